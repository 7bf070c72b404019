// CPU model of the decode kernel's tagged dataflow (test infrastructure).
//
// The reference synchronises its phases with grid barriers
// (/root/reference/src/barriers.cuh:38-73); the MI355X kernel replaces them
// with tagged words: a value and the number of the phase that produced it
// travel in one 64-bit word, and a consumer polls exactly the words it needs
// until every tag matches.  This program runs the kernel's phase structure on
// G threads ("workgroups") with the kernel's encodings and tag arithmetic:
//
//   x      [H/2]    packed pairs with 4-bit tags (residual rows 2i, 2i + 1 in
//                   word i: O and down publish them)
//   qkv    [QKV]    full 32-bit tags
//   part   [NS][NKV][W]  packed pairs with 4-bit tags tag % 15 + 1 (attention partials)
//   act    [F/2]    packed pairs with 4-bit tags (gate/up output)
//   amax   [2][G]   argmax slots, 14-bit tags tag % 16383 + 1, double-buffered
//                   by token parity
//
// with the phase order and per-token phase count of the kernel (5 phases per
// layer + the LM head, tags tag_base + 5 * layer + phase) and single-buffered
// activations.  Every producer writes values that are a known function of
// (token, layer, index), so a consumer that accepts a word with the right tag
// but the wrong value -- a stale word whose tag aliases, or a buffer
// overwritten before every reader consumed it -- is detected.  Threads sleep
// for random short intervals to vary the interleaving.  All shared words are
// std::atomic with relaxed order, as in the kernel; ThreadSanitizer checks the
// model for data races.
//
// The encodings and tag arithmetic are the kernel's own (mk_protocol.h).  G_IDLE
// of the threads have no role in any layer, like the workgroups of a large grid
// that only join the LM head: they wait for the last layer's QKV output
// before polling x (the kernel's wait_last_qkv).
//
// Usage: dataflow_model [drop | alias | nogate]
//   drop:   one producer omits one word of one phase; every waiting thread must
//           time out or see the error word and unwind ("timeout detected", 0);
//   alias:  a planted mistake -- 4-bit tags that repeat every 5 phases, so the
//           gate/up output of consecutive layers carries the same tag; the
//           model must report stale values (exit 2);
//   nogate: a planted mistake -- the idle threads poll x without waiting for
//           the last QKV output, so an x word 15 phases old passes its 4-bit
//           tag check; the model must report stale values (exit 2).
// Exit 0 and "ok" without arguments.
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <thread>
#include <vector>

#include "../../megakernel_amd/csrc/mk_protocol.h"

using mk::ll_pack;
using mk::ll_tag;
using mk::ll_val;
using mk::pk_pack;
using mk::pk_ready;
using mk::tag14;
using mk::u64;

constexpr int G_ROLE = 16, G_IDLE = 4;  // workgroups with layer roles / LM head only
constexpr int G = G_ROLE + G_IDLE;
constexpr int H = 64, NQ = 4, NKV = 2, D = 16, F = 96;
constexpr int QD = NQ * D, KVD = NKV * D, QKV = QD + 2 * KVD, GQA = NQ / NKV;
constexpr int NS = 3;                 // attention splits per kv head
constexpr int W = GQA * D / 2 + GQA;  // words of one split partial
constexpr int L = 4, T = 24;          // layers, tokens
constexpr int PHASES = mk::PHASES_PER_LAYER;

bool alias_mode = false, nogate_mode = false;
// the kernel's tag4; alias mode plants a period of 5 phases (= one layer)
unsigned tag4(unsigned tag) { return alias_mode ? tag % 5u + 1u : mk::tag4(tag); }
float pk_f(unsigned h) { return mk::f32_from(h & ~15u); }

// ---- shared state
std::atomic<u64> x[H / 2], qkv[QKV], part[NS * NKV * W], act[F / 2], amax[2 * G];
std::atomic<int> err{0}, bad{0};
std::atomic<long> polls{0};
bool drop_mode = false;

// values: small integers, exact in fp32 and in the 19-bit packed pairs
float val(int token, int layer, int buf, int i) { return (float)((token * 131 + layer * 37 + buf * 11 + i) % 4093); }

struct Ctx {
  int wg;
  std::mt19937 rng;
  void jitter() {
    const unsigned r = rng() % 8;
    if (r == 0) std::this_thread::sleep_for(std::chrono::microseconds(rng() % 50));
    else if (r < 3) std::this_thread::yield();
  }
};

// Bounded wait on one word (the kernel's Spin): false when it timed out or
// another thread already failed.
template <class Ok>
bool wait_word(std::atomic<u64>& w, Ok ok, u64* out) {
  const auto t0 = std::chrono::steady_clock::now();
  for (long n = 0;; ++n) {
    const u64 v = w.load(std::memory_order_relaxed);
    polls.fetch_add(1, std::memory_order_relaxed);
    if (ok(v)) {
      *out = v;
      return true;
    }
    if ((n & 255) == 255) {
      if (err.load(std::memory_order_relaxed)) return false;
      if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(300)) {
        err.store(1, std::memory_order_relaxed);
        return false;
      }
    }
    std::this_thread::yield();
  }
}

void expect(bool c, const char* what, int token, int layer, int i) {
  if (!c && bad.fetch_add(1) < 8) fprintf(stderr, "stale or wrong value: %s token %d layer %d index %d\n", what, token, layer, i);
}

// item -> workgroup offsets as in the kernel (phases on disjoint workgroups)
int first_item(int wg, int off) { return (wg + G_ROLE - off % G_ROLE) % G_ROLE; }

// Wait for x rows i, i + 1 (word i / 2, i even) of tag `tag` and check them
// against the values of (token, layer, buf).
bool need_x2(int i, unsigned tag, int token, int layer, int buf, const char* what) {
  u64 v;
  const unsigned t4 = tag4(tag);
  if (!wait_word(x[i / 2], [&](u64 w) { return pk_ready(w, t4); }, &v)) return false;
  expect(pk_f((unsigned)v) == val(token, layer, buf, i) && pk_f((unsigned)(v >> 32)) == val(token, layer, buf, i + 1),
         what, token, layer, i);
  return true;
}
void put_x2(int i, unsigned tag, int token, int layer, int buf) {
  x[i / 2].store(pk_pack(val(token, layer, buf, i), val(token, layer, buf, i + 1), tag4(tag)), std::memory_order_relaxed);
}

void run(int wg) {
  Ctx c{wg, std::mt19937(1234 + wg)};
  const unsigned per_token = PHASES * L + 1;
  const bool idle = wg >= G_ROLE;
  const int it_qkv = idle ? G : first_item(wg, G_ROLE / 4), it_att = idle ? G : first_item(wg, 0);
  const int it_o = idle ? G : first_item(wg, 3 * G_ROLE / 4);
  const int it_gu = idle ? G : first_item(wg, G_ROLE / 4), it_dn = idle ? G : first_item(wg, 0);
  const int RB_QKV = QKV / 16, RB_H = H / 16, RB_F = F / 16;
  for (int t = 0; t < T; ++t) {
    const unsigned tb = 1 + (unsigned)t * per_token;
    if (t > 0) {  // every workgroup reads the previous token's argmax slots
      for (int i = 0; i < G; ++i) {
        u64 v;
        const unsigned want = tag14(tb - 1u);
        if (!wait_word(amax[((t - 1) & 1) * G + i], [&](u64 w) { return (w & 0x3FFF) == want; }, &v)) return;
        expect((v >> 14) == (u64)(t - 1) * 1000 + i, "amax", t, -1, i);
      }
    }
    for (int layer = 0; layer < L; ++layer) {
      const unsigned tg = tb + PHASES * layer;
      c.jitter();
      // P1: QKV rows (needs all of x from the previous layer's down phase)
      if (it_qkv < RB_QKV) {
        if (layer > 0)
          for (int i = 0; i < H; i += 2)
            if (!need_x2(i, tg - 1u, t, layer - 1, 4, "x (down)")) return;
        for (int r = it_qkv; r < RB_QKV; r += G)
          for (int i = r * 16; i < r * 16 + 16; ++i) qkv[i].store(ll_pack(val(t, layer, 0, i), tg), std::memory_order_relaxed);
      }
      c.jitter();
      // P2: attention item (kv head g, split s): its head's q, k, v rows
      if (it_att < NKV * NS) {
        const int g = it_att / NS, s = it_att % NS;
        auto need = [&](int i) {
          u64 v;
          if (!wait_word(qkv[i], [&](u64 w) { return ll_tag(w) == tg; }, &v)) return false;
          expect(ll_val(v) == val(t, layer, 0, i), "qkv", t, layer, i);
          return true;
        };
        for (int j = 0; j < GQA; ++j)
          for (int d = 0; d < D; ++d)
            if (!need((g * GQA + j) * D + d)) return;
        for (int d = 0; d < D; ++d)
          if (!need(QD + g * D + d) || !need(QD + KVD + g * D + d)) return;
        const unsigned t4 = tag4(tg + 1u);
        for (int i = 0; i < W; ++i) {
          if (drop_mode && t == T / 2 && layer == 1 && g == 1 && s == 2 && i == 3) continue;  // the lost word
          const int k = (s * NKV + g) * W + i;
          part[k].store(pk_pack(val(t, layer, 1, 2 * k), val(t, layer, 1, 2 * k + 1), t4), std::memory_order_relaxed);
        }
      }
      c.jitter();
      // P3: O rows: every split partial of every head, plus this block's x rows
      if (it_o < RB_H) {
        const unsigned t4 = tag4(tg + 1u);
        for (int k = 0; k < NS * NKV * W; ++k) {
          u64 v;
          if (!wait_word(part[k], [&](u64 w) { return pk_ready(w, t4); }, &v)) return;
          expect(pk_f((unsigned)v) == val(t, layer, 1, 2 * k) && pk_f((unsigned)(v >> 32)) == val(t, layer, 1, 2 * k + 1),
                 "part", t, layer, k);
        }
        for (int i = it_o * 16; i < it_o * 16 + 16; i += 2) {
          if (layer > 0 && !need_x2(i, tg - 1u, t, layer - 1, 4, "x rows (O)")) return;
          put_x2(i, tg + 2u, t, layer, 2);
        }
      }
      c.jitter();
      // P4: gate/up pairs (needs all of x from the O phase)
      if (it_gu < RB_F) {
        for (int i = 0; i < H; i += 2)
          if (!need_x2(i, tg + 2u, t, layer, 2, "x (O)")) return;
        const unsigned t4 = tag4(tg + 3u);
        for (int r = it_gu; r < RB_F; r += G)
          for (int i = r * 8; i < r * 8 + 8; ++i)
            act[i].store(pk_pack(val(t, layer, 3, 2 * i), val(t, layer, 3, 2 * i + 1), t4), std::memory_order_relaxed);
      }
      c.jitter();
      // P5: down rows (all of act, plus this block's x rows from O)
      if (it_dn < RB_H) {
        const unsigned t4 = tag4(tg + 3u);
        for (int i = 0; i < F / 2; ++i) {
          u64 v;
          if (!wait_word(act[i], [&](u64 w) { return pk_ready(w, t4); }, &v)) return;
          expect(pk_f((unsigned)v) == val(t, layer, 3, 2 * i) && pk_f((unsigned)(v >> 32)) == val(t, layer, 3, 2 * i + 1),
                 "act", t, layer, i);
        }
        for (int i = it_dn * 16; i < it_dn * 16 + 16; i += 2) {
          if (!need_x2(i, tg + 2u, t, layer, 2, "x rows (down)")) return;
          put_x2(i, tg + 4u, t, layer, 4);
        }
      }
    }
    // LM head: every workgroup needs all of x from the last down phase and
    // publishes its argmax slot for this token
    const unsigned tl = tb + PHASES * L;
    if (idle && !nogate_mode) {  // wait_last_qkv: the last layer's QKV output, full tag
      u64 v;
      if (!wait_word(qkv[0], [&](u64 w) { return ll_tag(w) == tl - (unsigned)PHASES; }, &v)) return;
    }
    for (int i = 0; i < H; i += 2)
      if (!need_x2(i, tl - 1u, t, L - 1, 4, "x (final)")) return;
    amax[(t & 1) * G + wg].store(((u64)t * 1000 + wg) << 14 | tag14(tl), std::memory_order_relaxed);
  }
}

int main(int argc, char** argv) {
  drop_mode = argc > 1 && strcmp(argv[1], "drop") == 0;
  alias_mode = argc > 1 && strcmp(argv[1], "alias") == 0;
  nogate_mode = argc > 1 && strcmp(argv[1], "nogate") == 0;
  // the host clears every tagged buffer (tag 0) when a handle is created (and
  // the packed-pair buffers again when the position moves back); consecutive
  // launches continue the tag sequence, so the T tokens here stand for any
  // split of them into launches
  for (auto& w : x) w.store(0);
  for (auto& w : qkv) w.store(0);
  for (auto& w : part) w.store(0);
  for (auto& w : act) w.store(0);
  for (auto& w : amax) w.store(0);
  std::vector<std::thread> th;
  for (int i = 0; i < G; ++i) th.emplace_back(run, i);
  for (auto& t : th) t.join();
  const int e = err.load(), b = bad.load();
  printf("threads %d tokens %d layers %d polls %ld error %d wrong values %d\n", G, T, L, polls.load(), e, b);
  if (b) return 2;
  if (drop_mode) {
    if (!e) return 3;
    printf("timeout detected\n");
    return 0;
  }
  if (e) return 4;
  printf("ok\n");
  return 0;
}
