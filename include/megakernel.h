/* megakernel.h - C ABI of megakernel.so, the MI355X (gfx950) persistent
 * decode megakernel for a Qwen3-0.6B-shaped decoder.
 *
 * Drop-in boundary: the first six functions have exactly the signatures and
 * meaning of the reference library built by `make lib`
 * (/root/reference/src/megakernel.cu:535-624, bound through ctypes in
 * /root/reference/host/bridge.py:39-67).  Everything after them is additive.
 *
 * Conventions (all functions):
 *   - plain pointers and sizes only; no framework types cross the boundary;
 *   - the device is the caller's current HIP device;
 *   - functions returning int return >= 0 on success and -1 on failure, with
 *     a message available from megakernel_last_error(); functions returning a
 *     handle return NULL on failure (the reference never does, but its bridge
 *     already treats NULL as failure, bridge.py:106-107);
 *   - a handle is not reentrant: one host thread drives it at a time, as in
 *     the reference.
 *
 * Flat weight format (reference host/weight_loader.py:141-192): bf16 tensors
 * stored back to back; the offset array lists byte offsets in the order
 *   [embedding, final_norm, then per layer: attn_norm, w_q, w_k, w_v, q_norm,
 *    k_norm, w_o, ffn_norm, w_gate, w_up, w_down]
 * (reference megakernel.cu:518-532, bridge.py:86-93); matrices are row-major
 * [out, in].  The library repacks the weights into its own device layout at
 * init, so the caller's buffer is no longer read afterwards (the reference
 * requires it to outlive the handle; keeping it alive remains harmless).
 */
#ifndef MEGAKERNEL_H
#define MEGAKERNEL_H

#ifdef __cplusplus
extern "C" {
#endif

#define MK_DEFAULT_VOCAB 151936
#define MK_DEFAULT_MAX_SEQ 33024 /* >= 32768 prefill + 128 decode */

#define MK_PRESET_BASELINE 0  /* hidden 1024, 16/8 heads, head_dim 64, ffn 2816 */
#define MK_PRESET_QWEN3_06B 1 /* hidden 1024, 16/8 heads, head_dim 128, ffn 3072 */
#define MK_PRESET_TINY 2      /* hidden 256, 4/2 heads, head_dim 64, ffn 512 */

/* ---- reference entry points ------------------------------------------- */

/* Replaces megakernel_init (reference src/megakernel.cu:544-585).
 * d_weights: device pointer to the flat weight buffer; offsets: host array of
 * num_offsets = 2 + 11 * layers byte offsets (310 for 28 layers) of the
 * reference's contiguous weights.bin (host/weight_loader.py:141-192).  The
 * preset (BASELINE, QWEN3_06B or TINY) and the vocabulary are inferred from
 * the offset differences; offsets that match no supported shape exactly are
 * rejected (use megakernel_init_ex).  KV capacity MK_DEFAULT_MAX_SEQ.
 * Returns an opaque handle, or NULL on failure. */
void* megakernel_init(void* d_weights, long long* offsets, int num_offsets);

/* Replaces megakernel_decode (reference src/megakernel.cu:588-591).
 * Consumes input_token at the current position, returns the greedy next token
 * (argmax of fp32 logits, lowest index on ties) and advances the position by
 * one.  Blocking.  Returns -1 on error (bad token, KV full, device fault). */
int megakernel_decode(void* handle, int input_token);

/* Replaces megakernel_reset (reference src/megakernel.cu:594-601): zeroes the
 * KV cache and sets the position to 0. */
void megakernel_reset(void* handle);

/* Replaces megakernel_get_pos (reference src/megakernel.cu:604-607). */
int megakernel_get_pos(void* handle);

/* Replaces megakernel_free (reference src/megakernel.cu:610-617). */
void megakernel_free(void* handle);

/* Replaces megakernel_sync (reference src/megakernel.cu:620-622):
 * device-wide synchronize. */
void megakernel_sync(void);

/* ---- additive extensions ------------------------------------------------ */

/* Message of the last failure on this thread ("" if none). */
const char* megakernel_last_error(void);

/* megakernel_init with an explicit preset (MK_PRESET_*), vocabulary size
 * (multiple of 16) and KV capacity in positions.  When the offsets describe
 * a contiguous file of another preset or vocabulary the call fails; tensors
 * of a non-contiguous layout must not overlap at the preset's sizes. */
void* megakernel_init_ex(void* d_weights, const long long* offsets, int num_offsets, int preset, int vocab,
                         int max_seq);

/* Same, from a host copy of the flat weight file: the library uploads it, so
 * a caller needs no GPU framework at all (the reference bridge uploads with
 * torch, host/bridge.py:80-84). */
void* megakernel_init_from_host(const void* host_weights, unsigned long long nbytes, const long long* offsets,
                                int num_offsets, int preset, int vocab, int max_seq);

/* n greedy steps in ONE resident kernel launch: step 0 consumes first_token,
 * step i consumes the token step i-1 produced; out_tokens[i] (host, n ints)
 * receives step i's output.  Equivalent to n calls of megakernel_decode
 * without a host round trip per token.  Returns 0 or -1. */
int megakernel_generate(void* handle, int first_token, int n, int* out_tokens);

/* One decode step that also returns the residual stream after the embedding
 * and after every layer (layers_out: host float[(layers + 1) * hidden]) and
 * the fp32 logits (logits_out: host float[vocab]).  Validation only; either
 * pointer may be NULL.  Returns the next token or -1. */
int megakernel_debug_forward(void* handle, int token, float* layers_out, float* logits_out);

/* Set the decode position without touching the cache. */
int megakernel_set_pos(void* handle, int pos);

/* Copy a host KV prefix into the cache and set the position to len.
 * host_kv: bf16 [layers][2 (K, V)][n_kv_heads][len][head_dim], K after
 * QK-norm + RoPE (the reference's cache layout, src/kv_cache.cuh:11-32, with
 * len in place of MAX_SEQ_LEN). */
int megakernel_set_kv(void* handle, const void* host_kv, int len);

/* Copy positions [0, len) of the cache out in the megakernel_set_kv layout. */
int megakernel_get_kv(void* handle, void* host_kv, int len);

/* Fill positions [0, len) of the cache on the device with the synthetic
 * N(0, std^2) stream of oracle/synth.py (kv_prefill_bits) and set the
 * position to len. */
int megakernel_fill_kv_synthetic(void* handle, int len, unsigned long long seed, float std);

/* megakernel_generate that also records, for step trace_token, the device
 * wall clock (100 MHz on MI355X) when each workgroup's inputs of every phase
 * were ready and when it finished the phase, followed by 16 finer events of
 * the middle layer: host_trace receives u64[(5 * layers + 1) * 2 + 16][grid]
 * (0 = the workgroup had no such event).  Profiling only.  Returns the number
 * of entries or -1. */
int megakernel_trace_generate(void* handle, int first_token, int n, int trace_token,
                              unsigned long long* host_trace);

/* Device time of the last decode launch in milliseconds (HIP events). */
float megakernel_last_kernel_ms(void* handle);

/* Number of resident workgroups of the decode kernel (one per CU). */
int megakernel_grid_size(void* handle);

/* Minimum positions per attention work item (default 512). */
int megakernel_set_attention_chunk(void* handle, int chunk_min);

/* Above this many attention splits per kv head (default 20: contexts beyond
 * 10,240 positions at the default chunk) the workgroup of each head's first
 * split merges the head's splits and the O phase reads one merged partial; at
 * or below it every O workgroup merges the splits itself.  Tuning and testing
 * only. */
int megakernel_set_attention_merge(void* handle, int merge_min);

/* Which persistent kernel decodes (no counterpart in the reference, whose
 * kernel has one shape).  MK_KERNEL_AUTO (default): the class-specialised
 * kernel -- every workgroup keeps one role class for the launch and loads a
 * role's next weights right after computing it -- whenever a role table
 * holds all attention items of the launch (up to 4 splits per kv head on the
 * BASELINE and TINY presets), else the spread kernel; MK_KERNEL_SPREAD: always
 * the spread kernel.  megakernel_decode_kernel_for reports which kernel a
 * launch of n_tokens from the current position would use. */
#define MK_KERNEL_AUTO 0
#define MK_KERNEL_SPREAD 1
#define MK_KERNEL_CLASS 2
int megakernel_set_decode_kernel(void* handle, int variant);
int megakernel_decode_kernel_for(void* handle, int n_tokens);

/* FP8 LM head (no counterpart in the reference kernel, which plans FP8
 * weights in RESEARCH.md:434-436,463).  A mode other than MK_LMHEAD_BF16
 * builds, once, an OCP e4m3 copy of the tied LM head with one power-of-two
 * scale per row (2^e, the smallest e with max|row| <= 448 * 2^e; weights
 * rounded to nearest even after the exact scaling) and a per-row bound of its
 * error.  MK_LMHEAD_FP8: decode launches stream the copy, 1 byte per weight
 * instead of 2 for 32 % of the bytes of a token (logits and tokens of the FP8
 * weights).  MK_LMHEAD_SCREENED: the copy only screens -- every row whose
 * FP8 logit plus its error bound reaches the largest FP8 logit minus its
 * bound is scored again from the bf16 tiles, and the argmax runs over those
 * exact bf16 logits, so the tokens are the bf16 head's (class-specialised
 * kernel; the other launches use the bf16 head).  The embedding gather and the
 * prefill context keep the bf16 table.  MK_LMHEAD_BF16 (0) returns to bf16.
 * Returns 0, or -1 (unknown mode, vocab not a multiple of 16, hidden not of
 * 64, no memory). */
#define MK_LMHEAD_BF16 0
#define MK_LMHEAD_FP8 1
#define MK_LMHEAD_SCREENED 2
int megakernel_set_lmhead_fp8(void* handle, int enable);

/* FP8 KV cache (no counterpart in the reference kernel, which plans FP8 KV in
 * RESEARCH.md:434-436,463).  enable = 1 switches the handle's cache to OCP e4m3
 * codes with one power-of-two scale per (layer, kv head, position) row of K
 * and of V (2^e, the smallest e with max|row| <= 448 * 2^e; values rounded to
 * nearest even after the exact scaling), quantised as they are appended: half
 * the attention bytes of a token.  The cache is emptied (as megakernel_reset)
 * in either direction.  set_kv / get_kv / fill_kv_synthetic keep the bf16
 * reference layout at the boundary (quantised on the way in, exact bf16 of
 * code x scale on the way out); megakernel_prefill appends FP8 rows the same
 * way.  Returns 0 or -1. */
int megakernel_set_kv_fp8(void* handle, int enable);

/* The FP8 LM head as built: codes[V * H] row-major e4m3 bytes, scales[V]
 * (validation).  -1 when it has not been built. */
int megakernel_get_lmhead_fp8(void* handle, unsigned char* codes, float* scales);

/* FP8 layer weights (no counterpart in the reference kernel, which plans FP8
 * weights in RESEARCH.md:434-436,463).  enable = 1 builds, once, an OCP e4m3
 * copy of every layer's QKV, O, gate, up and down matrices with one
 * power-of-two scale per row (the quantisation of megakernel_set_lmhead_fp8)
 * and makes decode launches stream it: 1 byte per weight instead of 2 for 68 %
 * of the bytes of a token.  Norm gains, the embedding and the prefill context
 * keep bf16.  Served by the class-specialised kernel only: a launch that needs
 * the spread kernel (megakernel_set_decode_kernel(MK_KERNEL_SPREAD), or more
 * attention splits per kv head than the class kernel's role tables hold)
 * returns -1 while it is on.  enable = 0 returns to bf16.  Returns 0 or -1. */
int megakernel_set_layer_fp8(void* handle, int enable);

/* One FP8 layer matrix as built: codes[R * K] row-major e4m3 bytes and
 * scales[R] of matrix `which` of layer `layer` (validation): QKV = the fused
 * q | k | v rows [QD + 2 KVD][H], O [H][QD], GATE / UP [F][H], DOWN [H][F].
 * -1 when not built or out of range. */
#define MK_LAYER_QKV 0
#define MK_LAYER_O 1
#define MK_LAYER_GATE 2
#define MK_LAYER_UP 3
#define MK_LAYER_DOWN 4
int megakernel_get_layer_fp8(void* handle, int layer, int which, unsigned char* codes, float* scales);

/* Device fill of n bf16 values: bf16(float32(S_i - 131070) * c [+ 1.0f]),
 * S_i the Irwin-Hall(4) sum of the 16-bit fields of splitmix64(key, i). */
int megakernel_synth_fill(void* d_dst, unsigned long long n, unsigned long long key, float c, int add_one);

/* splitmix64 stream key of (seed, tensor_id); host-only arithmetic. */
unsigned long long megakernel_synth_key(unsigned long long seed, unsigned long long tensor_id);

/* The RoPE inverse-frequency table the kernel uses (host-only). Returns the
 * number of entries (head_dim / 2) or -1. */
int megakernel_rope_inv_freq(int preset, float* out, int n);

/* Thin device-memory helpers so ctypes callers need no GPU framework.
 * kind: 0 host->device, 1 device->host, 2 device->device. */
void* megakernel_device_alloc(unsigned long long nbytes);
void megakernel_device_free(void* d);
int megakernel_memcpy(void* dst, const void* src, unsigned long long nbytes, int kind);

/* CU count, wall-clock rate (kHz) and "name (gcnArch)" of the current device. */
int megakernel_device_info(int* cus, int* wall_clock_khz, char* name, int name_len);

/* ---- batched decode ------------------------------
 * megakernel_decode_batch is the additive entry point of the 16-sequence
 * configuration; the reference has no batched path (its
 * engine decodes one sequence, src/megakernel.cu:377-413).  A batch handle
 * holds its own weight copy (matrix-core tile layout) and n_seq KV caches;
 * every call advances all n_seq sequences by one greedy step per step.
 * Presets: MK_PRESET_BASELINE and MK_PRESET_TINY. */

/* Create a batch handle for n_seq (1..16) sequences of KV capacity max_seq
 * from the flat device weight buffer (same arguments as megakernel_init_ex).
 * All positions start at 0.  Returns NULL on failure. */
void* megakernel_batch_init(void* d_weights, const long long* offsets, int num_offsets, int preset, int vocab,
                            int n_seq, int max_seq);
void megakernel_batch_free(void* handle);

/* Position (number of cached positions) of sequence seq / of all sequences
 * (pos: host int[n_seq]). */
int megakernel_batch_set_pos(void* handle, int seq, int pos);
int megakernel_batch_get_pos(void* handle, int* pos);

/* KV prefix of one sequence: synthetic fill (the megakernel_fill_kv_synthetic
 * stream) or a host copy in the megakernel_set_kv layout; both set the
 * sequence's position to len. */
int megakernel_batch_fill_kv_synthetic(void* handle, int seq, int len, unsigned long long seed, float std);
int megakernel_batch_set_kv(void* handle, int seq, const void* host_kv, int len);
int megakernel_batch_get_kv(void* handle, int seq, void* host_kv, int len);

/* One greedy step of every sequence: tokens_in[b] is consumed at sequence b's
 * position, tokens_out[b] (may be NULL) receives its argmax next token
 * (lowest index on ties); positions advance by one.  Returns 0 or -1. */
int megakernel_decode_batch(void* handle, const int* tokens_in, int* tokens_out);

/* n_steps greedy steps of every sequence (one graph replay per step, no host
 * round trip in between): tokens_out[i * n_seq + b] receives step i's token
 * of sequence b. */
int megakernel_generate_batch(void* handle, const int* first_tokens, int n_steps, int* tokens_out);

/* megakernel_decode_batch that also returns the fp32 logits
 * (logits: host float[n_seq * vocab]).  Validation only. */
int megakernel_batch_debug_logits(void* handle, const int* tokens_in, int* tokens_out, float* logits);

/* Prefill for a batch-1 handle (the reference's generate feeds the prompt
 * through decode token by token, host/bridge.py:136-163).  attach builds a
 * prefill context bound to the handle's KV cache: the batched kernels'
 * matrix-core weight copy (a second copy of the weights) and work buffers,
 * from the same flat device weights and offsets the handle was built from
 * (d_weights NULL: the library's own upload, for handles made by
 * megakernel_init_from_host).  Presets BASELINE and TINY.  prefill consumes n
 * prompt tokens at the handle's position, 16 per weight pass (the tokens are
 * the matrix columns, each attending causally to the cache and to the earlier
 * prompt tokens), advances the position by n and returns the greedy token
 * after the prompt in *next_token (may be NULL).  Both return 0 or -1. */
int megakernel_prefill_attach(void* handle, void* d_weights, const long long* offsets, int num_offsets);
int megakernel_prefill(void* handle, const int* tokens, int n, int* next_token);

/* Prefill (the reference feeds a prompt token by token
 * through its decode, host/bridge.py:136-163): the n prompt tokens of
 * sequence seq are consumed at positions pos .. pos + n - 1 in passes of up
 * to 1,024 (64 groups of 16 matrix columns), each pass one sweep over the
 * weights; token i attends causally to the cache and to tokens < i.  Their
 * K / V are appended, the position advances by n, *next_token (may be NULL)
 * receives the greedy token after the last prompt token and logits (may be
 * NULL; host float[vocab]) its fp32 logits.  Returns 0 or -1. */
int megakernel_batch_prefill(void* handle, int seq, const int* tokens, int n, int* next_token, float* logits);

/* FP8 KV caches for every sequence of a batch handle (no counterpart in the
 * reference, which plans FP8 KV in RESEARCH.md:434-436,463): the format of
 * megakernel_set_kv_fp8 (e4m3 codes, one power-of-two scale per K / V row).
 * Every cache is emptied and every position reset to 0, in either direction;
 * batch set_kv / get_kv / fill keep the bf16 reference layout; batch prefill
 * appends FP8 rows.  Returns 0 or -1. */
int megakernel_batch_set_kv_fp8(void* handle, int enable);

/* FP8 LM head for a batch handle (no counterpart in the reference): the copy
 * of megakernel_set_lmhead_fp8, built once from the handle's bf16 tiles; the
 * step graph is captured again.  Returns 0 or -1. */
int megakernel_batch_set_lmhead_fp8(void* handle, int enable);

/* How a batched step runs its layers (no counterpart in the reference):
 * MK_BATCH_STEP_PER_PHASE (the default) launches one kernel per phase and
 * layer (five per layer); MK_BATCH_STEP_PERSISTENT runs every layer in one
 * persistent kernel of two workgroups per CU whose phases hand off through
 * per-producer flags.  Both compute the same sums in the same order, so
 * tokens and logits are identical.  Returns 0, or -1 (unknown variant, or the
 * persistent kernel does not fit two workgroups per CU). */
#define MK_BATCH_STEP_PERSISTENT 0
#define MK_BATCH_STEP_PER_PHASE 1
int megakernel_batch_set_step_kernel(void* handle, int variant);

/* Diagnostics of the persistent step (no counterpart in the reference): one
 * step as megakernel_decode_batch, recording the device wall clock (100 MHz)
 * per layer, event and workgroup into stamps[L][11][G] (events: layer start,
 * then inputs ready / done of QKV, attention, O, gate/up, down; 0 where the
 * workgroup has no role).  Returns G (the workgroup count), or -1. */
int megakernel_batch_trace_step(void* handle, const int* tokens_in, unsigned long long* stamps, long long n_stamps);

/* Device time of the last megakernel_generate_batch / decode_batch / prefill call (ms). */
float megakernel_batch_last_ms(void* handle);

/* ---- operator microbench ---------------------------
 * Each op of one decode step as a standalone launch, for measuring it against
 * its roofline.  The reference has these only as device functions inside its
 * kernel (no host entry points); each declaration names the device code it
 * restates.  Every call runs `reps` independent instances of the op in ONE
 * launch: instance r reads weight copy r % n_copies (copies copy_bytes
 * apart), input r % n_in and writes output slot r % n_out (instances sharing
 * a slot leave one of their results, or for the LM head the max over them).
 * All pointers are device pointers; inputs and outputs are fp32 unless noted.
 * Calls are blocking, run on the null stream and return 0, or -1 with
 * megakernel_last_error() set (arguments are checked before any GPU work).
 * megakernel_op_last_ms() gives the device time of the last call. */

#define MK_OP_LAYOUT_TILE 1    /* 16x32 tiles (layer matrices, LM head): K % 32 == 0 */
#define MK_OP_LAYOUT_GATE_UP 2 /* [gate; up] rows (2F x K) -> interleaved tile blocks */

#define MK_OP_GEMV_PLAIN 0     /* y = W x                     (QKV, O) */
#define MK_OP_GEMV_RESIDUAL 1  /* y = res + W x               (down + residual) */
#define MK_OP_GEMV_GATE_UP 2   /* y = silu(Wg x) * (Wu x)     (gate/up + SiLU) */

/* Bytes of one packed rows x k bf16 matrix (== rows * k * 2), or -1. */
long long megakernel_op_packed_bytes(int rows, int k);

/* Repack a row-major bf16 [rows][k] matrix (device) into `layout` at d_dst
 * (megakernel_op_packed_bytes(rows, k) bytes); both 16-byte aligned.  For
 * MK_OP_LAYOUT_GATE_UP, rows = 2F: gate rows first, then up rows. */
int megakernel_op_pack(const void* d_src, int rows, int k, int layout, void* d_dst);

/* rmsnorm_float_in (src/rmsnorm.cuh:87-108): y = x * rsqrt(mean(x^2) + eps) * gain
 * over n = 512 / 1024 / 2048; x bf16 [n_in][n], gain bf16 [n], y fp32 [n_out][n]. */
int megakernel_op_rmsnorm(const void* x, const void* gain, float* y, int n, int n_in, int n_out, int reps,
                          float eps);

/* gemv_qkv / gemv_block / gemv_gate_up_silu (src/gemv.cuh:36-279) and the
 * down projection with its residual (src/megakernel.cu:270-290).  w: packed
 * (MK_OP_LAYOUT_TILE, or MK_OP_LAYOUT_GATE_UP for kind 2), rows outputs,
 * k in {256, 512, 1024, 2048, 2816, 3072}; x [n_in][k]; res [n_in][rows]
 * (kind 1); y [n_out][rows]. */
int megakernel_op_gemv(const void* w, long long copy_bytes, int n_copies, int rows, int k, int kind, const float* x,
                       const float* res, int n_in, float* y, int n_out, int reps);

/* apply_rope_inplace (src/attention.cuh:22-44), out of place: x, y
 * [n][n_heads][head_dim] with instance r at position pos[r % n_in],
 * angle = pos * theta^(-2i/head_dim) in fp32 (HF convention). */
int megakernel_op_rope(const float* x, const int* pos, float* y, int n_heads, int head_dim, int n_in, int n_out,
                       int reps, float theta);

/* lm_head_argmax_phase1/2 (src/sampling.cuh:32-117): logits = E h, token =
 * argmax with the lowest index on ties.  w: MK_OP_LAYOUT_TILE [vocab][k],
 * k in {256, 512, 1024}; h [n_in][k]; logits [n_out][vocab] or NULL; keys
 * [n_out] (workspace, left holding ordered(logit) << 32 | ~index); tokens
 * [n_out]. */
int megakernel_op_lmhead_argmax(const void* w, long long copy_bytes, int n_copies, int vocab, int k, const float* h,
                                int n_in, float* logits, unsigned long long* keys, int* tokens, int n_out,
                                int reps);

/* megakernel_op_lmhead_argmax without the keys workspace: allocates nothing
 * (no device allocation, no event, no wait).  It has no counterpart in the
 * reference; it is for callers that cannot allocate -- tight serving loops,
 * harnesses that forbid allocation.  It enqueues on the null stream, so it is
 * not meant for code under stream capture (no capture is tested).  The keys
 * live in a static device array of MK_NOALLOC_KEYS_MAX entries per GPU, so
 * n_out <= MK_NOALLOC_KEYS_MAX (larger calls fail with an error); calls that
 * overlap on one GPU share that array and race.  The work is enqueued on the
 * null stream; outputs are complete after the caller synchronises. */
#define MK_NOALLOC_KEYS_MAX 4096
int megakernel_op_lmhead_argmax_noalloc(const void* w, long long copy_bytes, int n_copies, int vocab, int k,
                                        const float* h, int n_in, float* logits, int* tokens, int n_out, int reps);

/* Device time of this thread's last megakernel_op_* call (ms). */
float megakernel_op_last_ms(void);

/* Self-test of the hand-off primitive that replaces the reference's grid
 * barrier (src/barriers.cuh:38-73): one workgroup per CU runs `rounds`
 * all-gather rounds of tagged words (full tags and 4-bit packed pairs,
 * double-buffered by round parity) with the decode kernel's stores and
 * loads, counting words accepted with the right tag but a wrong value.
 * *mismatches receives that count (0 expected), *us_per_round (may be NULL)
 * the mean time of a round.  Returns -1 if a wait timed out. */
int megakernel_selftest_dataflow(int rounds, int* mismatches, float* us_per_round);

#ifdef __cplusplus
}
#endif
#endif /* MEGAKERNEL_H */
