"""GPU parity of the operator microbench kernels (``megakernel_op_*``,
BASELINE configs[1]) against the CPU oracle's single ops
(oracle/qwen3_ref.py: rmsnorm, the fp32 matrix-vector product, silu_mul,
rope, argmax_first).

Tolerances (fp32 arithmetic on both sides, different summation order):
RMSNorm and RoPE outputs within 1e-5 relative + 1e-6 absolute; GEMV and LM-head
outputs (magnitude ~1) within 5e-5 absolute; argmax tokens identical unless
the oracle's top-1/top-2 margin is below 1e-4; exact ties resolve to the
lowest index.  Every case rotates several weight copies holding different
values and several inputs, so a wrong copy, input or output index fails.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from megakernel_amd import ops
from oracle import qwen3_ref

pytestmark = pytest.mark.gpu

GEMV_ATOL = 5e-5
NORM_RTOL, NORM_ATOL = 1e-5, 1e-6
ARGMAX_MARGIN = 1e-4


def _print(*a):
    print(*a, flush=True)


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def _bf16(shape, std: float, g: torch.Generator, mean: float = 0.0) -> torch.Tensor:
    return (torch.randn(shape, generator=g) * std + mean).to(torch.bfloat16)


def _packed(mats: list[torch.Tensor], layout: int) -> tuple[torch.Tensor, int]:
    """Pack row-major bf16 CPU matrices as consecutive copies in one device buffer."""
    rows, k = mats[0].shape
    nb = ops.packed_bytes(rows, k)
    buf = torch.empty(len(mats) * nb, dtype=torch.uint8, device="cuda")
    for c, m in enumerate(mats):
        src = m.contiguous().cuda()
        ops.pack(src, rows, k, layout, buf.data_ptr() + c * nb)
        del src
    return buf, nb


# ------------------------------------------------------------------ RMSNorm
@pytest.mark.parametrize("n", [1024, 512, 2048])
def test_op_rmsnorm(n):
    g = _gen(100 + n)
    n_in, reps = 5, 9
    x = _bf16((n_in, n), 1.0, g)
    x[3] = 0  # all-zero input: rsqrt(eps) * 0 == 0
    gain = _bf16((n,), 0.1, g, mean=1.0)
    y = torch.full((reps, n), float("nan"), device="cuda")
    _print(f"op_rmsnorm n={n} n_in={n_in} reps={reps}")
    ops.rmsnorm(x.cuda(), gain.cuda(), y, n, n_in, reps, reps, 1e-6)
    got = y.cpu()
    for r in range(reps):
        want = qwen3_ref.rmsnorm(x[r % n_in].float(), gain.float(), 1e-6)
        torch.testing.assert_close(got[r], want, rtol=NORM_RTOL, atol=NORM_ATOL, msg=f"instance {r}")
    assert torch.all(got[3] == 0)


# -------------------------------------------------------------------- GEMVs
GEMV_CASES = [
    # name, rows, k, kind       (BASELINE shapes first)
    ("qkv", 2048, 1024, ops.GEMV_PLAIN),
    ("o", 1024, 1024, ops.GEMV_PLAIN),
    ("down_residual", 1024, 2816, ops.GEMV_RESIDUAL),
    ("gate_up_silu", 2816, 1024, ops.GEMV_GATE_UP),
    ("qwen3_o", 1024, 2048, ops.GEMV_PLAIN),
    ("qwen3_down", 1024, 3072, ops.GEMV_RESIDUAL),
    ("tiny_gate_up", 512, 256, ops.GEMV_GATE_UP),
    ("tiny_down", 256, 512, ops.GEMV_RESIDUAL),
]


def _gemv_ref(w: torch.Tensor, x: torch.Tensor, kind: int, res: torch.Tensor | None) -> torch.Tensor:
    wf = w.float()
    if kind == ops.GEMV_GATE_UP:
        f = wf.shape[0] // 2
        return qwen3_ref.silu_mul(qwen3_ref.Qwen3Oracle._mv(wf[:f], x), qwen3_ref.Qwen3Oracle._mv(wf[f:], x))
    y = qwen3_ref.Qwen3Oracle._mv(wf, x)
    return y + res if kind == ops.GEMV_RESIDUAL else y


def _run_gemv(rows, k, kind, n_copies, n_in, reps, seed):
    g = _gen(seed)
    wrows = 2 * rows if kind == ops.GEMV_GATE_UP else rows
    mats = [_bf16((wrows, k), 0.02, g) for _ in range(n_copies)]
    layout = ops.LAYOUT_GATE_UP if kind == ops.GEMV_GATE_UP else ops.LAYOUT_TILE
    buf, nb = _packed(mats, layout)
    x = torch.randn((n_in, k), generator=g)
    res = torch.randn((n_in, rows), generator=g) if kind == ops.GEMV_RESIDUAL else None
    y = torch.full((reps, rows), float("nan"), device="cuda")
    ops.gemv(buf, nb, n_copies, rows, k, kind, x.cuda(), None if res is None else res.cuda(), n_in, y, reps, reps)
    got = y.cpu()
    worst = 0.0
    for r in range(reps):
        want = _gemv_ref(mats[r % n_copies], x[r % n_in], kind, None if res is None else res[r % n_in])
        err = float((got[r] - want).abs().max())
        worst = max(worst, err)
        assert err <= GEMV_ATOL, f"instance {r}: max abs err {err:.3e}"
    return worst


@pytest.mark.parametrize("name,rows,k,kind", GEMV_CASES, ids=[c[0] for c in GEMV_CASES])
def test_op_gemv(name, rows, k, kind):
    """3 weight copies x 2 inputs: 6 instances cover every (copy, input) pair."""
    _print(f"op_gemv {name} rows={rows} k={k} kind={kind}")
    worst = _run_gemv(rows, k, kind, n_copies=3, n_in=2, reps=6, seed=sum(map(ord, name)))
    _print(f"  worst abs err {worst:.2e}")


@pytest.mark.parametrize("n_in", [1, 3])
def test_op_gemv_many_items_per_workgroup(n_in):
    """More items than workgroups: a workgroup reuses (n_in = 1) or restages
    (n_in = 3) the input vector between its items."""
    _print(f"op_gemv qkv reps=40 n_in={n_in}")
    _run_gemv(2048, 1024, ops.GEMV_PLAIN, n_copies=2, n_in=n_in, reps=40, seed=7 + n_in)


# --------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("head_dim,positions", [
    (64, [0, 1, 7, 1023, 1279, 8191, 32767]),
    (128, [0, 3, 64, 100]),
])
def test_op_rope(head_dim, positions):
    g = _gen(head_dim)
    n_heads, n_in = 24, len(positions)
    reps = 2 * n_in
    x = torch.randn((n_in, n_heads, head_dim), generator=g)
    pos = torch.tensor(positions, dtype=torch.int32)
    y = torch.full((reps, n_heads, head_dim), float("nan"), device="cuda")
    _print(f"op_rope D={head_dim} positions={positions}")
    ops.rope(x.cuda(), pos.cuda(), y, n_heads, head_dim, n_in, reps, reps, 1e6)
    got = y.cpu()
    for r in range(reps):
        want = qwen3_ref.rope(x[r % n_in], positions[r % n_in], 1e6)
        torch.testing.assert_close(got[r], want, rtol=NORM_RTOL, atol=NORM_ATOL,
                                   msg=f"instance {r} pos {positions[r % n_in]}")
    assert torch.equal(got[0], x[0])  # position 0 is the identity
    # rotation preserves each (i, i + D/2) pair's norm
    h = head_dim // 2
    n_in_ = x[:, :, :h] ** 2 + x[:, :, h:] ** 2
    n_out = got[:n_in, :, :h] ** 2 + got[:n_in, :, h:] ** 2
    torch.testing.assert_close(n_out, n_in_, rtol=1e-5, atol=1e-6)


# --------------------------------------------------------- LM head + argmax
def _lm_case(vocab, k, n_copies, n_in, reps, seed, mats=None, h=None):
    g = _gen(seed)
    if mats is None:
        mats = [_bf16((vocab, k), 0.02, g) for _ in range(n_copies)]
    if h is None:
        h = torch.randn((n_in, k), generator=g)
    buf, nb = _packed(mats, ops.LAYOUT_TILE)
    logits = torch.full((reps, vocab), float("nan"), device="cuda")
    keys = torch.zeros(reps, dtype=torch.int64, device="cuda")
    toks = torch.full((reps,), -1, dtype=torch.int32, device="cuda")
    ops.lmhead_argmax(buf, nb, n_copies, vocab, k, h.cuda(), n_in, logits, keys, toks, reps, reps)
    del buf
    return mats, h, logits.cpu(), toks.cpu()


def test_op_lmhead_argmax_full_vocab():
    """BASELINE shape (151936 x 1024), 2 weight copies x 3 inputs."""
    vocab, k = 151936, 1024
    _print("op_lmhead_argmax vocab=151936 copies=2 reps=4")
    mats, h, logits, toks = _lm_case(vocab, k, n_copies=2, n_in=3, reps=4, seed=11)
    for r in range(4):
        want = qwen3_ref.Qwen3Oracle._mv(mats[r % 2].float(), h[r % 3])
        err = float((logits[r] - want).abs().max())
        assert err <= GEMV_ATOL, f"instance {r}: logits max abs err {err:.3e}"
        ref_tok = qwen3_ref.argmax_first(want)
        if int(toks[r]) != ref_tok:
            assert qwen3_ref.top2_margin(want) <= ARGMAX_MARGIN, f"instance {r}: {int(toks[r])} != {ref_tok}"
        assert int(toks[r]) == qwen3_ref.argmax_first(logits[r])  # token agrees with its own logits


def test_op_lmhead_argmax_ties_and_edges():
    """Two identical dominant rows -> the lower index; a dominant last row
    -> vocab - 1 (the final block of the final chunk)."""
    vocab, k = 4096 + 16 * 3, 1024  # last chunk partial
    g = _gen(12)
    h = torch.randn((2, k), generator=g)
    base = _bf16((vocab, k), 0.02, g)
    tie = base.clone()
    dom = (0.5 * torch.sign(h[0])).to(torch.bfloat16)
    tie[100] = dom
    tie[3000] = dom
    last = base.clone()
    last[vocab - 1] = (0.5 * torch.sign(h[1])).to(torch.bfloat16)
    _print("op_lmhead_argmax ties/edges")
    _, _, logits, toks = _lm_case(vocab, k, n_copies=2, n_in=2, reps=2, seed=12, mats=[tie, last], h=h)
    assert int(toks[0]) == 100
    assert logits[0, 100].item() == logits[0, 3000].item()
    assert int(toks[1]) == vocab - 1


def test_op_lmhead_argmax_tiny_k():
    """k = 256 (the TINY preset's hidden size)."""
    _print("op_lmhead_argmax vocab=2048 k=256")
    mats, h, logits, toks = _lm_case(2048, 256, n_copies=3, n_in=2, reps=6, seed=13)
    for r in range(6):
        want = qwen3_ref.Qwen3Oracle._mv(mats[r % 3].float(), h[r % 2])
        assert float((logits[r] - want).abs().max()) <= GEMV_ATOL
        assert int(toks[r]) == qwen3_ref.argmax_first(want) or qwen3_ref.top2_margin(want) <= ARGMAX_MARGIN


def test_op_pack_layouts_match_reference_layout():
    """The packed bytes follow the documented layout: element (row, col) of a
    tile block sits where mk_config.h says, and the gate/up layout interleaves
    gate block p at 2p and up block p at 2p + 1."""
    g = _gen(14)
    rows, k = 64, 512
    w = _bf16((rows, k), 1.0, g)
    wb = w.view(torch.int16).numpy().view(np.uint16)
    out = {}
    for layout in (ops.LAYOUT_TILE, ops.LAYOUT_GATE_UP):
        buf, _ = _packed([w], layout)
        out[layout] = buf.cpu().numpy().view(np.uint16)
    kt_n, half = k // 32, rows // 2
    for row, col in [(0, 0), (1, 7), (2, 8), (17, 300), (31, 511), (15, 256), (33, 40), (63, 511)]:
        kt, lt = col // 32, (row % 16) + 16 * ((col % 32) // 8)
        u = ((row // 16) * kt_n + kt) * 64 + lt
        assert out[ops.LAYOUT_TILE][u * 8 + col % 8] == wb[row, col]
        # gate rows [0, half): gate block p -> block 2p; up rows [half, rows): up block p -> 2p + 1
        db = 2 * (row // 16) if row < half else 2 * ((row - half) // 16) + 1
        u = (db * kt_n + kt) * 64 + lt
        assert out[ops.LAYOUT_GATE_UP][u * 8 + col % 8] == wb[row, col]
