"""The allocation-free LM head + argmax (megakernel_op_lmhead_argmax_noalloc)
against the workspace entry point it varies (megakernel_op_lmhead_argmax),
through the C ABI: identical logits and tokens (the same kernels), on two
calls in a row, the second with fewer outputs, so keys left in the static
array by the first call must not leak into the second."""
from __future__ import annotations

import ctypes

import pytest
import torch

from megakernel_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _p(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _case(lib, vocab: int, k: int, n_copies: int, n_in: int, n_out: int, reps: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    nb = ops.packed_bytes(vocab, k)
    w = torch.empty(n_copies * nb, dtype=torch.uint8, device="cuda")
    for c in range(n_copies):
        m = (torch.randn((vocab, k), generator=g) * 0.02).to(torch.bfloat16).cuda()
        ops.pack(m, vocab, k, ops.LAYOUT_TILE, w.data_ptr() + c * nb)
    h = torch.randn((n_in, k), generator=g).cuda()
    out = {}
    for name in ("workspace", "noalloc"):
        logits = torch.full((n_out, vocab), float("nan"), device="cuda")
        toks = torch.full((n_out,), -1, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        if name == "workspace":
            keys = torch.empty(n_out, dtype=torch.int64, device="cuda")
            rc = lib.megakernel_op_lmhead_argmax(_p(w), nb, n_copies, vocab, k, _p(h), n_in, _p(logits), _p(keys),
                                                 _p(toks), n_out, reps)
        else:
            rc = lib.megakernel_op_lmhead_argmax_noalloc(_p(w), nb, n_copies, vocab, k, _p(h), n_in, _p(logits),
                                                         _p(toks), n_out, reps)
        assert rc == 0, _lib.last_error(lib)
        lib.megakernel_sync()
        out[name] = (logits.cpu(), toks.cpu())
    return out


def test_noalloc_lmhead_matches_workspace_entry_point():
    lib = _lib.load()
    # first call: 64 outputs; second call: 5 outputs with another model and
    # inputs (the static keys still hold the first call's 64 maxima)
    for vocab, k, n_copies, n_in, n_out, reps, seed in [(8192, 1024, 2, 3, 64, 64, 1), (4096 + 48, 1024, 1, 2, 5, 5, 2)]:
        print(f"noalloc lmhead vocab {vocab} k {k} n_out {n_out} reps {reps}", flush=True)
        out = _case(lib, vocab, k, n_copies, n_in, n_out, reps, seed)
        (la, ta), (lb, tb) = out["workspace"], out["noalloc"]
        assert torch.equal(la, lb), "logits differ"
        assert torch.equal(ta, tb), f"tokens differ: {ta.tolist()} vs {tb.tolist()}"
        assert int(ta.min()) >= 0 and int(ta.max()) < vocab
        for r in range(n_out):  # each token is its own row's argmax (lowest index on ties)
            assert int(tb[r]) == int(torch.argmax(lb[r]))


def test_noalloc_rejects_more_outputs_than_the_static_array():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x10000)
    rc = lib.megakernel_op_lmhead_argmax_noalloc(fake, 0, 1, 4096, 1024, fake, 1, None, fake, 4097, 4097)
    assert rc == -1
    assert "static key array" in _lib.last_error(lib)
