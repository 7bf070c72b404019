"""Host-side logic that needs no GPU: the flat weight format and its offset
order, byte accounting of the roofline, the tag arithmetic, the bench's
--gpus contract."""
import json
import os
import subprocess
import sys

from megakernel_amd import config, weights
from oracle import layout

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_flat_layout_matches_reference_order_and_independent_restatement():
    s = config.BASELINE
    fl = weights.flat_layout(s)
    ol = layout.offsets(layout.BASELINE)
    assert fl.total_bytes == ol["__total__"]
    names = layout.ordered_names(layout.BASELINE)
    assert [fl.offsets[n] for n in names] == [ol[n] for n in names]
    # reference order (src/megakernel.cu:518-532, host/bridge.py:86-93)
    assert names[:2] == ["embedding", "final_norm"]
    assert names[2:13] == [f"layer.0.{k}" for k in ("attn_norm", "w_q", "w_k", "w_v", "q_norm", "k_norm",
                                                    "w_o", "ffn_norm", "w_gate", "w_up", "w_down")]
    assert len(fl.ordered_offsets()) == 2 + 11 * 28 == 310
    # every tensor starts 16-byte aligned (the library loads 16-byte units)
    assert all(o % 16 == 0 for o in fl.ordered_offsets())


def test_byte_accounting():
    s = config.BASELINE
    assert s.layer_weight_bytes == 23_597_312
    assert s.weight_bytes == 971_891_712 == weights.flat_layout(s).total_bytes
    assert s.kv_bytes_per_pos == 57_344 == 2 * 8 * 64 * 2 * 28
    assert s.token_bytes(1024) == 971_891_712 + 57_344 * 1026
    # 8 TB/s roofline at ctx 1024: 7,762 tok/s
    assert round(8e12 / s.token_bytes(1024)) == 7762


def test_w_o_shape_is_hidden_by_qdim():
    # the reference's validate_shapes has it transposed (reference host/weight_loader.py:128); the
    # matrix is [out = hidden, in = q_dim] row-major
    assert weights.tensor_dims(config.QWEN3_06B, "w_o") == (1024, 16 * 128)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]
