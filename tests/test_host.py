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


def _pmc_csv(path, counter, rows):
    """A rocprofv3 counter_collection.csv with (dispatch id, kernel, value) rows."""
    with open(path, "w") as f:
        f.write("Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value\n")
        for d, k, v in rows:
            f.write(f"{d},{k},{counter},{v}\n")
    return str(path)


def test_step_traffic_sums_kernels_per_unit(tmp_path):
    """step-traffic: counters summed over the matching kernels' dispatches
    (rows of one dispatch added), divided by the unit kernel's dispatch count
    and scaled by what the copy of known size read; other kernels ignored."""
    from megakernel_amd import profiling
    bench = tmp_path / "b.json"
    bench.write_text("# noise\n" + json.dumps({"algorithmic_bytes_per_unit": 1000, "traffic_key": {"k": 1}}) + "\n")
    kf = [(1, "mk::batch::bk_qkv", 10), (1, "mk::batch::bk_qkv", 2), (2, "mk::batch::bk_tok", 3),
          (3, "mk::synth_kv_kernel", 500), (4, "mk::batch::bk_qkv", 5), (5, "mk::batch::bk_tok", 0)]
    kw = [(1, "mk::batch::bk_qkv", 4), (2, "mk::batch::bk_tok", 1), (4, "mk::batch::bk_qkv", 2),
          (5, "mk::batch::bk_tok", 1)]
    a = profiling.argparse.Namespace(
        fetch=_pmc_csv(tmp_path / "f.csv", "FETCH_SIZE", kf), write=_pmc_csv(tmp_path / "w.csv", "WRITE_SIZE", kw),
        copy_fetch=_pmc_csv(tmp_path / "cf.csv", "FETCH_SIZE", [(1, "copyBuffer", 50)]),
        copy_write=_pmc_csv(tmp_path / "cw.csv", "WRITE_SIZE", [(1, "copyBuffer", 100)]),
        copy_kernel="copyBuffer", copy_bytes=100.0, kernels="mk::batch::", unit_kernel="bk_tok",
        bench_json=str(bench))
    r = profiling.step_traffic(a)
    assert r["units"] == 2 and r["dispatches"] == 4
    assert r["fetch_bytes_per_unit"] == (10 + 2 + 3 + 5 + 0) / 2 * 2.0
    assert r["write_bytes_per_unit"] == (4 + 1 + 2 + 1) / 2 * 1.0
    assert r["traffic_over_algorithmic"] == (20.0 + 4.0) / 1000
    assert r["traffic_key"] == {"k": 1}


def test_bench_reports_step_traffic_only_for_its_workload(tmp_path):
    """bench.py takes a measured step / prompt traffic only when the summary's
    workload key is the run's, scaled to the run's algorithmic bytes; the
    committed summaries carry the keys the bench lines use."""
    sys.path.insert(0, ROOT)
    import bench
    p = tmp_path / "t.json"
    p.write_text(json.dumps({"traffic_key": {"what": "prefill", "prompt": 8}, "traffic_over_algorithmic": 1.5}))
    assert bench.measured_traffic(str(p), {"what": "prefill", "prompt": 8}, 1000) == 1500
    assert bench.measured_traffic(str(p), {"what": "prefill", "prompt": 16}, 1000) is None
    assert bench.measured_traffic(str(tmp_path / "none.json"), {"what": "prefill", "prompt": 8}, 1000) is None
    with open(os.path.join(ROOT, "profiles", "prefill1024_traffic.json")) as f:
        assert json.load(f)["traffic_key"] == {"what": "prefill", "prompt": 1024, "pass_tokens": 1024}
    with open(os.path.join(ROOT, "profiles", "batch16_traffic.json")) as f:
        key = json.load(f)["traffic_key"]
    assert key["what"] == "batch" and key["sequences"] == 16 and key["step"] == "per-phase"
    assert not key["kv_fp8"] and not key["lmhead_fp8"] and len(key["kv_lengths"]) == 16
