"""CPU oracle for the batch-1 Qwen3 decode hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``megakernel_amd``) imports
this package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker / the
reported CPU baseline, never as the thing that is measured or shipped.

Contents
--------
synth      bit-exact restatement of the counter-based synthetic generator
           (splitmix64 -> Irwin-Hall(4) -> fp32 scale -> bf16 RNE) that the HIP
           library implements on the device.
layout     the reference's flat ``weights.bin`` layout and its 310-entry offset
           order (/root/reference/host/weight_loader.py:141-192,
           /root/reference/host/bridge.py:86-93), restated independently of the
           product's own layout code.
qwen3_ref  fp32-activation PyTorch forward of one decode step, following the
           reference kernel's phase order (/root/reference/src/megakernel.cu:132-332)
           and numerics policy (bf16 weights, fp32 activations/accumulation,
           bf16 KV cache, fp32 softmax).

Parity pins (what checks each function; see tests/test_oracle_*.py):
  * synth.splitmix64 / stream values: published splitmix64 known answers.
  * qwen3_ref forward: HF transformers ``Qwen3ForCausalLM`` golden fixtures
    (tests/golden/), plus closed-form checks of every op.
  * layout: the reference's own offset order and tensor shapes.
"""
