"""Write the golden fixtures that pin the CPU oracle.

Runs ONLY in the build container (needs the locally installed HF
``transformers``; nothing is downloaded: the model is built from a local
``Qwen3Config`` and random-initialised, then its weights are overwritten with
the repo's deterministic synthetic weights).  The fixtures are plain data
(``.npz``: inputs = config + seed + token stream, expected outputs = per-layer
residual stream, fp32 logits and greedy next tokens per decode step).

The HF model runs in fp32 with eager attention and an fp32 KV cache, so it is
the mathematical forward the reference's validation compares against
(/root/reference/host/validate.py:20-30,55-92) with fp32 activations.  The
oracle is checked against it in its fp32-KV mode (tests/test_oracle_golden.py);
its default bf16-KV mode adds only the rounding the reference applies when
appending to the cache (/root/reference/src/kv_cache.cuh:72,76).

Usage:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import layout, qwen3_ref, synth  # noqa: E402

FIXTURES = {
    # name: (shape, seed, gain_std, n_prompt, n_gen)
    "tiny": (layout.Shape(256, 4, 2, 64, 512, 2, 1024), 11, 0.1, 5, 6),
    "baseline_2l": (layout.Shape(1024, 16, 8, 64, 2816, 2, 4096), 7, 0.1, 4, 4),
}


def build_hf(shape: layout.Shape, bits: dict[str, np.ndarray]):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(
        vocab_size=shape.vocab, hidden_size=shape.hidden, intermediate_size=shape.ffn,
        num_hidden_layers=shape.n_layers, num_attention_heads=shape.n_q_heads,
        num_key_value_heads=shape.n_kv_heads, head_dim=shape.head_dim,
        rms_norm_eps=shape.eps, rope_parameters={"rope_type": "default", "rope_theta": shape.theta},
        tie_word_embeddings=True, hidden_act="silu", attention_bias=False,
        use_sliding_window=False, max_position_embeddings=4096)
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    model = Qwen3ForCausalLM(cfg).float().eval()
    f = lambda n: qwen3_ref.bits_to_torch(bits[n]).float()  # noqa: E731
    sd = {"model.embed_tokens.weight": f("embedding"), "model.norm.weight": f("final_norm"),
          "lm_head.weight": f("embedding")}
    hf_names = {
        "attn_norm": "input_layernorm.weight", "w_q": "self_attn.q_proj.weight",
        "w_k": "self_attn.k_proj.weight", "w_v": "self_attn.v_proj.weight",
        "q_norm": "self_attn.q_norm.weight", "k_norm": "self_attn.k_norm.weight",
        "w_o": "self_attn.o_proj.weight", "ffn_norm": "post_attention_layernorm.weight",
        "w_gate": "mlp.gate_proj.weight", "w_up": "mlp.up_proj.weight",
        "w_down": "mlp.down_proj.weight"}
    for i in range(shape.n_layers):
        for k, hk in hf_names.items():
            sd[f"model.layers.{i}.{hk}"] = f(f"layer.{i}.{k}")
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("rotary" in m for m in missing), missing
    return model


@torch.no_grad()
def run_hf(model, shape: layout.Shape, tokens_in: list[int], n_gen: int):
    from transformers import DynamicCache
    captured = []
    hooks = [model.model.embed_tokens.register_forward_hook(
        lambda m, i, o: captured.append(o[0, -1].clone()))]
    for layer in model.model.layers:
        hooks.append(layer.register_forward_hook(
            lambda m, i, o: captured.append((o[0] if isinstance(o, tuple) else o)[0, -1].clone())))
    cache = DynamicCache()
    feed = list(tokens_in)
    fed, layers, logits, nxt = [], [], [], []
    pos = 0
    while feed or len(nxt) < len(tokens_in) + n_gen:
        tok = feed.pop(0) if feed else nxt[-1]
        captured.clear()
        out = model(input_ids=torch.tensor([[tok]]), past_key_values=cache, use_cache=True,
                    position_ids=torch.tensor([[pos]]))
        cache = out.past_key_values
        lg = out.logits[0, -1].float()
        fed.append(tok)
        layers.append(torch.stack(captured).numpy())
        logits.append(lg.numpy())
        nxt.append(int(torch.argmax(lg)))
        pos += 1
    for h in hooks:
        h.remove()
    return np.array(fed), np.stack(layers), np.stack(logits), np.array(nxt)


def main():
    for name, (shape, seed, gain_std, n_prompt, n_gen) in FIXTURES.items():
        bits = qwen3_ref.synthetic_bits(shape, seed, std=0.02, gain_std=gain_std)
        prompt = synth.prompt_tokens(seed, n_prompt, shape.vocab)
        model = build_hf(shape, bits)
        fed, layers, logits, nxt = run_hf(model, shape, prompt, n_gen)
        path = os.path.join(HERE, f"hf_qwen3_{name}.npz")
        np.savez_compressed(
            path,
            shape=np.array([shape.hidden, shape.n_q_heads, shape.n_kv_heads, shape.head_dim,
                            shape.ffn, shape.n_layers, shape.vocab]),
            eps=shape.eps, theta=shape.theta, seed=seed, gain_std=gain_std, std=0.02,
            tokens_fed=fed, layers=layers.astype(np.float32), logits=logits.astype(np.float32),
            next_tokens=nxt)
        print(f"{path}: steps={len(fed)} layers={layers.shape} logits={logits.shape} "
              f"next={nxt.tolist()}")


if __name__ == "__main__":
    main()
