"""The local-checkpoint path (reference host/weight_loader.py without the Hub
download): an HF Qwen3 safetensors directory -> weights.bin + offsets, and the
engine built from that file (GPU part)."""
import json
import os

import numpy as np
import pytest
import torch

from megakernel_amd import config, weights
from oracle import qwen3_ref

from ._helpers import check_step, oracle_shape


def _tiny_checkpoint(tmp_path, seed=3):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    s = config.TINY
    cfg = Qwen3Config(vocab_size=s.vocab, hidden_size=s.hidden, intermediate_size=s.ffn,
                      num_hidden_layers=s.n_layers, num_attention_heads=s.n_q_heads,
                      num_key_value_heads=s.n_kv_heads, head_dim=s.head_dim, rms_norm_eps=1e-6,
                      rope_theta=1e6, tie_word_embeddings=True, max_position_embeddings=512)
    torch.manual_seed(seed)
    model = Qwen3ForCausalLM(cfg).to(torch.bfloat16)
    with torch.no_grad():  # non-trivial norm gains so the mapping of every tensor is checked
        for n, p in model.named_parameters():
            if n.endswith("norm.weight"):
                p.copy_(1 + 0.1 * torch.randn_like(p))
    d = tmp_path / "ckpt"
    model.save_pretrained(d, safe_serialization=True)
    return d, model.state_dict()


def test_convert_matches_state_dict(tmp_path):
    d, state = _tiny_checkpoint(tmp_path)
    offs_path, shape = weights.convert_safetensors(str(d), str(tmp_path / "weights.bin"))
    assert shape == config.TINY
    flat = np.fromfile(tmp_path / "weights.bin", dtype=np.uint16)
    offs = weights.load_offsets(offs_path)
    assert list(offs) == weights.names(shape)  # reference order
    hf = {"embedding": "model.embed_tokens.weight", "final_norm": "model.norm.weight"}
    for i in range(shape.n_layers):
        for k, v in weights._HF_KEYS.items():
            hf[f"layer.{i}.{k}"] = f"model.layers.{i}.{v}"
    for name, key in hf.items():
        t = state[key].to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)
        got = flat[offs[name] // 2: offs[name] // 2 + t.size]
        assert np.array_equal(got, t), name


def test_unknown_shape_is_rejected():
    cfg = {"hidden_size": 512, "num_attention_heads": 8, "num_key_value_heads": 4, "head_dim": 64,
           "intermediate_size": 1024, "num_hidden_layers": 2, "vocab_size": 1024}
    with pytest.raises(ValueError):
        weights.shape_from_hf_config(cfg)


def test_wrong_tensor_shape_is_rejected(tmp_path):
    _, state = _tiny_checkpoint(tmp_path)
    state["model.layers.0.mlp.down_proj.weight"] = state["model.layers.0.mlp.down_proj.weight"].t()
    with pytest.raises(ValueError):
        weights.flat_from_state(state, config.TINY.with_(n_layers=2))


@pytest.mark.gpu
def test_engine_from_converted_checkpoint(tmp_path):
    from megakernel_amd.bridge import MegakernelEngine
    d, _ = _tiny_checkpoint(tmp_path, seed=5)
    wpath = str(tmp_path / "weights.bin")
    offs_path, shape = weights.convert_safetensors(str(d), wpath)
    eng = MegakernelEngine(weights_path=wpath, offsets_path=offs_path, shape=shape, max_seq=64)
    try:
        osh = oracle_shape(shape)
        bits = qwen3_ref.unpack_flat(osh, np.fromfile(wpath, dtype=np.uint8), weights.load_offsets(offs_path))
        orc = qwen3_ref.Qwen3Oracle(osh, bits, 64)
        tok = 17
        for i in range(4):
            nxt, layers, logits = eng.debug_forward(tok)
            ref = orc.step(tok, capture=True)
            check_step(layers, logits, ref, f"converted step {i}")
            tok = ref["token"]
    finally:
        eng.close()


def _write_tokenizer(d):
    """A small byte-level BPE tokenizer.json (ids < 300) beside the checkpoint."""
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers
    tok = Tokenizer(models.BPE(unk_token="<unk>"))
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=300, special_tokens=["<unk>", "<|endoftext|>"],
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(["a persistent kernel decodes one token per step on every CU"] * 40, trainer)
    tok.save(str(d / "tokenizer.json"))
    (d / "tokenizer_config.json").write_text(json.dumps({"eos_token": "<|endoftext|>"}))


@pytest.mark.gpu
def test_converted_checkpoint_tokenizer_prefill_generate(tmp_path):
    """The product surface end to end, offline: a local HF checkpoint and its
    tokenizer.json -> weights.bin -> engine built from the file with the
    prefill context (the library's own upload) -> generate(text).  The greedy
    ids after the prompt, fed back to the oracle, match its argmax wherever
    the margin exceeds 2e-2; the returned text is the decoded prompt +
    generation."""
    from megakernel_amd.bridge import MegakernelEngine
    from megakernel_amd.tokenizer import load_tokenizer

    from ._helpers import check_tokens_teacher_forced
    d, _ = _tiny_checkpoint(tmp_path, seed=6)
    _write_tokenizer(d)
    wpath = str(tmp_path / "weights.bin")
    offs_path, shape = weights.convert_safetensors(str(d), wpath)
    tok = load_tokenizer(str(d))
    eng = MegakernelEngine(weights_path=wpath, offsets_path=offs_path, shape=shape, max_seq=128, tokenizer=tok,
                           prefill=True)
    try:
        osh = oracle_shape(shape)
        bits = qwen3_ref.unpack_flat(osh, np.fromfile(wpath, dtype=np.uint8), weights.load_offsets(offs_path))
        orc = qwen3_ref.Qwen3Oracle(osh, bits, 128)
        prompt = "a persistent kernel decodes"
        ids = tok.encode(prompt)
        gen, _ = eng.generate_ids(ids, max_tokens=8)
        for t in ids[:-1]:
            orc.step(t)
        check_tokens_teacher_forced([ids[-1]] + gen[:-1], gen, orc)
        gen_eos, _ = eng.generate_ids(ids, max_tokens=8, eos_id=tok.eos_token_id)
        text, _ = eng.generate(prompt, max_tokens=8)
        assert text == tok.decode(ids + gen_eos, skip_special_tokens=True)
    finally:
        eng.close()
