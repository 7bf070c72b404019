"""Offline tokenizers for MegakernelEngine.generate (megakernel_amd/tokenizer.py):
a local tokenizer.json (the reference's AutoTokenizer is a Hub download,
/root/reference/host/weight_loader.py:48-60) and the byte tokenizer of the
synthetic models."""
import json

import pytest

from megakernel_amd.tokenizer import ByteTokenizer, load_tokenizer


def test_byte_tokenizer_round_trip():
    t = ByteTokenizer(vocab=1024, eos_token_id=300)
    text = "megakernel on MI355X: ok ✓"
    ids = t.encode(text)
    assert all(0 <= i < 256 for i in ids) and len(ids) == len(text.encode("utf-8"))
    assert t.decode(ids) == text
    assert t.encode(text, add_bos=True)[0] == t.bos_token_id
    assert t.decode(ids + [300, 700], skip_special_tokens=True) == text
    assert t.decode([65, 300]) == "A<|300|>"
    assert t.eos_token_id == 300
    with pytest.raises(ValueError):
        ByteTokenizer(vocab=100)


def _tiny_bpe(tmp_path):
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers
    tok = Tokenizer(models.BPE(unk_token="<unk>"))
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=300, special_tokens=["<unk>", "<|endoftext|>"],
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    corpus = ["the persistent decode kernel streams the weights once per token"] * 50
    tok.train_from_iterator(corpus, trainer)
    tok.save(str(tmp_path / "tokenizer.json"))
    return tok


def test_local_tokenizer_json_and_eos(tmp_path):
    tok = _tiny_bpe(tmp_path)
    (tmp_path / "tokenizer_config.json").write_text(json.dumps({"eos_token": "<|endoftext|>"}))
    t = load_tokenizer(str(tmp_path))
    assert t.eos_token_id == tok.token_to_id("<|endoftext|>")
    text = "the decode kernel streams weights"
    ids = t.encode(text)
    assert ids == tok.encode(text).ids
    assert t.decode(ids) == text
    assert t.decode(ids + [t.eos_token_id], skip_special_tokens=True) == text
    # generation_config.json takes precedence (the HF Qwen3 checkpoints carry one)
    (tmp_path / "generation_config.json").write_text(json.dumps({"eos_token_id": [7, 8]}))
    assert load_tokenizer(str(tmp_path)).eos_token_id == 7


def test_missing_tokenizer_json(tmp_path):
    with pytest.raises(FileNotFoundError, match="tokenizer.json"):
        load_tokenizer(str(tmp_path))
