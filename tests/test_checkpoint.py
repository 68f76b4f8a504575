"""On-disk format (dequant_project_amd.checkpoint): save a quantized model,
rebuild it into a fresh skeleton, and check that every byte comes back.

The reference keeps quantized models only in memory; the state it holds is
the QuantLinear buffers (dequant/quant_linear.py:103-106) and QuantConfig
(:102), which is what the file carries. CPU only: the packer runs on the CPU
and no kernel is launched.
"""

import json

import pytest
import torch
from torch import nn

from dequant_project_amd import checkpoint as ck
from dequant_project_amd.packer import QuantConfig
from dequant_project_amd.quant_linear import PROJ, QuantLinear, quantize_model

transformers = pytest.importorskip("transformers")


def tiny_llama(seed, tie=False):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(hidden_size=128, intermediate_size=384, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=300, max_position_embeddings=64,
                      tie_word_embeddings=tie)
    torch.manual_seed(seed)
    return LlamaForCausalLM(cfg).half().eval()


def quant_state(model):
    return {k: v.clone() for k, v in model.state_dict().items()}


@pytest.mark.parametrize("cfg", [QuantConfig(4, 128, False, "sequential"), QuantConfig(2, 64, True, "interleaved"),
                                 QuantConfig(8, None, True, "sequential")], ids=repr)
def test_roundtrip_is_bit_exact(tmp_path, cfg):
    model = tiny_llama(1)
    stats = quantize_model(model, cfg)
    assert stats["replaced"] == 2 * len(PROJ)
    before = quant_state(model)
    path = tmp_path / "m.safetensors"
    info = ck.save_quantized(model, path, metadata={"note": "unit test"})
    assert info["quant_modules"] == 2 * len(PROJ)

    fresh = tiny_llama(2)  # different random init: every value must come from the file
    ck.load_quantized(fresh, path)
    after = fresh.state_dict()
    assert set(after) == set(before)
    for k, v in before.items():
        assert after[k].dtype == v.dtype and torch.equal(after[k], v), k
    for name, mod in model.named_modules():
        if isinstance(mod, QuantLinear):
            other = fresh.get_submodule(name)
            assert isinstance(other, QuantLinear)
            assert other.config == mod.config
            assert (other.out_features, other.in_features) == (mod.out_features, mod.in_features)
    meta = ck.read_metadata(path)
    assert meta["format"] == ck.FORMAT and meta["note"] == "unit test"
    assert len(meta["quant_modules"]) == 2 * len(PROJ)


def test_tied_embeddings_stored_once(tmp_path):
    model = tiny_llama(3, tie=True)
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    quantize_model(model, QuantConfig(4, 128, False))
    path = tmp_path / "t.safetensors"
    ck.save_quantized(model, path)
    meta = ck.read_metadata(path)
    assert meta["aliases"] in ({"lm_head.weight": "model.embed_tokens.weight"},
                               {"model.embed_tokens.weight": "lm_head.weight"})
    fresh = tiny_llama(4, tie=True)
    ck.load_quantized(fresh, path)
    assert torch.equal(fresh.lm_head.weight, model.lm_head.weight)
    assert fresh.lm_head.weight.data_ptr() == fresh.model.embed_tokens.weight.data_ptr()


def test_rejects_foreign_and_mismatched_files(tmp_path):
    from safetensors.torch import save_file

    plain = tmp_path / "plain.safetensors"
    save_file({"w": torch.zeros(2)}, str(plain))
    with pytest.raises(ValueError, match="not a"):
        ck.read_metadata(plain)

    model = tiny_llama(5)
    quantize_model(model, QuantConfig(4, 128, False))
    path = tmp_path / "m.safetensors"
    ck.save_quantized(model, path)
    # a skeleton of another shape cannot take the file
    from transformers import LlamaConfig, LlamaForCausalLM

    other = LlamaForCausalLM(LlamaConfig(hidden_size=128, intermediate_size=384, num_hidden_layers=1,
                                         num_attention_heads=4, num_key_value_heads=2, vocab_size=300,
                                         max_position_embeddings=64)).half()
    with pytest.raises(AttributeError):
        ck.load_quantized(other, path)

    # a tampered header (wrong packed shape) is refused before anything is built
    from safetensors import safe_open

    with safe_open(str(path), framework="pt") as f:
        meta = dict(f.metadata())
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    spec = json.loads(meta["quant_modules"])
    spec["model.layers.0.self_attn.q_proj"]["in_features"] = 256
    meta["quant_modules"] = json.dumps(spec)
    bad = tmp_path / "bad.safetensors"
    save_file(tensors, str(bad), metadata=meta)
    with pytest.raises(ValueError, match="qweight"):
        ck.load_quantized(tiny_llama(6), bad)


def test_reserved_metadata_keys(tmp_path):
    model = nn.Sequential(nn.Linear(128, 64, bias=False))
    with pytest.raises(ValueError, match="reserved"):
        ck.save_quantized(model, tmp_path / "x.safetensors", metadata={"format": "mine"})
