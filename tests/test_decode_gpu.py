"""End-to-end: a locally built Llama with QuantLinear projections decodes on
the GPU (dequant_project_amd.decode), saved and reloaded through the on-disk
format (dequant_project_amd.checkpoint).

Reference for the logits: the same model with every projection replaced by
an nn.Linear holding packer.dequantize's fp16 weight (the reference's own
materialized form, packer.py:177-189), run by PyTorch. The two differ only
in arithmetic rounding (fp32-accumulated fused GEMV with the exact (q - z)*s
weight vs fp16 weight GEMMs); through two layers and the lm_head the logits
must agree to rel-L2 <= 2e-3.
"""

import copy

import pytest
import torch
from torch import nn

from dequant_project_amd import checkpoint as ck
from dequant_project_amd import decode
from dequant_project_amd.packer import QuantConfig
from dequant_project_amd.quant_linear import QuantLinear, dequantize_cuda, quantize_model

pytestmark = pytest.mark.gpu
pytest.importorskip("transformers")

LOGITS_REL_L2 = 2e-3


def rel_l2(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


def dequantized_twin(model):
    """Copy of `model` with each QuantLinear as an fp16 nn.Linear of packer.dequantize's weight."""
    twin = copy.deepcopy(model)
    for name, mod in list(twin.named_modules()):
        if isinstance(mod, QuantLinear):
            lin = nn.Linear(mod.in_features, mod.out_features, bias=mod.bias is not None,
                            device="cuda", dtype=torch.float16)
            with torch.no_grad():
                lin.weight.copy_(dequantize_cuda(mod._packed()))
                if mod.bias is not None:
                    lin.bias.copy_(mod.bias)
            parent_name, leaf = name.rsplit(".", 1)
            setattr(twin.get_submodule(parent_name), leaf, lin)
    return twin


@pytest.mark.parametrize("cfg", [QuantConfig(4, 128, False, "sequential"), QuantConfig(2, 64, False, "interleaved"),
                                 QuantConfig(8, None, True, "sequential")], ids=repr)
def test_decode_logits_match_dequantized_model(torch_gpu, cfg):
    model = decode.build_llama("tiny", seed=11)
    stats = quantize_model(model, cfg)
    assert stats["replaced"] == 14
    twin = dequantized_twin(model)
    for seq_len in (8, 40):  # prefill of seq_len - 1 tokens (M > 8 for 40: the dequantize + F.linear branch)
        step, restore, out = decode.decode_step_fn(model, seq_len)
        step()
        got = out["logits"].float()
        tstep, _, tout = decode.decode_step_fn(twin, seq_len)
        tstep()
        want = tout["logits"].float()
        err = rel_l2(got, want)
        print(f"{cfg} seq {seq_len}: logits rel-L2 {err:.2e}", flush=True)
        assert torch.isfinite(got).all()
        assert err <= LOGITS_REL_L2, f"{cfg} seq {seq_len}: rel-L2 {err:.3e}"


def test_graph_replay_matches_eager_and_is_repeatable(torch_gpu):
    model = decode.build_llama("tiny", seed=12)
    quantize_model(model, QuantConfig(4, 128, False))
    step, restore, out = decode.decode_step_fn(model, 32)
    step()
    eager = out["logits"].clone()
    restore()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
        restore()
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        step()
    for i in range(4):
        restore()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out["logits"], eager), f"replay {i} differs from the eager step"
        step()  # eager work between replays
        torch.cuda.synchronize()
        restore()


def test_timing_harness_reports(torch_gpu):
    model = decode.build_llama("tiny", seed=13)
    quantize_model(model, QuantConfig(4, 128, False))
    for mode in ("eager", "graph"):
        t, out = decode.time_decode(model, 16, mode, warmup=2, iters=5)
        assert t["gpu_ms"]["n"] == 5 and t["gpu_ms"]["median"] > 0
        assert t["total_ms"]["median"] >= t["host_ms"]["min"]
    assert decode.quantized_bytes_per_token(model, 16) > 0


def test_checkpoint_reload_gives_identical_logits(torch_gpu, tmp_path):
    model = decode.build_llama("tiny", seed=14)
    quantize_model(model, QuantConfig(4, 128, False))
    step, _, out = decode.decode_step_fn(model, 24)
    step()
    want = out["logits"].clone()
    path = tmp_path / "tiny.safetensors"
    ck.save_quantized(model, path)
    fresh = decode.build_llama("tiny", seed=15)
    ck.load_quantized(fresh, path, device="cuda")
    step2, _, out2 = decode.decode_step_fn(fresh, 24)
    step2()
    assert torch.equal(out2["logits"], want)
