"""Fused activation prologues: RMSNorm -> projections, SwiGLU -> down_proj.

The reference plans these fusions as its next step (MODEL_SELECTION.md:211-218:
fold the norms and the SwiGLU into the GEMVs so a decoder layer stops paying a
kernel, and an activation round trip, per elementwise op; byte_model.py:227-228
counts those activation bytes). Here they are prologues of the M = 1 GEMV
kernel (dq_gemv_prologue_batched):

  gemv_rmsnorm(x, gamma, eps, pws)  [W_i (rmsnorm(x) * gamma)] in ONE launch
                                    (q|k|v or gate|up of a layer share x)
  gemv_swiglu(gate, up, pw)         W (silu(gate) * up)

and `fuse_llama(model)` routes a Hugging Face Llama's decode steps through
them: per layer, input_layernorm + q|k|v become one launch, and
post_attention_layernorm + gate|up, then SwiGLU + down_proj, two more. Batches
of more than one row (prefill) run the model's own modules unchanged.

Numerics: RMSNorm is computed as (W (x * gamma)) / sqrt(mean(x^2) + eps) with
fp32 sums and fp16 products x * gamma, where the unfused module rounds
x / rms to fp16 and multiplies by gamma in fp16; SwiGLU rounds like the
unfused fp16 ops (silu in fp32, rounded; times up, rounded). Both match the
unfused composition to the fp16 rounding of the activations. Valid input
range of the RMSNorm prologue: every product x_i * gamma_i must be a finite
fp16 value (|x_i * gamma_i| <= 65504), since it is formed before the
division by rms(x); the unfused module divides first. Decoder residual
streams (entries up to a few thousand, gamma of order one) are far inside it.
"""

import torch
from torch import nn

from . import _native
from .packer import PackedWeight
from .quant_linear import QuantLinear

PROLOGUE_RMSNORM = 1
PROLOGUE_SWIGLU = 2


def _check_group(pws):
    cfg0 = pws[0].config
    if any(pw.config.bits != cfg0.bits or pw.config.symmetric != cfg0.symmetric
           or pw.config.layout != cfg0.layout for pw in pws):
        raise ValueError("fused GEMV: all weights must share bits, symmetric and layout")
    return cfg0


def _launch(xs, auxs, prologue, eps, pws):
    cfg0 = _check_group(pws)
    return _native.ext().gemv_prologue(
        xs, auxs, prologue, float(eps), [pw.qweight for pw in pws], [pw.scales for pw in pws],
        [pw.zeros for pw in pws], cfg0.bits, [pw.config.effective_group_size(pw.shape[1]) for pw in pws],
        cfg0.symmetric, cfg0.layout == "interleaved")


def gemv_rmsnorm(x, gamma, eps, pws):
    """[y_i = rmsnorm(x; gamma, eps) @ W_i^T] for one activation row, one launch.

    x fp16 [..., K] holding one row; gamma fp16 [K]; every W_i [N_i, K] packed
    in one format (up to 16). Returns fp16 [..., N_i] per weight.
    """
    pws = list(pws)
    k = pws[0].shape[1]
    x2 = x.reshape(-1, k).contiguous()
    g = gamma.contiguous()
    ys = _launch([x2] * len(pws), [g] * len(pws), PROLOGUE_RMSNORM, eps, pws)
    return [y.view(*x.shape[:-1], pw.shape[0]) for y, pw in zip(ys, pws)]


def gemv_swiglu(gate, up, pw: PackedWeight):
    """y = (silu(gate) * up) @ W^T for one activation row, one launch.

    gate, up fp16 [..., K] (the gate and up projections' outputs); W [N, K].
    """
    k = pw.shape[1]
    g2 = gate.reshape(-1, k).contiguous()
    u2 = up.reshape(-1, k).contiguous()
    (y,) = _launch([g2], [u2], PROLOGUE_SWIGLU, 0.0, [pw])
    return y.view(*gate.shape[:-1], pw.shape[0])


# --------------------------------------------------------- Llama integration
class _Pending:
    """Hand-off between a deferred norm and the projections that consume it."""

    def __init__(self):
        self.x = None        # the raw (un-normalized) activation the norm let through
        self.gamma = None
        self.eps = 0.0
        self.outputs = {}    # role -> projection output computed by the fused launch


def _rows(x):
    return x.numel() // x.shape[-1]


def _norm_eps(norm):
    for name in ("variance_epsilon", "eps"):
        if hasattr(norm, name):
            return float(getattr(norm, name))
    raise ValueError(f"cannot find the epsilon of {type(norm).__name__}")


class _DeferredNorm(nn.Module):
    """Stands in for an RMSNorm whose consumers fuse it: for one-row inputs it
    returns x unchanged and records it (the fused projections normalize);
    otherwise it is the norm."""

    def __init__(self, norm, pending):
        super().__init__()
        self.norm = norm
        self.pending = pending
        self.eps = _norm_eps(norm)

    def forward(self, x):
        p = self.pending
        p.outputs = {}
        if _rows(x) == 1 and x.dtype == torch.float16:
            p.x, p.gamma = x, self.norm.weight
            p.eps = self.eps
            return x
        p.x = None
        return self.norm(x)


class _FusedProjection(nn.Module):
    """One of a group of QuantLinear projections fed by a deferred norm: the
    first member called with the deferred activation runs the whole group in
    one launch; the others return their share."""

    def __init__(self, linear: QuantLinear, role, group, pending):
        super().__init__()
        self.linear = linear
        self.role = role
        self.group = group  # [(role, QuantLinear)], shared by the members
        self.pending = pending

    def forward(self, x):
        p = self.pending
        if p.x is None or x is not p.x:
            return self.linear(x)
        if self.role not in p.outputs:
            lins = [lin for _, lin in self.group]
            ys = gemv_rmsnorm(x, p.gamma, p.eps, [lin._packed() for lin in lins])
            for (role, lin), y in zip(self.group, ys):
                p.outputs[role] = y if lin.bias is None else y + lin.bias
        return p.outputs.pop(self.role)


class _FusedMLP(nn.Module):
    """LlamaMLP for one-row inputs behind a deferred norm: gate|up with the
    RMSNorm prologue in one launch, then down_proj with the SwiGLU prologue."""

    def __init__(self, mlp, pending):
        super().__init__()
        self.mlp = mlp
        self.pending = pending

    def forward(self, x):
        p = self.pending
        if p.x is None or x is not p.x:
            return self.mlp(x)
        m = self.mlp
        gate, up = gemv_rmsnorm(x, p.gamma, p.eps, [m.gate_proj._packed(), m.up_proj._packed()])
        if m.gate_proj.bias is not None:
            gate = gate + m.gate_proj.bias
        if m.up_proj.bias is not None:
            up = up + m.up_proj.bias
        y = gemv_swiglu(gate, up, m.down_proj._packed())
        return y if m.down_proj.bias is None else y + m.down_proj.bias


def _is_silu(act):
    # torch's nn.SiLU, or transformers' SiLUActivation (ACT2FN["silu"]), which
    # applies torch.nn.functional.silu
    return isinstance(act, nn.SiLU) or type(act).__name__ == "SiLUActivation"


def _fmt(lin):
    return lin.config.bits, lin.config.symmetric, lin.config.layout


def _fusable_mlp(mlp):
    """gate | up run as one grouped launch, so they must share bits, symmetry
    and layout; down_proj is a launch of its own and may differ."""
    return (all(isinstance(getattr(mlp, n, None), QuantLinear) for n in ("gate_proj", "up_proj", "down_proj"))
            and _is_silu(getattr(mlp, "act_fn", None))
            and _fmt(mlp.gate_proj) == _fmt(mlp.up_proj))


def fuse_llama(model):
    """Route the one-row (decode) steps of a quantized Llama through the fused
    prologues, in place. Layers whose projections are not QuantLinear of one
    format per group, or whose MLP activation is not SiLU, are left as they
    are. Returns {"attention": layers fused, "mlp": layers fused}."""
    stats = {"attention": 0, "mlp": 0}
    for layer in model.modules():
        attn = getattr(layer, "self_attn", None)
        mlp = getattr(layer, "mlp", None)
        if attn is None or not hasattr(layer, "input_layernorm"):
            continue
        qkv = [(r, getattr(attn, r, None)) for r in ("q_proj", "k_proj", "v_proj")]
        if all(isinstance(lin, QuantLinear) for _, lin in qkv) and len({_fmt(lin) for _, lin in qkv}) == 1:
            pending = _Pending()
            layer.input_layernorm = _DeferredNorm(layer.input_layernorm, pending)
            group = list(qkv)
            for role, lin in qkv:
                setattr(attn, role, _FusedProjection(lin, role, group, pending))
            stats["attention"] += 1
        if mlp is not None and hasattr(layer, "post_attention_layernorm") and _fusable_mlp(mlp):
            pending = _Pending()
            layer.post_attention_layernorm = _DeferredNorm(layer.post_attention_layernorm, pending)
            layer.mlp = _FusedMLP(mlp, pending)
            stats["mlp"] += 1
    return stats
