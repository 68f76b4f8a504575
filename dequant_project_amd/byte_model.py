"""Analytical byte model of batch-1 decode, extended with the MI355X roofline.

Restates the reference's dequant/byte_model.py (BITS :20, ModelSpec :23-49,
spec_from_hf_config :52-99, param_counts :121-150, _quant_bytes :165-176,
decode_bytes :179-251, predicted_latency_s :254-256) and adds what the
MI355X engine is graded against:

  MI355X_HBM_PEAK_BYTES_S   8.0e12 B/s, the vendor HBM3E peak (the denominator
                            of every "% of peak" this project reports)
  gemv_call_bytes()         algorithmic bytes of one fused dequant-GEMV call:
                            qweight + scales (+ zeros) + x + y, i.e.
                            PackedWeight.nbytes + M*K*2 + M*N*2 -- the
                            reference's per-call figure
                            (scripts/bench_dequant_kernel.py:156)
  roofline_us() / pct_of_peak()
"""

from dataclasses import dataclass

# Storage cost of one element, in bits.
BITS = {"fp32": 32, "bf16": 16, "fp16": 16, "fp8": 8, "int8": 8, "int4": 4, "int2": 2}

# ---- MI355X (gfx950, CDNA4) ------------------------------------------------
MI355X_HBM_PEAK_BYTES_S = 8.0e12        # HBM3E, 8 stacks, vendor peak
MI355X_HBM_BYTES = 288 * 2 ** 30
MI355X_INFINITY_CACHE_BYTES = 256 * 2 ** 20
MI355X_CUS = 256
MI355X_XCDS = 8
MI355X_LDS_BYTES_PER_CU = 160 * 1024
MI355X_L2_BYTES_PER_XCD = 4 * 2 ** 20


@dataclass(frozen=True)
class ModelSpec:
    """Architecture reduced to the numbers that drive byte counts."""

    name: str
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    tied_embedding: bool
    gated_mlp: bool
    qkv_bias: bool
    proj_bias: bool
    norm_bias: bool
    n_positions: int
    max_context: int

    @property
    def q_dim(self):
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim

    def linear_shapes(self):
        """(name, N, K) of the seven quantized projections of one layer (gated MLP)."""
        h, i = self.hidden, self.intermediate
        return [("q_proj", self.q_dim, h), ("k_proj", self.kv_dim, h), ("v_proj", self.kv_dim, h),
                ("o_proj", h, self.q_dim), ("gate_proj", i, h), ("up_proj", i, h),
                ("down_proj", h, i)]


def spec_from_hf_config(cfg, name=None):
    """ModelSpec from a HuggingFace config dict (gpt2 / llama / qwen2 / mistral)."""
    mt = cfg.get("model_type")
    name = name or mt
    if mt == "gpt2":
        hidden = cfg["n_embd"]
        return ModelSpec(name=name, n_layers=cfg["n_layer"], hidden=hidden, n_heads=cfg["n_head"],
                         n_kv_heads=cfg["n_head"], head_dim=hidden // cfg["n_head"],
                         intermediate=cfg.get("n_inner") or 4 * hidden, vocab=cfg["vocab_size"],
                         tied_embedding=cfg.get("tie_word_embeddings", True), gated_mlp=False,
                         qkv_bias=True, proj_bias=True, norm_bias=True,
                         n_positions=cfg["n_positions"], max_context=cfg["n_positions"])
    if mt in ("llama", "qwen2", "mistral"):
        hidden = cfg["hidden_size"]
        n_heads = cfg["num_attention_heads"]
        return ModelSpec(name=name, n_layers=cfg["num_hidden_layers"], hidden=hidden, n_heads=n_heads,
                         n_kv_heads=cfg.get("num_key_value_heads", n_heads),
                         head_dim=cfg.get("head_dim") or hidden // n_heads,
                         intermediate=cfg["intermediate_size"], vocab=cfg["vocab_size"],
                         tied_embedding=cfg.get("tie_word_embeddings", False), gated_mlp=True,
                         qkv_bias=cfg.get("attention_bias", mt == "qwen2"), proj_bias=False,
                         norm_bias=False, n_positions=0, max_context=cfg["max_position_embeddings"])
    raise ValueError(f"unsupported model_type: {mt!r}")


# Published architecture numbers of the two stacks the benchmark configs use.
LLAMA_3_8B_CONFIG = {
    "model_type": "llama", "num_hidden_layers": 32, "hidden_size": 4096,
    "num_attention_heads": 32, "num_key_value_heads": 8, "head_dim": 128,
    "intermediate_size": 14336, "vocab_size": 128256, "tie_word_embeddings": False,
    "attention_bias": False, "max_position_embeddings": 8192,
}
LLAMA_3_70B_CONFIG = {
    "model_type": "llama", "num_hidden_layers": 80, "hidden_size": 8192,
    "num_attention_heads": 64, "num_key_value_heads": 8, "head_dim": 128,
    "intermediate_size": 28672, "vocab_size": 128256, "tie_word_embeddings": False,
    "attention_bias": False, "max_position_embeddings": 8192,
}
LLAMA_3_2_1B_CONFIG = {
    "model_type": "llama", "num_hidden_layers": 16, "hidden_size": 2048,
    "num_attention_heads": 32, "num_key_value_heads": 8, "head_dim": 64,
    "intermediate_size": 8192, "vocab_size": 128256, "tie_word_embeddings": True,
    "attention_bias": False, "max_position_embeddings": 131072,
}


def param_counts(s: ModelSpec):
    """Parameter counts per component (a tied LM head counts once)."""
    norm_mult = 2 if s.norm_bias else 1
    if s.gated_mlp:
        mlp, mlp_bias = 3 * s.hidden * s.intermediate, 0
    else:
        mlp = 2 * s.hidden * s.intermediate
        mlp_bias = (s.intermediate + s.hidden) if s.proj_bias else 0
    qkv = s.hidden * (s.q_dim + 2 * s.kv_dim)
    qkv_b = (s.q_dim + 2 * s.kv_dim) if s.qkv_bias else 0
    out = s.q_dim * s.hidden
    out_b = s.hidden if s.proj_bias else 0
    counts = {
        "attn_qkv": s.n_layers * (qkv + qkv_b),
        "attn_out": s.n_layers * (out + out_b),
        "mlp": s.n_layers * (mlp + mlp_bias),
        "norms": s.n_layers * 2 * norm_mult * s.hidden + norm_mult * s.hidden,
        "embedding": s.vocab * s.hidden,
        "pos_embedding": s.n_positions * s.hidden,
        "lm_head": 0 if s.tied_embedding else s.vocab * s.hidden,
    }
    counts["total"] = sum(counts.values())
    return counts


def _bias_params(s: ModelSpec):
    per_layer = 0
    if s.qkv_bias:
        per_layer += s.q_dim + 2 * s.kv_dim
    if s.proj_bias:
        per_layer += s.hidden
        if not s.gated_mlp:
            per_layer += s.intermediate + s.hidden
    return s.n_layers * per_layer


def _quant_bytes(numel, dtype, group_size=None, asymmetric=False):
    """Bytes of numel values at dtype plus fp16 scale (+ zero) per group."""
    body = numel * BITS[dtype] / 8
    if group_size is None or BITS[dtype] >= 16:
        return body
    return body + (numel / group_size) * 2 * (2 if asymmetric else 1)


def decode_bytes(s: ModelSpec, seq_len, weight_dtype="fp16", lm_head_dtype=None, kv_dtype="fp16",
                 group_size=128, asymmetric=False):
    """Bytes read by ONE batch-1 decode step: layer weights, LM head, KV cache, activations."""
    lm_head_dtype = lm_head_dtype or weight_dtype
    p = param_counts(s)
    biases = _bias_params(s)
    quantizable = p["attn_qkv"] + p["attn_out"] + p["mlp"] - biases
    small = p["norms"] + biases
    layer_weights = _quant_bytes(quantizable, weight_dtype, group_size, asymmetric)
    layer_weights += small * BITS["fp16"] / 8
    lm_head = _quant_bytes(s.vocab * s.hidden, lm_head_dtype, group_size, asymmetric)
    embed_lookup = s.hidden * BITS[lm_head_dtype] / 8
    kv_cache = 2 * s.n_layers * s.kv_dim * seq_len * BITS[kv_dtype] / 8
    if BITS[kv_dtype] < 16:
        kv_cache += 2 * s.n_layers * s.n_kv_heads * seq_len * 2
    h, i = s.hidden, s.intermediate
    qkv_out = s.q_dim + 2 * s.kv_dim
    mlp_act = (h + 2 * i + 2 * i + i + i + h) if s.gated_mlp else (h + i + i + i + h)
    per_layer_act = (2 * h + h + qkv_out + qkv_out + s.q_dim + h + 2 * h + 2 * h + mlp_act + 2 * h)
    activations = (s.n_layers * per_layer_act + 2 * h + s.vocab) * BITS["fp16"] / 8
    out = {"layer_weights": layer_weights, "lm_head": lm_head, "kv_cache": kv_cache,
           "activations": activations + embed_lookup}
    out["total"] = sum(out.values())
    return out


def predicted_latency_s(total_bytes, bandwidth_gb_s):
    """Bandwidth-bound floor: bytes / bandwidth."""
    return total_bytes / (bandwidth_gb_s * 1e9)


# ---- per-call accounting of the fused kernel --------------------------------

def packed_weight_bytes(n, k, bits, group_size, symmetric):
    """PackedWeight.nbytes for an [N, K] weight (group_size None = per-channel)."""
    g = 1 if group_size is None else k // group_size
    nb = n * k * bits // 8 + n * g * 2
    if not symmetric:
        nb += n * g * 2
    return nb


def gemv_call_bytes(n, k, bits, group_size, symmetric, m=1):
    """Algorithmic HBM bytes of one dequant-GEMV call: weights + metadata + x + y."""
    return packed_weight_bytes(n, k, bits, group_size, symmetric) + m * k * 2 + m * n * 2


def gemv_call_flops(n, k, m=1):
    return 2 * m * n * k


def roofline_us(nbytes, peak_bytes_s=MI355X_HBM_PEAK_BYTES_S):
    """Time floor in microseconds at the HBM peak."""
    return nbytes / peak_bytes_s * 1e6


def pct_of_peak(nbytes, seconds, peak_bytes_s=MI355X_HBM_PEAK_BYTES_S):
    return 100.0 * nbytes / seconds / peak_bytes_s
