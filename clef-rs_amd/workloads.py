"""Synthetic workloads of the hybrid-prefill path (seeded, generated on device).

Values come from torch's device generator seeded per workload, so a workload
is reproducible bit for bit on the same software stack; parity tests copy the
very same tensors to the host for the CPU oracle.
"""
from __future__ import annotations

import torch


def _gen(seed, device):
    return torch.Generator(device=device).manual_seed(seed)


def scan_inputs(seed, T, Hk, Hv, dk, dv, dtype=torch.float32, device="cuda"):
    """Scan workloads: q,k ~ N(0,1) then per-head L2-normalised; v ~ N(0,1);
    beta = sigmoid(N(0,1)); g = -softplus(N(0,1)).  Returns q, k, v, g, beta
    cast to `dtype` (the state and accumulation stay f32 inside the scan)."""
    gen = _gen(seed, device)
    q = torch.randn((T, Hk, dk), generator=gen, device=device)
    k = torch.randn((T, Hk, dk), generator=gen, device=device)
    v = torch.randn((T, Hv, dv), generator=gen, device=device)
    beta = torch.sigmoid(torch.randn((T, Hv), generator=gen, device=device))
    g = -torch.nn.functional.softplus(torch.randn((T, Hv), generator=gen, device=device))
    q = q / q.norm(dim=-1, keepdim=True)
    k = k / k.norm(dim=-1, keepdim=True)
    return [x.to(dtype) for x in (q, k, v, g, beta)]


# Scan shapes: small CPU-runnable case and the full layer.
SCAN_SMALL = dict(seed=0, T=256, Hk=4, Hv=4, dk=64, dv=64)
SCAN_LAYER = dict(seed=2, T=4096, Hk=16, Hv=32, dk=128, dv=128)


def gemm_inputs(seed, M, N, K, dtype=torch.float16, device="cuda"):
    """Projection GEMM workload: x ~ N(0,1) [M,K], W ~ N(0,0.02) [N,K]."""
    gen = _gen(seed, device)
    x = torch.randn((M, K), generator=gen, device=device)
    w = torch.randn((N, K), generator=gen, device=device) * 0.02
    return x.to(dtype), w.to(dtype)


# Projection shapes (M tokens, K hidden): fused in-proj, out-proj, SwiGLU gate/up.
GEMM_M, GEMM_K = 2048, 2048
GEMM_N = {"in_proj": 8192, "out_proj": 2048, "swiglu": 6144}


def scan_bytes(T, Hk, Hv, dk, dv, in_bytes, out_bytes, initial=False):
    """Algorithmic HBM bytes of one scan call: q,k read once per k-head, v, g,
    beta, the output and the final f32 state (plus an initial state)."""
    b = 2 * T * Hk * dk * in_bytes + T * Hv * dv * in_bytes + 2 * T * Hv * in_bytes
    b += T * Hv * dv * out_bytes + Hv * dk * dv * 4
    if initial:
        b += Hv * dk * dv * 4
    return b


def scan_flops(T, Hk, Hv, dk, dv, C=64):
    """Chunked-algorithm flops (secondary figure)."""
    n = T / C
    return n * (Hk * 4 * C * C * dk + Hv * (2 * C * C * dk + 4 * C * C * dv + 6 * C * dk * dv
                                             + (2.0 / 3.0) * C ** 3))


# ---------------------------------------------------------------------------
# Hybrid block stack: 3 DeltaNet layers then 1 gated GQA attention layer,
# hidden 2048, SwiGLU 6144, DeltaNet heads 16 (q/k) / 32 (v) x 128, conv k=4,
# attention 16 q / 2 kv heads x 256 with rotary on 64 dims; every weight
# ~ N(0, 0.02); token ids uniform in [0, 151936).  Names follow the
# reference's checkpoint naming (qwen.rs:193-310).
# ---------------------------------------------------------------------------
def block_config(layers=("linear_attention",) * 3 + ("full_attention",)):
    return {
        "hidden_size": 2048, "intermediate_size": 6144, "vocab_size": 151936,
        "num_attention_heads": 16, "num_key_value_heads": 2, "head_dim": 256,
        "rms_norm_eps": 1e-6, "layer_types": list(layers),
        "linear_num_key_heads": 16, "linear_num_value_heads": 32,
        "linear_key_head_dim": 128, "linear_value_head_dim": 128, "linear_conv_kernel_dim": 4,
        "rope_parameters": {"rope_theta": 10000000.0, "partial_rotary_factor": 0.25,
                            "mrope_section": [11, 11, 10]},
    }


def weight_shapes(c):
    """(name, shape) of every tensor of a backbone config, in a fixed order."""
    P = "model.language_model."
    H, I = c["hidden_size"], c["intermediate_size"]
    key = c["linear_num_key_heads"] * c["linear_key_head_dim"]
    Hv = c["linear_num_value_heads"]
    value = Hv * c["linear_value_head_dim"]
    heads, kvh, d = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
    out = [(P + "embed_tokens.weight", (c["vocab_size"], H)), (P + "norm.weight", (H,))]
    for i, kind in enumerate(c["layer_types"]):
        p = f"{P}layers.{i}."
        out += [(p + "input_layernorm.weight", (H,)), (p + "post_attention_layernorm.weight", (H,)),
                (p + "mlp.gate_proj.weight", (I, H)), (p + "mlp.up_proj.weight", (I, H)),
                (p + "mlp.down_proj.weight", (H, I))]
        if kind == "full_attention":
            a = p + "self_attn."
            out += [(a + "q_proj.weight", (2 * heads * d, H)), (a + "k_proj.weight", (kvh * d, H)),
                    (a + "v_proj.weight", (kvh * d, H)), (a + "o_proj.weight", (H, heads * d)),
                    (a + "q_norm.weight", (d,)), (a + "k_norm.weight", (d,))]
        else:
            a = p + "linear_attn."
            out += [(a + "in_proj_qkv.weight", (2 * key + value, H)), (a + "in_proj_z.weight", (value, H)),
                    (a + "in_proj_a.weight", (Hv, H)), (a + "in_proj_b.weight", (Hv, H)),
                    (a + "out_proj.weight", (H, value)),
                    (a + "conv1d.weight", (2 * key + value, 1, c["linear_conv_kernel_dim"])),
                    (a + "dt_bias", (Hv,)), (a + "A_log", (Hv,)), (a + "norm.weight", (c["linear_value_head_dim"],))]
    return out


def block_weights(config, seed=3, device="cuda", std=0.02, dtype=torch.float32):
    gen = _gen(seed, device)
    return {name: (torch.randn(shape, generator=gen, device=device) * std).to(dtype)
            for name, shape in weight_shapes(config)}


def block_ids(config, T, seed=3, device="cpu"):
    gen = torch.Generator(device=device).manual_seed(seed + 1000)
    return torch.randint(0, config["vocab_size"], (T,), generator=gen, device=device, dtype=torch.int32)


def block_head(config, seed=3, n_logits=3, device="cuda"):
    """Last-token pooled linear head: [n_logits, H] ~ N(0, 0.02)."""
    gen = _gen(seed + 2000, device)
    return torch.randn((n_logits, config["hidden_size"]), generator=gen, device=device) * 0.02


def block_flops_per_token(config, T):
    """Projection + attention-core flops per token of one prefill of T tokens."""
    c = config
    H, I = c["hidden_size"], c["intermediate_size"]
    key = c["linear_num_key_heads"] * c["linear_key_head_dim"]
    Hv = c["linear_num_value_heads"]
    value = Hv * c["linear_value_head_dim"]
    heads, kvh, d = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
    f = 0.0
    for kind in c["layer_types"]:
        f += 2 * 3 * H * I
        if kind == "full_attention":
            f += 2 * H * (2 * heads * d + 2 * kvh * d) + 2 * heads * d * H
            f += 4 * heads * d * (T + 1) / 2  # causal QK^T and PV, averaged over positions
        else:
            f += 2 * H * (2 * key + 2 * value + 2 * Hv) + 2 * value * H
    return f


def ragged_workload(config, seed=4, requests=32, lo=128, hi=4096, prefix=512):
    """Ragged batch: `requests` lengths uniform in [lo, hi], one shared prefix
    of `prefix` token ids and the packed request ids (numpy, seeded).
    Returns (prefix_ids, lens, packed_ids, cu_seqlens)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, requests)
    prefix_ids = rng.integers(0, config["vocab_size"], prefix)
    packed = rng.integers(0, config["vocab_size"], int(lens.sum()))
    cu = np.concatenate([[0], np.cumsum(lens)])
    return prefix_ids, lens, packed, cu
