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
