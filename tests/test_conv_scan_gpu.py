"""The mixer's conv + SiLU followed by the scan, as the block runs them
(clef_conv_silu / clef_conv_silu_varlen, then clef_delta_scan /
clef_delta_scan_varlen; qwen.rs:603-618, 765-796, 826-882), against the
oracle's conv (history rows prepended, as qwen.rs:609-617) + SiLU +
recurrence, within the scan's bars: one sequence with history rows and a
captured state, and a ragged batch with and without a shared history."""
import numpy as np
import pytest
import torch

import oracle
from test_scan_gpu import _check

gpu = pytest.mark.gpu


@pytest.fixture(scope="module")
def clef():
    import clef_hip
    clef_hip.lib()
    return clef_hip


def _inputs(seed, T, Hk, Hv, d, dtype):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    W = 2 * Hk * d + Hv * d
    mixed = torch.randn((T, W + 64), generator=gen, device="cuda").to(dtype)  # + 64 columns as z would be
    conv_w = 0.5 * torch.randn((W, 4), generator=gen, device="cuda")
    g = -torch.nn.functional.softplus(torch.randn((T, Hv), generator=gen, device="cuda"))
    beta = torch.sigmoid(torch.randn((T, Hv), generator=gen, device="cuda"))
    hist = torch.randn((3, W), generator=gen, device="cuda")
    return mixed, conv_w, g, beta, hist, W


def _split(y, T, Hk, Hv, d):
    q = y[:, :Hk * d].view(T, Hk, d)
    k = y[:, Hk * d:2 * Hk * d].view(T, Hk, d)
    v = y[:, 2 * Hk * d:].view(T, Hv, d)
    return q, k, v


def _oracle_conv_scan(x, conv_w, hist, g, beta, Hk, Hv, d, initial, capture=0):
    """qwen.rs:603-618 then 826-882 on the CPU: conv over [history; x] with
    taps oldest -> newest, the history rows' outputs dropped, SiLU, split,
    recurrence."""
    W = x.shape[1]
    xin = np.concatenate([hist, x]) if hist is not None and len(hist) else x
    y = oracle.causal_conv(xin, conv_w)[len(xin) - len(x):]
    y = (y / (1.0 + np.exp(-y.astype(np.float64)))).astype(np.float32)
    T = x.shape[0]
    q = y[:, :Hk * d].reshape(T, Hk, d)
    k = y[:, Hk * d:2 * Hk * d].reshape(T, Hk, d)
    v = y[:, 2 * Hk * d:W].reshape(T, Hv, d)
    return oracle.delta_scan(q, k, v, g, beta, initial=initial, capture=capture)


@gpu
@pytest.mark.parametrize("precision", ["strict", "mixed"])
@pytest.mark.parametrize("T,Hk,Hv,d,hist_rows,capture", [(300, 2, 4, 64, 3, 128), (200, 2, 4, 64, 1, 77),
                                                         (65, 1, 2, 32, 2, 65), (3, 1, 1, 8, 3, 2),
                                                         (1024, 4, 8, 128, 3, 0)])
def test_conv_then_scan_matches_oracle(clef, precision, T, Hk, Hv, d, hist_rows, capture):
    dt = torch.float32 if precision == "strict" else torch.float16
    mixed, conv_w, g, beta, hist, W = _inputs(T + 7 * d, T, Hk, Hv, d, dt)
    history = hist[3 - hist_rows:].contiguous() if hist_rows else None
    init = 0.1 * torch.randn((Hv, d, d), generator=torch.Generator(device="cuda").manual_seed(3), device="cuda")
    scan = clef.DeltaScan(d, d, precision)
    y = clef.conv_silu(mixed[:, :W], conv_w, history=history, out_dtype=dt)
    q, k, v = _split(y, T, Hk, Hv, d)
    out, cap, fin = scan.prefill(q, k, v, g, beta, initial=init, capture=capture)
    x = mixed[:, :W].float().cpu().numpy()
    h = history.cpu().numpy() if history is not None else None
    eo, ec, ef = _oracle_conv_scan(x, conv_w.cpu().numpy(), h, g.cpu().numpy(), beta.cpu().numpy(), Hk, Hv, d,
                                   init.cpu().numpy(), capture)
    _check(out.cpu().numpy(), eo, precision)
    _check(fin.cpu().numpy(), ef, precision)
    if capture:
        _check(cap.cpu().numpy(), ec, precision)


@gpu
@pytest.mark.parametrize("precision", ["strict", "mixed"])
@pytest.mark.parametrize("with_history", [False, True])
def test_conv_then_scan_ragged_batch_matches_oracle(clef, precision, with_history):
    """Each sequence of the ragged batch equals the oracle's conv over its own
    rows (after the shared history rows, or zeros) and its recurrence from the
    shared initial state."""
    lens = [200, 0, 1, 63, 64, 65, 130, 7]
    Hk, Hv, d = 2, 4, 64
    T = sum(lens)
    dt = torch.float32 if precision == "strict" else torch.float16
    mixed, conv_w, g, beta, hist, W = _inputs(12, T, Hk, Hv, d, dt)
    history = hist if with_history else None
    cuh = np.concatenate([[0], np.cumsum(lens)])
    cu = torch.tensor(cuh, dtype=torch.int32, device="cuda")
    init = 0.1 * torch.randn((Hv, d, d), generator=torch.Generator(device="cuda").manual_seed(4), device="cuda")
    scan = clef.DeltaScan(d, d, precision)
    y = clef.conv_silu_varlen(mixed[:, :W], conv_w, cu, history=history, out_dtype=dt)
    q, k, v = _split(y, T, Hk, Hv, d)
    out, fin = scan.prefill_varlen(q, k, v, g, beta, cu, initial=init)
    x = mixed[:, :W].float().cpu().numpy()
    h = history.cpu().numpy() if history is not None else None
    o_all, f_all = out.cpu().numpy(), fin.cpu().numpy()
    gn, bn, wn, ini = g.cpu().numpy(), beta.cpu().numpy(), conv_w.cpu().numpy(), init.cpu().numpy()
    for s, (a, b) in enumerate(zip(cuh[:-1], cuh[1:])):
        if a == b:
            np.testing.assert_array_equal(f_all[s], ini)
            continue
        eo, _, ef = _oracle_conv_scan(x[a:b], wn, h, gn[a:b], bn[a:b], Hk, Hv, d, ini)
        _check(o_all[a:b], eo, precision)
        _check(f_all[s], ef, precision)
