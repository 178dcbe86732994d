"""Parity of the gfx950 chunked DeltaNet scan against the CPU oracle.

Bars: strict f32 profile rtol 1e-4 / atol 1e-5 against the CPU
F32 recurrence (qwen.rs:826-882); mixed f16-MFMA profile rtol 2e-2 with an
absolute floor of 1e-2 * RMS(expected) (the f16 operands perturb every
output by a fraction of the outputs' typical size, so elements near zero
need a floor).  Capture/resume at chunk-aligned boundaries must be
bit-exact (metal.rs:819-868 contract).  Achieved errors are appended to the
JSON file named by CLEF_PARITY_LOG.
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle

gpu = pytest.mark.gpu
STRICT_RTOL, STRICT_ATOL = 1e-4, 1e-5
MIXED_RTOL = 2e-2


def _close(actual, expected, rtol, atol):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert np.isfinite(actual).all()
    err = np.abs(actual - expected)
    bad = err > atol + rtol * np.abs(expected)
    assert not bad.any(), (f"{bad.sum()} of {bad.size} out of tolerance; max err {err.max():.3e}"
                           f" at {np.unravel_index(err.argmax(), err.shape)}")


def _record(name, actual, expected):
    path = os.environ.get("CLEF_PARITY_LOG")
    if path:
        a, e = np.asarray(actual, np.float64), np.asarray(expected, np.float64)
        err = np.abs(a - e)
        rms = float(np.sqrt(np.mean(e * e)))
        with open(path, "a") as f:
            f.write(json.dumps({"test": name, "max_abs": float(err.max()),
                                "max_abs_over_rms": float(err.max() / max(rms, 1e-30)),
                                "frac_outside_rtol_2e-2": float((err > 2e-2 * np.abs(e)).mean())}) + "\n")


def _check(actual, expected, precision, name=None):
    if name:
        _record(name, actual, expected)
    if precision == "strict":
        _close(actual, expected, STRICT_RTOL, STRICT_ATOL)
    else:
        e = np.asarray(expected, np.float64)
        _close(actual, expected, MIXED_RTOL, 1e-2 * np.sqrt(np.mean(e * e)))


def case_inputs(seed, T, Hk, Hv, dk, dv, dtype=torch.float32, device="cuda"):
    import workloads
    return workloads.scan_inputs(seed, T, Hk, Hv, dk, dv, dtype=dtype, device=device)


def _np(*ts):
    return [t.float().cpu().numpy() for t in ts]


@pytest.fixture(scope="module")
def clef():
    import clef_hip
    clef_hip.lib()
    return clef_hip


@gpu
@pytest.mark.parametrize("precision", ["strict", "mixed"])
def test_scan_small_config_seed0(clef, precision):
    """B=1, T=256, H=4, dk=dv=64, chunk 64, f32 inputs, zero initial state."""
    q, k, v, g, beta = case_inputs(0, 256, 4, 4, 64, 64)
    out, _, final = clef.DeltaScan(64, 64, precision).prefill(q, k, v, g, beta)
    eo, _, ef = oracle.delta_scan(*_np(q, k, v, g, beta))
    _check(out.cpu().numpy(), eo, precision, f"scan T=256 H=4 64/64 {precision}: out")
    _check(final.cpu().numpy(), ef, precision, f"scan T=256 H=4 64/64 {precision}: final state")


@gpu
@pytest.mark.parametrize("T,H,dk,dv", [(1, 1, 1, 1), (33, 2, 4, 5), (33, 2, 32, 13),
                                       (257, 2, 64, 13), (257, 2, 128, 13), (17, 2, 128, 128)])
def test_scan_reference_tail_shapes(clef, T, H, dk, dv):
    """metal.rs:741-815 generator and shapes (segment and column tails)."""
    i = torch.arange(T * H * dk, dtype=torch.float32)
    q = torch.sin(i * 0.017).reshape(T, H, dk)
    k = q * 0.7 + 0.1
    v = torch.cos(torch.arange(T * H * dv, dtype=torch.float32) * 0.031).reshape(T, H, dv)
    g = torch.full((T, H), -0.03)
    beta = torch.full((T, H), 0.65)
    eo, _, ef = oracle.delta_scan(*_np(q, k, v, g, beta))
    out, _, final = clef.DeltaScan(dk, dv).prefill(*(x.cuda() for x in (q, k, v, g, beta)))
    _check(out.cpu().numpy(), eo, "strict")
    _check(final.cpu().numpy(), ef, "strict")


@gpu
@pytest.mark.parametrize("decay", [-0.03, -1000.0])
@pytest.mark.parametrize("T,H,dk,dv", [(1, 2, 4, 13), (31, 2, 32, 17), (32, 1, 128, 128),
                                       (33, 2, 64, 3), (139, 2, 128, 13), (512, 2, 128, 17),
                                       (1024, 1, 128, 32)])
def test_scan_chunk_candidate_shapes(clef, T, H, dk, dv, decay):
    """chunk.rs:177-230 shapes and generators, including decay -1000 (underflow)."""
    q = (torch.sin(torch.arange(T * H * dk, dtype=torch.float32) * 0.071) * 0.02).reshape(T, H, dk)
    k = torch.cos(torch.arange(T * H * dk, dtype=torch.float32) * 0.037).reshape(T, H, dk)
    v = torch.sin(torch.arange(T * H * dv, dtype=torch.float32) * 0.033).reshape(T, H, dv)
    g = torch.full((T, H), decay)
    beta = torch.full((T, H), 0.65)
    eo, _, ef = oracle.delta_scan(*_np(q, k, v, g, beta))
    for precision in ("strict", "mixed"):
        out, _, final = clef.DeltaScan(dk, dv, precision).prefill(*(x.cuda() for x in (q, k, v, g, beta)))
        _check(out.cpu().numpy(), eo, precision)
        _check(final.cpu().numpy(), ef, precision)


@gpu
@pytest.mark.parametrize("precision", ["strict", "mixed"])
def test_scan_gqa_initial_state_and_f16_io(clef, precision):
    T, Hk, Hv, dk, dv = 200, 2, 6, 64, 48
    q, k, v, g, beta = case_inputs(11, T, Hk, Hv, dk, dv, dtype=torch.float16)
    init = torch.randn((Hv, dk, dv), device="cuda") * 0.1
    out, _, final = clef.DeltaScan(dk, dv, precision).prefill(q, k, v, g, beta, initial=init,
                                                              out_dtype=torch.float16)
    eo, _, ef = oracle.delta_scan(*_np(q, k, v, g, beta), initial=init.cpu().numpy())
    if precision == "strict":  # f16 output rounding dominates: compare at half precision
        _close(out.float().cpu().numpy(), eo, 1e-3, 1e-4)
        _check(final.cpu().numpy(), ef, "strict")
    else:
        _check(out.float().cpu().numpy(), eo, precision)
        _check(final.cpu().numpy(), ef, precision)


@gpu
@pytest.mark.parametrize("precision,dtype,dk", [("mixed", torch.float16, 100), ("mixed", torch.float32, 100),
                                                ("strict", torch.float32, 48), ("strict", torch.float32, 20)])
def test_scan_key_rows_loaded_element_wise_over_many_chunks(clef, precision, dtype, dk):
    """dk below the padded key width: the carry loads the raw key rows element
    by element instead of by DMA.  Eleven chunks, so the ring wraps, and with
    f16 keys under f16 products or f32 under f32 the recurrence reads each
    chunk's keys one chunk early (written two chunks ahead by the loader)."""
    T, Hk, Hv, dv = 700, 2, 4, 32
    q, k, v, g, beta = case_inputs(23, T, Hk, Hv, dk, dv, dtype=dtype)
    out, _, final = clef.DeltaScan(dk, dv, precision).prefill(q, k, v, g, beta)
    eo, _, ef = oracle.delta_scan(*_np(q, k, v, g, beta))
    _check(out.cpu().numpy(), eo, precision)
    _check(final.cpu().numpy(), ef, precision)


@gpu
def test_scan_strided_views_of_packed_projection(clef):
    """q,k,v as views into one [T, 2*Hk*dk + Hv*dv] row (the conv output layout)."""
    T, Hk, Hv, dk, dv = 130, 2, 4, 64, 64
    gen = torch.Generator(device="cuda").manual_seed(3)
    W = 2 * Hk * dk + Hv * dv
    mixed = torch.randn((T, W), generator=gen, device="cuda")
    q = mixed[:, :Hk * dk].view(T, Hk, dk)
    k = mixed[:, Hk * dk:2 * Hk * dk].view(T, Hk, dk)
    v = mixed[:, 2 * Hk * dk:].view(T, Hv, dv)
    gb = torch.randn((T, 2 * Hv), generator=gen, device="cuda")
    g = -torch.nn.functional.softplus(gb[:, :Hv])
    beta = torch.sigmoid(gb[:, Hv:])
    out, _, final = clef.DeltaScan(dk, dv).prefill(q, k, v, g, beta)
    eo, _, ef = oracle.delta_scan(*_np(q, k, v, g, beta))
    _check(out.cpu().numpy(), eo, "strict")
    _check(final.cpu().numpy(), ef, "strict")


@gpu
@pytest.mark.parametrize("precision", ["strict", "mixed"])
def test_scan_capture_and_resume(clef, precision):
    T, H, dk, dv = 257, 2, 128, 128
    q, k, v, g, beta = case_inputs(5, T, H, H, dk, dv)
    scan = clef.DeltaScan(dk, dv, precision)
    full, _, final = scan.prefill(q, k, v, g, beta)
    for boundary in (1, 16, 64, 128, 256):
        out, cap, _ = scan.prefill(q, k, v, g, beta, capture=boundary)
        assert torch.equal(out, full)  # capturing never changes the outputs
        _, ecap, _ = oracle.delta_scan(*_np(q, k, v, g, beta), capture=boundary)
        _check(cap.cpu().numpy(), ecap, precision)
        tail = [x[boundary:].contiguous() for x in (q, k, v, g, beta)]
        rout, _, rfin = scan.prefill(*tail, initial=cap)
        if boundary % 64 == 0:  # chunk-aligned boundary: bit-exact resume
            assert torch.equal(rout, full[boundary:])
            assert torch.equal(rfin, final)
        else:
            eo, _, ef = oracle.delta_scan(*(x.cpu().numpy() for x in tail),
                                          initial=cap.cpu().numpy())
            _check(rout.cpu().numpy(), eo, precision)
            _check(rfin.cpu().numpy(), ef, precision)


@gpu
@pytest.mark.parametrize("precision", ["strict", "mixed"])
def test_scan_full_layer_config(clef, precision):
    """T=4096, Hk=16, Hv=32, dk=dv=128, f16 q/k/v/g/beta, f32 state and output."""
    q, k, v, g, beta = case_inputs(2, 4096, 16, 32, 128, 128, dtype=torch.float16)
    out, _, final = clef.DeltaScan(128, 128, precision).prefill(q, k, v, g, beta)
    eo, _, ef = oracle.delta_scan(*_np(q, k, v, g, beta))
    _check(out.cpu().numpy(), eo, precision, f"scan T=4096 16/32 128/128 {precision}: out")
    _check(final.cpu().numpy(), ef, precision, f"scan T=4096 16/32 128/128 {precision}: final state")


@gpu
def test_scan_is_deterministic(clef):
    q, k, v, g, beta = case_inputs(9, 1000, 4, 8, 128, 128, dtype=torch.float16)
    scan = clef.DeltaScan(128, 128, "mixed")
    a = scan.prefill(q, k, v, g, beta)[0].clone()
    b = scan.prefill(q, k, v, g, beta)[0]
    assert torch.equal(a, b)


@gpu
@pytest.mark.parametrize("precision", ["strict", "mixed"])
@pytest.mark.parametrize("shared", [True, False])
def test_scan_varlen_matches_per_sequence_oracle(clef, precision, shared):
    """Ragged batch (cu_seqlens): every sequence equals the reference recurrence
    (qwen.rs:826-882) run alone from its own initial state; an empty sequence
    hands its initial state through; sequences of 1, 63, 64, 65 tokens cover
    the partial-chunk edges."""
    lens = [200, 0, 1, 63, 64, 65, 130, 7]
    Hk, Hv, dk, dv = 2, 4, 64, 48
    T = sum(lens)
    dt = torch.float32 if precision == "strict" else torch.float16
    q, k, v, g, beta = case_inputs(5, T, Hk, Hv, dk, dv, dtype=dt)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(9)
    nseq = len(lens)
    shape = (Hv, dk, dv) if shared else (nseq, Hv, dk, dv)
    init = 0.1 * torch.randn(shape, generator=gen, device="cuda")
    out, final = clef.DeltaScan(dk, dv, precision).prefill_varlen(q, k, v, g, beta, cu, initial=init)
    qn, kn, vn, gn, bn = _np(q, k, v, g, beta)
    o_all, f_all = out.cpu().numpy(), final.cpu().numpy()
    ini = init.cpu().numpy()
    for s, (a, b) in enumerate(zip(cu[:-1].tolist(), cu[1:].tolist())):
        s0 = ini if shared else ini[s]
        if b == a:
            np.testing.assert_array_equal(f_all[s], s0)
            continue
        eo, _, ef = oracle.delta_scan(qn[a:b], kn[a:b], vn[a:b], gn[a:b], bn[a:b], initial=s0)
        _check(o_all[a:b], eo, precision)
        _check(f_all[s], ef, precision)
