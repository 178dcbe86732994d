"""Parity of the kernels around the scan and the attention core against the
oracle (f32) and the reference's rounding points (f16 activations)."""
import numpy as np
import pytest
import torch

import oracle

gpu = pytest.mark.gpu


@pytest.fixture(scope="module")
def clef():
    import clef_hip
    clef_hip.lib()
    return clef_hip


def _silu(x):
    return x / (1.0 + np.exp(-x))


@gpu
@pytest.mark.parametrize("W,T,hist", [(8192, 139, 0), (8192, 17, 3), (8192, 2, 1), (64, 33, 2),
                                      (16, 5, 0), (3, 4, 0)])
@pytest.mark.parametrize("dt_in,dt_out", [(torch.float32, torch.float32), (torch.float16, torch.float16),
                                          (torch.float16, torch.float32)])
def test_conv_silu_matches_oracle(clef, W, T, hist, dt_in, dt_out):
    """pointwise.rs:330-358 shapes; history rows precede the tokens (resume)."""
    gen = torch.Generator(device="cuda").manual_seed(W + T)
    x = torch.sin(torch.arange(T * W, device="cuda", dtype=torch.float32) * 0.073).reshape(T, W).to(dt_in)
    w = torch.cos(torch.arange(W * 4, device="cuda", dtype=torch.float32) * 0.027).reshape(W, 1, 4)
    h = torch.randn((hist, W), generator=gen, device="cuda") if hist else None
    y = clef.conv_silu(x, w, history=h, out_dtype=dt_out)
    full = np.concatenate([h.cpu().numpy(), x.float().cpu().numpy()]) if hist else x.float().cpu().numpy()
    exp = oracle.causal_conv(full, w.cpu().numpy())[hist:]
    exp = _silu(exp.astype(np.float64))
    got = y.float().cpu().numpy()
    if dt_out == torch.float32:
        np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-6)
    else:
        np.testing.assert_allclose(got, exp, rtol=2e-3, atol=1e-3)


@gpu
@pytest.mark.parametrize("rows,width", [(4096, 2048), (17, 1024), (139, 16), (3, 4096)])
@pytest.mark.parametrize("dt_out", [torch.float32, torch.float16])
def test_rms_matches_oracle(clef, rows, width, dt_out):
    """pointwise.rs:430-466 generator: x = sin(0.073 i), w = 0.7."""
    x = torch.sin(torch.arange(rows * width, device="cuda", dtype=torch.float32) * 0.073).reshape(rows, width)
    w = torch.full((width,), 0.7, device="cuda")
    y = clef.rms_norm(x, w, out_dtype=dt_out)
    exp = oracle.rms(x.cpu().numpy(), w.cpu().numpy())
    if dt_out == torch.float32:
        # the oracle sums sequentially, the kernel in a tree: compare both with the
        # exact (f64) result at the reference's 1e-6 bar (pointwise.rs:455) and
        # with each other within the f32 summation error of a 4096-wide row
        xd = x.double().cpu().numpy()
        exact = xd / np.sqrt((xd ** 2).mean(-1, keepdims=True) + 1e-6) * 0.7
        assert np.abs(y.cpu().numpy() - exact).max() <= 1e-6
        assert np.abs(y.cpu().numpy() - exp).max() <= 4e-6
    else:  # one half ulp at most after rounding
        np.testing.assert_allclose(y.float().cpu().numpy(), exp, rtol=2 ** -10, atol=2 ** -24)


@gpu
@pytest.mark.parametrize("T,Hv,width", [(300, 32, 128), (7, 3, 64)])
def test_gated_rms_silu_reads_rounded_scan_output(clef, T, Hv, width):
    """An f16 scan output gives exactly what rounding the f32 one inside the
    norm gives (the mixed block feeds the norm f16 o)."""
    gen = torch.Generator(device="cuda").manual_seed(T + 1)
    o = torch.randn((T, Hv, width), generator=gen, device="cuda")
    z = torch.randn((T, Hv * width), generator=gen, device="cuda").half()
    w = torch.randn((width,), generator=gen, device="cuda")
    assert torch.equal(clef.gated_rms_silu(o, z, w, out_dtype=torch.float16),
                       clef.gated_rms_silu(o.half(), z, w, out_dtype=torch.float16))


@gpu
@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
@pytest.mark.parametrize("T,Hv,width", [(300, 32, 128), (20, 2, 4), (7, 3, 64)])
def test_gated_rms_silu(clef, dt, T, Hv, width):
    gen = torch.Generator(device="cuda").manual_seed(T)
    o = torch.randn((T, Hv, width), generator=gen, device="cuda")
    z = torch.randn((T, Hv * width), generator=gen, device="cuda").to(dt)
    w = torch.randn((width,), generator=gen, device="cuda")
    y = clef.gated_rms_silu(o, z, w, out_dtype=dt)
    on = o.to(dt).float().cpu().numpy()
    n = oracle.rms(on.reshape(-1, width), w.cpu().numpy()).reshape(T, Hv * width)
    zf = z.float().cpu().numpy()
    if dt == torch.float16:
        n = n.astype(np.float16).astype(np.float32)
    exp = n * _silu(zf.astype(np.float64))
    tol = 1e-5 if dt == torch.float32 else 2e-3
    np.testing.assert_allclose(y.float().cpu().numpy(), exp, rtol=tol, atol=tol)


@gpu
@pytest.mark.parametrize("T,heads,d,offset", [(4096, 2, 256, 0), (1, 1, 64, 0), (65, 2, 128, 8), (4109, 2, 256, 512),
                                               (77, 3, 64, 5), (300, 2, 24, 0)])
@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_values_transposed_is_an_exact_transpose(clef, T, heads, d, offset, dt):
    """clef_values_transposed: y[h, e, offset + t] = x[t, h*d + e] exactly, the
    columns outside [offset, offset + T) untouched (the 16-byte f16 path for
    d % 64 == 0 and 8-aligned offsets, partial last tiles, and the element path)."""
    gen = torch.Generator(device="cuda").manual_seed(T + d)
    x = torch.randn((T, heads * d), generator=gen, device="cuda").to(dt)
    ld = ((offset + T + 63) // 64) * 64
    out = torch.full((heads, d, ld), 7.0, dtype=dt, device="cuda")
    clef.values_transposed(x, heads, d, out=out, dst_offset=offset)
    ref = torch.full((heads, d, ld), 7.0, dtype=dt, device="cuda")
    ref[:, :, offset:offset + T] = x.view(T, heads, d).permute(1, 2, 0)
    assert torch.equal(out, ref)


@gpu
@pytest.mark.parametrize("heads,kvh,qn,kn,d", [(16, 2, 300, 300, 256), (2, 1, 20, 20, 8), (4, 2, 17, 273, 64),
                                               (2, 1, 1, 256, 256), (8, 8, 130, 130, 128)])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_attention_gated_matches_oracle(clef, heads, kvh, qn, kn, d, dt):
    """ops.rs:62-148 tiled attention (lower-right causal mask with cached keys), gated."""
    gen = torch.Generator(device="cuda").manual_seed(qn * 7 + kn)
    q = torch.randn((heads, qn, d), generator=gen, device="cuda").to(dt)
    k = torch.randn((kvh, kn, d), generator=gen, device="cuda").to(dt)
    v = torch.randn((kvh, kn, d), generator=gen, device="cuda").to(dt)
    proj = torch.randn((qn, heads, 2 * d), generator=gen, device="cuda").to(dt)
    gate = proj[:, :, d:]
    vt = clef.values_transposed(v.permute(1, 0, 2).contiguous().reshape(kn, kvh * d), kvh, d)
    y = clef.attention_gated(q, k, vt, gate)
    att = oracle.attention(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(), True)
    att = att.transpose(1, 0, 2).reshape(qn, heads * d)
    g = gate.float().cpu().numpy().reshape(qn, heads * d)
    sig = 1.0 / (1.0 + np.exp(-g.astype(np.float64)))
    if dt == torch.float16:
        exp = att.astype(np.float16).astype(np.float64) * sig.astype(np.float16).astype(np.float64)
        np.testing.assert_allclose(y.float().cpu().numpy(), exp, rtol=1e-2, atol=5e-3)
    else:
        np.testing.assert_allclose(y.cpu().numpy(), att * sig, rtol=1e-4, atol=1e-5)


@gpu
@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
@pytest.mark.parametrize("heads,d,rot,pos0", [(4, 256, 64, 11), (5, 128, 64, 4000), (3, 64, 32, 0), (2, 96, 32, 5)])
def test_qk_norm_rotary_matches_oracle(clef, dt, heads, d, rot, pos0):
    """d = 64, 128, 256: one token per work-group, lanes of 1, 2, 4 features;
    d = 96: one wave per (token, head); pos0 = 4000 reaches large angles."""
    T = 37
    gen = torch.Generator(device="cuda").manual_seed(1)
    proj = torch.randn((T, heads, 2 * d), generator=gen, device="cuda").to(dt)
    w = 1.0 + 0.1 * torch.randn((d,), generator=gen, device="cuda")
    y = clef.qk_norm_rotary(proj, heads, d, w, rot, 1e7, pos0=pos0, head_stride=2 * d)
    q = proj[:, :, :d].float().cpu().numpy()
    n = oracle.rms(q.reshape(-1, d), w.cpu().numpy()).reshape(T, heads, d)
    if dt == torch.float16:
        n = n.astype(np.float16).astype(np.float32)
    exp = oracle.rotary(n, rot, 1e7, pos0=pos0).transpose(1, 0, 2)
    tol = 1e-5 if dt == torch.float32 else 2e-3
    np.testing.assert_allclose(y.float().cpu().numpy(), exp, rtol=tol, atol=tol)


@gpu
@pytest.mark.parametrize("heads,kvh,qn,kn", [(16, 2, 300, 300), (16, 2, 4096, 4096), (4, 2, 130, 642),
                                             (2, 1, 1, 256), (8, 8, 65, 65)])
def test_attention_with_query_norm_equals_norm_then_attention(clef, heads, kvh, qn, kn):
    """The query RMS norm + rotary (qwen.rs:459-468) inside the attention core
    equals clef_qk_norm_rotary followed by clef_attention_gated bit for bit,
    with the queries at positions kn - qn .. kn - 1 as in a resumed prefill;
    the rotary table equals the angles clef_qk_norm_rotary rotates by."""
    d, rot, theta, eps = 256, 64, 1e7, 1e-6
    gen = torch.Generator(device="cuda").manual_seed(qn + 3 * kn)
    proj = (2.0 * torch.randn((qn, heads, 2 * d), generator=gen, device="cuda")).half()
    x = proj.reshape(qn, heads * 2 * d)
    w = 1.0 + 0.1 * torch.randn((d,), generator=gen, device="cuda")
    k = torch.randn((kvh, kn, d), generator=gen, device="cuda").half()
    v = torch.randn((kvh, kn, d), generator=gen, device="cuda").half()
    vt = clef.values_transposed(v.permute(1, 0, 2).contiguous().reshape(kn, kvh * d), kvh, d)
    gate = proj[:, :, d:]
    pos0 = kn - qn
    q = clef.qk_norm_rotary(x, heads, d, w, rot, theta, pos0=pos0, head_stride=2 * d, eps=eps)
    ref = clef.attention_gated(q, k, vt, gate)
    tab = clef.rotary_table(qn, rot, theta, pos0=pos0)
    got = clef.attention_gated_qnorm(x, heads, w, eps, tab, k, vt, gate, 2 * d)
    assert torch.equal(got, ref)
    ang = (np.arange(pos0, pos0 + qn, dtype=np.float64)[:, None]
           * (theta ** (-np.arange(0, rot, 2, dtype=np.float64) / rot)).astype(np.float32)[None, :])
    t = tab.cpu().numpy()
    np.testing.assert_allclose(t[:, :, 0], np.cos(ang.astype(np.float32)), rtol=0, atol=2e-6)
    np.testing.assert_allclose(t[:, :, 1], np.sin(ang.astype(np.float32)), rtol=0, atol=2e-6)


@gpu
def test_attention_with_query_norm_rejects_other_shapes(clef):
    """d other than 256, or a misaligned head stride: an error before launch."""
    heads, kvh, qn, d = 2, 1, 8, 128
    x = torch.zeros((qn, heads * 2 * d), dtype=torch.float16, device="cuda")
    w = torch.ones((d,), device="cuda")
    k = torch.zeros((kvh, qn, d), dtype=torch.float16, device="cuda")
    vt = torch.zeros((kvh, d, 64), dtype=torch.float16, device="cuda")
    tab = clef.rotary_table(qn, 64, 1e7)
    with pytest.raises(clef.ClefError):
        clef.attention_gated_qnorm(x, heads, w, 1e-6, tab, k, vt, x.view(qn, heads, 2 * d)[:, :, d:], 2 * d)
    x2 = torch.zeros((qn, heads * 2 * 256 + 4), dtype=torch.float16, device="cuda")
    w2 = torch.ones((256,), device="cuda")
    k2 = torch.zeros((kvh, qn, 256), dtype=torch.float16, device="cuda")
    vt2 = torch.zeros((kvh, 256, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(clef.ClefError):  # head stride 516 halves: rows not 16-byte aligned
        clef.attention_gated_qnorm(x2, heads, w2, 1e-6, tab, k2, vt2, x2[:, :heads * 256].view(qn, heads, 256),
                                   516)


@gpu
def test_delta_gates_matches_reference_formula(clef):
    T, Hv = 333, 32
    gen = torch.Generator(device="cuda").manual_seed(2)
    ab = (torch.randn((T, 2 * Hv + 5), generator=gen, device="cuda") * 4).half()
    dt = torch.randn(Hv, generator=gen, device="cuda")
    alog = torch.randn(Hv, generator=gen, device="cuda")
    g, beta = clef.delta_gates(ab[:, :Hv], ab[:, Hv:2 * Hv], dt, alog)
    a = ab[:, :Hv].double().cpu() + dt.double().cpu()
    sp = a.clamp(min=0) + torch.log1p(torch.exp(-a.abs()))
    np.testing.assert_allclose(g.cpu().numpy(), (sp * -torch.exp(alog.double().cpu())).numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(beta.cpu().numpy(), torch.sigmoid(ab[:, Hv:2 * Hv].double().cpu()).numpy(),
                               rtol=1e-6, atol=1e-7)


@gpu
@pytest.mark.parametrize("T,K,Hv", [(4096, 2048, 32), (333, 256, 16), (1, 512, 64), (17, 2048, 32)])
def test_delta_gates_proj_matches_projection_then_gates(clef, T, K, Hv):
    """The fused a/b projections + gates equal the in-projection GEMM's a/b
    columns (f16) followed by the gates kernel: the two f32 accumulation
    orders may round a value to the neighbouring half, nothing more."""
    gen = torch.Generator(device="cuda").manual_seed(T + K)
    x = torch.randn((T, K), generator=gen, device="cuda").half()
    w_ab = (torch.randn((2 * Hv, K), generator=gen, device="cuda") * 0.05).half()
    dt = torch.randn(Hv, generator=gen, device="cuda")
    alog = torch.randn(Hv, generator=gen, device="cuda")
    g, beta = clef.delta_gates_proj(x, clef.delta_gates_pack(w_ab), Hv, dt, alog)
    ab = clef.gemm(x, w_ab)
    g0, beta0 = clef.delta_gates(ab[:, :Hv], ab[:, Hv:], dt, alog)
    for got, ref in ((g, g0), (beta, beta0)):
        assert (got == ref).float().mean().item() > 0.99
        np.testing.assert_allclose(got.cpu().numpy(), ref.cpu().numpy(), rtol=1e-2, atol=1e-3)


@gpu
@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
@pytest.mark.parametrize("hist", [0, 1, 3])
@pytest.mark.parametrize("W", [64, 12])
def test_conv_silu_varlen_matches_per_sequence_oracle(clef, dt, hist, W):
    """Ragged batch: each sequence is the conv of [shared history; its tokens]
    (qwen.rs:609-618 per request); sequences of 0, 1, 2 and 3 tokens sit at
    and inside the window's reach; W = 12 takes the any-layout kernel."""
    lens = [40, 0, 1, 2, 3, 17, 33, 5]
    T = sum(lens)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(11 + hist)
    x = torch.randn((T, W), generator=gen, device="cuda").to(dt)
    w = torch.randn((W, 1, 4), generator=gen, device="cuda") * 0.5
    h = torch.randn((hist, W), generator=gen, device="cuda") if hist else None
    y = clef.conv_silu_varlen(x, w, cu, history=h, out_dtype=dt)
    got = y.float().cpu().numpy()
    xf = x.float().cpu().numpy()
    for a, b in zip(cu[:-1].tolist(), cu[1:].tolist()):
        if a == b:
            continue
        full = np.concatenate([h.cpu().numpy(), xf[a:b]]) if hist else xf[a:b]
        exp = _silu(oracle.causal_conv(full, w.cpu().numpy())[hist:].astype(np.float64))
        if dt == torch.float32:
            np.testing.assert_allclose(got[a:b], exp, rtol=1e-5, atol=1e-6)
        else:
            np.testing.assert_allclose(got[a:b], exp, rtol=2e-3, atol=1e-3)


@gpu
@pytest.mark.parametrize("cu", [[0, 40, 0, 40, 0, 40], [-50, 10, 4, 30, 20, 40], [0, 5000, 6000],
                                [2 ** 31 - 1, -(2 ** 31), 7, 3]])
@pytest.mark.parametrize("W", [64, 12])
def test_conv_and_rotary_varlen_accept_malformed_tables(clef, cu, W):
    """Device offset tables the host cannot inspect (overlapping, negative,
    past T, extreme): the ragged conv and q/k rotary kernels clamp each
    sequence start into [0, t], so they run inside their buffers and give
    finite values; a valid table is unaffected (tests above)."""
    T, hist = 40, 3
    nseq = len(cu) - 1
    dcu = torch.tensor(cu, dtype=torch.int64).to(torch.int32).cuda()
    gen = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn((T, W), generator=gen, device="cuda")
    w = torch.randn((W, 1, 4), generator=gen, device="cuda") * 0.5
    h = torch.randn((nseq, hist, W), generator=gen, device="cuda")
    y = clef.conv_silu_varlen(x, w, dcu, history=h)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    proj = torch.randn((T, 2, 64), generator=gen, device="cuda")
    r = clef.qk_norm_rotary_varlen(proj, 2, 64, torch.ones(64, device="cuda"), 32, 1e7, dcu)
    torch.cuda.synchronize()
    assert torch.isfinite(r).all()


@gpu
def test_qk_norm_rotary_varlen_positions(clef):
    """Ragged batch: token t of sequence s rotates at pos0 + (t - cu[s]),
    i.e. each sequence equals the single-sequence kernel at the same pos0."""
    lens, heads, d, rot, pos0 = [5, 0, 12, 1], 2, 64, 32, 7
    T = sum(lens)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(3)
    proj = torch.randn((T, heads, d), generator=gen, device="cuda")
    w = 1.0 + 0.1 * torch.randn((d,), generator=gen, device="cuda")
    y = clef.qk_norm_rotary_varlen(proj, heads, d, w, rot, 1e7, cu, pos0=pos0)
    for a, b in zip(cu[:-1].tolist(), cu[1:].tolist()):
        if a == b:
            continue
        one = clef.qk_norm_rotary(proj[a:b].contiguous(), heads, d, w, rot, 1e7, pos0=pos0)
        torch.testing.assert_close(y[:, a:b], one, rtol=0, atol=0)


@gpu
@pytest.mark.parametrize("np_", [0, 64, 72])
@pytest.mark.parametrize("d", [64, 256])
def test_attention_varlen_matches_per_sequence_oracle(clef, np_, d):
    """Ragged batch with a shared prefix: each sequence equals causal attention
    over [prefix; own keys] (ops.rs:62-148, lower-right mask), gated; lengths
    cover single tokens, tile edges and several query tiles."""
    lens = [130, 1, 64, 300, 17, 128]
    heads, kvh = 8, 2
    T = sum(lens)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(np_ + d)
    dt = torch.float16
    q = torch.randn((heads, T, d), generator=gen, device="cuda").to(dt)
    k = torch.randn((kvh, T, d), generator=gen, device="cuda").to(dt)
    v = torch.randn((kvh, T, d), generator=gen, device="cuda").to(dt)
    proj = torch.randn((T, heads, 2 * d), generator=gen, device="cuda").to(dt)
    gate = proj[:, :, d:]
    vt = clef.values_transposed(v.permute(1, 0, 2).contiguous().reshape(T, kvh * d), kvh, d)
    pk = pvt = None
    if np_:
        pk = torch.randn((kvh, np_, d), generator=gen, device="cuda").to(dt)
        pv = torch.randn((kvh, np_, d), generator=gen, device="cuda").to(dt)
        pvt = clef.values_transposed(pv.permute(1, 0, 2).contiguous().reshape(np_, kvh * d), kvh, d)
    y = clef.attention_gated_varlen(q, k, vt, gate, cu, prefix_k=pk, prefix_vt=pvt).float().cpu().numpy()
    qf, kf, vf = (t.float().cpu().numpy() for t in (q, k, v))
    g = gate.float().cpu().numpy()
    for a, b in zip(cu[:-1].tolist(), cu[1:].tolist()):
        ks, vs = kf[:, a:b], vf[:, a:b]
        if np_:
            ks = np.concatenate([pk.float().cpu().numpy(), ks], axis=1)
            vs = np.concatenate([pv.float().cpu().numpy(), vs], axis=1)
        att = oracle.attention(qf[:, a:b], ks, vs, True).transpose(1, 0, 2).reshape(b - a, heads * d)
        sig = 1.0 / (1.0 + np.exp(-g[a:b].reshape(b - a, heads * d).astype(np.float64)))
        exp = att.astype(np.float16).astype(np.float64) * sig.astype(np.float16).astype(np.float64)
        np.testing.assert_allclose(y[a:b], exp, rtol=1e-2, atol=5e-3)
