"""Pins the CPU oracle before it is trusted as the parity checker.

Each check is chosen so that a plausible mistake (a dropped term, a wrong
sign, a transposed operand, a wrong head mapping) fails it:
  * the reference's golden backbone fixture (whole hybrid stack),
  * the reference's prefix capture/resume contract (mod.rs:113-171),
  * f64 brute force and the independent chunkwise f64 algebra,
  * closed forms of the gated delta rule,
  * the reference's own deterministic input generators (metal.rs:755-771,
    chunk.rs:191-219), including the g = -1000 underflow case.
"""
import json

import numpy as np
import pytest

import oracle

TOL_ABS, TOL_REL = 1e-5, 1e-4  # crates/core/src/models/mod.rs:75-86


def assert_close(actual, expected, atol=TOL_ABS, rtol=TOL_REL):
    actual, expected = np.asarray(actual), np.asarray(expected)
    assert actual.shape == expected.shape
    assert np.isfinite(actual).all()
    err = np.abs(actual - expected)
    bad = err > atol + rtol * np.abs(expected)
    assert not bad.any(), f"max err {err.max()} at {np.unravel_index(err.argmax(), err.shape)}"


@pytest.fixture(scope="module")
def fixture_backbone(golden_dir):
    from safetensors.numpy import load_file
    cfg = json.loads((golden_dir / "backbone-config.json").read_text())
    w = load_file(str(golden_dir / "backbone.safetensors"))
    exp = load_file(str(golden_dir / "backbone-output.safetensors"))["hidden"]
    return cfg, w, exp


def test_backbone_matches_reference_golden_hidden_states(fixture_backbone):
    cfg, w, exp = fixture_backbone
    hidden, _ = oracle.Backbone(cfg, w).prefill(np.arange(20))
    assert_close(hidden, exp)


def test_backbone_golden_detects_planted_mistakes(fixture_backbone):
    """The fixture is sensitive: perturbing one weight of each sub-block fails it.

    (Its decay path is only weakly observable in layers 0 and 2, whose decays
    are near zero or saturated; the f64 and closed-form checks below pin it.)"""
    cfg, w, exp = fixture_backbone
    for name in ("model.language_model.layers.1.linear_attn.A_log",
                 "model.language_model.layers.1.linear_attn.in_proj_b.weight",
                 "model.language_model.layers.1.linear_attn.conv1d.weight",
                 "model.language_model.layers.2.linear_attn.norm.weight",
                 "model.language_model.layers.3.self_attn.k_norm.weight",
                 "model.language_model.layers.3.mlp.down_proj.weight"):
        w2 = dict(w)
        w2[name] = w[name].copy()
        w2[name].flat[0] += 0.05
        hidden, _ = oracle.Backbone(cfg, w2).prefill(np.arange(20))
        err = np.abs(hidden - exp)
        assert (err > TOL_ABS + TOL_REL * np.abs(exp)).any(), name


def test_backbone_mixed_profile_stays_near_f32(fixture_backbone):
    cfg, w, exp = fixture_backbone
    hidden, _ = oracle.Backbone(cfg, w, mixed_f16=True).prefill(np.arange(20))
    assert np.abs(hidden - exp).max() < 2e-2 * np.abs(exp).max()


def test_backbone_prefix_capture_and_resume(fixture_backbone):
    """mod.rs:113-171: capture at a boundary, resume, changed suffix."""
    cfg, w, _ = fixture_backbone
    b = oracle.Backbone(cfg, w)
    ids = np.arange(20)
    expected, _ = b.prefill(ids)
    for boundary in (1, 2, 3, 8, 19):
        captured, state = b.prefill(ids, capture=boundary)
        assert_close(captured, expected)
        assert state["history_rows"][0] == min(boundary, 3)
        with pytest.raises(ValueError):
            b.prefill(ids[boundary:], initial=state, capture=1)
        resumed, _ = b.prefill(ids[boundary:], initial=state)
        assert_close(resumed, expected)
        changed = ids.copy()
        changed[boundary:] += 20
        resumed, _ = b.prefill(changed[boundary:], initial=state)
        assert_close(resumed, b.prefill(changed)[0])
        again, _ = b.prefill(ids[boundary:], initial=state)  # state is not mutated
        assert_close(again, expected)
    with pytest.raises(ValueError):
        b.prefill(ids, capture=20)
    with pytest.raises(ValueError):
        b.prefill(np.array([64]))


def _rand_inputs(rng, T, H, dk, dv, decay_scale=1.0):
    q = rng.standard_normal((T, H, dk))
    k = rng.standard_normal((T, H, dk))
    v = rng.standard_normal((T, H, dv))
    g = -np.log1p(np.exp(rng.standard_normal((T, H)))) * decay_scale
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((T, H))))
    return q, k, v, g, beta


@pytest.mark.parametrize("T,H,dk,dv,chunk", [(1, 1, 4, 4, 64), (7, 2, 8, 5, 4), (65, 2, 16, 8, 64),
                                             (130, 3, 32, 16, 64), (100, 1, 8, 8, 32)])
def test_chunked_f64_equals_per_token_f64(T, H, dk, dv, chunk):
    rng = np.random.default_rng(T * 7 + dk)
    q, k, v, g, beta = _rand_inputs(rng, T, H, dk, dv)
    init = rng.standard_normal((H, dk, dv)) * 0.3
    o1, s1 = oracle.delta_recurrence_f64(q, k, v, g, beta, init)
    o2, s2 = oracle.delta_chunked_f64(q, k, v, g, beta, chunk, init)
    np.testing.assert_allclose(o2, o1, rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(s2, s1, rtol=1e-10, atol=1e-11)


def test_chunked_f64_with_underflowing_decay():
    rng = np.random.default_rng(5)
    q, k, v, g, beta = _rand_inputs(rng, 70, 2, 8, 4)
    g[:] = -1000.0
    o1, s1 = oracle.delta_recurrence_f64(q, k, v, g, beta)
    o2, s2 = oracle.delta_chunked_f64(q, k, v, g, beta, 64)
    np.testing.assert_allclose(o2, o1, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(s2, s1, rtol=1e-10, atol=1e-12)


def _l2(x):
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-6)


def test_closed_form_single_token():
    rng = np.random.default_rng(1)
    q, k, v, g, beta = _rand_inputs(rng, 1, 3, 16, 8)
    out, _, final = oracle.delta_recurrence(q, k, v, g, beta)
    qn = _l2(q) / 4.0
    kn = _l2(k)
    expect = beta[0][:, None] * (qn[0] * kn[0]).sum(-1)[:, None] * v[0]
    np.testing.assert_allclose(out[0], expect, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(final, kn[0][:, :, None] * (beta[0][:, None] * v[0])[:, None, :],
                               rtol=1e-5, atol=1e-6)


def test_closed_form_zero_beta_keeps_decayed_state():
    rng = np.random.default_rng(2)
    q, k, v, g, beta = _rand_inputs(rng, 9, 2, 8, 6)
    beta[:] = 0.0
    init = rng.standard_normal((2, 8, 6)).astype(np.float32)
    out, _, final = oracle.delta_recurrence(q, k, v, g, beta, initial=init)
    qn = _l2(q) / np.sqrt(8.0)
    gam = np.cumsum(g, axis=0)
    expect = np.exp(gam)[:, :, None] * np.einsum("thk,hkv->thv", qn, init)
    np.testing.assert_allclose(out, expect, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(final, np.exp(gam[-1])[:, None, None] * init, rtol=1e-5, atol=1e-6)


def test_closed_form_full_decay_makes_tokens_independent():
    rng = np.random.default_rng(3)
    q, k, v, g, beta = _rand_inputs(rng, 12, 2, 8, 5)
    g[:] = -1000.0  # chunk.rs:213
    out, _, _ = oracle.delta_recurrence(q, k, v, g, beta)
    qn = _l2(q) / np.sqrt(8.0)
    kn = _l2(k)
    expect = beta[:, :, None] * (qn * kn).sum(-1)[:, :, None] * v
    np.testing.assert_allclose(out, expect, rtol=1e-5, atol=1e-6)


def test_closed_form_orthonormal_keys_write_exactly():
    rng = np.random.default_rng(4)
    T, dk, dv = 6, 8, 4
    basis, _ = np.linalg.qr(rng.standard_normal((dk, dk)))
    k = basis[:, :T].T.reshape(T, 1, dk)
    q = rng.standard_normal((T, 1, dk))
    v = rng.standard_normal((T, 1, dv))
    g = np.zeros((T, 1))
    beta = np.ones((T, 1))
    _, _, final = oracle.delta_recurrence(q, k, v, g, beta)
    recalled = np.einsum("kv,tk->tv", final[0], _l2(k[:, 0]))
    np.testing.assert_allclose(recalled, v[:, 0], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("T,H,dk,dv", [(1, 1, 1, 1), (33, 2, 4, 5), (33, 2, 32, 13),
                                       (257, 2, 64, 13), (257, 2, 128, 13), (17, 2, 128, 128)])
def test_reference_generator_f32_within_1e5_of_f64(T, H, dk, dv):
    """metal.rs:741-815 inputs and tolerance (1e-5 abs)."""
    i = np.arange(T * H * dk, dtype=np.float32)
    q = np.sin(i * np.float32(0.017)).reshape(T, H, dk).astype(np.float32)
    k = (q * np.float32(0.7) + np.float32(0.1)).astype(np.float32)
    v = np.cos(np.arange(T * H * dv, dtype=np.float32) * np.float32(0.031)).reshape(T, H, dv)
    g = np.full((T, H), -0.03, np.float32)
    beta = np.full((T, H), 0.65, np.float32)
    out, _, _ = oracle.delta_recurrence(q, k, v, g, beta)
    ref, _ = oracle.delta_recurrence_f64(q, k, v, g.astype(np.float64), beta.astype(np.float64))
    assert np.abs(out - ref).max() < 1e-5


def test_split_and_resume_is_bit_exact():
    """metal.rs:819-868 contract, on the oracle itself."""
    rng = np.random.default_rng(6)
    q, k, v, g, beta = (x.astype(np.float32) for x in _rand_inputs(rng, 257, 2, 16, 8))
    full, _, final = oracle.delta_recurrence(q, k, v, g, beta)
    for boundary in (1, 16, 256):
        out, cap, _ = oracle.delta_recurrence(q, k, v, g, beta, capture=boundary)
        assert np.array_equal(out, full)
        tail, _, fin2 = oracle.delta_recurrence(q[boundary:], k[boundary:], v[boundary:],
                                                g[boundary:], beta[boundary:], initial=cap)
        assert np.array_equal(tail, full[boundary:])
        assert np.array_equal(fin2, final)


def test_gqa_scan_uses_repeat_interleave():
    rng = np.random.default_rng(7)
    T, Hk, Hv, dk, dv = 20, 2, 4, 8, 8
    q = rng.standard_normal((T, Hk, dk)).astype(np.float32)
    k = rng.standard_normal((T, Hk, dk)).astype(np.float32)
    v = rng.standard_normal((T, Hv, dv)).astype(np.float32)
    g = -np.abs(rng.standard_normal((T, Hv))).astype(np.float32)
    beta = rng.random((T, Hv)).astype(np.float32)
    out, _, final = oracle.delta_scan(q, k, v, g, beta)
    rep = np.arange(Hv) // (Hv // Hk)  # qwen.rs:727-729
    out2, _, final2 = oracle.delta_recurrence(q[:, rep], k[:, rep], v, g, beta)
    assert np.array_equal(out, out2) and np.array_equal(final, final2)
    tiled = np.arange(Hv) % Hk
    out3, _, _ = oracle.delta_recurrence(q[:, tiled], k[:, tiled], v, g, beta)
    assert not np.allclose(out, out3)


def test_pointwise_pieces_against_numpy():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((17, 24)).astype(np.float32)
    w = rng.standard_normal((24, 4)).astype(np.float32)
    y = oracle.causal_conv(x, w)
    xp = np.concatenate([np.zeros((3, 24), np.float32), x])
    expect = sum(xp[3 - d:3 - d + 17] * w[:, 3 - d] for d in range(4))
    np.testing.assert_allclose(y, expect, rtol=1e-6, atol=1e-6)
    wn = rng.standard_normal(24).astype(np.float32)
    r = oracle.rms(x, wn)
    xe = x.astype(np.float64)
    np.testing.assert_allclose(r, xe / np.sqrt((xe ** 2).mean(-1, keepdims=True) + 1e-6) * wn,
                               rtol=1e-5, atol=1e-6)
    a = rng.standard_normal((33, 100)).astype(np.float32)
    b = rng.standard_normal((45, 100)).astype(np.float32)
    np.testing.assert_allclose(oracle.linear(a, b), a.astype(np.float64) @ b.T.astype(np.float64),
                               rtol=1e-4, atol=1e-4)


def test_attention_matches_dense_softmax():
    """ops.rs:238-263: tiled online softmax equals dense causal softmax (T=300)."""
    q = np.sin(np.arange(300 * 4, dtype=np.float32) * np.float32(0.013)).reshape(1, 300, 4)
    out = oracle.attention(q, q, q, causal=True)
    s = (q[0].astype(np.float64) @ q[0].T.astype(np.float64)) / 2.0
    s[np.triu_indices(300, 1)] = -np.inf
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    assert np.abs(out[0] - p @ q[0]).max() < 1e-5


def test_attention_gqa_and_cached_prefix():
    rng = np.random.default_rng(9)
    q = rng.standard_normal((4, 5, 8)).astype(np.float32)
    k = rng.standard_normal((2, 12, 8)).astype(np.float32)
    v = rng.standard_normal((2, 12, 8)).astype(np.float32)
    out = oracle.attention(q, k, v, causal=True)
    for h in range(4):
        kk, vv = k[h // 2].astype(np.float64), v[h // 2].astype(np.float64)
        s = q[h].astype(np.float64) @ kk.T / np.sqrt(8)
        for i in range(5):
            s[i, 12 - 5 + i + 1:] = -np.inf  # lower-right aligned causal mask
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        np.testing.assert_allclose(out[h], p @ vv, rtol=1e-5, atol=1e-6)


def test_rotary_rotate_half_convention():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((5, 2, 8)).astype(np.float32)
    y = oracle.rotary(x, 4, 10000.0, pos0=3)
    inv = 10000.0 ** (-np.arange(0, 4, 2) / 4.0)
    for t in range(5):
        ang = (t + 3) * inv
        c, s = np.cos(np.concatenate([ang, ang])), np.sin(np.concatenate([ang, ang]))
        r = x[t, :, :4]
        rot = np.concatenate([-r[:, 2:], r[:, :2]], -1)
        np.testing.assert_allclose(y[t, :, :4], r * c + rot * s, rtol=1e-5, atol=1e-5)
        np.testing.assert_array_equal(y[t, :, 4:], x[t, :, 4:])


def test_f16_helpers_match_numpy():
    L = oracle.lib()
    rng = np.random.default_rng(11)
    vals = np.concatenate([rng.standard_normal(2000) * s for s in (1e-7, 1e-5, 1e-2, 1, 1e3, 7e4)])
    vals = np.concatenate([vals, [0.0, -0.0, 65504.0, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8]])
    for x in vals.astype(np.float32):
        got = L.oracle_f32_to_f16(float(x))
        assert got == np.float32(x).astype(np.float16).view(np.uint16), x
        assert L.oracle_f16_to_f32(got) == np.float32(np.float16(x)) or np.isnan(x)
