"""Hybrid backbone prefill on the GPU against the reference's golden fixture
and the CPU oracle.

Bars: the f32 profile must reproduce the reference's golden hidden states of
the synthetic backbone fixture within the reference's own tolerance
(1e-5 + 1e-4|e|, mod.rs:75-111) and the oracle within the same bar; the
mixed-f16 profile must stay within rtol 2e-2 of the F32 path (elementwise,
with an absolute floor of 2e-2 * max|e| for near-zero entries) and give the
same argmax decision.
"""
import json

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


@pytest.fixture(scope="module")
def fixture(golden_dir):
    from safetensors.numpy import load_file
    cfg = json.loads((golden_dir / "backbone-config.json").read_text())
    w = load_file(str(golden_dir / "backbone.safetensors"))
    exp = load_file(str(golden_dir / "backbone-output.safetensors"))["hidden"]
    return cfg, w, exp


def _close(actual, expected, atol, rtol):
    actual, expected = np.asarray(actual, np.float64), np.asarray(expected, np.float64)
    assert np.isfinite(actual).all()
    err = np.abs(actual - expected)
    bad = err > atol + rtol * np.abs(expected)
    assert not bad.any(), f"{bad.sum()}/{bad.size} out of tolerance, max err {err.max():.3e}"


def _mixed_close(actual, expected):
    expected = np.asarray(expected, np.float64)
    _close(actual, expected, 2e-2 * np.abs(expected).max(), 2e-2)


def _to_dev(w):
    return {k: torch.from_numpy(np.ascontiguousarray(v)).cuda() for k, v in w.items()}


@gpu
def test_fixture_backbone_f32_matches_reference_golden(clef, fixture):
    cfg, w, exp = fixture
    b = clef.Backbone(cfg, _to_dev(w), profile="f32")
    hidden, _ = b.prefill(np.arange(20))
    _close(hidden.cpu().numpy(), exp, 1e-5, 1e-4)
    ref, _ = oracle.Backbone(cfg, w).prefill(np.arange(20))
    _close(hidden.cpu().numpy(), ref, 1e-5, 1e-4)


@gpu
@pytest.mark.parametrize("scan", ["mixed", "strict"])
def test_fixture_backbone_mixed_profile(clef, fixture, scan):
    cfg, w, exp = fixture
    b = clef.Backbone(cfg, _to_dev(w), profile="mixed", scan_precision=scan)
    hidden, _ = b.prefill(np.arange(20))
    _mixed_close(hidden.cpu().numpy(), exp)
    emul, _ = oracle.Backbone(cfg, w, mixed_f16=True).prefill(np.arange(20))
    _close(hidden.cpu().numpy(), emul, 5e-3, 5e-3)


@gpu
@pytest.mark.parametrize("profile", ["f32", "mixed"])
def test_fixture_prefix_capture_and_resume(clef, fixture, profile):
    """mod.rs:113-171 on the device path."""
    cfg, w, _ = fixture
    b = clef.Backbone(cfg, _to_dev(w), profile=profile)
    ids = np.arange(20)
    expected = b.prefill(ids)[0].cpu().numpy()
    check = (lambda a, e: _close(a, e, 1e-5, 1e-4)) if profile == "f32" else \
        (lambda a, e: _close(a, e, 2e-3, 2e-3))
    for boundary in (1, 2, 3, 8, 19):
        captured, state = b.prefill(ids, capture=boundary)
        assert np.array_equal(captured.cpu().numpy(), expected)  # capturing changes nothing
        with pytest.raises(clef.ClefError):
            b.prefill(ids[boundary:], initial=state, capture=1)
        resumed, _ = b.prefill(ids[boundary:], initial=state)
        check(resumed.cpu().numpy(), expected)
        changed = ids.copy()
        changed[boundary:] += 20
        resumed, _ = b.prefill(changed[boundary:], initial=state)
        check(resumed.cpu().numpy(), b.prefill(changed)[0].cpu().numpy())
        again, _ = b.prefill(ids[boundary:], initial=state)  # the state is not mutated
        check(again.cpu().numpy(), expected)
    with pytest.raises(clef.ClefError):
        b.prefill(ids, capture=20)
    with pytest.raises(clef.ClefError):
        b.prefill(np.array([64]))


@pytest.fixture(scope="module")
def block_case():
    import workloads
    cfg = workloads.block_config()
    w = workloads.block_weights(cfg, seed=3)
    ids = workloads.block_ids(cfg, 2048, seed=3).numpy()
    head = workloads.block_head(cfg, seed=3)
    # the oracle needs only the gathered embedding rows: remap ids onto them
    uniq, inv = np.unique(ids, return_inverse=True)
    wh = {k: v.cpu().numpy() for k, v in w.items() if k != "model.language_model.embed_tokens.weight"}
    emb = w["model.language_model.embed_tokens.weight"]
    wh["model.language_model.embed_tokens.weight"] = emb[torch.from_numpy(uniq).long().cuda()].cpu().numpy()
    cfg_small = dict(cfg, vocab_size=len(uniq))
    ref, _ = oracle.Backbone(cfg_small, wh).prefill(inv.astype(np.int32))
    ref_logits = ref[-1].astype(np.float64) @ head.cpu().numpy().astype(np.float64).T
    return cfg, w, ids, head, ref, ref_logits


@gpu
@pytest.mark.parametrize("profile", ["f32", "mixed"])
def test_block_prefill_matches_oracle(clef, block_case, profile):
    """3 DeltaNet + 1 gated attention layer, hidden 2048, T = 2048, seed 3."""
    cfg, w, ids, head, ref, ref_logits = block_case
    b = clef.Backbone(cfg, w, profile=profile)
    hidden, _ = b.prefill(ids)
    logits = clef.head_logits(hidden[-1], head).cpu().numpy()
    got = hidden.cpu().numpy()
    if profile == "f32":
        _close(got, ref, 1e-4, 1e-4)
    else:
        _mixed_close(got, ref)
    assert int(np.argmax(logits)) == int(np.argmax(ref_logits))


@gpu
@pytest.mark.parametrize("profile", ["f32", "mixed"])
def test_fixture_varlen_batch_equals_per_request_resume(clef, fixture, profile):
    """A ragged batch resumed from one shared prefix state (every request a
    prefix-cache hit, prefix_cache.rs:135-177): each request's rows equal the
    single-request resume (qwen.rs:337-364) and the oracle over prefix + request."""
    cfg, w, _ = fixture
    b = clef.Backbone(cfg, _to_dev(w), profile=profile)
    rng = np.random.default_rng(4)
    prefix = rng.integers(0, cfg["vocab_size"], 8)
    lens = [5, 1, 12, 3, 9]
    reqs = [rng.integers(0, cfg["vocab_size"], n) for n in lens]
    _, state = b.prefill(np.concatenate([prefix, reqs[0]]), capture=len(prefix))
    cu = np.concatenate([[0], np.cumsum(lens)])
    hidden = b.prefill_varlen(np.concatenate(reqs), cu, initial=state).cpu().numpy()
    orc = oracle.Backbone(cfg, w)
    for s, ids in enumerate(reqs):
        got = hidden[cu[s]:cu[s + 1]]
        single = b.prefill(ids, initial=state)[0].cpu().numpy()[len(prefix):]
        ref = orc.prefill(np.concatenate([prefix, ids]))[0][len(prefix):]
        if profile == "f32":
            _close(got, single, 1e-6, 1e-6)
            _close(got, ref, 1e-5, 1e-4)
        else:
            _close(got, single, 2e-3, 2e-3)
            _mixed_close(got, ref)


@gpu
@pytest.mark.parametrize("profile", ["f32", "mixed"])
def test_block_ragged_batch_behind_shared_prefix(clef, block_case, profile):
    """The ragged workload at the block shape: requests packed by cu_seqlens
    behind one 512-token prefix computed once (prefix_cache.rs:135-177), each
    request's rows and pooled-head decision equal to its single resume
    (qwen.rs:337-364), which the block oracle test pins."""
    cfg, w, ids, head, _, _ = block_case
    b = clef.Backbone(cfg, w, profile=profile, max_tokens=8192)
    rng = np.random.default_rng(4)
    prefix = rng.integers(0, cfg["vocab_size"], 512)
    lens = [700, 128, 1, 65, 1500, 64]
    reqs = [rng.integers(0, cfg["vocab_size"], n) for n in lens]
    _, state = b.prefill(np.concatenate([prefix, reqs[0]]), capture=512)
    cu = np.concatenate([[0], np.cumsum(lens)])
    hidden = b.prefill_varlen(np.concatenate(reqs), cu, initial=state)
    for s, r in enumerate(reqs):
        single = b.prefill(r, initial=state)[0][512:]
        got = hidden[cu[s]:cu[s + 1]]
        if profile == "f32":
            _close(got.cpu().numpy(), single.cpu().numpy(), 1e-5, 1e-5)
        else:
            _close(got.cpu().numpy(), single.cpu().numpy(), 2e-3, 2e-3)
        lg = clef.head_logits(got[-1], head).cpu().numpy()
        ls = clef.head_logits(single[-1], head).cpu().numpy()
        assert int(np.argmax(lg)) == int(np.argmax(ls))
