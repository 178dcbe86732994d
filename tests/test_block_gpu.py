"""Hybrid backbone prefill on the GPU against the reference's golden fixture
and the CPU oracle.

Bars (elementwise, |actual - expected| <= atol + rtol |expected|):
- f32 profile: the reference's own 1e-5 + 1e-4 |e| (mod.rs:75-111), against
  the golden hidden states of the synthetic fixture and the oracle; at the
  full block (T = 2048, hidden 2048) against the oracle with its projection
  dot products accumulated in f64 (two f32 evaluations that sum K = 6144
  products in different orders differ by about 1e-5 there, so the bar is
  taken against the more exact yardstick, and the distances of the device
  path and of the f32 oracle from it are both recorded);
- mixed-f16 profile: rtol 2e-2 with an absolute floor of 1e-2 x RMS(e) (f16
  rounding of intermediate activations perturbs every element by a fraction
  of the activations' typical size, so elements near zero need a floor; it is
  set by the RMS of the expected values, not their maximum);
- decisions (the argmax of the 3-logit pooled head, qwen.rs last-token
  pooling) must equal the oracle's exactly: at 64 positions of the block at
  T = 2048, at 64 positions of the benchmarked T = 4096 prefill, and at 128
  positions over eight independently seeded 1024-token sequences.
Achieved errors are appended to the JSON file named by CLEF_PARITY_LOG.
"""
import ctypes
import json
import os

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


def _record(name, **values):
    path = os.environ.get("CLEF_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps({"test": name, **values}) + "\n")


def _errors(actual, expected):
    a, e = np.asarray(actual, np.float64), np.asarray(expected, np.float64)
    err = np.abs(a - e)
    rms = float(np.sqrt(np.mean(e * e)))
    return {"max_abs": float(err.max()), "max_abs_over_rms": float(err.max() / rms),
            "max_rel_ge_1": float((err / np.maximum(np.abs(e), 1e-30))[np.abs(e) >= rms].max(initial=0.0)),
            "frac_outside_rtol_2e-2": float((err > 2e-2 * np.abs(e)).mean()), "rms": rms}


def _close(actual, expected, atol, rtol, name=None):
    actual, expected = np.asarray(actual, np.float64), np.asarray(expected, np.float64)
    assert np.isfinite(actual).all()
    err = np.abs(actual - expected)
    if name:
        _record(name, atol=atol, rtol=rtol, **_errors(actual, expected))
    bad = err > atol + rtol * np.abs(expected)
    assert not bad.any(), f"{bad.sum()}/{bad.size} out of tolerance, max err {err.max():.3e}"


def _mixed_close(actual, expected, name=None):
    expected = np.asarray(expected, np.float64)
    _close(actual, expected, 1e-2 * np.sqrt(np.mean(expected * expected)), 2e-2, name)


def _to_dev(w):
    return {k: torch.from_numpy(np.ascontiguousarray(v)).cuda() for k, v in w.items()}


@gpu
def test_fixture_backbone_f32_matches_reference_golden(clef, fixture):
    cfg, w, exp = fixture
    b = clef.Backbone(cfg, _to_dev(w), profile="f32")
    hidden, _ = b.prefill(np.arange(20))
    _close(hidden.cpu().numpy(), exp, 1e-5, 1e-4, "fixture f32 vs golden")
    ref, _ = oracle.Backbone(cfg, w).prefill(np.arange(20))
    _close(hidden.cpu().numpy(), ref, 1e-5, 1e-4, "fixture f32 vs oracle")


@gpu
@pytest.mark.parametrize("scan", ["mixed", "strict"])
def test_fixture_backbone_mixed_profile(clef, fixture, scan):
    cfg, w, exp = fixture
    b = clef.Backbone(cfg, _to_dev(w), profile="mixed", scan_precision=scan)
    hidden, _ = b.prefill(np.arange(20))
    _mixed_close(hidden.cpu().numpy(), exp, f"fixture mixed ({scan} scan) vs golden")
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


@gpu
def test_prefix_state_of_another_size_is_rejected(clef, fixture):
    """A state whose size does not match this backbone at its token count is
    refused before any launch (the reference's layer-count check, qwen.rs:355)."""
    cfg, w, _ = fixture
    b = clef.Backbone(cfg, _to_dev(w), profile="f32")
    _, state = b.prefill(np.arange(10), capture=4)
    wrong_tokens = clef.PrefixState(state.buffer, 5)
    with pytest.raises(clef.ClefError, match="size"):
        b.prefill(np.arange(3), initial=wrong_tokens)
    truncated = clef.PrefixState(state.buffer[:-256], 4)
    with pytest.raises(clef.ClefError, match="size"):
        b.prefill(np.arange(3), initial=truncated)
    with pytest.raises(clef.ClefError, match="size"):
        b.prefill_varlen(np.arange(3), [0, 3], initial=wrong_tokens)
    other = clef.Backbone(dict(cfg, layer_types=cfg["layer_types"][:3]), _to_dev(w), profile="f32")
    with pytest.raises(clef.ClefError, match="size"):
        other.prefill(np.arange(3), initial=state)
    resumed, _ = b.prefill(np.arange(4, 10), initial=state)  # the right one still resumes
    assert resumed.shape[0] == 10


@gpu
def test_cancellation_and_deadline(clef, fixture):
    """Control::check (models/mod.rs:45-59) at the start of a prefill and
    before each layer: a set flag or a passed deadline returns Cancelled /
    DeadlineExceeded; clearing it restores normal prefills."""
    cfg, w, _ = fixture
    b = clef.Backbone(cfg, _to_dev(w), profile="f32")
    expected = b.prefill(np.arange(20))[0].cpu().numpy()
    flag = ctypes.c_int32(1)
    b.set_control(cancel=flag)
    with pytest.raises(clef.ClefError) as e:
        b.prefill(np.arange(20))
    assert e.value.code == clef.CANCELLED
    with pytest.raises(clef.ClefError) as e:
        b.prefill_varlen(np.arange(20), [0, 7, 20])
    assert e.value.code == clef.CANCELLED
    flag.value = 0
    np.testing.assert_array_equal(b.prefill(np.arange(20))[0].cpu().numpy(), expected)
    b.set_control(deadline=clef.monotonic_seconds() - 1.0)
    with pytest.raises(clef.ClefError) as e:
        b.prefill(np.arange(20))
    assert e.value.code == clef.DEADLINE_EXCEEDED
    b.set_control(deadline=clef.monotonic_seconds() + 3600.0)
    np.testing.assert_array_equal(b.prefill(np.arange(20))[0].cpu().numpy(), expected)
    b.set_control()
    np.testing.assert_array_equal(b.prefill(np.arange(20))[0].cpu().numpy(), expected)


# ---------------------------------------------------------------------------
# The block at its real shape: hidden 2048, 3 DeltaNet + 1 attention layer
# ---------------------------------------------------------------------------
def _oracle_backbone(cfg, w, id_lists):
    """Oracle over the embedding rows the given id lists use (ids remapped)."""
    uniq = np.unique(np.concatenate([np.asarray(x).ravel() for x in id_lists]))
    emb_name = "model.language_model.embed_tokens.weight"
    wh = {k: v.cpu().numpy() for k, v in w.items() if k != emb_name}
    wh[emb_name] = w[emb_name][torch.from_numpy(uniq).long().cuda()].cpu().numpy()
    remap = lambda ids: np.searchsorted(uniq, np.asarray(ids)).astype(np.int32)
    return oracle.Backbone(dict(cfg, vocab_size=len(uniq)), wh), remap


DECISION_POSITIONS = np.arange(31, 2048, 32)  # 64 positions: a prefix of each length ends there


@pytest.fixture(scope="module")
def block_case():
    import workloads
    cfg = workloads.block_config()
    w = workloads.block_weights(cfg, seed=3)
    ids = workloads.block_ids(cfg, 2048, seed=3).numpy()
    head = workloads.block_head(cfg, seed=3)
    orc, remap = _oracle_backbone(cfg, w, [ids])
    ref, _ = orc.prefill(remap(ids))
    with oracle.exact_dots():
        exact, _ = orc.prefill(remap(ids))
    ref_logits = ref[DECISION_POSITIONS].astype(np.float64) @ head.cpu().numpy().astype(np.float64).T
    return cfg, w, ids, head, ref, ref_logits, exact


def _decisions(clef, hidden, head, positions):
    return np.stack([clef.head_logits(hidden[int(t)], head).cpu().numpy() for t in positions]).astype(np.float64)


def _margins(logits):
    s = np.sort(logits, axis=1)
    return s[:, -1] - s[:, -2]


@gpu
@pytest.mark.parametrize("profile", ["f32", "mixed"])
def test_block_prefill_matches_oracle(clef, block_case, profile):
    """3 DeltaNet + 1 gated attention layer, hidden 2048, T = 2048, seed 3:
    hidden states within the profile's bar and the pooled head's decision
    equal to the oracle's at 64 positions (each the last token of a prefix)."""
    cfg, w, ids, head, ref, ref_logits, exact = block_case
    b = clef.Backbone(cfg, w, profile=profile)
    hidden, _ = b.prefill(ids)
    got = hidden.cpu().numpy()
    if profile == "f32":
        _record("block T=2048 f32 vs f32 oracle", **_errors(got, ref))
        _record("block T=2048 f32 oracle vs exact-accumulation oracle", **_errors(ref, exact))
        _close(got, exact, 1e-5, 1e-4, "block T=2048 f32 vs exact-accumulation oracle")
    else:
        _mixed_close(got, ref, "block T=2048 mixed vs oracle")
    logits = _decisions(clef, hidden, head, DECISION_POSITIONS)
    margins = _margins(ref_logits)
    _record(f"block T=2048 {profile} decisions", decisions=len(DECISION_POSITIONS),
            min_margin=float(margins.min()), max_logit_err=float(np.abs(logits - ref_logits).max()))
    assert (np.argmax(logits, 1) == np.argmax(ref_logits, 1)).all(), (
        np.flatnonzero(np.argmax(logits, 1) != np.argmax(ref_logits, 1)), margins.min())


BENCH_T = 4096
BENCH_POSITIONS = np.arange(63, BENCH_T, 64)  # 64 decisions spread over the whole prefill


@pytest.fixture(scope="module")
def bench_case():
    """The benchmarked workload itself: the block at T = 4096, seed 3 (the
    token ids bench.py times), with the oracle's hidden states (f32, and with
    f64-accumulated projection dots) and its logits at 64 positions."""
    import workloads
    cfg = workloads.block_config()
    w = workloads.block_weights(cfg, seed=3)
    ids = workloads.block_ids(cfg, BENCH_T, seed=3).numpy()
    head = workloads.block_head(cfg, seed=3)
    orc, remap = _oracle_backbone(cfg, w, [ids])
    ref, _ = orc.prefill(remap(ids))
    with oracle.exact_dots():
        exact, _ = orc.prefill(remap(ids))
    ref_logits = ref[BENCH_POSITIONS].astype(np.float64) @ head.cpu().numpy().astype(np.float64).T
    return cfg, w, ids, head, ref, ref_logits, exact


@gpu
@pytest.mark.parametrize("profile", ["f32", "mixed"])
def test_block_bench_workload_T4096_matches_oracle(clef, bench_case, profile):
    """The prefill bench.py times (3 DeltaNet + 1 gated attention layer,
    hidden 2048, T = 4096, seed 3): hidden states within the profile's bar
    (f32 against the f64-dot oracle, as at T = 2048) and the pooled head's
    decision equal to the oracle's at 64 positions over all 4096 tokens."""
    cfg, w, ids, head, ref, ref_logits, exact = bench_case
    b = clef.Backbone(cfg, w, profile=profile, max_tokens=8192)
    hidden, _ = b.prefill(ids)
    got = hidden.cpu().numpy()
    if profile == "f32":
        _record("block T=4096 f32 vs f32 oracle", **_errors(got, ref))
        _close(got, exact, 1e-5, 1e-4, "block T=4096 f32 vs exact-accumulation oracle")
    else:
        _mixed_close(got, ref, "block T=4096 mixed vs oracle")
    logits = _decisions(clef, hidden, head, BENCH_POSITIONS)
    margins = _margins(ref_logits)
    err = np.abs(logits - ref_logits).max()
    _record(f"block T=4096 {profile} decisions", decisions=len(BENCH_POSITIONS), min_margin=float(margins.min()),
            max_logit_err=float(err), margin_over_err=float(margins.min() / max(err, 1e-30)))
    assert (np.argmax(logits, 1) == np.argmax(ref_logits, 1)).all(), (
        np.flatnonzero(np.argmax(logits, 1) != np.argmax(ref_logits, 1)), margins.min())


SEEDED_RUNS = tuple(range(10, 18))  # eight independently seeded token sequences
SEEDED_T = 1024
SEEDED_POSITIONS = np.arange(63, SEEDED_T, 64)


@pytest.fixture(scope="module")
def seeded_case(block_case):
    """Eight token sequences of 1024 ids (seeds 10..17) through the seed-3
    block weights, with the oracle's logits at 16 positions of each."""
    import workloads
    cfg, w, _, head, _, _, _ = block_case
    runs = [workloads.block_ids(cfg, SEEDED_T, seed=sd).numpy() for sd in SEEDED_RUNS]
    orc, remap = _oracle_backbone(cfg, w, runs)
    hv = head.cpu().numpy().astype(np.float64)
    refs = [orc.prefill(remap(r))[0][SEEDED_POSITIONS].astype(np.float64) @ hv.T for r in runs]
    return cfg, w, head, runs, refs


@gpu
@pytest.mark.parametrize("profile", ["f32", "mixed"])
def test_block_decisions_over_seeded_sequences(clef, seeded_case, profile):
    """128 decisions over eight independently seeded sequences (16 positions
    each): the device path's argmax equals the oracle's at every one.  The
    ratio of the smallest margin to the largest logit error is recorded."""
    cfg, w, head, runs, refs = seeded_case
    b = clef.Backbone(cfg, w, profile=profile)
    min_margin, max_err, wrong = np.inf, 0.0, []
    for i, (ids, ref_logits) in enumerate(zip(runs, refs)):
        hidden, _ = b.prefill(ids)
        logits = _decisions(clef, hidden, head, SEEDED_POSITIONS)
        min_margin = min(min_margin, float(_margins(ref_logits).min()))
        max_err = max(max_err, float(np.abs(logits - ref_logits).max()))
        wrong += [(SEEDED_RUNS[i], int(p)) for p in
                  SEEDED_POSITIONS[np.argmax(logits, 1) != np.argmax(ref_logits, 1)]]
    _record(f"block seeded sequences {profile} decisions", sequences=len(runs),
            decisions=len(runs) * len(SEEDED_POSITIONS), min_margin=min_margin, max_logit_err=max_err,
            margin_over_err=min_margin / max(max_err, 1e-30))
    assert not wrong, wrong


@gpu
@pytest.mark.parametrize("profile", ["f32", "mixed"])
def test_fixture_varlen_batch_equals_per_request_resume(clef, fixture, profile):
    """A ragged batch resumed from one shared prefix state (every request a
    prefix-cache hit, prefix_cache.rs:135-177): each request's rows equal the
    single-request resume (qwen.rs:337-364) and the oracle over prefix + request."""
    cfg, w, _ = fixture
    b = clef.Backbone(cfg, _to_dev(w), profile=profile)
    rng = np.random.default_rng(4)
    orc = oracle.Backbone(cfg, w)
    # prefixes that are and are not a multiple of 8 tokens (the packed
    # attention kernel needs 8-key runs; the others run per sequence)
    for plen in (8, 5, 13):
        prefix = rng.integers(0, cfg["vocab_size"], plen)
        lens = [5, 1, 12, 3, 9]
        reqs = [rng.integers(0, cfg["vocab_size"], n) for n in lens]
        _, state = b.prefill(np.concatenate([prefix, reqs[0]]), capture=len(prefix))
        cu = np.concatenate([[0], np.cumsum(lens)])
        hidden = b.prefill_varlen(np.concatenate(reqs), cu, initial=state).cpu().numpy()
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


@pytest.fixture(scope="module")
def ragged_case(block_case):
    """The ragged workload at full size: 32 requests, lengths uniform in
    [128, 4096] (seed 4, 81 588 tokens), one shared 512-token prefix."""
    import workloads
    cfg, w, _, head, _, _, _ = block_case
    prefix, lens, packed, cu = workloads.ragged_workload(cfg, seed=4)
    return cfg, w, head, prefix, lens, packed, cu


@gpu
@pytest.mark.parametrize("profile", ["f32", "mixed"])
def test_block_ragged_workload_equals_per_request_resume(clef, ragged_case, profile):
    """Every request of the full ragged workload: its packed rows equal its
    single-request resume from the shared prefix state (qwen.rs:337-364) and
    its pooled-head decision is the same."""
    cfg, w, head, prefix, lens, packed, cu = ragged_case
    b = clef.Backbone(cfg, w, profile=profile, max_tokens=512 + 4096)
    _, state = b.prefill(np.concatenate([prefix, packed[:1]]), capture=512)
    hidden = b.prefill_varlen(packed, cu, initial=state)
    worst = 0.0
    for s in range(len(lens)):
        single = b.prefill(packed[cu[s]:cu[s + 1]], initial=state)[0][512:]
        got = hidden[cu[s]:cu[s + 1]]
        g, e = got.cpu().numpy(), single.cpu().numpy()
        if profile == "f32":
            _close(g, e, 1e-5, 1e-5)
        else:
            _close(g, e, 2e-3, 2e-3)
        worst = max(worst, float(np.abs(g - e).max()))
        lg = clef.head_logits(got[-1], head).cpu().numpy()
        ls = clef.head_logits(single[-1], head).cpu().numpy()
        assert int(np.argmax(lg)) == int(np.argmax(ls)), s
    _record(f"ragged workload {profile}: packed vs single resume", requests=len(lens), tokens=int(cu[-1]),
            max_abs=worst)


ORACLE_REQUESTS = (368, 999, 3310)  # prefix + request within the reference's 4096 tokens (qwen.rs:349)


@pytest.fixture(scope="module")
def ragged_oracle(ragged_case):
    """The oracle's hidden rows for three requests of the ragged workload,
    resumed from its own capture of the shared 512-token prefix (projection
    dot products accumulated in f64, the yardstick of the block test)."""
    cfg, w, head, prefix, lens, packed, cu = ragged_case
    pick = [int(np.flatnonzero(lens == n)[0]) for n in ORACLE_REQUESTS]
    reqs = [packed[cu[s]:cu[s + 1]] for s in pick]
    orc, remap = _oracle_backbone(cfg, w, [prefix] + reqs)
    with oracle.exact_dots():
        _, ostate = orc.prefill(remap(np.concatenate([prefix, reqs[0][:1]])), capture=512)
        return reqs, [orc.prefill(remap(r), initial=ostate)[0][512:] for r in reqs]


@gpu
@pytest.mark.parametrize("profile", ["f32", "mixed"])
def test_block_ragged_requests_match_oracle(clef, ragged_case, ragged_oracle, profile):
    """Three requests of the ragged workload (368, 999 and 3310 tokens) packed
    behind the shared 512-token prefix, against the oracle: hidden rows within
    the profile's bar and the same decision at each request's last token."""
    cfg, w, head, prefix, lens, packed, cu = ragged_case
    reqs, refs = ragged_oracle
    b = clef.Backbone(cfg, w, profile=profile, max_tokens=512 + 4096)
    _, state = b.prefill(np.concatenate([prefix, reqs[0][:1]]), capture=512)
    sub_cu = np.concatenate([[0], np.cumsum([len(r) for r in reqs])])
    hidden = b.prefill_varlen(np.concatenate(reqs), sub_cu, initial=state)
    hv = head.cpu().numpy().astype(np.float64)
    for i, ref in enumerate(refs):
        got = hidden[sub_cu[i]:sub_cu[i + 1]]
        name = f"ragged request of {len(reqs[i])} tokens behind 512, {profile} vs oracle"
        if profile == "f32":
            _close(got.cpu().numpy(), ref, 1e-5, 1e-4, name)
        else:
            _mixed_close(got.cpu().numpy(), ref, name)
        lg = clef.head_logits(got[-1], head).cpu().numpy()
        lr = ref[-1].astype(np.float64) @ hv.T
        assert int(np.argmax(lg)) == int(np.argmax(lr))
