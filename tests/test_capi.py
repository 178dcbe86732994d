"""The C-ABI library loads and exports every entry point include/clef_hip.h
declares, and rejects invalid requests before touching the device.  No
kernel is launched here (these tests run without a GPU)."""
import ctypes as C
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "clef_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(clef_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def clef():
    import clef_hip
    clef_hip.lib()
    return clef_hip


def test_library_exports_every_declared_symbol(clef):
    names = declared_functions()
    assert len(names) >= 20
    lib = C.CDLL(str(clef.LIB_PATH))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(clef.SIGNATURES), set(names) ^ set(clef.SIGNATURES)


def test_abi_version(clef):
    assert clef.lib().clef_hip_abi_version() == 2


@pytest.mark.parametrize("shape", [(0, 32, 32, 128, 128), (4097 * 256, 16, 32, 128, 128),
                                   (1, 2, 3, 128, 128), (1, 1, 1, 129, 128), (1, 1, 1, 128, 129),
                                   (1, 1, 1, 0, 4)])
def test_scan_rejects_unsupported_shapes_before_launch(clef, shape):
    """metal.rs:945-956: dimension checks happen before any allocation."""
    T, Hk, Hv, dk, dv = shape
    assert clef.lib().clef_delta_scan_workspace(T, Hk, Hv, dk, dv, 64, 0) == 0
    rc = clef.lib().clef_delta_scan(1, 1, 1, 0, 0, 0, 1, 1, 0, 0, T, Hk, Hv, dk, dv, 64, 0, None, 0,
                                    1, 0, 0, None, None, 1, 1 << 30, None)
    assert rc < 0
    assert "DeltaNet scan" in clef.last_error()


def test_scan_rejects_bad_chunk_capture_and_workspace(clef):
    L = clef.lib()
    assert L.clef_delta_scan_workspace(256, 4, 4, 64, 64, 32, 0) == 0
    ws = L.clef_delta_scan_workspace(256, 4, 4, 64, 64, 64, 0)
    assert ws > 0
    args = lambda capture, wsb: (1, 1, 1, 0, 0, 0, 1, 1, 0, 0, 256, 4, 4, 64, 64, 64, 0, None,
                                 capture, 1, 0, 0, None, None, 256, wsb, None)
    assert L.clef_delta_scan(*args(300, ws)) < 0          # capture beyond T
    assert L.clef_delta_scan(*args(5, ws)) < 0            # capture without a buffer
    assert L.clef_delta_scan(*args(0, ws - 1)) < 0        # workspace too small
    assert "workspace" in clef.last_error()


def test_gemm_and_pointwise_validation(clef):
    L = clef.lib()
    assert L.clef_gemm(None, 0, 1, 0, 1, 0, 4, 4, 4, 1, 1, 0, None) < 0
    assert L.clef_gemm(1, 0, 1, 0, 1, 0, 0, 4, 4, 1, 1, 0, None) < 0
    assert L.clef_gemm(1, 2, 1, 0, 1, 0, 4, 4, 4, 1, 1, 0, None) < 0   # ldx < K
    assert L.clef_gemm(1, 0, 1, 0, 1, 0, 4, 4, 4, 7, 1, 0, None) < 0   # dtype
    assert L.clef_rms_norm(1, 0, 0, 1, 1, 0, 0, 4, 8, 0.0, None) < 0   # eps
    assert L.clef_conv_silu(1, 0, 0, None, 2, 1, 4, 1, 0, 0, 4, 8, None) < 0  # history rows w/o data
    assert L.clef_attention_gated(1, 64, 1, 64, 1, 64, 1, 3, 2, 4, 4, 64, 1, 128, 128, 1, 192, None) < 0
    assert L.clef_attention_gated(1, 64, 1, 64, 1, 64, 1, 4, 2, 8, 4, 64, 1, 128, 128, 1, 256, None) < 0


def test_backbone_create_rejects_bad_config(clef):
    cfg = clef.BackboneConfig()
    cfg.hidden, cfg.intermediate, cfg.vocab, cfg.n_layers = 16, 32, 64, 1
    cfg.eps, cfg.profile, cfg.max_tokens = 0.0, 0, 4096
    layers = (clef.LayerWeights * 1)()
    handle = C.c_void_p()
    assert clef.lib().clef_backbone_create(C.byref(cfg), layers, 1, 1, C.byref(handle)) < 0
    assert not handle.value


def _check_plan(clef, cu, T, unit):
    """The host evaluation of the ragged tables (the device kernels' code):
    monotone spans inside [0, T], units tiling each span, and never more
    units than the ceil(T / unit) + nseq the workspaces reserve."""
    import numpy as np
    cu = np.asarray(cu, np.int64)
    nseq = len(cu) - 1
    spans, units = clef.ragged_plan(cu, T, unit)
    assert spans[0] >= 0 and spans[-1] <= T and (np.diff(spans) >= 0).all()
    # the spans are the running maximum of the clamped offsets
    assert (spans == np.maximum.accumulate(np.clip(cu, 0, T))).all()
    assert len(units) <= (T + unit - 1) // unit + nseq
    lens = np.diff(spans)
    assert len(units) == int(((lens + unit - 1) // unit).sum())
    if unit == 64:
        covered = np.zeros(T, np.int64)
        for t0, n in units:
            assert 0 <= t0 and 1 <= n <= 64 and t0 + n <= T
            covered[t0:t0 + n] += 1
        inside = np.zeros(T, np.int64)
        for s in range(nseq):
            inside[spans[s]:spans[s + 1]] += 1
        assert (covered == inside).all()  # each token of a span in exactly one chunk
    else:
        seen = set()
        for s, t in units:
            assert 0 <= s < nseq and 0 <= t and t * 128 < lens[s]
            seen.add((int(s), int(t)))
        assert len(seen) == len(units)
    return spans


@pytest.mark.parametrize("unit", [64, 128])
def test_ragged_plan_valid_table_is_unchanged(clef, unit):
    import numpy as np
    rng = np.random.default_rng(4)
    lens = rng.integers(1, 700, 37)
    cu = np.concatenate([[0], np.cumsum(lens)])
    spans = _check_plan(clef, cu, int(cu[-1]), unit)
    assert (spans == cu).all()


@pytest.mark.parametrize("unit", [64, 128])
@pytest.mark.parametrize("cu,T", [
    ([0, 1000, 0, 1000, 0, 1000], 1000),          # overlapping sequences
    ([0, 5000, 6000], 1000),                      # offsets past T
    ([-50, 100, 40, 900, 300, 1000], 1000),       # negative and non-monotone
    ([0] * 4096 + [4096], 4096),                  # many empty sequences
    ([0, 4096] * 2048 + [4096], 4096),            # 4096 sequences, all overlapping
    ([2 ** 31 - 1, -(2 ** 31), 7, 3], 10),        # extreme values
])
def test_ragged_plan_malformed_tables_stay_in_bounds(clef, unit, cu, T):
    _check_plan(clef, cu, T, unit)


def _seq_of(cu, t):
    """The kernels' binary search: the last s with cu[s] <= t (0 if none)."""
    lo, hi = 0, len(cu) - 2
    while lo < hi:
        mid = (lo + hi + 1) >> 1
        if cu[mid] <= t:
            lo = mid
        else:
            hi = mid - 1
    return lo


def _conv_varlen_reads(cu, T, hrows, taps, run=16):
    """Every (buffer, sequence, row) the ragged conv kernels read for a
    cu_seqlens table, following their index arithmetic (pointwise.hip:
    conv_silu_varlen_kernel's per-run and per-token paths with rows clamped
    into [0, T), conv_silu_varlen_scalar, the sequence start clamped into
    [0, t] by both)."""
    nseq = len(cu) - 1
    reads = []
    if taps <= 4:  # vectorised kernel, runs of `run` tokens
        for t0 in range(0, T, run):
            t1 = min(t0 + run, T)
            reads += [("x", 0, min(max(t0 - 3 + r, 0), T - 1)) for r in range(run + 3)]
            s = _seq_of(cu, t0)
            if cu[s] <= t0 - 3 and (s + 1 >= nseq or cu[s + 1] >= t1):
                continue  # inside one sequence: only the clamped rows above
            for t in range(t0, t1):
                while s + 1 < nseq and cu[s + 1] <= t:
                    s += 1
                start = min(max(cu[s], 0), t)
                avail = hrows + (t - start)
                for k in range(4):
                    tap, tp = k - (4 - taps), t - 3 + k
                    if tap >= 0 and avail - (3 - k) >= 0 and tp < start:
                        reads.append(("hist", s, hrows + tp - start))
    for t in range(T):  # any-layout kernel
        s = _seq_of(cu, t)
        start = min(max(cu[s], 0), t)
        for tap in range(taps):
            tp = t - (taps - 1 - tap)
            hr = hrows + (tp - start)
            if hr < 0:
                continue
            reads.append(("x", 0, tp) if tp >= start and tp >= 0 else ("hist", s, hr))
    return reads


@pytest.mark.parametrize("cu,T", [
    ([0, 1000, 0, 1000, 0, 1000], 1000),
    ([0, 5000, 6000], 1000),
    ([-50, 100, 40, 900, 300, 1000], 1000),
    ([-7, -3, 2, 1, 40], 40),
    ([0] * 64 + [64], 64),
    ([2 ** 31 - 1, -(2 ** 31), 7, 3], 10),
])
@pytest.mark.parametrize("hrows,taps", [(0, 4), (3, 4), (1, 2), (7, 8)])
def test_conv_varlen_malformed_tables_stay_in_bounds(cu, T, hrows, taps):
    """Any device cu_seqlens table keeps the ragged conv inside x ([T] rows)
    and the history ([nseq] x [hrows] rows): the sequence start is clamped
    into [0, t] before any row is derived from it."""
    if hrows > taps - 1:
        pytest.skip("history of at most taps - 1 rows")
    nseq = len(cu) - 1
    for buf, s, row in _conv_varlen_reads(cu, T, hrows, taps):
        assert 0 <= s < nseq
        assert 0 <= row < (T if buf == "x" else hrows), (buf, s, row)


def _brute_attention_order(spans):
    """(sequence, tile) pairs in the attention launch order, from its
    definition: key count np + min(128 (t + 1), len) per query tile, most
    first, ties in table order; beyond 8192 tiles, table order."""
    import numpy as np
    lens = np.diff(np.asarray(spans, np.int64))
    items = [(s, t, min(128 * (t + 1), int(lens[s]))) for s in range(len(lens))
             for t in range((int(lens[s]) + 127) // 128)]
    if len(items) <= 8192:
        items = [it for _, it in sorted(enumerate(items), key=lambda e: (-e[1][2], e[0]))]
    return np.array([(s, t) for s, t, _ in items], np.int64).reshape(-1, 2)


@pytest.mark.parametrize("case", range(6))
def test_ragged_plan_attention_order_matches_definition(clef, case):
    """The closed-form ranks (counts of each sequence's tiles above a key
    count, and ties in earlier sequences) against a sort by key count."""
    import numpy as np
    rng = np.random.default_rng(40 + case)
    if case == 0:    # uniform lengths, many ties at multiples of 128
        lens = rng.integers(1, 9, 50) * 128
    elif case == 1:  # random lengths
        lens = rng.integers(1, 3000, 64)
    elif case == 2:  # near-multiples of 128, single tokens, empty sequences
        lens = rng.choice([0, 1, 127, 128, 129, 255, 256, 257, 4096], 200)
    elif case == 3:  # a 512-token prefix's ragged batch: 32 requests in [128, 4096]
        lens = rng.integers(128, 4097, 32)
    elif case == 4:  # 4096 sequences of 256: exactly 8192 tiles, ranked
        lens = np.full(4096, 256)
    else:            # past 8192 tiles (3000 x 3): table order
        lens = np.full(3000, 300)
    cu = np.concatenate([[0], np.cumsum(lens)])
    T = max(int(cu[-1]), 1)
    spans, units = clef.ragged_plan(cu, T, 128)
    expected = _brute_attention_order(spans)
    assert units.shape == expected.shape and (units == expected).all()


@pytest.mark.parametrize("cu,T", [([0, 1000, 0, 1000, 0, 1000], 1000), ([-50, 100, 40, 900, 300, 1000], 1000),
                                  ([0, 5000, 6000], 1000)])
def test_ragged_plan_attention_order_of_malformed_tables(clef, cu, T):
    spans, units = clef.ragged_plan(cu, T, 128)
    expected = _brute_attention_order(spans)
    assert units.shape == expected.shape and (units == expected).all()


def test_ragged_plan_rejects_bad_arguments(clef):
    import numpy as np
    cu = np.array([0, 10], np.int32)
    sp = np.zeros(2, np.int32)
    L = clef.lib()
    assert L.clef_ragged_plan(cu.ctypes.data, 1, 10, 32, sp.ctypes.data, None, 0) < 0
    assert L.clef_ragged_plan(cu.ctypes.data, 0, 10, 64, sp.ctypes.data, None, 0) < 0
    assert L.clef_ragged_plan(cu.ctypes.data, 1, 10, 64, sp.ctypes.data, sp.ctypes.data, 1) < 0
