"""clef_delta_scan_noalloc (the scan with its scratch in the library's own
per-GPU device array, for callers that cannot allocate) against
clef_delta_scan with a caller workspace: bit-identical outputs, captured and
final states on two calls in a row, the second smaller, in both precision
profiles, with the device's free memory unchanged across each call; shapes whose workspace exceeds the array are rejected before any
launch.  Every call goes through the C ABI."""
import ctypes as C

import pytest
import torch

gpu = pytest.mark.gpu


@pytest.fixture(scope="module")
def clef():
    import clef_hip
    clef_hip.lib()
    return clef_hip


def _inputs(seed, T, Hk, Hv, dk, dv, dtype):
    import workloads
    return workloads.scan_inputs(seed, T, Hk, Hv, dk, dv, dtype=dtype)


def _outputs(args):
    T, Hv, dk, dv, capture, out_dtype = args[7], args[9], args[10], args[11], args[6], args[13]
    return (torch.empty((T, Hv, dv), dtype=out_dtype, device="cuda"),
            torch.empty((Hv, dk, dv), device="cuda") if capture else None,
            torch.empty((Hv, dk, dv), device="cuda"))


def _call(clef, fn, args, ws=None, outs=None):
    q, k, v, g, beta, init, capture, T, Hk, Hv, dk, dv, precision, out_dtype = args
    out, cap, fin = outs if outs is not None else _outputs(args)
    common = (clef._ptr(q), clef._ptr(k), clef._ptr(v), q.stride(0), v.stride(0), clef._dt(q), clef._ptr(g),
              clef._ptr(beta), g.stride(0), clef._dt(g), T, Hk, Hv, dk, dv, 64, precision, clef._ptr(init),
              capture, clef._ptr(out), Hv * dv, clef._dt(out), clef._ptr(cap), clef._ptr(fin))
    if fn == "clef_delta_scan":
        rc = clef.lib().clef_delta_scan(*common, clef._ptr(ws), ws.numel(), clef._stream())
    else:
        rc = clef.lib().clef_delta_scan_noalloc(*common, clef._stream())
    clef._check(rc)
    return out, cap, fin


CASES = [  # (T, Hk, Hv, dk, dv, capture, in dtype, out dtype): the second of each pair is smaller
    (4096, 16, 32, 128, 128, 2048, torch.float16, torch.float32),
    (300, 2, 4, 64, 48, 65, torch.float32, torch.float16),
]


@gpu
@pytest.mark.parametrize("precision", ["mixed", "strict"])
def test_noalloc_scan_equals_workspace_scan(clef, precision):
    prec = clef.STRICT if precision == "strict" else clef.MIXED
    for i, (T, Hk, Hv, dk, dv, capture, dt_in, dt_out) in enumerate(CASES):
        if precision == "strict" and T == 4096:
            T, capture = 2048, 1024  # the strict workspace of 4096 tokens is above the array
        print(f"noalloc {precision}: call {i} T={T} Hk={Hk} Hv={Hv} dk={dk} dv={dv}", flush=True)
        q, k, v, g, beta = _inputs(20 + i, T, Hk, Hv, dk, dv, dt_in)
        init = 0.1 * torch.randn((Hv, dk, dv), generator=torch.Generator(device="cuda").manual_seed(i),
                                 device="cuda")
        args = (q, k, v, g, beta, init, capture, T, Hk, Hv, dk, dv, prec, dt_out)
        n = clef.lib().clef_delta_scan_workspace(T, Hk, Hv, dk, dv, 64, prec)
        assert 0 < n <= 96 << 20
        buf = torch.empty(n + 256, dtype=torch.uint8, device="cuda")
        off = (-buf.data_ptr()) % 256
        ref = _call(clef, "clef_delta_scan", args, buf[off:off + n])
        got = _call(clef, "clef_delta_scan_noalloc", args)
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a, b)
        # the entry point's defining property: a further call, outputs
        # allocated beforehand, leaves the device's free memory unchanged
        outs = _outputs(args)
        torch.cuda.synchronize()
        free_before = torch.cuda.mem_get_info()[0]
        again = _call(clef, "clef_delta_scan_noalloc", args, outs=outs)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free_before
        for a, b in zip(again, ref):
            assert torch.equal(a, b)


@gpu
def test_noalloc_scan_rejects_shapes_above_the_array(clef):
    """The strict workspace of the full layer shape (99 MiB) exceeds the
    96 MiB array: refused before any launch, and the next call still works."""
    T, Hk, Hv, dk, dv = 4096, 16, 32, 128, 128
    assert clef.lib().clef_delta_scan_workspace(T, Hk, Hv, dk, dv, 64, clef.STRICT) > 96 << 20
    q, k, v, g, beta = _inputs(5, T, Hk, Hv, dk, dv, torch.float16)
    with pytest.raises(clef.ClefError, match="SCRATCH"):
        _call(clef, "clef_delta_scan_noalloc", (q, k, v, g, beta, None, 0, T, Hk, Hv, dk, dv, clef.STRICT,
                                                torch.float32))
    q, k, v, g, beta = _inputs(6, 100, 1, 2, 32, 32, torch.float32)
    args = (q, k, v, g, beta, None, 0, 100, 1, 2, 32, 32, clef.STRICT, torch.float32)
    n = clef.lib().clef_delta_scan_workspace(100, 1, 2, 32, 32, 64, clef.STRICT)
    buf = torch.empty(n + 256, dtype=torch.uint8, device="cuda")
    off = (-buf.data_ptr()) % 256
    for a, b in zip(_call(clef, "clef_delta_scan_noalloc", args), _call(clef, "clef_delta_scan", args,
                                                                       buf[off:off + n])):
        assert a is None and b is None or torch.equal(a, b)
