"""Python binding of libclef_hip.so (the C ABI in include/clef_hip.h).

Device memory and streams come from PyTorch; every call goes through the C
ABI with raw device pointers.  There is no CPU fallback: if the library is
missing or a call fails, a ClefError is raised.
"""
from __future__ import annotations

import ctypes as C
import pathlib

import torch

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libclef_hip.so"

F32, F16 = 0, 1
STRICT, MIXED = 0, 1
EPI_STORE, EPI_RESIDUAL = 0, 1
_DT = {torch.float32: F32, torch.float16: F16}
_TORCH = {F32: torch.float32, F16: torch.float16}

_lib = None


class ClefError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"clef_hip error {code}: {message}")
        self.code = code


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ClefError(-100, f"{LIB_PATH} is not built; run __graft_entry__.build()")
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


# symbol -> (restype, argtypes); the list mirrors include/clef_hip.h
_i, _l, _p, _z, _f, _d = C.c_int, C.c_int64, C.c_void_p, C.c_size_t, C.c_float, C.c_double
SIGNATURES = {
    "clef_hip_last_error": (C.c_char_p, []),
    "clef_hip_abi_version": (_i, []),
    "clef_delta_scan_workspace": (_z, [_i] * 7),
    "clef_delta_scan": (_i, [_p, _p, _p, _l, _l, _i, _p, _p, _l, _i, _i, _i, _i, _i, _i, _i, _i,
                             _p, _i, _p, _l, _i, _p, _p, _p, _z, _p]),
    "clef_gemm": (_i, [_p, _l, _p, _l, _p, _l, _i, _i, _i, _i, _i, _i, _p]),
    "clef_gemm_swiglu": (_i, [_p, _l, _p, _p, _l, _p, _l, _i, _i, _i, _i, _p]),
    "clef_rms_norm": (_i, [_p, _l, _i, _p, _p, _l, _i, _i, _i, _f, _p]),
    "clef_conv_silu": (_i, [_p, _l, _i, _p, _i, _p, _i, _p, _l, _i, _i, _i, _p]),
    "clef_delta_gates": (_i, [_p, _l, _p, _l, _i, _p, _p, _p, _p, _i, _i, _p]),
    "clef_gated_rms_silu": (_i, [_p, _p, _l, _i, _p, _p, _i, _i, _i, _i, _f, _p]),
    "clef_qk_norm_rotary": (_i, [_p, _l, _i, _p, _p, _i, _i, _i, _i, _i, _d, _i, _i, _i, _f, _p]),
    "clef_head_major": (_i, [_p, _l, _i, _p, _i, _i, _i, _i, _i, _i, _p]),
    "clef_attention_gated": (_i, [_p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _l, _p, _l, _i, _p]),
    "clef_embed": (_i, [_p, _i, _p, _i, _i, _i, _p, _p]),
    "clef_head_logits": (_i, [_p, _i, _p, _i, _p, _p]),
}


def _declare(L):
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args


def exported_symbols():
    """Names from SIGNATURES that the loaded library exports."""
    L = lib()
    return [n for n in SIGNATURES if hasattr(L, n)]


def last_error() -> str:
    return lib().clef_hip_last_error().decode()


def _check(rc: int):
    if rc != 0:
        raise ClefError(rc, last_error())


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _dt(t):
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ClefError(-1, f"unsupported dtype {t.dtype}") from None


def _token_view(t, name, rows_last2):
    """Validates a [T, H, d] view with contiguous (H, d) and returns its token stride."""
    if t.dim() != 3:
        raise ClefError(-1, f"{name} must be [T, heads, width]")
    H, d = t.shape[1], t.shape[2]
    if t.stride(2) != 1 or t.stride(1) != d:
        raise ClefError(-1, f"{name} must have contiguous heads and features")
    if not t.is_cuda:
        raise ClefError(-1, f"{name} must be a device tensor")
    return t.stride(0)


class DeltaScan:
    """Gated-DeltaNet prefill scan (DeltaKernel, metal.rs:80-278, on gfx950).

    `precision`: "strict" (f32 MFMA, parity with the CPU F32 path) or
    "mixed" (f16 MFMA, f32 accumulation and state).
    """

    def __init__(self, key_dim: int, value_dim: int, precision: str = "strict", chunk: int = 64):
        if precision not in ("strict", "mixed"):
            raise ClefError(-1, "precision must be 'strict' or 'mixed'")
        self.key_dim, self.value_dim, self.chunk = key_dim, value_dim, chunk
        self.precision = STRICT if precision == "strict" else MIXED
        self._ws = None

    def workspace(self, T, Hk, Hv, device):
        n = lib().clef_delta_scan_workspace(T, Hk, Hv, self.key_dim, self.value_dim, self.chunk,
                                            self.precision)
        if n == 0:
            raise ClefError(-1, last_error())
        if self._ws is None or self._ws.numel() < n or self._ws.device != device:
            self._ws = torch.empty(n + 256, dtype=torch.uint8, device=device)
        off = (-self._ws.data_ptr()) % 256
        return self._ws[off:off + n]

    def prefill(self, q, k, v, g, beta, initial=None, capture=0, out_dtype=torch.float32,
                want_final=True, out=None):
        """Returns (out [T,Hv,dv], captured [Hv,dk,dv] or None, final [Hv,dk,dv] or None)."""
        T, Hk, dk = q.shape
        Hv, dv = v.shape[1], v.shape[2]
        if k.shape != q.shape or v.shape[0] != T or dk != self.key_dim or dv != self.value_dim:
            raise ClefError(-1, "DeltaNet tensor shapes")
        if g.shape != (T, Hv) or beta.shape != (T, Hv) or g.dtype != beta.dtype:
            raise ClefError(-1, "DeltaNet gate shapes")
        if g.stride(1) != 1 or beta.stride(1) != 1 or g.stride(0) != beta.stride(0):
            raise ClefError(-1, "g and beta must share a token stride with contiguous heads")
        if q.dtype != k.dtype or q.dtype != v.dtype or q.stride(0) != k.stride(0):
            raise ClefError(-1, "q, k, v must share a dtype; q and k a token stride")
        sqk = _token_view(q, "q", 2)
        _token_view(k, "k", 2)
        sv = _token_view(v, "v", 2)
        dev = q.device
        if out is None:
            out = torch.empty((T, Hv, dv), dtype=out_dtype, device=dev)
        so = _token_view(out, "out", 2)
        captured = torch.empty((Hv, dk, dv), dtype=torch.float32, device=dev) if capture else None
        final = torch.empty((Hv, dk, dv), dtype=torch.float32, device=dev) if want_final else None
        if initial is not None:
            if initial.shape != (Hv, dk, dv) or initial.dtype != torch.float32 or not initial.is_contiguous():
                raise ClefError(-1, "initial state must be contiguous f32 [Hv, dk, dv]")
        ws = self.workspace(T, Hk, Hv, dev)
        _check(lib().clef_delta_scan(
            _ptr(q), _ptr(k), _ptr(v), sqk, sv, _dt(q), _ptr(g), _ptr(beta), g.stride(0), _dt(g),
            T, Hk, Hv, dk, dv, self.chunk, self.precision, _ptr(initial), int(capture),
            _ptr(out), so, _dt(out), _ptr(captured), _ptr(final), _ptr(ws), ws.numel(), _stream()))
        return out, captured, final


def _rows(t, name):
    if t.dim() != 2 or t.stride(1) != 1 or not t.is_cuda:
        raise ClefError(-1, f"{name} must be a row-major 2-D device tensor")
    return t.stride(0)


def gemm(x, w, out=None, out_dtype=None, residual=None):
    """y = x . w^T (GemmKernel::forward, neural.rs:50-55).

    x [M,K], w [N,K] share a dtype (f16: f16 MFMA; f32: f32 MFMA), f32
    accumulation.  With `residual` (an f32 [M,N] tensor) the rounded product
    is added into it in place and `residual` is returned.
    """
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K or w.dtype != x.dtype:
        raise ClefError(-1, "GEMM operand shapes or dtypes")
    out_dtype = out_dtype or x.dtype
    if residual is not None:
        if residual.dtype != torch.float32 or residual.shape != (M, N):
            raise ClefError(-1, "residual must be f32 [M, N]")
        y, epi, dto = residual, EPI_RESIDUAL, _DT[out_dtype]
    else:
        y = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=x.device)
        epi, dto = EPI_STORE, _dt(y)
    _check(lib().clef_gemm(_ptr(x), _rows(x, "x"), _ptr(w), _rows(w, "w"), _ptr(y), _rows(y, "y"),
                           M, N, K, _dt(x), dto, epi, _stream()))
    return y


def gemm_swiglu(x, wg, wu, out=None):
    """silu(x wg^T) * (x wu^T) (GemmKernel::gated, neural.rs:56-58)."""
    M, K = x.shape
    N = wg.shape[0]
    if wg.shape != (N, K) or wu.shape != (N, K) or wg.stride(0) != wu.stride(0):
        raise ClefError(-1, "gated projection weight dimensions")
    y = out if out is not None else torch.empty((M, N), dtype=x.dtype, device=x.device)
    _check(lib().clef_gemm_swiglu(_ptr(x), _rows(x, "x"), _ptr(wg), _ptr(wu), _rows(wg, "wg"),
                                  _ptr(y), _rows(y, "y"), M, N, K, _dt(x), _stream()))
    return y
