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
    "clef_delta_scan_noalloc": (_i, [_p, _p, _p, _l, _l, _i, _p, _p, _l, _i, _i, _i, _i, _i, _i, _i, _i,
                                     _p, _i, _p, _l, _i, _p, _p, _p]),
    "clef_delta_scan_varlen_workspace": (_z, [_i] * 8),
    "clef_ragged_plan": (_i, [_p, _i, _i, _i, _p, _p, _z]),
    "clef_delta_scan_varlen": (_i, [_p, _p, _p, _l, _l, _i, _p, _p, _l, _i, _p, _i, _i, _i, _i, _i, _i, _i, _i,
                                    _p, _l, _p, _l, _i, _p, _p, _z, _p]),
    "clef_silu_mul": (_i, [_p, _p, _p, _l, _i, _p]),
    "clef_gemm": (_i, [_p, _l, _p, _l, _p, _l, _i, _i, _i, _i, _i, _i, _p]),
    "clef_gemm_swiglu": (_i, [_p, _l, _p, _p, _l, _p, _l, _i, _i, _i, _i, _p]),
    "clef_rms_norm": (_i, [_p, _l, _i, _p, _p, _l, _i, _i, _i, _f, _p]),
    "clef_conv_silu": (_i, [_p, _l, _i, _p, _i, _p, _i, _p, _l, _i, _i, _i, _p]),
    "clef_delta_gates": (_i, [_p, _l, _p, _l, _i, _p, _p, _p, _p, _i, _i, _p]),
    "clef_delta_gates_pack_bytes": (_z, [_i, _i]),
    "clef_delta_gates_pack": (_i, [_p, _l, _i, _i, _i, _p, _p]),
    "clef_delta_gates_proj": (_i, [_p, _l, _p, _i, _i, _p, _p, _p, _p, _i, _i, _p]),
    "clef_attention_varlen_workspace": (_z, [_i, _i]),
    "clef_attention_gated_varlen": (_i, [_p, _l, _p, _l, _p, _l, _p, _i, _i, _p, _l, _p, _l, _i, _i, _i, _i, _i,
                                         _p, _l, _l, _p, _l, _p, _z, _p]),
    "clef_conv_silu_varlen": (_i, [_p, _l, _i, _p, _i, _l, _p, _i, _p, _i, _p, _l, _i, _i, _i, _p]),
    "clef_qk_norm_rotary_varlen": (_i, [_p, _l, _l, _i, _p, _p, _l, _i, _i, _i, _i, _i, _d, _i, _p, _i, _i, _f,
                                        _p]),
    "clef_gated_rms_silu": (_i, [_p, _i, _p, _l, _i, _p, _p, _i, _i, _i, _i, _f, _p]),
    "clef_qk_norm_rotary": (_i, [_p, _l, _l, _i, _p, _p, _l, _i, _i, _i, _i, _i, _d, _i, _i, _f, _p]),
    "clef_values_transposed": (_i, [_p, _l, _i, _p, _l, _i, _i, _i, _i, _i, _p]),
    "clef_attention_gated": (_i, [_p, _l, _p, _l, _p, _l, _i, _i, _i, _i, _i, _i, _p, _l, _l, _p, _l,
                                  _p]),
    "clef_attention_gated_qnorm": (_i, [_p, _l, _l, _p, _f, _p, _p, _l, _p, _l, _i, _i, _i, _i, _i, _p, _l, _l,
                                        _p, _l, _p]),
    "clef_rotary_table": (_i, [_i, _i, _d, _i, _p, _p]),
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

    def prefill_varlen(self, q, k, v, g, beta, cu_seqlens, initial=None, out_dtype=torch.float32,
                       want_final=True, out=None):
        """Ragged batch: tokens cu_seqlens[s]..cu_seqlens[s+1]-1 form sequence s.

        cu_seqlens: int32 device tensor [nseq + 1].  initial: None, one shared
        [Hv, dk, dv] state, or [nseq, Hv, dk, dv] per-sequence states (f32).
        Returns (out [T, Hv, dv], final [nseq, Hv, dk, dv] or None).
        """
        T, Hk, dk = q.shape
        Hv, dv = v.shape[1], v.shape[2]
        nseq = cu_seqlens.numel() - 1
        if k.shape != q.shape or v.shape[0] != T or dk != self.key_dim or dv != self.value_dim:
            raise ClefError(-1, "DeltaNet tensor shapes")
        if g.shape != (T, Hv) or beta.shape != (T, Hv) or g.dtype != beta.dtype or g.stride(0) != beta.stride(0):
            raise ClefError(-1, "DeltaNet gate shapes")
        if cu_seqlens.dtype != torch.int32 or not cu_seqlens.is_cuda or not cu_seqlens.is_contiguous():
            raise ClefError(-1, "cu_seqlens must be a contiguous int32 device tensor")
        sqk = _token_view(q, "q", 2)
        _token_view(k, "k", 2)
        sv = _token_view(v, "v", 2)
        dev = q.device
        if out is None:
            out = torch.empty((T, Hv, dv), dtype=out_dtype, device=dev)
        so = _token_view(out, "out", 2)
        stride = 0
        if initial is not None:
            if initial.dtype != torch.float32 or not initial.is_contiguous():
                raise ClefError(-1, "initial states must be contiguous f32")
            if initial.shape == (nseq, Hv, dk, dv):
                stride = Hv * dk * dv
            elif initial.shape != (Hv, dk, dv):
                raise ClefError(-1, "initial state must be [Hv, dk, dv] or [nseq, Hv, dk, dv]")
        final = torch.empty((nseq, Hv, dk, dv), dtype=torch.float32, device=dev) if want_final else None
        n = lib().clef_delta_scan_varlen_workspace(T, nseq, Hk, Hv, dk, dv, self.chunk, self.precision)
        if n == 0:
            raise ClefError(-1, last_error())
        ws = torch.empty(n + 256, dtype=torch.uint8, device=dev)
        off = (-ws.data_ptr()) % 256
        ws = ws[off:off + n]
        _check(lib().clef_delta_scan_varlen(
            _ptr(q), _ptr(k), _ptr(v), sqk, sv, _dt(q), _ptr(g), _ptr(beta), g.stride(0), _dt(g),
            _ptr(cu_seqlens), nseq, T, Hk, Hv, dk, dv, self.chunk, self.precision, _ptr(initial), stride,
            _ptr(out), so, _dt(out), _ptr(final), _ptr(ws), ws.numel(), _stream()))
        return out, final


def ragged_plan(cu_seqlens, T, unit):
    """Host evaluation of a ragged batch's launch tables (clef_ragged_plan):
    returns (spans [nseq + 1], units [n, 2]) as numpy int32 arrays."""
    import numpy as np
    cu = np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int32))
    nseq = int(cu.shape[0]) - 1
    spans = np.zeros(nseq + 1, np.int32)
    cap = (T + unit - 1) // unit + nseq
    table = np.zeros((cap, 2), np.int32)
    n = lib().clef_ragged_plan(cu.ctypes.data, nseq, T, unit, spans.ctypes.data, table.ctypes.data, cap)
    if n < 0:
        raise ClefError(n, last_error())
    return spans, table[:n].copy()


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


# ---------------------------------------------------------------------------
# Pointwise pieces (thin wrappers used by the parity tests)
# ---------------------------------------------------------------------------
def rms_norm(x, w, eps=1e-6, out_dtype=None):
    rows, width = x.shape
    y = torch.empty((rows, width), dtype=out_dtype or x.dtype, device=x.device)
    _check(lib().clef_rms_norm(_ptr(x), _rows(x, "x"), _dt(x), _ptr(w), _ptr(y), width, _dt(y),
                               rows, width, float(eps), _stream()))
    return y


def silu_mul(gate, up):
    """silu(gate) * up elementwise (clef_silu_mul): the unfused SwiGLU product."""
    if gate.shape != up.shape or gate.dtype != up.dtype or not gate.is_contiguous() or not up.is_contiguous():
        raise ClefError(-1, "gate and up must be contiguous tensors of one shape and dtype")
    y = torch.empty_like(gate)
    _check(lib().clef_silu_mul(_ptr(gate), _ptr(up), _ptr(y), gate.numel(), _dt(gate), _stream()))
    return y


def conv_silu(x, w, history=None, out_dtype=torch.float32):
    T, W = x.shape
    taps = w.reshape(W, -1).shape[1]
    y = torch.empty((T, W), dtype=out_dtype, device=x.device)
    hist_rows = 0 if history is None else history.shape[0]
    _check(lib().clef_conv_silu(_ptr(x), _rows(x, "x"), _dt(x), _ptr(history), hist_rows,
                                _ptr(w.reshape(W, taps).contiguous()), taps, _ptr(y), W, _dt(y), T, W,
                                _stream()))
    return y


def conv_silu_varlen(x, w, cu_seqlens, history=None, out_dtype=torch.float32):
    """Ragged batch: history None, one [rows, W] history shared by every sequence,
    or [nseq, rows, W] per sequence (f32)."""
    T, W = x.shape
    taps = w.reshape(W, -1).shape[1]
    nseq = cu_seqlens.numel() - 1
    y = torch.empty((T, W), dtype=out_dtype, device=x.device)
    rows, stride = 0, 0
    if history is not None:
        rows = history.shape[-2]
        stride = rows * W if history.dim() == 3 else 0
    _check(lib().clef_conv_silu_varlen(_ptr(x), _rows(x, "x"), _dt(x), _ptr(history), rows, stride,
                                       _ptr(cu_seqlens), nseq, _ptr(w.reshape(W, taps).contiguous()), taps,
                                       _ptr(y), W, _dt(y), T, W, _stream()))
    return y


def delta_gates(a, b, dt, a_log):
    T, Hv = a.shape
    g = torch.empty((T, Hv), dtype=torch.float32, device=a.device)
    beta = torch.empty_like(g)
    _check(lib().clef_delta_gates(_ptr(a), _rows(a, "a"), _ptr(b), _rows(b, "b"), _dt(a), _ptr(dt),
                                  _ptr(a_log), _ptr(g), _ptr(beta), T, Hv, _stream()))
    return g, beta


def delta_gates_pack(w_ab):
    """w_ab [2 Hv, K] f16 in the fragment order clef_delta_gates_proj reads."""
    K = w_ab.shape[1]
    Hv = w_ab.shape[0] // 2
    n = lib().clef_delta_gates_pack_bytes(K, Hv)
    if n == 0:
        raise ClefError(-1, "gates projection dimensions")
    packed = torch.empty(n, dtype=torch.uint8, device=w_ab.device)
    _check(lib().clef_delta_gates_pack(_ptr(w_ab), _rows(w_ab, "w_ab"), K, Hv, _dt(w_ab), _ptr(packed), _stream()))
    return packed


def delta_gates_proj(x, packed, Hv, dt, a_log):
    """[a | b] = x w_ab^T (f16, each rounded to f16) and the gates in one launch."""
    T, K = x.shape
    g = torch.empty((T, Hv), dtype=torch.float32, device=x.device)
    beta = torch.empty_like(g)
    _check(lib().clef_delta_gates_proj(_ptr(x), _rows(x, "x"), _ptr(packed), K, _dt(x), _ptr(dt), _ptr(a_log),
                                       _ptr(g), _ptr(beta), T, Hv, _stream()))
    return g, beta


def gated_rms_silu(o, z, w, eps=1e-6, out_dtype=torch.float32):
    T, Hv, width = o.shape
    y = torch.empty((T, Hv * width), dtype=out_dtype, device=o.device)
    _check(lib().clef_gated_rms_silu(_ptr(o), _dt(o), _ptr(z), z.stride(0), _dt(z), _ptr(w), _ptr(y), _dt(y),
                                     T, Hv, width, float(eps), _stream()))
    return y


def qk_norm_rotary(x, heads, d, w, rot_dim, theta, pos0=0, head_stride=None, eps=1e-6,
                   out=None, dst_offset=0, out_dtype=None):
    T = x.shape[0]
    hs = head_stride or d
    if out is None:
        out = torch.empty((heads, T + dst_offset, d), dtype=out_dtype or x.dtype, device=x.device)
    _check(lib().clef_qk_norm_rotary(_ptr(x), x.stride(0), hs, _dt(x), _ptr(w), _ptr(out), out.shape[1],
                                     _dt(out), T, heads, d, rot_dim, float(theta), pos0, dst_offset,
                                     float(eps), _stream()))
    return out


def qk_norm_rotary_varlen(x, heads, d, w, rot_dim, theta, cu_seqlens, pos0=0, head_stride=None, eps=1e-6,
                          out_dtype=None):
    T = x.shape[0]
    hs = head_stride or d
    out = torch.empty((heads, T, d), dtype=out_dtype or x.dtype, device=x.device)
    _check(lib().clef_qk_norm_rotary_varlen(_ptr(x), x.stride(0), hs, _dt(x), _ptr(w), _ptr(out), T, _dt(out), T,
                                            heads, d, rot_dim, float(theta), pos0, _ptr(cu_seqlens),
                                            cu_seqlens.numel() - 1, 0, float(eps), _stream()))
    return out


def values_transposed(x, heads, d, ld_tok=None, out=None, dst_offset=0, out_dtype=None):
    T = x.shape[0]
    if out is None:
        ld_tok = ld_tok or max(64, ((T + dst_offset + 63) // 64) * 64)
        out = torch.zeros((heads, d, ld_tok), dtype=out_dtype or x.dtype, device=x.device)
    _check(lib().clef_values_transposed(_ptr(x), x.stride(0), _dt(x), _ptr(out), out.shape[2], _dt(out),
                                        T, heads, d, dst_offset, _stream()))
    return out


def attention_gated(q, k, vt, gate, kn=None):
    """q [heads, qn, d], k [kvh, kn, d], vt [kvh, d, ldv]; gate [qn, heads, *] view."""
    heads, qn, d = q.shape
    kvh, kn_, _ = k.shape
    kn = kn or kn_
    y = torch.empty((qn, heads * d), dtype=q.dtype, device=q.device)
    _check(lib().clef_attention_gated(_ptr(q), qn, _ptr(k), kn_, _ptr(vt), vt.shape[2], _dt(q), heads, kvh,
                                      qn, kn, d, _ptr(gate), gate.stride(0), gate.stride(1), _ptr(y),
                                      heads * d, _stream()))
    return y


def rotary_table(T, rot_dim, theta, pos0=0, device="cuda"):
    """(cos, sin) of positions pos0 .. pos0 + T - 1 per rotary frequency: [T, rot_dim // 2, 2] f32."""
    out = torch.empty((T, rot_dim // 2, 2), dtype=torch.float32, device=device)
    _check(lib().clef_rotary_table(T, rot_dim, float(theta), pos0, _ptr(out), _stream()))
    return out


def attention_gated_qnorm(x, heads, w, eps, rot_tab, k, vt, gate, head_stride, kn=None):
    """attention_gated of qk_norm_rotary(x) (rotary width 64, d = 256) with the query norm and
    rotary inside the attention core: x [qn, *] raw query rows (head h at h * head_stride),
    w [256] norm weights, rot_tab from rotary_table for the queries' positions."""
    qn = x.shape[0]
    kvh, kn_, d = k.shape
    kn = kn or kn_
    y = torch.empty((qn, heads * d), dtype=x.dtype, device=x.device)
    _check(lib().clef_attention_gated_qnorm(_ptr(x), x.stride(0), head_stride, _ptr(w), float(eps), _ptr(rot_tab),
                                            _ptr(k), kn_, _ptr(vt), vt.shape[2], heads, kvh, qn, kn, d, _ptr(gate),
                                            gate.stride(0), gate.stride(1), _ptr(y), heads * d, _stream()))
    return y


def attention_gated_varlen(q, k, vt, gate, cu_seqlens, prefix_k=None, prefix_vt=None):
    """Ragged batch: q [heads, T, d], k [kvh, T, d], vt [kvh, d, ldv] packed by
    cu_seqlens (int32 device); optional shared prefix keys [kvh, np, d] and
    values^T [kvh, d, ldpv] visible to every query."""
    heads, T, d = q.shape
    kvh = k.shape[0]
    nseq = cu_seqlens.numel() - 1
    y = torch.empty((T, heads * d), dtype=q.dtype, device=q.device)
    np_ = 0 if prefix_k is None else prefix_k.shape[1]
    n = lib().clef_attention_varlen_workspace(T, nseq)
    ws = torch.empty(n + 256, dtype=torch.uint8, device=q.device)
    off = (-ws.data_ptr()) % 256
    ws = ws[off:off + n]
    _check(lib().clef_attention_gated_varlen(
        _ptr(q), T, _ptr(k), k.shape[1], _ptr(vt), vt.shape[2], _ptr(cu_seqlens), nseq, T,
        _ptr(prefix_k), np_, _ptr(prefix_vt), 0 if prefix_vt is None else prefix_vt.shape[2], np_, _dt(q),
        heads, kvh, d, _ptr(gate), gate.stride(0), gate.stride(1), _ptr(y), heads * d, _ptr(ws), ws.numel(),
        _stream()))
    return y


# ---------------------------------------------------------------------------
# Hybrid backbone (Backbone::{load, prefill}, qwen.rs:193-426)
# ---------------------------------------------------------------------------
class BackboneConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "hidden", "intermediate", "vocab", "heads", "kv_heads", "head_dim", "rotary_dim",
        "lin_k_heads", "lin_v_heads", "lin_dk", "lin_dv", "conv_taps", "n_layers")] + [
        ("eps", C.c_float), ("rope_theta", C.c_double), ("profile", C.c_int),
        ("scan_precision", C.c_int), ("max_tokens", C.c_int)]


_LW = ("input_norm", "post_norm", "gate", "up", "down", "qkv", "z", "a", "b", "out", "conv", "dt",
       "a_log", "norm", "q", "k", "v", "o", "q_norm", "k_norm")


class LayerWeights(C.Structure):
    _fields_ = [("kind", C.c_int)] + [(n, C.c_void_p) for n in _LW]


class Control(C.Structure):
    _fields_ = [("cancel", C.POINTER(C.c_int32)), ("deadline", C.c_double)]


SIGNATURES.update({
    "clef_backbone_create": (_i, [C.POINTER(BackboneConfig), C.POINTER(LayerWeights), _p, _p,
                                  C.POINTER(C.c_void_p)]),
    "clef_backbone_destroy": (None, [_p]),
    "clef_backbone_workspace": (_z, [_p, _i, _i]),
    "clef_backbone_prefix_bytes": (_z, [_p, _i]),
    "clef_backbone_prefill": (_i, [_p, C.POINTER(C.c_int32), _i, _p, _i, _z, _i, _p, _z, _p, _p, _z, _p]),
    "clef_backbone_varlen_workspace": (_z, [_p, _i, _i, _i]),
    "clef_backbone_prefill_varlen": (_i, [_p, C.POINTER(C.c_int32), C.POINTER(C.c_int32), _i, _p, _i, _z, _p, _p,
                                          _z, _p]),
    "clef_backbone_set_control": (_i, [_p, C.POINTER(Control)]),
    "clef_monotonic_seconds": (_d, []),
    "clef_backbone_enable_timing": (_i, [_p, _i]),
    "clef_backbone_timings": (_i, [_p, C.POINTER(C.c_double), C.POINTER(C.c_int), C.POINTER(C.c_double),
                                   C.POINTER(C.c_double)]),
})

CATEGORIES = ("gemm", "scan", "attention", "conv", "norm", "other")
CANCELLED, DEADLINE_EXCEEDED = -20, -21


def monotonic_seconds() -> float:
    return lib().clef_monotonic_seconds()


class PrefixState:
    """Device copy of a captured prefix (PrefixState, qwen.rs:153-191)."""

    def __init__(self, buffer, tokens):
        self.buffer, self.tokens = buffer, tokens

    def bytes(self):
        return self.buffer.numel()


class Backbone:
    """Hybrid backbone over checkpoint tensors named as the reference names them.

    `weights` maps "model.language_model.*" names to device tensors; matrices
    are cast to the profile dtype (f16 for "mixed", f32 for "f32") and vectors
    to f32 here, once.
    """

    P = "model.language_model."

    def __init__(self, config: dict, weights: dict, profile: str = "f32", scan_precision=None,
                 max_tokens: int = 4096, device="cuda"):
        if profile not in ("f32", "mixed"):
            raise ClefError(-1, "profile must be 'f32' or 'mixed'")
        self.profile = profile
        self.dtype = torch.float32 if profile == "f32" else torch.float16
        if scan_precision is None:
            scan_precision = "strict" if profile == "f32" else "mixed"
        rp = config["rope_parameters"]
        c = BackboneConfig()
        c.hidden, c.intermediate, c.vocab = config["hidden_size"], config["intermediate_size"], config["vocab_size"]
        c.heads, c.kv_heads, c.head_dim = (config["num_attention_heads"], config["num_key_value_heads"],
                                           config["head_dim"])
        c.rotary_dim = int(config["head_dim"] * rp["partial_rotary_factor"])
        c.lin_k_heads, c.lin_v_heads = config["linear_num_key_heads"], config["linear_num_value_heads"]
        c.lin_dk, c.lin_dv = config["linear_key_head_dim"], config["linear_value_head_dim"]
        c.conv_taps = config["linear_conv_kernel_dim"]
        c.n_layers = len(config["layer_types"])
        c.eps, c.rope_theta = config["rms_norm_eps"], rp["rope_theta"]
        c.profile = 0 if profile == "f32" else 1
        c.scan_precision = STRICT if scan_precision == "strict" else MIXED
        c.max_tokens = max_tokens
        self.c, self.config = c, config
        self._keep = []
        P = self.P

        def mat(name):
            t = weights[name].to(device=device, dtype=self.dtype).contiguous()
            self._keep.append(t)
            return t.data_ptr()

        def vec(name):
            t = weights[name].to(device=device, dtype=torch.float32).contiguous()
            self._keep.append(t)
            return t.data_ptr()

        layers = (LayerWeights * c.n_layers)()
        for i, kind in enumerate(config["layer_types"]):
            L, p = layers[i], f"{P}layers.{i}."
            L.input_norm = vec(p + "input_layernorm.weight")
            L.post_norm = vec(p + "post_attention_layernorm.weight")
            L.gate, L.up, L.down = (mat(p + f"mlp.{n}_proj.weight") for n in ("gate", "up", "down"))
            if kind == "full_attention":
                L.kind = 1
                a = p + "self_attn."
                L.q, L.k, L.v, L.o = (mat(a + f"{n}_proj.weight") for n in "qkvo")
                L.q_norm, L.k_norm = vec(a + "q_norm.weight"), vec(a + "k_norm.weight")
            else:
                L.kind = 0
                a = p + "linear_attn."
                L.qkv, L.z = mat(a + "in_proj_qkv.weight"), mat(a + "in_proj_z.weight")
                L.a, L.b = mat(a + "in_proj_a.weight"), mat(a + "in_proj_b.weight")
                L.out = mat(a + "out_proj.weight")
                L.conv, L.dt, L.a_log = vec(a + "conv1d.weight"), vec(a + "dt_bias"), vec(a + "A_log")
                L.norm = vec(a + "norm.weight")
        emb = mat(P + "embed_tokens.weight")
        fin = vec(P + "norm.weight")
        handle = C.c_void_p()
        L = lib()
        _declare(L)
        _check(L.clef_backbone_create(C.byref(c), layers, emb, fin, C.byref(handle)))
        self._h = handle
        self._ws = None

    def __del__(self):
        try:
            if getattr(self, "_h", None):
                lib().clef_backbone_destroy(self._h)
                self._h = None
        except Exception:
            pass

    def _workspace(self, T, prefix, device):
        n = lib().clef_backbone_workspace(self._h, T, prefix)
        if n == 0:
            raise ClefError(-1, "backbone workspace")
        if self._ws is None or self._ws.numel() < n:
            self._ws = torch.empty(n, dtype=torch.uint8, device=device)
        return self._ws

    def enable_timing(self, enable=True):
        _check(lib().clef_backbone_enable_timing(self._h, int(enable)))

    def set_control(self, cancel=None, deadline=0.0):
        """Cooperative cancellation / deadline (Control, models/mod.rs:45-59).
        cancel: a ctypes.c_int32 flag another thread may set (kept referenced
        here); deadline: absolute seconds on monotonic_seconds()'s clock, 0 =
        none.  set_control() with no arguments clears it."""
        self._cancel = cancel
        if cancel is None and not deadline:
            _check(lib().clef_backbone_set_control(self._h, None))
            return
        c = Control(C.cast(C.pointer(cancel), C.POINTER(C.c_int32)) if cancel is not None else None,
                    float(deadline))
        _check(lib().clef_backbone_set_control(self._h, C.byref(c)))

    def timings(self):
        """Per-category {ms, launches, flops, bytes} of the prefills since the last call."""
        n = len(CATEGORIES)
        ms, cnt = (C.c_double * n)(), (C.c_int * n)()
        fl, by = (C.c_double * n)(), (C.c_double * n)()
        _check(lib().clef_backbone_timings(self._h, ms, cnt, fl, by))
        return {name: {"ms": ms[i], "launches": cnt[i], "flops": fl[i], "bytes": by[i]}
                for i, name in enumerate(CATEGORIES)}

    @classmethod
    def from_safetensors(cls, config: dict, paths, profile: str = "f32", **kw):
        """Backbone whose weights come from safetensors shards (load_backbone_weights)."""
        return cls(config, load_backbone_weights(config, paths, profile), profile=profile, **kw)

    def prefix_bytes(self, tokens):
        return lib().clef_backbone_prefix_bytes(self._h, tokens)

    def prefill(self, ids, initial: PrefixState = None, capture: int = 0, hidden=None):
        """Returns (hidden f32 [(prefix + T), H], PrefixState or None)."""
        import numpy as np
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
        T = int(ids.shape[0])
        prefix = initial.tokens if initial is not None else 0
        dev = torch.device("cuda", torch.cuda.current_device())
        if hidden is None:
            hidden = torch.empty((prefix + T, self.c.hidden), dtype=torch.float32, device=dev)
        saved = None
        if capture:
            nb = self.prefix_bytes(capture)
            if nb == 0:
                raise ClefError(-1, "prefill boundary or vocabulary")
            saved = PrefixState(torch.empty(nb, dtype=torch.uint8, device=dev), capture)
        ws = self._workspace(T, prefix, dev)
        _check(lib().clef_backbone_prefill(
            self._h, ids.ctypes.data_as(C.POINTER(C.c_int32)), T,
            _ptr(initial.buffer) if initial is not None else None, prefix,
            initial.bytes() if initial is not None else 0, int(capture),
            _ptr(saved.buffer) if saved is not None else None, saved.bytes() if saved is not None else 0,
            _ptr(hidden), _ptr(ws), ws.numel(), _stream()))
        return hidden, saved

    def prefill_varlen(self, ids, cu_seqlens, initial: PrefixState = None, hidden=None):
        """Ragged batch of requests resumed from one shared prefix: ids packed
        by cu_seqlens (host int arrays).  Returns hidden f32 [T, H] (no prefix
        rows); sequence s's rows equal prefill(ids[cu[s]:cu[s+1]], initial)."""
        import numpy as np
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
        cu = np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int32))
        T, nseq = int(ids.shape[0]), int(cu.shape[0]) - 1
        prefix = initial.tokens if initial is not None else 0
        dev = torch.device("cuda", torch.cuda.current_device())
        if hidden is None:
            hidden = torch.empty((T, self.c.hidden), dtype=torch.float32, device=dev)
        n = lib().clef_backbone_varlen_workspace(self._h, T, nseq, prefix)
        if n == 0:
            raise ClefError(-1, "prefill: ragged batch dimensions")
        if self._ws is None or self._ws.numel() < n:
            self._ws = torch.empty(n, dtype=torch.uint8, device=dev)
        _check(lib().clef_backbone_prefill_varlen(
            self._h, ids.ctypes.data_as(C.POINTER(C.c_int32)), cu.ctypes.data_as(C.POINTER(C.c_int32)), nseq,
            _ptr(initial.buffer) if initial is not None else None, prefix,
            initial.bytes() if initial is not None else 0, _ptr(hidden), _ptr(self._ws), self._ws.numel(),
            _stream()))
        return hidden


# ---------------------------------------------------------------------------
# Weights on disk (models/weights.rs:26-104)
# ---------------------------------------------------------------------------
SIGNATURES.update({
    "clef_st_open": (_i, [C.c_char_p, C.POINTER(_p)]),
    "clef_st_close": (None, [_p]),
    "clef_st_count": (_i, [_p]),
    "clef_st_info": (_i, [_p, _i, C.POINTER(C.c_char_p), C.POINTER(_i), C.POINTER(_i), C.POINTER(_l)]),
    "clef_st_find": (_i, [_p, C.c_char_p]),
    "clef_st_load": (_i, [_p, _i, _i, _p, _z, _p]),
})
_ST_NAMES = {0: "F32", 1: "F16", 2: "BF16"}


class SafeTensors:
    """A safetensors file opened and validated by the native reader."""

    def __init__(self, path):
        L = lib()
        _declare(L)
        h = _p()
        _check(L.clef_st_open(str(path).encode(), C.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            lib().clef_st_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self, i):
        name, dt, rank = C.c_char_p(), _i(), _i()
        shape = (_l * 8)()
        _check(lib().clef_st_info(self._h, i, C.byref(name), C.byref(dt), C.byref(rank), shape))
        return name.value.decode(), _ST_NAMES[dt.value], tuple(shape[d] for d in range(rank.value))

    def tensors(self):
        """{name: (dtype, shape)} of every tensor in the file."""
        out = {}
        for i in range(lib().clef_st_count(self._h)):
            name, dt, shape = self.info(i)
            out[name] = (dt, shape)
        return out

    def load(self, name, dtype=torch.float32, device=None):
        """The tensor on the device, converted there to f16 or f32."""
        i = lib().clef_st_find(self._h, name.encode())
        if i < 0:
            raise ClefError(-1, f"safetensors: no tensor {name}")
        _, _, shape = self.info(i)
        dev = device or torch.device("cuda", torch.cuda.current_device())
        t = torch.empty(shape, dtype=dtype, device=dev)
        _check(lib().clef_st_load(self._h, i, _DT[dtype], _ptr(t), t.numel() * t.element_size(), _stream()))
        return t


def backbone_tensor_specs(config: dict):
    """{checkpoint name: (shape, 'mat' | 'vec')} the hybrid backbone consumes
    (qwen.rs:193-310, 540-586 names and shapes)."""
    P = Backbone.P
    H, I = config["hidden_size"], config["intermediate_size"]
    specs = {P + "embed_tokens.weight": ((config["vocab_size"], H), "mat"), P + "norm.weight": ((H,), "vec")}
    key = config["linear_num_key_heads"] * config["linear_key_head_dim"]
    value = config["linear_num_value_heads"] * config["linear_value_head_dim"]
    hv, taps = config["linear_num_value_heads"], config["linear_conv_kernel_dim"]
    heads, kvh, d = config["num_attention_heads"], config["num_key_value_heads"], config["head_dim"]
    for i, kind in enumerate(config["layer_types"]):
        p = f"{P}layers.{i}."
        specs[p + "input_layernorm.weight"] = ((H,), "vec")
        specs[p + "post_attention_layernorm.weight"] = ((H,), "vec")
        specs[p + "mlp.gate_proj.weight"] = ((I, H), "mat")
        specs[p + "mlp.up_proj.weight"] = ((I, H), "mat")
        specs[p + "mlp.down_proj.weight"] = ((H, I), "mat")
        if kind == "full_attention":
            a = p + "self_attn."
            specs[a + "q_proj.weight"] = ((2 * heads * d, H), "mat")
            specs[a + "k_proj.weight"] = ((kvh * d, H), "mat")
            specs[a + "v_proj.weight"] = ((kvh * d, H), "mat")
            specs[a + "o_proj.weight"] = ((H, heads * d), "mat")
            specs[a + "q_norm.weight"] = ((d,), "vec")
            specs[a + "k_norm.weight"] = ((d,), "vec")
        else:
            a = p + "linear_attn."
            specs[a + "in_proj_qkv.weight"] = ((2 * key + value, H), "mat")
            specs[a + "in_proj_z.weight"] = ((value, H), "mat")
            specs[a + "in_proj_a.weight"] = ((hv, H), "mat")
            specs[a + "in_proj_b.weight"] = ((hv, H), "mat")
            specs[a + "out_proj.weight"] = ((H, value), "mat")
            specs[a + "conv1d.weight"] = ((2 * key + value, 1, taps), "vec")
            specs[a + "dt_bias"] = ((hv,), "vec")
            specs[a + "A_log"] = ((hv,), "vec")
            specs[a + "norm.weight"] = ((config["linear_value_head_dim"],), "vec")
    return specs


def load_backbone_weights(config: dict, paths, profile: str = "f32", device=None):
    """Backbone weights from safetensors shards, as Weights::load checks them
    (weights.rs:26-104): every required tensor present once with its shape,
    no unconsumed tensor under the language-model prefix (weights.rs:184-189;
    other namespaces, e.g. a vision tower, are skipped), matrices converted
    on the device to the profile's dtype and vectors to f32."""
    specs = backbone_tensor_specs(config)
    mat_dtype = torch.float32 if profile == "f32" else torch.float16
    out = {}
    for path in ([paths] if isinstance(paths, (str, bytes)) or hasattr(paths, "__fspath__") else paths):
        with SafeTensors(path) as st:
            for name, (_, shape) in st.tensors().items():
                if name not in specs:
                    if name.startswith(Backbone.P):
                        raise ClefError(-1, f"weights: unconsumed model tensor {name}")
                    continue
                want, kind = specs[name]
                if tuple(shape) != tuple(want) or name in out:
                    raise ClefError(-1, f"weights: tensor shape or duplicate {name}")
                out[name] = st.load(name, mat_dtype if kind == "mat" else torch.float32, device)
    missing = [n for n in specs if n not in out]
    if missing:
        raise ClefError(-1, f"weights: missing required tensor {missing[0]}")
    return out


def head_logits(x_row, w):
    """logits[j] = x . w[j] (f32), the pooled last-token head."""
    n, H = w.shape
    out = torch.empty(n, dtype=torch.float32, device=x_row.device)
    _check(lib().clef_head_logits(_ptr(x_row), H, _ptr(w), n, _ptr(out), _stream()))
    return out
