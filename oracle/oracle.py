"""ctypes binding of the CPU oracle (libclef_oracle.so).

TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module.  The product path (clef-rs_amd/) never imports or calls it.
"""
from __future__ import annotations

import ctypes as C
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libclef_oracle.so"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built (run `make -C oracle`)")
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


class OracleConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "hidden", "intermediate", "vocab", "heads", "kv_heads", "head_dim", "rotary_dim",
        "lin_k_heads", "lin_v_heads", "lin_dk", "lin_dv", "conv_taps", "n_layers")] + [
        ("eps", C.c_float), ("rope_theta", C.c_double)]


_FP = C.POINTER(C.c_float)
_LAYER_PTRS = ("input_norm", "post_norm", "gate", "up", "down", "qkv", "z", "a", "b", "out",
               "conv", "dt", "a_log", "norm", "q", "k", "v", "o", "q_norm", "k_norm")


class OracleLayer(C.Structure):
    _fields_ = [("kind", C.c_int)] + [(n, _FP) for n in _LAYER_PTRS]


class OracleBackbone(C.Structure):
    _fields_ = [("c", OracleConfig), ("embeddings", _FP), ("final_norm", _FP),
                ("layers", C.POINTER(OracleLayer)), ("mixed_f16", C.c_int)]


class OraclePrefix(C.Structure):
    _fields_ = [("tokens", C.c_int), ("hidden", _FP), ("recurrent", C.POINTER(_FP)),
                ("history", C.POINTER(_FP)), ("history_rows", C.POINTER(C.c_int)),
                ("key", C.POINTER(_FP)), ("value", C.POINTER(_FP))]


def _declare(L):
    i = C.c_int
    L.oracle_delta_recurrence.argtypes = [_f32p] * 5 + [i] * 4 + [C.c_void_p, i, _f32p, C.c_void_p, C.c_void_p]
    L.oracle_delta_recurrence.restype = i
    L.oracle_delta_scan.argtypes = [_f32p] * 5 + [i] * 5 + [C.c_void_p, i, _f32p, C.c_void_p, C.c_void_p]
    L.oracle_delta_scan.restype = i
    L.oracle_delta_recurrence_f64.argtypes = [_f64p] * 5 + [i] * 4 + [C.c_void_p, _f64p, C.c_void_p]
    L.oracle_delta_recurrence_f64.restype = i
    L.oracle_delta_chunked_f64.argtypes = [_f64p] * 5 + [i] * 5 + [C.c_void_p, _f64p, C.c_void_p]
    L.oracle_delta_chunked_f64.restype = i
    L.oracle_causal_conv.argtypes = [_f32p, i, i, _f32p, i, _f32p]
    L.oracle_rms.argtypes = [_f32p, i, i, _f32p, C.c_float, _f32p]
    L.oracle_linear.argtypes = [_f32p, i, i, _f32p, i, _f32p]
    L.oracle_attention.argtypes = [_f32p, _f32p, _f32p, i, i, i, i, i, i, _f32p]
    L.oracle_attention.restype = i
    L.oracle_rotary.argtypes = [_f32p, i, i, i, i, C.c_double, i]
    L.oracle_backbone_prefill.argtypes = [C.POINTER(OracleBackbone), C.POINTER(C.c_int), i,
                                          C.c_void_p, i, C.c_void_p, _f32p]
    L.oracle_backbone_prefill.restype = i
    L.oracle_set_threads.argtypes = [i]
    L.oracle_set_exact_dots.argtypes = [i]
    L.oracle_get_threads.restype = i
    L.oracle_f32_to_f16.argtypes = [C.c_float]
    L.oracle_f32_to_f16.restype = C.c_uint16
    L.oracle_f16_to_f32.argtypes = [C.c_uint16]
    L.oracle_f16_to_f32.restype = C.c_float


def _c32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def _c64(x):
    return np.ascontiguousarray(x, dtype=np.float64)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def set_threads(n: int):
    lib().oracle_set_threads(int(n))


class exact_dots:
    """Context in which the oracle accumulates its projection dot products
    in f64 (rounded to f32 once): a yardstick nearer the exact result."""

    def __enter__(self):
        lib().oracle_set_exact_dots(1)
        return self

    def __exit__(self, *exc):
        lib().oracle_set_exact_dots(0)


def threads() -> int:
    return lib().oracle_get_threads()


def delta_recurrence(q, k, v, g, beta, initial=None, capture=0):
    """Per-token recurrence on head-expanded q,k [T,H,dk]; returns (out, captured, final)."""
    q, k, v, g, beta = map(_c32, (q, k, v, g, beta))
    T, H, dk = q.shape
    dv = v.shape[2]
    out = np.empty((T, H, dv), np.float32)
    final = np.empty((H, dk, dv), np.float32)
    cap = np.empty((H, dk, dv), np.float32) if capture else None
    init = None if initial is None else _c32(initial)
    rc = lib().oracle_delta_recurrence(q, k, v, g, beta, T, H, dk, dv, _ptr(init), int(capture),
                                       out, _ptr(cap), _ptr(final))
    if rc:
        raise ValueError("oracle_delta_recurrence: invalid dimensions")
    return out, cap, final


def delta_scan(q, k, v, g, beta, initial=None, capture=0):
    """GQA scan: q,k [T,Hk,dk], v [T,Hv,dv], g,beta [T,Hv]; returns (out, captured, final)."""
    q, k, v, g, beta = map(_c32, (q, k, v, g, beta))
    T, Hk, dk = q.shape
    Hv, dv = v.shape[1], v.shape[2]
    out = np.empty((T, Hv, dv), np.float32)
    final = np.empty((Hv, dk, dv), np.float32)
    cap = np.empty((Hv, dk, dv), np.float32) if capture else None
    init = None if initial is None else _c32(initial)
    rc = lib().oracle_delta_scan(q, k, v, g, beta, T, Hk, Hv, dk, dv, _ptr(init), int(capture),
                                 out, _ptr(cap), _ptr(final))
    if rc:
        raise ValueError("oracle_delta_scan: invalid dimensions")
    return out, cap, final


def delta_recurrence_f64(q, k, v, g, beta, initial=None):
    q, k, v, g, beta = map(_c64, (q, k, v, g, beta))
    T, H, dk = q.shape
    dv = v.shape[2]
    out = np.empty((T, H, dv), np.float64)
    final = np.empty((H, dk, dv), np.float64)
    init = None if initial is None else _c64(initial)
    if lib().oracle_delta_recurrence_f64(q, k, v, g, beta, T, H, dk, dv, _ptr(init), out, _ptr(final)):
        raise ValueError("invalid dimensions")
    return out, final


def delta_chunked_f64(q, k, v, g, beta, chunk, initial=None):
    q, k, v, g, beta = map(_c64, (q, k, v, g, beta))
    T, H, dk = q.shape
    dv = v.shape[2]
    out = np.empty((T, H, dv), np.float64)
    final = np.empty((H, dk, dv), np.float64)
    init = None if initial is None else _c64(initial)
    if lib().oracle_delta_chunked_f64(q, k, v, g, beta, T, H, dk, dv, int(chunk), _ptr(init), out,
                                      _ptr(final)):
        raise ValueError("invalid dimensions")
    return out, final


def causal_conv(x, w):
    x, w = _c32(x), _c32(w)
    T, W = x.shape
    taps = w.reshape(W, -1).shape[1]
    y = np.empty_like(x)
    lib().oracle_causal_conv(x, T, W, _c32(w.reshape(W, taps)), taps, y)
    return y


def rms(x, w, eps=1e-6):
    x, w = _c32(x), _c32(w)
    width = w.shape[0]
    y = np.empty_like(x)
    lib().oracle_rms(x, x.size // width, width, w, float(eps), y)
    return y


def linear(x, w):
    x, w = _c32(x), _c32(w)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float32)
    lib().oracle_linear(x, M, K, w, N, y)
    return y


def attention(q, k, v, causal=True):
    q, k, v = map(_c32, (q, k, v))
    heads, qn, d = q.shape
    kvh, kn, _ = k.shape
    out = np.empty_like(q)
    if lib().oracle_attention(q, k, v, heads, kvh, qn, kn, d, int(causal), out):
        raise ValueError("attention tensor shapes")
    return out


def rotary(x, dim, theta, pos0=0):
    x = _c32(x).copy()
    T, heads, width = x.shape
    lib().oracle_rotary(x, T, heads, width, int(dim), float(theta), int(pos0))
    return x


def f16_round(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


class Backbone:
    """Hybrid backbone over raw checkpoint tensors (qwen.rs:193-310 naming).

    `config` carries the TextConfig fields; `weights` maps tensor names
    (model.language_model.*) to float arrays.
    """

    PREFIX = "model.language_model."

    def __init__(self, config: dict, weights: dict, mixed_f16: bool = False):
        self.cfg = config
        self._keep = []
        c = OracleConfig()
        rp = config["rope_parameters"]
        c.hidden = config["hidden_size"]
        c.intermediate = config["intermediate_size"]
        c.vocab = config["vocab_size"]
        c.heads = config["num_attention_heads"]
        c.kv_heads = config["num_key_value_heads"]
        c.head_dim = config["head_dim"]
        c.rotary_dim = int(config["head_dim"] * rp["partial_rotary_factor"])
        c.lin_k_heads = config["linear_num_key_heads"]
        c.lin_v_heads = config["linear_num_value_heads"]
        c.lin_dk = config["linear_key_head_dim"]
        c.lin_dv = config["linear_value_head_dim"]
        c.conv_taps = config["linear_conv_kernel_dim"]
        c.n_layers = len(config["layer_types"])
        c.eps = config["rms_norm_eps"]
        c.rope_theta = rp["rope_theta"]
        self.c = c
        P = self.PREFIX

        def fp(name):
            a = _c32(weights[name])
            self._keep.append(a)
            return a.ctypes.data_as(_FP)

        layers = (OracleLayer * c.n_layers)()
        self.kinds = []
        for i, kind in enumerate(config["layer_types"]):
            L = layers[i]
            p = f"{P}layers.{i}."
            L.input_norm = fp(p + "input_layernorm.weight")
            L.post_norm = fp(p + "post_attention_layernorm.weight")
            L.gate = fp(p + "mlp.gate_proj.weight")
            L.up = fp(p + "mlp.up_proj.weight")
            L.down = fp(p + "mlp.down_proj.weight")
            if kind == "full_attention":
                L.kind = 1
                a = p + "self_attn."
                L.q, L.k, L.v, L.o = (fp(a + n + "_proj.weight") for n in "qkvo")
                L.q_norm = fp(a + "q_norm.weight")
                L.k_norm = fp(a + "k_norm.weight")
            else:
                L.kind = 0
                a = p + "linear_attn."
                L.qkv = fp(a + "in_proj_qkv.weight")
                L.z = fp(a + "in_proj_z.weight")
                L.a = fp(a + "in_proj_a.weight")
                L.b = fp(a + "in_proj_b.weight")
                L.out = fp(a + "out_proj.weight")
                L.conv = fp(a + "conv1d.weight")
                L.dt = fp(a + "dt_bias")
                L.a_log = fp(a + "A_log")
                L.norm = fp(a + "norm.weight")
            self.kinds.append(L.kind)
        self._layers = layers
        b = OracleBackbone()
        b.c = c
        b.embeddings = fp(P + "embed_tokens.weight")
        b.final_norm = fp(P + "norm.weight")
        b.layers = layers
        b.mixed_f16 = int(mixed_f16)
        self.b = b

    def _alloc_prefix(self, tokens):
        c = self.c
        W = 2 * c.lin_k_heads * c.lin_dk + c.lin_v_heads * c.lin_dv
        n = c.n_layers
        pre = OraclePrefix()
        arrays = {"hidden": np.zeros((tokens, c.hidden), np.float32), "recurrent": [],
                  "history": [], "key": [], "value": []}
        rec, hist, key, val = (_FP * n)(), (_FP * n)(), (_FP * n)(), (_FP * n)()
        rows = (C.c_int * n)()
        for i, kind in enumerate(self.kinds):
            if kind == 0:
                r = np.zeros((c.lin_v_heads, c.lin_dk, c.lin_dv), np.float32)
                h = np.zeros((c.conv_taps - 1, W), np.float32)
                k = v = None
                rec[i] = r.ctypes.data_as(_FP)
                hist[i] = h.ctypes.data_as(_FP)
            else:
                r = h = None
                k = np.zeros((c.kv_heads, tokens, c.head_dim), np.float32)
                v = np.zeros((c.kv_heads, tokens, c.head_dim), np.float32)
                key[i] = k.ctypes.data_as(_FP)
                val[i] = v.ctypes.data_as(_FP)
            arrays["recurrent"].append(r)
            arrays["history"].append(h)
            arrays["key"].append(k)
            arrays["value"].append(v)
        pre.tokens = tokens
        pre.hidden = arrays["hidden"].ctypes.data_as(_FP)
        pre.recurrent, pre.history, pre.history_rows, pre.key, pre.value = rec, hist, rows, key, val
        arrays["_rows"] = rows
        arrays["_struct"] = pre
        arrays["_keep"] = (rec, hist, key, val)
        return pre, arrays

    def prefill(self, ids, initial=None, capture=0):
        """Returns (hidden [(offset+T), H], saved prefix dict or None)."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        T = ids.shape[0]
        offset = initial["_struct"].tokens if initial is not None else 0
        out = np.empty((offset + T, self.c.hidden), np.float32)
        saved_struct, saved = (None, None)
        if capture:
            saved_struct, saved = self._alloc_prefix(capture)
        rc = lib().oracle_backbone_prefill(
            C.byref(self.b), ids.ctypes.data_as(C.POINTER(C.c_int)), T,
            C.cast(C.pointer(initial["_struct"]), C.c_void_p) if initial is not None else None,
            int(capture), C.cast(C.pointer(saved_struct), C.c_void_p) if saved_struct else None,
            out)
        if rc:
            raise ValueError("prefill boundary or vocabulary")
        if saved is not None:
            saved["history_rows"] = list(saved["_rows"])
        return out, saved
