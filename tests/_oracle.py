"""ctypes binding of the CPU oracle (oracle/liboracle*.so) -- test infrastructure.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this,
and only as the checker or the timed CPU baseline.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_size_t, c_void_p

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(REPO, "oracle")

_P = c_void_p


class OraKV(ctypes.Structure):
    _fields_ = [
        ("n_layers", c_int),
        ("n_kv_heads", c_int),
        ("head_dim", c_int),
        ("max_seq", c_int),
        ("kv_dim", c_int),
        ("k_cache", c_void_p),
        ("v_cache", c_void_p),
        ("pos", c_int),
        ("len", c_int),
    ]


_SIGS = {
    "ora_f32_to_f16": (ctypes.c_uint16, [c_float]),
    "ora_f16_to_f32": (c_float, [ctypes.c_uint16]),
    "ora_cvt_f32_to_f16": (None, [_P, _P, c_int]),
    "ora_cvt_f16_to_f32": (None, [_P, _P, c_size_t]),
    "ora_precompute_rope_theta": (None, [c_float, c_int, _P]),
    "ora_apply_rope": (None, [_P, _P, c_int, _P, c_int, c_int, c_int]),
    "ora_apply_rope_batch": (None, [_P, _P, c_int, _P, c_int, c_int, c_int, c_int]),
    "ora_softmax_vec": (None, [_P, c_int]),
    "ora_gqa_attention": (None, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int]),
    "ora_kv_write_batch": (None, [POINTER(OraKV), c_int, c_int, _P, _P, c_int, c_int]),
    "ora_attention_batch": (
        None,
        [_P, _P, POINTER(OraKV), c_int, c_int, c_int, c_int, c_int, c_int, _P],
    ),
    "ora_decode_step": (
        None,
        [POINTER(OraKV), c_int, _P, _P, _P, c_int, _P, c_int, c_int, _P, _P],
    ),
    "ora_verify_steps": (
        None,
        [POINTER(OraKV), c_int, _P, _P, _P, c_int, c_int, _P, c_int, c_int, _P, _P],
    ),
    "ora_ref_gqa_attention": (None, [_P, _P, _P, _P, c_int, c_int, c_int, c_int]),
    "ora_prefill_chunk_attention": (
        None,
        [POINTER(OraKV), c_int, _P, _P, _P, _P, c_int, _P, c_int, c_int, _P, _P],
    ),
    "ora_decode_layers": (
        None,
        [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int],
    ),
    "ora_attention_batch_layers": (
        None,
        [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int],
    ),
    "ora_num_threads": (c_int, []),
    "ora_quantize_q8_0": (None, [_P, _P, c_int]),
    "ora_q4_0_q8_0_matvec": (None, [_P, _P, _P, c_int, c_int]),
    "ora_q4_0_q8_0_matvec_qkv": (None, [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int]),
    "ora_q4_0_q8_0_matvec_parallel": (None, [_P, _P, _P, c_int, c_int, c_int]),
    "ora_rmsnorm_batch": (None, [_P, _P, _P, c_int, c_int, c_float]),
    "ora_dequant_q4_0_rows": (None, [_P, _P, c_int, c_int]),
    "ora_q4_0_gemm": (None, [_P, c_int, c_int, _P, c_int, _P, c_int]),
    "ora_silu_mul": (None, [_P, _P, c_int]),
    "ora_prefill_layer": (
        None,
        [_P, POINTER(OraKV), _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_float, _P,
         c_int],
    ),
    "ora_typed_row_bytes": (ctypes.c_long, [c_int, c_int]),
    "ora_dequant_typed_rows": (c_int, [_P, c_int, _P, c_int, c_int]),
    "ora_typed_matvec": (c_int, [_P, c_int, _P, _P, c_int, c_int]),
    "ora_typed_matvec_q8": (c_int, [_P, c_int, _P, _P, c_int, c_int]),
    "ora_typed_gemm": (c_int, [_P, c_int, c_int, c_int, _P, c_int, _P, c_int]),
    "ora_decode_layer_typed": (
        c_int,
        [_P, POINTER(OraKV), _P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, _P],
    ),
    "ora_prefill_layer_typed": (
        c_int,
        [_P, POINTER(OraKV), _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_float, _P,
         c_int],
    ),
}


class OraLayerWeights(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "rms_att",
                                         "rms_ffn")]


class OraLayerWeightsTyped(ctypes.Structure):
    _fields_ = ([(n, c_void_p) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3")]
                + [(n + "_type", c_int) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3")]
                + [("rms_att", c_void_p), ("rms_ffn", c_void_p)])


_libs: dict = {}


def load(fast: bool = False) -> ctypes.CDLL:
    name = "liboracle_fast.so" if fast else "liboracle.so"
    if name in _libs:
        return _libs[name]
    path = os.path.join(ORACLE_DIR, name)
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
    lib = ctypes.CDLL(path)
    for fn, (res, args) in _SIGS.items():
        f = getattr(lib, fn)
        f.restype = res
        f.argtypes = args
    _libs[name] = lib
    return lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "array must be contiguous"
    return a.ctypes.data


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    load().ora_cvt_f32_to_f16(_p(x), _p(out), x.size)
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    load().ora_cvt_f16_to_f32(_p(h), _p(out), h.size)
    return out


def theta_inv(theta: float = 1e6, hd: int = 128) -> np.ndarray:
    out = np.empty(hd // 2, dtype=np.float32)
    load().ora_precompute_rope_theta(theta, hd, _p(out))
    return out


def apply_rope(q, k, pos, th, n_heads, n_kv, hd):
    """In place on float32 arrays (either may be None)."""
    load().ora_apply_rope(_p(q) if q is not None else None, _p(k) if k is not None else None,
                          pos, _p(th), n_heads, n_kv, hd)


def softmax(x: np.ndarray) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    load().ora_softmax_vec(_p(y), y.size)
    return y


def gqa_attention(q, kc, vc, n_heads, heads_per_kv, hd, max_seq, pos):
    """mistral_model.h:362-487 on a copy of q; kc/vc uint16 [max_seq, kv_dim]."""
    qq = np.array(q, dtype=np.float32, copy=True)
    att = np.zeros(n_heads * max_seq, dtype=np.float32)
    out = np.empty(n_heads * hd, dtype=np.float32)
    load().ora_gqa_attention(_p(qq), _p(att), _p(out), _p(kc), _p(vc), n_heads, heads_per_kv,
                             hd, max_seq, pos)
    return out


def make_kv(kc: np.ndarray, vc: np.ndarray, n_kv: int, hd: int, max_seq: int) -> OraKV:
    """OraKV (one layer) over caller-owned uint16 arrays [max_seq, kv_dim]."""
    assert kc.dtype == np.uint16 and kc.shape == (max_seq, n_kv * hd)
    return OraKV(1, n_kv, hd, max_seq, n_kv * hd, _p(kc), _p(vc), 0, 0)


def attention_batch(Q, kc, vc, n_heads, n_kv, hd, max_seq, start_pos, S):
    Q = np.ascontiguousarray(Q, dtype=np.float32)
    kv = make_kv(kc, vc, n_kv, hd, max_seq)
    out = np.empty((S, n_heads * hd), dtype=np.float32)
    att = np.zeros(n_heads * max_seq, dtype=np.float32)
    load().ora_attention_batch(_p(Q), _p(out), ctypes.byref(kv), 0, start_pos, n_heads, n_kv, hd,
                               S, _p(att))
    return out


def attention_batch_parallel(Q, kc, vc, n_heads, n_kv, hd, max_seq, start_pos, S, threads=0):
    """Same arithmetic as attention_batch, units spread over OpenMP threads."""
    Q = np.ascontiguousarray(Q, dtype=np.float32)
    out = np.empty((S, n_heads * hd), dtype=np.float32)
    load().ora_attention_batch_layers(_p(Q), _p(out), _p(kc), _p(vc), 1, n_heads, n_kv, hd,
                                      max_seq, start_pos, S, threads)
    return out


def kv_write_batch(kc, vc, K, V, n_kv, hd, max_seq, start_pos, S):
    kv = make_kv(kc, vc, n_kv, hd, max_seq)
    K = np.ascontiguousarray(K, dtype=np.float32)
    V = np.ascontiguousarray(V, dtype=np.float32)
    load().ora_kv_write_batch(ctypes.byref(kv), 0, start_pos, _p(K), _p(V), n_kv * hd, S)
    return kv.len


def decode_step(kc, vc, q, k, v, pos, th, n_heads, n_kv, hd, max_seq):
    """Steps 4-6 of mistral_model.h:849-863 on copies of q/k; kc/vc updated."""
    kv = make_kv(kc, vc, n_kv, hd, max_seq)
    qq = np.array(q, dtype=np.float32, copy=True)
    kk = np.array(k, dtype=np.float32, copy=True)
    vv = np.ascontiguousarray(v, dtype=np.float32)
    att = np.zeros(n_heads * max_seq, dtype=np.float32)
    out = np.empty(n_heads * hd, dtype=np.float32)
    load().ora_decode_step(ctypes.byref(kv), 0, _p(qq), _p(kk), _p(vv), pos, _p(th), n_heads, n_kv,
                           _p(att), _p(out))
    return out


def verify_steps(kc, vc, Q, K, V, start_pos, S, th, n_heads, n_kv, hd, max_seq):
    kv = make_kv(kc, vc, n_kv, hd, max_seq)
    QQ = np.array(Q, dtype=np.float32, copy=True)
    KK = np.array(K, dtype=np.float32, copy=True)
    VV = np.ascontiguousarray(V, dtype=np.float32)
    att = np.zeros(n_heads * max_seq, dtype=np.float32)
    out = np.empty((S, n_heads * hd), dtype=np.float32)
    load().ora_verify_steps(ctypes.byref(kv), 0, _p(QQ), _p(KK), _p(VV), start_pos, S, _p(th),
                            n_heads, n_kv, _p(att), _p(out))
    return out


def prefill_chunk_attention(kc, vc, Q, K, V, positions, th, n_heads, n_kv, hd, max_seq):
    """Phases 1 + 2 of mistral_layer_prefill_chunk on copies of Q/K; kc/vc
    updated.  Returns (out, len)."""
    kv = make_kv(kc, vc, n_kv, hd, max_seq)
    QQ = np.array(Q, dtype=np.float32, copy=True)
    KK = np.array(K, dtype=np.float32, copy=True)
    VV = np.ascontiguousarray(V, dtype=np.float32)
    P = np.ascontiguousarray(positions, dtype=np.int32)
    S = len(P)
    att = np.zeros(n_heads * max_seq, dtype=np.float32)
    out = np.empty((S, n_heads * hd), dtype=np.float32)
    load().ora_prefill_chunk_attention(ctypes.byref(kv), 0, _p(QQ), _p(KK), _p(VV), _p(P), S,
                                       _p(th), n_heads, n_kv, _p(att), _p(out))
    return out, kv.len


def ref_gqa_attention(q, k, v, S, n_heads, n_kv, hd):
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty((S, n_heads * hd), dtype=np.float32)
    load().ora_ref_gqa_attention(_p(out), _p(q), _p(k), _p(v), S, n_heads, n_kv, hd)
    return out


def decode_layers(Q, kcache, vcache, n_layers, n_heads, heads_per_kv, hd, max_seq, pos,
                  threads=0, fast=True):
    """CPU baseline: n_layers independent S=1 attentions (OpenMP over layer x head)."""
    Q = np.ascontiguousarray(Q, dtype=np.float32)
    out = np.empty((n_layers, n_heads * hd), dtype=np.float32)
    load(fast).ora_decode_layers(_p(Q), _p(out), _p(kcache), _p(vcache), n_layers, n_heads,
                                 heads_per_kv, hd, max_seq, pos, threads)
    return out


def attention_batch_layers(Q, kcache, vcache, n_layers, n_heads, n_kv, hd, max_seq, start_pos, S,
                           threads=0, fast=True):
    Q = np.ascontiguousarray(Q, dtype=np.float32)
    out = np.empty((n_layers, S, n_heads * hd), dtype=np.float32)
    load(fast).ora_attention_batch_layers(_p(Q), _p(out), _p(kcache), _p(vcache), n_layers,
                                          n_heads, n_kv, hd, max_seq, start_pos, S, threads)
    return out


def num_threads(fast: bool = True) -> int:
    return int(load(fast).ora_num_threads())


# --- Q4_0 x Q8_0 projections (oracle/q4_oracle.h) ---------------------------

Q8_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", (32,))])   # 36 bytes
Q4_BLOCK_BYTES = 18


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """fp32 [n] -> Q8_0 blocks [n/32] (structured array of (d, qs[32]))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size % 32 == 0
    out = np.zeros(x.size // 32, dtype=Q8_DTYPE)
    load().ora_quantize_q8_0(_p(x), out.ctypes.data, x.size)
    return out


def q4_0_q8_0_matvec(W: np.ndarray, xq: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
    """W: uint8 [out_dim, in_dim/32*18] Q4_0 rows; xq: Q8_0 blocks [in_dim/32]."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    assert W.size == out_dim * in_dim // 32 * Q4_BLOCK_BYTES and xq.dtype == Q8_DTYPE
    y = np.empty(out_dim, dtype=np.float32)
    load().ora_q4_0_q8_0_matvec(_p(W), xq.ctypes.data, _p(y), out_dim, in_dim)
    return y


def q4_0_q8_0_matvec_qkv(Wq, Wk, Wv, xq, dim, kv_dim, in_dim):
    Wq, Wk, Wv = (np.ascontiguousarray(w, dtype=np.uint8) for w in (Wq, Wk, Wv))
    yq = np.empty(dim, np.float32)
    yk = np.empty(kv_dim, np.float32)
    yv = np.empty(kv_dim, np.float32)
    load().ora_q4_0_q8_0_matvec_qkv(_p(Wq), _p(Wk), _p(Wv), xq.ctypes.data, _p(yq), _p(yk),
                                    _p(yv), dim, kv_dim, in_dim)
    return yq, yk, yv


def q4_0_q8_0_matvec_parallel(W, xq, out_dim, in_dim, threads=0, fast=True):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    y = np.empty(out_dim, dtype=np.float32)
    load(fast).ora_q4_0_q8_0_matvec_parallel(_p(W), xq.ctypes.data, _p(y), out_dim, in_dim,
                                             threads)
    return y


def make_q4_0(g: np.random.Generator, out_dim: int, in_dim: int) -> np.ndarray:
    """Random Q4_0 rows: N(0, 0.02)-sized fp16 scales, uniform nibbles."""
    nb = in_dim // 32
    W = np.empty((out_dim, nb, Q4_BLOCK_BYTES), np.uint8)
    d = (np.abs(g.standard_normal((out_dim, nb))) * 0.02 + 1e-3).astype(np.float16)
    W[:, :, 0:2] = d.view(np.uint8).reshape(out_dim, nb, 2)
    W[:, :, 2:] = g.integers(0, 256, (out_dim, nb, 16), dtype=np.uint8)
    return W.reshape(out_dim, nb * Q4_BLOCK_BYTES)


def dequant_q4_0(W: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
    """float64 weights [out_dim, in_dim] from Q4_0 rows (dequant.h:600-611 layout)."""
    nb = in_dim // 32
    B = np.ascontiguousarray(W, np.uint8).reshape(out_dim, nb, Q4_BLOCK_BYTES)
    d = B[:, :, 0:2].copy().view(np.float16).reshape(out_dim, nb).astype(np.float64)
    q = B[:, :, 2:].astype(np.int64)
    lo = (q & 0x0F) - 8
    hi = (q >> 4) - 8
    vals = np.concatenate([lo, hi], axis=2)          # weights 0..15, then 16..31
    return (vals * d[:, :, None]).reshape(out_dim, in_dim)


# ---- prefill layer (oracle/prefill_oracle.c) --------------------------------

def rmsnorm_batch(X, w, eps=1e-5):
    X = np.ascontiguousarray(X, np.float32)
    S, dim = X.shape
    out = np.empty_like(X)
    load().ora_rmsnorm_batch(_p(out), _p(X), _p(np.ascontiguousarray(w, np.float32)), dim, S, eps)
    return out


def dequant_q4_0_rows(W, rows, cols):
    out = np.empty((rows, cols), np.float32)
    load().ora_dequant_q4_0_rows(_p(np.ascontiguousarray(W, np.uint8)), _p(out), rows, cols)
    return out


def q4_0_gemm(W, out_dim, in_dim, X, threads=0):
    X = np.ascontiguousarray(X, np.float32)
    Y = np.empty((X.shape[0], out_dim), np.float32)
    load().ora_q4_0_gemm(_p(np.ascontiguousarray(W, np.uint8)), out_dim, in_dim, _p(X),
                         X.shape[0], _p(Y), threads)
    return Y


def silu_mul(gate, up):
    g = np.array(gate, np.float32, copy=True)
    load().ora_silu_mul(_p(g), _p(np.ascontiguousarray(up, np.float32)), g.size)
    return g


def prefill_layer(W, X, kc, vc, start_pos, S, dim, hidden, n_heads, n_kv, th, eps=1e-5,
                  threads=0):
    """One blas_prefill_layer on copies: returns X'; kc/vc (one layer) updated.
    W: dict of wq wk wv wo w1 w2 w3 (uint8 Q4_0 rows) and rms_att rms_ffn."""
    hd = dim // n_heads
    kv = make_kv(kc, vc, n_kv, hd, kc.shape[0])
    arrs = {k: np.ascontiguousarray(v) for k, v in W.items()}
    lw = OraLayerWeights(*[_p(arrs[n]) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3",
                                                  "rms_att", "rms_ffn")])
    Xo = np.array(X, np.float32, copy=True)
    load().ora_prefill_layer(ctypes.byref(lw), ctypes.byref(kv), _p(Xo), 0, start_pos, S, dim,
                             hidden, n_heads, n_kv, eps, _p(np.ascontiguousarray(th, np.float32)),
                             threads)
    return Xo


# ---- weight types other than Q4_0 (oracle/kquant_oracle.c) -----------------

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 2, 12, 14


def typed_row_bytes(t: int, cols: int) -> int:
    return int(load().ora_typed_row_bytes(t, cols))


def make_q4_k(g: np.random.Generator, rows: int, cols: int, d_scale: float = 1.0) -> np.ndarray:
    """Random Q4_K rows: small positive fp16 d / dmin (times d_scale), random
    6-bit scales and mins (all 12 bytes random), random nibbles."""
    nb = cols // 256
    B = np.empty((rows, nb, 144), np.uint8)
    d = ((np.abs(g.standard_normal((rows, nb))) * 0.002 + 1e-4) * d_scale).astype(np.float16)
    dm = ((np.abs(g.standard_normal((rows, nb))) * 0.002 + 1e-4) * d_scale).astype(np.float16)
    B[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    B[:, :, 2:4] = dm.view(np.uint8).reshape(rows, nb, 2)
    B[:, :, 4:] = g.integers(0, 256, (rows, nb, 140), dtype=np.uint8)
    return B.reshape(rows, nb * 144)


def make_q6_k(g: np.random.Generator, rows: int, cols: int, d_scale: float = 1.0) -> np.ndarray:
    """Random Q6_K rows: random ql / qh bits, int8 scales, small fp16 d (times
    d_scale)."""
    nb = cols // 256
    B = np.empty((rows, nb, 210), np.uint8)
    B[:, :, :208] = g.integers(0, 256, (rows, nb, 208), dtype=np.uint8)
    d = ((np.abs(g.standard_normal((rows, nb))) * 0.0005 + 1e-5) * d_scale).astype(np.float16)
    B[:, :, 208:210] = d.view(np.uint8).reshape(rows, nb, 2)
    return B.reshape(rows, nb * 210)


def make_typed(g: np.random.Generator, t: int, rows: int, cols: int,
               d_scale: float = 1.0) -> np.ndarray:
    """Random rows of type t; d_scale shrinks the K-quants' block scales
    (0.07 gives weights of a few hundredths, as a model's)."""
    if t == TYPE_Q4_K:
        return make_q4_k(g, rows, cols, d_scale)
    if t == TYPE_Q6_K:
        return make_q6_k(g, rows, cols, d_scale)
    if t == TYPE_Q4_0:
        return make_q4_0(g, rows, cols)
    w = (g.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    if t == TYPE_F16:
        return w.astype(np.float16).view(np.uint8).reshape(rows, cols * 2)
    return w.view(np.uint8).reshape(rows, cols * 4)


def dequant_typed(W, t: int, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    assert load().ora_dequant_typed_rows(_p(np.ascontiguousarray(W, np.uint8)), t, _p(out), rows,
                                         cols) == 0
    return out


def typed_matvec(W, t: int, x, out_dim: int, in_dim: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(out_dim, np.float32)
    assert load().ora_typed_matvec(_p(np.ascontiguousarray(W, np.uint8)), t, _p(x), _p(y),
                                   out_dim, in_dim) == 0
    return y


def typed_matvec_q8(W, t: int, xq, out_dim: int, in_dim: int) -> np.ndarray:
    y = np.empty(out_dim, np.float32)
    assert load().ora_typed_matvec_q8(_p(np.ascontiguousarray(W, np.uint8)), t, xq.ctypes.data,
                                      _p(y), out_dim, in_dim) == 0
    return y


def typed_gemm(W, t: int, out_dim: int, in_dim: int, X, threads: int = 0) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    Y = np.empty((X.shape[0], out_dim), np.float32)
    assert load().ora_typed_gemm(_p(np.ascontiguousarray(W, np.uint8)), t, out_dim, in_dim, _p(X),
                                 X.shape[0], _p(Y), threads) == 0
    return Y


MATS = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")


def prefill_layer_typed(W, types, X, kc, vc, start_pos, S, dim, hidden, n_heads, n_kv, th,
                        eps=1e-5, threads=0):
    """ora_prefill_layer_typed on copies: returns X'; kc/vc (one layer) updated.
    W: dict of the seven matrices (uint8 rows of their type) and rms_att,
    rms_ffn; types: dict of the seven GGML type ids."""
    hd = dim // n_heads
    kv = make_kv(kc, vc, n_kv, hd, kc.shape[0])
    arrs = {k: np.ascontiguousarray(v) for k, v in W.items()}
    lw = OraLayerWeightsTyped(*[_p(arrs[n]) for n in MATS], *[types[n] for n in MATS],
                              _p(arrs["rms_att"]), _p(arrs["rms_ffn"]))
    Xo = np.array(X, np.float32, copy=True)
    assert load().ora_prefill_layer_typed(ctypes.byref(lw), ctypes.byref(kv), _p(Xo), 0,
                                          start_pos, S, dim, hidden, n_heads, n_kv, eps,
                                          _p(np.ascontiguousarray(th, np.float32)), threads) == 0
    return Xo


def decode_layer_typed(W, types, x, kc, vc, pos, dim, hidden, n_heads, n_kv, th, eps=1e-5):
    """ora_decode_layer_typed on copies: returns x'; kc/vc (one layer) updated."""
    hd = dim // n_heads
    kv = make_kv(kc, vc, n_kv, hd, kc.shape[0])
    arrs = {k: np.ascontiguousarray(v) for k, v in W.items()}
    lw = OraLayerWeightsTyped(*[_p(arrs[n]) for n in MATS], *[types[n] for n in MATS],
                              _p(arrs["rms_att"]), _p(arrs["rms_ffn"]))
    xo = np.array(x, np.float32, copy=True)
    assert load().ora_decode_layer_typed(ctypes.byref(lw), ctypes.byref(kv), _p(xo), 0, pos, dim,
                                         hidden, n_heads, n_kv, eps,
                                         _p(np.ascontiguousarray(th, np.float32))) == 0
    return xo
