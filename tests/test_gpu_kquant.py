"""GPU parity of the weight types other than Q4_0 (Q4_K, Q6_K, F16, F32) in the
projections and the prefill layer against the oracle (oracle/kquant_oracle.c):
mia_dequant_f32, mia_matvec_f32, mia_matvec_q8, mia_gemm_f32,
mia_prefill_layer_typed and the drop-in q4_matvec_sdot_parallel for those
types.

Bars:
- Dequantisation is bit-exact (the Q4_K fp16 steps, the Q6_K value mapping,
  fp16 and fp32 rows).
- Matvec rows: the weights are exact and only the fp32 order of a row's sum
  differs from the oracle's, so |gpu - oracle| <= 2 * K * 2^-24 *
  sum_k |w_k x_k| (both within K * 2^-24 of the exact sum); a lost or doubled
  group, a wrong nibble, scale or min exceeds that by orders of magnitude.
  GEMM rows to the same bound: x enters as fp16 hi + lo (2^-22 relative,
  2^-25 absolute below 2^-3) and Q6_K / F32 weights as row-scaled hi + lo
  (2^-22 relative), both far inside it.
  The attention tolerance (2e-3 abs + 1e-2 rel) is checked as well.
- The layer normwise within 2e-3 of the oracle (the attention's fp16 ring and
  operands carried through Wo and the FFN), to fp32 level when Wo is zero;
  its ring rows within one fp16 ulp (plus 1e-5 of the row's scale)."""

import ctypes

import numpy as np
import pytest

import _data as D
import _gpu as G
import _oracle as O
import anetransformers_amd as mia
from anetransformers_amd import DeviceBuffer as DB
from anetransformers_amd import check

pytestmark = pytest.mark.gpu

U = 2.0 ** -24
NAMES = {O.TYPE_F32: "F32", O.TYPE_F16: "F16", O.TYPE_Q4_0: "Q4_0", O.TYPE_Q4_K: "Q4_K",
         O.TYPE_Q6_K: "Q6_K"}
Q4_K_M = {"wq": O.TYPE_Q4_K, "wk": O.TYPE_Q4_K, "wv": O.TYPE_Q6_K, "wo": O.TYPE_Q4_K,
          "w1": O.TYPE_Q4_K, "w3": O.TYPE_Q4_K, "w2": O.TYPE_Q6_K}


def _bound(Wd, x):
    """2 K 2^-24 sum |w x| per output, float64 (x [K] or [S][K])."""
    K = Wd.shape[1]
    return 2 * K * U * (np.abs(np.asarray(x, np.float64)) @ np.abs(Wd.astype(np.float64)).T)


def _assert_close(got, ref, bound, what):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    worst = np.unravel_index(int(np.argmax(err / (bound + 1e-30))), err.shape)
    assert np.all(err <= bound + 1e-30), (what, worst, float(err[worst]), float(bound[worst]))
    assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), what


def gpu_dequant(W, t, rows, cols):
    L = G.lib()
    dw, dy = DB.from_array(W), DB(rows * cols * 4)
    check(L.mia_dequant_f32(dw.ptr, t, dy.ptr, rows, cols, None), "dequant")
    check(L.mia_stream_sync(None), "sync")
    return dy.download((rows, cols), np.float32)


def gpu_matvec(W, t, x, rows, cols, q8=False):
    L = G.lib()
    dw, dx, dy = DB.from_array(W), DB.from_array(x), DB(rows * 4)
    fn = L.mia_matvec_q8 if q8 else L.mia_matvec_f32
    check(fn(dw.ptr, t, dx.ptr, dy.ptr, rows, cols, None), "matvec")
    check(L.mia_stream_sync(None), "sync")
    return dy.download(rows, np.float32)


def gpu_gemm(W, t, X, N, K):
    L = G.lib()
    S = X.shape[0]
    dw, dx, dy = DB.from_array(W), DB.from_array(np.ascontiguousarray(X, np.float32)), DB(
        S * N * 4)
    check(L.mia_gemm_f32(dw.ptr, t, dx.ptr, dy.ptr, N, K, S, None), "gemm")
    check(L.mia_stream_sync(None), "sync")
    return dy.download((S, N), np.float32)


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q6_K, O.TYPE_F16, O.TYPE_F32, O.TYPE_Q4_0])
def test_dequant_bit_exact(t):
    G.say(f"kquant: dequant {NAMES[t]} 72x4096")
    g = np.random.default_rng(100 + t)
    rows, cols = 72, 4096
    W = O.make_typed(g, t, rows, cols)
    if t == O.TYPE_Q4_K:
        # scales that round in fp16, mins that cancel, subnormal steps
        Wb = W.reshape(rows, cols // 256, 144)
        Wb[:8, :, 0:2] = np.frombuffer(np.float16(3.7).tobytes(), np.uint8)
        Wb[8:16, :, 2:4] = np.frombuffer(np.float16(61.3).tobytes(), np.uint8)
        Wb[16:24, :, 0:4] = np.frombuffer(np.float16(1e-6).tobytes() * 2, np.uint8)
        W = Wb.reshape(rows, -1)
    got = gpu_dequant(W, t, rows, cols)
    want = O.dequant_typed(W, t, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t,rows,cols", [
    (O.TYPE_Q4_K, 4096, 4096), (O.TYPE_Q4_K, 1024, 4096), (O.TYPE_Q4_K, 14336, 4096),
    (O.TYPE_Q6_K, 4096, 14336), (O.TYPE_Q6_K, 1024, 4096), (O.TYPE_Q4_K, 37, 256),
    (O.TYPE_Q6_K, 9, 512), (O.TYPE_F16, 1024, 4096), (O.TYPE_F32, 100, 4096),
    (O.TYPE_F16, 13, 96), (O.TYPE_Q4_0, 4096, 4096), (O.TYPE_Q4_0, 11, 32),
])
def test_matvec_f32(t, rows, cols):
    G.say(f"kquant: matvec_f32 {NAMES[t]} {rows}x{cols}")
    g = np.random.default_rng(rows + cols + t)
    W = O.make_typed(g, t, rows, cols, d_scale=0.07)
    x = g.standard_normal(cols).astype(np.float32)
    got = gpu_matvec(W, t, x, rows, cols)
    ref = O.typed_matvec(W, t, x, rows, cols)
    _assert_close(got, ref, _bound(O.dequant_typed(W, t, rows, cols), x), f"matvec {NAMES[t]}")


def _wide_q4_k(g, rows, cols):
    """Q4_K rows with large block scales: d up to 3.7 (sub-block steps vd far
    above 63.5) in half the rows, so waves mix both forms of the kernel's
    n * vd, and dmin up to 61.3."""
    W = O.make_q4_k(g, rows, cols)
    Wb = W.reshape(rows, cols // 256, 144)
    Wb[::2, :, 0:2] = np.frombuffer(np.float16(3.7).tobytes(), np.uint8)
    Wb[1::4, :, 2:4] = np.frombuffer(np.float16(61.3).tobytes(), np.uint8)
    return Wb.reshape(rows, -1)


@pytest.mark.parametrize("t,big", [(O.TYPE_Q4_K, False), (O.TYPE_Q4_K, True),
                                   (O.TYPE_Q6_K, False), (O.TYPE_F16, False),
                                   (O.TYPE_F32, False), (O.TYPE_Q4_0, False)])
@pytest.mark.parametrize("rows", [37, 4096, 14336])
def test_matvec_weights_exact(t, big, rows):
    # x = a one-hot vector e_k: y = column k of W, every product w * 1 and
    # every sum with zeros exact, so each weight the matvec forms must equal
    # the reference's (the bound tests cannot see one weight off by an ulp);
    # compared as values, so that a zero weight may come out as +0 or -0;
    # fp32 x and Q8_0 x (d = 1, q = 1) alike, rows per wave 1, 2, 4
    G.say(f"kquant: exact weights {NAMES[t]} big={big} rows={rows}")
    g = np.random.default_rng(900 + t + rows)
    cols = 1024
    W = _wide_q4_k(g, rows, cols) if big else O.make_typed(g, t, rows, cols, d_scale=0.07)
    Wd = O.dequant_typed(W, t, rows, cols)
    for k in (0, 1, 17, 31, 32, 255, 256, 511, 1000, 1023):
        x = np.zeros(cols, np.float32)
        x[k] = 1.0
        got = gpu_matvec(W, t, x, rows, cols)
        assert np.array_equal(got, Wd[:, k]), k
        if t in (O.TYPE_Q4_K, O.TYPE_Q6_K):
            xq = O.quantize_q8_0(x)
            xq["d"][:] = 0.0
            xq["qs"][:] = 0
            xq["d"][k // 32] = 1.0
            xq["qs"][k // 32][k % 32] = 1
            got = gpu_matvec(W, t, xq, rows, cols, q8=True)
            assert np.array_equal(got, Wd[:, k]), ("q8", k)


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_F16])
def test_gemm_weights_exact(t):
    # one-hot token rows: Y = columns of W; fp16-valued weights enter the GEMM
    # exactly, so Y is bit-exact
    G.say(f"kquant: gemm exact weights {NAMES[t]}")
    g = np.random.default_rng(950 + t)
    N, K = 96, 512
    W = _wide_q4_k(g, N, K) if t == O.TYPE_Q4_K else O.make_typed(g, t, N, K)
    ks = [0, 3, 31, 255, 256, 300, 511]
    X = np.zeros((len(ks), K), np.float32)
    X[np.arange(len(ks)), ks] = 1.0
    got = gpu_gemm(W, t, X, N, K)
    Wd = O.dequant_typed(W, t, N, K)
    assert np.array_equal(got, Wd[:, ks].T)


@pytest.mark.parametrize("t,rows,cols", [
    (O.TYPE_Q4_K, 4096, 4096), (O.TYPE_Q6_K, 4096, 14336), (O.TYPE_F16, 96, 512),
    (O.TYPE_F32, 40, 1024),
])
def test_matvec_q8(t, rows, cols):
    # q4_matvec_sdot_parallel's non-Q4_0 branch: x as the Q8_0 values d * q
    G.say(f"kquant: matvec_q8 {NAMES[t]} {rows}x{cols}")
    g = np.random.default_rng(7 * rows + cols + t)
    W = O.make_typed(g, t, rows, cols, d_scale=0.07)
    xq = O.quantize_q8_0(g.standard_normal(cols).astype(np.float32))
    got = gpu_matvec(W, t, xq, rows, cols, q8=True)
    ref = O.typed_matvec_q8(W, t, xq, rows, cols)
    xv = (xq["d"][:, None] * xq["qs"].astype(np.float32)).astype(np.float32).reshape(-1)
    _assert_close(got, ref, _bound(O.dequant_typed(W, t, rows, cols), xv), f"q8 {NAMES[t]}")


def test_matvec_q8_q4_0_is_the_w4a8_kernel():
    G.say("kquant: matvec_q8 Q4_0 == mia_q4_0_matvec")
    L = G.lib()
    g = np.random.default_rng(5)
    rows, cols = 512, 4096
    W = O.make_q4_0(g, rows, cols)
    xq = O.quantize_q8_0(g.standard_normal(cols).astype(np.float32))
    dw, dx, dy = DB.from_array(W), DB.from_array(xq), DB(rows * 4)
    check(L.mia_q4_0_matvec(dw.ptr, dx.ptr, dy.ptr, rows, cols, None), "q4_0_matvec")
    check(L.mia_stream_sync(None), "sync")
    want = dy.download(rows, np.float32)
    assert np.array_equal(gpu_matvec(W, O.TYPE_Q4_0, xq, rows, cols, q8=True), want)


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q6_K, O.TYPE_F16])
def test_dropin_sdot_parallel_other_types(t):
    G.say(f"kquant: drop-in q4_matvec_sdot_parallel {NAMES[t]}")
    L = G.lib()
    g = np.random.default_rng(50 + t)
    rows, cols = 1024, 4096
    W = O.make_typed(g, t, rows, cols, d_scale=0.07)
    xq = O.quantize_q8_0(g.standard_normal(cols).astype(np.float32))
    dw = DB.from_array(W)
    y = np.zeros(rows, np.float32)
    L.mia_dropin_set_abort(0)
    try:
        L.mia_dropin_q4_matvec_sdot_parallel(dw.ptr, ctypes.c_uint32(t), xq.ctypes.data,
                                             y.ctypes.data, rows, cols)
        assert L.mia_dropin_status() == 0, L.mia_last_error()
    finally:
        L.mia_dropin_set_abort(1)
    assert np.array_equal(y, gpu_matvec(W, t, xq, rows, cols, q8=True))


@pytest.mark.parametrize("t,S,N,K", [
    (O.TYPE_Q4_K, 5, 96, 512), (O.TYPE_Q6_K, 5, 96, 512), (O.TYPE_F16, 5, 96, 512),
    (O.TYPE_F32, 3, 40, 256), (O.TYPE_Q4_K, 64, 1024, 4096), (O.TYPE_Q6_K, 32, 4096, 14336),
    (O.TYPE_Q4_K, 130, 4096, 4096),
])
def test_gemm_f32(t, S, N, K):
    G.say(f"kquant: gemm {NAMES[t]} S={S} {N}x{K}")
    g = np.random.default_rng(S + N + K + t)
    W = O.make_typed(g, t, N, K, d_scale=0.07)
    X = g.standard_normal((S, K)).astype(np.float32)
    got = gpu_gemm(W, t, X, N, K)
    ref = O.typed_gemm(W, t, N, K, X)
    _assert_close(got, ref, _bound(O.dequant_typed(W, t, N, K), X), f"gemm {NAMES[t]}")


@pytest.mark.parametrize("t", [O.TYPE_F32, O.TYPE_Q6_K])
def test_gemm_rows_of_every_magnitude(t):
    # the row-scaled hi + lo split of weights that are not fp16 values: rows
    # from 1e-7 to 1e4 in size (F32), Q6_K steps from fp16 subnormals up, an
    # all-zero row, and a single-token batch
    G.say(f"kquant: gemm {NAMES[t]} row magnitudes")
    g = np.random.default_rng(600 + t)
    N, K = 64, 512
    if t == O.TYPE_F32:
        w = g.standard_normal((N, K)).astype(np.float32)
        w *= (10.0 ** np.linspace(-7, 4, N)).astype(np.float32)[:, None]
        w[5] = 0
        W = w.view(np.uint8).reshape(N, K * 4)
    else:
        W = O.make_q6_k(g, N, K)
        d = (2.0 ** np.linspace(-24, 2, N)).astype(np.float16)     # subnormal to 4
        Wb = W.reshape(N, K // 256, 210)
        Wb[:, :, 208:210] = d.view(np.uint8).reshape(N, 1, 2)
        Wb[5, :, 208:210] = 0
        W = Wb.reshape(N, -1)
    for S in (1, 9):
        X = g.standard_normal((S, K)).astype(np.float32)
        got = gpu_gemm(W, t, X, N, K)
        ref = O.typed_gemm(W, t, N, K, X)
        _assert_close(got, ref, _bound(O.dequant_typed(W, t, N, K), X),
                      f"gemm {NAMES[t]} S={S}")
        assert np.all(got[:, 5] == 0)


@pytest.mark.parametrize("t,N,K", [
    (O.TYPE_Q4_K, 4096, 4096), (O.TYPE_Q4_K, 1024, 4096), (O.TYPE_Q6_K, 1024, 4096),
    (O.TYPE_Q4_K, 14336, 4096), (O.TYPE_Q6_K, 4096, 14336),
])
def test_gemm_f32_prefill_shapes_sampled(t, N, K):
    # The Q4_K_M prefill layer's GEMMs at S = 512 (each shape's GEMM algorithm
    # is picked on its first call): 64 sampled output columns against a
    # float64 product of the oracle's dequantised rows, and a second call
    # bit-identical to the first.
    S = 512
    G.say(f"kquant: gemm {NAMES[t]} S={S} {N}x{K}, sampled columns")
    g = np.random.default_rng(800 + N + K + t)
    W = O.make_typed(g, t, N, K, d_scale=0.07)
    X = g.standard_normal((S, K)).astype(np.float32)
    got = gpu_gemm(W, t, X, N, K)
    again = gpu_gemm(W, t, X, N, K)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    rows = np.sort(g.choice(N, 64, replace=False))
    Wd = O.dequant_typed(np.ascontiguousarray(W[rows]), t, 64, K)
    ref = X.astype(np.float64) @ Wd.astype(np.float64).T
    _assert_close(got[:, rows], ref, _bound(Wd, X), f"gemm {NAMES[t]} S={S} {N}x{K}")


def test_gemm_f32_many_shapes():
    # More GEMM shapes than the library remembers algorithms for (64): every
    # batch size from 1 to 80 on one Q4_K and one Q6_K matrix, each against
    # the oracle; the shapes past the limit run the heuristic's first
    # algorithm untimed.
    G.say("kquant: gemm at 80 batch sizes x 2 types")
    g = np.random.default_rng(910)
    N, K = 96, 512
    for t in (O.TYPE_Q4_K, O.TYPE_Q6_K):
        W = O.make_typed(g, t, N, K, d_scale=0.07)
        Wd = O.dequant_typed(W, t, N, K)
        for S in range(1, 81):
            X = g.standard_normal((S, K)).astype(np.float32)
            got = gpu_gemm(W, t, X, N, K)
            ref = X.astype(np.float64) @ Wd.astype(np.float64).T
            _assert_close(got, ref, _bound(Wd, X), f"gemm {NAMES[t]} S={S}")


def gpu_pack(W, t, N, K):
    L = G.lib()
    dw = DB.from_array(W)
    nb = L.mia_gemm_pack_bytes(t, N, K)
    assert nb > 0
    dp = DB(nb)
    check(L.mia_gemm_pack(dw.ptr, t, dp.ptr, N, K, None), "pack")
    check(L.mia_stream_sync(None), "sync")
    return dp


@pytest.mark.parametrize("t,S,N,K", [
    (O.TYPE_Q4_K, 64, 1024, 4096), (O.TYPE_Q6_K, 32, 4096, 14336), (O.TYPE_F16, 5, 96, 512),
    (O.TYPE_F32, 3, 40, 256), (O.TYPE_Q4_0, 20, 1024, 4096),
])
def test_packed_gemm_is_bit_identical(t, S, N, K):
    G.say(f"kquant: packed gemm {NAMES[t]} S={S} {N}x{K}")
    L = G.lib()
    g = np.random.default_rng(700 + S + N + t)
    W = O.make_typed(g, t, N, K, d_scale=0.07)
    X = g.standard_normal((S, K)).astype(np.float32)
    dp = gpu_pack(W, t, N, K)
    dx, dy = DB.from_array(X), DB(S * N * 4)
    check(L.mia_gemm_packed_f32(dp.ptr, t, dx.ptr, dy.ptr, N, K, S, None), "packed gemm")
    check(L.mia_stream_sync(None), "sync")
    got = dy.download((S, N), np.float32)
    assert np.array_equal(got.view(np.uint32), gpu_gemm(W, t, X, N, K).view(np.uint32))


def test_gemm_q4_0_is_the_q4_0_gemm():
    G.say("kquant: gemm Q4_0 == mia_q4_0_gemm_f32")
    L = G.lib()
    g = np.random.default_rng(9)
    S, N, K = 20, 1024, 4096
    W = O.make_q4_0(g, N, K)
    X = g.standard_normal((S, K)).astype(np.float32)
    dw, dx, dy = DB.from_array(W), DB.from_array(X), DB(S * N * 4)
    check(L.mia_q4_0_gemm_f32(dw.ptr, dx.ptr, dy.ptr, N, K, S, None), "q4_0_gemm")
    check(L.mia_stream_sync(None), "sync")
    want = dy.download((S, N), np.float32)
    assert np.array_equal(gpu_gemm(W, O.TYPE_Q4_0, X, N, K), want)


def _layer(g, types, dim, hidden, nh, nkv):
    kvd = dim // nh * nkv
    shapes = {"wq": (dim, dim), "wk": (kvd, dim), "wv": (kvd, dim), "wo": (dim, dim),
              "w1": (hidden, dim), "w3": (hidden, dim), "w2": (dim, hidden)}
    W = {k: O.make_typed(g, types[k], *shapes[k], d_scale=0.07) for k in O.MATS}
    W["rms_att"] = (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    W["rms_ffn"] = (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    return W


def _zero_weights(W, t):
    """The same bytes with every block scale (and min) zeroed: all weights 0."""
    W = W.copy()
    if t == O.TYPE_Q4_K:
        W.reshape(W.shape[0], -1, 144)[:, :, 0:4] = 0
    elif t == O.TYPE_Q6_K:
        W.reshape(W.shape[0], -1, 210)[:, :, 208:210] = 0
    elif t == O.TYPE_Q4_0:
        W.reshape(W.shape[0], -1, 18)[:, :, 0:2] = 0
    else:
        W[:] = 0
    return W


MIXES = {
    "q4_k_m": Q4_K_M,
    "mixed": {"wq": O.TYPE_F16, "wk": O.TYPE_F32, "wv": O.TYPE_Q6_K, "wo": O.TYPE_Q4_0,
              "w1": O.TYPE_Q4_K, "w3": O.TYPE_Q4_0, "w2": O.TYPE_F16},
}


def _run_layer(L, W, types, X, th, kc, vc, dim, hidden, nh, nkv, M, start, S):
    dev = {k: DB.from_array(v) for k, v in W.items()}
    lw = mia.LayerWeightsTyped(*[dev[n].ptr for n in O.MATS], *[types[n] for n in O.MATS],
                               dev["rms_att"].ptr, dev["rms_ffn"].ptr)
    dX, dth, dkc, dvc = DB.from_array(X), DB.from_array(th), DB.from_array(kc), DB.from_array(vc)
    check(L.mia_prefill_layer_typed(dX.ptr, ctypes.byref(lw), dth.ptr, dkc.ptr, dvc.ptr, dim,
                                    hidden, nh, nkv, 1e-5, M, start, S, None), "layer_typed")
    check(L.mia_stream_sync(None), "sync")
    return (dX.download(X.shape, np.float32), dkc.download(kc.shape, np.uint16),
            dvc.download(vc.shape, np.uint16))


@pytest.mark.parametrize("mix,dim,hidden,nh,nkv,M,start,S,wo_zero", [
    ("q4_k_m", 512, 1024, 4, 1, 64, 10, 20, False),
    ("q4_k_m", 512, 1024, 4, 1, 64, 10, 20, True),
    ("mixed", 512, 1024, 4, 1, 64, 50, 30, False),      # the chunk wraps the ring
    ("q4_k_m", 4096, 14336, 32, 8, 4096, 100, 64, False),
    ("q4_k_m", 4096, 14336, 32, 8, 4096, 100, 64, True),
])
def test_prefill_layer_typed_matches_oracle(mix, dim, hidden, nh, nkv, M, start, S, wo_zero):
    G.say(f"kquant: layer {mix} dim={dim} hidden={hidden} M={M} start={start} S={S} "
          f"wo0={wo_zero}")
    L = G.lib()
    types = MIXES[mix]
    g = np.random.default_rng(dim + S + (1 if wo_zero else 0))
    W = _layer(g, types, dim, hidden, nh, nkv)
    if wo_zero:
        W["wo"] = _zero_weights(W["wo"], types["wo"])
    kc, vc = D.ring(g, M, kv_dim=dim // nh * nkv, filled=start)
    X = g.standard_normal((S, dim)).astype(np.float32)
    th = O.theta_inv(D.THETA, 128)
    got, kc_g, vc_g = _run_layer(L, W, types, X, th, kc, vc, dim, hidden, nh, nkv, M, start, S)
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = O.prefill_layer_typed(W, types, X, kc_o, vc_o, start, S, dim, hidden, nh, nkv, th)
    err = float(np.abs(got - ref).max())
    scale = float(np.abs(ref).max())
    assert err <= (2e-5 if wo_zero else 2e-3) * scale, (err, scale)
    slots = np.arange(start, start + S) % M
    untouched = np.setdiff1d(np.arange(M), slots)
    assert np.array_equal(kc_g[untouched], kc[untouched])
    assert np.array_equal(vc_g[untouched], vc[untouched])
    for a, b in ((kc_g, kc_o), (vc_g, vc_o)):
        fa, fb = D.f16_bits_to_f32(a[slots]), D.f16_bits_to_f32(b[slots])
        ulp = np.spacing(np.maximum(np.abs(fa), np.abs(fb)).astype(np.float16)).astype(np.float32)
        row = np.abs(fb).max(axis=1, keepdims=True)
        assert np.all(np.abs(fa - fb) <= ulp + 1e-5 * row)


@pytest.mark.parametrize("mix", ["q4_k_m", "mixed"])
def test_prefill_layer_typed_packed_is_bit_identical(mix):
    G.say(f"kquant: packed layer {mix}")
    L = G.lib()
    dim, hidden, nh, nkv, M, start, S = 512, 1024, 4, 1, 64, 10, 20
    types = MIXES[mix]
    g = np.random.default_rng(71 + len(mix))
    W = _layer(g, types, dim, hidden, nh, nkv)
    kc, vc = D.ring(g, M, kv_dim=dim // nh * nkv, filled=start)
    X = g.standard_normal((S, dim)).astype(np.float32)
    th = O.theta_inv(D.THETA, 128)
    want, kc_w, vc_w = _run_layer(L, W, types, X, th, kc, vc, dim, hidden, nh, nkv, M, start, S)
    kvd = dim // nh * nkv
    shapes = {"wq": (dim, dim), "wk": (kvd, dim), "wv": (kvd, dim), "wo": (dim, dim),
              "w1": (hidden, dim), "w3": (hidden, dim), "w2": (dim, hidden)}
    packs = {n: gpu_pack(W[n], types[n], *shapes[n]) for n in O.MATS}
    norms = {n: DB.from_array(W[n]) for n in ("rms_att", "rms_ffn")}
    lw = mia.LayerWeightsTyped(*[packs[n].ptr for n in O.MATS], *[types[n] for n in O.MATS],
                               norms["rms_att"].ptr, norms["rms_ffn"].ptr)
    dX, dth, dkc, dvc = DB.from_array(X), DB.from_array(th), DB.from_array(kc), DB.from_array(vc)
    check(L.mia_prefill_layer_typed_packed(dX.ptr, ctypes.byref(lw), dth.ptr, dkc.ptr, dvc.ptr,
                                           dim, hidden, nh, nkv, 1e-5, M, start, S, None),
          "layer_typed_packed")
    check(L.mia_stream_sync(None), "sync")
    assert np.array_equal(dX.download(X.shape, np.float32).view(np.uint32), want.view(np.uint32))
    assert np.array_equal(dkc.download(kc.shape, np.uint16), kc_w)
    assert np.array_equal(dvc.download(vc.shape, np.uint16), vc_w)


def test_prefill_layer_typed_all_q4_0_is_prefill_layer():
    G.say("kquant: layer_typed all Q4_0 == mia_prefill_layer")
    L = G.lib()
    dim, hidden, nh, nkv, M, start, S = 512, 1024, 4, 1, 64, 7, 16
    types = {k: O.TYPE_Q4_0 for k in O.MATS}
    g = np.random.default_rng(77)
    W = _layer(g, types, dim, hidden, nh, nkv)
    kc, vc = D.ring(g, M, kv_dim=dim // nh * nkv, filled=start)
    X = g.standard_normal((S, dim)).astype(np.float32)
    th = O.theta_inv(D.THETA, 128)
    got, kc_g, vc_g = _run_layer(L, W, types, X, th, kc, vc, dim, hidden, nh, nkv, M, start, S)
    dev = {k: DB.from_array(v) for k, v in W.items()}
    lw = mia.LayerWeights(*[dev[n].ptr for n in O.MATS], dev["rms_att"].ptr, dev["rms_ffn"].ptr)
    dX, dth, dkc, dvc = DB.from_array(X), DB.from_array(th), DB.from_array(kc), DB.from_array(vc)
    check(L.mia_prefill_layer(dX.ptr, ctypes.byref(lw), dth.ptr, dkc.ptr, dvc.ptr, dim, hidden,
                              nh, nkv, 1e-5, M, start, S, None), "prefill_layer")
    check(L.mia_stream_sync(None), "sync")
    assert np.array_equal(got, dX.download(X.shape, np.float32))
    assert np.array_equal(kc_g, dkc.download(kc.shape, np.uint16))
    assert np.array_equal(vc_g, dvc.download(vc.shape, np.uint16))
