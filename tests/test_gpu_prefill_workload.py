"""GPU parity of the prefill layer's GEMM launches at the benchmarked shapes
(Mistral-7B width, S = 512 new tokens after 1536 cached) against float64
products of the dequantised weights (mistral/mistral_ane_prefill.h:1018-1042,
1081-1110: dequantised tiles, cblas_sgemm, vDSP_vadd, SwiGLU).

At S = 512 the launches take other grids than the small-S tests: QKV, Wo and
W2 split K over workgroups (partial products summed by a second kernel), W1 and
W3 run unsplit, and W3's SwiGLU epilogue writes W2's input as fp16 hi + lo
planes.  Each output checked is held to an elementwise bound derived from the
arithmetic (fp32 sums of K products, x carried as hi + lo to 2^-22 relative
and 2^-25 absolute), computed alongside the float64 reference."""

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

U = 2.0 ** -24  # unit roundoff of fp32


def _gemm_bound(x_abs, w_abs, K, ex=None, rel=0.0):
    """Bound on |y - x.W^T| for the GPU GEMM: fp32 sums of K terms (each
    split into hi and lo products) over x = hi + lo (to 2^-22 relative,
    2^-25 absolute below fp16's normal range), plus the inputs' own error:
    ex elementwise, or rel * |x|."""
    b = ((2 * K * U + 2.0 ** -22 + rel) * (x_abs @ w_abs.T)
         + 2.0 ** -25 * w_abs.sum(axis=1)[None, :])
    if ex is not None:
        b = b + ex @ w_abs.T
    return b


@pytest.mark.parametrize("layout", ["gguf", "packed"])
@pytest.mark.parametrize("N,K", [(6144, 4096), (4096, 4096), (14336, 4096), (4096, 14336)])
def test_gemm_workload_shapes_sampled_columns(N, K, layout):
    # QKV (stacked 6144 rows), Wo, W1 / W3, W2 at S 512: 96 sampled output
    # columns (weight rows) of each against the float64 product
    S = 512
    G.say(f"gemm workload shape S={S} N={N} K={K} {layout}")
    L = G.lib()
    g = np.random.default_rng(N + 3 * K)
    W = O.make_q4_0(g, N, K)
    X = g.standard_normal((S, K)).astype(np.float32)
    X[3, :256] *= 1e-5  # tiny activations: the lo halves underflow in fp16
    dw = DB.from_array(W)
    dx, dy = DB.from_array(X), DB(S * N * 4)
    if layout == "packed":
        dp = DB(W.size)
        check(L.mia_q4_0_pack_gemm(dw.ptr, dp.ptr, N, K, None), "pack")
        check(L.mia_q4_0_gemm_packed_f32(dp.ptr, dx.ptr, dy.ptr, N, K, S, None), "gemm packed")
    else:
        check(L.mia_q4_0_gemm_f32(dw.ptr, dx.ptr, dy.ptr, N, K, S, None), "gemm")
    check(L.mia_stream_sync(None), "sync")
    got = dy.download((S, N), np.float32).astype(np.float64)
    cols = np.sort(g.choice(N, 96, replace=False))
    cols[0], cols[-1] = 0, N - 1
    Wd = O.dequant_q4_0(W[cols], len(cols), K)
    x64 = X.astype(np.float64)
    ref = x64 @ Wd.T
    bound = _gemm_bound(np.abs(x64), np.abs(Wd), K)
    err = np.abs(got[:, cols] - ref)
    assert np.all(err <= bound), float((err / bound).max())
    D.check_close(got[:, cols], ref, what=f"gemm S={S} N={N} K={K}")


def _layer(g, dim, hidden, nh, nkv):
    kvd = dim // nh * nkv
    return {"wq": O.make_q4_0(g, dim, dim), "wk": O.make_q4_0(g, kvd, dim),
            "wv": O.make_q4_0(g, kvd, dim), "wo": O.make_q4_0(g, dim, dim),
            "w1": O.make_q4_0(g, hidden, dim), "w3": O.make_q4_0(g, hidden, dim),
            "w2": O.make_q4_0(g, dim, hidden),
            "rms_att": (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32),
            "rms_ffn": (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32)}


def _run_layer(W, X, kc, vc, dim, hidden, nh, nkv, M, start, S, packed):
    L = G.lib()
    kvd = dim // nh * nkv
    shapes = {"wq": (dim, dim), "wk": (kvd, dim), "wv": (kvd, dim), "wo": (dim, dim),
              "w1": (hidden, dim), "w3": (hidden, dim), "w2": (dim, hidden)}
    dev = {k: DB.from_array(v) for k, v in W.items()}
    if packed:
        for k, (n, kk) in shapes.items():
            dp = DB(W[k].size)
            check(L.mia_q4_0_pack_gemm(dev[k].ptr, dp.ptr, n, kk, None), "pack")
            dev[k] = dp
    lw = mia.LayerWeights(*[dev[n].ptr for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3",
                                                  "rms_att", "rms_ffn")])
    th = O.theta_inv(D.THETA, 128)
    dX, dth, dkc, dvc = DB.from_array(X), DB.from_array(th), DB.from_array(kc), DB.from_array(vc)
    fn = "mia_prefill_layer_packed" if packed else "mia_prefill_layer"
    check(getattr(L, fn)(dX.ptr, ctypes.byref(lw), dth.ptr, dkc.ptr, dvc.ptr, dim, hidden, nh, nkv,
                         1e-5, M, start, S, None), fn)
    check(L.mia_stream_sync(None), "sync")
    return (dX.download(X.shape, np.float32), dkc.download(kc.shape, np.uint16),
            dvc.download(vc.shape, np.uint16))


def _rmsnorm64(X, w, eps=1e-5):
    x = X.astype(np.float64)
    return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)


def _zero_scales(Wq):
    B = Wq.reshape(Wq.shape[0], -1, 18).copy()
    B[:, :, 0:2] = 0
    return B.reshape(Wq.shape)


@pytest.mark.parametrize("packed", [False, True])
def test_prefill_layer_ffn_at_workload_shape(packed):
    # Wo = 0: the attention still runs and writes the ring but adds nothing,
    # so X' = X + W2 . (silu(W1 h) * (W3 h)), h = RMSNorm(X) * w_ffn.  W1 and
    # W3 run unsplit at this shape, W3's epilogue forms the SwiGLU product as
    # W2's hi + lo input planes, and W2 splits K four ways with the residual
    # add in the sum kernel.  128 output columns against float64, each within
    # the bound propagated through the chain.
    dim, hidden, nh, nkv, M, start, S = 4096, 14336, 32, 8, 4096, 1536, 512
    G.say(f"prefill layer FFN at the workload shape S={S} after {start}, packed={packed}")
    g = np.random.default_rng(4242)
    W = _layer(g, dim, hidden, nh, nkv)
    W["wo"] = _zero_scales(W["wo"])
    kc, vc = D.ring(g, M, kv_dim=dim // nh * nkv, filled=start)
    X = g.standard_normal((S, dim)).astype(np.float32)
    got, _, _ = _run_layer(W, X, kc, vc, dim, hidden, nh, nkv, M, start, S, packed)

    h = _rmsnorm64(X, W["rms_ffn"])
    rh = (np.log2(dim) + 8) * U                      # the GPU RMSNorm's relative error
    ah = np.abs(h)
    W1d = O.dequant_q4_0(W["w1"], hidden, dim)
    g1 = h @ W1d.T
    e1 = _gemm_bound(ah, np.abs(W1d), dim, rel=rh)
    del W1d
    W3d = O.dequant_q4_0(W["w3"], hidden, dim)
    g3 = h @ W3d.T
    e3 = _gemm_bound(ah, np.abs(W3d), dim, rel=rh)
    del W3d
    sig = 1.0 / (1.0 + np.exp(-g1))
    silu = g1 * sig
    a = silu * g3
    dsilu = np.abs(sig * (1.0 + g1 * (1.0 - sig)))
    # first-order propagation, the epilogue's own fp32 work (sigmoid through
    # exp and a divide, two products: 16 roundings) and the plane split
    ea = (dsilu * e1 * np.abs(g3) + np.abs(silu) * e3 + 16 * U * np.abs(a)
          + 2.0 ** -22 * np.abs(a) + 2.0 ** -25)
    del g1, g3, sig, silu, dsilu, e1, e3
    cols = np.sort(g.choice(dim, 128, replace=False))
    W2d = O.dequant_q4_0(W["w2"][cols], len(cols), hidden)
    ref = X.astype(np.float64)[:, cols] + a @ W2d.T
    bound = (_gemm_bound(np.abs(a), np.abs(W2d), hidden, ea)
             + U * (np.abs(ref) + np.abs(X[:, cols])))
    err = np.abs(got[:, cols].astype(np.float64) - ref)
    assert np.all(err <= bound), float((err / bound).max())


def test_prefill_layer_qkv_and_attention_at_workload_shape():
    # Wo = identity (exact in Q4_0) and W2 = 0: X' - X is the attention
    # output, held to the attention tolerance (2e-3 abs / 1e-2 rel) against
    # the oracle's attention of the oracle's Q over the ring as the GPU wrote
    # it; the new ring rows (the QKV launch's K and V, K rotated) within one
    # fp16 ulp of the float64 K / V, plus 1e-5 of the row's scale for rotated
    # keys near zero.
    dim, hidden, nh, nkv, M, start, S = 4096, 14336, 32, 8, 4096, 1536, 512
    G.say(f"prefill layer QKV + attention at the workload shape S={S} after {start}")
    g = np.random.default_rng(2424)
    W = _layer(g, dim, hidden, nh, nkv)
    n = dim // 32
    B = np.zeros((dim, n, 18), np.uint8)                 # identity Wo
    B[:, :, 2:] = 0x88
    r = np.arange(dim)
    b, i = r // 32, r % 32
    B[r, b, 0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    lo = i < 16
    B[r[lo], b[lo], 2 + i[lo]] = 0x8C
    B[r[~lo], b[~lo], 2 + i[~lo] - 16] = 0xC8
    W["wo"] = B.reshape(dim, n * 18)
    W["w2"] = _zero_scales(W["w2"])
    kvd = dim // nh * nkv
    kc, vc = D.ring(g, M, kv_dim=kvd, filled=start)
    X = g.standard_normal((S, dim)).astype(np.float32)
    got, kc_g, vc_g = _run_layer(W, X, kc, vc, dim, hidden, nh, nkv, M, start, S, False)
    att = got.astype(np.float64) - X
    th = O.theta_inv(D.THETA, 128)
    Qo = np.ascontiguousarray(O.q4_0_gemm(W["wq"], dim, dim, O.rmsnorm_batch(X, W["rms_att"])),
                              np.float32)
    O.load().ora_apply_rope_batch(Qo.ctypes.data, None, start, th.ctypes.data, nh, nkv, 128, S)
    ref = O.attention_batch_parallel(Qo, kc_g, vc_g, nh, nkv, 128, M, start, S)
    D.check_close(att, ref, what="layer attention at the workload shape")
    # new ring rows against float64 K / V
    h = _rmsnorm64(X, W["rms_att"])
    K64 = h @ O.dequant_q4_0(W["wk"], kvd, dim).T
    V64 = h @ O.dequant_q4_0(W["wv"], kvd, dim).T
    pos = np.arange(start, start + S)
    K64 = np.stack([D.rope_f64(K64[t], int(p), th, nkv, 128) for t, p in enumerate(pos)])
    slots = pos % M
    for ring_g, exact in ((kc_g, K64), (vc_g, V64)):
        fa = D.f16_bits_to_f32(ring_g[slots]).astype(np.float64)
        ulp = np.spacing(np.maximum(np.abs(fa), np.abs(exact)).astype(np.float16)).astype(np.float64)
        row = np.abs(exact).max(axis=1, keepdims=True)
        assert np.all(np.abs(fa - exact) <= ulp + 1e-5 * row)
    untouched = np.setdiff1d(np.arange(M), slots)
    assert np.array_equal(kc_g[untouched], kc[untouched])
    assert np.array_equal(vc_g[untouched], vc[untouched])
