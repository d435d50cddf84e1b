"""GPU tests of the Q4_0 GEMM tile layout (mia_q4_0_pack_gemm) and of the GEMM
and prefill layer on packed weights.

The layout has no reference counterpart: the reference dequantises the GGUF
blocks per 128-row tile (mistral/mistral_ane_prefill.h:1018-1042).  So:
  - the packed bytes are checked against the layout as the header states it,
    restated with numpy index arithmetic in tests/_gemm_layout.py (every byte
    of the input lands exactly once, which a permutation check confirms; the
    CPU tests of test_gemm_layout.py pin the restatement);
  - the GEMM and the layer on packed weights must be bit-identical to the
    same calls on the GGUF-layout weights, which test_gpu_prefill.py holds to
    the oracle; the small GEMM shapes are also held to the oracle's bound
    directly."""

import ctypes

import numpy as np
import pytest

import _data as D
import _gemm_layout as GL
import _gpu as G
import _oracle as O
import anetransformers_amd as mia
from anetransformers_amd import DeviceBuffer as DB
from anetransformers_amd import check

pytestmark = pytest.mark.gpu

def gpu_pack(dw, N, K):
    L = G.lib()
    dp = DB(N * K // 32 * 18)
    check(L.mia_q4_0_pack_gemm(dw.ptr, dp.ptr, N, K, None), "pack")
    return dp


def gemm(fn, dw, X, N, K):
    L = G.lib()
    S = X.shape[0]
    dx, dy = DB.from_array(np.ascontiguousarray(X, np.float32)), DB(S * N * 4)
    check(getattr(L, fn)(dw.ptr, dx.ptr, dy.ptr, N, K, S, None), fn)
    check(L.mia_stream_sync(None), "sync")
    return dy.download((S, N), np.float32)


@pytest.mark.parametrize("N,K", [(64, 64), (128, 256), (320, 1024), (64, 14336)])
def test_pack_layout(N, K):
    G.say(f"gemm tiles: pack N={N} K={K}")
    g = np.random.default_rng(N + K)
    W = O.make_q4_0(g, N, K)
    dp = gpu_pack(DB.from_array(W), N, K)
    check(G.lib().mia_stream_sync(None), "sync")
    got = dp.download((W.size,), np.uint8)
    want = GL.pack_layout(W, N, K)
    assert np.array_equal(got, want)
    # every input byte lands exactly once: the layout is a permutation
    perm = GL.pack_layout(np.arange(W.size, dtype=np.int64), N, K)
    assert np.array_equal(np.sort(perm), np.arange(W.size))


@pytest.mark.parametrize("S,N,K", [(1, 64, 64), (37, 128, 256), (128, 128, 4096),
                                   (200, 384, 4096), (130, 64, 14336)])
def test_packed_gemm_matches_gguf_layout_and_oracle(S, N, K):
    G.say(f"gemm tiles: packed gemm S={S} N={N} K={K}")
    g = np.random.default_rng(S * 5 + N)
    W = O.make_q4_0(g, N, K)
    X = g.standard_normal((S, K)).astype(np.float32)
    X[0, :64] *= 1e-6
    dw = DB.from_array(W)
    dp = gpu_pack(dw, N, K)
    got = gemm("mia_q4_0_gemm_packed_f32", dp, X, N, K)
    base = gemm("mia_q4_0_gemm_f32", dw, X, N, K)
    assert np.array_equal(got.view(np.uint32), base.view(np.uint32))
    ref = O.q4_0_gemm(W, N, K, X)
    Wd = O.dequant_q4_0(W, N, K)
    mag = np.abs(X.astype(np.float64)) @ np.abs(Wd).T
    bound = 2 * K * 2.0 ** -24 * mag + K * 6e-8 * np.abs(Wd).max()
    assert np.all(np.abs(got.astype(np.float64) - ref) <= bound)


@pytest.mark.parametrize("S,N,K", [(512, 6144, 4096), (512, 4096, 4096), (512, 14336, 4096),
                                   (512, 4096, 14336), (77, 1088, 4096)])
def test_packed_gemm_bit_identical_at_mistral_shapes(S, N, K):
    # the layer's shapes at S 512 (split-K for QKV, Wo and W2) and a ragged
    # grid (N not a multiple of the 256-row workgroup, S of the 64-token one)
    G.say(f"gemm tiles: packed gemm bit-identity S={S} N={N} K={K}")
    g = np.random.default_rng(N + K + S)
    W = O.make_q4_0(g, N, K)
    X = g.standard_normal((S, K)).astype(np.float32)
    dw = DB.from_array(W)
    dp = gpu_pack(dw, N, K)
    got = gemm("mia_q4_0_gemm_packed_f32", dp, X, N, K)
    base = gemm("mia_q4_0_gemm_f32", dw, X, N, K)
    assert np.array_equal(got.view(np.uint32), base.view(np.uint32))
    assert np.isfinite(got).all()


def _layer(g, dim, hidden, nh, nkv):
    kvd = dim // nh * nkv
    return {"wq": O.make_q4_0(g, dim, dim), "wk": O.make_q4_0(g, kvd, dim),
            "wv": O.make_q4_0(g, kvd, dim), "wo": O.make_q4_0(g, dim, dim),
            "w1": O.make_q4_0(g, hidden, dim), "w3": O.make_q4_0(g, hidden, dim),
            "w2": O.make_q4_0(g, dim, hidden),
            "rms_att": (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32),
            "rms_ffn": (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32)}


@pytest.mark.parametrize("dim,hidden,nh,nkv,M,start,S", [
    (1024, 1024, 8, 2, 4096, 1536, 512),
    (512, 1024, 4, 1, 64, 10, 20),
    (4096, 14336, 32, 8, 4096, 100, 64),
])
def test_packed_layer_bit_identical(dim, hidden, nh, nkv, M, start, S):
    G.say(f"gemm tiles: packed layer dim={dim} hidden={hidden} M={M} start={start} S={S}")
    L = G.lib()
    g = np.random.default_rng(dim + S + 1)
    W = _layer(g, dim, hidden, nh, nkv)
    kvd = dim // nh * nkv
    shapes = {"wq": (dim, dim), "wk": (kvd, dim), "wv": (kvd, dim), "wo": (dim, dim),
              "w1": (hidden, dim), "w3": (hidden, dim), "w2": (dim, hidden)}
    kc, vc = D.ring(g, M, kv_dim=kvd, filled=start)
    X = g.standard_normal((S, dim)).astype(np.float32)
    th = O.theta_inv(D.THETA, 128)
    dev = {k: DB.from_array(v) for k, v in W.items()}
    packed = {k: gpu_pack(dev[k], *shapes[k]) for k in shapes}
    names = ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "rms_att", "rms_ffn")
    outs = []
    for fn, src in (("mia_prefill_layer", dev), ("mia_prefill_layer_packed", {**dev, **packed})):
        lw = mia.LayerWeights(*[src[n].ptr for n in names])
        dX, dth = DB.from_array(X), DB.from_array(th)
        dkc, dvc = DB.from_array(kc), DB.from_array(vc)
        check(getattr(L, fn)(dX.ptr, ctypes.byref(lw), dth.ptr, dkc.ptr, dvc.ptr, dim, hidden, nh,
                             nkv, 1e-5, M, start, S, None), fn)
        check(L.mia_stream_sync(None), "sync")
        outs.append((dX.download(X.shape, np.float32), dkc.download(kc.shape, np.uint16),
                     dvc.download(vc.shape, np.uint16)))
    (x0, k0, v0), (x1, k1, v1) = outs
    assert np.array_equal(x0.view(np.uint32), x1.view(np.uint32))
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
