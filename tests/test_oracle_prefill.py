"""CPU checks that pin the prefill-layer oracle (oracle/prefill_oracle.c) to the
reference's BLAS prefill layer (mistral/mistral_ane_prefill.h:163-175,
907-1110; mistral_model.h:174-199) by known answers and float64
restatements, not by retyping its formulas."""

import numpy as np
import pytest

import _data as D
import _oracle as O


def test_rmsnorm_known_answers():
    dim = 64
    w = np.linspace(0.5, 2.0, dim).astype(np.float32)
    X = np.zeros((3, dim), np.float32)
    X[1] = 3.0                                      # constant row: 3 / sqrt(9 + eps) * w
    X[2, 0] = 8.0                                   # one spike: 8 / sqrt(64/dim + eps) * w0
    out = O.rmsnorm_batch(X, w, 1e-5)
    assert not out[0].any()
    assert np.allclose(out[1], 3.0 / np.sqrt(9.0 + 1e-5) * w, rtol=1e-6)
    assert np.isclose(out[2, 0], 8.0 / np.sqrt(1.0 + 1e-5) * w[0], rtol=1e-6)
    assert not out[2, 1:].any()


def test_rmsnorm_matches_float64():
    g = np.random.default_rng(1)
    X = (g.standard_normal((5, 4096)) * 3).astype(np.float32)
    w = g.standard_normal(4096).astype(np.float32)
    out = O.rmsnorm_batch(X, w, 1e-5)
    x = X.astype(np.float64)
    ref = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + 1e-5) * w
    assert np.allclose(out, ref, rtol=2e-6, atol=1e-6)


def test_dequant_rows_is_exact():
    g = np.random.default_rng(2)
    W = O.make_q4_0(g, 9, 256)
    assert np.array_equal(O.dequant_q4_0_rows(W, 9, 256).astype(np.float64),
                          O.dequant_q4_0(W, 9, 256))


@pytest.mark.parametrize("S,out_dim,in_dim", [(1, 16, 64), (7, 33, 256), (16, 64, 1024)])
def test_gemm_matches_float64(S, out_dim, in_dim):
    g = np.random.default_rng(S + out_dim)
    W = O.make_q4_0(g, out_dim, in_dim)
    X = g.standard_normal((S, in_dim)).astype(np.float32)
    Y = O.q4_0_gemm(W, out_dim, in_dim, X)
    Wd = O.dequant_q4_0(W, out_dim, in_dim)
    ref = X.astype(np.float64) @ Wd.T
    bound = in_dim * 2.0 ** -24 * (np.abs(X.astype(np.float64)) @ np.abs(Wd).T) + 1e-30
    assert np.all(np.abs(Y - ref) <= bound)
    # one token alone gives the same row as within the batch
    assert np.array_equal(O.q4_0_gemm(W, out_dim, in_dim, X[-1:])[0], Y[-1])


def test_silu_mul_known_answers_and_float64():
    g = np.array([0.0, 50.0, -50.0, 1.0, -1.0], np.float32)
    u = np.array([3.0, 2.0, 2.0, 1.0, 1.0], np.float32)
    h = O.silu_mul(g, u)
    assert h[0] == 0.0 and h[1] == np.float32(100.0) and abs(h[2]) < 1e-18
    x = np.random.default_rng(3).standard_normal(1000).astype(np.float32) * 6
    y = np.random.default_rng(4).standard_normal(1000).astype(np.float32)
    ref = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64))) * y
    assert np.allclose(O.silu_mul(x, y), ref, rtol=1e-6, atol=1e-7)


def _rope64(x, pos, th, n_heads, hd):
    x = x.reshape(n_heads, hd // 2, 2).astype(np.float64)
    ang = (th.astype(np.float32) * np.float32(pos)).astype(np.float64)  # fp32 angle
    c, s = np.cos(ang), np.sin(ang)
    e, o = x[..., 0], x[..., 1]
    return np.stack([e * c - o * s, o * c + e * s], axis=-1).reshape(-1)


def _layer64(W, X, kc, vc, start, S, dim, hidden, nh, nkv, th, eps, types=None):
    """The prefill layer in float64 (fp16 ring entries as the ring holds them);
    types: GGML type of each matrix (default all Q4_0)."""
    hd, M = dim // nh, kc.shape[0]
    kvd = nkv * hd
    types = types or {k: O.TYPE_Q4_0 for k in O.MATS}
    dq = {k: O.dequant_typed(W[k], types[k], *shape).astype(np.float64) for k, shape in
          (("wq", (dim, dim)), ("wk", (kvd, dim)), ("wv", (kvd, dim)), ("wo", (dim, dim)),
           ("w1", (hidden, dim)), ("w3", (hidden, dim)), ("w2", (dim, hidden)))}

    def rms(x, w):
        return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)

    x = X.astype(np.float64)
    xn = rms(x, W["rms_att"])
    Q, K, V = xn @ dq["wq"].T, xn @ dq["wk"].T, xn @ dq["wv"].T
    kring = D.f16_bits_to_f32(kc).astype(np.float64)
    vring = D.f16_bits_to_f32(vc).astype(np.float64)
    for t in range(S):
        slot = (start + t) % M
        kring[slot] = _rope64(K[t], start + t, th, nkv, hd).astype(np.float16)
        vring[slot] = V[t].astype(np.float16)
    A = np.zeros((S, dim))
    for t in range(S):
        p = start + t
        q = _rope64(Q[t], p, th, nh, hd).reshape(nh, hd)
        lo = max(0, p + 1 - M)
        slots = [pp % M for pp in range(lo, p + 1)]
        for h in range(nh):
            kvh = h // (nh // nkv)
            ks = kring[slots][:, kvh * hd:(kvh + 1) * hd]
            vs = vring[slots][:, kvh * hd:(kvh + 1) * hd]
            sc = ks @ q[h] / np.sqrt(hd)
            pr = np.exp(sc - sc.max())
            A[t, h * hd:(h + 1) * hd] = (pr / pr.sum()) @ vs
    x1 = x + A @ dq["wo"].T
    xn2 = rms(x1, W["rms_ffn"])
    G, U = xn2 @ dq["w1"].T, xn2 @ dq["w3"].T
    H = G / (1.0 + np.exp(-G)) * U
    return x1 + H @ dq["w2"].T, kring


def make_layer(g, dim, hidden, nh, nkv):
    kvd = dim // nh * nkv
    W = {"wq": O.make_q4_0(g, dim, dim), "wk": O.make_q4_0(g, kvd, dim),
         "wv": O.make_q4_0(g, kvd, dim), "wo": O.make_q4_0(g, dim, dim),
         "w1": O.make_q4_0(g, hidden, dim), "w3": O.make_q4_0(g, hidden, dim),
         "w2": O.make_q4_0(g, dim, hidden),
         "rms_att": (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32),
         "rms_ffn": (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32)}
    return W


def test_prefill_layer_matches_float64():
    g = np.random.default_rng(7)
    dim, hidden, nh, nkv, M, start, S = 256, 512, 4, 1, 32, 5, 8
    W = make_layer(g, dim, hidden, nh, nkv)
    kvd = dim // nh * nkv
    kc = np.zeros((M, kvd), np.uint16)
    vc = np.zeros((M, kvd), np.uint16)
    kc[:start] = D.to_f16_bits(g.standard_normal((start, kvd)).astype(np.float32))
    vc[:start] = D.to_f16_bits(g.standard_normal((start, kvd)).astype(np.float32))
    X = g.standard_normal((S, dim)).astype(np.float32)
    th = O.theta_inv(1e6, dim // nh)
    ref, kring = _layer64(W, X, kc, vc, start, S, dim, hidden, nh, nkv, th, 1e-5)
    kc_o, vc_o = kc.copy(), vc.copy()
    out = O.prefill_layer(W, X, kc_o, vc_o, start, S, dim, hidden, nh, nkv, th)
    assert np.abs(out - ref).max() <= 2e-4 * max(1.0, np.abs(ref).max())
    # the ring holds the layer's fp16 keys and values at the chunk's slots
    slots = np.arange(start, start + S) % M
    assert np.abs(D.f16_bits_to_f32(kc_o[slots]) - kring[slots]).max() <= 2e-3 * max(
        1.0, np.abs(kring[slots]).max())
    untouched = np.setdiff1d(np.arange(M), slots)
    assert np.array_equal(kc_o[untouched], kc[untouched])
