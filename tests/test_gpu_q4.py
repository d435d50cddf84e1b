"""GPU parity of the W4A8 projections either side of the attention step
(mia_quantize_q8_0, mia_q4_0_matvec, mia_q4_0_matvec_qkv and their drop-in
forms) against the oracle (oracle/q4_oracle.c).

Bars:
- Q8_0 quantisation is bit-exact (scale bits and every int8).
- Matvec rows: each block term (wd * xd) * isum is rounded as the reference
  rounds it and only the fp32 order of the sum over a row's blocks differs, so
  |y - oracle| <= 2 * bpr * 2^-24 * sum_b |term_b| (the worst-case bound of two
  reassociated fp32 sums of bpr terms); a lost or doubled block, a wrong nibble
  or a wrong scale is larger than that by orders of magnitude.  The stated
  attention tolerance (2e-3 abs + 1e-2 rel) is checked as well.
- Where every term is an exact integer (unit scales), y is bit-exact."""

import ctypes

import numpy as np
import pytest

import _gpu as G
import _oracle as O
import anetransformers_amd as mia
from anetransformers_amd import DeviceBuffer as DB
from anetransformers_amd import check

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def _q8_bytes(q):
    return np.ascontiguousarray(q).view(np.uint8).reshape(-1)


def gpu_quantize(x):
    L = G.lib()
    dx = DB.from_array(np.ascontiguousarray(x, np.float32))
    dq = DB(x.size // 32 * 36)
    check(L.mia_quantize_q8_0(dx.ptr, dq.ptr, x.size, None), "quantize")
    check(L.mia_stream_sync(None), "sync")
    return dq.download(x.size // 32, O.Q8_DTYPE)


def gpu_matvec(W, xq, out_dim, in_dim):
    L = G.lib()
    dw, dx = DB.from_array(W), DB.from_array(xq)
    dy = DB(out_dim * 4)
    check(L.mia_q4_0_matvec(dw.ptr, dx.ptr, dy.ptr, out_dim, in_dim, None), "q4_0_matvec")
    check(L.mia_stream_sync(None), "sync")
    return dy.download(out_dim, np.float32)


def gpu_matvec_qkv(Wq, Wk, Wv, xq, dim, kv_dim, in_dim):
    L = G.lib()
    dwq, dwk, dwv, dx = (DB.from_array(a) for a in (Wq, Wk, Wv, xq))
    dyq, dyk, dyv = DB(dim * 4), DB(kv_dim * 4), DB(kv_dim * 4)
    check(L.mia_q4_0_matvec_qkv(dwq.ptr, dwk.ptr, dwv.ptr, dx.ptr, dyq.ptr, dyk.ptr, dyv.ptr, dim,
                                kv_dim, in_dim, None), "q4_0_matvec_qkv")
    check(L.mia_stream_sync(None), "sync")
    return (dyq.download(dim, np.float32), dyk.download(kv_dim, np.float32),
            dyv.download(kv_dim, np.float32))


def term_abs_sum(W, xq, out_dim, in_dim):
    """sum_b |(wd * xd) * isum_b| per row, in float64."""
    nb = in_dim // 32
    B = np.ascontiguousarray(W, np.uint8).reshape(out_dim, nb, 18)
    wd = B[:, :, 0:2].copy().view(np.float16).reshape(out_dim, nb).astype(np.float64)
    q = B[:, :, 2:].astype(np.int64)
    w = np.concatenate([(q & 0x0F) - 8, (q >> 4) - 8], axis=2)         # [out, nb, 32]
    isum = np.einsum("rbj,bj->rb", w, xq["qs"].astype(np.int64))
    return (np.abs(wd * xq["d"].astype(np.float64)[None, :] * isum)).sum(axis=1)


def assert_rows_close(y, ref, W, xq, out_dim, in_dim, what):
    bound = 2 * (in_dim // 32) * U * term_abs_sum(W, xq, out_dim, in_dim) + 1e-30
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    worst = int(np.argmax(err / bound))
    assert np.all(err <= bound), (what, worst, float(err[worst]), float(bound[worst]))
    assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), what


def special_activation(g, n):
    x = (g.standard_normal(n) * 3.0).astype(np.float32)
    x[0:32] = 0.0                                          # all-zero block
    x[32:64] = 0.0
    x[32:40] = [127.0, -127.0, 63.5, 62.5, 0.5, 1.5, 2.5, -2.5]   # d = 1: ties to even
    x[64:96] = np.float32(1e-30) * (np.arange(32) - 16)    # tiny block
    x[96:128] = 0.0
    x[100] = -5e4                                          # one huge negative value
    return x


@pytest.mark.parametrize("n", [32, 4096, 14336])
def test_quantize_bit_exact(n):
    G.say(f"q4: quantize n={n}")
    g = np.random.default_rng(n)
    x = special_activation(g, n) if n >= 128 else (g.standard_normal(n) * 0.1).astype(np.float32)
    got, want = gpu_quantize(x), O.quantize_q8_0(x)
    assert np.array_equal(_q8_bytes(got), _q8_bytes(want))


@pytest.mark.parametrize("out_dim,in_dim", [(4096, 4096), (37, 256), (1, 64), (130, 14336),
                                            (9, 192)])
def test_matvec_matches_oracle(out_dim, in_dim):
    G.say(f"q4: matvec {out_dim}x{in_dim}")
    g = np.random.default_rng(out_dim * 7 + in_dim)
    W = O.make_q4_0(g, out_dim, in_dim)
    xq = O.quantize_q8_0(special_activation(g, in_dim) if in_dim >= 128
                         else g.standard_normal(in_dim).astype(np.float32))
    y = gpu_matvec(W, xq, out_dim, in_dim)
    ref = O.q4_0_q8_0_matvec(W, xq, out_dim, in_dim)
    assert_rows_close(y, ref, W, xq, out_dim, in_dim, f"{out_dim}x{in_dim}")


def test_matvec_exact_on_integer_terms():
    # wd = xd = 1: every term is an integer below 2^24, so any summation order
    # gives the exact result; extreme nibbles 0 and 15 (weights -8 and +7)
    G.say("q4: matvec integer terms")
    g = np.random.default_rng(5)
    out_dim, in_dim = 6, 14336
    nb = in_dim // 32
    B = np.empty((out_dim, nb, 18), np.uint8)
    B[:, :, 0:2] = np.array([0x00, 0x3C], np.uint8)        # fp16 1.0
    B[0, :, 2:] = 0x00                                      # all -8
    B[1, :, 2:] = 0xFF                                      # all +7
    B[2:, :, 2:] = g.integers(0, 256, (out_dim - 2, nb, 16), dtype=np.uint8)
    W = B.reshape(out_dim, nb * 18)
    xq = np.zeros(nb, O.Q8_DTYPE)
    xq["d"] = 1.0
    xq["qs"] = g.integers(-128, 128, (nb, 32))
    xq["qs"][:, 0] = -128
    y = gpu_matvec(W, xq, out_dim, in_dim)
    want = O.q4_0_q8_0_matvec(W, xq, out_dim, in_dim)
    assert np.array_equal(y, want)
    assert y[0] == np.float32(-8 * xq["qs"].astype(np.int64).sum())


@pytest.mark.parametrize("dim,kv_dim,in_dim", [(4096, 1024, 4096), (37, 5, 128), (8, 8, 64)])
def test_matvec_qkv_matches_oracle(dim, kv_dim, in_dim):
    G.say(f"q4: qkv {dim}/{kv_dim}x{in_dim}")
    g = np.random.default_rng(dim + kv_dim)
    Wq, Wk, Wv = (O.make_q4_0(g, r, in_dim) for r in (dim, kv_dim, kv_dim))
    xq = O.quantize_q8_0(g.standard_normal(in_dim).astype(np.float32))
    got = gpu_matvec_qkv(Wq, Wk, Wv, xq, dim, kv_dim, in_dim)
    want = O.q4_0_q8_0_matvec_qkv(Wq, Wk, Wv, xq, dim, kv_dim, in_dim)
    for y, ref, W, r, name in zip(got, want, (Wq, Wk, Wv), (dim, kv_dim, kv_dim), "qkv"):
        assert_rows_close(y, ref, W, xq, r, in_dim, name)


def test_quantize_then_matvec_chain_on_device():
    # the decode layer's order: quantize(xb) -> QKV, quantize(attn out) -> Wo,
    # with the Q8_0 blocks never leaving the device
    G.say("q4: device chain")
    L = G.lib()
    g = np.random.default_rng(11)
    dim, kv_dim = 4096, 1024
    x = g.standard_normal(dim).astype(np.float32)
    Wq, Wk, Wv, Wo = (O.make_q4_0(g, r, dim) for r in (dim, kv_dim, kv_dim, dim))
    dx, dq8 = DB.from_array(x), DB(dim // 32 * 36)
    dwq, dwk, dwv, dwo = (DB.from_array(a) for a in (Wq, Wk, Wv, Wo))
    dyq, dyk, dyv, dyo = DB(dim * 4), DB(kv_dim * 4), DB(kv_dim * 4), DB(dim * 4)
    check(L.mia_quantize_q8_0(dx.ptr, dq8.ptr, dim, None), "quantize")
    check(L.mia_q4_0_matvec_qkv(dwq.ptr, dwk.ptr, dwv.ptr, dq8.ptr, dyq.ptr, dyk.ptr, dyv.ptr, dim,
                                kv_dim, dim, None), "qkv")
    check(L.mia_quantize_q8_0(dyq.ptr, dq8.ptr, dim, None), "quantize 2")
    check(L.mia_q4_0_matvec(dwo.ptr, dq8.ptr, dyo.ptr, dim, dim, None), "wo")
    check(L.mia_stream_sync(None), "sync")
    xq = O.quantize_q8_0(x)
    yq, yk, yv = O.q4_0_q8_0_matvec_qkv(Wq, Wk, Wv, xq, dim, kv_dim, dim)
    got_q = dyq.download(dim, np.float32)
    assert_rows_close(got_q, yq, Wq, xq, dim, dim, "q")
    assert_rows_close(dyk.download(kv_dim, np.float32), yk, Wk, xq, kv_dim, dim, "k")
    assert_rows_close(dyv.download(kv_dim, np.float32), yv, Wv, xq, kv_dim, dim, "v")
    # the second stage from the device's own q (the reference feeds its own)
    xq2 = O.quantize_q8_0(got_q)
    assert np.array_equal(_q8_bytes(dq8.download(dim // 32, O.Q8_DTYPE)), _q8_bytes(xq2))
    assert_rows_close(dyo.download(dim, np.float32), O.q4_0_q8_0_matvec(Wo, xq2, dim, dim), Wo,
                      xq2, dim, dim, "o")


def test_dropin_projections():
    # mistral_model.h:833-842 and 866-867 through the reference's names, with
    # host activations and device weights
    G.say("q4: drop-in")
    L = G.lib()
    L.mia_dropin_set_abort(0)
    g = np.random.default_rng(13)
    dim, kv_dim = 256, 64
    xb = g.standard_normal(dim).astype(np.float32)
    Wq, Wk, Wv = (O.make_q4_0(g, r, dim) for r in (dim, kv_dim, kv_dim))
    dwq, dwk, dwv = (DB.from_array(a) for a in (Wq, Wk, Wv))
    xq = np.zeros(dim // 32, O.Q8_DTYPE)
    L.mia_dropin_quantize_q8_0(xb.ctypes.data, xq.ctypes.data, dim)
    assert L.mia_dropin_status() == 0, L.mia_last_error()
    want_xq = O.quantize_q8_0(xb)
    assert np.array_equal(_q8_bytes(xq), _q8_bytes(want_xq))
    yq, yk, yv = (np.zeros(n, np.float32) for n in (dim, kv_dim, kv_dim))
    L.mia_dropin_q4_matvec_sdot_parallel_fused_qkv(dwq.ptr, dwk.ptr, dwv.ptr, xq.ctypes.data,
                                                   yq.ctypes.data, yk.ctypes.data,
                                                   yv.ctypes.data, dim, kv_dim, dim)
    assert L.mia_dropin_status() == 0, L.mia_last_error()
    for y, ref, W, r in zip((yq, yk, yv), O.q4_0_q8_0_matvec_qkv(Wq, Wk, Wv, xq, dim, kv_dim, dim),
                            (Wq, Wk, Wv), (dim, kv_dim, kv_dim)):
        assert_rows_close(y, ref, W, xq, r, dim, "dropin qkv")
    yo = np.zeros(dim, np.float32)
    L.mia_dropin_q4_matvec_sdot_parallel(dwq.ptr, ctypes.c_uint32(2), xq.ctypes.data,
                                         yo.ctypes.data, dim, dim)
    assert L.mia_dropin_status() == 0
    assert np.array_equal(yo, yq)       # same kernel, same rows
    L.mia_dropin_q4_matvec_sdot_parallel(dwq.ptr, ctypes.c_uint32(8), xq.ctypes.data,
                                         yo.ctypes.data, dim, dim)   # Q8_0 weights
    assert L.mia_dropin_status() == mia.MIA_ERR_UNSUPPORTED
    L.mia_dropin_set_abort(1)


@pytest.mark.parametrize("out_dim,in_dim", [(4096, 4096), (37, 256), (130, 8192), (9, 64),
                                            (20, 2112)])
def test_fused_f32_input_is_bit_identical(out_dim, in_dim):
    # mia_q4_0_matvec_f32 quantises in every workgroup: y must equal
    # mia_quantize_q8_0 + mia_q4_0_matvec bit for bit, and the oracle's chain
    # within the reassociation bound
    G.say(f"q4: fused f32 {out_dim}x{in_dim}")
    L = G.lib()
    g = np.random.default_rng(out_dim + 3 * in_dim)
    W = O.make_q4_0(g, out_dim, in_dim)
    x = special_activation(g, in_dim) if in_dim >= 128 else g.standard_normal(in_dim).astype(
        np.float32)
    dw, dx, dy = DB.from_array(W), DB.from_array(x), DB(out_dim * 4)
    check(L.mia_q4_0_matvec_f32(dw.ptr, dx.ptr, dy.ptr, out_dim, in_dim, None), "matvec_f32")
    check(L.mia_stream_sync(None), "sync")
    y = dy.download(out_dim, np.float32)
    xq = gpu_quantize(x)
    assert np.array_equal(y, gpu_matvec(W, xq, out_dim, in_dim))
    assert_rows_close(y, O.q4_0_q8_0_matvec(W, O.quantize_q8_0(x), out_dim, in_dim), W, xq,
                      out_dim, in_dim, "fused")


@pytest.mark.parametrize("dim,kv_dim,in_dim", [(4096, 1024, 4096), (37, 5, 128)])
def test_fused_f32_qkv_is_bit_identical(dim, kv_dim, in_dim):
    G.say(f"q4: fused f32 qkv {dim}/{kv_dim}x{in_dim}")
    L = G.lib()
    g = np.random.default_rng(dim * 5 + kv_dim)
    Wq, Wk, Wv = (O.make_q4_0(g, r, in_dim) for r in (dim, kv_dim, kv_dim))
    x = g.standard_normal(in_dim).astype(np.float32)
    dwq, dwk, dwv, dx = (DB.from_array(a) for a in (Wq, Wk, Wv, x))
    dyq, dyk, dyv = DB(dim * 4), DB(kv_dim * 4), DB(kv_dim * 4)
    check(L.mia_q4_0_matvec_qkv_f32(dwq.ptr, dwk.ptr, dwv.ptr, dx.ptr, dyq.ptr, dyk.ptr, dyv.ptr,
                                    dim, kv_dim, in_dim, None), "qkv_f32")
    check(L.mia_stream_sync(None), "sync")
    got = (dyq.download(dim, np.float32), dyk.download(kv_dim, np.float32),
           dyv.download(kv_dim, np.float32))
    two = gpu_matvec_qkv(Wq, Wk, Wv, gpu_quantize(x), dim, kv_dim, in_dim)
    for a, b in zip(got, two):
        assert np.array_equal(a, b)
