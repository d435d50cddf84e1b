"""GPU parity of the decode layer (mia_decode_layer: mistral_layer_decode_parallel,
mistral/mistral_model.h:818-899) and of the fused gate / up matvec
(mia_q4_0_matvec_pair[_f32], drop-in q4_matvec_sdot_parallel_fused_pair,
mistral_model.h:750-811) against the oracle (oracle/kquant_oracle.c,
oracle/q4_oracle.c).

Bars:
- The pair matvec: rows within the W4A8 bound of tests/test_gpu_q4.py; the
  fp32-input form bit-identical to quantize + matvec.
- The all-Q4_0 layer, and layers of Q4_K / Q6_K weights, bit-identical to the
  same steps issued one C-ABI call at a time (the fused prologues and
  epilogues add no arithmetic of their own).
- The layer against the oracle normwise within 1e-2 of the output's scale.
  fp32 reassociation, the attention's fp16 operands and the GPU's exp / sin /
  cos differ from the oracle's by ulps; the layer then re-quantises its
  activations to Q8_0 four times (as the reference does), and an activation
  that sits at a rounding boundary can take the neighbouring step: one value
  of a block moves by d = amax / 127, which moves each output by d times its
  weight, ~1e-3 of the output's scale per flipped value at Mistral-7B's width
  when the activations are heavy-tailed (measured: 3.3e-3 after four
  requantisations of a Q4_K_M layer).  The steps themselves are held to their
  own bars elsewhere, and the all-Q4_0 layer bit for bit to its steps (above).
  The ring's new row within one fp16 ulp (plus 1e-5 of the row's scale),
  every other slot untouched."""

import ctypes

import numpy as np
import pytest

import _data as D
import _gpu as G
import _oracle as O
import anetransformers_amd as mia
from anetransformers_amd import DeviceBuffer as DB
from anetransformers_amd import check

from test_gpu_q4 import assert_rows_close

pytestmark = pytest.mark.gpu

Q4_K_M = {"wq": O.TYPE_Q4_K, "wk": O.TYPE_Q4_K, "wv": O.TYPE_Q6_K, "wo": O.TYPE_Q4_K,
          "w1": O.TYPE_Q4_K, "w3": O.TYPE_Q4_K, "w2": O.TYPE_Q6_K}
MIXES = {
    "q4_0": {k: O.TYPE_Q4_0 for k in O.MATS},
    "q4_k_m": Q4_K_M,
    "mixed": {"wq": O.TYPE_Q4_0, "wk": O.TYPE_Q4_K, "wv": O.TYPE_Q4_0, "wo": O.TYPE_F16,
              "w1": O.TYPE_Q4_0, "w3": O.TYPE_Q6_K, "w2": O.TYPE_Q4_0},
}


def _layer(g, types, dim, hidden, nh, nkv):
    kvd = dim // nh * nkv
    shapes = {"wq": (dim, dim), "wk": (kvd, dim), "wv": (kvd, dim), "wo": (dim, dim),
              "w1": (hidden, dim), "w3": (hidden, dim), "w2": (dim, hidden)}
    W = {k: O.make_typed(g, types[k], *shapes[k], d_scale=0.07) for k in O.MATS}
    W["rms_att"] = (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    W["rms_ffn"] = (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    return W


def _gpu_layer(L, W, types, x, th, kc, vc, dim, hidden, nh, nkv, M, pos):
    dev = {k: DB.from_array(v) for k, v in W.items()}
    lw = mia.LayerWeightsTyped(*[dev[n].ptr for n in O.MATS], *[types[n] for n in O.MATS],
                               dev["rms_att"].ptr, dev["rms_ffn"].ptr)
    dx, dth, dkc, dvc = DB.from_array(x), DB.from_array(th), DB.from_array(kc), DB.from_array(vc)
    check(L.mia_decode_layer(dx.ptr, ctypes.byref(lw), dth.ptr, dkc.ptr, dvc.ptr, dim, hidden, nh,
                             nkv, 1e-5, M, pos, None), "decode_layer")
    check(L.mia_stream_sync(None), "sync")
    return (dx.download(x.shape, np.float32), dkc.download(kc.shape, np.uint16),
            dvc.download(vc.shape, np.uint16))


@pytest.mark.parametrize("mix,dim,hidden,nh,nkv,M,pos", [
    ("q4_0", 512, 1024, 4, 1, 64, 5),
    ("q4_k_m", 512, 1024, 4, 1, 64, 63),
    ("mixed", 512, 1024, 4, 1, 64, 100),          # the ring wraps
    ("q4_0", 4096, 14336, 32, 8, 4096, 100),
    ("q4_k_m", 4096, 14336, 32, 8, 1024, 5000),   # Mistral-7B, a wrapped 1024-slot ring
])
def test_decode_layer_matches_oracle(mix, dim, hidden, nh, nkv, M, pos):
    G.say(f"decode layer: {mix} dim={dim} hidden={hidden} M={M} pos={pos}")
    L = G.lib()
    types = MIXES[mix]
    g = np.random.default_rng(dim + pos)
    W = _layer(g, types, dim, hidden, nh, nkv)
    kc, vc = D.ring(g, M, kv_dim=dim // nh * nkv, filled=min(pos, M))
    x = g.standard_normal(dim).astype(np.float32)
    th = O.theta_inv(D.THETA, 128)
    got, kc_g, vc_g = _gpu_layer(L, W, types, x, th, kc, vc, dim, hidden, nh, nkv, M, pos)
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = O.decode_layer_typed(W, types, x, kc_o, vc_o, pos, dim, hidden, nh, nkv, th)
    err, scale = float(np.abs(got - ref).max()), float(np.abs(ref).max())
    assert err <= 1e-2 * scale, (err, scale)
    slot = pos % M
    others = np.setdiff1d(np.arange(M), [slot])
    assert np.array_equal(kc_g[others], kc[others]) and np.array_equal(vc_g[others], vc[others])
    for a, b in ((kc_g, kc_o), (vc_g, vc_o)):
        fa, fb = D.f16_bits_to_f32(a[slot]), D.f16_bits_to_f32(b[slot])
        ulp = np.spacing(np.maximum(np.abs(fa), np.abs(fb)).astype(np.float16)).astype(np.float32)
        assert np.all(np.abs(fa - fb) <= ulp + 1e-5 * np.abs(fb).max())


def test_decode_layer_is_its_steps_call_by_call():
    # all-Q4_0 layer == RMSNorm, fused QKV, mia_decode_step, Wo, residual,
    # RMSNorm, pair, SwiGLU, quantize, W2, residual issued one call at a time
    G.say("decode layer: call-by-call composition")
    L = G.lib()
    dim, hidden, nh, nkv, M, pos = 512, 1024, 4, 1, 64, 37
    kvd = dim // nh * nkv
    types = MIXES["q4_0"]
    g = np.random.default_rng(11)
    W = _layer(g, types, dim, hidden, nh, nkv)
    kc, vc = D.ring(g, M, kv_dim=kvd, filled=pos)
    x = g.standard_normal(dim).astype(np.float32)
    th = O.theta_inv(D.THETA, 128)
    got, kc_g, vc_g = _gpu_layer(L, W, types, x, th, kc, vc, dim, hidden, nh, nkv, M, pos)

    dev = {k: DB.from_array(v) for k, v in W.items()}
    dx, dth, dkc, dvc = DB.from_array(x), DB.from_array(th), DB.from_array(kc), DB.from_array(vc)
    xb, xb2, q, k, v = DB(dim * 4), DB(dim * 4), DB(dim * 4), DB(kvd * 4), DB(kvd * 4)
    hb, hb2, q8 = DB(hidden * 4), DB(hidden * 4), DB(hidden // 32 * 36)
    S = None
    check(L.mia_rmsnorm_f32(xb.ptr, dx.ptr, dev["rms_att"].ptr, dim, 1, 1e-5, S))
    check(L.mia_q4_0_matvec_qkv_f32(dev["wq"].ptr, dev["wk"].ptr, dev["wv"].ptr, xb.ptr, q.ptr,
                                    k.ptr, v.ptr, dim, kvd, dim, S))
    check(L.mia_decode_step(q.ptr, k.ptr, v.ptr, dth.ptr, dkc.ptr, dvc.ptr, xb2.ptr, nh, nkv, 128,
                            M, pos, S))
    check(L.mia_q4_0_matvec_f32(dev["wo"].ptr, xb2.ptr, xb.ptr, dim, dim, S))
    check(L.mia_stream_sync(S))
    x1 = dx.download(dim, np.float32) + xb.download(dim, np.float32)     # fp32 add, as vDSP_vadd
    dx.upload(x1)
    check(L.mia_rmsnorm_f32(xb.ptr, dx.ptr, dev["rms_ffn"].ptr, dim, 1, 1e-5, S))
    check(L.mia_q4_0_matvec_pair_f32(dev["w1"].ptr, dev["w3"].ptr, xb.ptr, hb.ptr, hb2.ptr,
                                     hidden, dim, S))
    check(L.mia_silu_mul_f32(hb.ptr, hb2.ptr, hidden, S))
    check(L.mia_quantize_q8_0(hb.ptr, q8.ptr, hidden, S))
    check(L.mia_q4_0_matvec(dev["w2"].ptr, q8.ptr, xb.ptr, dim, hidden, S))
    check(L.mia_stream_sync(S))
    want = x1 + xb.download(dim, np.float32)
    assert np.array_equal(kc_g, dkc.download(kc.shape, np.uint16))
    assert np.array_equal(vc_g, dvc.download(vc.shape, np.uint16))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


KMIXES = {
    "q4_k_m": Q4_K_M,
    "q6_k": {k: O.TYPE_Q6_K for k in O.MATS},
    # Q / K / V of three runs of types; gate and up of one type, as the
    # fused K-quant layer needs
    "kmix": {"wq": O.TYPE_Q6_K, "wk": O.TYPE_Q4_K, "wv": O.TYPE_Q6_K, "wo": O.TYPE_Q6_K,
             "w1": O.TYPE_Q6_K, "w3": O.TYPE_Q6_K, "w2": O.TYPE_Q4_K},
}


@pytest.mark.parametrize("mix,dim,hidden,nh,nkv", [
    ("q4_k_m", 512, 1024, 4, 1),      # inputs of 16 and 32 Q8_0 blocks
    ("q6_k", 1024, 2816, 8, 2),       # 32 and 88
    ("kmix", 2048, 5632, 16, 4),      # 64 and 176
])
def test_kquant_decode_layer_is_its_steps_call_by_call(mix, dim, hidden, nh, nkv):
    # Q4_K / Q6_K layer == RMSNorm, Q8_0 blocks, a typed matvec per matrix,
    # mia_decode_step, Q8_0 blocks, Wo, residual, RMSNorm, Q8_0 blocks,
    # W1, W3, SwiGLU, Q8_0 blocks, W2, residual, issued one call at a time
    G.say(f"decode layer: {mix} call-by-call composition dim={dim} hidden={hidden}")
    L = G.lib()
    M, pos = 64, 45
    kvd = dim // nh * nkv
    types = KMIXES[mix]
    g = np.random.default_rng(dim + hidden)
    W = _layer(g, types, dim, hidden, nh, nkv)
    kc, vc = D.ring(g, M, kv_dim=kvd, filled=pos)
    x = g.standard_normal(dim).astype(np.float32)
    th = O.theta_inv(D.THETA, 128)
    got, kc_g, vc_g = _gpu_layer(L, W, types, x, th, kc, vc, dim, hidden, nh, nkv, M, pos)

    dev = {k: DB.from_array(v) for k, v in W.items()}
    dx, dth, dkc, dvc = DB.from_array(x), DB.from_array(th), DB.from_array(kc), DB.from_array(vc)
    xb, xb2, q, k, v = DB(dim * 4), DB(dim * 4), DB(dim * 4), DB(kvd * 4), DB(kvd * 4)
    hb, hb2, q8 = DB(hidden * 4), DB(hidden * 4), DB(hidden // 32 * 36)
    S = None

    def mv(name, y, rows, cols):
        check(L.mia_matvec_q8(dev[name].ptr, types[name], q8.ptr, y.ptr, rows, cols, S), name)

    check(L.mia_rmsnorm_f32(xb.ptr, dx.ptr, dev["rms_att"].ptr, dim, 1, 1e-5, S))
    check(L.mia_quantize_q8_0(xb.ptr, q8.ptr, dim, S))
    mv("wq", q, dim, dim)
    mv("wk", k, kvd, dim)
    mv("wv", v, kvd, dim)
    check(L.mia_decode_step(q.ptr, k.ptr, v.ptr, dth.ptr, dkc.ptr, dvc.ptr, xb2.ptr, nh, nkv, 128,
                            M, pos, S))
    check(L.mia_quantize_q8_0(xb2.ptr, q8.ptr, dim, S))
    mv("wo", xb, dim, dim)
    check(L.mia_stream_sync(S))
    x1 = dx.download(dim, np.float32) + xb.download(dim, np.float32)
    dx.upload(x1)
    check(L.mia_rmsnorm_f32(xb.ptr, dx.ptr, dev["rms_ffn"].ptr, dim, 1, 1e-5, S))
    check(L.mia_quantize_q8_0(xb.ptr, q8.ptr, dim, S))
    mv("w1", hb, hidden, dim)
    mv("w3", hb2, hidden, dim)
    check(L.mia_silu_mul_f32(hb.ptr, hb2.ptr, hidden, S))
    check(L.mia_quantize_q8_0(hb.ptr, q8.ptr, hidden, S))
    mv("w2", xb, dim, hidden)
    check(L.mia_stream_sync(S))
    want = x1 + xb.download(dim, np.float32)
    assert np.array_equal(kc_g, dkc.download(kc.shape, np.uint16))
    assert np.array_equal(vc_g, dvc.download(vc.shape, np.uint16))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("out_dim,in_dim", [(14336, 4096), (37, 256), (130, 2112)])
def test_pair_matvec(out_dim, in_dim):
    G.say(f"pair matvec {out_dim}x{in_dim}")
    L = G.lib()
    g = np.random.default_rng(out_dim + in_dim)
    W1, W3 = O.make_q4_0(g, out_dim, in_dim), O.make_q4_0(g, out_dim, in_dim)
    xf = g.standard_normal(in_dim).astype(np.float32)
    xq = O.quantize_q8_0(xf)
    d1, d3, dq, dxf = DB.from_array(W1), DB.from_array(W3), DB.from_array(xq), DB.from_array(xf)
    y1, y3, z1, z3 = (DB(out_dim * 4) for _ in range(4))
    check(L.mia_q4_0_matvec_pair(d1.ptr, d3.ptr, dq.ptr, y1.ptr, y3.ptr, out_dim, in_dim, None))
    check(L.mia_q4_0_matvec_pair_f32(d1.ptr, d3.ptr, dxf.ptr, z1.ptr, z3.ptr, out_dim, in_dim,
                                     None))
    check(L.mia_stream_sync(None))
    a1, a3 = y1.download(out_dim, np.float32), y3.download(out_dim, np.float32)
    assert np.array_equal(a1, z1.download(out_dim, np.float32))
    assert np.array_equal(a3, z3.download(out_dim, np.float32))
    assert_rows_close(a1, O.q4_0_q8_0_matvec(W1, xq, out_dim, in_dim), W1, xq, out_dim, in_dim,
                      "pair w1")
    assert_rows_close(a3, O.q4_0_q8_0_matvec(W3, xq, out_dim, in_dim), W3, xq, out_dim, in_dim,
                      "pair w3")
    # the drop-in, host buffers
    h1, h3 = np.zeros(out_dim, np.float32), np.zeros(out_dim, np.float32)
    L.mia_dropin_q4_matvec_sdot_parallel_fused_pair(d1.ptr, d3.ptr, xq.ctypes.data,
                                                    h1.ctypes.data, h3.ctypes.data, out_dim,
                                                    in_dim)
    assert L.mia_dropin_status() == 0
    assert np.array_equal(h1, a1) and np.array_equal(h3, a3)
