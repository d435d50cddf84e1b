"""GPU parity: attention at caller-given positions, through the C ABI and the
drop-in, against the oracle's restatement of mistral_layer_prefill_chunk
(mistral/mistral_model.h:908-1075): phase 1 rotates and writes every token at
positions[t] (a later token in the same slot wins), phase 2 attends each
token's window over the ring as written."""

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

TH = O.theta_inv(D.THETA, D.HD)

CASES = [
    (4096, list(range(1000, 1032))),                    # mistral_prefill's contiguous chunk
    (64, [100, 130, 101, 37, 500]),                     # unsorted; 130 recycles a slot of 100's window
    (64, [10, 74, 11, 138]),                            # three tokens in slot 10
    (48, [1000, 999, 998, 997]),                        # descending on a wrapped ring
    (65536, [70000 + 3 * i for i in range(16)]),        # strided on the wrapped 65536 ring
    (65536, [70000, 66536, 131000, 5, 65535, 131071]),  # scattered over the whole ring
    # chunks longer than 64 tokens find each slot's last writer through the
    # per-slot area: every slot taken 2-3 times, then (the area must be back
    # at rest after the first) an unsorted chunk with collisions on a larger
    # ring
    (64, list(range(200, 330))),
    (4096, [int(x) for x in np.random.default_rng(5).permutation(np.arange(5000, 5100))]
     + [5003 + 4096, 5050 + 8192, 5099 - 4096]),
]


def _chunk_gpu(kc, vc, Q, K, V, positions, M):
    lib = G.lib()
    S = len(positions)
    P = np.ascontiguousarray(positions, np.int32)
    dkc, dvc = DB.from_array(kc), DB.from_array(vc)
    dq, dk, dv, dth, dp = (DB.from_array(x) for x in (Q, K, V, TH, P))
    dout = DB(S * 4096 * 4)
    check(lib.mia_attention_chunk(dq.ptr, dk.ptr, dv.ptr, dp.ptr, dth.ptr, dkc.ptr, dvc.ptr,
                                  dout.ptr, 32, 8, 128, M, S, None), "attention_chunk")
    check(lib.mia_stream_sync(None), "sync")
    return (dout.download((S, 4096), np.float32), dkc.download(kc.shape, np.uint16),
            dvc.download(vc.shape, np.uint16))


@pytest.mark.parametrize("M,positions", CASES)
def test_attention_chunk_vs_oracle(M, positions):
    G.say(f"attention_chunk M={M} S={len(positions)} positions[:4]={positions[:4]}")
    g = D.rng(800 + M + len(positions))
    S = len(positions)
    kc, vc = D.ring(g, M)
    Q, K, V = D.normal(g, (S, 4096)), D.normal(g, (S, 1024)), D.normal(g, (S, 1024))
    out, kc_g, vc_g = _chunk_gpu(kc, vc, Q, K, V, positions, M)
    kc_o, vc_o = kc.copy(), vc.copy()
    ref, _ = O.prefill_chunk_attention(kc_o, vc_o, Q, K, V, positions, TH, 32, 8, 128, M)
    D.check_close(out, ref, what=f"chunk M={M}")
    # the ring: each written slot holds its last writer
    owner = {}
    for t, p in enumerate(positions):
        owner[p % M] = t
    slots = np.array(sorted(owner))
    toks = [owner[s] for s in slots]
    D.check_ring(kc_g, kc_o, vc_g, vc_o, slots, K[toks], np.asarray(positions)[toks], TH,
                 f"chunk ring M={M}")


def test_attention_positions_ring_as_it_stands():
    # phase 2 alone: rotated q, the ring untouched, each token at its own
    # position == the S=1 attention per token (gqa_attention_neon)
    G.say("attention_positions M=8192 S=24 scattered")
    lib = G.lib()
    g = D.rng(820)
    M = 8192
    positions = np.array([5, 8191, 8192, 12000, 100, 20000, 3, 16383] * 3, np.int32)
    S = len(positions)
    kc, vc = D.ring(g, M, spike_every=512)
    Q = D.normal(g, (S, 4096))
    dkc, dvc, dq, dp = DB.from_array(kc), DB.from_array(vc), DB.from_array(Q), DB.from_array(positions)
    dout = DB(S * 4096 * 4)
    check(lib.mia_attention_positions(dq.ptr, dout.ptr, dkc.ptr, dvc.ptr, dp.ptr, 32, 8, 128, M,
                                      S, None), "attention_positions")
    check(lib.mia_stream_sync(None), "sync")
    out = dout.download((S, 4096), np.float32)
    for t, p in enumerate(positions):
        ref = O.gqa_attention(Q[t], kc, vc, 32, 4, 128, M, int(p))
        D.check_close(out[t], ref, what=f"positions t={t} pos={p}")
    assert np.array_equal(dkc.download(kc.shape, np.uint16), kc)


def test_attention_positions_negative_position_gives_zero_row():
    G.say("attention_positions with a negative position")
    lib = G.lib()
    g = D.rng(821)
    M = 256
    kc, vc = D.ring(g, M)
    positions = np.array([40, -1, 300], np.int32)
    Q = D.normal(g, (3, 4096))
    dkc, dvc, dq, dp = DB.from_array(kc), DB.from_array(vc), DB.from_array(Q), DB.from_array(positions)
    dout = DB(3 * 4096 * 4)
    check(lib.mia_attention_positions(dq.ptr, dout.ptr, dkc.ptr, dvc.ptr, dp.ptr, 32, 8, 128, M,
                                      3, None), "attention_positions")
    check(lib.mia_stream_sync(None), "sync")
    out = dout.download((3, 4096), np.float32)
    assert np.all(out[1] == 0.0)
    for t in (0, 2):
        ref = O.gqa_attention(Q[t], kc, vc, 32, 4, 128, M, int(positions[t]))
        D.check_close(out[t], ref, what=f"t={t}")


def test_attention_positions_largest_positions():
    # positions up to INT_MAX: the window is the whole ring (its length is
    # formed without pos + 1), checked against the float64 brute force
    G.say("attention_positions with positions up to INT_MAX")
    lib = G.lib()
    g = D.rng(823)
    M = 1024
    kc, vc = D.ring(g, M)
    positions = np.array([2**31 - 1, 2**31 - 2, M - 1, M], np.int32)
    S = len(positions)
    Q = D.normal(g, (S, 4096))
    dkc, dvc, dq, dp = DB.from_array(kc), DB.from_array(vc), DB.from_array(Q), DB.from_array(positions)
    dout = DB(S * 4096 * 4)
    check(lib.mia_attention_positions(dq.ptr, dout.ptr, dkc.ptr, dvc.ptr, dp.ptr, 32, 8, 128, M,
                                      S, None), "attention_positions")
    check(lib.mia_stream_sync(None), "sync")
    out = dout.download((S, 4096), np.float32)
    for t, p in enumerate(positions):
        ref = D.gqa_decode_f64(Q[t], kc, vc, 32, 8, 128, M, int(p))
        D.check_close(out[t], ref, what=f"t={t} pos={p}")


def test_dropin_prefill_chunk_attention_two_layers():
    # the reference's per-layer call: host buffers, len bookkeeping (:952)
    G.say("dropin prefill_chunk_attention 2 layers M=512")
    lib = G.lib()
    g = D.rng(822)
    n_layers, M = 2, 512
    kv = mia.KVCache()
    lib.mia_dropin_kv_alloc(ctypes.byref(kv), n_layers, 8, 128, M)
    rings = [D.ring(g, M, filled=300) for _ in range(n_layers)]
    for l, (kc, vc) in enumerate(rings):
        off = l * M * 1024 * 2
        check(lib.mia_memcpy_h2d(kv.k_cache + off, kc.ctypes.data, kc.nbytes), "h2d")
        check(lib.mia_memcpy_h2d(kv.v_cache + off, vc.ctypes.data, vc.nbytes), "h2d")
    positions = np.arange(300, 332, dtype=np.int32)
    try:
        for l in range(n_layers):
            Q, K, V = D.normal(g, (32, 4096)), D.normal(g, (32, 1024)), D.normal(g, (32, 1024))
            out = np.empty((32, 4096), np.float32)
            lib.mia_dropin_prefill_chunk_attention(ctypes.byref(kv), l, Q.ctypes.data,
                                                   K.ctypes.data, V.ctypes.data,
                                                   positions.ctypes.data, 32, TH.ctypes.data, 32,
                                                   8, out.ctypes.data)
            assert lib.mia_dropin_status() == 0
            kc_o, vc_o = rings[l][0].copy(), rings[l][1].copy()
            ref, _ = O.prefill_chunk_attention(kc_o, vc_o, Q, K, V, positions, TH, 32, 8, 128, M)
            D.check_close(out, ref, what=f"dropin chunk layer {l}")
        assert kv.len == 332
    finally:
        lib.mia_dropin_kv_free(ctypes.byref(kv))
