"""GPU parity of the speculative verify with accept-only commit
(mia_attention_step_staged, mia_commit_staged and the drop-in's
mia_dropin_verify_stage / mia_dropin_verify_commit) against the oracle.

- The staged step's output equals S sequential decode steps (the verify loop
  of mistral/speculative.h:92-101), within the attention tolerance.
- The ring is bit-identical before and after the staged step.
- The staged rows are the rows mia_attention_step writes into the ring (bit
  for bit) and faithful roundings of the exact rotation.
- Committing n_keep rows gives the ring n_keep sequential decode steps
  leave: the accepted slots hold the drafts, every other slot is untouched.
- On a wrapped ring the rejected drafts of the reference's loop overwrite the
  oldest positions of the next step's window (speculative.h:336-341); after
  an accept-only commit the next decode step matches the oracle run on the
  accepted tokens only."""

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
ROW = D.KV_DIM * 2          # bytes of one fp16 ring row


def _p(a):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def staged(kc, vc, Q, K, V, M, start, S):
    """mia_attention_step_staged on device copies; returns out, the ring after
    the call and the staged K/V rows."""
    L = G.lib()
    dkc, dvc = DB.from_array(kc), DB.from_array(vc)
    dq, dk, dv, dth = DB.from_array(Q), DB.from_array(K), DB.from_array(V), DB.from_array(TH)
    dks, dvs = DB(S * ROW), DB(S * ROW)
    dout = DB(S * 4096 * 4)
    check(L.mia_attention_step_staged(dq.ptr, dk.ptr, dv.ptr, dth.ptr, dkc.ptr, dvc.ptr, dks.ptr,
                                      dvs.ptr, dout.ptr, 32, 8, 128, M, start, S, None), "staged")
    check(L.mia_stream_sync(None), "sync")
    return (dout.download((S, 4096), np.float32), dkc.download(kc.shape, np.uint16),
            dvc.download(vc.shape, np.uint16), dks.download((S, D.KV_DIM), np.uint16),
            dvs.download((S, D.KV_DIM), np.uint16))


@pytest.mark.parametrize("M,start,S", [(300, 1000, 8), (4096, 100, 5), (64, 200, 1),
                                       (4096, 17, 1), (65536, 70000, 8), (128, 100, 40)])
def test_staged_step_matches_sequential_and_leaves_ring(M, start, S):
    G.say(f"staged verify M={M} start={start} S={S}")
    g = D.rng(7 * M + start + S)
    kc, vc = D.ring(g, M, filled=None if start >= M else start)
    Q, K, V = D.normal(g, (S, 4096)), D.normal(g, (S, 1024)), D.normal(g, (S, 1024))
    out, kc_g, vc_g, ks, vs = staged(kc, vc, Q, K, V, M, start, S)
    assert np.array_equal(kc_g, kc) and np.array_equal(vc_g, vc), "ring touched before commit"
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = O.verify_steps(kc_o, vc_o, Q, K, V, start, S, TH, 32, 8, 128, M)
    D.check_close(out, ref, what=f"staged M={M} start={start} S={S}")
    # the staged rows, placed in their slots, are the ring the oracle leaves
    pos = np.arange(start, start + S)
    kc_c, vc_c = kc.copy(), vc.copy()
    kc_c[pos % M], vc_c[pos % M] = ks, vs
    D.check_ring(kc_c, kc_o, vc_c, vc_o, pos % M, K, pos, TH, "staged rows")
    # and bit for bit what the writing form of the step puts in the ring
    _, kc_w, vc_w = G.attention_step(kc, vc, Q, K, V, TH, M, start, S)
    assert np.array_equal(kc_w[pos % M], ks) and np.array_equal(vc_w[pos % M], vs)


def test_commit_keeps_only_accepted_rows_across_layers():
    # two layers of one cache ([layer][slot][kv_dim]), each staged with its
    # own drafts; the commit of 3 of 6 writes 3 slots per layer and nothing else
    G.say("commit 3 of 6, 2 layers, M=64 start=200")
    L = G.lib()
    M, start, S, keep, NLAY = 64, 200, 6, 3, 2
    g = D.rng(99)
    rings = [D.ring(g, M) for _ in range(NLAY)]
    kc = np.stack([r[0] for r in rings])
    vc = np.stack([r[1] for r in rings])
    dkc, dvc = DB.from_array(kc), DB.from_array(vc)
    dks, dvs = DB(NLAY * S * ROW), DB(NLAY * S * ROW)
    dth = DB.from_array(TH)
    dout = DB(S * 4096 * 4)
    Ks, Vs = [], []
    for l in range(NLAY):
        Q, K, V = D.normal(g, (S, 4096)), D.normal(g, (S, 1024)), D.normal(g, (S, 1024))
        Ks.append(K)
        Vs.append(V)
        dq, dk, dv = DB.from_array(Q), DB.from_array(K), DB.from_array(V)
        check(L.mia_attention_step_staged(dq.ptr, dk.ptr, dv.ptr, dth.ptr, dkc.ptr + l * M * ROW,
                                          dvc.ptr + l * M * ROW, dks.ptr + l * S * ROW,
                                          dvs.ptr + l * S * ROW, dout.ptr, 32, 8, 128, M, start,
                                          S, None), f"staged layer {l}")
    check(L.mia_commit_staged(dkc.ptr, dvc.ptr, dks.ptr, dvs.ptr, NLAY, S, keep, start, M,
                              D.KV_DIM, None), "commit")
    check(L.mia_stream_sync(None), "sync")
    kc_g, vc_g = dkc.download(kc.shape, np.uint16), dvc.download(vc.shape, np.uint16)
    ks = dks.download((NLAY, S, D.KV_DIM), np.uint16)
    vs = dvs.download((NLAY, S, D.KV_DIM), np.uint16)
    slots = np.arange(start, start + keep) % M
    for l in range(NLAY):
        want_k, want_v = kc[l].copy(), vc[l].copy()
        want_k[slots], want_v[slots] = ks[l, :keep], vs[l, :keep]
        assert np.array_equal(kc_g[l], want_k) and np.array_equal(vc_g[l], want_v), l
        assert np.array_equal(vs[l], D.to_f16_bits(Vs[l]))
        D.check_rotated_k(ks[l], Ks[l], np.arange(start, start + S), TH, what=f"layer {l}")


def test_accept_only_commit_keeps_the_next_window_intact():
    # M = 64, drafts at 200..205 (slots 8..13), 2 accepted.  The next step, at
    # position 202, attends 139..202: slots 11..13 must still hold positions
    # 139..141.  Rejected drafts 3..5 carry keys aligned with the next query in
    # the lowest-frequency RoPE pair (rotation ~ identity there) and V = 100,
    # so a stale draft left in the ring dominates the next output.
    G.say("stale-draft check M=64 start=200 S=6 keep=2")
    M, start, S, keep = 64, 200, 6, 2
    g = D.rng(5)
    kc, vc = D.ring(g, M)
    Q, K, V = D.normal(g, (S, 4096)), D.normal(g, (S, 1024)), D.normal(g, (S, 1024))
    K.reshape(S, 8, 128)[3:, :, 126] = 40.0
    V[3:] = 100.0
    q2, k2, v2 = D.normal(g, 4096), D.normal(g, 1024), D.normal(g, 1024)
    q2.reshape(32, 128)[:, 126] = 40.0
    nxt = start + keep

    # accept-only: staged step, commit 2, then the decode step at 202
    L = G.lib()
    dkc, dvc = DB.from_array(kc), DB.from_array(vc)
    dq, dk, dv, dth = DB.from_array(Q), DB.from_array(K), DB.from_array(V), DB.from_array(TH)
    dks, dvs, dout = DB(S * ROW), DB(S * ROW), DB(S * 4096 * 4)
    check(L.mia_attention_step_staged(dq.ptr, dk.ptr, dv.ptr, dth.ptr, dkc.ptr, dvc.ptr, dks.ptr,
                                      dvs.ptr, dout.ptr, 32, 8, 128, M, start, S, None), "staged")
    check(L.mia_commit_staged(dkc.ptr, dvc.ptr, dks.ptr, dvs.ptr, 1, S, keep, start, M, D.KV_DIM,
                              None), "commit")
    dq2, dk2, dv2, dout2 = DB.from_array(q2), DB.from_array(k2), DB.from_array(v2), DB(4096 * 4)
    check(L.mia_decode_step(dq2.ptr, dk2.ptr, dv2.ptr, dth.ptr, dkc.ptr, dvc.ptr, dout2.ptr, 32, 8,
                            128, M, nxt, None), "next step")
    check(L.mia_stream_sync(None), "sync")
    got = dout2.download(4096, np.float32)

    # oracle: the accepted tokens only, then the next step
    kc_o, vc_o = kc.copy(), vc.copy()
    O.verify_steps(kc_o, vc_o, Q[:keep], K[:keep], V[:keep], start, keep, TH, 32, 8, 128, M)
    ref = O.decode_step(kc_o, vc_o, q2, k2, v2, nxt, TH, 32, 8, 128, M)
    D.check_close(got, ref, what="next step after accept-only commit")

    # the reference's loop (every draft written) corrupts that window
    kc_s, vc_s = kc.copy(), vc.copy()
    O.verify_steps(kc_s, vc_s, Q, K, V, start, S, TH, 32, 8, 128, M)
    stale = O.decode_step(kc_s, vc_s, q2, k2, v2, nxt, TH, 32, 8, 128, M)
    assert np.abs(stale - ref).max() > 10.0


def test_dropin_verify_stage_then_commit():
    G.say("dropin verify_stage/commit 3 layers M=300 start=1000 S=5 keep=4")
    L = G.lib()
    L.mia_dropin_set_abort(0)
    NLAY, M, start, S, keep = 3, 300, 1000, 5, 4
    kv = mia.KVCache()
    L.mia_dropin_kv_alloc(ctypes.byref(kv), NLAY, 8, 128, M)
    assert L.mia_dropin_status() == 0
    g = D.rng(31)
    rings, ins, staged_rows = [], [], []
    for l in range(NLAY):
        kc, vc = D.ring(g, M)
        rings.append((kc, vc))
        check(L.mia_memcpy_h2d(kv.k_cache + l * M * ROW, _p(kc), kc.nbytes), "load k")
        check(L.mia_memcpy_h2d(kv.v_cache + l * M * ROW, _p(vc), vc.nbytes), "load v")
    kv.len = M
    th = TH.copy()
    # commit before anything is staged fails
    L.mia_dropin_verify_commit(ctypes.byref(kv), start, keep)
    assert L.mia_dropin_status() == mia.MIA_ERR_INVALID
    for l in range(NLAY):
        Q, K, V = D.normal(g, (S, 4096)), D.normal(g, (S, 1024)), D.normal(g, (S, 1024))
        ins.append((Q, K, V))
        out = np.zeros((S, 4096), np.float32)
        L.mia_dropin_verify_stage(ctypes.byref(kv), l, _p(Q), _p(K), _p(V), start, S, _p(th), 32,
                                  8, _p(out))
        assert L.mia_dropin_status() == 0, L.mia_last_error()
        kc_o, vc_o = rings[l][0].copy(), rings[l][1].copy()
        ref = O.verify_steps(kc_o, vc_o, Q, K, V, start, S, TH, 32, 8, 128, M)
        D.check_close(out, ref, what=f"dropin staged layer {l}")
        staged_rows.append((kc_o, vc_o))
    # ring untouched so far; a commit at another position is refused
    for l in range(NLAY):
        a = np.empty((M, D.KV_DIM), np.uint16)
        check(L.mia_memcpy_d2h(_p(a), kv.k_cache + l * M * ROW, a.nbytes), "read")
        assert np.array_equal(a, rings[l][0])
    L.mia_dropin_verify_commit(ctypes.byref(kv), start + 1, keep)
    assert L.mia_dropin_status() == mia.MIA_ERR_INVALID
    L.mia_dropin_verify_commit(ctypes.byref(kv), start, keep)
    assert L.mia_dropin_status() == 0, L.mia_last_error()
    slots = np.arange(start, start + keep) % M
    for l in range(NLAY):
        a = np.empty((M, D.KV_DIM), np.uint16)
        b = np.empty((M, D.KV_DIM), np.uint16)
        check(L.mia_memcpy_d2h(_p(a), kv.k_cache + l * M * ROW, a.nbytes), "read k")
        check(L.mia_memcpy_d2h(_p(b), kv.v_cache + l * M * ROW, b.nbytes), "read v")
        kc, vc = rings[l]
        kc_o, vc_o = staged_rows[l]
        want_v = vc.copy()
        want_v[slots] = vc_o[slots]
        assert np.array_equal(b, want_v), l
        untouched = np.setdiff1d(np.arange(M), slots)
        assert np.array_equal(a[untouched], kc[untouched]), l
        D.check_rotated_k(a[slots], ins[l][1][:keep], np.arange(start, start + keep), TH,
                          what=f"committed k layer {l}")
    assert kv.len == M
    # the batch is spent: a second commit is refused
    L.mia_dropin_verify_commit(ctypes.byref(kv), start, keep)
    assert L.mia_dropin_status() == mia.MIA_ERR_INVALID
    L.mia_dropin_kv_free(ctypes.byref(kv))
    L.mia_dropin_set_abort(1)
