"""CPU tier: pins the oracle (oracle/miattn_oracle.c) before anything is
checked against it.  Each check is independent of the oracle's own code:
numpy's IEEE conversions, float64 closed forms and brute force over explicit
position lists, and the known-answer tests of the reference
(tests/test_mistral.m:414-518, 921-983; tests/test_blas_prefill.m:89-131).
"""

import ctypes

import numpy as np
import pytest

import _data as D
import _oracle as O


# ------------------------------------------------------------------ fp16 --

def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    got = O.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne():
    g = D.rng(1)
    halves = np.arange(65536, dtype=np.uint16).view(np.float16)
    finite = halves[np.isfinite(halves)].astype(np.float32)
    # exact values, midpoints between neighbours (ties) and random floats
    srt = np.unique(finite.astype(np.float64))
    mids = ((srt[:-1] + srt[1:]) / 2).astype(np.float32)
    rand = np.concatenate([
        D.normal(g, 200000),
        D.normal(g, 100000) * 1e-5,       # subnormal range
        D.normal(g, 100000) * 3e4,        # near overflow
        np.array([65504, 65519.99, 65520, 65536, 1e9, -1e9, 0.0, -0.0, 2**-25, 2**-24 * 1.5,
                  np.inf, -np.inf], dtype=np.float32),
    ])
    x = np.concatenate([finite, mids, rand]).astype(np.float32)
    got = O.f32_to_f16(x)
    with np.errstate(over="ignore"):  # values past 65520 round to inf on purpose
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_f16_nan_stays_nan():
    got = O.f32_to_f16(np.array([np.nan, -np.nan], dtype=np.float32))
    assert np.all(np.isnan(got.view(np.float16)))


# ------------------------------------------------------------------ RoPE --

def test_theta_inv_closed_form():
    for theta, hd in [(1e6, 128), (1e4, 128), (1e4, 32)]:
        th = O.theta_inv(theta, hd)
        ref = 1.0 / np.power(np.float64(theta), 2.0 * np.arange(hd // 2) / hd)
        assert np.allclose(th, ref, rtol=4e-7, atol=0), (theta, hd)


def test_rope_pos0_identity():
    # tests/test_mistral.m:414-452: position 0 is the identity
    g = D.rng(2)
    q = D.normal(g, 32 * 128)
    k = D.normal(g, 8 * 128)
    q0, k0 = q.copy(), k.copy()
    O.apply_rope(q, k, 0, O.theta_inv(1e6, 128), 32, 8, 128)
    assert np.array_equal(q, q0) and np.array_equal(k, k0)


@pytest.mark.parametrize("pos", [1, 511, 4096, 32768, 70007])
def test_rope_preserves_norm_and_matches_float64(pos):
    # tests/test_mistral.m:454-469 (norm to 1e-5) and a float64 rotation on the
    # same fp32 angle.  A swapped sign, a wrong pair index or a transposed
    # (cos, sin) fails the float64 comparison by O(1).
    g = D.rng(3 + pos)
    th = O.theta_inv(1e6, 128)
    q = D.normal(g, 32 * 128)
    k = D.normal(g, 8 * 128)
    qr, kr = q.copy(), k.copy()
    O.apply_rope(qr, kr, pos, th, 32, 8, 128)
    for x, y, n in [(q, qr, 32), (k, kr, 8)]:
        nx = np.linalg.norm(x.reshape(n, 128), axis=1)
        ny = np.linalg.norm(y.reshape(n, 128), axis=1)
        assert np.all(np.abs(nx - ny) / nx < 1e-5)
        ref = D.rope_f64(x, pos, th, n, 128)
        assert np.max(np.abs(y - ref)) < 2e-6


def test_rope_batch_is_per_token_rope():
    g = D.rng(4)
    th = O.theta_inv(1e6, 128)
    S = 5
    Q = D.normal(g, (S, 4096))
    ref = np.stack([D.rope_f64(Q[t], 100 + t, th, 32, 128) for t in range(S)])
    got = Q.copy()
    O.load().ora_apply_rope_batch(got.ctypes.data, None, 100, th.ctypes.data, 32, 8, 128, S)
    assert np.max(np.abs(got - ref)) < 2e-6


# --------------------------------------------------------------- softmax --

def test_softmax_known_answers():
    # tests/test_mistral.m:955-982
    assert np.allclose(O.softmax(np.ones(4, np.float32)), 0.25, atol=1e-6)
    d = O.softmax(np.array([100, 0, 0, 0], np.float32))
    assert d[0] > 0.999 and d[1] < 0.001


def test_softmax_float64():
    x = D.normal(D.rng(5), 1000) * 5
    ref = np.exp(x.astype(np.float64) - x.max())
    ref /= ref.sum()
    got = O.softmax(x)
    assert np.max(np.abs(got - ref)) < 1e-6 and abs(got.sum() - 1) < 1e-5


# -------------------------------------------------------------- KV cache --

def test_kv_slot_closed_form():
    # kv_cache.h:38-42: layer*M*kv_dim + (pos % M)*kv_dim elements
    lib = O.load()
    kv = O.OraKV()
    assert lib.ora_kv_alloc(ctypes.byref(kv), 3, 8, 128, 1000) == 0
    try:
        lib.ora_kv_k_at.restype = ctypes.c_void_p
        lib.ora_kv_k_at.argtypes = [ctypes.POINTER(O.OraKV), ctypes.c_int, ctypes.c_int]
        for layer, pos in [(0, 0), (1, 999), (2, 1000), (2, 70007), (1, 123456)]:
            addr = lib.ora_kv_k_at(ctypes.byref(kv), layer, pos)
            off = (addr - kv.k_cache) // 2
            assert off == layer * 1000 * 1024 + (pos % 1000) * 1024
    finally:
        lib.ora_kv_free(ctypes.byref(kv))


def test_kv_write_batch_slots_and_len():
    g = D.rng(6)
    M, S = 10, 4
    kc = np.zeros((M, 1024), np.uint16)
    vc = np.zeros((M, 1024), np.uint16)
    K = D.normal(g, (S, 1024))
    V = D.normal(g, (S, 1024))
    new_len = O.kv_write_batch(kc, vc, K, V, 8, 128, M, 8, S)   # positions 8..11
    for t in range(S):
        slot = (8 + t) % M
        assert np.array_equal(kc[slot], D.to_f16_bits(K[t]))
        assert np.array_equal(vc[slot], D.to_f16_bits(V[t]))
    assert new_len == M  # end_pos 12 > max_seq -> len = max_seq (mistral_ane_prefill.h:203)


# ----------------------------------------------------- S=1 attention ------

@pytest.mark.parametrize("n_heads,n_kv,hd,M,pos", [
    (8, 2, 32, 128, 40),      # mistral_test_config (tests/test_cpu_ref.h:33-41)
    (8, 2, 32, 128, 300),     # wrapped ring
    (32, 8, 128, 64, 63),     # full, not wrapped
    (32, 8, 128, 64, 200),    # wrapped
])
def test_gqa_attention_vs_float64(n_heads, n_kv, hd, M, pos):
    g = D.rng(7 + pos)
    kc, vc = D.ring(g, M, n_kv * hd)
    q = D.normal(g, n_heads * hd)
    got = O.gqa_attention(q, kc, vc, n_heads, n_heads // n_kv, hd, M, pos)
    ref = D.gqa_decode_f64(q, kc, vc, n_heads, n_kv, hd, M, pos)
    assert np.max(np.abs(got - ref)) < 2e-6


def test_gqa_single_position_returns_v_row():
    g = D.rng(8)
    kc, vc = D.ring(g, 16)
    q = D.normal(g, 4096)
    out = O.gqa_attention(q, kc, vc, 32, 4, 128, 16, 0)
    ref = D.f16_bits_to_f32(vc[0]).reshape(8, 128)[np.arange(32) // 4].reshape(-1)
    assert np.array_equal(out, ref)


def test_gqa_equal_keys_average_v():
    g = D.rng(9)
    kc, vc = D.ring(g, 50)
    kc[:] = kc[0]
    q = D.normal(g, 4096)
    out = O.gqa_attention(q, kc, vc, 32, 4, 128, 50, 29)   # window = slots 0..29
    mean = D.f16_bits_to_f32(vc[:30]).mean(axis=0).reshape(8, 128)
    assert np.max(np.abs(out.reshape(32, 128) - mean[np.arange(32) // 4])) < 1e-5


def test_gqa_broadcast_equals_expanded_mha():
    # tests/test_mistral.m:474-518: GQA == MHA over KV heads expanded 4x
    g = D.rng(10)
    M, pos = 40, 70
    kc, vc = D.ring(g, M, 2 * 32)
    q = D.normal(g, 8 * 32)
    gqa = O.gqa_attention(q, kc, vc, 8, 4, 32, M, pos)
    ke = kc.reshape(M, 2, 32)[:, np.arange(8) // 4].reshape(M, 256).copy()
    ve = vc.reshape(M, 2, 32)[:, np.arange(8) // 4].reshape(M, 256).copy()
    mha = O.gqa_attention(q, ke, ve, 8, 1, 32, M, pos)
    assert np.array_equal(gqa, mha)


def test_gqa_window_is_last_positions_oldest_first():
    # Index-revealing ring test: V carries the position id, keys are equal so
    # the output is the mean id of the attended window; out-of-window slots
    # are poisoned with keys that would dominate any leak.
    M, pos, hd = 16, 40, 32
    n_kv = 1
    kc = np.zeros((M, hd), np.uint16)
    vc = np.zeros((M, hd), np.uint16)
    win = D.window_positions(pos, M)
    for p in range(pos + 1):
        vc[p % M] = D.to_f16_bits(np.full(hd, p, np.float32))
    q = np.zeros(4 * hd, np.float32)
    out = O.gqa_attention(q, kc, vc, 4, 4, hd, M, pos)
    assert np.allclose(out, win.mean(), atol=1e-4)
    assert list(win) == list(range(25, 41))


# ----------------------------------------------------- S>1 attention ------

def test_attention_batch_equals_sequential_decode():
    # tests/test_blas_prefill.m:89-131: batched prefill == sequential S=1 steps
    g = D.rng(11)
    M, start, S = 256, 60, 12
    kc, vc = D.ring(g, M, 1024, filled=start + S)
    Q = D.normal(g, (S, 4096))
    batch = O.attention_batch(Q, kc, vc, 32, 8, 128, M, start, S)
    seq = np.stack([O.gqa_attention(Q[t], kc, vc, 32, 4, 128, M, start + t) for t in range(S)])
    assert np.max(np.abs(batch - seq)) < 2e-6


def test_attention_batch_matches_textbook_causal():
    # tests/test_cpu_ref.h:113-147 with contiguous K/V from position 0
    g = D.rng(12)
    S, M = 20, 64
    K = D.f16_bits_to_f32(D.to_f16_bits(D.normal(g, (S, 256))))
    V = D.f16_bits_to_f32(D.to_f16_bits(D.normal(g, (S, 256))))
    Q = D.normal(g, (S, 8 * 32))
    kc = np.zeros((M, 256), np.uint16)
    vc = np.zeros((M, 256), np.uint16)
    kc[:S] = D.to_f16_bits(K)
    vc[:S] = D.to_f16_bits(V)
    batch = O.attention_batch(Q, kc, vc, 8, 8, 32, M, 0, S)
    ref = O.ref_gqa_attention(Q, K, V, S, 8, 8, 32)
    assert np.max(np.abs(batch - ref)) < 2e-6


def test_ref_gqa_attention_vs_float64():
    g = D.rng(13)
    S, nh, nkv, hd = 9, 8, 2, 32
    q = D.normal(g, (S, nh * hd))
    k = D.normal(g, (S, nkv * hd))
    v = D.normal(g, (S, nkv * hd))
    got = O.ref_gqa_attention(q, k, v, S, nh, nkv, hd)
    for t in range(S):
        for h in range(nh):
            kvh = h // (nh // nkv)
            ref = D.attend_f64(q[t, h * hd:(h + 1) * hd], k[:t + 1, kvh * hd:(kvh + 1) * hd],
                               v[:t + 1, kvh * hd:(kvh + 1) * hd], 1 / np.sqrt(hd))
            assert np.max(np.abs(got[t, h * hd:(h + 1) * hd] - ref)) < 2e-6


def test_attention_batch_parallel_is_bitwise_same():
    g = D.rng(14)
    M, start, S = 128, 90, 6
    kc, vc = D.ring(g, M)
    Q = D.normal(g, (S, 4096))
    a = O.attention_batch(Q, kc, vc, 32, 8, 128, M, start, S)
    b = O.attention_batch_parallel(Q, kc, vc, 32, 8, 128, M, start, S, threads=4)
    assert np.array_equal(a, b)


# ------------------------------------------------------- step semantics --

def test_decode_step_writes_rounded_rotated_k_and_attends_it():
    g = D.rng(15)
    M, pos = 64, 100
    kc, vc = D.ring(g, M)
    th = O.theta_inv(1e6, 128)
    q, k, v = D.normal(g, 4096), D.normal(g, 1024), D.normal(g, 1024)
    kc2, vc2 = kc.copy(), vc.copy()
    out = O.decode_step(kc2, vc2, q, k, v, pos, th, 32, 8, 128, M)
    krot = D.rope_f64(k, pos, th, 8, 128)
    slot = pos % M
    assert np.max(np.abs(D.f16_bits_to_f32(kc2[slot]) - krot)) <= np.abs(krot).max() * 2**-10
    assert np.array_equal(vc2[slot], D.to_f16_bits(v))
    others = np.arange(M) != slot
    assert np.array_equal(kc2[others], kc[others])
    qrot = D.rope_f64(q, pos, th, 32, 128)
    ref = D.gqa_decode_f64(qrot, kc2, vc2, 32, 8, 128, M, pos)
    assert np.max(np.abs(out - ref)) < 1e-5


def test_verify_steps_wrapped_window_float64():
    # speculative.h:92-101: token t attends its own window, in which drafts
    # 0..t have replaced the oldest entries and later drafts have not.
    g = D.rng(16)
    M, start, S = 24, 100, 5
    kc, vc = D.ring(g, M)
    th = O.theta_inv(1e6, 128)
    Q, K, V = D.normal(g, (S, 4096)), D.normal(g, (S, 1024)), D.normal(g, (S, 1024))
    kc2, vc2 = kc.copy(), vc.copy()
    out = O.verify_steps(kc2, vc2, Q, K, V, start, S, th, 32, 8, 128, M)
    ktab, vtab = kc.copy(), vc.copy()
    for t in range(S):
        pos = start + t
        ktab[pos % M] = D.to_f16_bits(D.rope_f64(K[t], pos, th, 8, 128).astype(np.float32))
        vtab[pos % M] = D.to_f16_bits(V[t])
        qrot = D.rope_f64(Q[t], pos, th, 32, 128)
        ref = D.gqa_decode_f64(qrot, ktab, vtab, 32, 8, 128, M, pos)
        assert np.max(np.abs(out[t] - ref)) < 1e-5, t


# ------------------------------------------- chunked prefill (positions) --

def _chunk_inputs(g, S):
    return D.normal(g, (S, 4096)), D.normal(g, (S, 1024)), D.normal(g, (S, 1024))


def test_prefill_chunk_contiguous_equals_sequential_steps():
    # mistral_prefill's positions start + i (mistral_model.h:1089) on a ring
    # that does not wrap: phase 2 sees no later token in any window, so the
    # chunk is the verify loop's sequence of decode steps, bit for bit.
    g = D.rng(17)
    M, start, S = 128, 40, 32
    kc, vc = D.ring(g, M, filled=start)
    th = O.theta_inv(1e6, 128)
    Q, K, V = _chunk_inputs(g, S)
    kc1, vc1, kc2, vc2 = kc.copy(), vc.copy(), kc.copy(), vc.copy()
    out1, ln = O.prefill_chunk_attention(kc1, vc1, Q, K, V, np.arange(start, start + S), th, 32,
                                         8, 128, M)
    out2 = O.verify_steps(kc2, vc2, Q, K, V, start, S, th, 32, 8, 128, M)
    assert np.array_equal(out1, out2)
    assert np.array_equal(kc1, kc2) and np.array_equal(vc1, vc2)
    assert ln == start + S


@pytest.mark.parametrize("M,positions", [
    (64, [100, 130, 101, 37, 500]),      # unsorted; 130 lands in the window of 100
    (64, [10, 74, 11, 138]),             # 10, 74 and 138 share slot 10: the last wins
    (256, [0, 1, 2, 255, 3]),            # an unwrapped run plus a far token
    (48, [1000, 999, 998, 997]),         # descending on a wrapped ring
])
def test_prefill_chunk_positions_float64(M, positions):
    # Phase 1 writes every token (token order, last writer wins per slot),
    # then phase 2 attends each token's window [pos-L+1, pos] over that final
    # ring: float64 attention on the rotated q against the final ring, whose
    # rows are checked separately (V bit-exact, K the rounded rotation).
    g = D.rng(18 + M + len(positions))
    positions = np.asarray(positions)
    S = len(positions)
    kc, vc = D.ring(g, M)
    th = O.theta_inv(1e6, 128)
    Q, K, V = _chunk_inputs(g, S)
    kc2, vc2 = kc.copy(), vc.copy()
    out, ln = O.prefill_chunk_attention(kc2, vc2, Q, K, V, positions, th, 32, 8, 128, M)
    owner = {}
    for t, p in enumerate(positions):
        owner[int(p) % M] = t
    vt = vc.copy()
    for slot, t in owner.items():
        vt[slot] = D.to_f16_bits(V[t])
    assert np.array_equal(vc2, vt)
    slots = np.array(sorted(owner))
    D.check_rotated_k(kc2[slots], K[[owner[s] for s in slots]],
                      positions[[owner[s] for s in slots]], th, what="chunk ring")
    others = np.setdiff1d(np.arange(M), slots)
    assert np.array_equal(kc2[others], kc[others])
    for t, p in enumerate(positions):
        qrot = D.rope_f64(Q[t], int(p), th, 32, 128)
        ref = D.gqa_decode_f64(qrot, kc2, vc2, 32, 8, 128, M, int(p))
        assert np.max(np.abs(out[t] - ref)) < 1e-5, (t, p)
    # len bookkeeping of mistral_model.h:952 (it can pass max_seq once; never
    # read by the attention)
    want = 0
    for p in positions:
        if want < M and p + 1 > want:
            want = int(p) + 1
    assert ln == want


def test_prefill_chunk_sees_later_tokens_in_recycled_slots():
    # The write-all-then-attend order differs from sequential steps exactly
    # when a later token's slot falls in an earlier token's window: token 0
    # (position 100, window 37..100 on a 64-slot ring) sees position 130 in
    # slot 2, where sequential steps would still hold position 66.
    g = D.rng(19)
    M, positions = 64, np.array([100, 130])
    kc, vc = D.ring(g, M)
    th = O.theta_inv(1e6, 128)
    Q, K, V = _chunk_inputs(g, 2)
    V[1] = 50.0
    K[1] = 0.0
    out, _ = O.prefill_chunk_attention(kc.copy(), vc.copy(), Q, K, V, positions, th, 32, 8, 128, M)
    seq = O.verify_steps(kc.copy(), vc.copy(), Q, K, V, 100, 1, th, 32, 8, 128, M)
    assert np.max(np.abs(out[0] - seq[0])) > 1e-2
