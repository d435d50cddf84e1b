"""CPU checks that pin the K-quant / F16 / F32 weight oracle (oracle/kquant_oracle.c)
to the reference's paths for those types (mistral/dequant.h:23-29, 56-125,
283-307, 365-521; mistral_model.h:211-243, 581-670; mistral_ane_prefill.h:
907-1042) by known answers, the reference's own documented value table and
float64, not by restating its loops."""

import numpy as np
import pytest

import _data as D
import _oracle as O
import test_oracle_prefill as P


def _pack_q4_k_scales(sc, m):
    """The 12 scale bytes of a Q4_K block holding 6-bit sub-block scales
    sc[0..7] and mins m[0..7]: the inverse of get_scale_min_k4
    (dequant.h:58-66), which reads j < 4 from the low 6 bits of bytes j and
    j + 4, and j >= 4 from byte j + 4's nibbles plus the top 2 bits of bytes
    j - 4 and j."""
    q = np.zeros(12, np.uint8)
    for j in range(4):
        q[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    return q


def _q4_k_block(d, dmin, sc, m, nibbles):
    """nibbles[256] in value order: value 64 g + l (l < 32) is the low nibble
    of qs[32 g + l], value 64 g + 32 + l its high nibble (dequant.h:74-123)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    b[4:16] = _pack_q4_k_scales(np.asarray(sc), np.asarray(m))
    nib = np.asarray(nibbles).reshape(4, 2, 32)
    b[16:] = (nib[:, 0, :] | (nib[:, 1, :] << 4)).reshape(128)
    return b


def test_q4_k_known_answers_every_sub_block():
    # d = dmin = 1 (exact): every fp16 step is exact here, so value
    # 32 j + l = nibble * sc[j] - m[j], j the sub-block (both branches of
    # get_scale_min_k4: j < 4 and j >= 4, scales and mins up to 63)
    sc = [1, 7, 33, 63, 5, 48, 17, 60]
    m = [0, 3, 62, 9, 40, 2, 31, 63]
    g = np.random.default_rng(3)
    nib = g.integers(0, 16, 256)
    blk = _q4_k_block(1.0, 1.0, sc, m, nib)
    got = O.dequant_typed(blk[None], O.TYPE_Q4_K, 1, 256)[0]
    want = np.array([nib[i] * sc[i // 32] - m[i // 32] for i in range(256)], np.float32)
    assert np.array_equal(got, want)


def _q4_k_numpy(B, rows, cols):
    """The reference's fp16 arithmetic in numpy: every operation exact in
    float64 and rounded once to fp16 (numpy's float64 -> float16 is RNE)."""
    blk = np.ascontiguousarray(B, np.uint8).reshape(rows, cols // 256, 144)
    d = blk[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dmin = blk[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    q = blk[:, :, 4:16].astype(np.int64)
    sc = np.empty(q.shape[:2] + (8,), np.int64)
    mn = np.empty_like(sc)
    sc[..., :4] = q[..., 0:4] & 63
    mn[..., :4] = q[..., 4:8] & 63
    sc[..., 4:] = (q[..., 8:12] & 0xF) | ((q[..., 0:4] >> 6) << 4)
    mn[..., 4:] = (q[..., 8:12] >> 4) | ((q[..., 4:8] >> 6) << 4)
    vd = (d[..., None] * sc).astype(np.float16).astype(np.float64)
    vm = (dmin[..., None] * mn).astype(np.float16).astype(np.float64)
    qs = blk[:, :, 16:].astype(np.int64).reshape(rows, cols // 256, 4, 32)
    nib = np.stack([qs & 0xF, qs >> 4], axis=3)            # [r][b][group][lo/hi][32]
    nib = nib.reshape(rows, cols // 256, 8, 32)            # sub-block j = 2 group + half
    p = (nib * vd[..., None]).astype(np.float16).astype(np.float64)
    out = (p - vm[..., None]).astype(np.float16)
    return out.astype(np.float32).reshape(rows, cols)


def test_q4_k_fp16_arithmetic_matches_numpy():
    g = np.random.default_rng(5)
    W = O.make_q4_k(g, 64, 1024)
    # wide ranges: scales large enough to round in fp16, mins that cancel
    Wb = W.reshape(64, 4, 144).copy()
    Wb[:8, :, 0:2] = np.frombuffer(np.float16(3.7).tobytes(), np.uint8)
    Wb[8:16, :, 2:4] = np.frombuffer(np.float16(61.3).tobytes(), np.uint8)
    Wb[16:24, :, 0:4] = np.frombuffer(np.float16(1e-6).tobytes() * 2, np.uint8)  # subnormal steps
    W = Wb.reshape(64, 4 * 144)
    got = O.dequant_typed(W, O.TYPE_Q4_K, 64, 1024)
    want = _q4_k_numpy(W, 64, 1024)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _q6_k_encode(q6):
    """ql / qh bytes holding 6-bit values q6[256] per the value table the
    reference documents beside its Q6_K kernel (dequant.h:340-346):
      n =   0.. 63: ql[n]     & 0xF, qh[n]     >> 0 & 3
      n =  64..127: ql[n]     & 0xF, qh[n-64]  >> 4 & 3
      n = 128..191: ql[n-128] >> 4,  qh[n-128] >> 2 & 3
      n = 192..255: ql[n-128] >> 4,  qh[n-192] >> 6 & 3"""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for n in range(256):
        lo, hi = int(q6[n]) & 0xF, int(q6[n]) >> 4
        if n < 64:
            ql[n] |= lo
            qh[n] |= hi
        elif n < 128:
            ql[n] |= lo
            qh[n - 64] |= hi << 4
        elif n < 192:
            ql[n - 128] |= lo << 4
            qh[n - 128] |= hi << 2
        else:
            ql[n - 128] |= lo << 4
            qh[n - 192] |= hi << 6
    return ql, qh


def test_q6_k_value_table_and_scales():
    g = np.random.default_rng(6)
    q6 = g.permutation(np.tile(np.arange(64), 4))          # every 6-bit value 4 times
    ql, qh = _q6_k_encode(q6)
    sc = np.array([1, -2, 3, -4, 5, 127, -128, 8, 9, -10, 11, 12, -13, 14, 15, -16], np.int8)
    blk = np.concatenate([ql, qh, sc.view(np.uint8),
                          np.frombuffer(np.float16(0.5).tobytes(), np.uint8)])
    got = O.dequant_typed(blk[None], O.TYPE_Q6_K, 1, 256)[0]
    want = np.array([0.5 * sc[n // 16] * (int(q6[n]) - 32) for n in range(256)], np.float32)
    assert np.array_equal(got, want)


def test_f16_f32_and_q4_0_rows_exact():
    g = np.random.default_rng(7)
    for t in (O.TYPE_F16, O.TYPE_F32):
        W = O.make_typed(g, t, 8, 96)
        got = O.dequant_typed(W, t, 8, 96)
        dt = np.float16 if t == O.TYPE_F16 else np.float32
        assert np.array_equal(got, W.view(dt).astype(np.float32).reshape(8, 96))
    W = O.make_q4_0(g, 8, 96)
    assert np.array_equal(O.dequant_typed(W, O.TYPE_Q4_0, 8, 96), O.dequant_q4_0(W, 8, 96))


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q6_K, O.TYPE_F16, O.TYPE_F32, O.TYPE_Q4_0])
def test_typed_matvec_against_float64(t):
    g = np.random.default_rng(10 + t)
    rows, cols = 37, 1024
    W = O.make_typed(g, t, rows, cols)
    x = g.standard_normal(cols).astype(np.float32)
    y = O.typed_matvec(W, t, x, rows, cols).astype(np.float64)
    Wd = O.dequant_typed(W, t, rows, cols).astype(np.float64)
    exact = Wd @ x.astype(np.float64)
    bound = 2 * cols * 2.0 ** -24 * (np.abs(Wd) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y - exact) <= bound)


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q6_K])
def test_typed_matvec_q8_is_matvec_on_q8_values(t):
    g = np.random.default_rng(20 + t)
    rows, cols = 9, 512
    W = O.make_typed(g, t, rows, cols)
    xq = O.quantize_q8_0(g.standard_normal(cols).astype(np.float32))
    xv = (xq["d"][:, None] * xq["qs"].astype(np.float32)).astype(np.float32).reshape(-1)
    assert np.array_equal(O.typed_matvec_q8(W, t, xq, rows, cols),
                          O.typed_matvec(W, t, xv, rows, cols))


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q6_K, O.TYPE_Q4_0])
def test_typed_gemm_against_float64(t):
    g = np.random.default_rng(30 + t)
    S, N, K = 5, 33, 512
    W = O.make_typed(g, t, N, K)
    X = g.standard_normal((S, K)).astype(np.float32)
    Y = O.typed_gemm(W, t, N, K, X).astype(np.float64)
    Wd = O.dequant_typed(W, t, N, K).astype(np.float64)
    exact = X.astype(np.float64) @ Wd.T
    bound = 2 * K * 2.0 ** -24 * (np.abs(X.astype(np.float64)) @ np.abs(Wd).T)
    assert np.all(np.abs(Y - exact) <= bound)
    if t == O.TYPE_Q4_0:  # the Q4_0 branch is the existing GEMM oracle's
        assert np.array_equal(Y.astype(np.float32), O.q4_0_gemm(W, N, K, X))


def test_row_bytes():
    assert O.typed_row_bytes(O.TYPE_Q4_K, 4096) == 16 * 144
    assert O.typed_row_bytes(O.TYPE_Q6_K, 14336) == 56 * 210
    assert O.typed_row_bytes(O.TYPE_Q4_0, 4096) == 128 * 18
    assert O.typed_row_bytes(O.TYPE_Q4_K, 100) == 0
    assert O.typed_row_bytes(7, 256) == 0


def _ones_row(t, cols):
    """A row of weights all exactly 1.0 in type t (d = 1, q at its offset + 1)."""
    if t == O.TYPE_Q4_0:
        blk = np.zeros(18, np.uint8)
        blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        blk[2:] = 9 | (9 << 4)                                  # q - 8 = 1
        return np.tile(blk, cols // 32)[None]
    ql, qh = _q6_k_encode(np.full(256, 33))                     # q - 32 = 1
    blk = np.concatenate([ql, qh, np.ones(16, np.int8).view(np.uint8),
                          np.frombuffer(np.float16(1.0).tobytes(), np.uint8)])
    return np.tile(blk, cols // 256)[None]


@pytest.mark.parametrize("t", [O.TYPE_Q4_0, O.TYPE_Q6_K])
def test_typed_matvec_four_lane_order(t):
    # q4_0_matvec_f32 / q6_K_matvec_f32_neon keep four fp32 lane sums (value
    # i in lane i % 4) and add them at the end: with x0 = 2^24 and x1 = x5 = 1
    # lane 1 holds 2 and the row sums to 2^24 + 2 exactly, where a sum in k
    # order rounds 2^24 + 1 back to 2^24 twice
    cols = 256
    x = np.zeros(cols, np.float32)
    x[0], x[1], x[5] = 2.0 ** 24, 1.0, 1.0
    W = _ones_row(t, cols)
    assert np.array_equal(O.dequant_typed(W, t, 1, cols), np.ones((1, cols), np.float32))
    assert O.typed_matvec(W, t, x, 1, cols)[0] == 2.0 ** 24 + 2
    # the F32 path (sgemv, k order) on the same values
    Wf = np.ones((1, cols), np.float32).view(np.uint8)
    assert O.typed_matvec(Wf, O.TYPE_F32, x, 1, cols)[0] == 2.0 ** 24


# Q4_K_M's mix (the reference's target files, mistral/gguf_loader.h:1-2): Q4_K
# matrices with Q6_K for the value and down projections
Q4_K_M = {"wq": O.TYPE_Q4_K, "wk": O.TYPE_Q4_K, "wv": O.TYPE_Q6_K, "wo": O.TYPE_Q4_K,
          "w1": O.TYPE_Q4_K, "w3": O.TYPE_Q4_K, "w2": O.TYPE_Q6_K}


def make_layer_typed(g, types, dim, hidden, nh, nkv, d_scale=1.0):
    kvd = dim // nh * nkv
    shapes = {"wq": (dim, dim), "wk": (kvd, dim), "wv": (kvd, dim), "wo": (dim, dim),
              "w1": (hidden, dim), "w3": (hidden, dim), "w2": (dim, hidden)}
    W = {k: O.make_typed(g, types[k], *shapes[k], d_scale=d_scale) for k in O.MATS}
    W["rms_att"] = (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    W["rms_ffn"] = (1.0 + 0.1 * g.standard_normal(dim)).astype(np.float32)
    return W


def _ring(g, M, kvd, start):
    kc = np.zeros((M, kvd), np.uint16)
    vc = np.zeros((M, kvd), np.uint16)
    kc[:start] = D.to_f16_bits(g.standard_normal((start, kvd)).astype(np.float32))
    vc[:start] = D.to_f16_bits(g.standard_normal((start, kvd)).astype(np.float32))
    return kc, vc


def test_prefill_layer_typed_all_q4_0_is_prefill_layer():
    g = np.random.default_rng(41)
    dim, hidden, nh, nkv, M, start, S = 256, 512, 4, 1, 32, 3, 6
    W = P.make_layer(g, dim, hidden, nh, nkv)
    kc, vc = _ring(g, M, dim // nh * nkv, start)
    X = g.standard_normal((S, dim)).astype(np.float32)
    th = O.theta_inv(1e6, dim // nh)
    k1, v1, k2, v2 = kc.copy(), vc.copy(), kc.copy(), vc.copy()
    a = O.prefill_layer(W, X, k1, v1, start, S, dim, hidden, nh, nkv, th)
    b = O.prefill_layer_typed(W, {k: O.TYPE_Q4_0 for k in O.MATS}, X, k2, v2, start, S, dim,
                              hidden, nh, nkv, th)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


@pytest.mark.parametrize("mix", ["q4_k_m", "f16_f32"])
def test_prefill_layer_typed_matches_float64(mix):
    g = np.random.default_rng(42)
    types = Q4_K_M if mix == "q4_k_m" else {
        "wq": O.TYPE_F16, "wk": O.TYPE_F32, "wv": O.TYPE_F16, "wo": O.TYPE_Q4_0,
        "w1": O.TYPE_F32, "w3": O.TYPE_Q4_K, "w2": O.TYPE_F16}
    dim, hidden, nh, nkv, M, start, S = 512, 768, 4, 1, 32, 5, 8
    W = make_layer_typed(g, types, dim, hidden, nh, nkv)
    kc, vc = _ring(g, M, dim // nh * nkv, start)
    X = g.standard_normal((S, dim)).astype(np.float32)
    th = O.theta_inv(1e6, dim // nh)
    ref, kring = P._layer64(W, X, kc, vc, start, S, dim, hidden, nh, nkv, th, 1e-5, types)
    ko, vo = kc.copy(), vc.copy()
    out = O.prefill_layer_typed(W, types, X, ko, vo, start, S, dim, hidden, nh, nkv, th)
    assert np.abs(out - ref).max() <= 2e-4 * max(1.0, np.abs(ref).max())
    slots = np.arange(start, start + S) % M
    assert np.abs(D.f16_bits_to_f32(ko[slots]) - kring[slots]).max() <= 2e-3 * max(
        1.0, np.abs(kring[slots]).max())


def _q8_64(x):
    """Q8_0 quantisation in float64 (d = amax / 127, q = round-half-even(x / d)
    saturated; dequant.h:545-612): the values d * q."""
    b = x.reshape(-1, 32)
    amax = np.abs(b).max(axis=1, keepdims=True)
    d = amax / 127.0
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(d > 0, np.clip(np.rint(b / d), -128, 127), 0.0)
    return (q * d).reshape(-1)


def _decode_layer64(W, types, x, kc, vc, pos, dim, hidden, nh, nkv, th, eps):
    """mistral_layer_decode_parallel (mistral_model.h:818-899) in float64 with
    the Q8_0 rounding of the activations (fp16 ring entries as the ring holds
    them)."""
    hd, M = dim // nh, kc.shape[0]
    kvd = nkv * hd
    shapes = {"wq": (dim, dim), "wk": (kvd, dim), "wv": (kvd, dim), "wo": (dim, dim),
              "w1": (hidden, dim), "w3": (hidden, dim), "w2": (dim, hidden)}
    dq = {k: O.dequant_typed(W[k], types[k], *shapes[k]).astype(np.float64) for k in O.MATS}

    def rms(v, w):
        return v / np.sqrt((v * v).mean() + eps) * w.astype(np.float64)

    x = x.astype(np.float64)
    xq = _q8_64(rms(x, W["rms_att"]))
    q, k, v = dq["wq"] @ xq, dq["wk"] @ xq, dq["wv"] @ xq
    kring = D.f16_bits_to_f32(kc).astype(np.float64)
    vring = D.f16_bits_to_f32(vc).astype(np.float64)
    slot = pos % M
    kring[slot] = P._rope64(k, pos, th, nkv, hd).astype(np.float16)
    vring[slot] = v.astype(np.float16)
    qr = P._rope64(q, pos, th, nh, hd).reshape(nh, hd)
    L = min(pos + 1, M)
    slots = [(pos + 1 - L + t) % M for t in range(L)]
    a = np.zeros(dim)
    for h in range(nh):
        kvh = h // (nh // nkv)
        sc = kring[slots][:, kvh * hd:(kvh + 1) * hd] @ qr[h] / np.sqrt(hd)
        pr = np.exp(sc - sc.max())
        a[h * hd:(h + 1) * hd] = (pr / pr.sum()) @ vring[slots][:, kvh * hd:(kvh + 1) * hd]
    x = x + dq["wo"] @ _q8_64(a)
    xq = _q8_64(rms(x, W["rms_ffn"]))
    g, u = dq["w1"] @ xq, dq["w3"] @ xq
    h = g / (1.0 + np.exp(-g)) * u
    return x + dq["w2"] @ _q8_64(h), kring[slot]


@pytest.mark.parametrize("mix,pos", [("q4_0", 5), ("q4_k_m", 40), ("q4_k_m", 100)])
def test_decode_layer_typed_matches_float64(mix, pos):
    # the Q8_0 rounding is reproduced in float64, so the oracle's fp32
    # arithmetic differs from this only by fp32 rounding and the occasional
    # activation whose Q8_0 step differs when its value sits at a rounding
    # boundary: a normwise 2e-3 of the output's scale (a dropped residual, a
    # swapped gate / up or a missing requantisation errs by tens of percent)
    g = np.random.default_rng(60 + pos)
    types = {k: O.TYPE_Q4_0 for k in O.MATS} if mix == "q4_0" else Q4_K_M
    dim, hidden, nh, nkv, M = 512, 768, 4, 1, 64
    W = make_layer_typed(g, types, dim, hidden, nh, nkv, 0.07) if mix != "q4_0" else \
        P.make_layer(g, dim, hidden, nh, nkv)
    kc, vc = _ring(g, M, dim // nh * nkv, min(pos, M))
    x = g.standard_normal(dim).astype(np.float32)
    th = O.theta_inv(1e6, dim // nh)
    ref, krow = _decode_layer64(W, types, x, kc, vc, pos, dim, hidden, nh, nkv, th, 1e-5)
    ko, vo = kc.copy(), vc.copy()
    out = O.decode_layer_typed(W, types, x, ko, vo, pos, dim, hidden, nh, nkv, th)
    assert np.abs(out - ref).max() <= 2e-3 * np.abs(ref).max()
    assert np.abs(D.f16_bits_to_f32(ko[pos % M]) - krow).max() <= 2e-3 * np.abs(krow).max()
    others = np.setdiff1d(np.arange(M), [pos % M])
    assert np.array_equal(ko[others], kc[others]) and np.array_equal(vo[others], vc[others])
