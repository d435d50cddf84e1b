"""Seeded synthetic inputs, float64 brute-force references and the parity
tolerance shared by the tests (test infrastructure)."""

from __future__ import annotations

import numpy as np

# Parity bar for the floating-point outputs: max-abs <= ATOL over all outputs,
# and |gpu - ref| <= RTOL * |ref| wherever |ref| >= ATOL / RTOL.
ATOL = 2e-3
RTOL = 1e-2

N_HEADS, N_KV, HD = 32, 8, 128
KV_DIM = N_KV * HD
THETA = 1e6


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def normal(g: np.random.Generator, shape) -> np.ndarray:
    return g.standard_normal(shape, dtype=np.float32)


def to_f16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> IEEE binary16 bits with round-to-nearest-even (numpy)."""
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def ring(g, max_seq, kv_dim=KV_DIM, filled=None, spike_every=0, spike=4.0):
    """fp16 K/V ring of one layer ~ N(0,1); slots >= filled stay zero (calloc).
    With spike_every, keys at positions p % spike_every == 0 are scaled."""
    kc = np.zeros((max_seq, kv_dim), dtype=np.uint16)
    vc = np.zeros((max_seq, kv_dim), dtype=np.uint16)
    n = max_seq if filled is None else min(filled, max_seq)
    k = normal(g, (n, kv_dim))
    if spike_every:
        k[::spike_every] *= spike
    kc[:n] = to_f16_bits(k)
    vc[:n] = to_f16_bits(normal(g, (n, kv_dim)))
    return kc, vc


def check_close(got: np.ndarray, ref: np.ndarray, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    max_abs = float(err.max()) if err.size else 0.0
    big = np.abs(ref) >= atol / rtol
    max_rel = float((err[big] / np.abs(ref[big])).max()) if big.any() else 0.0
    assert max_abs <= atol, f"{what}: max_abs {max_abs:.3e} > {atol}"
    assert max_rel <= rtol, f"{what}: max_rel {max_rel:.3e} > {rtol}"
    return max_abs, max_rel


def window_positions(pos: int, max_seq: int) -> np.ndarray:
    """Positions attended at `pos`: the last min(pos+1, max_seq), oldest first."""
    L = min(pos + 1, max_seq)
    return np.arange(pos + 1 - L, pos + 1, dtype=np.int64)


def attend_f64(qh: np.ndarray, K: np.ndarray, V: np.ndarray, scale: float) -> np.ndarray:
    """float64 softmax(q.K^T * scale) . V for one head; K, V float rows."""
    s = (K.astype(np.float64) @ qh.astype(np.float64)) * scale
    s -= s.max()
    p = np.exp(s)
    p /= p.sum()
    return p @ V.astype(np.float64)


def gqa_decode_f64(q, kc, vc, n_heads, n_kv, hd, max_seq, pos):
    """Independent float64 S=1 GQA attention over a ring (slot = p % max_seq)."""
    slots = window_positions(pos, max_seq) % max_seq
    hpk = n_heads // n_kv
    out = np.empty((n_heads, hd), dtype=np.float64)
    Kf = f16_bits_to_f32(kc[slots]).reshape(len(slots), n_kv, hd)
    Vf = f16_bits_to_f32(vc[slots]).reshape(len(slots), n_kv, hd)
    qh = np.asarray(q, dtype=np.float64).reshape(n_heads, hd)
    for h in range(n_heads):
        kvh = h // hpk
        out[h] = attend_f64(qh[h], Kf[:, kvh], Vf[:, kvh], 1.0 / np.sqrt(hd))
    return out.reshape(-1)


def rope_f64(x: np.ndarray, pos: int, th: np.ndarray, n_vec: int, hd: int) -> np.ndarray:
    """Adjacent-pair rotation in float64 using the fp32 angle fl32(theta_inv*pos)."""
    ang = (th.astype(np.float32) * np.float32(pos)).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    y = np.asarray(x, dtype=np.float64).reshape(n_vec, hd // 2, 2).copy()
    e, o = y[..., 0].copy(), y[..., 1].copy()
    y[..., 0] = e * c - o * s
    y[..., 1] = o * c + e * s
    return y.reshape(-1)


def check_rotated_k(k16_bits, K_raw, positions, th, n_kv=N_KV, hd=HD, what=""):
    """fp16 ring keys against the exact rotation: float64 RoPE on the fp32
    angle fl32(theta_inv*pos).  Bound: half an fp16 ulp (the final rounding)
    plus 4e-7 x the pair norm (fp32 sin/cos and products; covers results
    that nearly cancel, where the two sides' libm/ocml ulps show up)."""
    K_raw = np.asarray(K_raw, np.float32).reshape(len(positions), n_kv * hd)
    exact = np.stack([rope_f64(K_raw[i], int(p), th, n_kv, hd) for i, p in enumerate(positions)])
    got = f16_bits_to_f32(k16_bits).astype(np.float64).reshape(exact.shape)
    pr = K_raw.astype(np.float64).reshape(len(positions), -1, 2)
    pair_norm = np.repeat(np.sqrt((pr ** 2).sum(-1)), 2, axis=-1)
    mag = np.maximum(np.abs(exact), np.abs(got)).astype(np.float16)
    bound = 0.5 * np.spacing(mag).astype(np.float64) + 4e-7 * pair_norm
    bad = np.abs(got - exact) > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} rotated keys off the exact rounding"


def check_ring(kc_g, kc_o, vc_g, vc_o, written_slots, K_raw=None, positions=None, th=None,
               what=""):
    """Ring after a write step: V and every slot outside `written_slots` are
    bit-exact with the oracle's ring, and the written slots' keys are faithful
    fp16 roundings of the exact rotation on both sides.  Rotated keys are not
    compared bit for bit: RoPE's sin/cos come from different libraries (device
    ocml, host libm, the reference's Accelerate) and an ulp of fp32 can flip
    the fp16 rounding."""
    written_slots = np.asarray(written_slots)
    assert np.array_equal(vc_g, vc_o), f"{what}: V ring differs"
    diff = kc_g != kc_o
    rows = np.unique(np.nonzero(diff)[0])
    assert set(rows.tolist()) <= set(written_slots.tolist()), \
        f"{what}: unwritten slots changed: {rows[:10]}"
    if K_raw is not None:
        check_rotated_k(kc_g[written_slots], K_raw, positions, th, what=what + " (gpu)")
        check_rotated_k(kc_o[written_slots], K_raw, positions, th, what=what + " (oracle)")
    return int(diff.sum())
