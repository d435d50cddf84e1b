"""GPU parity at the edges of the attention entry points, through the C ABI:

- more tokens than ring slots (S > max_seq): the reference writes the tokens in
  order (kv_write_batch, mistral/mistral_ane_prefill.h:189-204; the verify
  loop, mistral/speculative.h:92-101), so a slot keeps the last token written
  to it;
- ring offsets beyond 32 bits (slot * kv_dim >= 2^32 elements);
- the flash kernel's second pass: rows whose later scores sit far above the
  first tile's maximum (the fp16 P of the first pass overflows);
- attention_batch (mistral_ane_prefill.h:207-275) over a wrapped ring, where
  the window of query t is the oldest-first run of slots (pos+1-L+s) % M
  (mistral_ane_prefill.h:238-241)."""

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


# ---- S > max_seq -----------------------------------------------------------

def test_kv_write_more_tokens_than_slots():
    G.say("kv_write_f32 M=64 start=10 S=100")
    lib = G.lib()
    g = D.rng(700)
    M, start, S = 64, 10, 100
    kc, vc = D.ring(g, M)
    K, V = D.normal(g, (S, 1024)), D.normal(g, (S, 1024))
    dkc, dvc, dK, dV = DB.from_array(kc), DB.from_array(vc), DB.from_array(K), DB.from_array(V)
    check(lib.mia_kv_write_f32(dkc.ptr, dvc.ptr, dK.ptr, dV.ptr, S, start, M, 1024, None), "kv_write")
    check(lib.mia_stream_sync(None), "sync")
    kc_o, vc_o = kc.copy(), vc.copy()
    O.kv_write_batch(kc_o, vc_o, K, V, 8, 128, M, start, S)
    assert np.array_equal(dkc.download(kc.shape, np.uint16), kc_o)
    assert np.array_equal(dvc.download(vc.shape, np.uint16), vc_o)


@pytest.mark.parametrize("M,start,S", [(64, 10, 100), (64, 500, 100), (32, 3, 80)])
def test_attention_step_more_tokens_than_slots(M, start, S):
    G.say(f"attention_step M={M} start={start} S={S} (S > M)")
    g = D.rng(710 + M + start + S)
    kc, vc = D.ring(g, M)
    Q, K, V = D.normal(g, (S, 4096)), D.normal(g, (S, 1024)), D.normal(g, (S, 1024))
    out, kc_g, vc_g = G.attention_step(kc, vc, Q, K, V, TH, M, start, S)
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = O.verify_steps(kc_o, vc_o, Q, K, V, start, S, TH, 32, 8, 128, M)
    D.check_close(out, ref, what=f"S>M M={M} start={start} S={S}")
    # the ring holds the last M tokens, each at its slot
    last = np.arange(start + S - M, start + S)
    D.check_ring(kc_g, kc_o, vc_g, vc_o, last % M, K[S - M:], last, TH, "S>M ring")


# ---- ring offsets beyond 2^32 elements ---------------------------------------

def test_ring_offsets_beyond_32_bits():
    """16 kv heads (kv_dim 2048) and a ring of 2^21 + 48 slots: the last slots
    sit at element offsets >= 2^32.  Keys are zero, so every window position
    weighs 1/L and the output is the window's mean of V; only the 8 slots at
    the ring's end carry values.  With the window starting at slot 8, those
    slots are read through the per-lane path of the tile that crosses the
    ring's end (decode) and of the flash kernel's wrapped tile; a 32-bit
    offset would read slots 2^21 lower, which are zero."""
    n_heads, n_kv, kv_dim = 64, 16, 2048
    M = (1 << 21) + 48
    pos = M + 7                       # window = all M slots, oldest at slot 8
    G.say(f"decode/flash ring offsets > 2^32: M={M} kv_dim={kv_dim} pos={pos}")
    lib = G.lib()
    nbytes = M * kv_dim * 2
    dkc, dvc = DB(nbytes), DB(nbytes)
    dkc.zero()
    dvc.zero()
    hi_slots = np.arange(M - 8, M)
    assert hi_slots[0] * kv_dim >= 1 << 32
    vrow = (2048 + 64 * (np.arange(kv_dim) // 128) + 2 * (np.arange(kv_dim) % 32)).astype(np.float32)
    vbits = D.to_f16_bits(np.tile(vrow, (8, 1)))
    dvc.upload(vbits, offset=int(hi_slots[0]) * kv_dim * 2)
    expect = np.repeat((8.0 * vrow.reshape(n_kv, 128) / M)[:, None, :], 4, axis=1).reshape(-1)
    g = D.rng(720)
    q = D.normal(g, n_heads * 128)
    dq, dout = DB.from_array(q), DB(n_heads * 128 * 4)
    check(lib.mia_gqa_attention(dq.ptr, dout.ptr, dkc.ptr, dvc.ptr, n_heads, 4, 128, M, pos, None),
          "gqa_attention")
    check(lib.mia_stream_sync(None), "sync")
    out = dout.download(n_heads * 128, np.float32)
    np.testing.assert_allclose(out, expect, rtol=2e-3, atol=1e-6)
    # flash kernel: 4 queries at positions pos-3 .. pos, windows all M slots
    S = 4
    Q = D.normal(g, (S, n_heads * 128))
    dQ, dO = DB.from_array(Q), DB(S * n_heads * 128 * 4)
    check(lib.mia_attention_batch(dQ.ptr, dO.ptr, dkc.ptr, dvc.ptr, n_heads, n_kv, 128, M,
                                  pos - 3, S, None), "attention_batch")
    check(lib.mia_stream_sync(None), "sync")
    outb = dO.download((S, n_heads * 128), np.float32)
    for t in range(S):
        np.testing.assert_allclose(outb[t], expect, rtol=5e-3, atol=1e-6)


# ---- the flash kernel's second pass -------------------------------------------

RAMP_DIM = 126  # dims 126/127: the lowest-frequency RoPE pair, ~unrotated


def _ramp_inputs(g, Mfill, S, slope):
    """Ring keys whose score against every query grows by `slope` log2 units
    per position, plus N(0,1) noise in the other dims.  q[126] = 8 gives
    score_log2 = k[126] * 8 / sqrt(128) * log2(e) = 1.0202 k[126]."""
    Q = D.normal(g, (S, 4096)) * 0.25
    Q.reshape(S, 32, 128)[:, :, RAMP_DIM] = 8.0
    Q.reshape(S, 32, 128)[:, :, RAMP_DIM + 1] = 0.0
    per_pos = slope / 1.0202
    return Q, per_pos


def _tile_jump_ok(scores_log2, lo, hi, need=17.0):
    """Every 32-key tile of [lo, hi] (any alignment) is followed by one whose
    maximum is more than `need` log2 units higher: a first-pass reference set
    in any tile overflows fp16 P in the next."""
    s = scores_log2[lo:hi + 1]
    n = len(s) - 64
    if n < 0:
        return True
    m0 = np.array([s[i:i + 32].max() for i in range(0, n + 1)])
    m1 = np.array([s[i + 32:i + 64].max() for i in range(0, n + 1)])
    return bool((m1 - m0 > need).all())


def _score_log2(Qr_row_head, Kf_head):
    return (Kf_head.astype(np.float64) @ Qr_row_head.astype(np.float64)) / np.sqrt(128) * np.log2(np.e)


@pytest.mark.parametrize("M,start,S", [(4096, 256, 64), (4096, 1536, 512)])
def test_flash_second_pass_prefill(M, start, S):
    """Causal prefill whose scores climb 24 log2 units per 32 keys: every key
    group's first-tile reference is overflowed by its later tiles, so every
    wave with two or more tiles runs the second pass (exact maxima)."""
    G.say(f"flash second pass prefill M={M} start={start} S={S}")
    g = D.rng(730 + S)
    kc, vc = D.ring(g, M, filled=start)
    Q, per_pos = _ramp_inputs(g, start, S, 0.75)
    # cached keys: the ramp in dim 126 (fp16-exact steps), noise elsewhere
    Kf = D.f16_bits_to_f32(kc[:start]).reshape(start, 8, 128) * 0.25
    Kf[:, :, RAMP_DIM] = np.round(per_pos * np.arange(start))[:, None]
    Kf[:, :, RAMP_DIM + 1] = 0.0
    kc[:start] = D.to_f16_bits(Kf.reshape(start, 1024))
    K = D.normal(g, (S, 1024)) * 0.25
    K.reshape(S, 8, 128)[:, :, RAMP_DIM] = np.round(per_pos * np.arange(start, start + S))[:, None]
    K.reshape(S, 8, 128)[:, :, RAMP_DIM + 1] = 0.0
    V = D.normal(g, (S, 1024))
    out, kc_g, vc_g = G.attention_step(kc, vc, Q, K, V, TH, M, start, S)
    kc_o, vc_o = kc.copy(), vc.copy()
    Qr = Q.copy()
    O.load().ora_apply_rope_batch(Qr.ctypes.data, None, start, TH.ctypes.data, 32, 8, 128, S)
    Kr = K.copy()
    O.load().ora_apply_rope_batch(None, Kr.ctypes.data, start, TH.ctypes.data, 32, 8, 128, S)
    O.kv_write_batch(kc_o, vc_o, Kr, V, 8, 128, M, start, S)
    # the construction: for a sample of rows, every tile is overflowed by the next
    Kall = D.f16_bits_to_f32(kc_o[:start + S]).reshape(start + S, 8, 128)
    for t in (0, S // 2, S - 1):
        for h in (0, 13, 31):
            sl = _score_log2(Qr.reshape(S, 32, 128)[t, h], Kall[:, h // 4])
            assert _tile_jump_ok(sl, 0, start + t), (t, h)
    ref = O.attention_batch_parallel(Qr, kc_o, vc_o, 32, 8, 128, M, start, S)
    D.check_close(out, ref, what=f"second pass prefill S={S}")
    pos = np.arange(start, start + S)
    D.check_ring(kc_g, kc_o, vc_g, vc_o, pos % M, K, pos, TH, "second pass ring")


@pytest.mark.parametrize("start", [70000, 66536])
def test_flash_second_pass_verify_65536_ring(start):
    """8-draft verify on a wrapped 65536-slot ring whose keys climb 24 log2
    units per 32 positions in window order (oldest lowest): every split and
    key group of the wrapped window overflows its first-tile reference."""
    G.say(f"flash second pass verify M=65536 start={start} S=8")
    g = D.rng(740 + start)
    M, S = 65536, 8
    kc, vc = D.ring(g, M)
    Q, per_pos = _ramp_inputs(g, M, S, 0.75)
    # window order of the first draft: positions start-M+1 .. start-1 (old)
    old = np.arange(start - M + 1, start)
    rank = old - old[0]                               # 0 .. M-2, oldest first
    Kf = D.f16_bits_to_f32(kc).reshape(M, 8, 128) * 0.25
    ramp = np.round(per_pos * (rank % 2048))          # fp16-exact, < 2048
    Kf[old % M, :, RAMP_DIM] = ramp[:, None]
    Kf[:, :, RAMP_DIM + 1] = 0.0
    kc = D.to_f16_bits(Kf.reshape(M, 1024))
    K = D.normal(g, (S, 1024)) * 0.25
    K.reshape(S, 8, 128)[:, :, RAMP_DIM] = 1600.0
    V = D.normal(g, (S, 1024))
    out, kc_g, vc_g = G.attention_step(kc, vc, Q, K, V, TH, M, start, S)
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = O.verify_steps(kc_o, vc_o, Q, K, V, start, S, TH, 32, 8, 128, M)
    D.check_close(out, ref, what=f"second pass verify start={start}")
    pos = np.arange(start, start + S)
    D.check_ring(kc_g, kc_o, vc_g, vc_o, pos % M, K, pos, TH, "second pass verify ring")


def test_flash_second_pass_descending_and_flat():
    """The other direction: the first tile holds the largest scores and the
    rest fall 24 log2 units per tile (P underflows to zero there, the first
    pass stands), and a row whose scores are all far below zero."""
    G.say("flash descending scores M=2048 start=1024 S=64")
    g = D.rng(750)
    M, start, S = 2048, 1024, 64
    kc, vc = D.ring(g, M, filled=start + S)
    Q, per_pos = _ramp_inputs(g, start, S, 0.75)
    Kf = D.f16_bits_to_f32(kc).reshape(M, 8, 128) * 0.25
    Kf[:start + S, :, RAMP_DIM] = -np.round(per_pos * np.arange(start + S))[:, None]
    Kf[:, :, RAMP_DIM + 1] = 0.0
    kc = D.to_f16_bits(Kf.reshape(M, 1024))
    out = G.attention_batch(Q, kc, vc, M, start, S)
    ref = O.attention_batch(Q, kc, vc, 32, 8, 128, M, start, S)
    D.check_close(out, ref, what="descending")
    # all scores near -2000 and near -39800 log2 units: the reference is
    # applied as fp16 hi + lo, so it stays within ~2^-22 of the row maximum
    # (one fp16 would be off by up to 16 units at 39800 and overflow P)
    for kval in (-1960.0, -39008.0):
        Kf[:start + S, :, RAMP_DIM] = kval
        kc2 = D.to_f16_bits(Kf.reshape(M, 1024))
        out = G.attention_batch(Q, kc2, vc, M, start, S)
        ref = O.attention_batch(Q, kc2, vc, 32, 8, 128, M, start, S)
        D.check_close(out, ref, what=f"flat scores k126={kval}")


# ---- attention_batch over a wrapped ring ---------------------------------------

@pytest.mark.parametrize("M,start,S", [(300, 1000, 8), (300, 1000, 40), (65536, 70000, 8),
                                       (128, 400, 200)])
def test_attention_batch_wrapped_ring(M, start, S):
    G.say(f"attention_batch wrapped M={M} start={start} S={S}")
    g = D.rng(760 + M + S)
    kc, vc = D.ring(g, M)
    Q = D.normal(g, (S, 4096))
    out = G.attention_batch(Q, kc, vc, M, start, S)
    ref = O.attention_batch_parallel(Q, kc, vc, 32, 8, 128, M, start, S)
    D.check_close(out, ref, what=f"wrapped batch M={M} start={start} S={S}")
