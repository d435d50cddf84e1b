"""GPU parity: S=1 decode attention (split-K flash-decode kernel) against the
CPU oracle on the same seeded inputs, through the C ABI.

Bar: outputs within max-abs 2e-3 / max-rel 1e-2 of the oracle; after the
fused step the slot written is pos % max_seq, V and every other slot are
bit-exact, and the rotated key is a faithful fp16 rounding of the exact
rotation (the sin/cos library boundary rules out bit equality)."""

import numpy as np
import pytest

import _data as D
import _gpu as G
import _oracle as O

pytestmark = pytest.mark.gpu

TH = O.theta_inv(D.THETA, D.HD)


def _new_token(g):
    return D.normal(g, 4096), D.normal(g, 1024), D.normal(g, 1024)


def test_decode_step_single_layer_repo_cpu_case():
    # Single-layer case of the reference's CPU path: positions 0..511 cached,
    # new token at 512 (L = 513), M = 4096, theta 1e6, seed 0.
    G.say("decode_step L=513 M=4096 seed=0")
    g = D.rng(0)
    M, pos = 4096, 512
    kc, vc = D.ring(g, M, filled=pos)
    q, k, v = _new_token(g)
    out, kc_g, vc_g = G.decode_step(kc, vc, q, k, v, TH, M, pos)
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = O.decode_step(kc_o, vc_o, q, k, v, pos, TH, 32, 8, 128, M)
    D.check_close(out, ref, what="decode_step L=513")
    D.check_ring(kc_g, kc_o, vc_g, vc_o, [pos % M], k, [pos], TH, "decode ring")


@pytest.mark.parametrize("pos", [0, 1, 62, 63, 64, 255, 256, 257, 300, 512, 1000, 2047, 4096])
def test_gqa_attention_lengths(pos):
    G.say(f"gqa_attention unwrapped pos={pos}")
    g = D.rng(100 + pos)
    M = 8192
    kc, vc = D.ring(g, M, filled=pos + 1)
    q = D.normal(g, 4096)
    out = G.gqa_attention(q, kc, vc, M, pos)
    ref = O.gqa_attention(q, kc, vc, 32, 4, 128, M, pos)
    D.check_close(out, ref, what=f"pos={pos}")


@pytest.mark.parametrize("M,pos", [(1000, 1500), (1000, 2999), (4096, 4096), (4096, 9999),
                                   (257, 70000), (65536, 70007)])
def test_gqa_attention_wrapped_ring(M, pos):
    G.say(f"gqa_attention wrapped M={M} pos={pos}")
    g = D.rng(M + pos)
    kc, vc = D.ring(g, M)
    q = D.normal(g, 4096)
    out = G.gqa_attention(q, kc, vc, M, pos)
    ref = O.gqa_attention(q, kc, vc, 32, 4, 128, M, pos)
    D.check_close(out, ref, what=f"M={M} pos={pos}")


def test_decode_step_long_context_sharp_peaks():
    # Long-context case: M = 32768 ring full, new token at 32768 wraps into
    # slot 0; every 1024th key x4 gives sharp softmax peaks (LSE merge).
    G.say("decode_step M=32768 pos=32768 spikes/1024")
    g = D.rng(3)
    M, pos = 32768, 32768
    kc, vc = D.ring(g, M, spike_every=1024)
    q, k, v = _new_token(g)
    out, kc_g, vc_g = G.decode_step(kc, vc, q, k, v, TH, M, pos)
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = O.decode_step(kc_o, vc_o, q, k, v, pos, TH, 32, 8, 128, M)
    D.check_close(out, ref, what="32K spikes")
    D.check_ring(kc_g, kc_o, vc_g, vc_o, [pos % M], k, [pos], TH, "decode ring")


def test_decode_step_first_token_returns_v():
    G.say("decode_step pos=0")
    g = D.rng(4)
    M = 64
    kc, vc = D.ring(g, M)
    q, k, v = _new_token(g)
    out, _, _ = G.decode_step(kc, vc, q, k, v, TH, M, 0)
    vh = D.f16_bits_to_f32(D.to_f16_bits(v)).reshape(8, 128)
    assert np.array_equal(out.reshape(32, 128), vh[np.arange(32) // 4])


def _ids_to_v(ids, kv_dim=1024):
    """V rows carrying a position id exactly in fp16: (id // 64, id % 64)."""
    v = np.zeros((len(ids), kv_dim), np.float32)
    v[:, 0::2] = (ids // 64)[:, None]
    v[:, 1::2] = (ids % 64)[:, None]
    return D.to_f16_bits(v)


@pytest.mark.parametrize("M,pos", [(4096, 700), (1000, 2500), (32768, 40000)])
def test_decode_window_and_no_leak_index_revealing(M, pos):
    # Keys in the window are zero (uniform softmax) and every slot outside the
    # window holds a key that would dominate any leak; V carries the position
    # id, so the output is exactly the mean id of the attended set.
    G.say(f"index-revealing decode M={M} pos={pos}")
    kc = np.zeros((M, 1024), np.uint16)
    vc = np.zeros((M, 1024), np.uint16)
    win = D.window_positions(pos, M)
    in_win = np.zeros(M, bool)
    in_win[win % M] = True
    kc[~in_win] = D.to_f16_bits(np.full(1024, 8.0, np.float32))
    vc[~in_win] = D.to_f16_bits(np.full(1024, -1000.0, np.float32))
    vc[win % M] = _ids_to_v(win)
    q = np.full(4096, 1.0, np.float32)
    out = G.gqa_attention(q, kc, vc, M, pos).reshape(32, 128)
    hi, lo = (win // 64).mean(), (win % 64).mean()
    assert np.allclose(out[:, 0::2], hi, rtol=1e-4) and np.allclose(out[:, 1::2], lo, rtol=1e-4)
