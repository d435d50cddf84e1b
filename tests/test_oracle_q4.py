"""CPU checks that pin the Q4_0 x Q8_0 oracle (oracle/q4_oracle.c) to the
reference's W4A8 path (mistral/dequant.h:545-612, 1022-1137) by known answers,
brute force and float64 dequantisation, not by restating its formula."""

import numpy as np
import pytest

import _oracle as O


def q8_block(values, d):
    b = np.zeros(1, dtype=O.Q8_DTYPE)
    b["d"] = d
    b["qs"][0] = values
    return b


def test_quantize_known_answers_ties_to_even():
    # amax 127 -> d = 1 exactly, so q = round-to-nearest-even(x)
    x = np.zeros(32, np.float32)
    x[:8] = [127.0, -127.0, 63.5, 62.5, 0.5, 1.5, 2.5, -2.5]
    q = O.quantize_q8_0(x)
    assert q["d"][0] == np.float32(1.0)
    assert list(q["qs"][0][:8]) == [127, -127, 64, 62, 0, 2, 2, -2]
    assert not q["qs"][0][8:].any()


def test_quantize_zero_block_and_scale():
    x = np.zeros(64, np.float32)
    x[32:] = np.arange(32, dtype=np.float32) - 16.0      # amax 16
    q = O.quantize_q8_0(x)
    assert q["d"][0] == 0.0 and not q["qs"][0].any()
    assert q["d"][1] == np.float32(16.0) / np.float32(127.0)
    assert q["qs"][1][0] == -127                          # the amax element maps to +-127
    assert np.abs(q["qs"][1]).max() == 127


def test_quantize_error_bound():
    g = np.random.default_rng(1)
    x = (g.standard_normal(32 * 64) * 3.0).astype(np.float32)
    q = O.quantize_q8_0(x)
    d = q["d"].astype(np.float64)[:, None]
    rec = q["qs"].astype(np.float64) * d
    err = np.abs(rec - x.reshape(-1, 32).astype(np.float64))
    assert np.all(err <= d * 0.5 * (1 + 1e-5) + 1e-12)
    assert np.all(np.abs(q["qs"]).max(axis=1) == 127)


def _one_block_rows(nibbles_rows, scale_bits=0x3C00):
    """Q4_0 rows of one block each, scale fp16 (default 1.0)."""
    rows = []
    for nib in nibbles_rows:
        nib = np.asarray(nib, np.int64)        # 32 stored nibbles (value + 8)
        b = np.empty(18, np.uint8)
        b[0] = scale_bits & 0xFF
        b[1] = scale_bits >> 8
        b[2:] = (nib[:16] | (nib[16:] << 4)).astype(np.uint8)
        rows.append(b)
    return np.stack(rows)


def test_matvec_block_dot_is_exact_integer():
    # wd = xd = 1: y is the block's integer dot, checked against int64 brute force
    g = np.random.default_rng(2)
    nib = g.integers(0, 16, (8, 32))
    xq = g.integers(-127, 128, 32)
    W = _one_block_rows(nib)
    y = O.q4_0_q8_0_matvec(W, q8_block(xq, 1.0), 8, 32)
    want = ((nib - 8) * xq[None, :]).sum(axis=1)
    assert np.array_equal(y, want.astype(np.float32))


def test_matvec_nibble_order():
    # stored byte j: low nibble = weight j, high nibble = weight j + 16
    nib = np.full(32, 8)            # all weights 0
    nib[0] = 15                     # weight 0 -> +7
    nib[16] = 0                     # weight 16 -> -8
    W = _one_block_rows([nib])
    assert W[0, 2] == 0x0F
    xq = np.zeros(32, np.int64)
    xq[0], xq[16] = 3, 5
    y = O.q4_0_q8_0_matvec(W, q8_block(xq, 1.0), 1, 32)
    assert y[0] == 7 * 3 - 8 * 5


def test_matvec_scales_multiply():
    nib = np.full(32, 9)            # weights +1
    W = _one_block_rows([nib], scale_bits=0x3800)     # fp16 0.5
    y = O.q4_0_q8_0_matvec(W, q8_block(np.full(32, 2), 0.25), 1, 32)
    assert y[0] == np.float32(0.5 * 0.25 * 64)


@pytest.mark.parametrize("out_dim,in_dim", [(64, 4096), (37, 256), (16, 14336)])
def test_matvec_matches_float64_dequant(out_dim, in_dim):
    g = np.random.default_rng(out_dim + in_dim)
    x = g.standard_normal(in_dim).astype(np.float32)
    xq = O.quantize_q8_0(x)
    W = O.make_q4_0(g, out_dim, in_dim)
    y = O.q4_0_q8_0_matvec(W, xq, out_dim, in_dim)
    xd = (xq["qs"].astype(np.float64) * xq["d"].astype(np.float64)[:, None]).reshape(-1)
    ref = O.dequant_q4_0(W, out_dim, in_dim) @ xd
    scale = np.abs(O.dequant_q4_0(W, out_dim, in_dim)) @ np.abs(xd)
    assert np.all(np.abs(y - ref) <= 1e-6 * scale + 1e-7)


def test_matvec_qkv_is_three_matvecs():
    g = np.random.default_rng(3)
    dim, kv, ind = 256, 64, 512
    xq = O.quantize_q8_0(g.standard_normal(ind).astype(np.float32))
    Wq, Wk, Wv = O.make_q4_0(g, dim, ind), O.make_q4_0(g, kv, ind), O.make_q4_0(g, kv, ind)
    yq, yk, yv = O.q4_0_q8_0_matvec_qkv(Wq, Wk, Wv, xq, dim, kv, ind)
    assert np.array_equal(yq, O.q4_0_q8_0_matvec(Wq, xq, dim, ind))
    assert np.array_equal(yk, O.q4_0_q8_0_matvec(Wk, xq, kv, ind))
    assert np.array_equal(yv, O.q4_0_q8_0_matvec(Wv, xq, kv, ind))
