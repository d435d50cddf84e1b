"""CPU tier: the oracle reproduces the committed golden fixtures
(tests/golden/make_golden.py), and the fixture inputs are what the seeded
generator yields on this numpy."""

import os
import sys

import numpy as np

import _data as D
import _oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden as MG  # noqa: E402


def _load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def test_tiny_decode_fixture():
    f = _load("tiny_decode")
    nh, nkv, hd, M, pos = (int(x) for x in f["shape"])
    out = O.gqa_attention(f["q"], f["kc"], f["vc"], nh, nh // nkv, hd, M, pos)
    assert np.array_equal(out, f["out"])
    ref = D.gqa_decode_f64(f["q"], f["kc"], f["vc"], nh, nkv, hd, M, pos)
    assert np.max(np.abs(f["out"] - ref)) < 2e-6


def test_tiny_batch_fixture():
    f = _load("tiny_batch")
    nh, nkv, hd, M, start, S = (int(x) for x in f["shape"])
    out = O.attention_batch(f["Q"], f["kc"], f["vc"], nh, nkv, hd, M, start, S)
    assert np.array_equal(out, f["out"])


def test_decode_l513_fixture():
    f = _load("decode_l513")
    kc, vc, q, k, v, M, pos = MG.decode_l513_inputs()
    assert MG.sha(kc, vc, q, k, v) == str(f["inputs_sha256"]), "seeded generator drifted"
    th = O.theta_inv(D.THETA, D.HD)
    assert np.array_equal(th, f["theta_inv"])
    out = O.decode_step(kc, vc, q, k, v, pos, th, 32, 8, 128, M)
    assert np.array_equal(out, f["out"])
    assert np.array_equal(kc[pos % M], f["k_row"]) and np.array_equal(vc[pos % M], f["v_row"])
