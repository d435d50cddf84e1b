#!/usr/bin/env python3
"""Writes the golden fixtures in this directory from the strict CPU oracle.

The reference holds no vector files (its tests draw unseeded arc4random
inputs, tests/test_harness.h:146-149), so the fixtures are ours:
  tiny_decode.npz   mistral_test_config shapes (tests/test_cpu_ref.h:33-41:
                    8 q / 2 kv heads, hd 32, max_seq 128) on a wrapped ring,
                    full inputs and outputs of ora_gqa_attention
  tiny_batch.npz    same shapes, attention_batch over S=6 tokens
  decode_l513.npz   single-layer decode step of the reference's CPU case
                    (32 q / 8 kv, hd 128, 512 cached + new token at 512,
                    theta 1e6, seed 0): inputs are regenerated from the seed,
                    their sha256 is stored, with the output and the written
                    ring rows.
Run: python tests/golden/make_golden.py
"""

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import _data as D  # noqa: E402
import _oracle as O  # noqa: E402


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def tiny_decode():
    g = D.rng(2024)
    nh, nkv, hd, M, pos = 8, 2, 32, 128, 300
    kc, vc = D.ring(g, M, nkv * hd)
    q = D.normal(g, nh * hd)
    out = O.gqa_attention(q, kc, vc, nh, nh // nkv, hd, M, pos)
    return dict(kc=kc, vc=vc, q=q, out=out, shape=np.array([nh, nkv, hd, M, pos]))


def tiny_batch():
    g = D.rng(2025)
    nh, nkv, hd, M, start, S = 8, 2, 32, 128, 40, 6
    kc, vc = D.ring(g, M, nkv * hd, filled=start + S)
    Q = D.normal(g, (S, nh * hd))
    out = O.attention_batch(Q, kc, vc, nh, nkv, hd, M, start, S)
    return dict(kc=kc, vc=vc, Q=Q, out=out, shape=np.array([nh, nkv, hd, M, start, S]))


def decode_l513_inputs():
    g = D.rng(0)
    M, pos = 4096, 512
    kc, vc = D.ring(g, M, filled=pos)
    q, k, v = D.normal(g, 4096), D.normal(g, 1024), D.normal(g, 1024)
    return kc, vc, q, k, v, M, pos


def decode_l513():
    kc, vc, q, k, v, M, pos = decode_l513_inputs()
    th = O.theta_inv(D.THETA, D.HD)
    kc2, vc2 = kc.copy(), vc.copy()
    out = O.decode_step(kc2, vc2, q, k, v, pos, th, 32, 8, 128, M)
    return dict(inputs_sha256=np.array(sha(kc, vc, q, k, v)), theta_inv=th, out=out,
                k_row=kc2[pos % M], v_row=vc2[pos % M], shape=np.array([32, 8, 128, M, pos]))


def main():
    for name, fn in [("tiny_decode", tiny_decode), ("tiny_batch", tiny_batch),
                     ("decode_l513", decode_l513)]:
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
