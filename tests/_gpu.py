"""GPU-side helpers for the parity tests: every call goes through the C ABI of
libmiattn.so (test infrastructure)."""

from __future__ import annotations

import sys

import numpy as np

import anetransformers_amd as mia
from anetransformers_amd import DeviceBuffer as DB
from anetransformers_amd import check

N_HEADS, N_KV, HD = 32, 8, 128


def lib():
    return mia.init(0)


def say(msg: str) -> None:
    """Name the case on stdout before a GPU step, flushed."""
    print(msg, flush=True)
    sys.stdout.flush()


def decode_step(kc, vc, q, k, v, th, M, pos):
    """Fused mia_decode_step on copies of the ring; returns (out, kc', vc')."""
    L = lib()
    dkc, dvc = DB.from_array(kc), DB.from_array(vc)
    dq, dk, dv, dth = DB.from_array(q), DB.from_array(k), DB.from_array(v), DB.from_array(th)
    dout = DB(N_HEADS * HD * 4)
    check(L.mia_decode_step(dq.ptr, dk.ptr, dv.ptr, dth.ptr, dkc.ptr, dvc.ptr, dout.ptr, N_HEADS,
                            N_KV, HD, M, pos, None), "decode_step")
    check(L.mia_stream_sync(None), "sync")
    return (dout.download(N_HEADS * HD, np.float32), dkc.download(kc.shape, np.uint16),
            dvc.download(vc.shape, np.uint16))


def gqa_attention(q, kc, vc, M, pos):
    L = lib()
    dkc, dvc, dq = DB.from_array(kc), DB.from_array(vc), DB.from_array(q)
    dout = DB(N_HEADS * HD * 4)
    check(L.mia_gqa_attention(dq.ptr, dout.ptr, dkc.ptr, dvc.ptr, N_HEADS, N_HEADS // N_KV, HD, M,
                              pos, None), "gqa_attention")
    check(L.mia_stream_sync(None), "sync")
    return dout.download(N_HEADS * HD, np.float32)


def attention_batch(Q, kc, vc, M, start, S):
    L = lib()
    dkc, dvc, dq = DB.from_array(kc), DB.from_array(vc), DB.from_array(Q)
    dout = DB(S * N_HEADS * HD * 4)
    check(L.mia_attention_batch(dq.ptr, dout.ptr, dkc.ptr, dvc.ptr, N_HEADS, N_KV, HD, M, start, S,
                                None), "attention_batch")
    check(L.mia_stream_sync(None), "sync")
    return dout.download((S, N_HEADS * HD), np.float32)


def attention_step(kc, vc, Q, K, V, th, M, start, S):
    L = lib()
    dkc, dvc = DB.from_array(kc), DB.from_array(vc)
    dq, dk, dv, dth = DB.from_array(Q), DB.from_array(K), DB.from_array(V), DB.from_array(th)
    dout = DB(S * N_HEADS * HD * 4)
    check(L.mia_attention_step(dq.ptr, dk.ptr, dv.ptr, dth.ptr, dkc.ptr, dvc.ptr, dout.ptr, N_HEADS,
                               N_KV, HD, M, start, S, None), "attention_step")
    check(L.mia_stream_sync(None), "sync")
    return (dout.download((S, N_HEADS * HD), np.float32), dkc.download(kc.shape, np.uint16),
            dvc.download(vc.shape, np.uint16))
