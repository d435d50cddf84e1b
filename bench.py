#!/usr/bin/env python3
"""Benchmark of the Mistral-7B GQA attention hot path on one MI355X.

Headline metric: decode attention HBM GB/s (% of peak) at 32K context, and
prefill attention TFLOP/s (% of fp16 MFMA peak).

  decode  (value): 32 layers, each a 32768-slot fp16 ring already full, new
          token at position 32768 (wraps into slot 0), every 1024th key x4.
          One step = 32 fused launches of mia_decode_step (RoPE q/k, fp16
          ring write, split-K flash-decode with LSE merge).
  prefill:         32 layers, 1536 cached positions + 512 new tokens
          (positions 1536..2047, causal), fp32 Q, fp16-valued K/V.  One step = 32
          calls of mia_attention_step (K RoPE + ring write, flash kernel).

roofline.achieved divides the algorithmic bytes (decode) or FLOPs (prefill)
of one launch by the dominant kernel's average duration, taken from HIP event
pairs that the kernel's own dispatch stamps (mia_profile_begin/end) during a
second pass over the same timed loop.

configs: the other config shapes (a 513-position single layer, a 4097-position
32-layer decode, the 8-draft verify on a wrapped 65536-slot ring), each with
its oracle CPU timing: reported beside the headline, not as it.

peaks: measured roofs on this part (include/mia_peaks.h): a plain HBM read
stream, the decode kernel's own load pattern over the headline's rings with no
arithmetic, and an fp16 MFMA loop; the roofline objects quote their fraction
of both the published and the measured peak.

dropin: the same decode step through the C drop-in (mia_dropin_decode_step)
with host q/k/v/out buffers, synchronous per layer as the reference's call
site is: the PCIe-inclusive rate, reported beside the headline, never as it.

Inputs are synthetic (seeded) and resident in HBM before timing starts.
Prints one JSON line.
"""

from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

import anetransformers_amd as mia  # noqa: E402
from anetransformers_amd import DeviceBuffer, Event, check  # noqa: E402

N_LAYERS, N_HEADS, N_KV, HD = 32, 32, 8, 128
KV_DIM = N_KV * HD
THETA = 1e6
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
MFMA_F16_PEAK_TFS = 2500.0   # MI355X dense fp16 MFMA

DECODE_M, DECODE_POS = 32768, 32768
DECODE_L = min(DECODE_POS + 1, DECODE_M)
DECODE_BYTES_PER_LAYER = 2 * N_KV * HD * 2 * DECODE_L          # K and V, fp16, once

PF_M, PF_START, PF_S = 4096, 1536, 512
PF_PAIRS_PER_HEAD = sum(PF_START + 1 + i for i in range(PF_S))   # unmasked (query, key)
PF_FLOP_PER_LAYER = 4 * HD * N_HEADS * PF_PAIRS_PER_HEAD


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def theta_inv() -> np.ndarray:
    i = np.arange(HD // 2, dtype=np.float32)
    return (np.float32(1.0) / np.power(np.float32(THETA), (np.float32(2.0) * i) / np.float32(HD))
            ).astype(np.float32)


def f16_valued(g, shape) -> np.ndarray:
    return g.standard_normal(shape, dtype=np.float32).astype(np.float16).astype(np.float32)


class Decode:
    """32 layers x 32768-slot rings, fused decode step per layer."""

    def __init__(self, lib, seed: int = 0):
        self.lib = lib
        ring = (N_LAYERS * DECODE_M, KV_DIM)
        nbytes = ring[0] * ring[1] * 2
        self.kc = DeviceBuffer(nbytes)
        self.vc = DeviceBuffer(nbytes)
        check(lib.mia_fill_normal_f16(self.kc.ptr, ring[0] * ring[1], seed * 2 + 1, None))
        check(lib.mia_fill_normal_f16(self.vc.ptr, ring[0] * ring[1], seed * 2 + 2, None))
        # every 1024th key x4: ring full, so slot == position and rows of all
        # layers with global row % 1024 == 0 are exactly those positions
        check(lib.mia_scale_rows_f16(self.kc.ptr, ring[0], KV_DIM, 1024, 0, 4.0, None))
        g = np.random.default_rng(seed)
        self.q = DeviceBuffer.from_array(g.standard_normal((N_LAYERS, N_HEADS * HD), np.float32))
        self.k = DeviceBuffer.from_array(g.standard_normal((N_LAYERS, KV_DIM), np.float32))
        self.v = DeviceBuffer.from_array(g.standard_normal((N_LAYERS, KV_DIM), np.float32))
        self.th = DeviceBuffer.from_array(theta_inv())
        self.out = DeviceBuffer(N_LAYERS * N_HEADS * HD * 4)
        check(lib.mia_device_sync())

    def step(self) -> None:
        lay = DECODE_M * KV_DIM * 2
        for l in range(N_LAYERS):
            check(self.lib.mia_decode_step(
                self.q.ptr + l * N_HEADS * HD * 4, self.k.ptr + l * KV_DIM * 4,
                self.v.ptr + l * KV_DIM * 4, self.th.ptr, self.kc.ptr + l * lay,
                self.vc.ptr + l * lay, self.out.ptr + l * N_HEADS * HD * 4, N_HEADS, N_KV, HD,
                DECODE_M, DECODE_POS, None), "decode_step")


class DropinDecode:
    """The decode workload through the C drop-in: host buffers, one
    synchronous mia_dropin_decode_step per layer on the same device rings."""

    def __init__(self, lib, dec: Decode, seed: int = 0):
        self.lib = lib
        g = np.random.default_rng(seed + 100)
        self.kv = mia.KVCache(N_LAYERS, N_KV, HD, DECODE_M, KV_DIM, dec.kc.ptr, dec.vc.ptr, 0,
                              DECODE_M)
        self.q = g.standard_normal((N_LAYERS, N_HEADS * HD), np.float32)
        self.k = g.standard_normal((N_LAYERS, KV_DIM), np.float32)
        self.v = g.standard_normal((N_LAYERS, KV_DIM), np.float32)
        self.th = theta_inv()
        self.out = np.empty((N_LAYERS, N_HEADS * HD), np.float32)
        lib.mia_dropin_set_abort(0)

    def step(self) -> None:
        kv = ctypes.byref(self.kv)
        for l in range(N_LAYERS):
            self.lib.mia_dropin_decode_step(kv, l, self.q[l].ctypes.data, self.k[l].ctypes.data,
                                            self.v[l].ctypes.data, DECODE_POS,
                                            self.th.ctypes.data, N_HEADS, N_KV,
                                            self.out[l].ctypes.data)
            if self.lib.mia_dropin_status() != 0:
                raise mia.MiattnError(self.lib.mia_dropin_status(),
                                      self.lib.mia_last_error().decode())


def wall_ms(fn, steps: int, warmup: int) -> float:
    """Mean wall-clock ms per call of a synchronous fn."""
    for _ in range(warmup):
        fn()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    return (time.perf_counter() - t0) * 1e3 / steps


class Prefill:
    """32 layers, 1536 cached + 512 new tokens per layer."""

    def __init__(self, lib, seed: int = 7):
        self.lib = lib
        g = np.random.default_rng(seed)
        lay_elems = PF_M * KV_DIM
        self.kc = DeviceBuffer(N_LAYERS * lay_elems * 2)
        self.vc = DeviceBuffer(N_LAYERS * lay_elems * 2)
        self.kc.zero()
        self.vc.zero()
        for l in range(N_LAYERS):   # cached positions 0..1535 (calloc'd rest)
            check(lib.mia_fill_normal_f16(self.kc.ptr + l * lay_elems * 2, PF_START * KV_DIM,
                                          1000 + 2 * l, None))
            check(lib.mia_fill_normal_f16(self.vc.ptr + l * lay_elems * 2, PF_START * KV_DIM,
                                          1001 + 2 * l, None))
        self.Q = DeviceBuffer.from_array(g.standard_normal((N_LAYERS, PF_S, N_HEADS * HD),
                                                           np.float32))
        self.K = DeviceBuffer.from_array(f16_valued(g, (N_LAYERS, PF_S, KV_DIM)))
        self.V = DeviceBuffer.from_array(f16_valued(g, (N_LAYERS, PF_S, KV_DIM)))
        self.th = DeviceBuffer.from_array(theta_inv())
        self.out = DeviceBuffer(N_LAYERS * PF_S * N_HEADS * HD * 4)
        check(lib.mia_device_sync())

    def _ptrs(self, l):
        lay = PF_M * KV_DIM * 2
        return (self.Q.ptr + l * PF_S * N_HEADS * HD * 4, self.K.ptr + l * PF_S * KV_DIM * 4,
                self.V.ptr + l * PF_S * KV_DIM * 4, self.kc.ptr + l * lay, self.vc.ptr + l * lay,
                self.out.ptr + l * PF_S * N_HEADS * HD * 4)

    def step(self) -> None:
        for l in range(N_LAYERS):
            q, k, v, kc, vc, out = self._ptrs(l)
            check(self.lib.mia_attention_step(q, k, v, self.th.ptr, kc, vc, out, N_HEADS, N_KV, HD,
                                              PF_M, PF_START, PF_S, None), "attention_step")


def timed(lib, fn, steps: int, warmup: int) -> float:
    """Mean ms per call of fn over `steps`, HIP events on the library stream."""
    for _ in range(warmup):
        fn()
    check(lib.mia_device_sync())
    e0, e1 = Event(), Event()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    check(lib.mia_device_sync())
    return e0.elapsed_ms(e1) / steps


def kernel_stats(lib, fn, steps: int, kind: int):
    """(launch count, average duration in ms) of the kernels of this kind over
    `steps` calls of fn, from the library's per-kernel HIP event pairs."""
    check(lib.mia_device_sync())
    check(lib.mia_profile_begin())
    for _ in range(steps):
        fn()
    n = ctypes.c_int()
    tot = ctypes.c_double()
    check(lib.mia_profile_end(kind, ctypes.byref(n), ctypes.byref(tot)))
    return n.value, tot.value / max(n.value, 1)


def kernel_avg_ms(lib, fn, steps: int, kind: int) -> float:
    """Average duration of the main attention kernel (kind 0 decode, 1 flash)
    over `steps` calls of fn, from the library's per-kernel HIP event pairs on
    the kernel's own stream (merge kernels excluded)."""
    check(lib.mia_device_sync())
    check(lib.mia_profile_begin())
    for _ in range(steps):
        fn()
    n = ctypes.c_int()
    tot = ctypes.c_double()
    check(lib.mia_profile_end(kind, ctypes.byref(n), ctypes.byref(tot)))
    return tot.value / max(n.value, 1)


def measure_peaks(lib, dec: "Decode", reps: int = 10) -> dict:
    """Measured HBM read and fp16 MFMA peaks (mean over `reps` launches)."""
    nb = 2 << 30
    buf = DeviceBuffer(nb)
    # N(0,1) fp16 like the rings: random bits toggle the HBM bus (constant
    # data reads about 4 % faster on this part)
    check(lib.mia_fill_normal_f16(buf.ptr, nb // 2, 77, None))
    st_ms = timed(lib, lambda: check(lib.mia_peak_read_stream(buf.ptr, nb, None)), reps, 2)
    del buf
    lay = DECODE_M * KV_DIM * 2
    start = (DECODE_POS + 1 - DECODE_L) % DECODE_M

    def ring_pass():
        for l in range(N_LAYERS):
            check(lib.mia_peak_read_ring(dec.kc.ptr + l * lay, dec.vc.ptr + l * lay, N_KV,
                                         DECODE_M, DECODE_L, start, None))

    rg_ms = timed(lib, ring_pass, max(reps // 4, 2), 1) / N_LAYERS
    flop = ctypes.c_double()
    iters = 1024
    mf_ms = timed(lib, lambda: check(lib.mia_peak_mfma_f16(iters, ctypes.byref(flop), None)),
                  reps, 2)
    # the duration floor of a kernel, measured as the attention kernels' are
    # (dispatch-stamped events): an empty kernel of each of their grids
    empty = {}
    for name, wgs, threads in (("decode_grid_us", N_KV * 32, 512), ("flash_grid_us", N_KV * 32, 256)):
        kernel_avg_ms(lib, lambda: check(lib.mia_peak_empty(wgs, threads, None)), 3, 4)
        empty[name] = round(1e3 * kernel_avg_ms(
            lib, lambda: check(lib.mia_peak_empty(wgs, threads, None)), 20, 4), 2)
    return {
        "hbm_read_stream": {
            "value": round(nb / (st_ms * 1e-3) / 1e9, 1), "unit": "GB/s",
            "workload": "one 2 GiB grid-stride read (N(0,1) fp16 data), 1024 workgroups x "
                        "256 threads, four 16-byte loads in flight per thread",
            "ms_per_launch": round(st_ms, 4)},
        "hbm_read_decode_pattern": {
            "value": round(DECODE_BYTES_PER_LAYER / (rg_ms * 1e-3) / 1e9, 1), "unit": "GB/s",
            "workload": "the headline's 32 rings (K and V, 134 MB each layer) read back to back "
                        "in decode_kernel's chunking and load pattern, no arithmetic",
            "us_per_layer": round(rg_ms * 1e3, 2)},
        "mfma_f16": {
            "value": round(flop.value / (mf_ms * 1e-3) / 1e12, 1), "unit": "TFLOP/s",
            "workload": f"{iters} rounds of 4 independent v_mfma_f32_32x32x16_f16 chains, "
                        "2 waves per SIMD on every CU",
            "ms_per_launch": round(mf_ms, 4)},
        "empty_kernel": dict(empty, workload="a kernel with no body on the decode kernel's grid "
                             "(256 x 512 threads) and the flash kernel's (256 x 256), timed by "
                             "the same dispatch-stamped events as the kernel averages (rocprof "
                             "puts the same empty kernel at ~1.5 us: these events add ~2.5 us to "
                             "a kernel this short, ~0.3 us to the attention kernels)"),
        "published": {"hbm_gbs": HBM_PEAK_GBS, "mfma_f16_tfs": MFMA_F16_PEAK_TFS},
    }


def cpu_baseline_decode(n_layers: int = 8, reps: int = 3):
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import _oracle as O  # the oracle is the timed CPU baseline here

    g = np.random.default_rng(11)
    kc = g.standard_normal((n_layers, DECODE_M, KV_DIM), np.float32)
    kc[:, ::1024] *= 4.0
    kc = kc.astype(np.float16).view(np.uint16)
    vc = g.standard_normal((n_layers, DECODE_M, KV_DIM), np.float32).astype(np.float16).view(np.uint16)
    Q = g.standard_normal((n_layers, N_HEADS * HD), np.float32)
    threads = O.num_threads(fast=True)
    O.decode_layers(Q[:1], kc[:1], vc[:1], 1, N_HEADS, N_HEADS // N_KV, HD, DECODE_M, DECODE_POS,
                    threads=threads)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        O.decode_layers(Q, kc, vc, n_layers, N_HEADS, N_HEADS // N_KV, HD, DECODE_M, DECODE_POS,
                        threads=threads)
        ts.append(time.perf_counter() - t0)
    dt = float(np.median(ts))
    t0 = time.perf_counter()
    O.decode_layers(Q[:1], kc[:1], vc[:1], 1, N_HEADS, N_HEADS // N_KV, HD, DECODE_M, DECODE_POS,
                    threads=1)
    dt1 = time.perf_counter() - t0
    return {
        "value": round(n_layers * DECODE_BYTES_PER_LAYER / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{n_layers} of 32 layers of the same decode workload (32768-slot full ring, "
                  f"new token at 32768), median of {reps}; oracle AVX2+F16C timing build, "
                  f"OpenMP over (layer, head)",
        "single_thread_value": round(DECODE_BYTES_PER_LAYER / dt1 / 1e9, 3),
    }


def cpu_baseline_prefill(n_layers: int = 2):
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import _oracle as O

    g = np.random.default_rng(12)
    kc = np.zeros((n_layers, PF_M, KV_DIM), np.uint16)
    vc = np.zeros((n_layers, PF_M, KV_DIM), np.uint16)
    kc[:, :PF_START + PF_S] = g.standard_normal((n_layers, PF_START + PF_S, KV_DIM),
                                                np.float32).astype(np.float16).view(np.uint16)
    vc[:, :PF_START + PF_S] = g.standard_normal((n_layers, PF_START + PF_S, KV_DIM),
                                                np.float32).astype(np.float16).view(np.uint16)
    Q = g.standard_normal((n_layers, PF_S, N_HEADS * HD), np.float32)
    threads = O.num_threads(fast=True)
    t0 = time.perf_counter()
    O.attention_batch_layers(Q, kc, vc, n_layers, N_HEADS, N_KV, HD, PF_M, PF_START, PF_S,
                             threads=threads)
    dt = time.perf_counter() - t0
    # one thread: the last 64 tokens of one layer (the longest windows)
    n1 = 64
    t0 = time.perf_counter()
    O.attention_batch_layers(Q[:1, PF_S - n1:], kc[:1], vc[:1], 1, N_HEADS, N_KV, HD, PF_M,
                             PF_START + PF_S - n1, n1, threads=1)
    dt1 = time.perf_counter() - t0
    flop1 = 4 * N_HEADS * HD * sum(PF_START + PF_S - n1 + 1 + i for i in range(n1))
    return {
        "value": round(n_layers * PF_FLOP_PER_LAYER / dt / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{n_layers} of 32 layers of the same prefill chunk (attention_batch over "
                  f"1536 cached + 512 new); oracle AVX2+F16C timing build, OpenMP over "
                  f"(layer, token, head)",
        "single_thread_value": round(flop1 / dt1 / 1e12, 5),
        "single_thread_sample": f"one thread, the last {n1} tokens of one layer "
                                f"(windows of {PF_START + PF_S - n1 + 1}..{PF_START + PF_S} keys)",
    }


class OtherConfigs:
    """The remaining config shapes, reported beside the headline: a single
    512-position decode layer (M 4096), a 32-layer decode at 4097 positions
    (M 65536), and a 32-layer speculative verify of 8 drafts at positions
    70000..70007 on a wrapped 65536-slot ring (staged drafts, then commit)."""

    def __init__(self, lib, seed: int = 21):
        self.lib = lib
        g = np.random.default_rng(seed)
        self.th = DeviceBuffer.from_array(theta_inv())
        # config 1: one layer, M 4096, positions 0..511 filled
        self.c1_kc = DeviceBuffer(4096 * KV_DIM * 2)
        self.c1_vc = DeviceBuffer(4096 * KV_DIM * 2)
        self.c1_kc.zero()
        self.c1_vc.zero()
        check(lib.mia_fill_normal_f16(self.c1_kc.ptr, 512 * KV_DIM, 31, None))
        check(lib.mia_fill_normal_f16(self.c1_vc.ptr, 512 * KV_DIM, 32, None))
        # configs 2 and 5: 32 layers of 65536-slot rings, every slot filled
        self.big = N_LAYERS * 65536 * KV_DIM
        self.kc = DeviceBuffer(self.big * 2)
        self.vc = DeviceBuffer(self.big * 2)
        check(lib.mia_fill_normal_f16(self.kc.ptr, self.big, 33, None))
        check(lib.mia_fill_normal_f16(self.vc.ptr, self.big, 34, None))
        self.q = DeviceBuffer.from_array(g.standard_normal((N_LAYERS, 8, N_HEADS * HD), np.float32))
        self.k = DeviceBuffer.from_array(g.standard_normal((N_LAYERS, 8, KV_DIM), np.float32))
        self.v = DeviceBuffer.from_array(g.standard_normal((N_LAYERS, 8, KV_DIM), np.float32))
        self.out = DeviceBuffer(N_LAYERS * 8 * N_HEADS * HD * 4)
        # config 5, accept-only form: [layer][8][kv_dim] fp16 staged drafts
        self.kst = DeviceBuffer(N_LAYERS * 8 * KV_DIM * 2)
        self.vst = DeviceBuffer(N_LAYERS * 8 * KV_DIM * 2)
        check(lib.mia_device_sync())

    def _args(self, l, S):
        return (self.q.ptr + l * 8 * N_HEADS * HD * 4, self.k.ptr + l * 8 * KV_DIM * 4,
                self.v.ptr + l * 8 * KV_DIM * 4, self.th.ptr)

    def c1(self) -> None:
        q, k, v, th = self._args(0, 1)
        check(self.lib.mia_decode_step(q, k, v, th, self.c1_kc.ptr, self.c1_vc.ptr, self.out.ptr,
                                       N_HEADS, N_KV, HD, 4096, 512, None), "decode_step")

    def c2(self) -> None:
        lay = 65536 * KV_DIM * 2
        for l in range(N_LAYERS):
            q, k, v, th = self._args(l, 1)
            check(self.lib.mia_decode_step(q, k, v, th, self.kc.ptr + l * lay, self.vc.ptr + l * lay,
                                           self.out.ptr + l * N_HEADS * HD * 4, N_HEADS, N_KV, HD,
                                           65536, 4096, None), "decode_step")

    def c5(self) -> None:
        lay = 65536 * KV_DIM * 2
        for l in range(N_LAYERS):
            q, k, v, th = self._args(l, 8)
            check(self.lib.mia_attention_step(q, k, v, th, self.kc.ptr + l * lay,
                                              self.vc.ptr + l * lay,
                                              self.out.ptr + l * 8 * N_HEADS * HD * 4, N_HEADS,
                                              N_KV, HD, 65536, 70000, 8, None), "attention_step")

    def c5_sequential(self) -> None:
        """Config 5 as the reference verifies without a batch path
        (speculative.h:92-101): 8 decode steps per layer, drafts at positions
        70000..70007, each written and attended in turn."""
        lay = 65536 * KV_DIM * 2
        for l in range(N_LAYERS):
            for t in range(8):
                q = self.q.ptr + (l * 8 + t) * N_HEADS * HD * 4
                k = self.k.ptr + (l * 8 + t) * KV_DIM * 4
                v = self.v.ptr + (l * 8 + t) * KV_DIM * 4
                check(self.lib.mia_decode_step(q, k, v, self.th.ptr, self.kc.ptr + l * lay,
                                               self.vc.ptr + l * lay,
                                               self.out.ptr + (l * 8 + t) * N_HEADS * HD * 4,
                                               N_HEADS, N_KV, HD, 65536, 70000 + t, None),
                      "decode_step")

    def c5_staged(self, n_keep: int = 5) -> None:
        """Config 5 with the ring left alone during the 32 layers' attention
        and one commit of the accepted drafts for all layers afterwards."""
        lay = 65536 * KV_DIM * 2
        for l in range(N_LAYERS):
            q, k, v, th = self._args(l, 8)
            check(self.lib.mia_attention_step_staged(
                q, k, v, th, self.kc.ptr + l * lay, self.vc.ptr + l * lay,
                self.kst.ptr + l * 8 * KV_DIM * 2, self.vst.ptr + l * 8 * KV_DIM * 2,
                self.out.ptr + l * 8 * N_HEADS * HD * 4, N_HEADS, N_KV, HD, 65536, 70000, 8,
                None), "attention_step_staged")
        check(self.lib.mia_commit_staged(self.kc.ptr, self.vc.ptr, self.kst.ptr, self.vst.ptr,
                                         N_LAYERS, 8, n_keep, 70000, 65536, KV_DIM, None),
              "commit_staged")


DIM = N_HEADS * HD
Q4_ROW_BYTES = DIM // 32 * 18                    # a 4096-wide Q4_0 row
Q8_BYTES = DIM // 32 * 36                        # the quantised 4096-vector
QKV_ROWS = DIM + 2 * KV_DIM
# algorithmic bytes of one fused launch: Q4_0 weights + fp32 x + fp32 y
QKV_BYTES = QKV_ROWS * Q4_ROW_BYTES + DIM * 4 + QKV_ROWS * 4
WO_BYTES = DIM * Q4_ROW_BYTES + DIM * 4 + DIM * 4


class Projections:
    """The W4A8 projections either side of the attention step, 32 layers:
    per layer quantize(xb) -> fused QKV matvec, quantize(attention out) -> Wo
    (mistral_model.h:833-842, 866-867).  Each layer has its own Q4_0 weights
    (755 MB in all, far beyond the caches), filled with a seeded fp16 N(0,1)
    stream read as Q4_0 bytes (finite scales, uniform-looking nibbles), scaled
    so that the outputs are O(1)."""

    def __init__(self, lib, seed: int = 41):
        self.lib = lib
        g = np.random.default_rng(seed)
        self.lw = QKV_ROWS * Q4_ROW_BYTES + DIM * Q4_ROW_BYTES   # per layer: Wq Wk Wv Wo
        self.w = DeviceBuffer(N_LAYERS * self.lw)
        check(lib.mia_fill_normal_f16(self.w.ptr, N_LAYERS * self.lw // 2, seed, None))
        # x 2^-8 keeps the scales near 0.004, so q, k, v come out O(1) for the
        # attention block below
        check(lib.mia_scale_rows_f16(self.w.ptr, N_LAYERS * self.lw // 2048, 1024, 1, 0,
                                     1.0 / 256, None))
        self.x = DeviceBuffer.from_array(g.standard_normal((N_LAYERS, DIM), np.float32))
        self.a = DeviceBuffer.from_array(g.standard_normal((N_LAYERS, DIM), np.float32))
        self.q8 = DeviceBuffer(Q8_BYTES)
        self.y = DeviceBuffer(N_LAYERS * (QKV_ROWS + DIM) * 4)
        check(lib.mia_device_sync())

    def _w(self, l):
        base = self.w.ptr + l * self.lw
        wq = base
        wk = wq + DIM * Q4_ROW_BYTES
        wv = wk + KV_DIM * Q4_ROW_BYTES
        wo = wv + KV_DIM * Q4_ROW_BYTES
        return wq, wk, wv, wo

    def _y(self, l):
        yq = self.y.ptr + l * (QKV_ROWS + DIM) * 4
        yk = yq + DIM * 4
        yv = yk + KV_DIM * 4
        yo = yv + KV_DIM * 4
        return yq, yk, yv, yo

    def qkv(self, l, x_ptr):
        wq, wk, wv, _ = self._w(l)
        yq, yk, yv, _ = self._y(l)
        check(self.lib.mia_quantize_q8_0(x_ptr, self.q8.ptr, DIM, None), "quantize")
        check(self.lib.mia_q4_0_matvec_qkv(wq, wk, wv, self.q8.ptr, yq, yk, yv, DIM, KV_DIM, DIM,
                                           None), "qkv")
        return yq, yk, yv

    def wo(self, l, a_ptr):
        _, _, _, wo = self._w(l)
        _, _, _, yo = self._y(l)
        check(self.lib.mia_quantize_q8_0(a_ptr, self.q8.ptr, DIM, None), "quantize")
        check(self.lib.mia_q4_0_matvec(wo, self.q8.ptr, yo, DIM, DIM, None), "wo")

    def qkv_fused(self, l, x_ptr):
        wq, wk, wv, _ = self._w(l)
        yq, yk, yv, _ = self._y(l)
        check(self.lib.mia_q4_0_matvec_qkv_f32(wq, wk, wv, x_ptr, yq, yk, yv, DIM, KV_DIM, DIM,
                                               None), "qkv_f32")
        return yq, yk, yv

    def wo_fused(self, l, a_ptr):
        _, _, _, wo = self._w(l)
        _, _, _, yo = self._y(l)
        check(self.lib.mia_q4_0_matvec_f32(wo, a_ptr, yo, DIM, DIM, None), "wo_f32")

    def step_two_launch(self) -> None:
        """The reference's call pattern: quantize, then the matvec."""
        for l in range(N_LAYERS):
            self.qkv(l, self.x.ptr + l * DIM * 4)
            self.wo(l, self.a.ptr + l * DIM * 4)

    def step(self) -> None:
        """Quantize folded into the matvec launches."""
        for l in range(N_LAYERS):
            self.qkv_fused(l, self.x.ptr + l * DIM * 4)
            self.wo_fused(l, self.a.ptr + l * DIM * 4)

    def block_step(self, dec: "Decode") -> None:
        """The attention block of the decode step on the device: projections
        around the fused attention at 32K context (mia_decode_step)."""
        lay = DECODE_M * KV_DIM * 2
        for l in range(N_LAYERS):
            yq, yk, yv = self.qkv_fused(l, self.x.ptr + l * DIM * 4)
            out = dec.out.ptr + l * DIM * 4
            check(self.lib.mia_decode_step(yq, yk, yv, dec.th.ptr, dec.kc.ptr + l * lay,
                                           dec.vc.ptr + l * lay, out, N_HEADS, N_KV, HD, DECODE_M,
                                           DECODE_POS, None), "decode_step")
            self.wo_fused(l, out)


def cpu_baseline_projections(n_layers: int = 4, reps: int = 3):
    """The oracle's row-parallel W4A8 matvec (OpenMP) on n_layers layers of
    the same projections: quantize + QKV + quantize + Wo."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import _oracle as O

    g = np.random.default_rng(14)
    Ws = [(O.make_q4_0(g, QKV_ROWS, DIM), O.make_q4_0(g, DIM, DIM)) for _ in range(n_layers)]
    xs = g.standard_normal((n_layers, 2, DIM), np.float32)
    threads = O.num_threads(fast=True)

    def run():
        for l in range(n_layers):
            O.q4_0_q8_0_matvec_parallel(Ws[l][0], O.quantize_q8_0(xs[l, 0]), QKV_ROWS, DIM,
                                        threads=threads)
            O.q4_0_q8_0_matvec_parallel(Ws[l][1], O.quantize_q8_0(xs[l, 1]), DIM, DIM,
                                        threads=threads)

    run()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    dt = float(np.median(ts))
    return {"value": round(n_layers * (QKV_BYTES + WO_BYTES) / dt / 1e9, 3), "unit": "GB/s",
            "cores": threads, "kind": "port",
            "sample": f"{n_layers} of 32 layers (quantize + QKV rows 6144 + quantize + Wo rows "
                      f"4096, in_dim 4096), median of {reps}; oracle timing build, OpenMP over "
                      f"rows"}


HIDDEN = 14336
LAYER_GEMMS = ((QKV_ROWS, DIM), (DIM, DIM), (HIDDEN, DIM), (HIDDEN, DIM), (DIM, HIDDEN))
LAYER_GEMM_FLOP = sum(2 * PF_S * n * k for n, k in LAYER_GEMMS)      # per layer, S = 512


def q4_bytes(rows: int, cols: int) -> int:
    return rows * (cols // 32) * 18


class PrefillLayers:
    """The whole prefill layer on the GPU (mia_prefill_layer_packed), 32 layers
    with their own Q4_0 weights (3.9 GB, regrouped once into the GEMM tile
    layout by mia_q4_0_pack_gemm at set-up, as a loader would), S = 512 new
    tokens after 1536 cached positions, the residual stream X carried from
    layer to layer.  packed=False: mia_prefill_layer on the GGUF layout."""

    def __init__(self, lib, seed: int = 51, packed: bool = True):
        self.lib = lib
        self.packed = packed
        g = np.random.default_rng(seed)
        self.sizes = [("wq", DIM, DIM), ("wk", KV_DIM, DIM), ("wv", KV_DIM, DIM), ("wo", DIM, DIM),
                      ("w1", HIDDEN, DIM), ("w2", DIM, HIDDEN), ("w3", HIDDEN, DIM)]
        self.lw_bytes = sum(q4_bytes(r, c) for _, r, c in self.sizes)
        self.w = DeviceBuffer(N_LAYERS * self.lw_bytes)
        check(lib.mia_fill_normal_f16(self.w.ptr, N_LAYERS * self.lw_bytes // 2, seed, None))
        # x 2^-12 keeps the block scales near 2.4e-4: the residual stream stays O(1)
        check(lib.mia_scale_rows_f16(self.w.ptr, N_LAYERS * self.lw_bytes // 2048, 1024, 1, 0,
                                     1.0 / 4096, None))
        if packed:
            wp = DeviceBuffer(N_LAYERS * self.lw_bytes)
            off = 0
            for _ in range(N_LAYERS):
                for _, r, c in self.sizes:
                    check(lib.mia_q4_0_pack_gemm(self.w.ptr + off, wp.ptr + off, r, c, None))
                    off += q4_bytes(r, c)
            check(lib.mia_device_sync())
            self.w = wp                              # (the GGUF-layout copy is freed)
        self.norms = DeviceBuffer.from_array(
            (1.0 + 0.1 * g.standard_normal((N_LAYERS, 2, DIM))).astype(np.float32))
        lay = PF_M * KV_DIM
        self.kc = DeviceBuffer(N_LAYERS * lay * 2)
        self.vc = DeviceBuffer(N_LAYERS * lay * 2)
        self.kc.zero()
        self.vc.zero()
        for l in range(N_LAYERS):
            check(lib.mia_fill_normal_f16(self.kc.ptr + l * lay * 2, PF_START * KV_DIM, 2000 + l, None))
            check(lib.mia_fill_normal_f16(self.vc.ptr + l * lay * 2, PF_START * KV_DIM, 3000 + l, None))
        self.X = DeviceBuffer.from_array(g.standard_normal((PF_S, DIM)).astype(np.float32))
        self.th = DeviceBuffer.from_array(theta_inv())
        self.lws = []
        for l in range(N_LAYERS):
            ptrs, off = {}, self.w.ptr + l * self.lw_bytes
            for name, r, c in self.sizes:
                ptrs[name] = off
                off += q4_bytes(r, c)
            nb = self.norms.ptr + l * 2 * DIM * 4
            self.lws.append(mia.LayerWeights(ptrs["wq"], ptrs["wk"], ptrs["wv"], ptrs["wo"],
                                             ptrs["w1"], ptrs["w2"], ptrs["w3"], nb, nb + DIM * 4))
        check(lib.mia_device_sync())

    def step(self) -> None:
        lay = PF_M * KV_DIM * 2
        fn = self.lib.mia_prefill_layer_packed if self.packed else self.lib.mia_prefill_layer
        for l in range(N_LAYERS):
            check(fn(self.X.ptr, ctypes.byref(self.lws[l]), self.th.ptr, self.kc.ptr + l * lay,
                     self.vc.ptr + l * lay, DIM, HIDDEN, N_HEADS, N_KV, 1e-5, PF_M, PF_START, PF_S,
                     None), "prefill_layer")


# Q4_K_M's mix (the reference's target files): Q4_K everywhere but the value
# and down projections, which are Q6_K
TYPE_Q4_K, TYPE_Q6_K = mia.TYPE_Q4_K, mia.TYPE_Q6_K
KM_SIZES = (("wq", DIM, DIM, TYPE_Q4_K), ("wk", KV_DIM, DIM, TYPE_Q4_K),
            ("wv", KV_DIM, DIM, TYPE_Q6_K), ("wo", DIM, DIM, TYPE_Q4_K),
            ("w1", HIDDEN, DIM, TYPE_Q4_K), ("w2", DIM, HIDDEN, TYPE_Q6_K),
            ("w3", HIDDEN, DIM, TYPE_Q4_K))


def km_bytes(rows: int, cols: int, t: int) -> int:
    return rows * (cols // 256) * (144 if t == TYPE_Q4_K else 210)


def km_weights(lib, seed: int):
    """32 layers of Q4_K_M matrices in one device buffer: (buffer, offsets of
    the seven matrices in a layer, bytes per layer).  A seeded fp16 N(0,1)
    stream read as the blocks, with the block scales scaled down so that the
    activations stay O(1)."""
    offs, off = {}, 0
    for name, r, c, t in KM_SIZES:
        offs[name] = off
        off += (km_bytes(r, c, t) + 255) // 256 * 256
    w = DeviceBuffer(N_LAYERS * off)
    check(lib.mia_fill_normal_f16(w.ptr, N_LAYERS * off // 2, seed, None))
    for l in range(N_LAYERS):
        for name, r, c, t in KM_SIZES:
            base = w.ptr + l * off + offs[name]
            n16 = km_bytes(r, c, t) // 2
            if t == TYPE_Q4_K:   # d and dmin: the first 2 of each block's 72 fp16
                check(lib.mia_scale_rows_f16(base, n16 // 2, 2, 36, 0, 1.0 / 16384, None))
            else:                # d: fp16 104 of each block's 105
                check(lib.mia_scale_rows_f16(base, n16, 1, 105, 104, 1.0 / 65536, None))
    return w, offs, off


class DecodeLayers:
    """The whole decode layer on the GPU (mia_decode_layer), 32 layers, for the
    token at position 32768 over the headline's full 32768-slot rings: Q4_0
    weights (3.9 GB) or Q4_K_M weights (4.45 GB); x carried from layer to
    layer."""

    Q4_SIZES = (("wq", DIM, DIM), ("wk", KV_DIM, DIM), ("wv", KV_DIM, DIM), ("wo", DIM, DIM),
                ("w1", HIDDEN, DIM), ("w2", DIM, HIDDEN), ("w3", HIDDEN, DIM))

    def __init__(self, lib, dec: "Decode", kind: str, seed: int = 71):
        self.lib, self.dec, self.kind = lib, dec, kind
        g = np.random.default_rng(seed)
        if kind == "q4_0":
            offs, off = {}, 0
            for name, r, c in self.Q4_SIZES:
                offs[name] = off
                off += (q4_bytes(r, c) + 255) // 256 * 256
            self.w = DeviceBuffer(N_LAYERS * off)
            check(lib.mia_fill_normal_f16(self.w.ptr, N_LAYERS * off // 2, seed, None))
            # x 2^-12 keeps the block scales near 2.4e-4: the residual stream stays O(1)
            check(lib.mia_scale_rows_f16(self.w.ptr, N_LAYERS * off // 2048, 1024, 1, 0,
                                         1.0 / 4096, None))
            types = {n: mia.TYPE_Q4_0 for n, _, _ in self.Q4_SIZES}
            self.weight_bytes = sum(q4_bytes(r, c) for _, r, c in self.Q4_SIZES)
        else:
            self.w, offs, off = km_weights(lib, seed)
            types = {n: t for n, _, _, t in KM_SIZES}
            self.weight_bytes = sum(km_bytes(r, c, t) for _, r, c, t in KM_SIZES)
        self.norms = DeviceBuffer.from_array(
            (1.0 + 0.1 * g.standard_normal((N_LAYERS, 2, DIM))).astype(np.float32))
        self.x = DeviceBuffer.from_array(g.standard_normal(DIM).astype(np.float32))
        names = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")
        self.lws = []
        for l in range(N_LAYERS):
            nb = self.norms.ptr + l * 2 * DIM * 4
            self.lws.append(mia.LayerWeightsTyped(
                *(self.w.ptr + l * off + offs[n] for n in names), *(types[n] for n in names),
                nb, nb + DIM * 4))
        check(lib.mia_device_sync())

    def step(self) -> None:
        lay = DECODE_M * KV_DIM * 2
        for l in range(N_LAYERS):
            check(self.lib.mia_decode_layer(
                self.x.ptr, ctypes.byref(self.lws[l]), self.dec.th.ptr,
                self.dec.kc.ptr + l * lay, self.dec.vc.ptr + l * lay, DIM, HIDDEN, N_HEADS, N_KV,
                1e-5, DECODE_M, DECODE_POS, None), "decode_layer")


def decode_layer_leg(lib, dec: "Decode", steps: int, warmup: int) -> dict:
    out = {"workload": "mia_decode_layer x 32 (RMSNorm, QKV, fused RoPE + ring write + "
                       "attention at 32K context, Wo, residual, RMSNorm, gate / up, SwiGLU, W2, "
                       "residual) for the token at position 32768 over the headline's full "
                       "32768-slot rings"}
    for kind in ("q4_0", "q4_k_m"):
        dl = DecodeLayers(lib, dec, kind)
        ms = timed(lib, dl.step, steps, warmup)
        nbytes = N_LAYERS * (dl.weight_bytes + DECODE_BYTES_PER_LAYER)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[kind] = {"ms_per_token": round(ms, 4), "tokens_per_s": round(1e3 / ms, 2),
                     "value": round(gbs, 2), "unit": "GB/s",
                     "bytes_per_token": nbytes,
                     "bytes": "weights of all 32 layers + the K / V window (32768 positions)",
                     "roofline": {"bound": "hbm", "achieved": round(gbs, 2),
                                  "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                                  "note": "the whole layer's bytes over the step's time "
                                          "(6 launches per layer: 4 matvecs with the "
                                          "RMSNorms, quantisation, residuals and SwiGLU "
                                          "inside, the attention and its merge)"}}
        del dl
    return out


def cpu_baseline_decode_layer() -> dict:
    """The oracle's decode layer (strict build, one thread) on 1 of the 32
    layers at the same 32K context, Q4_0 weights."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import _oracle as O

    g = np.random.default_rng(17)
    types = {n: O.TYPE_Q4_0 for n in O.MATS}
    W = {n: O.make_q4_0(g, r, c) for n, r, c in DecodeLayers.Q4_SIZES}
    W["rms_att"] = np.ones(DIM, np.float32)
    W["rms_ffn"] = np.ones(DIM, np.float32)
    kc = g.standard_normal((DECODE_M, KV_DIM), np.float32).astype(np.float16).view(np.uint16)
    vc = g.standard_normal((DECODE_M, KV_DIM), np.float32).astype(np.float16).view(np.uint16)
    x = g.standard_normal(DIM).astype(np.float32)
    th = theta_inv()
    t0 = time.perf_counter()
    O.decode_layer_typed(W, types, x, kc, vc, DECODE_POS, DIM, HIDDEN, N_HEADS, N_KV, th)
    dt = time.perf_counter() - t0
    nbytes = sum(q4_bytes(r, c) for _, r, c in DecodeLayers.Q4_SIZES) + DECODE_BYTES_PER_LAYER
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "tokens_per_s": round(1.0 / (32 * dt), 4),
            "sample": "1 of 32 layers (Q4_0, token at 32768 over a full 32768-slot ring), "
                      "oracle strict build, one thread; tokens_per_s scaled by 32 layers"}


class TypedLayers:
    """32 layers of Q4_K_M weights (4.45 GB): the decode projections through
    mia_matvec_q8 (the reference's non-Q4_0 branch of q4_matvec_sdot_parallel,
    seven launches per layer on Q8_0 inputs) and the prefill layer (S = 512
    after 1536 cached, X carried) through mia_prefill_layer_typed_packed on
    the weights packed once (mia_gemm_pack), and through
    mia_prefill_layer_typed on the GGUF blocks.  The weight bytes are a seeded
    fp16 N(0,1) stream with the block scales scaled down so that the
    activations stay O(1)."""

    def __init__(self, lib, seed: int = 61):
        self.lib = lib
        g = np.random.default_rng(seed)
        self.w, self.offs, self.lw_bytes = km_weights(lib, seed)
        self.norms = DeviceBuffer.from_array(
            (1.0 + 0.1 * g.standard_normal((N_LAYERS, 2, DIM))).astype(np.float32))
        # decode: Q8_0 inputs (the 4096-wide and 14336-wide vectors of each layer)
        self.x_dim = DeviceBuffer.from_array(g.standard_normal(DIM, np.float32))
        self.x_hid = DeviceBuffer.from_array(g.standard_normal(HIDDEN, np.float32))
        self.q8_dim, self.q8_hid = DeviceBuffer(DIM // 32 * 36), DeviceBuffer(HIDDEN // 32 * 36)
        check(lib.mia_quantize_q8_0(self.x_dim.ptr, self.q8_dim.ptr, DIM, None))
        check(lib.mia_quantize_q8_0(self.x_hid.ptr, self.q8_hid.ptr, HIDDEN, None))
        self.y = DeviceBuffer(N_LAYERS * (DIM * 3 + 2 * KV_DIM + 2 * HIDDEN) * 4)
        # prefill
        lay = PF_M * KV_DIM
        self.kc = DeviceBuffer(N_LAYERS * lay * 2)
        self.vc = DeviceBuffer(N_LAYERS * lay * 2)
        self.kc.zero()
        self.vc.zero()
        for l in range(N_LAYERS):
            check(lib.mia_fill_normal_f16(self.kc.ptr + l * lay * 2, PF_START * KV_DIM, 4000 + l, None))
            check(lib.mia_fill_normal_f16(self.vc.ptr + l * lay * 2, PF_START * KV_DIM, 5000 + l, None))
        self.X = DeviceBuffer.from_array(g.standard_normal((PF_S, DIM)).astype(np.float32))
        self.th = DeviceBuffer.from_array(theta_inv())
        self.lws = []
        for l in range(N_LAYERS):
            p = {n: self.w.ptr + l * self.lw_bytes + self.offs[n] for n, _, _, _ in KM_SIZES}
            t = {n: tt for n, _, _, tt in KM_SIZES}
            nb = self.norms.ptr + l * 2 * DIM * 4
            self.lws.append(mia.LayerWeightsTyped(
                *(p[n] for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3")),
                *(t[n] for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3")), nb, nb + DIM * 4))
        check(lib.mia_device_sync())
        self.decode_bytes = sum(km_bytes(r, c, t) for _, r, c, t in KM_SIZES)
        # the GEMM operand form, converted once as a loader would (mia_gemm_pack)
        self.poffs, off = {}, 0
        for name, r, c, t in KM_SIZES:
            self.poffs[name] = off
            off += (lib.mia_gemm_pack_bytes(t, r, c) + 255) // 256 * 256
        self.plw_bytes = off
        self.wp = DeviceBuffer(N_LAYERS * self.plw_bytes)
        self.plws = []
        for l in range(N_LAYERS):
            p = {n: self.wp.ptr + l * self.plw_bytes + self.poffs[n] for n, _, _, _ in KM_SIZES}
            for name, r, c, t in KM_SIZES:
                check(lib.mia_gemm_pack(self.w.ptr + l * self.lw_bytes + self.offs[name], t,
                                        p[name], r, c, None), "gemm_pack")
            lw = self.lws[l]
            self.plws.append(mia.LayerWeightsTyped(
                *(p[n] for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3")),
                lw.wq_type, lw.wk_type, lw.wv_type, lw.wo_type, lw.w1_type, lw.w2_type,
                lw.w3_type, lw.rms_att, lw.rms_ffn))
        check(lib.mia_device_sync())

    def decode_step(self) -> None:
        y = self.y.ptr
        for l in range(N_LAYERS):
            for name, r, c, t in KM_SIZES:
                x = self.q8_hid.ptr if c == HIDDEN else self.q8_dim.ptr
                check(self.lib.mia_matvec_q8(self.w.ptr + l * self.lw_bytes + self.offs[name], t,
                                             x, y, r, c, None), "matvec_q8")
                y += r * 4

    def prefill_step(self, packed: bool = True) -> None:
        lay = PF_M * KV_DIM * 2
        fn = self.lib.mia_prefill_layer_typed_packed if packed else self.lib.mia_prefill_layer_typed
        lws = self.plws if packed else self.lws
        for l in range(N_LAYERS):
            check(fn(self.X.ptr, ctypes.byref(lws[l]), self.th.ptr, self.kc.ptr + l * lay,
                     self.vc.ptr + l * lay, DIM, HIDDEN, N_HEADS, N_KV, 1e-5, PF_M, PF_START, PF_S,
                     None), "prefill_layer_typed")


def typed_leg(lib, steps: int, warmup: int) -> dict:
    tl = TypedLayers(lib)
    dec_ms = timed(lib, tl.decode_step, steps, warmup)
    n, k_ms = kernel_stats(lib, tl.decode_step, steps, 5)
    per_launch = tl.decode_bytes / 7                 # mean weight bytes per launch
    kern_gbs = per_launch / (k_ms * 1e-3) / 1e9
    pf_steps = max(steps // 8, 2)
    pf_ms = timed(lib, tl.prefill_step, pf_steps, 1)
    pf_conv_ms = timed(lib, lambda: tl.prefill_step(packed=False), pf_steps, 1)
    layer_flop = LAYER_GEMM_FLOP + PF_FLOP_PER_LAYER
    out = {
        "workload": "Q4_K_M weights (Q4_K; Q6_K for Wv and W2), 32 layers, 4.45 GB",
        "decode_projections": {
            "workload": "7 matvecs per layer on Q8_0 inputs (mia_matvec_q8: Wq, Wk, Wv, Wo, W1, "
                        "W2, W3), 32 layers",
            "value": round(N_LAYERS * tl.decode_bytes / (dec_ms * 1e-3) / 1e9, 2), "unit": "GB/s",
            "ms_per_step": round(dec_ms, 4), "weight_bytes_per_layer": tl.decode_bytes,
            "matvec_kernel_us": round(k_ms * 1e3, 3), "matvec_launches": n,
            "roofline": {"bound": "hbm", "achieved": round(kern_gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
                         "traffic": load_traffic("kquant_matvec"),
                         "note": "mean weight bytes per launch over the kernel's mean duration; "
                                 "traffic: FETCH + WRITE bytes per launch, mean over the seven"},
        },
        "prefill_layer": {
            "workload": "mia_prefill_layer_typed_packed x 32, S 512 after 1536 cached: the "
                        "weights in the GEMM operand form made once at set-up (mia_gemm_pack: "
                        "fp16 values of Q4_K, row-scaled hi + lo halves of Q6_K, 18 GB), fp16 "
                        "MFMA GEMMs (hipBLASLt, each shape's algorithm picked by timing on its first "
                        "call, in the warm-up) on the activations' hi + lo halves",
            "value": round(N_LAYERS * layer_flop / (pf_ms * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
            "ms_per_step": round(pf_ms, 3), "flop_per_layer": layer_flop,
            "per_call_conversion_ms_per_step": round(pf_conv_ms, 3),
            "per_call_conversion": "mia_prefill_layer_typed on the GGUF blocks: the same "
                                   "layer converting each matrix on every call",
        },
    }
    del tl
    return out


def cpu_baseline_prefill_layer():
    """The oracle's prefill layer (timing build, OpenMP) on 1 of the 32 layers."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import _oracle as O

    g = np.random.default_rng(15)
    W = {"wq": O.make_q4_0(g, DIM, DIM), "wk": O.make_q4_0(g, KV_DIM, DIM),
         "wv": O.make_q4_0(g, KV_DIM, DIM), "wo": O.make_q4_0(g, DIM, DIM),
         "w1": O.make_q4_0(g, HIDDEN, DIM), "w3": O.make_q4_0(g, HIDDEN, DIM),
         "w2": O.make_q4_0(g, DIM, HIDDEN),
         "rms_att": np.ones(DIM, np.float32), "rms_ffn": np.ones(DIM, np.float32)}
    kc = np.zeros((PF_M, KV_DIM), np.uint16)
    vc = np.zeros((PF_M, KV_DIM), np.uint16)
    kc[:PF_START] = g.standard_normal((PF_START, KV_DIM), np.float32).astype(np.float16).view(np.uint16)
    vc[:PF_START] = g.standard_normal((PF_START, KV_DIM), np.float32).astype(np.float16).view(np.uint16)
    X = g.standard_normal((PF_S, DIM)).astype(np.float32)
    threads = O.num_threads(fast=True)
    lib = O.load(True)
    hd = HD
    kv = O.make_kv(kc, vc, N_KV, hd, PF_M)
    arrs = {k: np.ascontiguousarray(v) for k, v in W.items()}
    lw = O.OraLayerWeights(*[arrs[n].ctypes.data for n in ("wq", "wk", "wv", "wo", "w1", "w2",
                                                              "w3", "rms_att", "rms_ffn")])
    th = theta_inv()
    t0 = time.perf_counter()
    lib.ora_prefill_layer(ctypes.byref(lw), ctypes.byref(kv), X.ctypes.data, 0, PF_START, PF_S,
                          DIM, HIDDEN, N_HEADS, N_KV, 1e-5, th.ctypes.data, threads)
    dt = time.perf_counter() - t0
    return {"value": round((LAYER_GEMM_FLOP + PF_FLOP_PER_LAYER) / dt / 1e12, 4),
            "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": "1 of 32 layers (S 512 after 1536), oracle timing build: dequantised fp32 "
                      "GEMMs and attention, OpenMP over tokens / heads"}


def cpu_baseline_typed(n_layers: int = 2) -> dict:
    """The oracle on the Q4_K_M leg's shapes: the typed matvec on Q8_0 inputs
    (one thread, as the oracle's typed matvec is) over n_layers layers' seven
    matrices, and the typed prefill layer (timing build, OpenMP) on 1 of the
    32 layers."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import _oracle as O

    g = np.random.default_rng(16)
    types = {n: t for n, _, _, t in KM_SIZES}
    Ws = [{n: O.make_typed(g, t, r, c, d_scale=0.07) for n, r, c, t in KM_SIZES}
          for _ in range(n_layers)]
    xq = {DIM: O.quantize_q8_0(g.standard_normal(DIM).astype(np.float32)),
          HIDDEN: O.quantize_q8_0(g.standard_normal(HIDDEN).astype(np.float32))}
    t0 = time.perf_counter()
    for W in Ws:
        for n, r, c, t in KM_SIZES:
            O.typed_matvec_q8(W[n], t, xq[c], r, c)
    dt = time.perf_counter() - t0
    nbytes = n_layers * sum(km_bytes(r, c, t) for _, r, c, t in KM_SIZES)
    dec = {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": f"{n_layers} of 32 layers, the seven matvecs on Q8_0 inputs, oracle "
                     f"(scalar, one thread)"}
    W = dict(Ws[0])
    W["rms_att"] = np.ones(DIM, np.float32)
    W["rms_ffn"] = np.ones(DIM, np.float32)
    kc = np.zeros((PF_M, KV_DIM), np.uint16)
    vc = np.zeros((PF_M, KV_DIM), np.uint16)
    kc[:PF_START] = g.standard_normal((PF_START, KV_DIM), np.float32).astype(np.float16).view(np.uint16)
    vc[:PF_START] = g.standard_normal((PF_START, KV_DIM), np.float32).astype(np.float16).view(np.uint16)
    X = g.standard_normal((PF_S, DIM)).astype(np.float32)
    threads = O.num_threads(fast=True)
    lib = O.load(True)
    kv = O.make_kv(kc, vc, N_KV, HD, PF_M)
    arrs = {k: np.ascontiguousarray(v) for k, v in W.items()}
    lw = O.OraLayerWeightsTyped(*[arrs[n].ctypes.data for n in O.MATS],
                                *[types[n] for n in O.MATS], arrs["rms_att"].ctypes.data,
                                arrs["rms_ffn"].ctypes.data)
    th = theta_inv()
    t0 = time.perf_counter()
    rc = lib.ora_prefill_layer_typed(ctypes.byref(lw), ctypes.byref(kv), X.ctypes.data, 0,
                                     PF_START, PF_S, DIM, HIDDEN, N_HEADS, N_KV, 1e-5,
                                     th.ctypes.data, threads)
    dt = time.perf_counter() - t0
    assert rc == 0
    pf = {"value": round((LAYER_GEMM_FLOP + PF_FLOP_PER_LAYER) / dt / 1e12, 4),
          "unit": "TFLOP/s", "cores": threads, "kind": "port",
          "sample": "1 of 32 layers (S 512 after 1536), oracle timing build: dequantised fp32 "
                    "GEMMs and attention, OpenMP"}
    return {"decode_projections": dec, "prefill_layer": pf}


def gguf_upload(lib, n_layers: int = 8):
    """A GGUF file holding n_layers layers of Mistral-7B attention weights
    (Q4_0, written to a temp dir from the format): time to open (map + parse)
    and to upload the data section to HBM (PCIe-inclusive)."""
    import tempfile

    sys.path.insert(0, os.path.join(REPO, "tests"))
    import _gguf as GW

    g = np.random.default_rng(17)
    tensors = []
    for l in range(n_layers):
        for nm, rows in (("attn_q", DIM), ("attn_k", KV_DIM), ("attn_v", KV_DIM),
                         ("attn_output", DIM)):
            raw = g.integers(0, 256, rows * Q4_ROW_BYTES, dtype=np.uint8).tobytes()
            tensors.append((f"blk.{l}.{nm}.weight", GW.GGML_Q4_0, (DIM, rows), raw))
    meta = [("llama.embedding_length", GW.U32, DIM), ("llama.block_count", GW.U32, n_layers)]
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "attn.gguf")
        GW.write(path, meta, tensors)
        del tensors
        h = ctypes.c_void_p()
        t0 = time.perf_counter()
        check(lib.mia_gguf_open(path.encode(), ctypes.byref(h)), "gguf_open")
        t_open = time.perf_counter() - t0
        dev, nb = ctypes.c_void_p(), ctypes.c_size_t()
        t0 = time.perf_counter()
        check(lib.mia_gguf_upload(h, ctypes.byref(dev), ctypes.byref(nb)), "gguf_upload")
        t_up = time.perf_counter() - t0
        check(lib.mia_free(dev.value), "free")
        lib.mia_gguf_close(h.value)
    return {"workload": f"GGUF file of {n_layers} layers x (Wq, Wk, Wv, Wo) Q4_0 at 4096 width",
            "bytes": nb.value, "open_ms": round(t_open * 1e3, 3),
            "upload_ms": round(t_up * 1e3, 2),
            "upload_gbs": round(nb.value / t_up / 1e9, 2), "unit": "GB/s",
            "path": "mapped file -> hipMemcpy in 64 MiB pieces (host pages, PCIe), wall clock"}


def cpu_other_configs():
    """Oracle timing (same thread count as the headline baseline) on bounded
    samples of configs 1, 2 and 5."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import _oracle as O

    g = np.random.default_rng(13)
    threads = O.num_threads(fast=True)
    res = {}
    # config 1: 1 layer, M 4096, pos 512 (L 513)
    kc = g.standard_normal((1, 4096, KV_DIM), np.float32).astype(np.float16).view(np.uint16)
    vc = g.standard_normal((1, 4096, KV_DIM), np.float32).astype(np.float16).view(np.uint16)
    Q = g.standard_normal((1, N_HEADS * HD), np.float32)
    O.decode_layers(Q, kc, vc, 1, N_HEADS, N_HEADS // N_KV, HD, 4096, 512, threads=threads)
    t0 = time.perf_counter()
    for _ in range(20):
        O.decode_layers(Q, kc, vc, 1, N_HEADS, N_HEADS // N_KV, HD, 4096, 512, threads=threads)
    dt = (time.perf_counter() - t0) / 20
    t0 = time.perf_counter()
    for _ in range(5):
        O.decode_layers(Q, kc, vc, 1, N_HEADS, N_HEADS // N_KV, HD, 4096, 512, threads=1)
    dt1 = (time.perf_counter() - t0) / 5
    res["1"] = {"value": round(4096 * 513 / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
                "kind": "port", "sample": "the whole config (1 layer), mean of 20",
                "single_thread_value": round(4096 * 513 / dt1 / 1e9, 3)}
    # config 2: 4 of 32 layers, M 65536, pos 4096 (L 4097)
    n = 4
    kc = g.standard_normal((n, 65536, KV_DIM), np.float32).astype(np.float16).view(np.uint16)
    vc = g.standard_normal((n, 65536, KV_DIM), np.float32).astype(np.float16).view(np.uint16)
    Q = g.standard_normal((n, N_HEADS * HD), np.float32)
    t0 = time.perf_counter()
    O.decode_layers(Q, kc, vc, n, N_HEADS, N_HEADS // N_KV, HD, 65536, 4096, threads=threads)
    dt = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.decode_layers(Q[:1], kc[:1], vc[:1], 1, N_HEADS, N_HEADS // N_KV, HD, 65536, 4096, threads=1)
    dt1 = time.perf_counter() - t0
    res["2"] = {"value": round(n * 4096 * 4097 / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
                "kind": "port", "sample": f"{n} of 32 layers",
                "single_thread_value": round(4096 * 4097 / dt1 / 1e9, 3),
                "single_thread_sample": "1 layer"}
    # config 5: 1 of 32 layers, 8 queries over the wrapped 65536-slot window
    Q = g.standard_normal((1, 8, N_HEADS * HD), np.float32)
    t0 = time.perf_counter()
    O.attention_batch_layers(Q, kc[:1], vc[:1], 1, N_HEADS, N_KV, HD, 65536, 70000, 8,
                             threads=threads)
    dt = time.perf_counter() - t0
    Q1 = Q[:, :2]
    t0 = time.perf_counter()
    O.attention_batch_layers(Q1, kc[:1], vc[:1], 1, N_HEADS, N_KV, HD, 65536, 70000, 2, threads=1)
    dt1 = (time.perf_counter() - t0) * 4  # 2 of the 8 queries
    res["5"] = {"value": round(4096 * 65536 / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
                "single_thread_value": round(4096 * 65536 / dt1 / 1e9, 3),
                "single_thread_sample": "one thread, 2 of the 8 queries of 1 layer, scaled to 8",
                "kind": "port",
                "sample": "1 of 32 layers: attention of the 8 queries over the wrapped window "
                          "(attention_batch on the same shape; the drafts' ring writes are not "
                          "timed)"}
    return res


def load_traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/), or None.

    Each entry carries the SHA-256 of the kernel source it was measured on;
    once that source has changed the figure no longer describes the kernel
    that runs, and None is reported instead of a stale number."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f).get(name)
        src = os.path.join(REPO, entry["kernel_source"])
        with open(src, "rb") as f:
            if hashlib.sha256(f.read()).hexdigest() != entry["kernel_source_sha256"]:
                log(f"roofline.traffic for {name}: {entry['kernel_source']} changed since its "
                    "counters were measured; reported as null")
                return None
        return int(entry["bytes"])
    except (OSError, ValueError, KeyError, TypeError):
        return None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-prefill", action="store_true")
    ap.add_argument("--skip-decode", action="store_true", help="prefill only (profiling)")
    ap.add_argument("--skip-layer", action="store_true",
                    help="skip the whole-prefill-layer line (profiling)")
    ap.add_argument("--skip-projections", action="store_true",
                    help="skip the W4A8 projection line (profiling)")
    ap.add_argument("--skip-configs", action="store_true",
                    help="skip the side configs 1, 2 and 5 (profiling)")
    ap.add_argument("--skip-peaks", action="store_true", help="skip the measured-peaks leg")
    ap.add_argument("--skip-decode-layer", action="store_true",
                    help="skip the whole-decode-layer leg")
    ap.add_argument("--skip-typed", action="store_true",
                    help="skip the Q4_K_M weight leg (projections and prefill layer)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 5 device-to-device copies of 512 MiB (a copy kernel of known "
                         "size, to scale HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU only: the attention path has no multi-GPU mode "
                          "(it would shard by kv head, each GPU running these kernels on "
                          "its heads' slice of the ring)",
                          "n_gpus": args.gpus}))
        return 2

    lib = mia.init(0)
    if args.copy_calibration:
        nb = 512 << 20
        src, dst = DeviceBuffer(nb), DeviceBuffer(nb)
        src.zero()
        for _ in range(5):
            check(lib.mia_memcpy_d2d(dst.ptr, src.ptr, nb))
        check(lib.mia_device_sync())
        del src, dst
    dec_ms = kern_ms = float("nan")
    dropin = projections = peaks = decode_layer = None
    if not args.skip_decode:
        log("decode: allocating 32 x 32768-slot rings (4 GiB)")
        dec = Decode(lib)
        dec_ms = timed(lib, dec.step, args.steps, args.warmup)
        kern_ms = kernel_avg_ms(lib, dec.step, args.steps, 0)
        if not args.skip_peaks:
            log("peaks: HBM read stream, decode load pattern, fp16 MFMA loop")
            peaks = measure_peaks(lib, dec)
            log(f"peaks: stream {peaks['hbm_read_stream']['value']} GB/s, decode pattern "
                f"{peaks['hbm_read_decode_pattern']['value']} GB/s, fp16 MFMA "
                f"{peaks['mfma_f16']['value']} TFLOP/s, empty kernel "
                f"{peaks['empty_kernel']['decode_grid_us']} / "
                f"{peaks['empty_kernel']['flash_grid_us']} us")
        dd = DropinDecode(lib, dec)
        di_ms = wall_ms(dd.step, args.steps, args.warmup)
        dropin = {"value": round(N_LAYERS * DECODE_BYTES_PER_LAYER / (di_ms * 1e-3) / 1e9, 2),
                  "unit": "GB/s", "ms_per_step": round(di_ms, 4),
                  "path": "mia_dropin_decode_step per layer, host q/k/v/out (PCIe), "
                          "synchronous, wall clock"}
        log(f"decode via drop-in (host buffers): {di_ms:.3f} ms/step")
        del dd
        if not args.skip_projections:
            log("projections: 32 layers x (quantize, QKV 6144 x 4096, quantize, Wo 4096 x 4096)")
            pj = Projections(lib)
            pj_ms = timed(lib, pj.step, args.steps, args.warmup)
            pj2_ms = timed(lib, pj.step_two_launch, args.steps, args.warmup)
            mv_n, mv_ms = kernel_stats(lib, pj.step, args.steps, 2)
            blk_ms = timed(lib, lambda: pj.block_step(dec), args.steps, args.warmup)
            mv_bytes = (QKV_BYTES + WO_BYTES) / 2           # per launch, launches alternate
            mv_gbs = mv_bytes / (mv_ms * 1e-3) / 1e9
            log(f"projections: {pj_ms:.3f} ms/step ({pj2_ms:.3f} with separate quantize "
                f"launches), matvec kernel {mv_ms * 1e3:.2f} us avg "
                f"({mv_gbs:.0f} GB/s); attention block {blk_ms:.3f} ms/step")
            projections = {
                "workload": "W4A8 projections of the decode step, 32 layers: quantize + fused "
                            "QKV (6144 x 4096 Q4_0) + quantize + Wo (4096 x 4096 Q4_0), own "
                            "weights per layer (755 MB); quantize folded into each matvec "
                            "launch (mia_q4_0_matvec_qkv_f32, mia_q4_0_matvec_f32)",
                "value": round(N_LAYERS * (QKV_BYTES + WO_BYTES) / (pj_ms * 1e-3) / 1e9, 2),
                "unit": "GB/s", "ms_per_step": round(pj_ms, 4),
                "two_launch_ms_per_step": round(pj2_ms, 4),
                "bytes_per_layer": QKV_BYTES + WO_BYTES,
                "matvec_kernel_us": round(mv_ms * 1e3, 3), "matvec_launches": mv_n,
                "roofline": {"bound": "hbm", "achieved": round(mv_gbs, 2), "peak": HBM_PEAK_GBS,
                             "unit": "GB/s", "frac": round(mv_gbs / HBM_PEAK_GBS, 4),
                             "traffic": load_traffic("q4_matvec")},
                "attention_block_ms_per_step": round(blk_ms, 4),
                "attention_block": "per layer: mia_q4_0_matvec_qkv_f32, mia_decode_step at "
                                   "32K context (the headline's rings), mia_q4_0_matvec_f32 (Wo)",
            }
            del pj
        if not args.skip_decode_layer:
            log("decode layer: 32 layers x the whole layer at 32K context, Q4_0 and Q4_K_M")
            decode_layer = decode_layer_leg(lib, dec, args.steps, args.warmup)
            log(f"decode layer: Q4_0 {decode_layer['q4_0']['ms_per_token']:.3f} ms/token "
                f"({decode_layer['q4_0']['tokens_per_s']:.1f} tokens/s, "
                f"{decode_layer['q4_0']['value']:.0f} GB/s); Q4_K_M "
                f"{decode_layer['q4_k_m']['ms_per_token']:.3f} ms/token "
                f"({decode_layer['q4_k_m']['tokens_per_s']:.1f} tokens/s)")
        del dec
    achieved = DECODE_BYTES_PER_LAYER / (kern_ms * 1e-3) / 1e9
    value = N_LAYERS * DECODE_BYTES_PER_LAYER / (dec_ms * 1e-3) / 1e9
    log(f"decode: {dec_ms:.3f} ms/step, {value:.1f} GB/s; decode kernel {kern_ms * 1e3:.2f} us "
        f"({achieved:.1f} GB/s)")

    prefill = None
    if not args.skip_prefill:
        log("prefill: 32 layers x (1536 cached + 512 new)")
        pf = Prefill(lib)
        pf_steps = max(args.steps // 2, 3)
        pf_ms = timed(lib, pf.step, pf_steps, 2)
        fl_ms = kernel_avg_ms(lib, pf.step, pf_steps, 1)
        fl_tfs = PF_FLOP_PER_LAYER / (fl_ms * 1e-3) / 1e12
        log(f"prefill: {pf_ms:.3f} ms/step, flash kernel {fl_ms * 1e3:.1f} us, {fl_tfs:.1f} TFLOP/s")
        prefill = {
            "value": round(N_LAYERS * PF_FLOP_PER_LAYER / (pf_ms * 1e-3) / 1e12, 3),
            "unit": "TFLOP/s",
            "ms_per_step": round(pf_ms, 4),
            "workload": "causal prefill chunk: 32 layers, 512 new tokens after 1536 cached "
                        "positions, 32 q / 8 kv heads, hd 128, fp32 Q (fp16 hi + lo parts "
                        "on MFMA), fp16 K/V, fp32 accumulate",
            "flop_per_layer": PF_FLOP_PER_LAYER,
            "kernel_us": round(fl_ms * 1e3, 2),
            "roofline": {"bound": "mfma", "achieved": round(fl_tfs, 3),
                         "peak": MFMA_F16_PEAK_TFS, "unit": "TFLOP/s",
                         "frac": round(fl_tfs / MFMA_F16_PEAK_TFS, 4),
                         "traffic": load_traffic("flash_prefill")},
        }
        if peaks is not None:
            mp = peaks["mfma_f16"]["value"]
            prefill["roofline"]["measured_peak"] = mp
            prefill["roofline"]["frac_of_measured"] = round(fl_tfs / mp, 4)
        del pf

    gguf = None
    if not args.skip_projections:
        log("gguf: writing and uploading an 8-layer attention-weight file")
        gguf = gguf_upload(lib)
        log(f"gguf: open {gguf['open_ms']:.2f} ms, upload {gguf['upload_ms']:.1f} ms "
            f"({gguf['upload_gbs']:.1f} GB/s)")

    layer = None
    if not args.skip_prefill and not args.skip_layer:
        log("prefill layer: 32 layers x (RMSNorm, QKV, attention, Wo, RMSNorm, SwiGLU FFN), S 512")
        pl = PrefillLayers(lib)
        pl_steps = max(args.steps // 4, 2)
        pl_ms = timed(lib, pl.step, pl_steps, 1)
        g_n, g_ms = kernel_stats(lib, pl.step, pl_steps, 3)
        gemm_tfs = (LAYER_GEMM_FLOP / 5) / (g_ms * 1e-3) / 1e12
        layer_flop = LAYER_GEMM_FLOP + PF_FLOP_PER_LAYER
        log(f"prefill layer: {pl_ms:.2f} ms/step ({N_LAYERS * layer_flop / (pl_ms * 1e-3) / 1e12:.1f} "
            f"TFLOP/s), GEMM kernel {g_ms * 1e3:.1f} us avg ({gemm_tfs:.1f} TFLOP/s)")
        layer = {
            "workload": "prefill layer x 32 (mia_prefill_layer): RMSNorm, fused QKV GEMM, RoPE + "
                        "ring write + flash attention, Wo GEMM + residual, RMSNorm, gate / up "
                        "GEMMs + SwiGLU, down GEMM + residual; S 512 after 1536 cached, Q4_0 "
                        "weights per layer (3.9 GB)",
            "value": round(N_LAYERS * layer_flop / (pl_ms * 1e-3) / 1e12, 3),
            "unit": "TFLOP/s", "ms_per_step": round(pl_ms, 3),
            "flop_per_layer": layer_flop, "gemm_flop_per_layer": LAYER_GEMM_FLOP,
            "gemm_kernel_us": round(g_ms * 1e3, 2), "gemm_launches": g_n,
            "roofline": {"bound": "mfma", "achieved": round(gemm_tfs, 3),
                         "peak": MFMA_F16_PEAK_TFS, "unit": "TFLOP/s",
                         "frac": round(gemm_tfs / MFMA_F16_PEAK_TFS, 4),
                         "traffic": load_traffic("q4_gemm_prefill"),
                         "note": "algorithmic FLOPs of the fp32 GEMM; the kernel issues twice "
                                 "as many fp16 MFMA FLOPs (activations split hi + lo); the "
                                 "split-K sum kernel of Wo and W2 is in ms_per_step, not in "
                                 "the GEMM kernel average"},
        }
        del pl

    typed = None
    if not args.skip_typed:
        log("typed weights: Q4_K_M decode projections and prefill layer, 32 layers")
        typed = typed_leg(lib, args.steps, args.warmup)
        log(f"typed weights: decode projections {typed['decode_projections']['ms_per_step']:.3f} "
            f"ms/step ({typed['decode_projections']['value']:.0f} GB/s, kernel "
            f"{typed['decode_projections']['roofline']['achieved']:.0f} GB/s); prefill layer "
            f"{typed['prefill_layer']['ms_per_step']:.2f} ms/step "
            f"({typed['prefill_layer']['value']:.1f} TFLOP/s; converting per call "
            f"{typed['prefill_layer']['per_call_conversion_ms_per_step']:.2f} ms)")

    configs = None
    if not args.skip_configs and not args.skip_decode:
        log("other configs: 1 (L 513), 2 (32 x L 4097), 5 (32 x verify S 8 on a wrapped ring)")
        oc = OtherConfigs(lib)
        c1 = timed(lib, oc.c1, 200, 20)
        c2 = timed(lib, oc.c2, args.steps, args.warmup)
        c5 = timed(lib, oc.c5, args.steps, args.warmup)
        c5s = timed(lib, oc.c5_staged, args.steps, args.warmup)
        c5q = timed(lib, oc.c5_sequential, max(args.steps // 4, 2), 1)
        # the main kernel of each config (kind 0 decode, 1 flash) from the
        # dispatch-stamped events, against its algorithmic window bytes
        k1 = kernel_avg_ms(lib, oc.c1, 50, 0)
        k2 = kernel_avg_ms(lib, oc.c2, 2, 0)
        k5 = kernel_avg_ms(lib, oc.c5, 2, 1)
        del oc

        def kroof(nbytes: int, ms: float) -> dict:
            gbs = nbytes / (ms * 1e-3) / 1e9
            return {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}
        configs = {
            "1": {"workload": "1 layer decode step, 512 filled positions + new token (L 513), M 4096",
                  "value": round(4096 * 513 / (c1 * 1e-3) / 1e9, 2), "unit": "GB/s",
                  "ms_per_step": round(c1, 5), "kernel_us": round(k1 * 1e3, 2),
                  "roofline": kroof(4096 * 513, k1)},
            "2": {"workload": "32-layer decode step, 4096 filled + new token (L 4097), M 65536",
                  "value": round(N_LAYERS * 4096 * 4097 / (c2 * 1e-3) / 1e9, 2), "unit": "GB/s",
                  "ms_per_step": round(c2, 4), "kernel_us": round(k2 * 1e3, 2),
                  "roofline": kroof(4096 * 4097, k2)},
            "3": {"workload": "the headline (value)"},
            "4": {"workload": "the prefill object"},
            "5": {"workload": "32-layer speculative verify, 8 drafts at positions 70000..70007 "
                              "on a wrapped 65536-slot ring (staged drafts, committed after "
                              "attention)",
                  "value": round(N_LAYERS * 4096 * 65536 / (c5 * 1e-3) / 1e9, 2), "unit": "GB/s",
                  "ms_per_step": round(c5, 4),
                  "kernel_us": round(k5 * 1e3, 2),
                  "kernel": "flash_kernel (32-row tiles, key range split over workgroups); "
                            "the split merge and the commit of the drafts are in ms_per_step",
                  "roofline": kroof(4096 * 65536, k5),
                  "accept_only_ms_per_step": round(c5s, 4),
                  "sequential_ms_per_step": round(c5q, 4),
                  "sequential_value": round(N_LAYERS * 8 * 4096 * 65536 / (c5q * 1e-3) / 1e9, 2),
                  "sequential": "the reference's verify without a batch path: 8 x "
                                "mia_decode_step per layer (fused RoPE, ring write, attention) "
                                "at positions 70000..70007; value counts the window read once "
                                "per draft",
                  "accept_only": "mia_attention_step_staged per layer (ring untouched), then one "
                                 "mia_commit_staged of 5 accepted drafts for all 32 layers"},
        }
        log(f"config 1: {c1 * 1e3:.1f} us; config 2: {c2:.3f} ms; config 5: {c5:.3f} ms "
            f"({c5s:.3f} ms staged + accept-only commit); kernels {k1 * 1e3:.2f} / "
            f"{k2 * 1e3:.2f} / {k5 * 1e3:.2f} us")

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline: decode sample")
        cpu = cpu_baseline_decode()
        if prefill is not None:
            log("cpu baseline: prefill sample")
            prefill["cpu_baseline"] = cpu_baseline_prefill()
        if layer is not None:
            log("cpu baseline: prefill layer sample")
            layer["cpu_baseline"] = cpu_baseline_prefill_layer()
        if projections is not None:
            log("cpu baseline: projections sample")
            projections["cpu_baseline"] = cpu_baseline_projections()
        if decode_layer is not None:
            log("cpu baseline: decode layer sample")
            decode_layer["cpu_baseline"] = cpu_baseline_decode_layer()
        if typed is not None:
            log("cpu baseline: Q4_K_M projections and prefill layer samples")
            for k, v in cpu_baseline_typed().items():
                typed[k]["cpu_baseline"] = v
        if configs is not None:
            log("cpu baseline: configs 1, 2, 5")
            for k, v in cpu_other_configs().items():
                configs[k]["cpu_baseline"] = v

    roof = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": load_traffic("decode_32k")}
    if peaks is not None:
        mp = peaks["hbm_read_decode_pattern"]["value"]
        roof["measured_peak"] = mp
        roof["frac_of_measured"] = round(achieved / mp, 4)
        roof["measured_peak_is"] = "hbm_read_decode_pattern (peaks)"
    line = {
        "metric": "decode attn HBM GB/s (% peak) @32K ctx; prefill attn TFLOPS (% MFMA peak)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) fp16 rings generated on the GPU)",
        "config": {
            "workload": "decode attention step x 32 layers: 32768-slot fp16 ring full, new "
                        "token at position 32768, every 1024th key x4, 32 q / 8 kv heads, hd 128, "
                        "RoPE theta 1e6, fused RoPE + ring write + split-K flash-decode",
            "layers": N_LAYERS, "ctx": DECODE_L, "max_seq": DECODE_M,
            "bytes_per_layer": DECODE_BYTES_PER_LAYER,
            "decode_kernel_us": round(kern_ms * 1e3, 2),
            "arithmetic": "fp16 MFMA operands (q split hi+lo), fp32 accumulate and softmax",
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "peaks": peaks,
        "dropin": dropin,
        "prefill": prefill,
        "configs": configs,
        "projections": projections,
        "gguf": gguf,
        "prefill_layer": layer,
        "typed_weights": typed,
        "decode_layer": decode_layer,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
