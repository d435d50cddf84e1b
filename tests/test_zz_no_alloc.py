"""GPU: mia_decode_step_noalloc (partials in the library's fixed per-device
area, no allocation) against mia_decode_step on the same inputs, through the
C ABI: two calls in a row, the second with a smaller input, then a shape with
16 kv heads.  Outputs must match to the parity bar (the two entry points share
their kernels and, at these shapes, their chunk plan, so they are expected to
be bit-identical), and the rings bit-exactly; the oracle checks the decode
step itself.  A call is also captured into a HIP graph in global capture
mode, where allocating or synchronising the device is refused: the capture
succeeds only if the entry point does neither."""

import ctypes

import numpy as np
import pytest

import _data as D
import _gpu as G
import _oracle as O
from anetransformers_amd import DeviceBuffer as DB
from anetransformers_amd import check

pytestmark = pytest.mark.gpu

TH = O.theta_inv(D.THETA, D.HD)


def _both(lib, kc, vc, q, k, v, n_heads, n_kv, M, pos):
    outs, rings = [], []
    dth = DB.from_array(TH)
    dq, dk, dv = DB.from_array(q), DB.from_array(k), DB.from_array(v)
    for fn in (lib.mia_decode_step_noalloc, lib.mia_decode_step):
        dkc, dvc = DB.from_array(kc), DB.from_array(vc)
        dout = DB(n_heads * 128 * 4)
        check(fn(dq.ptr, dk.ptr, dv.ptr, dth.ptr, dkc.ptr, dvc.ptr, dout.ptr, n_heads, n_kv, 128, M,
                 pos, None), fn.__name__)
        check(lib.mia_stream_sync(None), "sync")
        outs.append(dout.download(n_heads * 128, np.float32))
        rings.append((dkc.download(kc.shape, np.uint16), dvc.download(vc.shape, np.uint16)))
    return outs, rings


def test_noalloc_matches_decode_step_two_calls():
    lib = G.lib()
    g = D.rng(900)
    for M, pos in ((32768, 32768), (4096, 700)):      # second call: smaller input
        G.say(f"decode_step_noalloc vs decode_step M={M} pos={pos}")
        kc, vc = D.ring(g, M, filled=min(pos, M), spike_every=1024)
        q, k, v = D.normal(g, 4096), D.normal(g, 1024), D.normal(g, 1024)
        (out_n, out_r), ((kn, vn), (kr, vr)) = _both(lib, kc, vc, q, k, v, 32, 8, M, pos)
        D.check_close(out_n, out_r, what=f"noalloc vs decode_step M={M}")
        assert np.array_equal(out_n, out_r)
        assert np.array_equal(kn, kr) and np.array_equal(vn, vr)
        kc_o, vc_o = kc.copy(), vc.copy()
        ref = O.decode_step(kc_o, vc_o, q, k, v, pos, TH, 32, 8, 128, M)
        D.check_close(out_n, ref, what=f"noalloc vs oracle M={M}")
        D.check_ring(kn, kc_o, vn, vc_o, [pos % M], k, [pos], TH, "noalloc ring")


def test_noalloc_sixteen_kv_heads():
    lib = G.lib()
    g = D.rng(901)
    M, pos, n_heads, n_kv = 8192, 9000, 64, 16
    G.say(f"decode_step_noalloc n_kv={n_kv} M={M} pos={pos}")
    kc, vc = D.ring(g, M, kv_dim=n_kv * 128)
    q, k, v = D.normal(g, n_heads * 128), D.normal(g, n_kv * 128), D.normal(g, n_kv * 128)
    (out_n, out_r), ((kn, vn), (kr, vr)) = _both(lib, kc, vc, q, k, v, n_heads, n_kv, M, pos)
    D.check_close(out_n, out_r, what="noalloc 16 kv heads")
    assert np.array_equal(kn, kr) and np.array_equal(vn, vr)
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = O.decode_step(kc_o, vc_o, q, k, v, pos, TH, n_heads, n_kv, 128, M)
    D.check_close(out_n, ref, what="noalloc 16 kv heads vs oracle")


def _hip():
    h = ctypes.CDLL("libamdhip64.so")
    v = ctypes.c_void_p
    for name, args in (("hipStreamBeginCapture", [v, ctypes.c_int]),
                       ("hipStreamEndCapture", [v, ctypes.POINTER(v)]),
                       ("hipGraphInstantiate", [ctypes.POINTER(v), v, v, v, ctypes.c_size_t]),
                       ("hipGraphLaunch", [v, v]),
                       ("hipGraphExecDestroy", [v]),
                       ("hipGraphDestroy", [v])):
        getattr(h, name).argtypes = args
        getattr(h, name).restype = ctypes.c_int
    return h


def test_noalloc_captured_in_graph():
    # Global capture mode: hipMalloc / hipFree / hipDeviceSynchronize from
    # any thread during the capture make it fail.  A 32K window takes 32
    # chunks, so the split-K partials are in use.  The graph is replayed
    # three times with eager work and synchronisations in between, each
    # replay checked against the eager mia_decode_step.
    lib = G.lib()
    hip = _hip()
    g = D.rng(902)
    M, pos = 32768, 40000
    G.say(f"decode_step_noalloc captured in a HIP graph M={M} pos={pos}")
    kc, vc = D.ring(g, M, spike_every=1024)
    q, k, v = D.normal(g, 4096), D.normal(g, 1024), D.normal(g, 1024)
    (_, out_r), _ = _both(lib, kc, vc, q, k, v, 32, 8, M, pos)
    dth = DB.from_array(TH)
    dq, dk, dv = DB.from_array(q), DB.from_array(k), DB.from_array(v)
    dkc, dvc = DB.from_array(kc), DB.from_array(vc)
    dout = DB(4096 * 4)
    stream = ctypes.c_void_p()
    check(lib.mia_stream_create(ctypes.byref(stream)), "stream")
    graph, gexec = ctypes.c_void_p(), ctypes.c_void_p()
    try:
        assert hip.hipStreamBeginCapture(stream, 0) == 0  # hipStreamCaptureModeGlobal
        rc = lib.mia_decode_step_noalloc(dq.ptr, dk.ptr, dv.ptr, dth.ptr, dkc.ptr, dvc.ptr,
                                         dout.ptr, 32, 8, 128, M, pos, stream)
        end = hip.hipStreamEndCapture(stream, ctypes.byref(graph))
        assert rc == 0, lib.mia_last_error().decode()
        assert end == 0, f"capture ended with hipError {end}"
        assert hip.hipGraphInstantiate(ctypes.byref(gexec), graph, None, None, 0) == 0
        for rep in range(3):
            check(lib.mia_memset(dout.ptr, 0, 4096 * 4), "clear")
            check(lib.mia_device_sync(), "sync")
            assert hip.hipGraphLaunch(gexec, stream) == 0
            check(lib.mia_stream_sync(stream), "sync")
            got = dout.download(4096, np.float32)
            assert np.array_equal(got, out_r), f"replay {rep}"
    finally:
        if gexec.value:
            hip.hipGraphExecDestroy(gexec)
        if graph.value:
            hip.hipGraphDestroy(graph)
        lib.mia_stream_destroy(stream)
