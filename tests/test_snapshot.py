"""KV-ring snapshots (mia_kv_snapshot_*, mia_dropin_kv_save / kv_load): the
header is checked field by field against the documented layout with Python's
struct, without a device; the round trips (host buffer and file) run on the
GPU and must give back the rings bit for bit with their cursors."""

import ctypes
import struct

import numpy as np
import pytest

import anetransformers_amd as mia

HDR = struct.Struct("<8sII7iIQQ")


def _header(n_layers=2, n_kv=8, hd=128, M=64, pos=70, length=64, magic=b"MIAKVRG1", hb=64,
            eb=2, kv_dim=None, payload=None):
    kv_dim = n_kv * hd if kv_dim is None else kv_dim
    payload = n_layers * M * n_kv * hd * 2 if payload is None else payload
    return HDR.pack(magic, hb, eb, n_layers, n_kv, hd, M, kv_dim, pos, length, 0, payload, 0)


def _info(buf):
    lib = mia.load()
    out = [ctypes.c_int(-7) for _ in range(6)]
    rc = lib.mia_kv_snapshot_info(buf, len(buf), *[ctypes.byref(o) for o in out])
    return rc, [o.value for o in out]


def test_snapshot_bytes_and_header_layout():
    lib = mia.load()
    assert HDR.size == 64
    assert lib.mia_kv_snapshot_bytes(32, 8, 128, 32768) == 64 + 2 * 32 * 32768 * 1024 * 2
    assert lib.mia_kv_snapshot_bytes(0, 8, 128, 64) == 0
    assert lib.mia_kv_snapshot_bytes(2, 8, 128, -1) == 0
    rc, f = _info(_header())
    assert rc == mia.MIA_OK and f == [2, 8, 128, 64, 70, 64]


@pytest.mark.parametrize("bad", [
    dict(magic=b"MIAKVRG2"), dict(hb=128), dict(eb=4), dict(kv_dim=1000), dict(payload=12),
    dict(pos=-1), dict(length=65),
])
def test_snapshot_header_rejected(bad):
    rc, _ = _info(_header(**bad))
    assert rc == mia.MIA_ERR_INVALID


def test_snapshot_argument_errors_without_device_work():
    lib = mia.load()
    buf = np.zeros(64, np.uint8)
    p = buf.ctypes.data
    assert lib.mia_kv_snapshot_info(p, 63, None, None, None, None, None, None) == \
        mia.MIA_ERR_INVALID                                                   # short header
    assert lib.mia_kv_snapshot_save(p, 64, p, p, 1, 8, 128, 4, 0, 0) == mia.MIA_ERR_INVALID
    assert b"too small" in lib.mia_last_error()
    assert lib.mia_kv_snapshot_save(p, 1 << 30, p, p, 1, 8, 128, 4, 0, 5) == mia.MIA_ERR_INVALID
    assert lib.mia_kv_snapshot_save(None, 1 << 30, p, p, 1, 8, 128, 4, 0, 0) == \
        mia.MIA_ERR_INVALID
    h = np.frombuffer(_header(n_layers=1, M=4, pos=3, length=3), np.uint8).copy()
    assert lib.mia_kv_snapshot_load(h.ctypes.data, 64, p, p, 1, 8, 128, 4, None, None) == \
        mia.MIA_ERR_INVALID                                                   # truncated
    assert b"truncated" in lib.mia_last_error()
    assert lib.mia_kv_snapshot_load(h.ctypes.data, 1 << 20, p, p, 2, 8, 128, 4, None, None) == \
        mia.MIA_ERR_INVALID                                                   # other shape
    kv = mia.KVCache()
    assert lib.mia_dropin_kv_save(ctypes.byref(kv), b"/nonexistent/x") == mia.MIA_ERR_INVALID
    assert lib.mia_dropin_kv_load(ctypes.byref(kv), b"/nonexistent/x") == mia.MIA_ERR_INVALID


def _ring_pair(lib, g, L, M, kvd):
    n = L * M * kvd
    k = g.integers(0, 1 << 16, n, dtype=np.uint16)
    v = g.integers(0, 1 << 16, n, dtype=np.uint16)
    return k, v


@pytest.mark.gpu
def test_snapshot_round_trip_host_buffer():
    from anetransformers_amd import DeviceBuffer as DB
    from anetransformers_amd import check
    lib = mia.init(0)
    g = np.random.default_rng(3)
    L, n_kv, hd, M = 3, 8, 128, 96
    k, v = _ring_pair(lib, g, L, M, n_kv * hd)
    dk, dv = DB.from_array(k), DB.from_array(v)
    nbytes = lib.mia_kv_snapshot_bytes(L, n_kv, hd, M)
    snap = np.empty(nbytes, np.uint8)
    check(lib.mia_kv_snapshot_save(snap.ctypes.data, nbytes, dk.ptr, dv.ptr, L, n_kv, hd, M,
                                   1000, 96), "save")
    f = HDR.unpack(snap[:64].tobytes())
    assert f[0] == b"MIAKVRG1" and f[3:10] == (L, n_kv, hd, M, n_kv * hd, 1000, 96)
    assert f[11] == k.nbytes
    assert np.array_equal(snap[64:64 + k.nbytes].view(np.uint16), k)
    assert np.array_equal(snap[64 + k.nbytes:].view(np.uint16), v)
    ek, ev = DB(k.nbytes), DB(v.nbytes)
    ek.zero()
    ev.zero()
    pos, length = ctypes.c_int(), ctypes.c_int()
    check(lib.mia_kv_snapshot_load(snap.ctypes.data, nbytes, ek.ptr, ev.ptr, L, n_kv, hd, M,
                                   ctypes.byref(pos), ctypes.byref(length)), "load")
    assert (pos.value, length.value) == (1000, 96)
    assert np.array_equal(ek.download(k.shape, np.uint16), k)
    assert np.array_equal(ev.download(v.shape, np.uint16), v)


@pytest.mark.gpu
def test_snapshot_round_trip_file(tmp_path):
    lib = mia.init(0)
    g = np.random.default_rng(4)
    L, n_kv, hd, M = 2, 8, 128, 40
    kv = mia.KVCache()
    lib.mia_dropin_kv_alloc(ctypes.byref(kv), L, n_kv, hd, M)
    assert lib.mia_dropin_status() == 0
    k, v = _ring_pair(lib, g, L, M, n_kv * hd)
    mia.check(lib.mia_memcpy_h2d(kv.k_cache, k.ctypes.data, k.nbytes))
    mia.check(lib.mia_memcpy_h2d(kv.v_cache, v.ctypes.data, v.nbytes))
    kv.pos, kv.len = 57, 40
    path = str(tmp_path / "ring.kv").encode()
    mia.check(lib.mia_dropin_kv_save(ctypes.byref(kv), path), "kv_save")
    data = open(path, "rb").read()
    assert len(data) == lib.mia_kv_snapshot_bytes(L, n_kv, hd, M)
    other = mia.KVCache()
    lib.mia_dropin_kv_alloc(ctypes.byref(other), L, n_kv, hd, M)
    mia.check(lib.mia_dropin_kv_load(ctypes.byref(other), path), "kv_load")
    assert (other.pos, other.len) == (57, 40)
    back_k, back_v = np.empty_like(k), np.empty_like(v)
    mia.check(lib.mia_memcpy_d2h(back_k.ctypes.data, other.k_cache, k.nbytes))
    mia.check(lib.mia_memcpy_d2h(back_v.ctypes.data, other.v_cache, v.nbytes))
    assert np.array_equal(back_k, k) and np.array_equal(back_v, v)
    # a truncated file and a ring of another shape are refused, the cache untouched
    zero = np.zeros(k.nbytes, np.uint8)
    mia.check(lib.mia_memcpy_h2d(other.k_cache, zero.ctypes.data, k.nbytes))
    open(path, "wb").write(data[:-10])
    assert lib.mia_dropin_kv_load(ctypes.byref(other), path) == mia.MIA_ERR_INVALID
    mia.check(lib.mia_memcpy_d2h(back_k.ctypes.data, other.k_cache, k.nbytes))
    assert not back_k.any()
    open(path, "wb").write(data)
    small = mia.KVCache()
    lib.mia_dropin_kv_alloc(ctypes.byref(small), L, n_kv, hd, M - 8)
    assert lib.mia_dropin_kv_load(ctypes.byref(small), path) == mia.MIA_ERR_INVALID
    for c in (kv, other, small):
        lib.mia_dropin_kv_free(ctypes.byref(c))
