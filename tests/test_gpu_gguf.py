"""GPU tier of the GGUF loader: the data section uploaded by mia_gguf_upload is
byte-identical to the file, and the Q4_0 projections read straight from the
uploaded tensors (device base + tensor offset) match the oracle run on the
written weights."""

import ctypes

import numpy as np
import pytest

import _gguf as W
import _gpu as G
import _oracle as O
import anetransformers_amd as mia
from anetransformers_amd import DeviceBuffer as DB
from anetransformers_amd import check

pytestmark = pytest.mark.gpu


def test_upload_and_projections_from_the_file(tmp_path):
    G.say("gguf: one Mistral-width layer, upload + QKV/Wo from the uploaded tensors")
    lib = G.lib()
    g = np.random.default_rng(3)
    dim, kv_dim = 4096, 1024
    meta, tensors = W.mistral_like(g, dim=dim, n_layers=1, n_heads=32, n_kv=8, hidden=14336,
                                   vocab=16, q4_maker=O.make_q4_0)
    path = tmp_path / "layer.gguf"
    offs = W.write(path, meta, tensors)
    h = ctypes.c_void_p()
    check(lib.mia_gguf_open(str(path).encode(), ctypes.byref(h)), "open")
    try:
        dev, nbytes = ctypes.c_void_p(), ctypes.c_size_t()
        check(lib.mia_gguf_upload(h, ctypes.byref(dev), ctypes.byref(nbytes)), "upload")
        blob = path.read_bytes()
        assert nbytes.value == len(blob) - offs["__data__"]
        back = np.empty(nbytes.value, np.uint8)
        check(lib.mia_memcpy_d2h(back.ctypes.data, dev.value, nbytes.value), "d2h")
        assert back.tobytes() == blob[offs["__data__"]:]

        def dptr(name):
            t = mia.GGUFTensor()
            check(lib.mia_gguf_find(h, name.encode(), ctypes.byref(t)), name)
            return dev.value + t.offset

        W4 = {name: np.frombuffer(raw, np.uint8).reshape(shape[1], -1)
              for name, ttype, shape, raw in tensors if ttype == W.GGML_Q4_0}
        x = g.standard_normal(dim).astype(np.float32)
        dx = DB.from_array(x)
        dyq, dyk, dyv, dyo = DB(dim * 4), DB(kv_dim * 4), DB(kv_dim * 4), DB(dim * 4)
        check(lib.mia_q4_0_matvec_qkv_f32(dptr("blk.0.attn_q.weight"), dptr("blk.0.attn_k.weight"),
                                          dptr("blk.0.attn_v.weight"), dx.ptr, dyq.ptr, dyk.ptr,
                                          dyv.ptr, dim, kv_dim, dim, None), "qkv")
        check(lib.mia_q4_0_matvec_f32(dptr("blk.0.attn_output.weight"), dx.ptr, dyo.ptr, dim, dim,
                                      None), "wo")
        check(lib.mia_stream_sync(None), "sync")
        xq = O.quantize_q8_0(x)
        want = O.q4_0_q8_0_matvec_qkv(W4["blk.0.attn_q.weight"], W4["blk.0.attn_k.weight"],
                                      W4["blk.0.attn_v.weight"], xq, dim, kv_dim, dim)
        want_o = O.q4_0_q8_0_matvec(W4["blk.0.attn_output.weight"], xq, dim, dim)
        for d, ref, n in zip((dyq, dyk, dyv, dyo), want + (want_o,), (dim, kv_dim, kv_dim, dim)):
            y = d.download(n, np.float32)
            # reassociation bound of tests/test_gpu_q4.py, in its simple form
            assert np.all(np.abs(y - ref) <= 2e-3 + 1e-2 * np.abs(ref))
            assert np.abs(y - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
        check(lib.mia_free(dev.value), "free")
    finally:
        lib.mia_gguf_close(h.value)
