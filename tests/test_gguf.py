"""CPU tier: libmiattn's GGUF loader (include/mia_gguf.h) on files written from
the format (tests/_gguf.py), checked against what was written and against the
reference's own parser (mistral/gguf_loader.h, built into oracle/_ref where
the reference tree is present), including the places where the two differ
on purpose (alignment key, K-quant sizes, bounds checks)."""

import ctypes
import os

import numpy as np
import pytest

import _gguf as W
import _oracle as O
import anetransformers_amd as mia

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SO = os.path.join(REPO, "oracle", "_ref", "libref_gguf.so")


class Loaded:
    def __init__(self, path):
        self.lib = mia.load()
        h = ctypes.c_void_p()
        self.rc = self.lib.mia_gguf_open(str(path).encode(), ctypes.byref(h))
        self.h = h.value

    def __enter__(self):
        mia.check(self.rc, "mia_gguf_open")
        return self

    def __exit__(self, *a):
        self.lib.mia_gguf_close(self.h)

    def config(self):
        c = mia.MistralConfig()
        mia.check(self.lib.mia_gguf_get_config(self.h, ctypes.byref(c)))
        return c

    def header(self):
        v, b, e, u = ctypes.c_uint32(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        mia.check(self.lib.mia_gguf_get_header(self.h, ctypes.byref(v), ctypes.byref(b),
                                               ctypes.byref(e), ctypes.byref(u)))
        return v.value, b.value, e.value, u.value

    def tensors(self):
        out = []
        for i in range(self.lib.mia_gguf_n_tensors(self.h)):
            t = mia.GGUFTensor()
            mia.check(self.lib.mia_gguf_tensor_at(self.h, i, ctypes.byref(t)))
            out.append(t)
        return out

    def data(self, t):
        p = self.lib.mia_gguf_host_data(self.h, ctypes.byref(t))
        return ctypes.string_at(p, t.bytes)


def open_rc(path):
    lib = mia.load()
    h = ctypes.c_void_p()
    rc = lib.mia_gguf_open(str(path).encode(), ctypes.byref(h))
    if rc == 0:
        lib.mia_gguf_close(h.value)
    return rc


def ref_lib():
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref not built (reference tree absent)")
    lib = ctypes.CDLL(REF_SO)
    lib.ref_gguf_open.restype = ctypes.c_void_p
    lib.ref_gguf_open.argtypes = [ctypes.c_char_p]
    lib.ref_gguf_close.argtypes = [ctypes.c_void_p]
    lib.ref_gguf_config.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.ref_gguf_tensor.argtypes = [ctypes.c_void_p, ctypes.c_int] + [ctypes.c_void_p] * 6
    lib.ref_gguf_data_offset.restype = ctypes.c_long
    lib.ref_gguf_data_offset.argtypes = [ctypes.c_void_p]
    return lib


def ref_parse(path):
    lib = ref_lib()
    h = lib.ref_gguf_open(str(path).encode())
    assert h, "reference parser refused the file"
    ints = np.zeros(14, np.int32)
    floats = np.zeros(2, np.float32)
    lib.ref_gguf_config(h, ints.ctypes.data, floats.ctypes.data)
    tensors = []
    for i in range(int(ints[10])):
        name = ctypes.create_string_buffer(256)
        nd, ty = ctypes.c_uint32(), ctypes.c_uint32()
        ne = np.zeros(4, np.uint64)
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        lib.ref_gguf_tensor(h, i, name, ctypes.byref(nd), ne.ctypes.data, ctypes.byref(ty),
                            ctypes.byref(off), ctypes.byref(nb))
        tensors.append((name.value, nd.value, tuple(int(x) for x in ne), ty.value, off.value,
                        nb.value))
    data_off = lib.ref_gguf_data_offset(h)
    lib.ref_gguf_close(h)
    return ints, floats, tensors, data_off


@pytest.fixture
def model_file(tmp_path):
    g = np.random.default_rng(0)
    meta, tensors = W.mistral_like(g, q4_maker=O.make_q4_0)
    path = tmp_path / "m.gguf"
    offs = W.write(path, meta, tensors)
    return path, meta, tensors, offs


def test_config_and_tensors_match_what_was_written(model_file):
    path, meta, tensors, offs = model_file
    with Loaded(path) as f:
        c = f.config()
        assert (c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim) == \
            (256, 512, 2, 8, 2, 32)
        assert (c.vocab_size, c.max_seq_len, c.sliding_window) == (40, 32768, 4096)
        assert c.rope_theta == np.float32(1e6) and c.rms_eps == np.float32(1e-5)
        assert f.header() == (3, 1, 2, 0)
        got = f.tensors()
        assert [t.name.decode() for t in got] == [t[0] for t in tensors]
        assert f.lib.mia_gguf_data_offset(f.h) == offs["__data__"]
        for t, (name, ttype, shape, raw) in zip(got, tensors):
            assert t.type == ttype and t.n_dims == len(shape)
            assert tuple(t.ne)[:len(shape)] == shape and all(x == 1 for x in tuple(t.ne)[len(shape):])
            assert t.offset == offs[name] and t.bytes == len(raw)
            assert f.data(t) == raw
        q = mia.GGUFTensor()
        mia.check(f.lib.mia_gguf_find(f.h, b"blk.1.attn_v.weight", ctypes.byref(q)))
        assert q.ne[0] == 256 and q.ne[1] == 64 and q.bytes == 64 * 8 * 18
        assert f.lib.mia_gguf_find(f.h, b"blk.9.attn_v.weight", ctypes.byref(q)) == \
            mia.MIA_ERR_INVALID


def test_matches_the_reference_parser(model_file):
    path, meta, tensors, offs = model_file
    ints, floats, rtensors, rdata = ref_parse(path)
    with Loaded(path) as f:
        c = f.config()
        v, bos, eos, unk = f.header()
        assert list(ints) == [c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads,
                              c.head_dim, c.vocab_size, c.max_seq_len, c.sliding_window, v,
                              len(tensors), bos, eos, unk]
        assert floats[0] == c.rope_theta and floats[1] == c.rms_eps
        assert rdata == f.lib.mia_gguf_data_offset(f.h)
        for t, r in zip(f.tensors(), rtensors):
            assert (t.name, t.n_dims, tuple(t.ne), t.type, t.offset, t.bytes) == r


def test_mistral_prefix_and_defaults(tmp_path):
    # "mistral." keys, and the defaults of gguf_loader.h:166-171 when absent
    meta = [("mistral.embedding_length", W.U32, 128),
            ("mistral.attention.head_count", W.I32, 4),
            ("mistral.attention.sliding_window", W.U64, 2048)]
    path = tmp_path / "d.gguf"
    W.write(path, meta, [("x", W.GGML_F32, (32,), bytes(128))])
    with Loaded(path) as f:
        c = f.config()
        assert (c.dim, c.n_heads, c.head_dim, c.sliding_window) == (128, 4, 32, 2048)
        assert c.rope_theta == np.float32(10000.0) and c.rms_eps == np.float32(1e-5)
        assert f.header()[1:] == (1, 2, 0)
    ints, floats, _, _ = ref_parse(path)
    assert (ints[0], ints[3], ints[5], ints[8]) == (128, 4, 32, 2048)
    assert floats[0] == np.float32(10000.0)


def test_alignment_key_is_honoured(tmp_path):
    # general.alignment = 64: the data section starts at the next multiple of
    # 64.  gguf_loader.h:280 always rounds to 32, so it misplaces the data
    # whenever the header ends in the first half of a 64-byte line.
    raw = np.arange(64, dtype=np.float32).tobytes()
    differs = 0
    for pad in range(0, 64, 4):
        path = tmp_path / f"a{pad}.gguf"
        offs = W.write(path, [("general.name", W.STR, "p" * pad)],
                       [("t", W.GGML_F32, (64,), raw)], alignment=64, write_alignment_key=True)
        with Loaded(path) as f:
            assert f.lib.mia_gguf_data_offset(f.h) == offs["__data__"]
            assert offs["__data__"] % 64 == 0
            assert f.data(f.tensors()[0]) == raw
        if os.path.exists(REF_SO):
            differs += ref_parse(path)[3] != offs["__data__"]
    if os.path.exists(REF_SO):
        assert differs > 0


def test_k_quant_sizes(tmp_path):
    # gguf_type_size (gguf_loader.h:361-371) knows Q4_K but returns 0 for
    # Q6_K, so the reference reports 0 bytes; the ggml block is 210 bytes
    path = tmp_path / "k.gguf"
    W.write(path, [], [("a", W.GGML_Q4_K, (512, 2), bytes(2 * 2 * 144)),
                       ("b", W.GGML_Q6_K, (256, 3), bytes(3 * 210))])
    with Loaded(path) as f:
        a, b = f.tensors()
        assert a.bytes == 576 and b.bytes == 630
    _, _, rt, _ = ref_parse(path)
    assert rt[0][5] == 576 and rt[1][5] == 0
    bb, bv = ctypes.c_uint32(), ctypes.c_uint32()
    assert mia.load().mia_gguf_type_block(2, ctypes.byref(bb), ctypes.byref(bv)) == 0
    assert (bb.value, bv.value) == (18, 32)


def test_malformed_files_are_errors_not_reads_past_the_end(tmp_path, model_file):
    path, meta, tensors, offs = model_file
    blob = path.read_bytes()
    cases = W.malformed_variants(blob, offs["__data__"])
    for name, data in cases.items():
        p = tmp_path / f"bad_{name}.gguf"
        p.write_bytes(data)
        rc = open_rc(p)
        assert rc in (mia.MIA_ERR_INVALID, mia.MIA_ERR_UNSUPPORTED), name
    # a tensor offset pointing past the file
    bad = tmp_path / "bad_offset.gguf"
    W.bad_offset_file(bad)
    assert open_rc(bad) == mia.MIA_ERR_INVALID
    assert open_rc(tmp_path / "missing.gguf") == mia.MIA_ERR_INVALID
