"""GPU parity of the C drop-in (include/mia_dropin.h): the reference's own call
sequences, with host q/out buffers and a device KVCache, against the oracle.

- decode, steps 4-6 of mistral/mistral_model.h:849-863: apply_rope, fp16
  round, kv_write(pos % max_seq), len update, gqa_attention_neon;
- the fused mia_dropin_decode_step of the same steps;
- prefill, mistral/mistral_ane_prefill.h:746-755: apply_rope_batch,
  kv_write_batch, attention_batch;
- verify, mistral/speculative.h:92-101, as one mia_dropin_verify_step.
The cache has 3 layers and the tests use layer 1, so the layer offset of
kv_k / kv_v and of every drop-in entry point is exercised."""

import ctypes

import numpy as np
import pytest

import _data as D
import _gpu as G
import _oracle as O
import anetransformers_amd as mia

pytestmark = pytest.mark.gpu

TH = O.theta_inv(D.THETA, D.HD)
NL, LAYER = 3, 1
P = ctypes.c_void_p


def _p(a):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class Cache:
    """A drop-in KVCache (device ring) with helpers to load and read a layer."""

    def __init__(self, M):
        self.lib = G.lib()
        self.lib.mia_dropin_set_abort(0)
        self.kv = mia.KVCache()
        self.lib.mia_dropin_kv_alloc(ctypes.byref(self.kv), NL, D.N_KV, D.HD, M)
        assert self.lib.mia_dropin_status() == 0, self.lib.mia_last_error()
        self.M = M
        self.layer_bytes = M * self.kv.kv_dim * 2

    def base(self, which, layer):  # kv_k / kv_v (kv_cache.h:61-68)
        ptr = self.kv.k_cache if which == "k" else self.kv.v_cache
        return ptr + layer * self.layer_bytes

    def load(self, layer, kc, vc):
        mia.check(self.lib.mia_memcpy_h2d(self.base("k", layer), _p(kc), kc.nbytes), "load k")
        mia.check(self.lib.mia_memcpy_h2d(self.base("v", layer), _p(vc), vc.nbytes), "load v")

    def read(self, layer):
        out = []
        for w in "kv":
            a = np.empty((self.M, self.kv.kv_dim), dtype=np.uint16)
            mia.check(self.lib.mia_memcpy_d2h(_p(a), self.base(w, layer), a.nbytes), "read")
            out.append(a)
        return out

    def ok(self, what):
        assert self.lib.mia_dropin_status() == 0, f"{what}: {self.lib.mia_last_error()}"

    def free(self):
        self.lib.mia_dropin_kv_free(ctypes.byref(self.kv))
        self.ok("kv_free")
        assert not self.kv.k_cache and not self.kv.v_cache


def _other_layers_zero(c):
    for layer in range(NL):
        if layer != LAYER:
            kc, vc = c.read(layer)
            assert not kc.any() and not vc.any(), f"layer {layer} touched"


@pytest.mark.parametrize("M,filled,pos", [(4096, 512, 512), (300, 300, 1000), (1024, 1024, 1024)])
def test_reference_decode_sequence(M, filled, pos):
    G.say(f"dropin decode sequence M={M} pos={pos}")
    g = D.rng(M + pos)
    kc, vc = D.ring(g, M, filled=filled)
    q, k, v = D.normal(g, 4096), D.normal(g, 1024), D.normal(g, 1024)
    c = Cache(M)
    c.load(LAYER, kc, vc)
    lib = c.lib
    c.kv.len = min(filled, M)
    # 4. RoPE (host buffers, in place)
    qg, kg = q.copy(), k.copy()
    lib.mia_dropin_apply_rope(_p(qg), _p(kg), pos, _p(TH), 32, 8, 128)
    c.ok("apply_rope")
    qo, ko = q.copy(), k.copy()
    O.apply_rope(qo, ko, pos, TH, 32, 8, 128)
    D.check_close(qg, qo, atol=1e-5, rtol=1e-5, what="apply_rope q")
    D.check_close(kg, ko, atol=1e-5, rtol=1e-5, what="apply_rope k")
    # 5. fp16 round (cvt_f32_to_f16_neon) and kv_write at pos % max_seq
    k16, v16 = D.to_f16_bits(kg), D.to_f16_bits(v)
    lib.mia_dropin_kv_write(ctypes.byref(c.kv), LAYER, pos % M, _p(k16), _p(v16))
    c.ok("kv_write")
    if c.kv.len < M and pos + 1 > c.kv.len:
        c.kv.len = pos + 1
    # 6. attention over the layer's ring
    att = np.zeros(32 * M, dtype=np.float32)
    out = np.zeros(4096, dtype=np.float32)
    qin = qg.copy()
    lib.mia_dropin_gqa_attention(_p(qin), _p(att), _p(out), P(c.base("k", LAYER)),
                                 P(c.base("v", LAYER)), 32, 4, 128, M, pos)
    c.ok("gqa_attention")
    assert np.array_equal(qin, qg), "q must not be modified"
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = O.decode_step(kc_o, vc_o, q, k, v, pos, TH, 32, 8, 128, M)
    D.check_close(out, ref, what=f"dropin decode M={M} pos={pos}")
    kc_g, vc_g = c.read(LAYER)
    D.check_ring(kc_g, kc_o, vc_g, vc_o, [pos % M], k[None], np.array([pos]), TH, "dropin ring")
    _other_layers_zero(c)
    c.free()


@pytest.mark.parametrize("M,filled,pos", [(4096, 512, 512), (300, 300, 1000)])
def test_fused_decode_step(M, filled, pos):
    G.say(f"dropin decode_step M={M} pos={pos}")
    g = D.rng(3 * M + pos)
    kc, vc = D.ring(g, M, filled=filled)
    q, k, v = D.normal(g, 4096), D.normal(g, 1024), D.normal(g, 1024)
    c = Cache(M)
    c.load(LAYER, kc, vc)
    c.kv.len = min(filled, M)
    out = np.zeros(4096, dtype=np.float32)
    qh, kh, vh = q.copy(), k.copy(), v.copy()
    c.lib.mia_dropin_decode_step(ctypes.byref(c.kv), LAYER, _p(qh), _p(kh), _p(vh), pos, _p(TH),
                                 32, 8, _p(out))
    c.ok("decode_step")
    assert np.array_equal(qh, q) and np.array_equal(kh, k), "inputs must not be modified"
    assert c.kv.len == (min(filled, M) if filled >= M else max(filled, pos + 1))
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = O.decode_step(kc_o, vc_o, q, k, v, pos, TH, 32, 8, 128, M)
    D.check_close(out, ref, what=f"dropin decode_step M={M} pos={pos}")
    kc_g, vc_g = c.read(LAYER)
    D.check_ring(kc_g, kc_o, vc_g, vc_o, [pos % M], k[None], np.array([pos]), TH, "decode ring")
    _other_layers_zero(c)
    c.free()


@pytest.mark.parametrize("start,S", [(1536, 512), (0, 37)])
def test_reference_prefill_sequence(start, S):
    G.say(f"dropin prefill sequence start={start} S={S}")
    g = D.rng(start + S)
    M = 4096
    kc, vc = D.ring(g, M, filled=start)
    Q, K, V = D.normal(g, (S, 4096)), D.normal(g, (S, 1024)), D.normal(g, (S, 1024))
    c = Cache(M)
    c.load(LAYER, kc, vc)
    c.kv.len = start
    lib = c.lib
    Qg, Kg = Q.copy(), K.copy()
    lib.mia_dropin_apply_rope_batch(_p(Qg), _p(Kg), start, _p(TH), 32, 8, 128, S)
    c.ok("apply_rope_batch")
    lib.mia_dropin_kv_write_batch(ctypes.byref(c.kv), LAYER, start, _p(Kg), _p(V), 1024, S)
    c.ok("kv_write_batch")
    assert c.kv.len == start + S
    cfg = mia.MistralConfig(4096, 14336, NL, 32, 8, 128, 32000, M, 1e6, 1e-5, 0)
    out = np.zeros((S, 4096), dtype=np.float32)
    lib.mia_dropin_attention_batch(_p(Qg), _p(out), ctypes.byref(c.kv), LAYER, start,
                                   ctypes.byref(cfg), S, None)
    c.ok("attention_batch")
    # oracle: the same three steps on the CPU
    Qo, Ko = Q.copy(), K.copy()
    O.load().ora_apply_rope_batch(_p(Qo), _p(Ko), start, _p(TH), 32, 8, 128, S)
    D.check_close(Qg, Qo, atol=1e-5, rtol=1e-5, what="apply_rope_batch Q")
    kc_o, vc_o = kc.copy(), vc.copy()
    O.kv_write_batch(kc_o, vc_o, Ko, V, 8, 128, M, start, S)
    ref = O.attention_batch_parallel(Qo, kc_o, vc_o, 32, 8, 128, M, start, S)
    D.check_close(out, ref, what=f"dropin prefill start={start} S={S}")
    kc_g, vc_g = c.read(LAYER)
    pos = np.arange(start, start + S)
    D.check_ring(kc_g, kc_o, vc_g, vc_o, pos % M, K, pos, TH, "prefill ring")
    _other_layers_zero(c)
    c.free()


@pytest.mark.parametrize("M,start,S", [(512, 1500, 8), (4096, 100, 8)])
def test_verify_step(M, start, S):
    G.say(f"dropin verify_step M={M} start={start} S={S}")
    g = D.rng(M * 7 + start)
    filled = M if start >= M else start
    kc, vc = D.ring(g, M, filled=filled)
    Q, K, V = D.normal(g, (S, 4096)), D.normal(g, (S, 1024)), D.normal(g, (S, 1024))
    c = Cache(M)
    c.load(LAYER, kc, vc)
    c.kv.len = filled
    out = np.zeros((S, 4096), dtype=np.float32)
    c.lib.mia_dropin_verify_step(ctypes.byref(c.kv), LAYER, _p(Q), _p(K), _p(V), start, S, _p(TH),
                                 32, 8, _p(out))
    c.ok("verify_step")
    assert c.kv.len == min(M, max(filled, start + S))
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = O.verify_steps(kc_o, vc_o, Q, K, V, start, S, TH, 32, 8, 128, M)
    D.check_close(out, ref, what=f"dropin verify M={M} start={start}")
    kc_g, vc_g = c.read(LAYER)
    pos = np.arange(start, start + S)
    D.check_ring(kc_g, kc_o, vc_g, vc_o, pos % M, K, pos, TH, "verify ring")
    _other_layers_zero(c)
    c.free()


def test_dropin_rejects_bad_layer_without_device_work():
    G.say("dropin bad layer")
    c = Cache(64)
    k16 = np.zeros(1024, dtype=np.uint16)
    c.lib.mia_dropin_kv_write(ctypes.byref(c.kv), NL, 0, _p(k16), _p(k16))
    assert c.lib.mia_dropin_status() == mia.MIA_ERR_INVALID
    c.free()
