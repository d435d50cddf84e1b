"""CPU tier: the C-ABI library loads, exports every symbol the headers declare,
the drop-in header compiles and links as C, and argument errors are reported
before any device work (no kernel is launched here)."""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import anetransformers_amd as mia

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(REPO, "include")
CLANG = "/opt/rocm/llvm/bin/clang"


def declared_functions():
    names = set()
    for h in ("miattn.h", "mia_dropin.h", "mia_gguf.h", "mia_peaks.h"):
        text = open(os.path.join(INCLUDE, h)).read()
        # top-level prototypes "type name(" ending in ");" (not static inline wrappers)
        for m in re.finditer(r"^(?:const\s+)?[A-Za-z_][\w \*]*?\b(mia_\w+)\s*\(", text, re.M):
            names.add(m.group(1))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = mia.load()
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding covers the same set
    assert set(names) <= set(mia.exported_symbols())


def test_library_exports_nothing_unprefixed():
    # every defined dynamic symbol (functions, data, weak) is the mia_ C ABI:
    # kernel stubs and C++ launch helpers stay local (csrc/exports.map)
    out = subprocess.run(["nm", "-D", "--defined-only", mia.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = [l.split()[-1] for l in out.splitlines() if l.strip()]
    ours = [n for n in exported if n.startswith("mia_")]
    assert len(ours) >= 30
    assert ours == exported, sorted(set(exported) - set(ours))
    assert "mia_internal_set_error" not in exported


@pytest.mark.skipif(not os.path.exists(CLANG), reason="ROCm clang not present")
def test_dropin_header_compiles_and_links(tmp_path):
    src = tmp_path / "use_dropin.c"
    src.write_text(r'''
#define MIA_DROPIN_Q4_REFERENCE_NAMES
#include "mia_dropin.h"
/* the reference's call sequence, mistral/mistral_model.h:849-863 */
void layer_attention(KVCache *kv, float *q, float *k, float *att, float *out, _Float16 *k16,
                     _Float16 *v16, const float *theta_inv, int layer, int pos) {
    apply_rope(q, k, pos, theta_inv, 32, 8, 128);
    int cache_pos = pos % kv->max_seq;
    kv_write(kv, layer, cache_pos, k16, v16);
    if (kv->len < kv->max_seq && pos + 1 > kv->len) kv->len = pos + 1;
    gqa_attention_neon(q, att, out, kv_k(kv, layer), kv_v(kv, layer), 32, 4, 128, kv->max_seq, pos);
}
void prefill(KVCache *kv, float *Q, float *K, float *V, float *out, const float *th,
             const MistralConfig *c, int start, int S) {
    apply_rope_batch(Q, K, start, th, c->n_heads, c->n_kv_heads, c->head_dim, S);
    kv_write_batch(kv, 0, start, K, V, kv->kv_dim, S);
    attention_batch(Q, out, kv, 0, start, c, S, 0);
}
/* the projections either side, mistral/mistral_model.h:833-842, 866-867 */
void projections(const void *wq, const void *wk, const void *wv, const void *wo, float *xb,
                 float *xb2, block_q8_0 *xb_q8, float *q, float *k, float *v, float *out) {
    quantize_f32_to_q8_0(xb, xb_q8, 4096);
    q4_matvec_sdot_parallel_fused_qkv(wq, wk, wv, xb_q8, q, k, v, 4096, 1024, 4096);
    quantize_f32_to_q8_0(xb2, xb_q8, 4096);
    q4_matvec_sdot_parallel(wo, 2, xb_q8, out, 4096, 4096);
}
_Static_assert(sizeof(block_q8_0) == 36, "block_q8_0 size");
int main(void) { KVCache kv = kv_alloc(1, 8, 128, 16); kv_free(&kv); return kv_k_at(&kv, 0, 0) != 0; }
''')
    exe = tmp_path / "use_dropin"
    r = subprocess.run([CLANG, "-std=c11", "-Wall", "-Werror", "-I", INCLUDE, str(src), "-o",
                        str(exe), "-L", mia.PKG_DIR, "-lmiattn",
                        f"-Wl,-rpath,{mia.PKG_DIR}"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


REF_MISTRAL = "/root/reference/mistral"


@pytest.mark.skipif(not os.path.exists(CLANG), reason="ROCm clang not present")
@pytest.mark.skipif(not os.path.exists(os.path.join(REF_MISTRAL, "gguf_loader.h")),
                    reason="reference tree absent")
def test_dropin_compiles_in_the_reference_translation_unit(tmp_path):
    """The header swap as the reference's own TU would see it: gguf_loader.h
    first (mistral/mistral_infer.m:12-14), whose MistralConfig the drop-in then
    uses, and the reference names called with that type."""
    src = tmp_path / "ref_tu.c"
    src.write_text(r'''
#include "gguf_loader.h"
#define MIA_GPU_ATTENTION
#include "mia_dropin.h"
void step(MistralConfig *c, float *q, float *k, float *att, float *out, const float *th,
          float *Q, float *O, int pos, int S) {
    KVCache kv = kv_alloc(c->n_layers, c->n_kv_heads, c->head_dim, 4096);
    apply_rope(q, k, pos, th, c->n_heads, c->n_kv_heads, c->head_dim);
    gqa_attention_neon(q, att, out, kv_k(&kv, 0), kv_v(&kv, 0), c->n_heads,
                       c->n_heads / c->n_kv_heads, c->head_dim, kv.max_seq, pos);
    attention_batch(Q, O, &kv, 0, pos, c, S, att);
    kv_free(&kv);
}
_Static_assert(sizeof(MistralConfig) == 44, "gguf_loader.h MistralConfig");
int main(int argc, char **argv) { return argc > 1 && argv[1][0] == 'x'; }
''')
    exe = tmp_path / "ref_tu"
    r = subprocess.run([CLANG, "-std=gnu11", "-Wall", "-Werror", "-Wno-unused-function",
                        "-I", REF_MISTRAL, "-I", INCLUDE, str(src), "-o", str(exe),
                        "-L", mia.PKG_DIR, "-lmiattn", f"-Wl,-rpath,{mia.PKG_DIR}"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # a translation unit with its own MistralConfig (same fields) opts out by macro
    src2 = tmp_path / "own_config.c"
    src2.write_text(r'''
typedef struct { int dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, vocab_size,
                 max_seq_len; float rope_theta, rms_eps; int sliding_window; } MistralConfig;
#define MIA_DROPIN_HAVE_MISTRAL_CONFIG
#include "mia_dropin.h"
void prefill(const MistralConfig *c, KVCache *kv, const float *Q, float *O, int start, int S) {
    attention_batch(Q, O, kv, 0, start, c, S, 0);
}
''')
    r = subprocess.run([CLANG, "-std=gnu11", "-Wall", "-Werror", "-I", INCLUDE, "-c", str(src2),
                        "-o", str(tmp_path / "own_config.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_kvcache_struct_layout_matches_reference():
    # mistral/metal_matvec.h:302 casts KVCache as {int a,b,c,d,e; ptr k, v; int f,g}
    assert mia.KVCache.k_cache.offset == 24 and mia.KVCache.v_cache.offset == 32
    assert mia.KVCache.pos.offset == 40 and ctypes.sizeof(mia.KVCache) == 48


def test_argument_errors_without_device_work():
    lib = mia.load()
    buf = np.zeros(16, np.float32)
    p = buf.ctypes.data
    rc = lib.mia_gqa_attention(p, p, p, p, 32, 4, 64, 128, 5, None)     # head_dim 64
    assert rc == mia.MIA_ERR_UNSUPPORTED and b"head_dim" in lib.mia_last_error()
    rc = lib.mia_gqa_attention(p, p, p, p, 32, 8, 128, 128, 5, None)    # GQA ratio 8
    assert rc == mia.MIA_ERR_UNSUPPORTED
    rc = lib.mia_gqa_attention(None, p, p, p, 32, 4, 128, 128, 5, None)
    assert rc == mia.MIA_ERR_INVALID
    rc = lib.mia_gqa_attention(p, p, p, p, 32, 4, 128, 128, -1, None)   # negative pos
    assert rc == mia.MIA_ERR_INVALID
    rc = lib.mia_attention_batch(p, p, p, p, 32, 8, 128, 1 << 23, 0, 4, None)  # max_seq too big
    assert rc == mia.MIA_ERR_UNSUPPORTED
    rc = lib.mia_attention_step(p, p, p, p, p, p, p, 32, 8, 128, 4096, 2**31 - 4, 8, None)
    assert rc == mia.MIA_ERR_INVALID and b"overflow" in lib.mia_last_error()
    rc = lib.mia_rope_f32(p, p, 1, 0, p, 32, 8, 96, None)
    assert rc == mia.MIA_ERR_UNSUPPORTED


def test_staged_verify_argument_errors_without_device_work():
    lib = mia.load()
    buf = np.zeros(64, np.float32)
    p = buf.ctypes.data
    rc = lib.mia_attention_step_staged(p, p, p, p, p, p, None, p, p, 32, 8, 128, 64, 0, 4, None)
    assert rc == mia.MIA_ERR_INVALID
    rc = lib.mia_attention_step_staged(p, p, p, p, p, p, p, p, p, 32, 8, 64, 64, 0, 4, None)
    assert rc == mia.MIA_ERR_UNSUPPORTED
    rc = lib.mia_commit_staged(p, p, p, p, 1, 4, 5, 0, 64, 1024, None)     # n_keep > S_staged
    assert rc == mia.MIA_ERR_INVALID
    rc = lib.mia_commit_staged(p, p, p, p, 0, 4, 2, 0, 64, 1024, None)     # no layers
    assert rc == mia.MIA_ERR_INVALID
    rc = lib.mia_commit_staged(p, p, p, p, 1, 4, 2, -1, 64, 1024, None)    # negative position
    assert rc == mia.MIA_ERR_INVALID
    lib.mia_dropin_set_abort(0)
    try:
        kv = mia.KVCache()
        kv.n_layers, kv.kv_dim, kv.max_seq = 2, 1024, 64
        lib.mia_dropin_verify_commit(ctypes.byref(kv), 10, 2)           # nothing staged
        assert lib.mia_dropin_status() == mia.MIA_ERR_INVALID
    finally:
        lib.mia_dropin_set_abort(1)


def test_prefill_argument_errors_without_device_work():
    lib = mia.load()
    buf = np.zeros(64, np.float32)
    p = buf.ctypes.data
    assert lib.mia_q4_0_gemm_f32(p, p, p, 64, 96, 4, None) == mia.MIA_ERR_UNSUPPORTED
    assert lib.mia_q4_0_gemm_f32(p, p, p, 64, 100, 4, None) == mia.MIA_ERR_INVALID
    assert lib.mia_q4_0_gemm_f32(p, p, p, 64, 128, 0, None) == mia.MIA_ERR_INVALID
    assert lib.mia_q4_0_gemm_f32(p + 2, p, p, 64, 128, 4, None) == mia.MIA_ERR_INVALID
    assert lib.mia_rmsnorm_f32(p, p, p, 6, 1, 1e-5, None) == mia.MIA_ERR_INVALID
    lw = mia.LayerWeights(*([p] * 9))
    # dim must be n_heads x 128
    assert lib.mia_prefill_layer(p, ctypes.byref(lw), p, p, p, 500, 1024, 4, 1, 1e-5, 64, 0, 4,
                                 None) == mia.MIA_ERR_UNSUPPORTED
    lw.w2 = None
    assert lib.mia_prefill_layer(p, ctypes.byref(lw), p, p, p, 512, 1024, 4, 1, 1e-5, 64, 0, 4,
                                 None) == mia.MIA_ERR_INVALID
    # the tile layout: multiples of 64, 16-byte aligned destination, no overlap
    big = np.zeros(64 * 128 // 32 * 18 // 4 + 8, np.float32)
    q = (big.ctypes.data + 15) // 16 * 16
    n = 64 * 128 // 32 * 18
    assert lib.mia_q4_0_pack_gemm(p, q, 100, 128, None) == mia.MIA_ERR_INVALID
    assert lib.mia_q4_0_pack_gemm(p, q, 64, 96, None) == mia.MIA_ERR_INVALID
    assert lib.mia_q4_0_pack_gemm(p, q + 4, 64, 128, None) == mia.MIA_ERR_INVALID
    assert lib.mia_q4_0_pack_gemm(q, q + n - 16, 64, 128, None) == mia.MIA_ERR_INVALID
    assert b"overlap" in lib.mia_last_error()
    assert lib.mia_q4_0_gemm_packed_f32(q, p, p, 96, 128, 4, None) == mia.MIA_ERR_INVALID
    assert lib.mia_q4_0_gemm_packed_f32(q + 4, p, p, 64, 128, 4, None) == mia.MIA_ERR_INVALID
    lw = mia.LayerWeights(*([q] * 9))
    lw.wo = q + 4
    assert lib.mia_prefill_layer_packed(p, ctypes.byref(lw), p, p, p, 512, 1024, 4, 1, 1e-5, 64,
                                        0, 4, None) == mia.MIA_ERR_INVALID
    assert b"16-byte" in lib.mia_last_error()


def test_typed_weight_entry_points_without_device_work(tmp_path):
    import _oracle as O
    lib = mia.load()
    for t in (mia.TYPE_F32, mia.TYPE_F16, mia.TYPE_Q4_0, mia.TYPE_Q4_K, mia.TYPE_Q6_K, 3, 8):
        for n in (32, 96, 256, 4096, 14336, 100):
            # the reference's sizes, where the library takes the shape (rows of
            # whole 32-value groups)
            want = O.typed_row_bytes(t, n) if t in (0, 1, 2, 12, 14) and n % 32 == 0 else 0
            assert lib.mia_weight_row_bytes(t, n) == want, (t, n)
    buf = np.zeros(64, np.float32)
    p = (buf.ctypes.data + 15) // 16 * 16
    assert lib.mia_matvec_f32(p, 3, p, p, 8, 256, None) == mia.MIA_ERR_UNSUPPORTED   # Q4_1
    assert lib.mia_matvec_f32(p, mia.TYPE_Q4_K, p, p, 8, 128, None) == mia.MIA_ERR_UNSUPPORTED
    assert lib.mia_matvec_f32(p + 2, mia.TYPE_Q4_K, p, p, 8, 256, None) == mia.MIA_ERR_INVALID
    assert lib.mia_matvec_f32(p + 2, mia.TYPE_Q6_K, p + 4, p, 8, 256, None) == mia.MIA_ERR_INVALID
    assert b"x must be 16-byte" in lib.mia_last_error()
    assert lib.mia_matvec_q8(p, mia.TYPE_Q6_K, p + 2, p, 8, 256, None) == mia.MIA_ERR_INVALID
    assert lib.mia_matvec_q8(p, mia.TYPE_Q4_0, p, p, 8, 96, None) == mia.MIA_ERR_UNSUPPORTED
    assert lib.mia_dequant_f32(p, mia.TYPE_F16, p + 4, 8, 64, None) == mia.MIA_ERR_INVALID
    assert lib.mia_dequant_f32(p, mia.TYPE_F16, p, 0, 64, None) == mia.MIA_ERR_INVALID
    assert lib.mia_gemm_f32(p, mia.TYPE_Q6_K, p, p, 8, 200, 4, None) == mia.MIA_ERR_UNSUPPORTED
    assert lib.mia_gemm_f32(p, mia.TYPE_F32, p, p + 4, 8, 64, 4, None) == mia.MIA_ERR_INVALID
    assert lib.mia_gemm_f32(p, mia.TYPE_Q4_0, p, p, 8, 96, 4, None) == mia.MIA_ERR_UNSUPPORTED
    lw = mia.LayerWeightsTyped(*([p] * 7), *([mia.TYPE_Q4_K] * 7), p, p)
    lw.w2_type = 5                                                            # Q5_0
    assert lib.mia_prefill_layer_typed(p, ctypes.byref(lw), p, p, p, 512, 1024, 4, 1, 1e-5, 64,
                                       0, 4, None) == mia.MIA_ERR_UNSUPPORTED
    lw.w2_type, lw.w1 = mia.TYPE_Q6_K, None
    assert lib.mia_prefill_layer_typed(p, ctypes.byref(lw), p, p, p, 512, 1024, 4, 1, 1e-5, 64,
                                       0, 4, None) == mia.MIA_ERR_INVALID
    # the C struct and the binding agree
    if os.path.exists(CLANG):
        src = tmp_path / "lw.c"
        src.write_text(r'''
#include <stddef.h>
#include "miattn.h"
_Static_assert(offsetof(mia_layer_weights_typed, wq_type) == %d, "types");
_Static_assert(offsetof(mia_layer_weights_typed, w3_type) == %d, "types");
_Static_assert(offsetof(mia_layer_weights_typed, rms_att) == %d, "rms");
_Static_assert(sizeof(mia_layer_weights_typed) == %d, "size");
''' % (mia.LayerWeightsTyped.wq_type.offset, mia.LayerWeightsTyped.w3_type.offset,
       mia.LayerWeightsTyped.rms_att.offset, ctypes.sizeof(mia.LayerWeightsTyped)))
        subprocess.run([CLANG, "-std=c11", "-fsyntax-only", "-I", INCLUDE, str(src)], check=True)


def test_typed_pack_sizes_and_errors_without_device_work():
    lib = mia.load()
    a = lambda n: (n + 255) // 256 * 256
    assert lib.mia_gemm_pack_bytes(mia.TYPE_Q4_K, 4096, 4096) == a(4096 * 4096 * 2)
    assert lib.mia_gemm_pack_bytes(mia.TYPE_F16, 100, 96) == a(100 * 96 * 2)
    assert lib.mia_gemm_pack_bytes(mia.TYPE_Q6_K, 4096, 14336) == \
        2 * a(4096 * 14336 * 2) + a(4096 * 4)
    assert lib.mia_gemm_pack_bytes(mia.TYPE_F32, 40, 1024) == 2 * a(40 * 1024 * 2) + a(40 * 4)
    assert lib.mia_gemm_pack_bytes(mia.TYPE_Q4_0, 4096, 4096) == 4096 * 128 * 18
    assert lib.mia_gemm_pack_bytes(mia.TYPE_Q4_0, 100, 4096) == 0        # tile layout: x 64
    assert lib.mia_gemm_pack_bytes(mia.TYPE_Q4_K, 64, 100) == 0
    assert lib.mia_gemm_pack_bytes(3, 64, 256) == 0
    buf = np.zeros(4096, np.float32)
    p = (buf.ctypes.data + 15) // 16 * 16
    assert lib.mia_gemm_pack(p, mia.TYPE_Q4_K, p + 8, 4, 256, None) == mia.MIA_ERR_INVALID
    assert lib.mia_gemm_pack(p, mia.TYPE_Q4_K, p + 512, 4, 256, None) == mia.MIA_ERR_INVALID
    assert b"overlap" in lib.mia_last_error()
    assert lib.mia_gemm_packed_f32(p + 8, mia.TYPE_Q4_K, p, p, 4, 256, 2, None) == \
        mia.MIA_ERR_INVALID
    lw = mia.LayerWeightsTyped(*([p] * 7), *([mia.TYPE_Q4_K] * 7), p, p)
    lw.wo = p + 32 + 2                      # Q6_K-legal alignment, not the packed form's
    lw.wo_type = mia.TYPE_Q6_K
    assert lib.mia_prefill_layer_typed_packed(p, ctypes.byref(lw), p, p, p, 512, 1024, 4, 1,
                                              1e-5, 64, 0, 4, None) == mia.MIA_ERR_INVALID
    assert b"16-byte" in lib.mia_last_error()


def test_q4_argument_errors_without_device_work():
    lib = mia.load()
    buf = np.zeros(64, np.float32)
    p = buf.ctypes.data
    rc = lib.mia_q4_0_matvec(p, p, p, 64, 96, None)           # 3 blocks per row (odd)
    assert rc == mia.MIA_ERR_UNSUPPORTED and b"even" in lib.mia_last_error()
    rc = lib.mia_q4_0_matvec(p, p, p, 64, 100, None)          # not a multiple of 32
    assert rc == mia.MIA_ERR_INVALID
    rc = lib.mia_q4_0_matvec(p, p, p, 0, 128, None)
    assert rc == mia.MIA_ERR_INVALID
    rc = lib.mia_q4_0_matvec(p + 2, p, p, 64, 128, None)      # misaligned weights
    assert rc == mia.MIA_ERR_INVALID and b"aligned" in lib.mia_last_error()
    rc = lib.mia_q4_0_matvec_qkv(p, None, p, p, p, p, p, 64, 16, 128, None)
    assert rc == mia.MIA_ERR_INVALID
    rc = lib.mia_q4_0_matvec_f32(p, p, p, 64, 16384, None)    # fused form: in_dim <= 8192
    assert rc == mia.MIA_ERR_UNSUPPORTED
    rc = lib.mia_q4_0_matvec_f32(p, p + 4, p, 64, 128, None)   # fp32 x needs 16-byte alignment
    assert rc == mia.MIA_ERR_INVALID
    rc = lib.mia_quantize_q8_0(p, p, 48, None)
    assert rc == mia.MIA_ERR_INVALID
    rc = lib.mia_quantize_q8_0(p + 4, p, 64, None)             # x needs 16-byte alignment
    assert rc == mia.MIA_ERR_INVALID


def test_no_device_is_reported(monkeypatch):
    lib = mia.load()
    n = ctypes.c_int(-1)
    rc = lib.mia_device_count(ctypes.byref(n))
    if rc == mia.MIA_OK and n.value > 0:
        pytest.skip("a device is present")
    rc = lib.mia_init(0)
    assert rc in (mia.MIA_ERR_NO_DEVICE, mia.MIA_ERR_INVALID)
    with pytest.raises(mia.MiattnError):
        mia.check(rc, "mia_init")


def test_dropin_error_path_returns_when_abort_disabled():
    lib = mia.load()
    lib.mia_dropin_set_abort(0)
    try:
        kv = mia.KVCache()
        lib.mia_dropin_kv_alloc(ctypes.byref(kv), 0, 8, 128, 16)   # invalid: no layers
        assert lib.mia_dropin_status() == mia.MIA_ERR_INVALID
        assert kv.k_cache is None and kv.kv_dim == 1024
    finally:
        lib.mia_dropin_set_abort(1)


def test_binding_fails_loudly_without_library(tmp_path):
    saved = mia._lib
    try:
        mia._lib = None
        with pytest.raises(mia.MiattnError):
            mia.load(str(tmp_path / "nope.so"))
    finally:
        mia._lib = saved


def test_positions_argument_errors_without_device_work():
    lib = mia.load()
    buf = np.zeros(64, np.float32)
    p = buf.ctypes.data
    pos = np.array([3, 4], np.int32)
    pp = pos.ctypes.data
    assert lib.mia_attention_positions(p, p, p, p, None, 32, 8, 128, 64, 2, None) == mia.MIA_ERR_INVALID
    assert lib.mia_attention_positions(p, p, p, p, pp, 32, 8, 128, 64, 0, None) == mia.MIA_ERR_INVALID
    assert lib.mia_attention_positions(p, p, p, p, pp + 2, 32, 8, 128, 64, 2,
                                       None) == mia.MIA_ERR_INVALID
    assert lib.mia_attention_positions(p, p, p, p, pp, 32, 8, 64, 64, 2,
                                       None) == mia.MIA_ERR_UNSUPPORTED
    assert lib.mia_attention_chunk(p, p, p, pp, None, p, p, p, 32, 8, 128, 64, 2,
                                   None) == mia.MIA_ERR_INVALID
    assert lib.mia_attention_chunk(p + 4, p, p, pp, p, p, p, p, 32, 8, 128, 64, 2,
                                   None) == mia.MIA_ERR_INVALID          # Q not 16-byte aligned
    lib.mia_dropin_set_abort(0)
    try:
        kv = mia.KVCache()
        kv.n_layers, kv.n_kv_heads, kv.head_dim, kv.kv_dim, kv.max_seq = 1, 8, 128, 1024, 64
        neg = np.array([5, -2], np.int32)
        lib.mia_dropin_prefill_chunk_attention(ctypes.byref(kv), 0, p, p, p, neg.ctypes.data, 2,
                                               p, 32, 8, p)
        assert lib.mia_dropin_status() == mia.MIA_ERR_INVALID
    finally:
        lib.mia_dropin_set_abort(1)
