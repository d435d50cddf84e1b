"""MI355X (gfx950) Mistral-7B GQA attention hot path.

The product is ``libmiattn.so`` (HIP kernels + ``extern "C"`` shim + the C
drop-in with the reference's signatures, see ``include/``).  This module is a
thin ctypes binding over that C ABI used by the tests and the benchmark; it
holds no compute of its own and raises if the library is missing.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_long, c_size_t, c_uint64, c_void_p

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libmiattn.so")

MIA_OK = 0
MIA_ERR_INVALID = 1
MIA_ERR_UNSUPPORTED = 2
MIA_ERR_HIP = 3
MIA_ERR_NO_DEVICE = 4

HEAD_DIM = 128


class MiattnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"miattn status {code}: {msg}")
        self.code = code


class KVCache(ctypes.Structure):
    """mistral/kv_cache.h:10-20 field order (k_cache/v_cache on the device)."""

    _fields_ = [
        ("n_layers", c_int),
        ("n_kv_heads", c_int),
        ("head_dim", c_int),
        ("max_seq", c_int),
        ("kv_dim", c_int),
        ("k_cache", c_void_p),
        ("v_cache", c_void_p),
        ("pos", c_int),
        ("len", c_int),
    ]


class MistralConfig(ctypes.Structure):
    """mistral/gguf_loader.h:51-63 field order."""

    _fields_ = [
        ("dim", c_int),
        ("hidden_dim", c_int),
        ("n_layers", c_int),
        ("n_heads", c_int),
        ("n_kv_heads", c_int),
        ("head_dim", c_int),
        ("vocab_size", c_int),
        ("max_seq_len", c_int),
        ("rope_theta", c_float),
        ("rms_eps", c_float),
        ("sliding_window", c_int),
    ]


class GGUFTensor(ctypes.Structure):
    """mia_gguf_tensor (include/mia_gguf.h): GGUFTensor (gguf_loader.h:43-49) + bytes."""

    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("n_dims", ctypes.c_uint32),
        ("ne", ctypes.c_uint64 * 4),
        ("type", ctypes.c_uint32),
        ("offset", ctypes.c_uint64),
        ("bytes", ctypes.c_uint64),
    ]


class LayerWeights(ctypes.Structure):
    """mia_layer_weights (include/miattn.h): device pointers of one layer."""

    _fields_ = [(n, c_void_p) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "rms_att",
                                         "rms_ffn")]


class LayerWeightsTyped(ctypes.Structure):
    """mia_layer_weights_typed (include/miattn.h): device pointers and GGML
    type ids of one layer."""

    _fields_ = ([(n, c_void_p) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3")]
                + [(n + "_type", c_int) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3")]
                + [("rms_att", c_void_p), ("rms_ffn", c_void_p)])


TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 2, 12, 14

_P = c_void_p
_SIGS = {
    # runtime plumbing
    "mia_init": (c_int, [c_int]),
    "mia_device_count": (c_int, [POINTER(c_int)]),
    "mia_last_error": (ctypes.c_char_p, []),
    "mia_version": (c_int, []),
    "mia_malloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "mia_free": (c_int, [_P]),
    "mia_memcpy_h2d": (c_int, [_P, _P, c_size_t]),
    "mia_memcpy_d2h": (c_int, [_P, _P, c_size_t]),
    "mia_memcpy_d2d": (c_int, [_P, _P, c_size_t]),
    "mia_memset": (c_int, [_P, c_int, c_size_t]),
    "mia_stream_create": (c_int, [POINTER(c_void_p)]),
    "mia_stream_destroy": (c_int, [_P]),
    "mia_stream_sync": (c_int, [_P]),
    "mia_device_sync": (c_int, []),
    "mia_event_create": (c_int, [POINTER(c_void_p)]),
    "mia_event_destroy": (c_int, [_P]),
    "mia_event_record": (c_int, [_P, _P]),
    "mia_event_elapsed_ms": (c_int, [POINTER(c_float), _P, _P]),
    "mia_profile_begin": (c_int, []),
    "mia_profile_end": (c_int, [c_int, POINTER(c_int), POINTER(ctypes.c_double)]),
    "mia_fill_normal_f16": (c_int, [_P, c_size_t, c_uint64, _P]),
    "mia_scale_rows_f16": (c_int, [_P, c_long, c_int, c_int, c_int, c_float, _P]),
    # measured peaks (bench)
    "mia_peak_read_stream": (c_int, [_P, c_size_t, _P]),
    "mia_peak_read_ring": (c_int, [_P, _P, c_int, c_int, c_int, c_int, _P]),
    "mia_peak_mfma_f16": (c_int, [c_int, POINTER(ctypes.c_double), _P]),
    "mia_peak_empty": (c_int, [c_int, c_int, _P]),
    # hot path
    "mia_rope_f32": (c_int, [_P, _P, c_int, c_int, _P, c_int, c_int, c_int, _P]),
    "mia_kv_write_f32": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int, _P]),
    "mia_gqa_attention": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P]),
    "mia_decode_step": (c_int, [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P]),
    "mia_decode_step_noalloc": (
        c_int,
        [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P],
    ),
    "mia_attention_batch": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, _P]),
    "mia_attention_positions": (
        c_int,
        [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P],
    ),
    "mia_attention_chunk": (
        c_int,
        [_P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P],
    ),
    "mia_attention_step": (
        c_int,
        [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, _P],
    ),
    "mia_attention_step_staged": (
        c_int,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, _P],
    ),
    "mia_commit_staged": (
        c_int,
        [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, _P],
    ),
    "mia_quantize_q8_0": (c_int, [_P, _P, c_int, _P]),
    "mia_q4_0_matvec": (c_int, [_P, _P, _P, c_int, c_int, _P]),
    "mia_q4_0_matvec_qkv": (
        c_int,
        [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, _P],
    ),
    "mia_q4_0_matvec_f32": (c_int, [_P, _P, _P, c_int, c_int, _P]),
    "mia_q4_0_matvec_qkv_f32": (
        c_int,
        [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, _P],
    ),
    "mia_q4_0_matvec_pair": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, _P]),
    "mia_q4_0_matvec_pair_f32": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, _P]),
    "mia_silu_mul_f32": (c_int, [_P, _P, c_long, _P]),
    "mia_decode_layer": (
        c_int,
        [_P, POINTER(LayerWeightsTyped), _P, _P, _P, c_int, c_int, c_int, c_int, c_float, c_int,
         c_int, _P],
    ),
    "mia_rmsnorm_f32": (c_int, [_P, _P, _P, c_int, c_int, c_float, _P]),
    "mia_q4_0_gemm_f32": (c_int, [_P, _P, _P, c_int, c_int, c_int, _P]),
    "mia_q4_0_pack_gemm": (c_int, [_P, _P, c_int, c_int, _P]),
    "mia_q4_0_gemm_packed_f32": (c_int, [_P, _P, _P, c_int, c_int, c_int, _P]),
    "mia_prefill_layer": (
        c_int,
        [_P, POINTER(LayerWeights), _P, _P, _P, c_int, c_int, c_int, c_int, c_float, c_int,
         c_int, c_int, _P],
    ),
    "mia_prefill_layer_packed": (
        c_int,
        [_P, POINTER(LayerWeights), _P, _P, _P, c_int, c_int, c_int, c_int, c_float, c_int,
         c_int, c_int, _P],
    ),
    # weight types other than Q4_0
    "mia_weight_row_bytes": (c_long, [c_int, c_int]),
    "mia_dequant_f32": (c_int, [_P, c_int, _P, c_int, c_int, _P]),
    "mia_matvec_f32": (c_int, [_P, c_int, _P, _P, c_int, c_int, _P]),
    "mia_matvec_q8": (c_int, [_P, c_int, _P, _P, c_int, c_int, _P]),
    "mia_gemm_f32": (c_int, [_P, c_int, _P, _P, c_int, c_int, c_int, _P]),
    "mia_gemm_pack_bytes": (c_size_t, [c_int, c_int, c_int]),
    "mia_gemm_pack": (c_int, [_P, c_int, _P, c_int, c_int, _P]),
    "mia_gemm_packed_f32": (c_int, [_P, c_int, _P, _P, c_int, c_int, c_int, _P]),
    "mia_prefill_layer_typed_packed": (
        c_int,
        [_P, POINTER(LayerWeightsTyped), _P, _P, _P, c_int, c_int, c_int, c_int, c_float, c_int,
         c_int, c_int, _P],
    ),
    "mia_prefill_layer_typed": (
        c_int,
        [_P, POINTER(LayerWeightsTyped), _P, _P, _P, c_int, c_int, c_int, c_int, c_float, c_int,
         c_int, c_int, _P],
    ),
    # KV-ring snapshots
    "mia_kv_snapshot_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "mia_kv_snapshot_save": (c_int, [_P, c_size_t, _P, _P, c_int, c_int, c_int, c_int, c_int,
                                     c_int]),
    "mia_kv_snapshot_load": (c_int, [_P, c_size_t, _P, _P, c_int, c_int, c_int, c_int,
                                     POINTER(c_int), POINTER(c_int)]),
    "mia_kv_snapshot_info": (c_int, [_P, c_size_t] + [POINTER(c_int)] * 6),
    # GGUF weight files (include/mia_gguf.h); the config struct is MistralConfig's layout
    "mia_gguf_open": (c_int, [ctypes.c_char_p, POINTER(c_void_p)]),
    "mia_gguf_close": (None, [_P]),
    "mia_gguf_get_config": (c_int, [_P, POINTER(MistralConfig)]),
    "mia_gguf_get_header": (
        c_int,
        [_P, POINTER(ctypes.c_uint32), POINTER(c_int), POINTER(c_int), POINTER(c_int)],
    ),
    "mia_gguf_n_tensors": (c_int, [_P]),
    "mia_gguf_tensor_at": (c_int, [_P, c_int, POINTER(GGUFTensor)]),
    "mia_gguf_find": (c_int, [_P, ctypes.c_char_p, POINTER(GGUFTensor)]),
    "mia_gguf_host_data": (c_void_p, [_P, POINTER(GGUFTensor)]),
    "mia_gguf_data_offset": (c_size_t, [_P]),
    "mia_gguf_data_bytes": (c_size_t, [_P]),
    "mia_gguf_type_block": (
        c_int,
        [ctypes.c_uint32, POINTER(ctypes.c_uint32), POINTER(ctypes.c_uint32)],
    ),
    "mia_gguf_upload": (c_int, [_P, POINTER(c_void_p), POINTER(c_size_t)]),
    # drop-in (reference signatures)
    "mia_dropin_set_abort": (None, [c_int]),
    "mia_dropin_status": (c_int, []),
    "mia_dropin_kv_alloc": (None, [POINTER(KVCache), c_int, c_int, c_int, c_int]),
    "mia_dropin_kv_write": (None, [POINTER(KVCache), c_int, c_int, _P, _P]),
    "mia_dropin_kv_free": (None, [POINTER(KVCache)]),
    "mia_dropin_apply_rope": (None, [_P, _P, c_int, _P, c_int, c_int, c_int]),
    "mia_dropin_gqa_attention": (None, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int]),
    "mia_dropin_apply_rope_batch": (None, [_P, _P, c_int, _P, c_int, c_int, c_int, c_int]),
    "mia_dropin_kv_write_batch": (None, [POINTER(KVCache), c_int, c_int, _P, _P, c_int, c_int]),
    "mia_dropin_attention_batch": (
        None,
        [_P, _P, POINTER(KVCache), c_int, c_int, POINTER(MistralConfig), c_int, _P],
    ),
    "mia_dropin_decode_step": (
        None,
        [POINTER(KVCache), c_int, _P, _P, _P, c_int, _P, c_int, c_int, _P],
    ),
    "mia_dropin_verify_step": (
        None,
        [POINTER(KVCache), c_int, _P, _P, _P, c_int, c_int, _P, c_int, c_int, _P],
    ),
    "mia_dropin_prefill_chunk_attention": (
        None,
        [POINTER(KVCache), c_int, _P, _P, _P, _P, c_int, _P, c_int, c_int, _P],
    ),
    "mia_dropin_verify_stage": (
        None,
        [POINTER(KVCache), c_int, _P, _P, _P, c_int, c_int, _P, c_int, c_int, _P],
    ),
    "mia_dropin_verify_commit": (None, [POINTER(KVCache), c_int, c_int]),
    "mia_dropin_quantize_q8_0": (None, [_P, _P, c_int]),
    "mia_dropin_kv_save": (c_int, [POINTER(KVCache), ctypes.c_char_p]),
    "mia_dropin_kv_load": (c_int, [POINTER(KVCache), ctypes.c_char_p]),
    "mia_dropin_q4_matvec_sdot_parallel": (None, [_P, ctypes.c_uint32, _P, _P, c_int, c_int]),
    "mia_dropin_q4_matvec_sdot_parallel_fused_pair": (
        None,
        [_P, _P, _P, _P, _P, c_int, c_int],
    ),
    "mia_dropin_q4_matvec_sdot_parallel_fused_qkv": (
        None,
        [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int],
    ),
}

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libmiattn.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise MiattnError(
            MIA_ERR_NO_DEVICE,
            f"{path} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')",
        )
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return list(_SIGS)


def check(rc: int, what: str = "") -> None:
    if rc != MIA_OK:
        msg = load().mia_last_error().decode(errors="replace")
        raise MiattnError(rc, f"{what}: {msg}" if what else msg)


def init(device: int = 0) -> ctypes.CDLL:
    lib = load()
    check(lib.mia_init(device), "mia_init")
    return lib


def ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class DeviceBuffer:
    """Device allocation owned by Python; frees itself on close()/GC."""

    def __init__(self, nbytes: int):
        self.lib = load()
        p = c_void_p()
        check(self.lib.mia_malloc(ctypes.byref(p), int(nbytes)), "mia_malloc")
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(self.lib.mia_memcpy_h2d(self.ptr + offset, ptr(a), a.nbytes), "upload")

    def download(self, shape, dtype, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(self.lib.mia_memcpy_d2h(ptr(out), self.ptr + offset, out.nbytes), "download")
        return out

    def zero(self) -> None:
        check(self.lib.mia_memset(self.ptr, 0, self.nbytes), "memset")

    def close(self) -> None:
        if self.ptr:
            self.lib.mia_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        self.lib = load()
        p = c_void_p()
        check(self.lib.mia_event_create(ctypes.byref(p)), "event_create")
        self.ptr = p.value

    def record(self, stream=None) -> None:
        check(self.lib.mia_event_record(self.ptr, stream), "event_record")

    def elapsed_ms(self, later: "Event") -> float:
        ms = c_float()
        check(self.lib.mia_event_elapsed_ms(ctypes.byref(ms), self.ptr, later.ptr), "elapsed")
        return float(ms.value)
