"""A small GGUF v3 writer for the loader tests, written from the format itself
(little-endian: magic "GGUF", version, tensor count, metadata count, typed
key/value pairs, tensor infos, padding to the alignment, data), so that test
files need no external package (test infrastructure)."""

from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 2, 8, 12, 14
BLOCK = {GGML_F32: (4, 1), GGML_F16: (2, 1), GGML_Q4_0: (18, 32), GGML_Q8_0: (34, 32),
         GGML_Q4_K: (144, 256), GGML_Q6_K: (210, 256)}


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def tensor_bytes(ttype: int, shape) -> int:
    bb, bv = BLOCK[ttype]
    n = int(np.prod(shape))
    assert n % bv == 0
    return n // bv * bb


def write(path, metadata, tensors, alignment: int = 32, version: int = 3,
          write_alignment_key: bool = False) -> dict:
    """metadata: list of (key, vtype, value); tensors: list of (name, ggml type,
    shape as ne (ne[0] first), raw bytes).  Returns {name: offset} and the data
    section offset under "__data__"."""
    meta = list(metadata)
    if write_alignment_key:
        meta.append(("general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for k, vt, v in meta:
        head += _str(k) + struct.pack("<I", vt) + _value(vt, v)
    offsets, off = {}, 0
    infos = b""
    for name, ttype, shape, raw in tensors:
        assert len(raw) == tensor_bytes(ttype, shape), name
        infos += _str(name) + struct.pack("<I", len(shape))
        infos += b"".join(struct.pack("<Q", d) for d in shape)
        infos += struct.pack("<IQ", ttype, off)
        offsets[name] = off
        off += len(raw)
        off = (off + alignment - 1) // alignment * alignment
    body = head + infos
    data_off = (len(body) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(body)
        f.write(b"\0" * (data_off - len(body)))
        pos = 0
        for name, ttype, shape, raw in tensors:
            f.write(b"\0" * (offsets[name] - pos))
            f.write(raw)
            pos = offsets[name] + len(raw)
    offsets["__data__"] = data_off
    return offsets


def mistral_like(g, dim=256, n_layers=2, n_heads=8, n_kv=2, hidden=512, vocab=40,
                 prefix="llama", q4_maker=None):
    """Metadata and tensors shaped like a small Mistral GGUF (blk.N.attn_q ...)."""
    kv_dim = dim // n_heads * n_kv
    meta = [
        ("general.architecture", STR, prefix),
        ("general.name", STR, "test model"),
        (f"{prefix}.context_length", U32, 32768),
        (f"{prefix}.embedding_length", U32, dim),
        (f"{prefix}.feed_forward_length", U32, hidden),
        (f"{prefix}.block_count", U32, n_layers),
        (f"{prefix}.attention.head_count", U32, n_heads),
        (f"{prefix}.attention.head_count_kv", U32, n_kv),
        (f"{prefix}.rope.freq_base", F32, 1000000.0),
        (f"{prefix}.attention.layer_norm_rms_epsilon", F32, 1e-5),
        ("tokenizer.ggml.model", STR, "llama"),
        ("tokenizer.ggml.tokens", ARR, (STR, [f"tok{i}" for i in range(vocab)])),
        ("tokenizer.ggml.scores", ARR, (F32, [float(-i) for i in range(vocab)])),
        ("tokenizer.ggml.token_type", ARR, (I32, [1] * vocab)),
        ("tokenizer.ggml.bos_token_id", U32, 1),
        ("tokenizer.ggml.eos_token_id", U32, 2),
        ("tokenizer.ggml.unknown_token_id", U32, 0),
        ("general.nested", ARR, (ARR, [(U8, [1, 2, 3]), (STR, ["a", "bc"])])),
        ("general.flag", BOOL, True),
    ]
    tensors = []
    for l in range(n_layers):
        for nm, rows in (("attn_q", dim), ("attn_k", kv_dim), ("attn_v", kv_dim),
                         ("attn_output", dim)):
            raw = q4_maker(g, rows, dim).tobytes()
            tensors.append((f"blk.{l}.{nm}.weight", GGML_Q4_0, (dim, rows), raw))
        for nm in ("attn_norm", "ffn_norm"):
            tensors.append((f"blk.{l}.{nm}.weight", GGML_F32, (dim,),
                            g.standard_normal(dim).astype(np.float32).tobytes()))
    tensors.append(("token_embd.weight", GGML_F16, (dim, vocab),
                    g.standard_normal(dim * vocab).astype(np.float16).tobytes()))
    tensors.append(("output_norm.weight", GGML_F32, (dim,),
                    np.ones(dim, np.float32).tobytes()))
    return meta, tensors


def malformed_variants(blob: bytes, data_offset: int) -> dict:
    """Byte-level corruptions of a valid file that a loader must refuse (each
    one is an error, never a read past the mapping): bad magic and versions,
    an absurd count, and cuts inside the metadata, the tensor records and
    the data section."""
    return {
        "magic": b"GGUX" + blob[4:],
        "version1": blob[:4] + (1).to_bytes(4, "little") + blob[8:],
        "version4": blob[:4] + (4).to_bytes(4, "little") + blob[8:],
        "huge_count": blob[:8] + (1 << 40).to_bytes(8, "little") + blob[16:],
        "cut_in_metadata": blob[:200],
        "cut_in_tensor_infos": blob[:data_offset - 40],
        "cut_in_data": blob[:data_offset + 100],
        "short": blob[:10],
    }


def bad_offset_file(path) -> None:
    """A one-tensor file whose tensor offset points past the end."""
    write(path, [], [("t", GGML_F32, (8,), bytes(32))])
    b = bytearray(open(path, "rb").read())
    i = b.index(b"t") + 1 + 4 + 8 + 4            # name, n_dims, ne[0], type
    b[i:i + 8] = (1 << 20).to_bytes(8, "little")
    open(path, "wb").write(bytes(b))
