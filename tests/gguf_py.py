"""Minimal GGUF v3 encoder for tests: builds arbitrary (including malformed)
files byte by byte, independently of the two C/C++ writers under test.

Layout (crates/t0-core/src/gguf.rs:299-345): magic "GGUF", u32 version, u64
tensor count, u64 metadata count, metadata (u64-length key, u32 type, value),
tensor infos (name, u32 n_dims, u64 dims innermost first, u32 type, u64 offset
relative to the blob), then the blob right after the infos with 32-byte aligned
offsets."""
import struct

import numpy as np

U32, F32, BOOL, STRING, ARRAY = 4, 6, 7, 8, 9


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def meta_value(kind, value):
    if kind == U32:
        return struct.pack("<II", U32, value)
    if kind == F32:
        return struct.pack("<If", F32, value)
    if kind == BOOL:
        return struct.pack("<IB", BOOL, 1 if value else 0)
    if kind == STRING:
        return struct.pack("<I", STRING) + _str(value)
    if kind == ARRAY:
        vals = np.asarray(value, np.float32)
        return struct.pack("<IIQ", ARRAY, F32, vals.size) + vals.tobytes()
    raise ValueError(kind)


def build(meta, tensors, version=3, magic=b"GGUF", offsets=None, raw_meta=None):
    """meta: list of (key, kind, value); tensors: list of (name, shape, ggml_type, data_bytes)."""
    out = bytearray(magic)
    out += struct.pack("<I", version)
    out += struct.pack("<QQ", len(tensors), len(meta) + (len(raw_meta) if raw_meta else 0))
    for k, kind, v in meta:
        out += _str(k) + meta_value(kind, v)
    for k, blob in raw_meta or []:
        out += _str(k) + blob
    offs, cur = [], 0
    for _, _, _, data in tensors:
        offs.append(cur)
        cur += len(data)
        cur += (-cur) % 32
    info_offs = offs if offsets is None else offsets  # the blob itself is always laid out naturally
    for (name, shape, ty, _), off in zip(tensors, info_offs):
        out += _str(name) + struct.pack("<I", len(shape))
        for d in reversed(shape):
            out += struct.pack("<Q", d)
        out += struct.pack("<IQ", ty, off)
    pos = 0
    for (_, _, _, data), off in zip(tensors, offs):
        if off > pos:
            out += b"\0" * (off - pos)
        out += data
        pos = off + len(data)
    return bytes(out)


def t0_meta(embed=128, layers=3, heads=2, hidden=256, patch=32, gen=3, levels=(0.1, 0.5, 0.9), extra=()):
    m = [("t0.embed_dim", U32, embed), ("t0.num_layers", U32, layers), ("t0.num_heads", U32, heads),
         ("t0.mlp_hidden_dim", U32, hidden), ("t0.patch_size", U32, patch), ("t0.group_every_n", U32, gen),
         ("t0.quantile_levels", ARRAY, list(levels))]
    return m + list(extra)
