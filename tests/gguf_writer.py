"""Minimal GGUF (v3) writer for tests: key/value metadata and tensors, data
section aligned to 32 bytes (GGUF spec; the reference loader assumes 32).

Written from the GGUF file-format description: magic "GGUF", u32 version,
u64 tensor count, u64 kv count, kv pairs (u64-length key, u32 type, value),
tensor infos (name, u32 n_dims, u64 dims[ne0..], u32 ggml type, u64 offset
relative to the data section), padding, data.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 2, 8, 12, 14
_BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q4_0: (32, 18), GGML_Q8_0: (32, 34), GGML_Q4_K: (256, 144),
          GGML_Q6_K: (256, 210)}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        at, items = v
        out = struct.pack("<IQ", at, len(items))
        return out + b"".join(_value(at, x) for x in items)
    return struct.pack(_FMT[t], v)


def tensor_bytes(ggml_type, shape):
    n = int(np.prod(shape)) if shape else 1
    be, bb = _BLOCK[ggml_type]
    return (n + be - 1) // be * bb


def write_gguf(path, kv, tensors, version=3, align=32, kv_count=None, tensor_count=None):
    """kv: list of (key, type, value); tensors: list of (name, shape, ggml_type,
    data bytes).  shape is GGUF order (ne0 first)."""
    head = b"GGUF" + struct.pack("<I", version)
    head += struct.pack("<QQ", len(tensors) if tensor_count is None else tensor_count,
                        len(kv) if kv_count is None else kv_count)
    for key, t, v in kv:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    offs, cur = [], 0
    for name, shape, gt, data in tensors:
        offs.append(cur)
        cur += len(data)
        cur = (cur + align - 1) // align * align
    for (name, shape, gt, data), off in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        head += struct.pack("<IQ", gt, off)
    pad = (-len(head)) % align
    body = bytearray()
    for (name, shape, gt, data), off in zip(tensors, offs):
        body += b"\0" * (off - len(body))
        body += bytes(data)
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad + bytes(body))
    return len(head) + pad


def llama_kv(dim=256, heads=4, heads_kv=2, layers=2, ff=512, ctx=1024, vocab=None, rope=10000.0, eps=1e-5):
    kv = [("general.architecture", STR, "llama"),
          ("llama.embedding_length", U32, dim),
          ("llama.attention.head_count", U32, heads),
          ("llama.attention.head_count_kv", U32, heads_kv),
          ("llama.block_count", U32, layers),
          ("llama.feed_forward_length", U32, ff),
          ("llama.context_length", U32, ctx),
          ("llama.rope.freq_base", F32, rope),
          ("llama.attention.layer_norm_rms_epsilon", F32, eps),
          ("llama.norm_eps", F32, eps),
          ("general.file_type", U32, 15),
          ("general.alignment", U32, 32)]
    if vocab is not None:
        kv.append(("tokenizer.ggml.tokens", ARR, (STR, vocab)))
        kv.append(("tokenizer.ggml.scores", ARR, (F32, [0.0] * len(vocab))))
    return kv
