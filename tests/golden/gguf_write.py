"""GGUF writer (TEST INFRASTRUCTURE) with the reference converter's framing:
version 3, the converter's 19 key/values in its order (hy3_convert.c:926-949,
no tokenizer), tensor infos with dims in HF [out, in] order (:894-901, :1044),
the directory padded with zeros to general.alignment = 32 (:1066-1077) and
every tensor's data padded to 32 (:1232-1239). tests/test_oracle_golden.py
pins the framing byte for byte against a file the converter wrote.

tensors: list of (name, ggml_type, dims, data) where data is a uint8 array of
the tensor's bytes, or None for zeros (written sparsely: a seek, so that
full-size layers cost no disk writes).
"""
import struct

import numpy as np

ALIGN = 32
TYPE_SIZE = {0: (1, 4), 1: (1, 2), 8: (32, 36), 12: (256, 144)}

KVS = [  # (key, type, value) as hy3_convert.c:928-949 writes them
    ("general.architecture", 8, "hy_v3"),
    ("general.name", 8, "HYV3"),
    ("hy_v3.block_count", 4, 80),
    ("hy_v3.context_length", 4, 262144),
    ("hy_v3.embedding_length", 4, 4096),
    ("hy_v3.feed_forward_length", 4, 13312),
    ("hy_v3.attention.head_count", 4, 64),
    ("hy_v3.attention.head_count_kv", 4, 8),
    ("hy_v3.attention.key_length", 4, 128),
    ("hy_v3.attention.value_length", 4, 128),
    ("hy_v3.rope.freq_base", 4, 11158840),
    ("hy_v3.expert_count", 4, 192),
    ("hy_v3.expert_used_count", 4, 8),
    ("hy_v3.expert_feed_forward_length", 4, 1536),
    ("hy_v3.expert_shared_count", 4, 1),
    ("hy_v3.vocab_size", 4, 120832),
    ("hy_v3.attention.layer_norm_rms_epsilon", 6, 1e-5),
    ("hy_v3.rope.dimension_count", 4, 64),
    ("general.alignment", 4, ALIGN),
]


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _align(v):
    return (v + ALIGN - 1) // ALIGN * ALIGN


def nbytes(ggml_type, dims):
    be, bb = TYPE_SIZE[ggml_type]
    return int(np.prod(dims)) // be * bb


def write_gguf(path, tensors):
    hdr = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(KVS))
    for k, t, v in KVS:
        hdr += _str(k) + struct.pack("<I", t)
        hdr += _str(v) if t == 8 else (struct.pack("<f", v) if t == 6 else struct.pack("<I", v))
    infos, off = b"", 0
    for name, ty, dims, _ in tensors:
        infos += _str(name) + struct.pack("<I", len(dims)) + b"".join(
            struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ty, off)
        off = _align(off + nbytes(ty, dims))
    head = hdr + infos
    start = _align(len(head))
    with open(path, "wb") as f:
        f.write(head + b"\0" * (start - len(head)))
        pos = start
        for name, ty, dims, data in tensors:
            n = nbytes(ty, dims)
            if data is None:
                f.seek(pos + n)
            else:
                b = np.ascontiguousarray(data, np.uint8).tobytes()
                assert len(b) == n, (name, len(b), n)
                f.write(b)
            pos = _align(pos + n)
            f.seek(pos)
        f.truncate(pos)
