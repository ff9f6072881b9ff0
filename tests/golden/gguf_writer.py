"""Minimal GGUF v3 writer for test models (TEST INFRASTRUCTURE ONLY).

Writes what the reference's reader accepts for a Llama model (cleanroom-transformer/src/gguf.c:134-219
for the container; src/model.c:60-107 and :349-388 for the keys and tensor names): a header,
scalar/string metadata, tensor infos with ne[0] as the contiguous dimension, and tensor data
aligned to 32 bytes (the default general.alignment). gguf-py is not installed here, so this
project writes its own files.
"""
import struct

import numpy as np

GV_U32, GV_F32, GV_STR = 4, 6, 8
ALIGN = 32


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def write(path, kv, tensors, alignment=ALIGN):
    """kv: list of (key, kind, value) with kind in {"u32", "f32", "str"}.
    tensors: list of (name, ne tuple (ne[0] contiguous), ggml type id, raw uint8 bytes).
    alignment != 32 is written as general.alignment (u32) and used for the data section."""
    if alignment != ALIGN:
        kv = list(kv) + [("general.alignment", "u32", alignment)]
    head = bytearray()
    head += b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for key, kind, val in kv:
        head += _str(key)
        if kind == "u32":
            head += struct.pack("<II", GV_U32, val)
        elif kind == "f32":
            head += struct.pack("<If", GV_F32, val)
        elif kind == "str":
            head += struct.pack("<I", GV_STR) + _str(val)
        else:
            raise ValueError(kind)
    offsets, off = [], 0
    for name, ne, gtype, data in tensors:
        offsets.append(off)
        off += np.asarray(data).nbytes
        off = (off + alignment - 1) // alignment * alignment
    for (name, ne, gtype, data), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(ne)) + struct.pack("<%dQ" % len(ne), *ne)
        head += struct.pack("<IQ", gtype, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        pos = 0
        for (name, ne, gtype, data), o in zip(tensors, offsets):
            f.write(b"\0" * (o - pos))
            buf = np.ascontiguousarray(data).view(np.uint8).tobytes()
            f.write(buf)
            pos = o + len(buf)


def write_tiny_llama(path, model):
    """model: synth.tiny_llama() dict. Q8_0 matrices (type 8), F32 norms (type 0)."""
    c = model["cfg"]
    H, I, V = c["hidden"], c["intermediate"], c["vocab"]
    qw, kvw = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    kv = [("general.architecture", "str", "llama"), ("llama.block_count", "u32", c["n_layers"]),
          ("llama.embedding_length", "u32", H), ("llama.feed_forward_length", "u32", I),
          ("llama.attention.head_count", "u32", c["n_heads"]),
          ("llama.attention.head_count_kv", "u32", c["n_kv_heads"]),
          ("llama.rope.freq_base", "f32", c["rope_theta"]),
          ("llama.attention.layer_norm_rms_epsilon", "f32", c["eps"]), ("llama.vocab_size", "u32", V)]
    t = [("token_embd.weight", (H, V), 8, model["embed"]), ("output_norm.weight", (H,), 0, model["final_norm"]),
         ("output.weight", (H, V), 8, model["lm_head"])]
    names = {"q": ("attn_q", H, qw), "k": ("attn_k", H, kvw), "v": ("attn_v", H, kvw), "o": ("attn_output", qw, H),
             "gate": ("ffn_gate", H, I), "up": ("ffn_up", H, I), "down": ("ffn_down", I, H)}
    for li, L in enumerate(model["layers"]):
        t.append((f"blk.{li}.attn_norm.weight", (H,), 0, L["in_norm"]))
        t.append((f"blk.{li}.ffn_norm.weight", (H,), 0, L["post_norm"]))
        for key, (gn, ne0, ne1) in names.items():
            t.append((f"blk.{li}.{gn}.weight", (ne0, ne1), 8, L[key]))
    if model.get("rope_freqs") is not None:  # per-frequency RoPE divisors (Llama 3.1 scaling in GGUF)
        t.append(("rope_freqs.weight", (c["rot_dim"] // 2,), 0, np.ascontiguousarray(model["rope_freqs"], np.float32)))
    write(path, kv, t)
