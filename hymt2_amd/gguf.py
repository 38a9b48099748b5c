"""Minimal GGUF v3 writer for synthetic Hy-MT2 ("hunyuan-dense") models.

Writes the keys and tensor names the reference loader reads (src/model.c:519-575,
src/tokenizer.c:120-171, src/gguf.c:92-149) so that the unchanged reference host can load the
same seeded weights the HIP backend receives. The tokenizer vocabulary is a list of plain
placeholder tokens ("t0", "t1", ...); the token loop is driven by ids, never by text.
"""
from __future__ import annotations

import struct

import numpy as np

from . import abi

ALIGN = 32
_T_U32, _T_F32, _T_STR, _T_ARR = 4, 6, 8, 9


def _s(b: bytes) -> bytes:
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, vtype: int, payload: bytes) -> bytes:
    return _s(key.encode()) + struct.pack("<I", vtype) + payload


def write_model(path: str, model: dict, name: str = "synthetic") -> None:
    s = model["shape"]
    arch = "hunyuan-dense"
    tensors = []  # (name, dims, ggml type, bytes)

    def add_w(nm, w):
        tensors.append((nm, (w.k, w.n), w.type, np.ascontiguousarray(w.data).tobytes()))

    def add_v(nm, v):
        tensors.append((nm, (len(v),), abi.GT_F32, np.ascontiguousarray(v, dtype=np.float32).tobytes()))

    add_w("token_embd.weight", model["embd"])
    if model["outw"] is not model["embd"]:
        add_w("output.weight", model["outw"])
    add_v("output_norm.weight", model["out_norm"])
    for i, L in enumerate(model["layers"]):
        add_v(f"blk.{i}.attn_norm.weight", L["attn_norm"])
        add_v(f"blk.{i}.ffn_norm.weight", L["ffn_norm"])
        add_v(f"blk.{i}.attn_q_norm.weight", L["q_norm"])
        add_v(f"blk.{i}.attn_k_norm.weight", L["k_norm"])
        for gnm, key in (("attn_q", "wq"), ("attn_k", "wk"), ("attn_v", "wv"), ("attn_output", "wo"),
                         ("ffn_gate", "wg"), ("ffn_up", "wu"), ("ffn_down", "wd")):
            add_w(f"blk.{i}.{gnm}.weight", L[key])

    kvs = [
        _kv("general.architecture", _T_STR, _s(arch.encode())),
        _kv("general.name", _T_STR, _s(name.encode())),
        _kv(f"{arch}.embedding_length", _T_U32, struct.pack("<I", s.hidden)),
        _kv(f"{arch}.block_count", _T_U32, struct.pack("<I", s.n_layer)),
        _kv(f"{arch}.feed_forward_length", _T_U32, struct.pack("<I", s.ffn)),
        _kv(f"{arch}.attention.head_count", _T_U32, struct.pack("<I", s.heads)),
        _kv(f"{arch}.attention.head_count_kv", _T_U32, struct.pack("<I", s.kv_heads)),
        _kv(f"{arch}.attention.key_length", _T_U32, struct.pack("<I", s.hdim)),
        _kv(f"{arch}.rope.dimension_count", _T_U32, struct.pack("<I", s.hdim)),
        _kv(f"{arch}.rope.freq_base", _T_F32, struct.pack("<f", s.rope_base)),
        _kv(f"{arch}.attention.layer_norm_rms_epsilon", _T_F32, struct.pack("<f", s.eps)),
        _kv("tokenizer.ggml.model", _T_STR, _s(b"gpt2")),
        _kv("tokenizer.ggml.pre", _T_STR, _s(arch.encode())),
        _kv("tokenizer.ggml.bos_token_id", _T_U32, struct.pack("<I", 1)),
        _kv("tokenizer.ggml.eos_token_id", _T_U32, struct.pack("<I", 2)),
        _kv("tokenizer.ggml.unknown_token_id", _T_U32, struct.pack("<I", 0)),
    ]
    if s.rope_alpha > 0:
        kvs.append(_kv(f"{arch}.rope.scaling.alpha", _T_F32, struct.pack("<f", s.rope_alpha)))
    vocab = model.get("tokenizer_vocab", s.vocab)
    toks = b"".join(_s(f"t{i}".encode()) for i in range(vocab))
    kvs.append(_kv("tokenizer.ggml.tokens", _T_ARR, struct.pack("<IQ", _T_STR, vocab) + toks))

    info = b""
    off = 0
    offsets = []
    for nm, dims, gtype, data in tensors:
        offsets.append(off)
        info += _s(nm.encode()) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        info += struct.pack("<IQ", gtype, off)
        off += (len(data) + ALIGN - 1) // ALIGN * ALIGN
    header = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kvs)) + b"".join(kvs) + info
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * ((-len(header)) % ALIGN))
        for (_, _, _, data) in tensors:
            f.write(data)
            f.write(b"\0" * ((-len(data)) % ALIGN))
