"""Minimal GGUF v3 writer for synthetic Hy-MT2 ("hunyuan-dense") models.

Writes the keys and tensor names the reference loader reads (src/model.c:519-575,
src/tokenizer.c:120-171, src/gguf.c:92-149) so that the unchanged reference host can load the
same seeded weights the HIP backend receives.

Two tokenizer vocabularies:
* "placeholder" (default): tokens "t0", "t1", ...; the token loop is driven by ids.
* "words": id 0 "<unk>", 1 the BOS and 3 / 4 the user / assistant markers of the reference's
  chat template (src/model.c:915-916), 2 the EOS, and from id 5 on "\u0120" + a distinct
  lower-case word. The reference tokenizer (src/tokenizer.c:193-247, 298-312, 361-401) maps the
  text " w1 w2 ..." piece by piece to exactly those ids, so a prompt of chosen ids can be given
  to the reference's text-driven greedy loop (gen_ids) as text: see :func:`chat_text`.
"""
from __future__ import annotations

import struct

import numpy as np

from . import abi

ALIGN = 32

# "words" vocabulary: special tokens of the chat template (src/model.c:915-916)
BOS, EOS, USER, ASSISTANT = 1, 2, 3, 4
WORD_SPECIALS = ["<unk>", "<\uff5chy_begin\u2581of\u2581sentence\uff5c>", "<\uff5chy_end\u2581of\u2581sentence\uff5c>",
                 "<\uff5chy_User\uff5c>", "<\uff5chy_Assistant\uff5c>"]
FIRST_WORD = len(WORD_SPECIALS)


def word(i: int) -> str:
    """The distinct lower-case word of id i >= FIRST_WORD (bijective base 26)."""
    assert i >= FIRST_WORD
    n, out = i - FIRST_WORD + 1, []
    while n:
        n, r = divmod(n - 1, 26)
        out.append(chr(ord("a") + r))
    return "".join(reversed(out))


def word_token(i: int) -> str:
    """Token string of id i in the "words" vocabulary (GPT-2 byte encoding: space -> U+0120)."""
    return WORD_SPECIALS[i] if i < FIRST_WORD else "\u0120" + word(i)


def chat_text(word_ids) -> str:
    """User text whose chat-templated encoding by the reference host is
    [BOS, USER, *word_ids, ASSISTANT] (ids >= FIRST_WORD, "words" vocabulary)."""
    return "".join(" " + word(int(i)) for i in word_ids)


def chat_ids(word_ids) -> list:
    return [BOS, USER] + [int(i) for i in word_ids] + [ASSISTANT]
_T_U32, _T_F32, _T_STR, _T_ARR = 4, 6, 8, 9


def _s(b: bytes) -> bytes:
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, vtype: int, payload: bytes) -> bytes:
    return _s(key.encode()) + struct.pack("<I", vtype) + payload


def write_model(path: str, model: dict, name: str = "synthetic", vocab_style: str | None = None) -> None:
    """Writes `model` (hymt2_amd.synth) as a GGUF v3 file; the vocabulary style defaults to the
    model's "vocab_style" entry, else "placeholder"."""
    s = model["shape"]
    vocab_style = vocab_style or model.get("vocab_style", "placeholder")
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
    if vocab_style == "words":
        toks = b"".join(_s(word_token(i).encode()) for i in range(vocab))
    else:
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
