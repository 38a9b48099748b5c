"""Seeded synthetic weights, activations and models for the Hy-MT2 token-loop workloads.

Every buffer is produced once in host memory from a numpy PCG64 stream and then handed, byte
for byte, to both the HIP backend and the CPU checkers, so the GPU and CPU legs always see
identical inputs. Block layouts follow the reference's GGUF blocks (src/internal.h:21-27):

* STQ1_0: 42 B / 256 weights: qs[32] 4-bit codebook slots, sign[8], f16 d
* Q2_0C: 130 B / 512 weights: f16 d, qs[128] four 2-bit codes per byte, value (2c-3)*d
* Q4_K: 144 B / 256: f16 d, f16 dmin, scales[12] (6-bit packed), qs[128] 4-bit
* Q6_K: 210 B / 256: ql[128], qh[64], int8 scales[16], f16 d

The panel layout produced by :func:`codes_to_panel` is the reference's load-time repack
(src/kernels.c:529-561): 64 bytes per 256-weight block, segment s holding chunk {0,2,1,3}[s],
byte (s*16+o) carrying in bits 2l..2l+1 the code of weight chunk*64 + o + 16*l.

The reference ships no Q4_K/Q6_K quantizer (only dequant and dot), so :func:`quantize_q4_k`
and :func:`quantize_q6_k` are this package's own: they choose per-sub-block scales from the
block's range and round to nearest. Any valid block is a fair input for the matvec parity
tests; the dequant of what they produce is checked for small error in tests.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

from . import abi

QK = 256
SEG_OF_CHUNK = np.array([0, 2, 1, 3])
# STQ1_0 4-weight group codebook (src/kernels.c:178-181): sign half = 0xAA - base half.
STQ_BASE = np.array([0xA9, 0x89, 0x29, 0x09, 0xA6, 0x86, 0x26, 0x06,
                     0x9A, 0x92, 0x1A, 0x12, 0x6A, 0x62, 0x4A, 0x42], dtype=np.uint8)
STQ_CODEBOOK = np.concatenate([STQ_BASE, (0xAA - STQ_BASE.astype(np.int32)).astype(np.uint8)])


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def f16_bits(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_value(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# ----------------------------------------------------------------------------- codes / panel

def codes_to_panel(codes: np.ndarray) -> np.ndarray:
    """Per-weight 2-bit codes [n, nb, 256] -> panel bytes [n, nb, 64]."""
    n, nb, _ = codes.shape
    c = codes.reshape(n, nb, 4, 4, 16).astype(np.uint8)  # [chunk, lane l, o]
    byte = c[:, :, :, 0, :] | (c[:, :, :, 1, :] << 2) | (c[:, :, :, 2, :] << 4) | (c[:, :, :, 3, :] << 6)
    out = np.empty((n, nb, 4, 16), dtype=np.uint8)
    out[:, :, SEG_OF_CHUNK, :] = byte
    return out.reshape(n, nb, 64)


def panel_to_codes(pk: np.ndarray) -> np.ndarray:
    """Inverse of :func:`codes_to_panel`: panel bytes [n, nb, 64] -> codes [n, nb, 256]."""
    n, nb, _ = pk.shape
    seg = pk.reshape(n, nb, 4, 16)[:, :, SEG_OF_CHUNK, :]  # [chunk, o]
    c = np.stack([(seg >> (2 * l)) & 3 for l in range(4)], axis=3)  # [chunk, l, o]
    return c.reshape(n, nb, 256)


def stq_codes(blocks: np.ndarray) -> np.ndarray:
    """STQ1_0 blocks [n, nb, 42] -> per-weight codes [n, nb, 256] (0=-1, 1=0, 2=+1)."""
    g = np.arange(64)
    slot = (blocks[:, :, g >> 1] >> ((g & 1) * 4)) & 15
    sign = (blocks[:, :, 32 + (g >> 3)] >> (g & 7)) & 1
    cb = STQ_CODEBOOK[(sign.astype(np.int32) << 4) | slot]  # [n, nb, 64 groups]
    n, nb = blocks.shape[:2]
    out = np.empty((n, nb, 4, 4, 16), dtype=np.uint8)  # [chunk, l, o]
    cbr = cb.reshape(n, nb, 4, 16)
    for l in range(4):
        out[:, :, :, l, :] = (cbr >> (2 * l)) & 3
    return out.reshape(n, nb, 256)


# Panel byte position of STQ1_0 group g: chunk g>>4 goes to segment {0,2,1,3}[chunk].
_STQ_PANEL_POS = SEG_OF_CHUNK[np.arange(64) >> 4] * 16 + (np.arange(64) & 15)


def stq_panel(blocks: np.ndarray) -> np.ndarray:
    """STQ1_0 blocks [n, nb, 42] -> panel bytes [n, nb, 64]: the codebook byte of group g
    (src/kernels.c:184-188) already holds lanes 0..3 in panel bit order, so each group's byte
    is written straight to its panel position."""
    qs = blocks[:, :, :32]
    slots = np.empty(blocks.shape[:2] + (64,), dtype=np.uint8)
    slots[:, :, 0::2] = qs & 15
    slots[:, :, 1::2] = qs >> 4
    signs = np.unpackbits(blocks[:, :, 32:40], axis=2, bitorder="little")
    cb = STQ_CODEBOOK[(signs.astype(np.intp) << 4) | slots]
    out = np.empty_like(cb)
    out[:, :, _STQ_PANEL_POS] = cb
    return out


def q2c_codes(blocks: np.ndarray) -> np.ndarray:
    """Q2_0C blocks [n, nb512, 130] -> codes [n, 2*nb512, 256] (value (2c-3)*d)."""
    qs = blocks[:, :, 2:]
    c = np.stack([(qs >> (2 * j)) & 3 for j in range(4)], axis=3)  # weight 4*byte + j
    n, nb512 = blocks.shape[:2]
    return c.reshape(n, nb512 * 2, 256).astype(np.uint8)


def panel_from_blocks(gtype: int, data: np.ndarray, n: int, k: int):
    """Host-side panel repack (the reference's build_panel, src/model.c:642-660)."""
    if gtype == abi.GT_STQ1_0:
        blocks = data.reshape(n, k // QK, 42)
        ps = f16_value(blocks[:, :, 40:42].copy().view(np.uint16)[..., 0])
        return stq_panel(blocks), ps.astype(np.float32), 0, 1
    if gtype == abi.GT_Q2_0C:
        blocks = data.reshape(n, k // 512, 130)
        codes = q2c_codes(blocks)
        d = f16_value(blocks[:, :, 0:2].copy().view(np.uint16)[..., 0])
        ps = np.repeat(d, 2, axis=1)
        return codes_to_panel(codes), ps.astype(np.float32), 1, 3
    raise ValueError("panel repack only for STQ1_0 / Q2_0C")


# ----------------------------------------------------------------------------- block builders

def stq1_0_blocks(g: np.random.Generator, n: int, k: int, dlo=0.005, dhi=0.05) -> np.ndarray:
    nb = k // QK
    b = g.integers(0, 256, size=(n, nb, 42), dtype=np.uint8)
    d = f16_bits(g.uniform(dlo, dhi, size=(n, nb)))
    b[:, :, 40:42] = d.view(np.uint8).reshape(n, nb, 2)
    return b.reshape(n, nb * 42)


def q2_0c_blocks(g: np.random.Generator, n: int, k: int, dlo=0.002, dhi=0.02) -> np.ndarray:
    nb = k // 512
    b = g.integers(0, 256, size=(n, nb, 130), dtype=np.uint8)
    d = f16_bits(g.uniform(dlo, dhi, size=(n, nb)))
    b[:, :, 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    return b.reshape(n, nb * 130)


def panel_uniform_codes(g: np.random.Generator, n: int, k: int, ncodes=3, slo=0.005, shi=0.05):
    """Config-0 style panel: i.i.d. uniform codes in [0, ncodes) and fp32 scales U(slo, shi)."""
    nb = k // QK
    codes = g.integers(0, ncodes, size=(n, nb, 256), dtype=np.uint8)
    ps = g.uniform(slo, shi, size=(n, nb)).astype(np.float32)
    return codes_to_panel(codes), ps


def quantize_q4_k(x: np.ndarray) -> np.ndarray:
    """fp32 [n, k] -> Q4_K blocks [n, k/256*144] (range-based scales, round to nearest)."""
    n, k = x.shape
    nb = k // QK
    xb = x.reshape(n, nb, 8, 32).astype(np.float32)
    lo = np.minimum(xb.min(axis=3), 0.0)
    hi = xb.max(axis=3)
    s_f = (hi - lo) / 15.0
    m_f = -lo
    d = f16_value(f16_bits(np.maximum(s_f.max(axis=2), 1e-12) / 63.0))
    dmin = f16_value(f16_bits(np.maximum(m_f.max(axis=2), 1e-12) / 63.0))
    sc = np.clip(np.rint(s_f / d[..., None]), 0, 63).astype(np.int32)
    mn = np.clip(np.rint(m_f / dmin[..., None]), 0, 63).astype(np.int32)
    scale = d[..., None] * sc
    q = np.where(scale[..., None] > 0,
                 np.rint((xb + (dmin[..., None] * mn)[..., None]) / np.where(scale > 0, scale, 1)[..., None]), 0)
    q = np.clip(q, 0, 15).astype(np.uint8)  # [n, nb, 8 sub, 32]
    out = np.zeros((n, nb, 144), dtype=np.uint8)
    out[:, :, 0:2] = f16_bits(d).view(np.uint8).reshape(n, nb, 2)
    out[:, :, 2:4] = f16_bits(dmin).view(np.uint8).reshape(n, nb, 2)
    s = np.zeros((n, nb, 12), dtype=np.int32)
    for j in range(4):
        s[:, :, j] = (sc[:, :, j] & 63) | ((sc[:, :, j + 4] >> 4) << 6)
        s[:, :, j + 4] = (mn[:, :, j] & 63) | ((mn[:, :, j + 4] >> 4) << 6)
        s[:, :, j + 8] = (sc[:, :, j + 4] & 0xF) | ((mn[:, :, j + 4] & 0xF) << 4)
    out[:, :, 4:16] = s.astype(np.uint8)
    for grp in range(4):
        out[:, :, 16 + 32 * grp:16 + 32 * grp + 32] = q[:, :, 2 * grp, :] | (q[:, :, 2 * grp + 1, :] << 4)
    return out.reshape(n, nb * 144)


def quantize_q6_k(x: np.ndarray) -> np.ndarray:
    """fp32 [n, k] -> Q6_K blocks [n, k/256*210] (per-16 int8 scales, round to nearest)."""
    n, k = x.shape
    nb = k // QK
    xb = x.reshape(n, nb, 16, 16).astype(np.float32)
    s_f = np.abs(xb).max(axis=3) / 31.0
    d = f16_value(f16_bits(np.maximum(s_f.max(axis=2), 1e-12) / 127.0))
    sc = np.clip(np.rint(s_f / d[..., None]), 1, 127).astype(np.int32)
    scale = d[..., None] * sc
    q = np.clip(np.rint(xb / scale[..., None]), -32, 31).astype(np.int32) + 32  # 0..63
    a = q.reshape(n, nb, 256).astype(np.uint8)
    out = np.zeros((n, nb, 210), dtype=np.uint8)
    for half in range(2):
        e = a[:, :, 128 * half:128 * half + 128]
        l = np.arange(32)
        ql = np.zeros((n, nb, 64), dtype=np.uint8)
        ql[:, :, l] = (e[:, :, l] & 0xF) | ((e[:, :, l + 64] & 0xF) << 4)
        ql[:, :, l + 32] = (e[:, :, l + 32] & 0xF) | ((e[:, :, l + 96] & 0xF) << 4)
        qh = ((e[:, :, l] >> 4) | ((e[:, :, l + 32] >> 4) << 2) | ((e[:, :, l + 64] >> 4) << 4)
              | ((e[:, :, l + 96] >> 4) << 6)).astype(np.uint8)
        out[:, :, 64 * half:64 * half + 64] = ql
        out[:, :, 128 + 32 * half:128 + 32 * half + 32] = qh
    out[:, :, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, :, 208:210] = f16_bits(d).view(np.uint8).reshape(n, nb, 2)
    return out.reshape(n, nb * 210)


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """fp32 [n, k] -> Q8_0 blocks [n, k/32*34]: f16 d = max|x| / 127 per 32 weights, int8 round to
    nearest (src/internal.h:22 block_q8_0: f16 d, int8 qs[32])."""
    n, k = x.shape
    xb = x.reshape(n, k // 32, 32).astype(np.float32)
    d = f16_value(f16_bits(np.abs(xb).max(axis=2) / 127.0))
    q = np.clip(np.rint(xb / np.where(d > 0, d, 1)[..., None]), -127, 127).astype(np.int8)
    out = np.zeros((n, k // 32, 34), dtype=np.uint8)
    out[:, :, 0:2] = f16_bits(d).view(np.uint8).reshape(n, k // 32, 2)
    out[:, :, 2:] = q.view(np.uint8)
    return out.reshape(n, k // 32 * 34)


def dequant_rows(w: "Weight", rows) -> np.ndarray:
    """fp32 rows of an F16 / F32 / Q8_0 / Q4_K / Q6_K weight, with the reference's dequant_row
    operations in its order (src/kernels.c:1304-1329; Q4_K :844-859, Q6_K :786-806), one float32
    rounding per operation, so the values are bit-identical to the reference host's embedding."""
    rows = np.asarray(rows)
    raw = np.ascontiguousarray(w.data.reshape(w.n, w.row_bytes)[rows])
    m, k, f32 = len(rows), w.k, np.float32
    if w.type == abi.GT_F16:
        return raw.view(np.float16).astype(np.float32)
    if w.type == abi.GT_F32:
        return raw.view(np.float32).copy()
    if w.type == abi.GT_Q8_0:
        b = raw.reshape(m, k // 32, 34)
        d = f16_value(b[:, :, 0:2].copy().view(np.uint16)[..., 0])
        return (d[..., None] * b[:, :, 2:].view(np.int8).astype(f32)).reshape(m, k)
    if w.type == abi.GT_Q4_K:
        b = raw.reshape(m, k // QK, 144)
        d = f16_value(b[:, :, 0:2].copy().view(np.uint16)[..., 0])
        dmin = f16_value(b[:, :, 2:4].copy().view(np.uint16)[..., 0])
        s = b[:, :, 4:16].astype(np.int32)
        sc = np.empty(b.shape[:2] + (8,), np.int32)
        mn = np.empty_like(sc)
        for j in range(4):
            sc[..., j], mn[..., j] = s[..., j] & 63, s[..., j + 4] & 63
            sc[..., j + 4] = (s[..., j + 8] & 0xF) | ((s[..., j] >> 6) << 4)
            mn[..., j + 4] = (s[..., j + 8] >> 4) | ((s[..., j + 4] >> 6) << 4)
        qs = b[:, :, 16:].reshape(m, k // QK, 4, 32)
        q = np.stack([qs & 0xF, qs >> 4], axis=3).reshape(m, k // QK, 8, 32).astype(f32)  # sub-block is
        d1 = (d[..., None] * sc.astype(f32)).astype(f32)
        m1 = (dmin[..., None] * mn.astype(f32)).astype(f32)
        return ((d1[..., None] * q).astype(f32) - m1[..., None]).reshape(m, k)
    if w.type == abi.GT_Q6_K:
        b = raw.reshape(m, k // QK, 210)
        ql, qh = b[:, :, :128].reshape(m, -1, 2, 64), b[:, :, 128:192].reshape(m, -1, 2, 32)
        sc = b[:, :, 192:208].view(np.int8).reshape(m, -1, 2, 8).astype(f32)
        d = f16_value(b[:, :, 208:210].copy().view(np.uint16)[..., 0])
        out = np.empty((m, k // QK, 2, 4, 32), f32)
        l = np.arange(32)
        for qd in range(4):
            lo = ql[..., (qd & 1) * 32 + l]
            nib = (lo & 0xF) if qd < 2 else (lo >> 4)
            q = (nib | (((qh >> (2 * qd)) & 3) << 4)).astype(np.int32) - 32
            scl = sc[..., l // 16 + 2 * qd]
            out[:, :, :, qd, :] = ((d[..., None, None] * scl).astype(f32) * q.astype(f32)).astype(f32)
        return out.reshape(m, k)
    raise ValueError(f"no dequant for type {w.type}")


def f16_matrix(g: np.random.Generator, n: int, k: int, sigma=0.02) -> np.ndarray:
    x = g.standard_normal(size=(n, k), dtype=np.float32)
    x *= np.float32(sigma)
    return f16_bits(x).view(np.uint8).reshape(n, 2 * k)


# ----------------------------------------------------------------------------- weights / models

@dataclasses.dataclass
class Weight:
    """One GGUF weight matrix (raw rows) plus its optional host panel (pk/ps)."""
    type: int
    k: int
    n: int
    data: np.ndarray | None          # uint8 [n, row_bytes]
    pk: np.ndarray | None = None     # uint8 [n, nb, 64]
    ps: np.ndarray | None = None     # float32 [n, nb]
    pshift: int = 0
    poff: int = 0

    @property
    def row_bytes(self) -> int:
        return abi.row_bytes(self.type, self.k)

    def with_panel(self) -> "Weight":
        if self.type in (abi.GT_STQ1_0, abi.GT_Q2_0C) and self.pk is None:
            self.pk, self.ps, self.pshift, self.poff = panel_from_blocks(self.type, self.data, self.n, self.k)
        return self

    def nbytes_device(self) -> int:
        """Bytes the matvec streams per call (panel codes + scales, or raw blocks)."""
        if self.pk is not None:
            return self.pk.nbytes + self.ps.nbytes
        return self.n * self.row_bytes


def make_weight(g: np.random.Generator, gtype: int, n: int, k: int, **kw) -> Weight:
    if gtype == abi.GT_STQ1_0:
        return Weight(gtype, k, n, stq1_0_blocks(g, n, k, **kw)).with_panel()
    if gtype == abi.GT_Q2_0C:
        return Weight(gtype, k, n, q2_0c_blocks(g, n, k, **kw)).with_panel()
    if gtype == abi.GT_Q4_K:
        return Weight(gtype, k, n, quantize_q4_k(g.normal(0, kw.get("sigma", 0.02), size=(n, k))))
    if gtype == abi.GT_Q6_K:
        return Weight(gtype, k, n, quantize_q6_k(g.normal(0, kw.get("sigma", 0.02), size=(n, k))))
    if gtype == abi.GT_Q8_0:
        return Weight(gtype, k, n, quantize_q8_0(g.normal(0, kw.get("sigma", 0.02), size=(n, k))))
    if gtype == abi.GT_F16:
        return Weight(gtype, k, n, f16_matrix(g, n, k, kw.get("sigma", 0.02)))
    if gtype == abi.GT_F32:
        return Weight(gtype, k, n, g.normal(0, kw.get("sigma", 0.02), size=(n, k)).astype(np.float32).view(np.uint8))
    raise ValueError(f"unsupported type {gtype}")


@dataclasses.dataclass
class ModelShape:
    n_layer: int = 32
    hidden: int = 2048
    ffn: int = 6144
    heads: int = 16
    kv_heads: int = 4
    hdim: int = 128
    vocab: int = 120818
    ctx: int = 256
    eps: float = 1e-5
    rope_base: float = 10000.0
    rope_alpha: float = 0.0

    @property
    def qdim(self):
        return self.heads * self.hdim

    @property
    def kvdim(self):
        return self.kv_heads * self.hdim

    @property
    def rope_half(self):
        return self.hdim // 2


# Hy-MT2-1.8B shapes (the 1.8B decode and chunked-prefill benchmark workloads)
HYMT2_1_8B = ModelShape()

LAYER_TYPES = {
    "stq": dict(wq=abi.GT_STQ1_0, wk=abi.GT_STQ1_0, wv=abi.GT_STQ1_0, wo=abi.GT_STQ1_0,
                wg=abi.GT_STQ1_0, wu=abi.GT_STQ1_0, wd=abi.GT_STQ1_0),
    "q2": dict(wq=abi.GT_Q2_0C, wk=abi.GT_Q2_0C, wv=abi.GT_Q2_0C, wo=abi.GT_Q2_0C,
               wg=abi.GT_Q2_0C, wu=abi.GT_Q2_0C, wd=abi.GT_Q2_0C),
    "q4km": dict(wq=abi.GT_Q4_K, wk=abi.GT_Q4_K, wv=abi.GT_Q6_K, wo=abi.GT_Q4_K,
                 wg=abi.GT_Q4_K, wu=abi.GT_Q4_K, wd=abi.GT_Q6_K),
}


def make_model(shape: ModelShape, mode: str = "stq", seed: int = 3, head_type: int = abi.GT_F16,
               embd_sigma: float = 0.02) -> dict:
    """Random Hy-MT2-shaped model: layers of `mode` weights and a tied F16 embedding/head."""
    g = rng(seed)
    types = LAYER_TYPES[mode]
    s = shape
    layers = []
    for _ in range(s.n_layer):
        L = dict(attn_norm=g.uniform(0.9, 1.1, s.hidden).astype(np.float32),
                 ffn_norm=g.uniform(0.9, 1.1, s.hidden).astype(np.float32),
                 q_norm=g.uniform(0.9, 1.1, s.hdim).astype(np.float32),
                 k_norm=g.uniform(0.9, 1.1, s.hdim).astype(np.float32))
        dims = dict(wq=(s.qdim, s.hidden), wk=(s.kvdim, s.hidden), wv=(s.kvdim, s.hidden),
                    wo=(s.hidden, s.qdim), wg=(s.ffn, s.hidden), wu=(s.ffn, s.hidden), wd=(s.hidden, s.ffn))
        for name, (n, k) in dims.items():
            L[name] = make_weight(g, types[name], n, k)
        layers.append(L)
    if head_type == abi.GT_F16:
        embd = Weight(abi.GT_F16, s.hidden, s.vocab, f16_matrix(g, s.vocab, s.hidden, embd_sigma))
    else:
        embd = make_weight(g, head_type, s.vocab, s.hidden, sigma=embd_sigma)
    out_norm = g.uniform(0.9, 1.1, s.hidden).astype(np.float32)
    cosv, sinv = rope_tables(s.ctx, s.rope_half, s.hdim, s.rope_base, s.rope_alpha)
    return dict(shape=s, mode=mode, layers=layers, embd=embd, outw=embd, out_norm=out_norm,
                rope_cos=cosv, rope_sin=sinv, vocab_out=s.vocab)


def damp_token_row(model: dict, tok: int, factor: float = 1e-3) -> None:
    """Scale row `tok` of the tied F16 embedding / LM head by `factor`, so that its logit never
    wins the greedy argmax. Used for the EOS row (id 2) of the benchmark models: the reference's
    greedy loop stops at EOS (src/model.c:949), and the damped row keeps every run at its full
    length on both the reference host and the device loop."""
    e = model["embd"].data.view(np.float16)
    e[tok] = (e[tok].astype(np.float32) * factor).astype(np.float16)


# BASELINE configs 3 and 4: the 1.8B-shaped models and their prompts. The prompts are chat
# prompts of the "words" vocabulary (hymt2_amd.gguf): [BOS, USER, words..., ASSISTANT], so the
# reference host's text-driven greedy loop sees exactly these ids.
CONFIG3 = dict(mode="stq", seed=3, prompt_seed=1234, n_prompt=64, n_gen=128)
CONFIG4 = dict(mode="q2", seed=4, prompt_seed=4096, n_prompt=1024, n_gen=256, chunk=128)


def baseline_model(cfg: dict, ctx: int) -> dict:
    """The config's model (Hy-MT2-1.8B shapes, tied F16 head with a damped EOS row). The
    weights do not depend on ctx, which only sizes the RoPE tables."""
    model = make_model(ModelShape(ctx=ctx), mode=cfg["mode"], seed=cfg["seed"])
    damp_token_row(model, 2)
    model["vocab_style"] = "words"
    return model


# A small "words"-vocabulary model whose greedy runs end at EOS (id 2): the tied embedding's EOS
# row is scaled by 2.5 so that it wins the argmax after some steps (13 ids on the first prompt of
# GEN_IDS_CALLS). It pins the stop rule and the prefix-KV reuse of the reference's greedy loop
# (gen_ids, src/model.c:914-958). Each call is (user word ids, max_tokens); the calls run in
# order on one model, so each sees the cache the one before it left: the second prompt shares
# its first 12 words with the first, the third repeats the second, the fourth is capped at 5 ids.
GEN_IDS_SHAPE = ModelShape(n_layer=2, hidden=512, ffn=1024, heads=4, kv_heads=2, hdim=128, vocab=1000, ctx=256)


def gen_ids_model() -> dict:
    model = make_model(GEN_IDS_SHAPE, mode="stq", seed=211)
    e = model["embd"].data.view(np.float16)
    e[2] = (e[2].astype(np.float32) * 2.5).astype(np.float16)
    model["vocab_style"] = "words"
    return model


def gen_ids_calls():
    from . import gguf
    v = GEN_IDS_SHAPE.vocab
    w1 = rng(212).integers(gguf.FIRST_WORD, v, size=20)
    w2 = np.concatenate([w1[:12], rng(213).integers(gguf.FIRST_WORD, v, size=6)])
    w3 = rng(214).integers(gguf.FIRST_WORD, v, size=10)
    return [(w1, 64), (w2, 64), (w2, 64), (w3, 5)]


def baseline_prompt(cfg: dict, vocab: int = HYMT2_1_8B.vocab):
    """(ids, user text) of the config's prompt: n_prompt ids whose chat-templated text the
    reference encodes to exactly these ids."""
    from . import gguf
    words = rng(cfg["prompt_seed"]).integers(gguf.FIRST_WORD, vocab, size=cfg["n_prompt"] - 3)
    return np.array(gguf.chat_ids(words), dtype=np.int32), gguf.chat_text(words)


def rope_tables(ctx: int, rope_half: int, hdim: int, base: float, alpha: float):
    """RoPE cos/sin tables computed with libm float functions in the reference's order
    (src/model.c:535-537, :576-586), so they equal the tables the reference host uploads."""
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    for fn in ("powf", "cosf", "sinf"):
        getattr(libm, fn).restype = ctypes.c_float
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    libm.cosf.argtypes = [ctypes.c_float]
    libm.sinf.argtypes = [ctypes.c_float]
    f32 = np.float32
    base = f32(base)
    if alpha > 0 and hdim > 2:
        base = f32(base * f32(libm.powf(f32(alpha), f32(f32(hdim) / f32(hdim - 2)))))
    cosv = np.empty((ctx, rope_half), dtype=np.float32)
    sinv = np.empty((ctx, rope_half), dtype=np.float32)
    pos = np.arange(ctx, dtype=np.float32)
    for i in range(rope_half):
        freq = f32(f32(1.0) / f32(libm.powf(base, f32(f32(i) / f32(rope_half)))))
        ang = (pos * freq).astype(np.float32)
        cosv[:, i] = [libm.cosf(float(a)) for a in ang]
        sinv[:, i] = [libm.sinf(float(a)) for a in ang]
    return cosv, sinv


def model_weight_bytes(model: dict) -> dict:
    """Algorithmic bytes streamed per decode token (weights only), by part."""
    lay = sum(L[nm].nbytes_device() for L in model["layers"] for nm in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"))
    head = model["outw"].nbytes_device()
    return dict(layers=lay, head=head)


def activations(g: np.random.Generator, nt: int, k: int) -> np.ndarray:
    return g.normal(0.0, 1.0, size=(nt, k)).astype(np.float32)


def rand_prompt(g: np.random.Generator, n: int, vocab: int) -> np.ndarray:
    return g.integers(0, vocab, size=n, dtype=np.int32)


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)




def model_digest(model: dict) -> str:
    """sha256 over every buffer of a synthetic model in a fixed order; golden fixtures record
    it so a test can tell that the generator still reproduces the model they were made from."""
    import hashlib
    h = hashlib.sha256()
    s = model["shape"]
    h.update(repr(dataclasses.astuple(s)).encode())

    def add(a):
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())

    for L in model["layers"]:
        for nm in ("attn_norm", "ffn_norm", "q_norm", "k_norm"):
            add(L[nm])
        for nm in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
            w = L[nm]
            h.update(repr((w.type, w.k, w.n, w.pshift, w.poff)).encode())
            add(w.data), add(w.pk), add(w.ps)
    for a in (model["embd"].data, model["out_norm"], model["rope_cos"], model["rope_sin"]):
        add(a)
    return h.hexdigest()


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("math",)]
