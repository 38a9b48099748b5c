"""Pins of the oracle that do not depend on the reference build: closed forms, format
invariants, brute force and an independent float64 numpy forward. Each is chosen so that a
plausible mistake in the oracle (a dropped term, a wrong sign, index or permutation, a swapped
operand) fails it; the reference's own tolerances are reused where a check is not exact
(kernel error / sum|term| < 1e-5, tests/test_kernels.c:175-219)."""
import numpy as np
import pytest

from hymt2_amd import abi, synth
from oracle import oracle as O

f32 = np.float32


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ----------------------------------------------------------------------------- conversions

def test_f16_all_inputs_match_numpy():
    L = O.lib()
    h = np.arange(65536, dtype=np.uint16)
    got = np.array([L.oc_f16_to_f32(int(v)) for v in h], dtype=np.float32)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(ref)[~nan])


def test_bf16_round_to_nearest_even_brute_force():
    """Each result is the nearer of the two bf16 neighbours, ties to the even one."""
    L = O.lib()
    g = synth.rng(3)
    u = g.integers(0, 0x7F7F0000, size=20000, dtype=np.uint32)
    u[:64] = (np.arange(64, dtype=np.uint32) << 16) | 0x8000  # exact ties
    x = u.view(np.float32)
    for v, ub in zip(x, u):
        r = L.oc_f32_to_bf16(float(v))
        lo, hi = int(ub) >> 16, (int(ub) >> 16) + 1
        dlo = abs(float(v) - float(np.uint32(lo << 16).view(np.float32)))
        dhi = abs(float(np.uint32(hi << 16).view(np.float32)) - float(v))
        want = lo if (dlo < dhi or (dlo == dhi and lo % 2 == 0)) else hi
        assert r == want, (hex(ub), r, want)


def test_argmax_first_index_on_ties():
    L = O.lib()
    a = np.array([1.0, 3.0, -2.0, 3.0, 3.0], dtype=np.float32)
    assert L.oc_argmax(a.ctypes.data, 5) == 1
    b = np.full(7, -1.0, dtype=np.float32)
    assert L.oc_argmax(b.ctypes.data, 7) == 0


# ----------------------------------------------------------------------------- Q8_K

def test_q8k_closed_form():
    g = synth.rng(4)
    x = synth.activations(g, 4, 1024)
    x[0, :256] = 0.0
    x[1, 3], x[1, 9] = -5.0, 5.0
    y = O.quantize_q8k(x)
    blocks = x.reshape(-1, 256)
    for b, rec in zip(blocks, y):
        qs = rec["qs"].astype(np.int64)
        if not np.any(b):
            assert rec.tobytes() == bytes(576)
            continue
        j = int(np.argmax(np.abs(b)))  # first index of the largest magnitude
        assert qs[j] == -127, "the signed max maps to -127 (iscale = -127/max)"
        d = float(rec["d"])
        assert d == float(f32(1) / (f32(-127) / f32(b[j])))
        err = np.abs(b.astype(np.float64) - qs * d)
        assert np.all(err <= 0.5 * abs(d) * (1 + 1e-5) + 1e-30)
        assert np.array_equal(rec["bsums"], qs.reshape(16, 16).sum(axis=1))
        assert int(rec["sum"]) == int(qs.sum())
        perm = np.array([[c * 64 + l * 16 + i for c in (0, 2, 1, 3) for i in range(16)] for l in range(4)]).ravel()
        assert np.array_equal(rec["qp"], rec["qs"][perm])
    assert int(y[4]["qs"][3]) == -127 and int(y[4]["qs"][9]) == 127  # row 1, block 0: the first (negative) wins


# ----------------------------------------------------------------------------- block formats

def test_stq_codebook_one_zero_per_group_and_sign_half_negates():
    for i, byte in enumerate(synth.STQ_CODEBOOK):
        codes = [(int(byte) >> (2 * l)) & 3 for l in range(4)]
        assert codes.count(1) == 1 and all(c in (0, 1, 2) for c in codes), (i, codes)
        if i < 16:
            neg = [(int(synth.STQ_CODEBOOK[i + 16]) >> (2 * l)) & 3 for l in range(4)]
            assert neg == [2 - c for c in codes]
    assert len(set(synth.STQ_CODEBOOK[:16].tolist())) == 16


@pytest.mark.parametrize("gt", [abi.GT_STQ1_0, abi.GT_Q2_0C])
def test_panel_enc_equals_natural_order_dot(gt):
    """The panel's per-block int dot (codes x qp in panel order) equals the plain dot of the
    weights' codes with the activation's qs in natural order: pins the {0,2,1,3} segment order,
    the 2-bit lane layout and the qp permutation together."""
    g = synth.rng(5)
    n, k = 9, 1024
    w = synth.make_weight(g, gt, n, k)
    codes = (synth.stq_codes(w.data.reshape(n, k // 256, 42)) if gt == abi.GT_STQ1_0
             else synth.q2c_codes(w.data.reshape(n, k // 512, 130))).astype(np.int64)
    x = synth.activations(g, 2, k)
    xq = O.quantize_q8k(x)
    enc = O.block_ints(w, xq, 2, 0)
    qs = xq["qs"].astype(np.int64).reshape(2, k // 256, 256)
    want = np.einsum("rbj,tbj->trb", codes, qs)
    assert np.array_equal(enc, want)
    assert np.array_equal(synth.panel_to_codes(w.pk), codes)


def test_stq_q2_dequant_from_block_format():
    g = synth.rng(6)
    w = synth.make_weight(g, abi.GT_STQ1_0, 4, 512)
    d = synth.f16_value(w.data.reshape(4, 2, 42)[:, :, 40:42].copy().view(np.uint16)[..., 0])
    want = (synth.stq_codes(w.data.reshape(4, 2, 42)).astype(np.float32) - 1) * d[..., None]
    assert np.array_equal(bits(O.dequant(w)), bits(want.reshape(4, 512)))
    w = synth.make_weight(g, abi.GT_Q2_0C, 4, 1024)
    d = synth.f16_value(w.data.reshape(4, 2, 130)[:, :, 0:2].copy().view(np.uint16)[..., 0])
    want = (2 * synth.q2c_codes(w.data.reshape(4, 2, 130)).astype(np.float32) - 3) * np.repeat(d, 2, axis=1)[..., None]
    assert np.array_equal(bits(O.dequant(w)), bits(want.reshape(4, 1024)))


@pytest.mark.parametrize("gt,quant", [(abi.GT_Q4_K, synth.quantize_q4_k), (abi.GT_Q6_K, synth.quantize_q6_k)])
def test_kquant_roundtrip(gt, quant):
    """This package's Q4_K/Q6_K quantizer (written from the block format) and the oracle's
    dequant invert each other to quantization accuracy; a mis-indexed scale or nibble would
    give O(1) relative error."""
    g = synth.rng(7)
    x = g.normal(0, 0.02, size=(16, 2048)).astype(np.float32)
    w = synth.Weight(gt, 2048, 16, quant(x))
    deq = O.dequant(w)
    rel = np.sqrt(np.mean((deq - x) ** 2) / np.mean(x ** 2))
    assert rel < (0.08 if gt == abi.GT_Q4_K else 0.04), rel
    assert np.corrcoef(deq.ravel(), x.ravel())[0, 1] > 0.99


# ----------------------------------------------------------------------------- matvec

@pytest.mark.parametrize("gt", [abi.GT_STQ1_0, abi.GT_Q2_0C, abi.GT_Q4_K, abi.GT_Q6_K, abi.GT_F16, abi.GT_F32])
def test_matvec_vs_float64_dequant_dot(gt):
    """out[t, r] against sum_j dequant(W)[r, j] * x'[t, j] in float64, where x' is the Q8_K
    reconstruction q*d (quantized kinds) or x itself (F16/F32)."""
    g = synth.rng(8 + gt)
    n, k, nt = 33, 6144, 3
    w = synth.make_weight(g, gt, n, k)
    x = synth.activations(g, nt, k)
    xq = O.quantize_q8k(x)
    out = O.matvec(w, x, xq, nt).astype(np.float64)
    W = O.dequant(w).astype(np.float64)
    if gt in (abi.GT_F16, abi.GT_F32):
        xr = x.astype(np.float64)
    else:
        xr = (xq["qs"].astype(np.float64) * xq["d"].astype(np.float64)[:, None]).reshape(nt, k)
    terms = W[None, :, :] * xr[:, None, :]
    ref, mag = terms.sum(axis=2), np.abs(terms).sum(axis=2)
    assert np.all(np.abs(out - ref) <= 1e-5 * mag + 1e-30), np.max(np.abs(out - ref) / mag)


# ----------------------------------------------------------------------------- forward

TINY = synth.ModelShape(n_layer=2, hidden=512, ffn=1024, heads=4, kv_heads=2, hdim=128, vocab=600, ctx=32)


def _q8k_reconstruct(v):
    """Q8_K round trip of one fp32 vector (float32 arithmetic as the closed form states)."""
    out = np.empty(len(v), dtype=np.float64)
    for b in range(0, len(v), 256):
        blk = v[b:b + 256].astype(np.float32)
        if not np.any(blk):
            out[b:b + 256] = 0
            continue
        vmax = blk[int(np.argmax(np.abs(blk)))]
        iscale = f32(-127) / vmax
        q = np.clip(np.rint(iscale * blk), -127, 127)
        out[b:b + 256] = q * float(f32(1) / iscale)
    return out


def _bf16(v):
    u = np.asarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def numpy_forward(model, toks):
    """Float64 restatement of the Hy-MT2 forward (src/model.c:798-901): RMSNorm, Q8_K
    activations for the layer matvecs, NeoX RoPE then per-head q/k RMSNorm, bf16 KV, GQA
    softmax attention, SwiGLU, residuals, final norm, tied F16 head. Returns last logits."""
    s = model["shape"]
    W = {}
    for i, L in enumerate(model["layers"]):
        for nm in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
            W[i, nm] = O.dequant(L[nm]).astype(np.float64)
    E = O.dequant(model["embd"]).astype(np.float64)

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + s.eps) * w

    cos, sin = model["rope_cos"].astype(np.float64), model["rope_sin"].astype(np.float64)
    half = s.rope_half

    def rope(v, pos):
        v = v.reshape(-1, s.hdim).copy()
        a, b = v[:, :half].copy(), v[:, half:].copy()
        v[:, :half] = a * cos[pos] - b * sin[pos]
        v[:, half:] = a * sin[pos] + b * cos[pos]
        return v

    K = np.zeros((s.n_layer, s.ctx, s.kvdim))
    V = np.zeros((s.n_layer, s.ctx, s.kvdim))
    group = s.heads // s.kv_heads
    h = None
    for pos, tok in enumerate(toks):
        h = E[tok].copy()
        for i, L in enumerate(model["layers"]):
            xn = _q8k_reconstruct(rms(h, L["attn_norm"]).astype(np.float32))
            q = rope(W[i, "wq"] @ xn, pos)
            k = rope(W[i, "wk"] @ xn, pos)
            q = np.stack([rms(r, L["q_norm"]) for r in q])
            k = np.stack([rms(r, L["k_norm"]) for r in k])
            K[i, pos] = _bf16(k.ravel())
            V[i, pos] = _bf16(W[i, "wv"] @ xn)
            o = np.zeros(s.qdim)
            for hh in range(s.heads):
                kv = (hh // group) * s.hdim
                sc = K[i, :pos + 1, kv:kv + s.hdim] @ q[hh] / np.sqrt(s.hdim)
                p = np.exp(sc - sc.max())
                o[hh * s.hdim:(hh + 1) * s.hdim] = (p / p.sum()) @ V[i, :pos + 1, kv:kv + s.hdim]
            h = h + W[i, "wo"] @ _q8k_reconstruct(o.astype(np.float32))
            xn = _q8k_reconstruct(rms(h, L["ffn_norm"]).astype(np.float32))
            gt, up = W[i, "wg"] @ xn, W[i, "wu"] @ xn
            a = gt / (1 + np.exp(-gt)) * up
            h = h + W[i, "wd"] @ _q8k_reconstruct(a.astype(np.float32))
    return E @ rms(h, model["out_norm"])


@pytest.mark.parametrize("mode", ["stq", "q4km"])
def test_forward_vs_float64_numpy(mode):
    model = synth.make_model(TINY, mode=mode, seed=31)
    toks = synth.rand_prompt(synth.rng(32), 9, TINY.vocab)
    om = O.OracleModel(model, threads=4)
    om.forward(toks[:8], 0, False)
    lo = om.forward(toks[8:], 8, True).astype(np.float64)
    ref = numpy_forward(model, toks)
    err = np.max(np.abs(lo - ref)) / np.max(np.abs(ref))
    assert err < 2e-3, err  # float32 vs float64 rounding, amplified only by rare Q8_K rounding flips
    assert int(np.argmax(lo)) == int(np.argmax(ref))


def test_batched_equals_stepwise_and_prefix_reuse():
    """Prefill in one chunk equals token-by-token (tests/test_model.py:369-374), and continuing
    from a warm cache equals a cold run over the whole sequence (:394-399); bit-exact."""
    model = synth.make_model(TINY, mode="q2", seed=33)
    toks = synth.rand_prompt(synth.rng(34), 12, TINY.vocab)
    a = O.OracleModel(model, threads=4)
    a.forward(toks[:8], 0, False)
    la = a.forward(toks[8:], 8, True)
    b = O.OracleModel(model, threads=4)
    for i, t in enumerate(toks):
        lb = b.forward(toks[i:i + 1], i, i == len(toks) - 1)
    assert np.array_equal(bits(la), bits(lb))
    c = O.OracleModel(model, threads=4)
    c.forward(toks[:8], 0, False)
    c.forward(np.array([5, 6, 7], dtype=np.int32), 8, False)  # a different continuation first
    lc = c.forward(toks[8:], 8, True)  # then overwrite the same positions
    assert np.array_equal(bits(la), bits(lc))


def test_forward_rejects_out_of_range():
    model = synth.make_model(TINY, mode="stq", seed=35)
    om = O.OracleModel(model, threads=1)
    with pytest.raises(ValueError):
        om.forward(np.zeros(17, dtype=np.int32), 0)
    with pytest.raises(ValueError):
        om.forward(np.zeros(2, dtype=np.int32), TINY.ctx - 1)
    with pytest.raises(ValueError):
        om.forward(np.array([TINY.vocab], dtype=np.int32), 0)
