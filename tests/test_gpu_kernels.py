"""HIP kernels against the oracle and the golden vectors, bit for bit, through the C-ABI.

Covers the scalar conversions the kernels share (f16 -> f32 over every input, expf), Q8_K
activation quantization (src/kernels.c:128-165) with its edge cases, the panel / Q4_K / Q6_K
matvec (src/kernels.c:565-581, :808-877) at the layer shapes of BASELINE configs 0-2 and at
ragged row counts, the per-op `matmul` vtable entry (src/cuda.c:258-279 semantics), the F16
LM head with its fused argmax (src/kernels.c:1279-1289, src/model.c:945-948) and the entry
points' argument checks."""
import ctypes as C
import os
import zlib

import numpy as np
import pytest

from conftest import GOLDEN
from hymt2_amd import abi, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


# torch fills and copies on its own stream, the backend on the context stream: each helper
# waits for its torch work before the tensor is handed to the backend.
def dev(a):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
    torch.cuda.synchronize()
    return t


def empty_f32(n):
    import torch
    t = torch.zeros(n, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    return t


def sync():
    import torch
    torch.cuda.synchronize()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def q8k_dev(backend, x):
    """Quantize fp32 rows on the device; returns (device act tensor, host copy as Q8K records)."""
    import torch
    x = np.ascontiguousarray(x, dtype=np.float32)
    nt, k = x.shape
    act = torch.zeros(nt * (k // 256) * abi.Q8K_BYTES, dtype=torch.uint8, device="cuda:0")
    xd = dev(x)
    backend.quantize_q8k(xd.data_ptr(), act.data_ptr(), k, nt)
    sync()
    return act, act.cpu().numpy().view(O.Q8K_DTYPE)


# ----------------------------------------------------------------------------- conversions

def test_f16_to_f32_all_inputs(backend):
    src = np.arange(65536, dtype=np.uint16)
    out = empty_f32(65536)
    assert backend.L.hymt2_hip_selftest_f16(backend.impl, dev(src.view(np.int16)).data_ptr(), out.data_ptr(), 65536) == 0
    sync()
    got = out.cpu().numpy()
    ref = np.array([O.lib().oc_f16_to_f32(int(h)) for h in src], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan) and np.array_equal(bits(got)[~nan], bits(ref)[~nan])


def test_expf_matches_libm(backend):
    g = np.random.default_rng(0)
    x = np.concatenate([g.uniform(-104, 89, 1 << 21), g.uniform(-1, 1, 1 << 19), g.uniform(-20, 0, 1 << 19),
                        [0.0, -0.0, 88.72, 88.8, -103.9, -104.0, -200.0, 1e-30, -1e-30, np.inf, -np.inf]]
                       ).astype(np.float32)
    out = empty_f32(len(x))
    assert backend.L.hymt2_hip_selftest_expf(backend.impl, dev(x).data_ptr(), out.data_ptr(), len(x)) == 0
    sync()
    assert np.array_equal(bits(out.cpu().numpy()), bits(O.expf(x)))


def _mfma_operands(nw, g):
    """nw wavefronts of 64 (a, b) fp32 pairs, six kinds by wavefront: attention scores (q x bf16
    key), attention outputs (p in (0, 1] x bf16 value), random bit patterns over +-40 binades,
    products in and near the denormal range, denormal inputs and signed zeros, products that
    overflow."""
    def bf16(x):
        u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)

    def pattern(shape, lo, hi):
        s = g.integers(0, 2, shape, dtype=np.uint32) << 31
        e = g.integers(lo, hi, shape, dtype=np.uint32) << 23
        m = g.integers(0, 1 << 23, shape, dtype=np.uint32)
        return (s | e | m).view(np.float32)

    a = np.empty((nw, 64), np.float32)
    b = np.empty((nw, 64), np.float32)
    for k in range(6):
        w = slice(k, nw, 6)
        shape = a[w].shape
        if k == 0:
            a[w], b[w] = g.standard_normal(shape) * 3, bf16(g.standard_normal(shape))
        elif k == 1:
            a[w], b[w] = g.random(shape) ** 4, bf16(g.standard_normal(shape) * 0.1)
        elif k == 2:
            a[w], b[w] = pattern(shape, 127 - 40, 127 + 41), pattern(shape, 127 - 40, 127 + 41)
        elif k == 3:
            a[w], b[w] = pattern(shape, 1, 31), pattern(shape, 40, 110)
        elif k == 4:
            a[w] = np.where(g.random(shape) < 0.5, pattern(shape, 0, 1), np.where(g.random(shape) < 0.5, -0.0, 0.0))
            b[w] = pattern(shape, 100, 160)
        else:
            a[w], b[w] = pattern(shape, 200, 220), pattern(shape, 170, 190)
    return a, b


def test_mfma_zero_accumulator_products(backend):
    """The four-token chunk attention's products (a4_products: v_mfma_f32_16x16x1f32 with a zero
    accumulator) against numpy's IEEE single products, bit for bit, placed by the layout the
    kernel assumes: out[w][r][l] = a[w][16 (r / 4) + 4 (l / 16) + r % 4] * b[w][16 (r / 4) + l % 16].
    A -0 product may come back as +0 (no sum that starts at +0 can tell them apart); no other
    output may differ."""
    import torch
    nw = 3072
    a, b = _mfma_operands(nw, np.random.default_rng(23))
    out = torch.zeros(nw * 16 * 64, dtype=torch.float32, device="cuda:0")
    sync()
    ad, bd = dev(a), dev(b)
    assert backend.L.hymt2_hip_selftest_mfma(backend.impl, ad.data_ptr(), bd.data_ptr(), out.data_ptr(), nw) == 0
    sync()
    got = bits(out.cpu().numpy().reshape(nw, 16, 64))
    r, lane = np.arange(16)[:, None], np.arange(64)[None, :]
    with np.errstate(over="ignore", under="ignore"):
        want = bits(a[:, 16 * (r // 4) + 4 * (lane // 16) + r % 4] * b[:, 16 * (r // 4) + lane % 16])
    diff = got != want
    zero_sign = diff & (want == 0x80000000) & (got == 0)
    assert not (diff & ~zero_sign).any(), f"{int((diff & ~zero_sign).sum())} products differ"
    # the cases the operands were built for occur
    assert (want & 0x7F800000 == 0).sum() > 10000 and (want & 0x7FFFFFFF == 0x7F800000).sum() > 1000


def _sq_inputs(mode, m, n, g):
    x = g.standard_normal((m, n)).astype(np.float32)
    if mode == "small":
        x *= np.float32(0.02)
    elif mode == "outliers":
        x[:, ::64] *= np.float32(30)
    elif mode == "coarse":  # many halfway cases
        x = (np.trunc(x * 4) * np.float32(0.25)).astype(np.float32)
    elif mode == "wide":
        x *= np.exp(3 * g.standard_normal((m, n))).astype(np.float32)
    elif mode == "spike":
        x[np.arange(m), g.integers(0, n, m)] *= np.float32(1e6)
    elif mode == "regimes":
        x[:, : n // 2] *= np.float32(1e-3)
    elif mode == "zeros":
        x[g.random((m, n)) < 0.3] = 0
        x[: m // 4, :] = 0
    elif mode == "extreme":
        x[:, 0] = np.float32(3e19)  # squares overflow to inf
        x[m // 2:, 1] = np.nan
    return np.ascontiguousarray(x)


@pytest.mark.parametrize("mode", ["normal", "small", "outliers", "coarse", "wide", "spike", "regimes", "zeros",
                                  "extreme"])
@pytest.mark.parametrize("n", [2048, 1024, 132, 4])
def test_rmsnorm_sum_of_squares(backend, mode, n):
    """The RMSNorm's sequential sum of squares (src/model.c:719-739) by the lane-serial chain and
    by the exact segmented form, against numpy's sequential float32 accumulation."""
    g = np.random.default_rng(zlib.crc32(f"{mode}/{n}".encode()))
    m = 4096 if n == 2048 else 512
    x = _sq_inputs(mode, m, n, g)
    sq = (x * x).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        want = np.add.accumulate(sq, axis=1, dtype=np.float32)[:, -1]
    xd = dev(x)
    for method in (0, 1, 2):
        out = empty_f32(m)
        assert backend.L.hymt2_hip_selftest_sqsum(backend.impl, xd.data_ptr(), n, m, out.data_ptr(), method) == 0
        sync()
        got = out.cpu().numpy()
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(bits(got)[~nan], bits(want)[~nan]), f"method {method}"


def _softmax_addends(mode, m, n, g):
    """Non-negative addends like the attention's e_j = expf(s_j - max) in (0, 1], plus hard cases
    for the exact sum: long runs below half an ulp of the running sum (ties to even), equal
    values, zeros."""
    if mode == "uniform":
        s = g.standard_normal((m, n)).astype(np.float32)
    elif mode == "peaked":
        s = (g.standard_normal((m, n)) * 10).astype(np.float32)
    elif mode == "flat":
        s = (g.standard_normal((m, n)) * 1e-3).astype(np.float32)
    else:
        s = None
    if s is not None:
        s -= s.max(axis=1, keepdims=True)
        return np.exp(s).astype(np.float32)
    x = np.zeros((m, n), dtype=np.float32)
    if mode == "ties":      # 1, then addends of exactly half an ulp (and a quarter) of the sum
        x[:, 0] = 1.0
        x[:, 1:] = np.float32(2.0 ** -24)
        x[m // 2:, 1::3] = np.float32(2.0 ** -25)
    elif mode == "ones":
        x[:] = 1.0
        x[:, n // 2:] = np.float32(0.5)
    elif mode == "sparse":
        x[g.random((m, n)) < 0.05] = 1.0
        x[:, n - n // 4:] = 0.0
        x *= g.random((m, n)).astype(np.float32)
    return np.ascontiguousarray(x)


@pytest.mark.parametrize("mode", ["uniform", "peaked", "flat", "ties", "ones", "sparse"])
@pytest.mark.parametrize("n", [4096, 1280, 1000, 132, 4])
def test_softmax_denominator_sum(backend, mode, n):
    """The attention's softmax denominator: the sequential sum of e_j in position order
    (src/model.c:785-787) by the 8-wavefront exact form, against numpy's sequential float32
    accumulation."""
    g = np.random.default_rng(zlib.crc32(f"sm/{mode}/{n}".encode()))
    m = 256
    x = _softmax_addends(mode, m, n, g)
    want = np.add.accumulate(x, axis=1, dtype=np.float32)[:, -1]
    xd = dev(x)
    out = empty_f32(m)
    assert backend.L.hymt2_hip_selftest_sqsum(backend.impl, xd.data_ptr(), n, m, out.data_ptr(), 3) == 0
    sync()
    assert np.array_equal(bits(out.cpu().numpy()), bits(want))


# ----------------------------------------------------------------------------- Q8_K

def test_q8k_golden(backend):
    f = np.load(os.path.join(GOLDEN, "q8k.npz"), allow_pickle=False)
    _, got = q8k_dev(backend, f["x"])
    assert np.array_equal(got.view(np.uint8).ravel(), f["q8k"].ravel())


@pytest.mark.parametrize("k,nt", [(256, 1), (2048, 1), (2048, 16), (6144, 3), (6144, 16)])
def test_q8k_vs_oracle(backend, k, nt):
    g = synth.rng(k + nt)
    x = synth.activations(g, nt, k)
    x[0, :256] = 0.0
    x[-1, 11], x[-1, 40] = -4.0, 4.0        # the block's maximum magnitude with both signs: -max first
    if k >= 1024:
        x[-1, 261], x[-1, 456] = 5.0, -5.0  # +max first, in another lane
        x[-1, 520], x[-1, 523] = -6.0, 6.0  # both in one lane's eight elements
        x[-1, 770], x[-1, 771] = 7.0, -7.0
    x[nt // 2, 300 % k] = 1e25
    _, got = q8k_dev(backend, x)
    assert got.tobytes() == O.quantize_q8k(x).tobytes()


# ----------------------------------------------------------------------------- matvec

def run_matvec(backend, w, x):
    """Device quantize + matvec of an uploaded weight; returns out [nt, n] and the act."""
    nt = x.shape[0]
    h = backend.upload(w)
    try:
        act, xq = q8k_dev(backend, x)
        out = empty_f32(nt * w.n)
        backend.matvec(h, act.data_ptr(), out.data_ptr(), nt)
        sync()
        return out.cpu().numpy().reshape(nt, w.n), xq
    finally:
        backend.release(h)


@pytest.mark.parametrize("name", ["stq1_0", "q2_0c", "q4_k", "q6_k"])
def test_matvec_golden(backend, name):
    f = np.load(os.path.join(GOLDEN, f"matvec_{name}.npz"), allow_pickle=False)
    w = synth.Weight(int(f["type"]), int(f["k"]), int(f["n"]), f["data"]).with_panel()
    out, xq = run_matvec(backend, w, f["x"])
    assert np.array_equal(xq.view(np.uint8).ravel(), f["q8k"].ravel())
    assert np.array_equal(bits(out), bits(f["out"]))


SHAPES = [
    (abi.GT_STQ1_0, 12288, 2048),  # config 0: gate+up panel
    (abi.GT_STQ1_0, 3072, 2048),   # qkv
    (abi.GT_STQ1_0, 2048, 6144),   # down
    (abi.GT_Q2_0C, 2048, 2048),    # config 1: o
    (abi.GT_Q2_0C, 2048, 6144),
    (abi.GT_Q4_K, 3072, 2048),     # config 2: q/k
    (abi.GT_Q6_K, 2048, 6144),     # config 2: down
    (abi.GT_Q4_K, 37, 1536),       # ragged rows, odd block count
    (abi.GT_Q6_K, 65, 512),
    (abi.GT_STQ1_0, 1, 256),       # one row, one block
    (abi.GT_Q2_0C, 129, 512),
    (abi.GT_Q4_K, 37, 2048),       # ragged row counts at the decode kernel's two input sizes
    (abi.GT_STQ1_0, 129, 6144),
    (abi.GT_Q6_K, 65, 2048),
    (abi.GT_Q4_K, 11, 6144),
]


@pytest.mark.parametrize("gt,n,k", SHAPES)
def test_matvec_vs_oracle(backend, gt, n, k):
    g = synth.rng(gt * 7 + n + k)
    w = synth.make_weight(g, gt, n, k)
    for nt in (1, 2, 5, 16):
        x = synth.activations(g, nt, k)
        out, xq = run_matvec(backend, w, x)
        assert np.array_equal(bits(out), bits(O.matvec(w, x, xq, nt))), f"nt={nt}"


def test_config0_uniform_codes_panel(backend):
    """Config 0's panel (i.i.d. uniform codes 0..2, fp32 scales U(0.005, 0.05)) handed straight
    to upload as pk/ps, as the reference host does after its load-time repack."""
    g = synth.rng(0xC0DE0)
    n, k = 12288, 2048
    pk, ps = synth.panel_uniform_codes(g, n, k)
    w = synth.Weight(abi.GT_STQ1_0, k, n, np.zeros((n, abi.row_bytes(abi.GT_STQ1_0, k)), np.uint8), pk, ps, 0, 1)
    x = synth.activations(g, 1, k)
    out, xq = run_matvec(backend, w, x)
    assert np.array_equal(bits(out), bits(O.matvec(w, x, xq, 1)))


def test_per_op_matmul_groups(backend):
    """matmul() with q/k/v sharing one Q8_K activation (src/model.c:697-713 groups)."""
    g = synth.rng(77)
    ws = [synth.make_weight(g, abi.GT_Q4_K, 256, 2048), synth.make_weight(g, abi.GT_Q4_K, 128, 2048),
          synth.make_weight(g, abi.GT_Q6_K, 128, 2048)]
    hs = [backend.upload(w) for w in ws]
    try:
        for nt in (1, 7, 16):
            x = synth.activations(g, nt, 2048)
            xq = O.quantize_q8k(x)
            outs = backend.matmul(hs, [w.n for w in ws], xq, nt)
            for w, o in zip(ws, outs):
                assert np.array_equal(bits(o), bits(O.matvec(w, x, xq, nt)))
    finally:
        for h in hs:
            backend.release(h)


# ----------------------------------------------------------------------------- prefill GEMM

GEMM_SHAPES = [
    (abi.GT_STQ1_0, 3072, 2048),  # qkv of the 1.8B layer
    (abi.GT_Q2_0C, 2048, 6144),   # config 4: down
    (abi.GT_STQ1_0, 129, 512),    # ragged rows (row tiles of 32 / 64)
    (abi.GT_STQ1_0, 1, 256),      # one row, one block
    (abi.GT_Q2_0C, 1, 512),       # one row, one Q2_0C block (two panel pieces)
    (abi.GT_STQ1_0, 100, 1536),
    (abi.GT_Q2_0C, 8200, 2048),   # the large-contraction tiles at 128 tokens, ragged rows
    (abi.GT_Q2_0C, 16390, 2048),  # 256 row tiles of 64 and 6 rows (64 x 32 tiles), ragged tokens
]


@pytest.mark.parametrize("gt,n,k", GEMM_SHAPES)
def test_gemm_vs_oracle(backend, gt, n, k):
    """Chunks of more than 4 tokens run panel weights on the int8-MFMA GEMM (k_gemm_panel): every
    token's row equals panel_rows_scalar (src/kernels.c:565-581) bit for bit, for token counts
    that fill, straddle and undershoot the 16-, 32- and 64-token tiles (5 and 13: the reference
    host's batches of up to 16). Each call runs three times: a result that depends on wave
    timing shows up as a repeat that differs."""
    g = synth.rng(gt * 11 + n + k)
    w = synth.make_weight(g, gt, n, k)
    for nt in (5, 13, 17, 64, 77, 128):
        x = synth.activations(g, nt, k)
        out, xq = run_matvec(backend, w, x)
        assert np.array_equal(bits(out), bits(O.matvec(w, x, xq, nt))), f"nt={nt}"
        for rep in range(2):
            again, _ = run_matvec(backend, w, x)
            assert np.array_equal(bits(again), bits(out)), f"nt={nt} repeat {rep}"


def test_upload_rejects_partial_q2_0c_block(backend):
    """A Q2_0C row is whole 512-weight blocks (src/model.c:138): K = 256 is refused before
    any host bytes are read."""
    w = synth.Weight(abi.GT_Q2_0C, 256, 1, np.zeros((1, 0), dtype=np.uint8))
    w.pk = np.zeros((1, 1, 64), dtype=np.uint8)
    w.ps = np.zeros((1, 1), dtype=np.float32)
    with pytest.raises(RuntimeError):
        backend.upload(w)


def test_gemm_small_grid_repeats(backend):
    """The smallest GEMM grids (one row tile, one or two token tiles: one wavefront per SIMD,
    the tightest instruction timing) give the same bits on every one of 40 calls."""
    g = synth.rng(977)
    for gt, n, k in ((abi.GT_STQ1_0, 1, 256), (abi.GT_Q2_0C, 16, 512)):
        w = synth.make_weight(g, gt, n, k)
        h = backend.upload(w)
        try:
            for nt in (20, 64):
                x = synth.activations(g, nt, k)
                act, xq = q8k_dev(backend, x)
                want = bits(O.matvec(w, x, xq, nt))
                out = empty_f32(nt * n)
                for rep in range(20):
                    backend.matvec(h, act.data_ptr(), out.data_ptr(), nt)
                    sync()
                    got = bits(out.cpu().numpy().reshape(nt, n))
                    assert np.array_equal(got, want), f"type {gt} n={n} k={k} nt={nt} call {rep}"
        finally:
            backend.release(h)


def test_gemm_full_gate_up_vs_single_token(backend):
    """Config 4's widest contraction (2 x 6144 rows, K 2048, 128 tokens): the GEMM equals 128
    single-token decode-matvec calls on the same activations (each pinned to the oracle by
    test_matvec_vs_oracle), and the oracle on a sample of tokens."""
    g = synth.rng(0x6E77)
    n, k, nt = 12288, 2048, 128
    w = synth.make_weight(g, abi.GT_Q2_0C, n, k)
    x = synth.activations(g, nt, k)
    x[5] *= 1e-3   # small and large activation scales
    x[77] *= 50.0
    h = backend.upload(w)
    try:
        act, xq = q8k_dev(backend, x)
        out = empty_f32(nt * n)
        one = empty_f32(nt * n)
        backend.matvec(h, act.data_ptr(), out.data_ptr(), nt)
        for t in range(nt):
            backend.matvec(h, act.data_ptr() + t * (k // 256) * abi.Q8K_BYTES, one.data_ptr() + t * n * 4, 1)
        sync()
        got = out.cpu().numpy().reshape(nt, n)
        assert np.array_equal(bits(got), bits(one.cpu().numpy().reshape(nt, n)))
        nb = k // 256
        for t in (0, 5, 77, 127):
            xt = np.ascontiguousarray(xq[t * nb:(t + 1) * nb])
            assert np.array_equal(bits(got[t]), bits(O.matvec(w, x[t:t + 1], xt, 1)[0])), f"t={t}"
    finally:
        backend.release(h)


@pytest.mark.parametrize("gt", [abi.GT_Q4_K, abi.GT_Q6_K])
def test_multi_token_non_panel_groups(backend, gt):
    """Q4_K / Q6_K chunks above 16 tokens run the general matvec over groups of 16."""
    g = synth.rng(gt + 500)
    w = synth.make_weight(g, gt, 300, 2048)
    x = synth.activations(g, 45, 2048)
    out, xq = run_matvec(backend, w, x)
    assert np.array_equal(bits(out), bits(O.matvec(w, x, xq, 45)))


def test_per_op_matmul_128_tokens(backend):
    """matmul() with a 128-token chunk (a host built with MAX_BATCH = 128): panel weights on the
    GEMM, a Q6_K weight of the same group on the general kernel."""
    g = synth.rng(78)
    ws = [synth.make_weight(g, abi.GT_STQ1_0, 512, 1024), synth.make_weight(g, abi.GT_Q2_0C, 256, 1024),
          synth.make_weight(g, abi.GT_Q6_K, 128, 1024)]
    hs = [backend.upload(w) for w in ws]
    try:
        x = synth.activations(g, 128, 1024)
        xq = O.quantize_q8k(x)
        outs = backend.matmul(hs, [w.n for w in ws], xq, 128)
        for w, o in zip(ws, outs):
            assert np.array_equal(bits(o), bits(O.matvec(w, x, xq, 128)))
    finally:
        for h in hs:
            backend.release(h)


def test_per_op_weight_out(backend):
    """weight_out (src/device.h:76): a pinned host buffer per weight; matmul writes it from the
    kernels when the host passes it as the output (src/model.c:662-667), and still copies into any
    other host buffer. Both against the oracle, for a q/k/v-like group at 1, 7 and 16 tokens."""
    g = synth.rng(81)
    ws = [synth.make_weight(g, abi.GT_STQ1_0, 512, 1024), synth.make_weight(g, abi.GT_Q4_K, 256, 1024),
          synth.make_weight(g, abi.GT_Q6_K, 128, 1024)]
    hs = [backend.upload(w) for w in ws]
    try:
        ops = [backend.ops.weight_out(h) for h in hs]
        assert all(ops)
        for nt in (1, 7, 16):
            x = synth.activations(g, nt, 1024)
            xq = O.quantize_q8k(x)
            host = np.zeros((nt, 128), np.float32)  # the third weight's output in a host buffer
            outs = (C.c_void_p * 3)(ops[0], ops[1], host.ctypes.data)
            assert backend.ops.matmul(backend.impl, (C.c_void_p * 3)(*hs), outs, 3, xq.ctypes.data, nt)
            for i, w in enumerate(ws):
                got = host if i == 2 else np.ctypeslib.as_array(
                    C.cast(ops[i], C.POINTER(C.c_float)), shape=(16 * w.n,))[:nt * w.n].reshape(nt, w.n)
                assert np.array_equal(bits(got), bits(O.matvec(w, x, xq, nt))), (i, nt)
        assert backend.ops.weight_out(hs[0]) == ops[0]  # one buffer per weight, kept
    finally:
        for h in hs:
            backend.release(h)


# ----------------------------------------------------------------------------- LM head

@pytest.mark.parametrize("gt,n", [(abi.GT_F16, 120818), (abi.GT_F16, 1000), (abi.GT_F32, 777), (abi.GT_Q8_0, 120818),
                                  (abi.GT_Q8_0, 999)])
def test_head_and_argmax(backend, gt, n):
    import torch
    g = synth.rng(n)
    k = 2048
    w = synth.make_weight(g, gt, n, k, sigma=0.02)
    hvec = synth.activations(g, 1, k)[0]
    nw = g.uniform(0.9, 1.1, k).astype(np.float32)
    eps = 1e-5
    h = backend.upload(w)
    try:
        logits = empty_f32(n)
        key = torch.zeros(1, dtype=torch.int64, device="cuda:0")
        n_arg = n - 3
        assert backend.L.hymt2_hip_head(backend.impl, h, dev(hvec).data_ptr(), dev(nw).data_ptr(), C.c_float(eps),
                                        logits.data_ptr(), n_arg, key.data_ptr()) == 0
        sync()
        got = logits.cpu().numpy()
        xn = O.rmsnorm(hvec, nw, eps)
        ref = O.matvec(w, xn[None, :], None, 1)[0]
        assert np.array_equal(bits(got), bits(ref))
        tok = 0xFFFFFFFF - (int(key.cpu().numpy()[0]) & 0xFFFFFFFF)
        assert tok == int(np.argmax(ref[:n_arg]))
    finally:
        backend.release(h)


def test_argmax_nan_rules(backend):
    """The greedy argmax follows src/model.c:945-948 (best = 0, bv = logits[0], take j only when
    logits[j] > bv): a NaN logit at row 0 wins, a NaN elsewhere never does. Rows of an F32 head
    weight set to NaN give NaN logits at exactly those rows."""
    import torch
    g = synth.rng(4242)
    n, k = 600, 256
    w = synth.make_weight(g, abi.GT_F32, n, k, sigma=0.02)
    hvec = synth.activations(g, 1, k)[0]
    nw = np.ones(k, np.float32)
    for nan_rows, want in (([0], 0), ([5, 77], None)):
        data = w.data.copy().view(np.float32).reshape(n, k)
        data[nan_rows] = np.nan
        wn = synth.Weight(abi.GT_F32, k, n, data.view(np.uint8).reshape(n, 4 * k))
        h = backend.upload(wn)
        try:
            logits = empty_f32(n)
            key = torch.zeros(1, dtype=torch.int64, device="cuda:0")
            assert backend.L.hymt2_hip_head(backend.impl, h, dev(hvec).data_ptr(), dev(nw).data_ptr(),
                                            C.c_float(1e-5), logits.data_ptr(), n, key.data_ptr()) == 0
            sync()
            ref = logits.cpu().numpy()
            assert np.isnan(ref[nan_rows]).all()
            best, bv = 0, ref[0]  # the reference's loop, literally
            for j in range(1, n):
                if ref[j] > bv:
                    best, bv = j, ref[j]
            tok = 0xFFFFFFFF - (int(key.cpu().numpy()[0]) & 0xFFFFFFFF)
            assert tok == best and (want is None or tok == want)
        finally:
            backend.release(h)


# ----------------------------------------------------------------------------- FFN input step

@pytest.mark.parametrize("gt,n,k", [(abi.GT_STQ1_0, 6144, 2048), (abi.GT_Q2_0C, 1536, 1024), (abi.GT_Q4_K, 512, 2048),
                                    (abi.GT_Q6_K, 101, 2048), (abi.GT_STQ1_0, 7, 2048)])
def test_ffn_in_step(backend, gt, n, k):
    """hymt2_hip_ffn_in: RMSNorm -> Q8_K -> gate/up matvecs -> g / (1 + expf(-g)) * u, the decode
    step's fused feed-forward input (src/model.c:870-876), against the oracle's pieces."""
    g = synth.rng(n + k)
    wg, wu = synth.make_weight(g, gt, n, k), synth.make_weight(g, gt, n, k)
    hvec = synth.activations(g, 1, k)[0]
    nw = g.uniform(0.9, 1.1, k).astype(np.float32)
    hg, hu = backend.upload(wg), backend.upload(wu)
    try:
        out = empty_f32(n)
        assert backend.L.hymt2_hip_ffn_in(backend.impl, hg, hu, dev(hvec).data_ptr(), dev(nw).data_ptr(),
                                          C.c_float(1e-5), out.data_ptr()) == 0
        sync()
        xn = O.rmsnorm(hvec, nw, 1e-5)[None, :]
        xq = O.quantize_q8k(xn)
        gate, up = O.matvec(wg, xn, xq, 1)[0], O.matvec(wu, xn, xq, 1)[0]
        ref = (gate / (np.float32(1) + O.expf(-gate)) * up).astype(np.float32)
        assert np.array_equal(bits(out.cpu().numpy()), bits(ref))
    finally:
        backend.release(hg)
        backend.release(hu)


# ----------------------------------------------------------------------------- argument checks

def test_entry_points_reject_bad_arguments(backend):
    L = backend.L
    g = synth.rng(5)
    w = synth.make_weight(g, abi.GT_STQ1_0, 64, 512)
    h = backend.upload(w)
    try:
        act, _ = q8k_dev(backend, synth.activations(g, 1, 512))
        out = empty_f32(64 * 129)
        assert L.hymt2_hip_matvec(backend.impl, h, act.data_ptr(), out.data_ptr(), 0) < 0
        assert L.hymt2_hip_matvec(backend.impl, h, act.data_ptr(), out.data_ptr(), 129) < 0  # > MAX_CHUNK
        assert L.hymt2_hip_quantize_q8k(backend.impl, out.data_ptr(), act.data_ptr(), 300, 1) < 0
        xq = O.quantize_q8k(synth.activations(g, 1, 512))
        ws = (C.c_void_p * 1)(h)
        outs = (C.c_void_p * 1)(np.zeros(64, np.float32).ctypes.data)
        assert not backend.ops.matmul(backend.impl, ws, outs, 1, xq.ctypes.data, 129)
        # an unsupported tensor type (Q4_0, ggml type 2) is refused at upload (NULL), as the
        # reference backend does
        bad = abi.WeightT(w.data.ctypes.data, 2, 512, 64, 512 // 32 * 18, None, None, 0, 0, None)
        assert not backend.ops.upload(backend.impl, C.byref(bad))
        # F16 / Q8_0 weights take fp32 activations in the reference (src/kernels.c:1099-1107,
        # :1279-1289), which the per-op path does not receive: matmul refuses them
        for gt in (abi.GT_F16, abi.GT_Q8_0):
            hw = backend.upload(synth.make_weight(g, gt, 64, 512))
            try:
                assert not backend.ops.matmul(backend.impl, (C.c_void_p * 1)(hw), outs, 1, xq.ctypes.data, 1)
            finally:
                backend.release(hw)
        # the context is still usable afterwards
        backend.matvec(h, act.data_ptr(), out.data_ptr(), 1)
        sync()
    finally:
        backend.release(h)
