"""The fused token loop on the GPU against the golden vectors and the oracle, bit for bit.

Each model runs through the backend's hy_device_ops vtable exactly as the reference host
drives it (upload, fused_prepare, fused_forward per chunk of <= 16 tokens with the host
embedding; src/model.c:384-406, :325-381, :798-909), and through the device-resident greedy
loop (hymt2_hip_generate / gen_begin / gen_steps). Logits are compared as bit patterns and
greedy ids exactly."""
import ctypes
import os

import numpy as np
import pytest

from conftest import GOLDEN
from hymt2_amd import abi, lib, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def golden_model(mode):
    f = np.load(os.path.join(GOLDEN, f"model_{mode}.npz"), allow_pickle=False)
    shape = synth.ModelShape(**{k[6:]: int(f[k]) for k in f.files if k.startswith("shape_")})
    model = synth.make_model(shape, mode=str(f["mode"]), seed=int(f["seed"]))
    assert synth.model_digest(model) == str(f["digest"])
    return f, model


@pytest.mark.parametrize("mode", ["stq", "q2", "q4km"])
def test_golden_models(backend, mode):
    f, model = golden_model(mode)
    fm = lib.FusedModel(backend, model)
    try:
        prompt = f["prompt"]
        lg = fm.prefill(list(prompt), batch=8)  # the reference's scalar-ISA chunking
        assert np.array_equal(bits(lg), bits(f["logits"]))
        n = len(f["greedy"])
        assert np.array_equal(fm.generate_host(prompt, n, batch=8), f["greedy"])
        ids, st = fm.generate_device(prompt, n)
        assert np.array_equal(ids, f["greedy"])
        assert st.prefill_steps == len(prompt) and st.decode_steps == n - 1
    finally:
        fm.close()


SHAPE = synth.ModelShape(n_layer=3, hidden=512, ffn=1536, heads=8, kv_heads=2, hdim=64, vocab=900, ctx=320)


@pytest.mark.parametrize("mode", ["stq", "q2", "q4km"])
def test_chunking_and_prefix_reuse(backend, mode):
    """Chunks of 16, 5 and 1 tokens all give the oracle's logits; re-running a suffix over a warm
    cache (positions overwritten) equals a cold run (tests/test_model.py:369-374, :394-399)."""
    model = synth.make_model(SHAPE, mode=mode, seed=41)
    prompt = synth.rand_prompt(synth.rng(42), 37, SHAPE.vocab)
    om = O.OracleModel(model, threads=8)
    ref = None
    for i in range(0, len(prompt), 16):
        c = prompt[i:i + 16]
        ref = om.forward(c, i, want_logits=(i + len(c) == len(prompt)))
    fm = lib.FusedModel(backend, model)
    try:
        for batch in (16, 5, 1):
            assert np.array_equal(bits(fm.prefill(list(prompt), batch=batch)), bits(ref)), f"batch={batch}"
        fm.forward([1, 2, 3, 4], 30, False)           # scribble over positions 30..33
        lg = fm.forward(list(prompt[30:]), 30, True)  # then recompute them from the warm prefix
        assert np.array_equal(bits(lg), bits(ref))
    finally:
        fm.close()


@pytest.mark.parametrize("mode", ["stq", "q2", "q4km"])
def test_chunked_prefill_vs_oracle(backend, mode):
    """Prompt chunks above the reference's 16-token batch (128, and ragged 100 / 33): panel
    weights on the int8-MFMA GEMM (Q4_K / Q6_K on the general kernel in groups of 16), causal
    attention over the growing KV cache. The last prompt position's logits through
    fused_forward, and the device loop's greedy ids after gen_prefill, vs the oracle."""
    model = synth.make_model(SHAPE, mode=mode, seed=51)
    prompt = synth.rand_prompt(synth.rng(52), 290, SHAPE.vocab)
    om = O.OracleModel(model, threads=8)
    ref = None
    for i in range(0, len(prompt), 16):
        c = prompt[i:i + 16]
        ref = om.forward(c, i, want_logits=(i + len(c) == len(prompt)))
    want = O.OracleModel(model, threads=8).generate(prompt, 24, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        for batch in (128, 100):
            assert np.array_equal(bits(fm.prefill(list(prompt), batch=batch)), bits(ref)), f"batch={batch}"
        for chunk in (128, 33):
            ids, st = fm.generate_device(prompt, 24, chunk=chunk)
            assert np.array_equal(ids, want), f"chunk={chunk}"
            assert st.prefill_steps == len(prompt) and st.decode_steps == 23
        # the step API: prefill, then steps in pieces
        fm.gen_begin(prompt, len(prompt) + 10)
        fm.gen_prefill(128)
        fm.gen_steps(4)
        fm.gen_steps(5)
        assert np.array_equal(fm.gen_read(len(prompt), 10), want[:10])
        with pytest.raises(RuntimeError):
            fm.gen_prefill(128)  # only on a fresh loop
    finally:
        fm.close()


@pytest.mark.parametrize("mode", ["stq", "q4km"])
def test_long_greedy_device_vs_oracle(backend, mode):
    """A 300-position greedy run (attention past several 64-key tiles; softmax over > 256 keys)."""
    model = synth.make_model(SHAPE, mode=mode, seed=43)
    prompt = synth.rand_prompt(synth.rng(44), 40, SHAPE.vocab)
    n_gen = SHAPE.ctx - len(prompt)
    want = O.OracleModel(model, threads=8).generate(prompt, n_gen, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        ids, _ = fm.generate_device(prompt, n_gen)
        assert np.array_equal(ids, want)
        # the step API: begin, steps in pieces, read back
        fm.gen_begin(prompt, len(prompt) + 20)
        fm.gen_steps(len(prompt))
        fm.gen_steps(19)
        assert np.array_equal(fm.gen_read(len(prompt), 20), want[:20])
    finally:
        fm.close()


@pytest.mark.parametrize("mode", ["stq", "q2", "q4km"])
def test_hidden2048_models(backend, mode):
    """Two layers at the 1.8B layer shapes (hidden 2048, ffn 6144, 16/4 heads, hd 128): the
    single-token steps run the decode matvec kernel (K = 2048 and 6144); logits of a one-token
    forward after a prefill, and 20 device greedy ids, vs the oracle."""
    shape = synth.ModelShape(n_layer=2, vocab=1000, ctx=96)
    model = synth.make_model(shape, mode=mode, seed=47)
    prompt = synth.rand_prompt(synth.rng(48), 9, shape.vocab)
    om = O.OracleModel(model, threads=8)
    om.forward(prompt[:8], 0, False)
    ref = om.forward(prompt[8:], 8, True)
    fm = lib.FusedModel(backend, model)
    try:
        fm.forward(list(prompt[:8]), 0, False)
        assert np.array_equal(bits(fm.forward([int(prompt[8])], 8, True)), bits(ref))
        want = O.OracleModel(model, threads=8).generate(prompt, 20, batch=16)
        ids, _ = fm.generate_device(prompt, 20)
        assert np.array_equal(ids, want)
    finally:
        fm.close()


@pytest.mark.parametrize("mode", ["stq", "q2"])
def test_hidden2048_chunked_prefill(backend, mode):
    """Chunked prefill at the 1.8B layer shapes: a 150-token prompt as chunks of 128 + 22, both
    above the 16-token batch, so every qkv / o / gate-up / down contraction runs on the GEMM."""
    shape = synth.ModelShape(n_layer=2, vocab=1000, ctx=192)
    model = synth.make_model(shape, mode=mode, seed=53)
    prompt = synth.rand_prompt(synth.rng(54), 150, shape.vocab)
    om = O.OracleModel(model, threads=8)
    ref = None
    for i in range(0, len(prompt), 16):
        c = prompt[i:i + 16]
        ref = om.forward(c, i, want_logits=(i + len(c) == len(prompt)))
    want = O.OracleModel(model, threads=8).generate(prompt, 12, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        assert np.array_equal(bits(fm.prefill(list(prompt), batch=128)), bits(ref))
        ids, _ = fm.generate_device(prompt, 12, chunk=128)
        assert np.array_equal(ids, want)
    finally:
        fm.close()


def test_hidden2048_long_context_decode(backend):
    """The single-token attention at hd 128 over long rows: one layer at the 1.8B shapes, a
    640-token prompt fed one token at a time (every position through the decode attention: up
    to 7 product tiles of 96 positions, the exact segmented softmax sum past 256 keys), the last
    logits vs the oracle bit for bit, then 40 device greedy ids (rows up to 680)."""
    shape = synth.ModelShape(n_layer=1, vocab=1000, ctx=700)
    model = synth.make_model(shape, mode="stq", seed=59)
    prompt = synth.rand_prompt(synth.rng(60), 640, shape.vocab)
    om = O.OracleModel(model, threads=16)
    ref = None
    for i in range(0, len(prompt), 16):
        c = prompt[i:i + 16]
        ref = om.forward(c, i, want_logits=(i + len(c) == len(prompt)))
    want = O.OracleModel(model, threads=16).generate(prompt, 40, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        assert np.array_equal(bits(fm.prefill(list(prompt), batch=1)), bits(ref))
        ids, _ = fm.generate_device(prompt, 40)
        assert np.array_equal(ids, want)
    finally:
        fm.close()


@pytest.mark.parametrize("head", [abi.GT_Q6_K, abi.GT_Q4_K, abi.GT_Q8_0, abi.GT_F32])
def test_tied_head_types(backend, head):
    """Tied embedding / LM head of the other types the reference reads: Q6_K is the head of its own
    bench and test models (tools/make_bench_gguf.c:30, tests/test_model.py:216-222) and the only
    head its CUDA backend uploads (src/cuda.c:209-212). Q6_K / Q4_K heads run on the quantized
    matvec with the RMSNorm + Q8_K prologue and a separate argmax; Q8_0 / F32 on the fp32-activation
    LM head kernel. The device loop dequantizes the embedding rows itself (dequant_row,
    src/kernels.c:1304-1329). Two layers at the 1.8B layer shapes; logits after a chunked prefill
    and after a single-token step, and 20 greedy ids of the device loop (single-token and
    chunked prompt), against the oracle."""
    shape = synth.ModelShape(n_layer=2, vocab=1000, ctx=96)
    model = synth.make_model(shape, mode="stq", seed=61 + head, head_type=head)
    prompt = synth.rand_prompt(synth.rng(62), 21, shape.vocab)
    om = O.OracleModel(model, threads=8)
    om.forward(prompt[:16], 0, False)
    ref = om.forward(prompt[16:20], 16, True)
    ref1 = om.forward(prompt[20:], 20, True)
    want = O.OracleModel(model, threads=8).generate(prompt, 20, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        assert np.array_equal(bits(fm.prefill(list(prompt[:20]), batch=16)), bits(ref))
        assert np.array_equal(bits(fm.forward([int(prompt[20])], 20, True)), bits(ref1))
        for chunk in (1, 8):
            ids, _ = fm.generate_device(prompt, 20, chunk=chunk)
            assert np.array_equal(ids, want), f"chunk={chunk}"
        assert np.array_equal(fm.generate_host(prompt, 6, batch=16), want[:6])
    finally:
        fm.close()


def test_full_vocab_q6k_head(backend):
    """A Q6_K tied embedding / head at the full vocabulary (120818 x 2048, 203 MB), one layer:
    logits of a prefill and 6 greedy ids of the device loop against the oracle."""
    shape = synth.ModelShape(n_layer=1, ctx=64)
    model = synth.make_model(shape, mode="stq", seed=65, head_type=abi.GT_Q6_K)
    prompt = synth.rand_prompt(synth.rng(66), 10, shape.vocab)
    om = O.OracleModel(model, threads=16)
    ref = om.forward(prompt, 0, True)
    want = O.OracleModel(model, threads=16).generate(prompt, 6, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        assert np.array_equal(bits(fm.forward(list(prompt), 0, True)), bits(ref))
        ids, _ = fm.generate_device(prompt, 6)
        assert np.array_equal(ids, want)
    finally:
        fm.close()


def test_generate_rejects_overlong_runs(backend):
    model = synth.make_model(synth.ModelShape(n_layer=1, hidden=256, ffn=512, heads=2, kv_heads=1, hdim=128,
                                              vocab=300, ctx=64), mode="stq", seed=45)
    fm = lib.FusedModel(backend, model)
    try:
        prompt = synth.rand_prompt(synth.rng(46), 10, 300)
        with pytest.raises(RuntimeError):
            fm.gen_begin(prompt, 65)      # more positions than ctx
        fm.gen_begin(prompt, 12)
        fm.gen_steps(11)
        with pytest.raises(RuntimeError):
            fm.gen_steps(1)               # past n_total - 1 steps
        a = fm.args
        a.nt, a.pos0, a.want_logits, a.h, a.logits = 129, 0, 1, fm.h.ctypes.data, fm.logits.ctypes.data
        assert not fm.b.ops.fused_forward(fm.b.impl, ctypes.byref(a))  # nt > HYMT2_HIP_MAX_CHUNK
        a.nt, a.pos0 = 2, 63
        assert not fm.b.ops.fused_forward(fm.b.impl, ctypes.byref(a))  # past ctx
        # still usable
        ids, _ = fm.generate_device(prompt, 5)
        assert np.array_equal(ids, O.OracleModel(model, threads=4).generate(prompt, 5, batch=16))
    finally:
        fm.close()


@pytest.mark.parametrize("mode", ["stq", "q2"])
def test_full_size_model_short_run(backend, mode):
    """Hy-MT2-1.8B shapes (BASELINE configs 3 and 4): 32 layers, hidden 2048, ffn 6144, 16/4 heads,
    vocab 120818, tied F16 head. 12 prompt ids then 4 greedy ids, logits and ids vs the oracle."""
    shape = synth.ModelShape(ctx=64)
    model = synth.make_model(shape, mode=mode, seed=3)
    prompt = synth.rand_prompt(synth.rng(1234), 12, shape.vocab)
    om = O.OracleModel(model, threads=16)
    ref = om.forward(prompt, 0, True)
    fm = lib.FusedModel(backend, model)
    try:
        assert np.array_equal(bits(fm.forward(list(prompt), 0, True)), bits(ref))
        want = O.OracleModel(model, threads=16).generate(prompt, 4, batch=16)
        ids, _ = fm.generate_device(prompt, 4)
        assert np.array_equal(ids, want)
    finally:
        fm.close()


@pytest.mark.parametrize("mode,heads,kv_heads,hdim", [("q2", 16, 4, 128), ("stq", 16, 4, 128),
                                                      ("q2", 16, 8, 128), ("stq", 32, 8, 64)])
def test_pipelined_prefill_matches_sequential(backend, mode, heads, kv_heads, hdim):
    """The device loop's chunked prefill pipelined over the layers (up to 8 chunks in flight,
    chunk i's layer l in the same launches as chunk i + 1's layer l - 1) against one chunk after
    another and the oracle: a 300-token prompt in chunks of 33 (ten chunks, the last of 3
    tokens), so the default depth runs a group of eight and a group of two, and depth 3 four
    groups. At every depth the 10 greedy ids equal the oracle's, and so do the logits of a
    fused_forward at position 310 after them, bit for bit: that forward reads every layer's K/V
    of all 310 earlier positions, which the pipelined launches wrote for the prompt. Query
    heads per KV head and head dims 4 x 128, 2 x 128 and 4 x 64 run the three pipelined
    attention kernels k_attn_chunk_pipe<128, 4>, <128, 2> and <64, 4>."""
    shape = synth.ModelShape(n_layer=3, heads=heads, kv_heads=kv_heads, hdim=hdim, vocab=1000, ctx=320)
    model = synth.make_model(shape, mode=mode, seed=59)
    prompt = synth.rand_prompt(synth.rng(60), 300, shape.vocab)
    want = O.OracleModel(model, threads=8).generate(prompt, 10, batch=16)
    om = O.OracleModel(model, threads=8)
    for i in range(0, len(prompt), 16):
        om.forward(prompt[i:i + 16], i, want_logits=False)
    ref = om.forward(want, len(prompt), want_logits=True)
    fm = lib.FusedModel(backend, model)
    try:
        for depth in (8, 3, 1):
            prev = backend.prefill_pipeline(depth)
            try:
                ids, _ = fm.generate_device(prompt, 10, chunk=33)
            finally:
                backend.prefill_pipeline(prev)
            assert np.array_equal(ids, want), f"depth={depth}"
            assert np.array_equal(bits(fm.forward([int(ids[-1])], 309, True)), bits(ref)), f"depth={depth}"
        assert backend.prefill_pipeline(0) == 8
    finally:
        fm.close()


def test_full_size_chunked_prefill_config4(backend):
    """BASELINE config 4 at full size: the 1.8B Q2_0C model, a 1024-token prompt in 128-token
    chunks. The last position's logits equal those of a token-by-token prefill (single-token
    decode kernels, pinned to the oracle at this size by test_full_size_model_short_run), bit for
    bit, and the device loop's greedy ids after the chunked prefill equal those after 1024
    single-token steps (batched == stepwise, tests/test_model.py:369-374)."""
    shape = synth.ModelShape(ctx=1040)
    model = synth.make_model(shape, mode="q2", seed=4)
    prompt = synth.rand_prompt(synth.rng(4096), 1024, shape.vocab)
    fm = lib.FusedModel(backend, model)
    try:
        chunked = fm.prefill(list(prompt), batch=128)
        stepwise = fm.prefill(list(prompt), batch=1)
        assert np.array_equal(bits(chunked), bits(stepwise))
        a, _ = fm.generate_device(prompt, 8, chunk=128)
        b, _ = fm.generate_device(prompt, 8, chunk=1)
        assert np.array_equal(a, b)
        assert a[0] == int(np.argmax(stepwise[:fm.vocab_out]))
    finally:
        fm.close()


def _stepwise_logits(om, prompt):
    """The oracle's logits after the prompt, fed 16 positions at a time."""
    ref = None
    for i in range(0, len(prompt), 16):
        c = prompt[i:i + 16]
        ref = om.forward(c, i, want_logits=(i + len(c) == len(prompt)))
    return ref


@pytest.mark.parametrize("hd", [128, 64])
def test_split_attention_matches_one_kernel(backend, hd):
    """The split single-token attention (scores over many workgroups, then softmax and output)
    against the one-workgroup-per-head kernel and the oracle: two layers (the second layer's keys
    and values depend on the first layer's attention at every position, so the last logits cover
    all of them), a 600-token prompt fed one position at a time with the split form forced from
    position 0, then from 10**9 (never), last logits bit for bit equal to the oracle's; then 30
    device greedy ids (positions 600-629) under each form, equal to the oracle's."""
    if hd == 128:
        shape = synth.ModelShape(n_layer=2, vocab=1000, ctx=640)
    else:
        shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1536, heads=8, kv_heads=2, hdim=64, vocab=900, ctx=640)
    model = synth.make_model(shape, mode="stq", seed=71 + hd)
    prompt = synth.rand_prompt(synth.rng(72), 600, shape.vocab)
    ref = _stepwise_logits(O.OracleModel(model, threads=16), prompt)
    want = O.OracleModel(model, threads=16).generate(prompt, 30, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        for split_from in (0, 10 ** 9):
            backend.attn_split_from(split_from)
            assert np.array_equal(bits(fm.prefill(list(prompt), batch=1)), bits(ref)), f"split_from={split_from}"
            ids, _ = fm.generate_device(prompt, 30)
            assert np.array_equal(ids, want), f"split_from={split_from}"
    finally:
        backend.attn_split_from(-1)
        fm.close()


def test_split_attention_head_dim_256(backend):
    """Head dim 256 (the one-kernel form takes 64 and 128 only, so every single-token step runs
    the split form): a 150-token prompt one position at a time, logits and 20 greedy ids vs the
    oracle."""
    shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1024, heads=2, kv_heads=1, hdim=256, vocab=700, ctx=192)
    model = synth.make_model(shape, mode="q4km", seed=77)
    prompt = synth.rand_prompt(synth.rng(78), 150, shape.vocab)
    ref = _stepwise_logits(O.OracleModel(model, threads=16), prompt)
    want = O.OracleModel(model, threads=16).generate(prompt, 20, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        assert np.array_equal(bits(fm.prefill(list(prompt), batch=1)), bits(ref))
        ids, _ = fm.generate_device(prompt, 20)
        assert np.array_equal(ids, want)
    finally:
        fm.close()


@pytest.mark.parametrize("kv_heads", [1, 2])
def test_chunk_attention_long_rows(backend, kv_heads):
    """Chunk attention at head dim 128 over rows of up to 1500 positions, 4 or 2 query heads per
    KV head: each row's softmax sum by the 16-lane row chain in rounds of 512 positions (one to
    three rounds here), the running sum carried from one round into the next. The last logits of
    a 1500-token prompt in 128-token chunks and 16 device greedy ids after it, against the
    oracle."""
    shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1024, heads=4, kv_heads=kv_heads, hdim=128, vocab=600, ctx=1536)
    model = synth.make_model(shape, mode="q2", seed=83 + kv_heads)
    prompt = synth.rand_prompt(synth.rng(85 + kv_heads), 1500, shape.vocab)
    om = O.OracleModel(model, threads=16)
    ref = _stepwise_logits(om, prompt)
    want = O.OracleModel(model, threads=16).generate(prompt, 16, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        assert np.array_equal(bits(fm.prefill(list(prompt), batch=128)), bits(ref))
        ids, _ = fm.generate_device(prompt, 16, chunk=128)
        assert np.array_equal(ids, want)
    finally:
        fm.close()


def test_four_token_attention_one_chunk(backend):
    """The four-token chunk attention (k_attn_chunk4_pipe) through the one-chunk launch: 8 KV
    heads of 4 query heads at head dim 128, so a 128-token chunk is 32 groups x 8 KV heads = 256
    workgroups, the least that takes that kernel (the 44-token last chunk, 88, takes the
    per-token one). A 300-token prompt through fused_forward in chunks of 128, 128 and 44: the
    last logits against the oracle's bit for bit; then the device loop's chunked prefill (its
    pipelined launches, every step on the four-token kernel) and 8 greedy ids against the
    oracle's."""
    shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1024, heads=32, kv_heads=8, hdim=128, vocab=600, ctx=320)
    model = synth.make_model(shape, mode="q2", seed=91)
    prompt = synth.rand_prompt(synth.rng(92), 300, shape.vocab)
    om = O.OracleModel(model, threads=8)
    ref = _stepwise_logits(om, prompt)
    want = O.OracleModel(model, threads=8).generate(prompt, 8, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        assert np.array_equal(bits(fm.prefill(list(prompt), batch=128)), bits(ref))
        ids, _ = fm.generate_device(prompt, 8, chunk=128)
        assert np.array_equal(ids, want)
    finally:
        fm.close()


def test_four_token_attention_unaligned_long_rows(backend):
    """The four-token chunk attention over long rows at unaligned positions: a 1000-token prompt
    in chunks of 99 (ten full chunks and one of 10; every chunk after the first starts at a
    position that is not a multiple of 4 and ends in a 3-token group), pipelined, rows up to 1000
    positions. The 8 greedy ids, and the logits of a fused_forward of those ids at positions
    1000-1007 (reading every layer's K/V of the prompt, which layer 0's attention output shapes
    from layer 1 on), against the oracle's."""
    shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1024, heads=16, kv_heads=4, hdim=128, vocab=600, ctx=1040)
    model = synth.make_model(shape, mode="stq", seed=95)
    prompt = synth.rand_prompt(synth.rng(96), 1000, shape.vocab)
    want = O.OracleModel(model, threads=16).generate(prompt, 8, batch=16)
    om = O.OracleModel(model, threads=16)
    for i in range(0, len(prompt), 16):
        om.forward(prompt[i:i + 16], i, want_logits=False)
    ref = om.forward(want, len(prompt), want_logits=True)
    fm = lib.FusedModel(backend, model)
    try:
        ids, _ = fm.generate_device(prompt, 8, chunk=99)
        assert np.array_equal(ids, want)
        got = fm.forward(list(ids), len(prompt), True)
        assert np.array_equal(bits(got), bits(ref))
    finally:
        fm.close()


def test_long_context_beyond_4096(backend):
    """Context 4400 (past the one-kernel form's 4096 and the chunk kernel's 2048): two layers, a
    4150-token prompt in 128-token chunks (the general chunk attention, rows up to 4150), the last
    logits vs the oracle bit for bit; then single-token forwards at positions 4150 and 4151 (the
    split form's softmax sum in two chunks, the second continuing the first's running sum), logits
    vs the oracle; then 40 device greedy ids after the chunked prompt vs the oracle."""
    shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1024, heads=4, kv_heads=2, hdim=128, vocab=600, ctx=4400)
    model = synth.make_model(shape, mode="stq", seed=79)
    prompt = synth.rand_prompt(synth.rng(80), 4150, shape.vocab)
    om = O.OracleModel(model, threads=16)
    ref = _stepwise_logits(om, prompt)
    extra = [int(t) for t in synth.rand_prompt(synth.rng(81), 2, shape.vocab)]
    ref1 = om.forward(extra[:1], 4150, True)
    ref2 = om.forward(extra[1:], 4151, True)
    want = O.OracleModel(model, threads=16).generate(prompt, 40, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        assert np.array_equal(bits(fm.prefill(list(prompt), batch=128)), bits(ref))
        assert np.array_equal(bits(fm.forward(extra[:1], 4150, True)), bits(ref1))
        assert np.array_equal(bits(fm.forward(extra[1:], 4151, True)), bits(ref2))
        ids, _ = fm.generate_device(prompt, 40, chunk=128)
        assert np.array_equal(ids, want)
    finally:
        fm.close()
