"""Shapes the reference's CPU path takes that leave the backend's fast kernels for its general ones,
against the oracle, bit for bit (src/model.c:767-795, :857-876, :887-900):

* chunk attention at head dim 256 (k_attention<4>: the per-(KV head, token) chunk kernel takes
  head dims 64 and 128 only);
* chunk attention at head dim 64 past 2048 positions (k_attention<1>: the chunk kernel's rows
  end at 2048);
* gate and up weights of different types (Q4_K gate, Q6_K up), so the two matvecs cannot share
  row tiles and the SwiGLU runs as its own kernel (k_silu_mul), in the single-token step and in
  chunks;
* a quantized (Q6_K / Q4_K) LM head at hidden 1024: the decode matvec with the argmax epilogue
  takes K = 2048 and 6144 only, so the head runs on the general matvec with the RMSNorm + Q8_K
  prologue and a separate argmax kernel (k_argmax over the logits).

Each test compares the logits of the reference host's boundary (fused_forward per chunk) and the
device loop's greedy ids with the oracle's."""
import numpy as np
import pytest

from hymt2_amd import abi, lib, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def oracle_logits(model, prompt, batch=16):
    om = O.OracleModel(model, threads=16)
    ref = None
    for i in range(0, len(prompt), batch):
        c = prompt[i:i + batch]
        ref = om.forward(c, i, want_logits=(i + len(c) == len(prompt)))
    return ref


def check_model(backend, model, prompt, n_gen, batches, chunks):
    ref = oracle_logits(model, prompt)
    want = O.OracleModel(model, threads=16).generate(prompt, n_gen, batch=16)
    fm = lib.FusedModel(backend, model)
    try:
        for batch in batches:
            assert np.array_equal(bits(fm.prefill(list(prompt), batch=batch)), bits(ref)), f"batch={batch}"
        for chunk in chunks:
            ids, _ = fm.generate_device(prompt, n_gen, chunk=chunk)
            assert np.array_equal(ids, want), f"chunk={chunk}: first difference at {np.argmax(ids != want)}"
        assert np.array_equal(fm.generate_host(prompt, 4, batch=16), want[:4])
    finally:
        fm.close()


def test_chunk_attention_head_dim_256(backend):
    """Head dim 256, two query heads per KV head: a 150-token prompt in chunks of 16 (the general
    matvec) and 128 (the panel GEMM), each chunk's attention by k_attention<4>; 12 greedy ids
    with the prompt in chunks of 8 and 128 and one position at a time."""
    shape = synth.ModelShape(n_layer=2, hidden=1024, ffn=2048, heads=4, kv_heads=2, hdim=256, vocab=800, ctx=192)
    model = synth.make_model(shape, mode="q2", seed=91)
    prompt = synth.rand_prompt(synth.rng(92), 150, shape.vocab)
    check_model(backend, model, prompt, 12, batches=(16, 128), chunks=(8, 128, 1))


def test_chunk_attention_head_dim_64_past_2048(backend):
    """Head dim 64 at context 2304, four query heads per KV head: a 2200-token prompt in
    128-token chunks, every chunk's attention by k_attention<1> (rows up to 2200 positions; the
    second layer's keys and values depend on the first layer's attention at every position), the
    last logits bit for bit, then 8 greedy ids."""
    shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1024, heads=8, kv_heads=2, hdim=64, vocab=500, ctx=2304)
    model = synth.make_model(shape, mode="stq", seed=93)
    prompt = synth.rand_prompt(synth.rng(94), 2200, shape.vocab)
    check_model(backend, model, prompt, 8, batches=(128,), chunks=(128,))


@pytest.mark.parametrize("hidden", [2048, 512])
def test_unpaired_gate_up(backend, hidden):
    """Q4_K gate with a Q6_K up (the reference's Q4_K_M mix of q/k/o/gate in Q4_K and v/down in
    Q6_K, with up moved to Q6_K): the gate and up matvecs run as two jobs and the SwiGLU
    g = g / (1 + expf(-g)) * u as k_silu_mul, after the single-token matvec (hidden 2048: the
    decode kernel; 512: the general one) and after chunks of 16 and 5; 12 greedy ids."""
    shape = synth.ModelShape(n_layer=1, hidden=hidden, ffn=3 * hidden, heads=hidden // 128, kv_heads=hidden // 512,
                             hdim=128, vocab=1000, ctx=64)
    model = synth.make_model(shape, mode="q4km", seed=95 + hidden)
    g = synth.rng(96 + hidden)
    for L in model["layers"]:
        assert L["wg"].type == abi.GT_Q4_K
        L["wu"] = synth.make_weight(g, abi.GT_Q6_K, shape.ffn, shape.hidden)
    prompt = synth.rand_prompt(synth.rng(97), 21, shape.vocab)
    check_model(backend, model, prompt, 12, batches=(16, 5, 1), chunks=(1, 8))


@pytest.mark.parametrize("head", [abi.GT_Q6_K, abi.GT_Q4_K])
def test_quantized_head_hidden_1024(backend, head):
    """Tied Q6_K / Q4_K embedding and LM head at hidden 1024: the head on the general matvec
    (RMSNorm + Q8_K prologue) and the greedy argmax by k_argmax over the logits; the device loop
    dequantizes the embedding rows at hidden 1024. Logits after chunks of 16 and one position at
    a time, and 12 greedy ids."""
    shape = synth.ModelShape(n_layer=1, hidden=1024, ffn=2048, heads=8, kv_heads=2, hdim=128, vocab=1000, ctx=64)
    model = synth.make_model(shape, mode="stq", seed=98 + head, head_type=head)
    prompt = synth.rand_prompt(synth.rng(99), 21, shape.vocab)
    check_model(backend, model, prompt, 12, batches=(16, 1), chunks=(1, 8))
