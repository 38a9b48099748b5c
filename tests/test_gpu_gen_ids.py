"""The device loop with the reference greedy loop's semantics (hymt2_hip_generate_ids against
gen_ids, src/model.c:914-958): the stop ids end the loop before they are emitted, and the K/V
of the prompt prefix the previous call left is reused (at most n - 1 positions). Compared with
what the reference host computes on the same model (tests/golden/gen_ids.npz, from
make_golden.py --gen-ids) and with the oracle."""
import os

import numpy as np
import pytest

from conftest import GOLDEN
from hymt2_amd import gguf, lib, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu

STOP = [gguf.EOS]  # the words vocabulary's eos; it has no eog token, so eog = eos (src/tokenizer.c:147-149)


def fixture():
    f = np.load(os.path.join(GOLDEN, "gen_ids.npz"), allow_pickle=False)
    model = synth.gen_ids_model()
    assert synth.model_digest(model) == str(f["digest"]), "the generator no longer reproduces the fixture's model"
    return f, model


@pytest.mark.parametrize("chunk", [1, 8, 16])
def test_gen_ids_matches_reference(backend, chunk):
    """The fixture's calls in order on one context: 13 ids and then EOS (the 14th argmax), a
    second prompt sharing 14 positions with the first (64 ids, no stop), the same prompt again
    (n - 1 positions reused), and a run capped at 5 ids. Ids, reused positions and prefilled
    positions equal the reference host's, with the prompt as single-token steps or chunks."""
    f, model = fixture()
    fm = lib.FusedModel(backend, model)
    try:
        for i in range(len(synth.gen_ids_calls())):
            ids, st = fm.generate_ids(f[f"prompt{i}"], int(f[f"max{i}"]), stop_ids=STOP, chunk=chunk,
                                      reuse_prefix=True)
            assert np.array_equal(ids, f[f"ids{i}"]), f"call {i}: {ids.tolist()} != {f[f'ids{i}'].tolist()}"
            assert st.cached_tokens == int(f[f"cached{i}"]), f"call {i}"
            assert st.prefill_steps == int(f[f"prefill{i}"]), f"call {i}"
    finally:
        fm.close()


def test_gen_ids_reuse_equals_cold(backend):
    """A second prompt that shares its first 30 positions with the first prompt's sequence
    (prompt and fed-back ids) gives the same ids reusing them as computed cold; a fused_forward
    in between drops the record (nothing reused); the oracle agrees on both runs."""
    shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1024, heads=4, kv_heads=2, hdim=128, vocab=900, ctx=192)
    model = synth.make_model(shape, mode="q2", seed=301)
    a = synth.rand_prompt(synth.rng(302), 24, shape.vocab)
    om = O.OracleModel(model, threads=8)
    ids_a, keep_a = om.gen_ids(a, 20)
    b = np.concatenate([a, ids_a[:6], synth.rand_prompt(synth.rng(303), 9, shape.vocab)]).astype(np.int32)
    ids_b, keep_b = om.gen_ids(b, 40)
    assert keep_a == 0 and keep_b == 30
    fm = lib.FusedModel(backend, model)
    try:
        got_a, st = fm.generate_ids(a, 20, reuse_prefix=True)
        assert np.array_equal(got_a, ids_a) and st.cached_tokens == 0
        got_b, st = fm.generate_ids(b, 40, chunk=8, reuse_prefix=True)
        assert np.array_equal(got_b, ids_b) and st.cached_tokens == 30 and st.prefill_steps == len(b) - 30
        cold, st = fm.generate_ids(b, 40, chunk=8)
        assert np.array_equal(cold, ids_b) and st.cached_tokens == 0
        fm.generate_ids(a, 20, reuse_prefix=True)
        fm.forward([int(a[0])], 0, True)  # the host path writes K/V: the record is dropped
        again, st = fm.generate_ids(b, 40, reuse_prefix=True)
        assert np.array_equal(again, ids_b) and st.cached_tokens == 0
    finally:
        fm.close()


def test_gen_ids_limits(backend):
    """max_tokens capped at ctx - n (src/model.c:925-926); a prompt that fills the context is an
    error; a stop id that comes up first returns no ids."""
    shape = synth.ModelShape(n_layer=1, hidden=512, ffn=1024, heads=4, kv_heads=2, hdim=128, vocab=700, ctx=48)
    model = synth.make_model(shape, mode="stq", seed=305)
    p = synth.rand_prompt(synth.rng(306), 40, shape.vocab)
    want, _ = O.OracleModel(model, threads=8).gen_ids(p, 100)
    assert len(want) == 8
    fm = lib.FusedModel(backend, model)
    try:
        ids, _ = fm.generate_ids(p, 100)
        assert np.array_equal(ids, want)
        ids, st = fm.generate_ids(p, 100, stop_ids=[int(want[0])])
        assert len(ids) == 0 and st.decode_steps <= 16
        with pytest.raises(RuntimeError):
            fm.generate_ids(synth.rand_prompt(synth.rng(307), 48, shape.vocab), 4)
    finally:
        fm.close()
