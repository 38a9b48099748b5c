"""The oracle against the golden vectors (tests/golden/, written by make_golden.py from the
reference's own C code at the scalar ISA). Bit-exact throughout: int8/int32 records compared
byte for byte, fp32 outputs compared as bit patterns."""
import os

import numpy as np
import pytest

from conftest import GOLDEN
from hymt2_amd import synth
from oracle import oracle as O

TYPES = ("stq1_0", "q2_0c", "q4_k", "q6_k", "f16", "f32", "q8_0")


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def weight_of(f):
    w = synth.Weight(int(f["type"]), int(f["k"]), int(f["n"]), f["data"])
    return w.with_panel()


def test_q8k_golden():
    f = load("q8k")
    got = O.quantize_q8k(f["x"]).view(np.uint8)
    assert np.array_equal(got, f["q8k"])


@pytest.mark.parametrize("name", ["stq1_0", "q2_0c"])
def test_panel_golden(name):
    f = load("panel_" + name)
    w = synth.Weight(int(f["type"]), int(f["k"]), int(f["n"]), f["data"])
    pk, ps = O.panel_repack(w)
    assert np.array_equal(pk, f["pk"]) and np.array_equal(bits(ps), bits(f["ps"]))
    # the package's own numpy repack (used to build device panels) agrees too
    w.with_panel()
    assert np.array_equal(w.pk, f["pk"]) and np.array_equal(bits(w.ps), bits(f["ps"]))


@pytest.mark.parametrize("name", TYPES)
def test_matvec_golden(name):
    f = load("matvec_" + name)
    w = weight_of(f)
    xq = O.quantize_q8k(f["x"])
    assert np.array_equal(xq.view(np.uint8), f["q8k"])
    out = O.matvec(w, f["x"], xq, int(f["nt"]))
    assert np.array_equal(bits(out), bits(f["out"]))
    deq = O.dequant(synth.Weight(w.type, w.k, 4, w.data[:4]))
    assert np.array_equal(bits(deq), bits(f["dequant4"]))


def test_bf16_golden():
    f = load("bf16")
    L = O.lib()
    q, kv = np.ascontiguousarray(f["q"]), np.ascontiguousarray(f["kv"])
    assert bits(L.oc_dot_bf16(q.ctypes.data, kv.ctypes.data, len(q))) == bits(f["dot"])
    o = f["o"].copy()
    L.oc_axpy_bf16(o.ctypes.data, kv.ctypes.data, float(f["p"]), len(o))
    assert np.array_equal(bits(o), bits(f["axpy"]))
    got = np.array([L.oc_f32_to_bf16(float(v)) for v in f["vals"]], dtype=np.uint16)
    assert np.array_equal(got, f["to_bf16"])


def golden_model(mode):
    f = load("model_" + mode)
    shape = synth.ModelShape(**{k[6:]: int(f[k]) for k in f.files if k.startswith("shape_")})
    model = synth.make_model(shape, mode=str(f["mode"]), seed=int(f["seed"]))
    assert synth.model_digest(model) == str(f["digest"]), "the generator no longer reproduces the golden model"
    return f, model


@pytest.mark.parametrize("mode", ["stq", "q2", "q4km"])
def test_model_golden(mode):
    f, model = golden_model(mode)
    prompt = f["prompt"]
    om = O.OracleModel(model, threads=4)
    logits = None
    for i in range(0, len(prompt), 8):  # the reference's scalar-ISA prefill chunk (src/model.c:619)
        nt = min(8, len(prompt) - i)
        logits = om.forward(prompt[i:i + nt], i, want_logits=(i + nt == len(prompt)))
    assert np.array_equal(bits(logits), bits(f["logits"]))
    ids = O.OracleModel(model, threads=4).generate(prompt, len(f["greedy"]), batch=8)
    assert np.array_equal(ids, f["greedy"])


def test_baseline_config3_oracle():
    """The oracle at full size against the reference's scalar-ISA greedy loop on BASELINE config
    3 (tests/golden/baseline_config3.npz): the 1.8B-shaped STQ1_0 model, 64 chat-template prompt
    ids; the logits at the end of the prompt (sha256 of the bits) and the first greedy ids."""
    import hashlib
    f = load("baseline_config3")
    model = synth.baseline_model(synth.CONFIG3, int(f["ctx"]))
    assert synth.model_digest(model) == str(f["digest"]), "the generator no longer reproduces the fixture's model"
    prompt = f["prompt"]
    om = O.OracleModel(model, threads=8)
    logits = None
    for i in range(0, len(prompt), 8):
        nt = min(8, len(prompt) - i)
        logits = om.forward(prompt[i:i + nt], i, want_logits=(i + nt == len(prompt)))
    assert hashlib.sha256(bits(logits).tobytes()).hexdigest() == str(f["prompt_logits_sha256"])
    ids = O.OracleModel(model, threads=8).generate(prompt, 4, batch=8)
    assert np.array_equal(ids, f["greedy"][:4])


def test_gen_ids_golden():
    """The oracle's gen_ids (src/model.c:914-958 from the prompt ids on) against the reference's
    own loop on the EOS-ending model: the calls in order on one state, each reusing the cache the
    one before it left; ids before the stop id and the reused prefix length, call by call. A
    mutant that feeds or emits the stop id, drops the n - 1 bound on the reuse, or feeds the last
    id of a full run fails one of the calls (13 ids then EOS; 14 positions reused; n - 1 reused;
    a run capped at 5)."""
    f = load("gen_ids")
    model = synth.gen_ids_model()
    assert synth.model_digest(model) == str(f["digest"])
    om = O.OracleModel(model, threads=8)
    for i in range(len(synth.gen_ids_calls())):
        ids, keep = om.gen_ids(f[f"prompt{i}"], int(f[f"max{i}"]), stop_ids=[2])
        assert np.array_equal(ids, f[f"ids{i}"]), f"call {i}"
        assert keep == int(f[f"cached{i}"]), f"call {i}: reused {keep}, the reference {int(f[f'cached{i}'])}"
        assert len(f[f"prompt{i}"]) - keep == int(f[f"prefill{i}"])
