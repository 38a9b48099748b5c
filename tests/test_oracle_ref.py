"""The oracle (oracle/hymt2_oracle.c) against the reference itself, compiled from its sources
into oracle/_ref/ (oracle/Makefile) and run at its scalar ISA. Seeded random inputs over more
shapes than the golden vectors hold; bit-exact. Skipped where the reference tree was not
available to build _ref/."""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from hymt2_amd import abi, gguf, synth
from oracle import oracle as O

KINDS = [abi.GT_STQ1_0, abi.GT_Q2_0C, abi.GT_Q4_K, abi.GT_Q6_K, abi.GT_F16, abi.GT_F32, abi.GT_Q8_0]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_reference_kernel_selftest(ref):
    """The reference's own kernel test (tests/test_kernels.c) passes on this build."""
    exe = os.path.join(ROOT, "oracle", "_ref", "test_kernels")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/test_kernels not built")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "ALL KERNEL TESTS PASSED" in r.stdout, r.stdout[-2000:]


@pytest.mark.parametrize("k", [256, 2048, 6144])
def test_q8k_vs_ref(ref, k):
    g = synth.rng(k)
    x = synth.activations(g, 5, k)
    x[0, :256] = 0.0
    x[1, 7], x[1, 200] = -9.0, 9.0
    x[2] *= np.float32(1e-20)
    x[3, 1] = np.float32(3e38)
    assert O.quantize_q8k(x).tobytes() == ref.quantize_q8k(x).tobytes()


@pytest.mark.parametrize("gt", KINDS)
@pytest.mark.parametrize("n,k", [(37, 2048), (5, 6144)])
def test_matvec_vs_ref(ref, gt, n, k):
    g = synth.rng(gt * 1000 + n)
    w = synth.make_weight(g, gt, n, k)
    for nt in (1, 3, 16):
        x = synth.activations(g, nt, k)
        xq = O.quantize_q8k(x)
        assert np.array_equal(bits(O.matvec(w, x, xq, nt)), bits(ref.matvec(w, x, xq, nt, use_panel=True)))
    if w.pk is not None:  # the reference's native (un-repacked) STQ1_0 / Q2_0C dots agree too
        nat = synth.Weight(w.type, w.k, w.n, w.data)
        assert np.array_equal(bits(O.matvec(nat, x, xq, nt)), bits(ref.matvec(w, x, xq, nt, use_panel=False)))
        pk, ps = ref.panel_repack(w)
        assert np.array_equal(pk, w.pk) and np.array_equal(bits(ps), bits(w.ps))
    assert np.array_equal(bits(O.dequant(w)), bits(ref.dequant(w)))


def test_bf16_ops_vs_ref(ref):
    L, R = O.lib(), ref.load()
    g = synth.rng(9)
    for n in (64, 128, 131):
        q = synth.activations(g, 1, n)[0]
        kv = (synth.activations(g, 1, n)[0].view(np.uint32) >> 16).astype(np.uint16)
        assert bits(L.oc_dot_bf16(q.ctypes.data, kv.ctypes.data, n)) == bits(R.dot_bf16(q.ctypes.data, kv.ctypes.data, n))
        o1, o2 = q.copy(), q.copy()
        L.oc_axpy_bf16(o1.ctypes.data, kv.ctypes.data, 0.123, n)
        R.axpy_bf16(o2.ctypes.data, kv.ctypes.data, 0.123, n)
        assert np.array_equal(bits(o1), bits(o2))
    for h in range(0, 65536, 7):
        assert bits(L.oc_f16_to_f32(h)) == bits(R.f16_to_f32(h)) or np.isnan(R.f16_to_f32(h))


@pytest.mark.parametrize("mode", ["stq", "q2", "q4km"])
def test_model_vs_ref(ref, tmp_path, mode, monkeypatch):
    """Whole forward through the reference host (GGUF load, prefill in chunks of 8 at the scalar
    ISA, greedy with first-index argmax) against the oracle, on a tiny model with ctx 64 and a
    prompt that crosses a chunk boundary; also prefix reuse (warm == cold)."""
    monkeypatch.setenv("HYMT2_DEVICE", "cpu")
    monkeypatch.setenv("HYMT2_REPACK", "1")
    monkeypatch.setenv("HYMT2_PREFAULT", "0")
    shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1536, heads=8, kv_heads=2, hdim=64, vocab=700, ctx=64)
    model = synth.make_model(shape, mode=mode, seed=21)
    path = str(tmp_path / f"m_{mode}.gguf")
    gguf.write_model(path, model)
    rm = ref.RefModel(path, threads=2, ctx=shape.ctx)
    prompt = synth.rand_prompt(synth.rng(22), 13, shape.vocab)
    om = O.OracleModel(model, threads=4)
    lo = om.forward(prompt[:8], 0, False)
    lo = om.forward(prompt[8:], 8, True)
    assert np.array_equal(bits(lo), bits(rm.logits(prompt)))
    assert np.array_equal(bits(lo), bits(rm.logits(prompt, stepwise=True)))
    ids = O.OracleModel(model, threads=4).generate(prompt, 6, batch=8)
    assert np.array_equal(ids, rm.greedy(prompt, 6))
    rm.close()
