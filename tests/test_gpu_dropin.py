"""The drop-in: the reference's own C host, unchanged, with libhymt2_hip.so linked in place of
its CUDA backend (oracle/Makefile `host`), selects the HIP device through hy_cuda_create
(HYMT2_DEVICE=cuda, src/model.c:424-450), uploads every weight, enables the fused path and
produces the same logits and greedy ids, bit for bit, as the same host on the CPU at the scalar
ISA. Each leg runs in a fresh process (the backend's weak reference to the host's
hy_device_wrap binds when the host library loads it)."""
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import ROOT
from hymt2_amd import gguf, synth
from oracle import refbind

pytestmark = pytest.mark.gpu

RUNNER = os.path.join(ROOT, "tests", "helpers", "dropin_run.py")


def run_leg(env_extra, path, ctx, out, prompt, text, max_tokens, unset=()):
    env = dict(os.environ, HYMT2_ISA="scalar", HYMT2_REPACK="1", HYMT2_PREFAULT="0", HYMT2_THREADS="4",
               HYMT2_VERBOSE="1", **env_extra)
    for k in unset:
        env.pop(k, None)
    r = subprocess.run([sys.executable, RUNNER, path, str(ctx), out, ",".join(str(int(t)) for t in prompt), text,
                        str(max_tokens)], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return np.load(out, allow_pickle=False), r.stderr


@pytest.mark.parametrize("mode", ["stq", "q2", "q4km"])
def test_reference_host_on_hip_backend(tmp_path, mode):
    if not (refbind.available(refbind.HOST_LIB) and refbind.available(refbind.REF_LIB)):
        pytest.skip("oracle/_ref host libraries not built (needs the reference tree at build time)")
    shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1024, heads=4, kv_heads=2, hdim=128, vocab=1000, ctx=128)
    model = synth.make_model(shape, mode=mode, seed=51)
    path = str(tmp_path / f"m_{mode}.gguf")
    gguf.write_model(path, model)
    prompt = synth.rand_prompt(synth.rng(52), 21, shape.vocab)
    text = "t5 t17 t300 t42"
    gpu, log = run_leg({"HYMT2_DEVICE": "cuda"}, path, shape.ctx, str(tmp_path / "gpu.npz"), prompt, text, 24)
    cpu, _ = run_leg({"HYMT2_DEVICE": "cpu-ref"}, path, shape.ctx, str(tmp_path / "cpu.npz"), prompt, text, 24)
    assert "gpu=hip+fused" in str(gpu["info"]), str(gpu["info"]) + log[-2000:]
    assert "gpu=off" in str(cpu["info"])
    for key in ("logits", "stepwise"):
        assert np.array_equal(gpu[key].view(np.uint32), cpu[key].view(np.uint32)), key
    assert len(cpu["ids"]) > 0 and np.array_equal(gpu["ids"], cpu["ids"])


@pytest.mark.parametrize("mode", ["stq", "q4km"])
def test_reference_host_per_op_path(tmp_path, mode):
    """HYMT2_FUSED=0 (src/model.c:330-333): the host's per-op path. Every layer matvec group goes
    through the backend's matmul with the weight_out buffers as outputs (gpu_out,
    src/model.c:662-667); norms, RoPE and attention run on the host. The backend declines the F16
    head at upload, so the host computes it on the CPU and keeps the device for the layers
    (reported "gpu=hip", not "+fused"). Logits, stepwise logits and greedy ids equal the CPU's."""
    if not (refbind.available(refbind.HOST_LIB) and refbind.available(refbind.REF_LIB)):
        pytest.skip("oracle/_ref host libraries not built (needs the reference tree at build time)")
    shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1024, heads=4, kv_heads=2, hdim=128, vocab=1000, ctx=128)
    model = synth.make_model(shape, mode=mode, seed=57)
    path = str(tmp_path / f"m_{mode}.gguf")
    gguf.write_model(path, model)
    prompt = synth.rand_prompt(synth.rng(58), 19, shape.vocab)
    text = "t5 t17 t300 t42"
    gpu, log = run_leg({"HYMT2_DEVICE": "cuda", "HYMT2_FUSED": "0"}, path, shape.ctx, str(tmp_path / "gpu.npz"),
                       prompt, text, 12)
    cpu, _ = run_leg({"HYMT2_DEVICE": "cpu-ref"}, path, shape.ctx, str(tmp_path / "cpu.npz"), prompt, text, 12)
    info = str(gpu["info"])
    assert "gpu=hip" in info and "+fused" not in info, info + log[-2000:]
    for key in ("logits", "stepwise"):
        assert np.array_equal(gpu[key].view(np.uint32), cpu[key].view(np.uint32)), key
    assert len(cpu["ids"]) > 0 and np.array_equal(gpu["ids"], cpu["ids"])


def test_reference_host_auto_selects_hip(tmp_path):
    """HYMT2_DEVICE unset (auto): the host tries cuda first (src/device.c:112, src/model.c:457),
    uploads every weight, times a CPU step against a fused step and keeps the fused path only
    when it is at least 10% faster (src/model.c:338-373). On two 1.8B-shaped layers the backend
    wins its calibration against the host cores: the host reports gpu=hip+fused, and its logits,
    stepwise logits and greedy ids equal the same host's on the CPU."""
    if not (refbind.available(refbind.HOST_LIB) and refbind.available(refbind.REF_LIB)):
        pytest.skip("oracle/_ref host libraries not built (needs the reference tree at build time)")
    shape = synth.ModelShape(n_layer=2, vocab=4000, ctx=96)
    model = synth.make_model(shape, mode="stq", seed=59)
    path = str(tmp_path / "m_auto.gguf")
    gguf.write_model(path, model)
    prompt = synth.rand_prompt(synth.rng(60), 17, shape.vocab)
    text = "t5 t17 t300 t42"
    gpu, log = run_leg({}, path, shape.ctx, str(tmp_path / "gpu.npz"), prompt, text, 12,
                       unset=("HYMT2_DEVICE", "HYMT2_VK", "HYMT2_FUSED"))
    cpu, _ = run_leg({"HYMT2_DEVICE": "cpu-ref"}, path, shape.ctx, str(tmp_path / "cpu.npz"), prompt, text, 12)
    assert "gpu=hip+fused" in str(gpu["info"]), str(gpu["info"]) + log[-2000:]
    assert "auto -> hip+fused" in log, log[-2000:]
    for key in ("logits", "stepwise"):
        assert np.array_equal(gpu[key].view(np.uint32), cpu[key].view(np.uint32)), key
    assert len(cpu["ids"]) > 0 and np.array_equal(gpu["ids"], cpu["ids"])
