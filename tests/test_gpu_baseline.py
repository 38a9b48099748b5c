"""BASELINE configs 3 and 4 at full size on the GPU against the reference's own greedy loop.

The fixtures (tests/golden/baseline_config3.npz, baseline_config4.npz) hold what the reference
host compiled from its sources computes at the scalar ISA on the same seeded 1.8B-shaped models
and prompts (tests/golden/make_golden.py --baseline): gen_ids (src/model.c:914-958) on the chat
prompt whose encoding is the config's prompt ids, and hymt2_debug_logits at the end of the prompt
and at the input of the loop's last forward. Ids are compared exactly, logits by the sha256 of
their bits."""
import hashlib
import os

import numpy as np
import pytest

from conftest import GOLDEN
from hymt2_amd import lib, synth

pytestmark = pytest.mark.gpu

CFG = {"config3": synth.CONFIG3, "config4": synth.CONFIG4}


def fixture(name):
    f = np.load(os.path.join(GOLDEN, f"baseline_{name}.npz"), allow_pickle=False)
    model = synth.baseline_model(CFG[name], int(f["ctx"]))
    assert synth.model_digest(model) == str(f["digest"]), "the generator no longer reproduces the fixture's model"
    return f, model


def check_logits(f, prefix, lg):
    lg = np.ascontiguousarray(lg, dtype=np.float32)
    top = f[f"{prefix}_top_idx"]
    assert np.array_equal(lg[top].view(np.uint32), f[f"{prefix}_top_val"].view(np.uint32)), prefix
    assert hashlib.sha256(lg.view(np.uint32).tobytes()).hexdigest() == str(f[f"{prefix}_sha256"]), prefix


def test_config3_greedy_identity(backend):
    """64 prompt ids, then 128 greedy ids of the device loop (the bench's workload), with the
    prompt as single-token steps and as 64- and 16-position chunks; the logits at the end of the
    prompt and after 64 + 127 positions through the reference host's boundary (fused_forward in
    chunks of 16)."""
    f, model = fixture("config3")
    prompt, want = f["prompt"], f["greedy"]
    assert len(prompt) == 64 and len(want) == 128
    fm = lib.FusedModel(backend, model)
    try:
        for chunk in (1, 64, 16):
            ids, st = fm.generate_device(prompt, len(want), chunk=chunk)
            assert np.array_equal(ids, want), f"chunk={chunk}: first difference at {np.argmax(ids != want)}"
            assert st.decode_steps == len(want) - 1
        check_logits(f, "prompt_logits", fm.prefill(list(prompt), batch=16))
        check_logits(f, "last_logits", fm.prefill(list(prompt) + list(want[:-1]), batch=16))
        assert np.array_equal(fm.generate_host(prompt, 8, batch=16), want[:8])
    finally:
        fm.close()


def test_config4_greedy_identity(backend):
    """1024 prompt ids in 128-token chunks (int8-MFMA GEMMs, chunk attention over the growing KV
    cache, pipelined over the layers), then all 256 greedy ids of the decode (single-token steps
    at positions 1024-1279, the split attention); the logits at the end of the 128-token-chunk
    prefill and after 1024 + 255 positions (10 chunks, the last one ragged), through the reference
    host's boundary (fused_forward in chunks of 128)."""
    f, model = fixture("config4")
    prompt, want = f["prompt"], f["greedy"]
    assert len(prompt) == 1024 and len(want) == 256
    fm = lib.FusedModel(backend, model)
    try:
        ids, st = fm.generate_device(prompt, len(want), chunk=128)
        assert np.array_equal(ids, want), f"first difference at {np.argmax(ids != want)}"
        assert st.decode_steps == len(want) - 1
        check_logits(f, "prompt_logits", fm.prefill(list(prompt), batch=128))
        check_logits(f, "last_logits", fm.prefill(list(prompt) + list(want[:-1]), batch=128))
    finally:
        fm.close()
