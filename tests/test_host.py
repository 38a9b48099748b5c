"""Host-side logic without a GPU: the synthetic-model generator, the GGUF writer (read back by
the reference host), byte accounting used by the bench, and bench.py's one-GPU contract."""
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import ROOT
from hymt2_amd import abi, synth


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""


def test_panel_paths_agree():
    """The fast STQ1_0 panel builder (codebook bytes placed directly) equals the generic
    codes -> panel path, and panel_to_codes inverts codes_to_panel."""
    g = synth.rng(1)
    blocks = synth.stq1_0_blocks(g, 7, 1024).reshape(7, 4, 42)
    codes = synth.stq_codes(blocks)
    assert np.array_equal(synth.stq_panel(blocks), synth.codes_to_panel(codes))
    c = g.integers(0, 4, size=(3, 5, 256), dtype=np.uint8)
    assert np.array_equal(synth.panel_to_codes(synth.codes_to_panel(c)), c)


def test_decode_bytes_per_token_accounting():
    """Per-layer panel bytes of the 1.8B shapes: 68 B per 256 weights over q,k,v,o,gate,up,down
    = 12,812,288 B; 32 layers = 409,993,216 B; F16 head 494,870,528 B."""
    s = synth.HYMT2_1_8B
    g = synth.rng(2)
    rows = dict(wq=(s.qdim, s.hidden), wk=(s.kvdim, s.hidden), wv=(s.kvdim, s.hidden), wo=(s.hidden, s.qdim),
                wg=(s.ffn, s.hidden), wu=(s.ffn, s.hidden), wd=(s.hidden, s.ffn))
    per_layer = sum(synth.make_weight(g, abi.GT_STQ1_0, n, k).nbytes_device() for n, k in rows.values())
    assert per_layer == 12_812_288 and 32 * per_layer == 409_993_216
    assert s.vocab * s.hidden * 2 == 494_870_528


def test_model_generator_is_deterministic():
    shape = synth.ModelShape(n_layer=1, hidden=256, ffn=512, heads=2, kv_heads=1, hdim=128, vocab=50, ctx=16)
    a = synth.model_digest(synth.make_model(shape, "q4km", seed=9))
    assert a == synth.model_digest(synth.make_model(shape, "q4km", seed=9))
    assert a != synth.model_digest(synth.make_model(shape, "q4km", seed=10))


def test_gguf_roundtrip_through_reference_loader(ref, tmp_path, monkeypatch):
    """A GGUF written by hymt2_amd.gguf loads in the reference host with the intended shapes."""
    from hymt2_amd import gguf
    monkeypatch.setenv("HYMT2_DEVICE", "cpu")
    shape = synth.ModelShape(n_layer=2, hidden=512, ffn=1024, heads=4, kv_heads=2, hdim=128, vocab=300, ctx=32)
    model = synth.make_model(shape, "q2", seed=4)
    p = str(tmp_path / "m.gguf")
    gguf.write_model(p, model)
    rm = ref.RefModel(p, threads=1, ctx=32)
    assert "repack=panel" in rm.info() or "repack=native" in rm.info()
    lg = rm.logits(np.array([1, 2, 3], dtype=np.int32))
    assert lg.shape == (300,) and np.all(np.isfinite(lg))
    rm.close()


def test_product_package_does_not_import_the_oracle():
    """The product (hymt2_amd and its C-ABI library) never imports, loads or links the checker."""
    import re
    pat = re.compile(r"^\s*(from|import)\s+oracle\b|liboracle|hymt2_oracle|_ref/", re.M)
    for dirpath, _, files in os.walk(os.path.join(ROOT, "hymt2_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")) or f == "Makefile":
                text = open(os.path.join(dirpath, f), errors="replace").read()
                assert not pat.search(text), os.path.join(dirpath, f)
