"""Writes the golden vectors under tests/golden/ from the reference library.

The reference (zhangbo8418/hymt2) commits no golden vectors: its tests draw seeded random
inputs (tests/test_kernels.c, seed 12345) and compare its SIMD paths with its scalar path. The
fixtures here are therefore made by running the reference's own C code, compiled from its
sources by oracle/Makefile into oracle/_ref/libhymt2_ref.so, on small seeded inputs at the
scalar ISA (the bit-exact contract of the HIP backend):

* q8k.npz         quantize_q8k (src/kernels.c:128-165) on edge-case rows
* panel_<t>.npz   panel_repack_rows (src/kernels.c:535-561) of STQ1_0 / Q2_0C rows
* matvec_<t>.npz  matmul_rows (src/kernels.c:1241-1329) for every weight type the backend
                  accepts, nt = 3, plus dequant_row (src/kernels.c:1099-1109) of 4 rows
* bf16.npz        dot_bf16 / axpy_bf16 (src/kernels.c:1111-1124) and f32_to_bf16 (:107-111)
* model_<m>.npz   whole-model logits (hymt2_debug_logits) and 8 greedy ids of a tiny
                  synthetic model loaded from a GGUF by the reference host (src/model.c)
* gen_ids.npz     (with --gen-ids) the reference's greedy loop gen_ids (src/model.c:914-958) on
                  hymt2_amd.synth.gen_ids_model(), whose greedy runs end at EOS: the calls of
                  synth.gen_ids_calls() in order on one model, so each reuses the K/V prefix the
                  one before it left. Per call: the prompt ids, the returned ids (before the stop
                  id) and hymt2_model_stats's cached and prefilled token counts.
* baseline_config3.npz / baseline_config4.npz (with --baseline): the BASELINE decode
                  workloads on the Hy-MT2-1.8B-shaped models (hymt2_amd.synth.CONFIG3 / CONFIG4).
                  The reference's own greedy loop (gen_ids, src/model.c:914-958, through
                  hymt2_debug_generate_ids) runs the chat prompt whose encoding is the config's
                  prompt ids: config 3 = 64 prompt ids then 128 greedy ids; config 4 = 1024 prompt
                  ids then 256 greedy ids. Logits (hymt2_debug_logits) are stored as a sha256 of
                  their bits plus the top 32 (index, value) pairs: at the end of the prompt and
                  after the prompt and all generated ids but the last (the input of the loop's
                  last forward). A control run at the auto-detected ISA records how
                  many leading greedy ids agree with the scalar run.

Inputs are stored in the fixtures (or, for the models, regenerated from a seed and checked
against a stored digest). Run from the repository root: python tests/golden/make_golden.py
[--baseline [config3|config4]] [--gen-ids]
"""
import hashlib
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from hymt2_amd import abi, gguf, synth  # noqa: E402
from oracle import refbind as R  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

TYPE_NAMES = {abi.GT_STQ1_0: "stq1_0", abi.GT_Q2_0C: "q2_0c", abi.GT_Q4_K: "q4_k", abi.GT_Q6_K: "q6_k",
              abi.GT_F16: "f16", abi.GT_F32: "f32"}

# Tiny Hy-MT2-shaped models: every layer op, GQA (4 q heads over 2 kv heads), tied F16 head.
TINY = dict(n_layer=2, hidden=512, ffn=1024, heads=4, kv_heads=2, hdim=128, vocab=1000, ctx=64)
MODEL_SEED, PROMPT_SEED, N_PROMPT, N_GREEDY = 11, 5, 20, 8


def q8k_inputs() -> np.ndarray:
    """Rows of 2 blocks each that hit quantize_q8k's branches."""
    g = synth.rng(101)
    x = synth.activations(g, 6, 512)
    x[0, :256] = 0.0                     # all-zero block -> zeroed record
    x[1, 5], x[1, 77] = 3.0, -3.0        # |max| tie: the first index sets the sign
    x[1, 300], x[1, 301] = -7.0, 7.0     # tie, negative first
    x[2, 256:] = 1e-30                   # tiny (denormal scale) block
    x[3, 10] = 1e30                      # huge outlier
    x[4, :] = -1.0                       # constant block
    x[5, ::2] *= 1e-3                    # wide dynamic range
    return x


def logits_summary(prefix: str, lg: np.ndarray, top: int = 32) -> dict:
    lg = np.ascontiguousarray(lg, dtype=np.float32)
    order = np.argsort(-lg, kind="stable")[:top]
    s = np.sort(lg)[::-1]
    return {f"{prefix}_sha256": hashlib.sha256(lg.view(np.uint32).tobytes()).hexdigest(),
            f"{prefix}_top_idx": order.astype(np.int32), f"{prefix}_top_val": lg[order],
            f"{prefix}_top2_gap": np.float32(s[0] - s[1])}


# canonical context lengths of the fixtures' models (the weights do not depend on ctx)
BASELINE_CTX = {"config3": 256, "config4": 1344}


def baseline_fixture(name: str, cfg: dict, n_gen: int, last_logits: bool, threads: int = 8):
    ctx = BASELINE_CTX[name]
    t0 = time.time()
    model = synth.baseline_model(cfg, ctx)
    prompt, text = synth.baseline_prompt(cfg)
    rec = dict(name=name, mode=cfg["mode"], seed=cfg["seed"], ctx=ctx, digest=synth.model_digest(model),
               prompt=prompt, n_gen=n_gen, threads=threads)
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, f"{name}.gguf")
        gguf.write_model(path, model)
        del model
        for isa in ("scalar", "auto"):
            rec_isa = R.set_isa(isa)
            if isa == "auto":
                rec["auto_isa"] = rec_isa
            rm = R.RefModel(path, threads=threads, ctx=ctx)
            ids = ref_greedy(rm, text, n_gen)
            if isa == "scalar":
                got = rm.encode_chat(text)
                assert np.array_equal(got, prompt), "chat text does not encode to the prompt ids"
                rec["greedy"] = ids
                rec["info"] = rm.info()
                rec.update(logits_summary("prompt_logits", rm.logits(prompt)))
                if last_logits:
                    rec.update(logits_summary("last_logits", rm.logits(np.concatenate([prompt, ids[:-1]]))))
            else:
                agree = 0
                while agree < min(len(ids), len(rec["greedy"])) and ids[agree] == rec["greedy"][agree]:
                    agree += 1
                rec["auto_agree"] = agree
                rec["auto_greedy"] = ids
            rm.close()
    R.set_isa("scalar")
    np.savez(os.path.join(OUT, f"baseline_{name}.npz"), **rec)
    print(name, f"{time.time() - t0:.0f} s: greedy", rec["greedy"][:12], "... auto agrees on", rec["auto_agree"],
          "of", n_gen, "ids", flush=True)


def ref_greedy(rm, text: str, n_gen: int) -> np.ndarray:
    ids, st = rm.generate_text(text, n_gen)
    assert len(ids) == n_gen, f"reference generated {len(ids)} ids, expected {n_gen} ({st})"
    return ids.astype(np.int32)


def baseline_fixtures(which=("config3", "config4")):
    os.environ.update(HYMT2_DEVICE="cpu", HYMT2_ISA="scalar", HYMT2_REPACK="1", HYMT2_PREFAULT="0")
    if "config3" in which:
        baseline_fixture("config3", synth.CONFIG3, synth.CONFIG3["n_gen"], last_logits=True)
    if "config4" in which:
        baseline_fixture("config4", synth.CONFIG4, synth.CONFIG4["n_gen"], last_logits=True)


def gen_ids_fixture(threads: int = 4):
    os.environ.update(HYMT2_DEVICE="cpu", HYMT2_ISA="scalar", HYMT2_REPACK="1", HYMT2_PREFAULT="0")
    model = synth.gen_ids_model()
    rec = dict(digest=synth.model_digest(model))
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "gen_ids.gguf")
        gguf.write_model(path, model)
        R.set_isa("scalar")
        rm = R.RefModel(path, threads=threads, ctx=synth.GEN_IDS_SHAPE.ctx)
        for i, (words, max_tokens) in enumerate(synth.gen_ids_calls()):
            text = gguf.chat_text(words)
            prompt = np.array(gguf.chat_ids(words), dtype=np.int32)
            assert np.array_equal(rm.encode_chat(text), prompt), "chat text does not encode to the prompt ids"
            ids, st = rm.generate_text(text, max_tokens)
            rec[f"prompt{i}"] = prompt
            rec[f"max{i}"] = np.int32(max_tokens)
            rec[f"ids{i}"] = ids.astype(np.int32)
            rec[f"cached{i}"] = np.int32(st["cached_tokens"])
            rec[f"prefill{i}"] = np.int32(st["prefill_tokens"])
            print(f"call {i}: {len(prompt)} prompt ids, {st['cached_tokens']} cached, {len(ids)} ids: {ids.tolist()}",
                  flush=True)
        rm.close()
    np.savez(os.path.join(OUT, "gen_ids.npz"), **rec)


def main():
    if "--gen-ids" in sys.argv:
        gen_ids_fixture()
        return
    if "--baseline" in sys.argv:
        rest = [a for a in sys.argv[sys.argv.index("--baseline") + 1:] if not a.startswith("-")]
        baseline_fixtures(tuple(rest) or ("config3", "config4"))
        return
    R.set_isa("scalar")
    L = R.load()
    g = synth.rng(202)

    x = q8k_inputs()
    np.savez(os.path.join(OUT, "q8k.npz"), x=x, q8k=R.quantize_q8k(x).view(np.uint8))

    for gt, name in TYPE_NAMES.items():
        n, k, nt = 32, 512, 3
        w = synth.make_weight(g, gt, n, k)
        xf = synth.activations(g, nt, k)
        xq = R.quantize_q8k(xf)
        out = R.matvec(w, xf, xq, nt, use_panel=True)
        deq = R.dequant(synth.Weight(w.type, w.k, 4, w.data[:4]))
        np.savez(os.path.join(OUT, f"matvec_{name}.npz"), type=gt, n=n, k=k, nt=nt, data=w.data, x=xf,
                 q8k=xq.view(np.uint8), out=out, dequant4=deq)
        if w.pk is not None:
            pk, ps = R.panel_repack(w)
            np.savez(os.path.join(OUT, f"panel_{name}.npz"), type=gt, n=n, k=k, data=w.data, pk=pk, ps=ps)

    # Q8_0 (the fp32-activation LM head of src/kernels.c:1099-1107), from its own stream so the
    # fixtures above keep their inputs
    gq = synth.rng(203)
    n, k, nt = 32, 512, 3
    w = synth.make_weight(gq, abi.GT_Q8_0, n, k)
    xf = synth.activations(gq, nt, k)
    out = R.matvec(w, xf, R.quantize_q8k(xf), nt, use_panel=False)
    deq = R.dequant(synth.Weight(w.type, w.k, 4, w.data[:4]))
    np.savez(os.path.join(OUT, "matvec_q8_0.npz"), type=abi.GT_Q8_0, n=n, k=k, nt=nt, data=w.data, x=xf,
             q8k=R.quantize_q8k(xf).view(np.uint8), out=out, dequant4=deq)

    n = 300
    q = synth.activations(g, 1, n)[0]
    kv = (synth.activations(g, 1, n)[0].view(np.uint32) >> 16).astype(np.uint16)  # bf16 bits
    o = synth.activations(g, 1, n)[0]
    o2 = o.copy()
    L.axpy_bf16(o2.ctypes.data, kv.ctypes.data, np.float32(0.37), n)
    vals = np.concatenate([synth.activations(g, 1, 256)[0],
                           np.array([0.0, -0.0, 1.0, 65504.0, 1e-40, -3.4e38, 1.00390625, 1.01171875],
                                    dtype=np.float32)])
    np.savez(os.path.join(OUT, "bf16.npz"), q=q, kv=kv, dot=np.float32(L.dot_bf16(q.ctypes.data, kv.ctypes.data, n)),
             o=o, p=np.float32(0.37), axpy=o2, vals=vals,
             to_bf16=np.array([L.f32_to_bf16(float(v)) for v in vals], dtype=np.uint16))

    os.environ.update(HYMT2_DEVICE="cpu", HYMT2_ISA="scalar", HYMT2_REPACK="1", HYMT2_PREFAULT="0")
    with tempfile.TemporaryDirectory() as td:
        for mode in ("stq", "q2", "q4km"):
            shape = synth.ModelShape(**TINY)
            model = synth.make_model(shape, mode=mode, seed=MODEL_SEED)
            path = os.path.join(td, f"tiny_{mode}.gguf")
            gguf.write_model(path, model)
            rm = R.RefModel(path, threads=1, ctx=shape.ctx)
            prompt = synth.rand_prompt(synth.rng(PROMPT_SEED), N_PROMPT, shape.vocab)
            logits = rm.logits(prompt)
            ids = rm.greedy(prompt, N_GREEDY)
            rm.close()
            np.savez(os.path.join(OUT, f"model_{mode}.npz"), mode=mode, seed=MODEL_SEED,
                     digest=synth.model_digest(model), prompt=prompt, logits=logits, greedy=ids,
                     **{f"shape_{k}": v for k, v in TINY.items()})
            print(mode, "greedy", ids)
    print("golden vectors written to", OUT)


if __name__ == "__main__":
    main()
