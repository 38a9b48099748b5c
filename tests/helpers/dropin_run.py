"""Runs the reference's unchanged C host (oracle/_ref/libhymt2_host.so: the reference sources
linked against libhymt2_hip.so in place of src/cuda.c) on a GGUF in a fresh process and saves
what it computed. Used by tests/test_gpu_dropin.py; run as

    python dropin_run.py <model.gguf> <ctx> <out.npz> <prompt ids comma-separated> <text> <max_tokens>

The environment chooses the device exactly as for the reference (HYMT2_DEVICE, HYMT2_ISA,
HYMT2_REPACK, HYMT2_FUSED)."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import refbind  # noqa: E402


def main():
    path, ctx, out = sys.argv[1], int(sys.argv[2]), sys.argv[3]
    prompt = np.array([int(t) for t in sys.argv[4].split(",")], dtype=np.int32)
    text, max_tokens = sys.argv[5], int(sys.argv[6])
    lib = refbind.HOST_LIB if os.environ.get("HYMT2_DEVICE") != "cpu-ref" else refbind.REF_LIB
    if os.environ.get("HYMT2_DEVICE") == "cpu-ref":
        os.environ["HYMT2_DEVICE"] = "cpu"
    refbind.load(lib)
    rm = refbind.RefModel(path, threads=int(os.environ.get("HYMT2_THREADS", "4")), ctx=ctx, path=lib)
    info = rm.info()
    print("model info:", info, flush=True)
    logits = rm.logits(prompt)
    step = rm.logits(prompt, stepwise=True)
    ids, st = rm.generate_text(text, max_tokens)
    print("generated", len(ids), "ids; stats", st, flush=True)
    rm.close()
    np.savez(out, info=info, logits=logits, stepwise=step, ids=ids)


if __name__ == "__main__":
    main()
