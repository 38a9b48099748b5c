"""Decode benchmark of the HIP backend on the Hy-MT2-1.8B-shaped STQ1_0 model.

One step = one greedy decode token at batch 1: the full 32-layer forward (STQ1_0 panel
matvecs, RoPE, q/k norms, bf16 KV, GQA attention, SwiGLU), the tied F16 LM head and the
argmax, all on the device with no host round trip (hymt2_hip_gen_steps). Weights are random
(seeded) with the config's shapes; the prompt is 64 random chat-template ids (hymt2_amd.synth
CONFIG3). The greedy ids are checked against the reference's own greedy loop on the same model
(tests/golden/baseline_config3.npz). Prints one JSON line.

  python bench.py [--steps K] [--warmup W] [--no-cpu]

The cpu_baseline leg times the reference library itself (oracle/_ref/libhymt2_ref.so, built
from the reference's sources) on the host with HYMT2_DEVICE=cpu, HYMT2_REPACK=1, the ISA it
auto-detects and HYMT2_THREADS = the host's physical cores, on the same workload: the chat
text that encodes to the same 64 prompt ids, then 128 greedy decode tokens. The same leg runs
the reference's unchanged host with this backend linked in place of its CUDA one
(oracle/_ref/libhymt2_host.so, HYMT2_DEVICE=cuda) in a child process, fused (host_dropin) and
per-op (HYMT2_FUSED=0, per_op), and reports the host's own decode rate (hymt2_model_stats).
"""
import argparse
import ctypes as C
import json
import os
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_model(ctx: int):
    """BASELINE config 3's model (hymt2_amd.synth.CONFIG3): 1.8B shapes, STQ1_0 layers, tied F16
    head whose EOS row is damped so that both legs decode their full length."""
    from hymt2_amd import synth
    model = synth.baseline_model(synth.CONFIG3, ctx)
    return model["shape"], model


FIXTURE = os.path.join(ROOT, "tests", "golden", "baseline_config3.npz")


def check_against_fixture(prompt, ids):
    """The device loop's greedy ids against the reference's own greedy loop at the scalar ISA on
    the same model and prompt (tests/golden/baseline_config3.npz, written by
    tests/golden/make_golden.py --baseline). Raises on any difference."""
    f = np.load(FIXTURE, allow_pickle=False)
    if not np.array_equal(f["prompt"], prompt):
        raise RuntimeError("bench prompt differs from the fixture's prompt")
    n = min(len(ids), len(f["greedy"]))
    bad = np.nonzero(ids[:n] != f["greedy"][:n])[0]
    if len(bad):
        raise RuntimeError(f"greedy id {bad[0]} differs from the reference: {ids[bad[0]]} != {f['greedy'][bad[0]]}")
    return dict(checked_ids=int(n), identical=True, reference=f"reference gen_ids at ISA scalar ({f['info']})",
                min_top2_gap_at_prompt_end=float(f["prompt_logits_top2_gap"]))


def _timed_launches(stream, launch, n):
    """Average seconds per launch of `launch(i)` over i = 0..n-1, from HIP events recorded on
    the backend stream (the stream the kernels run on)."""
    import torch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(n):
        launch(i)
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / n / 1000.0


def ffn_in_roofline(model, b, copies: int = 64, passes: int = 3):
    """The decode step's dominant kernel: the fused feed-forward input (RMSNorm + Q8_K prologue,
    gate and up STQ1_0 panel matvecs, SwiGLU epilogue; 2 x 6144 x 2048 weights), launched
    standalone through hymt2_hip_ffn_in over `copies` distinct device copies of layer 0's gate/up
    weights (64 x 6.7 MB = 430 MB, more than the 256 MB Infinity Cache, so every launch streams
    its weights from HBM as in the decode loop). Algorithmic bytes per launch = panel codes +
    panel scales of both weights + h + the norm weights + the SwiGLU output."""
    import torch
    s = model["shape"]
    L0 = model["layers"][0]
    wg, wu = L0["wg"], L0["wu"]
    handles = [(b.upload(wg), b.upload(wu)) for _ in range(copies)]
    stream = torch.cuda.ExternalStream(b.stream)
    h = torch.randn(s.hidden, device="cuda", dtype=torch.float32)
    nw = torch.from_numpy(L0["ffn_norm"]).to("cuda")
    out = torch.empty(wg.n, device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()

    def launch(i):
        g, u = handles[i % copies]
        if b.L.hymt2_hip_ffn_in(b.impl, g, u, h.data_ptr(), nw.data_ptr(), C.c_float(s.eps), out.data_ptr()) != 0:
            raise RuntimeError("hymt2_hip_ffn_in failed: " + b.last_error())

    for i in range(copies):
        launch(i)
    avg_s = _timed_launches(stream, launch, copies * passes)
    for g, u in handles:
        b.release(g)
        b.release(u)
    algo = wg.nbytes_device() + wu.nbytes_device() + 2 * s.hidden * 4 + wg.n * 4
    return dict(bound="hbm", achieved=round(algo / avg_s / 1e9, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(algo / avg_s / 1e9 / HBM_PEAK_GBS, 4), traffic=_pmc_traffic("ffn_in"),
                kernel="k_mv1<PANEL, SPL 1, ITERS 6, PRO_NORM> pair mode, 256 workgroups of 24 gate+up row pairs (hymt2_hip_ffn_in): fused FFN input of "
                       "one decode token (RMSNorm + Q8_K prologue, gate+up 2x6144x2048 STQ1_0 panel, SwiGLU)",
                avg_us=round(avg_s * 1e6, 2), bytes_per_launch=algo,
                timing=f"HIP events on the backend stream over {copies * passes} launches rotating {copies} "
                       f"weight copies",
                in_graph=_in_graph_figure(algo))


def head_roofline(fm, b, reps: int = 20):
    """LM head (F16 120818 x 2048 + argmax) from HIP events on the backend stream; algorithmic
    bytes = weight rows + input vector + norm + logits. Its 495 MB of weights exceed the
    Infinity Cache by themselves."""
    import torch
    s = fm.shape
    stream = torch.cuda.ExternalStream(b.stream)
    h = torch.randn(s.hidden, device="cuda", dtype=torch.float32)
    nw = torch.ones(s.hidden, device="cuda", dtype=torch.float32)
    logits = torch.empty(fm.model["outw"].n, device="cuda", dtype=torch.float32)
    key = torch.zeros(1, device="cuda", dtype=torch.int64)
    torch.cuda.synchronize()

    def launch(_):
        rc = b.L.hymt2_hip_head(b.impl, fm.outw, h.data_ptr(), nw.data_ptr(), C.c_float(s.eps), logits.data_ptr(),
                                fm.vocab_out, key.data_ptr())
        if rc != 0:
            raise RuntimeError("hymt2_hip_head failed: " + b.last_error())

    for i in range(3):
        launch(i)
    avg_s = _timed_launches(stream, launch, reps)
    w = fm.model["outw"]
    algo = w.n * w.k * 2 + 2 * s.hidden * 4 + w.n * 4
    return dict(achieved=round(algo / avg_s / 1e9, 1), frac=round(algo / avg_s / 1e9 / HBM_PEAK_GBS, 4),
                avg_us=round(avg_s * 1e6, 2), bytes_per_launch=algo,
                kernel="k_head<F16> (LM head 120818x2048 + argmax)")


def layer_sets(b, copies: int = 64, passes: int = 2):
    """BASELINE configs 0-2 on the single-token matvec entry point (hymt2_hip_matvec, Q8_K
    activation already on the device, the reference's matmul_rows contract), each timed with
    HIP events over `copies` rotating device copies of its weights (beyond the 256 MB Infinity
    Cache):
      config0: the fused gate/up 12288x2048 STQ1_0 panel (codes uniform 0..2, fp32 scales
               U(0.005, 0.05)), one call; also timed repeating one copy (cache-resident)
      config1: one Q2_0C layer: q, k, v, o, gate, up, down
      config2: one Q4_K_M layer: Q4_K q, k, o, gate, up; Q6_K v, down
    Algorithmic bytes: weights as stored + Q8_K activations + fp32 outputs."""
    import torch
    from hymt2_amd import abi, synth
    s = synth.HYMT2_1_8B
    g = synth.rng(0xC0DE0)
    stream = torch.cuda.ExternalStream(b.stream)
    shapes = [("wq", s.qdim, s.hidden), ("wk", s.kvdim, s.hidden), ("wv", s.kvdim, s.hidden), ("wo", s.hidden, s.qdim),
              ("wg", s.ffn, s.hidden), ("wu", s.ffn, s.hidden), ("wd", s.hidden, s.ffn)]
    act = {k: torch.zeros(k // 256 * abi.Q8K_BYTES, dtype=torch.uint8, device="cuda") for k in (s.hidden, s.ffn)}
    for k, a in act.items():
        x = torch.randn(k, device="cuda", dtype=torch.float32)
        b.quantize_q8k(x.data_ptr(), a.data_ptr(), k, 1)
    out = torch.empty(max(s.ffn * 2, s.hidden), device="cuda", dtype=torch.float32)
    res = {}

    def timed(weights, reps):
        """weights: list of (Weight, [device copies]); one unit = one pass over the list."""
        def launch(i):
            for w, hs in weights:
                b.matvec(hs[i % len(hs)], act[w.k].data_ptr(), out.data_ptr(), 1)
        n = max(len(hs) for _, hs in weights)
        for i in range(n):
            launch(i)
        return _timed_launches(stream, launch, reps)

    # config 0: per call (launch included), and streaming: one launch over `copies` stacked
    # copies of the panel (copies * 12288 rows, 430 MB), the kernel's sustained bandwidth
    pk, ps = synth.panel_uniform_codes(g, 2 * s.ffn, s.hidden)
    w0 = synth.Weight(abi.GT_STQ1_0, s.hidden, 2 * s.ffn,
                      np.zeros((2 * s.ffn, abi.row_bytes(abi.GT_STQ1_0, s.hidden)), np.uint8), pk, ps, 0, 1)
    hs = [b.upload(w0) for _ in range(copies)]
    algo0 = w0.nbytes_device() + (s.hidden // 256) * abi.Q8K_BYTES + 2 * s.ffn * 4
    t_call = timed([(w0, hs)], copies * passes)
    for h in hs:
        b.release(h)
    nrow = copies * 2 * s.ffn
    ws = synth.Weight(abi.GT_STQ1_0, s.hidden, nrow, np.zeros((nrow, abi.row_bytes(abi.GT_STQ1_0, s.hidden)), np.uint8),
                      np.tile(pk, (copies, 1, 1)), np.tile(ps, (copies, 1)), 0, 1)
    big = torch.empty(nrow, device="cuda", dtype=torch.float32)
    hb = b.upload(ws)

    def launch_big(_):
        b.matvec(hb, act[s.hidden].data_ptr(), big.data_ptr(), 1)

    launch_big(0)
    t_big = _timed_launches(stream, launch_big, 5)
    b.release(hb)
    algo_big = ws.nbytes_device() + (s.hidden // 256) * abi.Q8K_BYTES + nrow * 4
    res["config0"] = dict(unit="call", bytes=algo0, call_us=round(t_call * 1e6, 2),
                          call_GBs=round(algo0 / t_call / 1e9, 1), call_frac=round(algo0 / t_call / 1e9 / HBM_PEAK_GBS, 4),
                          stream_rows=nrow, stream_bytes=algo_big, stream_us=round(t_big * 1e6, 2),
                          stream_GBs=round(algo_big / t_big / 1e9, 1),
                          stream_frac=round(algo_big / t_big / 1e9 / HBM_PEAK_GBS, 4),
                          timing="call: HIP events over back-to-back launches rotating 64 copies (launch cost "
                                 "included); stream: one launch over 64 stacked copies")
    # configs 1 and 2: one layer's matvec set
    for name, mode in (("config1", "q2"), ("config2", "q4km")):
        types = synth.LAYER_TYPES[mode]
        ws = []
        for nm, n, k in shapes:
            w = synth.make_weight(g, types[nm], n, k)
            ws.append((w, [b.upload(w) for _ in range(copies)]))
        algo = sum(w.nbytes_device() if w.pk is not None else w.n * w.row_bytes for w, _ in ws)
        algo += sum((w.k // 256) * abi.Q8K_BYTES + w.n * 4 for w, _ in ws)
        t = timed(ws, copies * passes)
        for _, hh in ws:
            for h in hh:
                b.release(h)
        res[name] = dict(unit="layer (7 matvecs)", bytes=algo, us=round(t * 1e6, 2), GBs=round(algo / t / 1e9, 1),
                         frac=round(algo / t / 1e9 / HBM_PEAK_GBS, 4))
    return res


def gemm_roofline(b, nt: int = 128, copies: int = 8, reps: int = 64):
    """The prefill GEMM (k_gemm_panel, int8 MFMA) at config 4's widest contraction: 2 x 6144 rows
    of Q2_0C panel (gate and up stacked), K 2048, one 128-token chunk of Q8_K activations, through
    hymt2_hip_matvec; HIP events on the backend stream over launches rotating `copies` weight
    copies. int8 ops per launch = 2 * rows * K * tokens."""
    import torch
    from hymt2_amd import abi, synth
    s = synth.HYMT2_1_8B
    g = synth.rng(0x6E77)
    n, k = 2 * s.ffn, s.hidden
    w = synth.make_weight(g, abi.GT_Q2_0C, n, k)
    hs = [b.upload(w) for _ in range(copies)]
    stream = torch.cuda.ExternalStream(b.stream)
    act = torch.zeros(nt * (k // 256) * abi.Q8K_BYTES, dtype=torch.uint8, device="cuda")
    x = torch.randn(nt, k, device="cuda", dtype=torch.float32)
    out = torch.empty(nt * n, device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()
    b.quantize_q8k(x.data_ptr(), act.data_ptr(), k, nt)

    def launch(i):
        b.matvec(hs[i % copies], act.data_ptr(), out.data_ptr(), nt)

    for i in range(copies):
        launch(i)
    avg_s = _timed_launches(stream, launch, reps)
    for h in hs:
        b.release(h)
    ops = 2.0 * n * k * nt
    return dict(bound="mfma", achieved=round(ops / avg_s / 1e12, 1), peak=INT8_PEAK_TOPS, unit="TOP/s",
                frac=round(ops / avg_s / 1e12 / INT8_PEAK_TOPS, 4), avg_us=round(avg_s * 1e6, 2),
                ops_per_launch=int(ops), kernel="k_gemm_panel (int8 MFMA 16x16x64): 12288x2048 Q2_0C panel x "
                f"{nt} tokens", timing=f"HIP events on the backend stream over {reps} launches rotating {copies} "
                                       f"weight copies")


def config4(b):
    """BASELINE config 4 (hymt2_amd.synth.CONFIG4): the 1.8B-shaped model with Q2_0C weights, a
    1024-token prompt (random chat-template ids) in 128-token chunks on the device
    (hymt2_hip_generate_chunked: int8-MFMA GEMMs, causal GQA attention over the growing KV cache,
    LM head + argmax on the last position), then 256 greedy decode tokens. Prefill and decode are
    timed separately with HIP events on the backend stream. MFMA utilisation of the prefill =
    int8 ops of all layer contractions / (time x peak). The first greedy ids are checked against
    the reference's own greedy loop (tests/golden/baseline_config4.npz)."""
    from hymt2_amd import lib, synth
    cfg = synth.CONFIG4
    n_prompt, n_gen, chunk = cfg["n_prompt"], cfg["n_gen"], cfg["chunk"]
    t = time.time()
    model = synth.baseline_model(cfg, n_prompt + n_gen + 64)
    shape = model["shape"]
    log(f"config 4 model built in {time.time() - t:.1f} s")
    fm = lib.FusedModel(b, model)
    prompt, _ = synth.baseline_prompt(cfg)
    # warm: kernels loaded, graphs captured, every KV-cache and activation page touched by a whole
    # run; then three timed runs, the median run (by prefill time) reported
    fm.generate_device(prompt, n_gen, chunk=chunk)
    runs = [fm.generate_device(prompt, n_gen, chunk=chunk) for _ in range(3)]
    if any(not np.array_equal(r[0], runs[0][0]) for r in runs):
        raise RuntimeError("config 4: the timed runs' greedy ids differ")
    ids, st = sorted(runs, key=lambda r: r[1].prefill_ms)[1]
    f = np.load(os.path.join(ROOT, "tests", "golden", "baseline_config4.npz"), allow_pickle=False)
    if not (np.array_equal(f["prompt"], prompt) and np.array_equal(ids[:len(f["greedy"])], f["greedy"])):
        raise RuntimeError("config 4: greedy ids differ from the reference's (tests/golden/baseline_config4.npz)")

    def after(first2):
        """Logits of a fused_forward at position n_prompt + 1 after a two-id device run: they
        read every layer's K/V at all earlier positions, which the prefill wrote."""
        return fm.forward([int(first2[1])], n_prompt + 1, True).view(np.uint32)

    logits_pipe = after(ids)
    ids_step, st1 = fm.generate_device(prompt, 2, chunk=1)   # the same prompt one position per step
    logits_step = after(ids_step)
    depth = b.prefill_pipeline(1)                            # chunks one after another
    try:
        fm.generate_device(prompt[:chunk + 5], 2, chunk=chunk)
        ids_seq, st_seq = fm.generate_device(prompt, 2, chunk=chunk)
    finally:
        b.prefill_pipeline(depth)
    logits_seq = after(ids_seq)
    if not (np.array_equal(ids_seq, ids[:2]) and np.array_equal(ids_step, ids[:2]) and
            np.array_equal(logits_seq, logits_pipe) and np.array_equal(logits_step, logits_pipe)):
        raise RuntimeError("config 4: the pipelined, one-chunk-after-another and stepwise prefills disagree")
    weights = sum(L[nm].n * L[nm].k for L in model["layers"] for nm in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"))
    ops = 2.0 * weights * n_prompt
    pre_s = st.prefill_ms / 1e3
    wb = synth.model_weight_bytes(model)
    avg_pos = n_prompt + (n_gen - 1) / 2.0
    tok_bytes = wb["layers"] + wb["head"] + 2 * shape.n_layer * shape.kvdim * 2 * (avg_pos + 1)
    dec_tok_s = st.decode_steps / (st.decode_ms / 1e3)
    fm.close()
    return dict(workload=f"config4: Hy-MT2-1.8B-shaped Q2_0C, {n_prompt}-token random prompt in {chunk}-token "
                         f"chunks, then {n_gen} greedy tokens (device loop)",
                greedy_parity=f"first {len(f['greedy'])} ids identical to the reference's gen_ids at ISA scalar; "
                              f"logits at position {n_prompt + 1} bit-identical after the pipelined, the "
                              f"one-chunk-after-another and the stepwise prefill",
                prefill_schedule=f"{chunk}-token chunks pipelined over the layers, up to {depth} in flight "
                                 f"(chunk i's layer l in the launches of chunk i + 1's layer l - 1; the same bits "
                                 f"as one chunk after another)",
                timing="one whole warm-up run, then the median of three timed runs (by prefill time); HIP events "
                       "on the backend stream",
                prefill_tok_s=round(n_prompt / pre_s, 1), prefill_ms=round(st.prefill_ms, 3),
                prefill_sequential_tok_s=round(n_prompt / (st_seq.prefill_ms / 1e3), 1),
                prefill_int8_ops=int(ops), prefill_mfma_util=round(ops / pre_s / 1e12 / INT8_PEAK_TOPS, 4),
                prefill_stepwise_tok_s=round(st1.prefill_steps / (st1.prefill_ms / 1e3), 1),
                decode_tok_s=round(dec_tok_s, 2), decode_bytes_per_token=int(tok_bytes),
                decode_effective_GBs=round(tok_bytes * dec_tok_s / 1e9, 1),
                distinct_ids=len(set(ids.tolist())))


def q6k_head_leg(b, n_gen: int = 64, reps: int = 20):
    """The reference's own bench-model shape (tools/make_bench_gguf.c: the 1.8B shapes with
    STQ1_0 layers and a Q6_K tied embedding / LM head, 203 MB): device-loop decode after a
    64-token prompt, and the LM head matvec alone (Q6_K 120818 x 2048 through hymt2_hip_matvec on
    a Q8_K activation; HIP events on the backend stream, alternating two device copies of the
    head). Algorithmic head bytes = the Q6_K rows + the activation blocks + the logits."""
    import torch
    from hymt2_amd import abi, lib, synth
    shape = synth.ModelShape(ctx=64 + n_gen + 64)
    model = synth.make_model(shape, mode="stq", seed=3, head_type=abi.GT_Q6_K)
    prompt = synth.rand_prompt(synth.rng(1234), 64, shape.vocab)
    fm = lib.FusedModel(b, model)
    fm.generate_device(prompt[:8], 4)  # warm: kernels loaded, graphs captured
    ids, st = fm.generate_device(prompt, n_gen)
    w = model["outw"]
    stream = torch.cuda.ExternalStream(b.stream)
    act = torch.zeros((w.k // 256) * abi.Q8K_BYTES, dtype=torch.uint8, device="cuda")
    x = torch.randn(w.k, device="cuda", dtype=torch.float32)
    out = torch.empty(w.n, device="cuda", dtype=torch.float32)
    b.quantize_q8k(x.data_ptr(), act.data_ptr(), w.k, 1)
    # two device copies of the 203 MB head alternate (406 MB, beyond the 256 MB Infinity Cache)
    heads = [fm.outw, b.upload(w)]

    def launch(i):
        b.matvec(heads[i % 2], act.data_ptr(), out.data_ptr(), 1)

    for i in range(3):
        launch(i)
    avg_s = _timed_launches(stream, launch, reps)
    b.release(heads[1])
    algo = w.n * w.row_bytes + (w.k // 256) * abi.Q8K_BYTES + w.n * 4
    wb = synth.model_weight_bytes(model)
    dec = st.decode_steps / (st.decode_ms / 1e3)
    tok_bytes = wb["layers"] + wb["head"] + 2 * shape.n_layer * shape.kvdim * 2 * (64 + n_gen / 2.0)
    fm.close()
    return dict(workload="Hy-MT2-1.8B shapes, STQ1_0 layers, Q6_K tied embedding / LM head (the reference's "
                         "make_bench_gguf shape), 64 random prompt ids, device-loop greedy decode",
                decode_tok_s=round(dec, 2), decode_bytes_per_token=int(tok_bytes),
                decode_effective_GBs=round(tok_bytes * dec / 1e9, 1), distinct_ids=len(set(ids.tolist())),
                head_kernel="Q6_K LM head matvec 120818 x 2048 (hymt2_hip_matvec, one Q8_K token; two weight "
                            "copies alternate)",
                head_bytes=int(algo), head_us=round(avg_s * 1e6, 2), head_GBs=round(algo / avg_s / 1e9, 1),
                head_frac=round(algo / avg_s / 1e9 / HBM_PEAK_GBS, 4))


def summarize_trace(d: str):
    """Markdown table of a rocprofv3 --kernel-trace CSV (DIR/*kernel_trace.csv): per kernel the
    dispatches, average / min / max duration and share of GPU time; then, for the decode step's
    FFN-input kernel (the bench's roofline kernel), the average over the dispatches launched back
    to back by the roofline leg (each preceded by another dispatch of the same kernel) apart from
    the ones inside the decode graphs. No GPU needed."""
    import csv
    import glob
    fs = glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)
    if not fs:
        raise SystemExit(f"no *kernel_trace.csv under {d}")
    rows = []
    for f in fs:
        rows += list(csv.DictReader(open(f)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    dur = {}
    for r in rows:
        dur.setdefault(r["Kernel_Name"], []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    tot = sum(sum(v) for v in dur.values())
    print("| kernel | calls | avg us | min us | max us | % of GPU time |")
    print("|---|---:|---:|---:|---:|---:|")
    for k, v in sorted(dur.items(), key=lambda kv: -sum(kv[1]))[:24]:
        print(f"| `{k[:96]}` | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} | {100 * sum(v) / tot:.2f} |")
    # the FFN-input kernel is the RMSNorm-prologue decode matvec (k_mv1<0, 1, ITERS, 1>) that the
    # roofline leg launches back to back; the qkv matvec shares the form with other ITERS
    import re
    norm_mv = [k for k in dur if re.search(r"k_mv1<0, 1, \d+, 1>", k)]
    b2b = {k: sum(1 for i, r in enumerate(rows) if i and r["Kernel_Name"] == k and rows[i - 1]["Kernel_Name"] == k)
           for k in norm_mv}
    tgt = max(b2b, key=b2b.get) if b2b and max(b2b.values()) > 0 else None
    summary = {"kernel_avg_us": {k[:120]: round(sum(v) / len(v), 3) for k, v in dur.items() if "hy::" in k}}
    if tgt is None:
        print()
        print("warning: no back-to-back dispatches of an RMSNorm-prologue decode matvec (the roofline leg's "
              "FFN-input kernel) in this trace")
    else:
        alone, graph = [], []
        for i, r in enumerate(rows):
            if r["Kernel_Name"] != tgt:
                continue
            t = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
            (alone if i and rows[i - 1]["Kernel_Name"] == tgt else graph).append(t)
        print()
        print(f"`{tgt}`: {len(alone)} back-to-back dispatches (the roofline leg, hymt2_hip_ffn_in) average "
              f"{sum(alone) / len(alone):.2f} us; {len(graph)} dispatches inside the decode graphs average "
              f"{sum(graph) / max(len(graph), 1):.2f} us.")
        summary["ffn_in"] = dict(kernel=tgt, standalone_avg_us=round(sum(alone) / len(alone), 3),
                                 in_graph_avg_us=round(sum(graph) / max(len(graph), 1), 3), in_graph_dispatches=len(graph))
    # the longest run of pipelined-prefill dispatches (job-table kernels, with the chunks'
    # embedding lookups before them): per kernel and per launch step
    def pipe(n):
        return "_pipe" in n or "GemmLaunchT<24>" in n
    runs, cur = [], []
    for r in rows:
        n = r["Kernel_Name"]
        if pipe(n) or "k_embed_rows" in n:
            cur.append(r)
        elif cur:
            runs.append(cur)
            cur = []
    if cur:
        runs.append(cur)
    runs = [x for x in runs if any(pipe(r["Kernel_Name"]) for r in x)]
    if runs:
        main = max(runs, key=len)
        wall = (int(main[-1]["End_Timestamp"]) - int(main[0]["Start_Timestamp"])) / 1000.0
        acc = {}
        for r in main:
            n = r["Kernel_Name"].split("(")[0].replace("void ", "").replace("(anonymous namespace)::", "")
            if "GemmLaunchT<24>" in r["Kernel_Name"]:
                n = "k_gemm_panel<24, ...> (" + r["Kernel_Name"].split("<", 1)[1].split(">")[0] + ")"
            a = acc.setdefault(n, [0, 0.0])
            a[0] += 1
            a[1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
        ksum = sum(v[1] for v in acc.values())
        print()
        print(f"Pipelined prefill window: {len(main)} dispatches, {wall:.1f} us from the first start to the last end, "
              f"{ksum:.1f} us of kernel time.")
        print()
        print("| kernel | calls | total us | avg us | % of window kernel time |")
        print("|---|---:|---:|---:|---:|")
        for k, (c, s) in sorted(acc.items(), key=lambda kv: -kv[1][1]):
            print(f"| `{k[:96]}` | {c} | {s:.1f} | {s / c:.2f} | {100 * s / ksum:.1f} |")
        att = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0 for r in main
               if "k_attn_chunk_pipe" in r["Kernel_Name"] or "k_attn_chunk4_pipe" in r["Kernel_Name"]]
        if att:
            print()
            print("Chunk attention per launch step (us): " + " ".join(f"{x:.0f}" for x in att))
        # the decode that follows the window (config 4: 256 tokens at positions 1024-1279, 255
        # steps after the prompt's last forward): its split attention, per launch
        end = int(main[-1]["End_Timestamp"])
        after = [r for r in rows if int(r["Start_Timestamp"]) > end]
        dec = {}
        for name in ("k_attn_scores", "k_attn_out"):
            v = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0 for r in after
                 if name in r["Kernel_Name"]][:255 * 32]
            if v:
                dec[name] = (len(v), sum(v) / len(v))
        if dec:
            print()
            print("Split attention in the decode after the window: " +
                  ", ".join(f"{k} {n} launches {a:.2f} us" for k, (n, a) in dec.items()) +
                  f" ({sum(a for _, a in dec.values()):.2f} us a layer)")
            summary["decode_after_prefill"] = {k: dict(launches=n, avg_us=round(a, 3)) for k, (n, a) in dec.items()}
    print()
    print(json.dumps(summary))


def host_loop_rate(fm, prompt, n_tokens: int):
    """Decode rate of the reference host's own loop over the drop-in boundary: one
    fused_forward per token with the host embedding in (8 KB H2D), the 120818 logits out (483 KB
    D2H) and the argmax on the host (src/model.c:914-958). PCIe-inclusive, for comparison with the
    device-resident loop that `value` measures."""
    import numpy as np
    logits = fm.prefill(list(prompt), batch=16)
    pos = len(prompt)
    t0 = time.perf_counter()
    for _ in range(n_tokens):
        best = int(np.argmax(logits[:fm.vocab_out]))
        logits = fm.forward([best], pos, True)
        pos += 1
    dt = time.perf_counter() - t0
    return dict(value=round(n_tokens / dt, 2), unit="tok/s", tokens=n_tokens,
                note="hy_device_ops.fused_forward per token with logits D2H and host argmax")


def _in_graph_figure(algo: int):
    """The FFN-input kernel's average duration inside the decode graphs, from the committed
    kernel-trace summary of the decode bench (profiles/decode_config3_kernels.json, written by
    --summarize-trace from a rocprofv3 run of this bench): HIP events time graph launches, not the
    kernels inside them. None when the profile is missing."""
    p = os.path.join(ROOT, "profiles", "decode_config3_kernels.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        d = json.load(f).get("ffn_in")
    if not d:
        return None
    us = d["in_graph_avg_us"]
    return dict(avg_us=us, achieved=round(algo / (us * 1e-6) / 1e9, 1), frac=round(algo / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                kernel=d["kernel"], dispatches=d["in_graph_dispatches"], source="profiles/decode_config3_kernels.json")


def _pmc_traffic(kernel: str):
    """HBM bytes per launch of `kernel` measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    (profiles/traffic.json, scaled by the same counters on a copy kernel of known size), or
    None when not measured."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get(kernel, {}).get("hbm_bytes_per_launch")


def kernels_only(args):
    """Standalone launches for counter collection: the dominant kernel over rotating weight
    copies, then a plain copy kernel of known size (256 MiB read + 256 MiB written) that
    calibrates the FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    from hymt2_amd import lib
    shape, model = build_model(64)
    b = lib.Backend()
    roof = ffn_in_roofline(model, b, copies=64, passes=1)
    log(f"ffn_in: {roof['avg_us']} us, {roof['achieved']} GB/s")
    calibration_copy()
    b.close()


def calibration_copy():
    """The counter runs' calibration kernel: torch.neg over 64 Mi fp32 (268,435,456 B read and
    268,435,456 B written), whose FETCH_SIZE / WRITE_SIZE give the counters' scale."""
    import torch
    src = torch.randn(64 << 20, device="cuda", dtype=torch.float32)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    log("calibration copy: torch.neg over 67108864 fp32 (268435456 B read, 268435456 B written)")


def attn_traffic():
    """Decode steps for the attention kernels' counter passes, then the calibration copy: the
    config-3 model at positions 64-79 (k_attn1, one workgroup per head, short rows) and the
    config-4 model at positions 1024-1039 after its 1024-token prompt (the split form:
    k_attn_scores, k_attn_out)."""
    from hymt2_amd import lib, synth
    b = lib.Backend()
    for cfg, chunk in ((synth.CONFIG3, 64), (synth.CONFIG4, 128)):
        prompt, _ = synth.baseline_prompt(cfg)
        model = synth.baseline_model(cfg, len(prompt) + 128)
        fm = lib.FusedModel(b, model)
        log(f"{len(prompt)}-token prompt: model uploaded")
        fm.gen_begin(prompt, len(prompt) + 17)
        fm.gen_prefill(chunk)
        fm.gen_read(0, 1)
        log("prompt done")
        for _ in range(2):
            fm.gen_steps(8)
            fm.gen_read(0, 1)
            log("8 decode steps done")
        fm.close()
        del model
    calibration_copy()
    b.close()


def prefill_pass():
    """The config-4 prompt's pipelined chunked prefill alone, twice (hymt2_hip_gen_prefill, no
    decode step and so no graph replay): the launches the chunk kernels' counter passes read."""
    from hymt2_amd import lib, synth
    b = lib.Backend()
    cfg = synth.CONFIG4
    prompt, _ = synth.baseline_prompt(cfg)
    model = synth.baseline_model(cfg, len(prompt) + 64)
    fm = lib.FusedModel(b, model)
    log(f"{len(prompt)}-token prompt: model uploaded")
    for _ in range(2):
        fm.gen_begin(prompt, len(prompt) + 8)
        fm.gen_prefill(cfg["chunk"])
        fm.gen_read(0, 1)
        log("prefill done")
    fm.close()
    b.close()


def summarize_pmc(fetch_dir: str, write_dir: str):
    """HBM bytes per dispatch of every kernel in two rocprofv3 --pmc runs (FETCH_SIZE, then
    WRITE_SIZE; KiB per dispatch), each scaled by what the counter reads for the calibration copy
    (torch.neg of 268,435,456 B in and out). Prints a table and a JSON object."""
    import csv

    def load(d, counter):
        rows = list(csv.DictReader(open(os.path.join(d, "run_counter_collection.csv"))))
        acc = {}
        for r in rows:
            if r["Counter_Name"] != counter:
                continue
            a = acc.setdefault(r["Kernel_Name"], [0, 0.0])
            a[0] += 1
            a[1] += float(r["Counter_Value"])
        cal = [v[1] / v[0] for k, v in acc.items() if "neg" in k.lower()]
        if not cal:
            raise RuntimeError(f"no calibration kernel in {d}")
        scale = 268435456.0 / (max(cal) * 1024.0)
        return {k: (v[0], v[1] / v[0] * 1024.0 * scale) for k, v in acc.items()}, scale

    fetch, fs = load(fetch_dir, "FETCH_SIZE")
    write, ws = load(write_dir, "WRITE_SIZE")
    print(f"scale factors: FETCH_SIZE {fs:.4f}, WRITE_SIZE {ws:.4f}")
    print()
    print("| kernel | dispatches | fetch B / dispatch | write B / dispatch |")
    print("|---|---:|---:|---:|")
    out = {}
    for k in sorted(fetch, key=lambda k: -fetch[k][1]):
        if "neg" in k.lower():
            continue
        n, fb = fetch[k]
        wb = write.get(k, (0, 0.0))[1]
        out[k] = dict(dispatches=n, fetch_bytes=round(fb), write_bytes=round(wb))
        print(f"| `{k[:90]}` | {n} | {fb:,.0f} | {wb:,.0f} |")
    print()
    print(json.dumps(dict(fetch_scale=round(fs, 4), write_scale=round(ws, 4), kernels=out)))


def layer_sets_only():
    """The configs 0-2 matvec legs alone (for a kernel trace of their launches)."""
    from hymt2_amd import lib
    b = lib.Backend()
    print(json.dumps(layer_sets(b)), flush=True)
    b.close()


def host_leg_child(path: str, ctx: int, fused: bool, n_tokens: int, text: str):
    """In a fresh process: the reference's unchanged host (oracle/_ref/libhymt2_host.so, its
    sources linked with libhymt2_hip.a in place of src/cuda.c) on the GGUF with
    HYMT2_DEVICE=cuda, fused or per-op (HYMT2_FUSED=0), the ISA it detects; its own greedy loop
    gen_ids (src/model.c:914-958) on the chat text, as the CPU baseline runs it. Prints one JSON
    line: the model info, the ids and hymt2_model_stats."""
    from oracle import refbind
    os.environ.update(HYMT2_DEVICE="cuda", HYMT2_REPACK="1")
    os.environ.pop("HYMT2_ISA", None)
    if not fused:
        os.environ["HYMT2_FUSED"] = "0"
    L = refbind.load(refbind.HOST_LIB)
    isa = L.hymt2_isa().decode()
    threads = int(os.environ["HYMT2_THREADS"])  # the parent's choice (the host's physical cores)
    rm = refbind.RefModel(path, threads=threads, ctx=ctx, path=refbind.HOST_LIB)
    info = rm.info()
    rm.generate_text(text, 4)  # warm: graphs captured, page faults (the prompt KV is then reused)
    rm.logits([0])             # reset the prefix cache so the timed run prefills the whole prompt
    t0 = time.perf_counter()
    ids, st = rm.generate_text(text, n_tokens)
    wall = time.perf_counter() - t0
    rm.close()
    print(json.dumps(dict(info=info, isa=isa, threads=threads, ids=[int(i) for i in ids], stats=st, wall=wall)),
          flush=True)


def host_legs(path: str, ctx: int, prompt, text: str, gpu_ids, n_fused: int = 128, n_per_op: int = 32):
    """The reference host over this backend (host_leg_child), fused and per-op. The fused leg's
    ids must equal the device loop's (its numbers all come from the device; the host only takes
    the argmax); the per-op leg runs norms, RoPE, attention and the F16 head on the host at its
    ISA, so its ids follow that ISA's fp32 order (counted, not required)."""
    out = {}
    for name, fused, n in (("host_dropin", True, n_fused), ("per_op", False, n_per_op)):
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--host-leg", path, str(ctx),
                            "1" if fused else "0", str(n), text], capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            raise RuntimeError(f"{name} leg failed: {r.stdout[-2000:]} {r.stderr[-2000:]}")
        d = json.loads(r.stdout.strip().splitlines()[-1])
        st, ids = d["stats"], np.array(d["ids"], dtype=np.int32)
        if st["decode_tokens"] != n or st["prefill_tokens"] != len(prompt) or st["decode_ms"] <= 0:
            raise RuntimeError(f"{name} leg: {st}, expected a {len(prompt)}-token prompt and {n} tokens")
        m = min(len(ids), len(gpu_ids))
        agree = int(np.argmin(np.append(ids[:m] == gpu_ids[:m], False)))
        if fused and (agree != m or "gpu=hip+fused" not in d["info"]):
            raise RuntimeError(f"host_dropin leg: {d['info']}; ids agree with the device loop for {agree} of {m}")
        out[name] = dict(value=round(st["decode_tokens"] / (st["decode_ms"] / 1000.0), 2), unit="tok/s",
                         ms_per_token=round(st["decode_ms"] / st["decode_tokens"], 4),
                         prefill_tok_s=round(st["prefill_tokens"] / (st["prefill_ms"] / 1000.0), 1),
                         tokens=n, info=d["info"], isa=d["isa"], threads=d["threads"],
                         ids_agree_with_device_loop=f"{agree} of {m}",
                         note=("the reference's gen_ids with this backend linked in (HYMT2_DEVICE=cuda): "
                               + ("fused_forward per token, logits D2H, host argmax" if fused else
                                  "HYMT2_FUSED=0: the layer matvecs per op on the GPU (weight_out outputs), "
                                  "norms, RoPE, attention and the F16 head on the host")))
    return out


def cpu_baseline(model, prompt, text, gpu_ids, n_tokens: int, host: bool = True):
    """The reference's own greedy loop (gen_ids, src/model.c:914-958, compiled from the
    reference's sources into oracle/_ref/libhymt2_ref.so) on the host cores, on the same weights
    and the same 64 prompt ids: the chat text it is given encodes to exactly the GPU leg's prompt
    (checked), then n_tokens greedy tokens. HYMT2_DEVICE=cpu, HYMT2_REPACK=1, the ISA it detects,
    HYMT2_THREADS = the host's physical cores. Rate = decode tokens / decode time, as
    hymt2_model_stats and the reference's CLI report it (tools/hymt2_cli.c:92)."""
    from oracle import refbind
    from hymt2_amd import gguf
    if not refbind.available():
        raise RuntimeError("cpu baseline: oracle/_ref/libhymt2_ref.so is not built (run __graft_entry__.build() "
                           "where the reference tree is present, or pass --no-cpu)")
    os.environ.update(HYMT2_DEVICE="cpu", HYMT2_REPACK="1")
    os.environ.pop("HYMT2_ISA", None)
    L = refbind.load()
    isa = refbind.set_isa("auto")
    threads = int(os.environ.get("HYMT2_THREADS") or L.hy_physical_cpu_count())
    os.environ["HYMT2_THREADS"] = str(threads)
    ctx = len(prompt) + n_tokens + 64
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "cfg3.gguf")
        gguf.write_model(path, model)
        rm = refbind.RefModel(path, threads=threads, ctx=ctx)
        if not np.array_equal(rm.encode_chat(text), prompt):
            raise RuntimeError("cpu baseline: the chat text does not encode to the GPU leg's prompt ids")
        rm.generate_text(text, 4)  # warm: page faults, thread pool (the prompt KV is then reused)
        rm.logits([0])             # reset the prefix cache so the timed run prefills the whole prompt
        t0 = time.perf_counter()
        ids, st = rm.generate_text(text, n_tokens)
        wall = time.perf_counter() - t0
        info = rm.info()
        rm.close()
        legs = host_legs(path, ctx, prompt, text, gpu_ids) if host else {}
    if len(ids) != n_tokens or st["decode_tokens"] != n_tokens or st["decode_ms"] <= 0 or st["prefill_tokens"] != len(prompt):
        raise RuntimeError(f"cpu baseline: reference decoded {len(ids)} tokens ({st}), expected a "
                           f"{len(prompt)}-token prompt and {n_tokens} tokens")
    tok_s = st["decode_tokens"] / (st["decode_ms"] / 1000.0)
    n = min(len(ids), len(gpu_ids))
    agree = int(np.argmin(np.append(ids[:n] == gpu_ids[:n], False)))
    return dict(value=round(tok_s, 2), unit="tok/s", cores=threads, kind="reference",
                sample=f"reference hymt2 gen_ids ({info}, HYMT2_DEVICE=cpu, ISA {isa}): {st['prefill_tokens']}-token "
                       f"prompt then {st['decode_tokens']} greedy decode tokens of the same model and prompt ids, "
                       f"{wall:.1f} s wall",
                prefill_tok_s=round(st["prefill_tokens"] / (st["prefill_ms"] / 1000.0), 2),
                ids_agree_with_gpu=f"{agree} of {n} leading ids (the auto ISA's fp32 order differs from the "
                                   f"scalar order the GPU matches)"), legs


def boundary_costs(vocab: int, hidden: int, reps: int = 200):
    """Per-token pieces the reference host's loop adds to the device step (src/cuda.c:339-421 and
    src/model.c:945-948 for the reference's own backend): the input block H2D (the host's
    embedding row, the position and its RoPE row: 16 KB from pinned staging), the logits D2H into
    the host's pageable buffer (vocab floats), and an argmax over them (numpy's; the reference's is
    a scalar loop). Each timed alone with a synchronisation, as the loop runs them."""
    import torch
    dev = torch.empty(vocab, dtype=torch.float32, device="cuda")
    pageable = torch.empty(vocab, dtype=torch.float32)
    hin = torch.empty(4096, dtype=torch.float32, pin_memory=True)
    din = torch.empty(4096, dtype=torch.float32, device="cuda")
    lg = np.random.default_rng(0).standard_normal(vocab).astype(np.float32)

    def per_call_us(fn):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        return round((time.perf_counter() - t0) / reps * 1e6, 1)

    def h2d():
        din.copy_(hin, non_blocking=True)
        torch.cuda.synchronize()

    return dict(input_h2d_us=per_call_us(h2d), logits_d2h_us=per_call_us(lambda: pageable.copy_(dev)),
                host_argmax_us=per_call_us(lambda: np.argmax(lg)), hidden=hidden, vocab=vocab)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-tokens", type=int, default=128)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-layer-sets", action="store_true", help="skip the configs 0-2 matvec timings")
    ap.add_argument("--no-config4", action="store_true", help="skip the config 4 chunked-prefill run")
    ap.add_argument("--config4-only", action="store_true",
                    help="only the config 4 chunked-prefill run and the prefill GEMM timing (for profiling)")
    ap.add_argument("--kernels-only", action="store_true",
                    help="only the standalone kernel launches used for rocprofv3 counter passes")
    ap.add_argument("--no-q6k", action="store_true", help="skip the Q6_K-head model leg")
    ap.add_argument("--q6k-only", action="store_true", help="only the Q6_K-head model leg (for profiling)")
    ap.add_argument("--host-leg", nargs=5, metavar=("GGUF", "CTX", "FUSED", "TOKENS", "TEXT"),
                    help=argparse.SUPPRESS)  # child process of the cpu_baseline leg's host legs
    ap.add_argument("--no-host-legs", action="store_true", help="skip the reference-host legs (host_dropin, per_op)")
    ap.add_argument("--attn-traffic", action="store_true",
                    help="only decode steps of the config-3 and config-4 models and the calibration copy (counter runs)")
    ap.add_argument("--layer-sets-only", action="store_true", help="only the configs 0-2 matvec legs (kernel trace)")
    ap.add_argument("--prefill-pass", action="store_true",
                    help="only the config-4 prompt's pipelined prefill, twice, no decode (counter runs)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print HBM bytes per dispatch from two rocprofv3 --pmc output directories and exit")
    ap.add_argument("--summarize-trace", metavar="DIR",
                    help="print the kernel table of a rocprofv3 --kernel-trace output directory and exit")
    args = ap.parse_args()
    if args.host_leg:
        g, ctx, fused, n, text = args.host_leg
        host_leg_child(g, int(ctx), fused == "1", int(n), text)
        return
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the Hy-MT2 token loop at batch 1 runs on a single MI355X "
              "(multi-GPU figures are not part of this build); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    from hymt2_amd import lib, synth

    if args.kernels_only:
        kernels_only(args)
        return
    if args.attn_traffic:
        attn_traffic()
        return
    if args.prefill_pass:
        prefill_pass()
        return
    if args.layer_sets_only:
        layer_sets_only()
        return
    if args.q6k_only:
        b = lib.Backend()
        print(json.dumps(q6k_head_leg(b)), flush=True)
        b.close()
        return
    if args.config4_only:
        b = lib.Backend()
        c4 = config4(b)
        c4["gemm_roofline"] = gemm_roofline(b)
        print(json.dumps(c4), flush=True)
        b.close()
        return
    prompt, text = synth.baseline_prompt(synth.CONFIG3)
    n_total = len(prompt) + args.warmup + args.steps + 1  # steps fill positions 1..n_total-1
    ctx = (max(n_total, len(prompt) + 33) + 63) // 64 * 64  # also room for the host-loop sample
    t = time.time()
    shape, model = build_model(ctx)
    log(f"model built in {time.time() - t:.1f} s")
    b = lib.Backend()
    fm = lib.FusedModel(b, model)
    log(f"backend {b.info}; weights uploaded")
    fm.gen_begin(prompt, n_total)
    fm.gen_steps(len(prompt))          # prefill, one position per step (untimed)
    fm.gen_read(0, 1)
    fm.gen_steps(args.warmup)          # warmup decode steps
    fm.gen_read(0, 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fm.gen_steps(args.steps)
    fm.gen_read(0, 1)                  # waits for the stream
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ids = fm.gen_read(len(prompt), args.warmup + args.steps + 1)
    parity = check_against_fixture(prompt, ids)
    log(f"greedy ids identical to the reference for the first {parity['checked_ids']}")
    tok_s = args.steps / dt
    wb = synth.model_weight_bytes(model)
    log(f"decode: {tok_s:.1f} tok/s ({dt / args.steps * 1e3:.3f} ms/token), {len(set(ids.tolist()))} distinct ids")
    host = host_loop_rate(fm, prompt, 32)
    log(f"host-driven loop (fused_forward + logits D2H + host argmax): {host['value']} tok/s")
    roof = ffn_in_roofline(model, b)
    log(f"ffn_in kernel: {roof['avg_us']} us, {roof['achieved']} GB/s")
    head = head_roofline(fm, b)
    log(f"head kernel: {head['avg_us']} us, {head['achieved']} GB/s")
    sets = None
    if not args.no_layer_sets:
        sets = layer_sets(b)
        log(f"layer sets: {sets}")
    q6 = None
    if not args.no_q6k:
        q6 = q6k_head_leg(b)
        log(f"q6k head model: {q6}")
    c4 = None
    if not args.no_config4:
        c4 = config4(b)
        c4["gemm_roofline"] = gemm_roofline(b)
        log(f"config 4: {c4}")
    costs = boundary_costs(shape.vocab, shape.hidden)
    log(f"boundary pieces per token: {costs}")
    cpu, legs = None, {}
    if not args.no_cpu:
        t = time.time()
        cpu, legs = cpu_baseline(model, prompt, text, ids, args.cpu_tokens, host=not args.no_host_legs)
        log(f"cpu baseline in {time.time() - t:.1f} s: {cpu}")
        for k, v in legs.items():
            log(f"{k}: {v}")
    if "host_dropin" in legs:
        hd = legs["host_dropin"]
        hd["over_device_loop_us_per_token"] = round((hd["ms_per_token"] - dt / args.steps * 1e3) * 1e3, 1)
        hd["pieces"] = costs
    avg_pos = len(prompt) + args.warmup + (args.steps - 1) / 2.0
    kv_read = 2 * shape.n_layer * shape.kvdim * 2 * (avg_pos + 1)
    token_bytes = wb["layers"] + wb["head"] + kv_read
    out = {
        "metric": "decode tok/s @ batch 1 (1.8B STQ1_0) + achieved HBM GB/s vs peak",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8xint2->int32 + fp32 (bf16 KV, f16 head)", "data": "synthetic",
        "config": {"workload": "config3: Hy-MT2-1.8B-shaped STQ1_0 greedy decode at batch 1 on the device-resident "
                               "loop (32 layers, hidden 2048, 16/4 heads, hd 128, ffn 6144, vocab 120818, tied F16 "
                               "head, bf16 KV), 64 random prompt ids, random seeded weights",
                   "global_batch": 1, "prompt": len(prompt), "parallelism": "single GPU",
                   "decode_bytes_per_token": int(token_bytes),
                   "decode_effective_GBs": round(token_bytes * tok_s / 1e9, 1),
                   "distinct_ids": len(set(ids.tolist())), "greedy_parity": parity},
        "roofline": roof,
        "head_roofline": head,
        "host_loop": host,
        "host_dropin": legs.get("host_dropin"),
        "per_op": legs.get("per_op"),
        "layer_sets": sets,
        "q6k_head_model": q6,
        "config4_prefill": c4,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    fm.close()
    b.close()


if __name__ == "__main__":
    main()
