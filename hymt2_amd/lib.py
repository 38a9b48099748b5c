"""ctypes binding of libhymt2_hip.so and a host-side mirror of the reference's fused token loop.

The library is the product: a C-ABI HIP backend (include/hymt2_hip.h). This module only loads
it and marshals numpy buffers; there is no CPU fallback. If the shared library is missing,
:func:`load` raises.

:class:`FusedModel` mirrors what the reference host does around the device for one model
(src/model.c): it uploads every weight through the backend's ``upload`` (device_upload_all,
:384-406), prepares the fused path (enable_fused, :325-381), embeds tokens on the host
(dequant_row, :802), calls ``fused_forward`` per chunk of at most MAX_BATCH tokens
(forward_tokens, :904-909) and picks greedy tokens with the first-index argmax (gen_ids,
:945-948). ``generate_device`` instead runs the whole greedy loop on the GPU.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import abi

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhymt2_hip.so")


class GenStats(C.Structure):
    _fields_ = [("prefill_ms", C.c_double), ("decode_ms", C.c_double),
                ("prefill_steps", C.c_int), ("decode_steps", C.c_int), ("cached_tokens", C.c_int)]


class GenOpts(C.Structure):
    _fields_ = [("stop_ids", C.c_void_p), ("n_stop", C.c_int), ("chunk", C.c_int), ("reuse_prefix", C.c_int)]


_lib = None

# embedding types the device loop dequantizes on the GPU
EMBED_TYPES = (abi.GT_F16, abi.GT_F32, abi.GT_Q8_0, abi.GT_Q4_K, abi.GT_Q6_K)


def load():
    """Load libhymt2_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() or "
                           f"`make -C hymt2_amd/csrc`")
    L = C.CDLL(LIB_PATH)
    vp, i = C.c_void_p, C.c_int
    sig = {
        "hy_cuda_probe": (i, [C.c_char_p, i]),
        "hy_cuda_create": (vp, [C.c_char_p, C.c_char_p, C.c_size_t]),
        "hymt2_hip_open": (vp, [C.c_char_p, C.c_size_t]),
        "hymt2_hip_ops": (C.POINTER(abi.DeviceOps), []),
        "hymt2_hip_last_error": (i, [vp, C.c_char_p, i]),
        "hymt2_hip_abi_layout": (i, [C.c_char_p, i]),
        "hymt2_hip_stream": (vp, [vp]),
        "hymt2_hip_quantize_q8k": (i, [vp, vp, vp, i, i]),
        "hymt2_hip_matvec": (i, [vp, vp, vp, vp, i]),
        "hymt2_hip_selftest_f16": (i, [vp, vp, vp, i]),
        "hymt2_hip_selftest_expf": (i, [vp, vp, vp, i]),
        "hymt2_hip_selftest_sqsum": (i, [vp, vp, i, i, vp, i]),
        "hymt2_hip_selftest_mfma": (i, [vp, vp, vp, vp, i]),
        "hymt2_hip_generate": (i, [vp, C.POINTER(abi.FusedArgs), vp, i, vp, i, i, vp, C.POINTER(GenStats)]),
        "hymt2_hip_gen_begin": (i, [vp, C.POINTER(abi.FusedArgs), vp, i, vp, i, i]),
        "hymt2_hip_gen_steps": (i, [vp, i]),
        "hymt2_hip_gen_prefill": (i, [vp, C.POINTER(abi.FusedArgs), i]),
        "hymt2_hip_generate_chunked": (i, [vp, C.POINTER(abi.FusedArgs), vp, i, vp, i, i, i, vp,
                                           C.POINTER(GenStats)]),
        "hymt2_hip_gen_read": (i, [vp, vp, i, i]),
        "hymt2_hip_generate_ids": (i, [vp, C.POINTER(abi.FusedArgs), vp, i, vp, i, i, C.POINTER(GenOpts), vp,
                                       C.POINTER(GenStats)]),
        "hymt2_hip_head": (i, [vp, vp, vp, vp, C.c_float, vp, i, vp]),
        "hymt2_hip_ffn_in": (i, [vp, vp, vp, vp, vp, C.c_float, vp]),
        "hymt2_hip_matmul_static": (C.c_bool, [vp, C.POINTER(vp), C.POINTER(vp), i, vp, i]),
        "hymt2_hip_attn_split_from": (i, [vp, i]),
        "hymt2_hip_prefill_pipeline": (i, [vp, i]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    _lib = L
    return L


EXPORTS = ["hy_cuda_create", "hy_cuda_probe", "hymt2_hip_open", "hymt2_hip_ops", "hymt2_hip_last_error",
           "hymt2_hip_abi_layout", "hymt2_hip_stream", "hymt2_hip_quantize_q8k", "hymt2_hip_matvec",
           "hymt2_hip_selftest_f16", "hymt2_hip_selftest_expf", "hymt2_hip_selftest_sqsum", "hymt2_hip_selftest_mfma", "hymt2_hip_generate", "hymt2_hip_gen_begin",
           "hymt2_hip_gen_steps", "hymt2_hip_gen_read", "hymt2_hip_head", "hymt2_hip_ffn_in",
           "hymt2_hip_gen_prefill", "hymt2_hip_generate_chunked", "hymt2_hip_matmul_static",
           "hymt2_hip_attn_split_from", "hymt2_hip_prefill_pipeline", "hymt2_hip_generate_ids"]


def abi_layout() -> dict:
    buf = C.create_string_buffer(1024)
    load().hymt2_hip_abi_layout(buf, 1024)
    return {k: int(v) for k, v in (kv.split("=") for kv in buf.value.decode().split())}


def _p(a):
    return None if a is None else a.ctypes.data


class Backend:
    """One backend context (the impl pointer of the hy_device_ops vtable)."""

    def __init__(self):
        L = load()
        info = C.create_string_buffer(256)
        self.impl = L.hymt2_hip_open(info, 256)
        self.info = info.value.decode(errors="replace")
        if not self.impl:
            raise RuntimeError(f"hymt2_hip_open failed: {self.info}")
        self.ops = L.hymt2_hip_ops().contents
        self.L = L

    def attn_split_from(self, pos: int):
        """Single-token forwards at positions >= pos use the split attention (-1: default)."""
        if self.L.hymt2_hip_attn_split_from(self.impl, pos) != 0:
            raise RuntimeError("hymt2_hip_attn_split_from failed")

    def prefill_pipeline(self, depth: int) -> int:
        """Chunks in flight in the device loop's chunked prefill (1: one after another; < 1:
        query). Returns the previous depth."""
        return int(self.L.hymt2_hip_prefill_pipeline(self.impl, depth))

    def last_error(self) -> str:
        buf = C.create_string_buffer(512)
        self.L.hymt2_hip_last_error(self.impl, buf, 512)
        return buf.value.decode(errors="replace")

    @property
    def stream(self) -> int:
        return self.L.hymt2_hip_stream(self.impl)

    def upload(self, w) -> int:
        """synth.Weight -> device weight handle (hy_dweight*)."""
        wt = abi.WeightT(_p(w.data), w.type, w.k, w.n, w.row_bytes, _p(w.pk), _p(w.ps), w.pshift, w.poff, None)
        h = self.ops.upload(self.impl, C.byref(wt))
        if not h:
            raise RuntimeError(f"upload failed: {self.last_error()}")
        return h

    def release(self, h: int):
        if h:
            self.ops.release(h)

    def matmul(self, handles, ns, xq: np.ndarray, nt: int):
        """Per-op path: returns [out_i (nt, n_i)] for weights sharing the Q8_K activations xq."""
        outs = [np.zeros((nt, n), dtype=np.float32) for n in ns]
        ws = (C.c_void_p * len(handles))(*handles)
        os_ = (C.c_void_p * len(outs))(*[o.ctypes.data for o in outs])
        if not self.ops.matmul(self.impl, ws, os_, len(handles), xq.ctypes.data, nt):
            raise RuntimeError(f"matmul failed: {self.last_error()}")
        return outs

    def quantize_q8k(self, x_dev: int, act_dev: int, k: int, nt: int):
        if self.L.hymt2_hip_quantize_q8k(self.impl, x_dev, act_dev, k, nt) != 0:
            raise RuntimeError(f"quantize_q8k failed: {self.last_error()}")

    def matvec(self, h: int, act_dev: int, out_dev: int, nt: int):
        if self.L.hymt2_hip_matvec(self.impl, h, act_dev, out_dev, nt) != 0:
            raise RuntimeError(f"matvec failed: {self.last_error()}")

    def close(self):
        if getattr(self, "impl", None):
            self.ops.destroy_impl(self.impl)
            self.impl = None


class FusedModel:
    """A synthetic model resident on the device behind the fused path."""

    def __init__(self, backend: Backend, model: dict):
        self.b = backend
        self.model = model
        s = model["shape"]
        self.shape = s
        self.handles = []
        layers = (abi.FusedLayer * s.n_layer)()
        for i, L in enumerate(model["layers"]):
            fl = layers[i]
            for nm in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
                h = backend.upload(L[nm])
                self.handles.append(h)
                setattr(fl, nm, h)
            for nm in ("attn_norm", "ffn_norm", "q_norm", "k_norm"):
                setattr(fl, nm, L[nm].ctypes.data)
        self.outw = backend.upload(model["outw"])
        self.handles.append(self.outw)
        if model["embd"] is model["outw"]:
            self.embd_dev = self.outw
        elif model["embd"].type in EMBED_TYPES:
            self.embd_dev = backend.upload(model["embd"])
            self.handles.append(self.embd_dev)
        else:
            self.embd_dev = None
        self.layers = layers
        self.args = abi.FusedArgs(n_layer=s.n_layer, hidden=s.hidden, ffn=s.ffn, heads=s.heads,
                                  kv_heads=s.kv_heads, hdim=s.hdim, qdim=s.qdim, kvdim=s.kvdim, ctx=s.ctx,
                                  rope_half=s.rope_half, nt=0, pos0=0, eps=s.eps, want_logits=0,
                                  layers=layers, outw=self.outw, out_norm=model["out_norm"].ctypes.data,
                                  rope_cos=model["rope_cos"].ctypes.data, rope_sin=model["rope_sin"].ctypes.data,
                                  h=None, logits=None)
        if not backend.ops.fused_prepare(backend.impl, C.byref(self.args)):
            raise RuntimeError(f"fused_prepare failed: {backend.last_error()}")
        self.h = np.zeros((abi.MAX_CHUNK, s.hidden), dtype=np.float32)
        self.logits = np.zeros(model["outw"].n, dtype=np.float32)
        self.vocab_out = model["vocab_out"]

    def embed(self, toks) -> np.ndarray:
        """The host embedding of forward_batch (dequant_row, src/model.c:802)."""
        from .synth import dequant_rows
        return dequant_rows(self.model["embd"], toks)

    def forward(self, toks, pos0: int, want_logits: bool = True):
        """One fused_forward of len(toks) <= MAX_CHUNK tokens; returns logits or None."""
        nt = len(toks)
        self.h[:nt] = self.embed(toks)
        a = self.args
        a.nt, a.pos0, a.want_logits = nt, pos0, int(want_logits)
        a.h, a.logits = self.h.ctypes.data, self.logits.ctypes.data
        if not self.b.ops.fused_forward(self.b.impl, C.byref(a)):
            raise RuntimeError(f"fused_forward failed: {self.b.last_error()}")
        return self.logits.copy() if want_logits else None

    def prefill(self, prompt, batch: int = abi.MAX_BATCH):
        logits = None
        for i in range(0, len(prompt), batch):
            chunk = prompt[i:i + batch]
            logits = self.forward(chunk, i, want_logits=(i + len(chunk) == len(prompt)))
        return logits

    def generate_host(self, prompt, n_gen: int, batch: int = abi.MAX_BATCH):
        """The reference host's greedy loop over fused_forward (host argmax per token)."""
        logits = self.prefill(list(prompt), batch)
        pos = len(prompt)
        out = []
        for i in range(n_gen):
            best = int(np.argmax(logits[:self.vocab_out]))
            out.append(best)
            if i + 1 == n_gen:
                break
            logits = self.forward([best], pos, True)
            pos += 1
        return np.array(out, dtype=np.int32)

    def generate_device(self, prompt, n_gen: int, chunk: int = 1):
        """Greedy loop entirely on the device; the prompt runs as single-token steps (chunk 1)
        or as chunks of up to `chunk` positions. Returns (ids, GenStats)."""
        if self.embd_dev is None:
            raise ValueError("device generation needs an F16/F32/Q8_0/Q4_K/Q6_K embedding table")
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_gen, dtype=np.int32)
        st = GenStats()
        rc = self.b.L.hymt2_hip_generate_chunked(self.b.impl, C.byref(self.args), self.embd_dev, self.vocab_out,
                                                 prompt.ctypes.data, len(prompt), n_gen, chunk, out.ctypes.data,
                                                 C.byref(st))
        if rc != n_gen:
            raise RuntimeError(f"hymt2_hip_generate failed ({rc}): {self.b.last_error()}")
        return out, st

    def generate_ids(self, prompt, max_tokens: int, stop_ids=(), chunk: int = 1, reuse_prefix: bool = False):
        """The reference's greedy loop gen_ids (src/model.c:914-958) on the device: ids before a
        stop id (or max_tokens of them), the prompt in chunks of `chunk`, optionally reusing the
        K/V prefix of the previous call's sequence. Returns (ids, GenStats)."""
        if self.embd_dev is None:
            raise ValueError("device generation needs an F16/F32/Q8_0/Q4_K/Q6_K embedding table")
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        stop = np.ascontiguousarray(stop_ids, dtype=np.int32)
        out = np.zeros(max(max_tokens, 1), dtype=np.int32)
        opts = GenOpts(stop.ctypes.data if len(stop) else None, len(stop), chunk, int(reuse_prefix))
        st = GenStats()
        rc = self.b.L.hymt2_hip_generate_ids(self.b.impl, C.byref(self.args), self.embd_dev, self.vocab_out,
                                             prompt.ctypes.data, len(prompt), max_tokens, C.byref(opts),
                                             out.ctypes.data, C.byref(st))
        if rc < 0:
            raise RuntimeError(f"hymt2_hip_generate_ids failed ({rc}): {self.b.last_error()}")
        return out[:rc].copy(), st

    def gen_begin(self, prompt, n_total: int):
        if self.embd_dev is None:
            raise ValueError("device generation needs an F16/F32/Q8_0/Q4_K/Q6_K embedding table")
        self._prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        rc = self.b.L.hymt2_hip_gen_begin(self.b.impl, C.byref(self.args), self.embd_dev, self.vocab_out,
                                          self._prompt.ctypes.data, len(self._prompt), n_total)
        if rc != 0:
            raise RuntimeError(f"gen_begin failed ({rc}): {self.b.last_error()}")

    def gen_prefill(self, chunk: int):
        rc = self.b.L.hymt2_hip_gen_prefill(self.b.impl, C.byref(self.args), chunk)
        if rc != 0:
            raise RuntimeError(f"gen_prefill failed ({rc}): {self.b.last_error()}")

    def gen_steps(self, n: int):
        rc = self.b.L.hymt2_hip_gen_steps(self.b.impl, n)
        if rc != 0:
            raise RuntimeError(f"gen_steps failed ({rc}): {self.b.last_error()}")

    def gen_read(self, first: int, count: int) -> np.ndarray:
        out = np.zeros(count, dtype=np.int32)
        if self.b.L.hymt2_hip_gen_read(self.b.impl, out.ctypes.data, first, count) != count:
            raise RuntimeError(f"gen_read failed: {self.b.last_error()}")
        return out

    def close(self):
        for h in self.handles:
            self.b.release(h)
        self.handles = []
