"""ctypes binding of the reference library built from its own sources (oracle/_ref/):
TEST INFRASTRUCTURE ONLY.

``_ref/libhymt2_ref.so`` is the reference's C host + CPU kernels compiled by oracle/Makefile
straight from the read-only reference tree. Tests use it to pin the oracle bit-for-bit, and
bench.py's cpu_baseline leg times it. ``_ref/libhymt2_host.so`` is the reference's libhymt2 built
with its own flags (hidden visibility; only the public HYMT2_API symbols exported) and the HIP
backend's static archive linked in place of src/cuda.c (the drop-in, exercised by GPU tests).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_LIB = os.path.join(HERE, "_ref", "libhymt2_ref.so")
HOST_LIB = os.path.join(HERE, "_ref", "libhymt2_host.so")

_libs = {}

# The chat template of the reference's greedy loop (src/model.c:915-916).
CHAT_PRE = "<\uff5chy_begin\u2581of\u2581sentence\uff5c><\uff5chy_User\uff5c>"
CHAT_POST = "<\uff5chy_Assistant\uff5c>"


def available(path: str = REF_LIB) -> bool:
    return os.path.exists(path)


def load(path: str = REF_LIB):
    if path in _libs:
        return _libs[path]
    if not os.path.exists(path):
        raise RuntimeError(f"{path} not built (make -C oracle ref)")
    L = C.CDLL(path)
    vp, i, f = C.c_void_p, C.c_int, C.c_float
    sig = {
        "kernels_init": (None, []), "kernels_set_isa": (C.c_bool, [C.c_char_p]), "kernels_isa": (C.c_char_p, []),
        "quantize_q8k": (None, [vp, i, vp]), "panel_repack_rows": (None, [vp, vp, vp, i, i]),
        "matmul_rows": (None, [vp, i, i, vp, vp, i, vp]), "dequant_row": (None, [vp, i, vp]),
        "f16_to_f32": (f, [C.c_uint16]), "f32_to_bf16": (C.c_uint16, [f]),
        "dot_bf16": (f, [vp, vp, i]), "axpy_bf16": (None, [vp, vp, f, i]),
        "hymt2_model_load": (vp, [C.c_char_p, i, i, C.c_char_p, i]), "hymt2_model_free": (None, [vp]),
        "hymt2_debug_logits": (C.POINTER(C.c_float), [vp, vp, i, C.POINTER(C.c_int)]),
        "hymt2_debug_logits_stepwise": (C.POINTER(C.c_float), [vp, vp, i, C.POINTER(C.c_int)]),
        "hymt2_model_info": (i, [vp, C.c_char_p, i]),
        "hymt2_debug_device_matmul": (i, [C.c_char_p, C.c_uint, vp, i, i, vp, i, vp]),
        "hymt2_debug_matmul": (i, [C.c_uint, vp, i, i, vp, i, vp, i]),
        "hy_physical_cpu_count": (i, []),
        "hymt2_debug_generate_ids": (i, [vp, C.c_char_p, vp, i]),
        "hymt2_debug_encode": (i, [vp, C.c_char_p, C.POINTER(C.POINTER(C.c_int))]),
        "hymt2_model_stats": (None, [vp, C.POINTER(i), C.POINTER(i), C.POINTER(C.c_double), C.POINTER(i),
                                     C.POINTER(C.c_double)]),
        "hymt2_isa": (C.c_char_p, []),
    }
    for name, (res, args) in sig.items():
        if hasattr(L, name):
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
    if hasattr(L, "kernels_init"):  # internal symbol: exported by _ref/libhymt2_ref.so only
        L.kernels_init()
    _libs[path] = L
    return L


def set_isa(name: str, path: str = REF_LIB) -> str:
    L = load(path)
    L.kernels_set_isa(name.encode())
    return L.kernels_isa().decode()


def weight_t(w, use_panel: bool):
    """synth.Weight -> the reference's weight_t (hymt2_amd.abi.WeightT layout)."""
    from hymt2_amd import abi
    wt = abi.WeightT(w.data.ctypes.data if w.data is not None else None, w.type, w.k, w.n, w.row_bytes,
                     w.pk.ctypes.data if (use_panel and w.pk is not None) else None,
                     w.ps.ctypes.data if (use_panel and w.ps is not None) else None,
                     w.pshift if use_panel else 0, w.poff if use_panel else 0, None)
    wt._keep = (w.data, w.pk, w.ps)
    return wt


def quantize_q8k(x: np.ndarray, path: str = REF_LIB) -> np.ndarray:
    from oracle.oracle import q8k_empty
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
    nt, k = x.shape
    y = q8k_empty(nt * (k // 256))
    L = load(path)
    for t in range(nt):
        L.quantize_q8k(x[t].ctypes.data, k, y[t * (k // 256):].ctypes.data)
    return y


def matvec(w, xf, xq, nt: int, use_panel=True, path: str = REF_LIB) -> np.ndarray:
    L = load(path)
    out = np.zeros((nt, w.n), dtype=np.float32)
    wt = weight_t(w, use_panel)
    xf_c = None if xf is None else np.ascontiguousarray(xf, dtype=np.float32)
    L.matmul_rows(C.byref(wt), 0, w.n, None if xf_c is None else xf_c.ctypes.data,
                  None if xq is None else xq.ctypes.data, nt, out.ctypes.data)
    return out


def panel_repack(w, path: str = REF_LIB):
    L = load(path)
    nb = w.k // 256
    pk = np.zeros((w.n, nb, 64), dtype=np.uint8)
    ps = np.zeros((w.n, nb), dtype=np.float32)
    wt = weight_t(w, False)
    L.panel_repack_rows(C.byref(wt), pk.ctypes.data, ps.ctypes.data, 0, w.n)
    return pk, ps


def dequant(w, path: str = REF_LIB) -> np.ndarray:
    L = load(path)
    out = np.zeros((w.n, w.k), dtype=np.float32)
    wt = weight_t(w, False)
    for r in range(w.n):
        L.dequant_row(C.byref(wt), r, out[r].ctypes.data)
    return out


class RefModel:
    """A GGUF loaded by the reference host (hymt2_model_load)."""

    def __init__(self, gguf_path: str, threads: int = 1, ctx: int = 0, path: str = REF_LIB):
        self.L = load(path)
        err = C.create_string_buffer(512)
        self.m = self.L.hymt2_model_load(gguf_path.encode(), threads, ctx, err, 512)
        if not self.m:
            raise RuntimeError("hymt2_model_load failed: " + err.value.decode(errors="replace"))

    def info(self) -> str:
        buf = C.create_string_buffer(256)
        self.L.hymt2_model_info(self.m, buf, 256)
        return buf.value.decode()

    def logits(self, ids, stepwise=False) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        nv = C.c_int(0)
        fn = self.L.hymt2_debug_logits_stepwise if stepwise else self.L.hymt2_debug_logits
        p = fn(self.m, ids.ctypes.data, len(ids), C.byref(nv))
        return np.ctypeslib.as_array(p, shape=(nv.value,)).copy()

    def greedy(self, prompt, n_gen: int) -> np.ndarray:
        """Greedy ids by re-running the prompt + generated ids (hymt2_debug_logits resets the
        cache each call); first-index argmax as in src/model.c:945-948."""
        ids = list(int(t) for t in prompt)
        out = []
        for _ in range(n_gen):
            lg = self.logits(ids)
            best = int(np.argmax(lg))  # numpy argmax returns the first maximal index
            out.append(best)
            ids.append(best)
        return np.array(out, dtype=np.int32)

    def encode(self, text: str) -> np.ndarray:
        """The reference tokenizer's ids of `text` (tok_encode via hymt2_debug_encode)."""
        p = C.POINTER(C.c_int)()
        n = self.L.hymt2_debug_encode(self.m, text.encode(), C.byref(p))
        ids = np.array([p[i] for i in range(n)], dtype=np.int32)
        libc = C.CDLL(None)
        libc.free.argtypes = [C.c_void_p]
        libc.free(C.cast(p, C.c_void_p))
        return ids

    def encode_chat(self, user: str) -> np.ndarray:
        """Ids of the chat prompt gen_ids builds around `user` (src/model.c:915-921)."""
        return self.encode(CHAT_PRE + user + CHAT_POST)

    def generate_text(self, text: str, max_tokens: int):
        """The reference's own greedy loop (gen_ids via hymt2_debug_generate_ids) and its
        timing counters (hymt2_model_stats)."""
        ids = np.zeros(max_tokens, dtype=np.int32)
        n = self.L.hymt2_debug_generate_ids(self.m, text.encode(), ids.ctypes.data, max_tokens)
        pt, ct, dt = C.c_int(), C.c_int(), C.c_int()
        pms, dms = C.c_double(), C.c_double()
        self.L.hymt2_model_stats(self.m, C.byref(pt), C.byref(ct), C.byref(pms), C.byref(dt), C.byref(dms))
        return ids[:max(n, 0)], dict(prefill_tokens=pt.value, cached_tokens=ct.value, prefill_ms=pms.value,
                                     decode_tokens=dt.value, decode_ms=dms.value)

    def close(self):
        if self.m:
            self.L.hymt2_model_free(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
