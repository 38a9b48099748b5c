"""ctypes binding of liboracle.so: TEST INFRASTRUCTURE ONLY.

The CPU restatement of the reference's scalar path (hymt2_oracle.c). Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and only as the
checker. The product package (hymt2_amd) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q8K_DTYPE = np.dtype([("qp", np.int8, 256), ("d", np.float32), ("sum", np.int32),
                      ("bsums", np.int16, 16), ("pad", np.uint8, 24), ("qs", np.int8, 256)])
assert Q8K_DTYPE.itemsize == 576


class OcWeight(C.Structure):
    _fields_ = [("type", C.c_int), ("k", C.c_int), ("n", C.c_int), ("data", C.c_void_p),
                ("pk", C.c_void_p), ("ps", C.c_void_p), ("pshift", C.c_int), ("poff", C.c_int)]


class OcLayer(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p)] + [(n, OcWeight) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")]


class OcModel(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layer", "hidden", "ffn", "heads", "kv_heads", "hdim", "ctx",
                                        "rope_half", "vocab_out")] + [
        ("eps", C.c_float), ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
        ("embd", OcWeight), ("outw", OcWeight), ("out_norm", C.c_void_p), ("layers", C.POINTER(OcLayer))]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run `make -C oracle`)")
        L = C.CDLL(LIB_PATH)
        vp, i, f = C.c_void_p, C.c_int, C.c_float
        sig = {
            "oc_f16_to_f32": (f, [C.c_uint16]), "oc_f32_to_bf16": (C.c_uint16, [f]),
            "oc_quantize_q8k": (None, [vp, i, vp]), "oc_panel_repack": (None, [C.POINTER(OcWeight), vp, vp, i, i]),
            "oc_dequant_row": (None, [C.POINTER(OcWeight), i, vp]),
            "oc_matvec": (None, [C.POINTER(OcWeight), vp, vp, i, vp]),
            "oc_block_ints": (None, [C.POINTER(OcWeight), vp, i, i, vp]),
            "oc_dot_bf16": (f, [vp, vp, i]), "oc_axpy_bf16": (None, [vp, vp, f, i]),
            "oc_rope_tables": (None, [i, i, i, f, f, vp, vp]),
            "oc_state_new": (vp, [C.POINTER(OcModel)]), "oc_state_free": (None, [vp]),
            "oc_forward": (i, [vp, vp, i, i, i, vp]), "oc_state_hidden": (vp, [vp]),
            "oc_argmax": (i, [vp, i]), "oc_generate": (i, [vp, vp, i, i, i, vp]),
            "oc_gen_ids": (i, [vp, vp, i, i, i, vp, i, vp, C.POINTER(i)]),
            "oc_set_threads": (None, [i]), "oc_rmsnorm": (None, [vp, vp, vp, i, f]), "oc_expf_n": (None, [vp, vp, i]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().oc_expf_n(x.ctypes.data, y.ctypes.data, x.size)
    return y


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty_like(x)
    lib().oc_rmsnorm(x.ctypes.data, w.ctypes.data, y.ctypes.data, x.size, eps)
    return y


def q8k_empty(nblocks: int) -> np.ndarray:
    return np.zeros(nblocks, dtype=Q8K_DTYPE)


def quantize_q8k(x: np.ndarray) -> np.ndarray:
    """fp32 [nt, k] -> Q8_K records [nt * k/256]."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
    nt, k = x.shape
    y = q8k_empty(nt * (k // 256))
    for t in range(nt):
        lib().oc_quantize_q8k(x[t].ctypes.data, k, y[t * (k // 256):].ctypes.data)
    return y


def oc_weight(w) -> OcWeight:
    """hymt2_amd.synth.Weight -> OcWeight (keeps references alive on the struct)."""
    ow = OcWeight(w.type, w.k, w.n, _p(w.data), _p(w.pk), _p(w.ps), w.pshift, w.poff)
    ow._keep = (w.data, w.pk, w.ps)
    return ow


def panel_repack(w):
    nb = w.k // 256
    pk = np.zeros((w.n, nb, 64), dtype=np.uint8)
    ps = np.zeros((w.n, nb), dtype=np.float32)
    ow = OcWeight(w.type, w.k, w.n, _p(w.data), None, None, 0, 0)
    lib().oc_panel_repack(C.byref(ow), pk.ctypes.data, ps.ctypes.data, 0, w.n)
    return pk, ps


def matvec(w, xf: np.ndarray | None, xq: np.ndarray | None, nt: int) -> np.ndarray:
    out = np.zeros((nt, w.n), dtype=np.float32)
    ow = oc_weight(w)
    xf_c = None if xf is None else np.ascontiguousarray(xf, dtype=np.float32)
    lib().oc_matvec(C.byref(ow), _p(xf_c), _p(xq), nt, out.ctypes.data)
    return out


def block_ints(w, xq: np.ndarray, nt: int, kind: int) -> np.ndarray:
    nb = w.k // 256
    out = np.zeros((nt, w.n, nb), dtype=np.int32)
    ow = oc_weight(w)
    lib().oc_block_ints(C.byref(ow), xq.ctypes.data, nt, kind, out.ctypes.data)
    return out


def dequant(w) -> np.ndarray:
    out = np.zeros((w.n, w.k), dtype=np.float32)
    ow = oc_weight(w)
    for r in range(w.n):
        lib().oc_dequant_row(C.byref(ow), r, out[r].ctypes.data)
    return out


class OracleModel:
    """A model held by the oracle: KV cache and scratch live in C."""

    def __init__(self, model: dict, threads: int = 0):
        s = model["shape"]
        self.model = model
        layers = (OcLayer * s.n_layer)()
        keep = []
        for i, L in enumerate(model["layers"]):
            ol = layers[i]
            for nm in ("attn_norm", "ffn_norm", "q_norm", "k_norm"):
                setattr(ol, nm, L[nm].ctypes.data)
            for nm in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
                ow = oc_weight(L[nm])
                keep.append(ow)
                setattr(ol, nm, ow)
        m = OcModel(s.n_layer, s.hidden, s.ffn, s.heads, s.kv_heads, s.hdim, s.ctx, s.rope_half,
                    model["vocab_out"], s.eps, model["rope_cos"].ctypes.data, model["rope_sin"].ctypes.data,
                    oc_weight(model["embd"]), oc_weight(model["outw"]), model["out_norm"].ctypes.data, layers)
        self._keep = (layers, keep, m)
        if threads:
            lib().oc_set_threads(threads)
        self.state = lib().oc_state_new(C.byref(m))
        self.vocab_n = model["outw"].n

    def __del__(self):
        try:
            if getattr(self, "state", None):
                lib().oc_state_free(self.state)
                self.state = None
        except Exception:  # interpreter shutdown
            pass

    def forward(self, toks, pos0: int, want_logits=True):
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        logits = np.zeros(self.vocab_n, dtype=np.float32)
        if lib().oc_forward(self.state, toks.ctypes.data, len(toks), pos0, int(want_logits), logits.ctypes.data):
            raise ValueError(f"oc_forward rejected nt={len(toks)} pos0={pos0} (1 <= nt <= 16, pos0 + nt <= ctx)")
        return logits

    def hidden(self, nt: int) -> np.ndarray:
        s = self.model["shape"]
        ptr = lib().oc_state_hidden(self.state)
        return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_float)), shape=(nt * s.hidden,)).copy()

    def generate(self, prompt, n_gen: int, batch: int = 1) -> np.ndarray:
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_gen, dtype=np.int32)
        if lib().oc_generate(self.state, prompt.ctypes.data, len(prompt), n_gen, batch, out.ctypes.data) < 0:
            raise ValueError("oc_generate: prompt + generated ids exceed ctx, or an id is out of range")
        return out

    def gen_ids(self, prompt, max_tokens: int, stop_ids=(), batch: int = 16):
        """gen_ids (src/model.c:914-958) from the prompt ids: (ids before a stop id, positions of
        the prompt whose K/V this state's cache kept from the previous gen_ids call)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        stop = np.ascontiguousarray(stop_ids, dtype=np.int32)
        out = np.zeros(max(max_tokens, 1), dtype=np.int32)
        keep = C.c_int(0)
        n = lib().oc_gen_ids(self.state, prompt.ctypes.data, len(prompt), max_tokens, batch,
                             stop.ctypes.data if len(stop) else None, len(stop), out.ctypes.data, C.byref(keep))
        if n < 0:
            raise ValueError(f"oc_gen_ids: {n}")
        return out[:n].copy(), keep.value
