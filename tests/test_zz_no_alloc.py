"""hymt2_hip_matmul_static, the per-op matmul that allocates nothing (its device staging is a
static array per GPU), against the vtable's matmul (hy_device_ops.matmul, whose staging the
context allocates) and the oracle, bit for bit: two groups in a row, the second smaller, with
outputs in host buffers and in weight_out buffers; a group beyond the static staging is refused
and the context stays usable."""
import ctypes as C

import numpy as np
import pytest

from hymt2_amd import abi, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def static_matmul(backend, hs, outs, xq, nt):
    ws = (C.c_void_p * len(hs))(*hs)
    os_ = (C.c_void_p * len(outs))(*outs)
    return backend.L.hymt2_hip_matmul_static(backend.impl, ws, os_, len(hs), xq.ctypes.data, nt)


def test_matmul_static_matches_matmul(backend):
    g = synth.rng(91)
    groups = [  # (weights, tokens): a q/k/v group at the 1.8B shapes, then a smaller mixed group
        ([synth.make_weight(g, abi.GT_STQ1_0, 2048, 2048), synth.make_weight(g, abi.GT_STQ1_0, 512, 2048),
          synth.make_weight(g, abi.GT_STQ1_0, 512, 2048)], 16),
        ([synth.make_weight(g, abi.GT_Q4_K, 300, 1024), synth.make_weight(g, abi.GT_Q6_K, 77, 1024),
          synth.make_weight(g, abi.GT_Q2_0C, 256, 1024)], 3),
    ]
    for ws, nt in groups:
        hs = [backend.upload(w) for w in ws]
        try:
            x = synth.activations(g, nt, ws[0].k)
            xq = O.quantize_q8k(x)
            want = backend.matmul(hs, [w.n for w in ws], xq, nt)
            got = [np.zeros((nt, w.n), np.float32) for w in ws]
            assert static_matmul(backend, hs, [o.ctypes.data for o in got], xq, nt), backend.last_error()
            for w, a, b in zip(ws, got, want):
                assert np.array_equal(bits(a), bits(b))
                assert np.array_equal(bits(a), bits(O.matvec(w, x, xq, nt)))
            # the first output into its weight_out buffer (written by the kernels), the rest by copy
            op = backend.ops.weight_out(hs[0])
            got2 = [np.zeros((nt, w.n), np.float32) for w in ws]
            outs = [op] + [o.ctypes.data for o in got2[1:]]
            assert static_matmul(backend, hs, outs, xq, nt), backend.last_error()
            first = np.ctypeslib.as_array(C.cast(op, C.POINTER(C.c_float)), shape=(16 * ws[0].n,))
            assert np.array_equal(bits(first[:nt * ws[0].n].reshape(nt, ws[0].n)), bits(want[0]))
            for a, b in zip(got2[1:], want[1:]):
                assert np.array_equal(bits(a), bits(b))
        finally:
            for h in hs:
                backend.release(h)


def test_matmul_static_refuses_oversized_groups(backend):
    g = synth.rng(92)
    w = synth.make_weight(g, abi.GT_STQ1_0, 40000, 256)  # 40000 rows x 128 tokens x 4 B > 16 MiB
    h = backend.upload(w)
    try:
        x = synth.activations(g, 128, 256)
        xq = O.quantize_q8k(x)
        out = np.zeros((128, w.n), np.float32)
        assert not static_matmul(backend, [h], [out.ctypes.data], xq, 128)
        assert "static scratch" in backend.last_error()
        small = np.zeros((2, w.n), np.float32)  # still usable
        assert static_matmul(backend, [h], [small.ctypes.data], xq[:2], 2), backend.last_error()
        assert np.array_equal(bits(small), bits(O.matvec(w, x[:2], xq[:2], 2)))
    finally:
        backend.release(h)
