"""ctypes mirrors of the reference's device-backend ABI.

These structs must stay byte-identical to the C declarations in ``include/hymt2_hip.h``,
which in turn mirror the reference's ``src/internal.h`` and ``src/device.h``:

* ``WeightT``     <- ``weight_t``        (src/internal.h:48-61)
* ``FusedLayer``  <- ``hy_fused_layer``  (src/device.h:44-47)
* ``FusedArgs``   <- ``hy_fused_args``   (src/device.h:49-59)
* ``DeviceOps``   <- ``hy_device_ops``   (src/device.h:70-80)
* ``Q8K_BYTES``   <- ``sizeof(q8k_block)`` (src/internal.h:29-41)

The C side checks the sizes and offsets with static_asserts; ``tests/test_abi.py`` checks the
Python side against them through ``hymt2_hip_abi_layout``.
"""
import ctypes as C

QK_K = 256
MAX_BATCH = 16  # src/internal.h:12
MAX_CHUNK = 128  # tokens per call the backend accepts (HYMT2_HIP_MAX_CHUNK)
Q8K_BYTES = 576

# GGUF tensor type codes (src/internal.h:46)
GT_F32, GT_F16, GT_Q8_0, GT_Q4_K, GT_Q6_K, GT_Q2_0C, GT_STQ1_0 = 0, 1, 8, 12, 14, 40, 43

ROW_BYTES_PER_BLOCK = {GT_F32: (1, 4), GT_F16: (1, 2), GT_Q8_0: (32, 34), GT_Q4_K: (256, 144),
                       GT_Q6_K: (256, 210), GT_STQ1_0: (256, 42), GT_Q2_0C: (512, 130)}


def row_bytes(gtype: int, k: int) -> int:
    """Bytes of one GGUF row of ``k`` weights (src/kernels.c:113-124)."""
    blk, nbytes = ROW_BYTES_PER_BLOCK[gtype]
    return (k // blk) * nbytes


class WeightT(C.Structure):
    _fields_ = [("data", C.c_void_p), ("type", C.c_int), ("k", C.c_int), ("n", C.c_int),
                ("row_bytes", C.c_size_t), ("pk", C.c_void_p), ("ps", C.c_void_p),
                ("pshift", C.c_int), ("poff", C.c_int), ("gpu", C.c_void_p)]


class FusedLayer(C.Structure):
    _fields_ = [("wq", C.c_void_p), ("wk", C.c_void_p), ("wv", C.c_void_p), ("wo", C.c_void_p),
                ("wg", C.c_void_p), ("wu", C.c_void_p), ("wd", C.c_void_p),
                ("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
                ("q_norm", C.c_void_p), ("k_norm", C.c_void_p)]


class FusedArgs(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layer", "hidden", "ffn", "heads", "kv_heads", "hdim",
                                        "qdim", "kvdim", "ctx", "rope_half", "nt", "pos0")] + [
        ("eps", C.c_float), ("want_logits", C.c_int), ("layers", C.POINTER(FusedLayer)),
        ("outw", C.c_void_p), ("out_norm", C.c_void_p), ("rope_cos", C.c_void_p),
        ("rope_sin", C.c_void_p), ("h", C.c_void_p), ("logits", C.c_void_p)]


_VP = C.c_void_p
DESTROY_FN = C.CFUNCTYPE(None, _VP)
UPLOAD_FN = C.CFUNCTYPE(_VP, _VP, C.POINTER(WeightT))
RELEASE_FN = C.CFUNCTYPE(None, _VP)
MATMUL_FN = C.CFUNCTYPE(C.c_bool, _VP, C.POINTER(_VP), C.POINTER(_VP), C.c_int, _VP, C.c_int)
IS_SW_FN = C.CFUNCTYPE(C.c_bool, _VP)
WEIGHT_OUT_FN = C.CFUNCTYPE(_VP, _VP)
PREPARE_FN = C.CFUNCTYPE(C.c_bool, _VP, C.POINTER(FusedArgs))
FORWARD_FN = C.CFUNCTYPE(C.c_bool, _VP, C.POINTER(FusedArgs))


class DeviceOps(C.Structure):
    _fields_ = [("destroy_impl", DESTROY_FN), ("upload", UPLOAD_FN), ("release", RELEASE_FN),
                ("matmul", MATMUL_FN), ("is_software", IS_SW_FN), ("weight_out", WEIGHT_OUT_FN),
                ("fused_prepare", PREPARE_FN), ("fused_forward", FORWARD_FN)]


def abi_layout() -> dict:
    """Sizes/offsets of the Python mirrors, compared with the C side in tests."""
    return {
        "weight_t": C.sizeof(WeightT), "weight_t.row_bytes": WeightT.row_bytes.offset,
        "weight_t.pk": WeightT.pk.offset, "weight_t.gpu": WeightT.gpu.offset,
        "hy_fused_layer": C.sizeof(FusedLayer),
        "hy_fused_args": C.sizeof(FusedArgs), "hy_fused_args.eps": FusedArgs.eps.offset,
        "hy_fused_args.layers": FusedArgs.layers.offset, "hy_fused_args.logits": FusedArgs.logits.offset,
        "hy_device_ops": C.sizeof(DeviceOps), "q8k_block": Q8K_BYTES,
    }
