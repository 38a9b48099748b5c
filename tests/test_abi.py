"""The C-ABI boundary without a GPU: libhymt2_hip.so loads, exports every entry point that
include/hymt2_hip.h declares (and nothing else), its struct layouts equal the reference's own
declarations (src/internal.h:29-61, src/device.h:44-80), and the two drop-in entry points
behave as the reference's CUDA ones do when no device or host is present (src/cuda.c:18-34,
:151-167). No GPU work is launched."""
import ctypes as C
import os
import re
import subprocess

import pytest

from conftest import ROOT
from hymt2_amd import abi, lib

HEADER = os.path.join(ROOT, "include", "hymt2_hip.h")
HELPERS = os.path.join(ROOT, "tests", "helpers")
REF_SRC = "/root/reference/src"


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^HYMT2_HIP_API\s+[\w\s]+?\**\s*(\w+)\s*\(", text, re.M)))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    return sorted({ln.split()[-1] for ln in out.splitlines() if " T " in ln})


def test_header_declares_the_python_export_list():
    assert declared() == sorted(lib.EXPORTS)


def test_library_exports_exactly_the_declared_symbols():
    lib.load()
    assert exported() == declared()


def test_abi_layout_matches_python_mirrors():
    assert lib.abi_layout() == abi.abi_layout()


def _layout(tmp_path, name, extra):
    exe = tmp_path / name
    subprocess.run(["gcc", "-std=gnu11", os.path.join(HELPERS, "abi_layout.c"), "-o", str(exe)] + extra, check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    return {k: int(v) for k, v in (kv.split("=") for kv in out.split())}


def test_public_header_layout_matches_library(tmp_path):
    assert _layout(tmp_path, "pub", ["-I", os.path.join(ROOT, "include")]) == lib.abi_layout()


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_SRC, "device.h")), reason="reference tree not present")
def test_layout_matches_reference_declarations(tmp_path):
    assert _layout(tmp_path, "ref", ["-DFROM_REFERENCE", "-I", REF_SRC]) == lib.abi_layout()


def test_probe_reports_kfd_without_initialising_the_gpu():
    L = lib.load()
    buf = C.create_string_buffer(8)
    r = L.hy_cuda_probe(buf, 8)
    assert r == (1 if os.access("/dev/kfd", os.R_OK | os.W_OK) else 0)
    assert buf.value.decode() == str(r)


def test_create_without_host_returns_null_with_message():
    """Loaded on its own (no reference host providing hy_device_wrap), hy_cuda_create refuses
    before touching the GPU, with a message, as the reference's returns NULL when its runtime is
    unusable."""
    L = lib.load()
    info = C.create_string_buffer(256)
    assert not L.hy_cuda_create(b"cuda", info, 256)
    assert b"hy_device_wrap" in info.value


def test_header_compiles_as_c_and_links(tmp_path):
    src = tmp_path / "use.c"
    src.write_text('#include "hymt2_hip.h"\n#include <stdio.h>\n'
                   'int main(void){ char b[8]; char info[128] = ""; const hymt2_device_ops *o = hymt2_hip_ops();\n'
                   ' int p = hy_cuda_probe(b, 8); hy_device *d = hy_cuda_create("cuda", info, sizeof info);\n'
                   ' printf("%d %d %d\\n", p, d == NULL, o && o->upload && o->fused_forward); return 0; }\n')
    exe = tmp_path / "use"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src),
                    "-L", os.path.dirname(lib.LIB_PATH), "-lhymt2_hip", "-o", str(exe)], check=True)
    env = dict(os.environ, LD_LIBRARY_PATH=os.path.dirname(lib.LIB_PATH))
    out = subprocess.run([str(exe)], capture_output=True, text=True, env=env, check=True).stdout.split()
    assert out[1:] == ["1", "1"]


def test_vtable_is_complete():
    ops = lib.load().hymt2_hip_ops().contents
    for name, _ in abi.DeviceOps._fields_:
        assert C.cast(getattr(ops, name), C.c_void_p).value, name
