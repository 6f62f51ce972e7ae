"""CPU checks of the C ABI: libmoe_hip.so loads, exports every function
include/moe_hip.h declares, its struct layouts are the reference's, and its
argument validation rejects bad calls before touching a GPU."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import moe_hip as mh
from abi_types import FFNWeights, ForwardCache, Matrix, ModelConfig, MoEWeights
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "moe_hip.h")
REF_INCLUDE = "/root/reference/include"


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(moe_\w+)\s*\(", text, re.M)
    return sorted(set(names))


def test_library_exports_every_declared_function():
    lib = mh.lib()
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding types every one of them
    assert not [n for n in names if n not in mh.SIGNATURES]


LAYOUT_PROGRAM = r"""
#include <stdio.h>
#include <stddef.h>
%s
int main(void) {
    printf("%%zu %%zu %%zu %%zu %%zu\n", sizeof(Matrix), sizeof(FFNWeights), sizeof(MoEWeights),
           sizeof(ModelConfig), sizeof(ForwardCache));
    printf("%%zu %%zu %%zu %%zu %%zu %%zu\n", offsetof(MoEWeights, W_router),
           offsetof(MoEWeights, n_experts), offsetof(MoEWeights, top_k),
           offsetof(ModelConfig, ffn_hidden), offsetof(ForwardCache, router_probs),
           offsetof(ForwardCache, expert_ids));
    return 0;
}
"""


def compile_layout(includes, flags, tmp_path):
    src = tmp_path / "layout.c"
    exe = tmp_path / "layout"
    src.write_text(LAYOUT_PROGRAM % includes)
    subprocess.run(["gcc", "-std=c11", *flags, str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    return [int(v) for v in out]


def ctypes_layout():
    return [C.sizeof(Matrix), C.sizeof(FFNWeights), C.sizeof(MoEWeights), C.sizeof(ModelConfig),
            C.sizeof(ForwardCache), MoEWeights.W_router.offset, MoEWeights.n_experts.offset,
            MoEWeights.top_k.offset, ModelConfig.ffn_hidden.offset,
            ForwardCache.router_probs.offset, ForwardCache.expert_ids.offset]


def test_header_layout_matches_ctypes(tmp_path):
    got = compile_layout('#include "moe_hip.h"', ["-I" + os.path.join(ROOT, "include")], tmp_path)
    assert got == ctypes_layout()


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="reference headers not present")
def test_header_layout_matches_reference(tmp_path):
    """The reference's own headers give the same sizes and offsets, and
    moe_hip.h compiles after them (it reuses their types)."""
    inc = '#include "transformer.h"\n#include "moe_hip.h"'
    got = compile_layout(inc, ["-I" + REF_INCLUDE, "-I" + os.path.join(ROOT, "include")],
                         tmp_path)
    assert got == ctypes_layout()


def test_argument_validation_without_gpu():
    lib = mh.lib()
    h = C.c_void_p()
    assert lib.moe_hip_layer_create(0, 512, 4, 2, C.byref(h)) == 1        # bad shape
    assert lib.moe_hip_layer_create(128, 512, 4, 5, C.byref(h)) == 1      # k > E
    assert lib.moe_hip_layer_create(96, 512, 4, 2, C.byref(h)) == 2       # d % 64
    assert lib.moe_hip_layer_create(128, 48, 4, 2, C.byref(h)) == 2       # F % 32
    assert lib.moe_hip_layer_create(128, 512, 5000, 2, C.byref(h)) == 2   # E > 4096
    assert lib.moe_hip_layer_create(128, 512, 300, 257, C.byref(h)) == 2  # top_k > 256
    assert b"must be 0" in lib.moe_hip_last_error_message() or lib.moe_hip_last_error() == 2
    assert lib.moe_hip_forward(None, None, None, None, None) == 1
    assert lib.moe_hip_set_expert_path(7) == 1
    assert lib.moe_hip_error_string(4) == b"device out of memory"


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is visible")
def test_no_gpu_is_reported_not_faked():
    lib = mh.lib()
    assert lib.moe_hip_init(0) == 5
    buf = np.zeros(4, np.float32)
    assert lib.moe_hip_memcpy(buf.ctypes.data_as(C.c_void_p), buf.ctypes.data_as(C.c_void_p),
                              16, 1) == 5
