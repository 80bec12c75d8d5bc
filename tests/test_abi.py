"""CPU checks of the C-ABI boundary: the library loads, exports every symbol
include/*.h declares, the name registry covers the reference kernel names,
and argument validation reports errors without touching a GPU."""
import ctypes
import glob
import os
import re

import pytest

from conftest import ROOT
import ubridge_amd
from ubridge_amd import _lib, registry


def declared_symbols():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", src, re.M):
            if not m.group(0).startswith("typedef"):  # function-pointer types
                names.append(m.group(1))
    return sorted(set(names))


def test_header_parses():
    names = declared_symbols()
    assert "ubridge_qmatmul" in names and "dequantize_block_q8_0_bf16" in names


@pytest.mark.parametrize("name", declared_symbols())
def test_symbol_exported(name):
    assert hasattr(_lib.lib, name), f"{name} declared in include/ but not exported"


def test_reference_quant_names_registered():
    # the quant module names of src/device_executor.rs:295-308
    for q in ("q8_0", "q4_k"):
        for t in ("f16", "bf16", "f32"):
            assert registry.has_function(f"dequantize_block_{q}_{t}")
            assert registry.has_function(f"quantize_block_{q}_{t}")
    with pytest.raises(KeyError):
        registry.get_function("no_such_kernel", "quant")


def test_argument_errors_without_gpu():
    lib = _lib.lib
    lib.dequantize_block_q8_0_f32(None, None, 64, None)
    assert lib.ubridge_last_error() == 1
    lib.dequantize_block_q4_k_bf16(ctypes.c_void_p(256), ctypes.c_void_p(512), 100, None)
    assert lib.ubridge_last_error() == 1  # 100 is not a multiple of 256
    assert lib.ubridge_last_error() == 0  # reading clears it
    rc = lib.ubridge_qmatmul(12, ctypes.c_void_p(256), ctypes.c_void_p(256), 0, ctypes.c_void_p(256),
                             0, 1, 16, 300, ctypes.c_void_p(256), 1 << 20, None)
    assert rc == 1 and b"K=300" in lib.ubridge_last_error_string()
    lib.ubridge_last_error()
    lib.quantize_block_q4_k_f32(None, None, 0, 0, None)
    assert lib.ubridge_last_error() == 3



def test_status_returning_moe_errors_without_gpu():
    # topsaten_moe_wrapper.cpp:80-216: int status instead of void + last_error
    from ubridge_amd import moe  # noqa: F401  (registers the signatures)
    lib = _lib.lib
    p = ctypes.c_void_p(256)
    rc = lib.topsaten_fused_moe_gemm(p, p, p, p, p, p, p, p, 0, 2, 16, 4, 64, 64, 8, 8, None)
    assert rc == 3 and b"dtype_code 8" in lib.ubridge_last_error_string()
    lib.ubridge_last_error()
    rc = lib.topsaten_moe_align_block_size(p, p, p, p, 4, 2, 0, 16, None)
    assert rc == 1 and lib.ubridge_last_error() == 1
    rc = lib.topsaten_topk_softmax_f32(p, p, p, None, 4, 8, 2, 1, None)
    assert rc == 1 and b"token_expert_indices" in lib.ubridge_last_error_string()
    lib.ubridge_last_error()
    assert lib.topsaten_topk_softmax_f32(p, p, p, None, 0, 8, 2, 1, None) == 0
    lib.topsaten_release_graph_workspace_pool(None)
    assert lib.ubridge_last_error() == 0


def test_plain_c_caller(tmp_path):
    # include/ubridge_hip.h compiles as C99 and a C program links and calls the
    # library (no GPU work: version, argument errors, knobs)
    import shutil
    import subprocess
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    libdir = os.path.dirname(_lib.lib._name)
    exe = str(tmp_path / "c_caller")
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "abi_c_caller.c"), "-o", exe, "-L", libdir, "-lubridge_hip",
           "-Wl,-rpath," + libdir]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK"), r.stdout + r.stderr

def test_workspace_size():
    ws = _lib.lib.ubridge_qmatmul_workspace_size
    assert ws(12, 1, 4096) >= 4096 + 16 * 4 + 128 * 4  # codes, d per 256, sums per 32
    assert ws(2, 16, 14336) >= 16 * 14336 * (1 + 8 / 32)


def test_tune_knobs_roundtrip():
    from ubridge_amd import ops
    for name in ops.TUNE_KNOBS:
        old = ops.tune_get(name)
        ops.tune_set(name, 2)
        assert ops.tune_get(name) == 2
        ops.tune_set(name, old)
        assert ops.tune_get(name) == old
    with pytest.raises(Exception):
        ops.tune_set("no_such_knob", 1)
    assert _lib.lib.ubridge_last_error() == 0


def test_gemm_launch_params_struct_and_cache():
    # GEMM_OP_PARAS (src/gemm_tuner.rs:222-258): 132-byte C struct, one
    # cached entry per shape (the pointer is stable), this library's tile
    from ubridge_amd import ops
    import torch
    assert ctypes.sizeof(ops.GemmOpParas) == 132
    assert ops.GemmOpParas.sip_m.offset == 32 and ops.GemmOpParas.alpha.offset == 88
    p1 = _lib.lib.ubridge_get_gemm_launch_params(5, 15, 1, 2048, 4096, 14336, 0)
    p2 = _lib.lib.ubridge_get_gemm_launch_params(5, 15, 1, 2048, 4096, 14336, 0)
    assert ctypes.addressof(p1.contents) == ctypes.addressof(p2.contents)
    p = p1.contents
    assert (p.input_dtype, p.output_dtype, p.input_batch, p.input_m, p.input_k, p.input_n) == \
        (5, 5, 1, 2048, 4096, 14336)
    assert (p.sip_m, p.sip_n, p.sip_k) == (256, 256, 64)  # 8 x 56 = 448 tiles of 256 x 256
    assert p.rhs_multicore == 1 and p.lhs_multicore == 0 and p.alpha == 1.0
    small = ops.get_gemm_launch_params(torch.bfloat16, "i8", 1, 64, 256, 384, 1)
    # quantized weights: the pipelined kernel's split-K tile, 64 x 256 up to 64 rows (2 tiles)
    assert (small.sip_m, small.sip_n, small.rhs_transpose) == (64, 256, 1)
    dense = ops.get_gemm_launch_params(torch.bfloat16, torch.bfloat16, 1, 64, 256, 384, 1)
    assert (dense.sip_m, dense.sip_n) == (128, 128)
    # unsupported activation type (DataFp32 = 8): NULL and error 3
    assert not _lib.lib.ubridge_get_gemm_launch_params(8, 8, 1, 4, 4, 4, 0)
    assert _lib.lib.ubridge_last_error() == 3
    assert not _lib.lib.ubridge_get_gemm_launch_params(5, 15, 0, 4, 4, 4, 0)
    assert _lib.lib.ubridge_last_error() == 1


def test_workspace_api_without_gpu():
    # scratch bookkeeping entry points: argument checks and the counters,
    # which start at zero (no call has needed scratch in this process)
    from ubridge_amd import ops
    lib = _lib.lib
    assert ops.workspace_stats() == (0, 0, 0)
    assert lib.ubridge_set_workspace_allocator(ops._WS_ALLOC(lambda *a: 0), ops._WS_FREE(),
                                               None) == 1
    assert b"both functions" in lib.ubridge_last_error_string()
    lib.ubridge_last_error()
    alloc = ops.TorchWorkspaceAllocator(device=0)
    ops.set_workspace_allocator(alloc)  # registering touches no device
    ops.set_workspace_allocator(None)
    assert ops.workspace_stats() == (0, 0, 0)
