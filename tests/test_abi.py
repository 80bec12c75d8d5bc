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
