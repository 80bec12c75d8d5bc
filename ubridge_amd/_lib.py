"""ctypes binding of libubridge_hip.so (the C ABI in include/ubridge_hip.h).

The HIP library is the only compute path: if it is missing this module raises
at import time instead of falling back to anything else.
"""
import ctypes
import os

# torch ships the HIP runtime (same soname, libamdhip64.so.7); load it first so
# this library and torch share one runtime, one device context and one set of
# streams.
import torch  # noqa: F401

_HERE = os.path.dirname(os.path.abspath(__file__))
# UBRIDGE_LIB: another build of the same library (e.g. a debug build)
LIB_PATH = os.environ.get("UBRIDGE_LIB") or os.path.join(_HERE, "lib", "libubridge_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"libubridge_hip.so not found at {LIB_PATH}; build it first with "
        "`python ubridge_amd/build.py` (hipcc --offload-arch=gfx950)")

lib = ctypes.CDLL(LIB_PATH)

_vp, _i, _sz, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
_cp = ctypes.c_char_p

# name -> (restype, argtypes)
PROTOS = {
    "ubridge_last_error": (_i, []),
    "ubridge_last_error_string": (_cp, []),
    "ubridge_version": (_cp, []),
    "ubridge_tune_set": (_i, [_cp, _i]),
    "ubridge_tune_get": (_i, [_cp]),
    "ubridge_gguf_to_soa": (_i, [_i, _vp, _vp, _sz, _vp]),
    "ubridge_soa_to_gguf": (_i, [_i, _vp, _vp, _sz, _vp]),
    "ubridge_qmatmul_workspace_size": (_sz, [_i, _i, _i]),
    "ubridge_quantize_activations": (_i, [_i, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "ubridge_qmatmul_prequantized": (_i, [_i, _vp, _vp, _i, _i, _i, _i, _vp, _vp]),
    "ubridge_qmatmul": (_i, [_i, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
}
for _q in ("q8_0", "q4_k", "q4_0"):
    for _t in ("f16", "bf16", "f32"):
        PROTOS[f"dequantize_block_{_q}_{_t}"] = (None, [_vp, _vp, _sz, _vp])
for _q in ("q8_0", "q4_k"):
    for _t in ("f16", "bf16", "f32"):
        PROTOS[f"quantize_block_{_q}_{_t}"] = (None, [_vp, _vp, _sz, _sz, _vp])


def register(name, restype, argtypes):
    PROTOS[name] = (restype, argtypes)
    fn = getattr(lib, name)
    fn.restype = restype
    fn.argtypes = argtypes
    return fn


for _n, (_r, _a) in list(PROTOS.items()):
    register(_n, _r, _a)


class UbridgeError(RuntimeError):
    pass


def check(rc=None):
    """Raise UbridgeError if the last call (or the given return code) failed."""
    code = lib.ubridge_last_error()
    if rc:
        code = rc
    if code:
        msg = lib.ubridge_last_error_string().decode(errors="replace")
        raise UbridgeError(f"ubridge error {code}: {msg}")

# --- GEMM family (gemm.hip)
_REF_MM = [_i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _f, _f, _f, _i, _i, _i, _i]
for _n in ("matmul_bf16_4bit", "matmul_f16_4bit", "matmul_bf16_8bit", "matmul_f16_8bit"):
    register(_n, None, [_vp, _vp, _vp, _vp, _vp] + _REF_MM + [_i, _vp])
for _n in ("matmul_bf16", "matmul_f16"):
    register(_n, None, [_vp, _vp, _vp] + _REF_MM + [_vp])
for _n in ("dequant_bf16", "dequant_f16"):
    register(_n, None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp])
register("ubridge_w4a16_gemm", _i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp])
register("ubridge_gemm_dense", _i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp])
