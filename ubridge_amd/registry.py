"""Kernel-by-name lookup and launch, the host mirror of the reference's
GcuDevice::get_or_load_func(func, module) (src/gcu_device.rs:160-183) and
GcuLaunchAsync::launch(cfg, (params...)) (src/gcu_launch.rs:121-181).

    f = get_function("dequantize_block_q8_0_bf16", "quant")
    f.launch((c_void_p(w.data_ptr()), c_void_p(out.data_ptr()), c_size_t(n)))

Each argument is a ctypes scalar; the library receives an array of pointers to
them (the reference's as_kernel_param convention) and unpacks it with the
reference kernel's positional signature.
"""
import ctypes

from ._lib import check, lib, register

register("ubridge_get_function", ctypes.c_void_p, [ctypes.c_char_p, ctypes.c_char_p])
register("ubridge_has_function", ctypes.c_int, [ctypes.c_char_p])
register("ubridge_num_functions", ctypes.c_int, [])
register("ubridge_function_name", ctypes.c_char_p, [ctypes.c_int])
register("ubridge_launch", ctypes.c_int,
         [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p])


class Function:
    def __init__(self, name, module, handle):
        self.name, self.module, self.handle = name, module, handle

    def launch(self, args, stream=None):
        """Launch asynchronously on `stream` (a torch stream, default current)."""
        from .ops import stream_ptr
        keep = list(args)
        arr = (ctypes.c_void_p * max(len(keep), 1))(
            *[ctypes.cast(ctypes.pointer(a), ctypes.c_void_p) for a in keep])
        rc = lib.ubridge_launch(self.handle, arr, stream_ptr(stream))
        check(rc)

    def __repr__(self):
        return f"Function({self.module}.{self.name})"


def get_function(name, module=None):
    h = lib.ubridge_get_function(name.encode(), module.encode() if module else None)
    if not h:
        lib.ubridge_last_error()
        raise KeyError(f"no kernel '{name}' in module '{module or '*'}'")
    return Function(name, module, h)


def has_function(name):
    return bool(lib.ubridge_has_function(name.encode()))


def function_names():
    return [lib.ubridge_function_name(i).decode() for i in range(lib.ubridge_num_functions())]
