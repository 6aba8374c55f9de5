"""Locate and bind libevo_hip.so (the product library).

``load()`` raises if the library has not been built: there is no fallback
path, every call below runs the gfx950 kernels.
"""
from __future__ import annotations

import ctypes
import os
from functools import lru_cache

PACKAGE_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBRARY_PATH = os.path.join(PACKAGE_DIR, "lib", "libevo_hip.so")

c_size, c_void, c_float, c_int = (ctypes.c_size_t, ctypes.c_void_p,
                                   ctypes.c_float, ctypes.c_int)

HYENA_HCS, HYENA_HCM, HYENA_HCL = 0, 1, 2
DTYPE_F32, DTYPE_BF16, DTYPE_SPLIT, DTYPE_BF16_SPLIT, DTYPE_F16, DTYPE_BF16_F16 = 0, 1, 2, 3, 4, 5
DTYPE_PLANAR = 0x100  # OR-ed into the Hyena dtype: planar projection columns
DTYPE_BF16_TAPS = 0x200  # OR-ed into the Hyena dtype: inner taps are BF16 values
FP8_MFMA_K32, FP8_MFMA_K128, FP8_EXACT = 0, 1, 2

# name -> (restype, argtypes) for include/evo/hip_ops.h
_OPS = {
    "evo_hip_hyena_workspace_bytes": (c_size, [c_int, c_size, c_size, c_size]),
    "evo_hip_hyena_forward": (c_int, [c_int, c_int, c_void, c_size, c_size, c_void,
                                      c_size, c_void, c_size, c_size, c_void, c_void,
                                      c_void, c_size, c_void, c_void, c_void, c_void,
                                      c_size, c_void, c_void]),
    "evo_hip_hyena_static_scratch_bytes": (c_size, []),
    "evo_hip_hyena_forward_static": (c_int, [c_int, c_int, c_void, c_size, c_size, c_void,
                                             c_size, c_void, c_size, c_size, c_void, c_void,
                                             c_void, c_size, c_void, c_void, c_void, c_void,
                                             c_void]),
    "evo_hip_e4m3_quantize": (c_int, [c_int, c_void, c_size, c_float, c_void, c_void]),
    "evo_hip_fp8_linear": (c_int, [c_void, c_void, c_void, c_size, c_size, c_size,
                                   c_float, c_int, c_void]),
    "evo_hip_fp8_linear_bf16": (c_int, [c_void, c_void, c_void, c_size, c_size, c_size,
                                   c_float, c_int, c_void]),
    "evo_hip_split_f32": (c_int, [c_void, c_size, c_void, c_void, c_void]),
    "evo_hip_linear": (c_int, [c_void, c_void, c_void, c_void, c_void, c_size, c_size,
                               c_size, c_void, c_void]),
    "evo_hip_linear_normed": (c_int, [c_void, c_size, c_size, c_void, c_float, c_int, c_void,
                                      c_size, c_void, c_void]),
    "evo_hip_fp8_linear_normed": (c_int, [c_void, c_size, c_size, c_void, c_float, c_float,
                                          c_void, c_size, c_float, c_int, c_void, c_void]),
    "evo_hip_linear_split": (c_int, [c_void, c_void, c_void, c_void, c_void, c_size, c_size,
                                     c_size, c_void, c_void, c_size, c_void]),
    "evo_hip_pack_mlp": (c_int, [c_void, c_void, c_size, c_size, c_void, c_void]),
    "evo_hip_gated_mlp": (c_int, [c_void, c_void, c_void, c_void, c_size, c_size, c_size,
                                  c_int, c_void, c_void, c_void, c_void]),
    "evo_hip_rms_norm_e4m3": (c_int, [c_void, c_size, c_size, c_void, c_float, c_float,
                                      c_void, c_void]),
    "evo_hip_rms_norm": (c_int, [c_void, c_size, c_size, c_void, c_float, c_void, c_void,
                                 c_void, c_void]),
    "evo_hip_context_prefill_resident": (c_int, [c_void, c_void, c_size, c_void]),
    "evo_hip_context_set_product_timing": (c_int, [c_void, c_int]),
    "evo_hip_context_product_time": (c_int, [c_void, c_void, c_void]),
    "evo_hip_attention": (c_int, [c_void, c_size, c_size, c_size, c_int, c_void, c_float,
                                  c_size, c_void, c_void, c_void, c_size, c_void, c_void]),
    "evo_hip_attention_ws": (c_int, [c_void, c_size, c_size, c_size, c_int, c_void, c_float,
                                     c_size, c_void, c_void, c_void, c_size, c_void, c_void,
                                     c_size, c_void]),
}


class OpError(RuntimeError):
    pass


def share_hip_runtime() -> None:
    """PyTorch-ROCm ships its own libamdhip64 with the system soname
    (libamdhip64.so.7). Loading torch first makes libevo_hip.so bind to that
    same runtime, so device pointers and streams are shared; loading the
    library first would put two HIP runtimes in one process."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


@lru_cache(maxsize=None)
def load(path: str = LIBRARY_PATH) -> ctypes.CDLL:
    share_hip_runtime()
    if not os.path.exists(path):
        raise OpError(f"{path} is missing: build it with __graft_entry__.build() "
                      "(make -C evo.cpp_amd); there is no fallback implementation")
    lib = ctypes.CDLL(path)
    lib.evo_last_error.restype = ctypes.c_char_p
    for name, (restype, argtypes) in _OPS.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = restype, argtypes
    return lib


def call(name: str, *args) -> int:
    """Call an operator entry point; raise OpError on a non-OK status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if name.endswith("_bytes"):
        return status
    if status != 0:
        raise OpError(f"{name}: {lib.evo_last_error().decode()}")
    return status
