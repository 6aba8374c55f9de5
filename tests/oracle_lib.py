"""ctypes bindings to oracle/liboracle.so (the CPU checker).

Test infrastructure only: the product never loads this library.
"""
from __future__ import annotations

import ctypes
import os
from functools import lru_cache

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REFERENCE_LIB = os.path.join(ROOT, "oracle", "_ref", "libevo_ref.so")

P = ctypes.c_void_p
S = ctypes.c_size_t
F = ctypes.c_float
I = ctypes.c_int


@lru_cache(maxsize=None)
def lib() -> ctypes.CDLL:
    L = ctypes.CDLL(ORACLE_PATH)
    sig = {
        "oracle_e4m3_encode": (ctypes.c_uint8, [F]),
        "oracle_e4m3_decode": (F, [ctypes.c_uint8]),
        "oracle_e4m3_quantize_f32": (None, [P, S, F, P]),
        "oracle_e4m3_quantize_bf16": (None, [P, S, F, P]),
        "oracle_qgmma_linear": (I, [P, P, S, S, S, F, S, P]),
        "oracle_rms_norm": (I, [P, S, S, P, F, P]),
        "oracle_linear_f32": (I, [P, S, S, P, S, P, P]),
        "oracle_gated_mlp_f32": (I, [P, S, S, S, P, P, P, I, P]),
        "oracle_causal_fir": (I, [P, S, S, P, S, P, I, I, P]),
        "oracle_hcl_recurrence": (I, [P, P, P, S, S, P, P, P, S, P, P]),
        "oracle_apply_rope": (I, [P, P, S, S, S, P, S, F]),
        "oracle_causal_attention": (I, [P, P, P, S, S, S, P]),
        "oracle_linear_bf16w": (I, [P, S, S, P, S, P, P, I]),
        "oracle_hyena_mixer": (I, [I, P, S, S, P, S, P, S, S, P, P, P, S, P]),
        "oracle_model_load": (P, [ctypes.c_char_p, ctypes.c_char_p, S]),
        "oracle_model_free": (None, [P]),
        "oracle_model_width": (S, [P]),
        "oracle_model_vocab": (S, [P]),
        "oracle_model_layers": (S, [P]),
        "oracle_model_prefill": (I, [P, P, S, S, P, S, P, I]),
        "oracle_model_convert_fp8": (I, [P, F]),
        "oracle_last_error": (ctypes.c_char_p, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    return L


def ptr(array: np.ndarray):
    return array.ctypes.data if array is not None else None


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(lib().oracle_last_error().decode())


class OracleModel:
    def __init__(self, path: str):
        err = ctypes.create_string_buffer(512)
        self.handle = lib().oracle_model_load(path.encode(), err, 512)
        if not self.handle:
            raise RuntimeError(err.value.decode())
        self.width = lib().oracle_model_width(self.handle)
        self.vocab = lib().oracle_model_vocab(self.handle)
        self.layers = lib().oracle_model_layers(self.handle)

    def convert_fp8(self, input_amax: float = 8.0) -> "OracleModel":
        """Convert every BF16 Hyena projection to E4M3 codes with the
        converter's amax rule (what libevo_hip.so does at load under
        EVO_MODEL_FLAG_HIP_FP8_PROJECTIONS)."""
        check(lib().oracle_model_convert_fp8(self.handle, input_amax))
        return self

    def __del__(self):
        if getattr(self, "handle", None):
            lib().oracle_model_free(self.handle)

    def prefill(self, tokens: np.ndarray, chunk: int = 256, threads: int = 8,
                capture_layer: int = None):
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.zeros((len(tokens), self.vocab), np.float32)
        capture = None
        layer = 2 ** 62
        if capture_layer == "all":  # every block's output: [layers, n, width]
            capture = np.zeros((self.layers, len(tokens), self.width), np.float32)
            layer = 2 ** 64 - 1
        elif capture_layer is not None:
            capture = np.zeros((len(tokens), self.width), np.float32)
            layer = capture_layer
        check(lib().oracle_model_prefill(
            self.handle, ptr(tokens), len(tokens), chunk, ptr(logits), layer,
            ptr(capture), threads))
        return (logits, capture) if capture_layer is not None else logits


def hyena_mixer(kind, projection, width, short_w, inner_w=None, groups=1,
                inner_len=2, direct=None, log_poles=None, residues=None,
                state=0):
    projection = f32(projection)
    length = projection.shape[0]
    out = np.zeros((length, width), np.float32)
    short_w = f32(short_w)
    args = [f32(a) if a is not None else None
            for a in (inner_w, direct, log_poles, residues)]
    check(lib().oracle_hyena_mixer(kind, ptr(projection), length, width,
                                   ptr(short_w), short_w.shape[-1],
                                   ptr(args[0]), groups, inner_len, ptr(args[1]),
                                   ptr(args[2]), ptr(args[3]), state, ptr(out)))
    return out


def linear_bf16w(x, weight_bits, bias_bits=None, threads=8):
    x = f32(x)
    rows, k = x.shape
    n = weight_bits.shape[0]
    out = np.zeros((rows, n), np.float32)
    check(lib().oracle_linear_bf16w(ptr(x), rows, k, ptr(weight_bits), n,
                                    ptr(bias_bits), ptr(out), threads))
    return out


def qgmma(in_codes, w_codes, output_scale, group_k=32):
    rows, k = in_codes.shape
    n = w_codes.shape[0]
    out = np.zeros((rows, n), np.float32)
    check(lib().oracle_qgmma_linear(ptr(np.ascontiguousarray(in_codes)),
                                    ptr(np.ascontiguousarray(w_codes)), rows, k, n,
                                    output_scale, group_k, ptr(out)))
    return out


def quantize_f32(x, scale):
    x = f32(x)
    codes = np.zeros(x.shape, np.uint8)
    lib().oracle_e4m3_quantize_f32(ptr(x), x.size, scale, ptr(codes))
    return codes
