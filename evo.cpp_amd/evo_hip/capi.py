"""ctypes bindings to the ``evo.h`` C ABI.

The same bindings drive ``libevo_hip.so`` (this library, backend HIP) and,
in tests, a reference ``libevo.so`` built from evo.cpp's sources: both export
the symbols of `include/evo/evo.h:133-210`.
"""
from __future__ import annotations

import ctypes
import os
from typing import Callable, List, Optional

import numpy as np

EVO_STATUS_OK = 0
EVO_STATUS_UNSUPPORTED = 5
STATUS_NAMES = {0: "ok", 2: "invalid_argument", 3: "io", 4: "model_format",
                5: "unsupported", 6: "cuda", 7: "mps", 8: "hip", 70: "internal"}
BACKEND_AUTO, BACKEND_CUDA, BACKEND_CPU, BACKEND_MPS, BACKEND_HIP = 0, 1, 2, 3, 4


class ModelParams(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_size_t), ("backend", ctypes.c_int),
                ("devices", ctypes.POINTER(ctypes.c_int32)),
                ("device_count", ctypes.c_size_t), ("flags", ctypes.c_uint32)]


class ContextParams(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_size_t),
                ("context_size", ctypes.c_size_t), ("flags", ctypes.c_uint32)]


class SamplerParams(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_size_t), ("temperature", ctypes.c_float),
                ("top_k", ctypes.c_size_t), ("top_p", ctypes.c_float),
                ("seed", ctypes.c_uint64)]


LOGITS_CALLBACK = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(ctypes.c_float),
                                   ctypes.c_size_t, ctypes.c_size_t,
                                   ctypes.c_size_t, ctypes.c_void_p)


class EvoError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class EvoLibrary:
    """One loaded C-ABI library (``libevo_hip.so`` or a reference build)."""

    def __init__(self, path: str):
        self.path = os.path.abspath(path)
        if "libevo_hip" in os.path.basename(path):
            from .native import share_hip_runtime
            share_hip_runtime()
        lib = ctypes.CDLL(self.path)
        self.lib = lib
        lib.evo_abi_version.restype = ctypes.c_uint32
        lib.evo_version_string.restype = ctypes.c_char_p
        lib.evo_last_error.restype = ctypes.c_char_p
        lib.evo_status_name.restype = ctypes.c_char_p
        lib.evo_status_name.argtypes = [ctypes.c_int]
        lib.evo_backend_name.restype = ctypes.c_char_p
        lib.evo_backend_name.argtypes = [ctypes.c_int]
        lib.evo_model_default_params.restype = ModelParams
        lib.evo_context_default_params.restype = ContextParams
        lib.evo_model_load.argtypes = [ctypes.c_char_p, ctypes.POINTER(ModelParams),
                                       ctypes.POINTER(ctypes.c_void_p)]
        lib.evo_model_free.argtypes = [ctypes.c_void_p]
        lib.evo_model_backend.argtypes = [ctypes.c_void_p]
        lib.evo_model_backend.restype = ctypes.c_int
        for name in ("evo_model_vocab_size", "evo_model_max_context",
                     "evo_model_embedding_width", "evo_model_layer_count"):
            getattr(lib, name).argtypes = [ctypes.c_void_p]
            getattr(lib, name).restype = ctypes.c_size_t
        for name in ("evo_model_id", "evo_model_architecture", "evo_model_profile"):
            getattr(lib, name).argtypes = [ctypes.c_void_p]
            getattr(lib, name).restype = ctypes.c_char_p
        lib.evo_context_create.argtypes = [ctypes.c_void_p,
                                           ctypes.POINTER(ContextParams),
                                           ctypes.POINTER(ctypes.c_void_p)]
        lib.evo_context_free.argtypes = [ctypes.c_void_p]
        lib.evo_context_position.argtypes = [ctypes.c_void_p]
        lib.evo_context_position.restype = ctypes.c_size_t
        lib.evo_context_capacity.argtypes = [ctypes.c_void_p]
        lib.evo_context_capacity.restype = ctypes.c_size_t
        lib.evo_context_profile.argtypes = [ctypes.c_void_p]
        lib.evo_context_profile.restype = ctypes.c_char_p
        lib.evo_context_prefill.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                            LOGITS_CALLBACK, ctypes.c_void_p]
        lib.evo_context_decode.argtypes = [ctypes.c_void_p, ctypes.c_uint32,
                                           LOGITS_CALLBACK, ctypes.c_void_p]
        lib.evo_context_embed.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                          LOGITS_CALLBACK, ctypes.c_void_p]
        lib.evo_batch_create.argtypes = [ctypes.c_size_t,
                                         ctypes.POINTER(ctypes.c_void_p)]
        lib.evo_batch_free.argtypes = [ctypes.c_void_p]
        lib.evo_batch_add_sequence.argtypes = [ctypes.c_void_p, ctypes.c_char_p,
                                               ctypes.c_size_t]
        lib.evo_sampler_default_params.restype = SamplerParams
        lib.evo_sampler_create.argtypes = [ctypes.POINTER(SamplerParams),
                                           ctypes.POINTER(ctypes.c_void_p)]
        lib.evo_sampler_free.argtypes = [ctypes.c_void_p]
        lib.evo_sampler_sample.argtypes = [ctypes.c_void_p,
                                           ctypes.POINTER(ctypes.c_float),
                                           ctypes.c_size_t,
                                           ctypes.POINTER(ctypes.c_uint32)]

    def check(self, status: int) -> None:
        if status != EVO_STATUS_OK:
            raise EvoError(status, self.lib.evo_last_error().decode())

    def load(self, path: str, backend: int, flags: int = 0) -> "Model":
        params = self.lib.evo_model_default_params()
        params.backend = backend
        params.flags = flags
        handle = ctypes.c_void_p()
        self.check(self.lib.evo_model_load(path.encode(), ctypes.byref(params),
                                           ctypes.byref(handle)))
        return Model(self, handle)


class Model:
    def __init__(self, library: EvoLibrary, handle: ctypes.c_void_p):
        self.library, self.handle = library, handle

    def close(self) -> None:
        if self.handle:
            self.library.lib.evo_model_free(self.handle)
            self.handle = None

    __del__ = close

    @property
    def vocab(self) -> int:
        return self.library.lib.evo_model_vocab_size(self.handle)

    @property
    def width(self) -> int:
        return self.library.lib.evo_model_embedding_width(self.handle)

    def context(self, context_size: int, flags: int = 0) -> "Context":
        lib = self.library.lib
        params = lib.evo_context_default_params()
        params.context_size = context_size
        params.flags = flags
        handle = ctypes.c_void_p()
        self.library.check(lib.evo_context_create(self.handle, ctypes.byref(params),
                                                  ctypes.byref(handle)))
        return Context(self, handle)


class Context:
    def __init__(self, model: Model, handle: ctypes.c_void_p):
        self.model, self.handle = model, handle

    def close(self) -> None:
        if self.handle:
            self.model.library.lib.evo_context_free(self.handle)
            self.handle = None

    __del__ = close

    @property
    def position(self) -> int:
        return self.model.library.lib.evo_context_position(self.handle)

    @property
    def profile(self) -> str:
        return self.model.library.lib.evo_context_profile(self.handle).decode()

    def prefill(self, sequence: bytes,
                on_chunk: Optional[Callable[[np.ndarray, int], int]] = None
                ) -> np.ndarray:
        """Prefill one sequence; returns the [len, vocab] F32 logits."""
        lib = self.model.library.lib
        chunks: List[np.ndarray] = []
        offsets: List[int] = []

        def callback(logits, rows, columns, offset, _user):
            array = np.ctypeslib.as_array(logits, shape=(rows, columns)).copy()
            chunks.append(array)
            offsets.append(offset)
            return on_chunk(array, offset) if on_chunk else 0

        c_callback = LOGITS_CALLBACK(callback)
        batch = ctypes.c_void_p()
        self.model.library.check(lib.evo_batch_create(1, ctypes.byref(batch)))
        try:
            self.model.library.check(
                lib.evo_batch_add_sequence(batch, sequence, len(sequence)))
            self.model.library.check(
                lib.evo_context_prefill(self.handle, batch, c_callback, None))
        finally:
            lib.evo_batch_free(batch)
        if not chunks:
            return np.zeros((0, self.model.vocab), dtype=np.float32)
        return np.concatenate(chunks, axis=0)

    def embed(self, sequence: bytes, layer: int) -> np.ndarray:
        """Prefill one sequence and return block `layer`'s output hidden
        states [len, width] F32 (evo_context_embed; the context must be
        fresh)."""
        lib = self.model.library.lib
        chunks: List[np.ndarray] = []

        def callback(values, rows, columns, _offset, _user):
            chunks.append(np.ctypeslib.as_array(values, shape=(rows, columns)).copy())
            return 0

        c_callback = LOGITS_CALLBACK(callback)
        batch = ctypes.c_void_p()
        self.model.library.check(lib.evo_batch_create(1, ctypes.byref(batch)))
        try:
            self.model.library.check(
                lib.evo_batch_add_sequence(batch, sequence, len(sequence)))
            self.model.library.check(
                lib.evo_context_embed(self.handle, batch, layer, c_callback, None))
        finally:
            lib.evo_batch_free(batch)
        return np.concatenate(chunks, axis=0)

    def decode(self, token: int) -> np.ndarray:
        """One cached decode step; returns the [vocab] F32 logits of `token`
        at the current position."""
        lib = self.model.library.lib
        rows: List[np.ndarray] = []

        def callback(logits, count, columns, offset, _user):
            rows.append(np.ctypeslib.as_array(logits, shape=(count, columns)).copy())
            return 0

        c_callback = LOGITS_CALLBACK(callback)
        self.model.library.check(lib.evo_context_decode(self.handle, token, c_callback, None))
        return rows[0][0]
