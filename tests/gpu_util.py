"""Device-memory helpers for the GPU tests (torch is only the allocator)."""
from __future__ import annotations

import numpy as np


def torch():
    import torch as t
    return t


# Tensors handed to the C ABI as raw pointers must outlive the asynchronous
# launch: every tensor made here stays referenced until release() (called
# after each test by an autouse fixture), so the caching allocator cannot
# hand its memory to another operand of the same call.
_live = []


def release() -> None:
    torch().cuda.synchronize()
    _live.clear()


def dev(array: np.ndarray):
    """Copy a numpy array to cuda:0 as a tensor of the same bits."""
    t = torch()
    array = np.ascontiguousarray(array)
    if array.dtype == np.uint16:
        tensor = t.from_numpy(array.view(np.int16))
    elif array.dtype == np.uint32:
        tensor = t.from_numpy(array.view(np.int32))
    else:
        tensor = t.from_numpy(array)
    tensor = tensor.to("cuda:0")
    _live.append(tensor)
    return tensor


def empty(shape, dtype=np.float32):
    t = torch()
    mapping = {np.float32: t.float32, np.uint8: t.uint8, np.uint16: t.int16,
               np.int32: t.int32}
    tensor = t.empty(tuple(shape), dtype=mapping[np.dtype(dtype).type], device="cuda:0")
    _live.append(tensor)
    return tensor


def zeros(shape, dtype=np.float32):
    return empty(shape, dtype).zero_()


def host(tensor, dtype=None) -> np.ndarray:
    torch().cuda.synchronize()
    array = tensor.detach().cpu().numpy()
    if dtype is not None:
        array = array.view(dtype)
    return array


def p(tensor):
    return None if tensor is None else tensor.data_ptr()


def stream():
    return torch().cuda.current_stream().cuda_stream
