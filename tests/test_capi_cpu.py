"""The C-ABI library without a GPU: it loads, exports exactly the symbols the
headers declare, and its host-only entry points follow the reference's
contracts (status/backend names, default params, batch API, byte tokenizer,
sampler). Sampled token ids are compared bit-exactly with evo.cpp's own
sampler (oracle/_ref) where the reference library is built."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from evo_hip import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "evo.cpp_amd", "lib", "libevo_hip.so")
HEADERS = [os.path.join(ROOT, "include", "evo", name) for name in ("evo.h", "hip_ops.h")]
REF = os.path.join(ROOT, "oracle", "_ref", "libevo_ref.so")


def declared_symbols():
    names = set()
    for header in HEADERS:
        text = open(header).read()
        names |= set(re.findall(r"EVO_API[^;(]*?\b(evo_\w+)\s*\(", text, re.S))
    return names


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True,
                         text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_library_exports_exactly_the_declared_symbols():
    declared = declared_symbols()
    assert len(declared) >= 48
    assert exported_symbols() == declared


def test_reference_abi_subset_present():
    """Every symbol of evo.cpp's include/evo/evo.h:133-210 is exported."""
    reference = {
        "evo_abi_version", "evo_version_string", "evo_status_name", "evo_backend_name",
        "evo_last_error", "evo_model_default_params", "evo_context_default_params",
        "evo_sampler_default_params", "evo_embedding_default_options", "evo_model_load",
        "evo_model_free", "evo_model_backend", "evo_model_id", "evo_model_architecture",
        "evo_model_profile", "evo_model_vocab_size", "evo_model_max_context",
        "evo_model_embedding_width", "evo_model_layer_count", "evo_model_encode",
        "evo_model_decode_token", "evo_context_create", "evo_context_free",
        "evo_context_position", "evo_context_capacity", "evo_context_profile",
        "evo_context_prefill", "evo_context_decode", "evo_context_embed",
        "evo_context_embed_ex", "evo_batch_create", "evo_batch_free", "evo_batch_clear",
        "evo_batch_add_sequence", "evo_batch_sequence_count", "evo_batch_token_count",
        "evo_sampler_create", "evo_sampler_free", "evo_sampler_sample"}
    assert reference <= exported_symbols()


@pytest.fixture(scope="module")
def lib():
    return capi.EvoLibrary(LIB)


def test_version_status_and_backend_names(lib):
    L = lib.lib
    assert L.evo_abi_version() == (1 << 24) | (6 << 16)
    assert L.evo_status_name(0) == b"ok" and L.evo_status_name(8) == b"hip"
    assert L.evo_status_name(2) == b"invalid_argument" and L.evo_status_name(99) == b"unknown"
    assert L.evo_backend_name(4) == b"hip" and L.evo_backend_name(2) == b"cpu"
    params = L.evo_context_default_params()
    assert params.struct_size == ctypes.sizeof(capi.ContextParams) and params.context_size == 4096


def test_model_load_errors_without_gpu(lib):
    with pytest.raises(capi.EvoError) as error:
        lib.load("/nonexistent.safetensors", capi.BACKEND_CPU)
    assert error.value.status == 5  # HIP-only library: CPU backend unsupported
    with pytest.raises(capi.EvoError) as error:
        lib.load("", capi.BACKEND_HIP)
    assert error.value.status == 2


def test_batch_api(lib):
    L = lib.lib
    batch = ctypes.c_void_p()
    lib.check(L.evo_batch_create(2, ctypes.byref(batch)))
    lib.check(L.evo_batch_add_sequence(batch, b"ACGT", 4))
    lib.check(L.evo_batch_add_sequence(batch, b"AC", 2))
    L.evo_batch_sequence_count.argtypes = L.evo_batch_token_count.argtypes = [ctypes.c_void_p]
    L.evo_batch_sequence_count.restype = L.evo_batch_token_count.restype = ctypes.c_size_t
    assert L.evo_batch_sequence_count(batch) == 2 and L.evo_batch_token_count(batch) == 6
    assert L.evo_batch_add_sequence(batch, b"A", 1) == 2  # full
    L.evo_batch_free(batch)


def sample(library, logits, temperature, top_k, top_p, seed, draws):
    L = library.lib
    params = L.evo_sampler_default_params()
    params.temperature, params.top_k, params.top_p, params.seed = temperature, top_k, top_p, seed
    sampler = ctypes.c_void_p()
    library.check(L.evo_sampler_create(ctypes.byref(params), ctypes.byref(sampler)))
    token = ctypes.c_uint32()
    out = []
    data = logits.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    for _ in range(draws):
        library.check(L.evo_sampler_sample(sampler, data, logits.size, ctypes.byref(token)))
        out.append(token.value)
    L.evo_sampler_free(sampler)
    return out


def test_greedy_sampler_lowest_index_on_ties(lib):
    logits = np.zeros(512, np.float32)
    logits[[7, 300]] = 5.0
    assert sample(lib, logits, 1.0, 1, 1.0, 0, 3) == [7, 7, 7]


@pytest.mark.skipif(not os.path.exists(REF), reason="reference library not built")
@pytest.mark.parametrize("temperature,top_k,top_p,seed", [
    (1.0, 0, 1.0, 1), (0.7, 40, 0.9, 42), (1.3, 4, 1.0, 7), (1.0, 1, 1.0, 3)])
def test_sampler_ids_bit_exact_with_reference(lib, temperature, top_k, top_p, seed):
    logits = np.random.Generator(np.random.PCG64(seed)).standard_normal(512).astype(np.float32)
    ours = sample(lib, logits, temperature, top_k, top_p, seed, 64)
    theirs = sample(capi.EvoLibrary(REF), logits, temperature, top_k, top_p, seed, 64)
    assert ours == theirs
