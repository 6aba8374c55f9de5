"""GPU parity at the benchmark configurations' own sizes (configs 2-5 of the
benchmark plan; config 1 is in test_gpu_model.py), called through the C ABI.

* Config 2: one Hyena operator at 7B width, L = 8192, W = 4096, 256 filter
  groups, BF16 projection N(0, 1) in, split planes out (the model path),
  against the oracle mixer on the same BF16 projection: max error <= 2e-5 of
  the output scale.
* Config 3: the FP8 projection GEMM M = 1024, K = 4096, N = 12288 with amax
  scales: E4M3 codes bit-exact on every element; exact (QGMMA) mode
  bit-exact on 64 sampled rows x all 12288 columns; the MFMA K32 / K128
  modes within the RMS / max bounds of test_gpu_ops.py on those rows.
* Config 4: a 7B-width model with one block of each mixer type (HCS, HCM,
  HCL, attention; FFN 11264, 32 heads, 256 filter groups) at 8192 tokens
  against the oracle: logits and every block output within 1e-3 of the
  output scale, top-1 100 %. The full 32-block 7B shape at 1024 and 8192
  tokens: a smaller arena (256 / 1024 rows per chunk) equals the 8192-row
  arena within 1e-4, repeated runs are bit-identical, logits finite.
* Config 5: 131072 tokens through the 32-block 7B shape, arena 4096 against
  arena 8192 within 1e-4, finite.

The arena bound: chunking changes only F32 summation orders (split-K
partials of few-tile GEMMs, the modal-state carry across chunk boundaries,
the FIR history hand-over), which 32 blocks compound to ~3e-5 of the logit
scale (measured at 1024 tokens, arena 256); 1e-4 is 10x inside the 1e-3
parity tolerance.

Inputs follow the benchmark distributions ("survey" init: linears N(0, 0.02),
taps and D N(0, 0.02), log-poles log U[0.5, 0.99], residues N(0, 0.02)).
"""
import ctypes
import os
import time

import numpy as np
import pytest

import oracle_lib as O
from evo_hip import artifact as A
from evo_hip import capi
from evo_hip import native as N
from evo_hip.artifact import bf16_bits, bf16_to_f32
from gpu_util import dev, empty, host, p, stream
from test_gpu_ops import hyena_gpu, hyena_oracle, rel_err

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "evo.cpp_amd", "lib", "libevo_hip.so")
THREADS = 16  # the oracle's OpenMP threads (the GPU box's CPU share)


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def say(message):
    print(message, flush=True)


# -------------------------------------------------------------- config 2
@pytest.mark.parametrize("kind", [N.HYENA_HCS, N.HYENA_HCM, N.HYENA_HCL])
def test_config2_hyena_operator_7b_width(kind):
    length, width, groups = 8192, 4096, 256
    r = rng(2000 + kind)
    proj = bf16_to_f32(bf16_bits(r.standard_normal((length, 3 * width), dtype=np.float32)))
    case = dict(projection=proj, width=width,
                short=bf16_bits(r.standard_normal((3 * width, 3), dtype=np.float32) * 0.02))
    if kind != N.HYENA_HCL:
        taps = 7 if kind == N.HYENA_HCS else 128
        case["inner"] = bf16_to_f32(bf16_bits(
            r.standard_normal((groups, taps), dtype=np.float32) * 0.02))
        case["groups"], case["inner_len"] = groups, taps
    if kind != N.HYENA_HCS:
        case["direct"] = bf16_to_f32(bf16_bits(r.standard_normal(width, dtype=np.float32) * 0.02))
    if kind == N.HYENA_HCL:
        case["log_poles"] = np.log(r.uniform(0.5, 0.99, (width, 16))).astype(np.float32)
        case["residues"] = (r.standard_normal((width, 16)) * 0.02).astype(np.float32)
        case["state"] = 16
    expected = hyena_oracle(kind, case)
    actual = hyena_gpu(kind, case, dtype=N.DTYPE_BF16_SPLIT, bf16_taps=True, guard=8)
    error = rel_err(actual, expected)
    say(f"config 2 kind {kind}: max err {error:.3g} of the output scale")
    assert error < 2e-5
    # The operator's own format (BF16 in, BF16 out, as evo.cpp's
    # bf16_hcs/hcm/hcl_prefill write it): each output is the F32 result
    # rounded once to BF16, so every element lies within half a BF16 ulp of
    # the oracle (|y| in [2^(E-1), 2^E): ulp 2^(E-8)), plus the F32 error above.
    out16 = hyena_gpu(kind, case, dtype=N.DTYPE_BF16, bf16_taps=True, guard=8)
    half_ulp = np.ldexp(1.0, np.frexp(expected)[1] - 9)
    excess = np.abs(out16 - expected) - half_ulp
    scale = np.abs(expected).max()
    say(f"config 2 kind {kind} BF16 out: worst excess over half an ulp "
        f"{excess.max() / scale:.3g} of the output scale")
    assert excess.max() < 2e-5 * scale


# -------------------------------------------------------------- config 3
def test_config3_fp8_projection_gemm():
    m, k, n = 1024, 4096, 12288
    r = rng(3000)
    a_bits = bf16_bits(r.standard_normal((m, k), dtype=np.float32))
    w = bf16_to_f32(bf16_bits(r.standard_normal((n, k), dtype=np.float32) * 0.02))
    in_scale = np.float32(448.0) / np.float32(np.abs(bf16_to_f32(a_bits)).max())
    w_scale = np.float32(448.0) / np.float32(np.abs(w).max())
    out_scale = float(np.float32(1.0) / (in_scale * w_scale))
    w_codes = O.quantize_f32(w, float(w_scale))

    # activation codes on the GPU, bit-exact on all 4 Mi elements
    a_dev = dev(a_bits)
    codes = empty((m, k), np.uint8)
    N.call("evo_hip_e4m3_quantize", N.DTYPE_BF16, p(a_dev), m * k, float(in_scale), p(codes),
           stream())
    expected_codes = np.zeros((m, k), np.uint8)
    O.lib().oracle_e4m3_quantize_bf16(O.ptr(a_bits), m * k, float(in_scale),
                                      O.ptr(expected_codes))
    a_codes = host(codes)
    assert np.array_equal(a_codes, expected_codes)

    import torch
    w_dev = dev(w_codes)
    results = {}
    for mode in (N.FP8_EXACT, N.FP8_MFMA_K32, N.FP8_MFMA_K128):
        out = empty((m, n))
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        N.call("evo_hip_fp8_linear", p(codes), p(w_dev), p(out), m, n, k, out_scale, mode,
               stream())
        end.record()
        torch.cuda.synchronize()
        results[mode] = host(out)
        say(f"config 3 mode {mode}: {start.elapsed_time(end):.3f} ms (first call)")

    rows = np.unique(np.concatenate([[0, m - 1], rng(3001).choice(m, 62, replace=False)]))
    expected = O.qgmma(expected_codes[rows], w_codes, out_scale)
    assert np.array_equal(results[N.FP8_EXACT][rows].view(np.uint32), expected.view(np.uint32))
    rms = np.sqrt(np.mean(expected.astype(np.float64) ** 2))
    for mode, bound in ((N.FP8_MFMA_K32, 2.0 ** -7), (N.FP8_MFMA_K128, 2.0 ** -8)):
        diff = results[mode][rows].astype(np.float64) - expected
        say(f"config 3 mode {mode}: rms dev {np.sqrt(np.mean(diff ** 2)) / rms:.3g} of rms, "
            f"max {np.abs(diff).max() / np.abs(expected).max():.3g} of max")
        assert np.sqrt(np.mean(diff ** 2)) <= bound * rms
        assert np.abs(diff).max() <= 2.0 ** -6 * np.abs(expected).max()


# -------------------------------------------------------------- config 4
@pytest.fixture(scope="module")
def hip():
    return capi.EvoLibrary(LIB)


def context_of(model, capacity, flags=0, arena=None):
    hip = model.library
    if arena:
        os.environ["EVO_HIP_ARENA_ROWS"] = str(arena)
    try:
        params = hip.lib.evo_context_default_params()
        params.context_size = capacity
        params.flags = flags
        handle = ctypes.c_void_p()
        hip.check(hip.lib.evo_context_create(model.handle, ctypes.byref(params),
                                             ctypes.byref(handle)))
        return capi.Context(model, handle)
    finally:
        os.environ.pop("EVO_HIP_ARENA_ROWS", None)


def relmax(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


@pytest.fixture(scope="module")
def one_of_each_7b(tmp_path_factory):
    """7B-width blocks: 0 HCS, 1 HCM, 2 HCL, 3 attention."""
    shape = A.tiny_shape(width=4096, layers=4, heads=32, inner=11264, groups=256, attn=(3,),
                         rope_scale=128.0, model_id="random-init-evo2-7b-width-4-blocks")
    path = str(tmp_path_factory.mktemp("w4096") / "one_of_each.safetensors")
    A.random_artifact(shape, seed=4, init="survey").write(path)
    return path


@pytest.mark.timeout(900)  # the CPU oracle needs ~1-2 min at 8192 tokens
def test_config4_one_block_of_each_mixer_at_7b_width(hip, one_of_each_7b):
    tokens = A.acgt_tokens(8192, seed=4)
    sequence = tokens.astype(np.uint8).tobytes()
    t0 = time.time()
    expected, blocks = O.OracleModel(one_of_each_7b).prefill(
        tokens, chunk=8192, threads=THREADS, capture_layer="all")
    say(f"config 4 (4 blocks, 8192 tokens): oracle {time.time() - t0:.1f} s")
    model = hip.load(one_of_each_7b, capi.BACKEND_HIP)
    logits = context_of(model, 8192).prefill(sequence)
    error = relmax(logits, expected)
    say(f"  logits max err {error:.3g}, top-1 {np.mean(logits.argmax(1) == expected.argmax(1))}")
    assert error <= 1e-3
    assert np.array_equal(logits.argmax(1), expected.argmax(1))
    previous = None
    for layer in range(4):
        hidden = context_of(model, 8192).embed(sequence, layer)
        block_error = relmax(hidden, blocks[layer])
        line = f"  block {layer}: output max err {block_error:.3g}"
        assert block_error <= 1e-3
        if previous is not None:
            # the block's own contribution to the residual stream
            delta_error = relmax(hidden - previous[0], blocks[layer] - previous[1])
            line += f", contribution max err {delta_error:.3g}"
            assert delta_error <= 1e-3
        say(line)
        previous = (hidden, blocks[layer])


@pytest.fixture(scope="module")
def evo2_7b(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("evo2_7b") / "evo2_7b.safetensors")
    t0 = time.time()
    A.random_artifact(A.evo2_7b_shape(), seed=7, init="survey").write(path)
    say(f"7B artifact written in {time.time() - t0:.0f} s")
    return path


_loaded = {}


def loaded(hip, path, model_flags):
    """One resident copy of each (artifact, load flags) for the module."""
    key = (path, model_flags)
    if key not in _loaded:
        _loaded[key] = hip.load(path, capi.BACKEND_HIP, flags=model_flags)
    return _loaded[key]


def resident_prefill(hip, path, tokens, arena=None, flags=0, model_flags=0):
    """Logits of one prefill with tokens and logits in device memory."""
    ctx = context_of(loaded(hip, path, model_flags), len(tokens), flags=flags, arena=arena)
    ids = dev(tokens.astype(np.uint32))
    logits = empty((len(tokens), 512))
    N.call("evo_hip_context_prefill_resident", ctx.handle, p(ids), len(tokens), p(logits))
    return host(logits)


@pytest.mark.timeout(600)  # includes writing the 13 GB artifact once
@pytest.mark.parametrize("length", [1024, 8192])
def test_config4_full_7b_arena_and_determinism(hip, evo2_7b, length):
    tokens = A.acgt_tokens(length, seed=length)
    whole = resident_prefill(hip, evo2_7b, tokens)
    again = resident_prefill(hip, evo2_7b, tokens)
    chunked = resident_prefill(hip, evo2_7b, tokens, arena=1024 if length > 1024 else 256)
    assert np.isfinite(whole).all()
    assert np.array_equal(whole.view(np.uint32), again.view(np.uint32))
    error = relmax(chunked, whole)
    say(f"config 4 full 7B, {length} tokens: arena max err {error:.3g}")
    assert error <= 1e-4


def test_config4_full_7b_fp8_projections(hip, evo2_7b):
    """The benchmarked configuration (FP8 projections converted at load, MFMA
    K128): deterministic, finite, and close to the same weights with BF16
    projections. That is a different model (quantised weights), not a parity
    check: measured 1.4e-4 of the logit scale apart, one near-tie row of 8192
    flipping its top-1; bounds 1e-3 and 99.9 %."""
    tokens = A.acgt_tokens(8192, seed=8)
    fp8 = resident_prefill(hip, evo2_7b, tokens, model_flags=1 << 8)
    assert np.isfinite(fp8).all()
    assert np.array_equal(fp8.view(np.uint32),
                          resident_prefill(hip, evo2_7b, tokens, model_flags=1 << 8)
                          .view(np.uint32))
    f32 = resident_prefill(hip, evo2_7b, tokens)
    agree = float(np.mean(fp8.argmax(1) == f32.argmax(1)))
    say(f"config 4 FP8 K128 vs hip-f32: max err {relmax(fp8, f32):.3g}, top-1 {agree}")
    assert relmax(fp8, f32) <= 1e-3
    assert agree >= 0.999


# -------------------------------------------------------------- config 5
@pytest.mark.parametrize("model_flags,flags", [
    pytest.param(0, 0, id="bf16-projections"),
    # bench.py's configuration: FP8 projections, FP16 out-projections
    pytest.param(1 << 8, 1 << 12, id="fp8+f16-out")])
def test_config5_131072_tokens_arena_consistency(hip, evo2_7b, model_flags, flags):
    tokens = A.acgt_tokens(131072, seed=5)
    whole = resident_prefill(hip, evo2_7b, tokens, flags=flags, model_flags=model_flags)
    assert np.isfinite(whole).all()
    chunked = resident_prefill(hip, evo2_7b, tokens, arena=4096, flags=flags,
                               model_flags=model_flags)
    error = relmax(chunked, whole)
    say(f"config 5 (131072 tokens, flags {flags:#x}): arena 4096 vs 8192 max err {error:.3g}")
    assert error <= 1e-4


# --------------------------------------------- FP8 modes at 7B width
FP8_MODES = {"exact": 1 << 9, "k32": 1 << 10, "k128": 0}


@pytest.mark.timeout(900)
def test_fp8_projection_modes_at_7b_width(hip, evo2_7b):
    """The 32-block 7B shape with every Hyena input projection converted to
    E4M3 at load (the benchmarked configuration), 128 tokens, in the three
    FP8 modes against the oracle with the same conversion (codes and QGMMA
    per the reference's CUDA semantics). Per block: the E4M3 code agreement of
    the block's quantised input (the next block's codes recomputed from each
    side's captured hidden state by the oracle's norm and encoder), and the
    max error of the block's output; then the logits' max error and top-1."""
    tokens = A.acgt_tokens(128, seed=12)
    sequence = tokens.astype(np.uint8).tobytes()
    shape = A.evo2_7b_shape()
    t0 = time.time()
    oracle = O.OracleModel(evo2_7b).convert_fp8(8.0)
    expected, blocks = oracle.prefill(tokens, chunk=128, threads=THREADS, capture_layer="all")
    say(f"FP8 7B oracle (128 tokens): {time.time() - t0:.1f} s")
    art = A.random_artifact(shape, seed=7, init="survey")
    index = {spec.name: i for i, spec in enumerate(art.specs)}

    def codes(hidden, layer):
        scale = art._make(index[f"blocks.{layer}.pre_norm.scale"])
        normed = np.zeros_like(hidden)
        O.lib().oracle_rms_norm(O.ptr(hidden), hidden.shape[0], hidden.shape[1],
                                O.ptr(scale), np.float32(shape.eps), O.ptr(normed))
        return O.quantize_f32(normed, 448.0 / 8.0)

    summary = {}
    model = loaded(hip, evo2_7b, 1 << 8)
    for name, flags in FP8_MODES.items():
        logits = context_of(model, 128, flags).prefill(sequence)
        worst_block, worst_agreement = 0.0, 1.0
        previous = None
        for layer in range(shape.layers):
            hidden = context_of(model, 128, flags).embed(sequence, layer)
            worst_block = max(worst_block, relmax(hidden, blocks[layer]))
            if previous is not None and shape.mixer(layer) != "attn":
                agreement = float(np.mean(codes(previous, layer) ==
                                          codes(blocks[layer - 1], layer)))
                worst_agreement = min(worst_agreement, agreement)
            previous = hidden
        top1 = float(np.mean(logits.argmax(1) == expected.argmax(1)))
        summary[name] = (relmax(logits, expected), worst_block, worst_agreement, top1)
        say(f"  {name}: logits max err {summary[name][0]:.3g}, worst block max err "
            f"{worst_block:.3g}, worst code agreement {worst_agreement:.6f}, top-1 {top1}")
    # Measured (128 tokens, seed 12): logits 3.5-4.1e-5, worst block 3.7-4.4e-5,
    # worst code agreement 99.80-99.81 %, top-1 100 % in all three modes. The
    # bounds are that envelope with a 5x margin (0.5 % for the codes).
    for name, (logit_error, block_error, agreement, top1) in summary.items():
        assert top1 == 1.0
        assert logit_error <= 2e-4
        assert block_error <= 2e-4
        assert agreement >= 0.993


# ------------------------- the benchmarked configuration against the oracle
F16_PROJ = 1 << 11  # EVO_CONTEXT_FLAG_HIP_F16_PROJ
F16_OUT = 1 << 12   # EVO_CONTEXT_FLAG_HIP_F16_OUT
_fp8_oracle = {}


def fp8_oracle(path, tokens):
    """Oracle logits and every block output of the FP8-converted model (the
    reference CPU path's ops with the CUDA reference's FP8 semantics: codes
    of bf16(x) * input_scale, QGMMA K=32), computed once per model/input."""
    key = (path, len(tokens), tokens.tobytes())
    if key not in _fp8_oracle:
        t0 = time.time()
        _fp8_oracle[key] = O.OracleModel(path).convert_fp8(8.0).prefill(
            tokens, chunk=len(tokens), threads=THREADS, capture_layer="all")
        say(f"FP8 oracle ({os.path.basename(path)}, {len(tokens)} tokens): "
            f"{time.time() - t0:.1f} s")
    return _fp8_oracle[key]


def fp8_block_errors(model, sequence, blocks, layers, capacity, flags=0):
    """Max error of every block output (relative to that block's oracle
    output scale) under the given context flags."""
    errors = []
    for layer in range(layers):
        hidden = context_of(model, capacity, flags).embed(sequence, layer)
        errors.append(relmax(hidden, blocks[layer]))
    return errors


# Context flags of the compared profiles: 0 is the library's default context
# (FP8 MFMA K128, every other product split BF16); F16_OUT (out-projections
# on one FP16 pass) is the context bench.py measures.
CONTEXTS = [pytest.param(0, id="k128"), pytest.param(F16_OUT, id="k128+f16-out")]


@pytest.mark.timeout(1200)
@pytest.mark.parametrize("flags", CONTEXTS)
def test_benchmarked_fp8_k128_full_7b_at_1024_tokens(hip, evo2_7b, flags):
    """The benchmarked configuration as bench.py runs it: the 32-block 7B
    shape, every Hyena projection converted to E4M3 at load, MFMA K128, with
    (bench.py's context) and without FP16 out-projections, 1024 tokens,
    against the oracle with the same conversion. Every block output and the
    logits within 1e-3 of their scale, top-1 100 % (measured: logits 4.3e-5
    split, 1.8e-4 with FP16 out-projections)."""
    tokens = A.acgt_tokens(1024, seed=1024)
    sequence = tokens.astype(np.uint8).tobytes()
    expected, blocks = fp8_oracle(evo2_7b, tokens)
    model = loaded(hip, evo2_7b, 1 << 8)
    logits = resident_prefill(hip, evo2_7b, tokens, flags=flags, model_flags=1 << 8)
    errors = fp8_block_errors(model, sequence, blocks, A.evo2_7b_shape().layers, 1024, flags)
    top1 = float(np.mean(logits.argmax(1) == expected.argmax(1)))
    say(f"  flags {flags:#x}: logits max err {relmax(logits, expected):.3g}, worst block "
        f"{max(errors):.3g} (block {int(np.argmax(errors))}), top-1 {top1}")
    assert max(errors) <= 1e-3
    assert relmax(logits, expected) <= 1e-3
    assert top1 == 1.0


@pytest.mark.timeout(1200)
@pytest.mark.parametrize("flags", CONTEXTS)
def test_fp8_k128_one_block_of_each_mixer_at_8192_tokens(hip, one_of_each_7b, flags):
    """Config 4's one-of-each 7B-width model (HCS, HCM, HCL, attention) with
    FP8 Hyena projections converted at load, MFMA K128, 8192 tokens, against
    the oracle with the same conversion: every block output and the logits
    within 1e-3 of their scale, top-1 100 %."""
    tokens = A.acgt_tokens(8192, seed=48)
    sequence = tokens.astype(np.uint8).tobytes()
    expected, blocks = fp8_oracle(one_of_each_7b, tokens)
    model = hip.load(one_of_each_7b, capi.BACKEND_HIP, flags=1 << 8)
    logits = context_of(model, 8192, flags).prefill(sequence)
    errors = fp8_block_errors(model, sequence, blocks, 4, 8192, flags)
    top1 = float(np.mean(logits.argmax(1) == expected.argmax(1)))
    say(f"  flags {flags:#x}: logits max err {relmax(logits, expected):.3g}, block errors "
        f"{', '.join(f'{e:.3g}' for e in errors)}, top-1 {top1}")
    assert max(errors) <= 1e-3
    assert relmax(logits, expected) <= 1e-3
    assert top1 == 1.0


@pytest.mark.timeout(1200)
def test_f16_projection_profile_full_7b_at_1024_tokens(hip, evo2_7b):
    """The "+f16-proj" profile (EVO_CONTEXT_FLAG_HIP_F16_PROJ: out- and
    attention projections on one FP16 pass) on the benchmarked FP8 K128
    configuration, 1024 tokens, against the oracle: every block and the
    logits within 1e-3, top-1 100 % (measured 2.7e-4). At 8192 tokens on
    the one-of-each model it reaches 8.9e-5 but flips the top-1 of one
    near-tie row of 8192 (the attention block's error rises from 1.3e-5 to
    8.2e-5), which is why it is not the benchmarked context."""
    tokens = A.acgt_tokens(1024, seed=1024)
    sequence = tokens.astype(np.uint8).tobytes()
    expected, blocks = fp8_oracle(evo2_7b, tokens)
    model = loaded(hip, evo2_7b, 1 << 8)
    logits = resident_prefill(hip, evo2_7b, tokens, flags=F16_PROJ, model_flags=1 << 8)
    errors = fp8_block_errors(model, sequence, blocks, A.evo2_7b_shape().layers, 1024,
                              flags=F16_PROJ)
    top1 = float(np.mean(logits.argmax(1) == expected.argmax(1)))
    say(f"  +f16-proj: logits max err {relmax(logits, expected):.3g}, worst block "
        f"{max(errors):.3g}, top-1 {top1}")
    assert max(errors) <= 1e-3
    assert relmax(logits, expected) <= 1e-3
    assert top1 == 1.0
