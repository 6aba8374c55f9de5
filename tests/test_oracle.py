"""Pins the CPU oracle (oracle/liboracle.so) before it is trusted as the
checker of the HIP path.

* evo.cpp's golden op vectors (tests/golden/cpu_ops.json, a copy of the
  reference's tests/vectors/cpu_ops.json, atol 1e-5 / rtol 1e-4) on the exact
  inputs the reference generator used (tests/test_cpu_reference.cpp:28-136);
* the reference's closed-form cases (tests/test_cpu_reference.cpp:154-250);
* the 29 E4M3 code vectors (tests/test_fp8.cpp:22-33) and an exhaustive
  decode/encode round trip;
* QGMMA against exact rational arithmetic where the reference rule keeps
  every bit, and against a brute-force restatement on random codes;
* the whole-model forward against evo.cpp's own CPU library built from the
  reference sources (oracle/_ref, only where /root/reference is mounted) and
  against the committed reference logits.
"""
import json
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle_lib as O
from evo_hip import artifact as A

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def values(count, offset, divisor):
    """Input generator of tests/test_cpu_reference.cpp:28-38."""
    return np.array([(((i + offset) * 37 + 11) % 29 - 14) / divisor for i in range(count)],
                    np.float32)


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(GOLDEN, "cpu_ops.json")) as handle:
        data = json.load(handle)
    return data["vectors"], data["tolerance"]


def close(actual, expected, tol):
    np.testing.assert_allclose(actual, np.array(expected, np.float32),
                               atol=tol["atol"], rtol=tol["rtol"])


def test_rmsnorm_vector(oracle, golden):
    vec, tol = golden
    x = values(8, 0, 7.0)
    scale = (1.0 + values(4, 31, 19.0) * np.float32(0.1)).astype(np.float32)
    out = np.zeros(8, np.float32)
    oracle.oracle_rms_norm(O.ptr(x), 2, 4, O.ptr(scale), 1e-6, O.ptr(out))
    close(out, vec["rmsnorm"], tol)


def test_linear_vector(oracle, golden):
    vec, tol = golden
    x, w, b = values(8, 7, 9.0), values(12, 19, 13.0), values(3, 43, 17.0)
    out = np.zeros(6, np.float32)
    oracle.oracle_linear_f32(O.ptr(x), 2, 4, O.ptr(w), 3, O.ptr(b), O.ptr(out))
    close(out, vec["linear"], tol)


@pytest.mark.parametrize("gelu,name", [(1, "mlp_gelu"), (0, "mlp_identity")])
def test_mlp_vectors(oracle, golden, gelu, name):
    vec, tol = golden
    x = values(6, 3, 11.0)
    l1, l2, l3 = values(15, 17, 23.0), values(15, 41, 29.0), values(15, 67, 31.0)
    out = np.zeros(6, np.float32)
    oracle.oracle_gated_mlp_f32(O.ptr(x), 2, 3, 5, O.ptr(l1), O.ptr(l2), O.ptr(l3), gelu,
                                O.ptr(out))
    close(out, vec[name], tol)


@pytest.mark.parametrize("orientation,mode,name", [(0, 0, "fir"), (1, 1, "fir_causal_gated")])
def test_fir_vectors(oracle, golden, orientation, mode, name):
    vec, tol = golden
    x, w, b = values(15, 5, 13.0), values(9, 29, 17.0), values(3, 53, 19.0)
    out = np.zeros(15, np.float32)
    oracle.oracle_causal_fir(O.ptr(x), 5, 3, O.ptr(w), 3, O.ptr(b), orientation, mode,
                             O.ptr(out))
    close(out, vec[name], tol)


def test_hcl_vectors(oracle, golden):
    vec, tol = golden
    x2, x1, v = values(12, 2, 9.0), values(12, 37, 11.0), values(12, 71, 13.0)
    direct = values(3, 13, 17.0)
    log_poles = np.array([-0.03 * (i + 1) for i in range(6)], np.float32)
    residues = values(6, 23, 19.0)
    state = values(6, 47, 31.0)
    out = np.zeros(12, np.float32)
    oracle.oracle_hcl_recurrence(O.ptr(x2), O.ptr(x1), O.ptr(v), 4, 3, O.ptr(direct),
                                 O.ptr(log_poles), O.ptr(residues), 2, O.ptr(state),
                                 O.ptr(out))
    close(out, vec["hcl"], tol)
    close(state, vec["hcl_state"], tol)


def test_rope_and_attention_vectors(oracle, golden):
    vec, tol = golden
    q, k, v = values(24, 59, 13.0), values(24, 83, 17.0), values(24, 107, 19.0)
    inv = np.array([1.0, 0.01], np.float32)
    oracle.oracle_apply_rope(O.ptr(q), O.ptr(k), 3, 2, 4, O.ptr(inv), 5, 128.0)
    close(q, vec["rope_query"], tol)
    close(k, vec["rope_key"], tol)
    out = np.zeros(24, np.float32)
    oracle.oracle_causal_attention(O.ptr(q), O.ptr(k), O.ptr(v), 3, 2, 4, O.ptr(out))
    close(out, vec["attention"], tol)


def test_hyena_split_matches_vectors(golden):
    """The mixer's (x2, x1, v) de-interleave: with delta short taps (current
    row only) and an identity HCS filter, the oracle's mixer output is
    x2 * x1 * v, which must equal the product of the reference's split
    vectors hyena_x2 / hyena_x1 / hyena_value."""
    vec, tol = golden
    projection = values(24, 11, 15.0).reshape(2, 12)
    short = np.tile(np.array([0.0, 0.0, 1.0], np.float32), (12, 1))
    inner = np.zeros((1, 7), np.float32)
    inner[0, 6] = 1.0  # cross-correlation: last tap multiplies the current row
    out = O.hyena_mixer(0, projection, 4, short, inner_w=inner, groups=1, inner_len=7)
    expected = (np.array(vec["hyena_x2"]) * np.array(vec["hyena_x1"]) *
                np.array(vec["hyena_value"]))
    np.testing.assert_allclose(out.ravel(), expected, atol=tol["atol"], rtol=tol["rtol"])


# -------------------------------------------------- closed forms (KATs)
def test_kat_rmsnorm_eps_after_sqrt(oracle):
    x, s, out = np.array([3, 4], np.float32), np.array([1, 2], np.float32), np.zeros(2, np.float32)
    oracle.oracle_rms_norm(O.ptr(x), 1, 2, O.ptr(s), 0.25, O.ptr(out))
    den = np.sqrt(np.float32(12.5)) + np.float32(0.25)
    assert np.allclose(out, [3 / den, 8 / den], atol=1e-6)


def test_kat_fir_order_and_hcm(oracle):
    """Cross-correlation FIR of [1,2,3,4] with taps [1,2,3] gives [3,8,14,20];
    causal convolution with D=0.5 gives [1.5,5,11.5,18]
    (tests/test_cpu_reference.cpp:186-212)."""
    x = np.array([1, 2, 3, 4], np.float32)
    w = np.array([1, 2, 3], np.float32)
    out = np.zeros(4, np.float32)
    oracle.oracle_causal_fir(O.ptr(x), 4, 1, O.ptr(w), 3, None, 0, 0, O.ptr(out))
    assert out.tolist() == [3, 8, 14, 20]
    d = np.array([0.5], np.float32)
    oracle.oracle_causal_fir(O.ptr(x), 4, 1, O.ptr(w), 3, O.ptr(d), 1, 1, O.ptr(out))
    assert out.tolist() == [1.5, 5, 11.5, 18]


def test_kat_hcl_is_a_causal_convolution(oracle):
    """HCL == causal conv with h[t] = sum_m R_m p_m^t plus D*u (the modal
    identity), checked in float64 on a random case."""
    r = np.random.Generator(np.random.PCG64(0))
    L, W, S = 40, 3, 4
    x2, x1, v = (r.standard_normal((L, W)).astype(np.float32) for _ in range(3))
    lp = np.log(r.uniform(0.5, 0.99, (W, S))).astype(np.float32)
    res = r.standard_normal((W, S)).astype(np.float32) * 0.1
    d = r.standard_normal(W).astype(np.float32)
    state = np.zeros((W, S), np.float32)
    out = np.zeros((L, W), np.float32)
    oracle.oracle_hcl_recurrence(O.ptr(x2), O.ptr(x1), O.ptr(v), L, W, O.ptr(d), O.ptr(lp),
                                 O.ptr(res), S, O.ptr(state), O.ptr(out))
    u = (x1.astype(np.float64) * v)
    p = np.exp(lp.astype(np.float64))
    t = np.arange(L)
    h = (res[None, :, :] * p[None, :, :] ** t[:, None, None]).sum(-1)  # [L, W]
    conv = np.array([[np.dot(h[:i + 1, c][::-1], u[:i + 1, c]) for c in range(W)]
                     for i in range(L)])
    expected = x2 * (conv + d * u)
    np.testing.assert_allclose(out, expected, rtol=1e-4, atol=1e-5)


def test_kat_hcl_state(oracle):
    """Reference case tests/test_cpu_reference.cpp:215-229: outputs [22, 88.5]
    and final state 12.25."""
    x2 = np.array([2.0, 3.0], np.float32)
    x1 = np.array([1.0, 2.0], np.float32)
    v = np.array([4.0, 5.0], np.float32)
    d = np.array([0.5], np.float32)
    lp = np.array([np.log(0.5)], np.float32)
    res = np.array([2.0], np.float32)
    state = np.array([1.0], np.float32)
    out = np.zeros(2, np.float32)
    oracle.oracle_hcl_recurrence(O.ptr(x2), O.ptr(x1), O.ptr(v), 2, 1, O.ptr(d), O.ptr(lp),
                                 O.ptr(res), 1, O.ptr(state), O.ptr(out))
    assert np.allclose(out, [22.0, 88.5]) and np.isclose(state[0], 12.25)


# ------------------------------------------------------------ FP8 codec
FP8_VALUES = [-448.0, -432.0, -416.0, -1.25, -1.1875, -1.125, -1.0625, -1.0, -0.5,
              -0.015625, -0.00390625, -0.001953125, -0.0009765625, -0.0, 0.0,
              0.0009765625, 0.001953125, 0.0029296875, 0.00390625, 0.015625, 0.5,
              1.0, 1.0625, 1.125, 1.1875, 1.25, 416.0, 432.0, 448.0]
FP8_CODES = [0xfe, 0xfe, 0xfd, 0xba, 0xba, 0xb9, 0xb8, 0xb8, 0xb0, 0x88, 0x82, 0x81,
             0x80, 0x80, 0x00, 0x00, 0x01, 0x02, 0x02, 0x08, 0x30, 0x38, 0x38, 0x39,
             0x3a, 0x3a, 0x7d, 0x7e, 0x7e]


def test_e4m3_reference_codes(oracle):
    assert [oracle.oracle_e4m3_encode(v) for v in FP8_VALUES] == FP8_CODES


def test_e4m3_roundtrip_and_special_values(oracle):
    for code in range(256):
        value = oracle.oracle_e4m3_decode(code)
        if (code & 0x7f) == 0x7f:
            assert np.isnan(value)
            continue
        assert oracle.oracle_e4m3_encode(value) == code
    assert oracle.oracle_e4m3_encode(float("inf")) == 0x7e
    assert oracle.oracle_e4m3_encode(float("-inf")) == 0xfe
    assert oracle.oracle_e4m3_encode(float("nan")) & 0x7f == 0x7f
    assert oracle.oracle_e4m3_decode(0x7e) == 448.0
    assert oracle.oracle_e4m3_decode(0x01) == 2.0 ** -9


def test_e4m3_matches_numpy_codec_on_dense_grid(oracle):
    """The artifact writer's vectorised encoder agrees with the oracle on
    every BF16 value times several scales (RNE ties, subnormals, saturation)."""
    from evo_hip.fp8 import e4m3_encode
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = A.bf16_to_f32(bits)
    for scale in (1.0, 5.75, 0.03125):
        expected = np.zeros(bits.size, np.uint8)
        oracle.oracle_e4m3_quantize_bf16(O.ptr(bits), bits.size, scale, O.ptr(expected))
        got = e4m3_encode(x * np.float32(scale))
        finite = np.isfinite(x)
        assert np.array_equal(got[finite], expected[finite])


def _decode(codes):
    L = O.lib()
    return np.array([L.oracle_e4m3_decode(int(c)) for c in codes.ravel()],
                    np.float64).reshape(codes.shape)


def test_qgmma_exact_when_no_bits_are_lost():
    """Codes with significand 1.0 and exponents within 7 binades: every
    aligned term keeps all bits, so QGMMA == bf16(exact dot * scale)."""
    r = np.random.Generator(np.random.PCG64(3))
    exps = r.integers(4, 9, size=(5, 64))
    signs = r.integers(0, 2, size=(5, 64)) * 0x80
    a = ((exps << 3) | signs).astype(np.uint8)
    w = (((r.integers(5, 8, size=(7, 64))) << 3) | (r.integers(0, 2, (7, 64)) * 0x80)).astype(np.uint8)
    out = O.qgmma(a, w, 1.0)
    exact = _decode(a) @ _decode(w).T
    assert np.array_equal(out, A.bf16_to_f32(A.bf16_bits(exact.astype(np.float32))))


def _qgmma_bruteforce(a_vals, w_vals, scale, group=32):
    """Independent restatement over exact rationals of the QGMMA rule
    (tests/test_cuda_ops.cu:150-187): per group, top = max exponent over the
    accumulator and nonzero products; every term truncated toward zero to a
    multiple of 2^(top-13); sum; truncate to 14 significant bits."""
    def exponent(x):
        return int(np.floor(np.log2(abs(x))))
    acc = Fraction(0)
    for start in range(0, len(a_vals), group):
        terms = [(Fraction(a_vals[i]) * Fraction(w_vals[i]),
                  exponent(a_vals[i]) + exponent(w_vals[i]))
                 for i in range(start, start + group) if a_vals[i] != 0 and w_vals[i] != 0]
        top = max([e for _, e in terms] + ([exponent(float(acc))] if acc else []),
                  default=None)
        if top is None:
            continue
        quantum = Fraction(2) ** (top - 13)

        def trunc(x):
            q = abs(x) / quantum
            return (1 if x >= 0 else -1) * (q.numerator // q.denominator) * quantum
        total = sum(trunc(t) for t, _ in terms) + (trunc(acc) if acc else 0)
        if total == 0:
            acc = Fraction(0)
            continue
        e = exponent(float(total))
        q = abs(total) / Fraction(2) ** (e - 13)
        acc = (1 if total > 0 else -1) * (q.numerator // q.denominator) * Fraction(2) ** (e - 13)
    return float(A.bf16_to_f32(A.bf16_bits(np.array([float(acc) * scale], np.float32)))[0])


def test_qgmma_matches_bruteforce_rationals():
    r = np.random.Generator(np.random.PCG64(11))
    a = r.integers(0, 256, size=(3, 64)).astype(np.uint8)
    w = r.integers(0, 256, size=(5, 64)).astype(np.uint8)
    a[(a & 0x7f) == 0x7f] = 0x3c  # no NaN codes
    w[(w & 0x7f) == 0x7f] = 0x3c
    out = O.qgmma(a, w, 0.03125)
    da, dw = _decode(a), _decode(w)
    for i in range(3):
        for j in range(5):
            assert out[i, j] == _qgmma_bruteforce(da[i], dw[j], 0.03125)


# ------------------------------------------------------------ whole model
def test_oracle_matches_committed_reference_logits(tmp_path):
    golden = np.load(os.path.join(GOLDEN, "tiny_reference_logits.npz"))
    shape = A.tiny_shape(**{k: int(golden[k]) for k in ("width", "layers", "heads", "inner",
                                                         "groups")}, attn=(3,))
    path = str(tmp_path / "tiny.safetensors")
    A.random_artifact(shape, seed=int(golden["seed"])).write(path)
    logits = O.OracleModel(path).prefill(golden["tokens"])
    assert np.array_equal(logits.view(np.uint32), golden["logits"].view(np.uint32))


@pytest.mark.skipif(not os.path.exists(O.REFERENCE_LIB),
                    reason="reference CPU library not built (needs /root/reference)")
@pytest.mark.parametrize("width,heads,groups,inner,length,fp8", [
    (64, 4, 16, 96, 70, False), (40, 4, 8, 72, 300, False), (44, 2, 4, 52, 33, False)])
def test_oracle_bit_exact_with_reference_library(tmp_path, width, heads, groups, inner,
                                                 length, fp8):
    from evo_hip import capi
    shape = A.tiny_shape(width=width, heads=heads, groups=groups, inner=inner, hcm_len=16)
    path = str(tmp_path / "m.safetensors")
    A.random_artifact(shape, seed=width).write(path)
    tokens = A.acgt_tokens(length, seed=length)
    ref = capi.EvoLibrary(O.REFERENCE_LIB).load(path, capi.BACKEND_CPU)
    expected = ref.context(4096).prefill(tokens.astype(np.uint8).tobytes())
    for chunk in (256, 17):
        got = O.OracleModel(path).prefill(tokens, chunk=chunk)
        assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


def test_oracle_capture_matches_next_layer_input(tmp_path):
    shape = A.tiny_shape(width=64, layers=4, heads=4, inner=64, groups=16, attn=(3,))
    path = str(tmp_path / "c.safetensors")
    A.random_artifact(shape, seed=5).write(path)
    model = O.OracleModel(path)
    tokens = A.acgt_tokens(20, seed=5)
    logits, hidden = model.prefill(tokens, capture_layer=3)
    assert hidden.shape == (20, 64) and np.isfinite(hidden).all()
    assert np.array_equal(model.prefill(tokens), logits)


def test_qgmma_matches_bruteforce_on_quantised_normals():
    """Codes of quantised N(0, 1) activations and N(0, 0.02) weights (the
    config-3 distributions: many binades, subnormal codes, accumulators that
    grow across 16 groups of 32), against the rational restatement."""
    r = np.random.Generator(np.random.PCG64(12))
    x = r.standard_normal((4, 512)).astype(np.float32)
    w = (r.standard_normal((6, 512)) * 0.02).astype(np.float32)
    x[:, ::37] *= 1e-4  # a few values in the subnormal code range
    w[:, ::41] *= 1e-4
    a = O.quantize_f32(x, 448.0 / float(np.abs(x).max()))
    b = O.quantize_f32(w, 448.0 / float(np.abs(w).max()))
    assert np.any((a & 0x78) == 0) and np.any((b & 0x78) == 0)  # subnormal codes present
    out = O.qgmma(a, b, 0.0078125)
    da, dw = _decode(a), _decode(b)
    for i in range(4):
        for j in range(6):
            assert out[i, j] == _qgmma_bruteforce(da[i], dw[j], 0.0078125)


def test_oracle_fp8_conversion_matches_artifact_codes(tmp_path):
    """oracle_model_convert_fp8 (load-time conversion of BF16 projections)
    equals the same model written with codes and scales from the numpy
    encoder: weight_scale = 448 / amax(W), codes = E4M3(W * scale), input
    scale 448 / 8, output scale 1 / (input * weight)."""
    from evo_hip.fp8 import e4m3_encode
    shape = A.tiny_shape(width=64, layers=4, heads=4, inner=64, groups=16, attn=(3,))
    art = A.random_artifact(shape, seed=9)
    bf16_path = str(tmp_path / "bf16.safetensors")
    art.write(bf16_path)
    for index, spec in enumerate(list(art.specs)):
        if not spec.name.endswith(".projections.weight"):
            continue
        bits = art._make(index)
        weight = A.bf16_to_f32(bits)
        weight_scale = np.float32(448.0) / np.float32(np.abs(weight).max())
        input_scale = np.float32(448.0 / 8.0)
        codes = e4m3_encode(weight * weight_scale)
        scales = np.array([input_scale, np.float32(1) / (input_scale * weight_scale)],
                          np.float32)
        art.specs[index] = A.TensorSpec(spec.name, "F8_E4M3", spec.shape,
                                        lambda rng, c=codes: c)
        art.add(spec.name.replace(".weight", ".fp8_runtime_scales"), "F32", (2,),
                lambda rng, s=scales: s)
    fp8_path = str(tmp_path / "fp8.safetensors")
    art.write(fp8_path)
    tokens = A.acgt_tokens(40, seed=9)
    converted = O.OracleModel(bf16_path).convert_fp8(8.0).prefill(tokens)
    written = O.OracleModel(fp8_path).prefill(tokens)
    assert np.array_equal(converted.view(np.uint32), written.view(np.uint32))
    assert not np.array_equal(converted, O.OracleModel(bf16_path).prefill(tokens))


@pytest.mark.parametrize("group", [8, 16, 24, 12])
def test_qgmma_group_sizes_and_ragged_columns(group):
    """The vector walk (groups a multiple of 8: eight output columns per
    vector, ragged last column tile) and the scalar walk (other groups)
    against the rational restatement."""
    r = np.random.Generator(np.random.PCG64(100 + group))
    k = 4 * group * (2 if group < 16 else 1)
    a = r.integers(0, 256, size=(3, k)).astype(np.uint8)
    w = r.integers(0, 256, size=(11, k)).astype(np.uint8)
    a[(a & 0x7f) == 0x7f] = 0x41
    w[(w & 0x7f) == 0x7f] = 0x39
    out = O.qgmma(a, w, 0.0625, group_k=group)
    da, dw = _decode(a), _decode(w)
    for i in range(3):
        for j in range(11):
            assert out[i, j] == _qgmma_bruteforce(da[i], dw[j], 0.0625, group=group)


def test_e4m3_quantize_bf16_table_path_equals_direct_encode():
    """Large inputs encode through a 65536-entry table: every BF16 pattern,
    repeated past the table threshold, gets the code of the direct encoder."""
    L = O.lib()
    L.oracle_e4m3_quantize_bf16.argtypes = [O.P, O.S, O.F, O.P]
    patterns = np.arange(1 << 16, dtype=np.uint16)
    for scale in (1.0, 448.0 / 3.1, 2.0 ** -7):
        direct = np.zeros(patterns.size, np.uint8)
        L.oracle_e4m3_quantize_bf16(O.ptr(patterns), patterns.size, scale, O.ptr(direct))
        big = np.tile(patterns, 5)
        table = np.zeros(big.size, np.uint8)
        L.oracle_e4m3_quantize_bf16(O.ptr(big), big.size, scale, O.ptr(table))
        assert np.array_equal(table, np.tile(direct, 5))
        spot = [int(L.oracle_e4m3_encode(float(A.bf16_to_f32(np.array([p], np.uint16))[0])
                                          * np.float32(scale))) for p in patterns[::4099]]
        assert spot == list(direct[::4099])
