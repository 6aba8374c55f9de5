"""GPU parity of each gfx950 kernel, called through the operator C ABI
(include/evo/hip_ops.h), against the CPU oracle on identical seeded inputs.

Tolerances are stated per test: bit-exact for FP8 codes and the exact QGMMA
mode; relative (to the output scale) for floating-point kernels.
"""
import numpy as np
import pytest

import oracle_lib as O
from evo_hip import native as N
from evo_hip.artifact import bf16_bits, bf16_to_f32
from gpu_util import dev, empty, host, p, stream, zeros

pytestmark = pytest.mark.gpu


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def rel_err(actual, expected):
    scale = max(1e-30, float(np.abs(expected).max()))
    return float(np.abs(actual.astype(np.float64) - expected).max()) / scale


# ------------------------------------------------------------------ FP8
FP8_VALUES = [-448.0, -432.0, -416.0, -1.25, -1.1875, -1.125, -1.0625, -1.0, -0.5,
              -0.015625, -0.00390625, -0.001953125, -0.0009765625, -0.0, 0.0,
              0.0009765625, 0.001953125, 0.0029296875, 0.00390625, 0.015625, 0.5,
              1.0, 1.0625, 1.125, 1.1875, 1.25, 416.0, 432.0, 448.0]
FP8_CODES = [0xfe, 0xfe, 0xfd, 0xba, 0xba, 0xb9, 0xb8, 0xb8, 0xb0, 0x88, 0x82, 0x81,
             0x80, 0x80, 0x00, 0x00, 0x01, 0x02, 0x02, 0x08, 0x30, 0x38, 0x38, 0x39,
             0x3a, 0x3a, 0x7d, 0x7e, 0x7e]


def quantize_gpu(x: np.ndarray, scale: float, dtype=N.DTYPE_F32):
    d = dev(x)
    codes = empty(x.shape, np.uint8)
    N.call("evo_hip_e4m3_quantize", dtype, p(d), x.size, scale, p(codes), stream())
    return host(codes)


def test_e4m3_reference_vectors():
    """The 29 PyTorch code vectors of evo.cpp tests/test_cuda_ops.cu:371-431."""
    bits = bf16_bits(np.array(FP8_VALUES, np.float32))
    assert list(quantize_gpu(bits, 1.0, N.DTYPE_BF16)) == FP8_CODES
    assert list(quantize_gpu(np.array(FP8_VALUES, np.float32), 1.0)) == FP8_CODES


@pytest.mark.parametrize("scale", [1.0, 5.75, 3.25, 56.0, 0.03125, 448.0 / 6.1])
def test_e4m3_exhaustive_bf16(oracle, scale):
    """Every BF16 bit pattern (incl. inf/NaN/subnormals), bit-exact codes."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expected = np.zeros(65536, np.uint8)
    oracle.oracle_e4m3_quantize_bf16(O.ptr(bits), bits.size, scale, O.ptr(expected))
    assert np.array_equal(quantize_gpu(bits, scale, N.DTYPE_BF16), expected)


def test_e4m3_f32_rounds_through_bf16(oracle):
    x = rng(1).standard_normal(1 << 16).astype(np.float32) * 3
    assert np.array_equal(quantize_gpu(x, 56.0), O.quantize_f32(x, 56.0))


def fp8_case(seed, m, k, n, in_scale=5.75, w_scale=3.25):
    r = rng(seed)
    a = bf16_to_f32(bf16_bits(r.standard_normal((m, k)).astype(np.float32) * 2))
    w = bf16_to_f32(bf16_bits(r.standard_normal((n, k)).astype(np.float32) * 0.05))
    return O.quantize_f32(a, in_scale), O.quantize_f32(w, w_scale)


def fp8_gpu(a_codes, w_codes, out_scale, mode):
    m, k = a_codes.shape
    n = w_codes.shape[0]
    out = empty((m, n))
    N.call("evo_hip_fp8_linear", p(dev(a_codes)), p(dev(w_codes)), p(out), m, n, k,
           out_scale, mode, stream())
    return host(out)


@pytest.mark.parametrize("m,k,n", [(3, 64, 5), (1, 64, 5), (130, 256, 96), (64, 4096, 40)])
def test_qgmma_exact_bit_exact(m, k, n):
    """Reference case shape rows 3, K 64, N 5, scales 5.75/3.25/0.03125
    (tests/test_cuda_ops.cu:433-503) and larger ragged shapes."""
    a, w = fp8_case(7 + m, m, k, n)
    expected = O.qgmma(a, w, 0.03125)
    actual = fp8_gpu(a, w, 0.03125, N.FP8_EXACT)
    assert np.array_equal(actual.view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("mode", [N.FP8_MFMA_K32, N.FP8_MFMA_K128])
@pytest.mark.parametrize("m,k,n", [(128, 128, 128), (200, 512, 300), (1024, 4096, 256),
                                   (1, 4096, 300), (3, 8192, 96), (4, 1024, 1000)])
def test_fp8_mfma_close_to_qgmma(mode, m, k, n):
    """The MFMA modes do not reproduce QGMMA's per-term truncation (13
    fractional bits under each group's maximum) nor the hardware's own
    in-instruction rounding; measured against the exact emulation at
    K = 4096 their RMS deviation is about 2^-8 of the RMS output (one BF16
    ulp), the exact float64 dot itself sits 2^-9 away. Bounds: RMS deviation
    <= 2^-7 (k32) / 2^-8 (k128) of the RMS output, worst element <= 2^-6 of
    the output scale."""
    a, w = fp8_case(11 + m, m, k, n)
    expected = O.qgmma(a, w, 0.03125).astype(np.float64)
    actual = fp8_gpu(a, w, 0.03125, mode).astype(np.float64)
    rms = np.sqrt(np.mean(expected ** 2))
    bound = 2.0 ** -7 if mode == N.FP8_MFMA_K32 else 2.0 ** -8
    assert np.sqrt(np.mean((actual - expected) ** 2)) <= bound * rms
    assert np.abs(actual - expected).max() <= 2.0 ** -6 * np.abs(expected).max()


@pytest.mark.parametrize("mode", [N.FP8_MFMA_K32, N.FP8_MFMA_K128, N.FP8_EXACT])
def test_fp8_linear_bf16_output_equals_f32_output(mode):
    """BF16-output variant: bit-identical to the F32 output (every value is
    already a BF16 number)."""
    a, w = fp8_case(23, 300, 512, 200)
    f32 = fp8_gpu(a, w, 0.03125, mode)
    out = empty((300, 200), np.uint16)
    N.call("evo_hip_fp8_linear_bf16", p(dev(a)), p(dev(w)), p(out), 300, 200, 512, 0.03125,
           mode, stream())
    assert np.array_equal(host(out).view(np.uint16), bf16_bits(f32))
    assert np.array_equal(bf16_to_f32(bf16_bits(f32)), f32)


@pytest.mark.parametrize("m", [64, 1, 4])
def test_fp8_mfma_exact_on_representable_sums(m):
    """Codes restricted to +-{1, 1.5, 2}: every QGMMA term and partial sum is
    exact, so all three modes must agree bit for bit (m <= 4 runs the few-row
    kernel, whose codes are decoded by the hardware convert)."""
    r = rng(5 + m)
    choices = np.array([0x38, 0x3c, 0x40, 0xb8, 0xbc, 0xc0], np.uint8)
    a = choices[r.integers(0, 6, (m, 256))]
    w = choices[r.integers(0, 6, (96, 256))]
    exact = fp8_gpu(a, w, 1.0, N.FP8_EXACT)
    for mode in (N.FP8_MFMA_K32, N.FP8_MFMA_K128):
        assert np.array_equal(fp8_gpu(a, w, 1.0, mode), exact)
    dense = O.lib()  # closed form: plain dot of the decoded values
    dec = np.vectorize(lambda c: dense.oracle_e4m3_decode(int(c)))
    ref = dec(a).astype(np.float64) @ dec(w).astype(np.float64).T
    # the reference rounds the promoted accumulator to BF16 on output
    assert np.array_equal(exact, bf16_to_f32(bf16_bits(ref.astype(np.float32))))


# ---------------------------------------------------------------- GEMM
@pytest.mark.parametrize("m,n,k", [(1, 40, 64), (130, 200, 72), (256, 384, 1024),
                                   (2, 4096, 4096), (3, 77, 11264), (4, 520, 1920),
                                   (5, 96, 256)])
@pytest.mark.parametrize("bias,residual", [(False, False), (True, True), (False, True)])
def test_linear_split_matches_oracle(m, n, k, bias, residual):
    """m <= 4 runs the few-row (decode) kernel, m >= 5 the MFMA tile kernel."""
    r = rng(m + n + k)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = bf16_bits(r.standard_normal((n, k)).astype(np.float32) / np.sqrt(k))
    b = bf16_bits(r.standard_normal(n).astype(np.float32) * 0.1) if bias else None
    res = r.standard_normal((m, n)).astype(np.float32) if residual else None
    expected = O.linear_bf16w(x, w, b)
    if residual:
        expected = expected + res
    out = empty((m, n))
    hi, lo = split_gpu(x)
    N.call("evo_hip_linear", p(hi), p(lo), p(dev(w)), p(dev(b) if bias else None),
           p(dev(res) if residual else None), m, n, k, p(out), stream())
    # split-BF16 activations: ~2^-17 relative per product, F32 accumulation
    assert rel_err(host(out), expected) < 2e-5


@pytest.mark.parametrize("m,n,k", [(256, 512, 1920), (300, 1000, 2048), (5, 64, 512),
                                   (1024, 4096, 11264)])
@pytest.mark.parametrize("bias,residual", [(False, False), (True, True), (False, True)])
def test_linear_split_k_matches_oracle(m, n, k, bias, residual):
    """Few-tile launches split K over blocks (2-16 splits on these shapes) and
    sum the partials in split order before the epilogue: the result is the
    unsplit product up to the F32 summation order, and matches the oracle."""
    r = rng(m + n + k + 7)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = bf16_bits(r.standard_normal((n, k)).astype(np.float32) / np.sqrt(k))
    b = bf16_bits(r.standard_normal(n).astype(np.float32) * 0.1) if bias else None
    res = r.standard_normal((m, n)).astype(np.float32) if residual else None
    hi, lo = split_gpu(x)
    args = (p(hi), p(lo), p(dev(w)), p(dev(b) if bias else None),
            p(dev(res) if residual else None), m, n, k)
    unsplit, parted = empty((m, n)), empty((m, n))
    N.call("evo_hip_linear", *args, p(unsplit), stream())
    workspace = empty((16 * m * n,))
    N.call("evo_hip_linear_split", *args, p(parted), p(workspace), 16 * m * n * 4, stream())
    assert rel_err(host(parted), host(unsplit)) < 1e-5  # ~sqrt(K) F32 ulps
    if m * n * k <= 1 << 31:
        expected = O.linear_bf16w(x, w, b)
        if residual:
            expected = expected + res
        assert rel_err(host(parted), expected) < 2e-5
    # A workspace too small for any split runs the unsplit kernel.
    tiny = empty((m * n,))
    N.call("evo_hip_linear_split", *args, p(parted), p(tiny), m * n * 4, stream())
    assert np.array_equal(host(parted), host(unsplit))


@pytest.mark.parametrize("m,n,k,bias,residual", [(256, 76800, 512, True, True),
                                                  (600, 25000, 1024, False, False),
                                                  (600, 25000, 1024, False, True)])
def test_linear_tail_split_matches_unsplit(m, n, k, bias, residual):
    """A launch whose last round of 256 x 256 tiles would fill at most half
    of the 256 CUs (here 300 = 256 + 44 and 294 = 256 + 38 tiles, the second
    with ragged M and N) runs those last tiles as two K halves, summed in
    order before the epilogue: the unsplit product up to the F32 summation
    order, and the oracle's on the columns of the split tiles."""
    r = rng(m + n + k + 11)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = bf16_bits(r.standard_normal((n, k)).astype(np.float32) / np.sqrt(k))
    b = bf16_bits(r.standard_normal(n).astype(np.float32) * 0.1) if bias else None
    res = r.standard_normal((m, n)).astype(np.float32) if residual else None
    hi, lo = split_gpu(x)
    args = (p(hi), p(lo), p(dev(w)), p(dev(b) if bias else None),
            p(dev(res) if residual else None), m, n, k)
    unsplit, parted = empty((m, n)), empty((m, n))
    N.call("evo_hip_linear", *args, p(unsplit), stream())
    tiles = -(-m // 256) * -(-n // 256)
    tail = tiles % 256
    assert tiles > 256 and 0 < tail <= 128
    workspace = empty((2 * tail * 256 * 256,))
    N.call("evo_hip_linear_split", *args, p(parted), p(workspace), workspace.numel() * 4, stream())
    got, plain = host(parted), host(unsplit)
    assert rel_err(got, plain) < 1e-5
    assert not np.array_equal(got, plain)  # the split path ran
    cols = slice(n - 512, n)  # inside the split tiles (the last in tile order)
    expected = O.linear_bf16w(x, w[cols], b[cols] if bias else None)
    if residual:
        expected = expected + res[:, cols]
    assert rel_err(got[:, cols], expected) < 2e-5
    # One byte short of the partials: the unsplit launch, bit for bit.
    N.call("evo_hip_linear_split", *args, p(parted), p(workspace), workspace.numel() * 4 - 1,
           stream())
    assert np.array_equal(host(parted), plain)


def split_gpu(x):
    hi, lo = empty(x.shape, np.uint16), empty(x.shape, np.uint16)
    N.call("evo_hip_split_f32", p(dev(x)), x.size, p(hi), p(lo), stream())
    return hi, lo


def test_split_planes_exact():
    x = rng(2).standard_normal(4099).astype(np.float32) * 100
    hi, lo = split_gpu(x)
    h, l = host(hi).view(np.uint16), host(lo).view(np.uint16)
    assert np.array_equal(h, bf16_bits(x))
    assert np.array_equal(l, bf16_bits(x - bf16_to_f32(h)))
    # hi + lo carries 16 significant bits: |x - (hi + lo)| <= 2^-16 |x|
    assert np.all(np.abs(x - bf16_to_f32(h) - bf16_to_f32(l)) <= 2.0 ** -16 * np.abs(x))


def test_linear_bf16_profile_is_bf16_accurate():
    r = rng(3)
    x = r.standard_normal((96, 512)).astype(np.float32)
    w = bf16_bits(r.standard_normal((160, 512)).astype(np.float32) / 22.6)
    out = empty((96, 160))
    hi, _ = split_gpu(x)
    N.call("evo_hip_linear", p(hi), None, p(dev(w)), None, None, 96, 160, 512,
           p(out), stream())
    expected = O.linear_bf16w(bf16_to_f32(bf16_bits(x)), w)
    assert rel_err(host(out), expected) < 2e-5


@pytest.mark.parametrize("gelu", [1, 0])
@pytest.mark.parametrize("m", [70, 1, 3])
def test_gated_mlp(gelu, m):
    """m = 70: MFMA tiles; m = 1, 3: the few-row kernel's gated epilogue."""
    from scipy.special import erf
    r = rng(17 + gelu + m)
    width, inner = 96, 80  # inner not a multiple of 32: padded block
    x = r.standard_normal((m, width)).astype(np.float32)
    l1 = bf16_bits(r.standard_normal((inner, width)).astype(np.float32) / 10)
    l2 = bf16_bits(r.standard_normal((inner, width)).astype(np.float32) / 10)
    l3 = bf16_bits(r.standard_normal((width, inner)).astype(np.float32) / 9)
    res = r.standard_normal((m, width)).astype(np.float32)
    padded = (inner + 31) // 32 * 32
    w12 = zeros((2 * padded, width), np.uint16)
    N.call("evo_hip_pack_mlp", p(dev(l1)), p(dev(l2)), inner, width, p(w12), stream())
    scratch, out = empty((2 * m * inner,), np.uint16), empty((m, width))
    hi, lo = split_gpu(x)
    N.call("evo_hip_gated_mlp", p(hi), p(lo), p(w12), p(dev(l3)), m, width, inner, gelu,
           p(scratch), p(dev(res)), p(out), stream())
    first = O.linear_bf16w(x, l1).astype(np.float64)
    second = O.linear_bf16w(x, l2).astype(np.float64)
    act = 0.5 * first * (1 + erf(first / np.sqrt(2))) if gelu else first
    expected = O.linear_bf16w((act * second).astype(np.float32), l3) + res
    assert rel_err(host(out), expected) < 1e-4


def test_rms_norm(oracle):
    r = rng(9)
    for rows, width in [(3, 257), (64, 4096), (5, 1920)]:
        x = r.standard_normal((rows, width)).astype(np.float32) * 3
        scale = (1 + 0.1 * r.standard_normal(width)).astype(np.float32)
        expected = np.zeros_like(x)
        oracle.oracle_rms_norm(O.ptr(x), rows, width, O.ptr(scale), 1e-6, O.ptr(expected))
        out = empty((rows, width))
        hi, lo = empty((rows, width), np.uint16), empty((rows, width), np.uint16)
        N.call("evo_hip_rms_norm", p(dev(x)), rows, width, p(dev(scale)), 1e-6, p(out),
               p(hi), p(lo), stream())
        got = host(out)
        assert rel_err(got, expected) < 1e-5
        # the planes are the split of the F32 result
        assert np.array_equal(host(hi).view(np.uint16), bf16_bits(got))
        assert np.array_equal(host(lo).view(np.uint16),
                              bf16_bits(got - bf16_to_f32(bf16_bits(got))))


@pytest.mark.parametrize("rows,width,code_scale", [(64, 4096, 448.0 / 8.0), (5, 1920, 17.5),
                                                  (3, 257, 3.0)])
def test_rms_norm_e4m3_codes(rows, width, code_scale):
    """The norm fused with the FP8 input quantisation: codes are bit-exact
    E4M3(bf16(y) * scale) of the norm's own F32 output (oracle encoder)."""
    r = rng(rows + width)
    x = r.standard_normal((rows, width)).astype(np.float32) * 2
    scale = (1 + 0.1 * r.standard_normal(width)).astype(np.float32)
    out = empty((rows, width))
    N.call("evo_hip_rms_norm", p(dev(x)), rows, width, p(dev(scale)), 1e-6, p(out),
           None, None, stream())
    y = host(out)
    codes = empty((rows * width,), np.uint8)
    N.call("evo_hip_rms_norm_e4m3", p(dev(x)), rows, width, p(dev(scale)), 1e-6, code_scale,
           p(codes), stream())
    expected = np.zeros(rows * width, np.uint8)
    bits = np.ascontiguousarray(bf16_bits(y).ravel())
    O.lib().oracle_e4m3_quantize_bf16(O.ptr(bits), bits.size, code_scale, O.ptr(expected))
    assert np.array_equal(host(codes), expected)


@pytest.mark.parametrize("m,k,n", [(1, 4096, 12288), (3, 1920, 520), (4, 4096, 1000)])
@pytest.mark.parametrize("split", [1, 0])
def test_linear_normed_equals_norm_then_linear(m, k, n, split):
    """Decode's folded norm: the product of norm(x) formed inside the
    product's blocks is bit-identical to rms_norm's planes fed to the
    few-row product (and so within the linear tests' oracle bounds)."""
    r = rng(m * 7 + k + n + split)
    x = r.standard_normal((m, k)).astype(np.float32) * 3
    scale = (1 + 0.1 * r.standard_normal(k)).astype(np.float32)
    w = bf16_bits(r.standard_normal((n, k)).astype(np.float32) * 0.02)
    x_d, s_d, w_d = dev(x), dev(scale), dev(w)
    hi, lo = empty((m, k), np.uint16), empty((m, k), np.uint16)
    N.call("evo_hip_rms_norm", p(x_d), m, k, p(s_d), 1e-6, None, p(hi), p(lo), stream())
    two_step = empty((m, n))
    N.call("evo_hip_linear", p(hi), p(lo) if split else None, p(w_d), None, None, m, n, k,
           p(two_step), stream())
    folded = empty((m, n))
    N.call("evo_hip_linear_normed", p(x_d), m, k, p(s_d), 1e-6, split, p(w_d), n, p(folded),
           stream())
    assert np.array_equal(host(folded).view(np.uint32), host(two_step).view(np.uint32))


@pytest.mark.parametrize("m,k,n", [(1, 4096, 12288), (2, 1920, 1000), (4, 4096, 520)])
@pytest.mark.parametrize("mode", [0, 1])
def test_fp8_linear_normed_equals_norm_codes_then_linear(m, k, n, mode):
    """The folded FP8 projection forms the codes rms_norm_e4m3 writes, so
    its output equals the two-step path bit for bit."""
    r = rng(m * 11 + k + n + mode)
    x = r.standard_normal((m, k)).astype(np.float32) * 2
    scale = (1 + 0.1 * r.standard_normal(k)).astype(np.float32)
    w_codes = r.integers(0, 0x7e, (n, k), dtype=np.uint8)
    w_codes |= (r.integers(0, 2, (n, k), dtype=np.uint8) << 7)
    code_scale, out_scale = 448.0 / 8.0, 1.0 / 448.0
    x_d, s_d, w_d = dev(x), dev(scale), dev(w_codes)
    codes = empty((m * k,), np.uint8)
    N.call("evo_hip_rms_norm_e4m3", p(x_d), m, k, p(s_d), 1e-6, code_scale, p(codes),
           stream())
    two_step = empty((m, n), np.uint16)
    N.call("evo_hip_fp8_linear_bf16", p(codes), p(w_d), p(two_step), m, n, k, out_scale,
           mode, stream())
    folded = empty((m, n), np.uint16)
    N.call("evo_hip_fp8_linear_normed", p(x_d), m, k, p(s_d), 1e-6, code_scale, p(w_d), n,
           out_scale, mode, p(folded), stream())
    assert np.array_equal(host(folded), host(two_step))


def test_normed_products_reject_unsupported_shapes():
    x, scale = dev(np.ones((5, 256), np.float32)), dev(np.ones(256, np.float32))
    w = dev(np.zeros((8, 256), np.uint16))
    out = empty((5, 8))
    with pytest.raises(N.OpError):
        N.call("evo_hip_linear_normed", p(x), 5, 256, p(scale), 1e-6, 1, p(w), 8, p(out),
               stream())
    with pytest.raises(N.OpError):
        N.call("evo_hip_fp8_linear_normed", p(x), 1, 256, p(scale), 1e-6, 1.0, p(w), 8, 1.0,
               2, p(empty((1, 8), np.uint16)), stream())


# --------------------------------------------------------------- Hyena
def hyena_case(seed, kind, length, width, groups=16, inner_len=7, state=16):
    r = rng(seed)
    proj = r.standard_normal((length, 3 * width)).astype(np.float32)
    short = bf16_bits(r.standard_normal((3 * width, 3)).astype(np.float32) * 0.5)
    case = dict(projection=proj, short=short, width=width)
    if kind in (N.HYENA_HCS, N.HYENA_HCM):
        case["inner"] = bf16_to_f32(bf16_bits(
            r.standard_normal((groups, inner_len)).astype(np.float32) / np.sqrt(inner_len)))
        case["groups"], case["inner_len"] = groups, inner_len
    if kind in (N.HYENA_HCM, N.HYENA_HCL):
        case["direct"] = bf16_to_f32(bf16_bits(r.standard_normal(width).astype(np.float32) * 0.5))
    if kind == N.HYENA_HCL:
        case["log_poles"] = np.log(r.uniform(0.5, 0.99, (width, state))).astype(np.float32)
        case["residues"] = (r.standard_normal((width, state)) * 0.1).astype(np.float32)
        case["state"] = state
    return case


def hyena_oracle(kind, case, projection=None):
    return O.hyena_mixer(kind, case["projection"] if projection is None else projection,
                         case["width"], bf16_to_f32(case["short"]), case.get("inner"),
                         case.get("groups", 1), case.get("inner_len", 2),
                         case.get("direct"), case.get("log_poles"), case.get("residues"),
                         case.get("state", 0))


def planar(proj):
    """Interleaved projection columns (3c + s) -> planar (s * W + c)."""
    rows, cols = proj.shape
    return np.ascontiguousarray(proj.reshape(rows, cols // 3, 3).transpose(0, 2, 1)
                                .reshape(rows, cols))


CANARY = 0x7FC0DEAD  # a NaN payload no kernel writes


def guarded(shape, dtype, guard):
    """Output buffer with `guard` canary rows after it; returns (full, view)."""
    rows = int(np.prod(shape[:-1]))
    full = dev(np.full((rows + guard) * shape[-1] * np.dtype(dtype).itemsize // 4, CANARY,
                       np.uint32))
    return full, full.view(dev_dtype(dtype))[:rows * shape[-1]].view(shape)


def dev_dtype(dtype):
    import torch
    return {np.float32: torch.float32, np.uint16: torch.int16}[np.dtype(dtype).type]


def hyena_gpu(kind, case, dtype=N.DTYPE_F32, rows=None, caches=None, projection=None,
              planar_layout=False, bf16_taps=False, guard=0):
    proj = case["projection"] if projection is None else projection
    if planar_layout:
        proj = planar(proj)
    length = proj.shape[0] if rows is None else rows
    width = case["width"]
    state = case.get("state", 0)
    poles = np.exp(case["log_poles"]).astype(np.float32) if "log_poles" in case else None
    ws_bytes = N.call("evo_hip_hyena_workspace_bytes", kind, length, width, state)
    ws = empty((max(ws_bytes, 256),), np.uint8)
    out_shape, out_type = ((length, width), np.float32)
    if dtype in (N.DTYPE_BF16, N.DTYPE_F16, N.DTYPE_BF16_F16):
        out_shape, out_type = (length, width), np.uint16
    elif dtype in (N.DTYPE_SPLIT, N.DTYPE_BF16_SPLIT):
        out_shape, out_type = (2, length, width), np.uint16
    bf16_in = dtype in (N.DTYPE_BF16, N.DTYPE_BF16_SPLIT, N.DTYPE_BF16_F16)
    proj_d = dev(bf16_bits(proj) if bf16_in else proj)
    full = None
    if guard:
        full, out = guarded(out_shape, out_type, guard)
    else:
        out = empty(out_shape, out_type)
    caches = caches or {}
    flags = (N.DTYPE_PLANAR if planar_layout else 0) | (N.DTYPE_BF16_TAPS if bf16_taps else 0)
    N.call("evo_hip_hyena_forward", kind, dtype | flags,
           p(proj_d), length, width,
           p(dev(case["short"])), 3, p(dev(case["inner"]) if "inner" in case else None),
           case.get("groups", 1), case.get("inner_len", 0),
           p(dev(case["direct"]) if "direct" in case else None),
           p(dev(poles) if poles is not None else None),
           p(dev(case["residues"]) if "residues" in case else None), state,
           p(caches.get("short")), p(caches.get("inner")), p(caches.get("modal")),
           p(ws), ws_bytes, p(out), stream())
    result = host(out)
    if guard:
        tail = host(full)[out.numel() * np.dtype(out_type).itemsize // 4:]
        assert np.all(tail == CANARY), "rows past the output were written"
    if dtype in (N.DTYPE_SPLIT, N.DTYPE_BF16_SPLIT):
        planes = bf16_to_f32(result.view(np.uint16))
        return planes[0].astype(np.float64) + planes[1]
    if dtype in (N.DTYPE_F16, N.DTYPE_BF16_F16):
        return result.view(np.uint16).view(np.float16).astype(np.float32)
    return bf16_to_f32(result.view(np.uint16)) if dtype == N.DTYPE_BF16 else result


KINDS = [(N.HYENA_HCS, 7), (N.HYENA_HCM, 128), (N.HYENA_HCL, 0)]


@pytest.mark.parametrize("kind,inner_len", KINDS)
@pytest.mark.parametrize("length,width", [(1, 64), (300, 96), (1000, 128)])
def test_hyena_f32_matches_oracle(kind, inner_len, length, width):
    case = hyena_case(length + width + kind, kind, length, width, groups=16,
                      inner_len=inner_len or 7)
    expected = hyena_oracle(kind, case)
    assert rel_err(hyena_gpu(kind, case), expected) < 1e-5


@pytest.mark.parametrize("kind,inner_len", [(N.HYENA_HCS, 7), (N.HYENA_HCS, 5),
                                             (N.HYENA_HCM, 128), (N.HYENA_HCM, 33)])
@pytest.mark.parametrize("length,width,groups", [(1, 256, 16), (300, 256, 16),
                                                 (1000, 128, 4), (777, 512, 16)])
def test_hyena_fir_mfma_matches_oracle(kind, inner_len, length, width, groups):
    """Filter groups of 16k channels run the Toeplitz-MFMA FIR; F32 taps that
    are not BF16 numbers exercise the split-tap pass."""
    case = hyena_case(length + width + groups + inner_len, kind, length, width,
                      groups=groups, inner_len=inner_len)
    expected = hyena_oracle(kind, case)
    assert rel_err(hyena_gpu(kind, case), expected) < 1e-5
    proj = bf16_to_f32(bf16_bits(case["projection"]))
    expected = hyena_oracle(kind, case, projection=proj)
    actual = hyena_gpu(kind, case, dtype=N.DTYPE_BF16_SPLIT, projection=proj)
    assert rel_err(actual, expected) < 2e-5
    actual = hyena_gpu(kind, case, dtype=N.DTYPE_BF16_SPLIT, projection=proj,
                       planar_layout=True)
    assert rel_err(actual, expected) < 2e-5


@pytest.mark.parametrize("kind,inner_len", KINDS)
@pytest.mark.parametrize("dtype", [N.DTYPE_F32, N.DTYPE_BF16, N.DTYPE_SPLIT,
                                   N.DTYPE_BF16_SPLIT, N.DTYPE_BF16_F16])
@pytest.mark.parametrize("length", [2, 3, 295, 1025, 1031])
def test_hyena_leaves_rows_past_the_output(kind, inner_len, dtype, length):
    """Rows past the sequence end (the last chunk / segment / store pair is
    ragged: lengths not a multiple of 4) are never written: 64 canary rows
    after the output stay intact, and the rows inside match the oracle.
    Lengths 2 and 3 reach the prefill kernels' smallest chunks (a single row
    runs the decode kernel)."""
    case = hyena_case(3 * length + kind, kind, length, 64, groups=4, inner_len=inner_len or 7)
    proj = case["projection"]
    if dtype in (N.DTYPE_BF16, N.DTYPE_BF16_SPLIT, N.DTYPE_BF16_F16):
        proj = bf16_to_f32(bf16_bits(proj))
    expected = hyena_oracle(kind, case, projection=proj)
    actual = hyena_gpu(kind, case, dtype=dtype, projection=proj, guard=64,
                       bf16_taps=kind == N.HYENA_HCM)
    bound = {N.DTYPE_BF16: 2.0 ** -8, N.DTYPE_BF16_F16: 2.0 ** -11 + 2e-5}.get(dtype, 2e-5)
    assert rel_err(actual, expected) < bound


@pytest.mark.parametrize("kind,inner_len", KINDS)
def test_hyena_split_output(kind, inner_len):
    """F32 in, split planes out: hi + lo reproduces the F32 result to 2^-16."""
    case = hyena_case(91 + kind, kind, 513, 96, inner_len=inner_len or 7)
    expected = hyena_oracle(kind, case)
    assert rel_err(hyena_gpu(kind, case, dtype=N.DTYPE_SPLIT), expected) < 2e-5


@pytest.mark.parametrize("kind,inner_len", KINDS)
@pytest.mark.parametrize("length", [1, 777])
def test_hyena_f16_output(kind, inner_len, length):
    """One FP16 plane out (the one-pass FP16 out-projection's activation):
    with F32 input it is exactly fp16(y) of the F32-output kernel's y (RNE,
    saturated to +-65504), including a large-valued case that saturates; with
    BF16 input (the FP8 projection's output) it matches the oracle on the same
    BF16-rounded projection to FP16 rounding."""
    case = hyena_case(61 + kind + length, kind, length, 128, inner_len=inner_len or 7)
    for scale in (1.0, 3000.0):  # 3000: |y| ~ 1e5..1e7 exceeds the FP16 range
        big = dict(case, projection=(case["projection"] * scale).astype(np.float32))
        y = hyena_gpu(kind, big)
        expected16 = np.clip(y, -65504.0, 65504.0).astype(np.float16).astype(np.float32)
        actual16 = hyena_gpu(kind, big, dtype=N.DTYPE_F16)
        assert np.array_equal(actual16.view(np.uint32), expected16.view(np.uint32))
    proj = bf16_to_f32(bf16_bits(case["projection"]))
    expected = hyena_oracle(kind, case, projection=proj)
    actual = hyena_gpu(kind, case, dtype=N.DTYPE_BF16_F16, projection=proj,
                       bf16_taps=kind == N.HYENA_HCM)
    assert rel_err(actual, expected) <= 2.0 ** -11 + 2e-5


@pytest.mark.parametrize("kind,inner_len", KINDS)
def test_hyena_bf16_io(kind, inner_len):
    """BF16 projection in, BF16 output: compare with the oracle on the same
    BF16-rounded projection; the only extra error is the output rounding."""
    case = hyena_case(77 + kind, kind, 777, 128, inner_len=inner_len or 7)
    proj = bf16_to_f32(bf16_bits(case["projection"]))
    expected = hyena_oracle(kind, case, projection=proj)
    actual = hyena_gpu(kind, case, dtype=N.DTYPE_BF16)
    assert np.abs(actual - expected).max() <= 2.0 ** -8 * np.abs(expected).max()


@pytest.mark.parametrize("kind,inner_len", KINDS)
@pytest.mark.parametrize("groups", [16, 8])
def test_hyena_bf16_split_io(kind, inner_len, groups):
    """The model's FP8-projection path: BF16 projection in, split planes out."""
    case = hyena_case(55 + kind + groups, kind, 1029, 128, groups=groups,
                      inner_len=inner_len or 7)
    proj = bf16_to_f32(bf16_bits(case["projection"]))
    expected = hyena_oracle(kind, case, projection=proj)
    actual = hyena_gpu(kind, case, dtype=N.DTYPE_BF16_SPLIT, projection=proj)
    assert rel_err(actual, expected) < 2e-5
    actual = hyena_gpu(kind, case, dtype=N.DTYPE_BF16_SPLIT, projection=proj,
                       planar_layout=True)
    assert rel_err(actual, expected) < 2e-5


@pytest.mark.parametrize("kind,inner_len", KINDS)
@pytest.mark.parametrize("split", [1, 5, 130, 299])
@pytest.mark.parametrize("groups,layout", [(16, False), (4, False), (4, True)])
def test_hyena_continuation_equals_one_pass(kind, inner_len, split, groups, layout):
    """Two calls sharing the FIR histories / modal state equal one call
    (groups=4 gives 16-channel filter groups: the MFMA FIR; layout=True feeds
    the planar projection, whose short-FIR history is planar too)."""
    case = hyena_case(5 + kind, kind, 300, 64, groups=groups, inner_len=inner_len or 7)
    width = 64
    whole = hyena_gpu(kind, case)
    hist = inner_len - 1 if inner_len else 0
    caches = {"short": zeros((2, 3 * width)),
              "inner": zeros((max(hist, 1), width)) if hist else None,
              "modal": zeros((width, 16)) if kind == N.HYENA_HCL else None}
    first = hyena_gpu(kind, case, projection=case["projection"][:split], caches=caches,
                      planar_layout=layout)
    second = hyena_gpu(kind, case, projection=case["projection"][split:], caches=caches,
                       planar_layout=layout)
    joined = np.concatenate([first, second])
    assert rel_err(joined, whole) < 1e-5


@pytest.mark.parametrize("inner_len", [128, 33, 2])
@pytest.mark.parametrize("length,width,groups", [(1, 64, 4), (31, 128, 8), (1025, 64, 4),
                                                 (2100, 128, 8), (3000, 256, 16)])
@pytest.mark.parametrize("dtype", [N.DTYPE_F32, N.DTYPE_SPLIT, N.DTYPE_BF16_SPLIT])
def test_hcm_stream_mfma_matches_oracle(inner_len, length, width, groups, dtype):
    """BF16 taps (the artifact case) run the row-streaming MFMA FIR: segments
    of 1024 rows with a 128-row lead, 32-row steps, a register ring of the
    160-row window; lengths cross segment and step boundaries."""
    case = hyena_case(length + width + inner_len, N.HYENA_HCM, length, width, groups=groups,
                      inner_len=inner_len)
    proj = case["projection"]
    if dtype == N.DTYPE_BF16_SPLIT:
        proj = bf16_to_f32(bf16_bits(proj))
    expected = hyena_oracle(N.HYENA_HCM, case, projection=proj)
    actual = hyena_gpu(N.HYENA_HCM, case, dtype=dtype, projection=proj, bf16_taps=True)
    assert rel_err(actual, expected) < 2e-5


@pytest.mark.parametrize("split", [1, 31, 32, 300, 1024, 1500])
def test_hcm_stream_continuation(split):
    """Continuation through the caches with the streaming kernel: the first
    segment of each call fills its window from the inner and short histories."""
    width, length = 128, 2100
    case = hyena_case(split, N.HYENA_HCM, length, width, groups=8, inner_len=128)
    whole = hyena_gpu(N.HYENA_HCM, case, bf16_taps=True)
    caches = {"short": zeros((2, 3 * width)), "inner": zeros((127, width)), "modal": None}
    first = hyena_gpu(N.HYENA_HCM, case, projection=case["projection"][:split], caches=caches,
                      bf16_taps=True)
    second = hyena_gpu(N.HYENA_HCM, case, projection=case["projection"][split:],
                       caches=caches, bf16_taps=True)
    assert rel_err(np.concatenate([first, second]), whole) < 1e-5
    reference = hyena_gpu(N.HYENA_HCM, case)  # three-pass MFMA kernel
    assert rel_err(whole, reference) < 1e-6


# ----------------------------------------------------------- attention
@pytest.mark.parametrize("heads,head_dim,rows,prefix", [(2, 128, 300, 0), (2, 64, 200, 70),
                                                        (3, 32, 1, 500)])
def test_attention_uniform_scores(heads, head_dim, rows, prefix):
    """Q = 0: every score is 0, every probability exactly 1, so each output
    row is the plain mean of V over its keys: the P.V path (V^T split BF16
    planes, ~16 significant bits, F32 accumulation) to 2^-16 of max |v|.
    A product that lost V's lo plane would miss by ~2^-9."""
    r = rng(7 * heads + head_dim + rows)
    width = heads * head_dim
    total = prefix + rows
    proj = r.standard_normal((total, 3 * width)).astype(np.float32)
    qkv = proj.reshape(total, heads, 3, head_dim)
    qkv[:, :, 0] = 0.0
    v = qkv[:, :, 2].reshape(total, width).astype(np.float64)
    expected = (np.cumsum(v, axis=0) / np.arange(1, total + 1)[:, None])[prefix:]
    inv_freq = (1.0 / 10000 ** (np.arange(0, head_dim, 2) / head_dim)).astype(np.float32)
    capacity = (total + 63) // 64 * 64
    kc, vc = zeros((2, capacity, width), np.uint16), zeros((2, width, capacity), np.uint16)
    query, out = empty((2, total, width), np.uint16), empty((total, width))
    if prefix:
        N.call("evo_hip_attention", p(dev(proj[:prefix])), prefix, width, heads, 1,
               p(dev(inv_freq)), 8.0, 0, p(query), p(kc), p(vc), capacity, p(out), stream())
    N.call("evo_hip_attention", p(dev(proj[prefix:])), rows, width, heads, 1,
           p(dev(inv_freq)), 8.0, prefix, p(query), p(kc), p(vc), capacity, p(out), stream())
    error = np.abs(host(out)[:rows] - expected).max() / np.abs(v).max()
    assert error <= 2.0 ** -16


@pytest.mark.parametrize("rows,heads,head_dim,prefix", [
    (70, 4, 16, 0), (130, 2, 128, 0), (64, 3, 64, 33), (300, 2, 128, 129), (1, 4, 32, 0),
    (257, 1, 32, 0), (1000, 2, 128, 0)])
def test_attention_matches_oracle(oracle, rows, heads, head_dim, prefix):
    r = rng(rows + heads)
    width = heads * head_dim
    total = prefix + rows
    # projections of all `total` positions; the first `prefix` rows are
    # appended to the cache by a first call.
    proj = r.standard_normal((total, 3 * width)).astype(np.float32)
    inv_freq = (1.0 / 10000 ** (np.arange(0, head_dim, 2) / head_dim)).astype(np.float32)
    # oracle: column_split head-major layout [h][q,k,v][d]
    qkv = proj.reshape(total, heads, 3, head_dim)
    q = np.ascontiguousarray(qkv[:, :, 0]).reshape(total * heads * head_dim)
    k = np.ascontiguousarray(qkv[:, :, 1]).reshape(total * heads * head_dim)
    v = np.ascontiguousarray(qkv[:, :, 2]).reshape(total * heads * head_dim)
    O.check(oracle.oracle_apply_rope(O.ptr(q), O.ptr(k), total, heads, head_dim,
                                     O.ptr(inv_freq), 0, 8.0))
    expected = np.zeros_like(q)
    O.check(oracle.oracle_causal_attention(O.ptr(q), O.ptr(k), O.ptr(v), total, heads,
                                           head_dim, O.ptr(expected)))
    expected = expected.reshape(total, width)[prefix:]
    capacity = (total + 63) // 64 * 64  # whole 64-key tiles
    kc, vc = zeros((2, capacity, width), np.uint16), zeros((2, width, capacity), np.uint16)
    query, out = empty((2, total, width), np.uint16), empty((total, width))
    if prefix:
        N.call("evo_hip_attention", p(dev(proj[:prefix])), prefix, width, heads, 1,
               p(dev(inv_freq)), 8.0, 0, p(query), p(kc), p(vc), capacity, p(out), stream())
    N.call("evo_hip_attention", p(dev(proj[prefix:])), rows, width, heads, 1,
           p(dev(inv_freq)), 8.0, prefix, p(query), p(kc), p(vc), capacity, p(out), stream())
    assert rel_err(host(out)[:rows], expected) < 1e-5
    # value cache layout: V^T planes, positions permuted inside 16-blocks
    vt = bf16_to_f32(host(vc))
    v_rows = v.reshape(total, width)
    pos = np.arange(total)
    column = (pos & ~15) | (pos & 3) | ((pos & 4) << 1) | ((pos & 8) >> 1)
    stored = vt[0][:, column].T + vt[1][:, column].T
    assert np.abs(stored - v_rows).max() <= 2.0 ** -16 * np.abs(v_rows).max()


@pytest.mark.parametrize("heads,head_dim,prefix", [(2, 128, 0), (2, 128, 255), (2, 128, 256),
                                                  (2, 128, 1000), (4, 64, 3000), (3, 32, 77),
                                                  (2, 32, 84), (2, 128, 1003), (1, 64, 92)])
def test_single_query_attention_split_over_keys(oracle, heads, head_dim, prefix):
    """One query (the decode step) with a workspace: keys split in chunks of
    256 and the chunk partials combined; against the oracle and the same
    call without a workspace (MFMA flash kernel)."""
    r = rng(prefix + heads + head_dim)
    width = heads * head_dim
    total = prefix + 1
    proj = r.standard_normal((total, 3 * width)).astype(np.float32)
    inv_freq = (1.0 / 10000 ** (np.arange(0, head_dim, 2) / head_dim)).astype(np.float32)
    qkv = proj.reshape(total, heads, 3, head_dim)
    q = np.ascontiguousarray(qkv[:, :, 0]).reshape(total * heads * head_dim)
    k = np.ascontiguousarray(qkv[:, :, 1]).reshape(total * heads * head_dim)
    v = np.ascontiguousarray(qkv[:, :, 2]).reshape(total * heads * head_dim)
    O.check(oracle.oracle_apply_rope(O.ptr(q), O.ptr(k), total, heads, head_dim,
                                     O.ptr(inv_freq), 0, 8.0))
    expected = np.zeros_like(q)
    O.check(oracle.oracle_causal_attention(O.ptr(q), O.ptr(k), O.ptr(v), total, heads,
                                           head_dim, O.ptr(expected)))
    expected = expected.reshape(total, width)[prefix:]
    capacity = (total + 63) // 64 * 64
    results = []
    for workspace_floats in (heads * ((total + 255) // 256) * (head_dim + 2), 0):
        kc, vc = zeros((2, capacity, width), np.uint16), zeros((2, width, capacity), np.uint16)
        query, out = empty((2, total, width), np.uint16), empty((total, width))
        if prefix:
            N.call("evo_hip_attention", p(dev(proj[:prefix])), prefix, width, heads, 1,
                   p(dev(inv_freq)), 8.0, 0, p(query), p(kc), p(vc), capacity, p(out),
                   stream())
        workspace = empty((max(workspace_floats, 1),))
        N.call("evo_hip_attention_ws", p(dev(proj[prefix:])), 1, width, heads, 1,
               p(dev(inv_freq)), 8.0, prefix, p(query), p(kc), p(vc), capacity, p(out),
               p(workspace), workspace_floats * 4, stream())
        results.append(host(out)[:1].copy())
    assert rel_err(results[0], expected) < 1e-5
    assert rel_err(results[0], results[1]) < 1e-5


def test_attention_rejects_unaligned_capacity():
    width, heads = 64, 2
    proj = zeros((4, 3 * width))
    inv = dev(np.ones(16, np.float32))
    kc, vc = zeros((2, 70, width), np.uint16), zeros((2, width, 70), np.uint16)
    query, out = empty((2, 4, width), np.uint16), empty((4, width))
    with pytest.raises(N.OpError, match="multiple of 64"):
        N.call("evo_hip_attention", p(proj), 4, width, heads, 1, p(inv), 1.0, 0, p(query),
               p(kc), p(vc), 70, p(out), stream())
