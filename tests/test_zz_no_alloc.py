"""The allocation-free Hyena entry point (evo_hip_hyena_forward_static, the
library's fixed device scratch) against evo_hip_hyena_forward with a caller
workspace: same kernels, so the outputs and the updated caches must be
bit-identical. Each case runs two calls in a row on the shared scratch, the
second with a smaller input, so stale scratch contents from the first call
cannot leak into the second."""
import numpy as np
import pytest

from evo_hip import native as N
from evo_hip.artifact import bf16_bits, bf16_to_f32
from gpu_util import dev, empty, host, p, stream, torch, zeros
from test_gpu_ops import hyena_case

pytestmark = pytest.mark.gpu


def run(kind, case, length, static, dtype=N.DTYPE_F32, bf16_taps=False, caches=None):
    proj = case["projection"][:length]
    width, state = case["width"], case.get("state", 0)
    poles = np.exp(case["log_poles"]).astype(np.float32) if "log_poles" in case else None
    out = empty((length, width))
    args = [kind, dtype | (N.DTYPE_BF16_TAPS if bf16_taps else 0), p(dev(proj)), length, width,
            p(dev(case["short"])), 3, p(dev(case["inner"]) if "inner" in case else None),
            case.get("groups", 1), case.get("inner_len", 0),
            p(dev(case["direct"]) if "direct" in case else None),
            p(dev(poles) if poles is not None else None),
            p(dev(case["residues"]) if "residues" in case else None), state,
            p(caches.get("short")) if caches else None, p(caches.get("inner")) if caches else None,
            p(caches.get("modal")) if caches else None]
    if static:
        N.call("evo_hip_hyena_forward_static", *args, p(out), stream())
    else:
        ws_bytes = N.call("evo_hip_hyena_workspace_bytes", kind, length, width, state)
        ws = empty((max(ws_bytes, 256),), np.uint8)
        N.call("evo_hip_hyena_forward", *args, p(ws), ws_bytes, p(out), stream())
    return host(out)


def fresh_caches(kind, width, inner_len):
    return {"short": zeros((2, 3 * width)),
            "inner": zeros((inner_len - 1, width)) if kind != N.HYENA_HCL else None,
            "modal": zeros((width, 16)) if kind == N.HYENA_HCL else None}


@pytest.mark.parametrize("kind,inner_len,bf16_taps,width", [
    # W % 16 != 0: the three-pass HCL path, its chunk states in the scratch
    (N.HYENA_HCL, 0, False, 520),
    (N.HYENA_HCL, 0, False, 512),   # hcl_mfma_kernel: no scratch
    (N.HYENA_HCM, 128, False, 512),  # F32 taps: Toeplitz fragment table in the scratch
    (N.HYENA_HCS, 7, False, 512),    # streaming FIR: no scratch
    (N.HYENA_HCM, 128, True, 512)])  # streaming MFMA FIR: no scratch
def test_static_scratch_matches_workspace(kind, inner_len, bf16_taps, width):
    groups = 8 if width % 16 else 16
    case = hyena_case(70 + kind, kind, 3000, width, groups=groups, inner_len=inner_len or 7)
    for length in (3000, 777):  # second call smaller
        expected = run(kind, case, length, static=False, bf16_taps=bf16_taps)
        actual = run(kind, case, length, static=True, bf16_taps=bf16_taps)
        assert np.array_equal(actual.view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("kind,inner_len", [(N.HYENA_HCL, 0), (N.HYENA_HCM, 128)])
def test_static_scratch_with_caches(kind, inner_len):
    """Continuation through the caches: outputs and the caches left behind
    are identical to the workspace entry point's, over two calls."""
    width = 256
    inner = inner_len or 7
    case = hyena_case(90 + kind, kind, 2000, width, groups=16, inner_len=inner)
    results = []
    for static in (False, True):
        caches = fresh_caches(kind, width, inner)
        first = run(kind, case, 2000, static, caches=caches)
        second = run(kind, case, 1000, static, caches=caches)
        results.append((first, second, {k: host(v) for k, v in caches.items() if v is not None}))
    (a1, a2, ac), (b1, b2, bc) = results
    assert np.array_equal(a1, b1) and np.array_equal(a2, b2)
    for name in ac:
        assert np.array_equal(ac[name], bc[name])


def test_static_scratch_rejects_only_paths_that_need_more():
    """A three-pass HCL call (W % 16 != 0) whose chunk states exceed the
    scratch is refused before any launch."""
    limit = N.call("evo_hip_hyena_static_scratch_bytes")
    assert limit == 32 << 20
    width, length = 4104, 16384 + 128
    assert N.call("evo_hip_hyena_workspace_bytes", N.HYENA_HCL, length, width, 16) > limit
    proj = zeros((1, 1))
    with pytest.raises(N.OpError, match="static scratch"):
        N.call("evo_hip_hyena_forward_static", N.HYENA_HCL, N.DTYPE_F32, p(proj), length, width,
               p(proj), 3, None, 1, 0, p(proj), p(proj), p(proj), 16, None, None, None,
               p(proj), stream())


def test_static_scratch_accepts_hcl_mfma_at_131072_rows():
    """The model's HCL shape runs hcl_mfma_kernel, which needs no workspace:
    accepted at 131072 rows x 4096 channels (whose three-pass chunk states
    would exceed the scratch), bit-identical to the workspace entry point."""
    t = torch()
    width, length, state = 4096, 131072, 16
    assert N.call("evo_hip_hyena_workspace_bytes", N.HYENA_HCL, length, width, state) > \
        N.call("evo_hip_hyena_static_scratch_bytes")
    gen = t.Generator(device="cuda:0").manual_seed(131)
    projection = t.randn((length, 3 * width), generator=gen, device="cuda:0").to(t.bfloat16)
    r = np.random.default_rng(131)
    short = dev(bf16_bits(r.standard_normal((3 * width, 3)).astype(np.float32) * 0.5))
    direct = dev((r.standard_normal(width) * 0.5).astype(np.float32))
    poles = dev(r.uniform(0.5, 0.99, (width, state)).astype(np.float32))
    residues = dev((r.standard_normal((width, state)) * 0.1).astype(np.float32))
    outputs = []
    for static in (False, True):
        out = t.empty((length, width), dtype=t.bfloat16, device="cuda:0")
        args = [N.HYENA_HCL, N.DTYPE_BF16, projection.data_ptr(), length, width, p(short), 3,
                None, 1, 0, p(direct), p(poles), p(residues), state, None, None, None]
        if static:
            N.call("evo_hip_hyena_forward_static", *args, out.data_ptr(), stream())
        else:
            ws_bytes = N.call("evo_hip_hyena_workspace_bytes", N.HYENA_HCL, length, width, state)
            ws = t.empty((ws_bytes,), dtype=t.uint8, device="cuda:0")
            N.call("evo_hip_hyena_forward", *args, ws.data_ptr(), ws_bytes, out.data_ptr(),
                   stream())
        t.cuda.synchronize()
        outputs.append(out.view(t.int16).cpu().numpy())
    assert np.isfinite(bf16_to_f32(outputs[1][-8:])).all()
    assert np.array_equal(outputs[0], outputs[1])
