"""Prefill benchmark of the MI355X StripedHyena2 library (the 7B-shaped prefill).

Workload: Evo-2-7B-shaped model (32 blocks, width 4096, 32 heads, FFN 11264,
byte vocab 512; hyena short/medium-128/long striping with attention at blocks
3, 10, 17, 24, 31), seeded random-init weights (BF16 linears, Hyena input
projections converted to software E4M3 at load), batch-1 prefill of 8192
uniform ACGT tokens. One "step" = one full prefill with tokens and logits
resident in HBM (evo_hip_context_prefill_resident).

Also measured live (HIP events on the launching stream, algorithmic work
only): the dominant kernel (MLP l1/l2 GEMM, M=8192 N=2x11264 K=4096), the
three Hyena operators (config 2, BF16 projection in, L=8192 W=4096; the
headline `hyena_roofline` is the slowest of them) and the FP8 projection
GEMM (config 3, M=1024 K=4096 N=12288); and, on the host
cores, evo.cpp's own CPU library (oracle/_ref) on a bounded 16-token sample
of the same artifact.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--tokens L]
"""
import argparse
import ctypes
import json
import re
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "evo.cpp_amd"))

from evo_hip import artifact as A  # noqa: E402
from evo_hip import capi, native  # noqa: E402

METRIC = "prefill tok/s at 1 GPU, 7B-shape @1k/8k tok; % HBM BW and % FP8 MFMA peak"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F16_PROJ_FLAG = 1 << 11  # EVO_CONTEXT_FLAG_HIP_F16_PROJ
F16_OUT_FLAG = 1 << 12   # EVO_CONTEXT_FLAG_HIP_F16_OUT
FP8_PEAK_TFLOPS = 5000.0
LIB = os.path.join(ROOT, "evo.cpp_amd", "lib", "libevo_hip.so")
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libevo_ref.so")


def log(message):
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def artifact_path(directory):
    shape = A.evo2_7b_shape()
    art = A.random_artifact(shape, seed=0, init="survey")
    path = os.path.join(directory, "evo2_7b_shape_seed0_survey.safetensors")
    expected = sum(s.nbytes for s in art.specs)
    if not (os.path.exists(path) and os.path.getsize(path) > expected):
        os.makedirs(directory, exist_ok=True)
        log(f"writing 7B-shaped artifact ({expected / 1e9:.1f} GB) to {path}")
        start = time.time()
        art.write(path + ".tmp")
        os.replace(path + ".tmp", path)
        log(f"artifact written in {time.time() - start:.0f} s")
    return path, shape


def event_time(fn, repeats):
    """Average launch duration of fn() on torch's current stream (ms). A
    bounded spin kernel queued first holds the stream while the host
    enqueues the launches, so the timed launches run back to back and the
    host's per-call cost (ctypes, argument checks) is not counted."""
    import torch
    fn()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    torch.cuda._sleep(50_000_000)  # ~20 ms of GPU clock cycles
    start.record()
    for _ in range(repeats):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / repeats


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "roofline_kernels_hbm_traffic.md")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (copy-calibrated), or None."""
    try:
        with open(TRAFFIC_PROFILE) as handle:
            for line in handle:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 5 and cells[0] == f"`{kernel}`":
                    return int(float(cells[4]))
    except OSError:
        return None
    return None


def kernel_rooflines(split):
    import torch
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device="cuda").manual_seed(0)
    out = {}
    # Calibration launch for the HBM byte counters: a plain 1 GiB device copy
    # (torch's copy kernel) reads and writes exactly 2^30 bytes.
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    # dominant kernel: gated MLP l1/l2 GEMM of one block at L=8192
    m, n, k = 8192, 2 * 11264, 4096
    x = torch.randn(m, k, device="cuda", generator=g)
    planes = torch.empty(2, m, k, dtype=torch.int16, device="cuda")
    native.call("evo_hip_split_f32", x.data_ptr(), m * k, planes[0].data_ptr(),
                planes[1].data_ptr(), stream)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    y = torch.empty(m, n, device="cuda")
    lo = planes[1].data_ptr() if split else None
    ms = event_time(lambda: native.call("evo_hip_linear", planes[0].data_ptr(), lo,
                                        w.data_ptr(), None, None, m, n, k, y.data_ptr(),
                                        stream), 5)
    flops = 2.0 * m * n * k
    out["gemm"] = dict(kernel="gemm_kernel<%s>" % ("true" if split else "false"),
                       ms=ms, flops=flops, tflops=flops / ms / 1e9)
    del x, w, y, planes
    # Hyena operators at the model's shape: BF16 projection [8192, 12288] in
    # (the FP8 projection's output), out as one BF16 plane (config 2's
    # format), one FP16 plane (the benchmarked context's) and split BF16
    # planes [2, 8192, 4096] (contexts without +f16-out), 7B filter groups
    # (256) and tap counts (HCS 7, HCM 128, HCL 16 states).
    length, width, state, groups = 8192, 4096, 16, 256
    proj = torch.randn(length, 3 * width, device="cuda", generator=g).to(torch.bfloat16)
    short = (torch.randn(3 * width, 3, device="cuda", generator=g) * 0.3).to(torch.bfloat16)
    poles = torch.rand(width, state, device="cuda", generator=g) * 0.49 + 0.5
    residues = torch.randn(width, state, device="cuda", generator=g) * 0.02
    direct = torch.randn(width, device="cuda", generator=g) * 0.02
    planes_out = torch.empty(2, length, width, dtype=torch.int16, device="cuda")
    hbm_bytes = length * 3 * width * 2 + length * width * 4
    bf16_bytes = length * 3 * width * 2 + length * width * 2
    out["hyena"] = []
    for kind, name, taps, profiled in (
            (1, "HCM FIR, 128 taps (hyena_fir_mfma_stream_kernel)", 128,
             "hyena_fir_mfma_stream_kernel<unsigned short, unsigned short*>"),
            (0, "HCS FIR, 7 taps (hyena_fir_stream_kernel)", 7,
             "hyena_fir_stream_kernel<unsigned short, unsigned short*, 3, 7, false>"),
            (2, "HCL, 16 modal states (hcl_mfma_kernel)", 0,
             "hcl_mfma_kernel<unsigned short, unsigned short*>")):
        filt = (torch.randn(groups, max(taps, 1), device="cuda", generator=g)
                / max(taps, 1) ** 0.5).to(torch.bfloat16).float()
        st = state if kind == 2 else 0
        ws_bytes = native.call("evo_hip_hyena_workspace_bytes", kind, length, width, st)
        ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device="cuda")
        times = {}
        for dtype in (native.DTYPE_BF16, native.DTYPE_BF16_SPLIT, native.DTYPE_BF16_F16):
            times[dtype] = event_time(lambda: native.call(
                "evo_hip_hyena_forward", kind, dtype | native.DTYPE_BF16_TAPS,
                proj.data_ptr(), length,
                width, short.data_ptr(), 3, filt.data_ptr(), groups, taps, direct.data_ptr(),
                poles.data_ptr(), residues.data_ptr(), st, None, None, None, ws.data_ptr(),
                ws_bytes, planes_out.data_ptr(), stream), 10)
        ms, ms_split = times[native.DTYPE_BF16], times[native.DTYPE_BF16_SPLIT]
        ms_f16 = times[native.DTYPE_BF16_F16]
        out["hyena"].append(dict(kernel=name, profiled=profiled, ms=ms, bytes=bf16_bytes, gbs=bf16_bytes / ms / 1e6,
                                 ms_split=ms_split, bytes_split=hbm_bytes,
                                 gbs_split=hbm_bytes / ms_split / 1e6,
                                 ms_f16=ms_f16, gbs_f16=bf16_bytes / ms_f16 / 1e6))
    del proj, planes_out
    # config 3: FP8 projection GEMM M=1024 K=4096 N=12288 (promotion every 32 K)
    m, k, n = 1024, 4096, 12288

    def e4m3_codes(shape, std):
        """Config 3's operands: N(0, std) values quantised per tensor to
        E4M3 with amax scaling (the codes; the scale folds into the output
        scale)."""
        x = torch.randn(shape, device="cuda", generator=g) * std
        x = x * (448.0 / x.abs().max())
        return x.to(torch.float8_e4m3fn).view(torch.uint8)

    a8 = e4m3_codes((m, k), 1.0)
    w8 = e4m3_codes((n, k), 0.02)
    # BF16 output, the projection's own output type (each value is
    # bf16(acc * output_scale)), as the model writes it.
    y8 = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    for mode, name in ((0, "fp8_k32"), (1, "fp8_k128")):
        ms = event_time(lambda: native.call("evo_hip_fp8_linear_bf16", a8.data_ptr(),
                                            w8.data_ptr(), y8.data_ptr(), m, n, k, 1e-3,
                                            mode, stream), 10)
        flops = 2.0 * m * n * k
        out[name] = dict(kernel=f"fp8_mfma_kernel<{32 if mode == 0 else 128}>", ms=ms,
                         flops=flops, tflops=flops / ms / 1e9)
    # The bit-exact mode (the reference's per-term QGMMA semantics on the
    # VALU): one launch, for the cost of exact reference semantics.
    ms = event_time(lambda: native.call("evo_hip_fp8_linear_bf16", a8.data_ptr(),
                                        w8.data_ptr(), y8.data_ptr(), m, n, k, 1e-3, 2,
                                        stream), 1)
    out["fp8_exact"] = dict(kernel="qgmma_exact_kernel", ms=ms, flops=2.0 * m * n * k,
                            tflops=2.0 * m * n * k / ms / 1e9)
    del a8, w8, y8
    # Attention block body at the benchmarked shape (8192 rows from position
    # 0, 32 heads of 128): causal 2 * L^2 * W flop (Q.K^T and P.V over the
    # lower triangle); the timed op includes the Q/K/V split and RoPE.
    length, width, heads = 8192, 4096, 32
    cap = length
    projected = torch.randn(length, 3 * width, device="cuda", generator=g)
    inv_freq = (1.0 / (10000.0 ** (torch.arange(0, 128, 2, device="cuda").float() / 128)))
    query = torch.empty(2 * length * width, dtype=torch.int16, device="cuda")
    keys = torch.zeros(2 * cap * width, dtype=torch.int16, device="cuda")
    values = torch.zeros(2 * cap * width, dtype=torch.int16, device="cuda")
    att_out = torch.empty(length, width, device="cuda")
    ms = event_time(lambda: native.call("evo_hip_attention", projected.data_ptr(), length,
                                        width, heads, 1, inv_freq.data_ptr(), 1.0, 0,
                                        query.data_ptr(), keys.data_ptr(), values.data_ptr(),
                                        cap, att_out.data_ptr(), stream), 5)
    flops = 2.0 * length * length * width
    out["attention"] = dict(kernel="qkv_rope_kernel + flash_attention_kernel", ms=ms,
                            flops=flops, tflops=flops / ms / 1e9)
    return out


def composed_reference_8k():
    """The composed 8192-token figure of evo.cpp's CPU path on this pool's
    host (one core), as recorded by `--reference-cpu composed8k` in
    profiles/reference_cpu_7b_prefill.md: (tok/s, seconds) or None."""
    path = os.path.join(ROOT, "profiles", "reference_cpu_7b_prefill.md")
    if not os.path.exists(path):
        return None
    text = open(path).read()
    rate = re.search(r"\*\*([0-9.]+) tok/s\*\* at 8192 tokens", text)
    seconds = re.search(r"= ([0-9]+) s,\s*so", text)
    if not rate or not seconds:
        return None
    return float(rate.group(1)), float(seconds.group(1))


def cpu_baseline(path, sample_tokens):
    """evo.cpp's CPU F32 prefill (single-threaded by construction): the
    headline-length (8192-token) figure composed from per-block prefills
    timed on this host, with a live bounded sample of the same artifact
    through its own C ABI beside it."""
    if os.path.exists(REF_LIB):
        library, kind, backend = capi.EvoLibrary(REF_LIB), "reference", capi.BACKEND_CPU
    else:
        return None
    tokens = A.acgt_tokens(sample_tokens, seed=1).astype(np.uint8).tobytes()
    model = library.load(path, backend)
    context = model.context(sample_tokens)
    start = time.time()
    context.prefill(tokens)
    seconds = time.time() - start
    sample_rate = sample_tokens / seconds
    live = (f"live sample: {sample_tokens}-token prefill of the same 7B-shaped artifact "
            f"(BF16 projections; reference cpu-f32 path) in {seconds:.1f} s = "
            f"{sample_rate:.3f} tok/s; host has {os.cpu_count()} cores")
    composed = composed_reference_8k()
    if composed is None:
        return {"value": sample_rate, "unit": "tok/s", "cores": 1, "kind": kind,
                "sample": live, "sample_tok_s": round(sample_rate, 4)}
    rate, total = composed
    return {"value": rate, "unit": "tok/s", "cores": 1, "kind": kind, "composed": True,
            "sample": f"composed 8192-token prefill of the 7B shape ({total:.0f} s on one "
                      "core: 9 HCS + 9 HCM + 9 HCL + 5 attention blocks from one-block "
                      "8192-token prefills, profiles/reference_cpu_7b_prefill.md); " + live,
            "sample_tok_s": round(sample_rate, 4)}


def reference_cpu(part, directory, only=None):
    """evo.cpp's own CPU library (single-threaded F32 path) at the headline
    workload, timed on this host: `full1k` runs a 1024-token prefill of the
    7B-shaped artifact in full; `composed8k` times 8192-token prefills of
    one-block 7B-width models (one per mixer type, plus a two-block HCS model
    to separate the per-call embedding / final norm / unembedding) and
    composes the 32-block time as 9 HCS + 9 HCM + 9 HCL + 5 attention blocks
    plus one shared part."""
    import threading
    library = capi.EvoLibrary(REF_LIB)
    out = {"host_cores": os.cpu_count(), "threads": 1}
    # Progress line every minute (a single CPU prefill runs for minutes).
    started, done = time.time(), threading.Event()

    def heartbeat():
        while not done.wait(60):
            log(f"reference CPU run: {time.time() - started:.0f} s")
    threading.Thread(target=heartbeat, daemon=True).start()

    def time_prefill(path, length):
        model = library.load(path, capi.BACKEND_CPU)
        # untimed warm-up: maps the weights in and loads the library's state
        warm = model.context(64)
        warm.prefill(A.acgt_tokens(64, seed=9).astype(np.uint8).tobytes())
        warm.close()
        ctx = model.context(length)
        tokens = A.acgt_tokens(length, seed=1).astype(np.uint8).tobytes()
        start = time.time()
        ctx.prefill(tokens)
        seconds = time.time() - start
        ctx.close()
        model.close()
        log(f"{os.path.basename(path)} {length} tokens: {seconds:.1f} s")
        return seconds

    if part == "full1k":
        path, _ = artifact_path(directory)
        seconds = time_prefill(path, 1024)
        out.update(workload="7B-shaped, 32 blocks, 1024 ACGT tokens", seconds=round(seconds, 1),
                   tok_s=round(1024 / seconds, 4))
        done.set()
        return out
    os.makedirs(directory, exist_ok=True)
    base = A.evo2_7b_shape()
    layouts = {"hcs": dict(hcs=[0], hcm=[], hcl=[], attn=[]),
               "hcm": dict(hcs=[], hcm=[0], hcl=[], attn=[]),
               "hcl": dict(hcs=[], hcm=[], hcl=[0], attn=[]),
               "attn": dict(hcs=[], hcm=[], hcl=[], attn=[0]),
               "hcs2": dict(hcs=[0, 1], hcm=[], hcl=[], attn=[])}
    times = {}
    for name, lists in layouts.items():
        if only and name not in only:
            continue
        shape = A.ModelShape(width=base.width, layers=len(sum(lists.values(), [])),
                             heads=base.heads, inner=base.inner, rope_scale=base.rope_scale,
                             hcs_groups=base.hcs_groups, hcm_groups=base.hcm_groups,
                             hcs_len=base.hcs_len, hcm_len=base.hcm_len,
                             max_seqlen=base.max_seqlen,
                             model_id=f"random-init-evo2-7b-width-{name}", **lists)
        path = os.path.join(directory, f"evo2_7b_width_{name}.safetensors")
        if not os.path.exists(path):
            A.random_artifact(shape, seed=0, init="survey").write(path)
        times[name] = time_prefill(path, 8192)
    if set(times) != set(layouts):
        out.update(workload="one- and two-block 7B-width models, 8192 ACGT tokens",
                   measured_seconds={k: round(v, 1) for k, v in times.items()})
        done.set()
        return out
    shared = times["hcs"] - (times["hcs2"] - times["hcs"])
    block = {k: times[k] - shared for k in ("hcs", "hcm", "hcl", "attn")}
    composed = 9 * block["hcs"] + 9 * block["hcm"] + 9 * block["hcl"] + 5 * block["attn"] + shared
    out.update(workload="7B-shaped, 32 blocks, 8192 ACGT tokens (composed)",
               measured_seconds={k: round(v, 1) for k, v in times.items()},
               block_seconds={k: round(v, 1) for k, v in block.items()},
               shared_seconds=round(shared, 1), seconds=round(composed, 1),
               tok_s=round(8192 / composed, 4))
    done.set()
    return out


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=10)
    parser.add_argument("--warmup", type=int, default=2)
    parser.add_argument("--tokens", type=int, default=8192)
    parser.add_argument("--profile", choices=["f32", "bf16"], default="f32")
    parser.add_argument("--f16-projections", action="store_true",
                        help="out- and attention projections on one FP16 pass (the "
                             "+f16-proj context flag) instead of split BF16")
    parser.add_argument("--split-out", action="store_true",
                        help="out-projections on split BF16 too (context without the "
                             "+f16-out flag: every product except the FP8 ones split BF16)")
    parser.add_argument("--artifact-dir", default="/tmp/evo_bench")
    parser.add_argument("--cpu-sample", type=int, default=16)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-kernels", action="store_true")
    parser.add_argument("--long-tokens", type=int, default=131072,
                        help="config 5: one chunked prefill of this many tokens (0 = skip)")
    parser.add_argument("--decode-steps", type=int, default=32)
    parser.add_argument("--only-kernels", action="store_true",
                        help="run only the roofline launches (for rocprofv3 counter passes)")
    parser.add_argument("--reference-cpu", choices=["full1k", "composed8k"],
                        help="time only evo.cpp's CPU library at the headline workload")
    parser.add_argument("--reference-models", default="",
                        help="composed8k: comma-separated subset of hcs,hcm,hcl,attn,hcs2 "
                             "(to split the runs over several jobs)")
    args = parser.parse_args()
    if args.reference_cpu:
        only = set(filter(None, args.reference_models.split(",")))
        print(json.dumps(reference_cpu(args.reference_cpu, args.artifact_dir, only)),
              flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build runs on one "
              "MI355X (one process per GPU would each run this prefill on its own "
              "share; no collective is implemented)", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.only_kernels:
        native.load()
        print(json.dumps(kernel_rooflines(args.profile == "f32")), flush=True)
        return
    path, shape = artifact_path(args.artifact_dir)
    hip = capi.EvoLibrary(LIB)
    native.load()
    log("loading model (FP8 Hyena projections at load)")
    model = hip.load(path, capi.BACKEND_HIP, flags=1 << 8)
    params = hip.lib.evo_context_default_params()
    params.context_size = max(args.tokens, 1024)
    # The benchmarked context: FP8 K128 Hyena projections, out-projections on
    # one FP16 pass (EVO_CONTEXT_FLAG_HIP_F16_OUT: logits within 1.9e-4 of the
    # oracle, top-1 100 %), every other product split BF16. --split-out drops
    # the flag; --f16-projections adds the attention projections.
    f16_out = args.profile == "f32" and not args.split_out
    params.flags = (0 if args.profile == "f32" else (1 << 8)) | \
        (F16_PROJ_FLAG if args.f16_projections else 0) | (F16_OUT_FLAG if f16_out else 0)
    handle = ctypes.c_void_p()
    hip.check(hip.lib.evo_context_create(model.handle, ctypes.byref(params),
                                         ctypes.byref(handle)))
    context = capi.Context(model, handle)
    lib = native.load()
    lib.evo_hip_context_prefill_resident.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                                      ctypes.c_size_t, ctypes.c_void_p]
    # HIP events around every MLP l1/l2 product (the dominant kernel) of
    # each prefill, read after the timed region: its launch time inside the
    # timed prefills, for the roofline.
    native.call("evo_hip_context_set_product_timing", handle, 1)

    def product_time():
        ms, launches = ctypes.c_float(), ctypes.c_size_t()
        native.call("evo_hip_context_product_time", handle, ctypes.addressof(ms),
                    ctypes.addressof(launches))
        return ms.value / max(launches.value, 1), launches.value

    samples = {}

    def resident_rate(length, steps, warmup, ctx_handle=None):
        tokens = torch.from_numpy(A.acgt_tokens(length, seed=2).astype(np.int32)).cuda()
        logits = torch.empty(length, shape.vocab, device="cuda")
        target = handle if ctx_handle is None else ctx_handle

        def step():
            status = lib.evo_hip_context_prefill_resident(target, tokens.data_ptr(), length,
                                                         logits.data_ptr())
            if status != 0:
                raise RuntimeError(lib.evo_last_error().decode())
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        # Each prefill synchronises the context stream at its end, so the
        # per-step clock reads are the samples of the timed region.
        marks = [time.perf_counter()]
        for _ in range(steps):
            step()
            marks.append(time.perf_counter())
        torch.cuda.synchronize()
        seconds = time.perf_counter() - marks[0]
        samples.setdefault(length, [round(1e3 * (b - a), 3)
                                    for a, b in zip(marks, marks[1:])])
        return length * steps / seconds, 1e3 * seconds / steps

    log(f"timing {args.steps} prefills of {args.tokens} tokens")
    value, ms_per_step = resident_rate(args.tokens, args.steps, args.warmup)
    # (the last timed prefill's launches; every prefill rewrites the events)
    product_ms, product_launches = product_time()
    rate_1k, ms_1k = resident_rate(1024, max(args.steps, 5), 2)
    # The same prefill with every product but the FP8 ones on split BF16
    # (the context without EVO_CONTEXT_FLAG_HIP_F16_OUT), for reference.
    split_out = None
    if f16_out:
        sparams = hip.lib.evo_context_default_params()
        sparams.context_size = params.context_size
        sparams.flags = params.flags & ~F16_OUT_FLAG
        shandle = ctypes.c_void_p()
        hip.check(hip.lib.evo_context_create(model.handle, ctypes.byref(sparams),
                                             ctypes.byref(shandle)))
        split_ctx = capi.Context(model, shandle)
        srate, sms = resident_rate(args.tokens, max(args.steps // 2, 3), 1, shandle)
        split_out = {"tok_s": round(srate, 1), "ms_per_step": round(sms, 3),
                     "profile": split_ctx.profile}
        split_ctx.close()
    # C-ABI rate with host logits (PCIe-inclusive; not the headline value):
    # a prefill needs a fresh context, so each run opens one (not timed);
    # one warm-up run, then the median of three.
    # The callback only receives the host logits (a consumer that copies them
    # into Python arrays would time numpy, not the library).
    seq = A.acgt_tokens(args.tokens, seed=2).astype(np.uint8).tobytes()
    noop = capi.LOGITS_CALLBACK(lambda logits, rows, columns, offset, user: 0)
    batch = ctypes.c_void_p()
    hip.check(hip.lib.evo_batch_create(1, ctypes.byref(batch)))
    hip.check(hip.lib.evo_batch_add_sequence(batch, seq, len(seq)))
    cabi_seconds = []
    for run in range(4):
        ctx2 = model.context(args.tokens, params.flags)
        start = time.perf_counter()
        hip.check(hip.lib.evo_context_prefill(ctx2.handle, batch, noop, None))
        if run > 0:
            cabi_seconds.append(time.perf_counter() - start)
        ctx2.close()
    hip.lib.evo_batch_free(batch)
    cabi_rate = args.tokens / sorted(cabi_seconds)[1]

    # Cached decode after a 1024-token prefill (C ABI, host logits per step).
    decode_rate = None
    if args.decode_steps > 0:
        log(f"timing {args.decode_steps} decode steps after a 1024-token prefill")
        ctx3 = model.context(1024 + args.decode_steps + 8, params.flags)
        token = int(ctx3.prefill(A.acgt_tokens(1024, seed=3).astype(np.uint8)
                                 .tobytes())[-1].argmax())
        for _ in range(4):
            token = int(ctx3.decode(token).argmax())
        start = time.perf_counter()
        for _ in range(args.decode_steps):
            token = int(ctx3.decode(token).argmax())
        decode_rate = args.decode_steps / (time.perf_counter() - start)
        ctx3.close()

    # Config 5: one long prefill, chunked through the 8192-row arena.
    long_result = None
    if args.long_tokens > 0:
        log(f"timing one chunked prefill of {args.long_tokens} tokens")
        lparams = hip.lib.evo_context_default_params()
        lparams.context_size = args.long_tokens
        lparams.flags = params.flags
        lhandle = ctypes.c_void_p()
        hip.check(hip.lib.evo_context_create(model.handle, ctypes.byref(lparams),
                                             ctypes.byref(lhandle)))
        lctx = capi.Context(model, lhandle)
        ltokens = torch.from_numpy(A.acgt_tokens(args.long_tokens, seed=5)
                                   .astype(np.int32)).cuda()
        llogits = torch.empty(args.long_tokens, shape.vocab, device="cuda")
        torch.cuda.synchronize()
        start = time.perf_counter()
        status = lib.evo_hip_context_prefill_resident(lhandle, ltokens.data_ptr(),
                                                     args.long_tokens, llogits.data_ptr())
        torch.cuda.synchronize()
        seconds = time.perf_counter() - start
        if status != 0:
            raise RuntimeError(lib.evo_last_error().decode())
        long_result = {"tokens": args.long_tokens, "seconds": round(seconds, 3),
                       "tok_s": round(args.long_tokens / seconds, 1),
                       "chunk_rows": 8192, "finite": bool(torch.isfinite(llogits).all())}
        lctx.close()
        del ltokens, llogits

    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": ("fp8-e4m3 projections + f32 (split-bf16 MFMA"
                  + ("; fp16 out/attention projections" if args.f16_projections
                     else "; fp16 out-projections" if f16_out else "") + ")")
                 if args.profile == "f32"
                 else "fp8-e4m3 projections + bf16 MFMA",
        "data": "synthetic (seeded random-init weights, uniform ACGT tokens)",
        "config": {"workload": f"evo2-7b-shape prefill L={args.tokens}, batch 1, "
                               "fp8 hyena projections (config 4)",
                   "tokens": args.tokens, "layers": shape.layers, "width": shape.width,
                   "heads": shape.heads, "ffn": shape.inner,
                   "profile": context.profile, "tok_s_1k": round(rate_1k, 1),
                   "ms_per_step_1k": round(ms_1k, 3),
                   "samples_ms": samples.get(args.tokens),
                   "median_ms": round(float(np.median(samples[args.tokens])), 3),
                   "samples_ms_1k": samples.get(1024),
                   "c_abi_host_logits_tok_s": round(cabi_rate, 1),
                   "decode_tok_s_after_1k": round(decode_rate, 1) if decode_rate else None,
                   "long_context_prefill": long_result,
                   "split_out_projections": split_out},
    }
    if not args.no_kernels:
        log("kernel rooflines")
        kernels = kernel_rooflines(args.profile == "f32")
        g = kernels["gemm"]
        # achieved: the l1/l2 launches inside the timed prefills (HIP events
        # on the context stream); standalone_*: the same product launched
        # back to back outside the model (random activations), for the
        # counter passes.
        if args.tokens == 8192 and product_launches:
            in_model_ms = product_ms
        else:
            in_model_ms = g["ms"]
        tflops = g["flops"] / in_model_ms / 1e9
        result["roofline"] = {"bound": "mfma", "kernel": g["kernel"],
                              "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS,
                              "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                              "traffic": measured_traffic(g["kernel"]),
                              "ms": round(in_model_ms, 4),
                              "launches": product_launches,
                              "standalone_ms": round(g["ms"], 4),
                              "standalone_achieved": round(g["tflops"], 1),
                              "per_launch": "2*8192*22528*4096 flop (MLP l1/l2 of one block)"}
        # Config 2 is timed in the operator's own format (BF16 [8192, 12288]
        # in, BF16 [8192, 4096] out: 268435456 B per launch) -- `frac` --,
        # with one FP16 plane out (the same bytes; the benchmarked context's
        # mixer output) -- `frac_f16_out` -- and with split BF16 planes out
        # (335544320 B, the hip-f32 context without +f16-out) --
        # `frac_split_planes`, each from its own launch time.
        hyena = []
        for h in kernels["hyena"]:
            extra = {}
            if "HCM" in h["kernel"]:
                # HCM's 128-tap convolution is 2*128*8192*4096 = 8.6 GFLOP
                # per launch, on MFMA: its fraction of the BF16 peak too.
                tflops = 2 * 128 * 8192 * 4096 / h["ms"] / 1e9
                extra = {"mfma_tflops": round(tflops, 1),
                         "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4)}
            hyena.append({"kernel": h["kernel"], "achieved": round(h["gbs"], 1), **extra,
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(h["gbs"] / HBM_PEAK_GBS, 4),
                          "traffic": measured_traffic(h["profiled"]), "ms": round(h["ms"], 4),
                          "ms_split_planes": round(h["ms_split"], 4),
                          "frac_split_planes": round(h["gbs_split"] / HBM_PEAK_GBS, 4),
                          "ms_f16_out": round(h["ms_f16"], 4),
                          "frac_f16_out": round(h["gbs_f16"] / HBM_PEAK_GBS, 4)})
        per_launch = ("268435456 B: read BF16 [8192, 12288] projection, write BF16 "
                      "(or FP16) [8192, 4096]; split planes out: 335544320 B")
        worst = min(hyena, key=lambda h: h["frac"])
        result["hyena_roofline"] = dict(worst, bound="hbm", per_launch=per_launch)
        result["hyena_kernels"] = hyena
        for name in ("fp8_k32", "fp8_k128"):
            f = kernels[name]
            result[name + "_roofline"] = {"bound": "mfma", "kernel": f["kernel"],
                                          "achieved": round(f["tflops"], 1),
                                          "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                                          "frac": round(f["tflops"] / FP8_PEAK_TFLOPS, 4),
                                          "ms": round(f["ms"], 4)}
        f = kernels["fp8_exact"]
        result["fp8_exact"] = {"kernel": f["kernel"], "ms": round(f["ms"], 3),
                               "achieved": round(f["tflops"], 2), "unit": "TFLOP/s",
                               "frac": round(f["tflops"] / FP8_PEAK_TFLOPS, 5),
                               "note": "bit-exact reference QGMMA semantics (integer "
                                       "emulation on the VALU), config 3"}
        f = kernels["attention"]
        result["attention_roofline"] = {
            "bound": "mfma", "kernel": f["kernel"], "achieved": round(f["tflops"], 1),
            "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(f["tflops"] / BF16_PEAK_TFLOPS, 4), "ms": round(f["ms"], 4),
            "per_launch": "2*8192^2*4096 flop (causal Q.K^T and P.V, 32 heads of 128; "
                          "three BF16 MFMA passes per product)"}
    context.close()
    model.close()
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        log(f"CPU baseline: reference library, {args.cpu_sample}-token sample")
        result["cpu_baseline"] = cpu_baseline(path, args.cpu_sample)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
