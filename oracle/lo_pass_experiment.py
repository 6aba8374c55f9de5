"""Design experiment: how a GEMM whose lo pass runs on E4M3 (hi . W on BF16
plus E4M3(lo) . E4M3(W) with E8M0 scales per 32 K) would move the logits of
the benchmarked 7B configuration, per GEMM class, against the oracle's exact
F32 path. CPU only (the oracle's emulation mode, oracle_set_lo_emulation).

    python oracle/lo_pass_experiment.py [tokens] [threads] [masks]

Masks: bit 0 BF16 projections, 1 out-projection, 2 MLP l1/l2, 3 MLP l3 (the
E4M3-lo scheme); 16 attention keys and 32 values rounded to BF16 (two-pass
split attention products); 512 the attention probabilities rounded to FP16
before P.V (a two-pass FP16 P.V). A fourth argument "one-of-each" uses the 7B-width
model with one block of each mixer (HCS, HCM, HCL, attention) instead of the
32-block 7B shape.
"""
import ctypes
import os
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "evo.cpp_amd"))

import numpy as np  # noqa: E402

import oracle_lib as O  # noqa: E402
from evo_hip import artifact as A  # noqa: E402


def main():
    n = int(sys.argv[1]) if len(sys.argv) > 1 else 128
    threads = int(sys.argv[2]) if len(sys.argv) > 2 else 8
    masks = [int(x) for x in (sys.argv[3] if len(sys.argv) > 3 else "2,4,8,15").split(",")]
    if len(sys.argv) > 4 and sys.argv[4] == "one-of-each":
        shape, seed = A.tiny_shape(width=4096, layers=4, heads=32, inner=11264, groups=256,
                                   attn=(3,), rope_scale=128.0,
                                   model_id="random-init-evo2-7b-width-4-blocks"), 4
        path = "/tmp/evo_lo_pass/one_of_each_seed4_survey.safetensors"
    else:
        shape, seed = A.evo2_7b_shape(), 7
        path = "/tmp/evo_lo_pass/evo2_7b_seed7_survey.safetensors"
    if not os.path.exists(path):
        os.makedirs(os.path.dirname(path), exist_ok=True)
        A.random_artifact(shape, seed=seed, init="survey").write(path)
    tokens = A.acgt_tokens(n, seed=1024)
    model = O.OracleModel(path).convert_fp8(8.0)
    lib = O.lib()
    lib.oracle_set_lo_emulation.argtypes = [ctypes.c_uint]
    lib.oracle_set_lo_emulation(0)
    exact = model.prefill(tokens, chunk=n, threads=threads)
    for mask in masks:
        lib.oracle_set_lo_emulation(mask)
        start = time.time()
        out = model.prefill(tokens, chunk=n, threads=threads)
        error = float(np.abs(out.astype(np.float64) - exact).max() / np.abs(exact).max())
        top1 = float(np.mean(out.argmax(1) == exact.argmax(1)))
        print(f"mask {mask}: logits max err {error:.3g} of the scale, top-1 {top1:.4f} "
              f"({time.time() - start:.0f} s)", flush=True)
    lib.oracle_set_lo_emulation(0)


if __name__ == "__main__":
    main()
