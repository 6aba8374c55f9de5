"""Writes tests/golden/tiny_reference_logits.npz from evo.cpp's own CPU
library (oracle/_ref/libevo_ref.so, compiled from the reference sources by
oracle/Makefile) on a seeded random-init artifact.

The fixture holds data only: artifact seed and shape (the artifact is
regenerated bit-identically by evo_hip.artifact), the ACGT token ids and the
reference logits.

    make -C oracle ref && python tests/golden/make_golden.py
"""
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "evo.cpp_amd"))
from evo_hip import artifact as A  # noqa: E402
from evo_hip import capi  # noqa: E402

SHAPE = dict(width=64, layers=8, heads=4, inner=96, groups=16)
SEED, LENGTH = 2024, 96


def main():
    ref = capi.EvoLibrary(os.path.join(ROOT, "oracle", "_ref", "libevo_ref.so"))
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "tiny.safetensors")
        A.random_artifact(A.tiny_shape(**SHAPE, attn=(3,)), seed=SEED).write(path)
        tokens = A.acgt_tokens(LENGTH, seed=SEED)
        model = ref.load(path, capi.BACKEND_CPU)
        logits = model.context(4096).prefill(tokens.astype(np.uint8).tobytes())
    np.savez_compressed(os.path.join(ROOT, "tests", "golden", "tiny_reference_logits.npz"),
                        seed=SEED, tokens=tokens, logits=logits, **SHAPE)


if __name__ == "__main__":
    main()
