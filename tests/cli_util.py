"""Shared pieces of the evo-hip command-line tests: paths, the tiny artifact,
input files, and a runner for evo-hip and for the reference's own `evo`
command (oracle/_ref/evo, compiled from the reference sources by
oracle/Makefile)."""
import gzip
import json
import os
import subprocess

import numpy as np

from evo_hip import artifact as A

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "evo.cpp_amd", "bin", "evo-hip")
HIP_LIB = os.path.join(ROOT, "evo.cpp_amd", "lib", "libevo_hip.so")
REF_CLI = os.path.join(ROOT, "oracle", "_ref", "evo")
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libevo_ref.so")
TINY = dict(width=64, layers=8, heads=4, inner=96, groups=16, attn=(3,))


def byte_artifact(path, seed=7, shape=None):
    """Seeded tiny artifact whose embedding rows for token ids >= 256 are zero.
    The embedding is tied to the unembedding, so those ids get logit 0 while
    the 256 byte ids get random logits: greedy and top-k sampling then pick
    byte tokens, which generation can print."""
    art = A.random_artifact(shape or A.tiny_shape(**TINY), seed=seed)
    for spec in art.specs:
        if spec.name == "embedding_layer.weight":
            make = spec.make

            def masked(rng, make=make):
                table = np.array(make(rng))
                table[256:] = 0
                return table
            spec.make = masked
    art.write(path)
    return path


def write_inputs(directory, seed=1):
    """FASTA (two records, wrapped lines, a blank line, a header with a
    description), FASTQ (two records, one with a named + line), raw text, and
    a gzip copy of the FASTA. Returns {kind: path}."""
    rng = np.random.default_rng(seed)

    def dna(n):
        return "".join(rng.choice(list("ACGT"), n))
    paths = {}
    paths["fasta"] = os.path.join(directory, "in.fa")
    with open(paths["fasta"], "w") as f:
        f.write(">one some description\n" + dna(60) + "\n" + dna(40) + "\n\n>two\n"
                + dna(30) + "\n")
    paths["fastq"] = os.path.join(directory, "in.fq")
    with open(paths["fastq"], "w") as f:
        f.write("@r1\n" + dna(20) + "\n+\n" + "I" * 20 + "\n@r2\n" + dna(10) + "\n+r2\n"
                + "#" * 10 + "\n")
    paths["raw"] = os.path.join(directory, "in.txt")
    with open(paths["raw"], "w") as f:
        f.write(dna(77))
    paths["gzip"] = os.path.join(directory, "in.fa.gz")
    with open(paths["fasta"], "rb") as src, gzip.open(paths["gzip"], "wb") as dst:
        dst.write(src.read())
    return paths


def run(program, *args, library=None, backend="cpu", stdin=None, timeout=600):
    """Runs evo-hip (program CLI) or the reference `evo` (program REF_CLI)
    with the given subcommand and options. Returns CompletedProcess with
    bytes stdout/stderr."""
    argv = [program, *args]
    if backend is not None:
        argv += ["--backend", backend]
    if library is not None:
        argv += ["--library", library]
    return subprocess.run(argv, input=stdin, capture_output=True, timeout=timeout)


def jsonl(stdout):
    return [json.loads(line) for line in stdout.decode().splitlines() if line]
