"""The evo-hip front end without a GPU.

evo-hip opens any library that exports the evo C ABI. Driving evo.cpp's own
CPU library (oracle/_ref/libevo_ref.so) with it and comparing against the
reference's own `evo` command (oracle/_ref/evo) on the same artifact and
inputs checks everything the front end adds -- input parsing (FASTA, FASTQ,
raw, gzip, stdin), chunk bookkeeping, per-token log-likelihoods, the JSONL
records, generation's prefill/decode/sample loop, error codes -- byte for
byte, since both sides then compute the logits with the same code.
Log-likelihoods are also checked against numpy's log-softmax of the dumped
logits, which fixes them independently of either program.
"""
import os

import numpy as np
import pytest

import cli_util as C

needs_ref = pytest.mark.skipif(
    not (os.path.exists(C.REF_CLI) and os.path.exists(C.REF_LIB)),
    reason="reference CPU build (make -C oracle ref) is absent")
needs_cli = pytest.mark.skipif(not os.path.exists(C.CLI),
                               reason="evo-hip is not built (make -C evo.cpp_amd)")


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    directory = tmp_path_factory.mktemp("cli")
    paths = C.write_inputs(str(directory))
    paths["model"] = C.byte_artifact(str(directory / "tiny.safetensors"))
    return paths


def ours(*args, **kw):
    return C.run(C.CLI, *args, library=C.REF_LIB, **kw)


def reference(*args, **kw):
    return C.run(C.REF_CLI, *args, **kw)


@needs_cli
@needs_ref
@pytest.mark.parametrize("kind", ["fasta", "fastq", "raw", "gzip"])
def test_score_matches_reference_cli_bytes(files, kind):
    mine = ours("score", "-m", files["model"], "--input", files[kind])
    theirs = reference("score", "-m", files["model"], "--input", files[kind])
    assert mine.returncode == 0, mine.stderr
    assert theirs.returncode == 0, theirs.stderr
    assert mine.stdout == theirs.stdout
    records = C.jsonl(mine.stdout)
    assert len(records) == (1 if kind == "raw" else 2)
    for record in records:
        assert record["scored_tokens"] == record["tokens"] - 1
        assert len(record["token_log_likelihoods"]) == record["scored_tokens"]


@needs_cli
@needs_ref
def test_score_from_stdin(files):
    data = open(files["fasta"], "rb").read()
    mine = ours("score", "-m", files["model"], "--input", "-", stdin=data)
    theirs = reference("score", "-m", files["model"], "--input", files["fasta"])
    assert mine.returncode == 0, mine.stderr
    assert mine.stdout == theirs.stdout


@needs_cli
@needs_ref
def test_score_chunked_context(files, tmp_path):
    """A record longer than one chunk: the library streams several chunks;
    every token after the first is scored exactly once."""
    path = tmp_path / "long.txt"
    rng = np.random.default_rng(3)
    path.write_text("".join(rng.choice(list("ACGT"), 700)))
    args = ("score", "-m", files["model"], "--input", str(path), "--ctx", "1024")
    mine, theirs = ours(*args), reference(*args)
    assert mine.returncode == 0, mine.stderr
    assert mine.stdout == theirs.stdout
    assert C.jsonl(mine.stdout)[0]["scored_tokens"] == 699


@needs_cli
@needs_ref
def test_score_log_likelihoods_are_log_softmax_of_dumped_logits(files, tmp_path):
    out = tmp_path / "logits.npy"
    mine = ours("score", "-m", files["model"], "--input", files["raw"],
                "--dump-logits", str(out))
    assert mine.returncode == 0, mine.stderr
    logits = np.load(out)
    text = open(files["raw"], "rb").read()
    assert logits.shape == (len(text), 512) and logits.dtype == np.float32
    record = C.jsonl(mine.stdout)[0]
    # The difference to the row maximum is taken in F32, the rest in F64.
    shifted = (logits - logits.max(1, keepdims=True)).astype(np.float64)
    log_softmax = shifted - np.log(np.exp(shifted).sum(1, keepdims=True))
    expected = log_softmax[np.arange(len(text) - 1), np.frombuffer(text, np.uint8)[1:]]
    np.testing.assert_allclose(record["token_log_likelihoods"], expected, rtol=0,
                               atol=1e-9)
    assert record["log_likelihood"] == pytest.approx(expected.sum(), abs=1e-9)
    assert record["perplexity"] == pytest.approx(np.exp(-expected.mean()), rel=1e-12)
    theirs_path = tmp_path / "ref.npy"
    theirs = reference("score", "-m", files["model"], "--input", files["raw"],
                       "--dump-logits", str(theirs_path))
    assert theirs.returncode == 0, theirs.stderr
    assert np.array_equal(np.load(theirs_path), logits)


@needs_cli
@needs_ref
def test_bench_report_schema_matches_reference(files):
    args = ("bench", "-m", files["model"], "--input", files["fasta"], "--warmup", "0",
            "--repetitions", "3")
    mine, theirs = ours(*args), reference(*args)
    assert mine.returncode == 0, mine.stderr
    assert theirs.returncode == 0, theirs.stderr
    for a, b in zip(C.jsonl(mine.stdout), C.jsonl(theirs.stdout), strict=True):
        assert list(a) == list(b)
        timing = ("samples_seconds", "median_seconds", "median_tokens_per_second")
        assert {k: v for k, v in a.items() if k not in timing} == \
               {k: v for k, v in b.items() if k not in timing}
        assert len(a["samples_seconds"]) == 3 and min(a["samples_seconds"]) > 0
        assert a["median_seconds"] == sorted(a["samples_seconds"])[1]
        assert a["median_tokens_per_second"] == pytest.approx(
            a["tokens"] / a["median_seconds"], rel=1e-15)
        assert a["input"]["identity"].startswith("fnv1a64:")


@needs_cli
@needs_ref
@pytest.mark.parametrize("options", [
    (),
    ("--top-k", "4", "--temp", "0.8", "--seed", "9"),
    ("--top-k", "0", "--top-p", "0.9", "--seed", "123"),
    ("--force-prompt-threshold", "4", "--output-format", "raw"),
])
def test_run_matches_reference_cli(files, options):
    """Prefill, prompt-tail decode, sampling and byte output of generation."""
    args = ("run", "-m", files["model"], "-p", "ACGTACGTAACCGGTT", "-n", "24", *options)
    mine, theirs = ours(*args), reference(*args)
    assert theirs.returncode == 0, theirs.stderr
    assert mine.returncode == 0, mine.stderr
    assert mine.stdout == theirs.stdout and len(mine.stdout) == 24


@needs_cli
@needs_ref
def test_run_dump_logits_matches_reference(files, tmp_path):
    a, b = tmp_path / "a.npy", tmp_path / "b.npy"
    args = ("run", "-m", files["model"], "-p", "GATTACA", "-n", "5")
    assert ours(*args, "--dump-logits", str(a)).returncode == 0
    assert reference(*args, "--dump-logits", str(b)).returncode == 0
    assert np.array_equal(np.load(a), np.load(b)) and np.load(a).shape == (5, 512)


BAD_INPUTS = {
    "space.fa": b">a\nAC GT\n",
    "noheader.fa": b">\nACGT\n",
    "empty_record.fa": b">a\n>b\nACGT\n",
    "before.fa": b">a\nACGT\n",  # valid control
    "trunc.fq": b"@r\nACGT\n+\n",
    "qual.fq": b"@r\nACGT\n+\nII\n",
    "plus.fq": b"@r\nACGT\n+x\nIIII\n",
    "qbyte.fq": b"@r\nACGT\n+\nII I\n",
    "one.txt": b"A",
    "empty.txt": b"",
}


@needs_cli
@needs_ref
@pytest.mark.parametrize("name", sorted(BAD_INPUTS))
def test_input_errors_match_reference(files, tmp_path, name):
    path = tmp_path / name
    path.write_bytes(BAD_INPUTS[name])
    mine = ours("score", "-m", files["model"], "--input", str(path))
    theirs = reference("score", "-m", files["model"], "--input", str(path))
    assert mine.returncode == theirs.returncode
    assert mine.stdout == theirs.stdout
    if theirs.returncode != 0:
        # Same error class and message after the program-name prefix.
        assert mine.stderr.decode().strip().split(": ", 1)[1] == \
               theirs.stderr.decode().splitlines()[-1].split(": ", 1)[1]


@needs_cli
@needs_ref
def test_record_limit_and_option_errors(files):
    assert ours("score", "-m", files["model"], "--input", files["raw"],
                "--ctx", "50").returncode == 2
    assert reference("score", "-m", files["model"], "--input", files["raw"],
                     "--ctx", "50").returncode == 2
    for bad in (("--ctx", "0"), ("--warmup", "1001"), ("--repetitions", "0")):
        result = C.run(C.CLI, "bench", "-m", files["model"], "--input", files["raw"], *bad,
                       library=C.REF_LIB)
        assert result.returncode == 2, bad
    result = C.run(C.CLI, "run", "-m", files["model"], "-p", "ACGT", "-n", "10", "--ctx",
                   "8", library=C.REF_LIB)
    assert result.returncode == 2 and b"exceed --ctx" in result.stderr
    result = C.run(C.CLI, "score", "-m", files["model"], "--input", files["fasta"],
                   "--dump-logits", "/tmp/x.npy", library=C.REF_LIB)
    assert result.returncode == 2 and b"exactly one input record" in result.stderr
    assert C.run(C.CLI, "score", "-m", files["model"], "--input", "/nonexistent",
                 library=C.REF_LIB).returncode == 3


@needs_cli
def test_cli_reports_library_and_backend_errors(files):
    result = C.run(C.CLI, "score", "-m", files["model"], "--input", files["raw"],
                   library="/nonexistent/libevo.so")
    assert result.returncode == 3 and b"cannot load evo library" in result.stderr
    # libevo_hip.so is HIP-only: asking it for the CPU backend is unsupported.
    result = C.run(C.CLI, "score", "-m", files["model"], "--input", files["raw"],
                   library=C.HIP_LIB, backend="cpu")
    assert result.returncode == 5, result.stderr
    assert C.run(C.CLI, "--help", backend=None).returncode == 0
