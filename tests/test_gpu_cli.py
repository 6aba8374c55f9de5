"""evo-hip on the GPU (libevo_hip.so, backend HIP) against the reference's
own `evo` command (oracle/_ref/evo, CPU backend) on the same artifact and
inputs.

Tolerance (the logits contract of the "hip-f32" profile): dumped logits
satisfy max|hip - ref| <= 1e-3 * max|ref| with identical top-1 on every
row; a per-token log-likelihood is a difference of two logit-dependent terms,
so it agrees within 2e-3 * max|ref logits|. Greedy generation, which only
depends on top-1, is byte-identical.
"""
import os

import numpy as np
import pytest

import cli_util as C

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not os.path.exists(C.REF_CLI),
                                 reason="reference CPU build (make -C oracle ref) is absent")]
TOL = 1e-3


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    directory = tmp_path_factory.mktemp("gpucli")
    paths = C.write_inputs(str(directory))
    paths["model"] = C.byte_artifact(str(directory / "tiny.safetensors"))
    return paths


def hip(*args, **kw):
    return C.run(C.CLI, *args, backend="hip", **kw)


def reference(*args, **kw):
    return C.run(C.REF_CLI, *args, backend="cpu", **kw)


@pytest.mark.parametrize("kind", ["fasta", "fastq", "raw"])
def test_score_matches_reference(files, kind):
    mine = hip("score", "-m", files["model"], "--input", files[kind])
    theirs = reference("score", "-m", files["model"], "--input", files[kind])
    assert mine.returncode == 0, mine.stderr
    assert theirs.returncode == 0, theirs.stderr
    for a, b in zip(C.jsonl(mine.stdout), C.jsonl(theirs.stdout), strict=True):
        assert a["backend"] == "hip" and a["profile"] == "hip-f32"
        for key in ("name", "input_format", "model_id", "tokens", "scored_tokens"):
            assert a[key] == b[key]
        diff = np.abs(np.subtract(a["token_log_likelihoods"], b["token_log_likelihoods"]))
        print(f"{kind} {a['name']}: max |d log p| {diff.max():.3g}")
        assert diff.max() <= 2 * TOL * 60.0
        assert a["log_likelihood"] == pytest.approx(b["log_likelihood"],
                                                    abs=2 * TOL * 60.0 * a["scored_tokens"])


def test_score_dumped_logits_within_contract(files, tmp_path):
    a, b = tmp_path / "hip.npy", tmp_path / "ref.npy"
    mine = hip("score", "-m", files["model"], "--input", files["raw"], "--dump-logits", str(a))
    theirs = reference("score", "-m", files["model"], "--input", files["raw"],
                       "--dump-logits", str(b))
    assert mine.returncode == 0, mine.stderr
    assert theirs.returncode == 0, theirs.stderr
    actual, expected = np.load(a), np.load(b)
    assert actual.shape == expected.shape
    scale = float(np.abs(expected).max())
    assert scale <= 60.0  # the log-likelihood bound above assumes this
    assert float(np.abs(actual - expected).max()) <= TOL * scale
    assert np.array_equal(actual.argmax(1), expected.argmax(1))
    record, = C.jsonl(mine.stdout)
    text = np.frombuffer(open(files["raw"], "rb").read(), np.uint8)
    shifted = (actual - actual.max(1, keepdims=True)).astype(np.float64)
    log_softmax = shifted - np.log(np.exp(shifted).sum(1, keepdims=True))
    np.testing.assert_allclose(record["token_log_likelihoods"],
                               log_softmax[np.arange(len(text) - 1), text[1:]], atol=1e-9,
                               rtol=0)


@pytest.mark.parametrize("options", [(), ("--force-prompt-threshold", "5")])
def test_greedy_generation_matches_reference(files, options):
    args = ("run", "-m", files["model"], "-p", "ACGTACGTAACCGGTT", "-n", "24", *options)
    mine, theirs = hip(*args), reference(*args)
    assert theirs.returncode == 0, theirs.stderr
    assert mine.returncode == 0, mine.stderr
    assert mine.stdout == theirs.stdout and len(mine.stdout) == 24


def test_bench_report(files):
    mine = hip("bench", "-m", files["model"], "--input", files["fasta"], "--warmup", "1",
               "--repetitions", "3")
    theirs = reference("bench", "-m", files["model"], "--input", files["fasta"],
                       "--warmup", "0", "--repetitions", "3")
    assert mine.returncode == 0, mine.stderr
    for a, b in zip(C.jsonl(mine.stdout), C.jsonl(theirs.stdout), strict=True):
        assert list(a) == list(b)
        assert a["backend"] == "hip" and a["execution_profile"] == "hip-f32"
        assert a["input"] == b["input"] and a["tokens"] == b["tokens"]
        assert a["timing_scope"] == "prefill_with_host_logits"
        assert len(a["samples_seconds"]) == 3 and a["median_tokens_per_second"] > 0


def test_bf16_profile_scores(files):
    mine = hip("score", "-m", files["model"], "--input", files["raw"], "--profile", "hip-bf16")
    theirs = reference("score", "-m", files["model"], "--input", files["raw"])
    assert mine.returncode == 0, mine.stderr
    a, = C.jsonl(mine.stdout)
    b, = C.jsonl(theirs.stdout)
    assert a["profile"] == "hip-bf16"
    diff = np.abs(np.subtract(a["token_log_likelihoods"], b["token_log_likelihoods"]))
    assert diff.max() <= 2 * 1e-2 * 60.0


@pytest.mark.parametrize("profile", ["hip-f32+f16-out", "hip-f32+f16-proj", "hip-f32+fp8-k32"])
def test_composed_profiles_score(files, profile):
    """--profile takes a base profile and '+'-options as the library names
    them; the FP16 one-pass and FP8 options stay within the hip-f32 logits
    contract against the reference on this tiny BF16 model (the FP8 option
    only names the promotion mode: this artifact has no FP8 projections)."""
    mine = hip("score", "-m", files["model"], "--input", files["raw"], "--profile", profile)
    theirs = reference("score", "-m", files["model"], "--input", files["raw"])
    assert mine.returncode == 0, mine.stderr
    a, = C.jsonl(mine.stdout)
    b, = C.jsonl(theirs.stdout)
    assert a["profile"] == profile
    diff = np.abs(np.subtract(a["token_log_likelihoods"], b["token_log_likelihoods"]))
    assert diff.max() <= 2 * TOL * 60.0


def test_unknown_composed_profile_is_rejected(files):
    for profile in ("hip-f32+", "hip-bf16+f16-out", "hip-f32+fp8-exact+fp8-k32", "f16-out"):
        run = hip("score", "-m", files["model"], "--input", files["raw"], "--profile", profile)
        assert run.returncode != 0 and b"unknown --profile" in run.stderr
