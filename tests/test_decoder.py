"""The llama2c decoder on the CPU: the test oracle pinned against the
contract's known answers and closed forms, planted oracle mistakes caught, and
the application's argument and dimension checks (exit 2 before any GPU work).

Reference: applications/loom_private/decoder (contract.json, oracle.cpp,
tests/run_tests.sh)."""
import json
import os
import subprocess

import numpy as np
import pytest

import decoder_oracle as dorc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DECODER = os.path.join(ROOT, "cuda-elastic_amd", "bin", "llama2c_decoder_hip")


# contract.json "reference_only_upstream_configurations": upstream decodes one
# sequence; smoke = width 128, 16 rows, prompt 0 -> tokens [1, 2, 3, 4];
# validation = width 1024, 64 rows, prompt 1 -> tokens [2, 3, 4, 5].
@pytest.mark.parametrize("width,vocab,prompt,expected", [(128, 16, 0, [1, 2, 3, 4]),
                                                         (1024, 64, 1, [2, 3, 4, 5])])
def test_upstream_expected_tokens(width, vocab, prompt, expected):
    assert dorc.analytic_tokens(1, vocab, 4, first_prompt=prompt)[0].tolist() == expected
    *_, tokens = dorc.dense_double(prompt, width, vocab, 4)
    assert tokens.tolist() == expected


@pytest.mark.parametrize("width,vocab,steps", [(96, 16, 5), (2, 2, 2), (1000, 1000, 3), (4100, 300, 2),
                                               (200, 33, 4)])
def test_dense_double_matches_closed_form(width, vocab, steps):
    for prompt in (0, 1, vocab - 1):
        dense = dorc.dense_double(prompt, width, vocab, steps)
        closed = dorc.closed_form(prompt, width, vocab, steps)
        for got, want in zip(dense[:3], closed[:3]):
            np.testing.assert_allclose(got, want, rtol=1e-13, atol=0)
        assert np.array_equal(dense[3], closed[3])
        # The dense argmax reproduces the analytic progression.
        assert np.array_equal(dense[3], dorc.analytic_tokens(1, vocab, steps, prompt)[0])


def test_planted_classifier_offset_breaks_agreement():
    # A classifier with the wrong offset moves the argmax: the oracle's dense
    # path must then disagree with the analytic progression.
    *_, tokens = dorc.dense_double(3, 96, 16, 5, classifier_offset=0)
    assert not np.array_equal(tokens, dorc.analytic_tokens(1, 16, 5, 3)[0])


def test_probe_sequences():
    assert dorc.probe_sequences(1024) == [0, 146, 292, 438, 584, 730, 876, 1023]  # contract.json
    assert dorc.probe_sequences(1) == [0]
    assert dorc.probe_sequences(3) == [0, 1, 2]
    assert dorc.probe_sequences(40) == [0, 5, 11, 16, 22, 27, 33, 39]


def test_invariants_flag_planted_errors():
    width, vocab = 96, 16
    o, _, p, _ = dorc.closed_form(0, width, vocab, 2)
    o32, p32 = o.astype(np.float32), p.astype(np.float32)
    sq_ok, sum_ok = dorc.invariants(o32, p32, width, vocab)
    assert sq_ok.all() and sum_ok.all()
    bad_o = o32.copy()
    bad_o[1, 0] *= 2.0  # the contract's fault 2
    sq_ok, _ = dorc.invariants(bad_o, p32, width, vocab)
    assert sq_ok.tolist() == [True, False]
    bad_p = p32.copy()
    bad_p[0, 3] = np.nan
    _, sum_ok = dorc.invariants(o32, bad_p, width, vocab)
    assert sum_ok.tolist() == [False, True]


def test_rmsnorm_f32_order():
    # Synthetic rows: the square sum is width + 15, exact in float32.
    emb, _, w = dorc.model(1000, 10)
    got = dorc.rmsnorm_f32(emb[3:4], w)[0]
    scale = np.float32(1) / np.sqrt(np.float32(1015) / np.float32(1000) + np.float32(1e-5))
    assert got[3] == np.float32(4) * scale and got[0] == scale


def run(args):
    if not os.path.exists(DECODER):
        pytest.skip("decoder binary not built")
    proc = subprocess.run([DECODER] + args, capture_output=True, text=True, timeout=60)
    return proc.returncode, proc.stdout, proc.stderr


# tests/run_tests.sh:56-68: invalid dimensions and usage exit 2 with a clear
# message, before the GPU is touched.
@pytest.mark.parametrize("args,needle", [
    (["--set", "vocab=1", "--set", "width=8"], "vocab must satisfy"),
    (["--set", "vocab=17", "--set", "width=16"], "vocab must satisfy"),
    (["--set", "steps=1", "--set", "width=32", "--set", "vocab=8"], "steps must be"),
    (["--set", "batch=0"], "batch must be"),
    (["--set", "width=0"], "width must be"),
    (["--set", "batch=1", "--set", "width=16777201", "--set", "vocab=2", "--set", "steps=2"], "width must be"),
    (["--set", "batch=1048576"], "GiB"),
    (["--set", "batch=abc"], "not an integer"),
    (["--set", "rows=4"], "unsupported --set key 'rows'"),
    (["--preset", "smoke", "--set", "width=32", "--set", "vocab=8"], "unknown preset 'smoke'"),
    (["--set", "fault=4"], "fault must be"),
    (["--action", "bench"], "bench needs --launch direct or --launch graph"),
    (["--action", "profile", "--launch", "both"], "profile needs --launch direct or --launch graph"),
    (["--action", "bench", "--launch", "graph", "--set", "batch=2"], "--set is only valid with --action check"),
    (["--launch", "sideways"], "--launch must be direct, graph or both"),
    (["--iterations", "0"], "--iterations expects an integer >= 1"),
    (["--set", "novalue"], "--set expects key=value"),
    (["--asset", "weights=/nope"], "unsupported --asset name 'weights'"),
    (["--bogus", "1"], "unknown option --bogus"),
    (["--preset"], "--preset needs a value"),
])
def test_usage_errors_exit_2(args, needle):
    code, out, err = run(args)
    assert code == 2, err
    assert needle in err
    assert out == ""


def test_help_exits_0():
    code, out, err = run(["--help"])
    assert code == 0 and out.startswith("usage:")


def test_in_process_usage_error():
    import l2c
    code, record, _ = l2c.decoder(["--set", "vocab=1", "--set", "width=8"], in_process=True)
    assert code == 2 and record is None
    # The library keeps running after an error: a second call works too.
    code, record, _ = l2c.decoder(["--set", "steps=1"], in_process=True)
    assert code == 2
