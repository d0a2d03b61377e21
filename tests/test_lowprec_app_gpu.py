"""The lowprec classifier experiment's application on the GPU, case by case:
the cases of experiments/blackwell/lowprec/tests/run_tests.sh:37-60 (self-test,
the implementation check on the three dense fixtures, ragged tiles and one
sequence; the fp32 control at an odd width), planted faults in place of the
reference's mutant builds, the large preset, and the accuracy mode against
the reference's published accuracy (README.md "Numerical quality"), which
depends only on the formats, so a faithful implementation reproduces it."""
import pytest

pytestmark = pytest.mark.gpu

CASES = ["fp32", "bf16", "mxfp6", "nvfp4"]


def run(l2c, case, args, timeout=300, env=None):
    print(f"case lowprec {case} {' '.join(args)}{' ' + str(env) if env else ''}", flush=True)
    code, record, text = l2c.lowprec(case, args, timeout=timeout, env=env)
    print(text[-3000:], flush=True)
    return code, record, text


@pytest.mark.parametrize("case", CASES)
def test_selftest(torch_gpu, l2c, case):
    code, _, text = run(l2c, case, ["--selftest"])
    assert code == 0 and f"PASS: {case} quantizer self-test" in text


SHAPES = [("fixture1", ["--set", "fixture=1"]), ("fixture2", ["--set", "fixture=2"]),
          ("fixture3", ["--set", "fixture=3"]),
          ("ragged", ["--set", "batch=100", "--set", "width=1024", "--set", "vocab=200"]),
          ("one-sequence", ["--set", "batch=1", "--set", "width=256", "--set", "vocab=128", "--set", "steps=2"])]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("name,args", SHAPES)
def test_implementation_check(torch_gpu, l2c, case, name, args):
    code, record, text = run(l2c, case, args)
    assert code == 0, text[-2000:]
    assert "implementation check PASS" in text
    assert record["status"] == "pass" and record["outputs_agree"] is True
    assert record["identity"] == f"blackwell-experiments/lowprec-decoder-classifier/{case}"
    assert len({c["digest"] for c in record["checks"]}) == 1


def test_fp32_odd_width(torch_gpu, l2c):
    code, _, text = run(l2c, "fp32", ["--set", "batch=5", "--set", "width=1001", "--set", "vocab=999"])
    assert code == 0, text[-2000:]


@pytest.mark.parametrize("case,fault,needle", [
    ("bf16", 1, "code mismatch"), ("mxfp6", 1, "code mismatch"), ("mxfp6", 2, "scale mismatch"),
    ("nvfp4", 1, "code mismatch"), ("nvfp4", 2, "scale mismatch"), ("nvfp4", 3, "logit mismatch")])
def test_planted_faults_fail(torch_gpu, l2c, case, fault, needle):
    code, record, text = run(l2c, case, ["--set", "fixture=1", "--set", f"fault={fault}", "--launch", "direct"])
    assert code == 1
    assert needle in text and "implementation check FAIL" in text
    assert record["status"] == "fail"


@pytest.mark.parametrize("case", CASES)
def test_large_check(torch_gpu, l2c, case):
    """The experiment's check invocation (experiment.json "check": --preset
    large --action check --launch both)."""
    code, record, text = run(l2c, case, ["--preset", "large", "--action", "check", "--launch", "both"], timeout=600)
    assert code == 0, text[-2000:]
    assert record["dimensions"]["classifier_macs_per_step"] == 1024 * 8192 * 16384


# README.md "Numerical quality" (RTX 5090 runs): normalized RMS error of the
# classifier on the primary model and the fixtures, and token agreement of
# the fixtures' decodes (of 256).
PUBLISHED = {
    "fp32": {"primary_rms": 0.0, "fixture_rms": (5.7e-7, 5.8e-7), "tokens": (256, 256, 256), "production": True},
    "bf16": {"primary_rms": 4.6e-4, "fixture_rms": (0.0023, 0.0023), "tokens": (249, 256, 247), "production": False},
    "mxfp6": {"primary_rms": 0.124, "fixture_rms": (0.075, 0.077), "tokens": (174, 195, 204), "production": False},
    "nvfp4": {"primary_rms": 6.0e-8, "fixture_rms": (0.134, 0.136), "tokens": (163, 161, 171), "production": True},
}


@pytest.mark.parametrize("case", CASES)
def test_accuracy_matches_published(torch_gpu, l2c, case):
    code, record, text = run(l2c, case, ["--accuracy"], timeout=600)
    assert code == 0, text[-2000:]
    assert record["schema"] == "blackwell_experiments.lowprec_accuracy/1"
    ds = {d["dataset"]: d for d in record["datasets"]}
    want = PUBLISHED[case]
    primary = ds["primary"]
    assert primary["tokens"]["agree"] == 4096
    assert primary["production_fp32_tolerance_pass"] is want["production"]
    rms = primary["classifier_error"]["normalized_rms_error"]
    if want["primary_rms"] == 0.0:
        assert rms == 0.0
    else:
        assert abs(rms - want["primary_rms"]) <= 0.05 * want["primary_rms"], rms
    lo, hi = want["fixture_rms"]
    for i, tokens in enumerate(want["tokens"], start=1):
        d = ds[f"fixture{i}"]
        r = d["classifier_error"]["normalized_rms_error"]
        assert lo * 0.9 <= r <= hi * 1.1, (i, r)
        # Measured equal to the published counts. (A change of accumulation
        # order could move a near-tie; a token that differs then changes that
        # sequence's later steps.)
        assert d["tokens"]["agree"] == tokens, (i, d["tokens"])


@pytest.mark.parametrize("args", [["--set", "fixture=1"], ["--preset", "large", "--action", "check", "--launch", "both"]])
def test_nvfp4_amax_in_rmsnorm_changes_nothing(torch_gpu, l2c, args):
    """With L2C_LOWPREC_AMAX_IN_RMSNORM=1 the NVFP4 steps take the activations'
    maximum from the rmsnorm (l2c_decoder_rmsnorm_absmax and
    l2c_nvfp4_tensor_scales_absmax) instead of a pass of their own: the check
    passes and every output digest equals the default path's."""
    digests = []
    for env in (None, {"L2C_LOWPREC_AMAX_IN_RMSNORM": "1"}):
        code, record, text = run(l2c, "nvfp4", args, timeout=600, env=env)
        assert code == 0, text[-2000:]
        assert record["status"] == "pass"
        digests.append({c["digest"] for c in record["checks"]})
    assert len(digests[0]) == 1 and digests[0] == digests[1]
