"""The lowprec classifier experiment's application on the CPU: its host
reference (the implementation check's quantizer, fixture generator and
self-test matrix) against the test oracle, and the argument and dimension
checks of the case binaries (exit 2 before any GPU work).

Reference: experiments/blackwell/lowprec (spec.json, decoder_lowprec.cu,
tests/run_tests.sh)."""
import os

import numpy as np
import pytest

import lowprec_oracle as lo
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "cuda-elastic_amd", "bin", "lowprec")


@pytest.fixture(scope="module")
def host():
    import l2c
    try:
        l2c.load_host()
    except (FileNotFoundError, OSError) as e:
        pytest.skip(f"host library not loadable: {e}")
    return l2c


def matrices(host):
    yield "crafted-app", host.lowprec_crafted(130, 256)
    yield "crafted-oracle", lo.crafted(64, 512)
    emb, cls = lo.fixture(3, 1024, 32)
    yield "fixture-normalized", lo.rmsnorm_double(emb).astype(np.float32)
    yield "fixture-classifier", cls


@pytest.mark.parametrize("case", ["bf16", "mxfp6", "nvfp4"])
def test_host_reference_matches_oracle(host, orc, case):
    for name, m in matrices(host):
        rows, width = m.shape
        codes, scales, decode = host.lowprec_host_quantize(case, m, rows, width)
        if case == "bf16":
            np.testing.assert_array_equal(codes, orc.bf16(m.ravel()), err_msg=name)
        elif case == "mxfp6":
            c, s = orc.quantize_mxfp6(m, rows, width)
            np.testing.assert_array_equal(codes, c, err_msg=name)
            np.testing.assert_array_equal(scales, s, err_msg=name)
        else:
            enc, dec = orc.nvfp4_scales(m)
            c, s = orc.quantize_nvfp4(m, rows, width, enc)
            np.testing.assert_array_equal(codes, c, err_msg=name)
            np.testing.assert_array_equal(scales, s, err_msg=name)
            assert np.float32(decode) == dec


def test_fixture_generator_matches_oracle(host):
    for seed in (1, 2, 3):
        emb, cls = host.lowprec_fixture(seed, 1024, 8)
        oemb, ocls = lo.fixture(seed, 1024, 8)
        np.testing.assert_array_equal(emb.view(np.uint32), oemb.view(np.uint32))
        np.testing.assert_array_equal(cls.view(np.uint32), ocls.view(np.uint32))


def test_selftest_matrix_covers_the_edge_cases(host, orc):
    m = host.lowprec_crafted(130, 256)
    assert np.abs(m).max() == 2688.0
    c6, s6 = orc.quantize_mxfp6(m, 130, 256)
    s6 = s6.reshape(130, 8)
    assert (s6 == 0).any() and 127 in s6[2]  # zero blocks, 2^X = 1
    assert (c6.reshape(130, 256)[3, ::32] == 31).all()  # saturating block maxima
    enc, _ = orc.nvfp4_scales(m)
    _, s4 = orc.quantize_nvfp4(m, 130, 256, enc)
    assert (s4.reshape(130, 16)[4, 0] == 0)  # a block scale that rounds to zero


def run(case, args):
    exe = os.path.join(BIN, case)
    if not os.path.exists(exe):
        pytest.skip("lowprec binaries not built")
    import subprocess
    p = subprocess.run([exe] + args, capture_output=True, text=True, timeout=60)
    return p.returncode, p.stdout, p.stderr


# tests/run_tests.sh:50-51 (bf16-unaligned-width) and the dimension checks of
# decoder_lowprec.cu:1106-1127.
@pytest.mark.parametrize("case,args,needle", [
    ("bf16", ["--set", "batch=5", "--set", "width=1001", "--set", "vocab=999"], "width % 128 == 0"),
    ("mxfp6", ["--set", "batch=5", "--set", "width=1024", "--set", "vocab=998"], "vocab % 4 == 0"),
    ("nvfp4", ["--set", "fixture=4"], "fixture must be 0"),
    ("fp32", ["--set", "batch=0"], "batch must be in"),
    ("fp32", ["--set", "vocab=2000", "--set", "width=1024"], "vocab must satisfy"),
    ("mxfp6", ["--set", "steps=1"], "steps must be in"),
    ("bf16", ["--accuracy", "--bogus"], "--accuracy takes only --json-out"),
    ("nvfp4", ["--set", "batch=1048576"], "GiB of device memory"),
    ("fp32", ["--set", "rows=3"], "unsupported --set key 'rows'"),
])
def test_usage_errors_exit_2(case, args, needle):
    code, out, err = run(case, args)
    assert code == 2, err
    assert needle in err
