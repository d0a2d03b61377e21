"""The oracle against the committed golden fixtures (tests/golden/golden.json,
written from the reference's own host code by tests/golden/make_golden.py)
and against closed forms that hold without any fixture."""
import hashlib
import json
import math
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = json.load(open(os.path.join(HERE, "golden", "golden.json")))


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_uniform_spot_values(orc):
    for seed, stream, index, bits in GOLDEN["uniform_bits"]:
        v = np.float32(orc.lib().orc_uniform(seed, stream, index))
        assert v.view(np.uint32) == bits, (seed, stream, index)


@pytest.mark.parametrize("case", GOLDEN["fill_sha256"], ids=lambda c: f"m{c['mode']}s{c['size']}")
def test_fill_checksums(orc, case):
    inp = orc.fill(case["mode"], case["seed"], case["batch"], case["size"], case["rows"])
    assert sha(inp.input) == case["input"]
    assert sha(inp.probabilities) == case["probabilities"]
    assert sha(inp.weight) == case["weight"]
    assert sha(inp.matrix) == case["matrix"]


def test_gamma_values(orc):
    for n, g in GOLDEN["gamma"]:
        assert orc.gamma(n) == g


def test_format_tables(orc):
    e = GOLDEN["e2m1"]
    np.testing.assert_array_equal(orc.e2m1_encode(np.array(e["values"])), np.array(e["codes"], np.uint8))
    u = GOLDEN["ue4m3"]
    np.testing.assert_array_equal(orc.ue4m3_encode(np.array(u["values"])), np.array(u["codes"], np.uint8))
    b = GOLDEN["bf16"]
    v = np.array(b["bits"], np.uint32).view(np.float32)
    np.testing.assert_array_equal(orc.bf16(v), np.array(b["codes"], np.uint16))


def test_normals(orc):
    for case in GOLDEN["normals"]:
        got = orc.normal(case["seed"], case["stream"], 0, len(case["bits"]))
        np.testing.assert_array_equal(got.view(np.uint32), np.array(case["bits"], np.uint32))


def test_reference_dump_fixture(orc):
    """The dump the reference wrote: our reader parses it, its products sit
    inside its tolerances, and the oracle reproduces its tolerance and
    double-reference sections from regenerated inputs bit for bit."""
    d = GOLDEN["dump"]
    dump = orc.read_dump(os.path.join(HERE, "golden", d["file"]))
    assert (dump["batch"], dump["size"], dump["rows"], dump["seed"]) == (d["batch"], d["size"], d["rows"], d["seed"])
    inp = orc.fill("random", d["seed"], d["batch"], d["size"], d["rows"])
    ok, tol, refv, ratio, _ = orc.product_check(False, False, inp.input, inp.matrix, dump["product"],
                                                d["batch"], d["size"], d["rows"], [0])
    assert ok and d["valid"] == 1
    np.testing.assert_array_equal(tol, dump["product_tolerance"])
    np.testing.assert_array_equal(refv, dump["product_reference"])
    ok, err = orc.check_vectors(False, inp, dump["normalized"], dump["softmax"], d["batch"], d["size"])
    assert ok


# ---------------------------------------------------------------------------
# Closed forms and invariants (no fixture needed).

def test_deterministic_closed_forms(orc):
    """Deterministic inputs (llama2c_common.h:114-122): the shifted identity
    makes product[r] = input[r % size] exactly, the fp32 iteration's mean
    square of normalized/weight is 1, and softmax rows sum to 1."""
    batch, size, rows = 3, 10, 23
    inp = orc.fill("deterministic", 0, batch, size, rows)
    assert np.all(inp.input == np.tile([1, 2, 3, 4], batch * size // 4 + 1)[:batch * size])
    n, s, p = orc.iteration_f32(inp, batch, size, rows)
    np.testing.assert_array_equal(p, inp.input[np.arange(rows) % size])
    np.testing.assert_array_equal(orc.matvec_fma(inp.input, inp.matrix, size, rows), p)
    ms = np.mean(n.reshape(batch, size).astype(np.float64) ** 2, axis=1)
    np.testing.assert_allclose(ms, 1.0 / (1.0 + 1e-5 / np.mean(inp.input.reshape(batch, size).astype(np.float64) ** 2, axis=1)), rtol=1e-6)
    np.testing.assert_allclose(s.reshape(batch, size).sum(axis=1), 1.0, rtol=1e-6)


def test_rmsnorm_softmax_refs_against_numpy(orc):
    """The double references equal a numpy restatement of the textbook
    definitions (rmsnorm: x / sqrt(mean x^2 + eps) * w; softmax: exp(x - max) / sum)."""
    batch, size = 4, 333
    inp = orc.fill("random", 3, batch, size, 1)
    x = inp.input.reshape(batch, size).astype(np.float64)
    w = inp.weight.astype(np.float64)
    want = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + np.float64(np.float32(1e-5))) * w
    np.testing.assert_allclose(orc.rmsnorm_ref(inp.input, inp.weight, batch, size).reshape(batch, size),
                               want, rtol=1e-13, atol=0)
    p = inp.probabilities.reshape(batch, size).astype(np.float64)
    e = np.exp(p - p.max(axis=1, keepdims=True))
    np.testing.assert_allclose(orc.softmax_ref(inp.probabilities, batch, size).reshape(batch, size),
                               e / e.sum(axis=1, keepdims=True), rtol=1e-13, atol=0)


def test_product_check_catches_dropped_term(orc):
    """A product that drops its last 4 terms (the SOTA mutant the reference's
    bound is sized to catch, llama2c_common.h:222-223) fails the random check."""
    batch, size, rows = 1, 16384, 64
    inp = orc.fill("random", 1, batch, size, rows)
    M = inp.matrix.reshape(rows, size).astype(np.float64)
    x = inp.input[:size].astype(np.float64)
    good = (M @ x).astype(np.float32)
    bad = (M[:, :-4] @ x[:-4]).astype(np.float32)
    assert orc.product_check(False, False, inp.input, inp.matrix, good, 1, size, rows, [0])[0]
    assert not orc.product_check(False, False, inp.input, inp.matrix, bad, 1, size, rows, [0])[0]


def test_iteration_f32_within_bounds(orc):
    batch, size, rows = 4, 4096, 64
    inp = orc.fill("scaled", 2, batch, size, rows)
    n, s, p = orc.iteration_f32(inp, batch, size, rows, batched=True, vectors=batch)
    ok, err = orc.check_vectors(False, inp, n, s, batch, size)
    assert ok and err[1] < 1e-5 and err[3] < 1e-4
    ok, tol, refv, ratio, rel = orc.product_check(False, True, inp.input, inp.matrix, p, batch, size,
                                                  rows, list(range(batch)))
    assert ok


def test_mxfp4_exponent_closed_form(orc):
    rng = np.random.default_rng(5)
    a = np.concatenate([np.abs(rng.standard_normal(5000)).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 5000),
                        np.array([6.0, 12.0, 5.999999, 6.000001, 3.0, 1.5, 0.0], np.float32)])
    a = a[np.isfinite(a)].astype(np.float32)
    x = orc.mxfp4_exponent(a)
    for v, e in zip(a, x):
        if v == 0:
            assert e == -127
        elif -127 < e < 127:
            assert math.ldexp(6.0, int(e)) <= float(v) < math.ldexp(6.0, int(e) + 1)


def test_e2m1_roundtrip_and_ties(orc):
    codes = np.arange(16)
    vals = np.array([orc.lib().orc_e2m1_value(int(c)) for c in codes])
    back = orc.e2m1_encode(vals)
    # Every code round-trips except -0 (code 8), which encodes as +0.
    np.testing.assert_array_equal(back, np.where(codes == 8, 0, codes))
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    np.testing.assert_array_equal(orc.e2m1_encode(ties), [0, 2, 2, 4, 4, 6, 6])
    assert orc.e2m1_encode(np.array([100.0]))[0] == 7


@pytest.mark.parametrize("batched", [False, True])
def test_iteration_f32_threads_bit_equal(orc, batched):
    """The threaded CPU baseline computes every output with the scalar
    restatement's loops: equal bit for bit at any thread count."""
    batch, size, rows = 7, 333, 129
    inp = orc.fill("scaled", 3, batch, size, rows)
    ref = orc.iteration_f32(inp, batch, size, rows, batched=batched, vectors=batch)
    for threads in (1, 3, 8):
        got = orc.iteration_f32_mt(inp, batch, size, rows, batched=batched, vectors=batch, threads=threads)
        for a, b in zip(got, ref):
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
