"""Pins the oracle (oracle/l2c_oracle.c) against the reference's own host code
compiled as it lies (oracle/_ref/libl2c_ref.so): generator, input sets, the
gamma bound, validate_all decisions on planted errors, the dump layout and the
lowprec format encoders. Skipped where the reference tree was not available to
build oracle/_ref (the committed fixtures of test_golden.py still apply)."""
import os
import tempfile

import numpy as np
import pytest


@pytest.fixture(scope="module")
def R(orc):
    r = orc.ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return r


def test_uniform_matches(R, orc):
    for seed in (0, 1, 2, 3, 99, 2**63 + 5):
        for stream in range(4):
            for start in (0, 12345, 2**40):
                a = orc.uniform(seed, stream, start, 4096)
                b = np.empty(4096, np.float32)
                R.ref_uniform_array(seed, stream, start, 4096, b)
                np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("mode,seed,batch,size,rows", [
    (0, 0, 3, 17, 5), (1, 1, 2, 1001, 7), (1, 2, 1, 288, 288), (1, 3, 33, 64, 77), (0, 0, 5, 8, 40)])
def test_fill_matches(R, orc, mode, seed, batch, size, rows):
    ours = orc.fill(mode, seed, batch, size, rows)
    x = np.empty(batch * size, np.float32)
    p = np.empty(batch * size, np.float32)
    w = np.empty(size, np.float32)
    m = np.empty(rows * size, np.float32)
    R.ref_fill(mode, seed, batch, size, rows, x, p, w, m)
    for a, b in ((ours.input, x), (ours.probabilities, p), (ours.weight, w), (ours.matrix, m)):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_gamma_matches_and_closed_form(R, orc):
    for n in (1, 2, 288, 1001, 4096, 16384, 65536, 1 << 20):
        assert orc.gamma(n) == R.ref_gamma(n)
        first_order = 9.0 * np.sqrt(n) * 2.0**-24
        assert abs(orc.gamma(n) - first_order) <= first_order**2  # expm1(t) - t = O(t^2)
    assert abs(orc.gamma(16384) - 6.87e-5) < 1e-7


def _good_outputs(orc, inp, batch, size, rows):
    n = orc.rmsnorm_ref(inp.input, inp.weight, batch, size).astype(np.float32)
    s = orc.softmax_ref(inp.probabilities, batch, size).astype(np.float32)
    prod = (inp.matrix.reshape(rows, size).astype(np.float64) @ inp.input[:size].astype(np.float64))
    return n, s, prod.astype(np.float32)


def _both(R, orc, mode, seed, inp, n, s, prod, batch, size, rows):
    tol = np.empty(rows, np.float32)
    refv = np.empty(rows, np.float64)
    rv = R.ref_validate_all(mode, seed, inp.input, inp.probabilities, inp.weight, inp.matrix,
                            n, s, prod, batch, size, rows, tol, refv)
    ok_v, _ = orc.check_vectors(mode == 0, inp, n, s, batch, size)
    ok_p, otol, oref, _, _ = orc.product_check(mode == 0, False, inp.input, inp.matrix, prod, batch,
                                               size, rows, [0])
    return bool(rv), ok_v and ok_p, tol, refv, otol, oref


@pytest.mark.parametrize("mode,seed", [(0, 0), (1, 1), (1, 2)])
def test_validate_decisions_match(R, orc, mode, seed):
    batch, size, rows = 3, 257, 40
    inp = orc.fill(mode, seed, batch, size, rows)
    n, s, prod = _good_outputs(orc, inp, batch, size, rows)
    rv, ov, tol, refv, otol, oref = _both(R, orc, mode, seed, inp, n, s, prod, batch, size, rows)
    assert rv and ov
    np.testing.assert_array_equal(tol.view(np.uint32), otol.view(np.uint32))
    np.testing.assert_array_equal(refv, oref)
    # Planted errors: each must flip both oracles the same way.
    plants = [
        ("normalized", 5, 3.5e-4, False), ("normalized", 5, 2.5e-4, True),
        ("softmax", 9, None, False), ("product", 3, 1.5, False), ("product", 3, 0.4, True),
    ]
    for what, idx, amount, expect in plants:
        n2, s2, p2 = n.copy(), s.copy(), prod.copy()
        if what == "normalized":
            n2[idx] += np.float32(amount)
        elif what == "softmax":
            s2[idx] *= np.float32(1.0025)
        else:
            p2[idx] = np.float32(refv[idx] + amount * tol[idx])
        if mode == 0 and what == "product" and expect:
            expect = abs(p2[idx] - inp.input[idx % size]) <= 1e-4
        rv2, ov2, *_ = _both(R, orc, mode, seed, inp, n2, s2, p2, batch, size, rows)
        assert rv2 == expect and ov2 == expect, (what, amount, rv2, ov2)
    # NaN poison fails both.
    n3 = n.copy()
    n3[0] = np.nan
    rv3, ov3, *_ = _both(R, orc, mode, seed, inp, n3, s, prod, batch, size, rows)
    assert not rv3 and not ov3


def test_dump_layout_matches_reader(R, orc):
    batch, size, rows, seed = 3, 8, 6, 4
    inp = orc.fill(1, seed, batch, size, rows)
    n, s, prod = _good_outputs(orc, inp, batch, size, rows)
    tol = np.arange(rows, dtype=np.float32) + 0.5
    refv = np.arange(rows, dtype=np.float64) * 3.25
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "x.bin")
        assert R.ref_write_dump(path.encode(), 1, seed, batch, size, rows, n, s, prod, tol, refv) == 1
        dump = orc.read_dump(path)
        assert os.path.getsize(path) == 32 + 4 * (2 * batch * size + 2 * rows) + 8 * rows
    assert dump["magic"] == "L2CDUMP1" and dump["seed"] == seed and dump["inputs"] == 1
    np.testing.assert_array_equal(dump["normalized"], n)
    np.testing.assert_array_equal(dump["softmax"], s)
    np.testing.assert_array_equal(dump["product"], prod)
    np.testing.assert_array_equal(dump["product_tolerance"], tol)
    np.testing.assert_array_equal(dump["product_reference"], refv)


def test_e2m1_encoder_matches(R, orc):
    rng = np.random.default_rng(0)
    v = np.concatenate([np.arange(-8 * 64, 8 * 64 + 1) / 64.0, rng.standard_normal(20000) * 4,
                        [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -5.0, 1e300, -1e-300]])
    ref = np.empty(v.size, np.uint8)
    R.ref_encode_array(0, v, v.size, ref)
    np.testing.assert_array_equal(orc.e2m1_encode(v), ref)


def test_ue4m3_encoder_matches(R, orc):
    rng = np.random.default_rng(1)
    mags = np.array([orc.lib().orc_ue4m3_value(c) for c in range(127)])
    mids = (mags[:-1] + mags[1:]) / 2  # every tie
    v = np.concatenate([mags, mids, np.abs(rng.standard_normal(20000)) * 30,
                        np.abs(rng.standard_normal(2000)) * 1e-3, [448, 460, 464, 465, 1e9]])
    ref = np.empty(v.size, np.uint8)
    R.ref_encode_array(2, v, v.size, ref)
    np.testing.assert_array_equal(orc.ue4m3_encode(v), ref)
    # Signed: the oracle adds bit 7; magnitudes unchanged.
    neg = orc.ue4m3_encode(-v)
    np.testing.assert_array_equal(neg & 0x7F, ref)
    assert np.all((neg & 0x80) == np.where(ref != 0, 0x80, 0))


def test_bf16_matches(R, orc):
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    v = bits.view(np.float32)
    v = v[np.isfinite(v)]
    ref = np.empty(v.size, np.uint16)
    R.ref_to_bf16_array(v, v.size, ref)
    np.testing.assert_array_equal(orc.bf16(v), ref)


def test_normals_match(R, orc):
    for seed in (1, 2, 3):
        ref = np.empty(1000, np.float32)
        R.ref_normals_stream1(seed, 1000, ref)
        np.testing.assert_array_equal(orc.normal(seed, 1, 0, 1000).view(np.uint32), ref.view(np.uint32))


# --- MXFP6 / NVFP4 (experiments/blackwell/lowprec/reference.cpp:105-168) ----

def _lowprec_inputs():
    import lowprec_oracle as lo
    yield "crafted", lo.crafted(130, 256)
    emb, cls = lo.fixture(2, 1024, 16)
    yield "fixture-embedding", emb
    yield "fixture-classifier", cls
    rng = np.random.default_rng(3)
    wide = (rng.standard_normal((9, 4096)) * np.exp2(rng.integers(-20, 20, (9, 1)))).astype(np.float32)
    yield "scaled-rows", wide


def test_mxfp6_quantizer_matches(R, orc):
    for name, m in _lowprec_inputs():
        rows, width = m.shape
        c, s = orc.quantize_mxfp6(m, rows, width)
        c2 = np.empty_like(c)
        s2 = np.empty_like(s)
        R.ref_quantize_mxfp6(np.ascontiguousarray(m), rows, width, c2, s2)
        np.testing.assert_array_equal(c, c2, err_msg=name)
        np.testing.assert_array_equal(s, s2, err_msg=name)


def test_nvfp4_quantizer_matches(R, orc):
    for name, m in _lowprec_inputs():
        rows, width = m.shape
        enc, dec = orc.nvfp4_scales(m)
        amax = float(np.float32(np.abs(m).max()))
        assert np.float32(R.ref_nvfp4_encode_scale(amax)) == enc
        assert np.float32(R.ref_nvfp4_decode_scale(float(enc))) == dec
        c, s = orc.quantize_nvfp4(m, rows, width, enc)
        c2 = np.empty_like(c)
        s2 = np.empty_like(s)
        R.ref_quantize_nvfp4(np.ascontiguousarray(m), rows, width, float(enc), c2, s2)
        np.testing.assert_array_equal(c, c2, err_msg=name)
        np.testing.assert_array_equal(s, s2, err_msg=name)
    assert R.ref_nvfp4_encode_scale(0.0) == 1.0


def test_packing_matches_reference_unpack(R, orc):
    rng = np.random.default_rng(9)
    c6 = rng.integers(0, 64, 4 * 96).astype(np.uint8)
    p6 = orc.pack_e3m2(c6)
    assert p6.size == c6.size * 3 // 4
    assert [R.ref_unpack_e3m2(p6, i) for i in range(c6.size)] == c6.tolist()
    c4 = rng.integers(0, 16, 256).astype(np.uint8)
    p4 = orc.pack_e2m1(c4)
    assert [R.ref_unpack_e2m1(p4, i) for i in range(c4.size)] == c4.tolist()


def test_e3m2_encoder_matches(R, orc):
    v = np.concatenate([np.linspace(-40, 40, 20001), np.ldexp(np.arange(-64, 65) / 8.0, -4)])
    ours = orc.e3m2_encode(v)
    theirs = np.empty(v.size, np.uint8)
    R.ref_encode_array(1, np.ascontiguousarray(v, np.float64), v.size, theirs)
    np.testing.assert_array_equal(ours, theirs)
