"""The device format encoders and per-block quantizer rules
(cuda-elastic_amd/csrc/l2c_formats.h), built for the CPU as
lib/libl2c_formats_host.so, against the test oracle: every code, every
midpoint and its neighbours, a million random finite floats per format, and
whole-row MXFP6 / NVFP4 quantization of the crafted edge cases, fixtures and
random rows. The GPU tests then only have to show the kernels' lane layout
and packing."""
import ctypes
import os

import numpy as np
import pytest

import lowprec_oracle as lo
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATH = os.path.join(ROOT, "cuda-elastic_amd", "lib", "libl2c_formats_host.so")
f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


@pytest.fixture(scope="module")
def F():
    if not os.path.exists(PATH):
        pytest.skip("libl2c_formats_host.so not built")
    L = ctypes.CDLL(PATH)
    L.l2cf_encode_array.argtypes = [ctypes.c_int, f32p, ctypes.c_size_t, u8p]
    L.l2cf_values.argtypes = [ctypes.c_int, f32p]
    L.l2cf_quantize_mxfp6.argtypes = [f32p, ctypes.c_int, ctypes.c_int, u8p, u8p]
    L.l2cf_quantize_nvfp4.argtypes = [f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, u8p, u8p, ctypes.c_void_p]
    L.l2cf_nvfp4_encode_scale.argtypes, L.l2cf_nvfp4_encode_scale.restype = [ctypes.c_float], ctypes.c_float
    return L


def encode(F, fmt, v):
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(v.size, np.uint8)
    F.l2cf_encode_array(fmt, v, v.size, out)
    return out


def probes(table):
    """Every table value, every midpoint, and their float32 neighbours."""
    t = np.unique(np.abs(table.astype(np.float32)))
    mids = ((t[:-1].astype(np.float64) + t[1:]) / 2).astype(np.float32)
    pts = np.concatenate([t, mids, t * np.float32(1.5), [t.max() * np.float32(2), np.float32(1e-30), 0]]).astype(np.float32)
    pts = np.concatenate([pts, np.nextafter(pts, np.float32(np.inf)), np.nextafter(pts, np.float32(-np.inf))])
    return np.concatenate([pts, -pts]).astype(np.float32)


def random_floats(n, lo_exp, hi_exp, seed):
    rng = np.random.default_rng(seed)
    return (rng.uniform(1, 2, n) * np.exp2(rng.integers(lo_exp, hi_exp, n)) * rng.choice([-1, 1], n)).astype(np.float32)


def test_value_tables(F):
    e = np.empty(16, np.float32)
    F.l2cf_values(0, e)
    np.testing.assert_array_equal(e.astype(np.float64), np.abs(lo.E2M1) * np.where(np.arange(16) >= 8, -1, 1))
    u = np.empty(128, np.float32)
    F.l2cf_values(1, u)
    np.testing.assert_array_equal(u.astype(np.float64), lo.UE4M3)


@pytest.mark.parametrize("fmt,name,table,span", [(0, "e2m1", lo.E2M1, (-4, 5)), (1, "e3m2", lo.E3M2, (-8, 7))])
def test_element_encoders(F, orc, fmt, name, table, span):
    enc = orc.e2m1_encode if fmt == 0 else orc.e3m2_encode
    v = np.concatenate([probes(table), random_floats(1 << 20, span[0], span[1], fmt)])
    np.testing.assert_array_equal(encode(F, fmt, v), enc(v.astype(np.float64)))


def test_ue4m3_encoder(F, orc):
    v = np.abs(np.concatenate([probes(lo.UE4M3[:127]), random_floats(1 << 20, -14, 10, 7)]))
    np.testing.assert_array_equal(encode(F, 2, v), orc.ue4m3_encode(v.astype(np.float64)))


def _matrices():
    yield lo.crafted(130, 256)
    emb, cls = lo.fixture(1, 1024, 64)
    yield lo.rmsnorm_double(emb).astype(np.float32)
    yield cls
    rng = np.random.default_rng(2)
    yield (rng.standard_normal((17, 2048)) * np.exp2(rng.integers(-60, 60, (17, 1)))).astype(np.float32)


def test_row_quantizers(F, orc):
    for m in _matrices():
        rows, width = m.shape
        m = np.ascontiguousarray(m)
        c = np.empty(m.size, np.uint8)
        s = np.empty(m.size // 32, np.uint8)
        F.l2cf_quantize_mxfp6(m, rows, width, c, s)
        oc, os_ = orc.quantize_mxfp6(m, rows, width)
        np.testing.assert_array_equal(c, oc)
        np.testing.assert_array_equal(s, os_)
        enc, _ = orc.nvfp4_scales(m)
        assert np.float32(F.l2cf_nvfp4_encode_scale(float(np.abs(m).max()))) == enc
        c4 = np.empty(m.size, np.uint8)
        s4 = np.empty(m.size // 16, np.uint8)
        ex = np.empty(m.size, np.float32)
        F.l2cf_quantize_nvfp4(m, rows, width, float(enc), c4, s4, ex.ctypes.data)
        oc4, os4 = orc.quantize_nvfp4(m, rows, width, enc)
        np.testing.assert_array_equal(c4, oc4)
        np.testing.assert_array_equal(s4, os4)
        want = lo.dequantize_nvfp4(oc4, os4, rows, width).ravel()
        np.testing.assert_array_equal(ex.astype(np.float64), want)
        # The expansion is exact in bf16.
        assert not (ex.view(np.uint32) & 0xFFFF).any()
    assert F.l2cf_nvfp4_encode_scale(0.0) == 1.0


def test_host_mxfp8_exponent_matches_oracle(orc):
    """The harness's host MXFP8 block exponent (the closed form on the
    significand) equals the oracle's stepping definition."""
    import ctypes
    import l2c
    host = ctypes.CDLL(l2c.HOST_LIB_PATH)
    fn = host._ZN8l2c_host20mxfp8_block_exponentEf
    fn.argtypes, fn.restype = [ctypes.c_float], ctypes.c_int
    rng = np.random.default_rng(70)
    vals = np.concatenate([np.abs(rng.standard_normal(20000)).astype(np.float32) * np.float32(10.0) ** rng.integers(-40, 38, 20000).astype(np.float32),
                           np.array([448.0, 449.0, 1.75, 1.7500001, 0.0, 1e-45, 3e38, 224.0], np.float32)])
    for v in vals[np.isfinite(vals)]:
        assert fn(float(v)) == orc.lib().orc_mxfp8_exponent(float(v)), v
