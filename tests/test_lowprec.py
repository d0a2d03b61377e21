"""The low-precision classifier formats on the CPU: the oracle's E3M2, MXFP6
and NVFP4 quantizers against the golden codes written by the reference's own
quantizers, the value tables against the format definitions, packing, and
the implementation check's logit bound (it holds for float32 sums in any
order and rejects planted scale-layout and alpha mistakes).

Reference: experiments/blackwell/lowprec (spec.json, reference.cpp)."""
import json
import os

import numpy as np
import pytest

import lowprec_oracle as lo

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))


def test_e3m2_golden_codes(orc):
    g = GOLDEN["e3m2"]
    np.testing.assert_array_equal(orc.e3m2_encode(np.array(g["values"])), np.array(g["codes"], np.uint8))


def test_e3m2_table_definition(orc):
    # spec.json "formats.E3M2": bias 3, subnormal m/4 * 2^-2, largest 28 at 0x1f, bit 5 the sign.
    assert lo.E3M2[0x1F] == 28.0 and lo.E3M2[1] == 0.0625 and lo.E3M2[4] == 0.25
    assert lo.E3M2[0x3F] == -28.0
    mags = lo.E3M2[:32]
    assert np.all(np.diff(mags) > 0)
    for c in range(64):
        assert orc.e3m2_value(c) == lo.E3M2[c]
        want = 0 if c == 32 else c  # -0 encodes as +0
        assert orc.e3m2_encode(np.array([lo.E3M2[c]]))[0] == want
    # Every midpoint is a tie to the even code; just above goes up.
    mid = (mags[:-1] + mags[1:]) / 2
    codes = orc.e3m2_encode(mid)
    lower = np.arange(31)
    np.testing.assert_array_equal(codes, np.where(lower % 2 == 0, lower, lower + 1))
    np.testing.assert_array_equal(orc.e3m2_encode(np.nextafter(mid, 100)), lower + 1)


def test_mxfp6_exponent_closed_form(orc):
    rng = np.random.default_rng(1)
    v = np.concatenate([np.exp2(rng.uniform(-140, 127, 2000)), [1.0, 2.0, 0.9995, 1.999, 3e38, 1e-45]])
    v = v.astype(np.float32)
    v = v[v > 0]
    got = np.array([orc.lib().orc_mxfp6_exponent(float(x)) for x in v])
    want = np.clip(np.frexp(v.astype(np.float64))[1] - 1 - 4, -127, 127)
    np.testing.assert_array_equal(got, want)


def test_crafted_golden_codes(orc):
    g = GOLDEN["lowprec_crafted"]
    rows, width = g["rows"], g["width"]
    m = lo.crafted(rows, width)
    import hashlib
    assert hashlib.sha256(m.tobytes()).hexdigest() == g["input_sha256"]
    c6, s6 = orc.quantize_mxfp6(m, rows, width)
    assert orc.pack_e3m2(c6).tobytes().hex() == g["mxfp6_codes_packed_hex"]
    assert s6.tobytes().hex() == g["mxfp6_scales_hex"]
    enc, dec = orc.nvfp4_scales(m)
    assert int(enc.view(np.uint32)) == g["nvfp4_encode_bits"] and int(dec.view(np.uint32)) == g["nvfp4_decode_bits"]
    c4, s4 = orc.quantize_nvfp4(m, rows, width, enc)
    assert orc.pack_e2m1(c4).tobytes().hex() == g["nvfp4_codes_packed_hex"]
    assert s4.tobytes().hex() == g["nvfp4_scales_hex"]


def test_crafted_cases_behave_as_specified(orc):
    m = lo.crafted(40, 256)
    c6, s6 = orc.quantize_mxfp6(m, 40, 256)
    c6, s6 = c6.reshape(40, 256), s6.reshape(40, 8)
    # Row 2 block 0: maximum 30 -> X = 0; 26 ties between 24 and 28 -> 24 (even code 30);
    # 30 saturates to 28 (0x1f); 0.03125 ties to 0; -0.09375 ties to -0.125.
    assert s6[2, 0] == 127
    assert c6[2, 7] == 30 and c6[2, 8] == 31 and c6[2, 0] == 0 and c6[2, 10] == (32 | 2)
    # Row 3: every block maximum (2 - 2^-j) 2^e scales past 28 and saturates.
    for i in range(8):
        assert c6[3, 32 * i] == 31
    # Zero blocks: scale 0, codes 0; -0 encodes as +0.
    assert s6[6, 0] == 0 and s6[6, 1] == 0 and not c6[6, :64].any()
    enc, _ = orc.nvfp4_scales(m)
    assert enc == 1.0  # the tensor maximum 2688
    c4, s4 = orc.quantize_nvfp4(m, 40, 256, enc)
    c4, s4 = c4.reshape(40, 256), s4.reshape(40, 16)
    # Row 1 block 0: maximum 6.2 -> scale 1.0333 rounds to 1.0 (0x38); 6.2 saturates to 6.
    assert s4[1, 0] == 0x38 and c4[1, 15] == 7
    assert c4[1, :8].tolist() == [0, 2, 2, 4, 4, 6, 6, 7]  # ties to even codes
    # Row 4 block 0: maximum 8e-6 -> the block scale rounds to zero, codes zero.
    assert s4[4, 0] == 0 and not c4[4, :16].any()
    # Row 5: scale targets 1 + i / 16 tie between UE4M3 codes for odd i.
    targets = 1.0 + 0.0625 * (np.arange(16) % 16)
    np.testing.assert_array_equal(s4[5], orc.ue4m3_encode(targets))


def test_pack_unpack_roundtrip(orc):
    rng = np.random.default_rng(4)
    c = rng.integers(0, 64, 1024).astype(np.uint8)
    np.testing.assert_array_equal(lo.unpack_e3m2(orc.pack_e3m2(c), c.size), c)
    c4 = rng.integers(0, 16, 1024).astype(np.uint8)
    np.testing.assert_array_equal(lo.unpack_e2m1(orc.pack_e2m1(c4), c4.size), c4)
    # The first four values fill three bytes little-endian.
    assert orc.pack_e3m2(np.array([1, 2, 3, 4], np.uint8)).tolist() == [0x81, 0x30, 0x10]


def _dequantized(orc, fmt, m):
    rows, width = m.shape
    if fmt == "mxfp6":
        c, s = orc.quantize_mxfp6(m, rows, width)
        return lo.dequantize_mxfp6(c, s, rows, width), 1.0, (c, s)
    enc, dec = orc.nvfp4_scales(m)
    c, s = orc.quantize_nvfp4(m, rows, width, enc)
    return lo.dequantize_nvfp4(c, s, rows, width), float(dec), (c, s)


@pytest.mark.parametrize("fmt", ["mxfp6", "nvfp4"])
def test_logit_bound_holds_for_float32_orders(orc, fmt):
    emb, cls = lo.fixture(1, 1024, 32)
    a = lo.rmsnorm_double(emb[:6]).astype(np.float32)
    A, da, _ = _dequantized(orc, fmt, a)
    W, dw, _ = _dequantized(orc, fmt, cls)
    alpha = float(np.float32(da) * np.float32(dw))
    exp, bound = lo.logit_bound(A, W, alpha, 1024)
    A32, W32 = A.astype(np.float32), W.astype(np.float32)  # exact: every product is exact
    for order in (slice(None), slice(None, None, -1)):
        prods = A32[:, None, order] * W32[None, :, order]
        seq = np.zeros(prods.shape[:2], np.float32)
        for k in range(prods.shape[2]):
            seq = seq + prods[:, :, k]
        got = seq * np.float32(alpha)
        assert np.all(np.abs(got - exp) <= bound)
    blocked = (prods.reshape(6, 32, 32, 32).sum(axis=3, dtype=np.float32).sum(axis=2, dtype=np.float32)
               * np.float32(alpha))
    assert np.all(np.abs(blocked - exp) <= bound)


@pytest.mark.parametrize("mistake", ["scale-layout", "alpha", "rounding"])
def test_logit_bound_rejects_planted_mistakes(orc, mistake):
    """Planted on the CPU, in the oracle's operands: each block's scale read
    from its neighbour's slot, alpha left at 1 (NVFP4), element codes rounded
    down by one step when odd. The implementation check must reject each."""
    emb, cls = lo.fixture(1, 1024, 32)
    a = lo.rmsnorm_double(emb[:6]).astype(np.float32)
    fmt = "mxfp6" if mistake == "rounding" else "nvfp4"
    A, da, _ = _dequantized(orc, fmt, a)
    W, dw, (wc, ws) = _dequantized(orc, fmt, cls)
    alpha = float(np.float32(da) * np.float32(dw))
    exp, bound = lo.logit_bound(A, W, alpha, 1024)
    if mistake == "scale-layout":
        ws2 = ws.reshape(32, -1)[:, np.arange(64) ^ 1].ravel()
        got = (A @ lo.dequantize_nvfp4(wc, ws2, 32, 1024).T) * alpha
    elif mistake == "alpha":
        got = A @ W.T
    else:
        wc2 = np.where((wc & 31) > 1, wc & ~np.uint8(1), wc)
        got = A @ lo.dequantize_mxfp6(wc2, ws, 32, 1024).T
    assert np.any(np.abs(got - exp) > bound)
