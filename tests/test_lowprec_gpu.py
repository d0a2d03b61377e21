"""The low-precision classifier path on the GPU through the C ABI: the device
quantizers (MXFP6, NVFP4 with its tensor scales and alpha, BF16) bit for bit
against the oracle, and the bf16 and MXFP6 contractions against the double
product of the dequantized operands within the implementation check's bound
(experiments/blackwell/lowprec/spec.json "implementation_check")."""
import numpy as np
import pytest

import lowprec_oracle as lo
import oracle

pytestmark = pytest.mark.gpu


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def inputs(name, rows, width):
    if name == "crafted":
        return lo.crafted(rows, width)
    if name == "fixture":
        emb, _ = lo.fixture(1, width, rows)
        return lo.rmsnorm_double(emb).astype(np.float32)
    rng = np.random.default_rng(rows * 7 + width)
    return (rng.standard_normal((rows, width)) * np.exp2(rng.integers(-30, 30, (rows, 1)))).astype(np.float32)


CASES = [("crafted", 130, 256), ("crafted", 8, 128), ("fixture", 64, 1024), ("random", 1, 128 * 3),
         ("random", 333, 2048)]


def mxfp6_buffers(torch, l2c, rows, width):
    cb, sb = l2c.mxfp6_bytes(rows, width)
    assert cb == (rows + 31) // 32 * 32 * width * 3 // 4 and sb == (rows + 31) // 32 * 32 * width // 32
    return (torch.full((cb,), 0xAB, dtype=torch.uint8, device="cuda"),
            torch.full((sb,), 0xAB, dtype=torch.uint8, device="cuda"))


@pytest.mark.parametrize("name,rows,width", CASES)
def test_quantize_mxfp6_exact(torch_gpu, l2c, name, rows, width):
    """Codes and scales bit for bit in the tiled operand layout, padding rows zero."""
    torch = torch_gpu
    print(f"case quantize_mxfp6 {name} {rows}x{width}", flush=True)
    x = inputs(name, rows, width)
    codes, scales = mxfp6_buffers(torch, l2c, rows, width)
    l2c.quantize_mxfp6(codes, scales, dev(torch, x), rows, width)
    torch.cuda.synchronize()
    c, s = oracle.quantize_mxfp6(x, rows, width)
    pc, ps = lo.tile_mxfp6(c, s, rows, width)
    np.testing.assert_array_equal(codes.cpu().numpy(), pc)
    np.testing.assert_array_equal(scales.cpu().numpy(), ps)


NVFP4_CASES = [("crafted", 130, 256), ("crafted", 8, 128), ("fixture", 64, 1024), ("random", 1, 32 * 3),
               ("random", 333, 2048), ("random", 3, 16)]


@pytest.mark.parametrize("name,rows,width", NVFP4_CASES)
def test_quantize_nvfp4_exact(torch_gpu, l2c, name, rows, width):
    torch = torch_gpu
    print(f"case quantize_nvfp4 {name} {rows}x{width}", flush=True)
    x = inputs(name, rows, width)
    f32 = torch.float32
    ts = torch.full((2,), np.nan, dtype=f32, device="cuda")
    alpha = torch.full((1,), np.nan, dtype=f32, device="cuda")
    other = torch.tensor([0.75], dtype=f32, device="cuda")
    partials = torch.empty(l2c.NVFP4_PARTIALS, dtype=f32, device="cuda")
    codes = torch.full((rows * width // 2,), 0xAB, dtype=torch.uint8, device="cuda")
    scales = torch.full((rows * width // 16,), 0xAB, dtype=torch.uint8, device="cuda")
    expanded = torch.full((rows * width,), -1, dtype=torch.int16, device="cuda")
    xd = dev(torch, x)
    l2c.nvfp4_tensor_scales(ts, xd, rows * width, partials, alpha=alpha, other_decode=other)
    l2c.quantize_nvfp4(codes, scales, xd, ts, rows, width, expanded=expanded)
    torch.cuda.synchronize()
    s, d = oracle.nvfp4_scales(x)
    got = ts.cpu().numpy()
    assert got[0] == s and got[1] == d
    assert alpha.cpu().numpy()[0] == np.float32(d * np.float32(0.75))
    c, sc = oracle.quantize_nvfp4(x, rows, width, s)
    np.testing.assert_array_equal(codes.cpu().numpy(), oracle.pack_e2m1(c))
    np.testing.assert_array_equal(scales.cpu().numpy(), sc)
    exp = expanded.cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(lo.bf16_value(exp).reshape(rows, width), lo.dequantize_nvfp4(c, sc, rows, width))


def test_nvfp4_zero_tensor(torch_gpu, l2c):
    torch = torch_gpu
    f32 = torch.float32
    x = torch.zeros(4 * 64, dtype=f32, device="cuda")
    ts = torch.full((2,), np.nan, dtype=f32, device="cuda")
    partials = torch.empty(l2c.NVFP4_PARTIALS, dtype=f32, device="cuda")
    codes = torch.full((128,), 0xAB, dtype=torch.uint8, device="cuda")
    scales = torch.full((16,), 0xAB, dtype=torch.uint8, device="cuda")
    l2c.nvfp4_tensor_scales(ts, x, x.numel(), partials)
    l2c.quantize_nvfp4(codes, scales, x, ts, 4, 64)
    torch.cuda.synchronize()
    assert ts.cpu().numpy().tolist() == [1.0, 1.0]
    assert not codes.cpu().numpy().any() and not scales.cpu().numpy().any()


def test_to_bf16_x4_exact(torch_gpu, l2c):
    torch = torch_gpu
    x = np.concatenate([inputs("random", 33, 256).ravel(),
                        np.array([1.00390625, 1.01171875, -1.00390625, 3.3e38, 1e-40, -0.0, 0.0, 2.0], np.float32)])
    out = torch.empty(x.size, dtype=torch.int16, device="cuda")
    l2c.to_bf16_x4(out, dev(torch, x), x.size)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16), oracle.bf16(x))


def check_bound(got, A, W, alpha, K):
    exp, bound = lo.logit_bound(A, W, alpha, K)
    bad = np.abs(got.astype(np.float64) - exp) > bound
    assert not bad.any(), f"{bad.sum()} logits outside the bound; first at {np.argwhere(bad)[0]}"


# The last two: many tiles ragged on both edges, and the XCD-ordered tile map.
# (7, 64, 11) and (9, 192, 17): one step and as many steps as the DMA ring has
# stages (the prologue's clamped DMAs).
@pytest.mark.parametrize("batch,cols,rows", [(5, 128, 9), (300, 1024, 260), (1024, 4096, 512), (40, 96, 33),
                                             (257, 2080, 129), (1030, 640, 8000), (1024, 1024, 8192),
                                             (7, 64, 11), (9, 192, 17)])
def test_matmul_bf16_bound(torch_gpu, l2c, batch, cols, rows):
    torch = torch_gpu
    print(f"case matmul_bf16 {batch}x{cols}x{rows}", flush=True)
    rng = np.random.default_rng(batch + cols + rows)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    w = (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    xb, wb = oracle.bf16(x), oracle.bf16(w)
    out = torch.full((batch, rows), np.nan, dtype=torch.float32, device="cuda")
    alpha = torch.tensor([0.375], dtype=torch.float32, device="cuda")
    l2c.matmul_bf16(out, dev(torch, xb.view(np.int16)), dev(torch, wb.view(np.int16)), batch, cols, rows, alpha=alpha)
    torch.cuda.synchronize()
    A = lo.bf16_value(xb).reshape(batch, cols)
    W = lo.bf16_value(wb).reshape(rows, cols)
    check_bound(out.cpu().numpy(), A, W, 0.375, cols)
    # Without alpha, twice: equal bit for bit.
    l2c.matmul_bf16(out, dev(torch, xb.view(np.int16)), dev(torch, wb.view(np.int16)), batch, cols, rows)
    torch.cuda.synchronize()
    first = out.cpu().numpy().copy()
    check_bound(first, A, W, 1.0, cols)
    out.fill_(np.nan)
    l2c.matmul_bf16(out, dev(torch, xb.view(np.int16)), dev(torch, wb.view(np.int16)), batch, cols, rows)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), first.view(np.uint32))


@pytest.mark.parametrize("batch,cols,rows", [(3, 128, 5), (130, 256, 130), (257, 512, 130), (1024, 2048, 1024),
                                             (64, 1024, 128)])
def test_matmul_mxfp6_bound(torch_gpu, l2c, batch, cols, rows):
    """Operands quantized by the oracle and uploaded (the GEMM alone), then by
    the device quantizer (the case's conversion + GEMM)."""
    torch = torch_gpu
    print(f"case matmul_mxfp6 {batch}x{cols}x{rows}", flush=True)
    x = inputs("crafted" if batch >= 8 else "random", batch, cols)
    w = inputs("random", rows, cols) if rows != 128 else lo.fixture(2, cols, rows)[1]
    xc, xs = oracle.quantize_mxfp6(x, batch, cols)
    wc, ws = oracle.quantize_mxfp6(w, rows, cols)
    A = lo.dequantize_mxfp6(xc, xs, batch, cols)
    W = lo.dequantize_mxfp6(wc, ws, rows, cols)
    out = torch.full((batch, rows), np.nan, dtype=torch.float32, device="cuda")
    txc, txs = lo.tile_mxfp6(xc, xs, batch, cols)
    twc, tws = lo.tile_mxfp6(wc, ws, rows, cols)
    l2c.matmul_mxfp6(out, dev(torch, txc), dev(torch, txs), dev(torch, twc), dev(torch, tws), batch, cols, rows)
    torch.cuda.synchronize()
    check_bound(out.cpu().numpy(), A, W, 1.0, cols)
    dxc, dxs = mxfp6_buffers(torch, l2c, batch, cols)
    dwc, dws = mxfp6_buffers(torch, l2c, rows, cols)
    l2c.quantize_mxfp6(dxc, dxs, dev(torch, x), batch, cols)
    l2c.quantize_mxfp6(dwc, dws, dev(torch, w), rows, cols)
    out2 = torch.full((batch, rows), np.nan, dtype=torch.float32, device="cuda")
    l2c.matmul_mxfp6(out2, dxc, dxs, dwc, dws, batch, cols, rows)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out2.cpu().numpy(), out.cpu().numpy())


def test_nvfp4_classifier_bound(torch_gpu, l2c):
    """The NVFP4 case's classifier: device tensor scales, quantizers with bf16
    expansions, l2c_matmul_bf16 with alpha = d_X d_W."""
    torch = torch_gpu
    batch, cols, rows = 100, 1024, 200
    emb, cls = lo.fixture(3, cols, rows)
    x = lo.rmsnorm_double(emb[:batch]).astype(np.float32)
    f32, u8 = torch.float32, torch.uint8
    partials = torch.empty(l2c.NVFP4_PARTIALS, dtype=f32, device="cuda")

    def quant(m, r, alpha=None, other=None):
        ts = torch.empty(2, dtype=f32, device="cuda")
        md = dev(torch, m)
        l2c.nvfp4_tensor_scales(ts, md, m.size, partials, alpha=alpha, other_decode=other)
        codes = torch.empty(m.size // 2, dtype=u8, device="cuda")
        sc = torch.empty(m.size // 16, dtype=u8, device="cuda")
        ex = torch.empty(m.size, dtype=torch.int16, device="cuda")
        l2c.quantize_nvfp4(codes, sc, md, ts, r, cols, expanded=ex)
        return ts, ex

    wts, wex = quant(cls, rows)
    decode_w = wts[1:2]
    alpha = torch.empty(1, dtype=f32, device="cuda")
    _, xex = quant(x, batch, alpha=alpha, other=decode_w)
    out = torch.full((batch, rows), np.nan, dtype=f32, device="cuda")
    l2c.matmul_bf16(out, xex, wex, batch, cols, rows, alpha=alpha)
    torch.cuda.synchronize()
    sx, dx = oracle.nvfp4_scales(x)
    sw, dw = oracle.nvfp4_scales(cls)
    a = np.float32(dx * dw)
    assert alpha.cpu().numpy()[0] == a
    xc, xsc = oracle.quantize_nvfp4(x, batch, cols, sx)
    wc, wsc = oracle.quantize_nvfp4(cls, rows, cols, sw)
    check_bound(out.cpu().numpy(), lo.dequantize_nvfp4(xc, xsc, batch, cols),
                lo.dequantize_nvfp4(wc, wsc, rows, cols), float(a), cols)


@pytest.mark.parametrize("name,rows,width", [("crafted", 130, 256), ("random", 333, 2048), ("random", 3, 16)])
def test_nvfp4_tensor_scales_from_absmax(torch_gpu, l2c, name, rows, width):
    """The tensor scales from a maximum word (as l2c_decoder_rmsnorm_absmax
    leaves it) equal those of the two-pass reduction over x bit for bit, alpha
    included, and the word is cleared afterwards; a zero word gives s = d = 1."""
    torch = torch_gpu
    print(f"case nvfp4_tensor_scales_absmax {name} {rows}x{width}", flush=True)
    x = inputs(name, rows, width)
    f32 = torch.float32
    xd = dev(torch, x)
    other = torch.tensor([0.75], dtype=f32, device="cuda")
    partials = torch.empty(l2c.NVFP4_PARTIALS, dtype=f32, device="cuda")
    ts_a = torch.full((2,), np.nan, dtype=f32, device="cuda")
    ts_b = torch.full((2,), np.nan, dtype=f32, device="cuda")
    alpha_a = torch.full((1,), np.nan, dtype=f32, device="cuda")
    alpha_b = torch.full((1,), np.nan, dtype=f32, device="cuda")
    l2c.nvfp4_tensor_scales(ts_a, xd, rows * width, partials, alpha=alpha_a, other_decode=other)
    word = torch.from_numpy(np.array([np.max(np.abs(x))], np.float32).view(np.int32)).cuda()
    l2c.nvfp4_tensor_scales_absmax(ts_b, word, alpha=alpha_b, other_decode=other)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ts_a.cpu().numpy().view(np.uint32), ts_b.cpu().numpy().view(np.uint32))
    np.testing.assert_array_equal(alpha_a.cpu().numpy().view(np.uint32), alpha_b.cpu().numpy().view(np.uint32))
    assert word.cpu().numpy()[0] == 0
    l2c.nvfp4_tensor_scales_absmax(ts_b, word)
    torch.cuda.synchronize()
    assert ts_b.cpu().numpy().tolist() == [1.0, 1.0]


def test_quantize_nvfp4_rounds_every_value_like_the_oracle(torch_gpu, l2c):
    """The NVFP4 quantizer's E2M1 rounding (the hardware conversion, with its
    negative zeros made +0) against the oracle's nearest-even search: blocks
    [6, x1 .. x15] with tensor scale 1 have block scale 1, so each x's code is
    E2M1(x) itself. The values: every float within 2^16 ulps of each rounding
    threshold and of 6.0 (the top of the range, where codes saturate up to
    6.375), every 16th float in [2^-3, 6.375), and a sample below 2^-3 down
    to the subnormals, with both signs."""
    torch = torch_gpu
    print("case quantize_nvfp4 E2M1 rounding sweep", flush=True)
    bits = []
    for t in (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0):
        b = int(np.float32(t).view(np.uint32))
        bits.append(np.arange(b - 65536, b + 65536, dtype=np.uint32))
    lo_b, hi_b = int(np.float32(0.125).view(np.uint32)), int(np.float32(6.375).view(np.uint32))
    bits.append(np.arange(lo_b, hi_b, 16, dtype=np.uint32))
    bits.append(np.arange(0, lo_b, 4099, dtype=np.uint32))
    mag = np.unique(np.concatenate(bits)).view(np.float32)
    mag = mag[mag < np.float32(6.375)]
    vals = np.concatenate([mag, -mag])
    per = 15
    nblk = (vals.size + per - 1) // per
    x = np.zeros((nblk, 16), dtype=np.float32)
    x[:, 0] = 6.0
    flat = np.zeros(nblk * per, dtype=np.float32)
    flat[:vals.size] = vals
    x[:, 1:] = flat.reshape(nblk, per)
    rows, width = nblk, 16
    f32 = torch.float32
    ts = torch.tensor([1.0, 1.0], dtype=f32, device="cuda")
    codes = torch.full((rows * width // 2,), 0xAB, dtype=torch.uint8, device="cuda")
    scales = torch.full((rows * width // 16,), 0xAB, dtype=torch.uint8, device="cuda")
    expanded = torch.full((rows * width,), -1, dtype=torch.int16, device="cuda")
    l2c.quantize_nvfp4(codes, scales, dev(torch, x.reshape(-1)), ts, rows, width, expanded=expanded)
    torch.cuda.synchronize()
    assert np.all(scales.cpu().numpy() == 0x38)  # UE4M3 1.0: every block scale is 1
    got = lo.unpack_e2m1(codes.cpu().numpy(), rows * width).reshape(rows, width)
    want = oracle.e2m1_encode(x.reshape(-1).astype(np.float64)).reshape(rows, width)
    bad = np.argwhere(got != want)
    assert bad.size == 0, [(float(x[i, j]), int(got[i, j]), int(want[i, j])) for i, j in bad[:8]]
    exp = lo.bf16_value(expanded.cpu().numpy().view(np.uint16)).reshape(rows, width)
    values = np.array([oracle.lib().orc_e2m1_value(c) for c in range(16)], dtype=np.float64)
    np.testing.assert_array_equal(exp, values[want].astype(exp.dtype))
