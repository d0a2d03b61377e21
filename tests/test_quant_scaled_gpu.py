"""The block-scaled quantized-weight path on the GPU (l2c_matmul_qs): the
device MXFP8 activation quantizer bit-exact with the oracle, and the
contraction on the scaled matrix cores against the oracle's dequantize-both,
double-accumulate reference within the implementation-check bound of
experiments/blackwell/lowprec/spec.json:55-62 (gamma_K with u = 2^-23 times
sum |terms|, plus u |reference|). The error against the bf16-activation
reference (what activation quantization costs) is bounded by 2^-4 of sum
|terms| per output by construction and reported."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

U = 2.0 ** -23


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def untile_scales(tiled, batch, cols):
    """[cols/128][Bp][4] scale tiles to row-major [batch][cols/32]."""
    bp = (batch + 3) // 4 * 4
    t = tiled.reshape(cols // 128, bp, 4)
    return np.ascontiguousarray(t.transpose(1, 0, 2).reshape(bp, cols // 32)[:batch]), t[:, batch:, :]


def weights(torch, l2c, fmt, W, rows, cols):
    if fmt == 0:
        codes = torch.empty(rows * cols // 2, dtype=torch.uint8, device="cuda")
        scales = torch.empty(rows * cols // 32, dtype=torch.uint8, device="cuda")
        l2c.quantize_mxfp4(codes, scales, dev(torch, W), rows, cols)
    else:
        codes = torch.empty(rows * cols, dtype=torch.uint8, device="cuda")
        scales = torch.empty(rows, dtype=torch.float32, device="cuda")
        l2c.quantize_fp8(codes, scales, dev(torch, W), rows, cols)
    return codes, scales


def bf16_activations(torch, l2c, x):
    xbf = torch.empty(x.size, dtype=torch.int16, device="cuda")
    l2c.to_bf16(xbf, dev(torch, x), x.size)
    return xbf


@pytest.mark.parametrize("batch,cols", [(4, 128), (33, 1024), (256, 4096), (7, 384)])
def test_quantize_mxfp8_exact(torch_gpu, l2c, orc, batch, cols):
    torch = torch_gpu
    print(f"case quantize_mxfp8 {batch}x{cols}", flush=True)
    rng = np.random.default_rng(batch + cols)
    x = (rng.standard_normal(batch * cols) * 0.7).astype(np.float32)
    ties = np.array([448.0, 480.0, 464.0, 0.0, -0.0, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -11, 1e30, -1e-30,
                     17.0, 18.0, 19.0, 255.0, 256.0, 257.0], np.float32)
    x[:ties.size] = ties
    x[32:64] = 0.0                       # a zero block
    x[64:96] *= np.float32(1e-36)        # a block of bf16 subnormals and tiny normals
    x[96:128] *= np.float32(1e35)        # a block near the top of the range
    xbf = bf16_activations(torch, l2c, x)
    ws = torch.full((l2c.mxfp8_workspace_bytes(batch, cols),), 0xA5, dtype=torch.uint8, device="cuda")
    l2c.quantize_mxfp8(ws, xbf, batch, cols)
    torch.cuda.synchronize()
    codes, tiled = l2c.mxfp8_views(ws, batch, cols)
    oc, osc = orc.quantize_mxfp8(xbf.cpu().numpy().view(np.uint16), batch, cols)
    np.testing.assert_array_equal(codes.cpu().numpy(), oc)
    got_scales, padding = untile_scales(tiled.cpu().numpy(), batch, cols)
    np.testing.assert_array_equal(got_scales.reshape(-1), osc)
    assert np.all(padding == 0)


def check_qs(torch, l2c, orc, fmt, batch, size, rows, x, W, label):
    print(f"case matmul_qs {label} fmt={fmt} {batch}x{size}x{rows}", flush=True)
    xbf = bf16_activations(torch, l2c, x)
    codes, scales = weights(torch, l2c, fmt, W, rows, size)
    ws = torch.empty(l2c.mxfp8_workspace_bytes(batch, size), dtype=torch.uint8, device="cuda")
    out = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
    l2c.matmul_qs(out, xbf, codes, scales, fmt, batch, size, rows, ws)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    xb = xbf.cpu().numpy().view(np.uint16)
    oc, osc = orc.quantize_mxfp8(xb, batch, size)
    dc, dt = l2c.mxfp8_views(ws, batch, size)
    np.testing.assert_array_equal(dc.cpu().numpy(), oc)  # the activations the product used
    np.testing.assert_array_equal(untile_scales(dt.cpu().numpy(), batch, size)[0].reshape(-1), osc)
    vec = list(range(batch))
    wc, wsc = codes.cpu().numpy(), scales.cpu().numpy()
    ref, mag = orc.qsmatmul_ref(fmt, oc, osc, wc, wsc, size, rows, vec, batch)
    assert np.all(np.isfinite(got))
    err = np.abs(got - ref)
    gamma = size * U / (1 - size * U)
    bad = err > gamma * mag + U * np.abs(ref) + 1e-30
    assert not np.any(bad), (np.argwhere(bad.reshape(batch, rows))[:5], got[bad][:5], ref[bad][:5])
    # Against the bf16-activation reference: E4M3 keeps 4 significant bits, so
    # each term moves by at most 2^-4 of itself.
    ref16, mag16 = orc.qmatmul_ref(fmt, xb, wc, wsc, size, rows, vec, batch)
    rel16 = np.max(np.abs(got - ref16) / np.maximum(mag16, 1e-30))
    print(f"  max |p - ref_bf16| / sum|terms| = {rel16:.3e}; max err / bound = "
          f"{np.max(err / (gamma * mag + U * np.abs(ref) + 1e-30)):.3f}", flush=True)
    assert rel16 <= 2.0 ** -4 * (1 + 1e-6)
    # Deterministic: a second call gives the same bits.
    again = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
    l2c.matmul_qs(again, xbf, codes, scales, fmt, batch, size, rows, ws)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(again.cpu().numpy().view(np.uint32), out.cpu().numpy().view(np.uint32))
    return rel16


@pytest.mark.parametrize("fmt", [0, 1])
# One k-step (128), two, three (as many as the DMA ring has stages), ragged
# tiles on both axes, batches that are not a multiple of 4 (padded scale
# rows), and grids of many tiles with the XCD-ordered tile map. MXFP4 weights
# with size % 512 == 0 take the 128 x 256 tile with its four-step scale ring:
# one scale group (512), exactly as many groups as ring slots (1536), ragged
# tiles on both axes past one tile (600 and 513 rows, 130 and 257 vectors).
@pytest.mark.parametrize("batch,size,rows", [(8, 128, 16), (5, 128, 9), (3, 256, 5), (9, 384, 17),
                                             (300, 1024, 200), (33, 384, 77), (256, 4096, 256),
                                             (520, 1152, 1030), (1024, 2048, 1024), (5, 512, 9),
                                             (130, 1536, 600), (257, 2560, 513)])
def test_matmul_qs(torch_gpu, l2c, orc, fmt, batch, size, rows):
    inp = orc.fill("normal", 6, batch, size, rows)
    check_qs(torch_gpu, l2c, orc, fmt, batch, size, rows, inp.input, inp.matrix, "normal")


@pytest.mark.parametrize("fmt", [0, 1])
def test_matmul_qs_scale_spread(torch_gpu, l2c, orc, fmt):
    """Blocks of activations and weights whose magnitudes differ by up to
    2^+-12 within a row, zero blocks and tiny blocks: every scale byte class
    the realistic operands reach, to the same bound."""
    batch, size, rows = 64, 1024, 96
    rng = np.random.default_rng(60 + fmt)
    x = rng.standard_normal((batch, size // 32, 32))
    x *= np.exp2(rng.integers(-12, 13, (batch, size // 32, 1)))
    x[::7, 3] = 0.0
    W = rng.standard_normal((rows, size // 32, 32))
    W *= np.exp2(rng.integers(-12, 13, (rows, size // 32, 1)))
    W[::5, 6] = 0.0
    check_qs(torch_gpu, l2c, orc, fmt, batch, size, rows, x.astype(np.float32).reshape(-1),
             W.astype(np.float32).reshape(-1), "spread")


def test_matmul_qs_rejects_bad_arguments(torch_gpu, l2c):
    """cols % 128 != 0, a short workspace and a misaligned scale pointer are
    refused before anything is launched."""
    torch = torch_gpu
    lib = l2c.load()
    buf = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    p = buf.data_ptr()
    s = torch.cuda.current_stream().cuda_stream
    need = l2c.mxfp8_workspace_bytes(64, 1024)
    assert l2c.mxfp8_workspace_bytes(64, 1000) == 0
    assert lib.l2c_matmul_qs(p, p, p, p, 0, 64, 1000, 64, p, 1 << 20, s) == 1
    assert lib.l2c_matmul_qs(p, p, p, p, 0, 64, 1024, 64, p, need - 1, s) == 1
    assert lib.l2c_matmul_qs(p, p, p, p + 2, 0, 64, 1024, 64, p, need, s) == 1
    assert lib.l2c_matmul_qs(p, p, p, p, 2, 64, 1024, 64, p, need, s) == 1


@pytest.mark.parametrize("shift", [0, 10])
def test_quantize_mxfp8_every_bf16_value(torch_gpu, l2c, orc, shift):
    """Every bf16 value of magnitude <= 448 (both signs, subnormals, zeros),
    31 to a block beside a 448 * 2^shift that fixes the block's scale, times
    2^shift: the device codes (the hardware E4M3 conversion) equal the
    oracle's nearest-even encoder at every one, ties and -0 included."""
    torch = torch_gpu
    mags = np.arange(0, 0x43E1, dtype=np.uint32)            # bf16 patterns 0 .. 448
    vals = np.concatenate([mags, mags | 0x8000]).astype(np.uint32) << 16
    v = vals.view(np.float32).astype(np.float64) * 2.0 ** shift
    per = 31
    nblk = -(-v.size // per)
    blocks = np.zeros((nblk, 32))
    blocks[:, 0] = 448.0 * 2.0 ** shift
    flat = np.zeros(nblk * per)
    flat[:v.size] = v
    blocks[:, 1:] = flat.reshape(nblk, per)
    x = blocks.reshape(-1)
    cols = 128 * 64
    rows = -(-x.size // cols)
    x = np.concatenate([x, np.zeros(rows * cols - x.size)]).astype(np.float32)
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal((xb.astype(np.uint32) << 16).view(np.float32), x)  # exact in bf16
    print(f"case quantize_mxfp8 every bf16 value, shift {shift}, {rows}x{cols}", flush=True)
    xbf = torch.from_numpy(xb.view(np.int16)).cuda()
    ws = torch.empty(l2c.mxfp8_workspace_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    l2c.quantize_mxfp8(ws, xbf, rows, cols)
    torch.cuda.synchronize()
    codes, tiled = l2c.mxfp8_views(ws, rows, cols)
    oc, osc = orc.quantize_mxfp8(xb, rows, cols)
    assert np.all(osc[:nblk] == 127 + shift)  # each block's 448 * 2^shift sets its scale
    got = codes.cpu().numpy()
    bad = np.flatnonzero(got != oc)
    assert bad.size == 0, (bad[:8], x[bad[:8]], got[bad[:8]], oc[bad[:8]])
    np.testing.assert_array_equal(untile_scales(tiled.cpu().numpy(), rows, cols)[0].reshape(-1), osc)


def test_launch_shape_names_the_tile_the_product_runs(torch_gpu, l2c):
    """l2c_launch_shape reports the 128 x 256 grid for MXFP4 products with
    cols % 512 == 0 and the 256 x 128 grid otherwise (and for fp8)."""
    assert l2c.launch_shape(l2c.OP_MATMUL_QS, 300, 1024, 600, l2c.Q_MXFP4)[:2] == (3 * 3, 512)
    assert l2c.launch_shape(l2c.OP_MATMUL_QS, 300, 1152, 600, l2c.Q_MXFP4)[:2] == (2 * 5, 512)
    assert l2c.launch_shape(l2c.OP_MATMUL_QS, 300, 1024, 600, l2c.Q_FP8)[:2] == (2 * 5, 512)
    assert l2c.launch_shape(l2c.OP_MATMUL_QS, 1024, 16384, 8192, l2c.Q_MXFP4)[:2] == (256, 512)
    assert l2c.launch_shape(l2c.OP_MATMUL_QS, 1024, 16384, 8192, l2c.Q_MXFP4)[2] == 1


@pytest.mark.parametrize("batch,cols,rows", [(1, 512, 1), (257, 512, 257), (130, 1536, 600), (64, 2048, 4096),
                                             (1024, 16384, 1024)])
def test_wide_and_narrow_mxfp4_tiles_agree_bit_for_bit(torch_gpu, l2c, orc, batch, cols, rows):
    """MXFP4 products with cols % 512 == 0 run on the 128 x 256 tile when the
    scale array is 16-byte aligned and on the 256 x 128 tile otherwise; every
    output accumulates the same MFMA sequence in both, so the two agree bit for
    bit. The second call reads a copy of the scales 4 bytes past a 16-byte
    boundary (4-byte aligned, as the C ABI requires)."""
    torch = torch_gpu
    print(f"case wide/narrow mxfp4s {batch}x{cols}x{rows}", flush=True)
    inp = orc.fill("normal", 9, batch, cols, rows)
    codes, scales = weights(torch, l2c, 0, inp.matrix, rows, cols)
    xbf = bf16_activations(torch, l2c, inp.input)
    ws = torch.empty(l2c.mxfp8_workspace_bytes(batch, cols), dtype=torch.uint8, device="cuda")
    wide = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
    narrow = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
    holder = torch.zeros(scales.numel() + 16, dtype=torch.uint8, device="cuda")
    shifted = holder[4:4 + scales.numel()]
    shifted.copy_(scales)
    assert scales.data_ptr() % 16 == 0 and shifted.data_ptr() % 16 == 4
    l2c.matmul_qs(wide, xbf, codes, scales, 0, batch, cols, rows, ws)
    l2c.matmul_qs(narrow, xbf, codes, shifted, 0, batch, cols, rows, ws)
    torch.cuda.synchronize()
    w, n = wide.cpu().numpy(), narrow.cpu().numpy()
    assert np.isfinite(w).all()
    np.testing.assert_array_equal(w.view(np.uint32), n.view(np.uint32))


def test_wide_and_narrow_mxfp4_tiles_agree_on_random_shapes(torch_gpu, l2c):
    """Seeded random shapes (ragged batch and rows, K from 512 to 4096) through
    both MXFP4 tiles: bit-identical outputs, every one finite. Operands are
    random device data quantized by the library, so no oracle is involved; the
    oracle comparison of the narrow tile is in the tests above."""
    torch = torch_gpu
    rng = np.random.default_rng(2026)
    for case in range(12):
        batch = int(rng.integers(1, 700))
        rows = int(rng.integers(1, 1500))
        cols = 512 * int(rng.integers(1, 9))
        print(f"case random wide/narrow mxfp4s #{case} {batch}x{cols}x{rows}", flush=True)
        g = torch.Generator(device="cuda").manual_seed(case)
        x = torch.randn(batch * cols, device="cuda", generator=g) * float(rng.uniform(0.1, 4.0))
        w = torch.randn(rows * cols, device="cuda", generator=g) * float(rng.uniform(1e-3, 1.0))
        codes = torch.empty(rows * cols // 2, dtype=torch.uint8, device="cuda")
        scales = torch.empty(rows * cols // 32, dtype=torch.uint8, device="cuda")
        l2c.quantize_mxfp4(codes, scales, w, rows, cols)
        xbf = torch.empty(batch * cols, dtype=torch.int16, device="cuda")
        l2c.to_bf16(xbf, x, batch * cols)
        ws = torch.empty(l2c.mxfp8_workspace_bytes(batch, cols), dtype=torch.uint8, device="cuda")
        wide = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
        narrow = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
        holder = torch.zeros(scales.numel() + 16, dtype=torch.uint8, device="cuda")
        shifted = holder[4:4 + scales.numel()]
        shifted.copy_(scales)
        l2c.matmul_qs(wide, xbf, codes, scales, 0, batch, cols, rows, ws)
        l2c.matmul_qs(narrow, xbf, codes, shifted, 0, batch, cols, rows, ws)
        torch.cuda.synchronize()
        wn, nn = wide.cpu().numpy(), narrow.cpu().numpy()
        assert np.isfinite(wn).all(), case
        np.testing.assert_array_equal(wn.view(np.uint32), nn.view(np.uint32))
