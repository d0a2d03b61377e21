"""Quantized path on the GPU: device quantizers bit-exact with the oracle's
brute-force encoders, and the quantized contraction against the oracle's
dequantize-then-fp32 product (relative error 2e-3 of sum |terms|, plus the
Higham-Mary bound of the fp32 accumulation)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def special_values(rng, n):
    """Random normals plus exact e2m1 / e4m3 rounding ties and extremes."""
    v = rng.standard_normal(n).astype(np.float32) * 0.05
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0, 0.0, -0.0, 6.0, 12.0,
                     1e-30, -1e-30, 3e38, -3e38, 1.0000001, 0.9999999], np.float32)
    v[:ties.size] = ties
    return v


def test_to_bf16_exact(torch_gpu, l2c, orc):
    torch = torch_gpu
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.standard_normal(1 << 16).astype(np.float32),
                        rng.integers(0, 2**32, 1 << 16, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    v = np.concatenate([v[np.isfinite(v)],
                        np.array([3.4028235e38, -3.4028235e38, 3.3961e38, 1e-45, -1e-45], np.float32)])
    out = torch.empty(v.size, dtype=torch.int16, device="cuda")
    l2c.to_bf16(out, dev(torch, v), v.size)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16), orc.bf16(v))


@pytest.mark.parametrize("rows,cols", [(4, 64), (33, 1024), (256, 4096)])
def test_quantize_mxfp4_exact(torch_gpu, l2c, orc, rows, cols):
    torch = torch_gpu
    rng = np.random.default_rng(rows)
    W = special_values(rng, rows * cols)
    W[32:64] = 0.0                      # an all-zero block
    W[64:96] *= np.float32(1e-36)       # a block far below 1
    codes = torch.empty(rows * cols // 2, dtype=torch.uint8, device="cuda")
    scales = torch.empty(rows * cols // 32, dtype=torch.uint8, device="cuda")
    l2c.quantize_mxfp4(codes, scales, dev(torch, W), rows, cols)
    torch.cuda.synchronize()
    oc, os_ = orc.quantize_mxfp4(W, rows, cols)
    np.testing.assert_array_equal(scales.cpu().numpy(), os_)
    np.testing.assert_array_equal(codes.cpu().numpy(), orc.pack_e2m1(oc))


@pytest.mark.parametrize("rows,cols", [(4, 64), (33, 1000), (128, 4096)])
def test_quantize_fp8_exact(torch_gpu, l2c, orc, rows, cols):
    torch = torch_gpu
    rng = np.random.default_rng(cols)
    W = special_values(rng, rows * cols)
    W[cols:2 * cols] = 0.0  # an all-zero row: scale 1
    codes = torch.empty(rows * cols, dtype=torch.uint8, device="cuda")
    scales = torch.empty(rows, dtype=torch.float32, device="cuda")
    l2c.quantize_fp8(codes, scales, dev(torch, W), rows, cols)
    torch.cuda.synchronize()
    oc, osc = orc.quantize_fp8(W, rows, cols)
    np.testing.assert_array_equal(scales.cpu().numpy(), osc)
    np.testing.assert_array_equal(codes.cpu().numpy(), oc)


@pytest.mark.parametrize("fmt", [0, 1])
# K % 64 == 0 runs l2c_qgemm_ks.hip ((520, 1088, 1030), (1024, 2048, 1024):
# many tiles, ragged edges and the XCD-ordered tile map; K = 64, 192, 256: one
# step, three, and as many steps as the DMA ring has stages); K % 64 == 32
# runs l2c_qgemm.hip.
@pytest.mark.parametrize("batch,size,rows", [(8, 64, 16), (300, 1024, 200), (256, 4096, 256),
                                             (33, 96, 77), (5, 32, 9), (130, 2080, 140),
                                             (520, 1088, 1030), (1024, 2048, 1024), (3, 192, 5), (9, 256, 17)])
def test_matmul_q(torch_gpu, l2c, orc, fmt, batch, size, rows):
    torch = torch_gpu
    print(f"case matmul_q fmt={fmt} batch={batch} size={size} rows={rows}", flush=True)
    inp = orc.fill("normal", 5, batch, size, rows)
    x = dev(torch, inp.input)
    xbf = torch.empty(batch * size, dtype=torch.int16, device="cuda")
    l2c.to_bf16(xbf, x, batch * size)
    W = dev(torch, inp.matrix)
    if fmt == 0:
        codes = torch.empty(rows * size // 2, dtype=torch.uint8, device="cuda")
        scales = torch.empty(rows * size // 32, dtype=torch.uint8, device="cuda")
        l2c.quantize_mxfp4(codes, scales, W, rows, size)
    else:
        codes = torch.empty(rows * size, dtype=torch.uint8, device="cuda")
        scales = torch.empty(rows, dtype=torch.float32, device="cuda")
        l2c.quantize_fp8(codes, scales, W, rows, size)
    out = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
    l2c.matmul_q(out, xbf, codes, scales, fmt, batch, size, rows)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    ref, mag = orc.qmatmul_ref(fmt, xbf.cpu().numpy().view(np.uint16), codes.cpu().numpy(),
                               scales.cpu().numpy(), size, rows, list(range(batch)), batch)
    err = np.abs(got - ref)
    assert np.all(np.isfinite(got))
    assert np.max(err / np.maximum(mag, 1e-30)) <= 2e-3
    assert np.all(err <= orc.gamma(size) * mag + np.finfo(np.float32).tiny)
    # A second call into a fresh buffer: equal bit for bit (fixed reduction order).
    again = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
    l2c.matmul_q(again, xbf, codes, scales, fmt, batch, size, rows)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(again.cpu().numpy().view(np.uint32), out.cpu().numpy().view(np.uint32))


def extreme_blocks(rng, rows, size):
    """Weights whose 32-value blocks span every magnitude class of the MXFP4
    block scale: zero blocks, blocks below 6 * 2^-126 (scale byte 0, i.e.
    2^-127, whose bf16 expansions are subnormal), and 1e-20 to 1e30. Rows
    r % 8 == 7 hold only the smallest class."""
    W = rng.standard_normal(rows * size).astype(np.float32).reshape(rows, size // 32, 32)
    mags = np.array([0.0, 3e-38, 1e-20, 1.0, 1e20, 1e30], np.float32)
    for r in range(rows):
        for b in range(size // 32):
            W[r, b] *= mags[1] if r % 8 == 7 else mags[(r + b) % mags.size]
    return W.reshape(-1)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("batch,size,rows", [(64, 1024, 96), (40, 96, 72)])
def test_matmul_q_extreme_blocks(torch_gpu, l2c, orc, fmt, batch, size, rows):
    """Scale extremes through the contraction (K % 64 == 0 and == 32 kernels)
    against the exact dequantize-then-accumulate oracle, to the bound of
    test_matmul_q."""
    torch = torch_gpu
    print(f"case matmul_q extremes fmt={fmt} batch={batch} size={size} rows={rows}", flush=True)
    rng = np.random.default_rng(size + rows)
    W = extreme_blocks(rng, rows, size)
    x = rng.standard_normal(batch * size).astype(np.float32)
    xbf = torch.empty(batch * size, dtype=torch.int16, device="cuda")
    l2c.to_bf16(xbf, dev(torch, x), batch * size)
    if fmt == 0:
        codes = torch.empty(rows * size // 2, dtype=torch.uint8, device="cuda")
        scales = torch.empty(rows * size // 32, dtype=torch.uint8, device="cuda")
        l2c.quantize_mxfp4(codes, scales, dev(torch, W), rows, size)
    else:
        codes = torch.empty(rows * size, dtype=torch.uint8, device="cuda")
        scales = torch.empty(rows, dtype=torch.float32, device="cuda")
        l2c.quantize_fp8(codes, scales, dev(torch, W), rows, size)
    out = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
    l2c.matmul_q(out, xbf, codes, scales, fmt, batch, size, rows)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    ref, mag = orc.qmatmul_ref(fmt, xbf.cpu().numpy().view(np.uint16), codes.cpu().numpy(),
                               scales.cpu().numpy(), size, rows, list(range(batch)), batch)
    if fmt == 0:
        assert np.any(scales.cpu().numpy() == 0)  # the 2^-127 scale is exercised
    err = np.abs(got - ref)
    assert np.all(np.isfinite(got))
    bad = err > orc.gamma(size) * mag + np.finfo(np.float32).tiny
    assert not np.any(bad), (np.argwhere(bad.reshape(batch, rows))[:5], got[bad][:5], ref[bad][:5])
