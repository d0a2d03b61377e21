"""Full-size properties of the batched contractions at the C4 / C5 sheet shape
(batch 1024, k 16384, rows 8192), where the oracle would take minutes.

Every output is computed by the same arithmetic wherever its row and column
sit in the tile grid: the k order, the k-slice pairs' sum and the epilogue do
not depend on the tile or the lane. So rotating the batch rows of X rotates
the output's rows, and rotating the rows of W (quantized afresh) rotates its
columns, bit for bit. A tile-position-dependent mistake anywhere in the sheet
fails this: a row clamp, the XCD tile map, or a mixed-up k-slice pair. The
values themselves are checked against the oracle on smaller shapes
(test_kernels_gpu.py, test_quant_gpu.py, test_quant_scaled_gpu.py) and on
sampled rows of this shape through the harness (test_harness_gpu.py)."""
import pytest

pytestmark = pytest.mark.gpu

B, K, R = 1024, 16384, 8192
SHIFT_B, SHIFT_R = 300, 1000  # not multiples of any tile edge


def _operands(torch):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(20261202)
    X = torch.randn(B, K, generator=gen, device="cuda", dtype=torch.float32)
    W = torch.randn(R, K, generator=gen, device="cuda", dtype=torch.float32) / 128.0  # N(0, 1/K)
    return X, W


def _weights(torch, l2c, fmt, W):
    if fmt == 0:
        codes = torch.empty(R * K // 2, dtype=torch.uint8, device="cuda")
        scales = torch.empty(R * K // 32, dtype=torch.uint8, device="cuda")
        l2c.quantize_mxfp4(codes, scales, W, R, K)
    else:
        codes = torch.empty(R * K, dtype=torch.uint8, device="cuda")
        scales = torch.empty(R, dtype=torch.float32, device="cuda")
        l2c.quantize_fp8(codes, scales, W, R, K)
    return codes, scales


def _product(torch, l2c, kind, X, W):
    out = torch.full((B * R,), float("nan"), dtype=torch.float32, device="cuda")
    if kind == "fp32":
        l2c.matmul(out, X, W, B, K, R)
    else:
        fmt = 0 if kind.startswith("mxfp4") else 1
        xbf = torch.empty(B * K, dtype=torch.int16, device="cuda")
        l2c.to_bf16(xbf, X, B * K)
        codes, scales = _weights(torch, l2c, fmt, W)
        if kind.endswith("s"):
            ws = torch.empty(l2c.mxfp8_workspace_bytes(B, K), dtype=torch.uint8, device="cuda")
            l2c.matmul_qs(out, xbf, codes, scales, fmt, B, K, R, ws)
        else:
            l2c.matmul_q(out, xbf, codes, scales, fmt, B, K, R)
    torch.cuda.synchronize()
    return out.view(B, R)


def _bits(torch, t):
    return t.contiguous().view(torch.int32)


@pytest.mark.parametrize("kind", ["fp32", "mxfp4", "fp8", "mxfp4s", "fp8s"])
def test_rotations_commute_with_the_product(torch_gpu, l2c, kind):
    torch = torch_gpu
    print(f"case full-size rotations {kind} {B}x{K}x{R}", flush=True)
    X, W = _operands(torch)
    base = _product(torch, l2c, kind, X, W)
    assert bool(torch.isfinite(base).all())
    assert float(base.abs().max()) > 0.0

    rx = _product(torch, l2c, kind, torch.roll(X, SHIFT_B, dims=0).contiguous(), W)
    assert torch.equal(_bits(torch, rx), _bits(torch, torch.roll(base, SHIFT_B, dims=0)))
    del rx

    rw = _product(torch, l2c, kind, X, torch.roll(W, SHIFT_R, dims=0).contiguous())
    assert torch.equal(_bits(torch, rw), _bits(torch, torch.roll(base, SHIFT_R, dims=1)))
