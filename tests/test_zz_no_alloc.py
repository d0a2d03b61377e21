"""The allocation-free block-scaled product (l2c_matmul_qs_static) against the
workspace form (l2c_matmul_qs) through the C ABI: equal bit for bit on two
calls in a row (the second with a smaller input, so stale scratch contents
from the first call must not leak into it), no device memory taken by the
calls, and shapes beyond the fixed scratch refused before any launch."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def operands(torch, l2c, orc, fmt, batch, size, rows, seed):
    inp = orc.fill("normal", seed, batch, size, rows)
    x = torch.from_numpy(inp.input).cuda()
    xbf = torch.empty(batch * size, dtype=torch.int16, device="cuda")
    l2c.to_bf16(xbf, x, batch * size)
    W = torch.from_numpy(inp.matrix).cuda()
    if fmt == 0:
        codes = torch.empty(rows * size // 2, dtype=torch.uint8, device="cuda")
        scales = torch.empty(rows * size // 32, dtype=torch.uint8, device="cuda")
        l2c.quantize_mxfp4(codes, scales, W, rows, size)
    else:
        codes = torch.empty(rows * size, dtype=torch.uint8, device="cuda")
        scales = torch.empty(rows, dtype=torch.float32, device="cuda")
        l2c.quantize_fp8(codes, scales, W, rows, size)
    return xbf, codes, scales


def free_bytes():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


@pytest.mark.parametrize("fmt", [0, 1])
def test_static_scratch_matches_workspace_form(torch_gpu, l2c, orc, fmt):
    torch = torch_gpu
    lib = l2c.load()
    stream = torch.cuda.current_stream().cuda_stream
    # The benchmark shape first, then a smaller, ragged one.
    for batch, size, rows in ((1024, 16384, 1024), (96, 1152, 200)):
        print(f"case qs_static fmt={fmt} {batch}x{size}x{rows}", flush=True)
        xbf, codes, scales = operands(torch, l2c, orc, fmt, batch, size, rows, seed=batch)
        ws = torch.empty(l2c.mxfp8_workspace_bytes(batch, size), dtype=torch.uint8, device="cuda")
        want = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
        got = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
        l2c.matmul_qs(want, xbf, codes, scales, fmt, batch, size, rows, ws)
        torch.cuda.synchronize()
        before = free_bytes()
        rc = lib.l2c_matmul_qs_static(got.data_ptr(), xbf.data_ptr(), codes.data_ptr(), scales.data_ptr(), fmt,
                                      batch, size, rows, stream)
        torch.cuda.synchronize()
        assert rc == 0, l2c.load().l2c_strerror(rc)
        assert free_bytes() == before  # the call took no device memory
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32))


def test_static_scratch_refuses_oversized_shapes(torch_gpu, l2c):
    torch = torch_gpu
    lib = l2c.load()
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    p = buf.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    cols = 16384
    fits = max(b for b in range(1, 2048) if l2c.mxfp8_workspace_bytes(b, cols) <= l2c.QS_STATIC_SCRATCH_BYTES)
    too_many = fits + 1
    assert l2c.mxfp8_workspace_bytes(too_many, cols) > l2c.QS_STATIC_SCRATCH_BYTES
    assert lib.l2c_matmul_qs_static(p, p, p, p, 0, too_many, cols, 8, stream) == 1
    assert lib.l2c_matmul_qs_static(p, p, p, p, 0, 8, 1000, 8, stream) == 1  # cols % 128 != 0
    assert lib.l2c_matmul_qs_static(p, p, p, p, 0, 0, cols, 8, stream) == 0  # nothing to do
