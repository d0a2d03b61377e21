"""Parity of the HIP kernels (through the C ABI) with the CPU oracle.

Bars: rmsnorm and softmax within the reference's tolerances
(llama2c/llama2c_common.h:237-276) and a max relative error of 1e-5; the fp32
products within the Higham-Mary bound of every element
(llama2c_common.h:277-294) and a relative error (|p - ref| / sum|terms|) of
1e-4 * sqrt(size); the naive matrix-vector product bit-exact with the oracle's
sequential fmaf chain.
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROW_SHAPES = [  # (batch, size): aligned, register tiers, unaligned, generic two-pass
    (1, 288), (1, 4096), (8, 768), (64, 1000), (33, 1001), (3, 1), (2, 3), (5, 16384),
    (2, 65536), (2, 65537), (1, 100000),
]


def dev(torch, a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


@pytest.mark.parametrize("batch,size", ROW_SHAPES)
@pytest.mark.parametrize("mode", ["random", "deterministic", "scaled"])
def test_rmsnorm_softmax(torch_gpu, l2c, orc, batch, size, mode):
    torch = torch_gpu
    print(f"case rmsnorm/softmax batch={batch} size={size} mode={mode}", flush=True)
    inp = orc.fill(mode, 7, batch, size, 1)
    x, p, w = dev(torch, inp.input), dev(torch, inp.probabilities), dev(torch, inp.weight)
    out_n = torch.empty_like(x)
    out_s = torch.empty_like(p)
    l2c.rmsnorm(out_n, x, w, size, batch)
    l2c.softmax(out_s, p, size, batch)
    torch.cuda.synchronize()
    n, s = out_n.cpu().numpy(), out_s.cpu().numpy()
    ok, err = orc.check_vectors(mode == "deterministic", inp, n, s, batch, size)
    assert ok, f"reference tolerances violated: {err}"
    assert err[1] <= 1e-5, f"rmsnorm max relative error {err[1]}"
    assert err[3] <= 1e-5, f"softmax max relative error {err[3]}"


def test_unaligned_rows(torch_gpu, l2c, orc):
    """Rows starting one float past a 16-byte boundary take the scalar path."""
    torch = torch_gpu
    batch, size = 4, 4096
    inp = orc.fill("random", 3, batch, size, 1)
    big = torch.zeros(batch * size + 1, dtype=torch.float32, device="cuda")
    big[1:] = dev(torch, inp.input)
    x = big[1:]
    wbig = torch.zeros(size + 1, dtype=torch.float32, device="cuda")
    wbig[1:] = dev(torch, inp.weight)
    obig = torch.zeros(batch * size + 1, dtype=torch.float32, device="cuda")
    l2c.rmsnorm(obig[1:], x, wbig[1:], size, batch)
    pbig = torch.zeros(batch * size + 1, dtype=torch.float32, device="cuda")
    pbig[1:] = dev(torch, inp.probabilities)
    sbig = torch.zeros(batch * size + 1, dtype=torch.float32, device="cuda")
    l2c.softmax(sbig[1:], pbig[1:], size, batch)
    torch.cuda.synchronize()
    ok, err = orc.check_vectors(False, inp, obig[1:].cpu().numpy(), sbig[1:].cpu().numpy(), batch,
                                size)
    assert ok and err[1] <= 1e-5 and err[3] <= 1e-5, err
    assert obig[0].item() == 0.0 and sbig[0].item() == 0.0


def test_softmax_in_place(torch_gpu, l2c, orc):
    torch = torch_gpu
    for batch, size in [(4, 16384), (3, 100000), (5, 1001)]:
        inp = orc.fill("random", 5, batch, size, 1)
        p = dev(torch, inp.probabilities)
        l2c.softmax(p, p, size, batch)
        torch.cuda.synchronize()
        ref = orc.softmax_ref(inp.probabilities, batch, size)
        got = p.cpu().numpy().astype(np.float64)
        assert np.max(np.abs(got - ref) / ref) <= 1e-5


def test_large_logits_range(torch_gpu, l2c, orc):
    """Logits spread over [-80, 80]: exp must stay accurate far from the max."""
    torch = torch_gpu
    batch, size = 2, 4096
    rng = np.random.default_rng(11)
    p = (rng.random(batch * size, dtype=np.float32) * 160 - 80).astype(np.float32)
    dp = dev(torch, p)
    out = torch.empty_like(dp)
    l2c.softmax(out, dp, size, batch)
    torch.cuda.synchronize()
    ref = orc.softmax_ref(p, batch, size)
    got = out.cpu().numpy().astype(np.float64)
    mask = ref > 1e-30
    assert np.max(np.abs(got[mask] - ref[mask]) / ref[mask]) <= 1e-5
    assert np.all(np.isfinite(got)) and np.all(got >= 0)


MATVEC_SHAPES = [(288, 288), (4096, 11008), (768, 2048), (1000, 300), (1001, 77), (8188, 9), (8192, 5),
                 (8196, 9), (16384, 257), (16388, 20), (32768, 33), (4100, 16384), (1, 5), (7, 1)]


@pytest.mark.parametrize("cols,rows", MATVEC_SHAPES)
@pytest.mark.parametrize("variant", [0, 1])
@pytest.mark.parametrize("mode", ["random", "deterministic"])
def test_matvec(torch_gpu, l2c, orc, cols, rows, variant, mode):
    torch = torch_gpu
    print(f"case matvec cols={cols} rows={rows} variant={variant} mode={mode}", flush=True)
    inp = orc.fill(mode, 9, 1, cols, rows)
    x, W = dev(torch, inp.input), dev(torch, inp.matrix)
    out = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    l2c.matvec(out, x, W, cols, rows, variant)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ok, tol, ref, ratio, rel = orc.product_check(mode == "deterministic", False, inp.input,
                                                 inp.matrix, got, 1, cols, rows, [0])
    assert ok, f"tolerance ratio {ratio}"
    assert rel <= 1e-4 * math.sqrt(cols)
    if variant == 0:  # naive: the reference's sequential order, bit for bit
        np.testing.assert_array_equal(got, orc.matvec_fma(inp.input, inp.matrix, cols, rows))


@pytest.mark.parametrize("batch,size,rows", [(1, 288, 288), (8, 768, 2048), (64, 1000, 300),
                                             (33, 1001, 77), (4, 16384, 512), (2, 20000, 40)])
def test_fused(torch_gpu, l2c, orc, batch, size, rows):
    torch = torch_gpu
    inp = orc.fill("random", 2, batch, size, rows)
    x, p, w, M = (dev(torch, a) for a in (inp.input, inp.probabilities, inp.weight, inp.matrix))
    n = torch.full_like(x, float("nan"))
    s = torch.full_like(p, float("nan"))
    prod = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    l2c.fused(n, x, w, s, p, prod, M, size, batch, batch, rows)
    torch.cuda.synchronize()
    ok, err = orc.check_vectors(False, inp, n.cpu().numpy(), s.cpu().numpy(), batch, size)
    assert ok and err[1] <= 1e-5 and err[3] <= 1e-5, err
    ok, tol, ref, ratio, rel = orc.product_check(False, False, inp.input, inp.matrix,
                                                 prod.cpu().numpy(), batch, size, rows, [0])
    assert ok, ratio


def test_fused_partial_items(torch_gpu, l2c, orc):
    """Row counts that differ (leftover rmsnorm or softmax rows) and zero counts."""
    torch = torch_gpu
    size = 512
    inp = orc.fill("random", 4, 6, size, 9)
    x, p, w, M = (dev(torch, a) for a in (inp.input, inp.probabilities, inp.weight, inp.matrix))
    for rr, sr, mr in [(6, 2, 9), (1, 6, 0), (0, 0, 9), (6, 0, 0)]:
        n = torch.full_like(x, float("nan"))
        s = torch.full_like(p, float("nan"))
        prod = torch.full((9,), float("nan"), dtype=torch.float32, device="cuda")
        l2c.fused(n, x, w, s, p, prod, M, size, rr, sr, mr)
        torch.cuda.synchronize()
        nn, ss, pp = n.cpu().numpy(), s.cpu().numpy(), prod.cpu().numpy()
        if rr:
            ref = orc.rmsnorm_ref(inp.input[:rr * size], inp.weight, rr, size)
            err = np.abs(nn[:rr * size] - ref)
            assert np.all(err <= 1e-5 * np.abs(ref) + 1e-30)
        assert np.all(np.isnan(nn[rr * size:]))
        if sr:
            ref = orc.softmax_ref(inp.probabilities[:sr * size], sr, size)
            assert np.max(np.abs(ss[:sr * size] - ref) / ref) <= 1e-5
        assert np.all(np.isnan(ss[sr * size:]))
        if mr:
            ok, *_ = orc.product_check(False, False, inp.input, inp.matrix, pp, 1, size, 9, [0])
            assert ok
        else:
            assert np.all(np.isnan(pp))


@pytest.mark.parametrize("batch,size,rows", [
    (8, 768, 2048), (1, 4096, 11008), (4, 16384, 1024), (1024, 16384, 64), (5, 16384, 7),
    (3, 16388, 50), (2, 8196, 11), (2, 8192, 7), (2, 32768, 64), (2, 65536, 64), (1, 70000, 9), (2, 16385, 10), (33, 1001, 77),
    (3, 1, 5)])
def test_fused_equals_separate_launches(torch_gpu, l2c, orc, batch, size, rows):
    """The fused launch runs the row kernels' and the coalesced product's own code
    in one grid, so its outputs equal the three separate launches' bit for bit:
    every row-kernel lane count (192 to 1024 lanes, 1 to 16 float4 a lane), the
    two-pass and unaligned paths, and both matrix load choices (the 172 MiB
    matrix of 4096 x 11008 is read with ordinary loads)."""
    torch = torch_gpu
    print(f"case fused==separate batch={batch} size={size} rows={rows}", flush=True)
    inp = orc.fill("random", 5, batch, size, rows)
    x, p, w, M = (dev(torch, a) for a in (inp.input, inp.probabilities, inp.weight, inp.matrix))
    outs = [(torch.full_like(x, float("nan")), torch.full_like(p, float("nan")),
             torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")) for _ in range(2)]
    (n0, s0, g0), (n1, s1, g1) = outs
    l2c.fused(n0, x, w, s0, p, g0, M, size, batch, batch, rows)
    l2c.rmsnorm(n1, x, w, size, batch)
    l2c.softmax(s1, p, size, batch)
    l2c.matvec(g1, x, M, size, rows, l2c.MATVEC_COALESCED)
    torch.cuda.synchronize()
    for a, b in ((n0, n1), (s0, s1), (g0, g1)):
        np.testing.assert_array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))
    ok, err = orc.check_vectors(False, inp, n0.cpu().numpy(), s0.cpu().numpy(), batch, size)
    assert ok, err


def test_fused_launch_shape_every_row_size(torch_gpu, l2c):
    """Every row size maps to a fused kernel instance of the row kernels' size,
    and the launch takes one workgroup per rmsnorm and softmax row plus one per
    lanes / 64 matrix rows (lanes / 128 for aligned rows of >= 8192 floats,
    or of >= 4096 floats in a matrix of more than 128 MiB, whose matrix rows
    take a pair of wavefronts)."""
    sizes = list(range(1, 300)) + [767, 768, 1000, 1001, 4095, 4096, 4097, 8192, 8196, 16380, 16384,
                                   16388, 20000, 32768, 32772, 65536, 65537, 70000, 100000]
    for size in sizes:
        grid, block, per_cu = l2c.launch_shape(l2c.OP_FUSED, 3, size, 1000)
        rgrid, rblock, _ = l2c.launch_shape(l2c.OP_RMSNORM, 3, size, 1)
        assert block == rblock, (size, block, rblock)
        per_block = block // 64 // (2 if size % 4 == 0 and size >= 8192 else 1)
        assert grid == 6 + -(-1000 // per_block), (size, grid, block)
        assert per_cu >= 1, size
    for size, rows in [(4096, 8192), (4096, 8193), (4096, 11008), (4092, 11008), (4100, 16384), (6144, 16384),
                       (8188, 4097), (8192, 10)]:
        grid, block, _ = l2c.launch_shape(l2c.OP_FUSED, 3, size, rows)
        pair = size % 4 == 0 and (size >= 8192 or (size >= 4096 and 4 * size * rows > 128 << 20))
        assert grid == 6 + -(-rows // (block // 64 // (2 if pair else 1))), (size, rows, grid, block)


@pytest.mark.parametrize("size", [16384, 16388, 70000])
def test_fused_partial_items_long_rows(torch_gpu, l2c, orc, size):
    """Fused launches with differing row counts on rows of 512 and 576 lanes and
    on the two-pass path: the rows computed equal the separate launches' bit for
    bit and nothing else is written."""
    torch = torch_gpu
    inp = orc.fill("random", 6, 7, size, 9)
    x, p, w, M = (dev(torch, a) for a in (inp.input, inp.probabilities, inp.weight, inp.matrix))
    n1, s1 = torch.empty_like(x), torch.empty_like(p)
    g1 = torch.empty((9,), dtype=torch.float32, device="cuda")
    l2c.rmsnorm(n1, x, w, size, 7)
    l2c.softmax(s1, p, size, 7)
    l2c.matvec(g1, x, M, size, 9, l2c.MATVEC_COALESCED)
    ref = [t.cpu().numpy().view(np.uint32) for t in (n1, s1, g1)]
    for rr, sr, mr in [(5, 2, 9), (1, 6, 0), (0, 0, 9), (7, 0, 0), (3, 3, 1)]:
        print(f"case fused partial size={size} rms={rr} softmax={sr} matmul={mr}", flush=True)
        n = torch.full_like(x, float("nan"))
        s = torch.full_like(p, float("nan"))
        prod = torch.full((9,), float("nan"), dtype=torch.float32, device="cuda")
        l2c.fused(n, x, w, s, p, prod, M, size, rr, sr, mr)
        torch.cuda.synchronize()
        for got, want, k in ((n, ref[0], rr * size), (s, ref[1], sr * size), (prod, ref[2], mr)):
            g = got.cpu().numpy()
            np.testing.assert_array_equal(g[:k].view(np.uint32), want[:k])
            assert np.all(np.isnan(g[k:]))


@pytest.mark.parametrize("batch,size,rows", [(1, 288, 288), (8, 768, 2048), (64, 1000, 300),
                                             (33, 1001, 77), (256, 512, 128), (300, 96, 200),
                                             (512, 2048, 1024), (2, 5, 3), (3, 20, 5),
                                             (130, 4100, 257)])
@pytest.mark.parametrize("mode", ["scaled", "deterministic", "random"])
def test_matmul_batched(torch_gpu, l2c, orc, batch, size, rows, mode):
    torch = torch_gpu
    print(f"case matmul batch={batch} size={size} rows={rows} mode={mode}", flush=True)
    inp = orc.fill(mode, 1, batch, size, rows)
    X, W = dev(torch, inp.input), dev(torch, inp.matrix)
    out = torch.full((batch * rows,), float("nan"), dtype=torch.float32, device="cuda")
    l2c.matmul(out, X, W, batch, size, rows)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ok, tol, ref, ratio, rel = orc.product_check(mode == "deterministic", True, inp.input,
                                                 inp.matrix, got, batch, size, rows,
                                                 list(range(batch)))
    assert ok, f"tolerance ratio {ratio}"
    assert rel <= 1e-4 * math.sqrt(size)


def test_matmul_unaligned_operands(torch_gpu, l2c, orc):
    torch = torch_gpu
    batch, size, rows = 40, 256, 70
    inp = orc.fill("random", 8, batch, size, rows)
    xb = torch.zeros(batch * size + 1, dtype=torch.float32, device="cuda")
    xb[1:] = dev(torch, inp.input)
    out = torch.empty(batch * rows, dtype=torch.float32, device="cuda")
    l2c.matmul(out, xb[1:], dev(torch, inp.matrix), batch, size, rows)
    torch.cuda.synchronize()
    ok, *_ = orc.product_check(False, True, inp.input, inp.matrix, out.cpu().numpy(), batch, size,
                               rows, list(range(batch)))
    assert ok


def test_bad_arguments(torch_gpu, l2c):
    torch = torch_gpu
    x = torch.zeros(16, device="cuda")
    with pytest.raises(l2c.L2CError):
        l2c.rmsnorm(x, x, x, 0, 1)
    with pytest.raises(l2c.L2CError):
        l2c.matvec(x, x, x, 4, 4, variant=7)
    with pytest.raises(l2c.L2CError):
        l2c.matmul_q(x, x, x, x, 0, 1, 30, 1)  # cols % 32 != 0
    # Zero rows is a no-op.
    l2c.rmsnorm(x, x, x, 16, 0)
    l2c.matmul(x, x, x, 0, 16, 1)
