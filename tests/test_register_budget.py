"""Register budget that lets the row kernels run beside the block-scaled
contraction (CPU: compiles the device code only and reads the compiler's
resource report).

In the C5 iteration rmsnorm and softmax (1024 rows of 16384 floats: the
8-float4, 512-lane row kernels) run on their own streams while the MXFP4
contraction on 128 x 256 tiles holds one workgroup of two waves a SIMD on
every CU. A row workgroup adds two waves a SIMD, so the rows overlap the
product only while 2 x VGPRs(product) + 2 x VGPRs(row kernel), each rounded up
to the allocation granule of 8, fit the 512 registers of a SIMD lane. When
they did not (the product at 212 VGPRs), the graph iteration measured
166-168 against 140 us."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "cuda-elastic_amd")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

GRANULE = 8
REGISTERS_PER_LANE = 512
WAVES_PER_SIMD = 2  # both kernels run 512-lane workgroups: two waves on each SIMD


def resource_report(source):
    """{mangled kernel name: VGPRs} from one device-only compile."""
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-c", "-o", os.devnull,
           "-Rpass-analysis=kernel-resource-usage", "-I" + os.path.join(ROOT, "include"), source]
    out = subprocess.run(cmd, cwd=PKG, capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    vgprs, name = {}, None
    for line in out.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"remark:\s+VGPRs: (\d+)", line)
        if m and name:
            vgprs[name] = int(m.group(1))
    return vgprs


def allocated(v):
    return (v + GRANULE - 1) // GRANULE * GRANULE


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not available")
def test_row_kernels_fit_beside_the_wide_block_scaled_contraction():
    product = resource_report(os.path.join(PKG, "csrc", "l2c_scgemm.hip"))
    rows = resource_report(os.path.join(PKG, "csrc", "l2c_rowops.hip"))
    wide = [v for k, v in product.items() if "scaled_gemm_wide_kernel" in k]
    assert len(wide) == 1, sorted(product)
    # The row kernels the library picks for 16384-float rows: 8 float4 a lane,
    # vector loads, exact cover, 512 lanes.
    picked = {k: v for k, v in rows.items()
              if re.search(r"(rmsnorm|softmax)_kernelILi8ELb1ELb1ELi512E", k)}
    assert len(picked) == 2, sorted(rows)
    for name, v in picked.items():
        need = WAVES_PER_SIMD * (allocated(wide[0]) + allocated(v))
        assert need <= REGISTERS_PER_LANE, (name, v, wide[0], need)
