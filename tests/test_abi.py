"""The C-ABI libraries load and export every symbol include/*.h declares; the
command line rejects bad arguments before touching a GPU. No GPU needed."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "cuda-elastic_amd")


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(l2c_[a-z0-9_]+)\s*\(", text)))


def test_headers_declare_expected():
    import l2c
    assert set(declared("l2c.h")) == set(l2c.KERNEL_SYMBOLS)
    assert set(declared("l2c_harness.h")) == set(l2c.HOST_SYMBOLS)


def test_libraries_export_every_symbol():
    import l2c
    lib = ctypes.CDLL(l2c.LIB_PATH)
    for name in declared("l2c.h"):
        assert hasattr(lib, name), name
    host = ctypes.CDLL(l2c.HOST_LIB_PATH)
    for name in declared("l2c_harness.h"):
        assert hasattr(host, name), name
    lib.l2c_version.restype = ctypes.c_char_p
    assert b"gfx950" in lib.l2c_version()


def test_code_object_is_gfx950():
    import l2c
    out = subprocess.run(["/opt/rocm/llvm/bin/llvm-readelf", "-n", l2c.LIB_PATH],
                         capture_output=True, text=True)
    if out.returncode != 0:
        pytest.skip("llvm-readelf unavailable")
    blob = open(l2c.LIB_PATH, "rb").read()
    assert b"gfx950" in blob


@pytest.mark.parametrize("args,needle", [
    (["bogus"], "Usage"), (["graph", "0"], "Usage"), (["1", "2", "3", "4", "5", "6", "7"], "Usage"),
    (["random=abc"], "bad seed"), (["random="], "bad seed"), (["graph", "-5"], "Usage"),
    (["direct", "auto", "auto"], "Usage"),
])
def test_cli_usage_errors(args, needle):
    import l2c
    proc = subprocess.run([l2c.HARNESS] + args, capture_output=True, text=True, timeout=60)
    assert proc.returncode == 1
    assert needle in proc.stderr
    assert proc.stdout == ""


def test_compare_tool_on_reference_dump(tmp_path, orc):
    """l2c_compare accepts the reference's own dump against itself (bitwise
    identical) and rejects a copy with a product moved past its tolerance, a
    truncated copy and a different header."""
    import l2c
    src = os.path.join(ROOT, "tests", "golden", "ref_dump_random7_2x16x5.bin")
    data = bytearray(open(src, "rb").read())
    a = tmp_path / "a.bin"
    a.write_bytes(data)
    code, out = l2c.compare_dumps([src, str(a)])
    assert code == 0 and "bitwise identical" in out and "PASS" in out
    dump = orc.read_dump(src)
    off = 32 + 4 * 2 * 2 * 16  # first product element
    import numpy as np
    bad = bytearray(data)
    p0 = np.float32(dump["product_reference"][0] + 2.0 * dump["product_tolerance"][0])
    bad[off:off + 4] = p0.tobytes()
    b = tmp_path / "b.bin"
    b.write_bytes(bad)
    code, out = l2c.compare_dumps([src, str(b)])
    assert code == 1 and "FAIL" in out
    c = tmp_path / "c.bin"
    c.write_bytes(data[:-3])
    assert l2c.compare_dumps([src, str(c)])[0] == 1
    hdr = bytearray(data)
    hdr[24] ^= 1  # seed
    d = tmp_path / "d.bin"
    d.write_bytes(hdr)
    code, out = l2c.compare_dumps([src, str(d)])
    assert code == 1 and "header" in out
    assert l2c.compare_dumps([src])[0] == 2


def test_k_bound_rejects_offset_overflow():
    """Contractions whose per-lane byte offsets (row * K * element bytes, in
    int) would pass INT_MAX are refused before anything is launched, so the
    calls return on a machine without a GPU."""
    import l2c
    lib = ctypes.CDLL(l2c.LIB_PATH)
    p = ctypes.c_void_p(1 << 20)  # never dereferenced: the call returns first
    for fn in (lib.l2c_matmul_q, lib.l2c_matmul, lib.l2c_matmul_bf16):
        fn.restype = ctypes.c_int
    big = 1 << 22  # 256 rows x 2^22 bf16 = 2^31 bytes
    for fmt in (0, 1):
        assert lib.l2c_matmul_q(p, p, p, p, fmt, 1, big, 1, None) == 1
        assert lib.l2c_matmul_q(p, p, p, p, fmt, 1, big + 32, 1, None) == 1
    assert lib.l2c_matmul_bf16(p, p, p, None, 1, big, 1, None) == 1
    assert lib.l2c_matmul_bf16(p, p, p, None, 1, big + 32, 1, None) == 1
    assert lib.l2c_matmul(p, p, p, 1, 0x7fffffff - 31, 1, None) == 1


def test_make_fails_on_compile_error(tmp_path):
    """A HIP source that does not compile makes the package build exit
    non-zero and leaves no object behind (no stale object can reach a link)."""
    import shutil
    pkg = tmp_path / "pkg"
    (pkg / "csrc").mkdir(parents=True)
    (tmp_path / "include").mkdir()
    (tmp_path / "include" / "l2c.h").write_text("/* empty */\n")
    shutil.copy(os.path.join(PKG, "Makefile"), pkg / "Makefile")
    (pkg / "csrc" / "broken.hip").write_text("this is not C++;\n")
    proc = subprocess.run(["make", "-C", str(pkg), "_build/broken.o"], capture_output=True, text=True,
                          timeout=300)
    assert proc.returncode != 0
    assert not (pkg / "_build" / "broken.o").exists()
    (pkg / "csrc" / "broken.hip").write_text(
        "#include <hip/hip_runtime.h>\n__global__ void ok_kernel(int *p) { *p = 1; }\n")
    proc = subprocess.run(["make", "-C", str(pkg), "_build/broken.o"], capture_output=True, text=True,
                          timeout=300)
    assert proc.returncode == 0, proc.stderr
    assert (pkg / "_build" / "broken.o").exists()
