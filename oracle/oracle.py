"""numpy wrappers of the test oracle (liboracle.so) and of the reference's own
host code built as oracle/_ref/libl2c_ref.so.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product never imports it.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libl2c_ref.so")

MODES = {"deterministic": 0, "random": 1, "scaled": 2, "normal": 3}

_orc = None
_ref = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_c = ctypes


def build() -> None:
    import subprocess
    subprocess.run(["make", "-C", HERE], check=True)


def lib():
    global _orc
    if _orc is not None:
        return _orc
    if not os.path.exists(ORACLE_PATH):
        raise FileNotFoundError(f"{ORACLE_PATH} is not built (make -C oracle)")
    L = ctypes.CDLL(ORACLE_PATH)
    u64, i, sz, d, f = _c.c_uint64, _c.c_int, _c.c_size_t, _c.c_double, _c.c_float
    L.orc_uniform.argtypes, L.orc_uniform.restype = [u64, u64, u64], f
    L.orc_normal.argtypes, L.orc_normal.restype = [u64, u64, u64], f
    L.orc_uniform_array.argtypes = [u64, u64, u64, sz, _f32p]
    L.orc_normal_array.argtypes = [u64, u64, u64, sz, _f32p]
    L.orc_fill.argtypes = [i, u64, i, i, i, _f32p, _f32p, _f32p, _f32p]
    L.orc_gamma.argtypes, L.orc_gamma.restype = [i], d
    L.orc_rmsnorm_ref.argtypes = [_f32p, _f32p, i, i, f, _f64p]
    L.orc_softmax_ref.argtypes = [_f32p, i, i, _f64p]
    L.orc_check_vectors.argtypes = [i, _f32p, _f32p, _f32p, _f32p, _f32p, i, i, _f64p]
    L.orc_check_vectors.restype = i
    L.orc_product_check.argtypes = [i, i, _f32p, _f32p, _f32p, i, i, i, _i32p, i, _f32p, _f64p,
                                    _c.POINTER(d), _c.POINTER(d)]
    L.orc_product_check.restype = i
    L.orc_iteration_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, i, i, i, i, i, _f32p, _f32p, _f32p]
    L.orc_iteration_f32_mt.argtypes = [_f32p, _f32p, _f32p, _f32p, i, i, i, i, i, _f32p, _f32p, _f32p, i]
    L.orc_matvec_fma.argtypes = [_f32p, _f32p, i, i, _f32p]
    L.orc_e2m1_value.argtypes, L.orc_e2m1_value.restype = [_c.c_uint], d
    L.orc_ue4m3_value.argtypes, L.orc_ue4m3_value.restype = [_c.c_uint], d
    L.orc_e2m1_encode_array.argtypes = [_f64p, sz, _u8p]
    L.orc_ue4m3_encode_array.argtypes = [_f64p, sz, _u8p]
    L.orc_bf16_array.argtypes = [_f32p, sz, _u16p]
    L.orc_mxfp4_exponent_array.argtypes = [_f32p, sz, _i32p]
    L.orc_quantize_mxfp4.argtypes = [_f32p, i, i, _u8p, _u8p]
    L.orc_quantize_fp8.argtypes = [_f32p, i, i, _u8p, _f32p]
    L.orc_qmatmul_ref.argtypes = [i, _u16p, _u8p, _c.c_void_p, i, i, _i32p, i, _f64p, _f64p]
    L.orc_mxfp8_exponent.argtypes, L.orc_mxfp8_exponent.restype = [f], i
    L.orc_quantize_mxfp8.argtypes = [_u16p, i, i, _u8p, _u8p]
    L.orc_qsmatmul_ref.argtypes = [i, _u8p, _u8p, _u8p, _c.c_void_p, i, i, _i32p, i, _f64p, _f64p]
    L.orc_e3m2_value.argtypes, L.orc_e3m2_value.restype = [_c.c_uint], d
    L.orc_e3m2_encode_array.argtypes = [_f64p, sz, _u8p]
    L.orc_mxfp6_exponent.argtypes, L.orc_mxfp6_exponent.restype = [f], i
    L.orc_quantize_mxfp6.argtypes = [_f32p, i, i, _u8p, _u8p]
    L.orc_quantize_nvfp4.argtypes = [_f32p, i, i, f, _u8p, _u8p]
    L.orc_nvfp4_encode_scale.argtypes, L.orc_nvfp4_encode_scale.restype = [f], f
    L.orc_nvfp4_decode_scale.argtypes, L.orc_nvfp4_decode_scale.restype = [f], f
    L.orc_pack_e3m2.argtypes = [_u8p, _c.c_longlong, _u8p]
    _orc = L
    return L


def ref():
    """The reference's own host code, or None when it was not built."""
    global _ref
    if _ref is not None:
        return _ref
    if not os.path.exists(REF_PATH):
        return None
    R = ctypes.CDLL(REF_PATH)
    u64, i, sz, d, f = _c.c_uint64, _c.c_int, _c.c_size_t, _c.c_double, _c.c_float
    R.ref_uniform.argtypes, R.ref_uniform.restype = [u64, u64, u64], f
    R.ref_uniform_array.argtypes = [u64, u64, u64, sz, _f32p]
    R.ref_gamma.argtypes, R.ref_gamma.restype = [i], d
    R.ref_fill.argtypes = [i, u64, i, i, i, _f32p, _f32p, _f32p, _f32p]
    R.ref_validate_all.argtypes = [i, u64, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, i, i,
                                   i, _f32p, _f64p]
    R.ref_validate_all.restype = i
    R.ref_write_dump.argtypes = [_c.c_char_p, i, u64, i, i, i, _f32p, _f32p, _f32p, _f32p, _f64p]
    R.ref_write_dump.restype = i
    R.ref_encode_array.argtypes = [i, _f64p, sz, _u8p]
    R.ref_to_bf16_array.argtypes = [_f32p, sz, _u16p]
    R.ref_normals_stream1.argtypes = [i, _c.c_longlong, _f32p]
    R.ref_quantize_mxfp6.argtypes = [_f32p, i, i, _u8p, _u8p]
    R.ref_quantize_nvfp4.argtypes = [_f32p, i, i, f, _u8p, _u8p]
    R.ref_nvfp4_encode_scale.argtypes, R.ref_nvfp4_encode_scale.restype = [f], f
    R.ref_nvfp4_decode_scale.argtypes, R.ref_nvfp4_decode_scale.restype = [f], f
    R.ref_unpack_e3m2.argtypes, R.ref_unpack_e3m2.restype = [_u8p, _c.c_longlong], _c.c_uint
    R.ref_unpack_e2m1.argtypes, R.ref_unpack_e2m1.restype = [_u8p, _c.c_longlong], _c.c_uint
    _ref = R
    return R


# ---------------------------------------------------------------------------

class Inputs:
    def __init__(self, input, probabilities, weight, matrix):
        self.input, self.probabilities, self.weight, self.matrix = input, probabilities, weight, matrix


def fill(mode, seed, batch, size, rows) -> Inputs:
    m = MODES[mode] if isinstance(mode, str) else mode
    x = np.empty(batch * size, np.float32)
    p = np.empty(batch * size, np.float32)
    w = np.empty(size, np.float32)
    M = np.empty(rows * size, np.float32)
    lib().orc_fill(m, seed, batch, size, rows, x, p, w, M)
    return Inputs(x, p, w, M)


def uniform(seed, stream, start, n):
    out = np.empty(n, np.float32)
    lib().orc_uniform_array(seed, stream, start, n, out)
    return out


def normal(seed, stream, start, n):
    out = np.empty(n, np.float32)
    lib().orc_normal_array(seed, stream, start, n, out)
    return out


def gamma(n):
    return lib().orc_gamma(n)


def rmsnorm_ref(x, w, batch, size, eps=1.0e-5):
    out = np.empty(batch * size, np.float64)
    lib().orc_rmsnorm_ref(np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32),
                          batch, size, eps, out)
    return out


def softmax_ref(p, batch, size):
    out = np.empty(batch * size, np.float64)
    lib().orc_softmax_ref(np.ascontiguousarray(p, np.float32), batch, size, out)
    return out


def check_vectors(deterministic, inputs: Inputs, normalized, softmax, batch, size):
    err = np.zeros(4, np.float64)
    ok = lib().orc_check_vectors(int(deterministic), inputs.input, inputs.probabilities,
                                 inputs.weight, np.ascontiguousarray(normalized, np.float32),
                                 np.ascontiguousarray(softmax, np.float32), batch, size, err)
    return bool(ok), err


def product_check(deterministic, batched, x, W, product, batch, size, rows, vectors):
    vec = np.ascontiguousarray(vectors, np.int32)
    n = batch * rows if batched else rows
    tol = np.full(n, np.nan, np.float32)
    refv = np.full(n, np.nan, np.float64)
    ratio, rel = ctypes.c_double(), ctypes.c_double()
    ok = lib().orc_product_check(int(deterministic), int(batched), np.ascontiguousarray(x, np.float32),
                                 np.ascontiguousarray(W, np.float32),
                                 np.ascontiguousarray(product, np.float32), batch, size, rows, vec,
                                 len(vec), tol, refv, ctypes.byref(ratio), ctypes.byref(rel))
    return bool(ok), tol, refv, ratio.value, rel.value


def iteration_f32(inputs: Inputs, batch, size, rows, batched=False, vectors=None):
    nv = (vectors if vectors is not None else batch) if batched else 1
    normalized = np.empty(batch * size, np.float32)
    soft = np.empty(batch * size, np.float32)
    product = np.empty((batch * rows) if batched else rows, np.float32)
    lib().orc_iteration_f32(inputs.input, inputs.probabilities, inputs.weight, inputs.matrix, batch,
                            size, rows, int(batched), nv, normalized, soft, product)
    return normalized, soft, product


def iteration_f32_mt(inputs: Inputs, batch, size, rows, batched=False, vectors=None, threads=1):
    """iteration_f32 over OpenMP threads (the timed CPU baseline)."""
    nv = (vectors if vectors is not None else batch) if batched else 1
    normalized = np.empty(batch * size, np.float32)
    soft = np.empty(batch * size, np.float32)
    product = np.empty((batch * rows) if batched else rows, np.float32)
    lib().orc_iteration_f32_mt(inputs.input, inputs.probabilities, inputs.weight, inputs.matrix, batch,
                               size, rows, int(batched), nv, normalized, soft, product, threads)
    return normalized, soft, product


def matvec_fma(x, W, cols, rows):
    out = np.empty(rows, np.float32)
    lib().orc_matvec_fma(np.ascontiguousarray(x, np.float32), np.ascontiguousarray(W, np.float32),
                         cols, rows, out)
    return out


def e2m1_encode(v):
    v = np.ascontiguousarray(v, np.float64)
    out = np.empty(v.size, np.uint8)
    lib().orc_e2m1_encode_array(v, v.size, out)
    return out


def ue4m3_encode(v):
    v = np.ascontiguousarray(v, np.float64)
    out = np.empty(v.size, np.uint8)
    lib().orc_ue4m3_encode_array(v, v.size, out)
    return out


def bf16(v):
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(v.size, np.uint16)
    lib().orc_bf16_array(v, v.size, out)
    return out


def mxfp4_exponent(v):
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(v.size, np.int32)
    lib().orc_mxfp4_exponent_array(v, v.size, out)
    return out


def quantize_mxfp4(W, rows, cols):
    """Unpacked codes [rows*cols] and scale codes [rows*cols/32]."""
    codes = np.empty(rows * cols, np.uint8)
    scales = np.empty(rows * cols // 32, np.uint8)
    lib().orc_quantize_mxfp4(np.ascontiguousarray(W, np.float32), rows, cols, codes, scales)
    return codes, scales


def quantize_fp8(W, rows, cols):
    codes = np.empty(rows * cols, np.uint8)
    scales = np.empty(rows, np.float32)
    lib().orc_quantize_fp8(np.ascontiguousarray(W, np.float32), rows, cols, codes, scales)
    return codes, scales


def e3m2_encode(v):
    v = np.ascontiguousarray(v, np.float64)
    out = np.empty(v.size, np.uint8)
    lib().orc_e3m2_encode_array(v, v.size, out)
    return out


def e3m2_value(code):
    return lib().orc_e3m2_value(int(code))


def quantize_mxfp6(X, rows, width):
    """Unpacked E3M2 codes [rows*width] and UE8M0 scale codes [rows*width/32]."""
    codes = np.empty(rows * width, np.uint8)
    scales = np.empty(rows * width // 32, np.uint8)
    lib().orc_quantize_mxfp6(np.ascontiguousarray(X, np.float32), rows, width, codes, scales)
    return codes, scales


def nvfp4_scales(X):
    """(encode s, decode d) of a tensor from its largest magnitude."""
    a = np.float32(np.max(np.abs(np.asarray(X, np.float32)))) if np.size(X) else np.float32(0)
    s = lib().orc_nvfp4_encode_scale(float(a))
    return np.float32(s), np.float32(lib().orc_nvfp4_decode_scale(s))


def quantize_nvfp4(X, rows, width, s):
    """Unpacked E2M1 codes [rows*width] and UE4M3 scale codes [rows*width/16]."""
    codes = np.empty(rows * width, np.uint8)
    scales = np.empty(rows * width // 16, np.uint8)
    lib().orc_quantize_nvfp4(np.ascontiguousarray(X, np.float32), rows, width, float(s), codes, scales)
    return codes, scales


def pack_e3m2(codes):
    """Value i at bits 6i..6i+5 of a little-endian bit stream."""
    c = np.ascontiguousarray(codes, np.uint8)
    out = np.empty((c.size * 6 + 7) // 8, np.uint8)
    lib().orc_pack_e3m2(c, c.size, out)
    return out


def pack_e2m1(codes):
    """Two codes per byte, even index in the low nibble."""
    c = np.ascontiguousarray(codes, np.uint8).reshape(-1, 2)
    return (c[:, 0] | (c[:, 1] << 4)).astype(np.uint8)


def qmatmul_ref(fmt, xbf16, codes_packed, scales, size, rows, vectors, batch):
    vec = np.ascontiguousarray(vectors, np.int32)
    out = np.full(batch * rows, np.nan, np.float64)
    mag = np.full(batch * rows, np.nan, np.float64)
    scales = np.ascontiguousarray(scales)
    lib().orc_qmatmul_ref(fmt, np.ascontiguousarray(xbf16, np.uint16),
                          np.ascontiguousarray(codes_packed, np.uint8),
                          scales.ctypes.data_as(ctypes.c_void_p), size, rows, vec, len(vec), out, mag)
    return out, mag


def quantize_mxfp8(xbf16, rows, cols):
    """bf16 activations (uint16) to row-major e4m3 codes [rows*cols] and
    UE8M0 scale codes [rows*cols/32]."""
    codes = np.empty(rows * cols, np.uint8)
    scales = np.empty(rows * cols // 32, np.uint8)
    lib().orc_quantize_mxfp8(np.ascontiguousarray(xbf16, np.uint16), rows, cols, codes, scales)
    return codes, scales


def qsmatmul_ref(fmt, xcodes, xscales, wcodes_packed, wscales, size, rows, vectors, batch):
    """Both operands dequantized, double accumulation: (out, sum |terms|),
    each [batch * rows], NaN outside the listed vectors."""
    vec = np.ascontiguousarray(vectors, np.int32)
    out = np.full(batch * rows, np.nan, np.float64)
    mag = np.full(batch * rows, np.nan, np.float64)
    wscales = np.ascontiguousarray(wscales)
    lib().orc_qsmatmul_ref(fmt, np.ascontiguousarray(xcodes, np.uint8), np.ascontiguousarray(xscales, np.uint8),
                           np.ascontiguousarray(wcodes_packed, np.uint8), wscales.ctypes.data_as(ctypes.c_void_p),
                           size, rows, vec, len(vec), out, mag)
    return out, mag


# ---------------------------------------------------------------------------
# Dumps (llama2c/llama2c_common.h:16-32; L2CDUMP2 adds int32 matmul + pad and
# batch x rows product sections).

def read_dump(path):
    data = open(path, "rb").read()
    magic = data[:8]
    if magic not in (b"L2CDUMP1", b"L2CDUMP2"):
        raise ValueError(f"{path}: not a llama2c dump")
    batch, size, rows, inputs = np.frombuffer(data, "<i4", 4, 8)
    seed = int(np.frombuffer(data, "<u8", 1, 24)[0])
    off = 32
    matmul = -1
    if magic == b"L2CDUMP2":
        matmul = int(np.frombuffer(data, "<i4", 1, 32)[0])
        off = 40
    n = int(batch) * int(size)
    p = int(batch) * int(rows) if magic == b"L2CDUMP2" else int(rows)
    out = dict(magic=magic.decode(), batch=int(batch), size=int(size), rows=int(rows),
               inputs=int(inputs), seed=seed, matmul=matmul)
    for name, count, dt in (("normalized", n, "<f4"), ("softmax", n, "<f4"), ("product", p, "<f4"),
                            ("product_tolerance", p, "<f4"), ("product_reference", p, "<f8")):
        width = np.dtype(dt).itemsize
        if len(data) - off < count * width:
            raise ValueError(f"{path}: truncated in {name}")
        out[name] = np.frombuffer(data, dt, count, off)
        off += count * width
    if off != len(data):
        raise ValueError(f"{path}: {len(data) - off} trailing bytes")
    return out
