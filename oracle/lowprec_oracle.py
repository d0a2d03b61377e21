"""CPU oracle of the low-precision classifier cases (MXFP6, NVFP4, BF16) of
the llama2c decoder, in numpy over the C oracle's format encoders.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker. The product
never imports it.

Restates, from the reference repository (experiments/blackwell/lowprec):
  value tables       reference.cpp:27-45 (E2M1, E3M2, UE4M3, UE8M0 decode)
  dequantize_*       reference.cpp:152-158 (E3M2 x 2^(s-127); E2M1 x UE4M3, d apart)
  unpack_e3m2/e2m1   reference.cpp:159-168 and spec.json "layout"
  fixture            reference.cpp:199-213, spec.json "fixtures"
  logit_bound        spec.json "implementation_check.logits"
  rmsnorm_double     reference.cpp:215-220
The quantizers themselves are the C oracle's (oracle/l2c_oracle.c).

How it is pinned: the C quantizers equal the reference's own quantizers
(oracle/_ref) bit for bit on the crafted rows below and on random rows
(tests/test_oracle_vs_ref.py) and reproduce the committed golden codes
(tests/golden); the value tables are checked against the format definitions
at every code (tests/test_lowprec.py); the logit bound is checked to hold for
float32 sums in several orders and to fail on a dropped term.
"""
from __future__ import annotations

import numpy as np

import oracle

E2M1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6], np.float64)


def _e3m2_table():
    out = np.empty(64, np.float64)
    for c in range(64):
        e, m = (c >> 2) & 7, c & 3
        mag = np.ldexp(m / 4.0, -2) if e == 0 else np.ldexp(1.0 + m / 4.0, e - 3)
        out[c] = -mag if c & 32 else mag
    return out


def _ue4m3_table():
    out = np.empty(128, np.float64)
    for c in range(128):
        e, m = (c >> 3) & 15, c & 7
        out[c] = np.ldexp(m / 8.0, -6) if e == 0 else np.ldexp(1.0 + m / 8.0, e - 7)
    return out


E3M2 = _e3m2_table()
UE4M3 = _ue4m3_table()


def ue8m0(code):
    return np.ldexp(1.0, np.asarray(code, np.int64) - 127)


def dequantize_mxfp6(codes, scales, rows, width):
    c = np.asarray(codes, np.uint8).reshape(rows, width)
    s = np.asarray(scales, np.uint8).reshape(rows, width // 32)
    return E3M2[c] * np.repeat(ue8m0(s), 32, axis=1)


def dequantize_nvfp4(codes, scales, rows, width):
    """Element value times block scale, without the tensor decode scale."""
    c = np.asarray(codes, np.uint8).reshape(rows, width)
    s = np.asarray(scales, np.uint8).reshape(rows, width // 16)
    return E2M1[c] * np.repeat(UE4M3[s & 0x7f], 16, axis=1)


def bf16_value(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32).astype(np.float64)


def unpack_e3m2(packed, count):
    """Codes of a packed E3M2 row (value i at bits 6i..6i+5)."""
    p = np.asarray(packed, np.uint8).astype(np.uint32)
    i = np.arange(count)
    bit = 6 * i
    byte, off = bit // 8, bit % 8
    nxt = np.where(off > 2, p[np.minimum(byte + 1, p.size - 1)], 0)
    return (((p[byte] | (nxt << 8)) >> off) & 0x3F).astype(np.uint8)


def tile_mxfp6(codes, scales, rows, width):
    """Unpacked E3M2 codes [rows*width] and scale codes [rows*width/32] in the
    tiled operand layout of the MXFP6 contraction (rows padded to Rp, a
    multiple of 32, with zero codes and scales): code bytes
    [width/128][Rp/32][4][32][24 B] (each 24 B the block's packed stream) and
    scale bytes [width/128][Rp][4]."""
    rp = (rows + 31) // 32 * 32
    c = np.zeros((rp, width), np.uint8)
    c[:rows] = np.asarray(codes, np.uint8).reshape(rows, width)
    sc = np.zeros((rp, width // 32), np.uint8)
    sc[:rows] = np.asarray(scales, np.uint8).reshape(rows, width // 32)
    # [row][block][32] -> [t][group][b][r][32]
    blocks = c.reshape(rp // 32, 32, width // 128, 4, 32).transpose(2, 0, 3, 1, 4)
    packed = oracle.pack_e3m2(np.ascontiguousarray(blocks).ravel())
    sbytes = np.ascontiguousarray(sc.reshape(rp, width // 128, 4).transpose(1, 0, 2)).ravel()
    return packed, sbytes


def untile_mxfp6(code_bytes, scale_bytes, rows, width):
    """Inverse of tile_mxfp6: unpacked codes [rows*width], scales [rows*width/32]."""
    rp = (rows + 31) // 32 * 32
    n = rp * width
    codes = unpack_e3m2(np.asarray(code_bytes, np.uint8)[: n * 3 // 4], n)
    c = codes.reshape(width // 128, rp // 32, 4, 32, 32).transpose(1, 3, 0, 2, 4).reshape(rp, width)
    s = np.asarray(scale_bytes, np.uint8)[: rp * width // 32].reshape(width // 128, rp, 4).transpose(1, 0, 2)
    return np.ascontiguousarray(c[:rows]).ravel(), np.ascontiguousarray(s.reshape(rp, width // 32)[:rows]).ravel()


def unpack_e2m1(packed, count):
    p = np.asarray(packed, np.uint8)
    i = np.arange(count)
    return ((p[i // 2] >> (4 * (i % 2))) & 0xF).astype(np.uint8)


def pack_e2m1(codes):
    return oracle.pack_e2m1(codes)


def fixture(seed, width, vocab):
    """(embedding, classifier) float32 [vocab][width]: standard normals of
    stream 1, and of stream 2 times float(1 / sqrt(width))."""
    n = width * vocab
    emb = oracle.normal(seed, 1, 0, n).reshape(vocab, width)
    scale = np.float32(1.0 / np.sqrt(float(width)))
    cls = (oracle.normal(seed, 2, 0, n) * scale).astype(np.float32).reshape(vocab, width)
    return emb, cls


def rmsnorm_double(x):
    x = np.asarray(x, np.float64)
    scale = 1.0 / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) / x.shape[-1] + float(np.float32(1e-5)))
    return scale * x


def logit_bound(a, w, alpha, K):
    """Expected logits sum_k a_k w_k * alpha in double and the implementation
    check's bound gamma * sum|a w| * |alpha| + 2^-23 |expected| + 1e-30,
    gamma = K u / (1 - K u), u = 2^-23. a [B][K], w [V][K] (double)."""
    u = 2.0 ** -23
    gamma = K * u / (1.0 - K * u)
    exp = (a @ w.T) * alpha
    mag = np.abs(a) @ np.abs(w).T
    return exp, gamma * mag * abs(alpha) + u * np.abs(exp) + 1e-30


def crafted(rows=130, width=256, seed=5):
    """A [rows][width] float32 matrix of quantizer edge cases (rows >= 8,
    width >= 128, width % 32 == 0):
      row 0   the tensor maximum 2688 (NVFP4 encode scale exactly 1)
      row 1   E2M1 ties and saturation at block scale 1 (block maximum 6)
      row 2   E3M2 ties and saturation at 2^X = 1 (block maximum 16..31.9)
      row 3   blocks whose maximum rounds past 28 (mantissa above 1.75)
      row 4   tiny blocks: block scales that round to zero, subnormal inputs
      row 5   UE4M3 scale ties (block maxima 6 (1 + i / 16))
      row 6   zero blocks next to nonzero ones, negative zeros
      rest    random values of magnitude 2^-9 .. 4 per row"""
    m = np.zeros((rows, width), np.float32)
    m[0, 0] = 2688.0
    e2 = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 5.5, -0.25, -0.75, -2.5, -5.5, 0.26, -0.2, 6.0, 6.2]
    m[1, :16] = e2
    m[1, 16:32] = np.float32(e2) * np.float32(0.75)  # block maximum 4.875
    e3 = [0.03125, 0.09375, 0.15625, 0.21875, 1.125, 1.375, 2.75, 26.0, 30.0, -0.03125,
          -0.09375, -26.0, 0.0, 16.0, 18.0, 22.0]
    m[2, :16] = e3
    m[2, 16:32] = [31.9, 31.0, 29.9, 28.1] + [1.0] * 12
    m[2, 32:64] = np.float32(e3 * 2) / np.float32(4.0)
    for i in range(min(8, width // 32)):  # block maxima (2 - 2^-j) * 2^(i-4), then smaller values
        blk = m[3, 32 * i:32 * i + 32]
        blk[0] = np.float32((2.0 - 2.0 ** -(i + 2)) * 2.0 ** (i - 4))
        blk[1:] = np.float32(blk[0]) * np.linspace(-0.99, 0.98, 31, dtype=np.float32)
    m[4, :16] = np.float32(1e-6) * (np.arange(16, dtype=np.float32) - 8)
    m[4, 16:32] = np.float32(0.004) * (np.arange(16, dtype=np.float32) - 8)
    m[4, 32:64] = np.float32(1e-30) * (np.arange(32, dtype=np.float32) + 1)
    m[4, 64:96] = np.float32(1e-40) * (np.arange(32, dtype=np.float32) - 15)
    m[4, 96:128] = np.float32(2.0 ** -126) * np.arange(32, dtype=np.float32)
    for i in range(width // 16):
        m[5, 16 * i] = np.float32(6.0 * (1.0 + 0.0625 * (i % 16)))
        m[5, 16 * i + 1] = np.float32(-3.0)
    m[6, 32:64] = np.float32(-0.0)
    m[6, 64:96] = np.float32(0.5)
    rng = np.random.default_rng(seed)
    for r in range(7, rows):
        m[r] = ((rng.random(width) - 0.5) * np.ldexp(1.0, r % 12 - 8)).astype(np.float32)
    return m
