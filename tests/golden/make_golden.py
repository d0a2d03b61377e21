"""Writes the golden fixtures of tests/golden from the reference's own host
code (llama2c/llama2c_common.h and experiments/blackwell/lowprec/reference.cpp,
compiled as they lie into oracle/_ref/libl2c_ref.so by oracle/Makefile).

The reference holds no committed golden vectors for this path, so these
fixtures are produced by its code and kept as data: inputs and expected
outputs only. Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle  # noqa: E402


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    R = oracle.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libl2c_ref.so is not built (make -C oracle with the reference present)")
    g = {"source": "reference host code compiled by oracle/Makefile (llama2c_common.h, lowprec/reference.cpp)"}

    # Generator spot values (llama2c_common.h:100-103).
    spots = []
    for seed in (0, 1, 2, 3, 12345678901234567):
        for stream in (0, 1, 2, 3):
            for index in (0, 1, 2, 1023, 1 << 20, (1 << 33) + 7):
                v = float(np.float32(R.ref_uniform(seed, stream, index)))
                spots.append([seed, stream, index, np.float32(v).view(np.uint32).item()])
    g["uniform_bits"] = spots

    # Whole input sets (llama2c_common.h:105-132) as checksums.
    fills = []
    for mode, seed, b, s, r in ((0, 0, 3, 17, 5), (1, 1, 2, 1001, 7), (1, 2, 1, 288, 288),
                                (1, 3, 4, 64, 300), (0, 0, 2, 8, 20)):
        x = np.empty(b * s, np.float32)
        p = np.empty(b * s, np.float32)
        w = np.empty(s, np.float32)
        m = np.empty(r * s, np.float32)
        R.ref_fill(mode, seed, b, s, r, x, p, w, m)
        fills.append(dict(mode=mode, seed=seed, batch=b, size=s, rows=r, input=sha(x),
                          probabilities=sha(p), weight=sha(w), matrix=sha(m)))
    g["fill_sha256"] = fills

    # gamma~ (llama2c_common.h:231-235).
    g["gamma"] = [[n, R.ref_gamma(n)] for n in (1, 2, 77, 288, 768, 1000, 1001, 4096, 16384, 65536)]

    # E2M1 / UE4M3 encodings and bf16 (lowprec/reference.cpp:13-96).
    vals = np.concatenate([np.arange(-160, 161) / 16.0, [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0,
                                                          1e-9, -1e-9, 100.0, -100.0]])
    vals = vals.astype(np.float64)
    e2 = np.empty(vals.size, np.uint8)
    R.ref_encode_array(0, vals, vals.size, e2)
    g["e2m1"] = {"values": vals.tolist(), "codes": e2.tolist()}
    u = np.concatenate([np.ldexp(np.arange(0, 64) / 8.0, -9), np.arange(0, 480, 3.5),
                        [448.0, 460.0, 464.0, 470.0, 1e6, 0.0009765625, 0.00146484375]])
    u = u.astype(np.float64)
    e4 = np.empty(u.size, np.uint8)
    R.ref_encode_array(2, u, u.size, e4)
    g["ue4m3"] = {"values": u.tolist(), "codes": e4.tolist()}
    rng = np.random.default_rng(20261201)
    fv = np.concatenate([rng.standard_normal(200).astype(np.float32),
                         np.array([1.00390625, 1.01171875, -1.00390625, 3.0e38, 1e-40], np.float32)])
    b16 = np.empty(fv.size, np.uint16)
    R.ref_to_bf16_array(fv, fv.size, b16)
    g["bf16"] = {"bits": fv.view(np.uint32).tolist(), "codes": b16.tolist()}

    # Standard normals of the lowprec fixture generator (stream 1, seeds 1..3).
    g["normals"] = []
    for seed in (1, 2, 3):
        out = np.empty(64, np.float32)
        R.ref_normals_stream1(seed, 64, out)
        g["normals"].append({"seed": seed, "stream": 1, "bits": out.view(np.uint32).tolist()})

    # E3M2 encodings and the MXFP6 / NVFP4 quantizers (lowprec/reference.cpp:
    # 27-45, 105-150) on the crafted edge-case matrix of lowprec_oracle.
    import lowprec_oracle
    ev = np.concatenate([np.arange(-33 * 16, 33 * 16 + 1) / 16.0, np.arange(-64, 65) / 256.0,
                         [1e-9, -1e-9, 100.0, -100.0, 27.99, 28.0, 30.0, 30.01]]).astype(np.float64)
    e3 = np.empty(ev.size, np.uint8)
    R.ref_encode_array(1, ev, ev.size, e3)
    g["e3m2"] = {"values": ev.tolist(), "codes": e3.tolist()}
    rows, width = 40, 256
    m = lowprec_oracle.crafted(rows, width)
    c6 = np.empty(rows * width, np.uint8)
    s6 = np.empty(rows * width // 32, np.uint8)
    R.ref_quantize_mxfp6(m, rows, width, c6, s6)
    amax = np.float32(np.abs(m).max())
    enc = np.float32(R.ref_nvfp4_encode_scale(float(amax)))
    dec = np.float32(R.ref_nvfp4_decode_scale(float(enc)))
    c4 = np.empty(rows * width, np.uint8)
    s4 = np.empty(rows * width // 16, np.uint8)
    R.ref_quantize_nvfp4(m, rows, width, float(enc), c4, s4)
    g["lowprec_crafted"] = {
        "rows": rows, "width": width, "input_sha256": sha(m),
        "mxfp6_codes_packed_hex": oracle.pack_e3m2(c6).tobytes().hex(), "mxfp6_scales_hex": s6.tobytes().hex(),
        "nvfp4_encode_bits": int(enc.view(np.uint32)), "nvfp4_decode_bits": int(dec.view(np.uint32)),
        "nvfp4_codes_packed_hex": oracle.pack_e2m1(c4).tobytes().hex(), "nvfp4_scales_hex": s4.tobytes().hex()}

    # A whole dump of the reference's writer (llama2c_common.h:321-345) for a
    # small random case, with outputs computed by the reference's validate_all
    # on the double-reference outputs rounded to float.
    b, s, r, seed = 2, 16, 5, 7
    x = np.empty(b * s, np.float32)
    p = np.empty(b * s, np.float32)
    w = np.empty(s, np.float32)
    m = np.empty(r * s, np.float32)
    R.ref_fill(1, seed, b, s, r, x, p, w, m)
    nrm = oracle.rmsnorm_ref(x, w, b, s).astype(np.float32)
    sm = oracle.softmax_ref(p, b, s).astype(np.float32)
    prod = (m.reshape(r, s).astype(np.float64) @ x[:s].astype(np.float64)).astype(np.float32)
    tol = np.empty(r, np.float32)
    refv = np.empty(r, np.float64)
    valid = R.ref_validate_all(1, seed, x, p, w, m, nrm, sm, prod, b, s, r, tol, refv)
    path = os.path.join(HERE, "ref_dump_random7_2x16x5.bin")
    assert R.ref_write_dump(path.encode(), 1, seed, b, s, r, nrm, sm, prod, tol, refv) == 1
    g["dump"] = {"file": os.path.basename(path), "valid": int(valid), "batch": b, "size": s,
                 "rows": r, "seed": seed}

    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(g, f, indent=1)
    print("wrote", os.path.join(HERE, "golden.json"), "and", path)


if __name__ == "__main__":
    main()
