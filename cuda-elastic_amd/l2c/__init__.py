"""Python binding of the llama2c hot path on MI355X.

Loads the in-tree libl2c.so (HIP kernels behind the C ABI of include/l2c.h)
and libl2c_host.so (the harness, include/l2c_harness.h) with ctypes. Device
memory and streams come from torch: every wrapper takes torch tensors on the
GPU and enqueues on torch's current stream (or the stream passed in).

There is no fallback: if the built library is missing or a call fails, an
exception is raised.

The wrappers mirror the reference kernels' argument order and meaning
(llama2c/llama2c_cuda_graph.cu:58-162, llama2c_sota.cu:263-298).
"""
from __future__ import annotations

import ctypes
import os
import shlex
import subprocess

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG_DIR, "lib")
BIN_DIR = os.path.join(PKG_DIR, "bin")
LIB_PATH = os.path.join(LIB_DIR, "libl2c.so")
HOST_LIB_PATH = os.path.join(LIB_DIR, "libl2c_host.so")
HARNESS = os.path.join(BIN_DIR, "llama2c_hip")
DECODER = os.path.join(BIN_DIR, "llama2c_decoder_hip")
LOWPREC_CASES = ("fp32", "bf16", "mxfp6", "nvfp4")
LOWPREC_DIR = os.path.join(BIN_DIR, "lowprec")
COMPARE = os.path.join(BIN_DIR, "l2c_compare")

RMS_EPSILON = 1.0e-5  # llama2c/llama2c_common.h:44

MATVEC_NAIVE = 0
MATVEC_COALESCED = 1
Q_MXFP4 = 0
Q_FP8 = 1
OP_RMSNORM, OP_SOFTMAX, OP_MATVEC, OP_FUSED, OP_MATMUL, OP_MATMUL_Q, OP_MATMUL_QS = range(7)

# Symbols declared in include/l2c.h and include/l2c_harness.h.
KERNEL_SYMBOLS = (
    "l2c_rmsnorm", "l2c_softmax", "l2c_matvec", "l2c_fused", "l2c_matmul", "l2c_matmul_q",
    "l2c_quantize_mxfp4", "l2c_quantize_fp8", "l2c_to_bf16", "l2c_launch_shape",
    "l2c_strerror", "l2c_version",
    "l2c_decoder_init_model", "l2c_decoder_rmsnorm", "l2c_decoder_rmsnorm_absmax", "l2c_decoder_softmax_argmax",
    "l2c_quantize_mxfp6", "l2c_nvfp4_tensor_scales", "l2c_nvfp4_tensor_scales_absmax", "l2c_quantize_nvfp4",
    "l2c_to_bf16_x4",
    "l2c_matmul_bf16", "l2c_matmul_mxfp6", "l2c_mxfp6_bytes",
    "l2c_matmul_qs", "l2c_quantize_mxfp8", "l2c_mxfp8_workspace_bytes", "l2c_matmul_qs_static",
    "l2c_copy_to_host",
)
QS_STATIC_SCRATCH_BYTES = 24 << 20  # L2C_QS_STATIC_SCRATCH_BYTES
NVFP4_PARTIALS = 1024  # L2C_NVFP4_PARTIALS
HOST_SYMBOLS = ("l2c_harness_main", "l2c_compare_dumps", "l2c_decoder_main", "l2c_decoder_run",
                "l2c_lowprec_main", "l2c_lowprec_run", "l2c_lowprec_host_quantize", "l2c_lowprec_fixture",
                "l2c_lowprec_crafted")


class L2CError(RuntimeError):
    """A nonzero return code from the C ABI."""


def build(jobs: int = 8) -> None:
    """Compiles the package (make -C cuda-elastic_amd)."""
    subprocess.run(["make", "-C", PKG_DIR, f"-j{jobs}"], check=True)


_lib = None
_host = None


def _vp(x):
    return ctypes.c_void_p(x)


def load() -> ctypes.CDLL:
    """Loads libl2c.so (after torch, so both share one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(
            f"{LIB_PATH} is not built; run `make -C {PKG_DIR}` (or __graft_entry__.build())")
    try:
        import torch  # noqa: F401  (loads the HIP runtime torch was built with first)
    except ImportError:
        pass
    lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    i, f, p, sz = ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t
    sigs = {
        "l2c_rmsnorm": [p, p, p, i, i, f, p],
        "l2c_softmax": [p, p, i, i, p],
        "l2c_matvec": [p, p, p, i, i, i, p],
        "l2c_fused": [p, p, p, p, p, p, p, i, i, i, i, f, p],
        "l2c_matmul": [p, p, p, i, i, i, p],
        "l2c_matmul_q": [p, p, p, p, i, i, i, i, p],
        "l2c_quantize_mxfp4": [p, p, p, i, i, p],
        "l2c_quantize_fp8": [p, p, p, i, i, p],
        "l2c_to_bf16": [p, p, sz, p],
        "l2c_launch_shape": [i, i, i, i, i, ctypes.POINTER(i), ctypes.POINTER(i), ctypes.POINTER(i)],
        "l2c_decoder_init_model": [p, p, p, i, i, p],
        "l2c_decoder_rmsnorm": [p, p, p, p, i, i, i, p],
        "l2c_decoder_rmsnorm_absmax": [p, p, p, p, i, i, i, p, p],
        "l2c_decoder_softmax_argmax": [p, p, p, p, i, i, i, i, p],
        "l2c_quantize_mxfp6": [p, p, p, i, i, p],
        "l2c_nvfp4_tensor_scales": [p, p, p, p, ctypes.c_longlong, p, p],
        "l2c_nvfp4_tensor_scales_absmax": [p, p, p, p, p],
        "l2c_quantize_nvfp4": [p, p, p, p, p, i, i, p],
        "l2c_to_bf16_x4": [p, p, ctypes.c_longlong, p],
        "l2c_matmul_bf16": [p, p, p, p, i, i, i, p],
        "l2c_matmul_mxfp6": [p, p, p, p, p, i, i, i, p],
        "l2c_matmul_qs": [p, p, p, p, i, i, i, i, p, sz, p],
        "l2c_quantize_mxfp8": [p, sz, p, i, i, p],
        "l2c_matmul_qs_static": [p, p, p, p, i, i, i, i, p],
        "l2c_copy_to_host": [p, p, sz, p],
    }
    for name, args in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    lib.l2c_mxfp8_workspace_bytes.argtypes = [i, i]
    lib.l2c_mxfp8_workspace_bytes.restype = sz
    lib.l2c_mxfp6_bytes.argtypes = [i, i, ctypes.POINTER(sz), ctypes.POINTER(sz)]
    lib.l2c_mxfp6_bytes.restype = ctypes.c_int
    lib.l2c_strerror.argtypes = [ctypes.c_int]
    lib.l2c_strerror.restype = ctypes.c_char_p
    lib.l2c_version.argtypes = []
    lib.l2c_version.restype = ctypes.c_char_p
    _lib = lib
    return lib


def load_host() -> ctypes.CDLL:
    """Loads libl2c_host.so (the harness library)."""
    global _host
    if _host is not None:
        return _host
    load()
    if not os.path.exists(HOST_LIB_PATH):
        raise FileNotFoundError(f"{HOST_LIB_PATH} is not built")
    host = ctypes.CDLL(HOST_LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    host.l2c_harness_main.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
                                      ctypes.c_char_p, ctypes.c_size_t]
    host.l2c_harness_main.restype = ctypes.c_int
    host.l2c_compare_dumps.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]
    host.l2c_compare_dumps.restype = ctypes.c_int
    host.l2c_decoder_main.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.c_char_p,
                                      ctypes.c_size_t]
    host.l2c_decoder_main.restype = ctypes.c_int
    host.l2c_decoder_run.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]
    host.l2c_decoder_run.restype = ctypes.c_int
    host.l2c_lowprec_main.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.c_char_p,
                                      ctypes.c_size_t]
    host.l2c_lowprec_main.restype = ctypes.c_int
    host.l2c_lowprec_run.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]
    host.l2c_lowprec_run.restype = ctypes.c_int
    vp = ctypes.c_void_p
    host.l2c_lowprec_host_quantize.argtypes = [ctypes.c_int, vp, ctypes.c_int, ctypes.c_int, vp, vp, vp]
    host.l2c_lowprec_host_quantize.restype = ctypes.c_int
    host.l2c_lowprec_fixture.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
    host.l2c_lowprec_fixture.restype = ctypes.c_int
    host.l2c_lowprec_crafted.argtypes = [ctypes.c_int, ctypes.c_int, vp]
    host.l2c_lowprec_crafted.restype = ctypes.c_int
    _host = host
    return host


def _check(code: int, what: str) -> None:
    if code != 0:
        msg = load().l2c_strerror(code).decode()
        raise L2CError(f"{what} failed: {msg} ({code})")


def _stream(stream):
    if stream is not None:
        return stream if isinstance(stream, int) else stream.cuda_stream
    import torch
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("l2c wrappers take GPU tensors")
    return t.data_ptr()


# ---------------------------------------------------------------------------
# Kernel wrappers (torch tensors in, results in `out`).

def rmsnorm(out, inp, weight, size, batch, eps=RMS_EPSILON, stream=None):
    _check(load().l2c_rmsnorm(_vp(_ptr(out)), _vp(_ptr(inp)), _vp(_ptr(weight)), size, batch,
                              eps, _vp(_stream(stream))), "l2c_rmsnorm")


def softmax(out, logits, size, batch, stream=None):
    _check(load().l2c_softmax(_vp(_ptr(out)), _vp(_ptr(logits)), size, batch,
                              _vp(_stream(stream))), "l2c_softmax")


def matvec(out, x, W, cols, rows, variant=MATVEC_COALESCED, stream=None):
    _check(load().l2c_matvec(_vp(_ptr(out)), _vp(_ptr(x)), _vp(_ptr(W)), cols, rows, variant,
                             _vp(_stream(stream))), "l2c_matvec")


def fused(normalized, inp, weight, softmax_out, logits, product, matrix, size, rms_rows,
          softmax_rows, matmul_rows, eps=RMS_EPSILON, stream=None):
    _check(load().l2c_fused(_vp(_ptr(normalized)), _vp(_ptr(inp)), _vp(_ptr(weight)),
                            _vp(_ptr(softmax_out)), _vp(_ptr(logits)), _vp(_ptr(product)),
                            _vp(_ptr(matrix)), size, rms_rows, softmax_rows, matmul_rows, eps,
                            _vp(_stream(stream))), "l2c_fused")


def matmul(out, X, W, batch, cols, rows, stream=None):
    _check(load().l2c_matmul(_vp(_ptr(out)), _vp(_ptr(X)), _vp(_ptr(W)), batch, cols, rows,
                             _vp(_stream(stream))), "l2c_matmul")


def matmul_q(out, xbf16, wq, scales, fmt, batch, cols, rows, stream=None):
    _check(load().l2c_matmul_q(_vp(_ptr(out)), _vp(_ptr(xbf16)), _vp(_ptr(wq)), _vp(_ptr(scales)),
                               fmt, batch, cols, rows, _vp(_stream(stream))), "l2c_matmul_q")


def mxfp8_workspace_bytes(batch, cols):
    return load().l2c_mxfp8_workspace_bytes(batch, cols)


def mxfp8_views(workspace, batch, cols):
    """(codes [batch*cols], scales [cols/128][Bp][4]) views of an l2c_matmul_qs
    workspace (uint8 tensor), as include/l2c.h lays it out."""
    n = batch * cols
    off = (n + 255) // 256 * 256
    bp = (batch + 3) // 4 * 4
    return workspace[:n], workspace[off:off + (cols // 128) * bp * 4]


def matmul_qs(out, xbf16, wq, scales, fmt, batch, cols, rows, workspace, stream=None):
    _check(load().l2c_matmul_qs(_vp(_ptr(out)), _vp(_ptr(xbf16)), _vp(_ptr(wq)), _vp(_ptr(scales)), fmt, batch,
                                cols, rows, _vp(_ptr(workspace)), workspace.numel() * workspace.element_size(),
                                _vp(_stream(stream))), "l2c_matmul_qs")


def matmul_qs_static(out, xbf16, wq, scales, fmt, batch, cols, rows, stream=None):
    _check(load().l2c_matmul_qs_static(_vp(_ptr(out)), _vp(_ptr(xbf16)), _vp(_ptr(wq)), _vp(_ptr(scales)), fmt,
                                       batch, cols, rows, _vp(_stream(stream))), "l2c_matmul_qs_static")


def quantize_mxfp8(workspace, xbf16, batch, cols, stream=None):
    _check(load().l2c_quantize_mxfp8(_vp(_ptr(workspace)), workspace.numel() * workspace.element_size(),
                                     _vp(_ptr(xbf16)), batch, cols, _vp(_stream(stream))), "l2c_quantize_mxfp8")


def quantize_mxfp4(codes, scales, W, rows, cols, stream=None):
    _check(load().l2c_quantize_mxfp4(_vp(_ptr(codes)), _vp(_ptr(scales)), _vp(_ptr(W)), rows, cols,
                                     _vp(_stream(stream))), "l2c_quantize_mxfp4")


def quantize_fp8(codes, scales, W, rows, cols, stream=None):
    _check(load().l2c_quantize_fp8(_vp(_ptr(codes)), _vp(_ptr(scales)), _vp(_ptr(W)), rows, cols,
                                   _vp(_stream(stream))), "l2c_quantize_fp8")


def to_bf16(out, inp, n, stream=None):
    _check(load().l2c_to_bf16(_vp(_ptr(out)), _vp(_ptr(inp)), n, _vp(_stream(stream))),
           "l2c_to_bf16")


def decoder_init_model(embedding, classifier, norm_weight, width, vocab, stream=None):
    _check(load().l2c_decoder_init_model(_vp(_ptr(embedding)), _vp(_ptr(classifier)),
                                         _vp(_ptr(norm_weight)), width, vocab, _vp(_stream(stream))),
           "l2c_decoder_init_model")


def decoder_rmsnorm(normalized, tokens, embedding, weight, width, vocab, batch, stream=None):
    _check(load().l2c_decoder_rmsnorm(_vp(_ptr(normalized)), _vp(_ptr(tokens)), _vp(_ptr(embedding)),
                                      _vp(_ptr(weight)), width, vocab, batch, _vp(_stream(stream))),
           "l2c_decoder_rmsnorm")


def decoder_rmsnorm_absmax(normalized, tokens, embedding, weight, width, vocab, batch, absmax_bits, stream=None):
    _check(load().l2c_decoder_rmsnorm_absmax(_vp(_ptr(normalized)), _vp(_ptr(tokens)), _vp(_ptr(embedding)),
                                             _vp(_ptr(weight)), width, vocab, batch, _vp(_ptr(absmax_bits)),
                                             _vp(_stream(stream))), "l2c_decoder_rmsnorm_absmax")


def decoder_softmax_argmax(probabilities, logits, tokens, generated, vocab, batch, steps, step,
                           stream=None):
    _check(load().l2c_decoder_softmax_argmax(_vp(_ptr(probabilities)), _vp(_ptr(logits)),
                                             _vp(_ptr(tokens)), _vp(_ptr(generated)), vocab, batch,
                                             steps, step, _vp(_stream(stream))),
           "l2c_decoder_softmax_argmax")


def launch_shape(op, batch, cols, rows, variant=0):
    g, b, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _check(load().l2c_launch_shape(op, batch, cols, rows, variant, ctypes.byref(g),
                                   ctypes.byref(b), ctypes.byref(c)), "l2c_launch_shape")
    return g.value, b.value, c.value


# ---------------------------------------------------------------------------
# Harness

def parse_line(line: str) -> dict:
    """Parses the key=value result line into a dict (numbers converted)."""
    out = {}
    for token in line.split():
        if "=" not in token:
            continue
        k, v = token.split("=", 1)
        try:
            out[k] = int(v)
        except ValueError:
            try:
                out[k] = float(v)
            except ValueError:
                out[k] = v
    return out


def harness(args, in_process: bool = True, env=None, timeout=None):
    """Runs one harness invocation; returns (exit_code, parsed line, raw line).

    args is the argument list after the program name, e.g.
    ["graph", "3", "1024", "16384", "8192", "1", "1", "nocopy", "batched", "scaled"].
    """
    args = [str(a) for a in args]
    if in_process:
        host = load_host()
        argv = [b"llama2c_hip"] + [a.encode() for a in args]
        arr = (ctypes.c_char_p * len(argv))(*argv)
        buf = ctypes.create_string_buffer(8192)
        code = host.l2c_harness_main(len(argv), arr, buf, len(buf))
        line = buf.value.decode()
        return code, parse_line(line), line
    if not os.path.exists(HARNESS):
        raise FileNotFoundError(f"{HARNESS} is not built")
    proc = subprocess.run([HARNESS] + args, capture_output=True, text=True, env=env,
                          timeout=timeout)
    line = proc.stdout.strip().splitlines()[-1] if proc.stdout.strip() else ""
    if proc.returncode != 0 and proc.stderr:
        line = line or ""
    return proc.returncode, parse_line(line), line + ("\n" + proc.stderr if proc.stderr else "")


def compare_dumps(paths, in_process: bool = False):
    """Runs the dump comparer; returns (exit_code, report text)."""
    if in_process:
        host = load_host()
        arr = (ctypes.c_char_p * len(paths))(*[p.encode() for p in paths])
        return host.l2c_compare_dumps(len(paths), arr), ""
    proc = subprocess.run([COMPARE] + list(paths), capture_output=True, text=True)
    return proc.returncode, proc.stdout + proc.stderr


def decoder(args, in_process: bool = False, timeout=None):
    """Runs the llama2c decoder application (the loom_private protocol);
    returns (exit_code, record dict or None, stderr text).

    args is the argument list after the program name, e.g.
    ["--launch", "both", "--set", "batch=40", "--set", "width=96"].
    In-process runs return no stderr text (it goes to the process's stderr).
    """
    import json
    args = [str(a) for a in args]
    if in_process:
        host = load_host()
        argv = [b"llama2c_decoder_hip"] + [a.encode() for a in args]
        arr = (ctypes.c_char_p * len(argv))(*argv)
        buf = ctypes.create_string_buffer(1 << 16)
        code = host.l2c_decoder_main(len(argv), arr, buf, len(buf))
        text = buf.value.decode()
        return code, (json.loads(text) if text else None), ""
    if not os.path.exists(DECODER):
        raise FileNotFoundError(f"{DECODER} is not built")
    proc = subprocess.run([DECODER] + args, capture_output=True, text=True, timeout=timeout)
    record = None
    for line in proc.stdout.splitlines():
        if line.startswith("RESULT "):
            record = json.loads(line[len("RESULT "):])
    return proc.returncode, record, proc.stderr


def lowprec(case, args, in_process: bool = False, timeout=None, env=None):
    """Runs one case ("fp32", "bf16", "mxfp6", "nvfp4") of the lowprec
    classifier experiment; returns (exit_code, record dict or None, stdout +
    stderr text). args: the loom_private options, or ["--selftest"], or
    ["--accuracy"]. env: extra environment variables for the child process
    (e.g. {"L2C_LOWPREC_AMAX_IN_RMSNORM": "1"})."""
    import json
    args = [str(a) for a in args]
    index = LOWPREC_CASES.index(case)
    if in_process:
        host = load_host()
        argv = [case.encode()] + [a.encode() for a in args]
        arr = (ctypes.c_char_p * len(argv))(*argv)
        buf = ctypes.create_string_buffer(1 << 20)
        code = host.l2c_lowprec_main(index, len(argv), arr, buf, len(buf))
        text = buf.value.decode()
        return code, (json.loads(text) if text else None), ""
    exe = os.path.join(LOWPREC_DIR, case)
    if not os.path.exists(exe):
        raise FileNotFoundError(f"{exe} is not built")
    proc = subprocess.run([exe] + args, capture_output=True, text=True, timeout=timeout,
                          env=dict(os.environ, **env) if env else None)
    record = None
    for line in proc.stdout.splitlines():
        if line.startswith("RESULT "):
            record = json.loads(line[len("RESULT "):])
    return proc.returncode, record, proc.stdout + proc.stderr


def lowprec_host_quantize(case, x, rows, width):
    """The lowprec application's host reference quantizer (numpy in/out):
    (codes uint16 [rows*width], scales uint8 [blocks], decode float)."""
    import numpy as np
    x = np.ascontiguousarray(x, np.float32)
    codes = np.empty(rows * width, np.uint16)
    block = {"bf16": 0, "mxfp6": 32, "nvfp4": 16}[case]
    scales = np.empty(rows * width // block if block else 1, np.uint8)
    decode = ctypes.c_float(0)
    code = load_host().l2c_lowprec_host_quantize(LOWPREC_CASES.index(case), x.ctypes.data, rows, width,
                                                 codes.ctypes.data, scales.ctypes.data, ctypes.addressof(decode))
    if code:
        raise L2CError(f"l2c_lowprec_host_quantize failed ({code})")
    return codes, scales[: rows * width // block] if block else scales[:0], decode.value


def lowprec_fixture(seed, width, vocab):
    import numpy as np
    emb = np.empty(width * vocab, np.float32)
    cls = np.empty(width * vocab, np.float32)
    if load_host().l2c_lowprec_fixture(seed, width, vocab, emb.ctypes.data, cls.ctypes.data):
        raise L2CError("l2c_lowprec_fixture failed")
    return emb.reshape(vocab, width), cls.reshape(vocab, width)


def lowprec_crafted(rows, width):
    import numpy as np
    out = np.empty(rows * width, np.float32)
    if load_host().l2c_lowprec_crafted(rows, width, out.ctypes.data):
        raise L2CError("l2c_lowprec_crafted failed")
    return out.reshape(rows, width)


def command_line(args) -> str:
    return " ".join(shlex.quote(a) for a in [HARNESS] + [str(a) for a in args])


# ---------------------------------------------------------------------------
# Low-precision classifier formats and contractions.

def mxfp6_bytes(rows, width):
    """(code bytes, scale bytes) of a [rows][width] MXFP6 operand in the tiled layout."""
    c, s = ctypes.c_size_t(), ctypes.c_size_t()
    _check(load().l2c_mxfp6_bytes(rows, width, ctypes.byref(c), ctypes.byref(s)), "l2c_mxfp6_bytes")
    return c.value, s.value


def quantize_mxfp6(codes, scales, x, rows, width, stream=None):
    _check(load().l2c_quantize_mxfp6(_vp(_ptr(codes)), _vp(_ptr(scales)), _vp(_ptr(x)), rows, width,
                                     _vp(_stream(stream))), "l2c_quantize_mxfp6")


def nvfp4_tensor_scales(tensor_scales, x, n, partials, alpha=None, other_decode=None, stream=None):
    _check(load().l2c_nvfp4_tensor_scales(_vp(_ptr(tensor_scales)), _vp(_ptr(alpha)), _vp(_ptr(other_decode)),
                                          _vp(_ptr(x)), n, _vp(_ptr(partials)), _vp(_stream(stream))),
           "l2c_nvfp4_tensor_scales")


def nvfp4_tensor_scales_absmax(tensor_scales, absmax_bits, alpha=None, other_decode=None, stream=None):
    _check(load().l2c_nvfp4_tensor_scales_absmax(_vp(_ptr(tensor_scales)), _vp(_ptr(alpha)),
                                                 _vp(_ptr(other_decode)), _vp(_ptr(absmax_bits)),
                                                 _vp(_stream(stream))), "l2c_nvfp4_tensor_scales_absmax")


def quantize_nvfp4(codes, scales, x, tensor_scales, rows, width, expanded=None, stream=None):
    _check(load().l2c_quantize_nvfp4(_vp(_ptr(codes)), _vp(_ptr(scales)), _vp(_ptr(expanded)), _vp(_ptr(x)),
                                     _vp(_ptr(tensor_scales)), rows, width, _vp(_stream(stream))),
           "l2c_quantize_nvfp4")


def to_bf16_x4(out, inp, n, stream=None):
    _check(load().l2c_to_bf16_x4(_vp(_ptr(out)), _vp(_ptr(inp)), n, _vp(_stream(stream))), "l2c_to_bf16_x4")


def matmul_bf16(out, X, W, batch, cols, rows, alpha=None, stream=None):
    _check(load().l2c_matmul_bf16(_vp(_ptr(out)), _vp(_ptr(X)), _vp(_ptr(W)), _vp(_ptr(alpha)), batch, cols,
                                  rows, _vp(_stream(stream))), "l2c_matmul_bf16")


def matmul_mxfp6(out, X, Xscales, W, Wscales, batch, cols, rows, stream=None):
    _check(load().l2c_matmul_mxfp6(_vp(_ptr(out)), _vp(_ptr(X)), _vp(_ptr(Xscales)), _vp(_ptr(W)),
                                   _vp(_ptr(Wscales)), batch, cols, rows, _vp(_stream(stream))),
           "l2c_matmul_mxfp6")
