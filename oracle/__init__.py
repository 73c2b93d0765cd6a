"""CPU oracle of the INT8 weight linear -- TEST INFRASTRUCTURE ONLY.

Python (numpy + ctypes) front end of ``oracle/wq8_oracle.c``, the plain-C restatement of the reference's
arithmetic (wgpkernels/int8/int8_gemm.cu, wgpkernels/int8/__init__.py). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this package, and only as the
checker: the product path (``wgpkernels_amd``) never imports it.

Arrays are numpy. 16-bit floating-point tensors travel as ``uint16`` bit patterns with a ``dtype`` code
(0 = FP16, 1 = BF16, 2 = FP32), the codes of the reference's C-ABI (I:50).

Which oracle function is pinned by what (tests/test_oracle.py):
- exp / recip / logistic / gelu / swiglu: libm double precision error bounds over dense sweeps.
- ss_tree: float64 sum of squares within FP32 rounding; tree order pinned by a brute-force restatement.
- rotate_row: the closed form kron(H4, ...) of I:579-584.
- quantize_blocks / quantize: invariants (|q| <= 127, max |q| == 127 per nonzero block, scale * q
  reconstructs v within half a step, hi + lo / 254 within 1/508 step) and numpy restatements.
- block_sums / gemm: numpy int64 brute force for the sums, FP64 dequantize-and-matmul for the outputs.
- golden fixtures under tests/golden/ hold the oracle's outputs at the reference's config 1.
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
ACTS = {None: 0, "rms_norm": 1, "swiglu": 2, "gelu": 3}
DTYPES = {"float16": 0, "bfloat16": 1, "float32": 2}
_lib = None


def build(force=False):
    """Compiles liboracle.so with oracle/Makefile (gcc, -ffp-contract=off)."""
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < (HERE / "wq8_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-B" if force else "liboracle.so"], cwd=HERE, check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        p, i, i64, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        _lib.or_quantize_blocks.argtypes = [p, p, p, i, i, i64, i, i, i, p, f]
        _lib.or_quantize.argtypes = [p, p, p, p, i, i, i64, i, i, i, p, f]
        _lib.or_transform_rows.argtypes = [p, p, i, i, i64, i, i, i, p, f]
        _lib.or_rotate_groups.argtypes = [p, p, i, i, i64, i, i]
        _lib.or_block_sums.argtypes = [p, p, p, i, i, i]
        _lib.or_block_sums.restype = None
        _lib.or_gemm.argtypes = [p, p, p, p, p, p, p, p, p, i, i, i, i, i, i]
        _lib.or_gemm_pieces.argtypes = [p, p, p, p, p, p, p, p, p, i, i, i, i, i, i, i]
        _lib.or_linear_f64.argtypes = [p, i64, p, p, p, p, p, p, i, i, i, i]
        _lib.or_linear_f64.restype = None
        for name in ("or_to_dtype", "or_from_dtype"):
            getattr(_lib, name).argtypes = [p, p, i64, i]
            getattr(_lib, name).restype = None
        for name in ("or_exp_vec", "or_recip_vec", "or_logistic_vec", "or_gelu_vec"):
            getattr(_lib, name).argtypes = [p, p, i64]
            getattr(_lib, name).restype = None
        _lib.or_swiglu_vec.argtypes = [p, p, p, i64]
        _lib.or_swiglu_vec.restype = None
        _lib.or_ss_tree.argtypes = [p, i]
        _lib.or_ss_tree.restype = f
        _lib.or_rotate_row.argtypes = [p, i, i]
        _lib.or_rotate_row.restype = None
        _lib.or_check_div127.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        _lib.or_check_div127.restype = ctypes.c_longlong
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype=None):
    if a is None:
        return None
    a = np.ascontiguousarray(a if dtype is None else a.astype(dtype, copy=False))
    return a


def _check(code):
    if code:
        raise RuntimeError(f"oracle rejected the arguments (code {code})")


def _width(x, act):
    return x.shape[1] // 2 if act == "swiglu" else x.shape[1]


# ---- conversions ------------------------------------------------------------------------------
def to_dtype(v, dtype):
    """FP32 array -> uint16 bits (dtype 0 / 1, round to nearest even) or float32 (2)."""
    v = _c(v, np.float32)
    out = np.empty(v.shape, np.float32 if dtype == 2 else np.uint16)
    lib().or_to_dtype(_p(v), _p(out), v.size, dtype)
    return out


def from_dtype(bits, dtype):
    bits = _c(bits)
    out = np.empty(bits.shape, np.float32)
    lib().or_from_dtype(_p(bits), _p(out), bits.size, dtype)
    return out


# ---- element functions --------------------------------------------------------------------------
def _vec(name, x):
    x = _c(x, np.float32)
    out = np.empty_like(x)
    getattr(lib(), name)(_p(x), _p(out), x.size)
    return out


def exp(x):
    """exp on [-87, 80] (the range the logistic feeds it)."""
    return _vec("or_exp_vec", x)


def recip(x):
    """1 / x for x in [1, 2^116] by Newton steps."""
    return _vec("or_recip_vec", x)


def logistic(x):
    return _vec("or_logistic_vec", x)


def check_div127(lo, hi, step=1):
    """Bit patterns in [lo, hi) (every step-th) whose three-op division by 127 of the GPU kernels differs from the IEEE
    quotient."""
    return int(lib().or_check_div127(lo, hi, step))


def swiglu(g, u):
    g, u = _c(g, np.float32), _c(u, np.float32)
    out = np.empty_like(g)
    lib().or_swiglu_vec(_p(g), _p(u), _p(out), g.size)
    return out


def gelu(x):
    return _vec("or_gelu_vec", x)


def ss_tree(v):
    v = _c(v, np.float32)
    return float(lib().or_ss_tree(_p(v), v.shape[-1]))


def rotate_row(v, group):
    v = np.array(v, np.float32, copy=True)
    lib().or_rotate_row(_p(v), v.shape[-1], group)
    return v


# ---- quantizers (K8:269-485) ------------------------------------------------------------------
def quantize_blocks(x, dtype, group=0, act=None, act_weight=None, eps=0.0):
    """(q int8 (M, K), scale float32 (M, ceil(K/128))) of op(x)."""
    x = _c(x)
    m, k = x.shape[0], _width(x, act)
    q = np.empty((m, k), np.int8)
    scale = np.empty((m, (k + 127) // 128), np.float32)
    aw = _c(act_weight)
    _check(lib().or_quantize_blocks(_p(x), _p(q), _p(scale), m, k, x.shape[1], dtype, group, ACTS[act], _p(aw), eps))
    return q, scale


def quantize(x, dtype, group=0, hilo=False, act=None, act_weight=None, eps=0.0):
    """(hi int8, lo int8 or None, scale float32 (M,)) of op(x)."""
    x = _c(x)
    m, k = x.shape[0], _width(x, act)
    hi = np.empty((m, k), np.int8)
    lo = np.empty((m, k), np.int8) if hilo else None
    scale = np.empty(m, np.float32)
    aw = _c(act_weight)
    _check(lib().or_quantize(_p(x), _p(hi), _p(lo), _p(scale), m, k, x.shape[1], dtype, group, ACTS[act], _p(aw), eps))
    return hi, lo, scale


def transform_rows(x, dtype, group=0, act=None, act_weight=None, eps=0.0):
    x = _c(x)
    m, k = x.shape[0], _width(x, act)
    out = np.empty((m, k), np.float32 if dtype == 2 else np.uint16)
    aw = _c(act_weight)
    _check(lib().or_transform_rows(_p(x), _p(out), m, k, x.shape[1], dtype, group, ACTS[act], _p(aw), eps))
    return out


def rotate_groups(x, dtype, group):
    x = _c(x)
    out = np.empty(x.shape, np.float32 if dtype == 2 else np.uint16)
    _check(lib().or_rotate_groups(_p(x), _p(out), x.shape[0], x.shape[1], x.shape[1], dtype, group))
    return out


# ---- GEMM (K8:773-863) ------------------------------------------------------------------------
MODES = {"row": 0, "exact": 1, "block": 2, "block_biased": 3, "exact_combined": 4}


def block_sums(a, b):
    """Exact INT32 sums of each 128-element K block: (M, N, ceil(K/128))."""
    a, b = _c(a, np.int8), _c(b, np.int8)
    m, k = a.shape
    n = b.shape[0]
    out = np.empty((m, n, (k + 127) // 128), np.int32)
    lib().or_block_sums(_p(a), _p(b), _p(out), m, n, k)
    return out


def gemm(a, a_lo, sa, b, sb, bias, dtype, mode, residual=None, rscale=None, pieces=1):
    """Y (M, N) as uint16 bits in `dtype` (0 / 1). mode 'row' | 'exact' | 'block' (the reference's fold order) |
    'block_biased' (the single-FMA fold of the wide gfx950 kernel) | 'exact_combined' (weight groups only: the hi and lo
    block sums combined as integers, 254 H + L, then scaled by sb / 254: the gfx950 exact+g kernel's order); sb 2-D ->
    weight groups. pieces > 1: every output folded as a tile split along K into that many pieces of whole k-blocks (the
    split-K order: each piece folds its blocks from zero, the pieces add in order)."""
    a, b = _c(a, np.int8), _c(b, np.int8)
    a_lo = _c(a_lo, np.int8)
    sa, sb = _c(sa, np.float32), _c(sb, np.float32)
    bias, residual, rscale = _c(bias), _c(residual), _c(rscale)
    m, k = a.shape
    n = b.shape[0]
    y = np.empty((m, n), np.uint16)
    _check(lib().or_gemm_pieces(_p(a), _p(a_lo), _p(sa), _p(b), _p(sb), _p(bias), _p(residual), _p(rscale), _p(y), m, n, k, dtype,
                                MODES[mode], int(sb.ndim == 2), pieces))
    return y


def linear_f64(x, dtype, w, sw, bias=None, residual=None, rscale=None):
    """FP64-accumulated x @ (w * sw).T + bias (then residual) on prepared activations, as FP32 (unrounded)."""
    x, w, sw = _c(x), _c(w, np.int8), _c(sw, np.float32)
    bias, residual, rscale = _c(bias), _c(residual), _c(rscale)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    lib().or_linear_f64(_p(x), x.shape[1], _p(w), _p(sw), _p(bias), _p(residual), _p(rscale), _p(out), m, n, k, dtype)
    return out
