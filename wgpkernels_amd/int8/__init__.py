"""INT8 weight linears on AMD Instinct MI355X (gfx950):

    Y = op(X) @ (W * scales).T + bias            or, with a residual,   Y = R + residual_scale * (...)

W is a checkpoint's INT8 (N, K) matrix, used as stored (never dequantized or copied). scales are FP32 per channel (N,)
or per channel and 128-element K block (N, ceil(K / 128)). op is None, 'rms_norm', 'swiglu' or 'gelu', applied in FP32
while the activation is prepared.

A drop-in for the reference's `wgpkernels.int8` (wgpkernels/int8/__init__.py): the same public functions, arguments,
paths, fusions, errors and autotune behaviour. `from wgpkernels import int8` resolves to this module. The kernels are
hand-written HIP for gfx950 in libwgp_int8.so (built by `python -m wgpkernels_amd.build`), reached through its C-ABI
with ctypes. PyTorch supplies tensors and the current stream. Without the library every call raises: there is no CPU
fallback.

Paths:
- 'lines' (1-4 tokens): HBM-streaming GEMV with the activations unquantized.
- 'small' (up to 32 tokens): the INT8 weights converted exactly to BF16/FP16 on matrix cores.
- 'exact': INT8 matrix cores on x = s * (hi + lo / 254), two passes.
- 'block': one INT8 pass, one FP32 scale per token and 128-element K block.
- 'row': one scale per token (W8A8), on request only.
linear() picks a path per GPU, shape and token-count bucket by timing the candidates once (see choose_path()).
"""
import ctypes
import time
from contextvars import ContextVar
from pathlib import Path

import torch

from . import _native, _policy, _tuning
from ._native import ptr as _ptr
from ._policy import (DECIDE_MAX_ROWS, EXACT_ROWS, EXACT_TOLERANCE, LINE_MAX_ROWS, LINE_ROWS, SMALL_MAX_ROWS,  # noqa: F401
                      SMALL_ROWS, LinearShape)

# Quantized activations of the GEMM paths are made in row chunks of at most this many bytes. The reference allows
# 16 MiB (wgpkernels/int8/__init__.py:38); MI355X has 288 GB of HBM, so one chunk covers a 32760-token latent at
# K = 5120 and a long linear is one quantize launch and one GEMM launch.
SCRATCH_BYTES = 512 * 1024 * 1024
ACTS = {None: 0, "rms_norm": 1, "swiglu": 2, "gelu": 3}
DTYPES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
HIP_ARCHS = _native.HIP_ARCHS
# Rows of a chunk are a multiple of the long GEMM tile's token height.
CHUNK_ROW_MULTIPLE = 256

_lib = None
_sizes = (ctypes.c_int64 * 2)()
_tuning_quietly = ContextVar("wgpkernels_amd_int8_tuning_quietly", default=False)


# ---- library --------------------------------------------------------------------------------------------------------
def default_library_path():
    return Path(__file__).with_name("libwgp_int8.so")


def load_library(path=None):
    """Loads libwgp_int8.so (default: the one built next to this file), checks its ABI, binds its entry points,
    allocates each supported GPU's split counters and resolves its allocation-free GEMM array (so that nothing is
    allocated or looked up later under graph capture)."""
    global _lib
    lib = _native.Library(path or default_library_path())
    sizes = (ctypes.c_int64 * 2)()
    for index in _native.supported_gpus():
        _native.gpu(torch.device("cuda", index)).counters
        with torch.cuda.device(index):
            # a workspace query resolves the device's allocation-free GEMM array (no symbol lookup under capture later)
            lib.wq8_gemm_workspace(256, 256, 128, 10, 1, 0, sizes)
    _lib = lib
    return lib


def library():
    """The loaded library, loading the default one on first use."""
    return _lib if _lib is not None else load_library()


def weight_groups_supported():
    """Whether the loaded library takes per-(channel, 128-element K block) weight scales (N, ceil(K / 128))."""
    return _lib is not None and bool(_lib.features & _native.FEATURE_WEIGHT_GROUPS)


def segments_supported():
    """Whether the loaded library runs several linears of one input in one GEMM (linear_prepared_segments)."""
    return _lib is not None and _lib.has("wq8_gemm_segments")


def prepare_stream(stream):
    """Gives `stream` split counters of its own, so that its GEMMs may run at the same time as those of the GPU's other
    streams (which share one set). Call it outside graph capture, before the stream's first call."""
    if stream.cuda_stream not in _native.stream_counters:
        counters = torch.zeros(_native.COUNTER_INTS, dtype=torch.int32, device=stream.device)
        torch.cuda.current_stream(stream.device).synchronize()
        _native.stream_counters[stream.cuda_stream] = counters


# ---- argument checks ----------------------------------------------------------------------------------------------
def _op_width(x, act):
    """K of the linear fed by x: SwiGLU rows hold [gate | value]."""
    return x.shape[1] // 2 if act == "swiglu" else x.shape[1]


def _check_activation(x, aligned=True):
    """2-D with unit column stride; with `aligned`, 16-byte aligned start and row pitch (the quantizers load 16 bytes
    per lane from plain pointers; the few-token kernels load through buffer descriptors and take any pitch)."""
    if x.dim() != 2 or (x.shape[1] > 1 and x.stride(1) != 1):
        raise ValueError("activations must be 2-D with unit column stride")
    if aligned and (x.data_ptr() % 16 or (x.shape[0] > 1 and (x.stride(0) * x.element_size()) % 16)):
        raise ValueError("activation rows must be 16-byte aligned")
    if x.dtype not in DTYPES:
        raise ValueError(f"activations must be FP16, BF16 or FP32, not {x.dtype}")


def _row_pitch(x):
    """Elements between rows as the kernels read them. A one-row input's stride is meaningless (PyTorch reports
    (K, 1).t() as contiguous with stride (1, 1)), so its pitch is its width."""
    return x.stride(0) if x.shape[0] > 1 else x.shape[1]


def _is_block_mode(mode, sa):
    return mode.startswith("block") if mode else sa.dim() == 2


def _check_gemm(a, a_lo, sa, b, sb, y, mode):
    """Shapes the GEMM kernels read. They trust their arguments, so a mismatch raises here rather than reading past a
    buffer."""
    (m, k), n = a.shape, b.shape[0]
    kblocks = (k + 127) // 128
    if b.dim() != 2 or b.shape[1] != k or (a_lo is not None and a_lo.shape != a.shape) or tuple(y.shape) != (m, n):
        raise ValueError("INT8 GEMM operand shapes do not match")
    want_sa = m * kblocks if _is_block_mode(mode, sa) else m
    if sa.numel() != want_sa or sb.numel() not in (n, n * kblocks):
        raise ValueError(f"INT8 GEMM scale shapes do not match mode {mode or 'inferred'}: sa {tuple(sa.shape)}, sb {tuple(sb.shape)}")
    if any(t is not None and not t.is_contiguous() for t in (a, a_lo, sa, b, sb, y)):
        raise ValueError("INT8 GEMM operands must be contiguous")


def _has_weight_groups(sb):
    """Whether sb is per (channel, 128-element K block) rather than per channel."""
    if sb.dim() != 2:
        return False
    library()
    if not weight_groups_supported():
        raise RuntimeError("This INT8 library does not take per-(channel, k-block) weight scales; rebuild it")
    return True


# ---- activation preparation (reference: wgpkernels/int8/__init__.py:143-176) ---------------------------------------
def quantize_blocks(x, group=0, act=None, act_weight=None, eps=0.0):
    """INT8 of op(x) (ConvRot-rotated when group > 0) with one FP32 scale per row and 128-element block:
    (q (M, K) int8, scales (M, ceil(K / 128)) float32)."""
    lib = library()
    _check_activation(x)
    m, k = x.shape[0], _op_width(x, act)
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    scale = torch.empty((m, (k + 127) // 128), dtype=torch.float32, device=x.device)
    # RMSNorm over rows longer than the kernel keeps in registers computes the row norms first
    inv_rms = torch.empty(m, dtype=torch.float32, device=x.device) if act == "rms_norm" and k > 16384 else None
    lib.call("wq8_quantize_blocks", x.data_ptr(), q.data_ptr(), scale.data_ptr(), m, k, _row_pitch(x), DTYPES[x.dtype], group, ACTS[act],
             _ptr(act_weight), eps, _ptr(inv_rms), _native.gpu(x).stream())
    return q, scale


def quantize(x, group=0, hilo=False, act=None, act_weight=None, eps=0.0):
    """Row-wise symmetric INT8 of op(x) (ConvRot-rotated when group > 0): (hi, lo or None, FP32 row scales (M,))."""
    lib = library()
    _check_activation(x)
    m, k = x.shape[0], _op_width(x, act)
    hi = torch.empty((m, k), dtype=torch.int8, device=x.device)
    lo = torch.empty_like(hi) if hilo else None
    scale = torch.empty(m, dtype=torch.float32, device=x.device)
    lib.call("wq8_quantize", x.data_ptr(), hi.data_ptr(), _ptr(lo), scale.data_ptr(), m, k, _row_pitch(x), DTYPES[x.dtype], group, ACTS[act],
             _ptr(act_weight), eps, _native.gpu(x).stream())
    return hi, lo, scale


def transform_rows(x, group=0, act=None, act_weight=None, eps=0.0):
    """op(x), ConvRot-rotated, rounded once to x's dtype: the unquantized activation of the few-token paths."""
    lib = library()
    _check_activation(x)
    m, k = x.shape[0], _op_width(x, act)
    out = torch.empty((m, k), dtype=x.dtype, device=x.device)
    lib.call("wq8_transform_rows", x.data_ptr(), out.data_ptr(), m, k, _row_pitch(x), DTYPES[x.dtype], group, ACTS[act], _ptr(act_weight), eps,
             _native.gpu(x).stream())
    return out


def rotate_groups(x, group):
    """ConvRot rotation (groups of 16, 64 or 256), rounded once to the input dtype."""
    lib = library()
    _check_activation(x)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    lib.call("wq8_rotate_groups", x.data_ptr(), out.data_ptr(), x.shape[0], x.shape[1], _row_pitch(x), DTYPES[x.dtype], group,
             _native.gpu(x).stream())
    return out


# ---- GEMM tiles (reference: wgpkernels/int8/__init__.py:179-329) ------------------------------------------------------
# Variant ids keep the reference's modes (its int8_gemm.cu:1417-1432); the tiles behind them are this library's.
# Per mode: (long-tile variant, short-tile variant or None). The timed choice compares both, whole tiles only (split 0)
# and with the split-K tail (split 1: the tiles of an incomplete last wave split along K), as the reference times its
# stream-K (wgpkernels/int8/__init__.py:180-183).
# The block mode times 10 and 15, its tiles with the single-FMA biased fold (15, the short one, is an id the reference
# does not use); 11, the short tile in the reference's fold order, runs when asked for by id.
TILES = {"row": (0, 6), "exact": (1, 7), "block": (10, 15), "block+g": (12, 13), "exact+g": (14, None)}
VARIANT_MODES = {0: "row", 2: "row", 6: "row", 1: "exact", 7: "exact", 10: "block", 11: "block", 12: "block+g", 13: "block+g",
                 14: "exact+g", 15: "block"}


def tile_candidates(mode):
    """(variant, split) pairs the tile choice times for `mode`: the untimed default first."""
    return [(v, split) for v in TILES[mode] if v is not None for split in (1, 0)]


def _untimed_tile(mode, m, n, k, cus):
    """Tile of a shape nobody has timed yet (under capture): the library's wave-count estimate, with the split-K tail
    (as the reference's untimed choice, wgpkernels/int8/__init__.py:273-276)."""
    long_v, short_v = TILES[mode]
    base = "exact" if mode.startswith("exact") else "row"
    short = library().wq8_gemm_select(m, n, k, base == "exact", cus) in (6, 7)
    return (short_v if short and short_v is not None else long_v), 1


# (mode, M, N, K, device) -> (variant, split, slot bytes, counter bytes) of decided shapes
_plans = {}


def _tile_plan(a, a_lo, sa, b, sb, bias, y, mode, output_is_residual):
    (m, k), n = a.shape, b.shape[0]
    shape = (mode, m, n, k, b.device.index)
    plan = _plans.get(shape)
    if plan is not None:
        return plan
    state = _native.gpu(b)
    key = f"{mode}|{_tuning.gemm_rows_bucket(m)}x{n}x{k}|{state.name}"
    choice = _tuning.store.get(key)
    decided = choice is not None
    if choice is None and _tuning.is_capturing():
        choice = _untimed_tile(mode, m, n, k, state.cus)
    elif choice is None:
        # the timing writes its outputs: never into an output that is also the residual
        scratch = torch.empty_like(y) if output_is_residual else y
        label = f"INT8 GEMM {mode} {m}x{n}x{k}"
        loud = not _tuning_quietly.get()
        if loud:
            print(f"[WGPKernels] Autotuning {label}...", flush=True)
        started = time.time()
        runs = {c: (lambda c: lambda: gemm(a, a_lo, sa, b, sb, bias, y.dtype, c[1], c[0], scratch))(c) for c in tile_candidates(mode)}
        timings = _tuning.time_cold(library(), runs, b.device)
        choice = min(timings, key=timings.get)
        _tuning.store.put(key, list(choice))
        decided = True
        if loud:
            print(f"[WGPKernels] Selected {label}: tiles {choice[0]}, split {choice[1]} ({timings[choice] * 1000:.1f} us; "
                  f"tuned in {time.time() - started:.2f} s).", flush=True)
    variant, split = choice
    library().wq8_gemm_workspace(m, n, k, variant, state.cus, split, _sizes)
    plan = (variant, split, _sizes[0], _sizes[1])
    if decided:
        _plans[shape] = plan
    return plan


def _workspace(device, slot_bytes, counter_bytes, raw_stream):
    slots = torch.empty(slot_bytes, dtype=torch.uint8, device=device) if slot_bytes else None
    counters = _native.counters_for(_native.gpu(device), raw_stream, counter_bytes).data_ptr() if counter_bytes else None
    return slots, counters


def gemm(a, a_lo, sa, b, sb, bias, out_dtype, split=None, variant=None, out=None, mode=None, residual=None, residual_scale=None):
    """Y = epilogue(A @ B.T) of prepared INT8 activations. mode 'row' (sa per row), 'exact' (a_lo given) or 'block' (sa
    per row and 128-element block), inferred when omitted; sb per channel (N) or per (channel, K block) with 'exact' /
    'block'. residual (M, N) and residual_scale (N) in out_dtype: Y = residual + residual_scale * (A @ B.T + bias); out
    may be the residual. variant forces a tile configuration (no tuning), with split 0 (whole tiles) or 1 (the tiles of an
    incomplete last wave split along K, their partial sums added by the last piece to finish)."""
    lib = library()
    m, k = a.shape
    n = b.shape[0]
    y = torch.empty((m, n), dtype=out_dtype, device=a.device) if out is None else out
    forced = variant is not None
    if forced and variant not in VARIANT_MODES:
        raise ValueError(f"unknown INT8 GEMM variant {variant}")
    _check_gemm(a, a_lo, sa, b, sb, y, VARIANT_MODES[variant] if forced else mode)
    state = _native.gpu(a)
    if forced:
        split = split or 0
        lib.wq8_gemm_workspace(m, n, k, variant, state.cus, split, _sizes)
        slot_bytes, counter_bytes = _sizes[0], _sizes[1]
    else:
        mode = mode or ("exact" if a_lo is not None else "block" if sa.dim() == 2 else "row")
        if _has_weight_groups(sb):
            if mode == "row":
                raise ValueError("Weights with per-(n, k-block) scales run the 'block' or 'exact' path")
            mode += "+g"
        variant, split, slot_bytes, counter_bytes = _tile_plan(a, a_lo, sa, b, sb, bias, y, mode, residual is not None)
    stream = state.stream()
    slots, counters = _workspace(a.device, slot_bytes, counter_bytes, stream)
    lib.call("wq8_gemm", a.data_ptr(), _ptr(a_lo), sa.data_ptr(), b.data_ptr(), sb.data_ptr(), _ptr(bias), _ptr(residual), _ptr(residual_scale),
             y.data_ptr(), m, n, k, DTYPES[out_dtype], variant, state.cus, split, _ptr(slots), counters, stream)
    return y


# ---- few-token paths (reference: wgpkernels/int8/__init__.py:332-353) --------------------------------------------------
def small(x, weight, scale, bias=None, residual=None, residual_scale=None, out=None):
    """Up to 32 tokens, unquantized activations: INT8 weights converted exactly to 16-bit on matrix cores, FP32
    accumulation. K a multiple of 64."""
    lib = library()
    _check_activation(x, aligned=False)
    m, k = x.shape
    n = weight.shape[0]
    state = _native.gpu(x)
    y = torch.empty((m, n), dtype=x.dtype, device=x.device) if out is None else out
    lib.wq8_small_workspace(m, n, k, state.cus, _sizes)
    stream = state.stream()
    slots, counters = _workspace(x.device, _sizes[0], _sizes[1], stream)
    lib.call("wq8_small", x.data_ptr(), _row_pitch(x), weight.data_ptr(), scale.data_ptr(), _ptr(bias), _ptr(residual), _ptr(residual_scale),
             y.data_ptr(), m, n, k, DTYPES[x.dtype], state.cus, _ptr(slots), counters, stream)
    return y


def gemv_lines(x, weight, scale, bias=None, residual=None, residual_scale=None, out=None):
    """One to four tokens, unquantized activations: FP32 GEMV streaming the weight rows. K a multiple of 4."""
    lib = _lib if _lib is not None else load_library()
    _check_activation(x, aligned=False)
    m, k = x.shape
    y = torch.empty((m, weight.shape[0]), dtype=x.dtype, device=x.device) if out is None else out
    lib.call("wq8_gemv_lines", x.data_ptr(), _row_pitch(x), weight.data_ptr(), scale.data_ptr(), _ptr(bias), _ptr(residual),
             _ptr(residual_scale), y.data_ptr(), m, weight.shape[0], k, DTYPES[x.dtype], _native.gpu(x).stream())
    return y


# ---- prepared activations (reference: wgpkernels/int8/__init__.py:367-430) ----------------------------------------------
class Prepared:
    """An activation prepared for one path: unquantized (transformed, rotated) rows for 'lines' / 'small', INT8 rows and
    scales for 'exact' / 'block' / 'row'. One preparation serves every weight of the same K; rows() is a view."""
    __slots__ = ("path", "x", "lo", "scale", "dtype")

    def __init__(self, path, x, lo, scale, dtype):
        self.path, self.x, self.lo, self.scale, self.dtype = path, x, lo, scale, dtype

    def rows(self, start, stop):
        return Prepared(self.path, self.x[start:stop], None if self.lo is None else self.lo[start:stop],
                        None if self.scale is None else self.scale[start:stop], self.dtype)


def prepare(x, group=0, path="block", act=None, act_weight=None, eps=0.0):
    """op(x) prepared once for `path` (see choose_path()); x 2-D BF16/FP16 with 16-byte aligned rows, act_weight in
    x's dtype."""
    if path in ("lines", "small"):
        # the few-token kernels read 16-bit activations as they are: op and rotation are applied once, rounded to x's dtype
        if act:
            values = transform_rows(x, group, act, act_weight, eps)
        else:
            values = rotate_groups(x, group) if group else x
        return Prepared(path, values, None, None, x.dtype)
    if path == "block":
        q, scale = quantize_blocks(x, group, act, act_weight, eps)
        return Prepared(path, q, None, scale, x.dtype)
    if path in ("exact", "row"):
        hi, lo, scale = quantize(x, group, path == "exact", act, act_weight, eps)
        return Prepared(path, hi, lo, scale, x.dtype)
    raise ValueError(f"unknown INT8 path {path!r}")


def linear_prepared(prepared, weight, scale, bias=None, residual=None, residual_scale=None, out=None):
    """Y = prepared @ (weight * scale).T + bias (or residual + residual_scale * (...)); weight an INT8 (N, K) matrix or a
    row range of one."""
    if prepared.path in ("lines", "small"):
        if scale.dim() == 2:
            raise ValueError("Weights with per-(n, k-block) scales run the 'block' or 'exact' path")
        kernel = gemv_lines if prepared.path == "lines" else small
        return kernel(prepared.x, weight, scale, bias, residual, residual_scale, out)
    return gemm(prepared.x, prepared.lo, prepared.scale, weight, scale, bias, prepared.dtype, out=out, mode=prepared.path, residual=residual,
                residual_scale=residual_scale)


def linear_prepared_segments(prepared, weights, scales, biases, outputs):
    """outputs[s] = prepared @ (weights[s] * scales[s]).T + biases[s] for 1 to 4 linears in one GEMM launch ('exact',
    'block' or 'row' preparations, per-channel scales, equal row counts that are multiples of 8). The input is read once
    for all of them; the tile is the one decided for the joined shape."""
    lib = library()
    if not segments_supported():
        raise RuntimeError("the loaded INT8 library has no wq8_gemm_segments")
    a, count, rows = prepared.x, len(weights), weights[0].shape[0]
    m, k = a.shape
    n = count * rows
    plan = _plans.get((prepared.path, m, n, k, a.device.index))
    if plan is None:
        joined = torch.cat(weights)
        plan = _tile_plan(a, prepared.lo, prepared.scale, joined, torch.cat(scales), None, torch.empty((m, n), dtype=prepared.dtype, device=a.device),
                          prepared.path, False)
        del joined
    variant, split, slot_bytes, counter_bytes = plan
    state = _native.gpu(a)
    stream = state.stream()
    slots, counters = _workspace(a.device, slot_bytes, counter_bytes, stream)
    table = lambda tensors: (ctypes.c_void_p * 4)(*[_ptr(t) for t in tensors])
    lib.call("wq8_gemm_segments", a.data_ptr(), _ptr(prepared.lo), prepared.scale.data_ptr(), table(weights), table(scales), table(biases),
             table(outputs), count, rows, m, k, DTYPES[prepared.dtype], variant, state.cus, split, _ptr(slots), counters, stream)
    return outputs


# ---- linear (reference: wgpkernels/int8/__init__.py:433-520) ----------------------------------------------------------
def chunk_rows(mode, k):
    """Token rows per chunk of a GEMM path: the chunk's quantized activations stay within SCRATCH_BYTES."""
    kblocks = (k + 127) // 128
    row_bytes = {"exact": 2 * k + 4, "block": k + 4 * kblocks}.get(mode, k + 4)
    return max(CHUNK_ROW_MULTIPLE, SCRATCH_BYTES // row_bytes // CHUNK_ROW_MULTIPLE * CHUNK_ROW_MULTIPLE)


def _gemm_linear(path, x, weight, scale, bias, group, act, act_weight, eps, residual, residual_scale, out):
    m = x.shape[0]
    y = torch.empty((m, weight.shape[0]), dtype=x.dtype, device=x.device) if out is None else out
    step = chunk_rows(path, weight.shape[1])
    for start in range(0, m, step):
        stop = min(m, start + step)
        prepared = prepare(x[start:stop], group, path, act, act_weight, eps)
        linear_prepared(prepared, weight, scale, bias, None if residual is None else residual[start:stop], residual_scale, y[start:stop])
    return y


def _run_path(path, x, weight, scale, bias, group, act=None, act_weight=None, eps=0.0, residual=None, residual_scale=None, out=None):
    if path in ("lines", "small"):
        return linear_prepared(prepare(x, group, path, act, act_weight, eps), weight, scale, bias, residual, residual_scale, out)
    return _gemm_linear(path, x, weight, scale, bias, group, act, act_weight, eps, residual, residual_scale, out)


_decided_paths = {}  # (m, n, k, group, act, precise, weight groups, device index) -> path


def choose_path(x, weight, scale, bias=None, group=0, precise=False, act=None, act_weight=None, eps=0.0):
    """The path linear() takes: the fastest full-precision path while it costs at most EXACT_TOLERANCE more than 'block'
    (always a full-precision one with precise=True). Timed once per GPU, shape, input operation and token-count bucket on
    this call's input, with cold caches, and cached; a fixed rule applies where nothing may be timed."""
    m, k, n = x.shape[0], weight.shape[1], weight.shape[0]
    if m > DECIDE_MAX_ROWS and not precise:
        return "block"
    weight_groups = _has_weight_groups(scale)
    # a plain tuple: a decided call returns here without building the shape object (host time of a decode step)
    memo = (m, n, k, group, act, precise, weight_groups, x.get_device())
    path = _decided_paths.get(memo)
    if path is not None:
        return path
    shape = LinearShape(m, n, k, group, act, precise, weight_groups)
    state = _native.gpu(x)
    key = shape.key(_tuning.path_rows_bucket(m), state.name)
    path = _tuning.store.get(key)
    if path is None:
        if _tuning.is_capturing():
            return shape.untimed()
        label = (f"INT8 path {m}x{n}x{k}{f' ConvRot {group}' if group else ''}{f' {act}' if act else ''}"
                 f"{' (precise)' if precise else ''}")
        print(f"[WGPKernels] Autotuning {label}...", flush=True)
        started = time.time()
        quiet = _tuning_quietly.set(True)
        try:
            runs = {p: (lambda p: lambda: _run_path(p, x, weight, scale, bias, group, act, act_weight, eps))(p) for p in shape.candidates()}
            timings = _tuning.time_cold(library(), runs, x.device)
        finally:
            _tuning_quietly.reset(quiet)
        path = _policy.decide(timings, precise)
        _tuning.store.put(key, path)
        print(f"[WGPKernels] Selected {label}: {path} ({timings[path] * 1000:.1f} us; tuned in {time.time() - started:.2f} s).", flush=True)
    _decided_paths[memo] = path
    return path


def linear(x, weight, scale, bias=None, group=0, precise=False, mode=None, act=None, act_weight=None, eps=0.0, residual=None,
           residual_scale=None, out=None):
    """Y = op(X) @ (INT8 weight * FP32 scales).T + bias for 2-D BF16/FP16 X (16-byte aligned rows, unit column stride), or
    residual + residual_scale * (...) (X's dtype; out may be the residual). act: None, 'rms_norm' (act_weight: K values
    in X's dtype or None; eps), 'swiglu' (X rows [gate | value]) or 'gelu' (tanh approximation). mode forces a path
    ('lines', 'small', 'exact', 'block', 'row'); otherwise choose_path() decides."""
    path = mode or choose_path(x, weight, scale, bias, group, precise, act, act_weight, eps)
    return _run_path(path, x, weight, scale, bias, group, act, act_weight, eps, residual, residual_scale, out)


from ._selftest import reference_linear as _reference, reference_rotation as _reference_rotation, selftest  # noqa: E402,F401
