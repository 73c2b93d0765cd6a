"""INT8 weight linears on AMD Instinct MI355X (gfx950): Y = op(X) @ (W * scales).T + bias, with W the checkpoint's INT8
(N, K) matrix (never dequantized or copied) and FP32 per-channel scales (N,) or per-(channel, 128-element K block) scales
(N, ceil(K / 128)).

Drop-in for the reference's ``wgpkernels.int8`` (wgpkernels/int8/__init__.py, cited as I:<line>): the same functions,
argument meanings, paths, fusions, errors and autotune behaviour, over a C library built by ``python -m
wgpkernels_amd.build`` (``libwgp_int8.so``, hand-written HIP for gfx950, loaded with ctypes; PyTorch supplies tensors and
the current stream).

Paths, by precision:
- full precision: 'lines' (1-4 tokens, FP32 GEMV streaming the weights), 'small' (up to 32 tokens, INT8 weights converted
  exactly to BF16/FP16 on matrix cores), 'exact' (INT8 matrix cores on x ~= scale * (hi + lo / 254), two passes);
- 'block': one INT8 pass with one FP32 scale per token and 128-element K block;
- 'row': one scale per token (W8A8), on request only.
linear() takes the fastest full-precision path while it costs at most EXACT_TOLERANCE more than 'block', else 'block'; the
choice is timed per GPU, shape, input operation and token-count bucket on first use and cached in a JSON file.

Fusions: act='rms_norm' (optional weight), 'swiglu' (rows [gate | value]) or 'gelu' (tanh approximation), applied in FP32
while the activation is quantized; residual epilogue Y = R + residual_scale * (X @ W.T + bias) in FP32 with one rounding,
optionally in place of R.
"""
import ctypes
import functools
import json
import os
import time
from contextvars import ContextVar
from pathlib import Path

import torch

# Quantized activations of the GEMM paths are produced in row chunks of at most this many bytes (I:38). MI355X has 288 GB
# of HBM: one chunk covers a 32760-token video latent at K = 5120, so a long linear is one quantize + one GEMM launch.
SCRATCH_BYTES = 512 * 1024 * 1024
MAX_GRID_Y = 2 ** 31 - 1  # the gfx950 kernels put rows on grid X: no 65535-row limit (I:40)
EXACT_TOLERANCE = 0.10
# Fixed thresholds used when a choice cannot be timed (graph capture, torch.compile), and the candidate limits of the
# few-token paths (I:43-44).
EXACT_ROWS, LINE_ROWS, SMALL_ROWS = 64, 4, 32
LINE_MAX_ROWS, SMALL_MAX_ROWS, DECIDE_MAX_ROWS = 4, 32, 4096
ACTS = {None: 0, "rms_norm": 1, "swiglu": 2, "gelu": 3}
HIP_ARCHS = ("gfx950",)
_COUNTERS = 1024  # split counters of the C-ABI, as the workspace queries size them (this library's kernels ask for none)
_DTYPES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}

_lib = None
_weight_groups = False
_sms = {}
_counters = {}          # device index -> counters shared by the device's streams
_stream_counters = {}   # raw stream handle -> counters of a stream given its own (prepare_stream)
_sizes = (ctypes.c_int64 * 2)()


def default_library_path():
    return Path(__file__).with_name("libwgp_int8.so")


def weight_groups_supported():
    """Whether the loaded library takes per-(n, 128-element k-block) weight scales (N, ceil(K / 128))."""
    return _weight_groups


def load_library(path=None):
    """Loads the C library (default: the one built next to this file), checks its ABI and registers its argument types."""
    global _lib, _weight_groups
    target = Path(path or default_library_path()).resolve()
    if not target.exists():
        raise RuntimeError(f"INT8 library {target} not found: build it with `python -m wgpkernels_amd.build`")
    lib = ctypes.CDLL(str(target))
    if lib.wq8_abi() != 11:
        raise RuntimeError("INT8 GEMM library ABI mismatch; rebuild it")
    features = getattr(lib, "wq8_features", None)
    _weight_groups = bool(features and features() & 1)
    p, i, i64, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    lib.wq8_quantize.argtypes = [p, p, p, p, i, i, i64, i, i, i, p, f, p]
    lib.wq8_quantize_blocks.argtypes = [p, p, p, i, i, i64, i, i, i, p, f, p, p]
    lib.wq8_transform_rows.argtypes = [p, p, i, i, i64, i, i, i, p, f, p]
    lib.wq8_rotate_groups.argtypes = [p, p, i, i, i64, i, i, p]
    lib.wq8_l2_flush.argtypes = [i, i64, p]
    lib.wq8_l2_flush_release.restype = None
    lib.wq8_gemm.argtypes = [p, p, p, p, p, p, p, p, p, i, i, i, i, i, i, i, p, p, p]
    lib.wq8_gemm_workspace.argtypes = [i, i, i, i, i, i, p]
    lib.wq8_gemm_workspace.restype = None
    lib.wq8_gemm_select.argtypes = [i, i, i, i, i]
    lib.wq8_small.argtypes = [p, i64, p, p, p, p, p, p, i, i, i, i, i, p, p, p]
    lib.wq8_small_workspace.argtypes = [i, i, i, i, p]
    lib.wq8_small_workspace.restype = None
    lib.wq8_gemv_lines.argtypes = [p, i64, p, p, p, p, p, p, i, i, i, i, p]
    if hasattr(lib, "wq8_gemm_segments"):
        lib.wq8_gemm_segments.argtypes = [p, p, p, p, p, p, p, i, i, i, i, i, i, i, i, p, p, p]
    for index in range(torch.cuda.device_count()):
        # only the GPUs the library is built for
        if torch.cuda.get_device_properties(index).gcnArchName.split(":")[0] in HIP_ARCHS:
            _counters.setdefault(index, torch.zeros(_COUNTERS, dtype=torch.int32, device=torch.device("cuda", index)))
    _lib = lib
    return lib


def _library():
    """The loaded library; loads the default one on first use. Raises when it is missing (there is no CPU fallback)."""
    return _lib if _lib is not None else load_library()


def _check(code):
    if code:
        raise RuntimeError(f"INT8 GEMM launch failed (HIP error {code})" if code > 0 else f"INT8 GEMM call rejected its arguments (code {code})")


def _ptr(tensor):
    return None if tensor is None else tensor.data_ptr()


def _stream(device):
    # the raw hipStream_t of the device's current stream (I:107-108); 0.07 us per call against 1.8 for current_stream()
    return torch._C._cuda_getCurrentRawStream(device.index if device.index is not None else torch.cuda.current_device())


def _sm_count(device):
    index = device.index if device.index is not None else torch.cuda.current_device()
    count = _sms.get(index)
    if count is None:
        count = _sms[index] = torch.cuda.get_device_properties(index).multi_processor_count
    return count


def prepare_stream(stream):
    """Gives `stream` its own split-K counters so that its GEMMs may run concurrently with those of the device's other
    streams (which share one set). Call outside graph capture, before the stream's first call. The reference's API: this
    library's kernels request no counters (their split partials are per-call scratch), so the set is never used."""
    if stream.cuda_stream not in _stream_counters:
        counters = torch.zeros(_COUNTERS, dtype=torch.int32, device=stream.device)
        torch.cuda.current_stream(stream.device).synchronize()
        _stream_counters[stream.cuda_stream] = counters


def _zeroed_counters(device, size, stream):
    """Split counters (zero, left zero by the kernels): the stream's own (prepare_stream) or the device's shared set."""
    if size > _COUNTERS * 4:
        raise RuntimeError("INT8 GEMM split-K counters exceeded")
    own = _stream_counters.get(stream)
    if own is not None:
        return own
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _counters:
        _counters[index] = torch.zeros(_COUNTERS, dtype=torch.int32, device=device)
    return _counters[index]


def _width(x, act):
    """K of the linear fed by x: SwiGLU rows hold the gate and value halves."""
    return x.shape[1] // 2 if act == "swiglu" else x.shape[1]


def _check_rows(x):
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("activations must be 2-D with unit column stride")
    if x.data_ptr() % 16 or (x.shape[0] > 1 and (x.stride(0) * x.element_size()) % 16):
        raise ValueError("activation rows must be 16-byte aligned")


# ---- activation preparation (I:143-176) ---------------------------------------------------------------------
def quantize_blocks(x, group=0, act=None, act_weight=None, eps=0.0):
    """INT8 of op(x) (optionally ConvRot-rotated) with one FP32 scale per row and 128-element block:
    (q (M, K) int8, scales (M, ceil(K / 128)) float32)."""
    lib = _library()
    _check_rows(x)
    m, k = x.shape[0], _width(x, act)
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    scale = torch.empty((m, (k + 127) // 128), dtype=torch.float32, device=x.device)
    inv_rms = torch.empty(m, dtype=torch.float32, device=x.device) if act == "rms_norm" and k > 16384 else None
    _check(lib.wq8_quantize_blocks(x.data_ptr(), q.data_ptr(), scale.data_ptr(), m, k, x.stride(0), _DTYPES[x.dtype], group, ACTS[act],
                                   _ptr(act_weight), eps, _ptr(inv_rms), _stream(x.device)))
    return q, scale


def quantize(x, group=0, hilo=False, act=None, act_weight=None, eps=0.0):
    """Row-wise symmetric INT8 of op(x) (optionally ConvRot-rotated): (hi, lo or None, FP32 row scales (M,))."""
    lib = _library()
    _check_rows(x)
    m, k = x.shape[0], _width(x, act)
    hi = torch.empty((m, k), dtype=torch.int8, device=x.device)
    lo = torch.empty_like(hi) if hilo else None
    scale = torch.empty(m, dtype=torch.float32, device=x.device)
    _check(lib.wq8_quantize(x.data_ptr(), hi.data_ptr(), _ptr(lo), scale.data_ptr(), m, k, x.stride(0), _DTYPES[x.dtype], group, ACTS[act],
                            _ptr(act_weight), eps, _stream(x.device)))
    return hi, lo, scale


def transform_rows(x, group=0, act=None, act_weight=None, eps=0.0):
    """op(x), ConvRot-rotated, rounded once to x's dtype: the unquantized activation of the few-token paths."""
    lib = _library()
    _check_rows(x)
    m, k = x.shape[0], _width(x, act)
    out = torch.empty((m, k), dtype=x.dtype, device=x.device)
    _check(lib.wq8_transform_rows(x.data_ptr(), out.data_ptr(), m, k, x.stride(0), _DTYPES[x.dtype], group, ACTS[act], _ptr(act_weight), eps,
                                  _stream(x.device)))
    return out


def rotate_groups(x, group):
    """ConvRot rotation (groups of 16, 64 or 256), rounded once to the input dtype."""
    lib = _library()
    _check_rows(x)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _check(lib.wq8_rotate_groups(x.data_ptr(), out.data_ptr(), x.shape[0], x.shape[1], x.stride(0), _DTYPES[x.dtype], group, _stream(x.device)))
    return out


# ---- GEMM tile autotuning (I:179-293) -------------------------------------------------------------------------
# (variant, split) candidates per mode; the first is the untuned default. The gfx950 library runs whole tiles (split is
# accepted and ignored), its variants differ by tile height: 128 (0, 1, 10, 12, 14) or 32 tokens (6, 7, 11, 13).
_CANDIDATES = {'row': ((0, 0), (6, 0)), 'exact': ((1, 0), (7, 0)), 'block': ((10, 0), (11, 0)),
               'exact+g': ((14, 0),), 'block+g': ((12, 0), (13, 0))}
_MODES = {0: 'row', 2: 'row', 6: 'row', 1: 'exact', 7: 'exact', 10: 'block', 11: 'block', 12: 'block+g', 13: 'block+g', 14: 'exact+g'}
_TUNING_VERSION = 1
_TUNING_PATH = Path(os.environ.get("WGPKERNELS_AMD_CACHE", Path.home() / ".triton" / "autotune" / "wgpkernels_amd_int8.json"))
_tuned = None
_path_tuning = ContextVar("wgpkernels_amd_int8_path_tuning", default=False)


@functools.cache
def _device_name(index):
    props = torch.cuda.get_device_properties(index)
    return f"{props.gcnArchName.split(':')[0]}x{props.multi_processor_count}"


def _rows_bucket(m):
    return -(-m // 64) * 64 if m <= 4096 else min(1 << (m - 1).bit_length(), 16384)


def _cache():
    global _tuned
    if _tuned is None:
        try:
            payload = json.loads(_TUNING_PATH.read_text(encoding="utf-8"))
            _tuned = payload["configs"] if payload.get("version") == _TUNING_VERSION else {}
            if not isinstance(_tuned, dict):
                _tuned = {}
        except (OSError, ValueError, KeyError, TypeError, AttributeError):
            _tuned = {}
    return _tuned


def _save_cache():
    try:
        _TUNING_PATH.parent.mkdir(parents=True, exist_ok=True)
        _TUNING_PATH.write_text(json.dumps({"version": _TUNING_VERSION, "configs": _cache()}, indent=1), encoding="utf-8")
    except OSError as error:
        print(f"[INT8] Could not save the INT8 GEMM tuning cache {_TUNING_PATH}: {error}")


def _flush_bytes(device):
    # more than every L2 (4 MiB per XCD, 8 XCDs) plus the 256 MiB Infinity Cache, so that weights come from HBM
    l2 = torch.cuda.get_device_properties(device).L2_cache_size
    return 2 * (8 * l2 + 256 * 1024 * 1024)


def _best_of(launches, device):
    """Best time in ms of each launch(): three rounds in alternating order, each timed launch after a cold-cache read of a
    library-owned buffer larger than L2 + MALL (outside PyTorch's allocator). Back-to-back launches when it cannot be
    allocated."""
    lib = _library()
    names = list(launches)
    for name in names:
        launches[name]()
    flush, stream = _flush_bytes(device), _stream(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    cold = lib.wq8_l2_flush(index, flush, stream) == 0
    timings = {name: float("inf") for name in names}
    try:
        for round_index in range(3):
            for name in (names if round_index % 2 == 0 else names[::-1]):
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                if cold:
                    _check(lib.wq8_l2_flush(index, flush, stream))
                start.record()
                for _ in range(1 if cold else 3):
                    launches[name]()
                end.record()
                end.synchronize()
                timings[name] = min(timings[name], start.elapsed_time(end) / (1 if cold else 3))
    finally:
        lib.wq8_l2_flush_release()
    return timings


def _tuned_config(a, a_lo, sa, b, sb, bias, y, mode):
    """((variant, split), tuned) for this shape bucket: cached, timed now, or the untuned default under capture."""
    (m, k), n = a.shape, b.shape[0]
    key = f"{mode}|{_rows_bucket(m)}x{n}x{k}|{_device_name(b.device.index)}"
    config = _cache().get(key)
    if config is not None:
        return tuple(config), True
    if torch.cuda.is_current_stream_capturing() or torch.compiler.is_compiling():
        if mode in ('block', 'block+g', 'exact+g'):
            return _CANDIDATES[mode][0], False
        return (_library().wq8_gemm_select(m, n, k, mode == 'exact', _sm_count(b.device)), 0), False
    started = time.time()
    log = not _path_tuning.get()
    label = f"INT8 GEMM {mode} {m}x{n}x{k}"
    if log:
        print(f"[WGPKernels] Autotuning {label}...", flush=True)
    timings = _best_of({config: (lambda config: lambda: gemm(a, a_lo, sa, b, sb, bias, y.dtype, config[1], config[0], y))(config)
                        for config in _CANDIDATES[mode]}, b.device)
    best_ms, best = min((ms, config) for config, ms in timings.items())
    _cache()[key] = list(best)
    _save_cache()
    if log:
        print(f"[WGPKernels] Selected {label}: tiles {best[0]}, split {best[1]} ({best_ms * 1000:.1f} us; tuned in {time.time() - started:.2f} s).",
              flush=True)
    return best, True


_plans = {}  # (mode, M, N, K, device) -> (variant, split, slot bytes, counter bytes)


def _plan(a, a_lo, sa, b, sb, bias, y, mode, scratch_output):
    (m, k), n = a.shape, b.shape[0]
    shape = (mode, m, n, k, b.device.index)
    plan = _plans.get(shape)
    if plan is not None:
        return plan
    (variant, split), tuned = _tuned_config(a, a_lo, sa, b, sb, bias, torch.empty_like(y) if scratch_output else y, mode)
    _library().wq8_gemm_workspace(m, n, k, variant, _sm_count(b.device), split, _sizes)
    plan = (variant, split, _sizes[0], _sizes[1])
    if tuned:
        _plans[shape] = plan
    return plan


def _weight_scale_groups(sb):
    """Whether sb holds one scale per output channel and 128-element K block (N, ceil(K / 128))."""
    if sb.dim() != 2:
        return False
    if not _weight_groups:
        raise RuntimeError("This INT8 library predates per-(n, k-block) weight scales; rebuild it")
    return True


def _check_gemm_operands(a, a_lo, sa, b, sb, y, mode):
    """Shapes the kernels read (they trust their arguments, as the reference's do): a mismatch raises instead of reading
    past a buffer."""
    (m, k), n, kb = a.shape, b.shape[0], (a.shape[1] + 127) // 128
    block = (mode or '').startswith('block') or (mode is None and sa.dim() == 2)
    if b.shape[1] != k or (a_lo is not None and a_lo.shape != a.shape) or tuple(y.shape) != (m, n):
        raise ValueError("INT8 GEMM operand shapes do not match")
    if sa.numel() != (m * kb if block else m) or sb.numel() not in (n, n * kb):
        raise ValueError(f"INT8 GEMM scale shapes do not match mode {mode or 'inferred'}: sa {tuple(sa.shape)}, sb {tuple(sb.shape)}")
    for t in (a, a_lo, sa, b, sb, y):
        if t is not None and not t.is_contiguous():
            raise ValueError("INT8 GEMM operands must be contiguous")


def gemm(a, a_lo, sa, b, sb, bias, out_dtype, split=None, variant=None, out=None, mode=None, residual=None, residual_scale=None):
    """Y = epilogue(A @ B.T): mode 'row' (sa per row), 'exact' (a_lo given) or 'block' (sa per row and 128-element block),
    inferred when omitted; sb per channel (N) or per (channel, 128-element K block) with 'exact' / 'block'. residual (M, N) and
    residual_scale (N) in out_dtype: Y = residual + residual_scale * (A @ B.T + bias); out may be the residual."""
    lib = _library()
    m, k = a.shape
    n = b.shape[0]
    sms = _sm_count(a.device)
    y = torch.empty((m, n), dtype=out_dtype, device=a.device) if out is None else out
    _check_gemm_operands(a, a_lo, sa, b, sb, y, mode if variant is None else _MODES.get(variant, mode))
    if variant is None and split is None:
        mode = mode or ('exact' if a_lo is not None else 'block' if sa.dim() == 2 else 'row')
        if _weight_scale_groups(sb):
            if mode == 'row':
                raise ValueError("Weights with per-(n, k-block) scales run the 'block' or 'exact' path")
            mode += '+g'
        variant, split, slot_bytes, counter_bytes = _plan(a, a_lo, sa, b, sb, bias, y, mode, residual is not None)
    else:
        split = 0 if split is None else split
        lib.wq8_gemm_workspace(m, n, k, variant, sms, split, _sizes)
        slot_bytes, counter_bytes = _sizes[0], _sizes[1]
    slots = torch.empty(slot_bytes, dtype=torch.uint8, device=a.device) if slot_bytes else None
    stream = _stream(a.device)
    counters = _zeroed_counters(a.device, counter_bytes, stream).data_ptr() if counter_bytes else None
    _check(lib.wq8_gemm(a.data_ptr(), _ptr(a_lo), sa.data_ptr(), b.data_ptr(), sb.data_ptr(), _ptr(bias), _ptr(residual), _ptr(residual_scale),
                        y.data_ptr(), m, n, k, _DTYPES[out_dtype], variant, sms, split, _ptr(slots), counters, stream))
    return y


def small(x, weight, scale, bias=None, residual=None, residual_scale=None, out=None):
    """Weight-only INT8 for at most 32 tokens: unquantized activations, FP32 accumulation on matrix cores. K multiple of 64."""
    lib = _library()
    m, k = x.shape
    n = weight.shape[0]
    sms = _sm_count(x.device)
    y = torch.empty((m, n), dtype=x.dtype, device=x.device) if out is None else out
    lib.wq8_small_workspace(m, n, k, sms, _sizes)
    slots = torch.empty(_sizes[0] // 4, dtype=torch.float32, device=x.device) if _sizes[0] else None
    stream = _stream(x.device)
    counters = _zeroed_counters(x.device, _sizes[1], stream).data_ptr() if _sizes[1] else None
    _check(lib.wq8_small(x.data_ptr(), x.stride(0), weight.data_ptr(), scale.data_ptr(), _ptr(bias), _ptr(residual), _ptr(residual_scale),
                         y.data_ptr(), m, n, k, _DTYPES[x.dtype], sms, _ptr(slots), counters, stream))
    return y


def gemv_lines(x, weight, scale, bias=None, residual=None, residual_scale=None, out=None):
    """One to four tokens, unquantized activations, FP32 GEMV streaming the weight rows (K multiple of 4)."""
    lib = _library()
    m, k = x.shape
    y = torch.empty((m, weight.shape[0]), dtype=x.dtype, device=x.device) if out is None else out
    _check(lib.wq8_gemv_lines(x.data_ptr(), x.stride(0), weight.data_ptr(), scale.data_ptr(), _ptr(bias), _ptr(residual), _ptr(residual_scale),
                              y.data_ptr(), m, weight.shape[0], k, _DTYPES[x.dtype], _stream(x.device)))
    return y


class Prepared:
    """An activation prepared for one path: the unquantized (transformed, rotated) rows of 'lines' / 'small', or the INT8
    rows and scales of 'exact' / 'block' / 'row'. Rows can be sliced; one preparation serves every weight of the same K."""
    __slots__ = ("path", "x", "lo", "scale", "dtype")

    def __init__(self, path, x, lo, scale, dtype):
        self.path, self.x, self.lo, self.scale, self.dtype = path, x, lo, scale, dtype

    def rows(self, start, stop):
        cut = lambda t: None if t is None else t[start:stop]
        return Prepared(self.path, self.x[start:stop], cut(self.lo), cut(self.scale), self.dtype)


def prepare(x, group=0, path="block", act=None, act_weight=None, eps=0.0):
    """op(x) prepared once for `path` (choose_path()); x 2-D BF16/FP16 with 16-byte aligned rows; act_weight in x's dtype."""
    if path in ("lines", "small"):
        prepared = transform_rows(x, group, act, act_weight, eps) if act else rotate_groups(x, group) if group else x
        return Prepared(path, prepared, None, None, x.dtype)
    if path == "block":
        q, scale = quantize_blocks(x, group, act, act_weight, eps)
        return Prepared(path, q, None, scale, x.dtype)
    if path not in ("exact", "row"):
        raise ValueError(f"unknown INT8 path {path!r}")
    hi, lo, scale = quantize(x, group, path == "exact", act, act_weight, eps)
    return Prepared(path, hi, lo, scale, x.dtype)


def linear_prepared(prepared, weight, scale, bias=None, residual=None, residual_scale=None, out=None):
    """Y = prepared @ (weight * scale).T + bias (or residual + residual_scale * (...)); weight an INT8 (N, K) matrix or row range."""
    if prepared.path in ("lines", "small") and scale.dim() == 2:
        raise ValueError("Weights with per-(n, k-block) scales run the 'block' or 'exact' path")
    if prepared.path == "lines":
        return gemv_lines(prepared.x, weight, scale, bias, residual, residual_scale, out)
    if prepared.path == "small":
        return small(prepared.x, weight, scale, bias, residual, residual_scale, out)
    return gemm(prepared.x, prepared.lo, prepared.scale, weight, scale, bias, prepared.dtype, out=out, mode=prepared.path, residual=residual,
                residual_scale=residual_scale)


def segments_supported():
    """Whether the loaded library computes several linears of one input in one GEMM (linear_prepared_segments)."""
    return _lib is not None and hasattr(_lib, "wq8_gemm_segments")


def linear_prepared_segments(prepared, weights, scales, biases, outputs):
    """outputs[s] = prepared @ (weights[s] * scales[s]).T + biases[s] for 1 to 4 linears in one GEMM ('exact', 'block' or 'row'
    preparations; per-channel scales; rows a multiple of 8): the input is read once for all of them."""
    lib = _library()
    a, count, rows = prepared.x, len(weights), weights[0].shape[0]
    m, k = a.shape
    n = count * rows
    plan = _plans.get((prepared.path, m, n, k, a.device.index))
    if plan is None:  # planned once as one weight of N rows: the launch's own shape
        joined = torch.cat(weights)
        plan = _plan(a, prepared.lo, prepared.scale, joined, torch.cat(scales), None, torch.empty((m, n), dtype=prepared.dtype, device=a.device),
                     prepared.path, False)
        del joined
    variant, split, slot_bytes, counter_bytes = plan
    slots = torch.empty(slot_bytes, dtype=torch.uint8, device=a.device) if slot_bytes else None
    stream = _stream(a.device)
    counters = _zeroed_counters(a.device, counter_bytes, stream).data_ptr() if counter_bytes else None
    pointers = lambda tensors: (ctypes.c_void_p * 4)(*[None if t is None else t.data_ptr() for t in tensors])
    _check(lib.wq8_gemm_segments(a.data_ptr(), _ptr(prepared.lo), prepared.scale.data_ptr(), pointers(weights), pointers(scales), pointers(biases),
                                 pointers(outputs), count, rows, m, k, _DTYPES[prepared.dtype], variant, _sm_count(a.device), split, _ptr(slots),
                                 counters, stream))
    return outputs


def _gemm_path(x, weight, scale, bias, group, mode, act=None, act_weight=None, eps=0.0, residual=None, residual_scale=None, out=None):
    """'exact', 'block' or 'row' over row chunks whose quantized activations stay within SCRATCH_BYTES (I:433-444)."""
    m, k = x.shape[0], weight.shape[1]
    out = torch.empty((m, weight.shape[0]), dtype=x.dtype, device=x.device) if out is None else out
    row_bytes = (2 * k if mode == 'exact' else k) + 4 * (-(-k // 128) if mode == 'block' else 1)
    rows = max(128, SCRATCH_BYTES // row_bytes // 128 * 128)
    for start in range(0, m, rows):
        stop = min(start + rows, m)
        prepared = prepare(x[start:stop], group, mode, act, act_weight, eps)
        linear_prepared(prepared, weight, scale, bias, None if residual is None else residual[start:stop], residual_scale, out[start:stop])
        del prepared
    return out


def _run(path, x, weight, scale, bias, group, act=None, act_weight=None, eps=0.0, residual=None, residual_scale=None, out=None):
    if path in ('lines', 'small'):
        return linear_prepared(prepare(x, group, path, act, act_weight, eps), weight, scale, bias, residual, residual_scale, out)
    return _gemm_path(x, weight, scale, bias, group, path, act, act_weight, eps, residual, residual_scale, out)


# ---- path choice (I:453-509) --------------------------------------------------------------------------------------
def _precise_paths(m, k, groups=False):
    """Full-precision candidates; weights with per-(n, k-block) scales only have 'exact'."""
    return [path for path, ok in (('lines', m <= LINE_MAX_ROWS and k % 4 == 0 and not groups),
                                  ('small', m <= SMALL_MAX_ROWS and k % 64 == 0 and not groups), ('exact', True)) if ok]


def _static_path(m, k, precise, groups=False):
    if m <= LINE_ROWS and k % 4 == 0 and not groups:
        return 'lines'
    if m <= SMALL_ROWS and k % 64 == 0 and not groups:
        return 'small'
    return 'exact' if precise or m <= EXACT_ROWS else 'block'


def _path_bucket(m):
    return m if m <= 16 else -(-m // 8) * 8 if m <= 128 else _rows_bucket(m)


_paths = {}  # (M, N, K, group, act, precise, device, groups) -> path


def choose_path(x, weight, scale, bias=None, group=0, precise=False, act=None, act_weight=None, eps=0.0):
    """Fastest full-precision path while it costs at most EXACT_TOLERANCE more than 'block' (always with precise=True), timed
    on this call's input per GPU, shape, input operation and token-count bucket."""
    (m, k), n = (x.shape[0], weight.shape[1]), weight.shape[0]
    if m > DECIDE_MAX_ROWS and not precise:
        return 'block'
    groups = _weight_scale_groups(scale)
    shape = (m, n, k, group, act, precise, x.device.index, groups)
    path = _paths.get(shape)
    if path is not None:
        return path
    key = (f"path{'+precise' if precise else ''}|{_path_bucket(m)}x{n}x{k}|g{group}{f'|{act}' if act else ''}{'|wgroups' if groups else ''}"
           f"|{_device_name(x.device.index)}")
    path = _cache().get(key)
    if path is not None:
        _paths[shape] = path
        return path
    if torch.cuda.is_current_stream_capturing() or torch.compiler.is_compiling():
        return _static_path(m, k, precise, groups)
    candidates = _precise_paths(m, k, groups) + ([] if precise else ['block'])
    label = f"INT8 path {m}x{n}x{k}{f' ConvRot {group}' if group else ''}{f' {act}' if act else ''}{' (precise)' if precise else ''}"
    started = time.time()
    print(f"[WGPKernels] Autotuning {label}...", flush=True)
    token = _path_tuning.set(True)
    try:
        timings = _best_of({p: (lambda p: lambda: _run(p, x, weight, scale, bias, group, act, act_weight, eps))(p) for p in candidates}, x.device)
    finally:
        _path_tuning.reset(token)
    full_ms, path = min((timings[p], p) for p in candidates if p != 'block')
    if not precise and full_ms > (1 + EXACT_TOLERANCE) * timings['block']:
        path = 'block'
    _cache()[key] = _paths[shape] = path
    _save_cache()
    print(f"[WGPKernels] Selected {label}: {path} ({timings[path] * 1000:.1f} us; tuned in {time.time() - started:.2f} s).", flush=True)
    return path


def linear(x, weight, scale, bias=None, group=0, precise=False, mode=None, act=None, act_weight=None, eps=0.0, residual=None,
           residual_scale=None, out=None):
    """Y = op(X) @ (INT8 weight * FP32 scales).T + bias for 2-D BF16/FP16 X (rows 16-byte aligned, unit column stride), or
    residual + residual_scale * (...) (X's dtype; out may be the residual). act: None, 'rms_norm' (act_weight: K values in X's
    dtype or None; eps), 'swiglu' (X rows: gate | value) or 'gelu'. mode forces a path ('lines', 'small', 'exact', 'block',
    'row'); by default the path is chosen by choose_path()."""
    path = mode or choose_path(x, weight, scale, bias, group, precise, act, act_weight, eps)
    return _run(path, x, weight, scale, bias, group, act, act_weight, eps, residual, residual_scale, out)


# ---- self test (I:523-576) --------------------------------------------------------------------------------------
def _reference(x, w, s, bias, group, act, act_weight, eps, residual, residual_scale, round_input):
    """FP32 reference of linear(); round_input rounds op(x) to x's dtype as the few-token paths do."""
    v = x.float()
    if act == "swiglu":
        gate, value = v.chunk(2, dim=-1)
        v = torch.nn.functional.silu(gate) * value
    elif act == "rms_norm":
        v = v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps) * (1 if act_weight is None else act_weight.float())
    elif act == "gelu":
        v = torch.nn.functional.gelu(v, approximate="tanh")
    if group:
        v = _reference_rotation(v, group)
    if round_input:
        v = v.to(x.dtype).float()
    scale = s.repeat_interleave(128, dim=1)[:, :w.shape[1]] if s.dim() == 2 else s[:, None]
    out = v @ (w.float() * scale).T + (0 if bias is None else bias.float())
    return out if residual is None else residual.float() + (1 if residual_scale is None else residual_scale.float()) * out


def _reference_rotation(v, group):
    """ConvRot: each group of `group` values times kron(H4, ..., H4) / sqrt(group), H4 = ones - 2 * antidiagonal."""
    h = torch.ones(4, 4, device=v.device) - 2 * torch.eye(4, device=v.device).flip(0)
    rotation = h
    while rotation.shape[0] < group:
        rotation = torch.kron(rotation, h)
    return (v.reshape(v.shape[0], -1, group) @ (rotation * group ** -0.5)).reshape(v.shape)


def selftest(device=None):
    """Runs every kernel once on small inputs with fixed configurations (no tuning): None when the results match PyTorch,
    else the reason."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    generator = torch.Generator(device=device).manual_seed(0)
    variants = {"exact": 7, "block": 11, "row": 6, "exact+g": 14, "block+g": 13}
    cases = [(1, "lines", 0, None, False), (5, "small", 0, None, False), (5, "small", 64, None, False), (40, "exact", 0, None, False),
             (40, "block", 256, None, False), (40, "row", 16, None, False), (2, "lines", 0, "swiglu", True), (5, "small", 64, "rms_norm", True),
             (40, "exact", 256, "rms_norm", False), (40, "block", 0, "swiglu", True), (40, "block", 16, "rms_norm", True),
             (40, "exact", 64, None, True), (3, "lines", 64, "gelu", False), (5, "small", 0, "gelu", True), (40, "exact", 16, "gelu", False),
             (40, "block", 256, "gelu", True)]
    _library()
    if _weight_groups:  # weights with per-(n, k-block) scales
        cases += [(40, "exact+g", 0, None, True), (40, "block+g", 64, "rms_norm", False), (40, "block+g", 0, None, True)]
    for dtype in (torch.bfloat16, torch.float16):
        w = torch.randint(-127, 128, (96, 256), dtype=torch.int8, device=device, generator=generator)
        s = torch.rand(96, device=device, generator=generator) / 127
        s_groups = torch.rand(96, 2, device=device, generator=generator) / 127
        bias = torch.randn(96, dtype=dtype, device=device, generator=generator)
        norm_weight = (torch.rand(256, device=device, generator=generator) + 0.5).to(dtype)
        for m, path, group, act, with_residual in cases:
            x = torch.randn(m, 512 if act == "swiglu" else 256, dtype=dtype, device=device, generator=generator)
            act_weight = norm_weight if act == "rms_norm" else None
            residual = torch.randn(m, 96, dtype=dtype, device=device, generator=generator) * 4 if with_residual else None
            residual_scale = torch.rand(96, dtype=dtype, device=device, generator=generator) if with_residual else None
            scale = s_groups if path.endswith("+g") else s
            ref = _reference(x, w, scale, bias, group, act, act_weight, 1e-6, residual, residual_scale, path in ("lines", "small"))
            prepared = prepare(x, group, path.removesuffix("+g"), act, act_weight, 1e-6)
            if path in ("lines", "small"):
                y = linear_prepared(prepared, w, scale, bias, residual, residual_scale, residual)
            else:
                y = gemm(prepared.x, prepared.lo, prepared.scale, w, scale, bias, dtype, 0, variants[path], out=residual, residual=residual,
                         residual_scale=residual_scale)
            error = ((y.float() - ref).norm() / ref.norm()).item()
            if not error < (5e-3 if path in ("lines", "small", "exact", "exact+g") else 3e-2):
                return (f"{path} kernel mismatch ({dtype}, {m} rows, group {group}, {act or 'no input op'}"
                        f"{', residual' if with_residual else ''}): relative error {error:.3g}")
    torch.cuda.synchronize(device)
    return None
