"""The ctypes side of libwgp_int8.so: one table of C signatures (include/wq8.h), the loaded library, and what each GPU
needs from the host (compute-unit count, raw current stream, the zeroed split counters of the C-ABI).

Every entry point takes raw device pointers, plain sizes and the raw hipStream_t last, and returns 0 or an error code
(negative: arguments rejected before any launch; positive: a HIP error). Library.call() turns a nonzero code into
RuntimeError naming the entry point, so nothing fails silently and nothing falls back to another implementation.
"""
import ctypes
from pathlib import Path

import torch

ABI_VERSION = 11
HIP_ARCHS = ("gfx950",)
FEATURE_WEIGHT_GROUPS = 1

# C types by letter: p pointer, i int, l int64_t, q long long, f float; "-" = void result.
_CTYPES = {"p": ctypes.c_void_p, "i": ctypes.c_int, "l": ctypes.c_int64, "q": ctypes.c_longlong, "f": ctypes.c_float}

# name -> (result, arguments), in the order include/wq8.h declares them. The reference's ctypes layer binds the same
# argument lists (wgpkernels/int8/__init__.py:73-89); the *_at and scratch entry points are this library's extras.
SIGNATURES = {
    "wq8_abi": ("i", ""),
    "wq8_features": ("i", ""),
    "wq8_quantize": ("i", "ppppiilii" "ipfp"),
    "wq8_quantize_blocks": ("i", "pppiilii" "ipfpp"),
    "wq8_quantize_at": ("i", "ppppiilii" "ipf" "pqq" "p"),
    "wq8_quantize_blocks_at": ("i", "pppiilii" "ipfp" "pqq" "p"),
    "wq8_transform_rows": ("i", "ppiilii" "ipfp"),
    "wq8_rotate_groups": ("i", "ppiilii" "p"),
    "wq8_gemm": ("i", "ppppppppp" "iiiiiii" "ppp"),
    "wq8_gemm_workspace": ("-", "iiiiii" "p"),
    "wq8_gemm_select": ("i", "iiiii"),
    "wq8_gemm_at": ("i", "ppppppppp" "iiiiiii" "pp" "pqqqqqq" "p"),
    "wq8_gemm_segments": ("i", "ppppppp" "iiiiiiii" "ppp"),
    "wq8_gemm_noalloc": ("i", "ppppppppp" "iiiiiii" "p"),
    "wq8_small": ("i", "plpppppp" "iiiii" "ppp"),
    "wq8_small_workspace": ("-", "iiii" "p"),
    "wq8_gemv_lines": ("i", "plpppppp" "iiii" "p"),
    "wq8_l2_flush": ("i", "il" "p"),
    "wq8_l2_flush_release": ("-", ""),
}
# entry points an older or foreign build may lack: bound when present (segments_supported() reports the first)
OPTIONAL = {"wq8_gemm_segments", "wq8_gemm_noalloc", "wq8_quantize_at", "wq8_quantize_blocks_at", "wq8_gemm_at"}
# the test library's entry points (include/wq8_test.h; libwgp_int8_test.so, not part of the product library)
TEST_SIGNATURES = {
    "wq8_debug_block_sums": ("i", "ppp" "iii" "i" "p"),
    "wq8_debug_mfma_probe": ("i", "pp" "iii" "p"),
}


def _bind(fn, signature):
    result, args = signature
    fn.restype = None if result == "-" else _CTYPES[result]
    fn.argtypes = [_CTYPES[c] for c in args]
    return fn


class Library:
    """A loaded libwgp_int8.so with every declared entry point bound (or, with the test table, libwgp_int8_test.so).
    Attributes are the ctypes functions."""

    def __init__(self, path, signatures=None, optional=OPTIONAL):
        self.path = Path(path).resolve()
        if not self.path.exists():
            raise RuntimeError(f"INT8 library {self.path} not found: build it with `python -m wgpkernels_amd.build`")
        self.cdll = ctypes.CDLL(str(self.path))
        for name, signature in (signatures or SIGNATURES).items():
            fn = getattr(self.cdll, name, None)
            if fn is None:
                if name in optional:
                    continue
                raise RuntimeError(f"INT8 library {self.path} lacks {name}; rebuild it")
            setattr(self, name, _bind(fn, signature))
        if signatures is None:
            abi = self.wq8_abi()
            if abi != ABI_VERSION:
                raise RuntimeError(f"INT8 library ABI {abi}, expected {ABI_VERSION}; rebuild it")
            self.features = self.wq8_features()

    def has(self, name):
        return hasattr(self, name)

    def call(self, name, *args):
        """Calls entry point `name`; a nonzero return raises RuntimeError (there is no fallback path)."""
        code = getattr(self, name)(*args)
        if code:
            raise_code(code, name)


def load_test_library(path=None):
    """libwgp_int8_test.so (built with `python -m wgpkernels_amd.build --library int8_test`): the test-only entry points
    of include/wq8_test.h, for the parity tests and bench.py."""
    return Library(path or Path(__file__).with_name("libwgp_int8_test.so"), TEST_SIGNATURES, optional=())


def raise_code(code, name="INT8 kernel"):
    if code < 0:
        raise RuntimeError(f"{name} rejected its arguments (code {code})")
    raise RuntimeError(f"{name} launch failed (HIP error {code})")


def ptr(tensor):
    return None if tensor is None else tensor.data_ptr()


# ---- per-GPU host state -----------------------------------------------------------------------------------------
COUNTER_INTS = 1024  # the C-ABI's split counters, as its workspace queries size them (zero on entry, left zero)


class Gpu:
    """What the host keeps per GPU: its name for tuning keys, compute units, and the split counters its streams share
    (allocated lazily, never under graph capture: load_library() allocates them up front)."""
    __slots__ = ("index", "name", "cus", "arch", "_counters")

    def __init__(self, index):
        props = torch.cuda.get_device_properties(index)
        self.index = index
        self.arch = props.gcnArchName.split(":")[0]
        self.cus = props.multi_processor_count
        self.name = f"{self.arch}x{self.cus}"
        self._counters = None

    @property
    def counters(self):
        if self._counters is None:
            self._counters = torch.zeros(COUNTER_INTS, dtype=torch.int32, device=torch.device("cuda", self.index))
        return self._counters

    def stream(self):
        """The raw hipStream_t of this GPU's current torch stream (what every entry point takes last)."""
        return torch._C._cuda_getCurrentRawStream(self.index)


_gpus = {}


def gpu(device):
    """The Gpu of a torch device (or of a tensor's device); None index means the current device."""
    if isinstance(device, torch.Tensor):
        index = device.get_device()  # an int, without building a torch.device (host time per call)
        if index < 0:
            index = torch.cuda.current_device()
    else:
        index = device.index if device.index is not None else torch.cuda.current_device()
    state = _gpus.get(index)
    if state is None:
        state = _gpus[index] = Gpu(index)
    return state


def supported_gpus():
    """Indices of the visible GPUs the library is built for."""
    return [i for i in range(torch.cuda.device_count()) if gpu(torch.device("cuda", i)).arch in HIP_ARCHS]


# streams given their own counters (prepare_stream): raw handle -> int32 tensor
stream_counters = {}


def counters_for(state, raw_stream, nbytes):
    """Zeroed split counters for a call on `raw_stream` needing `nbytes` of them."""
    if nbytes > COUNTER_INTS * 4:
        raise RuntimeError("INT8 GEMM split-K counters exceeded")
    own = stream_counters.get(raw_stream)
    return own if own is not None else state.counters
