"""Per-GPU autotuning of the INT8 linear: the persistent store of decisions and the cold-cache timer.

Behaviour kept from the reference (wgpkernels/int8/__init__.py:195-293, :474-509): decisions are timed once per GPU,
shape and token-count bucket, persisted as JSON under ~/.triton/autotune, silent on a hit, and announced with one
"Autotuning ..." and one "Selected ..." line when measured. Key strings keep the reference's formats, so a cache file
reads the same way.

How this build times (its own design):
- Every candidate runs once untimed (kernel loading, allocator growth).
- Then ROUNDS rounds. Round r visits the candidates in a rotated order starting at candidate r, so none is always
  first after the flush or always last before a sync.
- Before each timed launch the library reads a buffer larger than every L2 plus the 256 MiB Infinity Cache (MALL) with
  allocating loads (wq8_l2_flush). The timed launch then streams its weights from HBM, as a layer of a model does.
- A round is synchronized once. A candidate's time is the median of its rounds.
"""
import json
import os
import statistics
import tempfile
from pathlib import Path

import torch

from . import _native

TUNING_VERSION = 2
DEFAULT_PATH = Path.home() / ".triton" / "autotune" / "wgpkernels_amd_int8.json"
ROUNDS = 5
# 4 MiB of L2 per XCD x 8 XCDs plus the 256 MiB MALL, read twice over
MALL_BYTES = 256 * 1024 * 1024


class Store:
    """Decisions by key, loaded on first use and rewritten whole (through a temporary file and a rename) after each new
    decision. A missing, unreadable or other-version file is an empty store."""

    def __init__(self, path):
        self.path = Path(path)
        self._entries = None

    def entries(self):
        if self._entries is None:
            self._entries = {}
            try:
                payload = json.loads(self.path.read_text(encoding="utf-8"))
                if isinstance(payload, dict) and payload.get("version") == TUNING_VERSION and isinstance(payload.get("configs"), dict):
                    self._entries = payload["configs"]
            except (OSError, ValueError):
                pass
        return self._entries

    def get(self, key):
        return self.entries().get(key)

    def put(self, key, value):
        self.entries()[key] = value
        try:
            self.path.parent.mkdir(parents=True, exist_ok=True)
            fd, tmp = tempfile.mkstemp(prefix=".wgp-int8-", dir=self.path.parent)
            with os.fdopen(fd, "w", encoding="utf-8") as f:
                json.dump({"version": TUNING_VERSION, "configs": self._entries}, f, indent=1, sort_keys=True)
            os.replace(tmp, self.path)
        except OSError as error:
            print(f"[INT8] Could not save the INT8 tuning cache {self.path}: {error}")


store = Store(os.environ.get("WGPKERNELS_AMD_CACHE", DEFAULT_PATH))


def gemm_rows_bucket(m):
    """Token-count bucket of the tile choice: multiples of 64 through 4096, then powers of two capped at 16384
    (reference buckets, wgpkernels/int8/__init__.py:195-197)."""
    if m <= 4096:
        return (m + 63) // 64 * 64
    bucket = 8192
    while bucket < m and bucket < 16384:
        bucket *= 2
    return bucket


def path_rows_bucket(m):
    """Token-count bucket of the path choice: exact through 16, multiples of 8 through 128, then as the tile choice
    (reference buckets, wgpkernels/int8/__init__.py:467-468)."""
    if m <= 16:
        return m
    if m <= 128:
        return (m + 7) // 8 * 8
    return gemm_rows_bucket(m)


def flush_bytes(index):
    l2 = torch.cuda.get_device_properties(index).L2_cache_size
    return 2 * (8 * l2 + MALL_BYTES)


def is_capturing():
    """Under graph capture or compilation nothing may be timed (no synchronization, no extra launches)."""
    return torch.cuda.is_current_stream_capturing() or torch.compiler.is_compiling()


def time_cold(lib, launches, device):
    """Median milliseconds per candidate of `launches` (name -> zero-argument callable), each timed launch after a
    cold-cache flush. Falls back to the median of warm back-to-back launches if the flush buffer cannot be allocated."""
    names = list(launches)
    for name in names:
        launches[name]()
    state = _native.gpu(device)
    stream = state.stream()
    nbytes = flush_bytes(state.index)
    cold = lib.wq8_l2_flush(state.index, nbytes, stream) == 0
    samples = {name: [] for name in names}
    try:
        for r in range(ROUNDS):
            order = names[r % len(names):] + names[:r % len(names)]
            marks = []
            for name in order:
                if cold:
                    lib.call("wq8_l2_flush", state.index, nbytes, stream)
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
                launches[name]()
                if not cold:
                    launches[name]()
                end.record()
                marks.append((name, start, end))
            marks[-1][2].synchronize()
            for name, start, end in marks:
                samples[name].append(start.elapsed_time(end) / (1 if cold else 2))
    finally:
        lib.wq8_l2_flush_release()
    return {name: statistics.median(values) for name, values in samples.items()}
