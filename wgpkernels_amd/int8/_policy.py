"""Which path serves a linear: the timed choice between the full-precision paths and 'block', and the fixed rule used
where nothing may be timed (graph capture, compilation).

The rule is the reference's (wgpkernels/int8/__init__.py:453-509): take the fastest full-precision path ('lines',
'small', 'exact') while it costs at most EXACT_TOLERANCE more than 'block', else 'block'; precise=True never takes
'block'; above DECIDE_MAX_ROWS tokens 'block' is taken untimed. Per-(channel, k-block) weight scales leave 'exact' as
the only full-precision path.

The fixed rule's thresholds are MI355X measurements, not the reference's RTX 5090 ones: with cold weights 'lines' is
the fastest path up to 4 tokens and 'small' up to 32 at the Wan widths (K, N in {5120, 13824}), where 'exact' (two
INT8 passes plus a quantize launch) was 20-45% slower.
"""
from dataclasses import dataclass

EXACT_TOLERANCE = 0.10
# few-token kernel limits (their C-ABI bounds) and the alignment their loads need
LINE_MAX_ROWS, SMALL_MAX_ROWS = 4, 32
LINE_K_MULTIPLE, SMALL_K_MULTIPLE = 4, 64
# the untimed rule: lines up to LINE_ROWS tokens, small up to SMALL_ROWS, exact up to EXACT_ROWS, then block
LINE_ROWS, SMALL_ROWS, EXACT_ROWS = 4, 32, 64
DECIDE_MAX_ROWS = 4096


@dataclass(frozen=True)
class LinearShape:
    """What a path decision depends on besides the GPU."""
    m: int
    n: int
    k: int
    group: int = 0
    act: str = None
    precise: bool = False
    weight_groups: bool = False

    def few_token_ok(self, max_rows, k_multiple):
        return not self.weight_groups and self.m <= max_rows and self.k % k_multiple == 0

    def candidates(self):
        """Paths the timed choice compares, full-precision ones first."""
        paths = []
        if self.few_token_ok(LINE_MAX_ROWS, LINE_K_MULTIPLE):
            paths.append("lines")
        if self.few_token_ok(SMALL_MAX_ROWS, SMALL_K_MULTIPLE):
            paths.append("small")
        paths.append("exact")
        if not self.precise:
            paths.append("block")
        return paths

    def untimed(self):
        """The fixed rule."""
        if self.few_token_ok(LINE_ROWS, LINE_K_MULTIPLE):
            return "lines"
        if self.few_token_ok(SMALL_ROWS, SMALL_K_MULTIPLE):
            return "small"
        return "exact" if self.precise or self.m <= EXACT_ROWS else "block"

    def key(self, rows_bucket, device_name):
        """Cache key, in the reference's format (wgpkernels/int8/__init__.py:485-486)."""
        parts = [f"path{'+precise' if self.precise else ''}", f"{rows_bucket}x{self.n}x{self.k}", f"g{self.group}"]
        if self.act:
            parts.append(self.act)
        if self.weight_groups:
            parts.append("wgroups")
        parts.append(device_name)
        return "|".join(parts)


def decide(timings, precise):
    """The path of measured `timings` (path -> ms): the fastest full-precision path unless it costs more than
    (1 + EXACT_TOLERANCE) x 'block'."""
    full = {p: t for p, t in timings.items() if p != "block"}
    best = min(full, key=full.get)
    if not precise and "block" in timings and full[best] > (1 + EXACT_TOLERANCE) * timings["block"]:
        return "block"
    return best
