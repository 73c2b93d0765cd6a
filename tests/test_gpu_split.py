"""GPU parity of the split-K launches (wq8_gemm with split != 0; the reference's stream-K, int8_gemm.cu:912-973,
K8:1479-1528) through the C-ABI, against the CPU oracle. Two forms: the tail split (the tiles of an incomplete last wave
split into 2-4 pieces, added by the last piece to arrive) and the deep split (at most half as many tiles as resident
workgroups: every tile split into up to 16 pieces, added by a second launch):
- every split tile's outputs bit for bit against the oracle's split-K order (pieces of whole k-blocks folded from zero,
  added in piece order), the whole tiles' against the unsplit order, for every GEMM variant;
- the INT32 modes (row, exact) bit-exact whatever the split;
- the workspace query (split slots and counters) matching the tiles and pieces the launch runs;
- the counters left at zero, also across back-to-back calls and replays of a captured HIP graph.
Which tiles are split, and into how many pieces, follows from the CU count the call passes: tests pass their own."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import DT, bits
from test_gpu_gemm import BIASED, operands

pytestmark = pytest.mark.gpu

# variant -> (mode, tile rows, tile channels or None for the exact width choice, workgroups per CU)
TILES = {0: ("row", 256, 256, 1), 6: ("row", 64, 128, 2), 1: ("exact", 128, None, 1), 7: ("exact", 32, 128, 2),
         10: ("block", 256, 192, 1), 11: ("block", 64, 128, 2), 12: ("block+g", 256, 192, 1), 13: ("block+g", 64, 128, 2),
         14: ("exact+g", 128, 192, 1), 15: ("block", 64, 128, 2)}


def tile_shape(variant, m, n, cus):
    mode, bm, bn, per_cu = TILES[variant]
    if bn is None:  # the long exact tile: 128 x 192 when its last wave of workgroups is fuller than with 128 x 256
        padded = lambda w: -(-(-(-m // 128) * -(-n // w)) // cus) * 128 * w
        bn = 192 if padded(192) < padded(256) else 256
    return bm, bn, per_cu


def deep_pieces(tiles, kblocks, slots):
    """Pieces of the deep split (every tile split; 0: no deep split)."""
    pieces = min(16, kblocks // 2, slots // tiles)
    return pieces if pieces >= 2 else 0


def plan(tiles, kblocks, slots):
    """(whole tiles, split tiles, pieces): the library's plan of a split launch."""
    deep = deep_pieces(tiles, kblocks, slots)
    if deep:
        return 0, tiles, deep
    sk = tiles if tiles < slots else tiles % slots
    pieces = min(4, kblocks // 4, slots // sk) if sk else 0
    return (tiles, 0, 1) if pieces < 2 else (tiles - sk, sk, pieces)


def raster(v, tiles_m, tiles_n, group=4):
    """Tile (tm, tn) of virtual tile v: GROUP_M token tiles sweep the channel tiles."""
    width = group * tiles_n
    first = v // width * group
    rows = min(group, tiles_m - first)
    return first + v % width % rows, v % width // rows


def split_tiles(variant, m, n, k, cus):
    bm, bn, per_cu = tile_shape(variant, m, n, cus)
    tiles_m, tiles_n = -(-m // bm), -(-n // bn)
    dp, sk, pieces = plan(tiles_m * tiles_n, (k + 127) // 128, cus * per_cu)
    return bm, bn, [raster(v, tiles_m, tiles_n) for v in range(dp, dp + sk)], pieces


def is_deep(variant, m, n, k, cus):
    bm, bn, per_cu = tile_shape(variant, m, n, cus)
    return deep_pieces(-(-m // bm) * -(-n // bn), (k + 127) // 128, cus * per_cu) > 0


def p(t):
    return None if t is None else t.data_ptr()


def run(wq, variant, a, a_lo, sa, b, sb, bias, res, rs, dtype, cus, split, counters):
    lib = wq.library()
    m, k = a.shape
    n = b.shape[0]
    sizes = (ctypes.c_int64 * 2)()
    lib.wq8_gemm_workspace(m, n, k, variant, cus, split, sizes)
    ws = torch.empty(max(1, sizes[0]), dtype=torch.uint8, device="cuda")
    y = res.clone() if res is not None else torch.empty(m, n, dtype=dtype, device="cuda")
    rc = lib.wq8_gemm(p(a), p(a_lo), p(sa), p(b), p(sb), p(bias), p(y if res is not None else None), p(rs), p(y), m, n, k, DT[dtype], variant,
                      cus, split, p(ws), p(counters), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return y, sizes[0], sizes[1]


@pytest.fixture
def counters():
    return torch.zeros(1024, dtype=torch.int32, device="cuda")


def oracle_split(oracle, variant, m, n, k, cus, ops, dtype):
    """The oracle's outputs of a split launch: the split tiles in the split-K order, the rest unsplit."""
    mode = TILES[variant][0]
    base, groups = mode.removesuffix("+g"), mode.endswith("+g")
    om = "block_biased" if base == "block" and not groups and variant in BIASED else "exact_combined" if groups and base == "exact" else base
    a, a_lo, sa, b, sb, bias, res, rs = ops
    args = (a.numpy(), None if a_lo is None else a_lo.numpy(), sa.numpy(), b.numpy(), sb.numpy(), None if bias is None else bits(bias),
            DT[dtype], om, None if res is None else bits(res), None if rs is None else bits(rs))
    whole = oracle.gemm(*args)
    bm, bn, tiles, pieces = split_tiles(variant, m, n, k, cus)
    if pieces > 1:
        split = oracle.gemm(*args, pieces=pieces)
        for tm, tn in tiles:
            rows, cols = slice(tm * bm, (tm + 1) * bm), slice(tn * bn, (tn + 1) * bn)
            whole[rows, cols] = split[rows, cols]
    return whole, len(tiles), pieces


# (m, n, k, CUs counted): deep splits (few tiles: every tile in up to 16 pieces), every tile split by the tail rule
# (fewer tiles than CUs), and whole waves plus a split last wave
SHAPES = [(200, 300, 1024, 256), (520, 700, 2048, 4), (97, 130, 16 * 130, 64), (70, 900, 4096, 256), (40, 2000, 3072, 32)]


@pytest.mark.parametrize("variant", sorted(TILES))
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_split_matches_oracle(wq, oracle, counters, variant, shape):
    m, n, k, cus = shape
    mode = TILES[variant][0]
    base, groups = mode.removesuffix("+g"), mode.endswith("+g")
    dtype = torch.bfloat16 if variant % 2 == 0 else torch.float16
    ops = operands(m, n, k, 100 + variant, groups, base == "exact", base == "block", dtype, residual=variant in (0, 10, 12, 14))
    print(f"split variant={variant} m={m} n={n} k={k} cus={cus} {dtype}", flush=True)
    want, sk, pieces = oracle_split(oracle, variant, m, n, k, cus, ops, dtype)
    cu = [None if t is None else t.cuda() for t in ops]
    y, ws_bytes, counter_bytes = run(wq, variant, *cu, dtype, cus, 1, counters)
    torch.cuda.synchronize()
    assert (sk == 0) == (pieces == 1)
    assert counter_bytes == (0 if is_deep(variant, m, n, k, cus) else 4 * sk)
    np.testing.assert_array_equal(bits(y), want)
    assert int(counters.abs().sum()) == 0  # left at zero


def test_split_plans(wq):
    """The workspace query reports the split tiles (one counter each) and their slots (4 bytes per output element and
    piece, 8 for the exact mode's two INT32 sums), after the block scales; the deep split no counters and whole m x n
    planes per piece; split 0 needs neither."""
    lib = wq.library()
    sizes = (ctypes.c_int64 * 2)()
    for variant, (m, n, k, cus) in [(0, (520, 700, 2048, 4)), (1, (200, 300, 1024, 256)), (10, (97, 130, 2080, 64)), (7, (33, 500, 4096, 8)),
                                    (11, (70, 900, 4096, 256)), (1, (64, 700, 4096, 256))]:
        bm, bn, tiles, pieces = split_tiles(variant, m, n, k, cus)
        assert tiles and pieces > 1
        lib.wq8_gemm_workspace(m, n, k, variant, cus, 0, sizes)
        scales = sizes[0]
        assert sizes[1] == 0
        lib.wq8_gemm_workspace(m, n, k, variant, cus, 1, sizes)
        words = 2 if TILES[variant][0] == "exact" else 1
        if is_deep(variant, m, n, k, cus):
            assert sizes[1] == 0
            assert sizes[0] - scales == -(-pieces * words * m * n * 4 // 256) * 256
        else:
            assert sizes[1] == 4 * len(tiles)
            assert sizes[0] - scales == -(-len(tiles) * pieces * bm * bn * 4 * words // 256) * 256
    # whole waves need no split
    lib.wq8_gemm_workspace(256 * 4, 256 * 8, 4096, 0, 32, 1, sizes)
    assert sizes[1] == 0


@pytest.mark.parametrize("variant,shape", [(10, (300, 500, 3072, 4)), (11, (70, 900, 4096, 256))], ids=["tail", "deep"])
def test_split_repeated_and_graph_replay(wq, oracle, counters, variant, shape):
    """Back-to-back split calls and replays of a captured split GEMM (the tail split, whose counters start and end at
    zero every time, and the deep split with its second launch): every result equals the eager one."""
    m, n, k, cus = shape
    ops = operands(m, n, k, 7, False, False, True, torch.bfloat16)
    cu = [None if t is None else t.cuda() for t in ops]
    want, sk, pieces = oracle_split(oracle, variant, m, n, k, cus, ops, torch.bfloat16)
    assert sk and pieces > 1
    lib = wq.library()
    sizes = (ctypes.c_int64 * 2)()
    lib.wq8_gemm_workspace(m, n, k, variant, cus, 1, sizes)
    ws = torch.empty(sizes[0], dtype=torch.uint8, device="cuda")
    y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    a, a_lo, sa, b, sb, bias, _, _ = cu

    def call():
        assert lib.wq8_gemm(p(a), None, p(sa), p(b), p(sb), p(bias), None, None, p(y), m, n, k, DT[torch.bfloat16], variant, cus, 1, p(ws),
                            p(counters), torch.cuda.current_stream().cuda_stream) == 0

    for _ in range(3):
        y.zero_()
        call()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(y), want)
        assert int(counters.abs().sum()) == 0
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            call()
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(4):
        y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(y), want)
        assert int(counters.abs().sum()) == 0
