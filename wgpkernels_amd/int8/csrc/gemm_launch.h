// The INT8 GEMM's launch side, shared by the translation units of the library: variant table, tile choice, split-K plan,
// launchers and the per-dtype dispatch (instantiated once per output dtype, in gemm_bf16.hip and gemm_f16.hip, so that
// the two compile in parallel), and the workspace layout.
#pragma once
#include "gemm_ring.h"
#include "gemm_pingpong.h"

namespace wq8 {

// ---- variants: the reference's variant ids keep their mode (K8:1417-1432); the tiles are this library's -------
// long: row 256 tokens x 256 channels, block (biased fold) and block with weight groups 256 x 192, hi/lo 128 x 256 or
// 128 x 192, hi/lo with weight groups 128 x 192, all on two groups of 4 waves in ping-pong (gemm_pingpong.h).
// short: 64 x 128 (hi/lo 32 x 128) on 4 waves, for inputs of few tokens. Variants 10 and 15 (15: the short block
// tile, an id the reference does not use) fold block sums with the single-FMA biased form; 11 and the weight-group
// variants fold in the reference's order.
enum { TILE_LONG = 0, TILE_SHORT = 1 };
struct Variant { int mode; bool wgroup; int tile; bool biased; };
inline bool variant_info(int v, Variant& out) {
    switch (v) {
        case 0: case 2: out = {MODE_ROW, false, TILE_LONG, false}; return true;
        case 6: out = {MODE_ROW, false, TILE_SHORT, false}; return true;
        case 1: out = {MODE_EXACT, false, TILE_LONG, false}; return true;
        case 7: out = {MODE_EXACT, false, TILE_SHORT, false}; return true;
        case 10: out = {MODE_BLOCK, false, TILE_LONG, true}; return true;
        case 11: out = {MODE_BLOCK, false, TILE_SHORT, false}; return true;
        case 12: out = {MODE_BLOCK, true, TILE_LONG, false}; return true;
        case 13: out = {MODE_BLOCK, true, TILE_SHORT, false}; return true;
        case 14: out = {MODE_EXACT, true, TILE_LONG, false}; return true;
        case 15: out = {MODE_BLOCK, false, TILE_SHORT, true}; return true;
    }
    return false;
}

// ---- split-K tail (the reference's stream-K for an incomplete last wave, K8:1479-1504, in this library's form) -------
// With split != 0, when the tiles do not fill whole waves of workgroups (or are fewer than one wave), the tiles of the
// last, incomplete wave are split along K into `pieces` ranges of whole 128-element k-blocks: at most 4, at least 4
// k-blocks each, and no more pieces than fill the CUs. The first dp tiles run whole, the split tiles' pieces after
// them; the last piece of a tile to finish adds the partial sums in piece order and runs
// the epilogue. INT32 sums (row, exact) add exactly; the FP32 folds (block, +g) add their pieces' partial folds.
struct SplitPlan { int dp, sk, pieces; };
inline SplitPlan plan_split(int tiles, int kblocks, int slots, int split) {
    const SplitPlan whole{tiles, 0, 1};
    if (!split || tiles <= 0 || slots <= 0) return whole;
    const int sk = tiles < slots ? tiles : tiles % slots;
    if (!sk) return whole;
    int pieces = 4;
    pieces = pieces < kblocks / 4 ? pieces : kblocks / 4;
    pieces = pieces < slots / sk ? pieces : slots / sk;
    if (pieces < 2) return whole;
    return {tiles - sk, sk, pieces};
}

// Deep split (split != 0 and at most half as many tiles as resident workgroups): every tile splits into
// min(16, KB / 2, slots / tiles) pieces of whole k-blocks (at least 2, else no deep split), so that the launch fills the
// chip; the pieces' partial sums go to row-major planes that a second kernel (gemm_split_finish) adds in piece order.
// Shapes of few tiles (up to a few hundred tokens at the Wan widths) otherwise leave most CUs idle, and the last-arriver
// reduction of the split-K tail is serial in the number of pieces; with more tiles than that the tail split remains.
inline int deep_pieces(int tiles, int kblocks, int slots, int split) {
    if (!split || tiles <= 0) return 0;
    int pieces = 16;
    pieces = pieces < kblocks / 2 ? pieces : kblocks / 2;
    pieces = pieces < slots / tiles ? pieces : slots / tiles;
    return pieces >= 2 ? pieces : 0;
}

// grid of a launch over g.tiles_m x g.tiles_n tiles with `slots` workgroups resident at once (CUs x workgroups per CU)
inline int plan_grid(GemmArgs& g, int split, int slots) {
    const int tiles = g.tiles_m * g.tiles_n;
    if (const int deep = g.seg_rows ? 0 : deep_pieces(tiles, g.kblocks, slots, split)) {
        g.dp_tiles = 0;
        g.pieces = deep;
        g.defer = 1;
        return tiles * deep;
    }
    const SplitPlan p = plan_split(tiles, g.kblocks, slots, split);
    g.dp_tiles = p.dp;
    g.pieces = p.pieces;
    g.defer = 0;
    return p.dp + p.sk * p.pieces;
}

// the deep split's second launch
template <int DT, int MODE, bool WG>
static int launch_finish(GemmArgs& g, hipStream_t stream) {
    constexpr bool FP = MODE == MODE_BLOCK || (MODE == MODE_EXACT && WG);
    constexpr int WORDS = MODE == MODE_EXACT && !WG ? 2 : 1;
    const int64_t elements = int64_t(g.m) * g.n;
    gemm_split_finish<DT, MODE, WG, FP, WORDS><<<int((elements + 1023) / 1024), 256, 0, stream>>>(g);  // 4 elements a thread
    return int(hipGetLastError());
}

inline int cus_of(const GemmArgs& g) { return g.sms > 0 ? g.sms : 256; }

// short tiles: two workgroups per CU (3 stages of 24 KiB); every other tile: one
template <int BM, int BN, int WAVES_N, int WAVES_M, int MODE, bool WG, bool BIASED, int DT, bool SUMS, bool SEG, int BK = 128, int STAGES = 3>
static int launch_ring(GemmArgs& g, hipStream_t stream, int split = 0) {
    g.tiles_m = (g.m + BM - 1) / BM;
    g.tiles_n = (g.n + BN - 1) / BN;
    g.n_first = 0;
    const int grid = plan_grid(g, SUMS ? 0 : split, cus_of(g) * (WAVES_N * WAVES_M == 4 ? 2 : 1));
    if constexpr (!SUMS && !SEG) {  // segments run whole tiles
        if (g.pieces > 1) {
            gemm_ring<BM, BN, WAVES_N, WAVES_M, BK, STAGES, MODE, WG, BIASED, DT, false, SEG, true><<<grid, 64 * WAVES_N * WAVES_M, 0, stream>>>(g);
            if (const int rc = int(hipGetLastError())) return rc;
            return g.defer ? launch_finish<DT, MODE, WG>(g, stream) : 0;
        }
    }
    gemm_ring<BM, BN, WAVES_N, WAVES_M, BK, STAGES, MODE, WG, BIASED, DT, SUMS, SEG><<<grid, 64 * WAVES_N * WAVES_M, 0, stream>>>(g);
    return int(hipGetLastError());
}

// MFMA shape of the ping-pong mainloops: v_mfma_i32_16x16x64_i8 for every mode. Against the 32x32x32 form, measured
// interleaved on one box at the Wan widths: row and exact 8-12% faster (row 8192 x 13824 x 5120: 460 against 524 us);
// the block folds 8-10% faster (headline shape 2098 against 2272 us), weight groups 3-5%, once each tile folds two
// tiles behind its chain (gemm_pingpong.h, LAG); folding one tile behind, the block modes ran 3-12% slower than with
// 32x32x32. The outputs are the same bits either way: each element's fold order does not depend on the MFMA shape.
// WQ8_PINGPONG_MF_BLOCK / _INT = 32 build the other form for comparison.
#ifndef WQ8_PINGPONG_MF_BLOCK
#define WQ8_PINGPONG_MF_BLOCK 16
#endif
#ifndef WQ8_PINGPONG_MF_INT
#define WQ8_PINGPONG_MF_INT 16
#endif
template <int MODE>
constexpr int pp_mf = MODE == MODE_BLOCK ? WQ8_PINGPONG_MF_BLOCK : WQ8_PINGPONG_MF_INT;

// channels [n_first, n_first + n_count) of the output (all of them by default)
template <int BM, int BN, int WAVES_N, int WAVES_M, int MODE, bool WG, bool BIASED, int DT, bool SEG>
static int launch_pingpong(GemmArgs& g, hipStream_t stream, int split = 0, int n_first = 0, int n_count = -1) {
    g.tiles_m = (g.m + BM - 1) / BM;
    g.tiles_n = ((n_count < 0 ? g.n : n_count) + BN - 1) / BN;
    g.n_first = n_first;
    const int grid = plan_grid(g, split, cus_of(g));
    // K % 128 == 0: the copies need no K-tail select (one VALU compare-select fewer per copy)
    if (!SEG && g.pieces > 1) {  // segments run whole tiles
        if constexpr (!SEG) {
            if (g.k % 128 == 0) gemm_pingpong<BM, BN, WAVES_N, WAVES_M, MODE, WG, BIASED, DT, false, false, true, false, pp_mf<MODE>><<<grid, 512, 0, stream>>>(g);
            else gemm_pingpong<BM, BN, WAVES_N, WAVES_M, MODE, WG, BIASED, DT, false, true, true, false, pp_mf<MODE>><<<grid, 512, 0, stream>>>(g);
            if (g.defer) {
                if (const int rc = int(hipGetLastError())) return rc;
                return launch_finish<DT, MODE, WG>(g, stream);
            }
        }
    } else if (g.k % 128 == 0) {
        gemm_pingpong<BM, BN, WAVES_N, WAVES_M, MODE, WG, BIASED, DT, SEG, false, false, false, pp_mf<MODE>><<<grid, 512, 0, stream>>>(g);
    } else {
        gemm_pingpong<BM, BN, WAVES_N, WAVES_M, MODE, WG, BIASED, DT, SEG, true, false, false, pp_mf<MODE>><<<grid, 512, 0, stream>>>(g);
    }
    return int(hipGetLastError());
}

// The kernels address operands with 32-bit buffer offsets: each operand (plus a tile of rows) below 2^31 bytes.
inline bool offsets_fit(const GemmArgs& g) {
    const int64_t lim = int64_t(1) << 31;
    const int64_t rows_b = g.seg_rows ? int64_t(g.seg_rows) : int64_t(g.n);
    return (int64_t(g.m) + 256) * g.k < lim && (rows_b + 256) * g.k < lim && (int64_t(g.m) + 256) * g.kblocks * 4 < lim &&
           (int64_t(g.n) + 256) * g.kblocks * 4 < lim;
}

// Tile area times the waves of workgroups a bm x bn tiling runs (one workgroup per CU at a time): the padded work of the
// launch, including the idle CUs of its last wave.
inline int64_t padded_work(const GemmArgs& g, int bm, int bn) {
    const int64_t tiles = int64_t((g.m + bm - 1) / bm) * ((g.n + bn - 1) / bn), cus = g.sms > 0 ? g.sms : 256;
    return (tiles + cus - 1) / cus * bm * bn;
}

// Channel split of the long biased block tiles: the number of channels (a multiple of 192) run as 256 x 192 tiles, the
// rest as 256 x 128 tiles (0: all of them), or -1 for 256 x 192 tiles only. Chosen when the estimated time, in waves of
// 256 x 192 workgroups with a 256 x 128 one counted as 0.8 of one (measured: 256 x 128 tiles alone ran 15% slower than
// 256 x 192 at K = 13824, N = 5120, which is 0.805 per tile), beats 256 x 192 tiles alone by more than 2%.
inline int block_channel_split(const GemmArgs& g) {
    const int64_t cus = g.sms > 0 ? g.sms : 256, tm = (g.m + 255) / 256;
    auto waves = [&](int64_t tiles) { return (tiles + cus - 1) / cus; };
    const double one = double(waves(tm * ((g.n + 191) / 192)));
    double best = one * 0.98;
    int split = -1;
    auto pick = [&](int c) {
        const int rest = g.n - 192 * c;
        if (rest <= 0 || rest % 128) return;
        const double t = double(waves(tm * c)) + 0.8 * double(waves(tm * (rest / 128)));
        if (t < best) {
            best = t;
            split = 192 * c;
        }
    };
    for (int c = g.n / 192; c > 0 && c >= g.n / 192 - 8; --c) pick(c);
    pick(0);  // 256 x 128 tiles only: fewer than a wave of 256 x 192 workgroups leaves CUs idle
    return split;
}

// The tile of a launch (tokens x channels) and whether its kernel runs two workgroups per CU. The launchers below take
// the same decisions; wq8_gemm_workspace sizes the split slots from them.
struct TileShape { int bm, bn, per_cu; };
inline TileShape tile_shape(const GemmArgs& g, const Variant& v) {
    const bool hilo = v.mode == MODE_EXACT;
    if (v.tile == TILE_SHORT) return {hilo ? 32 : 64, 128, 2};
    if (hilo && !v.wgroup) return {128, padded_work(g, 128, 192) < padded_work(g, 128, 256) ? 192 : 256, 1};
    if (hilo) return {128, 192, 1};
    if (v.mode == MODE_ROW) return {256, 256, 1};
    return {256, 192, 1};  // block: biased (10) or with weight groups (12)
}

template <int MODE, bool WG, bool BIASED, int DT, bool SEG>
static int launch_tiles(GemmArgs& g, int tile, int split, hipStream_t stream) {
    constexpr bool HILO = MODE == MODE_EXACT;
    if (tile == TILE_SHORT) {
        if constexpr (HILO) return launch_ring<32, 128, 4, 1, MODE, WG, BIASED, DT, false, SEG>(g, stream, split);
        else return launch_ring<64, 128, 4, 1, MODE, WG, BIASED, DT, false, SEG>(g, stream, split);
    }
    // hi/lo: 128 x 256 or 128 x 192 ping-pong (waves of 32 tokens x 128 or 96 channels, two INT32 accumulators per
    // tile), 128 x 192 when its last wave of workgroups is fuller; a stage holds the 128 tokens' hi and lo rows. 10-12%
    // faster than the 2-stage ring at config 4 (M = 4096, N = 3 x 5120 through the segments entry point: 533-542 against
    // 603-652 us, the same bits); the two tiles measure within 2% of each other there.
    if constexpr (HILO && !WG) {
        if (padded_work(g, 128, 192) < padded_work(g, 128, 256)) return launch_pingpong<128, 192, 2, 4, MODE, false, false, DT, SEG>(g, stream, split);
        return launch_pingpong<128, 256, 2, 4, MODE, false, false, DT, SEG>(g, stream, split);
    }
    // hi/lo with weight groups: 128 x 192 ping-pong (waves of 32 tokens x 96 channels). 23% faster than the 128 x 128
    // ring at M = 8192, N = 12288, K = 3072 (652 against 803 us), the same bits.
    else if constexpr (HILO) {
        static_assert(!SEG, "weight groups take no segments");
        return launch_pingpong<128, 192, 2, 4, MODE, true, false, DT, false>(g, stream, split);
    }
    // row: 256 x 256 ping-pong (waves of 64 tokens x 128 channels); block with the biased fold: 256 x 192 ping-pong
    // (waves of 64 tokens x 96 channels, whose FP32 accumulators, fragments and fold chain fit 256 registers)
    else if constexpr (MODE == MODE_ROW) return launch_pingpong<256, 256, 2, 4, MODE, false, false, DT, SEG>(g, stream, split);
    else if constexpr (MODE == MODE_BLOCK && BIASED && !WG) {
        // Whole tiles only (split 0): when the last wave of 256 x 192 workgroups would be at most half full, the channels
        // split in two launches: 256 x 192 tiles over a range that fills whole waves and 256 x 128 tiles over the rest
        // (K = 13824, N = 5120: 12 + 2 waves instead of 13.5 in 14); when 256 x 192 tiles would not fill one wave, one
        // launch of 256 x 128 tiles over every channel. The tiles are the same tiles, so are the bits.
        const int channels = split ? -1 : block_channel_split(g);
        if (channels >= 0) {
            if (channels > 0) {
                if (const int rc = launch_pingpong<256, 192, 2, 4, MODE, false, true, DT, SEG>(g, stream, 0, 0, channels)) return rc;
            }
            return launch_pingpong<256, 128, 2, 4, MODE, false, true, DT, SEG>(g, stream, 0, channels, g.n - channels);
        }
        return launch_pingpong<256, 192, 2, 4, MODE, false, true, DT, SEG>(g, stream, split);
    }
    // block with weight groups: 256 x 192 ping-pong, folding in the reference's order
    else if constexpr (MODE == MODE_BLOCK && WG) {
        static_assert(!SEG, "weight groups take no segments");
        return launch_pingpong<256, 192, 2, 4, MODE, true, false, DT, false>(g, stream, split);
    }
    // block in the reference's fold order has only the short tile (variant 11)
    else return -3;
}

template <int DT, bool SEG>
int dispatch_gemm(GemmArgs& g, const Variant& v, int split, hipStream_t stream) {
    if (!offsets_fit(g)) return -2;
    if (v.mode == MODE_ROW) return launch_tiles<MODE_ROW, false, false, DT, SEG>(g, v.tile, split, stream);
    if (v.mode == MODE_EXACT && !v.wgroup) return launch_tiles<MODE_EXACT, false, false, DT, SEG>(g, v.tile, split, stream);
    if (v.mode == MODE_BLOCK && !v.wgroup) {
        if (v.biased) return launch_tiles<MODE_BLOCK, false, true, DT, SEG>(g, v.tile, split, stream);
        return launch_tiles<MODE_BLOCK, false, false, DT, SEG>(g, v.tile, split, stream);
    }
    if constexpr (!SEG) {
        if (v.mode == MODE_BLOCK) return launch_tiles<MODE_BLOCK, true, false, DT, false>(g, v.tile, split, stream);
        return launch_tiles<MODE_EXACT, true, false, DT, false>(g, v.tile, split, stream);
    }
    return -4;
}

// workspace bytes of the transposed block scales: [sa_t (m x kblocks)][sb_t (n x kblocks)], each 256-byte aligned
inline int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }
inline void scale_workspace(int m, int n, int k, const Variant& v, int64_t& sa_bytes, int64_t& sb_bytes) {
    const int64_t kb = (k + 127) / 128;
    sa_bytes = v.mode == MODE_BLOCK ? align256(int64_t(m) * kb * 4) : 0;
    sb_bytes = v.wgroup ? align256(int64_t(n) * kb * 4) : 0;
}

// The split-K part of the workspace, after the scales: one slot of partial sums per piece of a split tile (4 bytes per
// output element, 8 for the INT32 hi and lo sums of the exact mode), and one counter per split tile.
inline void split_workspace(const GemmArgs& g, const Variant& v, int split, int64_t& slot_bytes, int64_t& counter_bytes) {
    slot_bytes = counter_bytes = 0;
    if (!split) return;
    const TileShape t = tile_shape(g, v);
    const int tiles = ((g.m + t.bm - 1) / t.bm) * ((g.n + t.bn - 1) / t.bn);
    const int words = v.mode == MODE_EXACT && !v.wgroup ? 2 : 1;
    if (const int deep = g.seg_rows ? 0 : deep_pieces(tiles, g.kblocks, cus_of(g) * t.per_cu, split)) {
        // deep split: `deep` planes (two per piece with the exact mode's hi and lo) of m x n words, no counters
        slot_bytes = align256(int64_t(deep) * words * g.m * g.n * 4);
        return;
    }
    const SplitPlan p = plan_split(tiles, g.kblocks, cus_of(g) * t.per_cu, split);
    if (!p.sk) return;
    slot_bytes = align256(int64_t(p.sk) * p.pieces * t.bm * t.bn * 4 * words);
    counter_bytes = int64_t(p.sk) * 4;
}

// The reference's tile estimate (K8:1554-1568) restated for this library's tiles: padded work of the waves of
// workgroups that run at once, divided by a relative mainloop efficiency.
inline double estimate_tiles(int m, int n, int k, int sms, int bm, int bn, int per_cu, double efficiency) {
    const long long tm = (m + bm - 1) / bm, tn = (n + bn - 1) / bn, tiles = tm * tn;
    const long long slots = (long long)per_cu * sms, waves = (tiles + slots - 1) / slots;
    return double(waves) * double(bm) * double(bn) * double(k) / efficiency;
}


// the per-dtype dispatch is instantiated in gemm_bf16.hip and gemm_f16.hip
extern template int dispatch_gemm<DT_BF16, false>(GemmArgs&, const Variant&, int, hipStream_t);
extern template int dispatch_gemm<DT_BF16, true>(GemmArgs&, const Variant&, int, hipStream_t);
extern template int dispatch_gemm<DT_F16, false>(GemmArgs&, const Variant&, int, hipStream_t);
extern template int dispatch_gemm<DT_F16, true>(GemmArgs&, const Variant&, int, hipStream_t);

}  // namespace wq8
