// INT8 GEMM mainloop with two wave groups in ping-pong, for long inputs: row mode, block mode with the biased fold, the
// exact mode, and the block and exact modes with per-(channel, k-block) weight scales.
//
// A workgroup of 8 waves computes a BM x BN tile; waves w and w + 4 run on the same SIMD. Group 0 (waves 0-3) and
// group 1 (waves 4-7) execute the same per-k-tile program, MEM (read every MFMA fragment of the k-tile from LDS into
// registers, issue DMA copies of later k-tiles) then COMP (the k-tile's MFMAs and, in the folding modes, its fold), but
// group 1 runs half an iteration behind: while one wave of a SIMD issues its dense MFMA block, the other one talks to LDS and
// memory, and the MFMA pipe of every SIMD always has a wave to feed it. s_barrier keeps the two groups in step; every
// barrier is met by group 0 and group 1 at different points of the program:
//
//   group 0:  bar0  [MEM k + copies of k+1]  bar(2k+1) [COMP k]              bar(2k+2) ...   bar(2KT+1)
//   group 1:  bar0  bar1  [MEM k + copies of k+1, k+2] bar(2k+2) [COMP k]    bar(2k+3) ...
//
// COMP runs at raised wave priority (s_setprio), so that the SIMD's arbiter issues the MFMA stream first when both waves
// are ready: 6% faster in row mode, 0.4-0.9% in block mode (whose MEM phase carries little VALU besides one tile's fold).
//
// The ring has two stages of BK = 128 k-elements; k-tile k lives in stage k % 2. Which group copies which rows, and when,
// is set out at the DMA code below: copies go in MEM phases only, and each lands in rows that no group still has to read.
//
// LDS layout, DMA and swizzle as in gemm_ring.h: rows of 128 bytes in 16-byte chunks, chunk c of row r at physical
// chunk c ^ ((r >> 1) & 7); filled by buffer_load ... lds with zero-filled tails past M, N and K. A stage holds the
// token rows (with hi / lo: both rows of each token), then the channel rows, then (block mode) the k-block's token
// scales. With weight groups the k-block's channel scales go to a three-slot ring of their own (both groups read them
// during COMP).
#pragma once
#include "gemm_ring.h"

namespace wq8 {

template <int BM, int BN, int WAVES_N, int WAVES_M, int MODE, bool WG, bool BIASED, int DT, bool SEG, bool KTAIL = true, bool SPLIT = false,
          bool SUMS = false, int MF = 32, int STAGES = 2>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) gemm_pingpong(GemmArgs g) {
    static_assert(WAVES_N * WAVES_M == 8, "two groups of four waves");
    static_assert(STAGES == 2, "k-tile kt + 2 is copied into the stage of k-tile kt");
    // row mode; block mode with the biased fold; block mode with weight-group scales (the reference's fold order); the
    // exact mode, with or without weight-group scales
    static_assert(MODE == MODE_ROW || (MODE == MODE_BLOCK && BIASED != WG) || (MODE == MODE_EXACT && !BIASED),
                  "row, block (biased fold), block+g, exact and exact+g modes");
    static_assert(!(WG && SEG), "segments take per-channel scales");
    constexpr bool BLOCK = MODE == MODE_BLOCK;
    constexpr bool BIAS_FOLD = BLOCK && BIASED;
    // exact: two activation operands (hi, lo). With weight groups their block sums combine exactly in INT32 (254 hi +
    // lo) before each k-tile's fold; without, INT32 hi and lo accumulators run over the whole of K and the epilogue
    // combines them.
    constexpr bool HILO = MODE == MODE_EXACT;
    // block+g: the fold scales each block sum by sa[token, kb] * sb[channel, kb]; exact+g by sb[channel, kb] / 254 (the
    // token scale goes to the epilogue). Three VALU ops per element either way.
    constexpr bool GROUPED = WG;
    constexpr bool FOLD = BLOCK || (HILO && WG);  // FP32 accumulators, one fold per k-tile
    constexpr int WAVES = 8, BK = 128, CPR = 8, RPG = 8;
    constexpr int WN = BN / WAVES_N, WM = BM / WAVES_M;
    // MFMA tiles of MF x MF outputs: v_mfma_i32_32x32x32_i8 (MF 32, 4 k-steps of 32 per 128-element k-tile, 16 sums per
    // lane) or v_mfma_i32_16x16x64_i8 (MF 16, 2 k-steps of 64, 4 sums per lane)
    static_assert(MF == 32 || MF == 16, "MFMA tile");
    constexpr int FN = WN / MF, FM = WM / MF, KSTEPS = MF == 32 ? 4 : 2, EPT = MF * MF / 64;
    using Acc = typename MfmaI8<MF>::acc;
    using AccF = typename MfmaI8<MF>::accf;
    // token rows of a stage: BM, or with hi / lo 2 BM laid out as [hi, lo] of tokens [0, BM / 2), then [hi, lo] of
    // tokens [BM / 2, BM), so that each group's rows stay one contiguous half as in the other modes
    constexpr int AR = HILO ? 2 * BM : BM;
    static_assert(!HILO || (BM / 2) % WM == 0, "a wave's tokens lie in one half of the tile");
    constexpr int ROWS = AR + BN;
    constexpr int TILE_BYTES = ROWS * BK;
    constexpr int STAGE_BYTES = TILE_BYTES + (BLOCK ? WAVES * 256 : 0);
    constexpr int EPI_BYTES = WAVES * epilogue_stage_bytes<WN, WM>();
    constexpr int RING_BYTES = STAGES * STAGE_BYTES > EPI_BYTES ? STAGES * STAGE_BYTES : EPI_BYTES;
    static_assert(RING_BYTES <= 160 * 1024, "ring");
    using R = Ring<STAGES, STAGE_BYTES, RING_BYTES>;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int group = wave >> 2;
    const int wn = wave % WAVES_N, wm = wave / WAVES_N;
    const int m = g.m, n = g.n, k = g.k, kblocks = g.kblocks;
    const Work w = work_of_block(g);
    const int m0 = w.tm * BM, n0 = g.n_first + w.tn * BN;
    const long long in_shift = g.counter && (g.in_first || g.in_step) ? g.in_first + __ldg(g.counter) * g.in_step : 0;
    const float* sa = g.sa + in_shift * (BLOCK ? kblocks : 1);
    using Params = EpilogueParams<DT, MODE, WG, SEG, BM, BN>;
    static_assert(WAVES * 64 >= BN && WAVES * 64 >= BM, "one thread per channel and token of the tile");
    __shared__ __attribute__((aligned(16))) uint8_t params_lds[Params::BYTES];
    Params params;

    // ---- DMA: who copies what. Group 0 (waves 0-3) reads token rows [0, AR / 2) and every channel row, group 1 token
    // rows [AR / 2, AR) and every channel row (AR = BM, or 2 BM with hi / lo). The copies go in the MEM phases only (a wave stalled at the texture-address
    // unit in COMP would stall its MFMA stream), about half in each group's:
    //   group 0, MEM of k-tile kt: k-tile kt + 1's channel rows and block scales, into the other stage (its previous
    //     k-tile has been read by both groups);
    //   group 1, MEM of k-tile kt: first k-tile kt + 1's token rows [AR / 2, AR) (only group 1 reads them, two phases
    //     later), then k-tile kt + 2's token rows [0, AR / 2) into the stage it is reading itself (group 0 is done with
    //     them and group 1 never reads them).
    // Row groups are 8 rows of 128 bytes (one 1 KiB DMA instruction); wave u = wave % 4 of a group takes row groups
    // u + 4 i of each share.
    static_assert(WAVES_N == 2 && WAVES_M == 4 && AR % 128 == 0 && BN % 32 == 0, "groups split the token rows in halves");
    constexpr uint32_t OUT_OF_RANGE = 0x80000000u;
    constexpr int PA = AR / 64, PB = BN / 32;  // per wave: token row groups of a half, channel row groups
    // copies per wave and k-tile, groups 0 and 1 (group 0: channel row groups, then the token scales, then with
    // weight groups the channel scales)
    constexpr int L0 = PB + (BLOCK ? 1 : 0) + (GROUPED ? 1 : 0), L1 = 2 * PA;
    const int lr = lane / CPR, u = wave & 3;
    auto swz_of = [](int r) { return (r >> 1) & 7; };
    const sgpr4 rs_a = buffer_rsrc(g.a + in_shift * k, uint32_t(m) * uint32_t(k));
    const sgpr4 rs_lo = HILO ? buffer_rsrc(g.a_lo + in_shift * k, uint32_t(m) * uint32_t(k)) : rs_a;
    // row group u + 4 i starts at a row of the same parity as u: one chunk swizzle per wave
    const uint32_t chunk = uint32_t((lane % CPR) ^ swz_of(u * RPG + lr)) * 16u;
    // the k-tiles [kb0, kb1) of this workgroup (one k-tile = one 128-element k-block): all of K, or (SPLIT launches
    // only) a piece of a split tile. k-tile indices below are relative to kb0, whose byte offset is part of every copy's
    // base offset. Launches without split tiles keep the trip count in terms of K: the compiler then keeps the copy
    // addressing scalar (8 VALU ops fewer per k-tile in group 0's loop).
    const int kbase = SPLIT ? w.kb0 : 0;
    const int k_tiles = SPLIT ? w.kb1 - w.kb0 : (k + BK - 1) / BK;
    const uint32_t lane_part = uint32_t(lr) * uint32_t(k) + chunk;
    const uint32_t k_off = uint32_t(kbase) * 128u;  // byte offset of k-tile kb0 in a row
    // group 0: descriptors of its channel row groups
    sgpr4 rs_b[PB];
    uint32_t base_b[PB];
#pragma unroll
    for (int j = 0; j < PB; ++j) {
        const int c0 = n0 + (u + 4 * j) * RPG;
        if constexpr (SEG) {
            const int count = n / g.seg_rows;
            int s = c0 / g.seg_rows;
            s = s < count ? s : count - 1;
            rs_b[j] = buffer_rsrc(g.seg_b[s], uint32_t(g.seg_rows) * uint32_t(k));
            base_b[j] = uint32_t(c0 - s * g.seg_rows) * uint32_t(k) + k_off;
        } else {
            rs_b[j] = buffer_rsrc(g.b, uint32_t(n) * uint32_t(k));
            base_b[j] = uint32_t(c0) * uint32_t(k) + k_off;
        }
    }
    // block mode: the k-tile's activation scales (transposed, one row per k-block) land after the tile's rows, wave u of
    // group 0 copying tokens 64 u ..
    static_assert(!BLOCK || BM == 256, "one scale copy of 64 tokens per wave of group 0");
    const sgpr4 rs_s = buffer_rsrc(g.sa_t, uint32_t(m) * uint32_t(kblocks) * 4u);
    const uint32_t stride_s = uint32_t(m) * 4u, voff_s = uint32_t(m0 + 64 * u + lane) * 4u + stride_s * uint32_t(kbase);
    // weight groups: the k-tile's channel scales (transposed, one row per k-block) go to a ring of their own with three
    // slots, wave u of group 0 copying channels 64 u .. (waves past BN / 64 read zeros into the slot's padding). Both
    // groups read them in COMP, and group 1's COMP of k-tile kt overlaps group 0's copies of k-tile kt + 2: a third slot
    // keeps those copies off the scales still being read.
    // A slot holds a copy of each of the four waves: a copy past BN (out of range) still writes its 256 bytes of zeros to
    // LDS, which must land inside the slot, not in the next one (whose scales another group may be reading then).
    constexpr int CH_SLOT = 4 * 256;
    static_assert(BN <= 256, "one 64-channel copy per wave of group 0");
    __shared__ __attribute__((aligned(16))) uint8_t ch_lds[GROUPED ? 3 * CH_SLOT : 16];
    const sgpr4 rs_c = buffer_rsrc(GROUPED ? g.sb_t : g.sa_t, GROUPED ? uint32_t(n) * uint32_t(kblocks) * 4u : 0u);
    const uint32_t stride_c = uint32_t(n) * 4u;
    const uint32_t voff_c = GROUPED && 64 * u < BN ? uint32_t(n0 + 64 * u + lane) * 4u + stride_c * uint32_t(kbase) : OUT_OF_RANGE;
    // copies are branch free (a branch would split the phase they are spread over into blocks the compiler schedules
    // apart); the K tail reads zeros through out-of-range offsets
    const int k_lim = k - int(chunk) - kbase * BK;  // this lane's chunk of k-tile kt is inside the row when kt * BK < k_lim
    auto copy_rows = [&](int kt, const sgpr4& rs, uint32_t base, int r0) {
        const uint32_t kk = uint32_t(kt) * uint32_t(BK);
        // without a K tail (KTAIL false: K % BK == 0) every copy of k-tiles 0 .. k_tiles - 1 lies inside its rows; the
        // copies past the last k-tile then read other rows' bytes (zeros past the buffer) into stage rows nobody reads
        const uint32_t off = lane_part + (base + kk);
        bdma16(rs, !KTAIL || int(kk) < k_lim ? off : OUT_OF_RANGE, R::base() + (kt % STAGES) * STAGE_BYTES + r0 * BK);
    };
    // copy j of group G in the MEM of k-tile kt
    auto issue_part = [&](int kt, int j, auto group_tag) {
        constexpr int G = decltype(group_tag)::value;
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (G == 0) {
            if (j < PB) {
                copy_rows(kt + 1, rs_b[j], base_b[j], AR + (u + 4 * j) * RPG);
            } else if (BLOCK && j == PB) {
                bdma4(rs_s, voff_s + stride_s * uint32_t(kt + 1), R::base() + ((kt + 1) % STAGES) * STAGE_BYTES + TILE_BYTES + 256 * u);
            } else if constexpr (GROUPED) {
                bdma4(rs_c, voff_c + stride_c * uint32_t(kt + 1), ch_lds + ((kt + 1) % 3) * CH_SLOT + 256 * u);
            }
        } else {
            const int r0 = (j < PA ? AR / 2 : 0) + (u + 4 * (j % PA)) * RPG;
            if constexpr (HILO) {
                // stage row r0 of half h: hi row of token h BM / 2 + q, or the lo row of token h BM / 2 + q - BM / 2
                const int h = r0 / (AR / 2), q = r0 % (AR / 2), lo = q >= BM / 2;
                copy_rows(j < PA ? kt + 1 : kt + 2, lo ? rs_lo : rs_a, uint32_t(m0 + h * (BM / 2) + q - (lo ? BM / 2 : 0)) * uint32_t(k) + k_off, r0);
            } else {
                copy_rows(j < PA ? kt + 1 : kt + 2, rs_a, uint32_t(m0 + r0) * uint32_t(k) + k_off, r0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // ---- accumulators and fragments
    Acc acc[FOLD ? 1 : FN][FOLD ? 1 : FM], acc_lo[HILO && !FOLD ? FN : 1][HILO && !FOLD ? FM : 1];
    AccF accf[FOLD ? FN : 1][FOLD ? FM : 1];
    float corr[FM];
    Acc start = {};
    if constexpr (BIAS_FOLD) {
#pragma unroll
        for (int x = 0; x < EPT; ++x) start[x] = FOLD_BIAS_BITS;
    }
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) {
            if constexpr (FOLD) accf[i][j] = AccF{};
            else acc[i][j] = Acc{};
            if constexpr (HILO && !FOLD) acc_lo[i][j] = Acc{};
        }
#pragma unroll
    for (int j = 0; j < FM; ++j) corr[j] = 0.0f;
    // fragment row of the lane, and the 16-byte chunk of a 128-byte row it reads at k-step ks: MF 32: row lane % 32,
    // chunk 2 ks + lane / 32 (32 k a step); MF 16: row lane % 16, chunk 4 ks + lane / 16 (64 k a step)
    const int frag_row = lane & (MF - 1);
    auto swz = [&](int ks) { return ((MF == 32 ? 2 * ks + (lane >> 5) : 4 * ks + (lane >> 4)) ^ swz_of(frag_row)) << 4; };
    // per k-step fragment offsets of this lane within a stage (loop invariant: a read adds only the stage offset, and
    // the fragment index is an instruction immediate); with hi / lo the wave's hi rows start at its tokens' half and
    // its lo rows follow BM / 2 rows later
    constexpr int A_LO = HILO ? BM / 2 * BK : 0;  // byte offset of a token's lo row from its hi row
    const int a_row = HILO ? (wm * WM) / (BM / 2) * BM + (wm * WM) % (BM / 2) : wm * WM;
    uint32_t off_a[KSTEPS], off_b[KSTEPS];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
        off_a[ks] = uint32_t((a_row + frag_row) * BK + swz(ks));
        off_b[ks] = uint32_t(AR * BK + (wn * WN + frag_row) * BK + swz(ks));
    }
    v4i af[FM][KSTEPS], bf[FN][KSTEPS], lf[HILO ? FM : 1][KSTEPS];
    float s_tok[FM];
    // block mode: tiles [0, TC) of a k-tile fold during its COMP, each behind a later tile's chain; the last tiles have no
    // chain to hide behind and keep their block sums through the barrier to fold in the next MEM (with the copies in the
    // MEM phases, folding more tiles in COMP measured faster: with 32 x 32 tiles 5 of 6 > 4 > 3).
    // MF 16: a tile folds behind the chains of the next two tiles (its 4 sums wait 2 more MFMAs, without which each fold
    // stalls on its chain's last MFMA), so at least the last two tiles keep their sums for the MEM phase.
    // With weight groups (block+g) a fold costs three VALU ops per element instead of one, and moving more of them to the
    // MEM phase balances the phases: 6 of the 24 16 x 16 tiles kept, 4% faster than 2 at M = 8192, N = 12288, K = 3072
    // (8 measured the same as 6, 4 half way). exact+g gained nothing from keeping more than 2, but folds three tiles
    // behind (its fold waits on two chains, hi and lo): 1-1.4% faster than two at that shape, the same bits; the other
    // modes lose 0.7-1.2% with three.
#ifndef WQ8_FOLD_LAG16
#define WQ8_FOLD_LAG16 2
#endif
#ifndef WQ8_FOLD_LAG_EG
#define WQ8_FOLD_LAG_EG 3
#endif
    constexpr int LAG = MF == 16 ? (HILO && GROUPED ? WQ8_FOLD_LAG_EG : WQ8_FOLD_LAG16) : 1;
    constexpr int KEEP = GROUPED && !HILO ? (MF == 16 ? 6 : DT == DT_BF16 ? 2 : 1) : 1;
    constexpr int T = FN * FM, TC = FOLD ? T - (KEEP > LAG ? KEEP : LAG) : T;
    Acc sums[T - TC > 0 ? T - TC : 1], sums_lo[HILO && T > TC ? T - TC : 1];
    // before the first k-tile the MEM fold adds (1.5 * 2^23) * 0
#pragma unroll
    for (int j = 0; j < FM; ++j) s_tok[j] = 0.0f;
#pragma unroll
    for (int t = 0; t < T - TC; ++t) sums[t] = start;
    if constexpr (HILO) {
#pragma unroll
        for (int t = 0; t < T - TC; ++t) sums_lo[t] = Acc{};
    }

    // weight groups: the EPT channel scales of a lane in channel fragment i (MF 32: channels 8 (x / 4) + 4 (lane / 32) + x % 4
    // of the fragment; MF 16: 4 (lane / 16) + x), read from the k-tile's slot when fragment i's first tile starts its chain
    v4f ch_scale[GROUPED ? FN : 1][EPT / 4];
    // the first MEM folds the kept tiles' zero sums: with zero scales, not uninitialized registers (0 * NaN is NaN)
#pragma unroll
    for (int i = 0; i < (GROUPED ? FN : 1); ++i)
#pragma unroll
        for (int q = 0; q < EPT / 4; ++q) ch_scale[i][q] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    auto load_channel_scales = [&](int kt, int i) {
        if constexpr (GROUPED) {
            const float* sc = reinterpret_cast<const float*>(ch_lds + (kt % 3) * CH_SLOT) + wn * WN + i * MF + 4 * (lane / (MF == 32 ? 32 : 16));
#pragma unroll
            for (int q = 0; q < EPT / 4; ++q) ch_scale[i][q] = *reinterpret_cast<const v4f*>(sc + 8 * q);
        }
    };
    // fold of element x of tile (i, j) whose block sum is `sum` (the reference's order with weight groups:
    // accf = fmaf(float(S), sa * sb, accf)); exact+g: hi and lo sums combined exactly in INT32 (one v_mad_i32_i24:
    // |hi| <= 128 * 127^2 < 2^23), scaled by the channel scale / 254 that the launcher stored
    auto fold_grouped = [&](int i, int j, const Acc& sum, const Acc& sum_lo, int x) {
        const float cs = ch_scale[GROUPED ? i : 0][x >> 2][x & 3];
        if constexpr (HILO) accf[i][j][x] = __builtin_fmaf(float(__mul24(sum[x], 254) + sum_lo[x]), cs, accf[i][j][x]);
        else accf[i][j][x] = __builtin_fmaf(float(sum[x]), s_tok[j] * cs, accf[i][j][x]);
    };

    // fold of the block sums of tile t >= TC (previous k-tile, scales s_tok)
    auto fold_kept = [&](int t) {
        const int i = t / FM, j = t % FM;
        if constexpr (GROUPED) {
#pragma unroll
            for (int x = 0; x < EPT; ++x) fold_grouped(i, j, sums[t - TC], sums_lo[HILO ? t - TC : 0], x);
        } else {
            const AccF bits = __builtin_bit_cast(AccF, sums[t - TC]);
#pragma unroll
            for (int x = 0; x < EPT; ++x) accf[i][j][x] = __builtin_fmaf(bits[x], s_tok[j], accf[i][j][x]);
        }
    };

    // MEM of k-tile kt; the DMA of k-tile dma_kt (if any) is spread over the fragment reads; in block mode the kept
    // tiles of k-tile kt - 1 fold between the reads (each fold frees the registers of the next reads)
    auto mem = [&](int kt, auto group_tag) {
        constexpr int G = decltype(group_tag)::value, LOADS = G == 0 ? L0 : L1;
        const uint8_t* as = R::base() + (kt % STAGES) * STAGE_BYTES;
        constexpr int RPK = FM * (HILO ? 2 : 1) + FN, RD = KSTEPS * RPK;  // fragment reads per k-step, per k-tile
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            if constexpr (T > TC) {
                // the kept tiles fold over k-steps 1 .. KSTEPS - 1
                constexpr int NM = T - TC;
                const int lo = ks == 0 ? TC : TC + (ks - 1) * NM / (KSTEPS - 1), hi = ks == 0 ? TC : TC + ks * NM / (KSTEPS - 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int t = TC; t < T; ++t)
                    if (t >= lo && t < hi) fold_kept(t);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int j = 0; j < FM; ++j) af[j][ks] = *reinterpret_cast<const v4i*>(as + off_a[ks] + j * MF * BK);
            if constexpr (HILO) {
#pragma unroll
                for (int j = 0; j < FM; ++j) lf[j][ks] = *reinterpret_cast<const v4i*>(as + off_a[ks] + A_LO + j * MF * BK);
            }
#pragma unroll
            for (int i = 0; i < FN; ++i) bf[i][ks] = *reinterpret_cast<const v4i*>(as + off_b[ks] + i * MF * BK);
#pragma unroll
            for (int p = 0; p < LOADS; ++p) {
                const int at = p * RD / LOADS;  // read index after which part p goes
                if (at / RPK == ks) issue_part(kt, p, group_tag);
            }
        }
        if constexpr (BLOCK) {
            const float* scales = reinterpret_cast<const float*>(as + TILE_BYTES);
#pragma unroll
            for (int j = 0; j < FM; ++j) s_tok[j] = scales[wm * WM + j * MF + frag_row];
        }
    };

    // fold of elements [x0, x1) of tile (i, j) whose block sums are `sum` (tiles folded during COMP)
    auto fold_part = [&](int i, int j, const Acc& sum, const Acc& sum_lo, int x0, int x1) {
        if constexpr (GROUPED) {
#pragma unroll
            for (int x = x0; x < x1; ++x) fold_grouped(i, j, sum, sum_lo, x);
        } else if constexpr (BIAS_FOLD) {
            const AccF bits = __builtin_bit_cast(AccF, sum);
#pragma unroll
            for (int x = x0; x < x1; ++x) accf[i][j][x] = __builtin_fmaf(bits[x], s_tok[j], accf[i][j][x]);
        } else {
#pragma unroll
            for (int x = x0; x < x1; ++x) accf[i][j][x] = __builtin_fmaf(float(sum[x]), s_tok[j], accf[i][j][x]);
        }
    };
    // the fold of the previous tile follows k-steps 1, 2 and 3 of the next chain (6 + 5 + 5 elements; MF 16: all 4 after
    // k-step 1): its last MFMA has finished by then
    auto fold_slice = [](int ks, int& x0, int& x1) {
        if constexpr (MF == 16) {
            x0 = ks == 1 ? 0 : 4;
            x1 = 4;
        } else {
            x0 = ks == 1 ? 0 : ks == 2 ? 6 : ks == 3 ? 11 : 16;
            x1 = ks == 1 ? 6 : ks == 2 ? 11 : 16;
        }
    };

    // COMP of the k-tile in registers; the DMA of k-tile dma_kt (if any) is spread over the MFMAs
    auto comp = [&](int kt) {
        if constexpr (FOLD) {
            // tile-major: each MF x MF tile chains its KSTEPS MFMAs on a fresh accumulator; the fold of tile t - LAG < TC
            // follows k-steps 1 .. KSTEPS - 1 of chain t, the sums of tiles t >= TC are kept for the next MEM
            if constexpr (BIAS_FOLD) {
#pragma unroll
                for (int j = 0; j < FM; ++j) corr[j] = __builtin_fmaf(FOLD_BIAS, s_tok[j], corr[j]);
            }
            Acc prev[LAG], prev_lo[LAG];  // sums of tiles t - 1 .. t - LAG
#pragma unroll
            for (int l = 0; l < LAG; ++l) prev[l] = start, prev_lo[l] = Acc{};
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    const int t = i * FM + j, pt = t - LAG, pi = (pt + FM * LAG) / FM - LAG, pj = (pt + FM * LAG) % FM;
                    if (GROUPED && j == 0) load_channel_scales(kt, i);
                    Acc c = start, c_lo = Acc{};
#pragma unroll
                    for (int ks = 0; ks < KSTEPS; ++ks) {
                        __builtin_amdgcn_sched_barrier(0);
                        c = MfmaI8<MF>::run(bf[i][ks], af[j][ks], c);
                        if constexpr (HILO) c_lo = MfmaI8<MF>::run(bf[i][ks], lf[j][ks], c_lo);
                        if (pt >= 0 && pt < TC && ks > 0) {
                            int x0, x1;
                            fold_slice(ks, x0, x1);
                            fold_part(pi, pj, prev[LAG - 1], prev_lo[LAG - 1], x0, x1);
                        }
                    }
#pragma unroll
                    for (int l = LAG - 1; l > 0; --l) {
                        prev[l] = prev[l - 1];
                        if constexpr (HILO) prev_lo[l] = prev_lo[l - 1];
                    }
                    prev[0] = c;
                    if constexpr (HILO) prev_lo[0] = c_lo;
                    if constexpr (SUMS) {
                        // test builds only: the exact INT32 block sums of tile (i, j), sums[(t * N + ch) * ceil(K / 128) + kb]
                        const int t_row = m0 + wm * WM + j * MF + frag_row;
#pragma unroll
                        for (int x = 0; x < EPT; ++x) {
                            const int ch = n0 + wn * WN + i * MF + (MF == 32 ? 8 * (x >> 2) + 4 * (lane >> 5) + (x & 3) : 4 * (lane >> 4) + x);
                            if (t_row < m && ch < n) g.sums[(int64_t(t_row) * n + ch) * kblocks + kbase + kt] = c[x] - start[x];
                        }
                    }
                    if (t >= TC) {
                        sums[t - TC] = c;
                        if constexpr (HILO) sums_lo[t - TC] = c_lo;
                    }
                }

            __builtin_amdgcn_sched_barrier(0);
        } else {
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
                for (int i = 0; i < FN; ++i)
#pragma unroll
                    for (int j = 0; j < FM; ++j) {
                        acc[i][j] = MfmaI8<MF>::run(bf[i][ks], af[j][ks], acc[i][j]);
                        if constexpr (HILO) acc_lo[i][j] = MfmaI8<MF>::run(bf[i][ks], lf[j][ks], acc_lo[i][j]);
                    }
        }
    };

    auto barrier = []() {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    // ---- prologue: k-tile 0 whole and k-tile 1's token rows [0, BM / 2), all landed before bar0; in the MEM of k-tile 0
    // group 0 copies k-tile 1's channel rows and scales, group 1 its token rows [BM / 2, BM)
    if (group == 0) {
#pragma unroll
        for (int j = 0; j < L0; ++j) issue_part(-1, j, IntC<0>{});
    } else {
#pragma unroll
        for (int j = 0; j < PA; ++j) issue_part(-1, j, IntC<1>{});  // k-tile 0, rows [BM / 2, BM)
#pragma unroll
        for (int j = PA; j < L1; ++j) issue_part(-2, j, IntC<1>{});  // k-tile 0, rows [0, BM / 2)
#pragma unroll
        for (int j = PA; j < L1; ++j) issue_part(-1, j, IntC<1>{});  // k-tile 1, rows [0, BM / 2)
    }
    // the epilogue parameters load behind the first DMA and are parked in their own LDS array before the first barrier
    // (vector loads complete in issue order: the prologue's wait covers them; no registers held through the mainloop)
    params.load(g, m0, n0, sa, tid);
    wait_vmcnt<0>();
    params.park(params_lds, tid);
    barrier();  // bar0
    if (group == 0) {
        for (int kt = 0; kt < k_tiles; ++kt) {
            mem(kt, IntC<0>{});
            wait_lgkm0();
            barrier();  // bar(2kt+1)
            __builtin_amdgcn_s_setprio(1);
            comp(kt);
            __builtin_amdgcn_s_setprio(0);
            wait_vmcnt<0>();  // k-tile kt + 1's copies have landed
            barrier();  // bar(2kt+2)
        }
        barrier();  // bar(2KT+1)
    } else {
        barrier();  // bar1
        for (int kt = 0; kt < k_tiles; ++kt) {
            mem(kt, IntC<1>{});
            wait_lgkm0();
            wait_vmcnt<L1>();  // the previous MEM's copies (k-tile kt + 1's token rows [0, BM / 2)) have landed
            barrier();  // bar(2kt+2)
            __builtin_amdgcn_s_setprio(1);
            comp(kt);
            __builtin_amdgcn_s_setprio(0);
            wait_vmcnt<PA>();  // this MEM's copies of k-tile kt + 1 (token rows [BM / 2, BM)), issued first, have landed
            barrier();  // bar(2kt+3)
        }
    }
    wait_vmcnt<0>();
#pragma unroll
    for (int t = TC; t < T; ++t) fold_kept(t);  // the kept tiles of the last k-tile
    // every wave is done with the ring (the last barrier follows the last LDS read of both groups) and, after each
    // wave's vmcnt(0), no copy (the zero-filled slots past the last k-tile included) is in flight
    __syncthreads();
    uint8_t* stage = R::base() + wave * epilogue_stage_bytes<WN, WM>();
    if constexpr (SUMS) return;
    if (SPLIT && w.tail >= 0) {
        if (g.defer) {
            // deep split: the piece's pre-epilogue values (FP32, with the biased fold's bias taken off) or INT32 sums go
            // to its planes; gemm_split_finish adds the pieces and runs the epilogue
            defer_store<FN, FM, WN, WM, MF, HILO && !FOLD ? 2 : 1>(g, m0, n0, wn, wm, w.piece, [&](int i, int j, int x, int h) -> uint32_t {
                if constexpr (FOLD) return __builtin_bit_cast(uint32_t, BIAS_FOLD ? accf[i][j][x] - corr[j] : accf[i][j][x]);
                else if constexpr (HILO) return uint32_t(h == 0 ? acc[i][j][x] : acc_lo[i][j][x]);
                else return uint32_t(acc[i][j][x]);
            });
            return;
        }
        // a piece of a split tile: its pre-epilogue values (FP32, with the biased fold's bias taken off) or INT32 sums go
        // to its slot; the last piece to arrive runs the epilogue on the sums of all pieces
        constexpr int NT = FN * FM * EPT, NV = NT * (HILO && !FOLD ? 2 : 1);
        // word v: element v % EPT of tile ((v % NT) / EPT) / FM, ((v % NT) / EPT) % FM; with hi / lo, v >= NT is the lo sum
        const bool last = split_arrive<NV, 512>(g, w, [&](int v) -> uint32_t {
            const int e = v % NT, i = e / EPT / FM, j = e / EPT % FM, x = e % EPT;
            if constexpr (FOLD) return __builtin_bit_cast(uint32_t, BIAS_FOLD ? accf[i][j][x] - corr[j] : accf[i][j][x]);
            else if constexpr (HILO) return uint32_t(v < NT ? acc[i][j][x] : acc_lo[i][j][x]);
            else return uint32_t(acc[i][j][x]);
        });
        if (!last) return;
        gemm_epilogue<DT, MODE, WG, SEG, BM, BN, FN, FM, WN, WM, MF>(g, m0, n0, wn, wm, params_lds, stage, [&](int i, int j, int x) {
            const int e = (i * FM + j) * EPT + x;
            if constexpr (FOLD) return __builtin_bit_cast(float, split_sum<NV, 512, true>(g, w, e));
            else if constexpr (HILO)
                return __builtin_fmaf(float(int32_t(split_sum<NV, 512, false>(g, w, NT + e))), 1.0f / 254.0f,
                                      float(int32_t(split_sum<NV, 512, false>(g, w, e))));
            else return float(int32_t(split_sum<NV, 512, false>(g, w, e)));
        });
        return;
    }
    gemm_epilogue<DT, MODE, WG, SEG, BM, BN, FN, FM, WN, WM, MF>(g, m0, n0, wn, wm, params_lds, stage, [&](int i, int j, int x) {
        if constexpr (BIAS_FOLD) return accf[i][j][x] - corr[j];
        else if constexpr (FOLD) return accf[i][j][x];
        // exact: the reference's combination of the two products (K8:790-799)
        else if constexpr (HILO) return __builtin_fmaf(float(acc_lo[i][j][x]), 1.0f / 254.0f, float(acc[i][j][x]));
        else return float(acc[i][j][x]);
    });
}

}  // namespace wq8
