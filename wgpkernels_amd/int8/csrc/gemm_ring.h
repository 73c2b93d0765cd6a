// INT8 GEMM mainloop for every mode: BM tokens x BN channels per workgroup, k-steps of 32 on v_mfma_i32_32x32x32_i8,
// operands streamed through a deep LDS ring.
//
// - Fetch: each ring stage holds one BK-element slice of the tile's token rows and channel rows (BK = 64 or 128 bytes per row),
//   filled straight from global memory by buffer_load ... lds (SGPR resource descriptors; out-of-range offsets read
//   zeros, which pads rows past M / N and the K tail). The ring is STAGES deep and STAGES - 2 stages stay in flight
//   while one is computed: the L2 / Infinity-Cache fetch rate of a CU is bounded by the bytes it has in flight (about
//   100 KiB are needed for a 128 x 256 tile at a high MFMA rate), so shallow rings of big stages starve.
// - LDS layout: rows of BK bytes in 16-byte chunks, chunk c of row r at physical chunk c ^ f(r) with
//   f(r) = (r >> 1) & 7 for 128-byte rows and (r >> 2) & 3 for 64-byte rows. gfx950 serves a ds_read_b128 16 lanes at a
//   time over 64 banks (256 bytes); a fragment read (32 rows, one logical chunk) is then conflict free (measured with
//   SQ_LDS_BANK_CONFLICT).
// - The weights are the MFMA A operand (32 channels), the activations the B operand (32 tokens): a lane of a 32x32
//   accumulator holds one token and 16 channels, so a block fold needs one activation scale per lane and fragment.
// - Folds (block modes) run once per 128-element K block, after the k-steps of that block:
//     reference order  accf = fmaf(float(S), scale, accf)                                   (block+g, SUMS)
//     combined hi/lo   accf = fmaf(float(254 S_hi + S_lo), sb / 254, accf), the INT32 combination exact  (exact+g)
//     biased           accumulation starts at 1.5 * 2^23 in every element, so the INT32 result is the bit pattern of
//                      the float 1.5 * 2^23 + S (|S| < 2^22): accf = fmaf(bits, sa, accf), one VALU op instead of two;
//                      the bias part 1.5 * 2^23 * sum(sa) is common to all channels of a token (corr) and subtracted in
//                      the epilogue. Adds ~1e-4 relative error, far inside the block quantization error.
#pragma once
#include "gemm_common.h"

namespace wq8 {

// LDS ring of STAGES stages of BYTES each, one contiguous array of TOTAL >= STAGES * BYTES bytes (the epilogue reuses
// it as staging).
template <int STAGES, int BYTES, int TOTAL> struct Ring {
    static WQ8_DEVICE uint8_t* base() {
        __shared__ __attribute__((aligned(1024))) uint8_t ring[TOTAL];
        return ring;
    }
    template <int S> static WQ8_DEVICE uint8_t* at() {
        static_assert(S < STAGES, "stage index");
        return base() + S * BYTES;
    }
};

constexpr float FOLD_BIAS = 12582912.0f;  // 1.5 * 2^23
constexpr int FOLD_BIAS_BITS = 0x4B400000;

// Scheduling groups (LLVM AMDGPU sched_group_barrier masks: 0x008 MFMA, 0x100 LDS read): k-step KS issues its MF MFMAs
// one at a time, with the RD LDS reads of k-step KS + 2 spread between them.
template <int RD, int MF, int X, bool AHEAD> WQ8_DEVICE void sched_slots() {
    if constexpr (X < MF) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        constexpr int reads = (X + 1) * RD / MF - X * RD / MF;
        if constexpr (AHEAD && reads > 0) __builtin_amdgcn_sched_group_barrier(0x100, reads, 0);
        sched_slots<RD, MF, X + 1, AHEAD>();
    }
}
template <int RD, int MF, int KS, int KSTEPS> WQ8_DEVICE void sched_ksteps() {
    if constexpr (KS < KSTEPS) {
        sched_slots<RD, MF, 0, (KS + 2 < KSTEPS)>();
        sched_ksteps<RD, MF, KS + 1, KSTEPS>();
    }
}

// s_waitcnt vmcnt(n) for a runtime n (the counter field is an immediate)
WQ8_DEVICE void wait_vmcnt_rt(int n) {
    switch (n) {
        case 0: wait_vmcnt<0>(); break;   case 1: wait_vmcnt<1>(); break;   case 2: wait_vmcnt<2>(); break;
        case 3: wait_vmcnt<3>(); break;   case 4: wait_vmcnt<4>(); break;   case 5: wait_vmcnt<5>(); break;
        case 6: wait_vmcnt<6>(); break;   case 7: wait_vmcnt<7>(); break;   case 8: wait_vmcnt<8>(); break;
        case 9: wait_vmcnt<9>(); break;   case 10: wait_vmcnt<10>(); break; case 11: wait_vmcnt<11>(); break;
        case 12: wait_vmcnt<12>(); break; case 13: wait_vmcnt<13>(); break; case 14: wait_vmcnt<14>(); break;
        case 15: wait_vmcnt<15>(); break; case 16: wait_vmcnt<16>(); break; case 17: wait_vmcnt<17>(); break;
        case 18: wait_vmcnt<18>(); break; case 19: wait_vmcnt<19>(); break; case 20: wait_vmcnt<20>(); break;
        case 21: wait_vmcnt<21>(); break; case 22: wait_vmcnt<22>(); break; case 23: wait_vmcnt<23>(); break;
        default: wait_vmcnt<24>(); break;
    }
}

template <int BM, int BN, int WAVES_N, int WAVES_M, int BK, int STAGES, int MODE, bool WG, bool BIASED, int DT, bool SUMS, bool SEG,
          bool SPLIT = false>
__global__ void __launch_bounds__(64 * WAVES_N * WAVES_M)
__attribute__((amdgpu_waves_per_eu((WAVES_N * WAVES_M + 3) / 4, (WAVES_N * WAVES_M + 3) / 4))) gemm_ring(GemmArgs g) {
    constexpr bool HILO = MODE == MODE_EXACT;
    constexpr bool FOLD = (MODE == MODE_BLOCK || WG) && !SUMS;
    constexpr bool BIAS_FOLD = BIASED && FOLD && MODE == MODE_BLOCK && !WG;
    constexpr int WAVES = WAVES_N * WAVES_M;
    constexpr int WN = BN / WAVES_N, WM = BM / WAVES_M;
    constexpr int FN = WN / 32, FM = WM / 32;
    constexpr int A_ROWS = BM * (HILO ? 2 : 1);
    constexpr int ROWS = A_ROWS + BN;
    constexpr int CPR = BK / 16;                  // 16-byte chunks per row
    constexpr int RPG = 1024 / BK;                // rows per 1 KiB DMA group
    constexpr int GROUPS = ROWS / RPG, G_PER_WAVE = GROUPS / WAVES;
    constexpr int TILE_BYTES = ROWS * BK;
    constexpr int STAGE_BYTES = TILE_BYTES + ((MODE == MODE_BLOCK || WG) ? WAVES * 256 : 0);
    constexpr int LOADS = G_PER_WAVE + ((MODE == MODE_BLOCK || WG) ? 1 : 0);  // DMA instructions per wave and stage
    constexpr int KSTEPS = BK / 32;
    constexpr int PER_BLOCK = 128 / BK;           // stages per 128-element scale block
    static_assert(BK == 64 || BK == 128, "stage depth");
    static_assert(BM % 32 == 0 && BN % 32 == 0 && FN >= 1 && FM >= 1, "tile");
    static_assert(GROUPS % WAVES == 0, "whole DMA groups per wave");
    static_assert(((MODE == MODE_BLOCK) ? BM : 0) + (WG ? BN : 0) <= WAVES * 64, "one scale DMA per wave");
    constexpr int EPI_BYTES = WAVES * epilogue_stage_bytes<WN, WM>();
    constexpr int RING_BYTES = STAGES * STAGE_BYTES > EPI_BYTES ? STAGES * STAGE_BYTES : EPI_BYTES;
    static_assert(STAGES >= 2 && RING_BYTES <= 160 * 1024, "ring");
    using R = Ring<STAGES, STAGE_BYTES, RING_BYTES>;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave % WAVES_N, wm = wave / WAVES_N;
    const int m = g.m, n = g.n, k = g.k, kblocks = g.kblocks;
    const Work w = work_of_block(g);
    const int m0 = w.tm * BM, n0 = g.n_first + w.tn * BN;
    const long long in_shift = g.counter && (g.in_first || g.in_step) ? g.in_first + __ldg(g.counter) * g.in_step : 0;
    const float* sa = g.sa + in_shift * (MODE == MODE_BLOCK ? kblocks : 1);
    using Params = EpilogueParams<DT, MODE, WG, SEG, BM, BN>;
    static_assert(WAVES * 64 >= BN && WAVES * 64 >= BM, "one thread per channel and token of the tile");
    __shared__ __attribute__((aligned(16))) uint8_t params_lds[Params::BYTES];
    // the parameters' registers stay live through the mainloop: prefetched only where registers are not the limit
    constexpr bool PREFETCH_PARAMS = true;
    Params params;
    if constexpr (!SUMS && PREFETCH_PARAMS) params.load(g, m0, n0, sa, tid);

    // ---- DMA: wave w copies row groups w + WAVES j (RPG rows = 1 KiB); lane l fills physical chunk l % CPR of row
    // l / CPR of the group, i.e. logical chunk (l % CPR) ^ f(r). Token rows [0, BM) (hi), [BM, 2 BM) (lo), then channel
    // rows. All offsets are 32-bit byte offsets inside per-operand buffer descriptors.
    constexpr uint32_t OUT_OF_RANGE = 0x80000000u;
    const int lr = lane / CPR;
    auto swz_of = [](int r) { return CPR == 8 ? (r >> 1) & 7 : (r >> 2) & 3; };
    const sgpr4 rs_a = buffer_rsrc(g.a + in_shift * k, uint32_t(m) * uint32_t(k));
    const sgpr4 rs_lo = HILO ? buffer_rsrc(g.a_lo + in_shift * k, uint32_t(m) * uint32_t(k)) : rs_a;
    // the swizzle of row r0 + lr is the same for every group of a wave (r0 = (wave + WAVES j) RPG, WAVES even), so a
    // lane's offset is lane_part plus a per-group uniform row base (SGPRs)
    static_assert(WAVES % 2 == 0 || CPR == 4, "group-independent swizzle");
    const uint32_t chunk = uint32_t((lane % CPR) ^ swz_of(wave * RPG + lr)) * 16u;  // byte offset of the lane's chunk
    const uint32_t lane_part = uint32_t(lr) * uint32_t(k) + chunk;
    sgpr4 rs_row[G_PER_WAVE];
    uint32_t base_row[G_PER_WAVE];
#pragma unroll
    for (int j = 0; j < G_PER_WAVE; ++j) {
        const int r0 = (wave + WAVES * j) * RPG;  // first row of the group (uniform)
        if (r0 < A_ROWS) {
            rs_row[j] = HILO && r0 >= BM ? rs_lo : rs_a;
            base_row[j] = uint32_t(m0 + (r0 % BM)) * uint32_t(k);
        } else {
            const int c0 = n0 + (r0 - A_ROWS);
            if constexpr (SEG) {
                const int count = n / g.seg_rows;
                int s = c0 / g.seg_rows;
                s = s < count ? s : count - 1;
                rs_row[j] = buffer_rsrc(g.seg_b[s], uint32_t(g.seg_rows) * uint32_t(k));
                base_row[j] = uint32_t(c0 - s * g.seg_rows) * uint32_t(k);
            } else {
                rs_row[j] = buffer_rsrc(g.b, uint32_t(n) * uint32_t(k));
                base_row[j] = uint32_t(c0) * uint32_t(k);
            }
        }
    }
    // scales of the k-tile's 128-element block: float slot wave * 64 + lane = sa of the tile's tokens (block mode), then
    // sb of its channels (weight groups); other slots read zeros. The launcher transposes the scales to one row per
    // k-block (sa_t[kb * m + t], sb_t[kb * n + c]), so a wave's 64 scales are 256 contiguous bytes.
    sgpr4 rs_s = buffer_rsrc(g.sa_t, uint32_t(m) * uint32_t(kblocks) * 4u);
    uint32_t voff_s = OUT_OF_RANGE, stride_s = 0;
    {
        // slot groups of 64 per wave: BM is a multiple of 64 in block mode, so the choice is uniform per wave
        constexpr int SA_SLOTS = MODE == MODE_BLOCK ? BM : 0;
        static_assert(SA_SLOTS % 64 == 0, "whole waves of activation scales");
        if (MODE == MODE_BLOCK && wave * 64 < SA_SLOTS) {
            voff_s = uint32_t(m0 + wave * 64 + lane) * 4u;
            stride_s = uint32_t(m) * 4u;
        }
        const int wslot = wave * 64 - SA_SLOTS;
        if (WG && wslot >= 0 && wslot < BN) {
            rs_s = buffer_rsrc(g.sb_t, uint32_t(n) * uint32_t(kblocks) * 4u);
            voff_s = uint32_t(n0 + wslot + lane) * 4u;
            stride_s = uint32_t(n) * 4u;
        }
    }
    // the k-tiles [kbase, kbase + k_tiles) of this workgroup: all of K, or (SPLIT launches only) the k-blocks of a piece
    // of a split tile; k-tile indices below are relative to kbase
    const int kbase = SPLIT ? w.kb0 * PER_BLOCK : 0;
    const int k_end = w.kb1 * 128 < k ? w.kb1 * 128 : k;
    const int k_tiles = SPLIT ? (k_end - w.kb0 * 128 + BK - 1) / BK : (k + BK - 1) / BK;
    auto issue = [&](auto st, int kt_rel) {
        uint8_t* base = R::template at<decltype(st)::value>();
        const int kt = kt_rel + kbase;
        const uint32_t kk = uint32_t(kt) * uint32_t(BK);
        if (kt * BK + BK <= k) {  // whole k-tile (uniform): no per-lane tail check
#pragma unroll
            for (int j = 0; j < G_PER_WAVE; ++j) bdma16(rs_row[j], lane_part + (base_row[j] + kk), base + (wave + WAVES * j) * 1024);
        } else {
#pragma unroll
            for (int j = 0; j < G_PER_WAVE; ++j)
                bdma16(rs_row[j], kt * BK + int(chunk) < k ? lane_part + (base_row[j] + kk) : OUT_OF_RANGE, base + (wave + WAVES * j) * 1024);
        }
        // waves without scales to copy read out of range (OUT_OF_RANGE plus a small offset stays out of range)
        if constexpr (MODE == MODE_BLOCK || WG) bdma4(rs_s, voff_s + stride_s * uint32_t(kt / PER_BLOCK), base + TILE_BYTES + wave * 256);
    };

    v16i acc[FN][FM];
    v16i acc_lo[HILO ? FN : 1][HILO ? FM : 1];
    v16f accf[FOLD ? FN : 1][FOLD ? FM : 1];
    float corr[FM];
    v16i start = {};
    if constexpr (BIAS_FOLD) {
#pragma unroll
        for (int x = 0; x < 16; ++x) start[x] = FOLD_BIAS_BITS;
    }
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) {
            acc[i][j] = start;
            if constexpr (HILO) acc_lo[i][j] = v16i{};
            if constexpr (FOLD) accf[i][j] = v16f{};
        }
#pragma unroll
    for (int j = 0; j < FM; ++j) corr[j] = 0.0f;
    const int frag_row = lane & 31;
    // physical chunk of logical chunk 2 ks + lane / 32 in fragment row lane % 32
    auto swz = [&](int ks) { return ((2 * ks + (lane >> 5)) ^ swz_of(frag_row)) << 4; };

    // fold of one 32x32 tile (i, j) whose block sums are `sum` (and `sum_lo` for hi/lo), scales from the stage
    // fold of elements [4 g0, 4 g1) of one 32x32 tile (i, j) whose block sums are `sum` (and `sum_lo` for hi/lo);
    // s_tok = the tile's activation scale of this lane's token (block mode)
    auto fold_part = [&](const float* scales, int i, int j, float s_tok, const v16i& sum, const v16i& sum_lo, int g0, int g1) {
        if constexpr (BIAS_FOLD) {
            // the whole vector is reinterpreted at once (element-wise bit casts of an MFMA result were merged into one
            // element by this compiler)
            const v16f bits = __builtin_bit_cast(v16f, sum);
#pragma unroll
            for (int x = 4 * g0; x < 4 * g1; ++x) accf[i][j][x] = __builtin_fmaf(bits[x], s_tok, accf[i][j][x]);
        } else if constexpr (WG) {
            const float* sbk = scales + (MODE == MODE_BLOCK ? BM : 0) + wn * WN + i * 32 + 4 * (lane >> 5);
#pragma unroll
            for (int gi = g0; gi < g1; ++gi) {
                const v4f s4 = *reinterpret_cast<const v4f*>(sbk + 8 * gi);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int x = 4 * gi + e;
                    if constexpr (MODE == MODE_BLOCK) {
                        accf[i][j][x] = __builtin_fmaf(float(sum[x]), s_tok * s4[e], accf[i][j][x]);
                    } else {
                        // hi and lo sums combined exactly in INT32 (one v_mad_i32_i24: |hi| <= 128 * 127^2 < 2^23), then
                        // scaled by the channel scale / 254 that the launcher stored: three VALU ops instead of four
                        const int32_t combined = __mul24(sum[x], 254) + sum_lo[x];
                        accf[i][j][x] = __builtin_fmaf(float(combined), s4[e], accf[i][j][x]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int x = 4 * g0; x < 4 * g1; ++x) accf[i][j][x] = __builtin_fmaf(float(sum[x]), s_tok, accf[i][j][x]);
        }
    };
    auto token_scale = [&](const float* scales, int j) { return MODE == MODE_BLOCK ? scales[wm * WM + j * 32 + frag_row] : 1.0f; };
    auto fold_tile = [&](const float* scales, int i, int j, const v16i& sum, const v16i& sum_lo) {
        fold_part(scales, i, j, token_scale(scales, j), sum, sum_lo, 0, 4);
    };

    auto compute = [&](auto st, int kt) {
        const uint8_t* as = R::template at<decltype(st)::value>();
        const uint8_t* bs = as + A_ROWS * BK;
        const float* scales = reinterpret_cast<const float*>(as + TILE_BYTES);
        constexpr bool TILE_MAJOR = FOLD && !HILO && PER_BLOCK == 1;
        if constexpr (TILE_MAJOR) {
            // one k-tile = one scale block: every 32x32 tile chains its KSTEPS MFMAs on a fresh accumulator, and a
            // quarter of the previous tile's fold follows each of them (MFMA and VALU pipes overlap; scheduling
            // barriers keep this order); the channel fragments of row i + 1 are read during row i
            static_assert(KSTEPS == 4, "one fold quarter per k-step");
            v4i af[FM][KSTEPS], bf[2][KSTEPS];
            float s_tok[FM];
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
                for (int j = 0; j < FM; ++j) af[j][ks] = *reinterpret_cast<const v4i*>(as + (wm * WM + j * 32 + frag_row) * BK + swz(ks));
#pragma unroll
            for (int j = 0; j < FM; ++j) s_tok[j] = token_scale(scales, j);
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) bf[0][ks] = *reinterpret_cast<const v4i*>(bs + (wn * WN + frag_row) * BK + swz(ks));
            if constexpr (BIAS_FOLD) {
#pragma unroll
                for (int j = 0; j < FM; ++j) corr[j] = __builtin_fmaf(FOLD_BIAS, s_tok[j], corr[j]);
            }
            v16i prev = start;
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                if (i + 1 < FN) {
#pragma unroll
                    for (int ks = 0; ks < KSTEPS; ++ks)
                        bf[(i + 1) & 1][ks] = *reinterpret_cast<const v4i*>(bs + (wn * WN + (i + 1) * 32 + frag_row) * BK + swz(ks));
                }
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    const int t = i * FM + j, pi = (t - 1) / FM, pj = (t - 1) % FM;
                    v16i c = start;
#pragma unroll
                    for (int ks = 0; ks < KSTEPS; ++ks) {
                        __builtin_amdgcn_sched_barrier(0);
                        c = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[i & 1][ks], af[j][ks], c, 0, 0, 0);
                        if (t > 0) fold_part(scales, pi, pj, s_tok[pj], prev, prev, ks, ks + 1);
                    }
                    prev = c;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            fold_part(scales, FN - 1, FM - 1, s_tok[FM - 1], prev, prev, 0, 4);
            return;
        }
        // every fragment of the k-tile is read first (the reads stay in flight while the MFMAs of earlier k-steps
        // issue), then the MFMAs run k-step by k-step
        v4i bf[KSTEPS][FN], af[KSTEPS][FM], lf[KSTEPS][HILO ? FM : 1];
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            const int sw = swz(ks);
#pragma unroll
            for (int i = 0; i < FN; ++i) bf[ks][i] = *reinterpret_cast<const v4i*>(bs + (wn * WN + i * 32 + frag_row) * BK + sw);
#pragma unroll
            for (int j = 0; j < FM; ++j) {
                af[ks][j] = *reinterpret_cast<const v4i*>(as + (wm * WM + j * 32 + frag_row) * BK + sw);
                if constexpr (HILO) lf[ks][j] = *reinterpret_cast<const v4i*>(as + (BM + wm * WM + j * 32 + frag_row) * BK + sw);
            }
        }
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[ks][i], af[ks][j], acc[i][j], 0, 0, 0);
                    if constexpr (HILO) acc_lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[ks][i], lf[ks][j], acc_lo[i][j], 0, 0, 0);
                }
        }
        // issue order (the compiler would otherwise sink every read next to its first use): the reads of k-steps 0 and
        // 1, then each k-step's MFMAs interleaved one for one with the reads of the k-step two ahead
        {
            constexpr int RD = FN + FM * (HILO ? 2 : 1), MF = FN * FM * (HILO ? 2 : 1);
            __builtin_amdgcn_sched_group_barrier(0x100, KSTEPS > 1 ? 2 * RD : RD, 0);
            sched_ksteps<RD, MF, 0, KSTEPS>();
        }
        if ((kt + 1) % PER_BLOCK != 0 && kt + 1 != k_tiles) return;  // the block continues in the next stage
        const int kb = (kt + kbase) / PER_BLOCK;
        if constexpr (SUMS) {
            // exact INT32 block sums, dumped as sums[(t * N + c) * kblocks + kb]
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    const int t = m0 + wm * WM + j * 32 + frag_row;
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int c = n0 + wn * WN + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                        if (t < m && c < n) g.sums[(int64_t(t) * n + c) * kblocks + kb] = acc[i][j][e];
                    }
                    acc[i][j] = v16i{};
                }
        } else if constexpr (FOLD) {
            if constexpr (BIAS_FOLD) {
#pragma unroll
                for (int j = 0; j < FM; ++j) corr[j] = __builtin_fmaf(FOLD_BIAS, scales[wm * WM + j * 32 + frag_row], corr[j]);
            }
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int i = 0; i < FN; ++i) {
                    fold_tile(scales, i, j, acc[i][j], acc_lo[HILO ? i : 0][HILO ? j : 0]);
                    acc[i][j] = start;
                    if constexpr (HILO) acc_lo[i][j] = v16i{};
                }
        }
    };

    // iteration kt: wait for this wave's DMA of k-tile kt (the later k-tiles' stay in flight), barrier (every wave's DMA
    // of kt landed; every wave done reading kt - 1), refill kt - 1's stage with kt + STAGES - 1, compute kt
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) {
        if (s < k_tiles) {
            if (s == 0) issue(IntC<0>{}, 0);
            if (s == 1) issue(IntC<1 % STAGES>{}, 1);
            if (s == 2) issue(IntC<2 % STAGES>{}, 2);
            if (s == 3) issue(IntC<3 % STAGES>{}, 3);
            if (s == 4) issue(IntC<4 % STAGES>{}, 4);
            if (s == 5) issue(IntC<5 % STAGES>{}, 5);
            if (s == 6) issue(IntC<6 % STAGES>{}, 6);
        }
    }
    auto iteration = [&](auto st, int kt) {
        if (kt + STAGES - 2 < k_tiles) {
            wait_vmcnt<(STAGES - 2) * LOADS>();  // steady state: the STAGES - 2 later k-tiles stay in flight
        } else {
            wait_vmcnt_rt((k_tiles - 1 - kt) * LOADS);
        }
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
        constexpr int NEXT = (decltype(st)::value + STAGES - 1) % STAGES;
        if (kt + STAGES - 1 < k_tiles) issue(IntC<NEXT>{}, kt + STAGES - 1);
        compute(st, kt);
    };
    for (int kt = 0; kt < k_tiles; kt += STAGES) {
        iteration(IntC<0>{}, kt);
        if (kt + 1 < k_tiles) iteration(IntC<1>{}, kt + 1);
        if constexpr (STAGES > 2) if (kt + 2 < k_tiles) iteration(IntC<2 % STAGES>{}, kt + 2);
        if constexpr (STAGES > 3) if (kt + 3 < k_tiles) iteration(IntC<3 % STAGES>{}, kt + 3);
        if constexpr (STAGES > 4) if (kt + 4 < k_tiles) iteration(IntC<4 % STAGES>{}, kt + 4);
        if constexpr (STAGES > 5) if (kt + 5 < k_tiles) iteration(IntC<5 % STAGES>{}, kt + 5);
        if constexpr (STAGES > 6) if (kt + 6 < k_tiles) iteration(IntC<6 % STAGES>{}, kt + 6);
    }
    if constexpr (SUMS) return;
    // every wave is done with the ring before its stages are reused as the epilogue's staging areas
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    if constexpr (!PREFETCH_PARAMS) params.load(g, m0, n0, sa, tid);
    params.park(params_lds, tid);
    __syncthreads();  // every copy has landed (vmcnt(0) costs nothing here) and the parameters are visible
    uint8_t* stage = R::base() + wave * epilogue_stage_bytes<WN, WM>();
    if (SPLIT && w.tail >= 0) {
        if (g.defer) {
            // deep split: the piece's pre-epilogue values (FP32, with the biased fold's bias taken off) or INT32 sums go
            // to its planes; gemm_split_finish adds the pieces and runs the epilogue
            defer_store<FN, FM, WN, WM, 32, HILO && !FOLD ? 2 : 1>(g, m0, n0, wn, wm, w.piece, [&](int i, int j, int x, int h) -> uint32_t {
                if constexpr (FOLD) return __builtin_bit_cast(uint32_t, BIAS_FOLD ? accf[i][j][x] - corr[j] : accf[i][j][x]);
                else if constexpr (HILO) return uint32_t(h == 0 ? acc[i][j][x] : acc_lo[i][j][x]);
                else return uint32_t(acc[i][j][x]);
            });
            return;
        }
        // a piece of a split tile: its pre-epilogue values (FP32, with the biased fold's bias taken off) or INT32 sums go
        // to its slot; the last piece to arrive runs the epilogue on the sums of all pieces
        constexpr int NT = FN * FM * 16, NV = NT * (HILO && !FOLD ? 2 : 1);
        // word v: element v % 16 of tile ((v % NT) / 16) / FM, ((v % NT) / 16) % FM; with hi / lo, v >= NT is the lo sum
        const bool last = split_arrive<NV, 64 * WAVES>(g, w, [&](int v) -> uint32_t {
            const int e = v % NT, i = e / 16 / FM, j = e / 16 % FM, x = e % 16;
            if constexpr (FOLD) return __builtin_bit_cast(uint32_t, BIAS_FOLD ? accf[i][j][x] - corr[j] : accf[i][j][x]);
            else if constexpr (HILO) return uint32_t(v < NT ? acc[i][j][x] : acc_lo[i][j][x]);
            else return uint32_t(acc[i][j][x]);
        });
        if (!last) return;
        gemm_epilogue<DT, MODE, WG, SEG, BM, BN, FN, FM, WN, WM>(g, m0, n0, wn, wm, params_lds, stage, [&](int i, int j, int x) {
            const int e = (i * FM + j) * 16 + x;
            if constexpr (FOLD) return __builtin_bit_cast(float, split_sum<NV, 64 * WAVES, true>(g, w, e));
            else if constexpr (HILO)
                return __builtin_fmaf(float(int32_t(split_sum<NV, 64 * WAVES, false>(g, w, NT + e))), 1.0f / 254.0f,
                                      float(int32_t(split_sum<NV, 64 * WAVES, false>(g, w, e))));
            else return float(int32_t(split_sum<NV, 64 * WAVES, false>(g, w, e)));
        });
        return;
    }
    gemm_epilogue<DT, MODE, WG, SEG, BM, BN, FN, FM, WN, WM>(g, m0, n0, wn, wm, params_lds, stage, [&](int i, int j, int x) {
        if constexpr (BIAS_FOLD) return accf[i][j][x] - corr[j];
        else if constexpr (FOLD) return accf[i][j][x];
        else if constexpr (HILO) return __builtin_fmaf(float(acc_lo[i][j][x]), 1.0f / 254.0f, float(acc[i][j][x]));
        else return float(acc[i][j][x]);
    });
}

}  // namespace wq8
