// MFMA skinny GEMM with W and x both staged through LDS (gfx950).
//
// Same contract as mfma_gemm_kernel (krk_mfma.h); reference counterparts
// engine/kernels/gemm.py:54-93, 116-157 and engine/kernels/gateup64.py:21-56.
//
// Why everything goes through LDS (measured on MI355X):
//   * HBM3E streams at ~6.5-7 TB/s only when each wave-wide load is a long
//     contiguous run.  The MFMA operand layout (lane (r, q) holds row r,
//     k0 + 8q .. +7) makes a direct fragment load touch 16 rows x 64 bytes.
//   * The same holds for x, which every workgroup re-reads from L2: a CU pulls
//     ~75 GB/s of L2 data with whole-row loads but only ~31 GB/s with the
//     fragment pattern, and at M = 32 a 32-row workgroup reads as many x bytes
//     as W bytes.
// So each stage of KC k (512, or 256 for large tiles or many workgroups per
// CU) is read row-contiguously
// — the NR = 16·NT weight rows and the MX = 16·MT x rows alike — into
// registers, PF stages ahead, written to an LDS tile, and the MFMA fragments
// of both operands are read back from LDS.
//
// Work split:
//   * a workgroup of 8 waves owns NR W rows (SILU: NT/2 gate tiles + the
//     matching NT/2 up tiles) and one of `splits` ranges of K stages;
//   * each wave loads (NR + MX) / 8 row pieces per stage (a piece is KC
//     elements: 1 KB = a whole wave load, or 512 B = half a wave load);
//   * tile rows are XOR-swizzled by 16-byte chunk (chunk c of row t sits at
//     c ^ (t % 16)), so fragment reads of 16 rows at one column hit distinct
//     banks without padding;
//   * two LDS tiles: stage i is written to tile i % 2 while other waves may
//     still read tile (i - 1) % 2, so one barrier per stage suffices;
//   * each wave runs KC/256 of the stage's KC/32 k-steps over every n and m
//     tile; waves are reduced in fixed order through LDS at the end, and
//     OutStage/splitk_finish store or combine the results (krk_epilogue.h).
// Rows past N and past M load clamped in-range rows (their outputs are never
// stored); k past K occurs only in the last stage of a K that is not a whole
// number of stages, and is zeroed there in both operands.
#pragma once

#include "krk_epilogue.h"
#include "krk_norm.h"
#include "krk_select.h"

namespace krk {

constexpr int kLdsWaves = 8;
// Stages of 512 k the fused RMSNorm prologue holds in registers: K <= 2560,
// the hidden size every normed projection reads.
constexpr int kLdsNormStages = 5;
// Most 512-k stages of x the XPRE variants hold in registers (o_proj's
// K = 4096 with one or two x tiles); shorter K uses kLdsNormStages.
constexpr int kLdsXpreStages = 8;
// With one x tile and one weight tile, up to down_proj's K = 9728.
constexpr int kLdsXpreLongStages = 19;

// k per stage: 512 fits two tiles of NR + MX rows in LDS up to four 16-row
// tiles (128 KB); 256 halves the footprint (more workgroups per CU when the
// grid is much larger than the chip).
__host__ __device__ constexpr bool mfma_lds_kc_ok(int MT, int NT, int KC) {
    return KC == 256 || (KC == 512 && MT + NT <= 4);
}
// Dynamic LDS bytes: two tiles, which the final reduction reuses (with token
// selection, followed by the bf16 outputs [16·MT][16·NT]).
__host__ __device__ constexpr size_t mfma_lds_bytes(int MT, int NT, int KC, bool sel = false) {
    const size_t tile = (size_t)2 * 16 * (NT + MT) * 2 * KC;
    const size_t red = (size_t)kLdsWaves * MT * NT * 64 * 16 + (sel ? (size_t)16 * MT * 16 * NT * 2 : 0);
    return tile > red ? tile : red;
}

// SEL: per-workgroup argmax keys for token selection (krk_select.h) instead
// of, or besides, storing y (y may be null); K unsplit.
// NORM: x is the residual stream and the projection input is
// rms_norm(x + na.d) with the rounding points of krk_norm.h, K unsplit in
// 512-k stages, at most kLdsNormStages of them.  Wave w owns x rows w, w + 8,
// ... (the rows it stages anyway): before the first stage it loads x, d and
// the gain for every stage of its rows, then the first weight stages, then
// forms s = bf16(x + d), takes each row's Σ s² with a wave butterfly and
// keeps the normalised rows in registers, from which every stage's x rows
// are staged; no x loads remain in the loop.  Workgroup 0 writes s to
// na.xout after the loop.
// XPRE (> 0): the same register-held x rows without the prologue: x for the
// whole K (at most XPRE 512-k stages, K unsplit) is loaded once before the
// first stage, and the stage loop loads weights only.
// cb: output channels per block (a multiple of 8, at most 16·NH).  Below
// 16·NH the last tile is partly padding: its rows past cb are not loaded
// (zeros in the tile) and their outputs not stored.  This lets a shape use
// all 256 CUs with whole K (qkv: 6144 = 256 x 24 channels) instead of
// leaving CUs idle or splitting K.
template <int MT, int NT, int PF, int KC, bool SILU, bool SEL = false, bool NORM = false, int XPRE = 0>
__global__ void __launch_bounds__(64 * kLdsWaves)
mfma_lds_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                const uint16_t* __restrict__ w, int64_t ldw,
                uint16_t* __restrict__ y, int64_t ldy,
                int M, int N, int K, int splits, int cb,
                float* __restrict__ part, uint32_t* __restrict__ ctr, SelectArgs sa, NormArgs na) {
    static_assert(!(SEL && SILU), "selection reads plain logits");
    static_assert(!(NORM || XPRE) || (KC == 512 && !SEL), "x rows held in registers are whole 512-k rows");
    static_assert(!(NORM && XPRE), "the fused prologue already holds x in registers");
    static_assert(XPRE == 0 || XPRE == kLdsNormStages || XPRE == kLdsXpreStages || (XPRE == kLdsXpreLongStages && MT == 1 && NT == 1),
                  "instantiated x-register depths");
    static_assert(MT >= 1 && MT <= 4, "MT covers up to 64 rows");
    static_assert(!SILU || (NT % 2 == 0), "SILU pairs gate and up tiles");
    static_assert(PF >= 2, "at least two stages in flight");
    static_assert(mfma_lds_kc_ok(MT, NT, KC), "k per stage");
    constexpr int WV = kLdsWaves;
    constexpr int PITCH = 2 * KC;             // bytes per tile row
    constexpr int KPW = (KC / 32) / WV;       // k-steps per wave per stage
    constexpr int RPL = 512 / KC;             // rows per wave load
    constexpr int LSH = KC == 512 ? 6 : 5;    // log2(lanes per row piece)
    constexpr int NR = 16 * NT, MX = 16 * MT, TR = NR + MX;
    constexpr int LW = NR / (WV * RPL), LX = MX / (WV * RPL), LPW = LW + LX;
    constexpr int NH = SILU ? NT / 2 : NT;
    static_assert(LW * WV * RPL == NR && LX * WV * RPL == MX, "rows split evenly over the loads");

    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int q = lane >> 4;
    const int lsub = lane & ((1 << LSH) - 1);  // lane within its row piece
    const int lrow = lane >> LSH;              // which row of the load (KC = 256)
    const int blk = blockIdx.x / splits;
    const int s = blockIdx.x - blk * splits;
    const int Nout = SILU ? (N >> 1) : N;
    const int c0 = blk * cb;

    // Row pieces this wave loads: tile rows RPL·(wave + WV·j) + lrow, W rows
    // first, then x rows.
    const uint16_t* rowp[LPW];
    bool rowok[LW];  // the piece is one of the block's cb channels (else padding: zeros, not loaded)
#pragma unroll
    for (int j = 0; j < LW; ++j) {
        const int tr = RPL * (wave + WV * j) + lrow;
        const int t = tr >> 4;
        const int cl = 16 * (t % NH) + (tr & 15);  // channel within the block
        rowok[j] = cl < cb;
        int ch = c0 + cl;
        ch = ch < Nout ? ch : Nout - 1;
        const int row = (SILU && t >= NH) ? ch + Nout : ch;
        rowp[j] = w + (int64_t)row * ldw + 8 * lsub;
    }
#pragma unroll
    for (int j = 0; j < LX; ++j) {
        const int m = RPL * (wave + WV * j) + lrow;
        rowp[LW + j] = x + (int64_t)(m < M ? m : M - 1) * ldx + 8 * lsub;
    }

    const int KST = (K + KC - 1) / KC;
    const int sb = (int)(((int64_t)s * KST) / splits);
    const int se = (int)(((int64_t)(s + 1) * KST) / splits);
    const bool ragged_k = (K % KC) != 0;

    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Stage st into registers.  Prefetches past the range read the start of
    // x row 0 instead (valid, L2-resident, never used).  The padding rows
    // past the block's cb channels are not loaded; the compiler then counts
    // only the unconditional loads in its waits, which wait for the next
    // stage's weight loads too (measured: loading the padding rows from x
    // instead, so that the waits keep a whole stage in flight, made qkv and
    // down at M = 64 3-6% slower).  NORM has its own unconditional loads.
    auto load = [&](u32x4 (&R)[LPW], int st, bool live) {
        const int kk = st * KC + 8 * lsub < K ? st * KC : -8 * lsub;  // past K: the row's start
        const int xo = 8 * lsub < K ? 8 * lsub : K - 8;
#pragma unroll
        for (int j = 0; j < LW; ++j)
            R[j] = rowok[j] ? load_stream16(live ? rowp[j] + kk : x + xo) : u32x4{0u, 0u, 0u, 0u};
        if constexpr (!NORM) {
#pragma unroll
            for (int j = 0; j < LX; ++j) R[LW + j] = load_cached16(live ? rowp[LW + j] + kk : x + xo);
        }
    };
    auto stash = [&](const u32x4 (&R)[LPW], int st, unsigned char* tile) {
        const bool rag = ragged_k && st == KST - 1;
        const uint32_t mk = (st * KC + 8 * lsub < K) ? 0xffffffffu : 0u;
#pragma unroll
        for (int j = 0; j < LPW; ++j) {
            const int tr = j < LW ? RPL * (wave + WV * j) + lrow : NR + RPL * (wave + WV * (j - LW)) + lrow;
            u32x4 v = R[j];
            if (rag) v &= mk;
            *reinterpret_cast<u32x4*>(tile + tr * PITCH + 16 * (lsub ^ (tr & 15))) = v;
        }
    };
    auto compute = [&](const unsigned char* tile) {
#pragma unroll
        for (int kk = 0; kk < KPW; ++kk) {
            // 16-byte chunk of this lane's fragment; every row read here is
            // 16-aligned + r, so its swizzled position is c ^ r.
            const int pos = 16 * ((4 * (KPW * wave + kk) + q) ^ r);
            bf16x8 b[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t)
                b[t] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(tile + (16 * t + r) * PITCH + pos));
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const bf16x8 a =
                    __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(tile + (NR + 16 * i + r) * PITCH + pos));
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[t], acc[i][t], 0, 0, 0);
            }
        }
    };

    if constexpr (NORM || XPRE) {
        // K unsplit (sb = 0) in nst <= XN stages of 512: lane l of wave w
        // holds k = 512·b + 8l of rows w + 8j for every stage b.  Rows past
        // M and k past K are zero.
        constexpr int XN = NORM ? kLdsNormStages : XPRE;
        const int nst = KST;
        u32x4 xr[XN][LX], dr[XN][LX], gv[XN];
        u32x4 sv[XN][LX];
#pragma unroll
        for (int b = 0; b < XN; ++b) {
            const int kb = b * KC + 8 * lsub;
            const int kc = (b < nst && kb < K) ? kb : 0;
            if constexpr (NORM) gv[b] = load_cached16(na.wn + kc);
#pragma unroll
            for (int j = 0; j < LX; ++j) {
                const int m = wave + WV * j;
                const int mm = m < M ? m : M - 1;
                xr[b][j] = load_cached16(x + (int64_t)mm * ldx + kc);
                if constexpr (NORM) dr[b][j] = load_cached16(na.d + (int64_t)mm * na.ldd + kc);
            }
        }
        // Weight rows only (the x rows come from xr), every load unconditional
        // (padding rows and stages past K read the start of x row 0 and are
        // zeroed when staged): a load under a branch would make the waits
        // of this prologue drain the first weight stages.
        auto load_w = [&](u32x4 (&Rw)[LW], int st, bool live) {
            const int kk = st * KC + 8 * lsub < K ? st * KC : -8 * lsub;
            const int xo = 8 * lsub < K ? 8 * lsub : K - 8;
#pragma unroll
            for (int j = 0; j < LW; ++j) Rw[j] = load_stream16(live && rowok[j] ? rowp[j] + kk : x + xo);
        };
        auto stash_norm = [&](const u32x4 (&Rw)[LW], const u32x4 (&Xr)[LX], int st, bool in, unsigned char* tile) {
            const bool rag = ragged_k && st == KST - 1;
            const uint32_t mk = (in && st * KC + 8 * lsub < K) ? 0xffffffffu : 0u;
#pragma unroll
            for (int j = 0; j < LPW; ++j) {
                const int tr = j < LW ? wave + WV * j : NR + wave + WV * (j - LW);
                u32x4 v = j < LW ? Rw[j] : Xr[j - LW];
                if (j < LW && !rowok[j]) v = u32x4{0u, 0u, 0u, 0u};
                if (!in || rag) v &= mk;
                *reinterpret_cast<u32x4*>(tile + tr * PITCH + 16 * (lsub ^ (tr & 15))) = v;
            }
        };
        u32x4 RW[PF][LW];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < PF; ++p) load_w(RW[p], p < nst ? p : 0, p < nst);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NORM) {
            float ss[LX];
#pragma unroll
            for (int j = 0; j < LX; ++j) ss[j] = 0.0f;
#pragma unroll
            for (int b = 0; b < XN; ++b) {
                const int kb = b * KC + 8 * lsub;
#pragma unroll
                for (int j = 0; j < LX; ++j) {
                    const int m = wave + WV * j;
                    const bool live = b < nst && kb < K && m < M;
                    xr[b][j] = add_sumsq_bf16x8(live ? xr[b][j] : u32x4{0u, 0u, 0u, 0u},
                                                live ? dr[b][j] : u32x4{0u, 0u, 0u, 0u}, ss[j]);
                }
            }
            // s is kept for xout, which workgroup 0 writes after the stage loop:
            // a store under a branch before the loop's loads would make the
            // compiler's waits there drain every load in flight.
#pragma unroll
            for (int b = 0; b < XN; ++b)
#pragma unroll
                for (int j = 0; j < LX; ++j) sv[b][j] = xr[b][j];
#pragma unroll
            for (int j = 0; j < LX; ++j) {
                wave_fold<1, 32>(&ss[j], lane);
                const float rstd = rms_rstd(ss[j], K, na.eps);
                const int m = wave + WV * j;
#pragma unroll
                for (int b = 0; b < XN; ++b) {
                    const bool live = b < nst && b * KC + 8 * lsub < K && m < M;
                    xr[b][j] = live ? normalize_bf16x8(xr[b][j], rstd, gv[b]) : u32x4{0u, 0u, 0u, 0u};
                }
            }
        } else {
            // XPRE: rows past M and k past K (whole stages past K, and the
            // ragged tail, masked when staged) are zero.
#pragma unroll
            for (int b = 0; b < XN; ++b)
#pragma unroll
                for (int j = 0; j < LX; ++j) {
                    const bool live = b < nst && wave + WV * j < M;
                    xr[b][j] = live ? xr[b][j] : u32x4{0u, 0u, 0u, 0u};
                }
        }
        // Stage i: the weight rows from R[i % PF], the x rows from xr[i].
        // All XN stages run, with no branch around a load (the compiler's
        // waits then keep PF - 1 stages in flight); stages past K are zero
        // (their weight registers hold placeholder loads).
#pragma unroll
        for (int i = 0; i < XN; ++i) {
            unsigned char* const tile = smem + (i & 1) * (TR * PITCH);
            stash_norm(RW[i % PF], xr[i], i, i < nst, tile);
            __syncthreads();  // tile i complete; every wave is done with tile i - 2
            load_w(RW[i % PF], i + PF < nst ? i + PF : 0, i + PF < nst);
            compute(tile);
        }
        if (NORM && blockIdx.x == 0) {
#pragma unroll
            for (int b = 0; b < XN; ++b) {
                const int kb = b * KC + 8 * lsub;
#pragma unroll
                for (int j = 0; j < LX; ++j) {
                    const int m = wave + WV * j;
                    if (b < nst && kb < K && m < M) *reinterpret_cast<u32x4*>(na.xout + (int64_t)m * na.ldxo + kb) = sv[b][j];
                }
            }
        }
    } else if (sb < se) {
        const int nst = se - sb;
        u32x4 R[PF][LPW];
#pragma unroll
        for (int p = 0; p < PF; ++p) load(R[p], p < nst ? sb + p : sb, p < nst);
        // Step i stashes stage i (its registers then take stage i + PF), and
        // computes it after the barrier.  Unrolled by PF so the register
        // buffers rotate without copies (a copy would be an early use of the
        // newest loads, and vmcnt retires in order).
        auto step = [&](int i, u32x4 (&Rc)[LPW]) {
            const int st = sb + i;
            unsigned char* const tile = smem + (i & 1) * (TR * PITCH);
            stash(Rc, st, tile);
            __syncthreads();  // tile i complete; every wave is done with tile i - 2
            load(Rc, i + PF < nst ? st + PF : sb, i + PF < nst);
            compute(tile);
        };
        int i = 0;
        for (; i + PF <= nst; i += PF) {
#pragma unroll
            for (int p = 0; p < PF; ++p) step(i + p, R[p]);
        }
#pragma unroll
        for (int p = 0; p < PF - 1; ++p)
            if (i + p < nst) step(i + p, R[p]);
    }

    // Cross-wave reduction in fixed wave order (reuses the tile area).
    f32x4* red = reinterpret_cast<f32x4*>(smem);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) red[((wave * MT + i) * NT + t) * 64 + lane] = acc[i][t];
    __syncthreads();

    OutStage<SILU> o{y, ldy, part, M, N, Nout, splits, s};
    uint16_t* const selv = reinterpret_cast<uint16_t*>(smem + (size_t)WV * MT * NT * 64 * 16);  // [16·MT][16·NT]
    const int items = MT * NH * 64;
    for (int v = threadIdx.x; v < items; v += blockDim.x) {
        const int ln = v & 63;
        const int tl = (v >> 6) % NH;
        const int i = (v >> 6) / NH;
        f32x4 gsum = red[(i * NT + tl) * 64 + ln];
        f32x4 usum = SILU ? red[(i * NT + tl + NH) * 64 + ln] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int wv = 1; wv < WV; ++wv) {
            gsum += red[((wv * MT + i) * NT + tl) * 64 + ln];
            if (SILU) usum += red[((wv * MT + i) * NT + tl + NH) * 64 + ln];
        }
        const int cl = 16 * tl + (ln & 15);
        const int c = c0 + cl;
        const bool cok = cl < cb && c < Nout;
        const int mb = 16 * i + 4 * (ln >> 4);
        if constexpr (SEL) {
#pragma unroll
            for (int e = 0; e < 4; ++e) selv[(mb + e) * (16 * NT) + 16 * tl + (ln & 15)] = (uint16_t)f32_to_bf16(gsum[e]);
            if (y && cok) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (mb + e < M) o.put(mb + e, c, gsum[e], usum[e]);
            }
        } else if (cok) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (mb + e < M) o.put(mb + e, c, gsum[e], usum[e]);
        }
    }
    if constexpr (SEL) {
        __syncthreads();
        const int n = cb < Nout - c0 ? cb : Nout - c0;
        select_local(sa, selv, 16 * NT, n, c0, M, blockIdx.x);
    } else if (splits > 1) {
        splitk_finish<SILU>(o, ctr, blk, c0, cb);
    }
}

}  // namespace krk
