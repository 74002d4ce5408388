// MFMA skinny GEMM with the weight stream staged through LDS (gfx950).
//
// Same contract as mfma_gemm_kernel (krk_mfma.h); reference counterparts
// engine/kernels/gemm.py:54-93, 116-157 and engine/kernels/gateup64.py:21-56.
//
// Why LDS: HBM3E delivers ~6.5 TB/s only when each wave-wide load covers a
// long contiguous run.  The MFMA B-operand layout (lane (r, q) holds
// W[n0 + r][k0 + 8q .. +7]) makes every direct load touch 16 rows x 64 bytes,
// i.e. 16 concurrent DRAM streams per wave; measured on MI355X that pattern
// tops out near 3-5 TB/s, while whole-row streaming (lane l reads bytes
// [16 l, 16 l + 16) of a 1 KB row chunk) reaches 6.3-6.9 TB/s.  So W is read
// row-contiguously into registers, written to a padded LDS tile, and the MFMA
// fragments are read back from LDS.
//
// Work split:
//   * a workgroup of 8 waves (two per SIMD, so one wave's stalls are covered
//     by the other's work) owns NR = 16·NT W rows (SILU: NT/2 gate tiles +
//     the matching NT/2 up tiles) and one of `splits` ranges of K stages;
//   * a stage is KC = 512 k for all NR rows: each wave loads NR/8 row chunks of
//     1 KB (non-temporal), the tile goes to LDS (row pitch 1040 B so the 16
//     rows a fragment read touches fall in different banks), and each wave
//     then runs 2 of the stage's 16 k-steps over every n tile and m tile;
//   * two stages of W are in flight in registers while a stage is computed,
//     and x fragments (global, L2-resident) are fetched a stage ahead;
//   * waves hold partial sums over different k-steps and are reduced in fixed
//     order through LDS; OutStage/splitk_finish finish as in krk_mfma.h.
// Rows past N, rows past M and k past K load clamped in-range addresses and
// are zeroed by masks, so the loop has no data-dependent branches.
#pragma once

#include "krk_epilogue.h"

namespace krk {

constexpr int kLdsKC = 512;         // k per stage (one 1 KB row chunk)
constexpr int kLdsRowPitch = 1040;  // bytes per LDS row slot (1 KB + 16 B pad)
constexpr int kLdsWaves = 8;
constexpr int kLdsKPW = (kLdsKC / 32) / kLdsWaves;  // k-steps per wave per stage (2)

template <int MT, int NT, bool SILU>
__global__ void __launch_bounds__(64 * kLdsWaves)
mfma_lds_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                const uint16_t* __restrict__ w, int64_t ldw,
                uint16_t* __restrict__ y, int64_t ldy,
                int M, int N, int K, int splits,
                float* __restrict__ part, uint32_t* __restrict__ ctr) {
    static_assert(MT >= 1 && MT <= 4, "MT covers up to 64 rows");
    static_assert(!SILU || (NT % 2 == 0), "SILU pairs gate and up tiles");
    constexpr int WV = kLdsWaves;
    constexpr int KPW = kLdsKPW;
    constexpr int NR = 16 * NT;
    constexpr int RPW = NR / WV;  // row chunks each wave loads per stage
    static_assert(NR % WV == 0, "rows split evenly over the waves");
    constexpr int NH = SILU ? NT / 2 : NT;

    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int q = lane >> 4;
    const int blk = blockIdx.x / splits;
    const int s = blockIdx.x - blk * splits;
    const int Nout = SILU ? (N >> 1) : N;
    const int c0 = blk * (16 * NH);

    // Row chunks this wave streams: tile rows wave + WV·i.
    const uint16_t* wrow[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int tr = wave + WV * i;  // tile row 0..NR-1
        const int t = tr >> 4;
        int ch = c0 + 16 * (t % NH) + (tr & 15);
        ch = ch < Nout ? ch : Nout - 1;
        const int row = (SILU && t >= NH) ? ch + Nout : ch;
        wrow[i] = w + (int64_t)row * ldw + 8 * lane;
    }
    // x rows past M read row M - 1: output row m depends only on x row m, so
    // those rows only feed outputs that are never stored.
    const uint16_t* xrow[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int m = 16 * i + r;
        xrow[i] = x + (int64_t)(m < M ? m : M - 1) * ldx + 8 * q;
    }

    // Stage range of this workgroup.
    const int KST = (K + kLdsKC - 1) / kLdsKC;
    const int sb = (int)(((int64_t)s * KST) / splits);
    const int se = (int)(((int64_t)(s + 1) * KST) / splits);
    // Only the last stage of a K that is not a multiple of 512 has lanes past
    // K; there both W and x are zeroed (either one alone could still form
    // 0 * inf).  Every other stage uses the loaded values unmodified, so no
    // early use of a load makes the compiler wait for it.
    const bool ragged_k = (K % kLdsKC) != 0;

    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // W row chunks of stage st into registers.  Prefetches past the range
    // read the start of x row 0 instead (valid, L2-resident, never used), so
    // every step issues the same loads and the compiler's waits stay exact.
    auto load_w = [&](u32x4 (&Rb)[RPW], int st, bool live) {
        const int k = st * kLdsKC + 8 * lane;
        const int kk = k < K ? st * kLdsKC : -8 * lane;  // past K: row start
        const int xo = 8 * lane < K ? 8 * lane : K - 8;
#pragma unroll
        for (int i = 0; i < RPW; ++i) Rb[i] = load_stream16(live ? wrow[i] + kk : x + xo);
    };
    // x fragments of this wave's KPW k-steps of stage st.
    auto load_x = [&](u32x4 (&X)[KPW][MT], int st) {
#pragma unroll
        for (int kk = 0; kk < KPW; ++kk) {
            const int k = st * kLdsKC + 32 * (KPW * wave + kk) + 8 * q;
            const int ko = k < K ? k - 8 * q : -8 * q;  // offset from xrow (which includes 8q)
#pragma unroll
            for (int i = 0; i < MT; ++i) X[kk][i] = load_cached16(xrow[i] + ko);
        }
    };
    auto stash = [&](const u32x4 (&Rb)[RPW], int st, unsigned char* tile) {
        const bool rag = ragged_k && st == KST - 1;
        const uint32_t m = (st * kLdsKC + 8 * lane < K) ? 0xffffffffu : 0u;
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            u32x4 v = Rb[i];
            if (rag) v &= m;
            *reinterpret_cast<u32x4*>(tile + (wave + WV * i) * kLdsRowPitch + 16 * lane) = v;
        }
    };
    auto compute = [&](const u32x4 (&X)[KPW][MT], const unsigned char* tile, int st) {
        const bool rag = ragged_k && st == KST - 1;
#pragma unroll
        for (int kk = 0; kk < KPW; ++kk) {
            const int chunk = 4 * (KPW * wave + kk) + q;  // 16-byte chunk within the 1 KB row
            bf16x8 b[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t)
                b[t] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4*>(tile + (16 * t + r) * kLdsRowPitch + 16 * chunk));
            const uint32_t xm = (st * kLdsKC + 8 * chunk < K) ? 0xffffffffu : 0u;
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                u32x4 xv = X[kk][i];
                if (rag) xv &= xm;
                const bf16x8 a = __builtin_bit_cast(bf16x8, xv);
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[t], acc[i][t], 0, 0, 0);
            }
        }
    };

    if (sb < se) {
        // Two stages of W in flight in registers (ra, rb) and two LDS tiles:
        // stage i is stashed into tile i % 2 while the other tile may still be
        // read by stage i - 1's fragments, so one barrier per stage suffices.
        // x is double-buffered and fetched one stage ahead, before the W
        // prefetch: vmcnt retires loads in order, so waiting for this stage's
        // x never waits for the W stages behind it.  The loop is unrolled by
        // two so the buffers swap roles without register copies (a copy would
        // be a use of the newest loads).
        const int nst = se - sb;
        u32x4 ra[RPW], rb[RPW];
        u32x4 xa[KPW][MT], xb[KPW][MT];
        unsigned char* const tile0 = smem;
        unsigned char* const tile1 = smem + NR * kLdsRowPitch;
        load_w(ra, sb, true);
        load_w(rb, nst > 1 ? sb + 1 : sb, nst > 1);
        load_x(xa, sb);
        auto step = [&](int i, u32x4 (&rc)[RPW], u32x4 (&xc)[KPW][MT], u32x4 (&xn)[KPW][MT], unsigned char* tile) {
            const int st = sb + i;
            stash(rc, st, tile);
            load_x(xn, i + 1 < nst ? st + 1 : sb);
            load_w(rc, i + 2 < nst ? st + 2 : sb, i + 2 < nst);
            __syncthreads();  // tile i complete; every wave is done with tile i - 2
            compute(xc, tile, st);
        };
        int i = 0;
        for (; i + 1 < nst; i += 2) {
            step(i, ra, xa, xb, tile0);
            step(i + 1, rb, xb, xa, tile1);
        }
        if (i < nst) step(i, ra, xa, xb, tile0);
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
        const int c = c0 + 16 * tl + (ln & 15);
        const int mb = 16 * i + 4 * (ln >> 4);
        if (c < Nout) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (mb + e < M) o.put(mb + e, c, gsum[e], usum[e]);
        }
    }
    if (splits > 1) splitk_finish<SILU>(o, ctr, blk, c0, 16 * NH);
}

// Dynamic LDS bytes for a configuration: two W tiles, which the reduction
// reuses.
constexpr size_t mfma_lds_bytes(int MT, int NT) {
    const size_t tile = (size_t)2 * 16 * NT * kLdsRowPitch;
    const size_t red = (size_t)kLdsWaves * MT * NT * 64 * 16;
    return tile > red ? tile : red;
}

}  // namespace krk
