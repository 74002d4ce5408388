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
//   * a workgroup of 4 waves owns NR = 16·NT W rows (SILU: NT/2 gate tiles +
//     the matching NT/2 up tiles) and one of `splits` ranges of K stages;
//   * a stage is KC = 512 k for all NR rows: each wave loads NR/4 row chunks of
//     1 KB (non-temporal), the tile goes to LDS (row pitch 1040 B so the 16
//     rows a fragment read touches fall in different banks), and each wave
//     then runs 4 of the stage's 16 k-steps over every n tile and m tile;
//   * the next stage's W loads are in flight while the current stage is
//     computed; x fragments (global, L2-resident) are issued before that
//     prefetch so waiting for them never waits for W;
//   * waves hold partial sums over different k-steps and are reduced in fixed
//     order through LDS; OutStage/splitk_finish finish as in krk_mfma.h.
// Rows past N, rows past M and k past K load clamped in-range addresses and
// are zeroed by masks, so the loop has no data-dependent branches.
#pragma once

#include "krk_epilogue.h"

namespace krk {

constexpr int kLdsKC = 512;      // k per stage (one 1 KB row chunk)
constexpr int kLdsRowPitch = 1040;  // bytes per LDS row slot (1 KB + 16 B pad)
constexpr int kLdsWaves = 4;

template <int MT, int NT, bool SILU>
__global__ void __launch_bounds__(256)
mfma_lds_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                const uint16_t* __restrict__ w, int64_t ldw,
                uint16_t* __restrict__ y, int64_t ldy,
                int M, int N, int K, int splits,
                float* __restrict__ part, uint32_t* __restrict__ ctr) {
    static_assert(MT >= 1 && MT <= 4, "MT covers up to 64 rows");
    static_assert(!SILU || (NT % 2 == 0), "SILU pairs gate and up tiles");
    constexpr int WV = kLdsWaves;
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
    const uint16_t* xrow[MT];
    uint32_t xmask[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int m = 16 * i + r;
        xmask[i] = m < M ? 0xffffffffu : 0u;
        xrow[i] = x + (int64_t)(m < M ? m : M - 1) * ldx + 8 * q;
    }

    // Stage range of this workgroup.
    const int KST = (K + kLdsKC - 1) / kLdsKC;
    const int sb = (int)(((int64_t)s * KST) / splits);
    const int se = (int)(((int64_t)(s + 1) * KST) / splits);

    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 R[RPW];
    u32x4 X[4][MT];

    auto load_w = [&](int st) {
        const int k = st * kLdsKC + 8 * lane;
        const bool ok = k < K;
        const int kk = ok ? st * kLdsKC : -8 * lane;  // clamped: row start
        const uint32_t m = ok ? 0xffffffffu : 0u;
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            u32x4 v = load_stream16(wrow[i] + kk);
            v &= m;
            R[i] = v;
        }
    };
    auto load_x = [&](int st) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int k = st * kLdsKC + 32 * (4 * wave + kk) + 8 * q;
            const bool ok = k < K;
            const int ko = ok ? k - 8 * q : -8 * q;  // offset from xrow (which includes 8q)
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                u32x4 v = load_cached16(xrow[i] + ko);
                v &= (ok ? xmask[i] : 0u);
                X[kk][i] = v;
            }
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < RPW; ++i)
            *reinterpret_cast<u32x4*>(smem + (wave + WV * i) * kLdsRowPitch + 16 * lane) = R[i];
    };
    auto compute = [&]() {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int chunk = 4 * (4 * wave + kk) + q;  // 16-byte chunk within the 1 KB row
            bf16x8 b[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t)
                b[t] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4*>(smem + (16 * t + r) * kLdsRowPitch + 16 * chunk));
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const bf16x8 a = __builtin_bit_cast(bf16x8, X[kk][i]);
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[t], acc[i][t], 0, 0, 0);
            }
        }
    };

    if (sb < se) {
        load_w(sb);
        int st = sb;
        // All stages but the last prefetch the next one unconditionally.
        for (; st + 1 < se; ++st) {
            load_x(st);
            __syncthreads();  // previous stage's fragment reads are done
            stash();
            load_w(st + 1);
            __syncthreads();  // tile complete
            compute();
        }
        load_x(st);
        __syncthreads();
        stash();
        __syncthreads();
        compute();
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

// Dynamic LDS bytes for a configuration: the W tile, which the reduction reuses.
constexpr size_t mfma_lds_bytes(int MT, int NT) {
    const size_t tile = (size_t)16 * NT * kLdsRowPitch;
    const size_t red = (size_t)kLdsWaves * MT * NT * 64 * 16;
    return tile > red ? tile : red;
}

}  // namespace krk
