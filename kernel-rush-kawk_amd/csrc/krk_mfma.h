// MFMA skinny GEMM for gfx950: y = x[M,K] · W[N,K]ᵀ with M <= 64 per launch.
//
// Reference counterpart: _skinny_kernel / _gateup_kernel
// (engine/kernels/gemm.py:54-93, 116-157) and the M=64 gate/up kernels
// (engine/kernels/gateup64.py:21-56, gateup_n32.py:14-46).  Those tile A
// into a zero-padded 16/32-row block and use tensor-core dots; this kernel
// is organised around the HBM weight stream of an MI355X instead.
//
// Instruction: v_mfma_f32_16x16x32_bf16.  Per lane (l = 0..63, r = l % 16,
// q = l / 16) the A operand holds x[m0 + r][k0 + 8q .. k0 + 8q + 7] and the
// B operand holds W[n0 + r][k0 + 8q .. +7]: one 16-byte load each, and one
// wave-wide W load covers 16 rows x 64 contiguous bytes.  The accumulator
// returns D[m0 + 4q + e][n0 + r] in element e.
//
// Work split:
//   * a workgroup owns a block of NT W tiles (16 rows each; with SILU_MUL the
//     first NT/2 tiles are gate rows and the last NT/2 the matching up rows,
//     so the epilogue pairs stay in registers) and one of `splits` K ranges;
//   * its waves divide that K range again (32-wide k-steps) and stream their
//     W slice with non-temporal 16-byte loads, U k-steps per pipeline stage,
//     double-buffered in registers so a stage is in flight while the
//     previous one feeds the MFMAs;
//   * x fragments come straight from global memory: x is at most 64 x K bf16
//     and stays resident in L2 while W streams past it;
//   * waves are reduced in a fixed order through LDS, then OutStage stores y
//     (splits == 1) or the fp32 partials that splitk_finish reduces.
#pragma once

#include "krk_epilogue.h"

namespace krk {

template <int MT, int NT, int U, bool SILU>
__global__ void __launch_bounds__(256)
mfma_gemm_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                 const uint16_t* __restrict__ w, int64_t ldw,
                 uint16_t* __restrict__ y, int64_t ldy,
                 int M, int N, int K, int splits,
                 float* __restrict__ part, uint32_t* __restrict__ ctr) {
    static_assert(MT >= 1 && MT <= 4, "MT covers up to 64 rows");
    static_assert(!SILU || (NT % 2 == 0), "SILU pairs gate and up tiles");
    constexpr int NH = SILU ? NT / 2 : NT;  // output-channel tiles per block

    extern __shared__ f32x4 red[];  // [waves][MT][NT][64 lanes]

    const int waves = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int q = lane >> 4;
    const int blk = blockIdx.x / splits;
    const int s = blockIdx.x - blk * splits;
    const int Nout = SILU ? (N >> 1) : N;
    const int c0 = blk * (16 * NH);

    // Row pointers.  Rows past the end are clamped to a valid row; their
    // results are never stored.
    const uint16_t* wp[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        int ch = c0 + 16 * (t % NH) + r;
        ch = ch < Nout ? ch : Nout - 1;
        const int row = (SILU && t >= NH) ? ch + Nout : ch;
        wp[t] = w + (int64_t)row * ldw + 8 * q;
    }
    const uint16_t* xp[MT];
    bool xv[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int m = 16 * i + r;
        xv[i] = m < M;
        xp[i] = x + (int64_t)(xv[i] ? m : 0) * ldx + 8 * q;
    }

    // This wave's k-steps [kb, ke) (32 elements each).
    const int KS = (K + 31) >> 5;
    const int P = splits * waves;
    const int j = s * waves + wave;
    const int kb = (int)(((int64_t)j * KS) / P);
    const int ke = (int)(((int64_t)(j + 1) * KS) / P);
    const bool kfull = (K & 31) == 0;

    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    bf16x8 wa[U][NT], xa[U][MT];
    bf16x8 wb[U][NT], xb[U][MT];

    // Load the U k-steps starting at g into (wr, xr).  Steps at or past ke and
    // k positions at or past K load zeros.
    auto load_stage = [&](int g, bf16x8 (&wr)[U][NT], bf16x8 (&xr)[U][MT]) {
        if (g + U <= ke && kfull) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int koff = (g + u) << 5;
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    wr[u][t] = __builtin_bit_cast(bf16x8, load_stream16(wp[t] + koff));
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    u32x4 v = {0u, 0u, 0u, 0u};
                    if (xv[i]) v = load_cached16(xp[i] + koff);
                    xr[u][i] = __builtin_bit_cast(bf16x8, v);
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int koff = (g + u) << 5;
                const bool ok = (g + u) < ke && (koff + 8 * q) < K;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    u32x4 v = {0u, 0u, 0u, 0u};
                    if (ok) v = load_stream16(wp[t] + koff);
                    wr[u][t] = __builtin_bit_cast(bf16x8, v);
                }
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    u32x4 v = {0u, 0u, 0u, 0u};
                    if (ok && xv[i]) v = load_cached16(xp[i] + koff);
                    xr[u][i] = __builtin_bit_cast(bf16x8, v);
                }
            }
        }
    };

    auto mma_stage = [&](const bf16x8 (&wr)[U][NT], const bf16x8 (&xr)[U][MT]) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xr[u][i], wr[u][t],
                                                                         acc[i][t], 0, 0, 0);
    };

    // Two-stage register pipeline, unrolled by two so the buffers swap roles
    // without register copies.
    int g = kb;
    if (g < ke) load_stage(g, wa, xa);
    while (g < ke) {
        if (g + U < ke) load_stage(g + U, wb, xb);
        mma_stage(wa, xa);
        g += U;
        if (g >= ke) break;
        if (g + U < ke) load_stage(g + U, wa, xa);
        mma_stage(wb, xb);
        g += U;
    }

    // Cross-wave reduction in fixed wave order.
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
        for (int wv = 1; wv < waves; ++wv) {
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

}  // namespace krk
