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
//     double-buffered in registers so one stage is in flight while the
//     previous one feeds the MFMAs;
//   * x fragments come straight from global memory: x is at most 64 x K bf16
//     and stays resident in L1/L2 while W streams past it;
//   * waves are reduced in a fixed order through LDS, then OutStage stores y
//     (splits == 1) or the fp32 partials that splitk_finish reduces.
//
// The main loop is branch-free: rows past M (x) or N (W) load a clamped, valid
// row and are zeroed by a select or never stored, and the prefetch of the
// next stage is unconditional (the last stage is peeled), so the compiler can
// wait for exactly one stage's loads at a time.  K tails (K % 32 != 0) go
// through a separate masked single-step path.
#pragma once

#include "krk_epilogue.h"

namespace krk {

template <int MT, int NT>
struct MfmaFrag {
    const uint16_t* wp[NT];
    const uint16_t* xp[MT];
    uint32_t xmask[MT];  // all-ones for rows < M, zero for padding rows

    __device__ __forceinline__ void load_step(int koff, bf16x8 (&wr)[NT], bf16x8 (&xr)[MT]) const {
#pragma unroll
        for (int t = 0; t < NT; ++t) wr[t] = __builtin_bit_cast(bf16x8, load_stream16(wp[t] + koff));
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            u32x4 v = load_cached16(xp[i] + koff);
            v &= xmask[i];
            xr[i] = __builtin_bit_cast(bf16x8, v);
        }
    }

    // One k-step at koff whose 8-element groups may run past K: groups at or
    // past K load a valid in-range address and are zeroed.
    __device__ __forceinline__ void load_step_tail(int koff, int q, int K, bf16x8 (&wr)[NT],
                                                   bf16x8 (&xr)[MT]) const {
        const bool ok = koff + 8 * q < K;
        const int kk = ok ? koff : K - 8 - 8 * q;  // stays inside the row
        const uint32_t m = ok ? 0xffffffffu : 0u;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            u32x4 v = load_stream16(wp[t] + kk);
            v &= m;
            wr[t] = __builtin_bit_cast(bf16x8, v);
        }
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            u32x4 v = load_cached16(xp[i] + kk);
            v &= (xmask[i] & m);
            xr[i] = __builtin_bit_cast(bf16x8, v);
        }
    }
};

template <int MT, int NT>
__device__ __forceinline__ void mma_step(f32x4 (&acc)[MT][NT], const bf16x8 (&wr)[NT], const bf16x8 (&xr)[MT]) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t)
            acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xr[i], wr[t], acc[i][t], 0, 0, 0);
}

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

    MfmaFrag<MT, NT> f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        int ch = c0 + 16 * (t % NH) + r;
        ch = ch < Nout ? ch : Nout - 1;
        const int row = (SILU && t >= NH) ? ch + Nout : ch;
        f.wp[t] = w + (int64_t)row * ldw + 8 * q;
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int m = 16 * i + r;
        f.xmask[i] = m < M ? 0xffffffffu : 0u;
        f.xp[i] = x + (int64_t)(m < M ? m : M - 1) * ldx + 8 * q;
    }

    // This wave's k-steps [kb, ke) (32 elements each).
    const int KS = (K + 31) >> 5;
    const int P = splits * waves;
    const int j = s * waves + wave;
    const int kb = (int)(((int64_t)j * KS) / P);
    int ke = (int)(((int64_t)(j + 1) * KS) / P);
    const bool tail = (K & 31) && ke == KS;  // this wave owns the ragged last step
    if (tail) --ke;

    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    bf16x8 wa[U][NT], xa[U][MT];
    bf16x8 wb[U][NT], xb[U][MT];
    auto load_stage = [&](int g, bf16x8 (&wr)[U][NT], bf16x8 (&xr)[U][MT]) {
#pragma unroll
        for (int u = 0; u < U; ++u) f.load_step((g + u) << 5, wr[u], xr[u]);
    };
    auto mma_stage = [&](const bf16x8 (&wr)[U][NT], const bf16x8 (&xr)[U][MT]) {
#pragma unroll
        for (int u = 0; u < U; ++u) mma_step<MT, NT>(acc, wr[u], xr[u]);
    };

    // Full stages, double-buffered; the last stage is peeled so every
    // in-loop prefetch is unconditional.
    const int nst = (ke - kb) / U;
    int g = kb;
    if (nst > 0) {
        load_stage(g, wa, xa);
        int left = nst - 1;  // stages still to load
        while (left >= 2) {
            load_stage(g + U, wb, xb);
            mma_stage(wa, xa);
            load_stage(g + 2 * U, wa, xa);
            mma_stage(wb, xb);
            g += 2 * U;
            left -= 2;
        }
        if (left == 1) {
            load_stage(g + U, wb, xb);
            mma_stage(wa, xa);
            mma_stage(wb, xb);
            g += 2 * U;
        } else {
            mma_stage(wa, xa);
            g += U;
        }
    }
    // Remaining whole steps, one at a time.
    for (; g < ke; ++g) {
        f.load_step(g << 5, wa[0], xa[0]);
        mma_step<MT, NT>(acc, wa[0], xa[0]);
    }
    if (tail) {
        f.load_step_tail(ke << 5, q, K, wa[0], xa[0]);
        mma_step<MT, NT>(acc, wa[0], xa[0]);
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
