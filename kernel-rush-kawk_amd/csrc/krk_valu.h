// VALU row-streaming kernel for the GEMV regime (M <= 8).
//
// Each wave owns R rows of W and walks them along K in blocks of 512 elements:
// one global load per row and block, 64 lanes x 16 contiguous bytes, so every
// load instruction is a single 1 KB run of one row (the access pattern that
// reaches the HBM ceiling; the MFMA fragment layout cuts rows into 64-byte
// pieces and does not).  Lane l always multiplies W[row][k0 + 8l .. 8l+7] by
// x[m][k0 + 8l .. 8l+7]; products accumulate in fp32 with v_dot2c_f32_bf16
// (exact bf16 products, fp32 sums).  A wave issues the loads of up to D blocks
// of all its rows before it consumes the first, so with a few waves per SIMD
// the whole weight stream of a small projection is in flight at once.
//
// x comes from one of two places:
//   * MX <= 2: straight from global memory (L2-resident after the first
//     workgroup) into registers, issued just before the W loads of the same
//     blocks so it arrives first; no LDS, no barrier;
//   * MX >= 4: once per workgroup into LDS by LDS DMA (global_load_lds),
//     issued before the W loads, so the workgroup barrier that publishes x
//     waits only for x, never for W.
// At the end each wave folds its MX*R per-lane sums across the 64 lanes with
// a fixed butterfly (gfx950 permlane swaps across rows, DPP within a row), so
// the summation order — and the result — depends only on the shape.
//
// Replaces the reference's Gemv (_gemv_kernel, engine/kernels/gemm.py:248-281,
// 10-31 and the gate/up variant 35-73) and the M <= 8 SkinnyMatmul configs
// (gemm.py:364-375); K splits reduce through splitk_finish like the other
// kernels (gemm.py:96-104, 160-170).
#pragma once

#include "krk_epilogue.h"
#include "krk_norm.h"
#include "krk_select.h"
#include "krk_sync.h"

namespace krk {

constexpr int kValuBlock = 512;  // K elements per wave-wide 16-byte load
constexpr int kValuMaxWaves = 8;
constexpr int kValuLdsMinRows = 4;  // x rows from which x is staged in LDS
constexpr int kValuXcdBlocks = 4096;  // grids from which blocks are ordered by XCD (lm_head)

// Dynamic LDS of one workgroup: x rows [0, MX) of one split's K range, whole
// 512-element blocks (none when x stays in registers).
__host__ __device__ constexpr size_t valu_lds_bytes(int MX, int blocks) {
    return MX < kValuLdsMinRows ? 0 : (size_t)MX * blocks * kValuBlock * sizeof(uint16_t);
}
// With the fused RMSNorm prologue: the normalised rows of the whole K
// (nb blocks), then the per-wave partial sums of squares.
__host__ __device__ constexpr size_t valu_norm_lds_bytes(int MX, int nb) {
    return (size_t)MX * nb * kValuBlock * sizeof(uint16_t) + (size_t)MX * kValuMaxWaves * sizeof(float);
}

__device__ __forceinline__ bf16x2 as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2, v); }

// 16-byte loads at a wave-uniform row base plus a 32-bit byte offset (the
// scalar-base addressing form of gfx9 global loads: no 64-bit address math
// per load).
__device__ __forceinline__ u32x4 load_row16_nt(const uint16_t* base, uint32_t byte_off) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + byte_off));
}
__device__ __forceinline__ u32x4 load_row16(const uint16_t* base, uint32_t byte_off) {
    return *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + byte_off);
}

// MX: x rows held (>= M); R: W rows per wave (for SILU R/2 gate rows then the
// matching R/2 up rows); D: 512-element blocks loaded per row before the wave
// consumes them; EXACT: K is whole blocks and every split is whole chunks of D
// blocks, so no load needs clamping and no lane masking.  NORM: x is the
// residual stream and the projection input is rms_norm(x + na.d) with the
// rounding points of krk_norm.h (K unsplit, one 512-k block per wave at
// most): wave w takes block w of every row (x, d and the gain in 2·MX + 1
// registers of 16 bytes, loaded before the first W loads), the row sums of
// squares meet in LDS, and each wave writes its normalised block there while
// the W loads are in flight; workgroup 0 also writes na.xout.
// Grid: x = output blocks, y = K splits; blockDim = 64 x waves; each workgroup
// covers waves * R (SILU: waves * R/2) consecutive output channels.  Split s
// owns K blocks [s*per + min(s, rem), ...) where per = nb / splits and
// rem = nb % splits (nb = ceil(K / 512)), so no division runs on the device.
// SEL: per-workgroup argmax keys for token selection (krk_select.h) instead
// of, or besides, storing y (y may be null); K unsplit.
template <int MX, int R, int D, bool SILU, bool EXACT, bool NORM = false, bool SEL = false>
__global__ __launch_bounds__(64 * kValuMaxWaves) void valu_gemm_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ w, int64_t ldw,
    uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int per, int rem,
    float* __restrict__ part, uint32_t* __restrict__ ctr, NormArgs na, SelectArgs sa) {
    static_assert(!SILU || R % 2 == 0, "SILU pairs gate and up rows");
    static_assert(!(SEL && SILU), "selection reads plain logits");
    constexpr bool XLDS = MX >= kValuLdsMinRows || NORM;
    static_assert(((XLDS ? 0 : MX) + R) * D < 64, "vmcnt counts at most 63 loads");
    constexpr int RO = SILU ? R / 2 : R;  // output channels per wave
    constexpr int V = MX * R;
    constexpr int P = log2_exact<V>();
    extern __shared__ __align__(16) unsigned char xs[];

    const int lane = threadIdx.x & 63;
    // Wave-uniform values live in scalar registers, so every load below is a
    // scalar row base plus this lane's 32-bit offset.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int waves = blockDim.x >> 6;
    const int s = blockIdx.y;
    const int splits = gridDim.y;
    // Grids of thousands of blocks (lm_head) take each XCD's blocks adjacent,
    // so the 16-byte pieces of a y line that neighbouring blocks write merge
    // in one L2 (measured, bit-identical: lm_head M = 1 / 4 1.9 / 2.9 us
    // faster; on the smaller projections' grids within noise or slower).
    const int blk = gridDim.x >= kValuXcdBlocks ? xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
    const int Nout = SILU ? N / 2 : N;
    const int cb = waves * RO;
    const int c0 = blk * cb;

    // This split's K range in whole blocks: [b0, b1), the last possibly ragged.
    const int nb = (K + kValuBlock - 1) / kValuBlock;
    const int b0 = s * per + (s < rem ? s : rem);
    const int b1 = b0 + per + (s < rem ? 1 : 0);
    const uint32_t lane_k = 8u * (uint32_t)lane;

    // Row bases.  Channels past Nout read the last row (discarded at the end);
    // x rows past M read row M - 1 (their sums are never stored).
    const uint16_t* wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int c = c0 + wave * RO + (r % RO);
        c = c < Nout ? c : Nout - 1;
        const int row = (SILU && r >= RO) ? c + Nout : c;
        wrow[r] = w + (int64_t)row * ldw;
    }
    const uint16_t* xrow[MX];
#pragma unroll
    for (int m = 0; m < MX; ++m) xrow[m] = x + (int64_t)(m < M ? m : M - 1) * ldx;

    // Element offset of this lane's 8 elements of block bb.  Generic shapes
    // clamp bb into the split (surplus loads of a short last chunk repeat a
    // block and are not consumed) and send lanes past K to k = 0 (zeroed).
    auto koff = [&](int bb) -> uint32_t {
        if constexpr (EXACT) {
            return (uint32_t)bb * kValuBlock + lane_k;
        } else {
            bb = bb < b1 ? bb : b1 - 1;
            const uint32_t k = (uint32_t)bb * kValuBlock + lane_k;
            return k < (uint32_t)K ? k : 0u;
        }
    };

    u32x4 wv[D][R];
    u32x4 xv[XLDS ? 1 : D][MX];
    auto issue = [&](int b) {
        if constexpr (!XLDS) {
#pragma unroll
            for (int d = 0; d < D; ++d)
#pragma unroll
                for (int m = 0; m < MX; ++m) xv[d][m] = load_row16(xrow[m], 2u * koff(b + d));
        }
#pragma unroll
        for (int d = 0; d < D; ++d)
#pragma unroll
            for (int r = 0; r < R; ++r) wv[d][r] = load_row16_nt(wrow[r], 2u * koff(b + d));
    };

    // After this wave's LDS DMAs: issue the W loads of the first chunk and
    // wait until the DMAs have landed.  vmcnt retires in order, so with the
    // D·R W loads issued strictly after the DMAs, vmcnt <= D·R means every
    // DMA is done while the W loads stay in flight.  That holds when every
    // load stays between the scheduling barriers: in EXACT variants each
    // loaded block is used unconditionally, and the compiler keeps them
    // there (the library's disassembly is checked by a test); in the other
    // variants a load used under a condition can be sunk below the wait
    // (observed), so they drain vmcnt completely.
    auto issue_first_chunk = [&](int b) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        issue(b);
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if constexpr (EXACT) {
            vm_wait<D * R>();
        } else {
            vm_wait<0>();
        }
    };

    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;

    const bool ragged = (K % kValuBlock) != 0;
    // Consume the chunk of D blocks at b: each block as soon as its loads land.
    auto consume = [&](int b) {
        const int n = b1 - b;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (EXACT || d < n) {
                const int bb = b + d;
                // Keep each block's LDS reads of x with that block.
                if constexpr (XLDS) __builtin_amdgcn_sched_barrier(0);
                u32x4 xb[MX];
#pragma unroll
                for (int m = 0; m < MX; ++m) {
                    if constexpr (XLDS) {
                        xb[m] = *reinterpret_cast<const u32x4*>(
                            xs + ((size_t)(m * (b1 - b0) + (bb - b0)) * kValuBlock + lane_k) * 2);
                    } else {
                        xb[m] = xv[d][m];
                    }
                }
                if (!EXACT && ragged && bb == nb - 1 && (uint32_t)bb * kValuBlock + lane_k >= (uint32_t)K) {
#pragma unroll
                    for (int r = 0; r < R; ++r) wv[d][r] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
                    for (int m = 0; m < MX; ++m) xb[m] = u32x4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int m = 0; m < MX; ++m) {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float a = acc[m * R + r];
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wv[d][r][j]), as_bf16x2(xb[m][j]), a, false);
                        acc[m * R + r] = a;
                    }
                }
            }
        }
    };

    // Each chunk's loads are issued and consumed in the same iteration (no
    // registers carried across iterations); the whole K range of a split is
    // usually one chunk.
    int b = b0;
    if constexpr (NORM) {
        // Block bw = wave of every row (lane l: k = 512·bw + 8l); waves past
        // the last block, and k past K, hold zeros.  Rows past M read row
        // M - 1.
        const int bw = wave;
        const uint32_t k = (uint32_t)bw * kValuBlock + lane_k;
        const bool kin = bw < nb && k < (uint32_t)K;
        const uint32_t kc = kin ? k : 0u;
        const u32x4 gv = load_row16(na.wn, 2u * kc);
        u32x4 xr[MX], dr[MX];
#pragma unroll
        for (int m = 0; m < MX; ++m) {
            xr[m] = load_row16(xrow[m], 2u * kc);
            dr[m] = load_row16(na.d + (int64_t)(m < M ? m : M - 1) * na.ldd, 2u * kc);
        }
        issue_first_chunk(b0);
        // s = bf16(x + d) (workgroup 0 writes it to xout) and the wave's
        // partial Σ s² per row, folded in fixed order.
        const bool write_xout = blockIdx.x == 0 && blockIdx.y == 0;
        float ss[MX];
#pragma unroll
        for (int m = 0; m < MX; ++m) {
            ss[m] = 0.0f;
            xr[m] = add_sumsq_bf16x8(kin ? xr[m] : u32x4{0u, 0u, 0u, 0u}, kin ? dr[m] : u32x4{0u, 0u, 0u, 0u}, ss[m]);
            if (write_xout && kin && m < M) *reinterpret_cast<u32x4*>(na.xout + (int64_t)m * na.ldxo + k) = xr[m];
        }
        float* const red = reinterpret_cast<float*>(xs + (size_t)MX * nb * kValuBlock * 2);
        constexpr int PM = log2_exact<MX>();
        wave_fold<MX, 32>(ss, lane);
        {
            const int v = (lane >> (6 - PM)) & (MX - 1);
            if ((lane & ((64 >> PM) - 1)) == 0) red[wave * MX + v] = ss[0];
        }
        lds_wait();
        bare_barrier();
        // Row statistics (waves in order), then block bw of each row.
        if (bw < nb) {
#pragma unroll
            for (int m = 0; m < MX; ++m) {
                float t = red[m];
                for (int wv = 1; wv < waves; ++wv) t += red[wv * MX + m];
                const float rstd = rms_rstd(t, K, na.eps);
                *reinterpret_cast<u32x4*>(xs + ((size_t)(m * nb + bw) * kValuBlock + lane_k) * 2) =
                    normalize_bf16x8(xr[m], rstd, gv);
            }
        }
        lds_wait();
        bare_barrier();  // publishes the normalised rows
        consume(b0);
        b += D;
    } else if constexpr (XLDS) {
        // x[0:MX, b0*512 : b1*512) into LDS as [m][block][512], one 1 KB DMA
        // per (row, block), spread over the waves; the first W loads go out
        // behind them.  The barrier publishes x once the DMAs have landed
        // (issue_first_chunk), and in EXACT variants block 0 is consumed as
        // soon as its own W rows land.
        const int nblk = b1 - b0;
        int m = 0, bi = wave;
        while (bi >= nblk) bi -= nblk, ++m;
        for (int j = wave; j < MX * nblk; j += waves) {
            dma_row(xrow[m] + koff(b0 + bi), xs + (size_t)j * (kValuBlock * 2));
            bi += waves;
            while (bi >= nblk) bi -= nblk, ++m;
        }
        issue_first_chunk(b0);
        bare_barrier();
        consume(b0);
        b += D;
    }
    for (; b < b1; b += D) {
        issue(b);
        consume(b);
    }

    wave_fold<V, 32>(acc, lane);

    // Lane l now holds value v = (l >> (6 - P)) & (V - 1), i.e. (m, r) with
    // v = m * R + r; the first lane of each group of 2^(6-P) writes it.
    constexpr int G = 64 >> P;  // lanes per value
    const int v = (lane >> (6 - P)) & (V - 1);
    const int m = v / R;
    const int r = v - m * R;
    float u = 0.0f;
    if constexpr (SILU) u = __shfl_down(acc[0], RO * G);
    const OutStage<SILU> o{y, ldy, part, M, N, Nout, splits, s};
    const int c = c0 + wave * RO + r;
    if constexpr (SEL) {
        __shared__ uint16_t selv[MX * kValuMaxWaves * R];  // [m][channel of the workgroup]
        if ((lane & (G - 1)) == 0 && r < RO) selv[m * cb + wave * RO + r] = (uint16_t)f32_to_bf16(acc[0]);
        if (y && (lane & (G - 1)) == 0 && m < M && r < RO && c < Nout) o.put(m, c, acc[0], u);
        __syncthreads();
        select_local(sa, selv, cb, cb < Nout - c0 ? cb : Nout - c0, c0, M, blk);
    } else {
        if ((lane & (G - 1)) == 0 && m < M && r < RO && c < Nout) o.put(m, c, acc[0], u);
        if (splits > 1) splitk_finish<SILU, 4, 1>(o, ctr, blk, c0, cb);
    }
}

}  // namespace krk
