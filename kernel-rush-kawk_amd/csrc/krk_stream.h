// Persistent MFMA skinny GEMM: W streamed through an LDS DMA ring, x held in
// registers (gfx950).  y = epilogue(x[M,K] · W[N,K]ᵀ), M <= 64 per launch.
//
// Reference counterparts: _skinny_kernel / _gateup_kernel / _gemv_kernel
// (engine/kernels/gemm.py:54-93, 116-157, 200-245) and the M=64 gate/up
// kernels (engine/kernels/gateup64.py:21-56, gateup_n32.py:14-46).  Like
// gateup64's interleaved weight rows (gateup64.py:31-33), a gate/up block here
// pairs 8 gate rows with the matching 8 up rows inside one 16-row tile.
//
// Design (each point measured on MI355X):
//   * HBM3E streams at ~6.5 TB/s only when each wave-wide load is a long
//     contiguous run: every W load is a 1 KB row chunk (64 lanes x 16 B),
//     DMA'd straight into LDS (global_load_lds_dwordx4).  MFMA B fragments
//     are then read from LDS.
//   * A CU needs ~100 KB in flight: the ring holds `depth` stages of
//     16 rows x 512 k, depth-1 of them in flight while one is consumed, and
//     it keeps streaming across block boundaries.
//   * Workgroups are persistent (at most one per CU): workgroup g walks blocks
//     g, g + G, ...  x is loaded once per workgroup into VGPRs — wave w keeps
//     the fragments of its fixed share of k-steps (2 of every stage's 16) for
//     every stage of the workgroup's K range — so x costs one L2 read per CU
//     instead of one per block, and no load in the loop competes with the
//     ring in the in-order vmcnt counter.
//   * Waits are explicit (vmcnt = DMAs issued after the consumed stage) and
//     barriers carry no memory fence, so the compiler never drains the ring.
//
// Block = one 16-row MFMA tile (v_mfma_f32_16x16x32_bf16, A = x fragment,
// B = W fragment): 16 output channels, or with SILU_MUL 8 channels whose
// gate rows sit in tile rows 0-7 and up rows in tile rows 8-15.  Waves hold
// partial sums over different k-steps; at the end of a block they are
// reduced through LDS in fixed wave order.
#pragma once

#include "krk_epilogue.h"
#include "krk_sync.h"

namespace krk {

constexpr int kStreamWaves = 8;
constexpr int kStreamKC = 512;       // k per stage
constexpr int kStreamPitch = 1040;   // bytes per LDS row (1 KB + 16 B: fragment reads hit distinct banks)
constexpr int kStreamSlot = 16 * kStreamPitch;
constexpr int kStreamKPW = (kStreamKC / 32) / kStreamWaves;  // k-steps per wave per stage (2)
constexpr int kStreamLPW = 16 / kStreamWaves;                // DMAs per wave per stage (2)
constexpr int kStreamMaxDepth = 8;

// Bytes of dynamic LDS: reduction area [WV][MT][64] f32x4, then the ring.
__host__ __device__ constexpr size_t stream_red_bytes(int MT) { return (size_t)kStreamWaves * MT * 64 * 16; }
__host__ __device__ constexpr size_t stream_lds_bytes(int MT, int depth) {
    return stream_red_bytes(MT) + (size_t)depth * kStreamSlot;
}

// MT: 16-row m tiles (M <= 16·MT).  XS: most K stages a workgroup owns (its
// x fragments live in X[XS][2][MT]).  SILU: gate/up blocks with the epilogue.
template <int MT, int XS, bool SILU>
__global__ void __launch_bounds__(512)
stream_gemm_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                   const uint16_t* __restrict__ w, int64_t ldw,
                   uint16_t* __restrict__ y, int64_t ldy,
                   int M, int N, int K, int splits, int depth,
                   float* __restrict__ part, uint32_t* __restrict__ ctr) {
    static_assert(MT >= 1 && MT <= 4, "MT covers up to 64 rows");
    constexpr int WV = kStreamWaves;
    constexpr int KPW = kStreamKPW;
    constexpr int LPW = kStreamLPW;
    constexpr int CB = SILU ? 8 : 16;  // output channels per block

    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    f32x4* const red = reinterpret_cast<f32x4*>(smem);
    unsigned char* const ring = smem + stream_red_bytes(MT);

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int q = lane >> 4;

    // This workgroup's split and blocks: blocks gi, gi + Gs, ... of split s.
    const int s = blockIdx.x % splits;
    const int gi = blockIdx.x / splits;
    const int Gs = gridDim.x / splits;
    const int Nout = SILU ? (N >> 1) : N;
    const int nblocks = (Nout + CB - 1) / CB;
    const int KST = (K + kStreamKC - 1) / kStreamKC;
    const int sb = (int)(((int64_t)s * KST) / splits);
    const int se = (int)(((int64_t)(s + 1) * KST) / splits);
    const int nst = se - sb;
    const int myblocks = gi < nblocks ? (nblocks - 1 - gi) / Gs + 1 : 0;
    const int T = myblocks * nst;  // stages this workgroup consumes

    // DMA of the workgroup's t-th stage into ring slot t % depth.
    const int klane = 8 * lane;
    auto issue = [&](int t) {
        const int bi = t / nst;
        const int st = sb + (t - bi * nst);
        const int b = gi + bi * Gs;
        unsigned char* slot = ring + (size_t)(t % depth) * kStreamSlot;
        const int k = st * kStreamKC + klane;
        const int kc = k < K ? k : 0;  // past K: any in-range address, masked at use
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int row = wave + WV * i;  // tile row 0..15
            int wr;
            if (SILU) {
                int ch = b * CB + (row & 7);
                ch = ch < Nout ? ch : Nout - 1;
                wr = row < 8 ? ch : ch + Nout;
            } else {
                const int ch = b * CB + row;
                wr = ch < Nout ? ch : Nout - 1;
            }
            dma_row(w + (int64_t)wr * ldw + kc, slot + row * kStreamPitch);
        }
    };
    for (int d = 0; d < depth - 1 && d < T; ++d) issue(d);

    // x fragments of this wave's k-steps, rows past M and k past K zeroed.
    u32x4 X[XS][KPW][MT];
#pragma unroll
    for (int j = 0; j < XS; ++j) {
#pragma unroll
        for (int kk = 0; kk < KPW; ++kk) {
            const int k = (sb + j) * kStreamKC + 32 * (wave * KPW + kk) + 8 * q;
            const bool kok = j < nst && k < K;
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const int m = 16 * i + r;
                const bool ok = kok && m < M;
                u32x4 v = load_cached16(x + (int64_t)(m < M ? m : M - 1) * ldx + (kok ? k : 0));
                v &= ok ? 0xffffffffu : 0u;
                X[j][kk][i] = v;
            }
        }
    }

    // Everything issued so far — the ring prologue, then x — must land before
    // the first stage: x is read-only from here on and the compiler then
    // knows it is complete (it would otherwise wait for it behind the ring on
    // every use).  The x transfer overlaps the prologue's HBM latency.
    vm_wait<0>();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);


    OutStage<SILU> o{y, ldy, part, M, N, Nout, splits, s};
    int t = 0;
    for (int bi = 0; bi < myblocks; ++bi) {
        const int b = gi + bi * Gs;
        f32x4 acc[MT];
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
        for (int j = 0; j < XS; ++j) {
            if (j < nst) {
                vm_wait_stages<LPW>(min(depth - 2, T - 1 - t));
                bare_barrier();  // stage t landed for every wave; the slot of t-1 is free
                if (t + depth - 1 < T) issue(t + depth - 1);
                const unsigned char* slot = ring + (size_t)(t % depth) * kStreamSlot;
                const bool ktail = (sb + j + 1) * kStreamKC > K;
#pragma unroll
                for (int kk = 0; kk < KPW; ++kk) {
                    const int chunk = 4 * (wave * KPW + kk) + q;  // 16-byte chunk of the 1 KB row
                    u32x4 v = *reinterpret_cast<const u32x4*>(slot + r * kStreamPitch + 16 * chunk);
                    if (ktail) v &= ((sb + j) * kStreamKC + 8 * chunk < K) ? 0xffffffffu : 0u;
                    const bf16x8 bw = __builtin_bit_cast(bf16x8, v);
#pragma unroll
                    for (int i = 0; i < MT; ++i)
                        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, X[j][kk][i]), bw, acc[i], 0, 0, 0);
                }
                ++t;
            }
        }

        // Block epilogue: every wave parks its partial sums, one barrier, then
        // thread v sums lane-slot v over the waves in fixed order.  The area
        // is rewritten only after the next block's stage barriers.
#pragma unroll
        for (int i = 0; i < MT; ++i) red[(wave * MT + i) * 64 + lane] = acc[i];
        lds_wait();
        bare_barrier();
        const int v = threadIdx.x;
        if (v < MT * 64) {
            const int i = v >> 6;
            const int ln = v & 63;
            const int rr = ln & 15;
            const int mb = 16 * i + 4 * (ln >> 4);
            if (!SILU || rr < 8) {
                f32x4 g = red[(0 * MT + i) * 64 + ln];
                f32x4 u = SILU ? red[(0 * MT + i) * 64 + (ln ^ 8)] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int wv = 1; wv < WV; ++wv) {
                    g += red[(wv * MT + i) * 64 + ln];
                    if (SILU) u += red[(wv * MT + i) * 64 + (ln ^ 8)];
                }
                const int c = b * CB + rr;
                if (c < Nout) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (mb + e < M) o.put(mb + e, c, g[e], u[e]);
                }
            }
        }
        if (splits > 1) splitk_finish<SILU>(o, ctr, b, b * CB, CB);
    }
}

}  // namespace krk
