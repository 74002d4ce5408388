// Wave-sliced MFMA skinny GEMM (gfx950): every wave owns its own K chunks and
// streams both operands of them into a private LDS ring by LDS DMA, so the
// main loop has no workgroup barrier.  y = x[M,K] · W[N,K]ᵀ, plain epilogue,
// M <= 32 per launch.
//
// Reference counterparts: _skinny_kernel with split-K and its _sum_kernel
// (engine/kernels/gemm.py:54-104); like them it covers the decode shapes whose
// weight stream is short (o_proj and down_proj, N = 2560, and QKV).
//
// Why (measured on MI355X, graph replay over rotating weight copies):
//   * at M = 5-16 the other kernels pay for x: the VALU kernel stages x into
//     LDS in every workgroup and reads it back for every weight block, and
//     the LDS-staged MFMA kernel moves x and W through registers into LDS
//     with a workgroup barrier per stage;
//   * here the channels are split evenly over one workgroup per CU (N / 256:
//     10 channels for N = 2560, 24 for 6144), and each wave takes K chunks
//     c = wave, wave + 8, ... of the workgroup's K range.  A chunk is KC k
//     (64 or 128) of the block's cb weight rows and of the M x rows: the
//     eight waves' chunks of one round are adjacent pieces of the same rows;
//   * one LDS DMA (global_load_lds_dwordx4, 64 lanes x 16 B) moves one
//     "group": RG = 1024 / (2·KC) rows x 2·KC bytes, whole 128-byte lines, so
//     the weight stream needs no register round trip and no swizzle pass;
//   * a wave waits only for its own DMAs (vmcnt), reads its MFMA fragments
//     from its own ring slot and issues its next chunk before it computes the
//     current one; the workgroup synchronises once, for the final fixed-order
//     reduction across waves.
// Against the table's previous plans this measured 0.7-2.3 us faster per call
// for o and down at M = 5-16 (down M = 8: 10.6 against 12.9 us) and 0.5 us for
// qkv at M = 5-8.
//
// LDS layout of a wave's ring slot: NGV weight groups, then XGV x groups,
// 1 KB each.  Lane l of a DMA loads row ρ = l / LR of its group (LR = 64 / RG
// lanes per row) into 16-byte slot j = l % LR, which holds the row's 16-byte
// piece j ^ f(r) (r the row within its 16-row MFMA tile; f(r) = r for
// LR >= 16, r >> 1 for LR = 8).  A fragment read of 16 tile rows at one piece
// then lands in 16 distinct 16-byte bank slots of a 256-byte bank row, with
// no padding.
//
// Rows past the block's channels or past M, groups past NGV or XGV and k past
// K are never loaded; the MFMA rows they feed produce outputs that are not
// stored (a fragment of k past K is zeroed in both operands).
#pragma once

#include "krk_epilogue.h"
#include "krk_sync.h"

namespace krk {

constexpr int kSliceWaves = 8;
constexpr int kSliceGroup = 1024;  // bytes one DMA writes

// Groups of a 16-row tile and rows per group for KC k per chunk.
__host__ __device__ constexpr int slice_rg(int KC) { return 1024 / (2 * KC); }
__host__ __device__ constexpr int slice_gt(int KC) { return 16 / slice_rg(KC); }
// Dynamic LDS: every wave's ring of D slots, or the reduction area.
__host__ __device__ constexpr size_t slice_lds_bytes(int MT, int NT, int D, int NGV, int XGV) {
    const size_t ring = (size_t)kSliceWaves * D * (NGV + XGV) * kSliceGroup;
    const size_t red = (size_t)kSliceWaves * MT * NT * 64 * 16;
    return ring > red ? ring : red;
}

// MT, NT: 16-row x and W tiles.  D: chunks in flight per wave.  KC: k per
// chunk (64 or 128).  NGV / XGV: weight / x groups loaded per chunk
// (ceil(cb / RG), ceil(M / RG)), compile-time so every wait count is.
// Grid: (blocks, splits); split s owns chunks [s·cper + min(s, crem), ...)
// of K (cper + (s < crem) of them).
template <int MT, int NT, int D, int KC, int NGV, int XGV>
__global__ void __launch_bounds__(64 * kSliceWaves)
slice_gemm_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                  const uint16_t* __restrict__ w, int64_t ldw,
                  uint16_t* __restrict__ y, int64_t ldy,
                  int M, int N, int K, int splits, int cb, int cper, int crem,
                  float* __restrict__ part, uint32_t* __restrict__ ctr) {
    constexpr int WV = kSliceWaves;
    constexpr int RG = slice_rg(KC), LR = 64 / RG, KS = KC / 32, GT = slice_gt(KC);
    constexpr int G = NGV + XGV;  // DMAs per chunk
    constexpr int SLOT = G * kSliceGroup;
    static_assert(KC == 64 || KC == 128, "128 or 256 bytes of each row per chunk");
    static_assert(NGV >= 1 && NGV <= GT * NT && XGV >= 1 && XGV <= GT * MT, "groups fit the tiles");
    static_assert(D >= 2 && D <= 3, "chunks in flight per wave");
    static_assert(G * (D - 1) < 64, "vmcnt is 6 bits");
    static_assert(WV == 8, "chunk counts below divide by 8 with a shift");
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r = lane & 15, q = lane >> 4;
    const int blk = blockIdx.x;
    const int s = blockIdx.y;
    const int c0 = blk * cb;
    auto fsw = [](int rr) { return LR >= 16 ? rr : (rr >> 1); };
    const int lrho = lane / LR, lj = lane % LR;

    // Source of each lane per group: weight group g holds block channels
    // RG·g + ρ, x group g rows RG·g + ρ (tile row = the same index mod 16).
    const uint16_t* src[G];
    bool lok[G];
#pragma unroll
    for (int g = 0; g < NGV; ++g) {
        const int cl = RG * g + lrho;
        lok[g] = cl < cb;
        int ch = c0 + cl;
        ch = ch < N ? ch : N - 1;  // last block past N: an in-range row, its outputs not stored
        src[g] = w + (int64_t)ch * ldw + 8 * (lj ^ fsw(cl & 15));
    }
#pragma unroll
    for (int g = 0; g < XGV; ++g) {
        const int m = RG * g + lrho;
        lok[NGV + g] = m < M;
        src[NGV + g] = x + (int64_t)(m < M ? m : M - 1) * ldx + 8 * (lj ^ fsw(m & 15));
    }
    // A group is loaded unmasked when all its rows exist: every group but the
    // last of each operand, and the last one when cb (M) fills it.
    const bool wlast_full = RG * NGV <= cb;
    const bool xlast_full = RG * XGV <= M;

    const int cs = s * cper + (s < crem ? s : crem);
    const int cn = cper + (s < crem ? 1 : 0);
    const int nc = cn > wave ? (cn - wave + WV - 1) >> 3 : 0;  // this wave's chunks
    const bool ktail = (K % KC) != 0;
    unsigned char* const ring = smem + (size_t)wave * D * SLOT;

    auto issue = [&](int j) {
        const int k0 = (cs + wave + WV * j) * KC;
        unsigned char* const slot = ring + (j % D) * SLOT;
        const bool tailc = ktail && k0 + KC > K;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const bool weights = g < NGV;
            const bool full = weights ? (g < NGV - 1 || wlast_full) : (g < G - 1 || xlast_full);
            const uint16_t* p = src[g] + k0;
            unsigned char* d = slot + g * kSliceGroup;
            if (full && !tailc) {
                if (weights) dma_row_stream(p, d);
                else dma_row(p, d);
            } else {
                const int row = weights ? RG * g + lrho : RG * (g - NGV) + lrho;
                if (lok[g] && k0 + 8 * (lj ^ fsw(row & 15)) < K) {
                    if (weights) dma_row_stream(p, d);
                    else dma_row(p, d);
                }
            }
        }
    };

    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Fragment addresses within a slot: tile row r sits in group r / RG of its
    // tile at row r % RG; tile rows of groups that are not loaded read group 0
    // (their outputs are not stored).
    const int gr = r / RG, rrho = r % RG, fr = fsw(r);
    int boff[NT], aoff[MT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int g = GT * t + gr;
        boff[t] = (g < NGV ? g : 0) * kSliceGroup + 16 * LR * rrho;
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int g = GT * i + gr;
        aoff[i] = (g < XGV ? NGV + g : 0) * kSliceGroup + 16 * LR * rrho;
    }

    // Chunk j goes to slot j % D.  Step j first issues chunk j + D - 1 into
    // the slot chunk j - 1 used (read in step j - 1, which waited for those
    // reads), then waits until only the chunks after j are outstanding.
    for (int j = 0; j < D - 1 && j < nc; ++j) issue(j);
    for (int j = 0; j < nc; ++j) {
        const bool more = j + D - 1 < nc;
        if (more) issue(j + D - 1);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (more) {
            vm_wait<G * (D - 1)>();
        } else if (D == 3 && j + 1 < nc) {
            vm_wait<G>();
        } else {
            vm_wait<0>();
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        const unsigned char* const slot = ring + (j % D) * SLOT;
        const int k0 = (cs + wave + WV * j) * KC;
        const bool tail = ktail && k0 + KC > K;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            const int pc = 4 * kk + q;  // this lane's 16-byte piece of the chunk
            const int lo = 16 * (pc ^ fr);
            const bool kok = !tail || (k0 + 8 * pc < K);
            bf16x8 b[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                u32x4 v = *reinterpret_cast<const u32x4*>(slot + boff[t] + lo);
                if (!kok) v = u32x4{0u, 0u, 0u, 0u};
                b[t] = __builtin_bit_cast(bf16x8, v);
            }
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                u32x4 v = *reinterpret_cast<const u32x4*>(slot + aoff[i] + lo);
                if (!kok) v = u32x4{0u, 0u, 0u, 0u};
                const bf16x8 a = __builtin_bit_cast(bf16x8, v);
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[t], acc[i][t], 0, 0, 0);
            }
        }
        lds_wait();  // the slot's reads are done before step j + 1 refills it
    }

    // Cross-wave reduction in fixed wave order (reuses the rings).
    f32x4* red = reinterpret_cast<f32x4*>(smem);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) red[((wave * MT + i) * NT + t) * 64 + lane] = acc[i][t];
    __syncthreads();
    OutStage<false> o{y, ldy, part, M, N, N, splits, s};
    constexpr int items = MT * NT * 64;
    for (int v = threadIdx.x; v < items; v += blockDim.x) {
        const int ln = v & 63;
        const int t = (v >> 6) % NT;
        const int i = (v >> 6) / NT;
        f32x4 sum = red[(i * NT + t) * 64 + ln];
#pragma unroll
        for (int wv = 1; wv < WV; ++wv) sum += red[((wv * MT + i) * NT + t) * 64 + ln];
        const int cl = 16 * t + (ln & 15);
        const int c = c0 + cl;
        if (cl < cb && c < N) {
            const int mb = 16 * i + 4 * (ln >> 4);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (mb + e < M) o.put(mb + e, c, sum[e], 0.0f);
        }
    }
    if (splits > 1) splitk_finish<false>(o, ctr, blk, c0, cb);
}

}  // namespace krk
