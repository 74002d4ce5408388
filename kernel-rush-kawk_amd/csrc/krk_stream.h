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
//   * W is DMA'd straight into LDS in whole 128-byte lines
//     (global_load_lds_dwordx4, 64 lanes x 16 B): with one 16-row x tile as
//     1 KB row chunks, with more tiles as 8 rows x 128 B of the loading
//     wave's own k range (below).  MFMA B fragments are then read from LDS.
//   * A CU needs ~100 KB in flight: the ring holds `depth` stages of
//     16 rows x 512 k, depth-1 of them in flight while one is consumed, and
//     it keeps streaming across block boundaries.
//   * Workgroups are persistent (at most one per CU): workgroup g walks blocks
//     g', g' + G, ... (g' its XCD-aware index, below).  x is loaded once per
//     workgroup into VGPRs — wave w keeps the fragments of its fixed share of
//     k-steps (2 of every stage's 16) for every stage of the workgroup's K
//     range — so x costs one L2 read per CU
//     instead of one per block, and no load in the loop competes with the
//     ring in the in-order vmcnt counter.  It is read as whole 1 KB row
//     pieces and turned into fragments through LDS before the ring starts
//     (one 16-row tile: 8 rows x 128 B per load, fragments formed in
//     registers).
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
#include "krk_norm.h"
#include "krk_select.h"
#include "krk_sync.h"

namespace krk {

constexpr int kStreamWaves = 8;
constexpr int kStreamKC = 512;       // k per stage
constexpr int kStreamPitch = 1040;   // bytes per LDS row (1 KB + 16 B: fragment reads hit distinct banks)
constexpr int kStreamSlot = 16 * kStreamPitch;
constexpr int kStreamKPW = (kStreamKC / 32) / kStreamWaves;  // k-steps per wave per stage (2)
constexpr int kStreamLPW = 16 / kStreamWaves;                // DMAs per wave per stage (2)
constexpr int kStreamMaxDepth = 8;

// Bytes of dynamic LDS: `nred` reduction areas [WV][MT][64] f32x4, then the
// ring.  A block's partial sums are parked at its end and reduced during the
// next block's first stage.  With two or more stages per block one area
// suffices (the next block parks its sums only after its second stage's
// barrier, which every wave reaches after that reduction); with one stage
// per block the blocks alternate between two.  The area saved goes to the
// ring (measured: at 64 rows two areas left room for only 4 stages).  With
// two or more x tiles the launch takes two areas whenever they fit beside
// the ring and every output block, so that only a block's first stage ends
// in a barrier.
__host__ __device__ constexpr size_t stream_red_bytes(int MT) { return (size_t)kStreamWaves * MT * 64 * 16; }
__host__ __device__ constexpr int stream_nred(int stages_per_split) { return stages_per_split >= 2 ? 1 : 2; }
__host__ __device__ constexpr size_t stream_lds_bytes(int MT, int depth, int nred) {
    return (size_t)nred * stream_red_bytes(MT) + (size_t)depth * kStreamSlot;
}
// Output buffer behind the ring (unsplit K): the bf16 results of `obcap`
// blocks, [slot][16·MT rows][CB channels].
__host__ __device__ constexpr size_t stream_out_bytes(int MT, bool silu) { return (size_t)(silu ? 8 : 16) * 16 * MT * 2; }

// x staging before the ring starts: one stage of one 16-row tile is 16 KB;
// up to kStreamXStageMax bytes of stages go through LDS per round.
constexpr int kStreamXStageBytes = 16 * 1024;
constexpr size_t kStreamXStageMax = 128 * 1024;
__host__ __device__ constexpr int stream_xgroup(int MT) { return (int)(kStreamXStageMax / ((size_t)kStreamXStageBytes * MT)); }
// LDS the staging of XS stages needs (the launch allocates at least this).
__host__ __device__ constexpr size_t stream_xstage_bytes(int MT, int XS) {
    return (size_t)kStreamXStageBytes * MT * (XS < stream_xgroup(MT) ? XS : stream_xgroup(MT));
}

static_assert(kStreamKC == kFragKC, "fragment order is laid out in the stream kernel's stages");

// MT: 16-row m tiles (M <= 16·MT).  XS: most K stages a workgroup owns (its
// x fragments live in X[XS][2][MT]).  SILU: gate/up blocks with the epilogue.
// SK (K unsplit): 1 or kSelMaxK — each workgroup keeps every row's SK
// largest (value, index) keys over its blocks (krk_select.h) and writes them
// to sa.keys[m][workgroup * SK ...]; y (the logits) is written only when
// non-null.  0: no selection.
// XF: x is given in fragment order (frag_offset; rows past M and k
// past K hold zeros), as add_rmsnorm_frag_kernel writes the normalised rows
// of a normed call: every fragment is one contiguous 1 KB load, and the trip
// of x through LDS is skipped.
template <int MT, int XS, bool SILU, int SK = 0, bool XF = false>
__global__ void __launch_bounds__(512)
stream_gemm_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                   const uint16_t* __restrict__ w, int64_t ldw,
                   uint16_t* __restrict__ y, int64_t ldy,
                   int M, int N, int K, int splits, int depth, int obcap, int nred,
                   float* __restrict__ part, uint32_t* __restrict__ ctr, SelectArgs sa) {
    static_assert(MT >= 1 && MT <= 4, "MT covers up to 64 rows");
    constexpr bool SEL = SK > 0;
    static_assert(!(SEL && SILU), "selection reads plain logits");
    static_assert(SK == 0 || SK == 1 || SK == kSelMaxK, "argmax or top-kSelMaxK");
    static_assert(!(XF && SEL), "fragment-order x serves the normed plain calls");
    constexpr int WV = kStreamWaves;
    constexpr int KPW = kStreamKPW;
    constexpr int LPW = kStreamLPW;
    constexpr int CB = SILU ? 8 : 16;  // output channels per block

    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    f32x4* const red0 = reinterpret_cast<f32x4*>(smem);
    f32x4* const red1 = nred == 2 ? red0 + WV * MT * 64 : red0;
    unsigned char* const ring = smem + nred * stream_red_bytes(MT);
    uint16_t* const ob = reinterpret_cast<uint16_t*>(ring + (size_t)depth * kStreamSlot);
    constexpr int MP = 16 * MT;  // rows per output-buffer slot

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int q = lane >> 4;

    // This workgroup's split and blocks: blocks vg, vg + Gs, ... of split s.
    const int s = blockIdx.x % splits;
    const int gi = blockIdx.x / splits;
    const int Gs = gridDim.x / splits;
    const int Nout = SILU ? (N >> 1) : N;
    const int nblocks = (Nout + CB - 1) / CB;
    const int KST = (K + kStreamKC - 1) / kStreamKC;
    const int sb = (int)(((int64_t)s * KST) / splits);
    const int se = (int)(((int64_t)(s + 1) * KST) / splits);
    const int nst = se - sb;
    // XCD-aware order: workgroups go to the 8 XCDs round robin, so with K
    // unsplit the workgroups of one XCD (gi = x, x + 8, ...) take adjacent
    // blocks of each round, vg = x·Gs/8 + gi/8.  The partial lines of y that
    // neighbouring blocks write then meet in one XCD's L2 instead of being
    // written back from several.  Measured (bit-identical output): gate_up
    // at M = 16-64 0.4-0.9 us faster (M = 32: 22.57 -> 21.93 us), lm_head at
    // M = 32 / 64 4.3 / 6.2 us faster; M = 5-9 within 0.4 us.
    const int vg = (splits == 1 && (Gs & 7) == 0) ? (gi & 7) * (Gs >> 3) + (gi >> 3) : gi;
    const int myblocks = vg < nblocks ? (nblocks - 1 - vg) / Gs + 1 : 0;
    const int T = myblocks * nst;  // stages this workgroup consumes

    // DMA of the workgroup's t-th stage into ring slot t % depth.
    //   * One 16-row x tile: wave w loads tile rows w and w + 8 whole (1 KB
    //     each, row r at r·kStreamPitch), and every wave reads every row,
    //     so each stage ends in a workgroup barrier.
    //   * WPR (two or more x tiles): wave w loads only what it computes on,
    //     its 64 k of all 16 rows, into its own 2 KB of the slot: group h
    //     (tile rows 8h..8h+7) at byte 1024·h, lane l bringing row
    //     8h + l/8's 16-byte piece (l % 8) ^ (row >> 1) to byte 16·l, so a
    //     fragment read of 16 rows at one piece hits 16 distinct bank
    //     slots.  A wave's slots are then its own: its vmcnt wait alone
    //     makes a stage readable, and only the reduction needs barriers
    //     (measured, bit-identical, two alternating runs: gate_up M = 32 /
    //     48 / 64 22.1-22.2 -> 21.3, 24.6-24.7 -> 23.9, 26.3-26.5 -> 25.9-26.0
    //     us, lm_head M = 32 120.9-121.6 -> 119.6-119.7 us; with one tile
    //     the 8-row pieces ingest more slowly and the stage barrier costs
    //     less, lm_head M = 5-16 1.3-2.2 us slower).
    constexpr bool WPR = MT >= 2;
    const int klane = 8 * lane;
    const int rho = lane >> 3, lj = lane & 7;
    auto issue = [&](int t) {
        const int bi = t / nst;
        const int st = sb + (t - bi * nst);
        const int b = vg + bi * Gs;
        unsigned char* slot = ring + (size_t)(t % depth) * kStreamSlot + (WPR ? wave * 2048 : 0);
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int row = WPR ? 8 * i + rho : wave + WV * i;  // tile row 0..15
            const int k = st * kStreamKC + (WPR ? 64 * wave + 8 * (lj ^ (row >> 1)) : klane);
            const int kc = k < K ? k : 0;  // past K: any in-range address, masked at use
            int wr;
            if (SILU) {
                int ch = b * CB + (row & 7);
                ch = ch < Nout ? ch : Nout - 1;
                wr = row < 8 ? ch : ch + Nout;
            } else {
                const int ch = b * CB + row;
                wr = ch < Nout ? ch : Nout - 1;
            }
            dma_row_stream(w + (int64_t)wr * ldw + kc, slot + (WPR ? i * 1024 : row * kStreamPitch));
        }
    };
    // x fragments X[j][kk][i] of the workgroup's K stages: lane (r, q) =
    // x[16i + r][32·(KPW·wave + kk) + 8q .. +7] of stage sb + j.
    u32x4 X[XS][KPW][MT];
    if constexpr (XF) {
        // Stage sb + j, k-step KPW·wave + kk, tile i: one 1 KB run per wave.
        // Stages past the split's range are zero (their loads read stage sb).
        const unsigned char* xf = reinterpret_cast<const unsigned char*>(x);
#pragma unroll
        for (int j = 0; j < XS; ++j) {
            const int st = j < nst ? sb + j : sb;
#pragma unroll
            for (int kk = 0; kk < KPW; ++kk)
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    const u32x4 v = *reinterpret_cast<const u32x4*>(
                        xf + frag_offset(st, KPW * wave + kk, i, lane, MT));
                    X[j][kk][i] = j < nst ? v : u32x4{0u, 0u, 0u, 0u};
                }
        }
        // The ring starts once x has landed, as below (issuing it right
        // behind these loads measured 0.3-0.5 us slower per call).
        vm_wait<0>();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        for (int d = 0; d < depth - 1 && d < T; ++d) issue(d);
    } else {
        if constexpr (MT == 1) {
            // One 16-row tile: each wave loads only its own 128 bytes of every
            // row (k-steps KPW·w, KPW·w + 1 of each stage), as two loads of 8
            // rows x 128 B (whole lines): lane (q, b3, rho) of load h gets row
            // 8h + rho, 16-byte piece 4·(b3 ^ h) + q.  Fragment kk = 0 (pieces
            // 0-3) is load b3 taken lane by lane; kk = 1 (pieces 4-7) is load
            // 1 - b3 moved by 8 lanes within each 16-lane row (DPP row_ror:8).
            // No LDS trip and no barrier (measured: gate_up at M = 9-16 0.3-0.75
            // us faster, output bit-identical; with two or more tiles the 8-row
            // loads ingest more slowly than whole row pieces, 1.7-4.2 us slower).
            // Rows past M, k past K and stages past the split's range are zero.
            static_assert(KPW == 2, "two k-steps (128 bytes) per wave per stage");
            const int b3 = (lane >> 3) & 1;
            const int rho = lane & 7;
            u32x4 V[XS][2];
#pragma unroll
            for (int j = 0; j < XS; ++j)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int m = 8 * h + rho;
                    const int k = (sb + j) * kStreamKC + 32 * KPW * wave + 8 * (4 * (b3 ^ h) + q);
                    const bool kok = j < nst && k < K;
                    const u32x4 v = load_cached16(x + (int64_t)(m < M ? m : M - 1) * ldx + (kok ? k : 0));
                    V[j][h] = (kok && m < M) ? v : u32x4{0u, 0u, 0u, 0u};
                }
#pragma unroll
            for (int j = 0; j < XS; ++j) {
                X[j][0][0] = b3 ? V[j][1] : V[j][0];
                const u32x4 yv = b3 ? V[j][0] : V[j][1];
                constexpr int kRowRor8 = 0x128;  // DPP row_ror:8
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    X[j][1][0][e] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)yv[e], kRowRor8, 0xF, 0xF, false);
            }
        } else {
            // x for the workgroup's K range, loaded once.  Whole 1 KB row pieces (wave
            // w loads rows w, w + 8, ... of every stage): a CU pulls L2 data ~2.5x
            // faster this way than in the MFMA fragment pattern.  Rows past M, k past
            // K and stages past the split's range are zero.
            constexpr int LX = 2 * MT;  // 16·MT rows over 8 waves
            u32x4 XR[XS][LX];
#pragma unroll
            for (int j = 0; j < XS; ++j) {
                const int k = (sb + j) * kStreamKC + klane;
                const bool kok = j < nst && k < K;
#pragma unroll
                for (int i = 0; i < LX; ++i) {
                    const int m = wave + WV * i;
                    const u32x4 v = load_cached16(x + (int64_t)(m < M ? m : M - 1) * ldx + (kok ? k : 0));
                    XR[j][i] = (kok && m < M) ? v : u32x4{0u, 0u, 0u, 0u};
                }
            }
            // The rows go through LDS (16·MT rows of 1 KB per stage, up to XG
            // stages at a time from the start of the area, idle until the ring
            // starts and the first block ends; chunks XOR-swizzled by row so the
            // fragment reads hit distinct banks) and come back as this wave's MFMA
            // fragments X[j][kk][i]: one write, barrier, read, barrier round per
            // group of XG stages.
            constexpr int XG = stream_xgroup(MT);
            unsigned char* const xstage = smem;
#pragma unroll
            for (int j0 = 0; j0 < XS; j0 += XG) {
#pragma unroll
                for (int j = j0; j < j0 + XG && j < XS; ++j)
#pragma unroll
                    for (int i = 0; i < LX; ++i) {
                        const int m = wave + WV * i;
                        *reinterpret_cast<u32x4*>(xstage + (j - j0) * kStreamXStageBytes * MT + m * 1024 +
                                                  16 * (lane ^ (m & 15))) = XR[j][i];
                    }
                lds_wait();
                bare_barrier();
#pragma unroll
                for (int j = j0; j < j0 + XG && j < XS; ++j)
#pragma unroll
                    for (int kk = 0; kk < KPW; ++kk) {
                        const int c = 4 * (wave * KPW + kk) + q;
#pragma unroll
                        for (int i = 0; i < MT; ++i)
                            X[j][kk][i] = *reinterpret_cast<const u32x4*>(xstage + (j - j0) * kStreamXStageBytes * MT +
                                                                          (16 * i + r) * 1024 + 16 * (c ^ r));
                    }
                lds_wait();
                bare_barrier();
            }
        }
        // The weight ring starts only now.  Measured: with its prologue in flight
        // the first-touch HBM fills of x queue behind 256 workgroups' worth of
        // weight DMAs and the x preload takes ~1.7x longer than the ring latency
        // it would hide.
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        for (int d = 0; d < depth - 1 && d < T; ++d) issue(d);
    }

    OutStage<SILU> o{y, ldy, part, M, N, Nout, splits, s};
    // Global stores share vmcnt with the ring's DMAs on gfx9, so a store in
    // the stage loop makes the following ring waits stricter and stalls the
    // storing waves.  With K unsplit the block results therefore go to an
    // LDS output buffer, written to y with 16-byte stores only when the
    // buffer is full (rare) and at the end.  Split K keeps the fp32 partials
    // and the fix-up of splitk_finish.
    const bool vec_ok = ((reinterpret_cast<uintptr_t>(y) & 15) == 0) && ((ldy & 7) == 0);
    auto flush = [&](int base, int cnt) {  // local blocks base .. base+cnt-1 in slots 0 .. cnt-1
        constexpr int CPR = CB / 8;         // 16-byte chunks per row
        const int items = cnt * M * CPR;
        for (int it = threadIdx.x; it < items; it += blockDim.x) {
            const int ch = it % CPR;
            const int rest = it / CPR;
            const int m = rest % M;
            const int sl = rest / M;
            const int c0 = (vg + (base + sl) * Gs) * CB + 8 * ch;
            const u32x4 v = *reinterpret_cast<const u32x4*>(ob + ((size_t)(sl * MP + m) * CB + 8 * ch));
            uint16_t* dst = y + (int64_t)m * ldy + c0;
            if (vec_ok && c0 + 8 <= Nout) {
                *reinterpret_cast<u32x4*>(dst) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (c0 + e < Nout) dst[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
            }
        }
    };
    // SEL: item slots a thread visits in finish_block (the same rows every
    // block), each with its (row, channel)'s running largest keys.
    constexpr int kSelSlots = SEL ? (MT * 4 * (SILU ? 8 : 16) * 4 + 511) / 512 : 1;
    constexpr int KL = SK > 0 ? SK : 1;  // keys kept per slot, descending
    uint64_t best[kSelSlots][KL];
#pragma unroll
    for (int j = 0; j < kSelSlots; ++j)
#pragma unroll
        for (int q2 = 0; q2 < KL; ++q2) best[j][q2] = 0;
    // Block epilogue: each thread finishes output elements (m, c) of the
    // block, summing the eight waves' partials in fixed wave order (8 or 16
    // independent LDS reads, then the adds).  It runs inside the next
    // block's first stage, after that stage's barrier (which also publishes
    // the partials) and its DMA issue, so the ring keeps streaming while it
    // works.  Partial layout: rb[wave][m tile][lane] f32x4, lane (r, q) holds
    // rows 4q..4q+3 of channel r.
    auto finish_block = [&](int bl, const f32x4* rb) {
        const int b = vg + bl * Gs;
        const int sl = obcap > 0 ? bl % obcap : 0;
        if (splits == 1 && sl == 0 && bl > 0 && (!SEL || y)) {
            // Buffer full: write it out before slot 0 is reused.
            flush(bl - obcap, obcap);
            lds_wait();
            bare_barrier();
        }
        const float* rf = reinterpret_cast<const float*>(rb);
        constexpr int LS = SILU ? 8 : 16;    // channels of a 16-row tile with outputs
        constexpr int LSB = SILU ? 3 : 4;    // log2(LS)
        constexpr int ITEMS = MT * 4 * LS * 4;
        auto item = [&](int it, int n) {  // n = it / 512, the thread's item slot
            const int e = it & 3;
            const int rr = (it >> 2) & (LS - 1);
            const int qq = (it >> (2 + LSB)) & 3;
            const int i = it >> (4 + LSB);
            const int ln = rr + 16 * qq;
            const int m = 16 * i + 4 * qq + e;
            float gv[WV], uv[WV];
            if constexpr (MT >= 2) {
                // Byte offsets from one base: every wave's read is the same
                // address register plus an immediate (ds_read2st64 pairs).
                // Measured, bit-identical: gate_up M = 64 25.8-25.9 -> 24.7
                // us, M = 32-48 0.1-0.2 us; with one x tile lm_head M = 8-16
                // was 1.2-2.3 us slower, so that keeps per-wave addresses.
                const unsigned char* const rbb = reinterpret_cast<const unsigned char*>(rf);
                const unsigned go = (unsigned)((i * 64 + ln) * 4 + e) * 4u;
                const unsigned uo = (unsigned)((i * 64 + (ln ^ 8)) * 4 + e) * 4u;
#pragma unroll
                for (int wv = 0; wv < WV; ++wv) {
                    gv[wv] = *reinterpret_cast<const float*>(rbb + go + wv * MT * 1024);
                    if (SILU) uv[wv] = *reinterpret_cast<const float*>(rbb + uo + wv * MT * 1024);
                }
            } else {
#pragma unroll
                for (int wv = 0; wv < WV; ++wv) {
                    gv[wv] = rf[((wv * MT + i) * 64 + ln) * 4 + e];
                    if (SILU) uv[wv] = rf[((wv * MT + i) * 64 + (ln ^ 8)) * 4 + e];
                }
            }
            float g = gv[0], u = SILU ? uv[0] : 0.0f;
#pragma unroll
            for (int wv = 1; wv < WV; ++wv) {
                g += gv[wv];
                if (SILU) u += uv[wv];
            }
            const int c = b * CB + rr;
            if (splits == 1) {
                const uint32_t v = SILU ? silu_mul_bf16(g, u) : f32_to_bf16(g);
                ob[(size_t)(sl * MP + m) * CB + rr] = (uint16_t)v;
                if constexpr (SEL) {
                    // Per lane: the largest key of its channel of row m over
                    // the blocks so far (reduced across channels at the end).
                    if (m < M && c < Nout) {
                        const uint64_t key = sel_key(v, (uint32_t)c);
                        if constexpr (SK == 1) best[n][0] = umax64(best[n][0], key);
                        else topk_insert(best[n], key);
                    }
                }
            } else if (m < M && c < Nout) {
                o.put(m, c, g, u);
            }
        };
        if constexpr (ITEMS % 512 != 0 || (SILU && MT == 4)) {
            // Item counts that leave threads idle or give some two items
            // (gate_up at 1-3 x tiles, lm_head at 1 or 3): the thread's items
            // unrolled (512 threads), so the LDS reads of all of them go out
            // before the first sum waits.  Measured, bit-identical: gate_up
            // M = 9-16 / 32 / 48 0.6 / 0.35 / 1.1 us faster, lm_head plans at
            // M = 5-16 3.5-4.3 us and M = 48 3.3 us faster.  Counts that are a
            // multiple of 512 keep the loop: unrolled, lm_head at M = 24-32
            // was 1.8-2.4 us slower, and at four plain x tiles the kernel
            // spilled past 256 VGPRs (lm_head M = 64 18 us slower).  The
            // SwiGLU epilogue at four x tiles (512 items) is the exception:
            // unrolled it fits (255 VGPRs) and gate_up at M = 49-64 measured
            // 0.55-0.6 us faster (M = 64 24.66-24.69 -> 24.06-24.13 us).
#pragma unroll
            for (int n = 0; n < (ITEMS + 511) / 512; ++n) {
                const int it = threadIdx.x + 512 * n;
                if (ITEMS % 512 == 0 || it < ITEMS) item(it, n);
            }
        } else if constexpr (!SILU && !SEL && MT == 4) {
            // Four x tiles, plain: 1024 outputs, two per thread, taken as
            // two adjacent rows (e, e + 1) of one lane so each wave's pair is
            // one 8-byte read, summed in the same wave order (255 VGPRs, no
            // spill; measured, bit-identical: lm_head M = 64 135.1-136.4 ->
            // 132.1-133.1 us).
            const int p = threadIdx.x;
            const int e0 = 2 * (p & 1);
            const int rr = (p >> 1) & 15;
            const int qq = (p >> 5) & 3;
            const int i = p >> 7;
            const int ln = rr + 16 * qq;
            const unsigned char* const rbb = reinterpret_cast<const unsigned char*>(rf);
            const unsigned go = (unsigned)((i * 64 + ln) * 4 + e0) * 4u;
            f32x2 gv[WV];
#pragma unroll
            for (int wv = 0; wv < WV; ++wv) gv[wv] = *reinterpret_cast<const f32x2*>(rbb + go + wv * MT * 1024);
            f32x2 g = gv[0];
#pragma unroll
            for (int wv = 1; wv < WV; ++wv) g += gv[wv];
            const int c = b * CB + rr;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int m = 16 * i + 4 * qq + e0 + h;
                if (splits == 1) {
                    ob[(size_t)(sl * MP + m) * CB + rr] = (uint16_t)f32_to_bf16(g[h]);
                } else if (m < M && c < Nout) {
                    o.put(m, c, g[h], 0.0f);
                }
            }
        } else {
            for (int it = threadIdx.x; it < ITEMS; it += blockDim.x) item(it, it / 512);
        }
        if (splits > 1) splitk_finish<SILU, 1, 1>(o, ctr, b, b * CB, CB);
    };

    int t = 0;
    for (int bi = 0; bi < myblocks; ++bi) {
        f32x4 acc[MT];
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
        for (int j = 0; j < XS; ++j) {
            if (j < nst) {
                vm_wait_stages<LPW>(min(depth - 2, T - 1 - t));
                // One tile: stage t landed for every wave and the slot of t - 1
                // is free.  WPR: at a block's first stage the barrier
                // publishes the last block's partial sums; with one
                // reduction area, the second stage's barrier keeps this
                // block's sums from being parked before every wave has
                // read the last block's.
                if (!WPR || j == 0 || (j == 1 && nred == 1)) bare_barrier();
                if (t + depth - 1 < T) issue(t + depth - 1);
                if (j == 0 && bi > 0) finish_block(bi - 1, (bi & 1) ? red0 : red1);
                const unsigned char* slot = ring + (size_t)(t % depth) * kStreamSlot + (WPR ? wave * 2048 : 0);
                const bool ktail = (sb + j + 1) * kStreamKC > K;
#pragma unroll
                for (int kk = 0; kk < KPW; ++kk) {
                    const int chunk = 4 * (wave * KPW + kk) + q;  // 16-byte chunk of the 1 KB row
                    const int pc = 4 * kk + q;  // the piece within the wave's 64 k
                    u32x4 v = *reinterpret_cast<const u32x4*>(
                        slot + (WPR ? (r >> 3) * 1024 + (r & 7) * 128 + 16 * (pc ^ (r >> 1)) : r * kStreamPitch + 16 * chunk));
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

        // Park this block's partial sums; the next block's first barrier
        // publishes them.  Buffer bi % 2 was last read by the epilogue of
        // block bi - 2, which ran before at least one barrier this wave has
        // since passed (with one area: this block's second-stage barrier).
        f32x4* const rb = (bi & 1) ? red1 : red0;
#pragma unroll
        for (int i = 0; i < MT; ++i) rb[(wave * MT + i) * 64 + lane] = acc[i];
        lds_wait();
    }
    if (myblocks > 0) {
        bare_barrier();
        finish_block(myblocks - 1, ((myblocks - 1) & 1) ? red1 : red0);
        if (splits == 1 && (!SEL || y)) {
            lds_wait();
            bare_barrier();
            const int base = (myblocks - 1) / obcap * obcap;
            flush(base, myblocks - base);
        }
    }
    if constexpr (SEL) {
        // Reduce each row's keys over its 16 channels (lane bits 2..5: the
        // block size covers the items of one slot, so it and lane agree in
        // bits 0..5); the lane of channel 0 writes the row's keys.
#pragma unroll
        for (int j = 0; j < kSelSlots; ++j) {
#pragma unroll
            for (int off = 4; off < 64; off <<= 1) {
                if constexpr (SK == 1) best[j][0] = umax64(best[j][0], shfl_xor_u64(best[j][0], off));
                else xor_level(best[j], off);
            }
            const int it = threadIdx.x + 512 * j;
            const int e = it & 3;
            const int qq = (it >> 6) & 3;  // item layout of finish_block (LS = 16)
            const int i = it >> 8;
            const int m = 16 * i + 4 * qq + e;
            if (it < MT * 4 * 16 * 4 && ((it >> 2) & 15) == 0 && m < M) {
#pragma unroll
                for (int q2 = 0; q2 < KL; ++q2)
                    store_agent_u64(sa.keys + (int64_t)m * sa.ldk + (int64_t)blockIdx.x * KL + q2, best[j][q2]);
            }
        }
    }
}

}  // namespace krk
