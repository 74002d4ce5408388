// Residual-add + RMSNorm prologue computed inside a projection kernel by a
// few of its own waves (gfx950), so a normed projection at M >= 2 is one
// launch.  Reference counterpart: the normed prologue the reference folds
// into its GEMM tiles (engine/kernels/gemm.py:21-51 _norm_stats /
// _normed_tile, offered by pick_normed at gemm.py:501-560); rounding points
// of engine/kernels/add_rmsnorm.py:15-29 and engine/kernels/rmsnorm.py:34-43.
//
// Every workgroup of a projection needs all M normalised rows (for its K
// range), but each row costs a full pass over x, the branch d and the gain:
// computing them in every workgroup was measured to cost more than a separate
// prologue launch.  Here each row is computed once per L2:
//
//   * the normalised rows go to one copy per XCC (accelerator die), chosen by
//     the hardware XCC_ID register, written with plain stores and read back
//     with plain loads: producer and readers of a copy share that die's L2,
//     which is coherent for the CUs attached to it;
//   * producer waves are picked from the grid assuming the dispatcher's
//     round-robin order over the 8 dies (workgroup L on die L % 8); each
//     producer wave computes one row, stores it, waits for the stores
//     (vmcnt(0)) and then raises the row's flag with an agent-scope store;
//   * every workgroup issues its first weight loads, then waits (one wave
//     polls the M flags of its die's copy with agent-scope loads) and reads
//     x from the copy;
//   * the wait is bounded by the 100 MHz realtime clock.  A workgroup whose
//     rows are not all flagged in time (the dispatch order was not the
//     assumed one, or producers were not resident) computes the missing rows
//     itself into its die's copy — the same values, so duplicate writers are
//     harmless — raises their flags and counts a fallback.  Correctness never
//     depends on the dispatch assumption, only the speed does;
//   * xout = bf16(x + d) is written once per row: the first producer of a row
//     on any die claims it with an agent-scope exchange;
//   * every wave clears the flags it raised and the claims it won at its end
//     of the kernel, so the control block is zero for the next call (a later
//     kernel on the stream) with no count of finished workgroups: a single
//     counter hit by every workgroup was measured to serialise, and its
//     answer would wait in the in-order vmcnt queue ahead of the weight ring.
//
// The rows are those of krk_norm.h: s = bf16(x + d), rstd =
// 1/sqrt(sum(s²)/K + eps) with the sum taken per lane in k order and then by a
// xor butterfly (every lane ends with the same bits), n = bf16(bf16(s·rstd)·g).
#pragma once

#include "krk_epilogue.h"
#include "krk_norm.h"
#include "krk_sync.h"

namespace krk {

constexpr int kCoopSlots = 16;      // copies: the XCC_ID register field is 4 bits
constexpr int kCoopDies = 8;        // dies the dispatcher is assumed to round-robin over
constexpr int kCoopMaxRows = 64;
constexpr int kCoopMaxVec = 8;      // 16-byte vectors per lane and row: K <= 64 * 8 * 8
constexpr int kCoopMaxK = 64 * 8 * kCoopMaxVec;
constexpr uint32_t kCoopWaitTicks = 3000;  // default bound of the wait: 30 us of the 100 MHz realtime clock

// Control block (u32 words, zero between calls except the statistic).
constexpr int kCoopFlags = 0;                                   // [kCoopSlots][kCoopMaxRows]
constexpr int kCoopClaims = kCoopFlags + kCoopSlots * kCoopMaxRows;  // [kCoopMaxRows]
constexpr int kCoopFallbacks = kCoopClaims + kCoopMaxRows + 32;  // own 128-byte line; cumulative, never cleared
constexpr int kCoopCtlWords = kCoopFallbacks + 32;

__host__ __device__ constexpr size_t coop_ctl_bytes() { return (size_t)kCoopCtlWords * 4; }
// Bytes of one copy of the rows: enough for M rows of K row-major and for
// the fragment layout of the stream kernel (16-row tiles, 512-k stages).
// `tiles` 16-row tiles (at least ceil(M / 16)).
__host__ __device__ constexpr size_t coop_slot_bytes(int M, int K, int tiles) {
    return (size_t)((K + 511) / 512) * (tiles > (M + 15) / 16 ? tiles : (M + 15) / 16) * 16 * 512 * 2;
}
// Bytes of the copies (the control block precedes them, padded to 256 bytes).
__host__ __device__ constexpr size_t coop_copy_bytes(int M, int K, int tiles) {
    return kCoopSlots * coop_slot_bytes(M, K, tiles);
}

// Where element (m, k) of a copy lives.  RowLayout: row-major, row stride K.
struct RowLayout {
    uint16_t* base;
    int K;
    __device__ __forceinline__ uint16_t* at(int m, int k) const { return base + (int64_t)m * K + k; }
};

struct CoopNorm {
    const uint16_t* x;   // [M, K] residual rows
    int64_t ldx;
    NormArgs na;         // branch d, gain, eps, xout
    uint32_t* ctl;       // control block
    uint16_t* copies;    // kCoopSlots copies of the normalised rows
    int64_t slot_elems;  // elements per copy
    int M, K;
    int producers;       // 0: no producer waves (every workgroup computes the rows itself; for tests)
    uint32_t wait_ticks; // bound of the wait, 100 MHz ticks
};

__device__ __forceinline__ int coop_slot() {
    // s_getreg_b32 HW_REG_XCC_ID, bits [3:0]: this wave's accelerator die.
    return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & (kCoopSlots - 1);
}

// Flags are written and polled at agent scope (device-coherent memory): a
// workgroup-scope poll, which stays in the die's caches, was measured never
// to see another CU's store (every workgroup timed out).
__device__ __forceinline__ void store_flag(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_flag(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave computes row m into `copy` (elements placed by the layout), waits for its
// stores and raises the row's `flag`; only then does it claim the row's
// xout (an agent-scope exchange, off the readers' path) and write xout's row
// if the claim is its.  Returns whether it won the claim (wave-uniform).
template <class Layout>
__device__ __forceinline__ bool coop_row(const CoopNorm& c, const Layout& copy, uint32_t* flag, int m, int lane) {
    const uint16_t* xr = c.x + (int64_t)m * c.ldx;
    const uint16_t* dr = c.na.d + (int64_t)m * c.na.ldd;
    u32x4 s[kCoopMaxVec], g[kCoopMaxVec];
    float ss = 0.0f;
#pragma unroll
    for (int v = 0; v < kCoopMaxVec; ++v) {
        const int k = 8 * (lane + 64 * v);
        if (k < c.K) {
            s[v] = add_bf16x8(load_cached16(xr + k), load_cached16(dr + k));
            g[v] = load_cached16(c.na.wn + k);
            ss = sumsq_bf16x8(s[v], ss);
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    const float rstd = rms_rstd(ss, c.K, c.na.eps);
#pragma unroll
    for (int v = 0; v < kCoopMaxVec; ++v) {
        const int k = 8 * (lane + 64 * v);
        if (k < c.K) *reinterpret_cast<u32x4*>(copy.at(m, k)) = normalize_bf16x8(s[v], rstd, g[v]);
    }
    drain_memory();
    if (lane == 0) store_flag(flag, 1u);
    uint32_t claimed = 1u;
    if (lane == 0)
        claimed = __hip_atomic_exchange(c.ctl + kCoopClaims + m, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool won = __shfl(claimed, 0) == 0u;
    if (won) {
        uint16_t* xo = c.na.xout + (int64_t)m * c.na.ldxo;
#pragma unroll
        for (int v = 0; v < kCoopMaxVec; ++v) {
            const int k = 8 * (lane + 64 * v);
            if (k < c.K) *reinterpret_cast<u32x4*>(xo + k) = s[v];
        }
    }
    return won;
}

// What a wave raised during the call: its die slot, the rows whose flags it
// set and the rows whose xout claims it won.  The wave clears exactly these
// at its end (coop_finish), so the control block is back at zero once the
// kernel is done, without any count of finished workgroups.
struct CoopMarks {
    int slot;
    uint64_t flagged;
    uint64_t won;
};

// Producer index of this workgroup on its (assumed) die: workgroup L sits on
// die L % 8 as rank L / 8 of `count` there.  `from_end` numbers producers
// from the die's last rank (persistent grids, whose last workgroups carry the
// fewest blocks); otherwise from its first.
__device__ __forceinline__ int coop_producer_index(int L, int G, bool from_end) {
    const int die = L % kCoopDies;
    const int rank = L / kCoopDies;
    const int count = (G - 1 - die) / kCoopDies + 1;
    return from_end ? count - 1 - rank : rank;
}

// Producer phase: wave w of producer p computes row p * rows_per_wg + w (for
// w < rows_per_wg) into its die's copy and raises the row's flag.  The
// wave's xout stores may still be in flight when it returns.
template <class Layout>
__device__ __forceinline__ void coop_produce(const CoopNorm& c, const Layout& copy, CoopMarks& mk, int p,
                                             int rows_per_wg, int wave, int lane) {
    const int m = p * rows_per_wg + wave;
    if (c.producers && wave < rows_per_wg && m < c.M) {
        const bool won = coop_row(c, copy, c.ctl + kCoopFlags + mk.slot * kCoopMaxRows + m, m, lane);
        mk.flagged |= 1ull << m;
        if (won) mk.won |= 1ull << m;
    }
}

// Wait until the M rows of this die's copy are flagged; on time-out compute
// every row here (the producers' values, so concurrent writers agree) and
// raise the flags for other waiters.  Called by every thread of the
// workgroup (`waves` waves); `word` is an LDS word for the broadcast.
// On return every row of the copy has been stored.
template <class Layout>
__device__ __forceinline__ void coop_wait(const CoopNorm& c, const Layout& copy, CoopMarks& mk, int wave, int lane,
                                          int waves, int* word) {
    uint32_t* flags = c.ctl + kCoopFlags + mk.slot * kCoopMaxRows;
    if (wave == 0) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        uint64_t missing;
        while (true) {
            const uint32_t f = lane < c.M ? load_flag(flags + lane) : 1u;
            missing = __builtin_amdgcn_ballot_w64(f == 0u);
            if (missing == 0 || __builtin_amdgcn_s_memrealtime() - t0 > c.wait_ticks) break;
            __builtin_amdgcn_s_sleep(2);
        }
        if (lane == 0) *word = missing != 0;
    }
    lds_wait();
    bare_barrier();
    if (*word) {
        for (int m = wave; m < c.M; m += waves) {
            if (coop_row(c, copy, flags + m, m, lane)) mk.won |= 1ull << m;
            mk.flagged |= 1ull << m;
        }
        if (threadIdx.x == 0)
            __hip_atomic_fetch_add(c.ctl + kCoopFallbacks, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        drain_memory();
        bare_barrier();
    }
}

// This die's copy of the rows.
__device__ __forceinline__ uint16_t* coop_copy(const CoopNorm& c, int slot) {
    return c.copies + (int64_t)slot * c.slot_elems;
}

// At the wave's end: clear the flags it raised and the claims it won.  A
// reader still waiting on a cleared flag times out and computes the rows
// itself, so an early clear costs time, never correctness; in the stream
// kernel every wave ends long after the grid has passed its wait.
__device__ __forceinline__ void coop_finish(const CoopNorm& c, const CoopMarks& mk, int lane) {
    if ((mk.flagged >> lane) & 1ull) store_flag(c.ctl + kCoopFlags + mk.slot * kCoopMaxRows + lane, 0u);
    if ((mk.won >> lane) & 1ull) store_flag(c.ctl + kCoopClaims + lane, 0u);
}

}  // namespace krk
