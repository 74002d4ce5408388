// Token selection fused into the lm_head projection: per-row argmax / top-k
// of the bf16 logits without writing them (gfx950).
//
// Reference consumers: `logits.argmax(dim=-1)` (engine/engine.py:196,
// engine/model.py:365; lowest index on exact ties, OPTIMIZATION_GUIDE.md:213)
// and `torch.topk(logits, k).indices` (engine/recycle.py:170).
//
// Order.  A logit is compared as its bf16 value (the projection's rounding),
// with every NaN above +inf and -0 equal to +0, as torch.argmax compares.
// Equal values rank the lower index first; torch.topk leaves the order of
// equal values unspecified, this is one valid order and it is deterministic.
// Each candidate is one 64-bit key: the order-preserving 16-bit image of the
// value in the high half and ~index in the low half, so the largest key is the
// largest value at its lowest index, and keys of distinct indices never tie.
// Key 0 is below every real key and marks an empty slot.
//
// Reduction (no second launch):
//   * every workgroup writes, per row, the top-k keys of its output channels
//     to cand[g][m][0..k) (g = its linear index);
//   * workgroups form groups of kSelGroup; the last one of a group to finish
//     (agent-scope counter, as the split-K fix-up in krk_epilogue.h) merges
//     the group's lists into cand2[group][m][0..k);
//   * the last group to finish merges those lists and writes the indices
//     (and the values, when asked), then resets the counters for the next
//     call.
// A merge of L lists keeps, per row, a subgroup of P threads of one wave: each
// thread reduces its share of the lists to a sorted local top-k, then k rounds
// of a subgroup max pick the winners (each round's winner advances its list).
#pragma once

#include "krk_epilogue.h"

namespace krk {

constexpr int kSelMaxK = 8;
constexpr int kSelGroup = 256;

// Workspace layout of a selecting call with G workgroups, M rows and k.
struct SelectLayout {
    size_t ctr1, ctr2, cand1, cand2, total;
};
__host__ __device__ inline SelectLayout select_layout(int G, int M, int k) {
    auto al = [](size_t v) { return (v + 255) / 256 * 256; };
    const int ng = (G + kSelGroup - 1) / kSelGroup;
    SelectLayout l;
    l.ctr1 = 0;
    l.ctr2 = al((size_t)ng * 4);
    l.cand1 = l.ctr2 + 256;
    l.cand2 = l.cand1 + al((size_t)G * M * k * 8);
    l.total = l.cand2 + al((size_t)ng * M * k * 8);
    return l;
}

struct SelectArgs {
    unsigned char* ws;   // workspace (select_layout)
    int64_t* idx;        // [M, k] selected indices
    uint16_t* vals;      // [M, k] their bf16 values, or null
    int k;
};

__device__ __forceinline__ uint64_t sel_key(uint32_t bits, uint32_t index) {
    bits &= 0xffffu;
    uint32_t o;
    if ((bits & 0x7fffu) > 0x7f80u) {
        o = 0xffffu;                      // NaN: above everything
    } else {
        if (bits == 0x8000u) bits = 0u;   // -0 == +0
        o = (bits & 0x8000u) ? (~bits & 0xffffu) : (bits | 0x8000u);
    }
    return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - index);
}
__device__ __forceinline__ uint32_t sel_index(uint64_t key) { return 0xffffffffu - (uint32_t)key; }
__device__ __forceinline__ uint16_t sel_bits(uint64_t key) {
    const uint32_t o = (uint32_t)(key >> 32);
    if (o == 0xffffu) return 0x7fc0u;
    return (uint16_t)((o & 0x8000u) ? (o & 0x7fffu) : (~o & 0xffffu));
}

// Insert key into a descending list of K keys (a key already present is never
// offered: keys are unique).
template <int K>
__device__ __forceinline__ void topk_insert(uint64_t (&t)[K], uint64_t key) {
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const uint64_t cur = t[i];
        const bool take = key > cur;
        t[i] = take ? key : cur;
        key = take ? cur : key;
    }
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
    const uint32_t lo = __shfl_xor((uint32_t)v, mask);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), mask);
    return ((uint64_t)hi << 32) | lo;
}

// Rows per wave and threads per row for M rows over the workgroup's waves.
__device__ __forceinline__ int sel_threads_per_row(int M, int waves) {
    const int rows_per_wave = (M + waves - 1) / waves;
    int p = 64;
    while (p > 1 && p * rows_per_wave > 64) p >>= 1;
    return p;
}

// Merge, for every row m < M, the lists src[i][m][0..k) (i < L, row stride
// M·k keys) into the top k, handed to emit(m, j, key) for j < k.  All threads
// of the workgroup call this.
template <typename Emit>
__device__ void select_merge(const uint64_t* src, int L, int M, int k, Emit emit) {
    const int waves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int P = sel_threads_per_row(M, waves);
    const int rows_per_wave = 64 / P;
    const int sub = lane / P;       // subgroup in the wave
    const int t = lane - sub * P;   // thread in the subgroup
    for (int m0 = 0; m0 < M; m0 += waves * rows_per_wave) {
        const int m = m0 + wave * rows_per_wave + sub;
        const bool live = m < M;
        uint64_t top[kSelMaxK];
#pragma unroll
        for (int j = 0; j < kSelMaxK; ++j) top[j] = 0;
        if (live) {
            for (int i = t; i < L; i += P) {
                const uint64_t* lst = src + ((size_t)i * M + m) * k;
                for (int j = 0; j < k; ++j) {
                    const uint64_t key = __hip_atomic_load(lst + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (key <= top[kSelMaxK - 1]) break;  // the list is descending
                    topk_insert(top, key);
                }
            }
        }
        // k rounds of a subgroup max; the winner's thread advances its list.
        int head = 0;
        for (int j = 0; j < k; ++j) {
            uint64_t mine = 0;
#pragma unroll
            for (int q = 0; q < kSelMaxK; ++q) mine = (q == head) ? top[q] : mine;
            uint64_t best = mine;
            for (int off = 1; off < P; off <<= 1) {
                const uint64_t o = shfl_xor_u64(best, off);
                best = o > best ? o : best;
            }
            if (live && mine == best && best != 0) ++head;
            if (live && t == 0) emit(m, j, best);
        }
    }
}

// Called by every thread of a workgroup once its per-row top-k lists are in
// cand1 (written by the caller as slot g).  Runs the group and final merges.
__device__ void select_finish(const SelectArgs& sa, int g, int G, int M) {
    __shared__ int stage;
    const SelectLayout l = select_layout(G, M, sa.k);
    uint32_t* ctr1 = reinterpret_cast<uint32_t*>(sa.ws + l.ctr1);
    uint32_t* ctr2 = reinterpret_cast<uint32_t*>(sa.ws + l.ctr2);
    uint64_t* cand1 = reinterpret_cast<uint64_t*>(sa.ws + l.cand1);
    uint64_t* cand2 = reinterpret_cast<uint64_t*>(sa.ws + l.cand2);
    const int ng = (G + kSelGroup - 1) / kSelGroup;
    const int grp = g / kSelGroup;
    const int gsize = (grp + 1) * kSelGroup <= G ? kSelGroup : G - grp * kSelGroup;

    drain_memory();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(ctr1 + grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        stage = prev == (uint32_t)(gsize - 1);
    }
    __syncthreads();
    if (!stage) return;
    // Last of its group: merge the group's lists.
    select_merge(cand1 + (size_t)grp * kSelGroup * M * sa.k, gsize, M, sa.k, [&](int m, int j, uint64_t key) {
        __hip_atomic_store(cand2 + ((size_t)grp * M + m) * sa.k + j, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    });
    drain_memory();
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_store(ctr1 + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t prev = __hip_atomic_fetch_add(ctr2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        stage = prev == (uint32_t)(ng - 1);
    }
    __syncthreads();
    if (!stage) return;
    // Last group: final merge and the outputs.
    select_merge(cand2, ng, M, sa.k, [&](int m, int j, uint64_t key) {
        sa.idx[(int64_t)m * sa.k + j] = key ? (int64_t)sel_index(key) : -1;
        if (sa.vals) sa.vals[(int64_t)m * sa.k + j] = key ? sel_bits(key) : (uint16_t)0xff80u;  // empty: -inf
    });
    if (threadIdx.x == 0) __hip_atomic_store(ctr2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-row top-k of the workgroup's own bf16 outputs vals[m][0..n) (LDS, row
// stride ld, channel c0 + i at column i), written as list g of cand1.  All
// threads call this after the outputs are in LDS and a barrier.
__device__ void select_local(const SelectArgs& sa, const uint16_t* vals, int ld, int n, int c0, int M, int g, int G) {
    const SelectLayout l = select_layout(G, M, sa.k);
    uint64_t* cand1 = reinterpret_cast<uint64_t*>(sa.ws + l.cand1) + (size_t)g * M * sa.k;
    const int waves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int P = sel_threads_per_row(M, waves);
    const int rows_per_wave = 64 / P;
    const int sub = lane / P;
    const int t = lane - sub * P;
    for (int m0 = 0; m0 < M; m0 += waves * rows_per_wave) {
        const int m = m0 + wave * rows_per_wave + sub;
        const bool live = m < M;
        uint64_t top[kSelMaxK];
#pragma unroll
        for (int j = 0; j < kSelMaxK; ++j) top[j] = 0;
        if (live)
            for (int i = t; i < n; i += P) topk_insert(top, sel_key(vals[m * ld + i], (uint32_t)(c0 + i)));
        int head = 0;
        for (int j = 0; j < sa.k; ++j) {
            uint64_t mine = 0;
#pragma unroll
            for (int q = 0; q < kSelMaxK; ++q) mine = (q == head) ? top[q] : mine;
            uint64_t best = mine;
            for (int off = 1; off < P; off <<= 1) {
                const uint64_t o = shfl_xor_u64(best, off);
                best = o > best ? o : best;
            }
            if (live && mine == best && best != 0) ++head;
            if (live && t == 0)
                __hip_atomic_store(cand1 + (size_t)m * sa.k + j, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    select_finish(sa, g, G, M);
}

}  // namespace krk
