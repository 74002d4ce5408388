// Token selection after the lm_head projection: per-row argmax / top-k of the
// bf16 logits (gfx950).
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
// Two sources feed select_rows_kernel:
//   * bf16 logits [M, N] written by a plain projection (top-k, and argmax
//     where the projection is the stream kernel);
//   * for argmax behind the VALU and LDS-staged MFMA projections, one key per
//     row and projection workgroup, written by select_local in the
//     projection's epilogue (its per-workgroup max costs the projection about
//     1%, and the logits are never written).
// select_rows_kernel: workgroup (c, m) reduces chunk c of row m to its top k
// keys (a threshold pass leaves a handful of candidates, ranked in LDS),
// stores them with agent-scope stores and bumps row m's counter; the
// workgroup that sees the count reach chunks-1 ranks the row's lists, writes
// the row's outputs and resets the counter (the protocol of the split-K
// fix-up, krk_epilogue.h).  A row of one chunk writes its outputs directly.
#pragma once

#include "krk_epilogue.h"

namespace krk {

constexpr int kSelMaxK = 8;
constexpr int kSelThreads = 256;
constexpr int kSelVec = 8;                                   // 16-byte logit vectors per thread
constexpr int kSelKeyVec = 2;                                // 16-byte key vectors per thread
constexpr int kSelChunkVals = kSelThreads * kSelVec * 8;     // bf16 logits per workgroup
constexpr int kSelChunkKeys = kSelThreads * kSelKeyVec * 2;  // 64-bit keys per workgroup
constexpr int kSelMaxRows = 64;                              // rows per launch: one counter each
constexpr int kSelCtrStride = 32;                            // counters 128 bytes apart

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

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t umin64(uint64_t a, uint64_t b) { return a > b ? b : a; }

// Insert key into a descending list of K keys (keys are unique).
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

// a <- the K largest of two descending lists a and b, descending: the
// elementwise max of a and reversed b is bitonic and holds the K largest;
// half-cleaners of stride K/2 ... 1 sort it.
template <int K>
__device__ __forceinline__ void merge_sorted(uint64_t (&a)[K], const uint64_t (&b)[K]) {
#pragma unroll
    for (int i = 0; i < K; ++i) a[i] = umax64(a[i], b[K - 1 - i]);
#pragma unroll
    for (int s = K / 2; s >= 1; s >>= 1) {
#pragma unroll
        for (int i = 0; i < K; ++i) {
            if (i & s) continue;
            const uint64_t hi = umax64(a[i], a[i + s]);
            const uint64_t lo = umin64(a[i], a[i + s]);
            a[i] = hi;
            a[i + s] = lo;
        }
    }
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
    const uint32_t lo = __shfl_xor((uint32_t)v, mask);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), mask);
    return ((uint64_t)hi << 32) | lo;
}

// Merge the lists of lanes l ^ 1, ..., l ^ (span/2) into every lane's list.
// Lists longer than one key keep the levels in a loop: the kernels run once
// per workgroup, so straight-line code would be fetched cold.
template <int K>
__device__ __forceinline__ void xor_level(uint64_t (&a)[K], int off) {
    uint64_t b[K];
#pragma unroll
    for (int j = 0; j < K; ++j) b[j] = shfl_xor_u64(a[j], off);
    merge_sorted(a, b);
}
template <int K, int SPAN>
__device__ __forceinline__ void xor_tree(uint64_t (&a)[K]) {
    if constexpr (K == 1) {
#pragma unroll
        for (int off = 1; off < SPAN; off <<= 1) xor_level(a, off);
    } else {
#pragma unroll 1
        for (int off = 1; off < SPAN; off <<= 1) xor_level(a, off);
    }
}

// The workgroup's K largest keys, descending, in every lane of wave 0.
// lds: kSelThreads / 64 * K keys; a barrier separates two calls.
template <int K>
__device__ __forceinline__ void block_top(uint64_t (&a)[K], uint64_t* lds) {
    constexpr int W = kSelThreads / 64;
    xor_tree<K, 64>(a);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < K; ++j) lds[wave * K + j] = a[j];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int j = 0; j < K; ++j) a[j] = lds[(lane & (W - 1)) * K + j];
        xor_tree<K, W>(a);
    }
}

// Per-workgroup argmax in the projection's epilogue: for each row m the
// largest key of the workgroup's bf16 outputs vals[m][0..n) (LDS, row stride
// ld, channel c0 + i at column i) goes to keys[m * ldk + g].  All threads call
// this after the outputs are in LDS and a barrier.  Rows spread over the
// waves; a row takes a subgroup of P lanes (a power of two, no more than the
// channels need).
struct SelectArgs {
    uint64_t* keys;  // [M, ldk] one key per row and projection workgroup
    int64_t ldk;
};

__device__ void select_local(const SelectArgs& sa, const uint16_t* vals, int ld, int n, int c0, int M, int g) {
    const int waves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rows = (M + waves - 1) / waves;  // rows per wave
    int P = 64;
    while (P > 1 && P * rows > 64) P >>= 1;
    while (P > 1 && (P >> 1) >= n) P >>= 1;
    const int sub = lane / P;
    const int t = lane - sub * P;
    for (int m0 = 0; m0 < M; m0 += waves * (64 / P)) {
        const int m = m0 + wave * (64 / P) + sub;
        uint64_t best = 0;
        if (m < M)
            for (int i = t; i < n; i += P) best = umax64(best, sel_key(vals[m * ld + i], (uint32_t)(c0 + i)));
        for (int off = 1; off < P; off <<= 1) best = umax64(best, shfl_xor_u64(best, off));
        if (m < M && t == 0) sa.keys[(int64_t)m * sa.ldk + g] = best;
    }
}

struct RowSelectArgs {
    const void* src;   // [M, ld]: bf16 logits, or 64-bit keys
    int64_t ld;
    int n;             // elements of a row
    int vec;           // rows 16-byte aligned: whole vectors are loaded at once
    uint32_t* ctr;     // row m's counter at ctr[m * kSelCtrStride], zero between calls
    uint64_t* lists;   // [M, chunks, k] per-chunk winners
    int64_t* idx;      // [M, k] selected indices (-1: empty)
    uint16_t* vals;    // [M, k] their bf16 values, or null
    int k;
};

__device__ __forceinline__ void store_agent_u64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_agent_u64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Order-preserving 16-bit images of the two bf16 values packed in w (positive:
// bits | 0x8000, negative: ~bits), two lanes per VALU op.  Unlike sel_key they
// keep NaN payloads and -0 < +0; the filter below allows for both.
typedef __attribute__((ext_vector_type(2))) int16_t i16x2;
typedef __attribute__((ext_vector_type(2))) uint16_t u16x2;
__device__ __forceinline__ u16x2 ord2(uint32_t w) {
    const i16x2 sgn = __builtin_bit_cast(i16x2, w) >> (int16_t)15;  // 0 or -1 per half
    return __builtin_bit_cast(u16x2, w ^ (__builtin_bit_cast(uint32_t, sgn) | 0x80008000u));
}
__device__ __forceinline__ u16x2 max2(u16x2 a, u16x2 b) { return __builtin_elementwise_max(a, b); }
__device__ __forceinline__ u16x2 min2(u16x2 a, u16x2 b) { return __builtin_elementwise_min(a, b); }

// Eight bf16 logits row[e0 .. e0+8) as a vector; positions at or past n read
// as -inf, which neither raises a maximum nor passes for a NaN.
__device__ __forceinline__ u32x4 load_logits8(const uint16_t* row, int64_t e0, int n, int vec) {
    if (vec && e0 + 8 <= n) return *reinterpret_cast<const u32x4*>(row + e0);
    u32x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t lo = e0 + 2 * j < n ? row[e0 + 2 * j] : 0xff80u;
        const uint32_t hi = e0 + 2 * j + 1 < n ? row[e0 + 2 * j + 1] : 0xff80u;
        r[j] = lo | (hi << 16);
    }
    return r;
}

constexpr int kSelGroupLanes = 8;                       // lanes per maximum of the threshold pass
constexpr int kSelGroups = kSelThreads / kSelGroupLanes;
constexpr int kSelCap = 256;                            // LDS candidate slots
constexpr uint32_t kOrdNegInf = 0x007fu;                // ord2 image of -inf; NaN images lie outside
constexpr uint32_t kOrdPosInf = 0xff80u;                // [kOrdNegInf, kOrdPosInf]

// Wave 0: the k largest of the cnt distinct keys cand[0..cnt) (LDS) into
// res[0..k) (LDS), descending, 0 where fewer.  A key's slot is its rank, the
// number of larger keys; LDS accesses of one wave complete in order, so the
// zeroing lands before the ranked stores.
__device__ __forceinline__ void rank_select(const uint64_t* cand, int cnt, int k, uint64_t* res) {
    const int lane = threadIdx.x & 63;
    if (lane < k) res[lane] = 0;
    for (int i = lane; i < cnt; i += 64) {
        const uint64_t mine = cand[i];
        int rank = 0;
        for (int j = 0; j < cnt; ++j) rank += cand[j] > mine ? 1 : 0;
        if (rank < k) res[rank] = mine;
    }
}

// Grid (chunks, M): KM = 1 (argmax) or kSelMaxK (top-k, k <= KM); KEYS: src
// holds keys (one per row and projection workgroup for argmax, kSelMaxK per
// workgroup for top-k) instead of bf16 logits.
//
// Logits: a chunk of kSelChunkVals values, kSelVec 16-byte vectors per thread
// held in registers.  Pass 1 takes the ord2 maximum of every group of
// kSelGroupLanes lanes; the k-th largest group maximum T is a value that at
// least k distinct elements reach, so every element of the chunk's top k has
// ord2 >= T - 1 (ord2 differs from the exact order only by -0 < +0, one step
// apart, and by NaN payloads, handled below).  Pass 2 appends the few
// elements at or above T - 1 to an LDS list as exact keys, and rank_select
// picks the chunk's top k from it.  A chunk holding a NaN, or more than
// kSelCap candidates (heavy ties), takes the exact path instead: every
// thread inserts its keys into a sorted list and the lists meet in block_top.
template <int KM, bool KEYS>
__global__ void __launch_bounds__(kSelThreads) select_rows_kernel(RowSelectArgs a) {
    __shared__ uint64_t lds[kSelThreads / 64 * KM];
    __shared__ uint64_t cand[kSelCap];
    __shared__ uint64_t res[kSelMaxK];
    __shared__ uint32_t gmax[kSelGroups];
    __shared__ uint32_t thr;
    __shared__ int ncand;
    __shared__ int last;
    const int c = blockIdx.x;
    const int m = blockIdx.y;
    const int C = gridDim.x;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int k = a.k;
    uint64_t top[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) top[j] = 0;
    bool in_res = false;  // the chunk's winners are in res[] (else in top[] of wave 0)

    if constexpr (KEYS) {
        const uint64_t* row = static_cast<const uint64_t*>(a.src) + (int64_t)m * a.ld;
        uint64_t v[kSelKeyVec][2];
#pragma unroll
        for (int u = 0; u < kSelKeyVec; ++u) {
            const int64_t e = (int64_t)c * kSelChunkKeys + 2 * (u * kSelThreads + t);
            if (a.vec && e + 2 <= a.n) {
                const u32x4 q = *reinterpret_cast<const u32x4*>(row + e);
                v[u][0] = ((uint64_t)q[1] << 32) | q[0];
                v[u][1] = ((uint64_t)q[3] << 32) | q[2];
            } else {
                v[u][0] = e < a.n ? row[e] : 0;
                v[u][1] = e + 1 < a.n ? row[e + 1] : 0;
            }
        }
#pragma unroll
        for (int u = 0; u < kSelKeyVec; ++u) {
            if constexpr (KM == 1) {
                top[0] = umax64(top[0], umax64(v[u][0], v[u][1]));
            } else {
                topk_insert(top, v[u][0]);
                topk_insert(top, v[u][1]);
            }
        }
        block_top(top, lds);
    } else {
        const uint16_t* row = static_cast<const uint16_t*>(a.src) + (int64_t)m * a.ld;
        const int64_t base = (int64_t)c * kSelChunkVals;
        u32x4 v[kSelVec];
#pragma unroll
        for (int u = 0; u < kSelVec; ++u) v[u] = load_logits8(row, base + 8 * (u * kSelThreads + t), a.n, a.vec);
        // Pass 1: ord2 maximum and minimum (a NaN shows as one above +inf or
        // one below -inf).
        u16x2 mx = ord2(v[0][0]), mn = mx;
#pragma unroll
        for (int u = 0; u < kSelVec; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u16x2 o = ord2(v[u][j]);
                mx = max2(mx, o);
                mn = min2(mn, o);
            }
        uint32_t gm = mx[0] > mx[1] ? mx[0] : mx[1];
        const uint32_t lo = mn[0] < mn[1] ? mn[0] : mn[1];
#pragma unroll
        for (int off = 1; off < kSelGroupLanes; off <<= 1) {
            const uint32_t o = __shfl_xor(gm, off);
            gm = o > gm ? o : gm;
        }
        if ((lane & (kSelGroupLanes - 1)) == 0) gmax[t / kSelGroupLanes] = gm;
        if (t == 0) ncand = 0;
        const bool nan = __syncthreads_or(gm > kOrdPosInf || lo < kOrdNegInf);
        if (t < 64) {
            // T: the k-th largest group maximum (ties ranked by group index).
            uint32_t mine = t < kSelGroups ? gmax[t] : 0u;
            int rank = 0;
#pragma unroll 8
            for (int j = 0; j < kSelGroups; ++j) {
                const uint32_t o = gmax[j];
                rank += (o > mine || (o == mine && j < t)) ? 1 : 0;
            }
            if (t < kSelGroups && rank == k - 1) thr = nan ? 0u : mine;
        }
        __syncthreads();
        const uint32_t T = thr;
        // Pass 2: candidates at or above T - 1, as exact keys.  The vectors
        // holding one are rare; a loop reloads them (from cache) rather than
        // index the register array, so the hot path stays short.
        uint32_t hit = 0;
#pragma unroll
        for (int u = 0; u < kSelVec; ++u) {
            const u16x2 q = max2(max2(ord2(v[u][0]), ord2(v[u][1])), max2(ord2(v[u][2]), ord2(v[u][3])));
            const uint32_t qm = q[0] > q[1] ? q[0] : q[1];
            hit |= (qm + 1 >= T ? 1u : 0u) << u;
        }
#pragma unroll 1
        while (hit) {
            const int u = __builtin_ctz(hit);
            hit &= hit - 1;
            const int64_t e0 = base + 8 * (u * kSelThreads + t);
            const u32x4 q = load_logits8(row, e0, a.n, a.vec);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t bits = (q[j >> 1] >> (16 * (j & 1))) & 0xffffu;
                if (e0 + j < a.n && (uint32_t)ord2(bits)[0] + 1 >= T) {
                    const int slot = atomicAdd(&ncand, 1);
                    if (slot < kSelCap) cand[slot] = sel_key(bits, (uint32_t)(e0 + j));
                }
            }
        }
        __syncthreads();
        const int cnt = ncand;
        if (cnt <= kSelCap) {
            if (t < 64) rank_select(cand, cnt, k, res);
            in_res = true;
        } else {
            // Exact path: every position at or above T - 1 (all, after a NaN).
#pragma unroll 1
            for (int u = 0; u < kSelVec; ++u) {
                const int64_t e0 = base + 8 * (u * kSelThreads + t);
                const u32x4 q = load_logits8(row, e0, a.n, a.vec);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t bits = (q[j >> 1] >> (16 * (j & 1))) & 0xffffu;
                    if (e0 + j < a.n && (uint32_t)ord2(bits)[0] + 1 >= T) {
                        const uint64_t key = sel_key(bits, (uint32_t)(e0 + j));
                        if constexpr (KM == 1) top[0] = umax64(top[0], key);
                        else topk_insert(top, key);
                    }
                }
            }
            block_top(top, lds);
        }
    }
    // The chunk's winners, in the first k lanes of wave 0: lane j holds the
    // j-th (0 past them).
    uint64_t win = 0;
    if (t < 64) {
        if (in_res) {
            win = lane < k ? res[lane] : 0;
        } else {
#pragma unroll
            for (int j = 0; j < KM; ++j) win = lane == j ? top[j] : win;
        }
    }

    auto emit = [&](uint64_t key) {
        a.idx[(int64_t)m * k + lane] = key ? (int64_t)sel_index(key) : -1;
        if (a.vals) a.vals[(int64_t)m * k + lane] = key ? sel_bits(key) : (uint16_t)0xff80u;  // empty: -inf
    };
    if (C == 1) {
        if (t < k) emit(win);
        return;
    }
    if (t < 64) {
        if (lane < k) store_agent_u64(a.lists + ((int64_t)m * C + c) * k + lane, win);
        drain_memory();
        if (t == 0) {
            const uint32_t prev =
                __hip_atomic_fetch_add(a.ctr + m * kSelCtrStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = prev == (uint32_t)(C - 1);
        }
    }
    __syncthreads();
    if (!last) return;
    // The row's last workgroup: the top k of the C lists.
    const int total = C * k;
    if (total <= kSelCap) {
        for (int i = t; i < total; i += kSelThreads) cand[i] = load_agent_u64(a.lists + (int64_t)m * total + i);
        __syncthreads();
        if (t < 64) {
            rank_select(cand, total, k, res);
            if (lane < k) win = res[lane];
        }
    } else {
#pragma unroll
        for (int j = 0; j < KM; ++j) top[j] = 0;
        for (int i = t; i < C; i += kSelThreads) {
            const uint64_t* src = a.lists + ((int64_t)m * C + i) * k;
            uint64_t b[KM];
#pragma unroll
            for (int j = 0; j < KM; ++j) b[j] = j < k ? load_agent_u64(src + j) : 0;
            merge_sorted(top, b);
        }
        block_top(top, lds);
        if (t < 64) {
            win = 0;
#pragma unroll
            for (int j = 0; j < KM; ++j) win = lane == j ? top[j] : win;
        }
    }
    if (t < k) emit(win);
    if (t == 0) __hip_atomic_store(a.ctr + m * kSelCtrStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace krk
