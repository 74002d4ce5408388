// Output stage shared by the GEMM kernels: bf16 store or SwiGLU epilogue, and
// the deterministic split-K reduction.
//
// Split-K protocol (replaces the reference's second launch, _sum_kernel /
// _sum_gateup_kernel at engine/kernels/gemm.py:96-104 and 160-170, with an
// in-kernel fix-up):
//   * every workgroup (block b, split s) writes its fp32 sums to
//     part[s][m][col] (col indexes W rows: gate cols [0, Nout), up cols
//     [Nout, N) for SILU_MUL);
//   * it waits for those stores to complete and bumps the block's counter;
//   * the workgroup that sees the count reach splits-1 sums the partials in
//     the fixed order s = 0, 1, ..., splits-1 (so the result does not depend
//     on which split finished last), applies the epilogue, stores y and resets
//     the counter to zero for the next call.
//
// Coherence.  The workgroups of one block run on different XCDs, whose L2
// caches are not coherent with each other.  An agent-scope fence
// (__threadfence) makes plain stores visible by writing back and invalidating
// the whole L2 (buffer_wbl2 sc1 / buffer_inv sc1), which costs tens of
// microseconds over a few hundred workgroups.  Instead every access to the
// shared partials is an agent-scope atomic (global_store/global_load with sc1,
// coherent across XCDs on its own), and the only ordering needed — partials
// complete before the counter moves, partial reads after the counter is seen
// — is enforced by s_waitcnt vmcnt(0) before the counter update and by the
// counter's returned value gating the reads.  This is the agent-scope
// release/acquire sequence of the gfx942/gfx950 memory model without the
// L2 maintenance that only non-atomic accesses require.
#pragma once

#include "krk_common.h"

namespace krk {

__device__ __forceinline__ void store_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every memory operation this wave issued has completed; the
// signal fences keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void drain_memory() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <bool SILU>
struct OutStage {
    uint16_t* y;
    int64_t ldy;
    float* part;
    int M, N, Nout, splits, s;

    // One finished element of this workgroup's share: (m, c) output element,
    // g = gate (or plain) sum, u = up sum (SILU only).
    __device__ __forceinline__ void put(int m, int c, float g, float u) const {
        if (splits == 1) {
            const uint32_t v = SILU ? silu_mul_bf16(g, u) : f32_to_bf16(g);
            y[(int64_t)m * ldy + c] = (uint16_t)v;
        } else {
            float* p = part + ((int64_t)s * M + m) * N;
            store_agent(p + c, g);
            if (SILU) store_agent(p + Nout + c, u);
        }
    }
};

// Called by every thread of the workgroup after all put() calls.  `blk` is the
// block's counter index, [c0, c0 + cb) its output channels.
//
// The partials live beyond this XCD's L2, so each load is a full round trip
// (about a microsecond).  The last workgroup therefore issues the loads of
// kBatch splits for kElems elements before it adds anything, and adds them in
// split order afterwards: one round trip per batch instead of one per split.
// The loaded values occupy 2·kBatch·kElems VGPRs, so kernels that call this
// with their main-loop registers still live (the persistent stream kernel)
// use kBatch = kElems = 1.
template <bool SILU, int kBatch = 8, int kElems = 2>
__device__ void splitk_finish(const OutStage<SILU>& o, uint32_t* __restrict__ ctr,
                              int blk, int c0, int cb) {
    __shared__ int is_last;
    drain_memory();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(ctr + blk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = (prev == (uint32_t)(o.splits - 1));
    }
    __syncthreads();
    if (!is_last) return;
    const int n = cb < o.Nout - c0 ? cb : o.Nout - c0;
    const int total = o.M * n;
    const int64_t sstride = (int64_t)o.M * o.N;
    for (int e0 = threadIdx.x; e0 < total; e0 += kElems * blockDim.x) {
        const float* p[kElems];
        float g[kElems], u[kElems];
#pragma unroll
        for (int h = 0; h < kElems; ++h) {
            int e = e0 + h * blockDim.x;
            e = e < total ? e : e0;  // a spare slot re-reads element e0 and is not stored
            const int m = e / n;
            p[h] = o.part + (int64_t)m * o.N + c0 + (e - m * n);
            g[h] = 0.0f;
            u[h] = 0.0f;
        }
        for (int s0 = 0; s0 < o.splits; s0 += kBatch) {
            float gv[kElems][kBatch], uv[kElems][kBatch];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                if (s0 + b < o.splits) {
#pragma unroll
                    for (int h = 0; h < kElems; ++h) {
                        gv[h][b] = load_agent(p[h] + (s0 + b) * sstride);
                        if (SILU) uv[h][b] = load_agent(p[h] + (s0 + b) * sstride + o.Nout);
                    }
                }
            }
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                if (s0 + b < o.splits) {
#pragma unroll
                    for (int h = 0; h < kElems; ++h) {
                        // Split 0 starts the sum (0 + v would turn -0 into +0).
                        g[h] = (s0 + b == 0) ? gv[h][b] : g[h] + gv[h][b];
                        if (SILU) u[h] = (s0 + b == 0) ? uv[h][b] : u[h] + uv[h][b];
                    }
                }
            }
        }
#pragma unroll
        for (int h = 0; h < kElems; ++h) {
            const int e = e0 + h * blockDim.x;
            if (e < total) {
                const int m = e / n;
                const uint32_t v = SILU ? silu_mul_bf16(g[h], u[h]) : f32_to_bf16(g[h]);
                o.y[(int64_t)m * o.ldy + c0 + (e - m * n)] = (uint16_t)v;
            }
        }
    }
    if (threadIdx.x == 0) {
        __hip_atomic_store(ctr + blk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace krk
