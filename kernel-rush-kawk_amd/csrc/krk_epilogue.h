// Output stage shared by the GEMM kernels: bf16 store or SwiGLU epilogue, and
// the deterministic split-K reduction.
//
// Split-K protocol (replaces the reference's second launch, _sum_kernel /
// _sum_gateup_kernel at engine/kernels/gemm.py:96-104 and 160-170, with an
// in-kernel fix-up):
//   * every workgroup (block b, split s) writes its fp32 sums to
//     part[s][m][col] (col indexes W rows: gate cols [0, Nout), up cols
//     [Nout, N) for SILU_MUL);
//   * it then releases (agent-scope fence) and bumps the block's counter;
//   * the workgroup that sees the count reach splits-1 acquires, sums the
//     partials in the fixed order s = 0, 1, ..., splits-1 (so the result does
//     not depend on which split finished last), applies the epilogue, stores
//     y and resets the counter to zero for the next call.
#pragma once

#include "krk_common.h"

namespace krk {

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
            p[c] = g;
            if (SILU) p[Nout + c] = u;
        }
    }
};

// Called by every thread of the workgroup after all put() calls.  `blk` is the
// block's counter index, [c0, c0 + cb) its output channels.
template <bool SILU>
__device__ void splitk_finish(const OutStage<SILU>& o, uint32_t* __restrict__ ctr,
                              int blk, int c0, int cb) {
    __shared__ int is_last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = atomicAdd(ctr + blk, 1u);
        is_last = (prev == (uint32_t)(o.splits - 1));
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    const int n = cb < o.Nout - c0 ? cb : o.Nout - c0;
    const int64_t sstride = (int64_t)o.M * o.N;
    for (int e = threadIdx.x; e < o.M * n; e += blockDim.x) {
        const int m = e / n;
        const int c = c0 + (e - m * n);
        const float* p = o.part + (int64_t)m * o.N + c;
        float g = p[0];
        float u = SILU ? p[o.Nout] : 0.0f;
        for (int s = 1; s < o.splits; ++s) {
            g += p[s * sstride];
            if (SILU) u += p[s * sstride + o.Nout];
        }
        const uint32_t v = SILU ? silu_mul_bf16(g, u) : f32_to_bf16(g);
        o.y[(int64_t)m * o.ldy + c] = (uint16_t)v;
    }
    if (threadIdx.x == 0) {
        __hip_atomic_store(ctr + blk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace krk
