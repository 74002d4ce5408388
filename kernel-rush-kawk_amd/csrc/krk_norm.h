// Residual add + RMSNorm prologue of the normed projections (gfx950).
//
//   xout = bf16(x + d)
//   n    = bf16( bf16(xout · rstd) · w_norm ),  rstd = 1/sqrt(mean(xout²) + eps)
//
// with the mean of squares accumulated in fp32.  These are the rounding points
// of the reference's fused prologue and of its stand-alone kernel
// (engine/kernels/gemm.py:21-51 _norm_stats/_normed_tile,
// engine/kernels/add_rmsnorm.py:15-29, cast placement
// engine/kernels/rmsnorm.py:34-43: the normalised value rounds to bf16 before
// the weight multiply).  `d` is the branch output the reference calls `y`.
//
// rstd is the correctly rounded fp32 reciprocal square root of the fp32 mean
// plus eps.  Sums of squares are taken in a fixed order (per thread in k
// order, then a fixed butterfly, then waves in order), so results are
// deterministic.
//
// The projection kernels fuse the prologue with these same rounding points:
// each wave of a workgroup owns whole x rows (every k), so it takes a row's
// statistic with a wave butterfly and normalises the row itself before the
// projection consumes it; no workgroup waits for another.
#pragma once

#include "krk_common.h"

namespace krk {

// Operands of the prologue, passed by value to the kernels that apply it.
struct NormArgs {
    const uint16_t* d;   // [M, K] branch output added to x
    int64_t ldd;
    const uint16_t* wn;  // [K] RMSNorm gain
    float eps;
    uint16_t* xout;      // [M, K] bf16(x + d)
    int64_t ldxo;
};

constexpr int kNormThreads = 256;
constexpr int kNormMaxVec = 8;  // 16-byte vectors per thread: K <= 256 * 8 * 8 = 16384

// bf16 bits of 8 elements a + b (fp32 add, one rounding each).
__device__ __forceinline__ u32x4 add_bf16x8(const u32x4& a, const u32x4& b) {
    u32x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t lo = f32_to_bf16(bf16_to_f32(a[j] & 0xffffu) + bf16_to_f32(b[j] & 0xffffu));
        const uint32_t hi = f32_to_bf16(bf16_to_f32(a[j] >> 16) + bf16_to_f32(b[j] >> 16));
        r[j] = lo | (hi << 16);
    }
    return r;
}

// Sum of squares of 8 bf16 values, in element order, added to acc.
__device__ __forceinline__ float sumsq_bf16x8(const u32x4& s, float acc) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float lo = bf16_to_f32(s[j] & 0xffffu);
        const float hi = bf16_to_f32(s[j] >> 16);
        acc = __builtin_fmaf(lo, lo, acc);
        acc = __builtin_fmaf(hi, hi, acc);
    }
    return acc;
}

// bf16 bits of bf16(bf16(s · rstd) · wn) for 8 elements.
__device__ __forceinline__ u32x4 normalize_bf16x8(const u32x4& s, float rstd, const u32x4& wn) {
    u32x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float lo = round_bf16(bf16_to_f32(s[j] & 0xffffu) * rstd) * bf16_to_f32(wn[j] & 0xffffu);
        const float hi = round_bf16(bf16_to_f32(s[j] >> 16) * rstd) * bf16_to_f32(wn[j] >> 16);
        r[j] = f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
    }
    return r;
}

// Two fp32 values -> packed bf16 bits (lo in bits 0-15), round to nearest
// even by gfx950's v_cvt_pk_bf16_f32 (each half the bits f32_to_bf16 gives).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 v;
    v[0] = (__bf16)lo;
    v[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// s = bf16(x + d) for 8 elements; ss += Σ s² (two squares per v_dot2: exact
// bf16 products, fp32 sums, in element order).
__device__ __forceinline__ u32x4 add_sumsq_bf16x8(const u32x4& x, const u32x4& d, float& ss) {
    u32x4 s;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        // Through a scalar: clang reads a vector-element operand of
        // __builtin_bit_cast as element 0 (seen in the gfx950 code).
        const uint32_t sj = pack_bf16x2(bf16_to_f32(x[j] & 0xffffu) + bf16_to_f32(d[j] & 0xffffu),
                                        bf16_to_f32(x[j] >> 16) + bf16_to_f32(d[j] >> 16));
        const bf16x2 sp = __builtin_bit_cast(bf16x2, sj);
        ss = __builtin_amdgcn_fdot2_f32_bf16(sp, sp, ss, false);
        s[j] = sj;
    }
    return s;
}

__device__ __forceinline__ float rms_rstd(float sumsq, int K, float eps) {
    return __frsqrt_rn(sumsq / (float)K + eps);
}

// Stand-alone prologue: one workgroup per row m writes xout[m] and n[m].
// Replaces the reference's add_rms_norm launch (engine/kernels/add_rmsnorm.py:32-43)
// in front of projections that do not fuse it.
__global__ void __launch_bounds__(kNormThreads)
add_rmsnorm_kernel(const uint16_t* __restrict__ x, int64_t ldx, NormArgs a,
                   uint16_t* __restrict__ n, int64_t ldn, int K) {
    __shared__ float red[kNormThreads / 64];
    const int m = blockIdx.x;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const uint16_t* xr = x + (int64_t)m * ldx;
    const uint16_t* dr = a.d + (int64_t)m * a.ldd;
    uint16_t* xo = a.xout + (int64_t)m * a.ldxo;
    uint16_t* nr = n + (int64_t)m * ldn;

    // The gain is loaded with x and d, so the normalisation after the
    // reduction needs no further memory round trip.
    u32x4 s[kNormMaxVec], g[kNormMaxVec];
    float ss = 0.0f;
#pragma unroll
    for (int v = 0; v < kNormMaxVec; ++v) {
        const int k = 8 * (t + kNormThreads * v);
        if (k < K) {
            s[v] = add_bf16x8(*reinterpret_cast<const u32x4*>(xr + k), *reinterpret_cast<const u32x4*>(dr + k));
            g[v] = *reinterpret_cast<const u32x4*>(a.wn + k);
            *reinterpret_cast<u32x4*>(xo + k) = s[v];
            ss = sumsq_bf16x8(s[v], ss);
        }
    }
    // Fixed-order reduction: butterfly within the wave (every lane ends with
    // the same sum), then waves in order.
    wave_fold<1, 32>(&ss, lane);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = red[0];
#pragma unroll
    for (int wv = 1; wv < kNormThreads / 64; ++wv) tot += red[wv];
    const float rstd = rms_rstd(tot, K, a.eps);
#pragma unroll
    for (int v = 0; v < kNormMaxVec; ++v) {
        const int k = 8 * (t + kNormThreads * v);
        if (k < K) *reinterpret_cast<u32x4*>(nr + k) = normalize_bf16x8(s[v], rstd, g[v]);
    }
}

// x in MFMA fragment order (v_mfma_f32_16x16x32_bf16 A operands), as the
// prologue below writes it for the stream kernel (krk_stream.h): byte offset
// of fragment (st, ks, i) of lane `lane`, for 512-k stage st, 32-k step ks
// of that stage and 16-row tile i of MT.  The 64 lanes' 16-byte pieces of
// one fragment are one contiguous 1 KB run (lane (r, q) holds
// x[16i + r][512·st + 32·ks + 8q .. +7]).
constexpr int kFragKC = 512;
__host__ __device__ constexpr size_t frag_offset(int st, int ks, int i, int lane, int MT) {
    return ((((size_t)st * (kFragKC / 32) + ks) * MT + i) * 64 + lane) * 16;
}
// Bytes of x in fragment order: 16·MT rows x whole 512-k stages.
__host__ __device__ constexpr size_t frag_bytes(int MT, int K) {
    return (size_t)MT * 16 * ((K + kFragKC - 1) / kFragKC) * kFragKC * 2;
}

// The stand-alone residual-add + RMSNorm prologue (add_rmsnorm_kernel's
// arithmetic and rounding points) writing the normalised rows in the stream
// kernel's fragment order for MT tiles (frag_offset), so that a normed
// call's stream kernel loads x as whole 1 KB runs and skips its trip through
// LDS.  Workgroup m of 16·MT writes row m: for m < M the normalised row (and
// xout[m]) plus zeros for k from K up to whole 512-k stages; rows past M are
// zeros.
__global__ void __launch_bounds__(kNormThreads)
add_rmsnorm_frag_kernel(const uint16_t* __restrict__ x, int64_t ldx, NormArgs a, unsigned char* __restrict__ nf,
                        int M, int K, int MT) {
    __shared__ float red[kNormThreads / 64];
    const int m = blockIdx.x;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int KP = (K + kFragKC - 1) / kFragKC * kFragKC;
    const int i = m >> 4;
    const int r = m & 15;
    const u32x4 zero{0u, 0u, 0u, 0u};
    auto put = [&](int k, const u32x4& v) {
        const int st = k / kFragKC;
        const int ks = (k % kFragKC) / 32;
        const int q = (k % 32) / 8;
        *reinterpret_cast<u32x4*>(nf + frag_offset(st, ks, i, r + 16 * q, MT)) = v;
    };
    if (m >= M) {  // the whole workgroup: a padding row
        for (int k = 8 * t; k < KP; k += 8 * kNormThreads) put(k, zero);
        return;
    }
    const uint16_t* xr = x + (int64_t)m * ldx;
    const uint16_t* dr = a.d + (int64_t)m * a.ldd;
    uint16_t* xo = a.xout + (int64_t)m * a.ldxo;
    u32x4 s[kNormMaxVec], g[kNormMaxVec];
    float ss = 0.0f;
#pragma unroll
    for (int v = 0; v < kNormMaxVec; ++v) {
        const int k = 8 * (t + kNormThreads * v);
        if (k < K) {
            s[v] = add_bf16x8(*reinterpret_cast<const u32x4*>(xr + k), *reinterpret_cast<const u32x4*>(dr + k));
            g[v] = *reinterpret_cast<const u32x4*>(a.wn + k);
            *reinterpret_cast<u32x4*>(xo + k) = s[v];
            ss = sumsq_bf16x8(s[v], ss);
        }
    }
    for (int k = K + 8 * t; k < KP; k += 8 * kNormThreads) put(k, zero);
    // Fixed-order reduction, as add_rmsnorm_kernel.
    wave_fold<1, 32>(&ss, lane);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = red[0];
#pragma unroll
    for (int wv = 1; wv < kNormThreads / 64; ++wv) tot += red[wv];
    const float rstd = rms_rstd(tot, K, a.eps);
#pragma unroll
    for (int v = 0; v < kNormMaxVec; ++v) {
        const int k = 8 * (t + kNormThreads * v);
        if (k < K) put(k, normalize_bf16x8(s[v], rstd, g[v]));
    }
}

}  // namespace krk
