// Shared device helpers for the gfx950 skinny GEMM kernels: vector types,
// bf16 <-> fp32 conversion and the SwiGLU epilogue arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace krk {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

// bf16 bits -> fp32: exact (bf16 is the top half of an fp32).
__device__ __forceinline__ float bf16_to_f32(uint32_t bits) {
    return __uint_as_float(bits << 16);
}

// fp32 -> bf16 bits, round to nearest even: gfx950's v_cvt_pk_bf16_f32.
// Checked on an MI355X against the integer form
//   u = bits(f); NaN ? (u >> 16) | 0x40 : (u + 0x7fff + ((u >> 16) & 1)) >> 16
// for all 2^32 inputs: identical, NaN payloads included (NaN stays NaN with
// the quiet bit set; infinities and overflow follow IEEE rounding).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    bf16x2 v;
    v[0] = (__bf16)f;
    v[1] = (__bf16)0.0f;
    return __builtin_bit_cast(uint32_t, v) & 0xffffu;
}

__device__ __forceinline__ float round_bf16(float f) {
    return bf16_to_f32(f32_to_bf16(f));
}

// SwiGLU on one (gate, up) accumulator pair with the reference's three bf16
// rounding points (engine/kernels/gemm.py:107-113, engine/kernels/swiglu.py:14-24):
// both projections round to bf16, silu is evaluated in fp32 and rounds to bf16,
// and the product rounds to bf16.  expf is the HIP device library's expf.
__device__ __forceinline__ uint32_t silu_mul_bf16(float g, float u) {
    const float gb = round_bf16(g);
    const float ub = round_bf16(u);
    const float s = round_bf16(gb / (1.0f + expf(-gb)));
    return f32_to_bf16(s * ub);
}

// Wave-wide butterflies in a fixed order (gfx950 permlane swaps across rows,
// DPP within a row): the summation order, and so the result, depends only on
// the lane layout.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Partner of a lane in the butterfly step on bit STEP.  Across rows (32, 16)
// the gfx950 permlane swaps exchange whole rows; within a row DPP row_mirror
// (lane i <-> 15 - i), row_half_mirror (i <-> 7 - i) and quad_perm (i ^ 2,
// i ^ 1).  Each partner differs from the lane in bit STEP.
template <int STEP>
__device__ __forceinline__ float partner(float v) {
    if constexpr (STEP == 8) return dpp_move<0x140>(v);
    if constexpr (STEP == 4) return dpp_move<0x141>(v);
    if constexpr (STEP == 2) return dpp_move<0x4E>(v);
    if constexpr (STEP == 1) return dpp_move<0xB1>(v);
    return v;
}

// Sum of a lane's pair (lo, hi) with its partner's on the bit-STEP step:
// lanes with the bit clear get lo + partner's lo, the others hi + partner's hi.
template <int STEP>
__device__ __forceinline__ float fold_pair(float lo, float hi, int lane) {
    if constexpr (STEP == 32 || STEP == 16) {
        // permlane swap (vdst = lo, src = hi): with the bit clear vdst keeps
        // the lane's lo and src receives the partner's lo; with it set vdst
        // receives the partner's hi and src keeps the lane's hi.
        const auto r = STEP == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false)
                                  : __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
        const bool up = (lane & STEP) != 0;
        const float give = up ? lo : hi;
        const float keep = up ? hi : lo;
        return keep + partner<STEP>(give);
    }
}

// Fold N values per lane across the wave.  While N > 1 each step keeps half of
// the values (the lane's bit STEP picks which half) and adds the partner's
// copy of that half; once N == 1 each step adds the partner's value.
// Afterwards lane l holds the wave sum of value (l >> (6 - p)) & (N0 - 1),
// N0 = 2^p the starting count.
template <int N, int STEP>
__device__ __forceinline__ void wave_fold(float* v, int lane) {
    if constexpr (STEP >= 1) {
        if constexpr (N > 1) {
#pragma unroll
            for (int i = 0; i < N / 2; ++i) v[i] = fold_pair<STEP>(v[i], v[i + N / 2], lane);
            wave_fold<N / 2, STEP / 2>(v, lane);
        } else {
            v[0] = fold_pair<STEP>(v[0], v[0], lane);
            wave_fold<1, STEP / 2>(v, lane);
        }
    }
}

template <int V>
constexpr int log2_exact() {
    static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "power of two up to 64");
    if constexpr (V == 1) {
        return 0;
    } else {
        return 1 + log2_exact<V / 2>();
    }
}

// 16-byte loads.  W is streamed once per call, so its loads carry the
// non-temporal hint; x is re-read by every workgroup and stays cacheable.
__device__ __forceinline__ u32x4 load_stream16(const uint16_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
// Block index i of n with each XCD's blocks adjacent (workgroups go to the 8
// XCDs round robin): XCD x = i mod 8 gets blocks [x·n/8, (x+1)·n/8).  The
// identity unless 8 divides n.
__device__ __forceinline__ int xcd_block(int i, int n) { return (n & 7) == 0 ? (i & 7) * (n >> 3) + (i >> 3) : i; }

__device__ __forceinline__ u32x4 load_cached16(const uint16_t* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

}  // namespace krk
