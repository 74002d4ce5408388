// Shared device helpers for the gfx950 skinny GEMM kernels: vector types,
// bf16 <-> fp32 conversion and the SwiGLU epilogue arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace krk {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
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

// 16-byte loads.  W is streamed once per call, so its loads carry the
// non-temporal hint; x is re-read by every workgroup and stays cacheable.
__device__ __forceinline__ u32x4 load_stream16(const uint16_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x4 load_cached16(const uint16_t* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

}  // namespace krk
