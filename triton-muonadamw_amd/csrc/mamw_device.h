// Device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mamw_plan.h"

namespace mamw {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// bf16 bit pattern -> fp32 (exact).
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bit pattern, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16x2 (low half = lo), round to nearest even: one
// v_cvt_pk_bf16_f32 for the pair.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Multiply the 8 bf16 values in `v` by `s`, rounding each product to bf16.
__device__ __forceinline__ uint4 scale_bf16x8(uint4 v, float s) {
    uint4 r;
    r.x = pack_bf16x2(bf16_to_f32(v.x & 0xffffu) * s, bf16_to_f32(v.x >> 16) * s);
    r.y = pack_bf16x2(bf16_to_f32(v.y & 0xffffu) * s, bf16_to_f32(v.y >> 16) * s);
    r.z = pack_bf16x2(bf16_to_f32(v.z & 0xffffu) * s, bf16_to_f32(v.z >> 16) * s);
    r.w = pack_bf16x2(bf16_to_f32(v.w & 0xffffu) * s, bf16_to_f32(v.w >> 16) * s);
    return r;
}

// torch.lerp(start, end, weight) with fp32 opmath (ATen's Lerp.h formula):
// small weights interpolate from `start`, large ones from `end`.
__device__ __forceinline__ float lerp_torch(float start, float end, float w) {
    const float d = end - start;
    return fabsf(w) < 0.5f ? __builtin_fmaf(w, d, start) : __builtin_fmaf(w - 1.0f, d, end);
}

// Sum over the 64 lanes of a wavefront (fixed butterfly order: deterministic).
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

}  // namespace mamw
