// common.h - device helpers shared by the gfx950 kernels (wave64, CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QK_WAVE 64

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

// bf16 -> fp32 is an exact widening: the bf16 bits are the high half.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16 round to nearest even (finite inputs).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t b = __float_as_uint(f);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

// Dot of 8 bf16 weights (one 16-byte load) with 8 fp32 activations.
__device__ __forceinline__ float dot8_bf16(uint4 w, const float *x, float acc) {
    acc = fmaf(bf16_lo(w.x), x[0], acc);
    acc = fmaf(bf16_hi(w.x), x[1], acc);
    acc = fmaf(bf16_lo(w.y), x[2], acc);
    acc = fmaf(bf16_hi(w.y), x[3], acc);
    acc = fmaf(bf16_lo(w.z), x[4], acc);
    acc = fmaf(bf16_hi(w.z), x[5], acc);
    acc = fmaf(bf16_lo(w.w), x[6], acc);
    acc = fmaf(bf16_hi(w.w), x[7], acc);
    return acc;
}

// Streaming 16-byte weight load: each weight byte is used once per step, so
// the load is marked nontemporal to keep it from displacing activations and
// KV lines in the caches.
__device__ __forceinline__ uint4 ld_stream16(const uint16_t *p) {
    const uint4 *q = reinterpret_cast<const uint4 *>(p);
    uint4 v;
    v.x = __builtin_nontemporal_load(&q->x);
    v.y = __builtin_nontemporal_load(&q->y);
    v.z = __builtin_nontemporal_load(&q->z);
    v.w = __builtin_nontemporal_load(&q->w);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, QK_WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, QK_WAVE));
    return v;
}

// Sum over aligned groups of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int m = G / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, QK_WAVE);
    return v;
}

// Argmax order: larger value wins, lower index wins an exact tie.  This is
// the reference's strict '>' over increasing row index (qwen_asr_kernels_avx.c
// :223-226) and the in-order combine of per-thread winners
// (qwen_asr_kernels.c:534-541).
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// SiLU(g) * u as the reference writes it (qwen_asr_kernels.c:930-931).
__device__ __forceinline__ float swiglu1(float g, float u) {
    return (g / (1.0f + expf(-g))) * u;
}
