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

// ---------------------------------------------------------------------------
// Cross-lane exchange without the LDS crossbar.  DPP moves operate inside a
// row of 16 lanes at VALU latency; gfx950's v_permlane16_swap /
// v_permlane32_swap exchange rows.  dpp<CTRL>(v): lane i reads lane f(i):
//   0xB1 quad_perm [1,0,3,2] (xor 1)      0x4E quad_perm [2,3,0,1] (xor 2)
//   0x104 row_shl:4 (i+4)   0x114 row_shr:4 (i-4)   0x128 row_ror:8 (xor 8)
//   0x124 row_ror:4   0x140 row_mirror (15 - i)   0x141 row_half_mirror (7 - i
//   within each 8 lanes)
// ---------------------------------------------------------------------------
template <int CTRL, int BANKS = 0xF>
__device__ __forceinline__ float dpp_mov(float old, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, 0xF, BANKS, false));
}

// v of lane f(i) for a CTRL under which every lane reads a lane of its own
// row (quad_perm, row_ror, row_mirror, row_half_mirror).  With old 0 and
// bound_ctrl the compiler folds the move into the VALU op that uses it
// (one v_add_f32_dpp instead of a copy, a v_mov_b32_dpp and a v_add_f32).
template <int CTRL>
__device__ __forceinline__ float dpp_read(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// value of lane (i ^ M) for M in {1, 2, 4, 8}
template <int M>
__device__ __forceinline__ float xor_lane(float v) {
    if (M == 1) return dpp_read<0xB1>(v);
    if (M == 2) return dpp_read<0x4E>(v);
    if (M == 8) return dpp_read<0x128>(v);
    // M == 4: lanes with bit 2 clear read i+4 (banks 0, 2), the others i-4 (banks 1, 3)
    float t = dpp_mov<0x104, 0x5>(v, v);
    return dpp_mov<0x114, 0xA>(t, v);
}

// {v from lanes [0,32) of a, lanes [0,32) of b} / {hi halves}: the two results
// of v_permlane32_swap(a, b); likewise for odd/even rows with permlane16.
__device__ __forceinline__ void swap32(float &a, float &b) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}

__device__ __forceinline__ void swap16(float &a, float &b) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}

// Sum over each aligned group of G lanes (G a power of two <= 64); every lane
// of the group receives the group's sum, the same bits in every lane.  The
// xor 4 and xor 8 steps read through the mirrors: after the xor 1, 2 steps
// every quad is uniform, so lane 7 - i of the 8 holds the value of lane i ^ 4;
// after the xor 4 step every 8 lanes are, so lane 15 - i holds that of i ^ 8.
// Each step is one DPP add.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if (G >= 2) v += xor_lane<1>(v);
    if (G >= 4) v += xor_lane<2>(v);
    if (G >= 8) v += dpp_read<0x141>(v);
    if (G >= 16) v += dpp_read<0x140>(v);
    if (G >= 32) { float a = v, b = v; swap16(a, b); v = a + b; }
    if (G >= 64) { float a = v, b = v; swap32(a, b); v = a + b; }
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

// Maximum over each aligned group of G lanes, steps as group_sum's.
template <int G>
__device__ __forceinline__ float group_max(float v) {
    if (G >= 2) v = fmaxf(v, xor_lane<1>(v));
    if (G >= 4) v = fmaxf(v, xor_lane<2>(v));
    if (G >= 8) v = fmaxf(v, dpp_read<0x141>(v));
    if (G >= 16) v = fmaxf(v, dpp_read<0x140>(v));
    if (G >= 32) { float a = v, b = v; swap16(a, b); v = fmaxf(a, b); }
    if (G >= 64) { float a = v, b = v; swap32(a, b); v = fmaxf(a, b); }
    return v;
}

__device__ __forceinline__ float wave_max(float v) { return group_max<64>(v); }


// p[0] + p[stride] + ... + p[(n - 1) stride], 1 <= n <= N, added left to
// right as a plain loop would; the n loads are issued together, so summing n
// split-K partials costs one memory latency instead of n.
template <int N>
__device__ __forceinline__ float sum_splits(const float *p, int n, long stride) {
    float v[N];
#pragma unroll
    for (int s = 0; s < N; s++) v[s] = s < n ? p[s * stride] : 0.0f;
    float acc = v[0];
#pragma unroll
    for (int s = 1; s < N; s++)
        if (s < n) acc += v[s];
    return acc;
}

template <int N>
__device__ __forceinline__ float2 sum_splits2(const float2 *p, int n, long stride) {
    float2 v[N];
#pragma unroll
    for (int s = 0; s < N; s++) v[s] = s < n ? p[s * stride] : make_float2(0.0f, 0.0f);
    float2 acc = v[0];
#pragma unroll
    for (int s = 1; s < N; s++)
        if (s < n) {
            acc.x += v[s].x;
            acc.y += v[s].y;
        }
    return acc;
}

// max / sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four row groups of an
// MFMA 16 x 16 result that share a column) with row swaps at VALU latency
__device__ __forceinline__ float xor_max16_32(float v) {
    float a = v, b = v;
    swap16(a, b);
    v = fmaxf(a, b);
    a = v;
    b = v;
    swap32(a, b);
    return fmaxf(a, b);
}

__device__ __forceinline__ float xor_sum16_32(float v) {
    float a = v, b = v;
    swap16(a, b);
    v = a + b;
    a = v;
    b = v;
    swap32(a, b);
    return a + b;
}

// Argmax order: larger value wins, lower index wins an exact tie.  This is
// the reference's strict '>' over increasing row index (qwen_asr_kernels_avx.c
// :223-226) and the in-order combine of per-thread winners
// (qwen_asr_kernels.c:534-541).
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// The (value, index) that wins under argmax_better among the 64 lanes, in
// every lane, with no LDS round trip: the xor 1 / 2 partners by quad_perm,
// the xor 4 / 8 partners through the mirrors (each quad, then each 8 lanes,
// hold one winner by then), the xor 16 / 32 partners by the permlane swaps
// (both swap results are offered: one is the lane's own pair).  argmax_better
// is a total order, so the step order does not change the winner.
__device__ __forceinline__ void wave_argmax(float &bv, int &bi) {
    auto take = [&](float ov, float oi) {
        if (argmax_better(ov, __float_as_int(oi), bv, bi)) {
            bv = ov;
            bi = __float_as_int(oi);
        }
    };
    take(xor_lane<1>(bv), xor_lane<1>(__int_as_float(bi)));
    take(xor_lane<2>(bv), xor_lane<2>(__int_as_float(bi)));
    take(dpp_read<0x141>(bv), dpp_read<0x141>(__int_as_float(bi)));
    take(dpp_read<0x140>(bv), dpp_read<0x140>(__int_as_float(bi)));
    {
        float v0 = bv, v1 = bv, i0 = __int_as_float(bi), i1 = __int_as_float(bi);
        swap16(v0, v1);
        swap16(i0, i1);
        take(v0, i0);
        take(v1, i1);
    }
    {
        float v0 = bv, v1 = bv, i0 = __int_as_float(bi), i1 = __int_as_float(bi);
        swap32(v0, v1);
        swap32(i0, i1);
        take(v0, i0);
        take(v1, i1);
    }
}

// SiLU(g) * u as the reference writes it (qwen_asr_kernels.c:930-931), the
// division as a product with the hardware reciprocal (v_rcp_f32, within
// 1 ulp; the reference's -ffast-math build, Makefile:5, does not divide
// exactly either).  g -> -inf: 1 / inf = 0, the reference's -0 as well.
__device__ __forceinline__ float swiglu1(float g, float u) {
    return (g * __builtin_amdgcn_rcpf(1.0f + expf(-g))) * u;
}

// 1 / sqrt(x) of the RMS norms (qwen_asr_kernels.c:783, :846): the hardware
// reciprocal square root (v_rsq_f32, within 1 ulp) instead of a correctly
// rounded square root and division (about 24 dependent instructions on the
// norm's critical path).  The reference's build (-ffast-math, Makefile:5)
// computes 1.0f / sqrtf(x) with an approximate reciprocal square root too.
// x >= eps > 0 here, never denormal.
__device__ __forceinline__ float rsqrt_norm(float x) { return __builtin_amdgcn_rsqf(x); }


// ---------------------------------------------------------------------------
// Row reductions for GEMV tiles.  A wave owning ROWS rows holds one partial
// sum per row in every lane; these fold them across the 64 lanes.
// ---------------------------------------------------------------------------
// One halving step of the transposing reduction over lane bit M: a lane with
// bit M clear keeps values [0, n/2) and gains its partner's copies of them; a
// lane with bit M set keeps [n/2, n).  For M = 32 / 16 one permlane swap of
// (v[i], v[i + n/2]) delivers both halves at once: the sum of the two swap
// results is exactly "own kept value + partner's value of the same row".
template <int N, int M>
__device__ __forceinline__ void transpose_step(float (&v)[N], int n, int lane) {
#pragma unroll
    for (int i = 0; i < N / 2; i++) {
        if (i < n / 2) {
            if (M == 32 || M == 16) {
                float a = v[i], b = v[i + n / 2];
                if (M == 32) swap32(a, b); else swap16(a, b);
                v[i] = a + b;
            } else {
                const bool up = (lane & M) != 0;
                const float keep = up ? v[i + n / 2] : v[i];
                const float send = up ? v[i] : v[i + n / 2];
                v[i] = keep + xor_lane<M>(send);
            }
        }
    }
}

// Reduce ROWS per-lane partials to KEEP values per lane (KEEP = 1 or 2).
// Afterwards every lane of the aligned group of 64*KEEP/ROWS lanes holds the
// totals of rows [KEEP*(lane / (64*KEEP/ROWS)), +KEEP).
template <int ROWS, int KEEP>
__device__ __forceinline__ void reduce_rows(float (&v)[ROWS], int lane) {
    constexpr int T = ROWS / KEEP > 1 ? ROWS / KEEP : 1;   // 2^(number of transposing steps)
    if (T >= 2) transpose_step<ROWS, 32>(v, ROWS, lane);
    if (T >= 4) transpose_step<ROWS, 16>(v, ROWS / 2, lane);
    if (T >= 8) transpose_step<ROWS, 8>(v, ROWS / 4, lane);
    // all-reduce what remains over the lanes below the last transposed bit
    constexpr int G = 64 / T;
#pragma unroll
    for (int i = 0; i < KEEP; i++) v[i] = group_sum<G>(v[i]);
}

// One 128-wide head row held by a 16-lane group: lane c (= lane % 16) owns
// dims 4c .. 4c+3 (lo) and 64+4c .. 64+4c+3 (hi), i.e. four NeoX RoPE pairs
// (d, d + 64).  RMSNorm with weights (wl, wh), then the rotation by (c4, s4)
// (qwen_asr_kernels.c:811-873, :1182-1247).  The sum of squares is this
// lane's 8 squares in pair order, then the 16 lanes' sums (xor 1, 2, 4, 8).
__device__ __forceinline__ void norm_rope_row16(float4 &lo, float4 &hi, float4 wl, float4 wh, float4 c4, float4 s4,
                                                float eps) {
    float ss = fmaf(lo.x, lo.x, hi.x * hi.x);
    ss = fmaf(lo.y, lo.y, ss);
    ss = fmaf(hi.y, hi.y, ss);
    ss = fmaf(lo.z, lo.z, ss);
    ss = fmaf(hi.z, hi.z, ss);
    ss = fmaf(lo.w, lo.w, ss);
    ss = fmaf(hi.w, hi.w, ss);
    ss = group_sum<16>(ss);
    const float rinv = rsqrt_norm(ss / 128.0f + eps);
    const float a0 = (lo.x * wl.x) * rinv, a1 = (lo.y * wl.y) * rinv, a2 = (lo.z * wl.z) * rinv,
                a3 = (lo.w * wl.w) * rinv;
    const float b0 = (hi.x * wh.x) * rinv, b1 = (hi.y * wh.y) * rinv, b2 = (hi.z * wh.z) * rinv,
                b3 = (hi.w * wh.w) * rinv;
    lo = make_float4(fmaf(a0, c4.x, -(b0 * s4.x)), fmaf(a1, c4.y, -(b1 * s4.y)), fmaf(a2, c4.z, -(b2 * s4.z)),
                     fmaf(a3, c4.w, -(b3 * s4.w)));
    hi = make_float4(fmaf(b0, c4.x, a0 * s4.x), fmaf(b1, c4.y, a1 * s4.y), fmaf(b2, c4.z, a2 * s4.z),
                     fmaf(b3, c4.w, a3 * s4.w));
}

// four consecutive elements summed over n split-K partials (stride floats
// apart), each element in split order as sum_splits
template <int N>
__device__ __forceinline__ float4 sum_splits4(const float *p, int n, long stride) {
    float4 v[N];
#pragma unroll
    for (int s = 0; s < N; s++)
        v[s] = s < n ? *reinterpret_cast<const float4 *>(p + s * stride) : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 acc = v[0];
#pragma unroll
    for (int s = 1; s < N; s++)
        if (s < n) {
            acc.x += v[s].x;
            acc.y += v[s].y;
            acc.z += v[s].z;
            acc.w += v[s].w;
        }
    return acc;
}

// one lane pair (l, l+64) of a 128-wide head: RMSNorm with weight, then RoPE
__device__ __forceinline__ void norm_rope_pair(float &x1, float &x2, const float *nw, float eps, float c, float sn,
                                               int lane) {
    float ss = wave_sum(fmaf(x1, x1, x2 * x2));
    const float rinv = rsqrt_norm(ss / 128.0f + eps);
    const float a = (x1 * nw[lane]) * rinv, b = (x2 * nw[lane + 64]) * rinv;
    x1 = fmaf(a, c, -(b * sn));
    x2 = fmaf(b, c, a * sn);
}

