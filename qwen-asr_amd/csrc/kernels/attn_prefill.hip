// attn_prefill.hip - causal GQA attention over many query rows (the prefill
// half of qwen_causal_attention, reference qwen_asr_kernels.c:1050-1141) on
// the bf16 matrix cores of gfx950, fp32-accurate.
//
// Every fp32 operand x is carried as hi = bf16(x) and lo = bf16(x - hi)
// (together ~16 significant bits; |x - hi - lo| <= 2^-17 |x|), and each
// product a.b is taken as hi_a.hi_b + hi_a.lo_b + lo_a.hi_b on
// v_mfma_f32_16x16x32_bf16 with fp32 accumulation: the dropped lo.lo term and
// the split error leave ~2^-16 relative per product, against 2^-24 for fp32
// products, at a fifth of the matrix-core time of v_mfma_f32_16x16x4_f32.
// Softmax statistics, exponentials and the output stay fp32.
//
// Operand layout of the 16x16x32 bf16 MFMA: lane l supplies A[l & 15][8 (l >> 4)
// + i] and B[8 (l >> 4) + i][l & 15], i = 0..7; the result D[4 (l >> 4) + r][l & 15],
// r = 0..3, lands in lane l.
//
// A block owns one kv head, 64 (or 128) consecutive queries of both query
// heads that share it (4 or 8 waves: head = wave & 1, queries 32 (wave >> 1)
// .. + 32) and one split of the key range.  Per 32-key tile staged in LDS (K rows and V^T,
// split into hi / lo once per block):
//   S^T = K Q^T   A = K rows (keys), B = this wave's queries, 32 dims per
//                 k-step; Q is split once, in registers.
//   online softmax per query: a query's 32 scores live in the 4 lanes
//                 l & 15 = query (keys 16 kt + 4 (l >> 4) + r), so the row
//                 max / sum are in-lane over 8 values plus two cross-lane
//                 steps; the rescale factor is lane-local.
//   O^T += V^T P^T  B = the probabilities exactly where S^T left them: k-slot
//                 8 (l >> 4) + i of the MFMA is key 4 (l >> 4) + i (i < 4) and
//                 16 + 4 (l >> 4) + i - 4 (i >= 4), and A = V^T reads the same
//                 keys, so no value crosses lanes.  A V^T row (one dim, 64
//                 bytes) stores the 32 keys in that order, so a lane's 8 keys
//                 are one 16-byte chunk: chunk c of row d sits in slot
//                 c ^ ((d / 2) % 4), and a fragment is one 16-byte read free of
//                 bank conflicts (the swizzle of the ring GEMM's tiles).
// O^T lands as lane l: dims 16 dt + 4 (l >> 4) + r of query l & 15, written
// back as float4 per dt.
//
// Splits: the key range is cut into chunks (a multiple of 32 keys) so the
// launch fills the chip; each split writes unnormalised partials (o[128], m,
// l) and attn_prefill_merge combines them in split order.  Query tiles are
// dispatched longest first (causal tiles grow with the query index).
#include "common.h"
#include "qk_kernels.h"
#include "qwen_asr_hip.h"

#include <math.h>

#define PF_Q 64                   // queries per block (per query head)
#define PF_KT 32                  // keys per LDS tile
// K tile: four 32-dim slices of 32 keys x 64-byte rows (chunk c of key row r
// in slot c ^ ((r / 2) % 4): the fragment reads are the ring GEMM's pattern,
// free of bank conflicts), slices 64 bytes apart beyond their 2 KB so the
// four slices a store instruction touches fall in different banks
#define PF_KSL (PF_KT * 32 + 32)         // bf16 per K slice
#define PF_VLDB PF_KT                     // bf16 row stride of the V^T tiles: 64 B, swizzled chunks
#define PF_MINIT (-1.0e30f)       // running-max start, as the reference's -1e30 (:1069)

typedef float pf_f32x4 __attribute__((ext_vector_type(4)));
typedef float pf_f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 pf_bf16x4 __attribute__((ext_vector_type(4)));

// x = hi + lo + O(2^-17 |x|), hi and lo bf16 (round to nearest even)
__device__ __forceinline__ void pf_split8(pf_f32x8 x, bf16x8 &hi, bf16x8 &lo) {
    hi = __builtin_convertvector(x, bf16x8);
    lo = __builtin_convertvector(x - __builtin_convertvector(hi, pf_f32x8), bf16x8);
}

__device__ __forceinline__ void pf_split4(float4 v, pf_bf16x4 &hi, pf_bf16x4 &lo) {
    const pf_f32x4 x = {v.x, v.y, v.z, v.w};
    hi = __builtin_convertvector(x, pf_bf16x4);
    lo = __builtin_convertvector(x - __builtin_convertvector(hi, pf_f32x4), pf_bf16x4);
}

// hi.hi + hi.lo + lo.hi of one 16x16x32 block
__device__ __forceinline__ f32x4 pf_mfma3(bf16x8 ah, bf16x8 al, bf16x8 bh, bf16x8 bl, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
}

// The next K/V tile, held in registers while the current one is consumed.
// V: lane l of wave w holds dim pf_vdim(w, l, j) of keys 4 pf_vgrp(l) + e: per
// store instruction a wave covers 8 dims x 8 key groups, which the swizzled
// V^T rows take without bank conflicts (the 32 lanes of a half wave land in
// 32 distinct bank pairs).
// NW waves stage a tile (NW = 4 or 8): per thread 16 / NW K float4s and
// 16 / NW V groups of 4 keys.
template <int NW>
struct PfStage {
    float4 k[16 / NW];   // K rows: float4 (tid + 64 NW i): key (.. >> 5), dims 4 (.. & 31)
    float v[64 / NW];    // V: dim pf_vdim<NW>(wave, lane, j), keys 4 pf_vgrp(lane) + e
};

__device__ __forceinline__ int pf_vgrp(int lane) { return (lane >> 2) & 7; }
template <int NW>
__device__ __forceinline__ int pf_vdim(int wave, int lane, int j) {
    return 8 * (wave + NW * j) + (lane & 3) + 4 * (lane >> 5);
}

template <int NW>
__device__ __forceinline__ void pf_load(PfStage<NW> &st, const float *kb, const float *vb, long ps, int k0, int kend,
                                        int tid) {
    constexpr int NI = 16 / NW;
    if (k0 + PF_KT <= kend) {                       // a whole tile (block-uniform): no bounds tests
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int idx = tid + 64 * NW * i;
            st.k[i] = *reinterpret_cast<const float4 *>(kb + (size_t)(k0 + (idx >> 5)) * ps + (idx & 31) * 4);
        }
        const int wave = tid >> 6, lane = tid & 63;
        const float *vr = vb + (size_t)(k0 + 4 * pf_vgrp(lane)) * ps;
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int d = pf_vdim<NW>(wave, lane, j);
#pragma unroll
            for (int e = 0; e < 4; e++) st.v[4 * j + e] = vr[(size_t)e * ps + d];
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int idx = tid + 64 * NW * i, key = k0 + (idx >> 5);
        st.k[i] = key < kend ? *reinterpret_cast<const float4 *>(kb + (size_t)key * ps + (idx & 31) * 4)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const int wave = tid >> 6, lane = tid & 63, g = pf_vgrp(lane);
#pragma unroll
    for (int j = 0; j < NI; j++) {
        const int d = pf_vdim<NW>(wave, lane, j);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int key = k0 + 4 * g + e;
            st.v[4 * j + e] = key < kend ? vb[(size_t)key * ps + d] : 0.0f;
        }
    }
}

__device__ __forceinline__ int pf_kslot(int key, int c) { return key * 32 + 8 * (c ^ ((key >> 1) & 3)); }

template <int NW>
__device__ __forceinline__ void pf_store(const PfStage<NW> &st, __bf16 (*sKh)[PF_KSL], __bf16 (*sKl)[PF_KSL],
                                         __bf16 (*sVh)[PF_VLDB], __bf16 (*sVl)[PF_VLDB], int tid) {
    constexpr int NI = 16 / NW;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int idx = tid + 64 * NW * i;
        pf_bf16x4 h, l;
        pf_split4(st.k[i], h, l);
        // dims 4 (idx & 31) .. + 3 of key idx >> 5: slice (idx & 31) / 8, chunk (idx & 7) / 2, half idx & 1
        const int o = pf_kslot(idx >> 5, (idx & 7) >> 1) + 4 * (idx & 1);
        *reinterpret_cast<pf_bf16x4 *>(&sKh[(idx & 31) >> 3][o]) = h;
        *reinterpret_cast<pf_bf16x4 *>(&sKl[(idx & 31) >> 3][o]) = l;
    }
    // keys 4 g .. 4 g + 3 go to chunk g % 4, half g / 4 of the row (key order
    // of the MFMA's k slots, see the header)
    const int wave = tid >> 6, lane = tid & 63, g = pf_vgrp(lane);
#pragma unroll
    for (int j = 0; j < NI; j++) {
        const int d = pf_vdim<NW>(wave, lane, j);
        const int o = 8 * ((g & 3) ^ ((d >> 1) & 3)) + 4 * (g >> 2);
        pf_bf16x4 h, l;
        pf_split4(make_float4(st.v[4 * j], st.v[4 * j + 1], st.v[4 * j + 2], st.v[4 * j + 3]), h, l);
        *reinterpret_cast<pf_bf16x4 *>(&sVh[d][o]) = h;
        *reinterpret_cast<pf_bf16x4 *>(&sVl[d][o]) = l;
    }
}

// 8 bf16 of V^T row d: keys 4 kq .. + 3 and 16 + 4 kq .. + 3 (the keys of this
// lane's scores), chunk kq of the row
__device__ __forceinline__ bf16x8 pf_vrow(const __bf16 *row, int d, int kq) {
    return *reinterpret_cast<const bf16x8 *>(row + 8 * (kq ^ ((d >> 1) & 3)));
}

__device__ __forceinline__ void pf_write_out(const qk_attn_args &a, size_t base, float4 v) {
    if (a.out) {
        *reinterpret_cast<float4 *>(a.out + base) = v;
    } else {
        const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint16_t hi = f32_to_bf16_rne(e[i]);
            a.out_hi[base + i] = hi;
            a.out_lo[base + i] = f32_to_bf16_rne(e[i] - bf16_to_f32(hi));
        }
    }
}

// NW waves: 16 NW queries per block (64 with 4 waves, two blocks per CU; 128
// with 8 waves, one block per CU, for long unsplit prefills: each staged K/V
// tile, split once, then serves twice the queries)
template <int NW>
__global__ __launch_bounds__(64 * NW, 8 / NW) void attn_prefill(qk_attn_args a) {
    constexpr int QT = 16 * NW;                           // queries per block
    constexpr int hd = QWEN_HIP_HEAD_DIM;
    __shared__ __attribute__((aligned(16))) __bf16 sKh[4][PF_KSL];
    __shared__ __attribute__((aligned(16))) __bf16 sKl[4][PF_KSL];
    __shared__ __attribute__((aligned(16))) __bf16 sVh[hd][PF_VLDB];
    __shared__ __attribute__((aligned(16))) __bf16 sVl[hd][PF_VLDB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ql = lane & 15, kq = lane >> 4;
    const int nq = (a.seq_q + QT - 1) / QT;
    // blocks go out in x order: query tiles longest first, all kv heads of a
    // tile next to each other, so the causal triangle's long tiles start first
    const int t = nq - 1 - (int)blockIdx.x / a.kv_heads;
    const int g = (int)blockIdx.x % a.kv_heads, split = blockIdx.z;
    const int q0 = t * QT;
    const int qn = min(QT, a.seq_q - q0);
    const int kend_tile = min(a.seq_k, a.q_offset + q0 + qn);
    const int ks0 = split * a.chunk;
    if (ks0 >= kend_tile) return;                         // block-uniform
    const int ks1 = min(kend_tile, ks0 + a.chunk);
    const int h = g * 2 + (wave & 1);
    const int qs = q0 + 32 * (wave >> 1);                 // first query of this wave
    const bool wave_on = qs < a.seq_q;
    const int qstride = a.heads * hd;
    const float *kb = a.k + (size_t)g * a.head_stride;
    const float *vb = a.v + (size_t)g * a.head_stride;

    // this lane's query rows (16 per tile qt), dims 32 s + 8 kq .. + 7, split once
    bf16x8 qh[2][4], qo[2][4];
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const int qi = qs + 16 * qt + ql;
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) {
            float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
            if (qi < a.seq_q) {
                const float *qp = a.q + (size_t)qi * qstride + h * hd + 32 * s4 + 8 * kq;
                x0 = *reinterpret_cast<const float4 *>(qp);
                x1 = *reinterpret_cast<const float4 *>(qp + 4);
            }
            pf_split8((pf_f32x8){x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w}, qh[qt][s4], qo[qt][s4]);
        }
    }
    f32x4 o[2][8];
#pragma unroll
    for (int qt = 0; qt < 2; qt++)
#pragma unroll
        for (int dt = 0; dt < 8; dt++) o[qt][dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m[2] = {PF_MINIT, PF_MINIT}, l[2] = {0.f, 0.f};

    PfStage<NW> st;
    pf_load<NW>(st, kb, vb, a.pos_stride, ks0, ks1, tid);
    for (int k0 = ks0; k0 < ks1; k0 += PF_KT) {
        __syncthreads();                                  // previous tile fully consumed
        pf_store<NW>(st, sKh, sKl, sVh, sVl, tid);
        __syncthreads();
        if (k0 + PF_KT < ks1) pf_load<NW>(st, kb, vb, a.pos_stride, k0 + PF_KT, ks1, tid);
        if (!wave_on) continue;

        // scores: s[qt][kt][r] = q(query qs + 16 qt + ql) . k(key k0 + 16 kt + 4 kq + r)
        f32x4 s[2][2];
#pragma unroll
        for (int qt = 0; qt < 2; qt++)
#pragma unroll
            for (int kt = 0; kt < 2; kt++) s[qt][kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) {
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                const int o = pf_kslot(16 * kt + ql, kq);
                const bf16x8 kh = *reinterpret_cast<const bf16x8 *>(&sKh[s4][o]);
                const bf16x8 kl = *reinterpret_cast<const bf16x8 *>(&sKl[s4][o]);
#pragma unroll
                for (int qt = 0; qt < 2; qt++) s[qt][kt] = pf_mfma3(kh, kl, qh[qt][s4], qo[qt][s4], s[qt][kt]);
            }
        }

        // online softmax (causal mask: key <= q_offset + query; keys past ks1 belong elsewhere).
        // A tile wholly below the wave's diagonal and inside the split needs no
        // mask (wave-uniform test; the unmasked scores are the same values).
        // The statistics run in base 2: m holds max(score) * scale * log2(e) and
        // p = 2^(score * scale * log2(e) - m) = e^(score * scale - max), the
        // scale and the subtraction in one fma (the merge takes 2^(m_i - M)).
        const bool open = k0 + PF_KT - 1 <= a.q_offset + qs && k0 + PF_KT <= ks1;
        const float scale2 = a.scale * 1.44269504088896341f;
        float p[2][2][4];
#pragma unroll
        for (int qt = 0; qt < 2; qt++) {
            const int qpos = a.q_offset + qs + 16 * qt + ql;
            float sc[2][4], mx = -INFINITY;
            if (open) {
#pragma unroll
                for (int kt = 0; kt < 2; kt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        sc[kt][r] = s[qt][kt][r];
                        mx = fmaxf(mx, sc[kt][r]);
                    }
            } else {
#pragma unroll
                for (int kt = 0; kt < 2; kt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int key = k0 + 16 * kt + 4 * kq + r;
                        sc[kt][r] = (key <= qpos && key < ks1) ? s[qt][kt][r] : -INFINITY;
                        mx = fmaxf(mx, sc[kt][r]);
                    }
            }
            // scaling by a positive factor keeps the maximum where it is
            mx = xor_max16_32(mx) * scale2;
            const float mn = fmaxf(m[qt], mx);
            const float corr = __builtin_amdgcn_exp2f(m[qt] - mn);
            float sum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    p[qt][kt][r] = __builtin_amdgcn_exp2f(fmaf(sc[kt][r], scale2, -mn));
                    sum += p[qt][kt][r];
                }
            sum = xor_sum16_32(sum);
            l[qt] = fmaf(l[qt], corr, sum);
            m[qt] = mn;
            if (!__all(corr == 1.0f)) {          // the running max moved for some query of the wave
#pragma unroll
                for (int dt = 0; dt < 8; dt++) o[qt][dt] *= corr;
            }
        }

        // O^T[d][query] += V^T[d][key] P^T[key][query]; B = this lane's 8 probabilities
        bf16x8 ph[2], po[2];
#pragma unroll
        for (int qt = 0; qt < 2; qt++)
            pf_split8((pf_f32x8){p[qt][0][0], p[qt][0][1], p[qt][0][2], p[qt][0][3], p[qt][1][0], p[qt][1][1],
                                 p[qt][1][2], p[qt][1][3]},
                      ph[qt], po[qt]);
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const bf16x8 vh = pf_vrow(&sVh[16 * dt + ql][0], 16 * dt + ql, kq);
            const bf16x8 vl = pf_vrow(&sVl[16 * dt + ql][0], 16 * dt + ql, kq);
#pragma unroll
            for (int qt = 0; qt < 2; qt++) o[qt][dt] = pf_mfma3(vh, vl, ph[qt], po[qt], o[qt][dt]);
        }
    }
    if (!wave_on) return;

#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const int qi = qs + 16 * qt + ql;
        if (qi >= a.seq_q) continue;
        if (a.nsplit == 1) {
            const float inv = l[qt] > 0.0f ? 1.0f / l[qt] : 0.0f;
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const f32x4 v = o[qt][dt];
                pf_write_out(a, (size_t)qi * qstride + h * hd + 16 * dt + 4 * kq,
                             make_float4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv));
            }
        } else {
            float *pp = a.part + ((size_t)(split * a.seq_q + qi) * a.heads + h) * QK_PF_PART;
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const f32x4 v = o[qt][dt];
                *reinterpret_cast<float4 *>(pp + 16 * dt + 4 * kq) = make_float4(v[0], v[1], v[2], v[3]);
            }
            if (kq == 0) {
                pp[hd] = m[qt];
                pp[hd + 1] = l[qt];
            }
        }
    }
}

// The splits of one (query, head) combined in split order (max, then
// rescaled sums) for the 4 dims of this lane: NB splits' loads in one round
// trip (splits at or past n read split 0, finite, and weigh 0).
template <int NB>
__device__ __forceinline__ void pf_merge_batch(const float *p0, size_t stride, int s0, int n, int sl, float &M, float &L,
                                               float4 &o, bool first_pass) {
    float mv[NB], lv[NB];
    float4 v[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const bool in = s0 + j < n;
        const float *p = p0 + (in ? s0 + j : 0) * stride;
        mv[j] = in ? p[QWEN_HIP_HEAD_DIM] : PF_MINIT;
        lv[j] = p[QWEN_HIP_HEAD_DIM + 1];
        if (!first_pass) v[j] = *reinterpret_cast<const float4 *>(p + 4 * sl);
    }
    if (first_pass) {                                     // the max over this batch only
#pragma unroll
        for (int j = 0; j < NB; j++) M = fmaxf(M, mv[j]);
        return;
    }
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const float w = s0 + j < n ? __builtin_amdgcn_exp2f(mv[j] - M) : 0.0f;
        L = fmaf(lv[j], w, L);
        o.x = fmaf(v[j].x, w, o.x);
        o.y = fmaf(v[j].y, w, o.y);
        o.z = fmaf(v[j].z, w, o.z);
        o.w = fmaf(v[j].w, w, o.w);
    }
}

// 32 lanes per (query, head), 4 dims each, eight per block: combine the splits
// of the query's tile in split order (max, then rescaled sums), normalise,
// store.  Up to 8 splits take one round trip (the max from the same loads).
__global__ __launch_bounds__(256) void attn_prefill_merge(qk_attn_args a) {
    constexpr int hd = QWEN_HIP_HEAD_DIM;
    const long u = 8L * blockIdx.x + (threadIdx.x >> 5);
    if (u >= (long)a.seq_q * a.heads) return;        // a whole half wave
    const int qi = (int)(u / a.heads), h = (int)(u % a.heads), sl = threadIdx.x & 31;
    const int t = qi / PF_Q;
    const int kend_tile = min(a.seq_k, a.q_offset + min(a.seq_q, (t + 1) * PF_Q));
    const int n = (kend_tile + a.chunk - 1) / a.chunk;
    const size_t stride = (size_t)a.seq_q * a.heads * QK_PF_PART;
    const float *p0 = a.part + ((size_t)qi * a.heads + h) * QK_PF_PART;
    float M = PF_MINIT, L = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    if (n >= 1 && n <= 4) {
        float mv[4], lv[4];
        float4 v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bool in = j < n;
            const float *p = p0 + (in ? j : 0) * stride;
            mv[j] = in ? p[hd] : PF_MINIT;
            lv[j] = p[hd + 1];
            v[j] = *reinterpret_cast<const float4 *>(p + 4 * sl);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) M = fmaxf(M, mv[j]);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float w = j < n ? __builtin_amdgcn_exp2f(mv[j] - M) : 0.0f;
            L = fmaf(lv[j], w, L);
            o.x = fmaf(v[j].x, w, o.x);
            o.y = fmaf(v[j].y, w, o.y);
            o.z = fmaf(v[j].z, w, o.z);
            o.w = fmaf(v[j].w, w, o.w);
        }
    } else if (n >= 5 && n <= 8) {
        float mv[8], lv[8];
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const bool in = j < n;
            const float *p = p0 + (in ? j : 0) * stride;
            mv[j] = in ? p[hd] : PF_MINIT;
            lv[j] = p[hd + 1];
            v[j] = *reinterpret_cast<const float4 *>(p + 4 * sl);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) M = fmaxf(M, mv[j]);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float w = j < n ? __builtin_amdgcn_exp2f(mv[j] - M) : 0.0f;
            L = fmaf(lv[j], w, L);
            o.x = fmaf(v[j].x, w, o.x);
            o.y = fmaf(v[j].y, w, o.y);
            o.z = fmaf(v[j].z, w, o.z);
            o.w = fmaf(v[j].w, w, o.w);
        }
    } else {
        // batches of 8: the max over all splits first, then the sums
        for (int s0 = 0; s0 < n; s0 += 8) pf_merge_batch<8>(p0, stride, s0, n, sl, M, L, o, true);
        for (int s0 = 0; s0 < n; s0 += 8) pf_merge_batch<8>(p0, stride, s0, n, sl, M, L, o, false);
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    const size_t base = (size_t)qi * a.heads * hd + h * hd + 4 * sl;
    const float e[4] = {o.x * inv, o.y * inv, o.z * inv, o.w * inv};
    if (a.out) {
        *reinterpret_cast<float4 *>(a.out + base) = make_float4(e[0], e[1], e[2], e[3]);
    } else {
        uint16_t hh[4], ll[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            hh[i] = f32_to_bf16_rne(e[i]);
            ll[i] = f32_to_bf16_rne(e[i] - bf16_to_f32(hh[i]));
        }
        *reinterpret_cast<uint2 *>(a.out_hi + base) = make_uint2(hh[0] | ((unsigned)hh[1] << 16), hh[2] | ((unsigned)hh[3] << 16));
        *reinterpret_cast<uint2 *>(a.out_lo + base) = make_uint2(ll[0] | ((unsigned)ll[1] << 16), ll[2] | ((unsigned)ll[3] << 16));
    }
}

extern "C" size_t qk_attn_prefill_plan(int seq_q, int seq_k, int q_offset, int heads, int kv_heads, int *chunk,
                                       int *nsplit) {
    const int nq = (seq_q + PF_Q - 1) / PF_Q;
    long tiles = 0;
    int kmax = 0;
    for (int t = 0; t < nq; t++) {
        const int qe = (t + 1) * PF_Q < seq_q ? (t + 1) * PF_Q : seq_q;
        int ke = q_offset + qe;
        if (ke > seq_k) ke = seq_k;
        if (ke > kmax) kmax = ke;
        tiles += (ke + PF_KT - 1) / PF_KT;
    }
    // about QK_PF_TARGET blocks in flight: enough to fill 256 CUs twice over
    long per = (tiles * kv_heads + QK_PF_TARGET - 1) / QK_PF_TARGET;
    if (per < 1) per = 1;
    long c = per * PF_KT;
    // no block walks more than a sixth of the longest query tile (at least 256
    // keys): the causal triangle's longest tiles then end with the rest
    long cap = ((kmax + 5) / 6 + PF_KT - 1) / PF_KT * PF_KT;
    if (cap < 256) cap = 256;
    if (c > cap) c = cap;
    // with several query tiles and up to 2048 keys, splits of a quarter of the
    // longest key range (nearest 32) at least: every split adds partials and a
    // merge pass (7 us at 401 rows), and the tiles themselves already spread
    // the work (C1 401 rows: 96-key splits 26.1 us against 32-key 28.3; C3
    // 1515 rows: 384-key 78.5 us against 224-key ~87, attention + merge)
    if (nq >= 4 && kmax <= 2048) {
        long q4 = (kmax / 4 + PF_KT / 2) / PF_KT * PF_KT;
        if (c < q4) c = q4;
    }
    // one query tile (a short continuation prefill over a long cache): 64-key
    // splits at least, half the partials of 32-key ones for the merge (C5's
    // 31 rows after ~1000 keys: 17.3 -> 15.7 us with the merge)
    if (nq == 1 && c < 2 * PF_KT) c = 2 * PF_KT;
    // with two (query tile, kv head) blocks per CU or more, the longest-first
    // order alone balances the CUs: no split, so no partials and no merge pass
    if ((long)nq * kv_heads >= 2L * 256) c = (kmax + PF_KT - 1) / PF_KT * PF_KT;
    if (c > kmax) c = (kmax + PF_KT - 1) / PF_KT * PF_KT;
    *chunk = (int)c;
    *nsplit = (int)((kmax + c - 1) / c);
    return *nsplit > 1 ? (size_t)*nsplit * seq_q * heads * QK_PF_PART : 0;
}

extern "C" int qk_attn_prefill_launch(const qk_attn_args *a, hipStream_t s) {
    if (!a || a->seq_q <= 0 || a->seq_k <= 0 || a->kv_heads <= 0 || a->heads != 2 * a->kv_heads)
        return QWEN_HIP_EINVAL;
    if (!a->out && (!a->out_hi || !a->out_lo)) return QWEN_HIP_EINVAL;
    if (a->chunk <= 0 || a->chunk % PF_KT || a->nsplit < 1 || (a->nsplit > 1 && !a->part)) return QWEN_HIP_EINVAL;
    const int nq = (a->seq_q + PF_Q - 1) / PF_Q;
    // every key the last query tile sees must fall in some split
    const int kmax = a->seq_k < a->q_offset + a->seq_q ? a->seq_k : a->q_offset + a->seq_q;
    if ((long)a->chunk * a->nsplit < kmax) return QWEN_HIP_EINVAL;
    // unsplit prefills with 128-query tiles enough for every CU: 8-wave blocks
    const int nq8 = (a->seq_q + 127) / 128;
    if (a->nsplit == 1 && (long)nq8 * a->kv_heads >= 256)
        attn_prefill<8><<<dim3(nq8 * a->kv_heads, 1, 1), 512, 0, s>>>(*a);
    else
        attn_prefill<4><<<dim3(nq * a->kv_heads, 1, a->nsplit), 256, 0, s>>>(*a);
    if (a->nsplit > 1)
        attn_prefill_merge<<<(unsigned)(((long)a->seq_q * a->heads + 7) / 8), 256, 0, s>>>(*a);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}
