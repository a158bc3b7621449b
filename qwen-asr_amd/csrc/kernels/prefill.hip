// prefill.hip - dense kernels of the multi-row prefill (gfx950 MFMA) and the
// elementwise operators of the op-level ABI.
//
// The reference prefill multiplies fp32 activations by bf16-exact weights in
// fp32 SGEMM (qwen_linear_nobias_bf16 -> bf16_get_f32_view -> cblas_sgemm,
// qwen_asr_kernels.c:462-472, :199-202).  Here the weights stay bf16 (they are
// exact) and each fp32 activation v is carried as two bf16 terms,
// hi = bf16(v) and lo = bf16(v - hi), so one tile step issues two bf16 MFMAs
// (hi.W and lo.W) into the same fp32 accumulator.  hi + lo represents v to
// about 2^-17 relative, close to the fp32 GEMM the reference runs.
#include "common.h"
#include "qk_kernels.h"
#include "qwen_asr_hip.h"

#include <math.h>

__device__ __forceinline__ void split2(float v, uint16_t &hi, uint16_t &lo) {
    hi = f32_to_bf16_rne(v);
    lo = f32_to_bf16_rne(v - bf16_to_f32(hi));
}

// sum over the NW waves of a block (red: NW floats of LDS)
template <int NW>
__device__ __forceinline__ float block_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; i++) s += red[i];
    return s;
}

__device__ __forceinline__ float block_sum256(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// ---------------------------------------------------------------------------
// RMSNorm (qwen_asr_kernels.c:750-809) writing the bf16 hi/lo split the GEMM
// consumes.  One block per row.  With nsum > 0 the row is first completed
// in place: x += part[0] + ... + part[nsum-1] (the split-K partials of the
// projection that produced it, summed in split order), which is the
// residual add of qwen_asr_decoder.c:318 / :331.
// ---------------------------------------------------------------------------
// 1024 threads per row: each thread's split partials are one batch of loads
// (D = 1024: one element per thread), so the row costs one memory latency.
#define RN_THREADS 1024
__global__ __launch_bounds__(RN_THREADS) void rmsnorm_split(float *x, const float *part, int nsum, long pstride,
                                                            const float *w, int D, float eps, uint16_t *hi,
                                                            uint16_t *lo) {
    __shared__ float red[RN_THREADS / 64];
    float *xr = x + (size_t)blockIdx.x * D;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < D; i += RN_THREADS) {
        float v = xr[i];
        if (nsum) {
            v += sum_splits<QK_GEMM_MAX_SPLIT>(part + (size_t)blockIdx.x * D + i, nsum, pstride);
            xr[i] = v;
        }
        ss = fmaf(v, v, ss);
    }
    float rinv = 1.0f;
    if (w) {
        ss = block_sum<RN_THREADS / 64>(ss, red);
        rinv = rsqrt_norm(ss / (float)D + eps);
    }
    if (!hi) return;
    uint16_t *h = hi + (size_t)blockIdx.x * D, *l = lo + (size_t)blockIdx.x * D;
    for (int i = threadIdx.x; i < D; i += RN_THREADS) {   // each thread re-reads only what it wrote
        const float v = w ? (xr[i] * w[i]) * rinv : xr[i];
        split2(v, h[i], l[i]);
    }
}

// Tall inputs: one wave per row, four rows per block, D / 64 elements per
// lane in 16-byte pieces (lane l holds elements 256 j + 4 l .. + 3); partials
// are summed in split order and then added, as above.
template <int Q>
__global__ __launch_bounds__(256) void rmsnorm_split_rows(float *x, const float *part, int nsum, long pstride,
                                                          const float *w, int S, float eps, uint16_t *hi,
                                                          uint16_t *lo) {
    constexpr int D = 256 * Q;
    const int row = 4 * blockIdx.x + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= S) return;                                   // whole wave
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)row * D) + lane;
    // the weights first: their loads pass under the row's
    float4 wv[Q];
    const float4 *w4 = w ? reinterpret_cast<const float4 *>(w) + lane : nullptr;
#pragma unroll
    for (int j = 0; j < Q; j++) wv[j] = w ? w4[64 * j] : make_float4(1.f, 1.f, 1.f, 1.f);
    float4 v[Q];
#pragma unroll
    for (int j = 0; j < Q; j++) v[j] = xr[64 * j];
    if (nsum) {
        const float4 *pr = reinterpret_cast<const float4 *>(part + (size_t)row * D) + lane;
        const long ps4 = pstride / 4;
        float4 ps[Q];
#pragma unroll
        for (int j = 0; j < Q; j++) ps[j] = pr[64 * j];
        for (int sp = 1; sp < nsum; sp += 2) {          // two splits' loads per round trip, summed in order
            const bool two = sp + 1 < nsum;
            float4 a[Q], b[Q];
#pragma unroll
            for (int j = 0; j < Q; j++) {
                a[j] = pr[sp * ps4 + 64 * j];
                b[j] = two ? pr[(sp + 1) * ps4 + 64 * j] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int j = 0; j < Q; j++) {
                ps[j].x += a[j].x; ps[j].y += a[j].y; ps[j].z += a[j].z; ps[j].w += a[j].w;
                if (two) { ps[j].x += b[j].x; ps[j].y += b[j].y; ps[j].z += b[j].z; ps[j].w += b[j].w; }
            }
        }
#pragma unroll
        for (int j = 0; j < Q; j++) {
            v[j].x += ps[j].x; v[j].y += ps[j].y; v[j].z += ps[j].z; v[j].w += ps[j].w;
            xr[64 * j] = v[j];
        }
    }
    float rinv = 1.0f;
    if (w) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < Q; j++) {
            ss = fmaf(v[j].x, v[j].x, ss);
            ss = fmaf(v[j].y, v[j].y, ss);
            ss = fmaf(v[j].z, v[j].z, ss);
            ss = fmaf(v[j].w, v[j].w, ss);
        }
        ss = wave_sum(ss);
        rinv = rsqrt_norm(ss / (float)D + eps);
    }
    if (!hi) return;
    uint2 *h = reinterpret_cast<uint2 *>(hi + (size_t)row * D) + lane;
    uint2 *l = reinterpret_cast<uint2 *>(lo + (size_t)row * D) + lane;
#pragma unroll
    for (int j = 0; j < Q; j++) {
        const float4 ww = wv[j];
        const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w}, we[4] = {ww.x, ww.y, ww.z, ww.w};
        uint16_t hh[4], ll[4];
#pragma unroll
        for (int k = 0; k < 4; k++) split2(w ? (e[k] * we[k]) * rinv : e[k], hh[k], ll[k]);
        h[64 * j] = make_uint2(hh[0] | ((unsigned)hh[1] << 16), hh[2] | ((unsigned)hh[3] << 16));
        l[64 * j] = make_uint2(ll[0] | ((unsigned)ll[1] << 16), ll[2] | ((unsigned)ll[3] << 16));
    }
}

// D = EPT * RN_THREADS: the same sums and products as rmsnorm_split, with
// the row and the weights held in registers (one memory round trip fewer)
template <int EPT>
__global__ __launch_bounds__(RN_THREADS) void rmsnorm_split_reg(float *x, const float *part, int nsum, long pstride,
                                                                const float *w, float eps, uint16_t *hi,
                                                                uint16_t *lo) {
    constexpr int D = EPT * RN_THREADS;
    __shared__ float red[RN_THREADS / 64];
    float *xr = x + (size_t)blockIdx.x * D;
    float v[EPT], wv[EPT];
#pragma unroll
    for (int e = 0; e < EPT; e++) {
        const int i = threadIdx.x + e * RN_THREADS;
        v[e] = xr[i];
        wv[e] = w ? w[i] : 1.0f;
    }
    if (nsum) {
#pragma unroll
        for (int e = 0; e < EPT; e++) {
            const int i = threadIdx.x + e * RN_THREADS;
            v[e] += sum_splits<QK_GEMM_MAX_SPLIT>(part + (size_t)blockIdx.x * D + i, nsum, pstride);
            xr[i] = v[e];
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < EPT; e++) ss = fmaf(v[e], v[e], ss);
    float rinv = 1.0f;
    if (w) {
        ss = block_sum<RN_THREADS / 64>(ss, red);
        rinv = rsqrt_norm(ss / (float)D + eps);
    }
    if (!hi) return;
    uint16_t *h = hi + (size_t)blockIdx.x * D, *l = lo + (size_t)blockIdx.x * D;
#pragma unroll
    for (int e = 0; e < EPT; e++) {
        const int i = threadIdx.x + e * RN_THREADS;
        split2(w ? (v[e] * wv[e]) * rinv : v[e], h[i], l[i]);
    }
}

// One 256-thread block per row, 4 consecutive elements per thread and
// 16-byte piece (D = 1024 V4): the same sums and products as rmsnorm_split
// (partials in split order, each split's loads issued together), a
// four-wave reduction of the squares.
template <int V4>
__global__ __launch_bounds__(256) void rmsnorm_split_vec(float *x, const float *part, int nsum, long pstride,
                                                         const float *w, float eps, uint16_t *hi, uint16_t *lo) {
    constexpr int D = 1024 * V4;
    __shared__ float red[4];
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)blockIdx.x * D) + threadIdx.x;
    // the weights first: their loads pass under the row's
    float4 wv[V4];
    const float4 *w4 = w ? reinterpret_cast<const float4 *>(w) + threadIdx.x : nullptr;
#pragma unroll
    for (int e = 0; e < V4; e++) wv[e] = w ? w4[256 * e] : make_float4(1.f, 1.f, 1.f, 1.f);
    float4 v[V4];
#pragma unroll
    for (int e = 0; e < V4; e++) v[e] = xr[256 * e];
    if (nsum) {
        const float4 *pr = reinterpret_cast<const float4 *>(part + (size_t)blockIdx.x * D) + threadIdx.x;
        const long ps4 = pstride / 4;
#pragma unroll
        for (int e = 0; e < V4; e++) {
            float4 q[QK_GEMM_MAX_SPLIT];
#pragma unroll
            for (int sp = 0; sp < QK_GEMM_MAX_SPLIT; sp++)
                q[sp] = sp < nsum ? pr[sp * ps4 + 256 * e] : make_float4(0.f, 0.f, 0.f, 0.f);
            float4 acc = q[0];
#pragma unroll
            for (int sp = 1; sp < QK_GEMM_MAX_SPLIT; sp++)
                if (sp < nsum) { acc.x += q[sp].x; acc.y += q[sp].y; acc.z += q[sp].z; acc.w += q[sp].w; }
            v[e].x += acc.x; v[e].y += acc.y; v[e].z += acc.z; v[e].w += acc.w;
            xr[256 * e] = v[e];
        }
    }
    float rinv = 1.0f;
    if (w) {
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < V4; e++) {
            ss = fmaf(v[e].x, v[e].x, ss);
            ss = fmaf(v[e].y, v[e].y, ss);
            ss = fmaf(v[e].z, v[e].z, ss);
            ss = fmaf(v[e].w, v[e].w, ss);
        }
        ss = block_sum<4>(ss, red);
        rinv = rsqrt_norm(ss / (float)D + eps);
    }
    if (!hi) return;
    uint2 *h = reinterpret_cast<uint2 *>(hi + (size_t)blockIdx.x * D) + threadIdx.x;
    uint2 *l = reinterpret_cast<uint2 *>(lo + (size_t)blockIdx.x * D) + threadIdx.x;
#pragma unroll
    for (int e = 0; e < V4; e++) {
        const float4 ww = wv[e];
        const float el[4] = {v[e].x, v[e].y, v[e].z, v[e].w}, we[4] = {ww.x, ww.y, ww.z, ww.w};
        uint16_t hh[4], ll[4];
#pragma unroll
        for (int k = 0; k < 4; k++) split2(w ? (el[k] * we[k]) * rinv : el[k], hh[k], ll[k]);
        h[256 * e] = make_uint2(hh[0] | ((unsigned)hh[1] << 16), hh[2] | ((unsigned)hh[3] << 16));
        l[256 * e] = make_uint2(ll[0] | ((unsigned)ll[1] << 16), ll[2] | ((unsigned)ll[3] << 16));
    }
}

extern "C" int qk_rmsnorm_split_launch(float *x, const float *part, int nsum, long pstride, const float *w, int S,
                                       int D, float eps, uint16_t *hi, uint16_t *lo, hipStream_t s) {
    if (S <= 0 || D <= 0 || !x || nsum < 0 || nsum > QK_GEMM_MAX_SPLIT || (nsum && !part) || (!hi) != (!lo) ||
        (!hi && !nsum))
        return QWEN_HIP_EINVAL;
    const bool a16 = ((uintptr_t)x | (uintptr_t)part | (uintptr_t)w) % 16 == 0 && (uintptr_t)hi % 8 == 0 &&
                     (uintptr_t)lo % 8 == 0 && (nsum <= 1 || pstride % 4 == 0);
    if (S >= 1024 && (D == 1024 || D == 2048) && a16) {
        // tall inputs: a wave per row keeps the grid at S / 4 blocks
        const unsigned blocks = (unsigned)((S + 3) / 4);
        if (D == 1024) rmsnorm_split_rows<4><<<blocks, 256, 0, s>>>(x, part, nsum, pstride, w, S, eps, hi, lo);
        else rmsnorm_split_rows<8><<<blocks, 256, 0, s>>>(x, part, nsum, pstride, w, S, eps, hi, lo);
    } else if ((D == 1024 || D == 2048) && a16) {
        if (D == 1024) rmsnorm_split_vec<1><<<S, 256, 0, s>>>(x, part, nsum, pstride, w, eps, hi, lo);
        else rmsnorm_split_vec<2><<<S, 256, 0, s>>>(x, part, nsum, pstride, w, eps, hi, lo);
    } else if (D == RN_THREADS) {
        rmsnorm_split_reg<1><<<S, RN_THREADS, 0, s>>>(x, part, nsum, pstride, w, eps, hi, lo);
    } else if (D == 2 * RN_THREADS) {
        rmsnorm_split_reg<2><<<S, RN_THREADS, 0, s>>>(x, part, nsum, pstride, w, eps, hi, lo);
    } else {
        rmsnorm_split<<<S, RN_THREADS, 0, s>>>(x, part, nsum, pstride, w, D, eps, hi, lo);
    }
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// ---------------------------------------------------------------------------
// GEMM on v_mfma_f32_16x16x32_bf16.  Block tile BM x BN = (WGM TM 16) x
// (WGN TN 16): 4 waves in a WGM x WGN grid, each TM x TN MFMA tiles of 16x16.
// K is walked QK_BK (64) at a time through LDS: the next tile's global loads
// are in flight (in registers) while the current one feeds the MFMAs, then
// land in the other of two buffers (one barrier per k tile) or, for 128-row
// tiles, in the single buffer after a second barrier (half the LDS, so two
// blocks share a CU).  Operand fragments:
// lane l supplies row (l & 15) and the 8 consecutive k values [8 (l >> 4), +8)
// of its 32-wide k step, for both the activation tile (A) and the weight tile
// (W rows play the B columns), so the k pairing is the same on both sides.
// Result: lane l holds D[4 (l >> 4) + r][l & 15], r = 0..3.
//
// Split-K: block z covers k in [z kc, (z + 1) kc).  With more than one split
// the STORE epilogue writes split z's partial product to y + z M N and the
// consumer sums the splits in order (fixed order: the result does not depend
// on scheduling).  ADD and SWIGLU epilogues run with one split only.
// ---------------------------------------------------------------------------
#define QK_BK 64
#define QK_LDK (QK_BK + 8)   // +16 B per row keeps the 16-row fragment reads conflict free

template <int WGM, int WGN, int TM, int TN, int EPI>
__global__ __launch_bounds__(256) void gemm_hilo(const uint16_t *__restrict__ ahi, const uint16_t *__restrict__ alo,
                                                 const uint16_t *__restrict__ W, int M, int N, int K, int kc,
                                                 float *y, uint16_t *ohi, uint16_t *olo) {
    static_assert(WGM * WGN == 4, "4 waves");
    constexpr int BM = WGM * TM * 16, BN = WGN * TN * 16;
    constexpr int CPR = QK_BK / 8;                                   // 16-byte chunks per row
    constexpr int ACH = BM * CPR, BCH = BN * CPR;                    // 16-byte chunks per tile
    constexpr int APT = (ACH + 255) / 256, BPT = (BCH + 255) / 256;
    // 128-row tiles keep one LDS buffer (two barriers per k tile, ~55 KB: two
    // blocks per CU); smaller tiles double-buffer (one barrier per k tile)
    constexpr int NBUF = BM >= 128 ? 1 : 2;
    __shared__ __attribute__((aligned(16))) uint16_t sA[NBUF][2][BM][QK_LDK];   // [buffer][hi, lo]
    __shared__ __attribute__((aligned(16))) uint16_t sB[NBUF][BN][QK_LDK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kb = blockIdx.z * kc, ke = min(K, kb + kc);

    uint4 ra[2][APT], rb[BPT];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < APT; i++) {
            const int c = tid + 256 * i, r = c / CPR, gm = m0 + r, gk = k0 + (c % CPR) * 8;
            const bool ok = (ACH % 256 == 0 || c < ACH) && gm < M && gk < ke;
            ra[0][i] = ok ? *reinterpret_cast<const uint4 *>(ahi + (size_t)gm * K + gk) : make_uint4(0u, 0u, 0u, 0u);
            ra[1][i] = ok ? *reinterpret_cast<const uint4 *>(alo + (size_t)gm * K + gk) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int i = 0; i < BPT; i++) {
            const int c = tid + 256 * i, r = c / CPR, gn = n0 + r, gk = k0 + (c % CPR) * 8;
            const bool ok = (BCH % 256 == 0 || c < BCH) && gn < N && gk < ke;
            rb[i] = ok ? ld_stream16(W + (size_t)gn * K + gk) : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < APT; i++) {
            const int c = tid + 256 * i;
            if (ACH % 256 == 0 || c < ACH) {
                *reinterpret_cast<uint4 *>(&sA[buf][0][c / CPR][(c % CPR) * 8]) = ra[0][i];
                *reinterpret_cast<uint4 *>(&sA[buf][1][c / CPR][(c % CPR) * 8]) = ra[1][i];
            }
        }
#pragma unroll
        for (int i = 0; i < BPT; i++) {
            const int c = tid + 256 * i;
            if (BCH % 256 == 0 || c < BCH) *reinterpret_cast<uint4 *>(&sB[buf][c / CPR][(c % CPR) * 8]) = rb[i];
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    const int nk = (ke - kb + QK_BK - 1) / QK_BK;
    gload(kb);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = NBUF == 2 ? (kt & 1) : 0;
        if (kt + 1 < nk) gload(kb + (kt + 1) * QK_BK);
#pragma unroll
        for (int kk = 0; kk < QK_BK; kk += 32) {
            const int koff = kk + (lane >> 4) * 8;
            bf16x8 bfr[TN];
#pragma unroll
            for (int j = 0; j < TN; j++)
                bfr[j] = *reinterpret_cast<const bf16x8 *>(&sB[buf][(wn * TN + j) * 16 + (lane & 15)][koff]);
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int ra_ = (wm * TM + i) * 16 + (lane & 15);
                const bf16x8 ah = *reinterpret_cast<const bf16x8 *>(&sA[buf][0][ra_][koff]);
                const bf16x8 al = *reinterpret_cast<const bf16x8 *>(&sA[buf][1][ra_][koff]);
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bfr[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bfr[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (NBUF == 1) __syncthreads();                   // every wave is done with the only buffer
        if (kt + 1 < nk) lstore(NBUF == 2 ? buf ^ 1 : 0);
        __syncthreads();
    }

    float *yz = y + (EPI == QK_GEMM_STORE ? (size_t)blockIdx.z * M * N : 0);
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + (wn * TN + j) * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + (wm * TM + i) * 16 + 4 * (lane >> 4) + r;
                const float v = acc[i][j][r];
                if (EPI == QK_GEMM_SWIGLU) {
                    const float u = __shfl_xor(v, 1, QK_WAVE);   // column n+1 lives in lane l^1
                    if ((lane & 1) == 0 && m < M && n < N) {
                        const size_t o = (size_t)m * (N / 2) + (n >> 1);
                        split2(swiglu1(v, u), ohi[o], olo[o]);
                    }
                } else if (m < M && n < N) {
                    if (EPI == QK_GEMM_STORE) yz[(size_t)m * N + n] = v;
                    else y[(size_t)m * N + n] += v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Large-M GEMM (same product and epilogues as gemm_hilo): block tile BM x 256
// with 8 waves, each 64 x (256 / WGN) (BM 128: 2 x 4 waves of 64 x 64; BM 256:
// 4 x 2 waves of 64 x 128).  K is walked 32 at a time through a ring of NST
// LDS stages filled by direct global -> LDS loads (global_load_lds, 16 bytes
// per lane), so no registers stage the operands and NST - 1 k tiles stay in
// flight behind the MFMAs; one barrier per k tile.  A stage holds A_hi
// [BM][32], A_lo [BM][32] and W [256][32] in bf16, rows of 64 bytes; a load
// instruction fills 1 KB (16 rows) with lane l at byte 16 l, i.e. row l / 4,
// 16-byte slot l % 4.  Slot p of row r holds k chunk p ^ ((r / 2) % 4): the
// 16 rows x 16 bytes a fragment read touches fall in 16 different 16-byte bank
// groups, and SQ_LDS_BANK_CONFLICT reads 0 for the fragment reads (with
// p ^ ((r / 4) % 4), also 16 distinct groups, it read 0.12 conflict cycles
// per active LDS cycle).
// ---------------------------------------------------------------------------
#define QK_GBK 32

template <int EPI, int BM>
__global__ __launch_bounds__(512, 1) void gemm_hilo_wide(const uint16_t *__restrict__ ahi,
                                                         const uint16_t *__restrict__ alo,
                                                         const uint16_t *__restrict__ W, int M, int N, int K, int kc,
                                                         float *y, uint16_t *ohi, uint16_t *olo) {
    constexpr int BN = 256, WGM = BM / 64, WGN = 8 / WGM, TM = 4, TN = BN / WGN / 16;
    constexpr int NST = BM == 128 ? 4 : 3;                 // stages: 4 x 32 KB or 3 x 48 KB
    constexpr int AB = BM * 64, STAGE = 2 * AB + BN * 64;  // bytes: one A half, one stage
    constexpr int AI = BM / 128;                           // 1 KB load instructions per wave: A half, W
    __shared__ __attribute__((aligned(1024))) unsigned char lds[NST][STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kb = blockIdx.z * kc, ke = min(K, kb + kc);
    const int nk = (ke - kb) / QK_GBK;

    // this lane's load slot: row rr of a 16-row group, k chunk cl (swizzled)
    const int rr = lane >> 2, cl = (lane & 3) ^ ((rr >> 1) & 3);
    const size_t ra0 = (size_t)min(m0 + 16 * (AI * wave) + rr, M - 1) * K + kb + 8 * cl;
    const size_t ra1 = (size_t)min(m0 + 16 * (AI * wave + 1) + rr, M - 1) * K + kb + 8 * cl;   // AI == 2 only
    const uint16_t *pw = W + (size_t)(n0 + 32 * wave + rr) * K + kb + 8 * cl;
    auto issue = [&](int kt) {
        unsigned char *st = lds[kt % NST];
        const int ko = kt * QK_GBK;
        // (written out per row group: the builtin on an array element, or in a
        // loop, made hipcc drop the kernel's host launch stub)
        __builtin_amdgcn_global_load_lds(ahi + ra0 + ko, st + 1024 * (AI * wave), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(alo + ra0 + ko, st + AB + 1024 * (AI * wave), 16, 0, 0);
        if constexpr (AI == 2) {
            __builtin_amdgcn_global_load_lds(ahi + ra1 + ko, st + 1024 * (AI * wave + 1), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(alo + ra1 + ko, st + AB + 1024 * (AI * wave + 1), 16, 0, 0);
        }
        __builtin_amdgcn_global_load_lds(pw + ko, st + 2 * AB + 2048 * wave, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(pw + (size_t)16 * K + ko, st + 2 * AB + 2048 * wave + 1024, 16, 0, 0);
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // fragment reads: row (lane & 15) of a 16-row tile, k chunk lane >> 4
    const int fr = lane & 15;
    const int fo = fr * 64 + 16 * ((lane >> 4) ^ ((fr >> 1) & 3));
    for (int t = 0; t < NST - 1 && t < nk; t++) issue(t);
    for (int kt = 0; kt < nk; kt++) {
        // this wave's loads of tile kt have landed once at most the later
        // tiles' loads (2 AI + 2 per tile) are outstanding
        const int later = min(nk - 1 - kt, NST - 2);
        if (later >= 2) __builtin_amdgcn_s_waitcnt(0x0f70 | (2 * (2 * AI + 2)));
        else if (later == 1) __builtin_amdgcn_s_waitcnt(0x0f70 | (2 * AI + 2));
        else __builtin_amdgcn_s_waitcnt(0x0f70);
        // every wave's share of tile kt is in LDS; tile kt-1's stage is free.  A
        // plain s_barrier: __syncthreads() would also wait for this wave's later
        // tiles still in flight (vmcnt(0)) and drain the ring every k tile
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (kt + NST - 1 < nk) issue(kt + NST - 1);
        const unsigned char *st = lds[kt % NST];
        bf16x8 bfr[TN];
#pragma unroll
        for (int j = 0; j < TN; j++)
            bfr[j] = *reinterpret_cast<const bf16x8 *>(st + 2 * AB + (wn * TN * 16 + j * 16) * 64 + fo);
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int ro = (wm * 64 + i * 16) * 64 + fo;
            const bf16x8 ah = *reinterpret_cast<const bf16x8 *>(st + ro);
            const bf16x8 al = *reinterpret_cast<const bf16x8 *>(st + AB + ro);
#pragma unroll
            for (int j = 0; j < TN; j++) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bfr[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bfr[j], acc[i][j], 0, 0, 0);
            }
        }
    }

    float *yz = y + (EPI == QK_GEMM_STORE ? (size_t)blockIdx.z * M * N : 0);
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn * TN * 16 + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
                const float v = acc[i][j][r];
                if (EPI == QK_GEMM_SWIGLU) {
                    const float u = __shfl_xor(v, 1, QK_WAVE);   // column n+1 lives in lane l^1
                    if ((lane & 1) == 0 && m < M) {
                        const size_t o = (size_t)m * (N / 2) + (n >> 1);
                        split2(swiglu1(v, u), ohi[o], olo[o]);
                    }
                } else if (m < M) {
                    if (EPI == QK_GEMM_STORE) yz[(size_t)m * N + n] = v;
                    else y[(size_t)m * N + n] += v;
                }
            }
        }
    }
}

template <int BM>
static void gemm_wide_dispatch(const uint16_t *a_hi, const uint16_t *a_lo, const uint16_t *W, int M, int N, int K,
                               const qk_gemm_plan *p, int epi, float *y, uint16_t *oh, uint16_t *ol, hipStream_t s) {
    const dim3 grid(N / 256, (M + BM - 1) / BM, p->nsplit);
    if (epi == QK_GEMM_STORE)
        gemm_hilo_wide<QK_GEMM_STORE, BM><<<grid, 512, 0, s>>>(a_hi, a_lo, W, M, N, K, p->kc, y, oh, ol);
    else if (epi == QK_GEMM_ADD)
        gemm_hilo_wide<QK_GEMM_ADD, BM><<<grid, 512, 0, s>>>(a_hi, a_lo, W, M, N, K, p->kc, y, oh, ol);
    else
        gemm_hilo_wide<QK_GEMM_SWIGLU, BM><<<grid, 512, 0, s>>>(a_hi, a_lo, W, M, N, K, p->kc, y, oh, ol);
}

// ---------------------------------------------------------------------------
// Mid-M GEMM (a few hundred rows, e.g. a 401-row prefill; same product and
// epilogues as gemm_hilo): block tile BM x BN with NW waves, each 32 x WTN
// (2 x WTN / 16 MFMA tiles), K walked 32 at a time through a ring of NST LDS
// stages filled by direct global -> LDS loads in the stage layout and swizzle
// of gemm_hilo_wide.  At this size a CU holds one or two tiles and walks
// their whole k range: the register-staged kernel (one k tile in flight)
// spends ~1.1 us per 64-deep k tile waiting for loads, ~5x its MFMA time.
// Here NST - 1 stages are in flight; four stages (64 KB at 64 x 128) let two
// blocks share a CU, which measured faster than deeper rings with one block
// per CU.  The 16-row load groups of a stage (A_hi, A_lo, W) are dealt
// round-robin to the waves: LPW 1 KB load instructions per wave and stage.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int ring_waves(int bm, int bn) { return bm / 32 * (bn / 64) < 4 ? 4 : bm / 32 * (bn / 64); }
__device__ constexpr int vmcnt_imm(int n) { return 0x0f70 | (n & 15) | ((n >> 4) << 14); }

// wait until at most later * LPW of this wave's loads are outstanding
// (later <= MAXL: the stages issued after the one about to be read)
template <int LPW, int MAXL>
__device__ __forceinline__ void ring_wait(int later) {
    if constexpr (MAXL > 0) {
        if (later >= MAXL) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(MAXL * LPW));
            return;
        }
        ring_wait<LPW, MAXL - 1>(later);
    } else {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
}

// 16 bytes per lane from global memory straight into LDS (lane l at byte 16 l
// of the 1 KB at l0).  Called through this helper: with the builtin written in
// the kernel on pointers held in an array, hipcc's host pass drops the
// kernel's launch stub.
__device__ __forceinline__ void lds_load16(const uint16_t *g, unsigned char *l0) {
    __builtin_amdgcn_global_load_lds(g, l0, 16, 0, 0);
}

template <int BM, int BN>
struct RingShape {
    static constexpr int NW = ring_waves(BM, BN), WGM = BM / 32, WGN = NW / WGM, WTN = BN / WGN, TM = 2,
                         TN = WTN / 16;
    static constexpr int AB = BM * 64, STAGE = 2 * AB + BN * 64;   // bytes: one A half, one stage
    static constexpr int GROUPS = (2 * BM + BN) / 16, LPW = GROUPS / NW;
    static_assert(WGM * WGN == NW && WTN % 16 == 0 && GROUPS % NW == 0, "wave grid / load split");
};

// The k walk of block (blockIdx.x, blockIdx.y, blockIdx.z) into acc: wave
// (wm, wn) = (wave / WGN, wave % WGN) holds rows m0 + 32 wm + 16 i + 4 (l >> 4)
// + r, columns n0 + WTN wn + 16 j + (l & 15) (lane l, acc[i][j][r]).  lds:
// NST stages of the kernel's shared memory.
template <int BM, int BN, int NST>
__device__ __forceinline__ void ring_tile(const uint16_t *__restrict__ ahi, const uint16_t *__restrict__ alo,
                                          const uint16_t *__restrict__ W, int M, int K, int kc, unsigned char *lds,
                                          f32x4 (&acc)[2][RingShape<BM, BN>::TN]) {
    using RS = RingShape<BM, BN>;
    constexpr int NW = RS::NW, WGN = RS::WGN, WTN = RS::WTN, TM = RS::TM, TN = RS::TN;
    constexpr int AB = RS::AB, STAGE = RS::STAGE, LPW = RS::LPW;
    static_assert((NST - 2) * LPW <= 63 && NST * STAGE <= 160 * 1024, "vmcnt / LDS range");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kb = blockIdx.z * kc, ke = min(K, kb + kc);
    const int nk = (ke - kb) / QK_GBK;

    // this lane's load slots: row rr of each of the wave's 16-row groups,
    // k chunk cl (swizzled); rows past M re-read row M - 1 (results dropped)
    const int rr = lane >> 2, cl = (lane & 3) ^ ((rr >> 1) & 3);
    const uint16_t *src[LPW];
    int dst[LPW];
#pragma unroll
    for (int j = 0; j < LPW; j++) {
        const int g = wave + NW * j;
        if (g < BM / 16) {
            src[j] = ahi + (size_t)min(m0 + 16 * g + rr, M - 1) * K + kb + 8 * cl;
            dst[j] = 1024 * g;
        } else if (g < BM / 8) {
            src[j] = alo + (size_t)min(m0 + 16 * (g - BM / 16) + rr, M - 1) * K + kb + 8 * cl;
            dst[j] = AB + 1024 * (g - BM / 16);
        } else {
            src[j] = W + (size_t)(n0 + 16 * (g - BM / 8) + rr) * K + kb + 8 * cl;
            dst[j] = 2 * AB + 1024 * (g - BM / 8);
        }
    }
    auto issue = [&](int kt) {
        unsigned char *st = lds + (kt % NST) * STAGE;
#pragma unroll
        for (int j = 0; j < LPW; j++) lds_load16(src[j] + kt * QK_GBK, st + dst[j]);
    };

#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    const int fr = lane & 15;
    const int fo = fr * 64 + 16 * ((lane >> 4) ^ ((fr >> 1) & 3));
    for (int t = 0; t < NST - 1 && t < nk; t++) issue(t);
    for (int kt = 0; kt < nk; kt++) {
        ring_wait<LPW, NST - 2>(min(nk - 1 - kt, NST - 2));
        // every wave's share of stage kt is in LDS and stage kt - 1 is free (a
        // plain s_barrier: __syncthreads() would also drain the later stages)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (kt + NST - 1 < nk) issue(kt + NST - 1);
        const unsigned char *st = lds + (kt % NST) * STAGE;
        bf16x8 bfr[TN];
#pragma unroll
        for (int j = 0; j < TN; j++)
            bfr[j] = *reinterpret_cast<const bf16x8 *>(st + 2 * AB + (wn * WTN + j * 16) * 64 + fo);
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int ro = (wm * 32 + i * 16) * 64 + fo;
            const bf16x8 ah = *reinterpret_cast<const bf16x8 *>(st + ro);
            const bf16x8 al = *reinterpret_cast<const bf16x8 *>(st + AB + ro);
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bfr[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bfr[j], acc[i][j], 0, 0, 0);
        }
    }
}

template <int EPI, int BM, int BN, int NST>
__global__ __launch_bounds__(ring_waves(BM, BN) * 64) void gemm_hilo_ring(const uint16_t *__restrict__ ahi,
                                                                           const uint16_t *__restrict__ alo,
                                                                           const uint16_t *__restrict__ W, int M,
                                                                           int N, int K, int kc, float *y,
                                                                           uint16_t *ohi, uint16_t *olo) {
    using RS = RingShape<BM, BN>;
    constexpr int WGN = RS::WGN, WTN = RS::WTN, TM = RS::TM, TN = RS::TN;
    __shared__ __attribute__((aligned(1024))) unsigned char lds[NST * RS::STAGE];
    f32x4 acc[TM][TN];
    ring_tile<BM, BN, NST>(ahi, alo, W, M, K, kc, lds, acc);
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    float *yz = y + (EPI == QK_GEMM_STORE ? (size_t)blockIdx.z * M * N : 0);
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn * WTN + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
                const float v = acc[i][j][r];
                if (EPI == QK_GEMM_SWIGLU) {
                    const float u = __shfl_xor(v, 1, QK_WAVE);   // column n+1 lives in lane l^1
                    if ((lane & 1) == 0 && m < M) {
                        const size_t o = (size_t)m * (N / 2) + (n >> 1);
                        split2(swiglu1(v, u), ohi[o], olo[o]);
                    }
                } else if (m < M) {
                    if (EPI == QK_GEMM_STORE) yz[(size_t)m * N + n] = v;
                    else y[(size_t)m * N + n] += v;
                }
            }
        }
    }
}

// Q|K|V projection with the RoPE / append epilogue (the work of rope_append
// on the product, reference qwen_asr_decoder.c:270-300): a 64 x 128 tile is
// 64 rows of one head (Q heads, then K heads, then V heads along N).  The
// tile goes to LDS (the ring is free after the k walk), then each wave takes
// 16 rows, four at a time on its four 16-lane groups, and runs rope_append's
// per-row code on them (norm_rope_row16): per-head RMSNorm and NeoX rotation
// of dims (d, d + 64) for Q and K (Q to q_out, K to the cache), V copied to
// the cache.  The sums and products are rope_append's, so the result equals
// GEMM (STORE, one split) + rope_append bit for bit.
#define RP_ROW (QWEN_HIP_HEAD_DIM + 4)        // floats per row of the staged tile
__global__ __launch_bounds__(256) void gemm_hilo_ring_rope(const uint16_t *__restrict__ ahi,
                                                           const uint16_t *__restrict__ alo,
                                                           const uint16_t *__restrict__ W, int M, int K,
                                                           qk_rope_append_args ra) {
    using RS = RingShape<64, QWEN_HIP_HEAD_DIM>;
    constexpr int WGN = RS::WGN, WTN = RS::WTN, TM = RS::TM, TN = RS::TN, hd = QWEN_HIP_HEAD_DIM, half = hd / 2;
    __shared__ __attribute__((aligned(1024))) unsigned char lds[QK_GEMM_RING_NST * RS::STAGE];
    static_assert(64 * RP_ROW * sizeof(float) <= sizeof(lds) && RP_ROW % 4 == 0, "staged tile");
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int m0 = blockIdx.y * 64, head = blockIdx.x;
    const int nqk = ra.heads + ra.kv_heads, qd = ra.heads * hd;
    const bool is_q = head < ra.heads, is_k = !is_q && head < nqk;
    // this wave's 16 rows of the tile: row rl0 + 4 k + g in pass k for the
    // 16-lane group g, whose lane c holds dims 4c .. 4c+3 and 64+4c .. 64+4c+3
    const int rl0 = 16 * wave, g = lane >> 4, c = lane & 15;
    // the epilogue's operands (the rows' cos / sin, the norm weights) are
    // loaded before the k walk, so their latency passes under it
    float4 cv[4], sv[4], wl = make_float4(0.f, 0.f, 0.f, 0.f), wh = wl;
    if (is_q || is_k) {
        const float *nw = is_q ? ra.q_norm : ra.k_norm;
        wl = *reinterpret_cast<const float4 *>(nw + 4 * c);
        wh = *reinterpret_cast<const float4 *>(nw + half + 4 * c);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const size_t p = (size_t)ra.start + min(m0 + rl0 + 4 * k + g, M - 1);
            cv[k] = *reinterpret_cast<const float4 *>(ra.rope_cos + p * hd + 4 * c);
            sv[k] = *reinterpret_cast<const float4 *>(ra.rope_sin + p * hd + 4 * c);
        }
    }
    f32x4 acc[TM][TN];
    ring_tile<64, QWEN_HIP_HEAD_DIM, QK_GEMM_RING_NST>(ahi, alo, W, M, K, K, lds, acc);

    __syncthreads();                                   // every wave is past its last k step
    float *T = reinterpret_cast<float *>(lds);         // [64][RP_ROW]
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                T[(wm * 32 + i * 16 + 4 * (lane >> 4) + r) * RP_ROW + wn * WTN + j * 16 + (lane & 15)] = acc[i][j][r];
    __syncthreads();

    // rows past M are computed on the tile's (finite) contents and not stored
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int rl = rl0 + 4 * k + g, srow = m0 + rl;
        float4 lo = *reinterpret_cast<const float4 *>(T + rl * RP_ROW + 4 * c);
        float4 hi = *reinterpret_cast<const float4 *>(T + rl * RP_ROW + half + 4 * c);
        float *d;
        if (is_q || is_k) {
            norm_rope_row16(lo, hi, wl, wh, cv[k], sv[k], ra.eps);
            d = is_q ? ra.q_out + (size_t)srow * qd + head * hd
                     : ra.k_cache + ((size_t)(head - ra.heads) * ra.cap + ra.start + srow) * hd;
        } else {
            d = ra.v_cache + ((size_t)(head - nqk) * ra.cap + ra.start + srow) * hd;
        }
        if (srow < M) {
            *reinterpret_cast<float4 *>(d + 4 * c) = lo;
            *reinterpret_cast<float4 *>(d + half + 4 * c) = hi;
        }
    }
}

extern "C" int qk_gemm_rope_fusable(const qk_gemm_plan *p) {
    return p && p->nst == QK_GEMM_RING_NST && p->bm == 64 && p->bn == QK_GEMM_BN && p->nsplit == 1;
}

extern "C" int qk_gemm_rope_launch(const uint16_t *a_hi, const uint16_t *a_lo, const uint16_t *W, int M, int K,
                                   const qk_gemm_plan *p, const qk_rope_append_args *ra, hipStream_t s) {
    if (M <= 0 || K <= 0 || K % QK_GBK || !a_hi || !a_lo || !W || !ra || !qk_gemm_rope_fusable(p) ||
        p->kc < K || ra->S != M || ra->pos_dev || ra->nsum > 1 || ra->heads <= 0 || ra->kv_heads <= 0 ||
        ra->heads % ra->kv_heads || !ra->q_norm || !ra->k_norm || !ra->rope_cos || !ra->rope_sin ||
        !ra->k_cache || !ra->v_cache || !ra->q_out || ra->start < 0 || ra->start + M > ra->cap)
        return QWEN_HIP_EINVAL;
    // 16-byte accesses in the epilogue
    if (((uintptr_t)ra->q_norm | (uintptr_t)ra->k_norm | (uintptr_t)ra->rope_cos | (uintptr_t)ra->rope_sin |
         (uintptr_t)ra->k_cache | (uintptr_t)ra->v_cache | (uintptr_t)ra->q_out) % 16)
        return QWEN_HIP_EINVAL;
    const dim3 grid(ra->heads + 2 * ra->kv_heads, (M + 63) / 64);
    gemm_hilo_ring_rope<<<grid, 256, 0, s>>>(a_hi, a_lo, W, M, K, *ra);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

template <int BM, int BN, int NST>
static void gemm_ring_dispatch(const uint16_t *a_hi, const uint16_t *a_lo, const uint16_t *W, int M, int N, int K,
                               const qk_gemm_plan *p, int epi, float *y, uint16_t *oh, uint16_t *ol, hipStream_t s) {
    const dim3 grid(N / BN, (M + BM - 1) / BM, p->nsplit), block(64 * ring_waves(BM, BN));
    if (epi == QK_GEMM_STORE)
        gemm_hilo_ring<QK_GEMM_STORE, BM, BN, NST><<<grid, block, 0, s>>>(a_hi, a_lo, W, M, N, K, p->kc, y, oh, ol);
    else if (epi == QK_GEMM_ADD)
        gemm_hilo_ring<QK_GEMM_ADD, BM, BN, NST><<<grid, block, 0, s>>>(a_hi, a_lo, W, M, N, K, p->kc, y, oh, ol);
    else
        gemm_hilo_ring<QK_GEMM_SWIGLU, BM, BN, NST><<<grid, block, 0, s>>>(a_hi, a_lo, W, M, N, K, p->kc, y, oh, ol);
}

// the ring configurations built: (bm, bn, nst); 0 when the plan names another
static int gemm_ring_launch(const uint16_t *a_hi, const uint16_t *a_lo, const uint16_t *W, int M, int N, int K,
                            const qk_gemm_plan *p, int epi, float *y, uint16_t *oh, uint16_t *ol, hipStream_t s) {
#define QK_RING(BM_, BN_, NST_)                                                                  \
    if (p->bm == BM_ && p->bn == BN_ && p->nst == NST_) {                                        \
        gemm_ring_dispatch<BM_, BN_, NST_>(a_hi, a_lo, W, M, N, K, p, epi, y, oh, ol, s);        \
        return 1;                                                                                \
    }
    QK_RING(64, 128, QK_GEMM_RING_NST) QK_RING(32, 128, QK_GEMM_RING_NST) QK_RING(128, 128, 3)
#undef QK_RING
    return 0;
}

template <int WGM, int WGN, int TM, int TN>
static void gemm_dispatch(const uint16_t *a_hi, const uint16_t *a_lo, const uint16_t *W, int M, int N, int K,
                          const qk_gemm_plan *p, int epi, float *y, uint16_t *oh, uint16_t *ol, hipStream_t s) {
    dim3 grid((N + WGN * TN * 16 - 1) / (WGN * TN * 16), (M + WGM * TM * 16 - 1) / (WGM * TM * 16), p->nsplit);
    if (epi == QK_GEMM_STORE)
        gemm_hilo<WGM, WGN, TM, TN, QK_GEMM_STORE><<<grid, 256, 0, s>>>(a_hi, a_lo, W, M, N, K, p->kc, y, oh, ol);
    else if (epi == QK_GEMM_ADD)
        gemm_hilo<WGM, WGN, TM, TN, QK_GEMM_ADD><<<grid, 256, 0, s>>>(a_hi, a_lo, W, M, N, K, p->kc, y, oh, ol);
    else
        gemm_hilo<WGM, WGN, TM, TN, QK_GEMM_SWIGLU><<<grid, 256, 0, s>>>(a_hi, a_lo, W, M, N, K, p->kc, y, oh, ol);
}

extern "C" void qk_gemm_plan_for(int M, int N, int K, qk_gemm_plan *p) { qk_gemm_plan_epi(M, N, K, QK_GEMM_STORE, p); }

extern "C" void qk_gemm_plan_epi(int M, int N, int K, int epi, qk_gemm_plan *p) {
    p->nst = 0;
    // 256 x 256 or 128 x 256 tiles (one block per CU) where they alone fill
    // every CU and the last round of blocks is not mostly empty (>= 85 % of
    // the rounds' slots used); the larger tile first
    for (int bm = 256; bm >= 128; bm -= 128) {
        const long wide = (long)((M + bm - 1) / bm) * (N / 256);
        const long slots = (wide + QK_GEMM_TARGET - 1) / QK_GEMM_TARGET * QK_GEMM_TARGET;
        if (M <= 512 || N % 256 || K % QK_GBK || wide < QK_GEMM_TARGET || wide * 100 < slots * 85) continue;
        p->bm = bm;
        p->bn = 256;
        p->nsplit = 1;
        p->kc = (K + QK_BK - 1) / QK_BK * QK_BK;
        return;
    }
    // otherwise 32 x 128 (M <= 32) or 64 x 128 tiles on the LDS ring where the
    // shape allows it (whole 128-column tiles, K in whole 32-deep steps), else
    // the register-staged kernel
    const int ring = N % QK_GEMM_BN == 0 && K % QK_GBK == 0;
    p->bn = QK_GEMM_BN;
    p->bm = M <= 32 ? 32 : (ring || M <= 512) ? 64 : 128;
    p->nst = ring ? QK_GEMM_RING_NST : 0;
    if (ring && (epi == QK_GEMM_SWIGLU || epi == QK_GEMM_STORE) && M > 512) {
        // more than 512 rows: 128 x 128 tiles (8 waves of 32 x 64, 3 stages =
        // 72 KB, two blocks per CU) move a quarter fewer bytes per MFMA (C3's
        // gate|up: 184 -> 156 us, down 103 -> 79 us, O 34.8 -> 33.8 us)
        p->bm = 128;
        p->nst = 3;
    }
    const long tiles = (long)((M + p->bm - 1) / p->bm) * ((N + QK_GEMM_BN - 1) / QK_GEMM_BN);
    const int kt = (K + QK_BK - 1) / QK_BK;
    long ns;
    if (ring) {
        // enough blocks for ~7/8 of the CUs (two ring blocks share a CU, so a
        // second round is cheap), and k walks of QK_GEMM_RING_KSPLIT or more
        // in two halves: measured faster even where the tiles alone fill the
        // chip (more splits cost their consumer more than they save), except
        // for a SwiGLU product, whose partials (twice the output) need a
        // reduce pass, and a Q|K|V product whose RoPE epilogue needs one split
        ns = (QK_GEMM_RING_TARGET + tiles - 1) / tiles;
        if (ns < 2 && K >= QK_GEMM_RING_KSPLIT && epi != QK_GEMM_SWIGLU && epi != QK_GEMM_ROPE) ns = 2;
        // 128 x 128 STORE tiles: two splits per 4096 of K.  Odd counts leave a
        // part-empty last round of blocks (C3's down, K 6144: 3 splits 93 us,
        // 4 splits 79 us, 2 splits 94 us; 1024-column products: 2 splits 29 us
        // against 3 splits 37 us)
        if (p->bm == 128 && epi == QK_GEMM_STORE) ns = 2 * ((K + 4095) / 4096);
    } else {
        ns = tiles >= QK_GEMM_TARGET ? 1 : (QK_GEMM_TARGET + tiles - 1) / tiles;
    }
    if (ns > QK_GEMM_MAX_SPLIT) ns = QK_GEMM_MAX_SPLIT;
    if (ns > kt) ns = kt;
    const int per = (int)((kt + ns - 1) / ns);      // k tiles per split
    p->kc = per * QK_BK;
    p->nsplit = (kt + per - 1) / per;
}

extern "C" int qk_gemm_launch(const uint16_t *a_hi, const uint16_t *a_lo, const uint16_t *W, int M, int N, int K,
                              const qk_gemm_plan *p, int epi, float *y, uint16_t *out_hi, uint16_t *out_lo,
                              hipStream_t s) {
    if (M <= 0 || N <= 0 || K <= 0 || (K & 7) || !a_hi || !a_lo || !W || !p) return QWEN_HIP_EINVAL;
    if (p->nsplit < 1 || p->kc <= 0 || p->kc % QK_BK || (long)p->kc * p->nsplit < K ||
        (long)p->kc * (p->nsplit - 1) >= K)
        return QWEN_HIP_EINVAL;
    if (p->nsplit > 1 && epi != QK_GEMM_STORE) return QWEN_HIP_EINVAL;
    if (epi == QK_GEMM_SWIGLU ? (!out_hi || !out_lo || (N & 1)) : !y) return QWEN_HIP_EINVAL;
    if (p->nst) {
        if (N % p->bn || K % QK_GBK || p->kc % QK_GBK) return QWEN_HIP_EINVAL;
        if (!gemm_ring_launch(a_hi, a_lo, W, M, N, K, p, epi, y, out_hi, out_lo, s)) return QWEN_HIP_EINVAL;
        return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
    }
    if (p->bn == 256) {
        if ((p->bm != 128 && p->bm != 256) || N % 256 || K % QK_GBK || p->kc % QK_GBK) return QWEN_HIP_EINVAL;
        if (p->bm == 128) gemm_wide_dispatch<128>(a_hi, a_lo, W, M, N, K, p, epi, y, out_hi, out_lo, s);
        else gemm_wide_dispatch<256>(a_hi, a_lo, W, M, N, K, p, epi, y, out_hi, out_lo, s);
        return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
    }
    if (p->bn != QK_GEMM_BN) return QWEN_HIP_EINVAL;
    if (p->bm == 32) gemm_dispatch<1, 4, 2, 2>(a_hi, a_lo, W, M, N, K, p, epi, y, out_hi, out_lo, s);
    else if (p->bm == 64) gemm_dispatch<2, 2, 2, 4>(a_hi, a_lo, W, M, N, K, p, epi, y, out_hi, out_lo, s);
    else if (p->bm == 128) gemm_dispatch<2, 2, 4, 4>(a_hi, a_lo, W, M, N, K, p, epi, y, out_hi, out_lo, s);
    else return QWEN_HIP_EINVAL;
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// Sum of the nsum split-K partials part[s][M][N] in split order, then the
// epilogue: STORE y = sum, ADD y += sum, SWIGLU hi/lo of silu(sum[2j]) sum[2j+1].
template <int EPI>
__global__ __launch_bounds__(256) void gemm_reduce(const float *part, int nsum, long M, long N, float *y,
                                                   uint16_t *ohi, uint16_t *olo) {
    const long pairs = M * N / 2, pstride = M * N;
    for (long t = blockIdx.x * 256L + threadIdx.x; t < pairs; t += (long)gridDim.x * 256) {
        const float2 v = sum_splits2<QK_GEMM_MAX_SPLIT>(reinterpret_cast<const float2 *>(part) + t, nsum, pstride / 2);
        if (EPI == QK_GEMM_SWIGLU) {
            split2(swiglu1(v.x, v.y), ohi[t], olo[t]);
        } else if (EPI == QK_GEMM_ADD) {
            float2 *o = reinterpret_cast<float2 *>(y) + t;
            float2 a = *o;
            a.x += v.x;
            a.y += v.y;
            *o = a;
        } else {
            reinterpret_cast<float2 *>(y)[t] = v;
        }
    }
}

extern "C" int qk_gemm_reduce_launch(const float *part, int nsum, int M, int N, int epi, float *y, uint16_t *out_hi,
                                     uint16_t *out_lo, hipStream_t s) {
    if (!part || nsum < 1 || nsum > QK_GEMM_MAX_SPLIT || M <= 0 || N <= 0 || (N & 1)) return QWEN_HIP_EINVAL;
    if (epi == QK_GEMM_SWIGLU ? (!out_hi || !out_lo) : !y) return QWEN_HIP_EINVAL;
    long blocks = ((long)M * N / 2 + 255) / 256;
    if (blocks > 2048) blocks = 2048;
    if (epi == QK_GEMM_STORE) gemm_reduce<QK_GEMM_STORE><<<(int)blocks, 256, 0, s>>>(part, nsum, M, N, y, out_hi, out_lo);
    else if (epi == QK_GEMM_ADD) gemm_reduce<QK_GEMM_ADD><<<(int)blocks, 256, 0, s>>>(part, nsum, M, N, y, out_hi, out_lo);
    else gemm_reduce<QK_GEMM_SWIGLU><<<(int)blocks, 256, 0, s>>>(part, nsum, M, N, y, out_hi, out_lo);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// ---------------------------------------------------------------------------
// Elementwise operators of the op-level ABI (reference qwen_asr_kernels.c).
// ---------------------------------------------------------------------------
__global__ void add_kernel(float *a, const float *b, long n) {
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
        a[i] += b[i];
}

extern "C" int qk_add_launch(float *a, const float *b, long n, hipStream_t s) {
    if (n <= 0) return n == 0 ? 0 : QWEN_HIP_EINVAL;
    long blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    add_kernel<<<(int)blocks, 256, 0, s>>>(a, b, n);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

__global__ __launch_bounds__(256) void rms_norm_kernel(float *out, const float *x, const float *w, int D, float eps) {
    __shared__ float red[4];
    const float *xr = x + (size_t)blockIdx.x * D;
    float *orow = out + (size_t)blockIdx.x * D;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < D; i += 256) ss = fmaf(xr[i], xr[i], ss);
    ss = block_sum256(ss, red);      // its trailing barrier orders all reads before in-place writes
    const float rinv = rsqrt_norm(ss / (float)D + eps);
    for (int i = threadIdx.x; i < D; i += 256) orow[i] = (xr[i] * w[i]) * rinv;
}

extern "C" int qk_rms_norm_launch(float *out, const float *x, const float *w, int S, int D, float eps, hipStream_t s) {
    if (S <= 0 || D <= 0) return QWEN_HIP_EINVAL;
    rms_norm_kernel<<<S, 256, 0, s>>>(out, x, w, D, eps);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

__global__ __launch_bounds__(64) void rms_norm_head_kernel(float *x, const float *w, int nh, int hd, float eps) {
    float *v = x + ((size_t)blockIdx.y * nh + blockIdx.x) * hd;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < hd; i += 64) ss = fmaf(v[i], v[i], ss);
    ss = wave_sum(ss);
    const float rinv = rsqrt_norm(ss / (float)hd + eps);
    for (int i = threadIdx.x; i < hd; i += 64) v[i] = (v[i] * w[i]) * rinv;
}

extern "C" int qk_rms_norm_per_head_launch(float *x, const float *w, int S, int nh, int hd, float eps, hipStream_t s) {
    if (S <= 0 || nh <= 0 || hd <= 0) return QWEN_HIP_EINVAL;
    rms_norm_head_kernel<<<dim3(nh, S), 64, 0, s>>>(x, w, nh, hd, eps);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

__global__ void rope_kernel(float *x, const float *cv, const float *sv, int nh, int hd) {
    const int half = hd / 2;
    const float *c = cv + (size_t)blockIdx.y * hd, *sn = sv + (size_t)blockIdx.y * hd;
    float *v = x + ((size_t)blockIdx.y * nh + blockIdx.x) * hd;
    for (int d = threadIdx.x; d < half; d += blockDim.x) {
        const float x1 = v[d], x2 = v[half + d];
        v[d] = fmaf(x1, c[d], -(x2 * sn[d]));
        v[half + d] = fmaf(x2, c[d], x1 * sn[d]);
    }
}

extern "C" int qk_rope_launch(float *x, const float *cos_v, const float *sin_v, int S, int nh, int hd, hipStream_t s) {
    if (S <= 0 || nh <= 0 || hd <= 0 || (hd & 1)) return QWEN_HIP_EINVAL;
    rope_kernel<<<dim3(nh, S), 64, 0, s>>>(x, cos_v, sin_v, nh, hd);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

__global__ void swiglu_kernel(float *out, const float *gu, int S, int inter) {
    const long n = (long)S * inter;
    for (long t = blockIdx.x * (long)blockDim.x + threadIdx.x; t < n; t += (long)gridDim.x * blockDim.x) {
        const long s = t / inter, j = t % inter;
        out[t] = swiglu1(gu[s * 2 * inter + 2 * j], gu[s * 2 * inter + 2 * j + 1]);
    }
}

// out == gate_up: row s of the output overwrites inputs of rows <= s only, so
// one block walks the rows in order, reading a whole row before writing it.
__global__ __launch_bounds__(256) void swiglu_inplace_kernel(float *buf, int S, int inter) {
    for (int s = 0; s < S; s++) {
        const float *gu = buf + (size_t)s * 2 * inter;
        float r[24];
        int n = 0;
        for (int j = threadIdx.x; j < inter && n < 24; j += 256, n++) r[n] = swiglu1(gu[2 * j], gu[2 * j + 1]);
        __syncthreads();
        n = 0;
        for (int j = threadIdx.x; j < inter && n < 24; j += 256, n++) buf[(size_t)s * inter + j] = r[n];
        __syncthreads();
    }
}

extern "C" int qk_swiglu_launch(float *out, const float *gate_up, int S, int inter, hipStream_t s) {
    if (S <= 0 || inter <= 0) return QWEN_HIP_EINVAL;
    if (out == gate_up) {
        if (inter > 24 * 256) return QWEN_HIP_EINVAL;
        swiglu_inplace_kernel<<<1, 256, 0, s>>>(out, S, inter);
    } else {
        long blocks = ((long)S * inter + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        swiglu_kernel<<<(int)blocks, 256, 0, s>>>(out, gate_up, S, inter);
    }
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

__global__ void split_kernel(const float *x, long n, uint16_t *hi, uint16_t *lo) {
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
        split2(x[i], hi[i], lo[i]);
}

extern "C" int qk_split_bf16_launch(const float *x, long n, uint16_t *hi, uint16_t *lo, hipStream_t s) {
    if (n <= 0) return QWEN_HIP_EINVAL;
    long blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    split_kernel<<<(int)blocks, 256, 0, s>>>(x, n, hi, lo);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}
