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
// consumes.  One block per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_split(const float *x, const float *w, int D, float eps,
                                                     uint16_t *hi, uint16_t *lo) {
    __shared__ float red[4];
    const float *xr = x + (size_t)blockIdx.x * D;
    float rinv = 1.0f;
    if (w) {
        float ss = 0.0f;
        for (int i = threadIdx.x; i < D; i += 256) ss = fmaf(xr[i], xr[i], ss);
        ss = block_sum256(ss, red);
        rinv = 1.0f / sqrtf(ss / (float)D + eps);
    }
    uint16_t *h = hi + (size_t)blockIdx.x * D, *l = lo + (size_t)blockIdx.x * D;
    for (int i = threadIdx.x; i < D; i += 256) {
        const float v = w ? (xr[i] * w[i]) * rinv : xr[i];
        split2(v, h[i], l[i]);
    }
}

extern "C" int qk_rmsnorm_split_launch(const float *x, const float *w, int S, int D, float eps,
                                       uint16_t *hi, uint16_t *lo, hipStream_t s) {
    if (S <= 0 || D <= 0 || !x || !hi || !lo) return QWEN_HIP_EINVAL;
    rmsnorm_split<<<S, 256, 0, s>>>(x, w, D, eps, hi, lo);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// ---------------------------------------------------------------------------
// GEMM on v_mfma_f32_16x16x32_bf16.  Block tile BM x BN (4 waves in 2x2, each
// WM x WN MFMA tiles of 16x16), K staged through LDS 64 at a time.  Operand
// fragments: lane l supplies row (l & 15) and the 8 consecutive k values
// [8*(l>>4), +8) of its 32-wide k step, for both the activation tile (A) and
// the weight tile (W rows play the B columns), so the k pairing is the same
// on both sides.  Result: lane l holds D[4*(l>>4) + r][l & 15], r = 0..3.
// ---------------------------------------------------------------------------
#define QK_BK 64
#define QK_LDK (QK_BK + 8)   // +16 B per row keeps the 16-row fragment reads conflict free

template <int WM, int WN, int EPI>
__global__ __launch_bounds__(256) void gemm_hilo(const uint16_t *__restrict__ ahi, const uint16_t *__restrict__ alo,
                                                 const uint16_t *__restrict__ W, int M, int N, int K,
                                                 float *y, uint16_t *ohi, uint16_t *olo) {
    constexpr int BM = 32 * WM, BN = 32 * WN;
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM][QK_LDK];
    __shared__ __attribute__((aligned(16))) uint16_t sB[BN][QK_LDK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    f32x4 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    for (int k0 = 0; k0 < K; k0 += QK_BK) {
        __syncthreads();
        for (int c = tid; c < BM * (QK_BK / 8); c += 256) {
            const int r = c / (QK_BK / 8), kc = (c % (QK_BK / 8)) * 8;
            const int gm = m0 + r, gk = k0 + kc;
            uint4 vh = make_uint4(0u, 0u, 0u, 0u), vl = vh;
            if (gm < M && gk < K) {
                vh = *reinterpret_cast<const uint4 *>(ahi + (size_t)gm * K + gk);
                vl = *reinterpret_cast<const uint4 *>(alo + (size_t)gm * K + gk);
            }
            *reinterpret_cast<uint4 *>(&sA[0][r][kc]) = vh;
            *reinterpret_cast<uint4 *>(&sA[1][r][kc]) = vl;
        }
        for (int c = tid; c < BN * (QK_BK / 8); c += 256) {
            const int r = c / (QK_BK / 8), kc = (c % (QK_BK / 8)) * 8;
            const int gn = n0 + r, gk = k0 + kc;
            uint4 vb = make_uint4(0u, 0u, 0u, 0u);
            if (gn < N && gk < K) vb = *reinterpret_cast<const uint4 *>(W + (size_t)gn * K + gk);
            *reinterpret_cast<uint4 *>(&sB[r][kc]) = vb;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < QK_BK; kk += 32) {
            const int koff = kk + (lane >> 4) * 8;
            bf16x8 bfr[WN];
#pragma unroll
            for (int j = 0; j < WN; j++)
                bfr[j] = *reinterpret_cast<const bf16x8 *>(&sB[wn * (BN / 2) + j * 16 + (lane & 15)][koff]);
#pragma unroll
            for (int i = 0; i < WM; i++) {
                const int ra = wm * (BM / 2) + i * 16 + (lane & 15);
                const bf16x8 ah = *reinterpret_cast<const bf16x8 *>(&sA[0][ra][koff]);
                const bf16x8 al = *reinterpret_cast<const bf16x8 *>(&sA[1][ra][koff]);
#pragma unroll
                for (int j = 0; j < WN; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bfr[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bfr[j], acc[i][j], 0, 0, 0);
                }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < WM; i++) {
#pragma unroll
        for (int j = 0; j < WN; j++) {
            const int n = n0 + wn * (BN / 2) + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * (BM / 2) + i * 16 + 4 * (lane >> 4) + r;
                const float v = acc[i][j][r];
                if (EPI == QK_GEMM_SWIGLU) {
                    const float u = __shfl_xor(v, 1, QK_WAVE);   // column n+1 lives in lane l^1
                    if ((lane & 1) == 0 && m < M && n < N) {
                        const size_t o = (size_t)m * (N / 2) + (n >> 1);
                        split2(swiglu1(v, u), ohi[o], olo[o]);
                    }
                } else if (m < M && n < N) {
                    if (EPI == QK_GEMM_STORE) y[(size_t)m * N + n] = v;
                    else y[(size_t)m * N + n] += v;
                }
            }
        }
    }
}

template <int WM, int WN>
static void gemm_dispatch(const uint16_t *a_hi, const uint16_t *a_lo, const uint16_t *W, int M, int N, int K,
                          int epi, float *y, uint16_t *oh, uint16_t *ol, hipStream_t s) {
    dim3 grid((N + 32 * WN - 1) / (32 * WN), (M + 32 * WM - 1) / (32 * WM));
    if (epi == QK_GEMM_STORE) gemm_hilo<WM, WN, QK_GEMM_STORE><<<grid, 256, 0, s>>>(a_hi, a_lo, W, M, N, K, y, oh, ol);
    else if (epi == QK_GEMM_ADD) gemm_hilo<WM, WN, QK_GEMM_ADD><<<grid, 256, 0, s>>>(a_hi, a_lo, W, M, N, K, y, oh, ol);
    else gemm_hilo<WM, WN, QK_GEMM_SWIGLU><<<grid, 256, 0, s>>>(a_hi, a_lo, W, M, N, K, y, oh, ol);
}

extern "C" int qk_gemm_launch(const uint16_t *a_hi, const uint16_t *a_lo, const uint16_t *W, int M, int N, int K,
                              int epi, float *y, uint16_t *out_hi, uint16_t *out_lo, hipStream_t s) {
    if (M <= 0 || N <= 0 || K <= 0 || (K & 7) || !a_hi || !a_lo || !W) return QWEN_HIP_EINVAL;
    if (epi == QK_GEMM_SWIGLU ? (!out_hi || !out_lo || (N & 1)) : !y) return QWEN_HIP_EINVAL;
    if (M >= 256) gemm_dispatch<2, 2>(a_hi, a_lo, W, M, N, K, epi, y, out_hi, out_lo, s);
    else gemm_dispatch<1, 2>(a_hi, a_lo, W, M, N, K, epi, y, out_hi, out_lo, s);
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
    const float rinv = 1.0f / sqrtf(ss / (float)D + eps);
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
    const float rinv = 1.0f / sqrtf(ss / (float)hd + eps);
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
