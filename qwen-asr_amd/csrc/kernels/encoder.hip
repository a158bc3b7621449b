// encoder.hip - kernels of the audio encoder (reference qwen_asr_encoder.c:
// Conv2D stem -> conv_out projection + sinusoidal positions -> pre-LayerNorm
// transformer layers with windowed bidirectional attention -> ln_post,
// proj1 + GELU, proj2).
//
// Every matrix product runs on the fp32 matrix cores (v_mfma_f32_16x16x4_f32):
// the reference computes the encoder in fp32 on weights widened from bf16
// (load_bf16_as_f32, qwen_asr_encoder.c:43-65), so products stay exact fp32
// and only the summation order differs.
//
//   enc_im2col   Conv2D(3x3, stride 2, pad 1) patches of all chunks at once:
//                row n = (chunk, oh, ow), column k = (ki, kj, ic) tap-major
//                (the reference's im2col, qwen_asr_kernels.c:566-590, with
//                the weight columns reordered to match); the stem
//                activations are channel-last [chunk][h][w][480], and with
//                bf16 weights conv2 / conv3 skip this pass: the GEMM reads
//                the same patches straight from the activations
//   enc_gemm     C[M][N] = A[M][K] . B[N][K]^T with the encoder epilogues:
//                bias along M or N, GELU, residual add, positional table add,
//                zeroing of the padded positions of a partial last chunk
//   enc_stem_rows conv3 output [chunk][16][w][480] -> token rows [t][480*16]
//                (qwen_asr_encoder.c:281-290)
//   enc_layernorm  (x - mean) * inv_std * w + b, two-pass mean / variance
//                (qwen_layer_norm, qwen_asr_kernels.c:640-748)
//   enc_attention  bidirectional attention inside fixed token windows
//                (qwen_bidirectional_attention, qwen_asr_kernels.c:1003-1048)
#include "common.h"
#include "qk_kernels.h"
#include "qwen_asr_hip.h"

#include <math.h>

__device__ __forceinline__ f32x4 enc_mfma(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// GELU, tanh form (qwen_gelu, qwen_asr_kernels.c:886-893)
__device__ __forceinline__ float enc_gelu(float v) {
    const float x3 = v * v * v;
    const float inner = 0.7978845608028654f * (v + 0.044715f * x3);
    return 0.5f * v * (1.0f + tanhf(inner));
}

// ---------------------------------------------------------------------------
// im2col of one stem layer over every chunk.  in: conv1 the mel [128][frames]
// (chunk c covering frames [c*cw, c*cw + cw), frames past `frames` read as
// 0); conv2 / conv3 channel-last [chunks][h_in][w_in][c_in].  cols:
// [chunks*h_out*w_out][kpad], the columns past c_in*9 zero.
// ---------------------------------------------------------------------------
// conv1 (one input channel, the mel read in place): thread = (row, k), 256 / kpad
// rows per block, 32-bit index math
__global__ __launch_bounds__(256) void enc_im2col_mel(const float *mel, float *cols, int rows, int h_in, int w_in,
                                                      int h_out, int w_out, int kpad, int mel_frames) {
    const int rpb = 256 / kpad, r = threadIdx.x / kpad, k = threadIdx.x % kpad;
    for (int n0 = blockIdx.x * rpb; n0 < rows; n0 += gridDim.x * rpb) {
        const int n = n0 + r;
        if (r >= rpb || n >= rows) continue;
        const int ow = n % w_out, t = n / w_out, oh = t % h_out, c = t / h_out;
        float v = 0.0f;
        if (k < 9) {
            const int ih = 2 * oh - 1 + k / 3, iw = 2 * ow - 1 + k % 3;
            const int f = c * w_in + iw;
            if (ih >= 0 && ih < h_in && iw >= 0 && iw < w_in && f < mel_frames) v = mel[(long)ih * mel_frames + f];
        }
        cols[(long)n * kpad + k] = v;
    }
}

// conv2 / conv3 on channel-last input [chunk][h_in][w_in][c_in]: one block
// per row n = (chunk, oh, ow); k = tap * c_in + ic, so each tap is c_in
// contiguous floats of one input pixel (float4 copies, both sides coalesced)
__global__ __launch_bounds__(256) void enc_im2col(const float *in, float *cols, int c_in, int chunks, int rows,
                                                  int h_in, int w_in, int h_out, int w_out, int kpad) {
    const int q4 = c_in / 4;
    for (int n = blockIdx.x; n < rows; n += gridDim.x) {
        const int ow = n % w_out, t = n / w_out, oh = t % h_out, c = t / h_out;
        float *dst = cols + (long)n * kpad;
        for (int i = threadIdx.x; i < 9 * q4; i += 256) {
            const int tap = i / q4, q = i - tap * q4;
            const int ih = 2 * oh - 1 + tap / 3, iw = 2 * ow - 1 + tap % 3;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (ih >= 0 && ih < h_in && iw >= 0 && iw < w_in)
                v = *reinterpret_cast<const float4 *>(in + (((long)c * h_in + ih) * w_in + iw) * c_in + 4 * q);
            *reinterpret_cast<float4 *>(dst + tap * c_in + 4 * q) = v;
        }
        for (int k = 9 * c_in + threadIdx.x; k < kpad; k += 256) dst[k] = 0.0f;
    }
}

extern "C" int qk_enc_im2col_launch(const float *in, float *cols, int c_in, int chunks, int h_in, int w_in,
                                    int h_out, int w_out, int kpad, int mel_frames, hipStream_t s) {
    if (!in || !cols || c_in <= 0 || chunks <= 0 || kpad < c_in * 9 || (kpad & 15)) return QWEN_HIP_EINVAL;
    if (mel_frames <= 0 && (c_in & 3)) return QWEN_HIP_EINVAL;
    const long rows = (long)chunks * h_out * w_out;
    if (rows > 0x7fffffffL) return QWEN_HIP_EINVAL;
    if (mel_frames > 0) {
        if (c_in != 1 || kpad > 256 || 256 % kpad) return QWEN_HIP_EINVAL;
        const long rpb = 256 / kpad, blocks = (rows + rpb - 1) / rpb;
        enc_im2col_mel<<<(int)(blocks < 65536 ? blocks : 65536), 256, 0, s>>>(in, cols, (int)rows, h_in, w_in, h_out,
                                                                              w_out, kpad, mel_frames);
    } else {
        enc_im2col<<<(int)(rows < 65536 ? rows : 65536), 256, 0, s>>>(in, cols, c_in, chunks, (int)rows, h_in, w_in,
                                                                     h_out, w_out, kpad);
    }
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// ---------------------------------------------------------------------------
// fp32 GEMM on v_mfma_f32_16x16x4_f32.  Block tile 64 x 64, 4 waves of 32 x 32
// (2 x 2 MFMA tiles), K walked 16 at a time through LDS with the next tile's
// loads in flight.  Within a 16-wide k block lane l supplies k = 4 (l >> 4) + c
// at k-step c for both operands (each lane reads one float4 per row).
// ---------------------------------------------------------------------------
#define EG_T 64
#define EG_K 16
#define EG_LD (EG_K + 4)

// the encoder epilogues on element (m, n) of C (y points at it)
__device__ __forceinline__ void enc_epilogue(const qk_enc_gemm_args &a, int m, int n, float v, float *y) {
    if (a.bias_m) v += a.bias_m[m];
    if (a.bias_n) v += a.bias_n[n];
    if (a.pe) v += a.pe[(long)(m % a.pe_rows) * a.N + n];
    if (a.gelu) v = enc_gelu(v);
    if (a.col_w > 0) {
        // stem output position (chunk, oh, ow) (column n, or row m when
        // pad_rows): the last chunk's positions past its valid width are the
        // zero padding the reference's next convolution sees
        const int p = a.pad_rows ? m : n;
        const int ow = p % a.col_w, c = p / (a.col_w * a.col_h);
        if (c == a.col_chunks - 1 && ow >= a.col_valid) v = 0.0f;
    }
    if (a.add) v += *y;                    // residual (qwen_add_inplace after the projection)
    *y = v;
}

__global__ __launch_bounds__(256) void enc_gemm(qk_enc_gemm_args a) {
    __shared__ __attribute__((aligned(16))) float sA[EG_T][EG_LD];
    __shared__ __attribute__((aligned(16))) float sB[EG_T][EG_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * EG_T, n0 = blockIdx.x * EG_T;
    const int lr = tid >> 2, lk = (tid & 3) * 4;      // loader: row lr, k lk .. lk+3 of the tile

    float4 ra, rb;
    auto gload = [&](int k0) {
        const int gm = m0 + lr, gn = n0 + lr, gk = k0 + lk;
        ra = (gm < a.M && gk < a.K) ? *reinterpret_cast<const float4 *>(a.A + (long)gm * a.lda + gk)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
        rb = (gn < a.N && gk < a.K) ? *reinterpret_cast<const float4 *>(a.B + (long)gn * a.ldb + gk)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // K slice of this block: [kb, ke); kc is a multiple of EG_K, so every
    // 16-wide step but the last one of the whole product lies inside K
    const int kb = blockIdx.z * a.kc, ke = min(a.K, kb + a.kc);
    gload(kb);
    for (int k0 = kb; k0 < ke; k0 += EG_K) {
        __syncthreads();
        *reinterpret_cast<float4 *>(&sA[lr][lk]) = ra;
        *reinterpret_cast<float4 *>(&sB[lr][lk]) = rb;
        __syncthreads();
        if (k0 + EG_K < ke) gload(k0 + EG_K);
        float4 af[2], bf[2];
#pragma unroll
        for (int i = 0; i < 2; i++) af[i] = *reinterpret_cast<const float4 *>(&sA[wm * 32 + i * 16 + (lane & 15)][4 * (lane >> 4)]);
#pragma unroll
        for (int j = 0; j < 2; j++) bf[j] = *reinterpret_cast<const float4 *>(&sB[wn * 32 + j * 16 + (lane & 15)][4 * (lane >> 4)]);
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) acc[i][j] = enc_mfma((&af[i].x)[c], (&bf[j].x)[c], acc[i][j]);
    }

    // D[4 (l >> 4) + r][l & 15] of each 16 x 16 tile: rows m, column n
    float *part = a.split > 1 ? a.ws + (long)blockIdx.z * a.M * a.N : nullptr;
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn * 32 + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
                if (m >= a.M || n >= a.N) continue;
                if (part)
                    part[(long)m * a.N + n] = acc[i][j][r];
                else
                    enc_epilogue(a, m, n, acc[i][j][r], a.C + (long)m * a.ldc + n);
            }
        }
    }
}

// split-K: C = epilogue(sum of the slices' partials, slice 0 first)
__global__ __launch_bounds__(256) void enc_gemm_reduce(qk_enc_gemm_args a) {
    const long MN = (long)a.M * a.N;
    for (long e = blockIdx.x * 256L + threadIdx.x; e < MN; e += (long)gridDim.x * 256) {
        float v = a.ws[e];
        for (int z = 1; z < a.split; z++) v += a.ws[z * MN + e];
        const int m = (int)(e / a.N), n = (int)(e % a.N);
        enc_epilogue(a, m, n, v, a.C + (long)m * a.ldc + n);
    }
}

// ---------------------------------------------------------------------------
// The same product with one operand bf16 (the weights, exact) and the other
// fp32, split on the way into LDS as hi = bf16(x), lo = bf16(x - hi):
// x.w = hi.w + lo.w on v_mfma_f32_16x16x32_bf16 (fp32 accumulation).  Block
// tile 64 x 64, 4 waves of 32 x 32, K 32 at a time (one MFMA k-step), the next
// tile's loads in flight during the MFMAs.  WA: the bf16 operand is A (rows
// M); otherwise B (rows N).  Fragments: lane l supplies row (l & 15), k
// 8 (l >> 4) .. + 7, for both operands.
// ---------------------------------------------------------------------------
#define EH_K 32
#define EH_LD (EH_K + 8)           // 80-byte rows: 16-row fragment reads conflict free
typedef float eh_f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 eh_bf16x4 __attribute__((ext_vector_type(4)));

template <bool WA, int TT>        // TT x TT MFMA tiles of 16 x 16 per wave: block tile 32 TT x 32 TT
__global__ __launch_bounds__(256) void enc_gemm_hl(qk_enc_gemm_args a) {
    constexpr int BT = 32 * TT;                       // block tile edge
    constexpr int XPT = BT * EH_K / 4 / 256;          // fp32 float4 loads per thread
    constexpr int WPT = BT * EH_K / 8 / 256;          // bf16 16-byte loads per thread
    __shared__ __attribute__((aligned(16))) __bf16 sX[2][BT][EH_LD];   // fp32 operand: [hi, lo]
    __shared__ __attribute__((aligned(16))) __bf16 sW[BT][EH_LD];      // bf16 operand
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BT, n0 = blockIdx.x * BT;
    // fp32 side: rows of X = M rows of A (WA false) or N rows of B (WA true)
    const float *X = WA ? a.B : a.A;
    const uint16_t *W = WA ? a.A16 : a.B16;
    const int ldx = WA ? a.ldb : a.lda, ldw = WA ? a.lda : a.ldb;
    const int xr0 = WA ? n0 : m0, xrn = WA ? a.N : a.M;
    const int wr0 = WA ? m0 : n0, wrn = WA ? a.M : a.N;
    // loaders: X rows xr + 32 i (4 floats at xk), W rows wr + 64 i (8 bf16 at wk)
    const int xr = tid >> 3, xk = (tid & 7) * 4;
    const int wr = tid >> 2, wk = (tid & 3) * 8;

    float4 rx[XPT];
    uint4 rw[WPT];
    // implicit im2col (A side only): this thread's rows as (input plane base,
    // top-left input row / column of the 3x3 window); -1 marks rows past M
    const bool conv = !WA && a.conv_c > 0;
    int cb[XPT], ci[XPT], cj[XPT];
    if (conv) {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int g = xr0 + xr + 32 * i;
            const int ow = g % a.col_w, t = g / a.col_w, oh = t % a.col_h, c = t / a.col_h;
            cb[i] = g < xrn ? c * a.conv_in_h * a.conv_in_w : -1;
            ci[i] = 2 * oh - 1;
            cj[i] = 2 * ow - 1;
        }
    }
    auto gload = [&](int k0) {
        if (conv) {
            // a 32-wide k tile lies in one tap: channels ic .. ic + 3 of one input pixel
            const int tap = k0 / a.conv_c, ic = k0 - tap * a.conv_c + xk;
            const int dy = tap / 3, dx = tap - 3 * dy;
#pragma unroll
            for (int i = 0; i < XPT; i++) {
                const int ih = ci[i] + dy, iw = cj[i] + dx;
                const bool ok = cb[i] >= 0 && ih >= 0 && ih < a.conv_in_h && iw >= 0 && iw < a.conv_in_w;
                rx[i] = ok ? *reinterpret_cast<const float4 *>(X + ((long)cb[i] + ih * a.conv_in_w + iw) * a.conv_c + ic)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        } else {
#pragma unroll
            for (int i = 0; i < XPT; i++) {
                const int g = xr0 + xr + 32 * i, gk = k0 + xk;
                rx[i] = (g < xrn && gk < a.K) ? *reinterpret_cast<const float4 *>(X + (long)g * ldx + gk)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int i = 0; i < WPT; i++) {
            const int g = wr0 + wr + 64 * i, gk = k0 + wk;
            rw[i] = (g < wrn && gk < a.K) ? *reinterpret_cast<const uint4 *>(W + (long)g * ldw + gk)
                                          : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const eh_f32x4 x = {rx[i].x, rx[i].y, rx[i].z, rx[i].w};
            const eh_bf16x4 hi = __builtin_convertvector(x, eh_bf16x4);
            const eh_bf16x4 lo = __builtin_convertvector(x - __builtin_convertvector(hi, eh_f32x4), eh_bf16x4);
            *reinterpret_cast<eh_bf16x4 *>(&sX[0][xr + 32 * i][xk]) = hi;
            *reinterpret_cast<eh_bf16x4 *>(&sX[1][xr + 32 * i][xk]) = lo;
        }
#pragma unroll
        for (int i = 0; i < WPT; i++) *reinterpret_cast<uint4 *>(&sW[wr + 64 * i][wk]) = rw[i];
    };
    f32x4 acc[TT][TT];
#pragma unroll
    for (int i = 0; i < TT; i++)
#pragma unroll
        for (int j = 0; j < TT; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    const int kb = blockIdx.z * a.kc, ke = min(a.K, kb + a.kc);
    gload(kb);
    for (int k0 = kb; k0 < ke; k0 += EH_K) {
        __syncthreads();
        lstore();
        __syncthreads();
        if (k0 + EH_K < ke) gload(k0 + EH_K);
        const int kf = 8 * (lane >> 4);
        bf16x8 fm[TT][2], fn[TT][2];    // [tile][hi / lo or weight]: M-side and N-side fragments
#pragma unroll
        for (int i = 0; i < TT; i++) {
            const int rm = wm * 16 * TT + i * 16 + (lane & 15), rn = wn * 16 * TT + i * 16 + (lane & 15);
            if (WA) {
                fm[i][0] = *reinterpret_cast<const bf16x8 *>(&sW[rm][kf]);
                fn[i][0] = *reinterpret_cast<const bf16x8 *>(&sX[0][rn][kf]);
                fn[i][1] = *reinterpret_cast<const bf16x8 *>(&sX[1][rn][kf]);
            } else {
                fm[i][0] = *reinterpret_cast<const bf16x8 *>(&sX[0][rm][kf]);
                fm[i][1] = *reinterpret_cast<const bf16x8 *>(&sX[1][rm][kf]);
                fn[i][0] = *reinterpret_cast<const bf16x8 *>(&sW[rn][kf]);
            }
        }
#pragma unroll
        for (int i = 0; i < TT; i++)
#pragma unroll
            for (int j = 0; j < TT; j++) {
                if (WA) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fm[i][0], fn[j][0], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fm[i][0], fn[j][1], acc[i][j], 0, 0, 0);
                } else {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fm[i][0], fn[j][0], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fm[i][1], fn[j][0], acc[i][j], 0, 0, 0);
                }
            }
    }

    float *part = a.split > 1 ? a.ws + (long)blockIdx.z * a.M * a.N : nullptr;
#pragma unroll
    for (int i = 0; i < TT; i++) {
#pragma unroll
        for (int j = 0; j < TT; j++) {
            const int n = n0 + wn * 16 * TT + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * 16 * TT + i * 16 + 4 * (lane >> 4) + r;
                if (m >= a.M || n >= a.N) continue;
                if (part)
                    part[(long)m * a.N + n] = acc[i][j][r];
                else
                    enc_epilogue(a, m, n, acc[i][j][r], a.C + (long)m * a.ldc + n);
            }
        }
    }
}

// split-K reduce of one row (block per row, N <= 1024) that then LayerNorms
// the finished row into ln_out, with enc_layernorm's element-to-thread map and
// reduction order (so the result equals a separate LayerNorm pass)
__global__ __launch_bounds__(256) void enc_gemm_reduce_ln(qk_enc_gemm_args a) {
    __shared__ float red[4];
    const int m = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long MN = (long)a.M * a.N;
    float v[4];
    float s = 0.0f;
    float x[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {      // every slice of the row's 4 columns in one batch of loads
        const int n = min(threadIdx.x + 256 * j, a.N - 1);
        x[j] = sum_splits<8>(a.ws + (long)m * a.N + n, a.split, MN);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = threadIdx.x + 256 * j;
        v[j] = 0.0f;
        if (n < a.N) {
            float *y = a.C + (long)m * a.ldc + n;
            enc_epilogue(a, m, n, x[j], y);
            v[j] = *y;
            s += v[j];
        }
    }
    s = wave_sum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    const float mean = (red[0] + red[1] + red[2] + red[3]) / (float)a.N;
    __syncthreads();
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = threadIdx.x + 256 * j;
        if (n < a.N) {
            const float d = v[j] - mean;
            q = fmaf(d, d, q);
        }
    }
    q = wave_sum(q);
    if (lane == 0) red[wave] = q;
    __syncthreads();
    const float var = (red[0] + red[1] + red[2] + red[3]) / (float)a.N;
    const float inv_std = 1.0f / sqrtf(var + a.ln_eps);
    float *o = a.ln_out + (long)m * a.N;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = threadIdx.x + 256 * j;
        if (n < a.N) o[n] = (v[j] - mean) * inv_std * a.ln_w[n] + a.ln_b[n];
    }
}

extern "C" int qk_enc_gemm_launch(const qk_enc_gemm_args *a, hipStream_t s) {
    if (!a || (a->A16 && a->B16)) return QWEN_HIP_EINVAL;
    const bool hl = a->A16 || a->B16;
    if (!(a->A || a->A16) || !(a->B || a->B16) || !a->C || a->M <= 0 || a->N <= 0 || a->K <= 0 || (a->K & 3) ||
        (a->lda & 3) || (a->ldb & 3) || a->lda < a->K || a->ldb < a->K || a->ldc < a->N || (a->pe && a->pe_rows <= 0))
        return QWEN_HIP_EINVAL;
    if (hl && ((a->K % EH_K) || (a->A16 ? (a->lda & 7) || !a->B : (a->ldb & 7) || !a->A))) return QWEN_HIP_EINVAL;
    if (a->conv_c > 0 && (!a->B16 || a->conv_c % EH_K || a->K != 9 * a->conv_c || a->col_w <= 0 || a->col_h <= 0 ||
                          a->conv_in_h <= 0 || a->conv_in_w <= 0 || !a->pad_rows))
        return QWEN_HIP_EINVAL;
    if (a->ln_out && (!a->ln_w || !a->ln_b)) return QWEN_HIP_EINVAL;
    const int kstep = hl ? EH_K : EG_K;
    qk_enc_gemm_args g = *a;
    const long tiles = (long)((a->N + EG_T - 1) / EG_T) * ((a->M + EG_T - 1) / EG_T);
    // slices so that the grid holds ~4 blocks per CU, each slice >= 128 deep
    int split = a->ws ? (int)((1024 + tiles - 1) / tiles) : 1;
    if (split > 8) split = 8;
    if (split > a->K / 128) split = a->K / 128;
    if (split < 1) split = 1;
    g.kc = ((a->K + split - 1) / split + kstep - 1) / kstep * kstep;
    g.split = (a->K + g.kc - 1) / g.kc;
    if (g.split > 1 && (long)g.split * a->M * a->N > a->ws_elems) g.kc = a->K, g.split = 1;
    if (g.split == 1) g.kc = a->K;
    dim3 grid((a->N + EG_T - 1) / EG_T, (a->M + EG_T - 1) / EG_T, g.split);
    // large products (the stem convolutions) take 128 x 128 tiles: half the
    // operand bytes per MFMA, which the per-CU load path needs at full rate
    const bool big = hl && g.split == 1 && (long)a->M * a->N >= (1L << 22);
    dim3 grid2((a->N + 127) / 128, (a->M + 127) / 128, 1);
    if (a->A16) {
        if (big) enc_gemm_hl<true, 4><<<grid2, 256, 0, s>>>(g);
        else enc_gemm_hl<true, 2><<<grid, 256, 0, s>>>(g);
    } else if (a->B16) {
        if (big) enc_gemm_hl<false, 4><<<grid2, 256, 0, s>>>(g);
        else enc_gemm_hl<false, 2><<<grid, 256, 0, s>>>(g);
    } else {
        enc_gemm<<<grid, 256, 0, s>>>(g);
    }
    const bool ln = a->ln_out != nullptr;
    if (g.split > 1 && g.split <= 8 && ln && a->N <= 1024 && a->ldc == a->N) {
        enc_gemm_reduce_ln<<<a->M, 256, 0, s>>>(g);
        return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
    }
    if (g.split > 1) {
        long blocks = ((long)a->M * a->N + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        enc_gemm_reduce<<<(int)blocks, 256, 0, s>>>(g);
    }
    if (hipGetLastError() != hipSuccess) return QWEN_HIP_EDEVICE;
    if (ln) {
        if (a->ldc != a->N) return QWEN_HIP_EINVAL;
        return qk_enc_layernorm_launch(a->C, a->ln_w, a->ln_b, a->ln_out, a->M, a->N, a->ln_eps, s);
    }
    return 0;
}

// conv3 output [480][chunks][16][w] -> rows [token][480*16], token = chunk*w + t for
// t < the chunk's token count (qwen_asr_encoder.c:281-290: column ch*16 + f)
__global__ __launch_bounds__(256) void enc_stem_rows(const float *c3, float *rows, int chunks, int w, int h,
                                                     int ch_n, int tokens) {
    const int D = ch_n * h;
    const long total = (long)tokens * D;
    for (long e = blockIdx.x * 256L + threadIdx.x; e < total; e += (long)gridDim.x * 256) {
        const int tok = (int)(e / D), col = (int)(e % D);
        const int ch = col / h, f = col % h;
        const int c = tok / w, t = tok % w;
        rows[e] = c3[(((long)c * h + f) * w + t) * ch_n + ch];   // c3 channel-last [chunk][h][w][ch]
    }
}

// conv1 directly from its patches (one input channel, 9 taps in cols[pos][kpad]):
// out[pos][ch] = GELU(b[ch] + sum_tap cols[pos][tap] w[ch][tap]) for 4
// channels per thread, float4 stores, so each position's 480 outputs are one
// contiguous run (the product is 9 multiply-adds per output: the pass is
// bound by the 4 bytes it writes per output).  Positions (chunk, oh, ow) of
// the last chunk with ow >= valid are the zero padding the next layer sees.
__global__ __launch_bounds__(256) void enc_conv1(const float *cols, int kpad, const float *w, const float *b, float *out,
                                                 int rows, int ch, int h_out, int w_out, int chunks, int valid) {
    // the grid stride is a multiple of ch / 4, so a thread keeps one channel
    // quad (its 36 weights and 4 biases in registers) for every position it visits
    const int q4 = ch / 4;
    const long i0 = blockIdx.x * 256L + threadIdx.x, stride = (long)gridDim.x * 256;
    const int c0 = 4 * (int)(i0 % q4);
    float wr[4][9], br[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        br[j] = b[c0 + j];
#pragma unroll
        for (int t = 0; t < 9; t++) wr[j][t] = w[(c0 + j) * kpad + t];
    }
    for (long i = i0; i < (long)rows * q4; i += stride) {
        const int pos = (int)(i / q4);
        const int ow = pos % w_out, cc = pos / (w_out * h_out);
        const float *x = cols + (long)pos * kpad;
        float v[4] = {br[0], br[1], br[2], br[3]};
#pragma unroll
        for (int t = 0; t < 9; t++) {
            const float xt = x[t];
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = fmaf(xt, wr[j][t], v[j]);
        }
        const bool pad = cc == chunks - 1 && ow >= valid;
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = pad ? 0.0f : enc_gelu(v[j]);
        *reinterpret_cast<float4 *>(out + (long)pos * ch + c0) = make_float4(v[0], v[1], v[2], v[3]);
    }
}

extern "C" int qk_enc_conv1_launch(const float *cols, int kpad, const float *w, const float *b, float *out, int rows,
                                   int ch, int h_out, int w_out, int chunks, int valid, hipStream_t s) {
    if (!cols || !w || !b || !out || rows <= 0 || (ch & 3) || kpad < 9 || h_out <= 0 || w_out <= 0 || chunks <= 0)
        return QWEN_HIP_EINVAL;
    // blocks: a multiple of q4 / gcd(q4, 256) so the grid stride is a multiple of q4
    const int q4 = ch / 4;
    int g = q4, t = 256;
    while (t) { const int r = g % t; g = t; t = r; }
    const long unit = q4 / g;
    long blocks = ((long)rows * q4 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    blocks = (blocks + unit - 1) / unit * unit;
    enc_conv1<<<(int)blocks, 256, 0, s>>>(cols, kpad, w, b, out, rows, ch, h_out, w_out, chunks, valid);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

extern "C" int qk_enc_stem_rows_launch(const float *c3, float *rows, int chunks, int w, int h, int ch_n, int tokens,
                                       hipStream_t s) {
    if (!c3 || !rows || tokens <= 0 || tokens > chunks * w) return QWEN_HIP_EINVAL;
    long blocks = ((long)tokens * ch_n * h + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    enc_stem_rows<<<(int)blocks, 256, 0, s>>>(c3, rows, chunks, w, h, ch_n, tokens);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// ---------------------------------------------------------------------------
// LayerNorm, one block per row (qwen_layer_norm: mean, then mean of squared
// deviations, then (x - mean) * inv_std * w + b).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void enc_layernorm(const float *x, const float *w, const float *b, float *out,
                                                     int D, float eps) {
    __shared__ float red[4];
    const float *xr = x + (long)blockIdx.x * D;
    float *orow = out + (long)blockIdx.x * D;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float s = 0.0f;
    for (int i = threadIdx.x; i < D; i += 256) s += xr[i];
    s = wave_sum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    const float mean = (red[0] + red[1] + red[2] + red[3]) / (float)D;
    __syncthreads();
    float v = 0.0f;
    for (int i = threadIdx.x; i < D; i += 256) {
        const float d = xr[i] - mean;
        v = fmaf(d, d, v);
    }
    v = wave_sum(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    const float var = (red[0] + red[1] + red[2] + red[3]) / (float)D;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (int i = threadIdx.x; i < D; i += 256) orow[i] = (xr[i] - mean) * inv_std * w[i] + b[i];
}

extern "C" int qk_enc_layernorm_launch(const float *x, const float *w, const float *b, float *out, int rows, int D,
                                       float eps, hipStream_t s) {
    if (!x || !w || !b || !out || rows <= 0 || D <= 0) return QWEN_HIP_EINVAL;
    enc_layernorm<<<rows, 256, 0, s>>>(x, w, b, out, D, eps);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// ---------------------------------------------------------------------------
// Windowed bidirectional attention, head_dim 64, on the fp32 matrix cores.
// Block = one wave: 16 queries of one window, one head.  S^T = K Q^T and
// O^T += V^T P^T on v_mfma_f32_16x16x4_f32: lane l holds query l & 15, keys
// (first product) and dims (second) 4 (l >> 4) + r of each 16-row tile, so
// the scores come out in the register layout the second product takes as
// its B operand.  Online softmax over blocks of 64 keys of the window
// [ws, we); K and V are read straight from qkv [T][3 H 64] (q | k | v).
// ---------------------------------------------------------------------------
#define EA_Q 16
#define EA_KB 64

__global__ __launch_bounds__(64) void enc_attention(const float *qkv, float *out, int T, int H, int win, float scale) {
    constexpr int hd = 64;
    const int lane = threadIdx.x, h = blockIdx.y;
    const int lq = lane & 15, lg = lane >> 4;
    const int tpw = (win + EA_Q - 1) / EA_Q;
    const int ws = (blockIdx.x / tpw) * win, we = min(T, ws + win);
    const int q0 = ws + (blockIdx.x % tpw) * EA_Q;
    if (q0 >= we) return;                              // whole block: a short last window
    const long stride = 3L * H * hd;
    const int qi = q0 + lq;
    const float *qrow = qkv + (long)min(qi, T - 1) * stride + h * hd;
    const float *kbase = qkv + (long)H * hd + h * hd, *vbase = qkv + 2L * H * hd + h * hd;

    float4 q[4];                                       // Q^T operand: dims 16 kb + 4 lg + c
#pragma unroll
    for (int kb = 0; kb < 4; kb++) q[kb] = *reinterpret_cast<const float4 *>(qrow + 16 * kb + 4 * lg);
    f32x4 o[4];                                        // O^T[16 dt + 4 lg + r][query lq]
#pragma unroll
    for (int dt = 0; dt < 4; dt++) o[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m = -1e30f, l = 0.0f;                        // the reference's max_score start

    for (int k0 = ws; k0 < we; k0 += EA_KB) {
        float p[4][4];                                 // key k0 + 16 t + 4 lg + r
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float *krow = kbase + (long)min(k0 + 16 * t + lq, T - 1) * stride;
            f32x4 acc = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                const float4 kk = *reinterpret_cast<const float4 *>(krow + 16 * kb + 4 * lg);
#pragma unroll
                for (int c = 0; c < 4; c++) acc = enc_mfma((&kk.x)[c], (&q[kb].x)[c], acc);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                p[t][r] = k0 + 16 * t + 4 * lg + r < we ? acc[r] * scale : -INFINITY;
                mx = fmaxf(mx, p[t][r]);
            }
        }
        mx = xor_max16_32(mx);
        const float mn = fmaxf(m, mx);
        const float corr = __expf(m - mn);
        float sum = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                p[t][r] = __expf(p[t][r] - mn);
                sum += p[t][r];
            }
        l = fmaf(l, corr, sum);                        // this lane's keys; lane groups summed at the end
        m = mn;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) o[dt] *= corr;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            if (k0 + 16 * t >= we) break;              // uniform: the tile holds no key of the window
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float *vrow = vbase + (long)min(k0 + 16 * t + 4 * lg + c, T - 1) * stride;
#pragma unroll
                for (int dt = 0; dt < 4; dt++) o[dt] = enc_mfma(vrow[16 * dt + lq], p[t][c], o[dt]);
            }
        }
    }
    l = xor_sum16_32(l);
    if (qi >= we) return;
    const float inv = 1.0f / l;
    float *orow = out + (long)qi * H * hd + h * hd + 4 * lg;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
        *reinterpret_cast<float4 *>(orow + 16 * dt) =
            make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
}

extern "C" int qk_enc_attention_launch(const float *qkv, float *out, int T, int H, int hd, int win, float scale,
                                       hipStream_t s) {
    if (!qkv || !out || T <= 0 || H <= 0 || hd != 64 || win <= 0) return QWEN_HIP_EINVAL;
    const long nwin = (T + win - 1) / win, tpw = (win + EA_Q - 1) / EA_Q;
    if (nwin * tpw > 0x7fffffffL) return QWEN_HIP_EINVAL;
    dim3 grid((unsigned)(nwin * tpw), H);
    enc_attention<<<grid, 64, 0, s>>>(qkv, out, T, H, win, scale);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}
