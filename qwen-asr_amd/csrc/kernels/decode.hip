// decode.hip - bandwidth-bound kernels of the per-token step (gfx950, wave64).
//
//  gemv_kernel        y = W x with bf16 W streamed once from HBM, fp32 x held
//                     in registers, fp32 accumulation (reference
//                     qwen_bf16_matvec_fused_avx, qwen_asr_kernels_avx.c:25-155),
//                     with fused prologues (RMSNorm qwen_asr_kernels.c:750-809;
//                     embedding gather qwen_asr.c:353-360) and epilogues
//                     (residual add :159-161; SwiGLU on interleaved rows
//                     :902-959; LM-head argmax :518-543).
//  argmax_finish      second pass of the argmax over the per-block winners.
//  rope_append        per-head q/k RMSNorm (:811-873) + NeoX RoPE
//                     (:1182-1247) + K/V append (qwen_asr_decoder.c:446-447).
//  attn_decode_split  one query row against the fp32 KV cache, split over
//  attn_combine       positions (qwen_causal_attention, :1050-1141); used by
//                     the op-level ABI.
//  attn_decode_fused  the decoder's per-layer attention: q/k norm + RoPE + K/V
//                     append + split attention + in-kernel combine.
#include "common.h"
#include "qk_kernels.h"
#include "qwen_asr_hip.h"

#include <math.h>

// ---------------------------------------------------------------------------
// GEMV.  A wave owns ROWS consecutive rows; lane l covers columns
// [c*512 + 8l, c*512 + 8l + 8) for chunk c < NC, so one 16-byte load per lane
// per row per chunk streams the row at full coalescing.  The ROWS partial
// sums per lane are reduced with a transposing butterfly: each exchange
// halves the values a lane carries, so the whole reduction costs
// log2(ROWS) + 6 - log2(ROWS) + (ROWS - 1) shuffles instead of 6 * ROWS.
// ---------------------------------------------------------------------------
template <int NC, int ROWS>
__device__ __forceinline__ void gemv_load(uint4 (&w)[ROWS][NC], const uint16_t *W, int R, int K,
                                          int rbase, int lane) {
#pragma unroll
    for (int j = 0; j < ROWS; j++) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int col = c * 512 + lane * 8;
            const int r = rbase + j;
            if (r < R && col < K) w[j][c] = ld_stream16(W + (size_t)r * K + col);
            else w[j][c] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
}

// MERGE: the input is merged from attention splits (the O projection);
// only the argmax epilogue walks several row groups per wave (iters), so the
// other instances hold no second weight buffer and no merge registers.
template <int NC, int ROWS, int EPI, bool MERGE>
__global__ __launch_bounds__(256) void gemv_kernel(qk_gemv_args a, int iters_arg) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int K = a.K, R = a.rows;
    constexpr bool LOOP = EPI == QK_EPI_ARGMAX;
    const int iters = LOOP ? iters_arg : 1;

    // The first rows' weights do not depend on the input row: issue their
    // loads before the prologue so HBM latency overlaps the gather / norm.
    const int rows_per_block = 4 * ROWS * iters;
    uint4 w[ROWS][NC];
    int rbase = blockIdx.x * rows_per_block + wave * ROWS;
    if (rbase < R) gemv_load<NC, ROWS>(w, a.W, R, K, rbase, lane);

    // ---- prologue: the input row, optionally gathered and RMS-normed ----
    float xr[NC][8];
    int tok = -1;
    if (a.tok) tok = *a.tok;
    if constexpr (MERGE) {
        // The input is the attention output, merged here from its position
        // splits (m, l, o): x = (sum_s o_s e^(m_s - M)) * (1 / sum_s l_s e^(m_s - M)).
        // Thread t merges columns [8t, 8t + 8) into LDS for the whole block.
        // Every one of the merge_nsplit slots is valid: splits past the live
        // count were written with m = -inf by the attention kernel, so they
        // weigh 0 and no position read is needed here.
        __shared__ __attribute__((aligned(16))) float xs[QK_MERGE_MAX_K];
        const int ns = a.merge_nsplit;
        for (int t = threadIdx.x; t * 8 < K; t += 256) {
            const int col = t * 8, h = col >> 7, d = col & 127;
            const float *pm = a.merge_m + (size_t)h * a.merge_nsplit;
            const float *pl = a.merge_l + (size_t)h * a.merge_nsplit;
            const float *po = a.merge_o + (size_t)h * a.merge_nsplit * 128 + d;
            float mv[QK_MERGE_MAX_SPLIT], lv[QK_MERGE_MAX_SPLIT];
            float4 oa[QK_MERGE_MAX_SPLIT], ob[QK_MERGE_MAX_SPLIT];
#pragma unroll
            for (int s = 0; s < QK_MERGE_MAX_SPLIT; s++)
                if (s < ns) {
                    mv[s] = pm[s];
                    lv[s] = pl[s];
                    oa[s] = *reinterpret_cast<const float4 *>(po + (size_t)s * 128);
                    ob[s] = *reinterpret_cast<const float4 *>(po + (size_t)s * 128 + 4);
                }
            float M = -INFINITY;
#pragma unroll
            for (int s = 0; s < QK_MERGE_MAX_SPLIT; s++) if (s < ns) M = fmaxf(M, mv[s]);
            float L = 0.0f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < QK_MERGE_MAX_SPLIT; s++)
                if (s < ns) {
                    const float e = (mv[s] == -INFINITY) ? 0.0f : __expf(mv[s] - M);
                    L = fmaf(lv[s], e, L);
                    acc[0] = fmaf(oa[s].x, e, acc[0]); acc[1] = fmaf(oa[s].y, e, acc[1]);
                    acc[2] = fmaf(oa[s].z, e, acc[2]); acc[3] = fmaf(oa[s].w, e, acc[3]);
                    acc[4] = fmaf(ob[s].x, e, acc[4]); acc[5] = fmaf(ob[s].y, e, acc[5]);
                    acc[6] = fmaf(ob[s].z, e, acc[6]); acc[7] = fmaf(ob[s].w, e, acc[7]);
                }
            const float inv = 1.0f / L;        // the reference scales by 1/sum (qwen_asr_kernels.c:1091-1094)
#pragma unroll
            for (int j = 0; j < 8; j++) xs[col + j] = acc[j] * inv;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int col = c * 512 + lane * 8;
#pragma unroll
            for (int j = 0; j < 8; j++) xr[c][j] = (col < K) ? xs[col + j] : 0.0f;
        }
    } else
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int col = c * 512 + lane * 8;
        if (col < K) {
            if (tok >= 0) {
                uint4 e = *reinterpret_cast<const uint4 *>(a.emb + (size_t)tok * K + col);
                xr[c][0] = bf16_lo(e.x); xr[c][1] = bf16_hi(e.x);
                xr[c][2] = bf16_lo(e.y); xr[c][3] = bf16_hi(e.y);
                xr[c][4] = bf16_lo(e.z); xr[c][5] = bf16_hi(e.z);
                xr[c][6] = bf16_lo(e.w); xr[c][7] = bf16_hi(e.w);
            } else {
                float4 p0 = *reinterpret_cast<const float4 *>(a.x + col);
                float4 p1 = *reinterpret_cast<const float4 *>(a.x + col + 4);
                xr[c][0] = p0.x; xr[c][1] = p0.y; xr[c][2] = p0.z; xr[c][3] = p0.w;
                xr[c][4] = p1.x; xr[c][5] = p1.y; xr[c][6] = p1.z; xr[c][7] = p1.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) xr[c][j] = 0.0f;
        }
    }
    if (tok >= 0 && a.x_store && blockIdx.x == 0 && wave == 0) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int col = c * 512 + lane * 8;
            if (col < K)
#pragma unroll
                for (int j = 0; j < 8; j++) a.x_store[col + j] = xr[c][j];
        }
    }
    if (a.norm_w) {
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int j = 0; j < 8; j++) ss = fmaf(xr[c][j], xr[c][j], ss);
        ss = wave_sum(ss);
        const float rinv = rsqrt_norm(ss / (float)K + a.eps);
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int col = c * 512 + lane * 8;
            if (col < K)
#pragma unroll
                for (int j = 0; j < 8; j++) xr[c][j] = (xr[c][j] * a.norm_w[col + j]) * rinv;
        }
    }
    if (a.normed_store && blockIdx.x == 0 && wave == 0) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int col = c * 512 + lane * 8;
            if (col < K)
#pragma unroll
                for (int j = 0; j < 8; j++) a.normed_store[col + j] = xr[c][j];
        }
    }

    // ---- rows ----
    float best_v = -1e30f;
    int best_i = 0x7fffffff;
    // residual add: the old value of the row this lane will own after the
    // reduction, loaded now so its latency overlaps the weight stream
    float resid = 0.0f;
    if constexpr (EPI == QK_EPI_ADD) {
        const int r = rbase + lane / (64 / ROWS);
        if (iters == 1 && r < R) resid = a.y[r];
    }
    for (int it = 0; it < iters; it++) {
        if (rbase >= R) break;
        const int rnext = rbase + 4 * ROWS;
        const bool more = LOOP && (it + 1 < iters) && (rnext < R);
        uint4 wn[ROWS][NC];
        if (more) gemv_load<NC, ROWS>(wn, a.W, R, K, rnext, lane);

        float acc[ROWS];
#pragma unroll
        for (int j = 0; j < ROWS; j++) {
            acc[j] = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; c++) acc[j] = dot8_bf16(w[j][c], xr[c], acc[j]);
        }

        if constexpr (EPI == QK_EPI_SWIGLU) {
            reduce_rows<ROWS, 2>(acc, lane);
            const int span = 128 / ROWS;                 // lanes per (g,u) pair
            const int r = rbase + 2 * (lane / span);
            if ((lane % span) == 0 && r < R)
                a.y[r >> 1] = swiglu1(acc[0], acc[1]);
        } else {
            reduce_rows<ROWS, 1>(acc, lane);
            const int span = 64 / ROWS;
            const int r = rbase + lane / span;
            if ((lane % span) == 0 && r < R) {
                if constexpr (EPI == QK_EPI_STORE) a.y[r] = acc[0];
                else if constexpr (EPI == QK_EPI_ADD) a.y[r] = (iters == 1 ? resid : a.y[r]) + acc[0];
                else {
                    if (a.logits) a.logits[r] = acc[0];
                    if (argmax_better(acc[0], r, best_v, best_i)) { best_v = acc[0]; best_i = r; }
                }
            }
        }
        if (more) {
#pragma unroll
            for (int j = 0; j < ROWS; j++)
#pragma unroll
                for (int c = 0; c < NC; c++) w[j][c] = wn[j][c];
        }
        rbase = rnext;
    }

    if constexpr (EPI == QK_EPI_ARGMAX) {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            float ov = __shfl_xor(best_v, m, QK_WAVE);
            int oi = __shfl_xor(best_i, m, QK_WAVE);
            if (argmax_better(ov, oi, best_v, best_i)) { best_v = ov; best_i = oi; }
        }
        __shared__ float sv[4];
        __shared__ int si[4];
        if (lane == 0) { sv[wave] = best_v; si[wave] = best_i; }
        __syncthreads();
        if (threadIdx.x == 0) {
            float bv = sv[0];
            int bi = si[0];
            for (int i = 1; i < 4; i++)
                if (argmax_better(sv[i], si[i], bv, bi)) { bv = sv[i]; bi = si[i]; }
            a.cand_val[blockIdx.x] = bv;
            a.cand_idx[blockIdx.x] = bi;
        }
    }
}

// Long rows (STORE or ADD, plain x; gemv_ks_fits): the block's four waves split
// each row's 512-column chunks (wave w takes chunks w, w + 4, w + 8, ...) for
// the block's ROWS rows, so x is held once per block instead of once per wave
// and a wave needs a quarter of the registers; the four partial sums of a row
// meet in LDS and are added in wave order.
template <int NCW, int ROWS, int EPI>
__global__ __launch_bounds__(256) void gemv_ks(qk_gemv_args a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = a.K, R = a.rows;
    const int r0 = blockIdx.x * ROWS;
    uint4 w[ROWS][NCW];
#pragma unroll
    for (int j = 0; j < ROWS; j++)
#pragma unroll
        for (int c = 0; c < NCW; c++) {
            const int col = (wave + 4 * c) * 512 + lane * 8, r = r0 + j;
            w[j][c] = (r < R && col < K) ? ld_stream16(a.W + (size_t)r * K + col) : make_uint4(0u, 0u, 0u, 0u);
        }
    float resid = 0.0f;
    if (EPI == QK_EPI_ADD && threadIdx.x < ROWS && r0 + (int)threadIdx.x < R) resid = a.y[r0 + threadIdx.x];
    float xr[NCW][8];
#pragma unroll
    for (int c = 0; c < NCW; c++) {
        const int col = (wave + 4 * c) * 512 + lane * 8;
        if (col < K) {
            const float4 p0 = *reinterpret_cast<const float4 *>(a.x + col);
            const float4 p1 = *reinterpret_cast<const float4 *>(a.x + col + 4);
            xr[c][0] = p0.x; xr[c][1] = p0.y; xr[c][2] = p0.z; xr[c][3] = p0.w;
            xr[c][4] = p1.x; xr[c][5] = p1.y; xr[c][6] = p1.z; xr[c][7] = p1.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) xr[c][j] = 0.0f;
        }
    }
    float acc[ROWS];
#pragma unroll
    for (int j = 0; j < ROWS; j++) {
        acc[j] = 0.0f;
#pragma unroll
        for (int c = 0; c < NCW; c++) acc[j] = dot8_bf16(w[j][c], xr[c], acc[j]);
    }
    reduce_rows<ROWS, 1>(acc, lane);            // lane l: row l / (64 / ROWS)
    __shared__ float part[4][ROWS];
    constexpr int span = 64 / ROWS;
    if (lane % span == 0) part[wave][lane / span] = acc[0];
    __syncthreads();
    if (threadIdx.x < ROWS) {
        const int t = threadIdx.x, r = r0 + t;
        if (r < R) {
            const float v = ((part[0][t] + part[1][t]) + part[2][t]) + part[3][t];
            a.y[r] = EPI == QK_EPI_ADD ? resid + v : v;
        }
    }
}

// gemv_ks takes the product: a plain input row, STORE or ADD, rows longer
// than 2048 columns, or of 2048 columns with 4096 rows or more (measured,
// cold weights, eager launches: 2048 x 6144 7.07 -> 6.25 us, 12288 x 2048
// 9.97 -> 9.14 us; 2048 x 2048 3.59 -> 3.78 us, so not below 4096 rows)
static bool gemv_ks_fits(const qk_gemv_args *a) {
    const bool shape = a->K > 4 * 512 || (a->K == 4 * 512 && a->rows >= 4096);
    return shape && (a->epi == QK_EPI_STORE || a->epi == QK_EPI_ADD) && a->x && !a->tok && !a->merge_o &&
           !a->norm_w && !a->normed_store && !a->x_store;
}

template <int NCW>
static void gemv_ks_dispatch(const qk_gemv_args *a, hipStream_t s) {
    // ROWS rows per block: at least 512 blocks where the rows allow
    const int rows = a->rows >= 4 * 512 ? 4 : a->rows >= 2 * 512 ? 2 : 1;
    const int blocks = (a->rows + rows - 1) / rows;
#define QK_KS(RW)                                                                                   \
    if (rows == RW) {                                                                                 \
        if (a->epi == QK_EPI_STORE) gemv_ks<NCW, RW, QK_EPI_STORE><<<blocks, 256, 0, s>>>(*a);        \
        else gemv_ks<NCW, RW, QK_EPI_ADD><<<blocks, 256, 0, s>>>(*a);                                 \
    }
    QK_KS(4) QK_KS(2) QK_KS(1)
#undef QK_KS
}

static int gemv_pick_rows(int R, int epi) {
    if (epi == QK_EPI_ARGMAX) return 4;
    if (R / 16 >= 256) return 4;
    if (R / 8 >= 256 || epi == QK_EPI_SWIGLU) return 2;
    return 1;
}

static int gemv_pick_iters(int K, int epi) {
    if (epi != QK_EPI_ARGMAX) return 1;
    return K <= 1024 ? 8 : 4;
}

extern "C" int qk_gemv_blocks(int rows, int K, int epi) {
    const int per = 4 * gemv_pick_rows(rows, epi) * gemv_pick_iters(K, epi);
    return (rows + per - 1) / per;
}

template <int NC, int ROWS>
static void gemv_dispatch_epi(const qk_gemv_args *a, int iters, int blocks, hipStream_t s) {
    switch (a->epi) {
    case QK_EPI_STORE: gemv_kernel<NC, ROWS, QK_EPI_STORE, false><<<blocks, 256, 0, s>>>(*a, iters); break;
    case QK_EPI_ADD:
        if (a->merge_o) gemv_kernel<NC, ROWS, QK_EPI_ADD, true><<<blocks, 256, 0, s>>>(*a, iters);
        else gemv_kernel<NC, ROWS, QK_EPI_ADD, false><<<blocks, 256, 0, s>>>(*a, iters);
        break;
    case QK_EPI_SWIGLU:
        if (ROWS >= 2) gemv_kernel<NC, (ROWS >= 2 ? ROWS : 2), QK_EPI_SWIGLU, false><<<blocks, 256, 0, s>>>(*a, iters);
        break;
    default:
        if (ROWS == 4) gemv_kernel<NC, 4, QK_EPI_ARGMAX, false><<<blocks, 256, 0, s>>>(*a, iters);
        break;
    }
}

template <int NC>
static void gemv_dispatch_rows(const qk_gemv_args *a, int rows_pw, int iters, int blocks, hipStream_t s) {
    if (rows_pw == 4) gemv_dispatch_epi<NC, 4>(a, iters, blocks, s);
    else if (rows_pw == 2) gemv_dispatch_epi<NC, 2>(a, iters, blocks, s);
    else gemv_dispatch_epi<NC, 1>(a, iters, blocks, s);
}

extern "C" int qk_gemv_launch(const qk_gemv_args *a, hipStream_t s) {
    if (!a || !a->W || a->rows <= 0 || a->K <= 0 || (a->K & 7) || a->K > 12 * 512) return QWEN_HIP_EINVAL;
    if (a->epi == QK_EPI_SWIGLU && (a->rows & 1)) return QWEN_HIP_EINVAL;
    if (a->epi == QK_EPI_ARGMAX && (!a->cand_val || !a->cand_idx)) return QWEN_HIP_EINVAL;
    if (a->epi != QK_EPI_ARGMAX && !a->y) return QWEN_HIP_EINVAL;
    if (!a->x && !a->tok && !a->merge_o) return QWEN_HIP_EINVAL;
    if (a->merge_o && (!a->merge_m || !a->merge_l || a->merge_nsplit <= 0 ||
                       a->merge_nsplit > QK_MERGE_MAX_SPLIT || a->K > QK_MERGE_MAX_K || (a->K & 127) || a->tok))
        return QWEN_HIP_EINVAL;
    if (a->tok && !a->emb) return QWEN_HIP_EINVAL;
    if (gemv_ks_fits(a)) {
        const int ncw = (a->K + 4 * 512 - 1) / (4 * 512);
        if (ncw == 1) gemv_ks_dispatch<1>(a, s);
        else if (ncw == 2) gemv_ks_dispatch<2>(a, s);
        else gemv_ks_dispatch<3>(a, s);
        return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
    }
    const int rows_pw = gemv_pick_rows(a->rows, a->epi);
    const int iters = gemv_pick_iters(a->K, a->epi);
    const int blocks = qk_gemv_blocks(a->rows, a->K, a->epi);
    const int nc = (a->K + 511) / 512;
    switch (nc) {
    case 1: gemv_dispatch_rows<1>(a, rows_pw, iters, blocks, s); break;
    case 2: gemv_dispatch_rows<2>(a, rows_pw, iters, blocks, s); break;
    case 3:
    case 4: gemv_dispatch_rows<4>(a, rows_pw, iters, blocks, s); break;
    case 5:
    case 6: gemv_dispatch_rows<6>(a, rows_pw, iters, blocks, s); break;
    case 7:
    case 8: gemv_dispatch_rows<8>(a, rows_pw, iters, blocks, s); break;
    default: gemv_dispatch_rows<12>(a, rows_pw, iters, blocks, s); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// ---------------------------------------------------------------------------
// Argmax, second pass: one block reduces the per-block winners.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void argmax_finish(const float *cv, const int *ci, int n, int *tok_out,
                                                     int *log, int *counter, int *pos, unsigned *epoch) {
    float bv = -1e30f;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += 256)
        if (argmax_better(cv[i], ci[i], bv, bi)) { bv = cv[i]; bi = ci[i]; }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        float ov = __shfl_xor(bv, m, QK_WAVE);
        int oi = __shfl_xor(bi, m, QK_WAVE);
        if (argmax_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    __shared__ float sv[4];
    __shared__ int si[4];
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < 4; i++)
            if (argmax_better(sv[i], si[i], sv[0], si[0])) { sv[0] = sv[i]; si[0] = si[i]; }
        // nothing above the reference's -1e30 floor: it returns its start row
        const int t = si[0] == 0x7fffffff ? 0 : si[0];
        if (tok_out) *tok_out = t;
        if (log) {
            const int c = *counter;
            log[c] = t;
            *counter = c + 1;
        }
        if (pos) *pos = *pos + 1;
        if (epoch) *epoch = *epoch + 1;
    }
}

extern "C" int qk_argmax_finish_launch(const float *cand_val, const int *cand_idx, int n, int *tok_out,
                                       int *log, int *counter, int *pos, unsigned *epoch, hipStream_t s) {
    if (n <= 0 || !cand_val || !cand_idx || (log && !counter)) return QWEN_HIP_EINVAL;
    argmax_finish<<<1, 256, 0, s>>>(cand_val, cand_idx, n, tok_out, log, counter, pos, epoch);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// ---------------------------------------------------------------------------
// q/k RMSNorm + NeoX RoPE + K/V append.  A 16-lane group per (row, head);
// lane c owns dims 4c .. 4c+3 and their RoPE partners 64+4c .. 64+4c+3
// (norm_rope_row16).  Every access is a 16-byte vector.
// ---------------------------------------------------------------------------
// Unit u = 16 block + 4 wave + lane / 16: head = u % (heads + kv_heads)
// ([0, heads) q, then k/v), row = u / (heads + kv_heads).  NS: the most
// split-K partials summed (1: the product as is).
template <int NS>
__global__ __launch_bounds__(256) void rope_append(qk_rope_append_args a) {
    const int hd = QWEN_HIP_HEAD_DIM, half = hd / 2;
    const int c = threadIdx.x & 15;
    const int nh = a.heads + a.kv_heads;
    const long u = 16L * blockIdx.x + (threadIdx.x >> 4);
    if (u >= (long)nh * a.S) return;            // the whole 16-lane group
    const int head = (int)(u % nh);
    const int srow = (int)(u / nh);
    const int start = a.pos_dev ? *a.pos_dev : a.start;
    const int p = start + srow;
    const int qd = a.heads * hd, kvd = a.kv_heads * hd;
    const float *row = a.qkv + (size_t)srow * (qd + 2 * kvd);
    const bool is_q = head < a.heads;
    const int kvh = head - a.heads;
    const float *src = is_q ? row + head * hd : row + qd + kvh * hd;
    const float *nw = is_q ? a.q_norm : a.k_norm;
    const int ns = a.nsum > 0 ? a.nsum : 1;
    float4 lo = sum_splits4<NS>(src + 4 * c, ns, a.pstride);
    float4 hi = sum_splits4<NS>(src + half + 4 * c, ns, a.pstride);
    const float4 wl = *reinterpret_cast<const float4 *>(nw + 4 * c);
    const float4 wh = *reinterpret_cast<const float4 *>(nw + half + 4 * c);
    const float4 c4 = *reinterpret_cast<const float4 *>(a.rope_cos + (size_t)p * hd + 4 * c);
    const float4 s4 = *reinterpret_cast<const float4 *>(a.rope_sin + (size_t)p * hd + 4 * c);
    norm_rope_row16(lo, hi, wl, wh, c4, s4, a.eps);
    float *dst = is_q ? a.q_out + (size_t)srow * qd + head * hd : a.k_cache + ((size_t)kvh * a.cap + p) * hd;
    *reinterpret_cast<float4 *>(dst + 4 * c) = lo;
    *reinterpret_cast<float4 *>(dst + half + 4 * c) = hi;
    if (!is_q) {
        const float *vs = row + qd + kvd + kvh * hd;
        float *vd = a.v_cache + ((size_t)kvh * a.cap + p) * hd;
        *reinterpret_cast<float4 *>(vd + 4 * c) = sum_splits4<NS>(vs + 4 * c, ns, a.pstride);
        *reinterpret_cast<float4 *>(vd + half + 4 * c) = sum_splits4<NS>(vs + half + 4 * c, ns, a.pstride);
    }
}

extern "C" int qk_rope_append_launch(const qk_rope_append_args *a, hipStream_t s) {
    if (!a || a->S <= 0 || a->heads <= 0 || a->kv_heads <= 0 || a->heads % a->kv_heads ||
        a->nsum > QK_GEMM_MAX_SPLIT)
        return QWEN_HIP_EINVAL;
    // 16-byte accesses throughout
    const uintptr_t al = (uintptr_t)a->qkv | (uintptr_t)a->q_norm | (uintptr_t)a->k_norm | (uintptr_t)a->rope_cos |
                         (uintptr_t)a->rope_sin | (uintptr_t)a->k_cache | (uintptr_t)a->v_cache | (uintptr_t)a->q_out;
    if (al % 16 || (a->nsum > 1 && a->pstride % 4)) return QWEN_HIP_EINVAL;
    const long units = (long)(a->heads + a->kv_heads) * a->S;
    if ((units + 15) / 16 > 0x7fffffffL) return QWEN_HIP_EINVAL;
    if (a->nsum > 1) rope_append<QK_GEMM_MAX_SPLIT><<<(unsigned)((units + 15) / 16), 256, 0, s>>>(*a);
    else rope_append<1><<<(unsigned)((units + 15) / 16), 256, 0, s>>>(*a);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// ---------------------------------------------------------------------------
// Decode attention.  Block (kv head, split) covers a contiguous range of
// positions for the HPK query heads sharing that kv head, so each K/V row is
// read once for all of them.  Sixteen lanes own one position (8 dims each);
// a wave advances four positions per step and the four waves interleave.
// Online softmax runs per 16-lane group; groups and waves merge in LDS, and
// the splits merge in attn_combine.  Partials: [head][split][m, l, o[128]].
// ---------------------------------------------------------------------------
#define QK_OPATTN_MIN_CHUNK 32

__device__ __host__ __forceinline__ int attn_chunk(int seq_k, int nsplit) {
    int c = (seq_k + nsplit - 1) / nsplit;
    return c < QK_OPATTN_MIN_CHUNK ? QK_OPATTN_MIN_CHUNK : c;
}

template <int HPK>
__global__ __launch_bounds__(256) void attn_decode_split(qk_attn_args a) {
    const int hd = QWEN_HIP_HEAD_DIM;
    const int kvh = blockIdx.x, split = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, gl = lane & 15;
    const int seq_k = a.pos_dev ? *a.pos_dev + 1 : a.seq_k;
    const int chunk = attn_chunk(seq_k, a.nsplit);
    const int nsplit = (seq_k + chunk - 1) / chunk;
    if (split >= nsplit) return;
    const int s0 = split * chunk;
    const int s1 = min(s0 + chunk, seq_k);

    float q[HPK][8];
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        const float *qp = a.q + (size_t)(kvh * HPK + h) * hd + gl * 8;
        float4 q0 = *reinterpret_cast<const float4 *>(qp);
        float4 q1 = *reinterpret_cast<const float4 *>(qp + 4);
        q[h][0] = q0.x; q[h][1] = q0.y; q[h][2] = q0.z; q[h][3] = q0.w;
        q[h][4] = q1.x; q[h][5] = q1.y; q[h][6] = q1.z; q[h][7] = q1.w;
    }
    float m[HPK], l[HPK], o[HPK][8];
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) o[h][j] = 0.0f;
    }
    const float *kb = a.k + (size_t)kvh * a.head_stride + gl * 8;
    const float *vb = a.v + (size_t)kvh * a.head_stride + gl * 8;
    for (int p = s0 + wave * 4 + g; p < s1; p += 16) {
        const float *kp = kb + (size_t)p * a.pos_stride;
        const float *vp = vb + (size_t)p * a.pos_stride;
        float4 k0 = *reinterpret_cast<const float4 *>(kp);
        float4 k1 = *reinterpret_cast<const float4 *>(kp + 4);
        float4 v0 = *reinterpret_cast<const float4 *>(vp);
        float4 v1 = *reinterpret_cast<const float4 *>(vp + 4);
        const float kv[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
        const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int h = 0; h < HPK; h++) {
            float d = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) d = fmaf(q[h][j], kv[j], d);
            d = group_sum<16>(d);
            const float sc = d * a.scale;
            const float mn = fmaxf(m[h], sc);
            const float corr = __expf(m[h] - mn);
            const float pw = __expf(sc - mn);
            l[h] = fmaf(l[h], corr, pw);
#pragma unroll
            for (int j = 0; j < 8; j++) o[h][j] = fmaf(o[h][j], corr, pw * vv[j]);
            m[h] = mn;
        }
    }

    __shared__ float sm_m[16][HPK], sm_l[16][HPK];
    __shared__ float sm_o[16][HPK][128];
    const int grp = wave * 4 + g;
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        if (gl == 0) { sm_m[grp][h] = m[h]; sm_l[grp][h] = l[h]; }
#pragma unroll
        for (int j = 0; j < 8; j++) sm_o[grp][h][gl * 8 + j] = o[h][j];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < HPK * hd; t += 256) {
        const int h = t / hd, d = t % hd;
        float M = -INFINITY;
        for (int i = 0; i < 16; i++) M = fmaxf(M, sm_m[i][h]);
        float L = 0.0f, acc = 0.0f;
        for (int i = 0; i < 16; i++) {
            const float mi = sm_m[i][h];
            const float e = (mi == -INFINITY) ? 0.0f : __expf(mi - M);
            L = fmaf(sm_l[i][h], e, L);
            acc = fmaf(sm_o[i][h][d], e, acc);
        }
        float *pp = a.part + ((size_t)(kvh * HPK + h) * a.nsplit + split) * (hd + 2);
        if (d == 0) { pp[0] = M; pp[1] = L; }
        pp[2 + d] = acc;
    }
}

__global__ __launch_bounds__(128) void attn_combine(qk_attn_args a) {
    const int hd = QWEN_HIP_HEAD_DIM;
    const int h = blockIdx.x, d = threadIdx.x;
    const int seq_k = a.pos_dev ? *a.pos_dev + 1 : a.seq_k;
    const int chunk = attn_chunk(seq_k, a.nsplit);
    const int nsplit = (seq_k + chunk - 1) / chunk;
    const float *pp = a.part + (size_t)h * a.nsplit * (hd + 2);
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, pp[(size_t)s * (hd + 2)]);
    float L = 0.0f, acc = 0.0f;
    for (int s = 0; s < nsplit; s++) {
        const float *q = pp + (size_t)s * (hd + 2);
        const float e = (q[0] == -INFINITY) ? 0.0f : __expf(q[0] - M);
        L = fmaf(q[1], e, L);
        acc = fmaf(q[2 + d], e, acc);
    }
    // the reference normalises by multiplying with 1/sum (qwen_asr_kernels.c:1091-1094)
    a.out[(size_t)h * hd + d] = acc * (1.0f / L);
}

extern "C" int qk_attn_decode_launch(const qk_attn_args *a, hipStream_t s) {
    if (!a || a->heads <= 0 || a->kv_heads <= 0 || a->heads % a->kv_heads || a->nsplit <= 0 || !a->part)
        return QWEN_HIP_EINVAL;
    if (!a->pos_dev && a->seq_k <= 0) return QWEN_HIP_EINVAL;
    const int hpk = a->heads / a->kv_heads;
    dim3 grid(a->kv_heads, a->nsplit);
    switch (hpk) {
    case 1: attn_decode_split<1><<<grid, 256, 0, s>>>(*a); break;
    case 2: attn_decode_split<2><<<grid, 256, 0, s>>>(*a); break;
    case 4: attn_decode_split<4><<<grid, 256, 0, s>>>(*a); break;
    default: return QWEN_HIP_EINVAL;
    }
    attn_combine<<<a->heads, 128, 0, s>>>(*a);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// ---------------------------------------------------------------------------
// Fused decode attention: one launch per layer does what the reference does
// in qwen_asr_decoder.c:439-455 -- q/k RMSNorm, NeoX RoPE, K/V append at
// `pos`, causal GQA attention over [0, pos] -- split over positions.  Each
// 16-lane group owns every 16th position of its split and prefetches the
// K/V rows of its next QK_AB positions into registers while it folds the
// current ones into its online softmax, so the position loop streams instead
// of paying one memory latency per position.  Splits write unnormalised
// partials (m, l, o[128]) with plain stores; the merge runs in the next
// kernel (the O-projection prologue for <= 8 splits, attn_merge otherwise).
// ---------------------------------------------------------------------------
#define QK_AB 4

template <int HPK>
__device__ __forceinline__ void attn_fold(const float (&q)[HPK][8], float4 k0, float4 k1, float4 v0, float4 v1,
                                          float scale, float (&m)[HPK], float (&l)[HPK], float (&o)[HPK][8]) {
    const float kv[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) d = fmaf(q[h][j], kv[j], d);
        d = group_sum<16>(d);
        const float sc = d * scale;
        const float mn = fmaxf(m[h], sc);
        const float corr = __expf(m[h] - mn), pw = __expf(sc - mn);
        l[h] = fmaf(l[h], corr, pw);
#pragma unroll
        for (int j = 0; j < 8; j++) o[h][j] = fmaf(o[h][j], corr, pw * vv[j]);
        m[h] = mn;
    }
}

template <int HPK>
__global__ __launch_bounds__(256) void attn_decode_fused(qk_attn_fused_args a) {
    const int hd = QWEN_HIP_HEAD_DIM;
    const int kvh = blockIdx.x, split = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, gl = lane & 15;
    const int pos = *a.pos_dev, seq_k = pos + 1;
    const int chunk = qk_attn_chunk(seq_k, a.nsplit);
    const int nsplit = (seq_k + chunk - 1) / chunk;
    if (split >= nsplit) {
        // an idle split marks its partial slot empty (m = -inf weighs 0 in the merge)
        if (threadIdx.x < HPK) a.part_m[(size_t)(kvh * HPK + threadIdx.x) * a.nsplit + split] = -INFINITY;
        return;
    }
    const int s0 = split * chunk, s1 = min(s0 + chunk, seq_k);
    const bool last_split = (s1 == seq_k);
    const int cached_end = last_split ? pos : s1;        // position pos itself comes from LDS
    const int qd = a.heads * hd, kvd = a.kv_heads * hd;

    // prefetch the first batch of cached K/V rows (independent of this step's q)
    const float *kb = a.k_cache + (size_t)kvh * a.cap * hd + gl * 8;
    const float *vb = a.v_cache + (size_t)kvh * a.cap * hd + gl * 8;
    const int p0 = s0 + wave * 4 + g;
    float4 ck[QK_AB][2], cv[QK_AB][2];
#pragma unroll
    for (int j = 0; j < QK_AB; j++) {
        const int p = p0 + 16 * j;
        if (p < cached_end) {
            ck[j][0] = *reinterpret_cast<const float4 *>(kb + (size_t)p * hd);
            ck[j][1] = *reinterpret_cast<const float4 *>(kb + (size_t)p * hd + 4);
            cv[j][0] = *reinterpret_cast<const float4 *>(vb + (size_t)p * hd);
            cv[j][1] = *reinterpret_cast<const float4 *>(vb + (size_t)p * hd + 4);
        }
    }

    __shared__ __attribute__((aligned(16))) float qs[HPK][128];
    __shared__ __attribute__((aligned(16))) float knew[128];
    __shared__ __attribute__((aligned(16))) float vnew[128];
    __shared__ float sm_m[16][HPK], sm_l[16][HPK];
    __shared__ float sm_o[16][HPK][128];

    const float c = a.rope_cos[(size_t)pos * hd + lane], sn = a.rope_sin[(size_t)pos * hd + lane];
    if (wave < HPK) {                       // query heads of this group
        const float *src = a.qkv + (size_t)(kvh * HPK + wave) * hd;
        float x1 = src[lane], x2 = src[lane + 64];
        norm_rope_pair(x1, x2, a.q_norm, a.eps, c, sn, lane);
        qs[wave][lane] = x1;
        qs[wave][lane + 64] = x2;
    }
    if (last_split && wave == (HPK < 4 ? HPK : 0)) {    // this step's key and value
        const float *ks = a.qkv + qd + (size_t)kvh * hd;
        const float *vs = a.qkv + qd + kvd + (size_t)kvh * hd;
        float x1 = ks[lane], x2 = ks[lane + 64];
        norm_rope_pair(x1, x2, a.k_norm, a.eps, c, sn, lane);
        const float v1 = vs[lane], v2 = vs[lane + 64];
        knew[lane] = x1; knew[lane + 64] = x2;
        vnew[lane] = v1; vnew[lane + 64] = v2;
        const size_t off = ((size_t)kvh * a.cap + pos) * hd;
        a.k_cache[off + lane] = x1; a.k_cache[off + lane + 64] = x2;
        a.v_cache[off + lane] = v1; a.v_cache[off + lane + 64] = v2;
    }
    __syncthreads();

    float q[HPK][8];
#pragma unroll
    for (int h = 0; h < HPK; h++)
#pragma unroll
        for (int j = 0; j < 8; j++) q[h][j] = qs[h][gl * 8 + j];
    float m[HPK], l[HPK], o[HPK][8];
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) o[h][j] = 0.0f;
    }
    for (int pb = p0; pb < cached_end; pb += 16 * QK_AB) {
        float4 nk[QK_AB][2], nv[QK_AB][2];
        const int pn = pb + 16 * QK_AB;
#pragma unroll
        for (int j = 0; j < QK_AB; j++) {
            const int p = pn + 16 * j;
            if (p < cached_end) {
                nk[j][0] = *reinterpret_cast<const float4 *>(kb + (size_t)p * hd);
                nk[j][1] = *reinterpret_cast<const float4 *>(kb + (size_t)p * hd + 4);
                nv[j][0] = *reinterpret_cast<const float4 *>(vb + (size_t)p * hd);
                nv[j][1] = *reinterpret_cast<const float4 *>(vb + (size_t)p * hd + 4);
            }
        }
#pragma unroll
        for (int j = 0; j < QK_AB; j++)
            if (pb + 16 * j < cached_end) attn_fold<HPK>(q, ck[j][0], ck[j][1], cv[j][0], cv[j][1], a.scale, m, l, o);
#pragma unroll
        for (int j = 0; j < QK_AB; j++) {
            ck[j][0] = nk[j][0]; ck[j][1] = nk[j][1];
            cv[j][0] = nv[j][0]; cv[j][1] = nv[j][1];
        }
    }
    if (last_split && wave == 0 && g == 0) {
        const float4 *kn = reinterpret_cast<const float4 *>(&knew[gl * 8]);
        const float4 *vn = reinterpret_cast<const float4 *>(&vnew[gl * 8]);
        attn_fold<HPK>(q, kn[0], kn[1], vn[0], vn[1], a.scale, m, l, o);
    }

    const int grp = wave * 4 + g;
#pragma unroll
    for (int h = 0; h < HPK; h++) {
        if (gl == 0) { sm_m[grp][h] = m[h]; sm_l[grp][h] = l[h]; }
#pragma unroll
        for (int j = 0; j < 8; j++) sm_o[grp][h][gl * 8 + j] = o[h][j];
    }
    __syncthreads();
    // merge the 16 groups; thread t -> (head t / 128, dim t % 128)
    for (int t = threadIdx.x; t < HPK * hd; t += 256) {
        const int h = t / hd, d = t % hd;
        float M = -INFINITY;
        for (int i = 0; i < 16; i++) M = fmaxf(M, sm_m[i][h]);
        float L = 0.0f, acc = 0.0f;
        for (int i = 0; i < 16; i++) {
            const float mi = sm_m[i][h];
            const float e = (mi == -INFINITY) ? 0.0f : __expf(mi - M);
            L = fmaf(sm_l[i][h], e, L);
            acc = fmaf(sm_o[i][h][d], e, acc);
        }
        const int hq = kvh * HPK + h;
        if (nsplit == 1 && a.out) {
            a.out[(size_t)hq * hd + d] = acc * (1.0f / L);
        } else {
            a.part_o[((size_t)hq * a.nsplit + split) * hd + d] = acc;
            if (d == 0) {
                a.part_m[(size_t)hq * a.nsplit + split] = M;
                a.part_l[(size_t)hq * a.nsplit + split] = L;
            }
        }
    }
}

extern "C" int qk_attn_fused_launch(const qk_attn_fused_args *a, hipStream_t s) {
    if (!a || a->heads <= 0 || a->kv_heads <= 0 || a->heads % a->kv_heads || a->nsplit <= 0 ||
        a->nsplit > QK_ATTN_MAX_SPLIT || !a->part_o || !a->part_m || !a->part_l || !a->pos_dev)
        return QWEN_HIP_EINVAL;
    dim3 grid(a->kv_heads, a->nsplit);
    switch (a->heads / a->kv_heads) {
    case 1: attn_decode_fused<1><<<grid, 256, 0, s>>>(*a); break;
    case 2: attn_decode_fused<2><<<grid, 256, 0, s>>>(*a); break;
    case 4: attn_decode_fused<4><<<grid, 256, 0, s>>>(*a); break;
    default: return QWEN_HIP_EINVAL;
    }
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// Merge of the split partials into out[head][128] (long contexts).
__global__ __launch_bounds__(128) void attn_merge(const float *part_o, const float *part_m, const float *part_l,
                                                   int nsplit_max, const int *pos_dev, float *out) {
    const int hd = QWEN_HIP_HEAD_DIM, h = blockIdx.x, d = threadIdx.x;
    const int seq_k = *pos_dev + 1;
    const int chunk = qk_attn_chunk(seq_k, nsplit_max);
    const int ns = (seq_k + chunk - 1) / chunk;
    const float *pm = part_m + (size_t)h * nsplit_max, *pl = part_l + (size_t)h * nsplit_max;
    const float *po = part_o + (size_t)h * nsplit_max * hd + d;
    float M = -INFINITY;
    for (int s = 0; s < ns; s++) M = fmaxf(M, pm[s]);
    float L = 0.0f, acc = 0.0f;
    for (int s = 0; s < ns; s++) {
        const float e = (pm[s] == -INFINITY) ? 0.0f : __expf(pm[s] - M);
        L = fmaf(pl[s], e, L);
        acc = fmaf(po[(size_t)s * hd], e, acc);
    }
    out[(size_t)h * hd + d] = acc * (1.0f / L);
}

extern "C" int qk_attn_merge_launch(const qk_attn_fused_args *a, hipStream_t s) {
    if (!a || !a->out || !a->pos_dev) return QWEN_HIP_EINVAL;
    attn_merge<<<a->heads, 128, 0, s>>>(a->part_o, a->part_m, a->part_l, a->nsplit, a->pos_dev, a->out);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}
