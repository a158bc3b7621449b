/*
 * ops.c - op-level ABI: the qwen_asr_kernels.h operators the decoder calls,
 * on device pointers.  Argument order and meaning follow the reference
 * (cited per function in include/qwen_asr_hip.h).
 *
 * Operators that need temporary device memory (the bf16 hi/lo split of a
 * GEMM input, attention split partials, argmax candidates) take it from a
 * per-device workspace owned by this file, grown on demand, and synchronise
 * their stream before returning so the workspace is free again.  Like the
 * reference's op layer (global scratch, qwen_asr_kernels.c:239-262), calls
 * on one device are not meant to run concurrently.
 */
#include "host_internal.h"

#include <pthread.h>
#include <stdlib.h>

#define QK_MAX_DEVICES 64
#define QK_OP_NSPLIT 32

static pthread_mutex_t g_ws_lock = PTHREAD_MUTEX_INITIALIZER;
static void *g_ws[QK_MAX_DEVICES];
static size_t g_ws_cap[QK_MAX_DEVICES];

/* Workspace of at least n bytes on the current device (lock held by caller). */
static int workspace(size_t n, void **out) {
    int dev = 0;
    QK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= QK_MAX_DEVICES) { qk_set_err("device index %d out of range", dev); return QWEN_HIP_EINVAL; }
    if (n > g_ws_cap[dev]) {
        size_t cap = g_ws_cap[dev] ? g_ws_cap[dev] : ((size_t)1 << 20);
        while (cap < n) cap *= 2;
        if (g_ws[dev]) (void)hipFree(g_ws[dev]);
        g_ws[dev] = NULL;
        g_ws_cap[dev] = 0;
        hipError_t e = hipMalloc(&g_ws[dev], cap);
        if (e != hipSuccess) {
            g_ws[dev] = NULL;
            qk_set_err("workspace hipMalloc(%zu): %s", cap, hipGetErrorString(e));
            return QWEN_HIP_ENOMEM;
        }
        g_ws_cap[dev] = cap;
    }
    *out = g_ws[dev];
    return 0;
}

int qwen_hip_add_inplace(float *a, const float *b, int n, hipStream_t s) {
    if (n < 0 || (n > 0 && (!a || !b))) return QWEN_HIP_EINVAL;
    return qk_add_launch(a, b, n, s);
}

int qwen_hip_rms_norm(float *out, const float *x, const float *w, int S, int D, float eps, hipStream_t s) {
    if (!out || !x || !w) return QWEN_HIP_EINVAL;
    return qk_rms_norm_launch(out, x, w, S, D, eps, s);
}

int qwen_hip_rms_norm_per_head(float *x, const float *w, int S, int nh, int hd, float eps, hipStream_t s) {
    if (!x || !w) return QWEN_HIP_EINVAL;
    return qk_rms_norm_per_head_launch(x, w, S, nh, hd, eps, s);
}

int qwen_hip_apply_rope_neox(float *x, const float *c, const float *sn, int S, int nh, int hd, hipStream_t s) {
    if (!x || !c || !sn) return QWEN_HIP_EINVAL;
    return qk_rope_launch(x, c, sn, S, nh, hd, s);
}

int qwen_hip_swiglu_multiply(float *out, const float *gu, int S, int inter, hipStream_t s) {
    if (!out || !gu) return QWEN_HIP_EINVAL;
    return qk_swiglu_launch(out, gu, S, inter, s);
}

/* Plan of the seq > 1 product: tiling as qk_gemm_plan_for, except that one
 * split is kept where the output tiles alone number QK_GEMM_TARGET or more
 * (they fill the chip, and the partials of a split plan would be at least
 * 2 x seq x out floats) and where the output width is odd (the split-K reduce
 * works on column pairs).  So the op splits K only for small tile grids. */
static void linear_plan(int S, int in_dim, int out_dim, qk_gemm_plan *p) {
    qk_gemm_plan_for(S, out_dim, in_dim, p);
    const long tiles = (long)((S + p->bm - 1) / p->bm) * ((out_dim + p->bn - 1) / p->bn);
    if (p->nsplit > 1 && ((out_dim & 1) || tiles >= QK_GEMM_TARGET)) {
        p->kc = ((in_dim + 63) / 64) * 64;
        p->nsplit = 1;
    }
}

size_t qk_linear_ws_bytes(int S, int in_dim, int out_dim) {
    qk_gemm_plan p;
    linear_plan(S, in_dim, out_dim, &p);
    const size_t n = (size_t)S * in_dim;
    const size_t part = p.nsplit > 1 ? (size_t)p.nsplit * S * out_dim : 0;
    return ((2 * n * sizeof(uint16_t) + 255) & ~(size_t)255) + part * sizeof(float);
}

int qk_linear_gemm(float *y, const float *x, const uint16_t *W, int S, int in_dim, int out_dim, void *ws,
                   hipStream_t s) {
    qk_gemm_plan p;
    linear_plan(S, in_dim, out_dim, &p);
    const size_t n = (size_t)S * in_dim;
    const size_t abytes = (2 * n * sizeof(uint16_t) + 255) & ~(size_t)255;
    uint16_t *ah = (uint16_t *)ws, *al = ah + n;
    float *pp = (float *)((char *)ws + abytes);
    int rc = qk_split_bf16_launch(x, (long)n, ah, al, s);
    if (!rc && p.nsplit > 1) {
        rc = qk_gemm_launch(ah, al, W, S, out_dim, in_dim, &p, QK_GEMM_STORE, pp, NULL, NULL, s);
        if (!rc) rc = qk_gemm_reduce_launch(pp, p.nsplit, S, out_dim, QK_GEMM_STORE, y, NULL, NULL, s);
    } else if (!rc) {
        rc = qk_gemm_launch(ah, al, W, S, out_dim, in_dim, &p, QK_GEMM_STORE, y, NULL, NULL, s);
    }
    return rc;
}

int qwen_hip_linear_nobias_bf16(float *y, const float *x, const uint16_t *W, int S, int in_dim, int out_dim,
                                hipStream_t s) {
    if (!y || !x || !W || S <= 0 || in_dim <= 0 || out_dim <= 0) return QWEN_HIP_EINVAL;
    if (S == 1) {
        qk_gemv_args g = {.W = W, .rows = out_dim, .K = in_dim, .x = x, .y = y, .epi = QK_EPI_STORE};
        return qk_gemv_launch(&g, s);
    }
    pthread_mutex_lock(&g_ws_lock);
    void *ws = NULL;
    int rc = workspace(qk_linear_ws_bytes(S, in_dim, out_dim), &ws);
    if (!rc) rc = qk_linear_gemm(y, x, W, S, in_dim, out_dim, ws, s);
    if (!rc && hipStreamSynchronize(s) != hipSuccess) rc = QWEN_HIP_EDEVICE;
    pthread_mutex_unlock(&g_ws_lock);
    return rc;
}

int qwen_hip_linear_nobias_bf16_qkv(float *q, float *k, float *v, const float *x, const uint16_t *Wq,
                                    const uint16_t *Wk, const uint16_t *Wv, int in_dim, int q_dim, int kv_dim,
                                    hipStream_t s) {
    int rc = qwen_hip_linear_nobias_bf16(q, x, Wq, 1, in_dim, q_dim, s);
    if (!rc) rc = qwen_hip_linear_nobias_bf16(k, x, Wk, 1, in_dim, kv_dim, s);
    if (!rc) rc = qwen_hip_linear_nobias_bf16(v, x, Wv, 1, in_dim, kv_dim, s);
    return rc;
}

int qwen_hip_causal_attention(float *out, const float *Q, const float *K, const float *V, int seq_q, int seq_k,
                              int n_heads, int n_kv_heads, int head_dim, float scale, int q_offset,
                              hipStream_t s) {
    if (!out || !Q || !K || !V || seq_q <= 0 || seq_k <= 0 || head_dim != QWEN_HIP_HEAD_DIM || q_offset < 0)
        return QWEN_HIP_EINVAL;
    qk_attn_args a = {.q = Q, .k = K, .v = V, .pos_stride = (long)n_kv_heads * head_dim, .head_stride = head_dim,
                      .seq_k = seq_k, .seq_q = seq_q, .q_offset = q_offset, .heads = n_heads,
                      .kv_heads = n_kv_heads, .scale = scale, .out = out};
    if (seq_q > 1) {
        const size_t pf = qk_attn_prefill_plan(seq_q, seq_k, q_offset, n_heads, n_kv_heads, &a.chunk, &a.nsplit);
        if (pf == 0) return qk_attn_prefill_launch(&a, s);
        pthread_mutex_lock(&g_ws_lock);
        void *ws = NULL;
        int rc = workspace(pf * sizeof(float), &ws);
        if (!rc) {
            a.part = (float *)ws;
            rc = qk_attn_prefill_launch(&a, s);
        }
        if (!rc && hipStreamSynchronize(s) != hipSuccess) rc = QWEN_HIP_EDEVICE;
        pthread_mutex_unlock(&g_ws_lock);
        return rc;
    }
    /* one query row: keys j <= q_offset, capped at seq_k (qwen_asr_kernels.c:1065-1067) */
    a.seq_k = q_offset + 1 < seq_k ? q_offset + 1 : seq_k;
    a.nsplit = QK_OP_NSPLIT;
    pthread_mutex_lock(&g_ws_lock);
    void *ws = NULL;
    int rc = workspace((size_t)n_heads * QK_OP_NSPLIT * (head_dim + 2) * sizeof(float), &ws);
    if (!rc) {
        a.part = (float *)ws;
        rc = qk_attn_decode_launch(&a, s);
    }
    if (!rc && hipStreamSynchronize(s) != hipSuccess) rc = QWEN_HIP_EDEVICE;
    pthread_mutex_unlock(&g_ws_lock);
    return rc;
}

int qwen_hip_argmax_matvec_bf16(const float *x, const uint16_t *W, int in_dim, int out_dim, hipStream_t s) {
    if (!x || !W || in_dim <= 0 || out_dim <= 0) return QWEN_HIP_EINVAL;
    const int nb = qk_gemv_blocks(out_dim, in_dim, QK_EPI_ARGMAX);
    pthread_mutex_lock(&g_ws_lock);
    void *ws = NULL;
    int rc = workspace((size_t)nb * 8 + 256, &ws);
    int result = -1;
    if (!rc) {
        float *cv = (float *)ws;
        int *ci = (int *)(cv + nb);
        int *tok = ci + nb;
        qk_gemv_args g = {.W = W, .rows = out_dim, .K = in_dim, .x = x, .cand_val = cv, .cand_idx = ci,
                          .epi = QK_EPI_ARGMAX};
        rc = qk_gemv_launch(&g, s);
        if (!rc) rc = qk_argmax_finish_launch(cv, ci, nb, tok, NULL, NULL, NULL, NULL, s);
        if (!rc && hipMemcpyAsync(&result, tok, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess)
            rc = QWEN_HIP_EDEVICE;
        if (!rc && hipStreamSynchronize(s) != hipSuccess) rc = QWEN_HIP_EDEVICE;
    }
    pthread_mutex_unlock(&g_ws_lock);
    return rc ? rc : result;
}
