/*
 * qwen_oracle.c - TEST INFRASTRUCTURE: a CPU restatement of the reference's
 * decoder token loop, used only as the checker by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg.  The product
 * path never links or calls this file.
 *
 * It restates, in plain C (fp32 activations, bf16 weights widened exactly by
 * a 16-bit shift, fp32 accumulation), the arithmetic of:
 *   qwen_asr_decoder.c:262-359 (prefill), :388-476 (forward), :122-170 (KV),
 *   :207-256 (RoPE tables); qwen_asr_kernels.c:159-161 (add), :750-809
 *   (rms_norm), :811-873 (per-head norm), :946-959 (swiglu), :1050-1097
 *   (causal attention, online softmax), :1182-1247 (NeoX RoPE), :518-543
 *   (argmax); qwen_asr_kernels_avx.c:25-97 (4-row bf16 matvec lane pattern),
 *   :357-400 (fp32 dot).
 * Dot products keep the reference's AVX-512 lane structure (32 lanes for the
 * bf16 matvec, 64 for the fp32 dot) so results land within a few ulp of the
 * reference build; each row is summed serially, so results do not depend on
 * the OpenMP thread count.
 *
 * How it is pinned (tests/test_oracle.py): against the compiled reference in
 * oracle/_ref (op by op and full trajectories), against fp64 brute force and
 * closed forms (RMSNorm, RoPE norm preservation and identity at position 0,
 * SwiGLU, softmax attention, single-key attention returning V, GQA head map),
 * and against the committed golden fixtures.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf16f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* Sum of 16 lanes in the order _mm512_reduce_add_ps folds them: halves of
 * 8, then 4, then 2, then the last pair. */
static inline float fold16(const float *a) {
    float t[8], u[4];
    for (int j = 0; j < 8; j++) t[j] = a[j] + a[j + 8];
    for (int j = 0; j < 4; j++) u[j] = t[j] + t[j + 4];
    float v0 = u[0] + u[2], v1 = u[1] + u[3];
    return v0 + v1;
}

/* One row of the bf16 matvec: qwen_asr_kernels_avx.c:42-95 (row 0 of the
 * 4-row block: two 16-lane accumulators over 32-wide steps, a 16-wide tail,
 * reduce, then a scalar tail). */
float orc_dot_bf16(const uint16_t *w, const float *x, int n) {
    float a[32];
    for (int j = 0; j < 32; j++) a[j] = 0.0f;
    int k = 0;
    for (; k + 32 <= n; k += 32)
        for (int j = 0; j < 32; j++) a[j] = fmaf(bf16f(w[k + j]), x[k + j], a[j]);
    for (; k + 16 <= n; k += 16)
        for (int j = 0; j < 16; j++) a[j] = fmaf(bf16f(w[k + j]), x[k + j], a[j]);
    float s16[16];
    for (int j = 0; j < 16; j++) s16[j] = a[j] + a[j + 16];
    float s = fold16(s16);
    for (; k < n; k++) s += bf16f(w[k]) * x[k];
    return s;
}

/* fp32 dot of the attention path: qwen_asr_kernels_avx.c:357-376 (four
 * 16-lane accumulators over 64-wide steps). */
static float orc_dot_f32(const float *a, const float *b, int n) {
    float acc[64];
    for (int j = 0; j < 64; j++) acc[j] = 0.0f;
    int i = 0;
    for (; i + 64 <= n; i += 64)
        for (int j = 0; j < 64; j++) acc[j] = fmaf(a[i + j], b[i + j], acc[j]);
    float s16[16];
    for (int j = 0; j < 16; j++)
        s16[j] = (acc[j] + acc[j + 16]) + (acc[j + 32] + acc[j + 48]);
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; j++) s16[j] = fmaf(a[i + j], b[i + j], s16[j]);
    float s = fold16(s16);
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

/* qwen_linear_nobias_bf16 / bf16 matvec, rows split over threads
 * (qwen_asr_kernels.c:351-373, :462-472).  y[s][o] = W[o] . x[s].  Each
 * (s, o) is one orc_dot_bf16 whatever the tiling, so the result does not
 * depend on it; input rows are taken 16 at a time so a weight row is read
 * once per 16 rows (the oracle's long prefills). */
#define ORC_ROW_TILE 16
void orc_linear_bf16(float *y, const float *x, const uint16_t *W,
                     int seq, int in_dim, int out_dim) {
    const long tiles = (seq + ORC_ROW_TILE - 1) / ORC_ROW_TILE;
    const long total = tiles * out_dim;
#pragma omp parallel for schedule(static)
    for (long t = 0; t < total; t++) {
        const int o = (int)(t % out_dim), s0 = (int)(t / out_dim) * ORC_ROW_TILE;
        const int s1 = s0 + ORC_ROW_TILE < seq ? s0 + ORC_ROW_TILE : seq;
        for (int s = s0; s < s1; s++)
            y[(size_t)s * out_dim + o] = orc_dot_bf16(W + (size_t)o * in_dim, x + (size_t)s * in_dim, in_dim);
    }
}

/* qwen_argmax_matvec_bf16 (qwen_asr_kernels.c:518-543 with the range kernel
 * qwen_asr_kernels_avx.c:157-249): strict '>' scanning upward, so ties keep
 * the lowest index; chunk winners combined in order with strict '>'. */
int orc_argmax_matvec_bf16(const float *x, const uint16_t *W, int in_dim, int out_dim,
                           float *best_val_out) {
    int nchunk = 64;
    int best_idx[64];
    float best_val[64];
    int chunk = (out_dim + nchunk - 1) / nchunk;
#pragma omp parallel for schedule(static)
    for (int c = 0; c < nchunk; c++) {
        int b = c * chunk, e = b + chunk;
        if (e > out_dim) e = out_dim;
        float bv = -1e30f;
        int bi = b < out_dim ? b : 0;
        for (int o = b; o < e; o++) {
            float v = orc_dot_bf16(W + (size_t)o * in_dim, x, in_dim);
            if (v > bv) { bv = v; bi = o; }
        }
        best_idx[c] = bi;
        best_val[c] = bv;
    }
    int best = best_idx[0];
    float bv = best_val[0];
    for (int c = 1; c < nchunk; c++)
        if (best_val[c] > bv) { bv = best_val[c]; best = best_idx[c]; }
    if (best_val_out) *best_val_out = bv;
    return best;
}

/* qwen_rms_norm (qwen_asr_kernels.c:750-809): 16-lane FMA sum of squares,
 * rinv = 1/sqrtf(ss/n + eps), out = (x*w)*rinv.  out may alias x. */
void orc_rms_norm(float *out, const float *x, const float *w, int seq, int hidden, float eps) {
    for (int s = 0; s < seq; s++) {
        const float *xr = x + (size_t)s * hidden;
        float *orow = out + (size_t)s * hidden;
        float acc[16] = {0};
        int i = 0;
        for (; i + 16 <= hidden; i += 16)
            for (int j = 0; j < 16; j++) acc[j] = fmaf(xr[i + j], xr[i + j], acc[j]);
        float ss = fold16(acc);
        for (; i < hidden; i++) ss += xr[i] * xr[i];
        float rinv = 1.0f / sqrtf(ss / (float)hidden + eps);
        for (int j = 0; j < hidden; j++) orow[j] = (xr[j] * w[j]) * rinv;
    }
}

/* qwen_rms_norm_per_head (qwen_asr_kernels.c:811-873): in place per head. */
void orc_rms_norm_per_head(float *x, const float *w, int seq, int n_heads, int head_dim, float eps) {
    for (int s = 0; s < seq; s++)
        for (int h = 0; h < n_heads; h++) {
            float *v = x + ((size_t)s * n_heads + h) * head_dim;
            orc_rms_norm(v, v, w, 1, head_dim, eps);
        }
}

/* RoPE tables (qwen_asr_decoder.c:207-256): inv[d] = 1/powf(theta, 2d/hd),
 * angle = (float)pos * inv[d], cos/sin duplicated across both halves. */
void orc_rope_table(float *cos_out, float *sin_out, int n_pos, int head_dim, float theta) {
    int half = head_dim / 2;
    float inv[512];
    for (int d = 0; d < half; d++)
        inv[d] = 1.0f / powf(theta, (float)(2 * d) / (float)head_dim);
    for (int p = 0; p < n_pos; p++) {
        float *c = cos_out + (size_t)p * head_dim, *sn = sin_out + (size_t)p * head_dim;
        for (int d = 0; d < half; d++) {
            float a = (float)p * inv[d];
            float cv = cosf(a), sv = sinf(a);
            c[d] = cv; c[half + d] = cv;
            sn[d] = sv; sn[half + d] = sv;
        }
    }
}

/* qwen_apply_rope_neox (qwen_asr_kernels.c:1182-1247), AVX-512 form
 * (:1208-1209): x1' = fma(x1, c, -(x2*s)), x2' = fma(x2, c, x1*s). */
void orc_apply_rope(float *x, const float *cos_v, const float *sin_v,
                    int seq, int n_heads, int head_dim) {
    int half = head_dim / 2;
    for (int s = 0; s < seq; s++) {
        const float *c = cos_v + (size_t)s * head_dim, *sn = sin_v + (size_t)s * head_dim;
        for (int h = 0; h < n_heads; h++) {
            float *v = x + ((size_t)s * n_heads + h) * head_dim;
            for (int d = 0; d < half; d++) {
                float x1 = v[d], x2 = v[half + d];
                v[d] = fmaf(x1, c[d], -(x2 * sn[d]));
                v[half + d] = fmaf(x2, c[d], x1 * sn[d]);
            }
        }
    }
}

/* qwen_causal_attention (qwen_asr_kernels.c:1050-1097): per query head h,
 * kv head h / (n_heads/n_kv_heads); keys j <= q_offset + i; single-pass
 * online softmax with max initialised to -1e30 and the reference's branch:
 * a new max rescales (o = o*corr + v, sum = sum*corr + 1), otherwise
 * o += exp(s - max) * v. */
void orc_causal_attention(float *out, const float *Q, const float *K, const float *V,
                          int seq_q, int seq_k, int n_heads, int n_kv_heads,
                          int head_dim, float scale, int q_offset) {
    int hpk = n_heads / n_kv_heads;
    int qh = n_heads * head_dim, kh = n_kv_heads * head_dim;
#pragma omp parallel for schedule(dynamic) collapse(2)
    for (int h = 0; h < n_heads; h++)
        for (int i = 0; i < seq_q; i++) {
            int kvh = h / hpk;
            const float *q = Q + (size_t)i * qh + (size_t)h * head_dim;
            float *o = out + (size_t)i * qh + (size_t)h * head_dim;
            int k_end = q_offset + i + 1;
            if (k_end > seq_k) k_end = seq_k;
            float m = -1e30f, sum = 0.0f;
            for (int d = 0; d < head_dim; d++) o[d] = 0.0f;
            for (int j = 0; j < k_end; j++) {
                const float *k = K + (size_t)j * kh + (size_t)kvh * head_dim;
                const float *v = V + (size_t)j * kh + (size_t)kvh * head_dim;
                float sc = orc_dot_f32(q, k, head_dim) * scale;
                if (sc > m) {
                    float corr = expf(m - sc);
                    sum = sum * corr + 1.0f;
                    for (int d = 0; d < head_dim; d++) o[d] = fmaf(o[d], corr, v[d]);
                    m = sc;
                } else {
                    float wt = expf(sc - m);
                    sum += wt;
                    for (int d = 0; d < head_dim; d++) o[d] = fmaf(v[d], wt, o[d]);
                }
            }
            if (sum > 0.0f) {
                float inv = 1.0f / sum;
                for (int d = 0; d < head_dim; d++) o[d] *= inv;
            }
        }
}

/* qwen_swiglu_multiply (qwen_asr_kernels.c:902-959): interleaved gate/up,
 * out[j] = (g / (1 + expf(-g))) * u.  out may alias gate_up. */
void orc_swiglu(float *out, const float *gate_up, int seq, int inter) {
    for (int s = 0; s < seq; s++) {
        const float *gu = gate_up + (size_t)s * 2 * inter;
        float *o = out + (size_t)s * inter;
        for (int j = 0; j < inter; j++) {
            float g = gu[2 * j], u = gu[2 * j + 1];
            g = g / (1.0f + expf(-g));
            o[j] = g * u;
        }
    }
}

void orc_add_inplace(float *a, const float *b, long n) {
    for (long i = 0; i < n; i++) a[i] += b[i];
}

/* ------------------------------------------------------------------------
 * Decoder (qwen_asr_decoder.c).  KV layout [layer][cap][kv_dim] fp32 as
 * kv_cache_init (:122-131); growth by doubling as kv_cache_grow (:133-160).
 * ------------------------------------------------------------------------ */
typedef struct {
    int hidden, layers, heads, kv_heads, head_dim, inter, vocab;
    float eps, theta;
    const uint16_t *wq[64], *wk[64], *wv[64], *wo[64], *gate[64], *up[64], *down[64];
    const float *qn[64], *kn[64], *inn[64], *postn[64];
    uint16_t *gate_up[64];
    const uint16_t *emb;
    const float *fnorm;
    float *kc, *vc;
    int kv_len, kv_cap;
    float *rcos, *rsin;
    int rope_cap;
    float *hidden_state;      /* final-normed hidden of the last forward */
} orc_model_t;

void *orc_create(int hidden, int layers, int heads, int kv_heads, int head_dim,
                 int inter, int vocab, float eps, float theta) {
    if (layers > 64) return NULL;
    orc_model_t *m = (orc_model_t *)calloc(1, sizeof(orc_model_t));
    m->hidden = hidden; m->layers = layers; m->heads = heads; m->kv_heads = kv_heads;
    m->head_dim = head_dim; m->inter = inter; m->vocab = vocab; m->eps = eps; m->theta = theta;
    m->hidden_state = (float *)calloc((size_t)hidden, sizeof(float));
    return m;
}

int orc_set_layer(void *mp, int l, const uint16_t *wq, const uint16_t *wk, const uint16_t *wv,
                  const uint16_t *wo, const uint16_t *gate, const uint16_t *up,
                  const uint16_t *down, const float *qn, const float *kn,
                  const float *inn, const float *postn) {
    orc_model_t *m = (orc_model_t *)mp;
    if (l < 0 || l >= m->layers) return -1;
    m->wq[l] = wq; m->wk[l] = wk; m->wv[l] = wv; m->wo[l] = wo;
    m->gate[l] = gate; m->up[l] = up; m->down[l] = down;
    m->qn[l] = qn; m->kn[l] = kn; m->inn[l] = inn; m->postn[l] = postn;
    /* interleave gate/up rows as qwen_asr_decoder.c:95-107 */
    size_t hid = (size_t)m->hidden, I = (size_t)m->inter;
    free(m->gate_up[l]);
    m->gate_up[l] = (uint16_t *)malloc(2 * I * hid * sizeof(uint16_t));
    for (size_t r = 0; r < I; r++) {
        memcpy(m->gate_up[l] + 2 * r * hid, gate + r * hid, hid * 2);
        memcpy(m->gate_up[l] + (2 * r + 1) * hid, up + r * hid, hid * 2);
    }
    return 0;
}

void orc_set_embeddings(void *mp, const uint16_t *emb, const float *fnorm) {
    orc_model_t *m = (orc_model_t *)mp;
    m->emb = emb;
    m->fnorm = fnorm;
}

static int orc_kv_reserve(orc_model_t *m, int need) {
    if (need <= m->kv_cap) return 0;
    int kvd = m->kv_heads * m->head_dim;
    int cap = m->kv_cap > 0 ? m->kv_cap : need + 1024;
    while (cap < need) cap *= 2;
    float *nk = (float *)calloc((size_t)m->layers * cap * kvd, sizeof(float));
    float *nv = (float *)calloc((size_t)m->layers * cap * kvd, sizeof(float));
    if (!nk || !nv) { free(nk); free(nv); return -1; }
    for (int l = 0; l < m->layers && m->kc; l++) {
        memcpy(nk + (size_t)l * cap * kvd, m->kc + (size_t)l * m->kv_cap * kvd, (size_t)m->kv_len * kvd * 4);
        memcpy(nv + (size_t)l * cap * kvd, m->vc + (size_t)l * m->kv_cap * kvd, (size_t)m->kv_len * kvd * 4);
    }
    free(m->kc); free(m->vc);
    m->kc = nk; m->vc = nv; m->kv_cap = cap;
    return 0;
}

static int orc_rope_reserve(orc_model_t *m, int need) {
    if (need <= m->rope_cap) return 0;
    int cap = m->rope_cap > 0 ? m->rope_cap : 1024;
    while (cap < need) cap *= 2;
    free(m->rcos); free(m->rsin);
    m->rcos = (float *)malloc((size_t)cap * m->head_dim * 4);
    m->rsin = (float *)malloc((size_t)cap * m->head_dim * 4);
    if (!m->rcos || !m->rsin) return -1;
    orc_rope_table(m->rcos, m->rsin, cap, m->head_dim, m->theta);
    m->rope_cap = cap;
    return 0;
}

/* The layer stack shared by prefill (:304-356) and forward (:428-469). */
static void orc_layers(orc_model_t *m, float *x, int S, int start) {
    int D = m->hidden, H = m->heads, KVH = m->kv_heads, hd = m->head_dim, I = m->inter;
    int qd = H * hd, kvd = KVH * hd;
    float scale = 1.0f / sqrtf((float)hd);
    float *xn = (float *)malloc((size_t)S * D * 4);
    float *q = (float *)malloc((size_t)S * qd * 4);
    float *k = (float *)malloc((size_t)S * kvd * 4);
    float *v = (float *)malloc((size_t)S * kvd * 4);
    float *att = (float *)malloc((size_t)S * qd * 4);
    float *proj = (float *)malloc((size_t)S * D * 4);
    float *gu = (float *)malloc((size_t)S * 2 * I * 4);
    float *g = (float *)malloc((size_t)S * I * 4);
    const float *rc = m->rcos + (size_t)start * hd, *rs = m->rsin + (size_t)start * hd;
    for (int l = 0; l < m->layers; l++) {
        orc_rms_norm(xn, x, m->inn[l], S, D, m->eps);
        orc_linear_bf16(q, xn, m->wq[l], S, D, qd);
        orc_linear_bf16(k, xn, m->wk[l], S, D, kvd);
        orc_linear_bf16(v, xn, m->wv[l], S, D, kvd);
        orc_rms_norm_per_head(q, m->qn[l], S, H, hd, m->eps);
        orc_rms_norm_per_head(k, m->kn[l], S, KVH, hd, m->eps);
        orc_apply_rope(q, rc, rs, S, H, hd);
        orc_apply_rope(k, rc, rs, S, KVH, hd);
        float *kl = m->kc + (size_t)l * m->kv_cap * kvd, *vl = m->vc + (size_t)l * m->kv_cap * kvd;
        memcpy(kl + (size_t)start * kvd, k, (size_t)S * kvd * 4);
        memcpy(vl + (size_t)start * kvd, v, (size_t)S * kvd * 4);
        orc_causal_attention(att, q, kl, vl, S, start + S, H, KVH, hd, scale, start);
        orc_linear_bf16(proj, att, m->wo[l], S, qd, D);
        orc_add_inplace(x, proj, (long)S * D);
        orc_rms_norm(xn, x, m->postn[l], S, D, m->eps);
        orc_linear_bf16(gu, xn, m->gate_up[l], S, D, 2 * I);
        orc_swiglu(g, gu, S, I);
        orc_linear_bf16(proj, g, m->down[l], S, I, D);
        orc_add_inplace(x, proj, (long)S * D);
    }
    free(xn); free(q); free(k); free(v); free(att); free(proj); free(gu); free(g);
}

/* qwen_decoder_prefill (qwen_asr_decoder.c:262-359). */
int orc_prefill(void *mp, const float *rows, int S) {
    orc_model_t *m = (orc_model_t *)mp;
    if (S <= 0) return 0;
    if (orc_kv_reserve(m, m->kv_len + S) || orc_rope_reserve(m, m->kv_len + S)) return -1;
    float *x = (float *)malloc((size_t)S * m->hidden * 4);
    memcpy(x, rows, (size_t)S * m->hidden * 4);
    orc_layers(m, x, S, m->kv_len);
    m->kv_len += S;
    free(x);
    return 0;
}

/* qwen_decoder_forward (qwen_asr_decoder.c:388-476).  hidden_out/logits_out
 * optional; returns the greedy token. */
int orc_forward(void *mp, const float *row, float *hidden_out, float *logits_out) {
    orc_model_t *m = (orc_model_t *)mp;
    if (orc_kv_reserve(m, m->kv_len + 1) || orc_rope_reserve(m, m->kv_len + 1)) return 151645;
    float *x = m->hidden_state;
    memcpy(x, row, (size_t)m->hidden * 4);
    orc_layers(m, x, 1, m->kv_len);
    m->kv_len += 1;
    orc_rms_norm(x, x, m->fnorm, 1, m->hidden, m->eps);
    if (hidden_out) memcpy(hidden_out, x, (size_t)m->hidden * 4);
    if (logits_out) orc_linear_bf16(logits_out, x, m->emb, 1, m->hidden, m->vocab);
    return orc_argmax_matvec_bf16(x, m->emb, m->hidden, m->vocab, NULL);
}

/* tok_embed_bf16_to_f32 (qwen_asr.c:353-360). */
void orc_embed_token(void *mp, int token, float *out) {
    orc_model_t *m = (orc_model_t *)mp;
    const uint16_t *src = m->emb + (size_t)token * m->hidden;
    for (int i = 0; i < m->hidden; i++) out[i] = bf16f(src[i]);
}

int orc_kv_len(void *mp) { return ((orc_model_t *)mp)->kv_len; }

int orc_set_kv_len(void *mp, int n) {
    orc_model_t *m = (orc_model_t *)mp;
    if (n < 0 || n > m->kv_len) return -1;
    m->kv_len = n;
    return 0;
}

void orc_destroy(void *mp) {
    orc_model_t *m = (orc_model_t *)mp;
    if (!m) return;
    for (int l = 0; l < 64; l++) free(m->gate_up[l]);
    free(m->kc); free(m->vc); free(m->rcos); free(m->rsin); free(m->hidden_state);
    free(m);
}

/* Host memory bandwidth for the CPU baseline's roofline (bench.py): a
 * STREAM-style triad a[i] = b[i] + s*c[i] over three n-float arrays on the
 * OpenMP threads in use, best of `reps` passes; returns GB/s counting 3 x 4
 * bytes per element (two reads, one write). Not part of the decoder checks. */
double orc_stream_triad(long n, int reps) {
    float *a = (float *)malloc((size_t)n * 4), *b = (float *)malloc((size_t)n * 4), *c = (float *)malloc((size_t)n * 4);
    if (!a || !b || !c) { free(a); free(b); free(c); return 0.0; }
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; i++) { a[i] = 0.0f; b[i] = 1.0f; c[i] = 2.0f; }
    double best = 0.0;
    for (int r = 0; r < reps; r++) {
#ifdef _OPENMP
        double t0 = omp_get_wtime();
#endif
#pragma omp parallel for schedule(static)
        for (long i = 0; i < n; i++) a[i] = b[i] + 3.0f * c[i];
#ifdef _OPENMP
        double dt = omp_get_wtime() - t0;
        double gbs = 12.0 * (double)n / dt / 1e9;
        if (gbs > best) best = gbs;
#endif
    }
    volatile float sink = a[n / 2];
    (void)sink;
    free(a); free(b); free(c);
    return best;
}
