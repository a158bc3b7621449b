/*
 * encoder.c - host side of the audio encoder on one MI355X (reference
 * qwen_encoder_load / qwen_encoder_forward, qwen_asr_encoder.c:67-372).
 *
 * Every chunk of chunk_size mel frames is its own 128 x w image for the
 * Conv2D stem; all chunks run as one batch (the image index is part of the
 * GEMM's column index), the mel zero-padded to whole chunks.  A partial last
 * chunk keeps the reference's geometry because each stem GEMM writes zeros
 * into the columns past that chunk's valid width, which is exactly the zero
 * padding the next convolution of the reference reads.  Tokens: the stem's
 * output columns of every chunk, chunk by chunk (w3 per full chunk).
 *
 * Weights live in HBM as fp32 (the reference widens bf16 at load time,
 * load_bf16_as_f32); Q|K|V of a layer are stacked [3d][d] so one GEMM and one
 * bias pass produce all three.  Attention windows are window_token_size =
 * tokens_per_chunk * (n_window_infer / chunk_size) tokens of the whole
 * sequence (:300-308).
 */
#include "host_internal.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ENC_CH 480            /* QWEN_CONV_HIDDEN, qwen_asr.h:39 */
#define ENC_MEL 128
#define ENC_K1 16             /* conv1 patch 1*3*3 padded to a multiple of 16 */
#define ENC_K2 (ENC_CH * 9)   /* 4320 */

/* A weight matrix on the device: a bf16 copy when every value is a bf16 value
 * (checkpoint weights are), used by the bf16 matrix-core GEMM; otherwise the
 * fp32 values, used by the fp32 one. */
typedef struct {
    float *f32;
    uint16_t *b16;
} enc_mat;

typedef struct {
    enc_mat wqkv, wo, fc1w, fc2w;
    float *bqkv, *bo, *ln1w, *ln1b, *fc1b, *fc2b, *ln2w, *ln2b;
    int loaded;
} enc_layer;

struct qwen_hip_encoder {
    qwen_hip_enc_config cfg;
    int device;
    hipStream_t stream;
    float *c1w, *c1b, *c2b, *c3b, *lnpw, *lnpb, *p1b, *p2b, *pe;
    enc_mat c2w, c3w, cow, p1w, p2w;
    int stem_loaded;
    enc_layer L[QWEN_HIP_ENC_MAX_LAYERS];
    /* activations, sized for cap_chunks chunks */
    int cap_chunks;
    float *mel, *cols, *c1, *c2, *c3, *rows, *x, *xn, *qkv, *att, *mid, *out;
    float *gws;   /* split-K partials of the GEMMs (QK_ENC_GEMM_WS_ELEMS floats) */
};

static int dmalloc(void **p, size_t n) {
    *p = NULL;
    if (hipMalloc(p, n ? n : 4) != hipSuccess) { *p = NULL; qk_set_err("hipMalloc(%zu) failed", n); return QWEN_HIP_ENOMEM; }
    return 0;
}

static void dfree(void **p) {
    if (*p) (void)hipFree(*p);
    *p = NULL;
}

void qwen_hip_enc_config_preset(qwen_hip_enc_config *c, int model_b) {
    if (!c) return;
    memset(c, 0, sizeof(*c));
    if (model_b) {          /* 1.7B, qwen_asr.c:149-161 */
        c->d_model = 1024; c->layers = 24; c->heads = 16; c->head_dim = 64; c->ffn_dim = 4096; c->output_dim = 2048;
    } else {                /* 0.6B, :163-176 */
        c->d_model = 896; c->layers = 18; c->heads = 14; c->head_dim = 64; c->ffn_dim = 3584; c->output_dim = 1024;
    }
    c->chunk_size = 100;    /* enc_n_window * 2, :182-184 */
    c->n_window_infer = 800;
}

static int conv_out(int w) { return (w + 2 - 3) / 2 + 1; }

int qwen_hip_encoder_tokens(const qwen_hip_enc_config *c, int mel_frames) {
    if (!c || c->chunk_size <= 0 || mel_frames <= 0) return QWEN_HIP_EINVAL;
    const int n_chunks = (mel_frames + c->chunk_size - 1) / c->chunk_size;
    const int last = mel_frames - (n_chunks - 1) * c->chunk_size;
    return (n_chunks - 1) * conv_out(conv_out(conv_out(c->chunk_size))) + conv_out(conv_out(conv_out(last)));
}

static int check_cfg(const qwen_hip_enc_config *c) {
    return c && c->d_model > 0 && c->d_model % 64 == 0 && c->layers > 0 && c->layers <= QWEN_HIP_ENC_MAX_LAYERS &&
           c->heads > 0 && c->head_dim == 64 && c->heads * c->head_dim == c->d_model && c->ffn_dim > 0 &&
           c->ffn_dim % 4 == 0 && c->output_dim > 0 && c->chunk_size >= 8 && c->n_window_infer >= c->chunk_size &&
           c->n_window_infer % c->chunk_size == 0;
}

static void act_free(qwen_hip_encoder *e) {
    void **b[] = {(void **)&e->mel, (void **)&e->cols, (void **)&e->c1, (void **)&e->c2, (void **)&e->c3,
                  (void **)&e->rows, (void **)&e->x, (void **)&e->xn, (void **)&e->qkv, (void **)&e->att,
                  (void **)&e->mid, (void **)&e->out, (void **)&e->gws};
    for (size_t i = 0; i < sizeof(b) / sizeof(b[0]); i++) dfree(b[i]);
    e->cap_chunks = 0;
}

void qwen_hip_encoder_destroy(qwen_hip_encoder *e) {
    if (!e) return;
    (void)hipSetDevice(e->device);
    (void)hipStreamSynchronize(e->stream);
    act_free(e);
    void **w[] = {(void **)&e->c1w,     (void **)&e->c1b,     (void **)&e->c2w.f32, (void **)&e->c2w.b16,
                  (void **)&e->c2b,     (void **)&e->c3w.f32, (void **)&e->c3w.b16, (void **)&e->c3b,
                  (void **)&e->cow.f32, (void **)&e->cow.b16, (void **)&e->lnpw,    (void **)&e->lnpb,
                  (void **)&e->p1w.f32, (void **)&e->p1w.b16, (void **)&e->p1b,     (void **)&e->p2w.f32,
                  (void **)&e->p2w.b16, (void **)&e->p2b,     (void **)&e->pe};
    for (size_t i = 0; i < sizeof(w) / sizeof(w[0]); i++) dfree(w[i]);
    for (int l = 0; l < QWEN_HIP_ENC_MAX_LAYERS; l++) {
        enc_layer *y = &e->L[l];
        void **v[] = {(void **)&y->wqkv.f32, (void **)&y->wqkv.b16, (void **)&y->bqkv,     (void **)&y->wo.f32,
                      (void **)&y->wo.b16,   (void **)&y->bo,       (void **)&y->ln1w,     (void **)&y->ln1b,
                      (void **)&y->fc1w.f32, (void **)&y->fc1w.b16, (void **)&y->fc1b,     (void **)&y->fc2w.f32,
                      (void **)&y->fc2w.b16, (void **)&y->fc2b,     (void **)&y->ln2w,     (void **)&y->ln2b};
        for (size_t i = 0; i < sizeof(v) / sizeof(v[0]); i++) dfree(v[i]);
    }
    if (e->stream) (void)hipStreamDestroy(e->stream);
    free(e);
}

/* sinusoidal position table of one chunk (qwen_sinusoidal_pe, qwen_asr_kernels.c:1147-1161) */
static void sinusoid(float *pe, int n_pos, int d) {
    const int half = d / 2;
    const float log_ts = logf(10000.0f) / (float)(half - 1);
    for (int p = 0; p < n_pos; p++)
        for (int i = 0; i < half; i++) {
            const float inv = expf(-(float)i * log_ts);
            const float ang = (float)p * inv;
            pe[(long)p * d + i] = sinf(ang);
            pe[(long)p * d + half + i] = cosf(ang);
        }
}

qwen_hip_encoder *qwen_hip_encoder_create(const qwen_hip_enc_config *cfg, int device) {
    if (!check_cfg(cfg)) {
        qk_set_err("unsupported encoder configuration (head_dim 64, heads*64 = d_model, d_model a multiple of 64, "
                   "at most %d layers)", QWEN_HIP_ENC_MAX_LAYERS);
        return NULL;
    }
    if (hipSetDevice(device) != hipSuccess) { qk_set_err("hipSetDevice(%d) failed", device); return NULL; }
    qwen_hip_encoder *e = (qwen_hip_encoder *)calloc(1, sizeof(*e));
    if (!e) { qk_set_err("out of host memory"); return NULL; }
    e->cfg = *cfg;
    e->device = device;
    if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess) {
        qk_set_err("hipStreamCreate failed");
        free(e);
        return NULL;
    }
    const int tpc = conv_out(conv_out(conv_out(cfg->chunk_size)));
    float *pe = (float *)malloc((size_t)tpc * cfg->d_model * sizeof(float));
    if (!pe || dmalloc((void **)&e->pe, (size_t)tpc * cfg->d_model * 4)) {
        free(pe);
        qwen_hip_encoder_destroy(e);
        return NULL;
    }
    sinusoid(pe, tpc, cfg->d_model);
    if (hipMemcpy(e->pe, pe, (size_t)tpc * cfg->d_model * 4, hipMemcpyHostToDevice) != hipSuccess) {
        free(pe);
        qk_set_err("position table upload failed");
        qwen_hip_encoder_destroy(e);
        return NULL;
    }
    free(pe);
    return e;
}

/* every value of src[0, n) is a bf16 value (its low 16 bits are zero) */
static int bf16_exact(const float *src, size_t n) {
    for (size_t i = 0; i < n; i++) {
        uint32_t u;
        memcpy(&u, src + i, 4);
        if (u & 0xffffu) return 0;
    }
    return 1;
}

/* rows [row0, row0 + n / cols) of a weight matrix: the bf16 copy when the whole
 * matrix (`exact`, decided by the caller) is bf16-valued, else fp32 */
static int up_mat(enc_mat *m, size_t total, size_t off, const float *src, size_t n, int exact) {
    if (!src) { qk_set_err("encoder weight pointer is NULL"); return QWEN_HIP_EINVAL; }
    if (exact) {
        if (m->f32) dfree((void **)&m->f32);
        if (!m->b16) QK_TRY(dmalloc((void **)&m->b16, total * 2));
        uint16_t *h = (uint16_t *)malloc(n * 2);
        if (!h) { qk_set_err("out of host memory"); return QWEN_HIP_ENOMEM; }
        for (size_t i = 0; i < n; i++) {
            uint32_t u;
            memcpy(&u, src + i, 4);
            h[i] = (uint16_t)(u >> 16);
        }
        const hipError_t r = hipMemcpy(m->b16 + off, h, n * 2, hipMemcpyHostToDevice);
        free(h);
        if (r != hipSuccess) { qk_set_err("hipMemcpy: %s", hipGetErrorString(r)); return QWEN_HIP_EDEVICE; }
    } else {
        if (m->b16) dfree((void **)&m->b16);
        if (!m->f32) QK_TRY(dmalloc((void **)&m->f32, total * 4));
        QK_HIP(hipMemcpy(m->f32 + off, src, n * 4, hipMemcpyHostToDevice));
    }
    return 0;
}

static int up(float **dst, const float *src, size_t n) {
    if (!src) { qk_set_err("encoder weight pointer is NULL"); return QWEN_HIP_EINVAL; }
    if (!*dst) QK_TRY(dmalloc((void **)dst, n * sizeof(float)));
    QK_HIP(hipMemcpy(*dst, src, n * sizeof(float), hipMemcpyHostToDevice));
    return 0;
}

int qwen_hip_encoder_load_layer(qwen_hip_encoder *e, int l, const qwen_hip_enc_layer_weights *w) {
    if (!e || !w || l < 0 || l >= e->cfg.layers) {
        qk_set_err("encoder: NULL argument or layer %d outside [0, %d)", l, e ? e->cfg.layers : 0);
        return QWEN_HIP_EINVAL;
    }
    QK_HIP(hipSetDevice(e->device));
    const size_t d = e->cfg.d_model, f = e->cfg.ffn_dim;
    enc_layer *y = &e->L[l];
    /* Q|K|V stacked: rows [0,d) q, [d,2d) k, [2d,3d) v */
    if (!y->bqkv) QK_TRY(dmalloc((void **)&y->bqkv, 3 * d * 4));
    const float *ws[3] = {w->wq, w->wk, w->wv}, *bs[3] = {w->bq, w->bk, w->bv};
    for (int i = 0; i < 3; i++)
        if (!ws[i] || !bs[i]) { qk_set_err("encoder layer %d: NULL q/k/v weight", l); return QWEN_HIP_EINVAL; }
    const int qkv_exact = bf16_exact(ws[0], d * d) && bf16_exact(ws[1], d * d) && bf16_exact(ws[2], d * d);
    for (int i = 0; i < 3; i++) {
        QK_TRY(up_mat(&y->wqkv, 3 * d * d, i * d * d, ws[i], d * d, qkv_exact));
        QK_HIP(hipMemcpy(y->bqkv + i * d, bs[i], d * 4, hipMemcpyHostToDevice));
    }
    QK_TRY(up_mat(&y->wo, d * d, 0, w->wo, d * d, w->wo && bf16_exact(w->wo, d * d)));
    QK_TRY(up(&y->bo, w->bo, d));
    QK_TRY(up(&y->ln1w, w->ln1_w, d));
    QK_TRY(up(&y->ln1b, w->ln1_b, d));
    QK_TRY(up_mat(&y->fc1w, f * d, 0, w->fc1_w, f * d, w->fc1_w && bf16_exact(w->fc1_w, f * d)));
    QK_TRY(up(&y->fc1b, w->fc1_b, f));
    QK_TRY(up_mat(&y->fc2w, d * f, 0, w->fc2_w, d * f, w->fc2_w && bf16_exact(w->fc2_w, d * f)));
    QK_TRY(up(&y->fc2b, w->fc2_b, d));
    QK_TRY(up(&y->ln2w, w->ln2_w, d));
    QK_TRY(up(&y->ln2b, w->ln2_b, d));
    y->loaded = 1;
    return 0;
}

int qwen_hip_encoder_load_stem(qwen_hip_encoder *e, const qwen_hip_enc_stem_weights *w) {
    if (!e || !w || !w->conv1_w) return QWEN_HIP_EINVAL;
    QK_HIP(hipSetDevice(e->device));
    const size_t d = e->cfg.d_model, o = e->cfg.output_dim;
    /* conv1 [480][1][3][3] -> rows of ENC_K1 with the 9 taps first */
    float c1[ENC_CH * ENC_K1];
    memset(c1, 0, sizeof(c1));
    for (int oc = 0; oc < ENC_CH; oc++) memcpy(c1 + oc * ENC_K1, w->conv1_w + oc * 9, 9 * sizeof(float));
    QK_TRY(up(&e->c1w, c1, ENC_CH * ENC_K1));
    QK_TRY(up(&e->c1b, w->conv1_b, ENC_CH));
    const size_t k2 = (size_t)ENC_CH * ENC_K2, ko = d * ENC_CH * 16;
    /* conv2 / conv3 [480][480][3][3]: columns reordered tap-major (k = tap *
     * 480 + ic) to match the channel-last stem activations */
    if (!w->conv2_w || !w->conv3_w) { qk_set_err("encoder weight pointer is NULL"); return QWEN_HIP_EINVAL; }
    float *tm = (float *)malloc(k2 * sizeof(float));
    if (!tm) { qk_set_err("out of host memory"); return QWEN_HIP_ENOMEM; }
    const float *cw[2] = {w->conv2_w, w->conv3_w};
    enc_mat *cm[2] = {&e->c2w, &e->c3w};
    int rc = 0;
    for (int i = 0; i < 2 && !rc; i++) {
        for (size_t oc = 0; oc < ENC_CH; oc++)
            for (size_t ic = 0; ic < ENC_CH; ic++)
                for (size_t tap = 0; tap < 9; tap++)
                    tm[oc * ENC_K2 + tap * ENC_CH + ic] = cw[i][oc * ENC_K2 + ic * 9 + tap];
        rc = up_mat(cm[i], k2, 0, tm, k2, bf16_exact(tm, k2));
    }
    free(tm);
    QK_TRY(rc);
    QK_TRY(up(&e->c2b, w->conv2_b, ENC_CH));
    QK_TRY(up(&e->c3b, w->conv3_b, ENC_CH));
    QK_TRY(up_mat(&e->cow, ko, 0, w->conv_out_w, ko, w->conv_out_w && bf16_exact(w->conv_out_w, ko)));
    QK_TRY(up(&e->lnpw, w->ln_post_w, d));
    QK_TRY(up(&e->lnpb, w->ln_post_b, d));
    QK_TRY(up_mat(&e->p1w, d * d, 0, w->proj1_w, d * d, w->proj1_w && bf16_exact(w->proj1_w, d * d)));
    QK_TRY(up(&e->p1b, w->proj1_b, d));
    QK_TRY(up_mat(&e->p2w, o * d, 0, w->proj2_w, o * d, w->proj2_w && bf16_exact(w->proj2_w, o * d)));
    QK_TRY(up(&e->p2b, w->proj2_b, o));
    e->stem_loaded = 1;
    return 0;
}

/* ---- synthetic weights: bf16 N(0, wstd) matrices widened to fp32 (what a
 * bf16 checkpoint gives the reference), fp32 biases N(0, wstd), LayerNorm
 * weights 1 + N(0, 0.1) and biases N(0, 0.02) ------------------------------ */
static float *syn_mat(size_t n, uint64_t seed, uint64_t id, double std) {
    uint16_t *b = (uint16_t *)malloc(n * 2);
    float *f = (float *)malloc(n * 4);
    if (!b || !f) { free(b); free(f); return NULL; }
    qwen_synth_normal_bf16(b, n, seed, id, 0.0, std, 0);
    for (size_t i = 0; i < n; i++) {
        const uint32_t u = (uint32_t)b[i] << 16;
        memcpy(&f[i], &u, 4);
    }
    free(b);
    return f;
}

static float *syn_vec(size_t n, uint64_t seed, uint64_t id, double mean, double std) {
    float *f = (float *)malloc(n * 4);
    if (f) qwen_synth_normal_f32(f, n, seed, id, mean, std, 0);
    return f;
}

int qwen_hip_encoder_load_synthetic(qwen_hip_encoder *e, uint64_t seed, double wstd) {
    if (!e) return QWEN_HIP_EINVAL;
    const qwen_hip_enc_config *c = &e->cfg;
    const size_t d = c->d_model, f = c->ffn_dim, o = c->output_dim;
    int rc = 0;
    for (int l = 0; l < c->layers && !rc; l++) {
#define ID(x) QWEN_SYNTH_ENC(l, QWEN_SYNTH_E_##x)
        float *p[16] = {syn_mat(d * d, seed, ID(WQ), wstd), syn_vec(d, seed, ID(BQ), 0, wstd),
                        syn_mat(d * d, seed, ID(WK), wstd), syn_vec(d, seed, ID(BK), 0, wstd),
                        syn_mat(d * d, seed, ID(WV), wstd), syn_vec(d, seed, ID(BV), 0, wstd),
                        syn_mat(d * d, seed, ID(WO), wstd), syn_vec(d, seed, ID(BO), 0, wstd),
                        syn_vec(d, seed, ID(LN1W), 1.0, 0.1), syn_vec(d, seed, ID(LN1B), 0, 0.02),
                        syn_mat(f * d, seed, ID(FC1W), wstd), syn_vec(f, seed, ID(FC1B), 0, wstd),
                        syn_mat(d * f, seed, ID(FC2W), wstd), syn_vec(d, seed, ID(FC2B), 0, wstd),
                        syn_vec(d, seed, ID(LN2W), 1.0, 0.1), syn_vec(d, seed, ID(LN2B), 0, 0.02)};
#undef ID
        int ok = 1;
        for (int i = 0; i < 16; i++) ok = ok && p[i];
        if (ok) {
            qwen_hip_enc_layer_weights w = {p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8],
                                            p[9], p[10], p[11], p[12], p[13], p[14], p[15]};
            rc = qwen_hip_encoder_load_layer(e, l, &w);
        } else {
            qk_set_err("out of host memory");
            rc = QWEN_HIP_ENOMEM;
        }
        for (int i = 0; i < 16; i++) free(p[i]);
    }
    if (rc) return rc;
#define SID(x) QWEN_SYNTH_ENC(QWEN_SYNTH_ENC_STEM, QWEN_SYNTH_S_##x)
    float *p[13] = {syn_mat(ENC_CH * 9, seed, SID(CONV1W), wstd * 10), syn_vec(ENC_CH, seed, SID(CONV1B), 0, wstd),
                    syn_mat((size_t)ENC_CH * ENC_K2, seed, SID(CONV2W), wstd), syn_vec(ENC_CH, seed, SID(CONV2B), 0, wstd),
                    syn_mat((size_t)ENC_CH * ENC_K2, seed, SID(CONV3W), wstd), syn_vec(ENC_CH, seed, SID(CONV3B), 0, wstd),
                    syn_mat(d * ENC_CH * 16, seed, SID(CONVOUT), wstd), syn_vec(d, seed, SID(LNPW), 1.0, 0.1),
                    syn_vec(d, seed, SID(LNPB), 0, 0.02), syn_mat(d * d, seed, SID(P1W), wstd),
                    syn_vec(d, seed, SID(P1B), 0, wstd), syn_mat(o * d, seed, SID(P2W), wstd),
                    syn_vec(o, seed, SID(P2B), 0, wstd)};
#undef SID
    int ok = 1;
    for (int i = 0; i < 13; i++) ok = ok && p[i];
    if (ok) {
        qwen_hip_enc_stem_weights w = {p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8], p[9], p[10], p[11], p[12]};
        rc = qwen_hip_encoder_load_stem(e, &w);
    } else {
        qk_set_err("out of host memory");
        rc = QWEN_HIP_ENOMEM;
    }
    for (int i = 0; i < 13; i++) free(p[i]);
    return rc;
}

/* ---- forward ------------------------------------------------------------ */
static int reserve(qwen_hip_encoder *e, int chunks, int tokens) {
    if (chunks <= e->cap_chunks) return 0;
    QK_HIP(hipStreamSynchronize(e->stream));
    act_free(e);
    const qwen_hip_enc_config *c = &e->cfg;
    const size_t cw = c->chunk_size;
    const size_t w1 = conv_out(cw), w2 = conv_out(w1), w3 = conv_out(w2);
    const size_t n1 = (size_t)chunks * 64 * w1, n2 = (size_t)chunks * 32 * w2, n3 = (size_t)chunks * 16 * w3;
    size_t cols = n1 * ENC_K1;
    if (n2 * ENC_K2 > cols) cols = n2 * ENC_K2;
    if (n3 * ENC_K2 > cols) cols = n3 * ENC_K2;
    const size_t T = (size_t)chunks * w3;   /* >= tokens */
    (void)tokens;
    const size_t d = c->d_model;
    int rc = dmalloc((void **)&e->mel, (size_t)ENC_MEL * chunks * cw * 4);
    if (!rc) rc = dmalloc((void **)&e->cols, cols * 4);
    if (!rc) rc = dmalloc((void **)&e->c1, (size_t)ENC_CH * n1 * 4);
    if (!rc) rc = dmalloc((void **)&e->c2, (size_t)ENC_CH * n2 * 4);
    if (!rc) rc = dmalloc((void **)&e->c3, (size_t)ENC_CH * n3 * 4);
    if (!rc) rc = dmalloc((void **)&e->rows, T * ENC_CH * 16 * 4);
    if (!rc) rc = dmalloc((void **)&e->x, T * d * 4);
    if (!rc) rc = dmalloc((void **)&e->xn, T * d * 4);
    if (!rc) rc = dmalloc((void **)&e->qkv, T * 3 * d * 4);
    if (!rc) rc = dmalloc((void **)&e->att, T * d * 4);
    if (!rc) rc = dmalloc((void **)&e->mid, T * (size_t)(c->ffn_dim > (int)d ? c->ffn_dim : (int)d) * 4);
    if (!rc) rc = dmalloc((void **)&e->out, T * (size_t)c->output_dim * 4);
    if (!rc) rc = dmalloc((void **)&e->gws, (size_t)QK_ENC_GEMM_WS_ELEMS * 4);
    if (rc) { act_free(e); return rc; }
    e->cap_chunks = chunks;
    return 0;
}

/* C = A . W^T with the activations A [M][K] and a weight matrix W [N][K] */
static int gemm(qwen_hip_encoder *e, const float *A, int lda, const enc_mat *W, int ldb, float *C, int ldc, int M,
                int N, int K, const float *bias_m, const float *bias_n, int gelu, int add) {
    qk_enc_gemm_args g = {.A = A, .B = W->f32, .C = C, .M = M, .N = N, .K = K, .lda = lda, .ldb = ldb, .ldc = ldc,
                          .bias_m = bias_m, .bias_n = bias_n, .gelu = gelu, .add = add,
                          .ws = e->gws, .ws_elems = QK_ENC_GEMM_WS_ELEMS, .B16 = W->b16};
    return qk_enc_gemm_launch(&g, e->stream);
}

/* x += A . W^T + bias (the residual projections), then xn = LayerNorm(x) (w, b) */
static int gemm_add_ln(qwen_hip_encoder *e, const float *A, int lda, const enc_mat *W, int K, const float *bias,
                       int T, const float *lnw, const float *lnb) {
    const int d = e->cfg.d_model;
    qk_enc_gemm_args g = {.A = A, .B = W->f32, .C = e->x, .M = T, .N = d, .K = K, .lda = lda, .ldb = K, .ldc = d,
                          .bias_n = bias, .add = 1, .ws = e->gws, .ws_elems = QK_ENC_GEMM_WS_ELEMS, .B16 = W->b16,
                          .ln_w = lnw, .ln_b = lnb, .ln_out = e->xn, .ln_eps = 1e-5f};
    return qk_enc_gemm_launch(&g, e->stream);
}

/* one stem layer, channel-last output [chunk][h_out][w_out][480] = GEMM rows
 * (position) x columns (output channel), bias + GELU, padding zeroed.  conv1
 * (mel_frames > 0): im2col of the mel, then a direct 9-tap pass.  conv2 / conv3 (input
 * channel-last): with bf16 weights the product reads the input as an
 * implicit im2col, else through a channel-last im2col into e->cols. */
static int stem_layer(qwen_hip_encoder *e, const float *in, int c_in, int chunks, int h_in, int w_in, int kpad,
                      int mel_frames, const float *w, const uint16_t *w16, const float *b, float *out,
                      int valid_last) {
    const int h_out = conv_out(h_in), w_out = conv_out(w_in);
    const int M = chunks * h_out * w_out;
    const int implicit = mel_frames == 0 && w16;
    if (!implicit)
        QK_TRY(qk_enc_im2col_launch(in, e->cols, c_in, chunks, h_in, w_in, h_out, w_out, kpad, mel_frames,
                                    e->stream));
    if (mel_frames > 0)   /* conv1: 9 taps per output, a direct pass */
        return qk_enc_conv1_launch(e->cols, kpad, w, b, out, M, ENC_CH, h_out, w_out, chunks, valid_last, e->stream);
    qk_enc_gemm_args g = {.A = implicit ? in : e->cols, .B = w, .C = out, .M = M, .N = ENC_CH, .K = kpad,
                          .lda = kpad, .ldb = kpad, .ldc = ENC_CH, .bias_n = b, .gelu = 1, .col_w = w_out,
                          .col_h = h_out, .col_chunks = chunks, .col_valid = valid_last, .pad_rows = 1,
                          .conv_c = implicit ? c_in : 0, .conv_in_h = h_in, .conv_in_w = w_in, .B16 = w16};
    return qk_enc_gemm_launch(&g, e->stream);
}

static int run(qwen_hip_encoder *e, int mel_frames, int *tokens_out) {
    const qwen_hip_enc_config *c = &e->cfg;
    const int cw = c->chunk_size, d = c->d_model, H = c->heads;
    const int chunks = (mel_frames + cw - 1) / cw;
    const int last = mel_frames - (chunks - 1) * cw;
    const int w1 = conv_out(cw), w2 = conv_out(w1), w3 = conv_out(w2);
    const int T = qwen_hip_encoder_tokens(c, mel_frames);
    /* conv stem (qwen_asr_encoder.c:237-279); the mel is [128][mel_frames] */
    QK_TRY(stem_layer(e, e->mel, 1, chunks, ENC_MEL, cw, ENC_K1, mel_frames, e->c1w, NULL, e->c1b, e->c1,
                      conv_out(last)));
    QK_TRY(stem_layer(e, e->c1, ENC_CH, chunks, 64, w1, ENC_K2, 0, e->c2w.f32, e->c2w.b16, e->c2b, e->c2,
                      conv_out(conv_out(last))));
    QK_TRY(stem_layer(e, e->c2, ENC_CH, chunks, 32, w2, ENC_K2, 0, e->c3w.f32, e->c3w.b16, e->c3b, e->c3,
                      conv_out(conv_out(conv_out(last)))));
    /* [480][16][w3] per chunk -> token rows [T][7680], project, add the chunk's positions (:281-301) */
    QK_TRY(qk_enc_stem_rows_launch(e->c3, e->rows, chunks, w3, 16, ENC_CH, T, e->stream));
    {
        qk_enc_gemm_args g = {.A = e->rows, .B = e->cow.f32, .C = e->x, .M = T, .N = d, .K = ENC_CH * 16,
                              .lda = ENC_CH * 16, .ldb = ENC_CH * 16, .ldc = d, .pe = e->pe, .pe_rows = w3,
                              .ws = e->gws, .ws_elems = QK_ENC_GEMM_WS_ELEMS, .B16 = e->cow.b16};
        QK_TRY(qk_enc_gemm_launch(&g, e->stream));
    }
    const int win = w3 * (c->n_window_infer / cw);
    const float scale = 1.0f / sqrtf((float)c->head_dim);
    /* pre-LayerNorm layers (:318-353): each residual projection's split-K
     * reduce also applies the next LayerNorm (ln2, the next layer's ln1, ln_post) */
    QK_TRY(qk_enc_layernorm_launch(e->x, e->L[0].ln1w, e->L[0].ln1b, e->xn, T, d, 1e-5f, e->stream));
    for (int l = 0; l < c->layers; l++) {
        const enc_layer *y = &e->L[l];
        QK_TRY(gemm(e, e->xn, d, &y->wqkv, d, e->qkv, 3 * d, T, 3 * d, d, NULL, y->bqkv, 0, 0));
        QK_TRY(qk_enc_attention_launch(e->qkv, e->att, T, H, 64, win, scale, e->stream));
        QK_TRY(gemm_add_ln(e, e->att, d, &y->wo, d, y->bo, T, y->ln2w, y->ln2b));
        QK_TRY(gemm(e, e->xn, d, &y->fc1w, d, e->mid, c->ffn_dim, T, c->ffn_dim, d, NULL, y->fc1b, 1, 0));
        const int last = l + 1 == c->layers;
        QK_TRY(gemm_add_ln(e, e->mid, c->ffn_dim, &y->fc2w, c->ffn_dim, y->fc2b, T,
                           last ? e->lnpw : e->L[l + 1].ln1w, last ? e->lnpb : e->L[l + 1].ln1b));
    }
    /* proj1 + GELU, proj2 on the ln_post rows (:358-371) */
    QK_TRY(gemm(e, e->xn, d, &e->p1w, d, e->mid, d, T, d, d, NULL, e->p1b, 1, 0));
    QK_TRY(gemm(e, e->mid, d, &e->p2w, d, e->out, c->output_dim, T, c->output_dim, d, NULL, e->p2b, 0, 0));
    *tokens_out = T;
    return 0;
}

static int ready(qwen_hip_encoder *e, int mel_frames) {
    if (!e || mel_frames <= 0) { qk_set_err("encoder: bad argument"); return QWEN_HIP_EINVAL; }
    if (!e->stem_loaded) { qk_set_err("encoder: stem weights not loaded"); return QWEN_HIP_ESTATE; }
    for (int l = 0; l < e->cfg.layers; l++)
        if (!e->L[l].loaded) { qk_set_err("encoder: layer %d not loaded", l); return QWEN_HIP_ESTATE; }
    QK_HIP(hipSetDevice(e->device));
    const int chunks = (mel_frames + e->cfg.chunk_size - 1) / e->cfg.chunk_size;
    return reserve(e, chunks, qwen_hip_encoder_tokens(&e->cfg, mel_frames));
}

int qwen_hip_encoder_forward(qwen_hip_encoder *e, const float *mel, int mel_frames, float *out) {
    int rc = ready(e, mel_frames);
    if (rc) return rc;
    if (!mel || !out) { qk_set_err("encoder: NULL mel or output"); return QWEN_HIP_EINVAL; }
    QK_HIP(hipMemcpyAsync(e->mel, mel, (size_t)ENC_MEL * mel_frames * 4, hipMemcpyHostToDevice, e->stream));
    int T = 0;
    QK_TRY(run(e, mel_frames, &T));
    QK_HIP(hipMemcpyAsync(out, e->out, (size_t)T * e->cfg.output_dim * 4, hipMemcpyDeviceToHost, e->stream));
    QK_HIP(hipStreamSynchronize(e->stream));
    return T;
}

int qwen_hip_encoder_forward_device(qwen_hip_encoder *e, const float *d_mel, int mel_frames, const float **d_out) {
    int rc = ready(e, mel_frames);
    if (rc) return rc;
    if (!d_mel || !d_out) { qk_set_err("encoder: NULL mel or output"); return QWEN_HIP_EINVAL; }
    QK_HIP(hipMemcpyAsync(e->mel, d_mel, (size_t)ENC_MEL * mel_frames * 4, hipMemcpyDeviceToDevice, e->stream));
    int T = 0;
    QK_TRY(run(e, mel_frames, &T));
    QK_HIP(hipStreamSynchronize(e->stream));
    *d_out = e->out;
    return T;
}

hipStream_t qwen_hip_encoder_stream(const qwen_hip_encoder *e) { return e ? e->stream : NULL; }

const qwen_hip_enc_config *qwen_hip_encoder_config(const qwen_hip_encoder *e) { return e ? &e->cfg : NULL; }
