/*
 * ref_harness.c - TEST INFRASTRUCTURE.  Drives the reference's own decoder
 * (qwen_decoder_prefill / qwen_decoder_forward, reference
 * qwen_asr_decoder.c:262 and :388) compiled unmodified from /root/reference
 * into oracle/_ref/.  Used only by tests, golden-fixture generation and the
 * CPU-baseline leg of bench.py; never by the product path.
 *
 * The reference loads weights from safetensors (qwen_decoder_load,
 * qwen_asr_decoder.c:45-116).  There are no checkpoints offline, so this
 * harness points the qwen_dec_layer_t fields at caller-owned synthetic host
 * buffers instead and does the two transformations the loader does: the
 * gate/up row interleave (:95-107) and fp32 norm vectors (:69-78, :112).
 * qwen_verbose normally lives in qwen_asr.c, which is not linked here.
 */
#include "qwen_asr.h"
#include "qwen_asr_kernels.h"

#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

int qwen_verbose = 0;

typedef struct {
    qwen_ctx_t *ctx;
    uint16_t *gate_up[QWEN_MAX_DEC_LAYERS];
} ref_model_t;

void *ref_create(int hidden, int layers, int heads, int kv_heads, int head_dim,
                 int intermediate, int vocab, float eps, float theta) {
    if (layers > QWEN_MAX_DEC_LAYERS) return NULL;
    ref_model_t *m = (ref_model_t *)calloc(1, sizeof(ref_model_t));
    if (!m) return NULL;
    m->ctx = (qwen_ctx_t *)calloc(1, sizeof(qwen_ctx_t));
    if (!m->ctx) { free(m); return NULL; }
    qwen_config_t *c = &m->ctx->config;
    c->dec_hidden = hidden;
    c->dec_layers = layers;
    c->dec_heads = heads;
    c->dec_kv_heads = kv_heads;
    c->dec_head_dim = head_dim;
    c->dec_intermediate = intermediate;
    c->vocab_size = vocab;
    c->dec_rms_norm_eps = eps;
    c->dec_rope_theta = theta;
    return m;
}

/* Borrow one layer's weights (bf16 [out][in], fp32 norms).  The caller keeps
 * the buffers alive for the model's lifetime, as the mmap does. */
int ref_set_layer(void *mp, int layer,
                  const uint16_t *wq, const uint16_t *wk, const uint16_t *wv,
                  const uint16_t *wo, const uint16_t *gate, const uint16_t *up,
                  const uint16_t *down, const float *q_norm, const float *k_norm,
                  const float *input_norm, const float *post_attn_norm) {
    ref_model_t *m = (ref_model_t *)mp;
    qwen_ctx_t *ctx = m->ctx;
    const qwen_config_t *c = &ctx->config;
    if (layer < 0 || layer >= c->dec_layers) return -1;
    qwen_dec_layer_t *l = &ctx->decoder.layers[layer];
    l->wq_weight_bf16 = (uint16_t *)wq;
    l->wk_weight_bf16 = (uint16_t *)wk;
    l->wv_weight_bf16 = (uint16_t *)wv;
    l->wo_weight_bf16 = (uint16_t *)wo;
    l->gate_weight_bf16 = (uint16_t *)gate;
    l->up_weight_bf16 = (uint16_t *)up;
    l->down_weight_bf16 = (uint16_t *)down;
    l->q_norm_weight = (float *)q_norm;
    l->k_norm_weight = (float *)k_norm;
    l->input_norm = (float *)input_norm;
    l->post_attn_norm = (float *)post_attn_norm;

    size_t hid = (size_t)c->dec_hidden, inter = (size_t)c->dec_intermediate;
    free(m->gate_up[layer]);
    uint16_t *gu = (uint16_t *)malloc(2 * inter * hid * sizeof(uint16_t));
    if (!gu) return -1;
    for (size_t r = 0; r < inter; r++) {
        memcpy(gu + (2 * r) * hid, gate + r * hid, hid * sizeof(uint16_t));
        memcpy(gu + (2 * r + 1) * hid, up + r * hid, hid * sizeof(uint16_t));
    }
    m->gate_up[layer] = gu;
    l->gate_up_fused_bf16 = gu;
    return 0;
}

void ref_set_embeddings(void *mp, const uint16_t *tok_emb, const float *final_norm) {
    ref_model_t *m = (ref_model_t *)mp;
    m->ctx->decoder.tok_embeddings_bf16 = (uint16_t *)tok_emb;
    m->ctx->decoder.norm = (float *)final_norm;
}

void ref_set_threads(int n) { qwen_set_threads(n); }

void ref_prefill(void *mp, const float *rows, int n) {
    qwen_decoder_prefill(((ref_model_t *)mp)->ctx, rows, n);
}

/* One reference forward.  hidden_out (optional) gets ctx->dec_x, the
 * final-normed hidden state (:474).  logits_out (optional) gets the full LM
 * head output computed with the same bf16 matvec the argmax streams over
 * (qwen_linear_nobias_bf16 with seq 1). */
int ref_forward(void *mp, const float *row, float *hidden_out, float *logits_out) {
    qwen_ctx_t *ctx = ((ref_model_t *)mp)->ctx;
    int tok = qwen_decoder_forward(ctx, row);
    const qwen_config_t *c = &ctx->config;
    if (hidden_out && ctx->dec_x)
        memcpy(hidden_out, ctx->dec_x, (size_t)c->dec_hidden * sizeof(float));
    if (logits_out && ctx->dec_x)
        qwen_linear_nobias_bf16(logits_out, ctx->dec_x, ctx->decoder.tok_embeddings_bf16,
                                1, c->dec_hidden, c->vocab_size);
    return tok;
}

/* tok_embed_bf16_to_f32 (qwen_asr.c:353-360) is static there; same widening. */
void ref_embed_token(void *mp, int token, float *out) {
    qwen_ctx_t *ctx = ((ref_model_t *)mp)->ctx;
    int dim = ctx->config.dec_hidden;
    const uint16_t *src = ctx->decoder.tok_embeddings_bf16 + (size_t)token * dim;
    for (int i = 0; i < dim; i++) {
        uint32_t b = (uint32_t)src[i] << 16;
        memcpy(&out[i], &b, 4);
    }
}

int ref_kv_len(void *mp) { return ((ref_model_t *)mp)->ctx->kv_cache_len; }
/* The widening of bf16_to_f32_buf (qwen_asr_kernels.c:232-236, static
 * there), which the reference's seq > 1 linear runs on every weight before
 * its GEMM (bf16_get_f32_view, :322-330); for the CPU baseline's BLAS-path
 * estimate. */
void ref_bf16_widen(float *dst, const uint16_t *src, long n) {
    uint32_t *d = (uint32_t *)(void *)dst;
    for (long i = 0; i < n; i++) d[i] = ((uint32_t)src[i]) << 16;
}

/* Capacity of the reference's KV cache (kv_cache_max, qwen_asr_decoder.c:122-160). */
int ref_kv_max(void *mp) { return ((ref_model_t *)mp)->ctx->kv_cache_max; }
void ref_set_kv_len(void *mp, int n) { ((ref_model_t *)mp)->ctx->kv_cache_len = n; }

/* Greedy loop of qwen_asr.c:729-759 without EOS stop: n_steps forwards, each
 * fed the previous token's embedding.  Returns wall seconds of the loop. */
double ref_generate(void *mp, int first_token, int n_steps, int *out_tokens) {
    qwen_ctx_t *ctx = ((ref_model_t *)mp)->ctx;
    int dim = ctx->config.dec_hidden;
    float *emb = (float *)malloc((size_t)dim * sizeof(float));
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    int tok = first_token;
    for (int i = 0; i < n_steps; i++) {
        ref_embed_token(mp, tok, emb);
        tok = qwen_decoder_forward(ctx, emb);
        out_tokens[i] = tok;
    }
    clock_gettime(CLOCK_MONOTONIC, &t1);
    free(emb);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

/* Wall-clock helper for the CPU baseline: prefill n rows, return seconds. */
double ref_time_prefill(void *mp, const float *rows, int n) {
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    qwen_decoder_prefill(((ref_model_t *)mp)->ctx, rows, n);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

void ref_destroy(void *mp) {
    ref_model_t *m = (ref_model_t *)mp;
    if (!m) return;
    qwen_ctx_t *ctx = m->ctx;
    for (int i = 0; i < QWEN_MAX_DEC_LAYERS; i++) free(m->gate_up[i]);
    free(ctx->kv_cache_k); free(ctx->kv_cache_v);
    free(ctx->dec_x); free(ctx->dec_x_norm); free(ctx->dec_q); free(ctx->dec_k);
    free(ctx->dec_v); free(ctx->dec_attn_out); free(ctx->dec_proj_out);
    free(ctx->dec_gate); free(ctx->dec_ffn_out); free(ctx->dec_rope_cos);
    free(ctx->dec_rope_sin);
    free(ctx->pref_x); free(ctx->pref_x_norm); free(ctx->pref_q); free(ctx->pref_k);
    free(ctx->pref_v); free(ctx->pref_attn_out); free(ctx->pref_proj_out);
    free(ctx->pref_ffn_out); free(ctx->pref_gate); free(ctx->pref_gate_up);
    free(ctx->rope_cache_cos); free(ctx->rope_cache_sin); free(ctx->rope_inv_freq);
    free(ctx);
    free(m);
}

/* ------------------------------------------------------------------------
 * The reference's audio encoder (qwen_encoder_forward, qwen_asr_encoder.c:
 * 171-372).  qwen_encoder_load (:67-168) reads safetensors; here the
 * qwen_encoder_t fields point at caller-owned fp32 buffers instead (the
 * loader's own output format: bf16 matrices widened to fp32).
 * ------------------------------------------------------------------------ */
void *ref_enc_create(int d_model, int layers, int heads, int head_dim, int ffn, int out_dim, int chunk,
                     int n_window_infer) {
    if (layers > QWEN_MAX_ENC_LAYERS) return NULL;
    qwen_ctx_t *ctx = (qwen_ctx_t *)calloc(1, sizeof(qwen_ctx_t));
    if (!ctx) return NULL;
    qwen_config_t *c = &ctx->config;
    c->enc_d_model = d_model;
    c->enc_layers = layers;
    c->enc_heads = heads;
    c->enc_head_dim = head_dim;
    c->enc_ffn_dim = ffn;
    c->enc_output_dim = out_dim;
    c->enc_chunk_size = chunk;
    c->enc_n_window = chunk / 2;
    c->enc_n_window_infer = n_window_infer;
    c->enc_conv_proj_dim = QWEN_CONV_HIDDEN * 16;
    return ctx;
}

int ref_enc_set_layer(void *p, int l, float *wq, float *bq, float *wk, float *bk, float *wv, float *bv, float *wo,
                      float *bo, float *ln1w, float *ln1b, float *fc1w, float *fc1b, float *fc2w, float *fc2b,
                      float *ln2w, float *ln2b) {
    qwen_ctx_t *ctx = (qwen_ctx_t *)p;
    if (l < 0 || l >= ctx->config.enc_layers) return -1;
    qwen_enc_layer_t *y = &ctx->encoder.layers[l];
    y->wq_weight = wq; y->wq_bias = bq; y->wk_weight = wk; y->wk_bias = bk;
    y->wv_weight = wv; y->wv_bias = bv; y->wo_weight = wo; y->wo_bias = bo;
    y->attn_norm_weight = ln1w; y->attn_norm_bias = ln1b;
    y->fc1_weight = fc1w; y->fc1_bias = fc1b; y->fc2_weight = fc2w; y->fc2_bias = fc2b;
    y->ffn_norm_weight = ln2w; y->ffn_norm_bias = ln2b;
    return 0;
}

int ref_enc_set_stem(void *p, float *c1w, float *c1b, float *c2w, float *c2b, float *c3w, float *c3b, float *cow,
                     float *lnpw, float *lnpb, float *p1w, float *p1b, float *p2w, float *p2b) {
    qwen_encoder_t *e = &((qwen_ctx_t *)p)->encoder;
    e->conv1_weight = c1w; e->conv1_bias = c1b; e->conv2_weight = c2w; e->conv2_bias = c2b;
    e->conv3_weight = c3w; e->conv3_bias = c3b; e->conv_out_weight = cow;
    e->ln_post_weight = lnpw; e->ln_post_bias = lnpb;
    e->proj1_weight = p1w; e->proj1_bias = p1b; e->proj2_weight = p2w; e->proj2_bias = p2b;
    return 0;
}

/* mel [128][frames] -> out [tokens][out_dim] (cap floats); returns tokens, -1 on failure */
int ref_enc_forward(void *p, const float *mel, int frames, float *out, long cap) {
    qwen_ctx_t *ctx = (qwen_ctx_t *)p;
    int T = 0;
    float *o = qwen_encoder_forward(ctx, mel, frames, &T);
    if (!o) return -1;
    if ((long)T * ctx->config.enc_output_dim > cap) { free(o); return -1; }
    memcpy(out, o, (size_t)T * ctx->config.enc_output_dim * sizeof(float));
    free(o);
    return T;
}

double ref_enc_time(void *p, const float *mel, int frames, float *out, long cap) {
    struct timespec a, b;
    clock_gettime(CLOCK_MONOTONIC, &a);
    int T = ref_enc_forward(p, mel, frames, out, cap);
    clock_gettime(CLOCK_MONOTONIC, &b);
    return T < 0 ? -1.0 : (b.tv_sec - a.tv_sec) + 1e-9 * (b.tv_nsec - a.tv_nsec);
}

void ref_enc_destroy(void *p) { free(p); }
