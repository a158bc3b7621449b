/*
 * decoder.c - host side of the Qwen3 decoder token loop on one MI355X.
 *
 * Mirrors the reference decoder (qwen_asr_decoder.c) with every tensor
 * resident in HBM:
 *   weights     per layer Wqkv [q_dim+2*kv_dim][hidden] (Wq|Wk|Wv stacked so
 *               one GEMV streams all three, as the fused-dispatch
 *               qwen_linear_nobias_bf16_qkv does, qwen_asr_kernels.c:434-460),
 *               Wo, Wgu [2*inter][hidden] with rows interleaved g0,u0,g1,u1
 *               (qwen_asr_decoder.c:95-107), Wdown; tied embedding / LM head.
 *   KV cache    fp32 like the reference (:122-131) but laid out
 *               [layer][kv_head][position][128] so one head's keys stream
 *               contiguously; grown by doubling (:133-160).
 *   RoPE table  fp32 cos/sin [position][128] from the reference's formulas
 *               (:207-256), computed on the host once per capacity.
 * The decode step is a fixed kernel sequence whose only per-step state lives
 * in device memory (position, input token), so it is captured once into a
 * HIP graph and replayed; generate() replays it n times with no host round
 * trip per token.
 */
#include "host_internal.h"

#include <math.h>
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[512];

void qk_set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

const char *qwen_hip_last_error(void) { return g_err; }

void qwen_hip_config_preset(qwen_hip_config *c, int model_b) {
    /* detect_config, qwen_asr.c:153-186 */
    c->hidden = model_b ? 2048 : 1024;
    c->layers = 28;
    c->heads = 16;
    c->kv_heads = 8;
    c->head_dim = 128;
    c->intermediate = model_b ? 6144 : 3072;
    c->vocab = QWEN_HIP_VOCAB_SIZE;
    c->rms_eps = 1e-6f;
    c->rope_theta = 1e6f;
}

/* Decode attention split budgets.  Up to QK_SHORT_MAX cached positions the
 * step uses at most QK_MERGE_MAX_SPLIT splits and the O-projection merges
 * them in its prologue (graph variant 0); beyond that it uses up to
 * QK_ATTN_MAX_SPLIT splits and a separate merge kernel (variant 1).  The
 * host knows every step's position, so it picks the variant per step. */
#define QK_SHORT_MAX 2048
enum { STEP_SHORT = 0, STEP_LONG = 1, STEP_VARIANTS = 2 };

/* Decode engines: one kernel per fused op replayed from a HIP graph, the same
 * kernels launched eagerly, or the whole greedy loop in one persistent kernel. */
enum { ENGINE_GRAPH = 0, ENGINE_EAGER = 1, ENGINE_PERSIST = 2 };

/* Control block (one device allocation): the input token of the next step,
 * its position (= kv_len) and the generate log cursor. */
enum { CTL_TOK = 0, CTL_POS = 1, CTL_COUNTER = 2, CTL_INTS = 64 };

struct qwen_hip_decoder {
    qwen_hip_config cfg;
    int device;
    hipStream_t stream;
    int qd, kvd, qkv_rows;
    float scale;

    /* weights (one allocation) */
    void *wbuf;
    uint16_t *w_qkv[QWEN_HIP_MAX_LAYERS], *w_o[QWEN_HIP_MAX_LAYERS];
    uint16_t *w_gu[QWEN_HIP_MAX_LAYERS], *w_down[QWEN_HIP_MAX_LAYERS];
    float *n_in[QWEN_HIP_MAX_LAYERS], *n_post[QWEN_HIP_MAX_LAYERS];
    float *n_q[QWEN_HIP_MAX_LAYERS], *n_k[QWEN_HIP_MAX_LAYERS];
    uint16_t *emb;
    float *fnorm;
    unsigned char loaded[QWEN_HIP_MAX_LAYERS];
    int emb_loaded;

    /* KV cache + RoPE table, both sized kv_cap positions */
    float *kc, *vc;
    float *rope_cos, *rope_sin;
    int kv_cap, kv_len;

    /* decode buffers */
    float *x, *qkv, *attn_out, *h, *hidden, *logits, *cand_val;
    float *part_o, *part_m, *part_l; /* attention split partials */
    int *cand_idx, n_cand;
    int *ctl;                 /* control block, see CTL_* */
    int *d_tok, *d_pos, *d_counter, *d_log, log_cap;
    float *h_row;             /* pinned staging */
    int *h_int;

    /* prefill buffers, sized pref_cap rows */
    int pref_cap;
    float *px, *pqkv, *pqrot;
    float *pattn;            /* prefill attention split partials */
    size_t pattn_floats;
    float *pgemm;            /* prefill split-K GEMM partials */
    size_t pgemm_floats;
    uint16_t *pxh, *pxl, *pah, *pal, *phh, *phl;

    hipGraph_t graph[STEP_VARIANTS];
    hipGraphExec_t gexec[STEP_VARIANTS];
    int engine, keep_logits;

    /* persistent engine: exchange words (one allocation), tickets + error word */
    int px_ok;
    unsigned long long *px_buf;
    size_t px_words;
    unsigned long long *xq, *xa, *xm, *xo, *xla, *xh, *xd, *xlb, *xc, *xv;
    unsigned *px_ctl;         /* [0, 16) per-XCD tickets, [16] error bits */
    unsigned px_epoch;
    unsigned long long *px_trace;   /* [256][QK_PX_TRACE] when tracing */
    int px_trace_step;              /* < 0: off */
    unsigned long long px_wait_ticks; /* bound of every in-kernel wait (device wall-clock ticks) */
    double px_ticks_per_s;
    int px_fallback;                /* 1: a failed persistent launch is redone by the graph engine */
    int px_fallbacks;               /* number of such fallbacks */

    /* relay kernel (0.6B shape): tiled weights and its own exchange words */
    int rl_ok, rl_on;
    char *wt;                       /* QK_RL_LAYER_BYTES per layer */
    unsigned long long *rl_buf;
    size_t rl_words;
    unsigned long long *rq, *ra, *rm, *ro, *rla, *rh, *rd, *rs, *rlb, *rc, *rv;
    int last_kernel;                /* QWEN_HIP_KERNEL_* of the last persistent launch */
};

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

static int dev_alloc(void **p, size_t n) {
    hipError_t e = hipMalloc(p, n ? n : 256);
    if (e != hipSuccess) {
        *p = NULL;
        qk_set_err("hipMalloc(%zu): %s", n, hipGetErrorString(e));
        return e == hipErrorOutOfMemory ? QWEN_HIP_ENOMEM : QWEN_HIP_EDEVICE;
    }
    return 0;
}

static void dev_free(void *p) {
    if (p) (void)hipFree(p);
}

static int use_device(const qwen_hip_decoder *d) {
    QK_HIP(hipSetDevice(d->device));
    return 0;
}

static void graph_drop(qwen_hip_decoder *d) {
    for (int v = 0; v < STEP_VARIANTS; v++) {
        if (d->gexec[v]) (void)hipGraphExecDestroy(d->gexec[v]);
        if (d->graph[v]) (void)hipGraphDestroy(d->graph[v]);
        d->gexec[v] = NULL;
        d->graph[v] = NULL;
    }
}

/* RoPE cos/sin table for positions [0, cap): ensure_rope_inv_freq and
 * ensure_rope_cache, qwen_asr_decoder.c:207-256. */
static int rope_build(qwen_hip_decoder *d, int cap) {
    const int hd = d->cfg.head_dim, half = hd / 2;
    size_t n = (size_t)cap * hd;
    float *hc = (float *)malloc(n * sizeof(float)), *hs = (float *)malloc(n * sizeof(float));
    float inv[QWEN_HIP_HEAD_DIM / 2];
    if (!hc || !hs) { free(hc); free(hs); qk_set_err("host alloc for RoPE table"); return QWEN_HIP_ENOMEM; }
    for (int i = 0; i < half; i++) inv[i] = 1.0f / powf(d->cfg.rope_theta, (float)(2 * i) / (float)hd);
    for (int p = 0; p < cap; p++) {
        float *c = hc + (size_t)p * hd, *s = hs + (size_t)p * hd;
        for (int i = 0; i < half; i++) {
            float a = (float)p * inv[i];
            float cv = cosf(a), sv = sinf(a);
            c[i] = cv; c[half + i] = cv;
            s[i] = sv; s[half + i] = sv;
        }
    }
    float *dc = NULL, *ds = NULL;
    int rc = dev_alloc((void **)&dc, n * sizeof(float));
    if (!rc) rc = dev_alloc((void **)&ds, n * sizeof(float));
    if (!rc && hipMemcpy(dc, hc, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) rc = QWEN_HIP_EDEVICE;
    if (!rc && hipMemcpy(ds, hs, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) rc = QWEN_HIP_EDEVICE;
    free(hc);
    free(hs);
    if (rc) { dev_free(dc); dev_free(ds); if (rc == QWEN_HIP_EDEVICE) qk_set_err("RoPE table upload failed"); return rc; }
    dev_free(d->rope_cos);
    dev_free(d->rope_sin);
    d->rope_cos = dc;
    d->rope_sin = ds;
    return 0;
}

/* kv_cache_grow (qwen_asr_decoder.c:133-160): double until >= required and
 * copy the live positions [0, kv_len) of every (layer, kv head). */
static int kv_reserve(qwen_hip_decoder *d, int required) {
    if (required <= d->kv_cap) return 0;
    int cap = d->kv_cap > 0 ? d->kv_cap : required;
    while (cap < required) {
        if (cap > (1 << 29)) { qk_set_err("KV capacity overflow"); return QWEN_HIP_EINVAL; }
        cap *= 2;
    }
    const int hd = d->cfg.head_dim;
    const size_t rows = (size_t)d->cfg.layers * d->cfg.kv_heads;
    const size_t bytes = rows * (size_t)cap * hd * sizeof(float);
    float *nk = NULL, *nv = NULL;
    int rc = dev_alloc((void **)&nk, bytes);
    if (!rc) rc = dev_alloc((void **)&nv, bytes);
    if (rc) { dev_free(nk); dev_free(nv); return rc; }
    QK_HIP(hipMemsetAsync(nk, 0, bytes, d->stream));
    QK_HIP(hipMemsetAsync(nv, 0, bytes, d->stream));
    if (d->kc && d->kv_len > 0) {
        const size_t w = (size_t)d->kv_len * hd * sizeof(float);
        const size_t sp = (size_t)d->kv_cap * hd * sizeof(float), dp = (size_t)cap * hd * sizeof(float);
        QK_HIP(hipMemcpy2DAsync(nk, dp, d->kc, sp, w, rows, hipMemcpyDeviceToDevice, d->stream));
        QK_HIP(hipMemcpy2DAsync(nv, dp, d->vc, sp, w, rows, hipMemcpyDeviceToDevice, d->stream));
    }
    QK_HIP(hipStreamSynchronize(d->stream));
    if ((rc = rope_build(d, cap))) { dev_free(nk); dev_free(nv); return rc; }
    dev_free(d->kc);
    dev_free(d->vc);
    d->kc = nk;
    d->vc = nv;
    d->kv_cap = cap;
    graph_drop(d);
    return 0;
}

static float *kc_layer(const qwen_hip_decoder *d, int l) {
    return d->kc + (size_t)l * d->cfg.kv_heads * d->kv_cap * d->cfg.head_dim;
}

static float *vc_layer(const qwen_hip_decoder *d, int l) {
    return d->vc + (size_t)l * d->cfg.kv_heads * d->kv_cap * d->cfg.head_dim;
}

static int set_dev_pos(qwen_hip_decoder *d) {
    d->h_int[1] = d->kv_len;
    QK_HIP(hipMemcpyAsync(d->d_pos, &d->h_int[1], sizeof(int), hipMemcpyHostToDevice, d->stream));
    QK_HIP(hipStreamSynchronize(d->stream));
    return 0;
}

static int check_cfg(const qwen_hip_config *c) {
    if (!c) return 0;
    if (c->head_dim != QWEN_HIP_HEAD_DIM) return 0;
    if (c->layers <= 0 || c->layers > QWEN_HIP_MAX_LAYERS) return 0;
    if (c->heads <= 0 || c->kv_heads <= 0 || c->heads % c->kv_heads) return 0;
    int hpk = c->heads / c->kv_heads;
    if (hpk != 1 && hpk != 2 && hpk != 4) return 0;
    if (c->hidden <= 0 || c->hidden % 64 || c->hidden > 6144) return 0;
    if (c->intermediate <= 0 || c->intermediate % 64 || c->intermediate > 6144) return 0;
    if (c->heads * c->head_dim > 6144) return 0;
    if (c->vocab <= 0) return 0;
    return 1;
}

/* Exchange words of the persistent engine, zero-initialised (tag 0 is never
 * expected: epochs start at 1). */
static int px_alloc(qwen_hip_decoder *d) {
    const size_t H = d->cfg.hidden, I = d->cfg.intermediate, P = 2 * QK_PX_XCD;
    const size_t n_q = P * 512, n_a = P * QK_PX_MAX_SPLIT * QK_PX_PART, n_h = P * H, n_i = P * (I / QK_PX_XCD);
    const size_t n_c = 2 * QK_PX_BLOCKS, n_v = QK_PX_BLOCKS, n_m = P * 256;
    d->px_words = n_q + n_a + n_m + 4 * n_h + n_i + n_c + n_v;
    QK_TRY(dev_alloc((void **)&d->px_buf, d->px_words * 8));
    QK_TRY(dev_alloc((void **)&d->px_ctl, 64 * sizeof(unsigned)));
    unsigned long long *p = d->px_buf;
    d->xq = p;  p += n_q;
    d->xa = p;  p += n_a;
    d->xm = p;  p += n_m;
    d->xo = p;  p += n_h;
    d->xla = p; p += n_h;
    d->xd = p;  p += n_h;
    d->xlb = p; p += n_h;
    d->xh = p;  p += n_i;
    d->xc = p;  p += n_c;
    d->xv = p;
    QK_HIP(hipMemset(d->px_buf, 0, d->px_words * 8));
    QK_HIP(hipMemset(d->px_ctl, 0, 64 * sizeof(unsigned)));
    d->px_epoch = 1;
    d->px_trace_step = -1;
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, d->device) != hipSuccess || khz <= 0)
        khz = 100000;                              /* the MI355X constant-rate clock: 100 MHz */
    d->px_ticks_per_s = (double)khz * 1e3;
    d->px_wait_ticks = (unsigned long long)d->px_ticks_per_s;   /* one second */
    d->px_fallback = 1;
    return 0;
}

/* The relay kernel's tiled weights and exchange words (zero-initialised). */
static int rl_alloc(qwen_hip_decoder *d) {
    const size_t T = 2 * QK_PX_XCD, H = d->cfg.hidden;
    const size_t n_q = T * 512, n_a = T * QK_RL_TEAM * QK_RL_PART, n_m = T * 256, n_h = T * H;
    const size_t n_i = T * (d->cfg.intermediate / QK_PX_XCD), n_c = (size_t)QK_PX_BLOCKS * QK_RL_LINE;
    d->rl_words = n_q + n_a + n_m + 5 * n_h + n_i + 2 * n_c;
    QK_TRY(dev_alloc((void **)&d->wt, (size_t)d->cfg.layers * QK_RL_LAYER_BYTES));
    QK_TRY(dev_alloc((void **)&d->rl_buf, d->rl_words * 8));
    unsigned long long *p = d->rl_buf;
    d->rq = p;  p += n_q;
    d->ra = p;  p += n_a;
    d->rm = p;  p += n_m;
    d->ro = p;  p += n_h;
    d->rla = p; p += n_h;
    d->rd = p;  p += n_h;
    d->rs = p;  p += n_h;
    d->rlb = p; p += n_h;
    d->rh = p;  p += n_i;
    d->rc = p;  p += n_c;
    d->rv = p;
    QK_HIP(hipMemset(d->rl_buf, 0, d->rl_words * 8));
    d->rl_ok = 1;
    d->rl_on = 1;
    return 0;
}

qwen_hip_decoder *qwen_hip_decoder_create(const qwen_hip_config *cfg, int device, int kv_capacity) {
    if (!check_cfg(cfg)) {
        qk_set_err("unsupported decoder configuration (head_dim must be 128; hidden, "
                   "intermediate multiples of 64 and <= 6144; heads/kv_heads in {1,2,4})");
        return NULL;
    }
    if (hipSetDevice(device) != hipSuccess) { qk_set_err("hipSetDevice(%d) failed", device); return NULL; }
    qwen_hip_decoder *d = (qwen_hip_decoder *)calloc(1, sizeof(*d));
    if (!d) { qk_set_err("host alloc"); return NULL; }
    d->cfg = *cfg;
    d->device = device;
    d->qd = cfg->heads * cfg->head_dim;
    d->kvd = cfg->kv_heads * cfg->head_dim;
    d->qkv_rows = d->qd + 2 * d->kvd;
    d->scale = 1.0f / sqrtf((float)cfg->head_dim);   /* qwen_asr_decoder.c:426 */
    if (hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking) != hipSuccess) {
        qk_set_err("hipStreamCreate failed");
        free(d);
        return NULL;
    }

    const size_t D = cfg->hidden, I = cfg->intermediate, L = cfg->layers;
    size_t per_layer = align256((size_t)d->qkv_rows * D * 2) + align256((size_t)D * d->qd * 2) +
                       align256(2 * I * D * 2) + align256(D * I * 2) + 2 * align256(D * 4) +
                       2 * align256((size_t)cfg->head_dim * 4);
    size_t total = L * per_layer + align256((size_t)cfg->vocab * D * 2) + align256(D * 4);
    if (dev_alloc(&d->wbuf, total)) goto fail;
    {
        char *p = (char *)d->wbuf;
        for (size_t l = 0; l < L; l++) {
            d->w_qkv[l] = (uint16_t *)p; p += align256((size_t)d->qkv_rows * D * 2);
            d->w_o[l] = (uint16_t *)p;   p += align256(D * d->qd * 2);
            d->w_gu[l] = (uint16_t *)p;  p += align256(2 * I * D * 2);
            d->w_down[l] = (uint16_t *)p; p += align256(D * I * 2);
            d->n_in[l] = (float *)p;     p += align256(D * 4);
            d->n_post[l] = (float *)p;   p += align256(D * 4);
            d->n_q[l] = (float *)p;      p += align256((size_t)cfg->head_dim * 4);
            d->n_k[l] = (float *)p;      p += align256((size_t)cfg->head_dim * 4);
        }
        d->emb = (uint16_t *)p; p += align256((size_t)cfg->vocab * D * 2);
        d->fnorm = (float *)p;
    }

    d->n_cand = qk_gemv_blocks(cfg->vocab, cfg->hidden, QK_EPI_ARGMAX);
    d->log_cap = 4096;
    if (dev_alloc((void **)&d->x, D * 4) || dev_alloc((void **)&d->qkv, (size_t)d->qkv_rows * 4) ||
        dev_alloc((void **)&d->part_o, (size_t)cfg->heads * QK_ATTN_MAX_SPLIT * cfg->head_dim * 4) ||
        dev_alloc((void **)&d->part_m, (size_t)cfg->heads * QK_ATTN_MAX_SPLIT * 4) ||
        dev_alloc((void **)&d->part_l, (size_t)cfg->heads * QK_ATTN_MAX_SPLIT * 4) ||
        dev_alloc((void **)&d->attn_out, (size_t)d->qd * 4) || dev_alloc((void **)&d->h, I * 4) ||
        dev_alloc((void **)&d->hidden, D * 4) || dev_alloc((void **)&d->logits, (size_t)cfg->vocab * 4) ||
        dev_alloc((void **)&d->cand_val, (size_t)d->n_cand * 4) ||
        dev_alloc((void **)&d->cand_idx, (size_t)d->n_cand * 4) ||
        dev_alloc((void **)&d->ctl, CTL_INTS * 4) || dev_alloc((void **)&d->d_log, (size_t)d->log_cap * 4))
        goto fail;
    d->d_tok = d->ctl + CTL_TOK;
    d->d_pos = d->ctl + CTL_POS;
    d->d_counter = d->ctl + CTL_COUNTER;
    if (hipHostMalloc((void **)&d->h_row, D * 4, hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc((void **)&d->h_int, 256, hipHostMallocDefault) != hipSuccess) {
        qk_set_err("hipHostMalloc failed");
        goto fail;
    }
    {
        int init[CTL_INTS] = {0};
        if (hipMemset(d->hidden, 0, D * 4) != hipSuccess ||
            hipMemset(d->part_o, 0, (size_t)cfg->heads * QK_ATTN_MAX_SPLIT * cfg->head_dim * 4) != hipSuccess ||
            hipMemset(d->part_l, 0, (size_t)cfg->heads * QK_ATTN_MAX_SPLIT * 4) != hipSuccess ||
            hipMemcpy(d->ctl, init, sizeof init, hipMemcpyHostToDevice) != hipSuccess) {
            qk_set_err("control block init failed");
            goto fail;
        }
    }
    if (kv_reserve(d, kv_capacity > 0 ? kv_capacity : 1024)) goto fail;
    d->engine = ENGINE_GRAPH;
    if (qk_persist_supported(cfg->hidden, cfg->intermediate, cfg->heads, cfg->kv_heads, device)) {
        if (px_alloc(d)) goto fail;
        d->px_ok = 1;
        d->engine = ENGINE_PERSIST;
        if (qk_relay_supported(cfg->hidden, cfg->intermediate, cfg->heads, cfg->kv_heads, device) && rl_alloc(d))
            goto fail;
    }
    return d;
fail:
    qwen_hip_decoder_destroy(d);
    return NULL;
}

static void prefill_free(qwen_hip_decoder *d) {
    dev_free(d->px); dev_free(d->pqkv); dev_free(d->pqrot);
    dev_free(d->pxh); dev_free(d->pxl); dev_free(d->pah); dev_free(d->pal);
    dev_free(d->phh); dev_free(d->phl);
    d->px = d->pqkv = d->pqrot = NULL;
    d->pxh = d->pxl = d->pah = d->pal = d->phh = d->phl = NULL;
    d->pref_cap = 0;
    dev_free(d->pattn);
    d->pattn = NULL;
    d->pattn_floats = 0;
    dev_free(d->pgemm);
    d->pgemm = NULL;
    d->pgemm_floats = 0;
}

void qwen_hip_decoder_destroy(qwen_hip_decoder *d) {
    if (!d) return;
    (void)hipSetDevice(d->device);
    if (d->stream) (void)hipStreamSynchronize(d->stream);
    graph_drop(d);
    dev_free(d->wbuf);
    dev_free(d->kc); dev_free(d->vc); dev_free(d->rope_cos); dev_free(d->rope_sin);
    dev_free(d->x); dev_free(d->qkv); dev_free(d->part_o); dev_free(d->part_m); dev_free(d->part_l);
    dev_free(d->attn_out); dev_free(d->h); dev_free(d->hidden); dev_free(d->logits);
    dev_free(d->cand_val); dev_free(d->cand_idx); dev_free(d->ctl); dev_free(d->d_log);
    dev_free(d->px_buf); dev_free(d->px_ctl); dev_free(d->px_trace);
    dev_free(d->wt); dev_free(d->rl_buf);
    prefill_free(d);
    if (d->h_row) (void)hipHostFree(d->h_row);
    if (d->h_int) (void)hipHostFree(d->h_int);
    if (d->stream) (void)hipStreamDestroy(d->stream);
    free(d);
}

/* ------------------------------------------------------------------------ */
/* weights                                                                   */
/* ------------------------------------------------------------------------ */
int qwen_hip_decoder_load_layer(qwen_hip_decoder *d, int l, const qwen_hip_layer_weights *w) {
    if (!d || !w || l < 0 || l >= d->cfg.layers) { qk_set_err("load_layer: bad argument"); return QWEN_HIP_EINVAL; }
    if (!w->wq || !w->wk || !w->wv || !w->wo || !w->gate || !w->up || !w->down || !w->q_norm ||
        !w->k_norm || !w->input_norm || !w->post_attn_norm) {
        qk_set_err("load_layer %d: missing tensor", l);
        return QWEN_HIP_EINVAL;
    }
    QK_TRY(use_device(d));
    const size_t D = d->cfg.hidden, I = d->cfg.intermediate, hd = d->cfg.head_dim;
    QK_HIP(hipMemcpy(d->w_qkv[l], w->wq, (size_t)d->qd * D * 2, hipMemcpyHostToDevice));
    QK_HIP(hipMemcpy(d->w_qkv[l] + (size_t)d->qd * D, w->wk, (size_t)d->kvd * D * 2, hipMemcpyHostToDevice));
    QK_HIP(hipMemcpy(d->w_qkv[l] + (size_t)(d->qd + d->kvd) * D, w->wv, (size_t)d->kvd * D * 2,
                     hipMemcpyHostToDevice));
    QK_HIP(hipMemcpy(d->w_o[l], w->wo, D * d->qd * 2, hipMemcpyHostToDevice));
    /* interleave gate/up rows: row 2r = gate[r], row 2r+1 = up[r] */
    QK_HIP(hipMemcpy2D(d->w_gu[l], 2 * D * 2, w->gate, D * 2, D * 2, I, hipMemcpyHostToDevice));
    QK_HIP(hipMemcpy2D(d->w_gu[l] + D, 2 * D * 2, w->up, D * 2, D * 2, I, hipMemcpyHostToDevice));
    QK_HIP(hipMemcpy(d->w_down[l], w->down, D * I * 2, hipMemcpyHostToDevice));
    QK_HIP(hipMemcpy(d->n_in[l], w->input_norm, D * 4, hipMemcpyHostToDevice));
    QK_HIP(hipMemcpy(d->n_post[l], w->post_attn_norm, D * 4, hipMemcpyHostToDevice));
    QK_HIP(hipMemcpy(d->n_q[l], w->q_norm, hd * 4, hipMemcpyHostToDevice));
    QK_HIP(hipMemcpy(d->n_k[l], w->k_norm, hd * 4, hipMemcpyHostToDevice));
    if (d->rl_ok) {   /* the relay kernel's tiled copy of the four matrices */
        QK_TRY(qk_relay_pack(d->wt + (size_t)l * QK_RL_LAYER_BYTES, d->w_qkv[l], d->w_o[l], d->w_gu[l], d->w_down[l],
                             d->stream));
        QK_HIP(hipStreamSynchronize(d->stream));
    }
    d->loaded[l] = 1;
    return 0;
}

int qwen_hip_decoder_load_embeddings(qwen_hip_decoder *d, const uint16_t *emb, const float *fnorm) {
    if (!d || !emb || !fnorm) { qk_set_err("load_embeddings: bad argument"); return QWEN_HIP_EINVAL; }
    QK_TRY(use_device(d));
    QK_HIP(hipMemcpy(d->emb, emb, (size_t)d->cfg.vocab * d->cfg.hidden * 2, hipMemcpyHostToDevice));
    QK_HIP(hipMemcpy(d->fnorm, fnorm, (size_t)d->cfg.hidden * 4, hipMemcpyHostToDevice));
    d->emb_loaded = 1;
    return 0;
}

static void norm_vec(float *out, size_t n, uint64_t seed, uint64_t tid, double norm_std) {
    if (norm_std == 0.0) {
        for (size_t i = 0; i < n; i++) out[i] = 1.0f;
    } else {
        qwen_synth_normal_f32(out, n, seed, tid, 1.0, norm_std, 0);
    }
}

int qwen_hip_decoder_load_synthetic(qwen_hip_decoder *d, uint64_t seed, double wstd, double norm_std) {
    if (!d) return QWEN_HIP_EINVAL;
    const qwen_hip_config *c = &d->cfg;
    const size_t D = c->hidden, I = c->intermediate, hd = c->head_dim;
    const size_t qd = d->qd, kvd = d->kvd;
    size_t big = (size_t)c->vocab * D;
    size_t need = qd * D + 2 * kvd * D + D * qd + 3 * I * D;
    uint16_t *buf = (uint16_t *)malloc((need > big ? need : big) * 2);
    float *nb = (float *)malloc((2 * D + 2 * hd) * 4);
    if (!buf || !nb) { free(buf); free(nb); qk_set_err("host alloc for synthetic weights"); return QWEN_HIP_ENOMEM; }
    int rc = 0;
    for (int l = 0; l < c->layers && !rc; l++) {
        qwen_hip_layer_weights w;
        uint16_t *p = buf;
        w.wq = p;   qwen_synth_normal_bf16(p, qd * D, seed, QWEN_SYNTH_LAYER(l, QWEN_SYNTH_WQ), 0, wstd, 0); p += qd * D;
        w.wk = p;   qwen_synth_normal_bf16(p, kvd * D, seed, QWEN_SYNTH_LAYER(l, QWEN_SYNTH_WK), 0, wstd, 0); p += kvd * D;
        w.wv = p;   qwen_synth_normal_bf16(p, kvd * D, seed, QWEN_SYNTH_LAYER(l, QWEN_SYNTH_WV), 0, wstd, 0); p += kvd * D;
        w.wo = p;   qwen_synth_normal_bf16(p, D * qd, seed, QWEN_SYNTH_LAYER(l, QWEN_SYNTH_WO), 0, wstd, 0); p += D * qd;
        w.gate = p; qwen_synth_normal_bf16(p, I * D, seed, QWEN_SYNTH_LAYER(l, QWEN_SYNTH_GATE), 0, wstd, 0); p += I * D;
        w.up = p;   qwen_synth_normal_bf16(p, I * D, seed, QWEN_SYNTH_LAYER(l, QWEN_SYNTH_UP), 0, wstd, 0); p += I * D;
        w.down = p; qwen_synth_normal_bf16(p, D * I, seed, QWEN_SYNTH_LAYER(l, QWEN_SYNTH_DOWN), 0, wstd, 0);
        float *n = nb;
        w.q_norm = n;         norm_vec(n, hd, seed, QWEN_SYNTH_LAYER(l, QWEN_SYNTH_QNORM), norm_std); n += hd;
        w.k_norm = n;         norm_vec(n, hd, seed, QWEN_SYNTH_LAYER(l, QWEN_SYNTH_KNORM), norm_std); n += hd;
        w.input_norm = n;     norm_vec(n, D, seed, QWEN_SYNTH_LAYER(l, QWEN_SYNTH_INNORM), norm_std); n += D;
        w.post_attn_norm = n; norm_vec(n, D, seed, QWEN_SYNTH_LAYER(l, QWEN_SYNTH_POSTNORM), norm_std);
        rc = qwen_hip_decoder_load_layer(d, l, &w);
    }
    if (!rc) {
        qwen_synth_normal_bf16(buf, big, seed, QWEN_SYNTH_EMBED, 0, wstd, 0);
        norm_vec(nb, D, seed, QWEN_SYNTH_FINAL_NORM, norm_std);
        rc = qwen_hip_decoder_load_embeddings(d, buf, nb);
    }
    free(buf);
    free(nb);
    return rc;
}

static int ready(qwen_hip_decoder *d) {
    if (!d) { qk_set_err("NULL decoder"); return QWEN_HIP_EINVAL; }
    if (!d->emb_loaded) { qk_set_err("embeddings not loaded"); return QWEN_HIP_ESTATE; }
    for (int l = 0; l < d->cfg.layers; l++)
        if (!d->loaded[l]) { qk_set_err("layer %d not loaded", l); return QWEN_HIP_ESTATE; }
    return use_device(d);
}

/* ------------------------------------------------------------------------ */
/* prefill: qwen_decoder_prefill, qwen_asr_decoder.c:262-359                */
/* ------------------------------------------------------------------------ */
static int prefill_reserve(qwen_hip_decoder *d, int S) {
    if (S <= d->pref_cap) return 0;
    int cap = d->pref_cap > 0 ? d->pref_cap : 64;       /* ensure_prefill_buffers :181-182 */
    while (cap < S) cap *= 2;
    prefill_free(d);
    const size_t D = d->cfg.hidden, I = d->cfg.intermediate;
    int rc = dev_alloc((void **)&d->px, (size_t)cap * D * 4);
    if (!rc) rc = dev_alloc((void **)&d->pqkv, (size_t)cap * d->qkv_rows * 4);
    if (!rc) rc = dev_alloc((void **)&d->pqrot, (size_t)cap * d->qd * 4);
    if (!rc) rc = dev_alloc((void **)&d->pxh, (size_t)cap * D * 2);
    if (!rc) rc = dev_alloc((void **)&d->pxl, (size_t)cap * D * 2);
    if (!rc) rc = dev_alloc((void **)&d->pah, (size_t)cap * d->qd * 2);
    if (!rc) rc = dev_alloc((void **)&d->pal, (size_t)cap * d->qd * 2);
    if (!rc) rc = dev_alloc((void **)&d->phh, (size_t)cap * I * 2);
    if (!rc) rc = dev_alloc((void **)&d->phl, (size_t)cap * I * 2);
    if (rc) { prefill_free(d); return rc; }
    d->pref_cap = cap;
    return 0;
}

static int prefill_layers(qwen_hip_decoder *d, int S) {
    const qwen_hip_config *c = &d->cfg;
    const int D = c->hidden, I = c->intermediate, hd = c->head_dim, start = d->kv_len;
    hipStream_t s = d->stream;
    int chunk = 0, nsplit = 0;
    const size_t pf = qk_attn_prefill_plan(S, start + S, start, c->heads, c->kv_heads, &chunk, &nsplit);
    /* GEMM tilings; with split-K the partials go to pgemm and their consumer
     * (RoPE/append, the next RMSNorm, the SwiGLU reduce) sums them in order */
    qk_gemm_plan gq, go, gg, gd;
    qk_gemm_plan_epi(S, d->qkv_rows, D, QK_GEMM_ROPE, &gq);
    const int rope_fused = qk_gemm_rope_fusable(&gq);   /* RoPE / append in the Q|K|V epilogue */
    qk_gemm_plan_for(S, D, d->qd, &go);
    qk_gemm_plan_epi(S, 2 * I, D, QK_GEMM_SWIGLU, &gg);
    qk_gemm_plan_for(S, D, I, &gd);
    size_t pg = 0;
    const size_t cand[4] = {gq.nsplit > 1 ? (size_t)gq.nsplit * S * d->qkv_rows : 0,
                            go.nsplit > 1 ? (size_t)go.nsplit * S * D : 0,
                            gg.nsplit > 1 ? (size_t)gg.nsplit * S * 2 * I : 0,
                            gd.nsplit > 1 ? (size_t)gd.nsplit * S * D : 0};
    for (int i = 0; i < 4; i++) pg = cand[i] > pg ? cand[i] : pg;
    if (pf > d->pattn_floats || pg > d->pgemm_floats) {
        QK_HIP(hipStreamSynchronize(s));          /* old buffers may still be in use */
        if (pf > d->pattn_floats) {
            dev_free(d->pattn);
            d->pattn = NULL;
            d->pattn_floats = 0;
            QK_TRY(dev_alloc((void **)&d->pattn, pf * sizeof(float)));
            d->pattn_floats = pf;
        }
        if (pg > d->pgemm_floats) {
            dev_free(d->pgemm);
            d->pgemm = NULL;
            d->pgemm_floats = 0;
            QK_TRY(dev_alloc((void **)&d->pgemm, pg * sizeof(float)));
            d->pgemm_floats = pg;
        }
    }
    float *const qkv = gq.nsplit > 1 ? d->pgemm : d->pqkv;
    int pending = 0;                 /* split-K partials of the last down projection not yet in px */
    for (int l = 0; l < c->layers; l++) {
        /* input RMSNorm (completing the previous layer's residual first) + Q|K|V */
        QK_TRY(qk_rmsnorm_split_launch(d->px, d->pgemm, pending, (long)S * D, d->n_in[l], S, D, c->rms_eps,
                                       d->pxh, d->pxl, s));
        qk_rope_append_args ra = {
            .qkv = qkv, .nsum = gq.nsplit, .pstride = (long)S * d->qkv_rows, .q_norm = d->n_q[l],
            .k_norm = d->n_k[l], .eps = c->rms_eps, .rope_cos = d->rope_cos, .rope_sin = d->rope_sin,
            .k_cache = kc_layer(d, l), .v_cache = vc_layer(d, l), .cap = d->kv_cap, .pos_dev = NULL,
            .start = start, .S = S, .heads = c->heads, .kv_heads = c->kv_heads, .q_out = d->pqrot};
        if (rope_fused) {
            QK_TRY(qk_gemm_rope_launch(d->pxh, d->pxl, d->w_qkv[l], S, D, &gq, &ra, s));
        } else {
            QK_TRY(qk_gemm_launch(d->pxh, d->pxl, d->w_qkv[l], S, d->qkv_rows, D, &gq, QK_GEMM_STORE, qkv, NULL,
                                  NULL, s));
            QK_TRY(qk_rope_append_launch(&ra, s));
        }
        qk_attn_args aa = {
            .q = d->pqrot, .k = kc_layer(d, l), .v = vc_layer(d, l), .pos_stride = hd,
            .head_stride = (long)d->kv_cap * hd, .pos_dev = NULL, .seq_k = start + S, .seq_q = S,
            .q_offset = start, .heads = c->heads, .kv_heads = c->kv_heads, .scale = d->scale,
            .part = d->pattn, .nsplit = nsplit, .chunk = chunk, .out = NULL, .out_hi = d->pah, .out_lo = d->pal};
        QK_TRY(qk_attn_prefill_launch(&aa, s));
        /* O projection + residual, post-attention RMSNorm */
        if (go.nsplit > 1) {
            QK_TRY(qk_gemm_launch(d->pah, d->pal, d->w_o[l], S, D, d->qd, &go, QK_GEMM_STORE, d->pgemm, NULL, NULL,
                                  s));
            QK_TRY(qk_rmsnorm_split_launch(d->px, d->pgemm, go.nsplit, (long)S * D, d->n_post[l], S, D, c->rms_eps,
                                           d->pxh, d->pxl, s));
        } else {
            QK_TRY(qk_gemm_launch(d->pah, d->pal, d->w_o[l], S, D, d->qd, &go, QK_GEMM_ADD, d->px, NULL, NULL, s));
            QK_TRY(qk_rmsnorm_split_launch(d->px, NULL, 0, 0, d->n_post[l], S, D, c->rms_eps, d->pxh, d->pxl, s));
        }
        /* gate|up + SwiGLU */
        if (gg.nsplit > 1) {
            QK_TRY(qk_gemm_launch(d->pxh, d->pxl, d->w_gu[l], S, 2 * I, D, &gg, QK_GEMM_STORE, d->pgemm, NULL, NULL,
                                  s));
            QK_TRY(qk_gemm_reduce_launch(d->pgemm, gg.nsplit, S, 2 * I, QK_GEMM_SWIGLU, NULL, d->phh, d->phl, s));
        } else {
            QK_TRY(qk_gemm_launch(d->pxh, d->pxl, d->w_gu[l], S, 2 * I, D, &gg, QK_GEMM_SWIGLU, NULL, d->phh, d->phl,
                                  s));
        }
        /* down projection + residual (split-K: completed by the next RMSNorm) */
        if (gd.nsplit > 1) {
            QK_TRY(qk_gemm_launch(d->phh, d->phl, d->w_down[l], S, D, I, &gd, QK_GEMM_STORE, d->pgemm, NULL, NULL,
                                  s));
            pending = gd.nsplit;
        } else {
            QK_TRY(qk_gemm_launch(d->phh, d->phl, d->w_down[l], S, D, I, &gd, QK_GEMM_ADD, d->px, NULL, NULL, s));
            pending = 0;
        }
    }
    if (pending) QK_TRY(qk_gemm_reduce_launch(d->pgemm, pending, S, D, QK_GEMM_ADD, d->px, NULL, NULL, s));
    return 0;
}

static int prefill_common(qwen_hip_decoder *d, const float *rows, int S, hipMemcpyKind kind) {
    int rc = ready(d);
    if (rc) return rc;
    if (S < 0 || (S > 0 && !rows)) { qk_set_err("prefill: bad rows"); return QWEN_HIP_EINVAL; }
    if (S == 0) return 0;
    if (d->kv_len + S > d->kv_cap) QK_TRY(kv_reserve(d, d->kv_len + S + 1024));   /* :278-279 */
    QK_TRY(prefill_reserve(d, S));
    QK_HIP(hipMemcpyAsync(d->px, rows, (size_t)S * d->cfg.hidden * 4, kind, d->stream));
    QK_TRY(prefill_layers(d, S));
    QK_HIP(hipStreamSynchronize(d->stream));
    d->kv_len += S;
    return set_dev_pos(d);
}

int qwen_hip_decoder_prefill(qwen_hip_decoder *d, const float *rows, int S) {
    return prefill_common(d, rows, S, hipMemcpyHostToDevice);
}

int qwen_hip_decoder_prefill_device(qwen_hip_decoder *d, const float *d_rows, int S) {
    return prefill_common(d, d_rows, S, hipMemcpyDeviceToDevice);
}

/* ------------------------------------------------------------------------ */
/* decode step: qwen_decoder_forward, qwen_asr_decoder.c:388-476            */
/* ------------------------------------------------------------------------ */
static int enqueue_step(qwen_hip_decoder *d, int variant) {
    const qwen_hip_config *c = &d->cfg;
    const int D = c->hidden, I = c->intermediate, L = c->layers;
    hipStream_t s = d->stream;
    for (int l = 0; l < L; l++) {
        /* input RMSNorm + Q|K|V; layer 0 also gathers the token embedding */
        qk_gemv_args g = {.W = d->w_qkv[l], .rows = d->qkv_rows, .K = D, .x = d->x, .norm_w = d->n_in[l],
                          .eps = c->rms_eps, .y = d->qkv, .epi = QK_EPI_STORE};
        if (l == 0) { g.tok = d->d_tok; g.emb = d->emb; g.x_store = d->x; }
        QK_TRY(qk_gemv_launch(&g, s));
        /* q/k norm + RoPE + K/V append + split attention (qwen_asr_decoder.c:439-455) */
        qk_attn_fused_args aa = {
            .qkv = d->qkv, .q_norm = d->n_q[l], .k_norm = d->n_k[l], .eps = c->rms_eps,
            .rope_cos = d->rope_cos, .rope_sin = d->rope_sin, .k_cache = kc_layer(d, l),
            .v_cache = vc_layer(d, l), .cap = d->kv_cap, .pos_dev = d->d_pos, .heads = c->heads,
            .kv_heads = c->kv_heads, .scale = d->scale, .part_o = d->part_o, .part_m = d->part_m,
            .part_l = d->part_l};
        /* O projection + residual (:457-458), merging the attention splits */
        qk_gemv_args go = {.W = d->w_o[l], .rows = D, .K = d->qd, .y = d->x, .epi = QK_EPI_ADD};
        if (variant == STEP_SHORT) {
            aa.nsplit = QK_MERGE_MAX_SPLIT;
            QK_TRY(qk_attn_fused_launch(&aa, s));
            go.merge_o = d->part_o; go.merge_m = d->part_m; go.merge_l = d->part_l;
            go.merge_nsplit = QK_MERGE_MAX_SPLIT;
        } else {
            aa.nsplit = QK_ATTN_MAX_SPLIT;
            aa.out = d->attn_out;
            QK_TRY(qk_attn_fused_launch(&aa, s));
            QK_TRY(qk_attn_merge_launch(&aa, s));
            go.x = d->attn_out;
        }
        QK_TRY(qk_gemv_launch(&go, s));
        /* post-attention RMSNorm + gate|up + SwiGLU (:460-466), down + residual (:467-468) */
        qk_gemv_args gu = {.W = d->w_gu[l], .rows = 2 * I, .K = D, .x = d->x, .norm_w = d->n_post[l],
                           .eps = c->rms_eps, .y = d->h, .epi = QK_EPI_SWIGLU};
        QK_TRY(qk_gemv_launch(&gu, s));
        qk_gemv_args gd = {.W = d->w_down[l], .rows = D, .K = I, .x = d->h, .y = d->x, .epi = QK_EPI_ADD};
        QK_TRY(qk_gemv_launch(&gd, s));
    }
    /* final RMSNorm (in place in the reference, :474) + tied LM head argmax */
    qk_gemv_args gl = {.W = d->emb, .rows = c->vocab, .K = D, .x = d->x, .norm_w = d->fnorm, .eps = c->rms_eps,
                       .normed_store = d->hidden, .logits = d->keep_logits ? d->logits : NULL,
                       .cand_val = d->cand_val, .cand_idx = d->cand_idx, .epi = QK_EPI_ARGMAX};
    QK_TRY(qk_gemv_launch(&gl, s));
    QK_TRY(qk_argmax_finish_launch(d->cand_val, d->cand_idx, d->n_cand, d->d_tok, d->d_log, d->d_counter,
                                   d->d_pos, NULL, s));
    return 0;
}

static int graph_ensure(qwen_hip_decoder *d, int v) {
    if (d->gexec[v]) return 0;
    QK_HIP(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(d, v);
    hipGraph_t g = NULL;
    hipError_t e = hipStreamEndCapture(d->stream, &g);
    if (rc) { if (g) (void)hipGraphDestroy(g); return rc; }
    if (e != hipSuccess) { qk_set_err("hipStreamEndCapture: %s", hipGetErrorString(e)); return QWEN_HIP_EDEVICE; }
    d->graph[v] = g;
    QK_HIP(hipGraphInstantiate(&d->gexec[v], g, NULL, NULL, 0));
    return 0;
}

/* n steps starting at position kv_len: step i attends over kv_len + i + 1 keys */
static int launch_steps(qwen_hip_decoder *d, int n) {
    for (int i = 0; i < n; i++) {
        const int v = (d->kv_len + i + 1 <= QK_SHORT_MAX) ? STEP_SHORT : STEP_LONG;
        if (d->engine == ENGINE_GRAPH) {
            QK_TRY(graph_ensure(d, v));
            QK_HIP(hipGraphLaunch(d->gexec[v], d->stream));
        } else {
            QK_TRY(enqueue_step(d, v));
        }
    }
    return 0;
}

static int log_reserve(qwen_hip_decoder *d, int n) {
    if (n <= d->log_cap) return 0;
    int cap = d->log_cap;
    while (cap < n) cap *= 2;
    int *p = NULL;
    QK_TRY(dev_alloc((void **)&p, (size_t)cap * 4));
    dev_free(d->d_log);
    d->d_log = p;
    d->log_cap = cap;
    graph_drop(d);
    return 0;
}

/* Bound of the launch check-in: QK_PX_CHECKIN_S, or the wait limit if that is
 * shorter.  The blocks of an idle device all start within microseconds; a grid
 * that is not fully resident by then shares the device with other work (its
 * missing blocks could wait behind it indefinitely), so the launch gives up
 * early instead of holding the CUs it has for the whole wait limit. */
#define QK_PX_CHECKIN_S 0.02
static unsigned long long checkin_ticks(const qwen_hip_decoder *d) {
    const unsigned long long c = (unsigned long long)(QK_PX_CHECKIN_S * d->px_ticks_per_s);
    return c < d->px_wait_ticks ? c : d->px_wait_ticks;
}

/* the relay kernel (rl_decode): two teams of CUs take the layers in turn */
static int rl_launch(qwen_hip_decoder *d, int first_tok, int n) {
    const qwen_hip_config *c = &d->cfg;
    const char *l0 = (const char *)d->n_in[0];
    qk_relay_args a = {
        .wt = d->wt, .layer0 = l0,
        .layer_stride = c->layers > 1 ? (long)((const char *)d->n_in[1] - l0) : 0,
        .off_nin = 0, .off_npost = (const char *)d->n_post[0] - l0, .off_nq = (const char *)d->n_q[0] - l0,
        .off_nk = (const char *)d->n_k[0] - l0, .emb = d->emb, .fnorm = d->fnorm, .k_cache = d->kc, .v_cache = d->vc,
        .cap = d->kv_cap, .rope_cos = d->rope_cos, .rope_sin = d->rope_sin, .layers = c->layers, .vocab = c->vocab,
        .eps = c->rms_eps, .scale = d->scale, .xq = d->rq, .xa = d->ra, .xm = d->rm, .xo = d->ro, .xla = d->rla,
        .xh = d->rh, .xd = d->rd, .xs = d->rs, .xlb = d->rlb, .xc = d->rc, .xv = d->rv, .cnt = d->px_ctl,
        .err = d->px_ctl + 16, .epoch = d->px_epoch, .wait_ticks = d->px_wait_ticks, .checkin_ticks = checkin_ticks(d),
        .pos0 = d->kv_len, .n_steps = n,
        .first_tok = first_tok, .x_in = d->x, .log = d->d_log, .tok_out = d->d_tok, .pos_out = d->d_pos,
        .hidden_out = d->hidden, .logits = d->keep_logits ? d->logits : NULL,
        .trace = d->px_trace_step >= 0 && d->px_trace_step < n ? d->px_trace : NULL, .trace_step = d->px_trace_step};
    return qk_relay_launch(&a, d->stream);
}

/* the split kernel (px_decode): every CU streams every layer's share */
static int sp_launch(qwen_hip_decoder *d, int first_tok, int n) {
    const qwen_hip_config *c = &d->cfg;
    const char *l0 = (const char *)d->w_qkv[0];
    qk_persist_args a = {
        .layer0 = l0, .layer_stride = c->layers > 1 ? (long)((const char *)d->w_qkv[1] - l0) : 0,
        .off_qkv = 0, .off_o = (const char *)d->w_o[0] - l0, .off_gu = (const char *)d->w_gu[0] - l0,
        .off_down = (const char *)d->w_down[0] - l0, .off_nin = (const char *)d->n_in[0] - l0,
        .off_npost = (const char *)d->n_post[0] - l0, .off_nq = (const char *)d->n_q[0] - l0,
        .off_nk = (const char *)d->n_k[0] - l0, .emb = d->emb, .fnorm = d->fnorm, .k_cache = d->kc,
        .v_cache = d->vc, .cap = d->kv_cap, .rope_cos = d->rope_cos, .rope_sin = d->rope_sin,
        .layers = c->layers, .vocab = c->vocab, .eps = c->rms_eps, .scale = d->scale,
        .xq = d->xq, .xa = d->xa, .xm = d->xm, .xo = d->xo, .xla = d->xla, .xh = d->xh, .xd = d->xd, .xlb = d->xlb,
        .xc = d->xc, .xv = d->xv, .cnt = d->px_ctl, .err = d->px_ctl + 16, .epoch = d->px_epoch,
        .wait_ticks = d->px_wait_ticks, .checkin_ticks = checkin_ticks(d),
        .pos0 = d->kv_len, .n_steps = n, .first_tok = first_tok, .x_in = d->x, .log = d->d_log,
        .tok_out = d->d_tok, .pos_out = d->d_pos, .hidden_out = d->hidden,
        .logits = d->keep_logits ? d->logits : NULL,
        .trace = d->px_trace_step >= 0 && d->px_trace_step < n ? d->px_trace : NULL, .trace_step = d->px_trace_step};
    return qk_persist_launch(&a, c->hidden, c->intermediate, d->stream);
}

/* The persistent engine: n steps from position kv_len in one persistent
 * launch of the relay kernel (where it is available, enabled and every
 * position stays below QK_RL_MAX_SEQ) or else the split kernel; the first
 * input is emb[first_tok] or, for first_tok < 0, the row staged in d->x.
 * Synchronises and checks the kernel's error bits. */
static int px_run(qwen_hip_decoder *d, int first_tok, int n) {
    const qwen_hip_config *c = &d->cfg;
    const int relay = d->rl_ok && d->rl_on && d->kv_len + n <= QK_RL_MAX_SEQ;
    const unsigned need = relay ? QK_RL_TAGS(c->layers, n) : QK_PX_TAGS(c->layers, n);
    if (d->px_epoch > 0xFFFFFF00u - need) {       /* tag space exhausted: start over on zeroed words */
        QK_HIP(hipMemsetAsync(d->px_buf, 0, d->px_words * 8, d->stream));
        if (d->rl_buf) QK_HIP(hipMemsetAsync(d->rl_buf, 0, d->rl_words * 8, d->stream));
        d->px_epoch = 1;
    }
    QK_HIP(hipMemsetAsync(d->px_ctl, 0, 64 * sizeof(unsigned), d->stream));
    QK_TRY(relay ? rl_launch(d, first_tok, n) : sp_launch(d, first_tok, n));
    d->last_kernel = relay ? QWEN_HIP_KERNEL_RELAY : QWEN_HIP_KERNEL_SPLIT;
    d->px_epoch += need;
    QK_HIP(hipMemcpyAsync(&d->h_int[16], d->px_ctl + 16, sizeof(int), hipMemcpyDeviceToHost, d->stream));
    QK_HIP(hipStreamSynchronize(d->stream));
    if (d->h_int[16]) {
        qk_set_err("persistent decode raised error bits 0x%x (%s)", (unsigned)d->h_int[16],
                   (d->h_int[16] & QK_PX_ERR_LAYOUT) ? "blocks not spread 32 per XCD" : "hand-over timed out");
        return QWEN_HIP_EDEVICE;
    }
    return 0;
}

/* Run n steps from position kv_len; first_tok as for px_run.  Tokens land in
 * d_log[0, n), the last one also in the control block.  Does not advance
 * kv_len.  If a persistent launch fails (a wait timed out, the grid was not
 * laid out one block per CU): with fallback on (the default) the decoder
 * switches to the graph engine, counts the fallback (qwen_hip_decoder_fallbacks)
 * and redoes the steps there (they rewrite the same K/V positions, so a
 * partial run leaves nothing behind); with fallback off the call fails with
 * QWEN_HIP_EDEVICE and the decoder state is as before the call. */
static int steps_run(qwen_hip_decoder *d, int first_tok, int n) {
    if (d->engine == ENGINE_PERSIST) {
        int rc = px_run(d, first_tok, n);
        if (rc == 0) return 0;
        char msg[512];
        snprintf(msg, sizeof msg, "%s", qwen_hip_last_error());
        QK_TRY(set_dev_pos(d));       /* the failed run may have advanced it */
        if (!d->px_fallback) {
            qk_set_err("%s", msg);
            return rc;
        }
        fprintf(stderr, "qwen_asr_hip: %s; using the graph engine\n", msg);
        d->px_fallbacks++;
        d->engine = ENGINE_GRAPH;
    }
    d->h_int[0] = first_tok;
    d->h_int[2] = 0;
    QK_HIP(hipMemcpyAsync(d->d_tok, &d->h_int[0], sizeof(int), hipMemcpyHostToDevice, d->stream));
    QK_HIP(hipMemcpyAsync(d->d_counter, &d->h_int[2], sizeof(int), hipMemcpyHostToDevice, d->stream));
    return launch_steps(d, n);
}

static int forward_prepare(qwen_hip_decoder *d, int steps) {
    int rc = ready(d);
    if (rc) return rc;
    if (d->kv_len + steps > d->kv_cap) QK_TRY(kv_reserve(d, d->kv_len + steps + 1024));   /* :416-418 */
    QK_TRY(log_reserve(d, steps));
    return 0;
}

/* one forward from the staged input (first_tok or the row in d->x) */
static int forward_one(qwen_hip_decoder *d, int first_tok) {
    if (steps_run(d, first_tok, 1)) return -1;
    if (hipMemcpyAsync(&d->h_int[8], d->ctl, 4 * sizeof(int), hipMemcpyDeviceToHost, d->stream) != hipSuccess ||
        hipStreamSynchronize(d->stream) != hipSuccess) {
        qk_set_err("forward: reading the token back failed");
        return -1;
    }
    d->kv_len += 1;
    return d->h_int[8 + CTL_TOK];
}

int qwen_hip_decoder_forward(qwen_hip_decoder *d, const float *row) {
    if (!row || forward_prepare(d, 1)) return QWEN_HIP_TOKEN_IM_END;
    memcpy(d->h_row, row, (size_t)d->cfg.hidden * 4);
    if (hipMemcpyAsync(d->x, d->h_row, (size_t)d->cfg.hidden * 4, hipMemcpyHostToDevice, d->stream) != hipSuccess) {
        qk_set_err("forward: staging copy failed");
        return QWEN_HIP_TOKEN_IM_END;
    }
    int t = forward_one(d, -1);
    return t < 0 ? QWEN_HIP_TOKEN_IM_END : t;
}

int qwen_hip_decoder_forward_token(qwen_hip_decoder *d, int token) {
    if (!d || token < 0 || token >= d->cfg.vocab) { qk_set_err("forward_token: bad token"); return QWEN_HIP_TOKEN_IM_END; }
    if (forward_prepare(d, 1)) return QWEN_HIP_TOKEN_IM_END;
    int t = forward_one(d, token);
    return t < 0 ? QWEN_HIP_TOKEN_IM_END : t;
}

int qwen_hip_decoder_generate(qwen_hip_decoder *d, int first, int n, int *out, int stop_on_eos) {
    if (!d || n < 0 || (n > 0 && !out) || first < 0 || first >= d->cfg.vocab) {
        qk_set_err("generate: bad argument");
        return QWEN_HIP_EINVAL;
    }
    if (n == 0) return 0;
    QK_TRY(forward_prepare(d, n));
    const int start = d->kv_len;
    int rc = steps_run(d, first, n);   /* keeps its own error message */
    if (rc) return rc;
    QK_HIP(hipMemcpyAsync(out, d->d_log, (size_t)n * 4, hipMemcpyDeviceToHost, d->stream));
    QK_HIP(hipStreamSynchronize(d->stream));
    int kept = n;
    if (stop_on_eos) {
        for (int i = 0; i < n; i++)
            if (out[i] == QWEN_HIP_TOKEN_ENDOFTEXT || out[i] == QWEN_HIP_TOKEN_IM_END) { kept = i + 1; break; }
    }
    d->kv_len = start + kept;
    QK_TRY(set_dev_pos(d));
    return kept;
}

int qwen_hip_decoder_kv_len(const qwen_hip_decoder *d) { return d ? d->kv_len : QWEN_HIP_EINVAL; }

const qwen_hip_config *qwen_hip_decoder_config(const qwen_hip_decoder *d) { return d ? &d->cfg : NULL; }

int qwen_hip_decoder_set_kv_len(qwen_hip_decoder *d, int n) {
    if (!d || n < 0 || n > d->kv_len) { qk_set_err("set_kv_len: %d outside [0, kv_len]", n); return QWEN_HIP_EINVAL; }
    QK_TRY(use_device(d));
    d->kv_len = n;
    return set_dev_pos(d);
}

int qwen_hip_decoder_set_keep_logits(qwen_hip_decoder *d, int on) {
    if (!d) return QWEN_HIP_EINVAL;
    if ((on != 0) != d->keep_logits) { d->keep_logits = on != 0; graph_drop(d); }
    return 0;
}

int qwen_hip_decoder_set_engine(qwen_hip_decoder *d, int engine) {
    if (!d || engine < ENGINE_GRAPH || engine > ENGINE_PERSIST) { qk_set_err("set_engine: unknown engine"); return QWEN_HIP_EINVAL; }
    if (engine == ENGINE_PERSIST && !d->px_ok) {
        qk_set_err("set_engine: the persistent engine needs 16 query / 8 kv heads, the 0.6B or 1.7B shape and 256 CUs");
        return QWEN_HIP_EINVAL;
    }
    d->engine = engine;
    return 0;
}

int qwen_hip_decoder_engine(const qwen_hip_decoder *d) { return d ? d->engine : QWEN_HIP_EINVAL; }

int qwen_hip_decoder_set_fallback(qwen_hip_decoder *d, int on) {
    if (!d) return QWEN_HIP_EINVAL;
    d->px_fallback = on != 0;
    return 0;
}

int qwen_hip_decoder_fallbacks(const qwen_hip_decoder *d) { return d ? d->px_fallbacks : QWEN_HIP_EINVAL; }

int qwen_hip_decoder_set_wait_limit(qwen_hip_decoder *d, double seconds) {
    if (!d || !(seconds >= 0.0) || seconds > 60.0) { qk_set_err("set_wait_limit: seconds outside [0, 60]"); return QWEN_HIP_EINVAL; }
    if (!d->px_ok) { qk_set_err("set_wait_limit: the persistent engine is not available"); return QWEN_HIP_ESTATE; }
    d->px_wait_ticks = (unsigned long long)(seconds * d->px_ticks_per_s);
    return 0;
}

int qwen_hip_decoder_set_tag_epoch(qwen_hip_decoder *d, unsigned epoch) {
    if (!d || epoch == 0u) { qk_set_err("set_tag_epoch: epoch must be at least 1"); return QWEN_HIP_EINVAL; }
    if (!d->px_ok) { qk_set_err("set_tag_epoch: the persistent engine is not available"); return QWEN_HIP_ESTATE; }
    QK_TRY(use_device(d));
    /* zeroed words carry tag 0, which no hand-over expects, so any epoch is safe after this */
    QK_HIP(hipMemsetAsync(d->px_buf, 0, d->px_words * 8, d->stream));
    if (d->rl_buf) QK_HIP(hipMemsetAsync(d->rl_buf, 0, d->rl_words * 8, d->stream));
    QK_HIP(hipStreamSynchronize(d->stream));
    d->px_epoch = epoch;
    return 0;
}

unsigned qwen_hip_decoder_tag_epoch(const qwen_hip_decoder *d) { return d ? d->px_epoch : 0u; }

int qwen_hip_decoder_set_trace(qwen_hip_decoder *d, int step) {
    if (!d) return QWEN_HIP_EINVAL;
    if (!d->px_ok) { qk_set_err("set_trace: the persistent engine is not available"); return QWEN_HIP_ESTATE; }
    QK_TRY(use_device(d));
    /* the relay kernel writes QK_RL_TRACE words per block into the same buffer;
     * cleared whenever tracing is (re)enabled, so a record holds one launch's stamps */
    if (step >= 0 && !d->px_trace) QK_TRY(dev_alloc((void **)&d->px_trace, (size_t)QK_PX_BLOCKS * QK_PX_TRACE * 8));
    if (step >= 0) QK_HIP(hipMemset(d->px_trace, 0, (size_t)QK_PX_BLOCKS * QK_PX_TRACE * 8));
    d->px_trace_step = step < 0 ? -1 : step;
    return 0;
}

int qwen_hip_decoder_read_trace(qwen_hip_decoder *d, uint64_t *out, size_t n) {
    const size_t need = (size_t)QK_PX_BLOCKS * QK_PX_TRACE;
    if (!d || !out || n < need) { qk_set_err("read_trace: need %zu words", need); return QWEN_HIP_EINVAL; }
    if (!d->px_trace) { qk_set_err("read_trace: tracing was never enabled"); return QWEN_HIP_ESTATE; }
    QK_TRY(use_device(d));
    if (d->last_kernel == QWEN_HIP_KERNEL_RELAY) {
        /* relay records are QK_RL_TRACE words per block */
        QK_HIP(hipMemcpy(out, d->px_trace, (size_t)QK_PX_BLOCKS * QK_RL_TRACE * 8, hipMemcpyDeviceToHost));
        return (int)QK_RL_TRACE;
    }
    QK_HIP(hipMemcpy(out, d->px_trace, need * 8, hipMemcpyDeviceToHost));
    return (int)QK_PX_TRACE;
}

int qwen_hip_decoder_set_relay(qwen_hip_decoder *d, int on) {
    if (!d) return QWEN_HIP_EINVAL;
    if (on && !d->rl_ok) {
        qk_set_err("set_relay: the relay kernel needs the 0.6B shape, the persistent engine and 256 CUs");
        return QWEN_HIP_EINVAL;
    }
    d->rl_on = on != 0;
    return 0;
}

int qwen_hip_decoder_last_kernel(const qwen_hip_decoder *d) { return d ? d->last_kernel : QWEN_HIP_EINVAL; }

int qwen_hip_decoder_read_hidden(qwen_hip_decoder *d, float *out) {
    if (!d || !out) return QWEN_HIP_EINVAL;
    QK_TRY(use_device(d));
    QK_HIP(hipMemcpyAsync(out, d->hidden, (size_t)d->cfg.hidden * 4, hipMemcpyDeviceToHost, d->stream));
    QK_HIP(hipStreamSynchronize(d->stream));
    return 0;
}

int qwen_hip_decoder_read_logits(qwen_hip_decoder *d, float *out) {
    if (!d || !out) return QWEN_HIP_EINVAL;
    if (!d->keep_logits) { qk_set_err("read_logits needs set_keep_logits(1) before the forward"); return QWEN_HIP_ESTATE; }
    QK_TRY(use_device(d));
    QK_HIP(hipMemcpyAsync(out, d->logits, (size_t)d->cfg.vocab * 4, hipMemcpyDeviceToHost, d->stream));
    QK_HIP(hipStreamSynchronize(d->stream));
    return 0;
}

hipStream_t qwen_hip_decoder_stream(const qwen_hip_decoder *d) { return d ? d->stream : NULL; }

double qwen_hip_decoder_step_bytes(const qwen_hip_decoder *d, int kv_len) {
    if (!d) return 0.0;
    const qwen_hip_config *c = &d->cfg;
    const double D = c->hidden, I = c->intermediate, L = c->layers;
    double w = L * 2.0 * (D * d->qkv_rows + (double)d->qd * D + 2.0 * I * D + I * D);
    double lm = 2.0 * c->vocab * D;
    double norms = 4.0 * (L * (2.0 * D + 2.0 * c->head_dim) + D);
    double kv_row = L * d->kvd * 4.0 * 2.0;         /* K and V, fp32, all layers */
    return w + lm + norms + kv_row * (kv_len + 1) + kv_row;
}
