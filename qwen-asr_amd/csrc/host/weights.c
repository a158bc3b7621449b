/*
 * weights.c - load the decoder of a Qwen3-ASR safetensors checkpoint into a
 * device decoder context (the reference's qwen_decoder_load,
 * qwen_asr_decoder.c:45-116, over its safetensors reader,
 * qwen_asr_safetensors.c:194-394, and the shape choice of detect_config,
 * qwen_asr.c:135-191).
 *
 * A checkpoint directory holds either model.safetensors or shards named
 * model-*.safetensors (all of them, in name order, as the reference scans
 * them).  Each file is mapped read-only; its header (little-endian u64
 * length + JSON object of name -> {dtype, shape, data_offsets}) is parsed into
 * a tensor table.  Matrices must be BF16 and are uploaded straight from the
 * mapping; norm vectors may be F32 or BF16 and are widened to fp32 (bf16 ->
 * fp32 is the exact bits << 16 widening).  The decoder shape is read from the
 * tensor shapes (hidden = embed_tokens columns, intermediate = gate_proj
 * rows, heads = q_proj rows / 128, ...); rms eps 1e-6 and rope theta 1e6 are
 * the reference's constants for both model sizes.
 */
#include "qwen_asr_hip.h"
#include "host_internal.h"

#include <dirent.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define ST_MAX_SHARDS 16
#define ST_NAME 256

typedef struct {
    char name[ST_NAME];
    int dtype;               /* QWEN_HIP_ST_* */
    int ndim;
    long long shape[8];
    size_t begin, end;       /* byte range inside the data section */
    int shard;
} st_tensor;

struct qwen_hip_checkpoint {
    int n_shards;
    void *map[ST_MAX_SHARDS];
    size_t map_size[ST_MAX_SHARDS];
    size_t data_off[ST_MAX_SHARDS];   /* 8 + header length */
    st_tensor *t;
    int n, cap;
};

/* ---- a small JSON scanner for the header ------------------------------- */
typedef struct { const char *p, *end; } js;

static void js_ws(js *j) {
    while (j->p < j->end && (*j->p == ' ' || *j->p == '\n' || *j->p == '\r' || *j->p == '\t')) j->p++;
}

static int js_expect(js *j, char c) {
    js_ws(j);
    if (j->p >= j->end || *j->p != c) return -1;
    j->p++;
    return 0;
}

static int js_peek(js *j, char c) {
    js_ws(j);
    return j->p < j->end && *j->p == c;
}

/* a JSON string into out; the escapes \" \\ \/ are decoded, any other escape is rejected */
static int js_string(js *j, char *out, size_t cap) {
    if (js_expect(j, '"')) return -1;
    size_t n = 0;
    while (j->p < j->end && *j->p != '"') {
        char c = *j->p++;
        if (c == '\\') {
            if (j->p >= j->end) return -1;
            c = *j->p++;
            if (c != '"' && c != '\\' && c != '/') return -1;
        }
        if (n + 1 >= cap) return -1;
        out[n++] = c;
    }
    if (j->p >= j->end) return -1;
    j->p++;
    out[n] = '\0';
    return 0;
}

static int js_int(js *j, long long *v) {
    js_ws(j);
    char *e = NULL;
    if (j->p >= j->end || (*j->p != '-' && (*j->p < '0' || *j->p > '9'))) return -1;
    *v = strtoll(j->p, &e, 10);
    if (!e || e > j->end || e == j->p) return -1;
    j->p = e;
    return 0;
}

/* skip any JSON value (objects/arrays by depth, strings with escapes) */
static int js_skip(js *j) {
    js_ws(j);
    if (j->p >= j->end) return -1;
    if (*j->p == '"') {
        char tmp[4096];
        return js_string(j, tmp, sizeof(tmp));
    }
    if (*j->p == '{' || *j->p == '[') {
        int depth = 0;
        while (j->p < j->end) {
            char c = *j->p;
            if (c == '"') { char tmp[4096]; if (js_string(j, tmp, sizeof(tmp))) return -1; continue; }
            j->p++;
            if (c == '{' || c == '[') depth++;
            else if (c == '}' || c == ']') { if (--depth == 0) return 0; }
        }
        return -1;
    }
    while (j->p < j->end && *j->p != ',' && *j->p != '}' && *j->p != ']') j->p++;
    return 0;
}

static int dtype_of(const char *s) {
    if (!strcmp(s, "BF16")) return QWEN_HIP_ST_BF16;
    if (!strcmp(s, "F32")) return QWEN_HIP_ST_F32;
    if (!strcmp(s, "F16")) return QWEN_HIP_ST_F16;
    return QWEN_HIP_ST_OTHER;
}

static int dtype_size(int d) { return d == QWEN_HIP_ST_F32 ? 4 : d == QWEN_HIP_ST_OTHER ? 0 : 2; }

static int add_tensor(qwen_hip_checkpoint *ck, const st_tensor *t) {
    if (ck->n == ck->cap) {
        int cap = ck->cap ? 2 * ck->cap : 512;
        st_tensor *nt = (st_tensor *)realloc(ck->t, (size_t)cap * sizeof(st_tensor));
        if (!nt) return QWEN_HIP_ENOMEM;
        ck->t = nt;
        ck->cap = cap;
    }
    ck->t[ck->n++] = *t;
    return 0;
}

/* one entry: {"dtype": "...", "shape": [...], "data_offsets": [b, e]} */
static int parse_entry(js *j, st_tensor *t) {
    if (js_expect(j, '{')) return -1;
    int have = 0;
    while (!js_peek(j, '}')) {
        char key[64];
        if (js_string(j, key, sizeof(key)) || js_expect(j, ':')) return -1;
        if (!strcmp(key, "dtype")) {
            char d[32];
            if (js_string(j, d, sizeof(d))) return -1;
            t->dtype = dtype_of(d);
            have |= 1;
        } else if (!strcmp(key, "shape")) {
            if (js_expect(j, '[')) return -1;
            t->ndim = 0;
            while (!js_peek(j, ']')) {
                long long v;
                if (t->ndim >= 8 || js_int(j, &v) || v < 0) return -1;
                t->shape[t->ndim++] = v;
                if (js_peek(j, ',')) j->p++;
            }
            j->p++;
            have |= 2;
        } else if (!strcmp(key, "data_offsets")) {
            long long b, e;
            if (js_expect(j, '[') || js_int(j, &b) || js_expect(j, ',') || js_int(j, &e) || js_expect(j, ']'))
                return -1;
            if (b < 0 || e < b) return -1;
            t->begin = (size_t)b;
            t->end = (size_t)e;
            have |= 4;
        } else if (js_skip(j)) {
            return -1;
        }
        if (js_peek(j, ',')) j->p++;
    }
    j->p++;
    return have == 7 ? 0 : -1;
}

static int open_shard(qwen_hip_checkpoint *ck, const char *path) {
    if (ck->n_shards >= ST_MAX_SHARDS) { qk_set_err("checkpoint: more than %d shards", ST_MAX_SHARDS); return QWEN_HIP_EINVAL; }
    const int fd = open(path, O_RDONLY);
    if (fd < 0) { qk_set_err("checkpoint: cannot open %s", path); return QWEN_HIP_EINVAL; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 8) { close(fd); qk_set_err("checkpoint: %s is not a safetensors file", path); return QWEN_HIP_EINVAL; }
    const size_t size = (size_t)st.st_size;
    void *m = mmap(NULL, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) { qk_set_err("checkpoint: mmap %s failed", path); return QWEN_HIP_ENOMEM; }
    const int s = ck->n_shards++;
    ck->map[s] = m;
    ck->map_size[s] = size;
    unsigned long long hlen = 0;
    memcpy(&hlen, m, 8);                       /* little-endian on every host this builds for */
    if (hlen > size - 8) { qk_set_err("checkpoint: %s header length %llu past the file end", path, hlen); return QWEN_HIP_EINVAL; }
    ck->data_off[s] = 8 + (size_t)hlen;
    js j = {(const char *)m + 8, (const char *)m + 8 + hlen};
    if (js_expect(&j, '{')) { qk_set_err("checkpoint: %s header is not a JSON object", path); return QWEN_HIP_EINVAL; }
    while (!js_peek(&j, '}')) {
        st_tensor t;
        memset(&t, 0, sizeof(t));
        if (js_string(&j, t.name, sizeof(t.name)) || js_expect(&j, ':')) goto bad;
        if (!strcmp(t.name, "__metadata__")) {
            if (js_skip(&j)) goto bad;
        } else {
            if (parse_entry(&j, &t)) goto bad;
            long long numel = 1;
            for (int i = 0; i < t.ndim; i++) numel *= t.shape[i];
            const size_t data = size - ck->data_off[s];
            if (t.end > data || (dtype_size(t.dtype) && (size_t)numel * dtype_size(t.dtype) != t.end - t.begin)) {
                qk_set_err("checkpoint: %s: tensor %s has a bad byte range", path, t.name);
                return QWEN_HIP_EINVAL;
            }
            t.shard = s;
            QK_TRY(add_tensor(ck, &t));
        }
        if (js_peek(&j, ',')) j.p++;
    }
    return 0;
bad:
    qk_set_err("checkpoint: %s: malformed header", path);
    return QWEN_HIP_EINVAL;
}

static int name_cmp(const void *a, const void *b) { return strcmp((const char *)a, (const char *)b); }

qwen_hip_checkpoint *qwen_hip_checkpoint_open(const char *model_dir) {
    if (!model_dir) { qk_set_err("checkpoint: NULL directory"); return NULL; }
    qwen_hip_checkpoint *ck = (qwen_hip_checkpoint *)calloc(1, sizeof(*ck));
    if (!ck) { qk_set_err("checkpoint: out of host memory"); return NULL; }
    char path[4096];
    snprintf(path, sizeof(path), "%s/model.safetensors", model_dir);
    if (access(path, R_OK) == 0) {
        if (open_shard(ck, path)) goto fail;
        return ck;
    }
    DIR *dir = opendir(model_dir);
    if (!dir) { qk_set_err("checkpoint: cannot read directory %s", model_dir); goto fail; }
    char names[ST_MAX_SHARDS][ST_NAME];
    int n = 0;
    struct dirent *e;
    while ((e = readdir(dir)) != NULL) {
        const size_t len = strlen(e->d_name);
        if (len < 18 || strncmp(e->d_name, "model-", 6) || strcmp(e->d_name + len - 12, ".safetensors")) continue;
        if (n == ST_MAX_SHARDS || len >= ST_NAME) { closedir(dir); qk_set_err("checkpoint: too many shards in %s", model_dir); goto fail; }
        memcpy(names[n++], e->d_name, len + 1);
    }
    closedir(dir);
    if (n == 0) { qk_set_err("checkpoint: no model.safetensors or model-*.safetensors in %s", model_dir); goto fail; }
    qsort(names, n, ST_NAME, name_cmp);
    for (int i = 0; i < n; i++) {
        const int w = snprintf(path, sizeof(path), "%s/%s", model_dir, names[i]);
        if (w < 0 || (size_t)w >= sizeof(path)) { qk_set_err("checkpoint: path too long in %s", model_dir); goto fail; }
        if (open_shard(ck, path)) goto fail;
    }
    return ck;
fail:
    qwen_hip_checkpoint_close(ck);
    return NULL;
}

void qwen_hip_checkpoint_close(qwen_hip_checkpoint *ck) {
    if (!ck) return;
    for (int s = 0; s < ck->n_shards; s++) munmap(ck->map[s], ck->map_size[s]);
    free(ck->t);
    free(ck);
}

int qwen_hip_checkpoint_count(const qwen_hip_checkpoint *ck) { return ck ? ck->n : QWEN_HIP_EINVAL; }

static const st_tensor *find(const qwen_hip_checkpoint *ck, const char *name) {
    for (int i = 0; i < ck->n; i++)
        if (!strcmp(ck->t[i].name, name)) return &ck->t[i];
    return NULL;
}

int qwen_hip_checkpoint_tensor(const qwen_hip_checkpoint *ck, const char *name, int *dtype, int *ndim,
                               long long *shape, const void **data) {
    if (!ck || !name) return QWEN_HIP_EINVAL;
    const st_tensor *t = find(ck, name);
    if (!t) return QWEN_HIP_EINVAL;
    if (dtype) *dtype = t->dtype;
    if (ndim) *ndim = t->ndim;
    if (shape) for (int i = 0; i < t->ndim; i++) shape[i] = t->shape[i];
    if (data) *data = (const char *)ck->map[t->shard] + ck->data_off[t->shard] + t->begin;
    return 0;
}

/* matrix of exactly rows x cols in BF16 */
static const uint16_t *mat(const qwen_hip_checkpoint *ck, const char *name, long long rows, long long cols) {
    const st_tensor *t = find(ck, name);
    if (!t) { qk_set_err("checkpoint: missing %s", name); return NULL; }
    if (t->dtype != QWEN_HIP_ST_BF16 || t->ndim != 2 || t->shape[0] != rows || t->shape[1] != cols) {
        qk_set_err("checkpoint: %s must be BF16 [%lld][%lld]", name, rows, cols);
        return NULL;
    }
    return (const uint16_t *)((const char *)ck->map[t->shard] + ck->data_off[t->shard] + t->begin);
}

/* vector of n, F32 or BF16, widened into out */
static int vec(const qwen_hip_checkpoint *ck, const char *name, long long n, float *out) {
    const st_tensor *t = find(ck, name);
    if (!t) { qk_set_err("checkpoint: missing %s", name); return QWEN_HIP_EINVAL; }
    if (t->ndim != 1 || t->shape[0] != n || (t->dtype != QWEN_HIP_ST_F32 && t->dtype != QWEN_HIP_ST_BF16)) {
        qk_set_err("checkpoint: %s must be F32 or BF16 [%lld]", name, n);
        return QWEN_HIP_EINVAL;
    }
    const char *p = (const char *)ck->map[t->shard] + ck->data_off[t->shard] + t->begin;
    if (t->dtype == QWEN_HIP_ST_F32) {
        memcpy(out, p, (size_t)n * 4);
    } else {
        for (long long i = 0; i < n; i++) {
            uint16_t b;
            memcpy(&b, p + 2 * i, 2);
            const uint32_t u = (uint32_t)b << 16;
            memcpy(&out[i], &u, 4);
        }
    }
    return 0;
}

#define LNAME(buf, l, what) snprintf(buf, sizeof(buf), "thinker.model.layers.%d.%s", l, what)

int qwen_hip_checkpoint_config(const qwen_hip_checkpoint *ck, qwen_hip_config *cfg) {
    if (!ck || !cfg) return QWEN_HIP_EINVAL;
    const st_tensor *e = find(ck, "thinker.model.embed_tokens.weight");
    if (!e || e->ndim != 2) { qk_set_err("checkpoint: missing thinker.model.embed_tokens.weight"); return QWEN_HIP_EINVAL; }
    char n[ST_NAME];
    LNAME(n, 0, "self_attn.q_proj.weight");
    const st_tensor *q = find(ck, n);
    LNAME(n, 0, "self_attn.k_proj.weight");
    const st_tensor *k = find(ck, n);
    LNAME(n, 0, "mlp.gate_proj.weight");
    const st_tensor *g = find(ck, n);
    if (!q || !k || !g || q->ndim != 2 || k->ndim != 2 || g->ndim != 2) {
        qk_set_err("checkpoint: layer 0 projections missing");
        return QWEN_HIP_EINVAL;
    }
    int layers = 0;
    while (layers < QWEN_HIP_MAX_LAYERS) {
        LNAME(n, layers, "self_attn.q_proj.weight");
        if (!find(ck, n)) break;
        layers++;
    }
    memset(cfg, 0, sizeof(*cfg));
    cfg->hidden = (int)e->shape[1];
    cfg->vocab = (int)e->shape[0];
    cfg->head_dim = QWEN_HIP_HEAD_DIM;
    cfg->heads = (int)(q->shape[0] / QWEN_HIP_HEAD_DIM);
    cfg->kv_heads = (int)(k->shape[0] / QWEN_HIP_HEAD_DIM);
    cfg->intermediate = (int)g->shape[0];
    cfg->layers = layers;
    cfg->rms_eps = 1e-6f;
    cfg->rope_theta = 1e6f;
    if (q->shape[0] % QWEN_HIP_HEAD_DIM || k->shape[0] % QWEN_HIP_HEAD_DIM || cfg->heads <= 0 || cfg->kv_heads <= 0) {
        qk_set_err("checkpoint: projection rows are not a multiple of head_dim %d", QWEN_HIP_HEAD_DIM);
        return QWEN_HIP_EINVAL;
    }
    return 0;
}

int qwen_hip_decoder_load_checkpoint(qwen_hip_decoder *d, const qwen_hip_checkpoint *ck) {
    if (!d || !ck) return QWEN_HIP_EINVAL;
    qwen_hip_config c;
    QK_TRY(qwen_hip_checkpoint_config(ck, &c));
    const qwen_hip_config *dc = qwen_hip_decoder_config(d);
    if (!dc || c.hidden != dc->hidden || c.layers != dc->layers || c.heads != dc->heads ||
        c.kv_heads != dc->kv_heads || c.intermediate != dc->intermediate || c.vocab != dc->vocab) {
        qk_set_err("checkpoint: shape differs from the decoder's configuration");
        return QWEN_HIP_EINVAL;
    }
    const long long D = c.hidden, I = c.intermediate, hd = c.head_dim;
    const long long qd = (long long)c.heads * hd, kvd = (long long)c.kv_heads * hd;
    float *nb = (float *)malloc((size_t)(2 * D + 2 * hd) * sizeof(float));
    if (!nb) { qk_set_err("checkpoint: out of host memory"); return QWEN_HIP_ENOMEM; }
    int rc = 0;
    char n[ST_NAME];
    for (int l = 0; l < c.layers && !rc; l++) {
        qwen_hip_layer_weights w;
        memset(&w, 0, sizeof(w));
        LNAME(n, l, "self_attn.q_proj.weight");   w.wq = mat(ck, n, qd, D);
        LNAME(n, l, "self_attn.k_proj.weight");   w.wk = mat(ck, n, kvd, D);
        LNAME(n, l, "self_attn.v_proj.weight");   w.wv = mat(ck, n, kvd, D);
        LNAME(n, l, "self_attn.o_proj.weight");   w.wo = mat(ck, n, D, qd);
        LNAME(n, l, "mlp.gate_proj.weight");      w.gate = mat(ck, n, I, D);
        LNAME(n, l, "mlp.up_proj.weight");        w.up = mat(ck, n, I, D);
        LNAME(n, l, "mlp.down_proj.weight");      w.down = mat(ck, n, D, I);
        if (!w.wq || !w.wk || !w.wv || !w.wo || !w.gate || !w.up || !w.down) { rc = QWEN_HIP_EINVAL; break; }
        float *qn = nb, *kn = nb + hd, *in = nb + 2 * hd, *pn = nb + 2 * hd + D;
        LNAME(n, l, "self_attn.q_norm.weight");          rc = vec(ck, n, hd, qn);
        if (!rc) { LNAME(n, l, "self_attn.k_norm.weight");         rc = vec(ck, n, hd, kn); }
        if (!rc) { LNAME(n, l, "input_layernorm.weight");          rc = vec(ck, n, D, in); }
        if (!rc) { LNAME(n, l, "post_attention_layernorm.weight"); rc = vec(ck, n, D, pn); }
        if (rc) break;
        w.q_norm = qn;
        w.k_norm = kn;
        w.input_norm = in;
        w.post_attn_norm = pn;
        rc = qwen_hip_decoder_load_layer(d, l, &w);
    }
    if (!rc) {
        const uint16_t *emb = mat(ck, "thinker.model.embed_tokens.weight", c.vocab, D);
        rc = emb ? vec(ck, "thinker.model.norm.weight", D, nb) : QWEN_HIP_EINVAL;
        if (!rc) rc = qwen_hip_decoder_load_embeddings(d, emb, nb);
    }
    free(nb);
    return rc;
}

qwen_hip_decoder *qwen_hip_decoder_create_from_checkpoint(const char *model_dir, int device, int kv_capacity) {
    qwen_hip_checkpoint *ck = qwen_hip_checkpoint_open(model_dir);
    if (!ck) return NULL;
    qwen_hip_config c;
    qwen_hip_decoder *d = NULL;
    if (qwen_hip_checkpoint_config(ck, &c) == 0) d = qwen_hip_decoder_create(&c, device, kv_capacity);
    if (d && qwen_hip_decoder_load_checkpoint(d, ck) != 0) {
        char msg[512];
        snprintf(msg, sizeof(msg), "%s", qwen_hip_last_error());
        qwen_hip_decoder_destroy(d);
        qk_set_err("%s", msg);
        d = NULL;
    }
    qwen_hip_checkpoint_close(ck);
    return d;
}

/* ---- the audio encoder (thinker.audio_tower.*; qwen_encoder_load,
 * qwen_asr_encoder.c:67-168, and the encoder part of detect_config) ------- */
#define ENAME(buf, fmt, ...) snprintf(buf, sizeof(buf), "thinker.audio_tower." fmt, __VA_ARGS__)

int qwen_hip_checkpoint_enc_config(const qwen_hip_checkpoint *ck, qwen_hip_enc_config *cfg) {
    if (!ck || !cfg) return QWEN_HIP_EINVAL;
    const st_tensor *co = find(ck, "thinker.audio_tower.conv_out.weight");
    const st_tensor *fc = find(ck, "thinker.audio_tower.layers.0.fc1.weight");
    const st_tensor *p2 = find(ck, "thinker.audio_tower.proj2.weight");
    if (!co || !fc || !p2 || co->ndim != 2 || fc->ndim != 2 || p2->ndim != 2) {
        qk_set_err("checkpoint: no audio encoder (thinker.audio_tower.conv_out / layers.0.fc1 / proj2)");
        return QWEN_HIP_EINVAL;
    }
    char n[ST_NAME];
    int layers = 0;
    for (; layers < QWEN_HIP_ENC_MAX_LAYERS; layers++) {
        ENAME(n, "layers.%d.self_attn.q_proj.weight", layers);
        if (!find(ck, n)) break;
    }
    memset(cfg, 0, sizeof(*cfg));
    cfg->d_model = (int)co->shape[0];
    cfg->head_dim = 64;
    cfg->heads = cfg->d_model / 64;
    cfg->ffn_dim = (int)fc->shape[0];
    cfg->output_dim = (int)p2->shape[0];
    cfg->layers = layers;
    cfg->chunk_size = 100;
    cfg->n_window_infer = 800;
    return 0;
}

/* any F32 / BF16 tensor of exactly n elements, widened into a new fp32 buffer */
static float *f32_of(const qwen_hip_checkpoint *ck, const char *name, long long n) {
    const st_tensor *t = find(ck, name);
    if (!t) { qk_set_err("checkpoint: missing %s", name); return NULL; }
    long long numel = 1;
    for (int i = 0; i < t->ndim; i++) numel *= t->shape[i];
    if (numel != n || (t->dtype != QWEN_HIP_ST_F32 && t->dtype != QWEN_HIP_ST_BF16)) {
        qk_set_err("checkpoint: %s must be F32 or BF16 with %lld elements", name, n);
        return NULL;
    }
    float *out = (float *)malloc((size_t)n * sizeof(float));
    if (!out) { qk_set_err("checkpoint: out of host memory"); return NULL; }
    const char *p = (const char *)ck->map[t->shard] + ck->data_off[t->shard] + t->begin;
    if (t->dtype == QWEN_HIP_ST_F32) {
        memcpy(out, p, (size_t)n * 4);
    } else {
        for (long long i = 0; i < n; i++) {
            uint16_t b;
            memcpy(&b, p + 2 * i, 2);
            const uint32_t u = (uint32_t)b << 16;
            memcpy(&out[i], &u, 4);
        }
    }
    return out;
}

int qwen_hip_encoder_load_checkpoint(qwen_hip_encoder *e, const qwen_hip_checkpoint *ck) {
    if (!e || !ck) return QWEN_HIP_EINVAL;
    qwen_hip_enc_config c;
    QK_TRY(qwen_hip_checkpoint_enc_config(ck, &c));
    /* the encoder's own shape must match what it was created with */
    const qwen_hip_enc_config *ec = qwen_hip_encoder_config(e);
    if (c.d_model != ec->d_model || c.layers != ec->layers || c.ffn_dim != ec->ffn_dim ||
        c.output_dim != ec->output_dim) {
        qk_set_err("checkpoint: encoder shape differs from the encoder's configuration");
        return QWEN_HIP_EINVAL;
    }
    const long long d = c.d_model, f = c.ffn_dim, o = c.output_dim;
    char n[ST_NAME];
    int rc = 0;
    for (int l = 0; l < c.layers && !rc; l++) {
        static const char *names[16] = {"self_attn.q_proj.weight", "self_attn.q_proj.bias", "self_attn.k_proj.weight",
                                        "self_attn.k_proj.bias", "self_attn.v_proj.weight", "self_attn.v_proj.bias",
                                        "self_attn.out_proj.weight", "self_attn.out_proj.bias",
                                        "self_attn_layer_norm.weight", "self_attn_layer_norm.bias", "fc1.weight",
                                        "fc1.bias", "fc2.weight", "fc2.bias", "final_layer_norm.weight",
                                        "final_layer_norm.bias"};
        const long long sizes[16] = {d * d, d, d * d, d, d * d, d, d * d, d, d, d, f * d, f, d * f, d, d, d};
        float *p[16] = {0};
        int ok = 1;
        for (int i = 0; i < 16 && ok; i++) {
            ENAME(n, "layers.%d.%s", l, names[i]);
            p[i] = f32_of(ck, n, sizes[i]);
            ok = p[i] != NULL;
        }
        if (ok) {
            qwen_hip_enc_layer_weights w = {p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7],
                                            p[8], p[9], p[10], p[11], p[12], p[13], p[14], p[15]};
            rc = qwen_hip_encoder_load_layer(e, l, &w);
        } else {
            rc = QWEN_HIP_EINVAL;
        }
        for (int i = 0; i < 16; i++) free(p[i]);
    }
    if (rc) return rc;
    static const char *snames[13] = {"conv2d1.weight", "conv2d1.bias", "conv2d2.weight", "conv2d2.bias",
                                     "conv2d3.weight", "conv2d3.bias", "conv_out.weight", "ln_post.weight",
                                     "ln_post.bias", "proj1.weight", "proj1.bias", "proj2.weight", "proj2.bias"};
    const long long ssizes[13] = {480 * 9, 480, 480LL * 4320, 480, 480LL * 4320, 480, d * 7680, d, d, d * d, d,
                                  o * d, o};
    float *p[13] = {0};
    int ok = 1;
    for (int i = 0; i < 13 && ok; i++) {
        ENAME(n, "%s", snames[i]);
        p[i] = f32_of(ck, n, ssizes[i]);
        ok = p[i] != NULL;
    }
    if (ok) {
        qwen_hip_enc_stem_weights w = {p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8], p[9], p[10], p[11], p[12]};
        rc = qwen_hip_encoder_load_stem(e, &w);
    } else {
        rc = QWEN_HIP_EINVAL;
    }
    for (int i = 0; i < 13; i++) free(p[i]);
    return rc;
}

qwen_hip_encoder *qwen_hip_encoder_create_from_checkpoint(const char *model_dir, int device) {
    qwen_hip_checkpoint *ck = qwen_hip_checkpoint_open(model_dir);
    if (!ck) return NULL;
    qwen_hip_enc_config c;
    qwen_hip_encoder *e = NULL;
    if (qwen_hip_checkpoint_enc_config(ck, &c) == 0) e = qwen_hip_encoder_create(&c, device);
    if (e && qwen_hip_encoder_load_checkpoint(e, ck) != 0) {
        char msg[512];
        snprintf(msg, sizeof(msg), "%s", qwen_hip_last_error());
        qwen_hip_encoder_destroy(e);
        qk_set_err("%s", msg);
        e = NULL;
    }
    qwen_hip_checkpoint_close(ck);
    return e;
}
