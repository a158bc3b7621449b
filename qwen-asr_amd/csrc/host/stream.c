/*
 * stream.c - the streaming caller of the token loop: per chunk, reuse the KV
 * cache of the longest unchanged prefix of the decoder input, prefill only the
 * rest, then decode greedily (reference qwen_asr.c:1747-1829, the decoder half
 * of qwen_transcribe_stream).
 *
 * The caller builds each chunk's full decoder input (prompt template, audio
 * rows, suffix, carried text tokens) as fp32 rows, exactly as the reference
 * assembles input_embeds.  The driver compares the prefill part (all rows but
 * the last) with the previous chunk's, row by row and bitwise (the
 * reference's memcmp), keeps that many cached positions (set_kv_len), prefills
 * the remaining rows, forwards the last row, and then appends and forwards
 * tokens until <|endoftext|> / <|im_end|> or max_new tokens, as the
 * reference's loop does (:1802-1814).  The previous rows are kept on the host.
 */
#include "host_internal.h"

#include <stdlib.h>
#include <string.h>

struct qwen_hip_stream {
    qwen_hip_decoder *dec;
    int hidden;
    float *prev;             /* previous chunk's prefill rows [prev_rows][hidden] */
    int prev_rows, prev_cap;
    long long rows_total, rows_reused;
};

qwen_hip_stream *qwen_hip_stream_create(qwen_hip_decoder *dec) {
    const qwen_hip_config *c = qwen_hip_decoder_config(dec);
    if (!c) { qk_set_err("stream: NULL decoder"); return NULL; }
    qwen_hip_stream *st = (qwen_hip_stream *)calloc(1, sizeof(*st));
    if (!st) { qk_set_err("stream: out of host memory"); return NULL; }
    st->dec = dec;
    st->hidden = c->hidden;
    return st;
}

void qwen_hip_stream_destroy(qwen_hip_stream *st) {
    if (!st) return;
    free(st->prev);
    free(st);
}

void qwen_hip_stream_reset(qwen_hip_stream *st) {
    if (st) st->prev_rows = 0;
}

int qwen_hip_stream_stats(const qwen_hip_stream *st, long long *rows_total, long long *rows_reused) {
    if (!st) return QWEN_HIP_EINVAL;
    if (rows_total) *rows_total = st->rows_total;
    if (rows_reused) *rows_reused = st->rows_reused;
    return 0;
}

static int is_eos(int t) { return t == QWEN_HIP_TOKEN_ENDOFTEXT || t == QWEN_HIP_TOKEN_IM_END; }

int qwen_hip_stream_chunk(qwen_hip_stream *st, const float *rows, int n_rows, int max_new, int *out_tokens,
                          int *reused_out) {
    if (!st || !rows || n_rows < 1 || max_new < 0 || (max_new > 0 && !out_tokens)) {
        qk_set_err("stream_chunk: bad argument");
        return QWEN_HIP_EINVAL;
    }
    qwen_hip_decoder *d = st->dec;
    const size_t D = (size_t)st->hidden;
    const int prefill_len = n_rows - 1;

    /* longest bitwise-equal prefix of the prefill rows (:1752-1761) */
    int reused = 0;
    const int cmp = prefill_len < st->prev_rows ? prefill_len : st->prev_rows;
    while (reused < cmp && memcmp(st->prev + (size_t)reused * D, rows + (size_t)reused * D, D * sizeof(float)) == 0)
        reused++;
    const int kv = qwen_hip_decoder_kv_len(d);
    if (kv < 0) return kv;
    if (reused > kv) reused = kv;                      /* the caller rolled the cache back further */
    QK_TRY(qwen_hip_decoder_set_kv_len(d, reused));    /* ctx->kv_cache_len = reused_prefill (:1764) */
    if (prefill_len > reused) QK_TRY(qwen_hip_decoder_prefill(d, rows + (size_t)reused * D, prefill_len - reused));
    st->rows_total += prefill_len;
    st->rows_reused += reused;

    /* keep this chunk's prefill rows for the next comparison (:1777-1794) */
    if (prefill_len > st->prev_cap) {
        int cap = st->prev_cap > 0 ? st->prev_cap : 64;
        while (cap < prefill_len) cap *= 2;
        float *p = (float *)realloc(st->prev, (size_t)cap * D * sizeof(float));
        if (!p) {
            st->prev_rows = 0;
            qk_set_err("stream_chunk: out of host memory");
            return QWEN_HIP_ENOMEM;
        }
        st->prev = p;
        st->prev_cap = cap;
    }
    memcpy(st->prev, rows, (size_t)prefill_len * D * sizeof(float));
    st->prev_rows = prefill_len;
    if (reused_out) *reused_out = reused;

    /* first token from the last row (:1773-1774) */
    const int before = qwen_hip_decoder_kv_len(d);
    const int t1 = qwen_hip_decoder_forward(d, rows + (size_t)prefill_len * D);
    if (qwen_hip_decoder_kv_len(d) != before + 1) return QWEN_HIP_EDEVICE;
    if (max_new == 0 || is_eos(t1)) return 0;

    /* the loop appends t and forwards it while t is not EOS and fewer than
     * max_new tokens are kept (:1802-1814): one generate call of max_new steps
     * from t1, truncated at the first EOS it produces */
    out_tokens[0] = t1;
    if (max_new == 1) {
        const int b = qwen_hip_decoder_kv_len(d);
        (void)qwen_hip_decoder_forward_token(d, t1);        /* the reference forwards the last kept token too */
        if (qwen_hip_decoder_kv_len(d) != b + 1) return QWEN_HIP_EDEVICE;
        return 1;
    }
    int *tmp = (int *)malloc((size_t)max_new * sizeof(int));
    if (!tmp) { qk_set_err("stream_chunk: out of host memory"); return QWEN_HIP_ENOMEM; }
    const int kept = qwen_hip_decoder_generate(d, t1, max_new, tmp, 1);
    if (kept < 0) { free(tmp); return kept; }
    int n = 1;
    for (int i = 0; i < kept && n < max_new; i++) {
        if (is_eos(tmp[i])) break;
        out_tokens[n++] = tmp[i];
    }
    free(tmp);
    return n;
}
