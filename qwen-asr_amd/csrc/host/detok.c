/*
 * detok.c - token ids -> UTF-8 text, the step after the token loop: the
 * decode half of the reference tokenizer (qwen_tokenizer_load /
 * qwen_tokenizer_decode, qwen_asr_tokenizer.c:500-609) and the transcript
 * assembly of the greedy loop (qwen_asr.c:729-754).
 *
 * vocab.json maps byte-level BPE strings to ids.  Each character of a string
 * stands for one byte under the GPT-2 byte <-> code point table: the printable
 * bytes 33-126, 161-172 and 174-255 map to themselves, the other 68 bytes to
 * code points 256, 257, ... in byte order.  A piece is the byte string its
 * characters map back to; a code point outside the table becomes '?', as in
 * the reference.  Ids missing from the file (and the special tokens past the
 * BPE vocabulary) decode to "".
 */
#include "host_internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct qwen_hip_vocab {
    int n;               /* max id + 1 */
    char **piece;        /* [n] decoded bytes, NUL terminated; NULL = absent */
};

/* code point -> byte of the byte-level table, -1 outside it */
static int cp_to_byte(unsigned cp) {
    static int table[512];
    static int ready = 0;
    if (!ready) {
        for (int i = 0; i < 512; i++) table[i] = -1;
        int extra = 0;
        for (int b = 0; b < 256; b++) {
            const int printable = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
            table[printable ? b : 256 + extra++] = b;
        }
        ready = 1;
    }
    return cp < 512 ? table[cp] : -1;
}

/* JSON string at *pp (after the opening quote) -> code points, as the
 * reference reads vocab keys: \n \t \" \\ \/ and \uXXXX escapes (a \u escape
 * is one code point; other escapes give their character), UTF-8 otherwise,
 * decoded by its lead byte with continuation bytes missing at the key's end
 * read as zero bits.  Writes the mapped bytes into out (cap includes the
 * NUL).  Returns 0 on success. */
static int read_key(const char **pp, const char *end, char *out, size_t cap) {
    const unsigned char *p = (const unsigned char *)*pp, *e = (const unsigned char *)end;
    const unsigned char *close = p;          /* the closing quote: escapes skip one character */
    while (close < e && *close != '"') close += (*close == '\\') ? 2 : 1;
    if (close >= e) return -1;
    size_t n = 0;
    while (p < close) {
        unsigned cp;
        if (*p == '\\') {
            const unsigned char c = *++p;
            p++;
            if (c == 'u') {
                cp = 0;
                for (int i = 0; i < 4 && p < close; i++, p++) {
                    const unsigned char h = *p;
                    cp <<= 4;
                    if (h >= '0' && h <= '9') cp |= h - '0';
                    else if (h >= 'a' && h <= 'f') cp |= h - 'a' + 10;
                    else if (h >= 'A' && h <= 'F') cp |= h - 'A' + 10;
                }
            } else {
                cp = c == 'n' ? '\n' : c == 't' ? '\t' : c;
            }
        } else {
            const unsigned char c = *p;
            int len = 1;
            if ((c & 0x80) == 0) { cp = c; }
            else if ((c & 0xE0) == 0xC0) { cp = c & 0x1F; len = 2; }
            else if ((c & 0xF0) == 0xE0) { cp = c & 0x0F; len = 3; }
            else if ((c & 0xF8) == 0xF0) { cp = c & 0x07; len = 4; }
            else { cp = c; }
            for (int i = 1; i < len; i++) cp = (cp << 6) | (p + i < close ? (p[i] & 0x3F) : 0);
            p = p + len < close ? p + len : close;
        }
        const int b = cp_to_byte(cp);
        if (n + 1 >= cap) return -1;
        out[n++] = (char)(b >= 0 ? b : '?');
    }
    *pp = (const char *)close + 1;
    out[n] = '\0';
    return 0;
}

static void ws(const char **p, const char *e) {
    while (*p < e && (**p == ' ' || **p == '\n' || **p == '\r' || **p == '\t')) (*p)++;
}

void qwen_hip_vocab_free(qwen_hip_vocab *v) {
    if (!v) return;
    if (v->piece)                              /* NULL when the first pass failed */
        for (int i = 0; i < v->n; i++) free(v->piece[i]);
    free(v->piece);
    free(v);
}

qwen_hip_vocab *qwen_hip_vocab_load(const char *vocab_json_path) {
    FILE *f = vocab_json_path ? fopen(vocab_json_path, "rb") : NULL;
    if (!f) { qk_set_err("vocab: cannot open %s", vocab_json_path ? vocab_json_path : "(null)"); return NULL; }
    fseek(f, 0, SEEK_END);
    const long size = ftell(f);
    fseek(f, 0, SEEK_SET);
    char *json = size > 0 ? (char *)malloc((size_t)size + 1) : NULL;   /* NUL-terminated for strtol */
    if (!json || fread(json, 1, (size_t)size, f) != (size_t)size) {
        fclose(f);
        free(json);
        qk_set_err("vocab: cannot read %s", vocab_json_path);
        return NULL;
    }
    fclose(f);
    json[size] = '\0';
    const char *end = json + size;
    char *key = (char *)malloc(65536);
    qwen_hip_vocab *v = (qwen_hip_vocab *)calloc(1, sizeof(*v));
    if (!key || !v) { free(key); free(v); free(json); qk_set_err("vocab: out of host memory"); return NULL; }
    /* two passes: the largest id sizes the table, then the pieces */
    for (int pass = 0; pass < 2; pass++) {
        const char *p = json;
        ws(&p, end);
        if (p >= end || *p != '{') goto bad;
        p++;
        for (;;) {
            ws(&p, end);
            if (p < end && *p == ',') { p++; continue; }
            if (p >= end || *p == '}') break;
            if (*p != '"') goto bad;
            p++;
            if (read_key(&p, end, key, 65536)) goto bad;
            ws(&p, end);
            if (p >= end || *p != ':') goto bad;
            p++;
            ws(&p, end);
            char *e = NULL;
            const long id = strtol(p, &e, 10);
            if (!e || e == p || e > end) goto bad;
            p = e;
            if (id < 0 || id >= (1L << 24)) continue;
            if (pass == 0) {
                if (id + 1 > v->n) v->n = (int)id + 1;
            } else {
                free(v->piece[id]);                       /* a repeated id keeps its last key */
                v->piece[id] = strdup(key);
                if (!v->piece[id]) goto oom;
            }
        }
        if (pass == 0) {
            v->piece = (char **)calloc(v->n > 0 ? (size_t)v->n : 1, sizeof(char *));
            if (!v->piece) goto oom;
        }
    }
    free(key);
    free(json);
    return v;
bad:
    qk_set_err("vocab: %s is not a JSON object of string -> id", vocab_json_path);
    goto fail;
oom:
    qk_set_err("vocab: out of host memory");
fail:
    free(key);
    free(json);
    qwen_hip_vocab_free(v);
    return NULL;
}

int qwen_hip_vocab_size(const qwen_hip_vocab *v) { return v ? v->n : QWEN_HIP_EINVAL; }

const char *qwen_hip_vocab_piece(const qwen_hip_vocab *v, int id) {
    if (!v || id < 0 || id >= v->n || !v->piece[id]) return "";
    return v->piece[id];
}

long qwen_hip_vocab_transcript(const qwen_hip_vocab *v, const int *tokens, int n, int past_asr_text, char *out,
                               size_t cap) {
    if (!v || n < 0 || (n > 0 && !tokens) || (cap > 0 && !out)) return QWEN_HIP_EINVAL;
    size_t len = 0;
    int started = past_asr_text != 0;
    for (int i = 0; i < n; i++) {
        const int t = tokens[i];
        if (t == QWEN_HIP_TOKEN_ENDOFTEXT || t == QWEN_HIP_TOKEN_IM_END) break;
        if (t == QWEN_HIP_TOKEN_ASR_TEXT) { started = 1; continue; }
        if (!started) continue;
        const char *piece = qwen_hip_vocab_piece(v, t);
        const size_t k = strlen(piece);
        if (len + k < cap) memcpy(out + len, piece, k);
        len += k;
    }
    if (cap > 0) out[len < cap ? len : cap - 1] = '\0';
    return (long)len;
}
