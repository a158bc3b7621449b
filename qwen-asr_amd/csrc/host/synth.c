/*
 * synth.c - deterministic synthetic inputs for the decoder token loop.
 *
 * No checkpoints exist offline, so every workload runs on seeded random
 * weights.  The generator is counter based: element i of tensor t under seed s
 * depends only on (s, t, i), so any range can be produced by any thread, on
 * any host, in any order, with identical results.  Both the product (bench,
 * smoke) and the CPU checkers draw their inputs from here, which is what makes
 * "same seeded weights and inputs" hold across the CPU and GPU paths.
 *
 *   stream value    u64(s,t,i) = mix64(key(s,t) + (i+1) * 0x9E3779B97F4A7C15)
 *   normal pair j   Box-Muller on u1 = (u64(2j)>>11 + 1)*2^-53 (in (0,1]),
 *                   u2 = (u64(2j+1)>>11)*2^-53: z0 = r cos(2 pi u2),
 *                   z1 = r sin(2 pi u2), r = sqrt(-2 ln u1), all in fp64
 *   fp32 value      (float)(mean + std * z)      (round to nearest even)
 *   bf16 value      round-to-nearest-even of the fp32 value's top 16 bits
 *
 * mix64 is the SplitMix64 finaliser (Steele, Lea, Flood 2014).
 */
#include "qwen_synth.h"

#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static inline uint64_t mix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xbf58476d1ce4e5b9ULL;
    z ^= z >> 27;
    z *= 0x94d049bb133111ebULL;
    z ^= z >> 31;
    return z;
}

uint64_t qwen_synth_key(uint64_t seed, uint64_t tensor_id) {
    return mix64(mix64(seed ^ 0x5157454e41535231ULL) + tensor_id * 0xd1342543de82ef95ULL);
}

static inline uint64_t stream_u64(uint64_t key, uint64_t i) {
    return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ULL);
}

uint16_t qwen_f32_to_bf16_rne(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    if ((b & 0x7f800000u) == 0x7f800000u) {           /* inf / nan */
        return (uint16_t)((b >> 16) | ((b & 0xffffu) ? 0x40u : 0u));
    }
    uint32_t lsb = (b >> 16) & 1u;
    b += 0x7fffu + lsb;
    return (uint16_t)(b >> 16);
}

static inline void normal_pair(uint64_t key, uint64_t j, double *z0, double *z1) {
    uint64_t h1 = stream_u64(key, 2 * j);
    uint64_t h2 = stream_u64(key, 2 * j + 1);
    double u1 = (double)((h1 >> 11) + 1) * 0x1.0p-53;
    double u2 = (double)(h2 >> 11) * 0x1.0p-53;
    double r = sqrt(-2.0 * log(u1));
    double a = 6.283185307179586476925286766559 * u2;
    *z0 = r * cos(a);
    *z1 = r * sin(a);
}

enum { KIND_BF16 = 0, KIND_F32 = 1, KIND_UNIF = 2 };

typedef struct {
    void *out;
    size_t begin, end;          /* element range [begin, end) */
    uint64_t key;
    double mean, std;           /* for uniform: lo, hi */
    int kind;
} synth_job_t;

static void *synth_worker(void *arg) {
    synth_job_t *j = (synth_job_t *)arg;
    if (j->kind == KIND_UNIF) {
        float *o = (float *)j->out;
        double lo = j->mean, hi = j->std;
        for (size_t i = j->begin; i < j->end; i++) {
            double u = (double)(stream_u64(j->key, i) >> 11) * 0x1.0p-53;
            o[i] = (float)(lo + (hi - lo) * u);
        }
        return NULL;
    }
    for (size_t i = j->begin; i < j->end; ) {
        double z[2];
        uint64_t pair = i >> 1;
        normal_pair(j->key, pair, &z[0], &z[1]);
        for (int h = (int)(i & 1); h < 2 && i < j->end; h++, i++) {
            float f = (float)(j->mean + j->std * z[h]);
            if (j->kind == KIND_BF16) ((uint16_t *)j->out)[i] = qwen_f32_to_bf16_rne(f);
            else ((float *)j->out)[i] = f;
        }
    }
    return NULL;
}

static int default_threads(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    if (n > 16) n = 16;
    return (int)n;
}

static void synth_run(void *out, size_t n, uint64_t key, double a, double b, int kind, int threads) {
    if (threads <= 0) threads = default_threads();
    if (n < ((size_t)1 << 20)) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t tid[64];
    synth_job_t jobs[64];
    size_t per = (n / (size_t)threads + 1) & ~(size_t)1;   /* even split keeps pairs whole */
    int started = 0;
    for (int t = 0; t < threads; t++) {
        size_t s = (size_t)t * per, e = s + per;
        if (s >= n) break;
        if (e > n) e = n;
        jobs[t] = (synth_job_t){ out, s, e, key, a, b, kind };
        if (threads == 1 || pthread_create(&tid[t], NULL, synth_worker, &jobs[t]) != 0) {
            synth_worker(&jobs[t]);
            tid[t] = 0;
        }
        started++;
    }
    for (int t = 0; t < started; t++)
        if (tid[t]) pthread_join(tid[t], NULL);
}

void qwen_synth_normal_bf16(uint16_t *out, size_t n, uint64_t seed, uint64_t tensor_id,
                            double mean, double std, int threads) {
    synth_run(out, n, qwen_synth_key(seed, tensor_id), mean, std, KIND_BF16, threads);
}

void qwen_synth_normal_f32(float *out, size_t n, uint64_t seed, uint64_t tensor_id,
                           double mean, double std, int threads) {
    synth_run(out, n, qwen_synth_key(seed, tensor_id), mean, std, KIND_F32, threads);
}

void qwen_synth_uniform_f32(float *out, size_t n, uint64_t seed, uint64_t tensor_id,
                            double lo, double hi, int threads) {
    synth_run(out, n, qwen_synth_key(seed, tensor_id), lo, hi, KIND_UNIF, threads);
}

void qwen_synth_tokens(int *out, size_t n, uint64_t seed, uint64_t tensor_id, int n_ids) {
    uint64_t key = qwen_synth_key(seed, tensor_id);
    for (size_t i = 0; i < n; i++)
        out[i] = (int)(stream_u64(key, i) % (uint64_t)n_ids);
}

uint64_t qwen_checksum_u16(const uint16_t *p, size_t n) {
    /* FNV-1a over the little-endian bytes, folded through mix64 every 4 KB
     * so that long tensors do not collapse to a low-entropy state. */
    uint64_t h = 0xcbf29ce484222325ULL;
    for (size_t i = 0; i < n; i++) {
        h ^= p[i];
        h *= 0x100000001b3ULL;
        if ((i & 2047) == 2047) h = mix64(h);
    }
    return mix64(h ^ (uint64_t)n);
}
