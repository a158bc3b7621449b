/*
 * qwen_synth.h - seeded synthetic inputs for the decoder token loop (host C,
 * no HIP dependency, so the CPU checkers link it too).  No counterpart in the
 * reference: there are no checkpoints offline, so every workload is drawn from
 * this counter-based generator (see synth.c for the exact recipe).
 */
#ifndef QWEN_SYNTH_H
#define QWEN_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Tensor ids for a decoder model. */
#define QWEN_SYNTH_EMBED        1u
#define QWEN_SYNTH_FINAL_NORM   2u
#define QWEN_SYNTH_LAYER(l, f)  (1000u + 32u * (uint64_t)(l) + (uint64_t)(f))
enum {
    QWEN_SYNTH_WQ = 0, QWEN_SYNTH_WK, QWEN_SYNTH_WV, QWEN_SYNTH_WO,
    QWEN_SYNTH_GATE, QWEN_SYNTH_UP, QWEN_SYNTH_DOWN,
    QWEN_SYNTH_QNORM, QWEN_SYNTH_KNORM, QWEN_SYNTH_INNORM, QWEN_SYNTH_POSTNORM
};
#define QWEN_SYNTH_AUDIO(chunk) (500000u + (uint64_t)(chunk))
/* Tensor ids for an audio encoder: layer l < 30, the stem / projections as
 * "layer" 30; the mel input of a workload. */
#define QWEN_SYNTH_ENC(l, f)    (700000u + 32u * (uint64_t)(l) + (uint64_t)(f))
#define QWEN_SYNTH_ENC_STEM     30u
#define QWEN_SYNTH_MEL(set)     (750000u + (uint64_t)(set))
enum {
    QWEN_SYNTH_E_WQ = 0, QWEN_SYNTH_E_BQ, QWEN_SYNTH_E_WK, QWEN_SYNTH_E_BK, QWEN_SYNTH_E_WV, QWEN_SYNTH_E_BV,
    QWEN_SYNTH_E_WO, QWEN_SYNTH_E_BO, QWEN_SYNTH_E_LN1W, QWEN_SYNTH_E_LN1B, QWEN_SYNTH_E_FC1W, QWEN_SYNTH_E_FC1B,
    QWEN_SYNTH_E_FC2W, QWEN_SYNTH_E_FC2B, QWEN_SYNTH_E_LN2W, QWEN_SYNTH_E_LN2B
};
enum {
    QWEN_SYNTH_S_CONV1W = 0, QWEN_SYNTH_S_CONV1B, QWEN_SYNTH_S_CONV2W, QWEN_SYNTH_S_CONV2B, QWEN_SYNTH_S_CONV3W,
    QWEN_SYNTH_S_CONV3B, QWEN_SYNTH_S_CONVOUT, QWEN_SYNTH_S_LNPW, QWEN_SYNTH_S_LNPB, QWEN_SYNTH_S_P1W,
    QWEN_SYNTH_S_P1B, QWEN_SYNTH_S_P2W, QWEN_SYNTH_S_P2B
};
#define QWEN_SYNTH_TOKENS(set)  (600000u + (uint64_t)(set))

uint64_t qwen_synth_key(uint64_t seed, uint64_t tensor_id);
uint16_t qwen_f32_to_bf16_rne(float f);
void qwen_synth_normal_bf16(uint16_t *out, size_t n, uint64_t seed, uint64_t tensor_id,
                            double mean, double std, int threads);
void qwen_synth_normal_f32(float *out, size_t n, uint64_t seed, uint64_t tensor_id,
                           double mean, double std, int threads);
void qwen_synth_uniform_f32(float *out, size_t n, uint64_t seed, uint64_t tensor_id,
                            double lo, double hi, int threads);
void qwen_synth_tokens(int *out, size_t n, uint64_t seed, uint64_t tensor_id, int n_ids);
uint64_t qwen_checksum_u16(const uint16_t *p, size_t n);

#ifdef __cplusplus
}
#endif
#endif /* QWEN_SYNTH_H */
