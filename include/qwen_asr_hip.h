/*
 * qwen_asr_hip.h - C ABI of the MI355X (gfx950) Qwen3 decoder token loop.
 *
 * This is the drop-in boundary for the reference's decoder hot path:
 *   - the decoder-level entry points replace qwen_decoder_prefill /
 *     qwen_decoder_forward (reference qwen_asr.h:313-317,
 *     qwen_asr_decoder.c:262 and :388) and the KV-length bookkeeping the
 *     callers do on ctx->kv_cache_len (qwen_asr.c:704, :1764);
 *   - the op-level entry points replace the operators of qwen_asr_kernels.h
 *     that the decoder calls, with the same argument meaning, but on DEVICE
 *     pointers and with a HIP stream (NULL = the legacy default stream).
 *
 * Plain C: no C++ or torch types cross this boundary.  Every function that can
 * fail returns 0 on success and a negative QWEN_HIP_E* code otherwise, except
 * where noted; qwen_hip_last_error() gives the message of the last failure on
 * the calling thread.  qwen_hip_decoder_forward keeps the reference
 * convention of returning QWEN_TOKEN_IM_END (151645) when it cannot run
 * (reference qwen_asr_decoder.c:417, :421).
 *
 * Numerics: bf16 weights (raw uint16 bit patterns, as the reference's
 * uint16_t *W_bf16), fp32 activations, fp32 accumulation, fp32 KV cache.
 */
#ifndef QWEN_ASR_HIP_H
#define QWEN_ASR_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "qwen_synth.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------
 * Constants (reference qwen_asr.h:23, :30-36)
 * ------------------------------------------------------------------------ */
#define QWEN_HIP_VOCAB_SIZE        151936
#define QWEN_HIP_TOKEN_ENDOFTEXT   151643
#define QWEN_HIP_TOKEN_IM_END      151645
#define QWEN_HIP_TOKEN_ASR_TEXT    151704      /* <asr_text>, qwen_asr.h:36 */
#define QWEN_HIP_MAX_LAYERS        28          /* QWEN_MAX_DEC_LAYERS, qwen_asr.h:27 */
#define QWEN_HIP_HEAD_DIM          128         /* the only head size the kernels build for */

#define QWEN_HIP_OK          0
#define QWEN_HIP_EINVAL     -1    /* bad argument / shape the kernels do not support */
#define QWEN_HIP_ENOMEM     -2    /* device or host allocation failed */
#define QWEN_HIP_EDEVICE    -3    /* a HIP runtime call failed */
#define QWEN_HIP_ESTATE     -4    /* call out of order (e.g. forward before weights) */

/* ------------------------------------------------------------------------
 * Model configuration: the decoder fields of qwen_config_t
 * (reference qwen_asr.h:60-68; values set by detect_config, qwen_asr.c:135-191)
 * ------------------------------------------------------------------------ */
typedef struct {
    int hidden;          /* dec_hidden: 1024 (0.6B) or 2048 (1.7B) */
    int layers;          /* dec_layers: 28 */
    int heads;           /* dec_heads: 16 */
    int kv_heads;        /* dec_kv_heads: 8 */
    int head_dim;        /* dec_head_dim: 128 */
    int intermediate;    /* dec_intermediate: 3072 or 6144 */
    int vocab;           /* vocab_size: 151936 */
    float rms_eps;       /* dec_rms_norm_eps: 1e-6 */
    float rope_theta;    /* dec_rope_theta: 1e6 */
} qwen_hip_config;

/* Fill cfg with the reference's 0.6B (model_b = 0) or 1.7B (model_b = 1)
 * decoder shape (qwen_asr.c:153-186). */
void qwen_hip_config_preset(qwen_hip_config *cfg, int model_b);

/* Host-side weights of one decoder layer, as qwen_dec_layer_t holds them
 * (reference qwen_asr.h:131-153): bf16 matrices row-major [out][in],
 * fp32 norm vectors. */
typedef struct {
    const uint16_t *wq;              /* [heads*head_dim][hidden] */
    const uint16_t *wk;              /* [kv_heads*head_dim][hidden] */
    const uint16_t *wv;              /* [kv_heads*head_dim][hidden] */
    const uint16_t *wo;              /* [hidden][heads*head_dim] */
    const uint16_t *gate;            /* [intermediate][hidden] */
    const uint16_t *up;              /* [intermediate][hidden] */
    const uint16_t *down;            /* [hidden][intermediate] */
    const float *q_norm;             /* [head_dim] */
    const float *k_norm;             /* [head_dim] */
    const float *input_norm;         /* [hidden] */
    const float *post_attn_norm;     /* [hidden] */
} qwen_hip_layer_weights;

/* ------------------------------------------------------------------------
 * Decoder-level ABI (the timed path)
 * ------------------------------------------------------------------------ */
typedef struct qwen_hip_decoder qwen_hip_decoder;

/* Create a decoder context on HIP device `device` with room for
 * `kv_capacity` cached positions (grown by doubling when exceeded, as
 * kv_cache_grow does, qwen_asr_decoder.c:133-160).  Returns NULL on failure. */
qwen_hip_decoder *qwen_hip_decoder_create(const qwen_hip_config *cfg, int device,
                                          int kv_capacity);
void qwen_hip_decoder_destroy(qwen_hip_decoder *dec);

/* Upload weights (replaces qwen_decoder_load, qwen_asr_decoder.c:45-116:
 * the gate/up rows are interleaved [g0,u0,g1,u1,...] as :95-107 does, and
 * Wq|Wk|Wv are concatenated so one GEMV pass streams all three). */
int qwen_hip_decoder_load_layer(qwen_hip_decoder *dec, int layer,
                                const qwen_hip_layer_weights *w);
int qwen_hip_decoder_load_embeddings(qwen_hip_decoder *dec,
                                     const uint16_t *tok_embeddings, /* [vocab][hidden] */
                                     const float *final_norm);       /* [hidden] */

/* Generate the seeded synthetic model directly (host generation with
 * qwen_synth_*, then upload).  norm_std = 0 gives the all-ones norms the
 * benchmark configs prescribe; norm_std > 0 draws 1 + norm_std*N(0,1). */
int qwen_hip_decoder_load_synthetic(qwen_hip_decoder *dec, uint64_t seed,
                                    double weight_std, double norm_std);

/* qwen_decoder_prefill (qwen_asr_decoder.c:262-359): run `seq_len` fp32 rows
 * [seq_len][hidden] through all layers starting at position kv_len, append
 * their K/V, advance kv_len.  `rows` is a HOST pointer; the _device variant
 * takes a device pointer.  Produces no token. */
int qwen_hip_decoder_prefill(qwen_hip_decoder *dec, const float *rows, int seq_len);
int qwen_hip_decoder_prefill_device(qwen_hip_decoder *dec, const float *d_rows, int seq_len);

/* qwen_decoder_forward (qwen_asr_decoder.c:388-476): one fp32 row (HOST
 * pointer) at position kv_len; returns the greedy token (argmax of the tied
 * LM head over the final-normed hidden state, lowest index on ties), or
 * QWEN_HIP_TOKEN_IM_END on failure. */
int qwen_hip_decoder_forward(qwen_hip_decoder *dec, const float *row);

/* Same step with the input row gathered on the device from the embedding
 * table (tok_embed_bf16_to_f32, qwen_asr.c:353-360, fused into the step). */
int qwen_hip_decoder_forward_token(qwen_hip_decoder *dec, int token);

/* The greedy loop of qwen_asr.c:729-759 kept on the device: starting from
 * `first_token`, run n_steps forwards, each fed the previous step's argmax,
 * with no host round trip per token.  Writes the n_steps produced tokens to
 * out_tokens (host).  stop_on_eos != 0 truncates at the first
 * <|endoftext|>/<|im_end|> (reference :733) and returns the count kept;
 * otherwise returns n_steps.  Negative on error. */
int qwen_hip_decoder_generate(qwen_hip_decoder *dec, int first_token, int n_steps,
                              int *out_tokens, int stop_on_eos);

/* KV bookkeeping: ctx->kv_cache_len.  set_kv_len accepts 0..kv_len and is
 * the rollback used by streaming reuse (qwen_asr.c:1764). */
int qwen_hip_decoder_kv_len(const qwen_hip_decoder *dec);
int qwen_hip_decoder_set_kv_len(qwen_hip_decoder *dec, int kv_len);

/* Validation taps.  read_hidden copies the final-normed hidden state of the
 * last forward (the reference's ctx->dec_x after :474) to host [hidden].
 * With keep_logits on, every forward also writes its full fp32 logits
 * [vocab], readable with read_logits (costs one extra vocab-sized write). */
int qwen_hip_decoder_set_keep_logits(qwen_hip_decoder *dec, int on);
int qwen_hip_decoder_read_hidden(qwen_hip_decoder *dec, float *out);
int qwen_hip_decoder_read_logits(qwen_hip_decoder *dec, float *out);

/* Decode engine: 0 = one kernel per fused op, replayed from a HIP graph;
 * 1 = the same kernels launched eagerly (no graph); 2 = the whole greedy loop
 * of a forward/generate call in one persistent kernel, one block per CU (default
 * where supported: 16 query / 8 kv heads, the 0.6B or 1.7B shape, 256 CUs in
 * 8 XCDs).  set_engine(2) returns QWEN_HIP_EINVAL where it is not supported.
 * Every wait inside the persistent kernel is bounded (set_wait_limit, default
 * 1 s of the device wall clock; the launch check-in, where every block of the
 * grid must have started, by 20 ms or the limit if shorter, so a grid that
 * shares the device with other work gives up early); a run that times out or
 * finds its grid not laid out one block per CU raises an error bit, and all
 * its blocks leave.
 * With fallback on (set_fallback, the default) the decoder then reports on
 * stderr, counts the event (fallbacks), switches to engine 0 and redoes the
 * steps there; with fallback off the call returns QWEN_HIP_EDEVICE (forward:
 * the failure token) and the decoder is left as before the call.  No
 * reference counterpart: the reference has one CPU path (qwen_asr_kernels.c). */
int qwen_hip_decoder_set_engine(qwen_hip_decoder *dec, int engine);
int qwen_hip_decoder_engine(const qwen_hip_decoder *dec);
int qwen_hip_decoder_set_fallback(qwen_hip_decoder *dec, int on);
int qwen_hip_decoder_fallbacks(const qwen_hip_decoder *dec);
/* seconds in [0, 60]; 0 makes every wait that is not satisfied by its first
 * poll give up (a test of the give-up path) */
int qwen_hip_decoder_set_wait_limit(qwen_hip_decoder *dec, double seconds);
/* Hand-over words carry a 32-bit tag that every launch takes from a running
 * epoch (each launch advances it by the tags it uses); when the next launch
 * would pass 0xFFFFFF00 the decoder zeroes the exchange words and starts again
 * at 1.  set_tag_epoch (epoch >= 1) zeroes the words and sets the epoch, so a
 * test can run launches at the top of the tag space and across the restart;
 * tag_epoch reads it (0 for a NULL decoder). */
int qwen_hip_decoder_set_tag_epoch(qwen_hip_decoder *dec, unsigned epoch);
unsigned qwen_hip_decoder_tag_epoch(const qwen_hip_decoder *dec);

/* Diagnostics of the persistent engine (no reference counterpart; the
 * reference only times whole phases with gettimeofday, qwen_asr.c:362-366).
 * set_trace(step >= 0): every later persistent launch records, for its step
 * index `step`, a 100 MHz wall-clock stamp per block at each hand-over point
 * (step < 0 turns it off).  read_trace copies the last record,
 * [256 blocks][704] uint64 (n >= 256*704), and returns the words per block.
 * Per layer l the stamps sit at 10*l + {0 Q entered, 1 Q input ready,
 * 2 attention entered, 3 its input ready, 4 O entered, 5 ready, 6 MLP entered,
 * 7 ready, 8 down entered, 9 ready}, then 10*layers + {0 LM head entered,
 * 1 ready, 2 token reduction entered, 3 token ready}; "entered" means the
 * block's compute of the previous stage is done (for the 1.7B shape, the
 * attention and down entries are where the sync wave starts polling, while
 * the previous dot may still run).  Compute-side stamps of
 * layer l sit at 320 + 10*l + {0 QKV dot done, 1 its stores and the next
 * prefetches issued, 2 q/k norm done, 3 attention fold done, 4 split partial
 * stored, 5 splits merged, 6 O dot done, 7 O stores and prefetches issued,
 * 8 gate/up dot done, 9 down dot done}; 640 + 2*l + {0, 1}: the cross-XCD
 * half of the residual update before QKV / before the MLP is done (640 + 2*layers:
 * the final one). */
int qwen_hip_decoder_set_trace(qwen_hip_decoder *dec, int step);
int qwen_hip_decoder_read_trace(qwen_hip_decoder *dec, uint64_t *out, size_t n);

/* The persistent engine has two kernels.  The split kernel (any supported
 * shape) has every CU stream its share of every layer.  The relay kernel (the
 * 0.6B shape; default where available) splits each XCD's CUs into two teams
 * that take the layers in turn: one team computes a layer from weights it
 * holds in registers while the other streams the next layer's weights, so a
 * computing CU's hand-overs never wait behind its own weight loads.  It keeps
 * each attention split's cached K/V rows in LDS, which bounds it to launches
 * whose positions stay below QWEN_HIP_RELAY_MAX_POS; longer contexts run on
 * the split kernel.  Both compute the same arithmetic (bf16 weights, fp32
 * activations and sums; the relay kernel's products run on the matrix cores
 * with each fp32 activation split exactly into three bf16 terms), so tokens
 * agree with the reference either way.  set_relay(0) forces the split kernel.
 * last_kernel: the kernel of the last persistent launch (its trace layout):
 * QWEN_HIP_KERNEL_SPLIT or QWEN_HIP_KERNEL_RELAY, 0 before any.
 *
 * Relay trace layout (read_trace returns 704 words per block): for layer l
 * of the block's team (team 0 even layers, team 1 odd), words 24*l + {0 input
 * wait entered, 1 cross-XCD half of the input residual in, 2 wave 0's
 * quarter of the input residual gathered, 4 Q stored, 5 q|k|v gathered,
 * 6 attention entered, 7 fold done, 8 split partials stored, 9 merge slices
 * in, 10 merged dims stored, 11 merged attention gathered, 12 O stored,
 * 13 cross-XCD half of the post-attention residual in, 14 wave 0's quarter
 * of the post-attention residual gathered, 16 gate|up
 * products reduced, 17 SwiGLU stored, 18 SwiGLU outputs gathered, 19 down
 * stored, 20 next layer's loads issued} (3 and 15 repeat 2 and 14); then
 * 24*layers + {0 LM entered, 1 final residual cross half in, 2 gathered,
 * 3 candidate stored, 4 token ready (team 0 only)}.  A record holds one
 * launch: set_trace clears it.  No
 * reference counterpart (the reference decodes on the CPU). */
#define QWEN_HIP_KERNEL_SPLIT 1
#define QWEN_HIP_KERNEL_RELAY 2
#define QWEN_HIP_RELAY_MAX_POS 1024
int qwen_hip_decoder_set_relay(qwen_hip_decoder *dec, int on);
int qwen_hip_decoder_last_kernel(const qwen_hip_decoder *dec);

/* The stream the decoder launches on (for event timing by callers). */
hipStream_t qwen_hip_decoder_stream(const qwen_hip_decoder *dec);

/* Per-step algorithmic HBM bytes of one forward at cache length kv_len
 * (weights + LM head + fp32 norms + K/V read + K/V write). */
double qwen_hip_decoder_step_bytes(const qwen_hip_decoder *dec, int kv_len);

const char *qwen_hip_last_error(void);

/* The configuration the decoder was created with (NULL for NULL). */
const qwen_hip_config *qwen_hip_decoder_config(const qwen_hip_decoder *dec);

/* ------------------------------------------------------------------------
 * Checkpoint loading: a Qwen3-ASR safetensors directory (model.safetensors,
 * or model-*.safetensors shards in name order) mapped read-only; replaces
 * multi_safetensors_open / multi_safetensors_find / safetensors_get_*
 * (reference qwen_asr_safetensors.h:47-73, qwen_asr_safetensors.c:194-394),
 * qwen_decoder_load (qwen_asr_decoder.c:45-116) and the decoder part of
 * detect_config (qwen_asr.c:135-191).  Only the decoder tensors
 * (thinker.model.*) are read.
 * ------------------------------------------------------------------------ */
#define QWEN_HIP_ST_F32    0       /* dtype codes, as safetensor_dtype_t (qwen_asr_safetensors.h:15-23) */
#define QWEN_HIP_ST_F16    1
#define QWEN_HIP_ST_BF16   2
#define QWEN_HIP_ST_OTHER -1

typedef struct qwen_hip_checkpoint qwen_hip_checkpoint;

/* NULL on failure (message in qwen_hip_last_error). */
qwen_hip_checkpoint *qwen_hip_checkpoint_open(const char *model_dir);
void qwen_hip_checkpoint_close(qwen_hip_checkpoint *ck);
/* number of tensors over all shards */
int qwen_hip_checkpoint_count(const qwen_hip_checkpoint *ck);
/* Look a tensor up by name (multi_safetensors_find): dtype, rank, shape
 * (up to 8 dims) and a pointer to its bytes inside the mapping (valid until
 * close).  Any output may be NULL.  QWEN_HIP_EINVAL when absent. */
int qwen_hip_checkpoint_tensor(const qwen_hip_checkpoint *ck, const char *name, int *dtype, int *ndim,
                               long long *shape, const void **data);
/* The decoder shape from the tensor shapes: hidden and vocab from
 * embed_tokens, heads / kv_heads from the q / k projection rows, the MLP
 * width from gate_proj, layers = count of consecutive layers present;
 * rms eps 1e-6 and rope theta 1e6 (qwen_asr.c:187-188). */
int qwen_hip_checkpoint_config(const qwen_hip_checkpoint *ck, qwen_hip_config *cfg);
/* Upload every decoder tensor: BF16 matrices straight from the mapping
 * (load_bf16_direct), F32 or BF16 norm vectors widened to fp32 (load_f32). */
int qwen_hip_decoder_load_checkpoint(qwen_hip_decoder *dec, const qwen_hip_checkpoint *ck);
/* open + config + create + load + close in one call; NULL on failure. */
qwen_hip_decoder *qwen_hip_decoder_create_from_checkpoint(const char *model_dir, int device, int kv_capacity);

/* ------------------------------------------------------------------------
 * Streaming driver: the decoder half of qwen_transcribe_stream (reference
 * qwen_asr.c:1747-1829).  Each call takes one chunk's complete decoder
 * input rows (the caller assembles template + audio + suffix + carried
 * tokens as the reference builds input_embeds), keeps the cached positions
 * of the longest prefix of rows[0..n_rows-1) that is bitwise equal to the
 * previous call's (the reference's memcmp, :1752-1764), prefills the rest,
 * forwards the last row and decodes greedily like the reference's loop
 * (:1802-1814): tokens are appended (and forwarded) until <|endoftext|> /
 * <|im_end|> or max_new of them.  Returns the number of tokens written to
 * out_tokens (room for max_new), negative on error; *reused_rows (may be
 * NULL) receives the reused prefix length.  The stream does not own the
 * decoder; one stream per decoder at a time.
 * ------------------------------------------------------------------------ */
typedef struct qwen_hip_stream qwen_hip_stream;
qwen_hip_stream *qwen_hip_stream_create(qwen_hip_decoder *dec);
void qwen_hip_stream_destroy(qwen_hip_stream *st);
/* forget the previous rows: the next chunk prefills from position 0 */
void qwen_hip_stream_reset(qwen_hip_stream *st);
int qwen_hip_stream_chunk(qwen_hip_stream *st, const float *rows, int n_rows, int max_new, int *out_tokens,
                          int *reused_rows);
/* prefill rows seen and reused so far (the reference's prefill_total_tokens /
 * prefill_reused_tokens, :1768-1769) */
int qwen_hip_stream_stats(const qwen_hip_stream *st, long long *rows_total, long long *rows_reused);

/* ------------------------------------------------------------------------
 * Audio encoder: qwen_encoder_load / qwen_encoder_forward (reference
 * qwen_asr_encoder.c:67-372) on the fp32 matrix cores.  mel [128][frames] ->
 * [tokens][output_dim] rows, the input the decoder's prefill consumes.
 * ------------------------------------------------------------------------ */
#define QWEN_HIP_ENC_MAX_LAYERS 24        /* QWEN_MAX_ENC_LAYERS, qwen_asr.h:26 */

/* The encoder fields of qwen_config_t (qwen_asr.h:48-57) */
typedef struct {
    int d_model;         /* 896 (0.6B) or 1024 (1.7B) */
    int layers;          /* 18 or 24 */
    int heads;           /* 14 or 16 */
    int head_dim;        /* 64 */
    int ffn_dim;         /* 3584 or 4096 */
    int output_dim;      /* 1024 or 2048 (the decoder's hidden) */
    int chunk_size;      /* mel frames per stem chunk: 100 */
    int n_window_infer;  /* 800: attention windows of n_window_infer / chunk_size chunks */
} qwen_hip_enc_config;

/* the reference's two presets (detect_config, qwen_asr.c:135-191) */
void qwen_hip_enc_config_preset(qwen_hip_enc_config *cfg, int model_b);

/* Host weights, fp32 as qwen_enc_layer_t / qwen_encoder_t hold them after
 * loading (qwen_asr.h:75-125); matrices row-major [out][in]. */
typedef struct {
    const float *wq, *bq, *wk, *bk, *wv, *bv, *wo, *bo;   /* [d][d], [d] */
    const float *ln1_w, *ln1_b;                           /* self_attn_layer_norm [d] */
    const float *fc1_w, *fc1_b, *fc2_w, *fc2_b;           /* [ffn][d], [ffn], [d][ffn], [d] */
    const float *ln2_w, *ln2_b;                           /* final_layer_norm [d] */
} qwen_hip_enc_layer_weights;

typedef struct {
    const float *conv1_w, *conv1_b;      /* [480][1][3][3], [480] */
    const float *conv2_w, *conv2_b;      /* [480][480][3][3], [480] */
    const float *conv3_w, *conv3_b;
    const float *conv_out_w;             /* [d][480*16] */
    const float *ln_post_w, *ln_post_b;  /* [d] */
    const float *proj1_w, *proj1_b;      /* [d][d], [d] */
    const float *proj2_w, *proj2_b;      /* [output_dim][d], [output_dim] */
} qwen_hip_enc_stem_weights;

typedef struct qwen_hip_encoder qwen_hip_encoder;
qwen_hip_encoder *qwen_hip_encoder_create(const qwen_hip_enc_config *cfg, int device);
void qwen_hip_encoder_destroy(qwen_hip_encoder *enc);
int qwen_hip_encoder_load_layer(qwen_hip_encoder *enc, int layer, const qwen_hip_enc_layer_weights *w);
int qwen_hip_encoder_load_stem(qwen_hip_encoder *enc, const qwen_hip_enc_stem_weights *w);
/* seeded synthetic encoder (qwen_synth ids QWEN_SYNTH_ENC): bf16 N(0, wstd)
 * matrices widened to fp32 (conv1: N(0, 10 wstd)), fp32 biases N(0, wstd),
 * LayerNorm weights 1 + N(0, 0.1), LayerNorm biases N(0, 0.02) */
int qwen_hip_encoder_load_synthetic(qwen_hip_encoder *enc, uint64_t seed, double wstd);
/* tokens the encoder produces for mel_frames frames (:193-214) */
int qwen_hip_encoder_tokens(const qwen_hip_enc_config *cfg, int mel_frames);
/* qwen_encoder_forward: mel (host) [128][mel_frames] -> out (host)
 * [tokens][output_dim]; returns tokens, negative on error. */
int qwen_hip_encoder_forward(qwen_hip_encoder *enc, const float *mel, int mel_frames, float *out);
/* Device in, device out: *d_out points at the encoder's own output buffer
 * (valid until the next call), ready for qwen_hip_decoder_prefill_device. */
int qwen_hip_encoder_forward_device(qwen_hip_encoder *enc, const float *d_mel, int mel_frames, const float **d_out);
hipStream_t qwen_hip_encoder_stream(const qwen_hip_encoder *enc);
const qwen_hip_enc_config *qwen_hip_encoder_config(const qwen_hip_encoder *enc);
/* Encoder from a checkpoint (thinker.audio_tower.*, qwen_encoder_load,
 * qwen_asr_encoder.c:67-168): shape from the tensor shapes (d_model from
 * conv_out rows, ffn from fc1 rows, output_dim from proj2 rows, layers
 * counted, 64-wide heads); F32 or BF16 tensors widened to fp32. */
int qwen_hip_checkpoint_enc_config(const qwen_hip_checkpoint *ck, qwen_hip_enc_config *cfg);
int qwen_hip_encoder_load_checkpoint(qwen_hip_encoder *enc, const qwen_hip_checkpoint *ck);
qwen_hip_encoder *qwen_hip_encoder_create_from_checkpoint(const char *model_dir, int device);

/* ------------------------------------------------------------------------
 * Token ids -> text: the decode half of the reference tokenizer
 * (qwen_tokenizer_load / qwen_tokenizer_decode, qwen_asr_tokenizer.c:500-609,
 * byte-level table :25-47, key decoding :70-121) and the transcript assembly
 * of the greedy loop (qwen_asr.c:729-754).  Host only.
 * ------------------------------------------------------------------------ */
typedef struct qwen_hip_vocab qwen_hip_vocab;
/* vocab.json (byte-level BPE string -> id); NULL on failure. */
qwen_hip_vocab *qwen_hip_vocab_load(const char *vocab_json_path);
void qwen_hip_vocab_free(qwen_hip_vocab *v);
/* max id + 1 */
int qwen_hip_vocab_size(const qwen_hip_vocab *v);
/* the bytes of one token ("" for ids absent from the file, as the reference) */
const char *qwen_hip_vocab_piece(const qwen_hip_vocab *v, int token_id);
/* Text of a generated token sequence as the reference's loop builds it:
 * stop at <|endoftext|> / <|im_end|>, emit pieces only after <asr_text>
 * (or from the start when past_asr_text != 0, the forced-language / carried-
 * text case).  Writes at most cap-1 bytes + NUL; returns the full length. */
long qwen_hip_vocab_transcript(const qwen_hip_vocab *v, const int *tokens, int n, int past_asr_text, char *out,
                               size_t cap);

/* ------------------------------------------------------------------------
 * Op-level ABI: the qwen_asr_kernels.h operators on device pointers.
 * Same argument order and meaning as the reference, plus a stream.
 * ------------------------------------------------------------------------ */

/* qwen_add_inplace (qwen_asr_kernels.h:18): a[i] += b[i] */
int qwen_hip_add_inplace(float *a, const float *b, int n, hipStream_t s);

/* qwen_rms_norm (qwen_asr_kernels.h:80): out = x * w / sqrt(mean(x^2)+eps);
 * out may equal x. */
int qwen_hip_rms_norm(float *out, const float *x, const float *w,
                      int seq_len, int hidden, float eps, hipStream_t s);

/* qwen_rms_norm_per_head (qwen_asr_kernels.h:86): in place per head_dim slice */
int qwen_hip_rms_norm_per_head(float *x, const float *w, int seq_len, int n_heads,
                               int head_dim, float eps, hipStream_t s);

/* qwen_apply_rope_neox (qwen_asr_kernels.h:151): in place, cos/sin [seq][head_dim] */
int qwen_hip_apply_rope_neox(float *x, const float *cos_vals, const float *sin_vals,
                             int seq_len, int n_heads, int head_dim, hipStream_t s);

/* qwen_swiglu_multiply (qwen_asr_kernels.h:97): out[s][j] = silu(gu[s][2j]) * gu[s][2j+1];
 * out may equal gate_up. */
int qwen_hip_swiglu_multiply(float *out, const float *gate_up, int seq_len,
                             int intermediate, hipStream_t s);

/* qwen_linear_nobias_bf16 (qwen_asr_kernels.h:41): y[seq][out] = x[seq][in] W^T.
 * seq_len == 1 runs the bandwidth-bound GEMV; seq_len > 1 the MFMA GEMM. */
int qwen_hip_linear_nobias_bf16(float *y, const float *x, const uint16_t *W_bf16,
                                int seq_len, int in_dim, int out_dim, hipStream_t s);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): the same product as qwen_hip_linear_nobias_bf16 with the same
 * kernels and results, but it never allocates or frees memory and never
 * synchronises; it only enqueues on s.  Its temporary memory is one fixed
 * per-GPU device array of qwen_hip_linear_noalloc_max_bytes() bytes (32 MiB),
 * held from library load to process exit.  A seq > 1 call needs 4*seq*in
 * bytes (the bf16 hi and lo halves of x, rounded up to 256), plus
 * 4*nsplit*seq*out bytes of split-K partials where the product splits K: only
 * products with fewer than 256 output tiles of 128 columns (32 rows for
 * seq <= 32, 64 up to 512 rows, 128 above) and an even out do, with nsplit at
 * most 16.  A call needing more than the array returns QWEN_HIP_EINVAL.  All
 * calls on one GPU share that array: calls whose kernels overlap in time on
 * one GPU race, so order them (one stream). */
int qwen_hip_linear_nobias_bf16_noalloc(float *y, const float *x, const uint16_t *W_bf16,
                                        int seq_len, int in_dim, int out_dim, hipStream_t s);
size_t qwen_hip_linear_noalloc_max_bytes(void);

/* qwen_linear_nobias_bf16_qkv (qwen_asr_kernels.h:45): the three seq=1 matvecs */
int qwen_hip_linear_nobias_bf16_qkv(float *q, float *k, float *v, const float *x,
                                    const uint16_t *Wq_bf16, const uint16_t *Wk_bf16,
                                    const uint16_t *Wv_bf16, int in_dim, int q_dim,
                                    int kv_dim, hipStream_t s);

/* qwen_causal_attention (qwen_asr_kernels.h:123): Q [seq_q][n_heads*hd],
 * K/V [seq_k][n_kv_heads*hd] (the reference's row layout), out like Q. */
int qwen_hip_causal_attention(float *out, const float *Q, const float *K, const float *V,
                              int seq_q, int seq_k, int n_heads, int n_kv_heads,
                              int head_dim, float scale, int q_offset, hipStream_t s);

/* qwen_argmax_matvec_bf16 (qwen_asr_kernels.h:156): index of the largest
 * W[o]·x, lowest index on exact ties.  Synchronous like the reference:
 * returns the index (>= 0) or a negative error code. */
int qwen_hip_argmax_matvec_bf16(const float *x, const uint16_t *W_bf16,
                                int in_dim, int out_dim, hipStream_t s);

#ifdef __cplusplus
}
#endif
#endif /* QWEN_ASR_HIP_H */
