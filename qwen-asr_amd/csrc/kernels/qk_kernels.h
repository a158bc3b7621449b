/*
 * qk_kernels.h - internal launcher interface between the C host code
 * (csrc/host, C) and the HIP kernels (csrc/kernels, .hip files).  Plain C structs
 * and functions; every launcher returns 0 or a negative QWEN_HIP_E* code and
 * only launches (never synchronises).
 */
#ifndef QK_KERNELS_H
#define QK_KERNELS_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bandwidth-bound GEMV (decode) ---------------------------------- */
enum { QK_EPI_STORE = 0, QK_EPI_ADD = 1, QK_EPI_SWIGLU = 2, QK_EPI_ARGMAX = 3 };

typedef struct {
    const uint16_t *W;        /* [rows][K] bf16 */
    int rows, K;
    const float *x;           /* [K] input row (unless gathered via tok) */
    const float *norm_w;      /* non-NULL: input is rms_norm(x) * norm_w */
    float eps;
    const int *tok;           /* non-NULL and *tok >= 0: x = emb[*tok] widened */
    const uint16_t *emb;      /* [vocab][K] bf16 for the gather */
    float *x_store;           /* gather mode: block 0 writes the gathered row */
    float *normed_store;      /* non-NULL: block 0 writes the (normed) input */
    float *y;                 /* STORE/ADD: [rows]; SWIGLU: [rows/2] */
    float *logits;            /* ARGMAX: optional [rows] */
    float *cand_val;          /* ARGMAX: per-block winners */
    int *cand_idx;
    int epi;
    /* merge prologue: the input row is the attention output merged from
     * merge_nsplit split partials (K = heads*128), unused slots holding
     * m = -inf; replaces x */
    const float *merge_o, *merge_m, *merge_l;
    int merge_nsplit;         /* split budget the partials were written with */
} qk_gemv_args;

#define QK_MERGE_MAX_SPLIT 8      /* merge prologue: at most this many splits */
#define QK_MERGE_MAX_K 2048       /* ... over an input row of at most this length */

int qk_gemv_launch(const qk_gemv_args *a, hipStream_t s);
/* number of blocks qk_gemv_launch uses (= candidates for ARGMAX) */
int qk_gemv_blocks(int rows, int K, int epi);

/* Reduce ARGMAX candidates: token = best; *tok_out = token (if non-NULL),
 * log[*counter] = token and ++*counter (if log non-NULL), ++*pos and
 * ++*epoch (each if non-NULL). */
int qk_argmax_finish_launch(const float *cand_val, const int *cand_idx, int n,
                            int *tok_out, int *log, int *counter, int *pos,
                            unsigned *epoch, hipStream_t s);

/* ---- q/k RMSNorm + NeoX RoPE + KV append ---------------------------- */
typedef struct {
    const float *qkv;         /* [S][q_dim + 2*kv_dim] raw projections, or nsum split-K */
    int nsum;                 /* partials pstride floats apart, summed in order (0: 1) */
    long pstride;
    const float *q_norm, *k_norm;
    float eps;
    const float *rope_cos, *rope_sin;   /* [cap][head_dim], indexed by position */
    float *k_cache, *v_cache; /* layer base, layout [kv_heads][cap][head_dim] */
    int cap;
    const int *pos_dev;       /* non-NULL: start position = *pos_dev */
    int start;                /* start position when pos_dev is NULL */
    int S, heads, kv_heads;
    float *q_out;             /* [S][q_dim] normed + rotated queries */
} qk_rope_append_args;

/* Every pointer 16-byte aligned and pstride a multiple of 4 when nsum > 1
 * (the kernel's accesses are 16-byte vectors); QWEN_HIP_EINVAL otherwise. */
int qk_rope_append_launch(const qk_rope_append_args *a, hipStream_t s);

/* ---- causal GQA attention -------------------------------------------- */
typedef struct {
    const float *q;           /* [seq_q][heads*head_dim] */
    const float *k, *v;       /* element (pos, kvh, d) at base + pos*pos_stride + kvh*head_stride + d */
    long pos_stride, head_stride;
    const int *pos_dev;       /* decode: seq_k = *pos_dev + 1 */
    int seq_k;                /* decode without pos_dev / prefill: keys [0, seq_k) */
    int seq_q, q_offset;      /* prefill: query i sees keys j <= q_offset + i */
    int heads, kv_heads;
    float scale;
    float *part;              /* decode: split partials [heads][nsplit][head_dim+2];
                                 prefill: [nsplit][seq_q][heads][QK_PF_PART] */
    int nsplit;
    int chunk;                /* prefill: keys per split (multiple of 32) */
    float *out;               /* fp32 [seq_q][heads*head_dim] */
    uint16_t *out_hi, *out_lo;/* prefill alternative: bf16 hi/lo split of out */
} qk_attn_args;

int qk_attn_decode_launch(const qk_attn_args *a, hipStream_t s);

/* Prefill attention (fp32 MFMA, heads == 2 * kv_heads, head_dim 128): the
 * key range of each 64-query tile is cut into splits of `chunk` keys; with
 * nsplit > 1 the splits write partials to `part` and a merge kernel follows.
 * qk_attn_prefill_plan picks chunk/nsplit for a launch of about
 * QK_PF_TARGET blocks and returns the partial buffer size in floats (0 when
 * nsplit == 1). */
#define QK_PF_PART 130              /* o[128], m, l */
#define QK_PF_TARGET 768
size_t qk_attn_prefill_plan(int seq_q, int seq_k, int q_offset, int heads, int kv_heads, int *chunk, int *nsplit);
int qk_attn_prefill_launch(const qk_attn_args *a, hipStream_t s);

/* ---- fused decode attention (one kernel per layer) -------------------- */
/* q/k RMSNorm + RoPE + K/V append + split attention.  Positions [0, pos]
 * are cut into nsplit' = ceil((pos+1)/chunk) splits of
 * chunk = max(QK_ATTN_MIN_CHUNK, ceil((pos+1)/nsplit)); each split writes the
 * unnormalised partials (m, l, o[head_dim]) of its query heads.  With a
 * single split the result goes straight to `out`.  The merge is
 * qk_attn_merge_launch or the O-projection GEMV prologue (QK_PRO_MERGE). */
#define QK_ATTN_MIN_CHUNK 64
#define QK_ATTN_MAX_SPLIT 32
#ifdef __cplusplus
__host__ __device__
#endif
static inline int qk_attn_chunk(int seq_k, int nsplit) {
    int c = (seq_k + nsplit - 1) / nsplit;
    return c < QK_ATTN_MIN_CHUNK ? QK_ATTN_MIN_CHUNK : c;
}

typedef struct {
    const float *qkv;                  /* raw [q_dim + 2*kv_dim] */
    const float *q_norm, *k_norm;
    float eps;
    const float *rope_cos, *rope_sin;  /* [cap][head_dim] */
    float *k_cache, *v_cache;          /* layer base [kv_heads][cap][head_dim] */
    int cap;
    const int *pos_dev;                /* position of this step (= kv_len) */
    int heads, kv_heads;
    float scale;
    float *part_o;                     /* [heads][nsplit][head_dim] */
    float *part_m, *part_l;            /* [heads][nsplit] */
    int nsplit;                        /* split budget (<= QK_ATTN_MAX_SPLIT) */
    float *out;                        /* [heads*head_dim] (single split / merge) */
} qk_attn_fused_args;

int qk_attn_fused_launch(const qk_attn_fused_args *a, hipStream_t s);
int qk_attn_merge_launch(const qk_attn_fused_args *a, hipStream_t s);

/* ---- persistent decode (the whole greedy loop in one launch) ----------- */
/* One block per CU, 8 XCDs x 32 CUs; XCD g owns kv head g.  Blocks exchange
 * activations through 64-bit words carrying (tag << 32 | fp32 bits): XCD-local
 * words go through the XCD's L2, cross-XCD words through memory-side coherent
 * accesses.  Word counts below are per buffer. */
#define QK_PX_XCD 8
#define QK_PX_LOC 32
#define QK_PX_BLOCKS (QK_PX_XCD * QK_PX_LOC)
#define QK_PX_MAX_SPLIT 32                 /* attention splits per kv head (one per CU) */
#define QK_PX_PART 260                     /* words per split: 2 heads x (m, l, o[128]) */
#define QK_PX_MIN_CHUNK 64                 /* positions per split, at least */
#define QK_PX_TPL 8                        /* exchange tags per layer */
enum { QK_PX_ERR_LAYOUT = 1, QK_PX_ERR_TIMEOUT = 2 };

typedef struct {
    /* layer l tensors live at layer0 + l * layer_stride + off_* (bytes) */
    const char *layer0;
    long layer_stride;
    long off_qkv, off_o, off_gu, off_down, off_nin, off_npost, off_nq, off_nk;
    const uint16_t *emb;       /* [vocab][hidden] tied embedding / LM head */
    const float *fnorm;
    float *k_cache, *v_cache;  /* [layer][kv_head][cap][128] */
    int cap;
    const float *rope_cos, *rope_sin;
    int layers, vocab;
    float eps, scale;
    /* exchange buffers (zero-initialised; each [2 parities][8 XCDs][...]) */
    unsigned long long *xq;    /* [2][8][512]  q|q|k|v of the group */
    unsigned long long *xa;    /* [2][8][32][QK_PX_PART] attention split partials */
    unsigned long long *xm;    /* [2][8][256] merged attention output of the group (2 heads x 128) */
    unsigned long long *xo;    /* [2][8][hidden] O-projection split-K partials (cross-XCD) */
    unsigned long long *xla;   /* [2][8][hidden] residual after attention (XCD-local copy) */
    unsigned long long *xh;    /* [2][8][inter/8] SwiGLU outputs of the group */
    unsigned long long *xd;    /* [2][8][hidden] down-projection split-K partials (cross-XCD) */
    unsigned long long *xlb;   /* [2][8][hidden] residual after the MLP (XCD-local copy) */
    unsigned long long *xc;    /* [256][2] LM-head argmax candidates (cross-XCD) */
    unsigned long long *xv;    /* [256] launch check-in words */
    unsigned *cnt;             /* [16] per-XCD tickets, zeroed before every launch */
    unsigned *err;             /* QK_PX_ERR_* bits, zeroed before every launch */
    unsigned epoch;            /* first tag of this launch (>= 1) */
    unsigned long long wait_ticks; /* bound of every wait, in ticks of the device wall clock */
    unsigned long long checkin_ticks; /* bound of the launch check-in wait (<= wait_ticks): every
                                         block of the grid must have started within it */
    /* the steps */
    int pos0, n_steps;
    int first_tok;             /* >= 0: step 0 input is emb[first_tok] */
    const float *x_in;         /* first_tok < 0: step 0 input row [hidden] */
    int *log;                  /* [n_steps] greedy tokens */
    int *tok_out;              /* last token */
    int *pos_out;              /* position after the last step (= pos0 + n_steps) */
    float *hidden_out;         /* final-normed hidden row of each step */
    float *logits;             /* optional [vocab] logits of each step */
    unsigned long long *trace; /* optional [256][QK_PX_TRACE] wall-clock stamps of step trace_step */
    int trace_step;
} qk_persist_args;

/* Trace points per block (100 MHz wall clock).  Sync wave, per layer l at
 * 10*l + {0: Q entered (previous compute done), 1: Q input ready, 2: A entered,
 * 3: A input ready, 4: O entered, 5: O input ready, 6: F entered, 7: F input
 * ready, 8: D entered, 9: D input ready}; then 10*L + {0: LM entered, 1: LM
 * input ready, 2: token reduce entered, 3: token ready}.  Compute wave 0 at
 * QK_PX_TRACE_CW + 10*l + {0: Q dot done, 1: Q stores + prefetch issued,
 * 2: q/k norm done, 3: fold done, 4: split merged + stored, 5: O splits merged,
 * 6: O dot done, 7: O stores + prefetch issued, 8: F dot done, 9: D dot done}.
 * Sync wave again at QK_PX_TRACE_XU + 2*l + {0: cross-XCD half of the residual
 * update before Q done, 1: the same before F}, and 2*L for the final one. */
#define QK_PX_TRACE_CW 320
#define QK_PX_TRACE_XU 640
#define QK_PX_TRACE 704

/* tags one launch of n steps consumes (the host advances epoch by this) */
#define QK_PX_TAGS(layers, n) (1u + (unsigned)(n) * (QK_PX_TPL * (unsigned)(layers) + 1u))

/* 1 if the persistent engine supports this shape on this device */
int qk_persist_supported(int hidden, int inter, int heads, int kv_heads, int device);
int qk_persist_launch(const qk_persist_args *a, int hidden, int inter, hipStream_t s);

/* ---- relay decode (0.6B shape): two teams of CUs take the layers in turn --
 * Blocks of XCD g with ticket rank r < 16 form team 0 (even layers), the
 * others team 1 (odd layers).  A team computes its layer from weights already
 * held in registers while the other team streams the next layer's weights
 * (and its K/V rows) from HBM, so no hand-over of the computing team waits
 * behind weight loads of its own CU.  Weights come pre-tiled (qk_relay_pack):
 * per layer, per (XCD, team rank, wave) QK_RL_TILES tiles of 1 KB, each the
 * B operand of one v_mfma_f32_16x16x32_bf16 (16 rows x 32 columns; lane l
 * holds row l % 16, columns 8 (l / 16) .. + 8). */
#define QK_RL_TEAM 16                      /* blocks of one team on one XCD */
#define QK_RL_WAVES 4                      /* waves per block (one per SIMD) */
#define QK_RL_TILES 60                     /* weight tiles per wave per layer */
#define QK_RL_TILE_BYTES 1024
#define QK_RL_KVP 64                       /* cached positions per split (held in LDS) */
#define QK_RL_MIN_CHUNK 16                 /* positions per split, at least */
#define QK_RL_MAX_SEQ (QK_RL_TEAM * QK_RL_KVP) /* the kernel attends over at most this many keys */
#define QK_RL_TPL 8                        /* exchange tags per layer */
#define QK_RL_PART 260                     /* words per split: 2 heads x (m, l, o[128]) */
#define QK_RL_TRACE 704                    /* trace words per block */
#define QK_RL_LINE 16                      /* words per cross-XCD single-word slot (one 128-byte line) */
/* bytes of one layer's tiled weights */
#define QK_RL_LAYER_BYTES ((long)QK_PX_XCD * QK_RL_TEAM * QK_RL_WAVES * QK_RL_TILES * QK_RL_TILE_BYTES)

typedef struct {
    const char *wt;            /* tiled weights, QK_RL_LAYER_BYTES per layer */
    /* norms of layer l at layer0 + l * layer_stride + off_* (bytes) */
    const char *layer0;
    long layer_stride;
    long off_nin, off_npost, off_nq, off_nk;
    const uint16_t *emb;       /* [vocab][1024] tied embedding / LM head */
    const float *fnorm;
    float *k_cache, *v_cache;  /* [layer][kv_head][cap][128] */
    int cap;
    const float *rope_cos, *rope_sin;
    int layers, vocab;
    float eps, scale;
    /* exchange words (zero-initialised); [2 teams][8 XCDs][...] unless noted */
    unsigned long long *xq;    /* [2][8][512] q|q|k|v of the group */
    unsigned long long *xa;    /* [2][8][16][QK_RL_PART] attention split partials */
    unsigned long long *xm;    /* [2][8][256] merged attention output of the group */
    unsigned long long *xo;    /* [2][8][1024] O-projection split-K partials (cross-XCD) */
    unsigned long long *xla;   /* [2][8][1024] residual after attention, republished */
    unsigned long long *xh;    /* [2][8][384] SwiGLU outputs of the group */
    unsigned long long *xd;    /* [2][8][1024] down-projection split-K partials (cross-XCD) */
    unsigned long long *xs;    /* [2][8][1024] residual after attention, slices for the next team */
    unsigned long long *xlb;   /* [2][8][1024] input residual of a layer, republished */
    unsigned long long *xc;    /* [256][QK_RL_LINE] LM-head candidates (value, index) */
    unsigned long long *xv;    /* [256][QK_RL_LINE] launch check-in words */
    unsigned *cnt;             /* [16] per-XCD tickets, zeroed before every launch */
    unsigned *err;             /* QK_PX_ERR_* bits, zeroed before every launch */
    unsigned epoch;            /* first tag of this launch (>= 1) */
    unsigned long long wait_ticks;
    unsigned long long checkin_ticks; /* bound of the launch check-in wait (<= wait_ticks) */
    int pos0, n_steps;
    int first_tok;             /* >= 0: step 0 input is emb[first_tok] */
    const float *x_in;         /* first_tok < 0: step 0 input row [1024] */
    int *log, *tok_out, *pos_out;
    float *hidden_out, *logits;
    unsigned long long *trace; /* optional [256][QK_RL_TRACE] stamps of step trace_step */
    int trace_step;
} qk_relay_args;

/* Trace points per block (100 MHz wall clock), written by wave 0 for the
 * block's own layers l at 24*l + {0: input wait entered, 1: cross-XCD half of
 * the input residual in, 2: wave 0's quarter of the input residual gathered (planes of x*w written; the product's barrier follows),
 * 3: = 2, 4: Q stored, 5: q|k|v gathered, 6: attention entered, 7: fold done,
 * 8: split partials stored, 9: merge slices in, 10: merged dims stored,
 * 11: merged output gathered, 12: O stored, 13: cross-XCD half of the
 * post-attention residual in, 14: wave 0's quarter of the post-attention residual gathered, 15: = 14,
 * 16: gate|up products reduced, 17: SwiGLU stored, 18: SwiGLU outputs
 * gathered, 19: down stored, 20: next layer's loads issued}; and at
 * 24*layers + {0: LM entered, 1: final residual cross half in, 2: final
 * residual gathered, 3: candidate stored, 4: token ready (team 0)}. */

/* tags one launch of n steps consumes */
#define QK_RL_TAGS(layers, n) (1u + (unsigned)(n) * (QK_RL_TPL * ((unsigned)(layers) + 1u)))

int qk_relay_supported(int hidden, int inter, int heads, int kv_heads, int device);
int qk_relay_launch(const qk_relay_args *a, hipStream_t s);
/* Tile layer l's row-major weights (stacked Wqkv, W_o, interleaved gate|up,
 * W_down; 0.6B shape) into dst (QK_RL_LAYER_BYTES). */
int qk_relay_pack(char *dst, const uint16_t *wqkv, const uint16_t *wo, const uint16_t *wgu, const uint16_t *wdown,
                  hipStream_t s);

/* ---- prefill (MFMA) ---------------------------------------------------- */
/* Optionally x += part[0] + ... + part[nsum-1] (rows of pstride floats apart,
 * in place, split order), then hi/lo = bf16 split of rms_norm(x)*w (w NULL:
 * of x itself): hi = bf16(v), lo = bf16(v - hi), so hi + lo carries v to
 * ~2^-17 relative.  hi/lo NULL: only the sum. */
int qk_rmsnorm_split_launch(float *x, const float *part, int nsum, long pstride, const float *w, int S, int D,
                            float eps, uint16_t *hi, uint16_t *lo, hipStream_t s);

enum { QK_GEMM_STORE = 0, QK_GEMM_ADD = 1, QK_GEMM_SWIGLU = 2, QK_GEMM_ROPE = 3 /* plans only */ };
/* Tiling of one M x N x K product: block rows bm x columns bn (32 / 64 x
 * QK_GEMM_BN on the LDS ring of nst stages, 128 x QK_GEMM_BN on a 3-stage
 * ring for STORE and SwiGLU products above 512 rows, 32 / 64 / 128 x
 * QK_GEMM_BN register-staged (nst 0), or 128 / 256 x 256 for large M), and
 * nsplit slices of kc (a multiple of 64) along K so a launch has enough
 * blocks.  Split rule on the ring: about QK_GEMM_RING_TARGET blocks, and two
 * splits at least for k walks of QK_GEMM_RING_KSPLIT or more; a STORE product
 * on the 128 x 128 tiles takes two splits per 4096 of K whatever its grid; a
 * SwiGLU product and a Q|K|V product with the RoPE epilogue split only to
 * fill the chip.  The op-level linear (qwen_hip_linear_nobias_bf16) keeps one
 * split where its output tiles alone number QK_GEMM_TARGET or more. */
#define QK_GEMM_BN 128
#define QK_GEMM_TARGET 256
#define QK_GEMM_MAX_SPLIT 16
#define QK_GEMM_RING_NST 4           /* 64 KB of LDS at 64 x 128: two blocks per CU */
#define QK_GEMM_RING_TARGET 224      /* blocks a ring launch aims for */
#define QK_GEMM_RING_KSPLIT 2048     /* ring k walks this long or longer: two splits at least */
typedef struct { int bm, nsplit, kc, bn, nst; } qk_gemm_plan;
void qk_gemm_plan_for(int M, int N, int K, qk_gemm_plan *p);
/* the plan for a product with epilogue epi: a SWIGLU product splits K only
 * to fill the chip (its split partials need a reduce pass), and so does a
 * ROPE one (the Q|K|V product of qk_gemm_rope_launch) */
void qk_gemm_plan_epi(int M, int N, int K, int epi, qk_gemm_plan *p);
/* Y[M][N] (=, +=) (A_hi + A_lo)[M][K] . W[N][K]^T on bf16 MFMA with fp32
 * accumulation; SWIGLU writes silu(Y[:,2j]) * Y[:,2j+1] as a bf16 hi/lo
 * split [M][N/2] into out_hi/out_lo.  With nsplit > 1 only STORE is allowed
 * and y is [nsplit][M][N]: split z's partial product at y + z M N. */
int qk_gemm_launch(const uint16_t *a_hi, const uint16_t *a_lo, const uint16_t *W, int M, int N, int K,
                   const qk_gemm_plan *p, int epi, float *y, uint16_t *out_hi, uint16_t *out_lo, hipStream_t s);
/* Sum nsum partials [nsum][M][N] in order and apply epi (N even). */
int qk_gemm_reduce_launch(const float *part, int nsum, int M, int N, int epi, float *y, uint16_t *out_hi,
                          uint16_t *out_lo, hipStream_t s);
/* Q|K|V product (A hi/lo [M][K] . W[(heads + 2 kv_heads) 128][K]^T) with
 * rope_append's work as its epilogue (qkv / nsum unused, pos_dev NULL, S ==
 * M, the other pointers 16-byte aligned): bit for bit qk_gemm_launch(STORE)
 * + qk_rope_append_launch.  Only for plans with qk_gemm_rope_fusable (64 x
 * 128 ring tiles, one split). */
int qk_gemm_rope_fusable(const qk_gemm_plan *p);
int qk_gemm_rope_launch(const uint16_t *a_hi, const uint16_t *a_lo, const uint16_t *W, int M, int K,
                        const qk_gemm_plan *p, const qk_rope_append_args *ra, hipStream_t s);
/* y[S][out] = x[S][in] . W[out][in]^T for S > 1 (the op-level linear's
 * product path, csrc/host/ops.c): split x to bf16 hi/lo, GEMM, split-K reduce,
 * all launched on s with ws (>= qk_linear_ws_bytes bytes) as the only
 * temporary memory. */
size_t qk_linear_ws_bytes(int S, int in_dim, int out_dim);
int qk_linear_gemm(float *y, const float *x, const uint16_t *W, int S, int in_dim, int out_dim, void *ws,
                   hipStream_t s);

/* ---- audio encoder (fp32 matrix cores) --------------------------------- */
/* C[M][N] (=, +=) A[M][K] . B[N][K]^T (+ bias_m[m] | bias_n[n]) (+ pe[m % pe_rows][n])
 * (GELU); K and the leading dimensions multiples of 4.  col_w > 0: stem
 * output, column n (row m when pad_rows) = (chunk, oh, ow) with col_h x col_w
 * per chunk; the last chunk's positions with ow >= col_valid are written as
 * 0.  conv_c > 0 (with B16 only): A is read as the implicit im2col of a 3x3,
 * stride 2, pad 1 convolution over channel-last activations
 * [chunk][conv_in_h][conv_in_w][conv_c]: row m = (chunk, oh, ow) of
 * col_h x col_w per chunk, column k = tap * conv_c + ic, 0 outside the
 * input; K = 9 conv_c, conv_c a multiple of 32, lda unused.  ws: optional
 * workspace of ws_elems floats; when the tile grid is too small to fill the
 * chip, K is split over up to 8 slices whose raw partials go to ws and are
 * summed in slice order by a second kernel that applies the epilogue
 * (deterministic).  kc / split are set by the launcher. */
typedef struct {
    const float *A, *B;
    float *C;
    int M, N, K, lda, ldb, ldc;
    const float *bias_m, *bias_n, *pe;
    int pe_rows, gelu, add;
    int col_w, col_h, col_chunks, col_valid, pad_rows;
    int conv_c, conv_in_h, conv_in_w;
    float *ws;
    long ws_elems;
    int kc, split;
    /* bf16 weights (exact copies of bf16-valued fp32 weights): when A16 (A side)
     * or B16 (B side) is set it replaces that operand, and the product runs on
     * the bf16 matrix cores with the other, fp32, operand split hi + lo (two
     * MFMAs per product, ~2^-17 relative per product); K and the bf16
     * operand's leading dimension must be multiples of 32 and 8. */
    const uint16_t *A16, *B16;
    /* optional LayerNorm of the finished rows of C into ln_out (weights ln_w,
     * ln_b, eps ln_eps): done in the split-K reduce when there is one (N <=
     * 1024), else by a LayerNorm pass after the product */
    const float *ln_w, *ln_b;
    float *ln_out;
    float ln_eps;
} qk_enc_gemm_args;
#define QK_ENC_GEMM_WS_ELEMS (2048L * 64 * 64)  /* split * M * N <= (1024 + tiles) * 4096 for every split the launcher picks */
int qk_enc_gemm_launch(const qk_enc_gemm_args *a, hipStream_t s);
int qk_enc_im2col_launch(const float *in, float *cols, int c_in, int chunks, int h_in, int w_in, int h_out,
                         int w_out, int kpad, int mel_frames, hipStream_t s);
/* conv1 from its im2col patches cols[rows][kpad] (taps 0..8) and weights
 * w[ch][kpad]: channel-last out[rows][ch] with bias, GELU and the last
 * chunk's padding positions zeroed */
int qk_enc_conv1_launch(const float *cols, int kpad, const float *w, const float *b, float *out, int rows, int ch,
                        int h_out, int w_out, int chunks, int valid, hipStream_t s);
int qk_enc_stem_rows_launch(const float *c3, float *rows, int chunks, int w, int h, int ch_n, int tokens,
                            hipStream_t s);
int qk_enc_layernorm_launch(const float *x, const float *w, const float *b, float *out, int rows, int D, float eps,
                            hipStream_t s);
int qk_enc_attention_launch(const float *qkv, float *out, int T, int H, int hd, int win, float scale, hipStream_t s);

/* ---- elementwise (op-level ABI) --------------------------------------- */
int qk_add_launch(float *a, const float *b, long n, hipStream_t s);
int qk_rms_norm_launch(float *out, const float *x, const float *w, int S, int D,
                       float eps, hipStream_t s);
int qk_rms_norm_per_head_launch(float *x, const float *w, int S, int nh, int hd,
                                float eps, hipStream_t s);
int qk_rope_launch(float *x, const float *cos_v, const float *sin_v, int S, int nh,
                   int hd, hipStream_t s);
int qk_swiglu_launch(float *out, const float *gate_up, int S, int inter, hipStream_t s);
int qk_split_bf16_launch(const float *x, long n, uint16_t *hi, uint16_t *lo, hipStream_t s);

#ifdef __cplusplus
}
#endif
#endif
