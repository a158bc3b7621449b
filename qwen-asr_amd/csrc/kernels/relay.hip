// relay.hip - the greedy decode loop of the 0.6B Qwen3 decoder as ONE
// persistent kernel in which two teams of CUs take the layers in turn:
// qwen_decoder_forward (reference qwen_asr_decoder.c:388-476) repeated by the
// token loop (qwen_asr.c:729-759), n steps per launch.
//
// Why two teams.  A decode step is a chain of dependent hand-overs between
// CUs (about 8 per layer); a hand-over is one or two round trips through the
// L2 or the memory side, and it is fast only on a CU whose own memory pipeline
// is quiet: a poll issued behind a CU's outstanding weight loads waits for
// them.  So the 32 CUs of each XCD split into two teams of 16.  Team 0 owns
// the even layers, team 1 the odd ones.  While one team computes layer l from
// weights it already holds in registers (and K/V rows it already holds in
// LDS), the other team streams layer l+1's weights and K/V rows from HBM.
// The computing team's CUs then issue nothing but hand-over traffic.
//
// Work layout (MI355X: 8 XCDs x 32 CUs, one block of 4 waves per CU, one
// wave per SIMD so each wave has 512 registers: the weights sit in 240 of
// them).  On XCD g a team owns kv head g with query heads 2g, 2g+1, 1/8 of the
// MLP rows and the matching split-K column slices of W_o and W_down; team
// rank q (0..15) holds 32 Q|K|V rows, 64 O rows x 256 columns, 48 gate|up rows
// and 64 down rows x 384 columns, 240 KB per layer, as 60 MFMA tiles per wave.
//
//   in  x = x' + sum of the previous layer's 8 down partials (its team's
//       slice q, cross-XCD), republished and gathered in the XCD; rms_norm
//   Q   32 Wqkv rows                                                -> local
//   A   q/k norm + RoPE + K/V append + attention over a position split
//   M   rank q merges 16 of the group's 256 attention dims           -> local
//   O   64 W_o rows over the group's columns                         -> cross
//   F   x' = x + sum of O partials (slice q, cross-XCD), republished;
//       rms_norm; 48 gate|up rows + SwiGLU                           -> local
//   D   64 W_down rows over the group's columns                      -> cross
//   LM  both teams: final residual, rms_norm, LM-head rows, argmax candidate
//   T   team 0: argmax over the 256 candidates, embedding of the token
//
// The products run on v_mfma_f32_16x16x32_bf16 with the weights as the B
// operand (16 rows x 32 columns per tile) and the fp32 activation split into
// three bf16 terms hi + mid + lo (exactly the fp32 value: 3 x 8 significant
// bits) as three A rows, so every product is exact and sums are fp32: the
// arithmetic of qwen_linear_nobias_bf16 (qwen_asr_kernels.c:462-472).
//
// Exchange words are 64-bit (tag << 32) | fp32 bits; a reader polls until
// each word carries the expected tag.  XCD-local words: plain stores (they
// land in the XCD's L2), agent-scope loads.  Cross-XCD words: agent-scope
// stores and loads, each producer's words on cache lines of its own.  Every
// wait is bounded in wall-clock time and also gives up when another block
// raised an error, so every wave reaches the end of the kernel.
#include "common.h"
#include "qk_kernels.h"
#include "qwen_asr_hip.h"

#include <math.h>

typedef unsigned long long u64;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

#define RL_H 1024
#define RL_I 3072
#define RL_XCD QK_PX_XCD
#define RL_NW QK_RL_WAVES
#define RL_HG (RL_I / RL_XCD)       // 384 SwiGLU outputs per XCD
#define RL_SO (RL_H / QK_RL_TEAM)   // 64 O / down rows per block
#define RL_NG 8                     // 32-lane attention groups (two per wave)
#define RL_TM 24                    // trace stamps per layer
static_assert(QK_RL_TRACE <= QK_PX_TRACE, "the two persistent kernels share one trace buffer");

static_assert(QK_RL_TEAM == 16 && RL_NW == 4 && QK_RL_TILES == 60, "layout constants");
static_assert(4 * 2 * RL_NG == QK_RL_KVP, "the fold's 4 batches of 2 positions per group cover a split's LDS rows");
static_assert(QK_RL_KVP * QK_RL_TEAM >= QK_RL_MAX_SEQ && QK_RL_MAX_SEQ == QWEN_HIP_RELAY_MAX_POS, "split capacity");

// ---------------------------------------------------------------------------
// exchange words
// ---------------------------------------------------------------------------
__device__ __forceinline__ u64 rl_word(float v, unsigned tag) { return ((u64)tag << 32) | __float_as_uint(v); }

__device__ __forceinline__ void rl_put_local(u64 *p, float v, unsigned tag) {
    __hip_atomic_store(p, rl_word(v, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}

__device__ __forceinline__ void rl_put_global(u64 *p, float v, unsigned tag) {
    __hip_atomic_store(p, rl_word(v, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ u64 rl_get(const u64 *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool rl_aborted(unsigned *err) {
    const unsigned e = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_amdgcn_readfirstlane(e) != 0u;
}

__device__ __forceinline__ void rl_raise(unsigned *err, unsigned bits) {
    __hip_atomic_fetch_or(err, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block barrier; this wave's LDS accesses are complete before it.  Global
// loads (the next layer's weights) stay in flight across it.
__device__ __forceinline__ void rl_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Wait for every load and store this wave issued.
__device__ __forceinline__ void rl_wait_vm() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// This wave waits until the words i in [i0, i1) (at most 64 * PER of them) at
// base + idx(i) carry `tag`, then calls put(i, value) for each.  False when
// the wait passed a.wait_ticks (QK_PX_ERR_TIMEOUT raised) or another block
// raised an error.  The clock is read while the pass's loads are in flight.
// The lane index is opaque to the optimiser, so no per-lane address of a poll
// is hoisted out of the layer loop (that would hold ~2 VGPRs per word for the
// whole kernel).  CHECKIN: the bound is a.checkin_ticks.
template <int PER, bool CHECKIN = false, typename Idx, typename Put>
__device__ __forceinline__ bool rl_poll(const qk_relay_args &a, const u64 *base, Idx idx, int i0, int i1, unsigned tag,
                                        Put put, int lane) {
    if (i1 <= i0) return true;
    int ln = lane;
    asm volatile("" : "+v"(ln));
    unsigned off[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = i0 + j * 64 + ln;
        off[j] = (unsigned)idx(i < i1 ? i : i0);
    }
    const u64 t0 = wall_clock64();
    for (unsigned spin = 1;; spin++) {
        u64 w[PER];
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int i = i0 + j * 64 + ln;
            w[j] = (i < i1) ? rl_get(base + off[j]) : ((u64)tag << 32);
        }
        const u64 now = wall_clock64();
        bool ok = true;
#pragma unroll
        for (int j = 0; j < PER; j++) ok = ok && ((unsigned)(w[j] >> 32) == tag);
        if (__all(ok)) {
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const int i = i0 + j * 64 + ln;
                if (i < i1) put(i, __uint_as_float((unsigned)w[j]));
            }
            return true;
        }
        if (now - t0 > (CHECKIN ? a.checkin_ticks : a.wait_ticks)) {
            if (lane == 0) rl_raise(a.err, QK_PX_ERR_TIMEOUT);
            return false;
        }
        if ((spin & 15u) == 0u && rl_aborted(a.err)) return false;
    }
}

// rl_poll over a contiguous range of exactly 64 * PER words with lane ln
// owning words [i0 + PER ln, + PER): on success v[j] holds word i0 + PER ln + j.
template <int PER>
__device__ __forceinline__ bool rl_poll_vec(const qk_relay_args &a, const u64 *base, int i0, unsigned tag,
                                            float (&v)[PER], int lane) {
    return rl_poll<PER>(
        a, base, [&](int i) { const int k = i - i0; return i0 + PER * (k & 63) + (k >> 6); }, i0, i0 + 64 * PER, tag,
        [&](int i, float x) { v[(i - i0) >> 6] = x; }, lane);
}

// ---------------------------------------------------------------------------
// weights and products
// ---------------------------------------------------------------------------
// One wave's tiles of one layer: Q (row tile w & 1, k tiles 16 (w >> 1) ..),
// O (row tile w, all 8 k tiles), F (row tiles 0..2, k tiles 8w ..), D (row
// tile w, all 12 k tiles).  Tile order in memory: q[0..16), o[0..8),
// f[0..24) (row tile major), d[0..12).
struct RlW {
    u32x4 q[16], o[8], f[24], d[12];
};

__device__ __forceinline__ u32x4 rl_ld16(const char *base, unsigned off) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + off));
}

// Tile i of the wave's 60 straight into accumulation registers (AGPRs): the
// weights then never compete with the working set for VGPRs, and the matrix
// cores read their B operand from them directly.  The compiler does not see
// these loads: every use sits behind an explicit wait for this wave's loads.
// The address is a 64-bit VGPR (no SGPR operand): the compiler's hazard
// checks do not look inside inline asm, and an SGPR base it had just reloaded
// with v_readlane would need 5 wait states before a memory instruction reads
// it; a VGPR address written by a VALU op needs none.
template <int I>
__device__ __forceinline__ u32x4 rl_ld_tile(const char *lane_base) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off offset:%2 nt"
                 : "=a"(v)
                 : "v"(lane_base + (I / 4) * 4096), "i"((I % 4) * 1024)
                 : "memory");
    return v;
}

template <int I, int N>
__device__ __forceinline__ void rl_ld_tiles(u32x4 *dst, const char *lane_base) {
    if constexpr (N > 0) {
        dst[0] = rl_ld_tile<I>(lane_base);
        rl_ld_tiles<I + 1, N - 1>(dst + 1, lane_base);
    }
}

__device__ __forceinline__ void rl_load_w(RlW &w, const char *base, int lane) {
    unsigned off = (unsigned)lane * 16u;
    asm volatile("" : "+v"(off));   // recomputed per call: no per-lane 64-bit bases held across the loops
    const char *lb = base + off;
    rl_ld_tiles<0, 16>(w.q, lb);
    rl_ld_tiles<16, 8>(w.o, lb);
    rl_ld_tiles<24, 24>(w.f, lb);
    rl_ld_tiles<48, 12>(w.d, lb);
}

__device__ __forceinline__ f32x4 rl_mfma(bf16x8 act, u32x4 wt, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(act, __builtin_bit_cast(bf16x8, wt), c, 0, 0, 0);
}

// Planes of an activation vector of K elements: hi, mid, lo, zeros, each
// padded by 64 bytes so the four planes start in different LDS banks and one
// fragment read (16 distinct 16-byte chunks) is conflict-free.
template <int K>
struct RlPlanes {
    static constexpr int STRIDE = K + 32;
    uint16_t v[4][STRIDE];
};

// A operand of k tile kt: lane l holds plane min(l % 16, 3) at columns
// 32 kt + 8 (l / 16) .. + 8.
template <int K>
__device__ __forceinline__ bf16x8 rl_afrag(const RlPlanes<K> &P, int kt, int lane) {
    const int p = min(lane & 15, 3);
    return *reinterpret_cast<const bf16x8 *>(&P.v[p][32 * kt + 8 * (lane >> 4)]);
}

// The 16 rows of one tile's product in lanes 0..15: hi + mid + lo terms.
__device__ __forceinline__ float rl_rowsum(f32x4 c) { return (c[0] + c[1]) + c[2]; }

// v = hi + mid + lo exactly: hi and mid truncated to bf16; lo, the rest, has
// at most 8 significant bits (v's 24 less the 8 of hi and of mid), so its
// bf16 truncation is exact too (v in the normal range).
__device__ __forceinline__ void rl_split3(float v, unsigned &h, unsigned &m, unsigned &l) {
    const unsigned hb = __float_as_uint(v) & 0xffff0000u;
    const float r1 = v - __uint_as_float(hb);
    const unsigned mb = __float_as_uint(r1) & 0xffff0000u;
    const float r2 = r1 - __uint_as_float(mb);
    h = hb >> 16;
    m = mb >> 16;
    l = __float_as_uint(r2) >> 16;
}

// planes P at element i of value v
template <int K>
__device__ __forceinline__ void rl_plane1(RlPlanes<K> &P, int i, float v) {
    unsigned h, m, l;
    rl_split3(v, h, m, l);
    P.v[0][i] = (uint16_t)h;
    P.v[1][i] = (uint16_t)m;
    P.v[2][i] = (uint16_t)l;
}

// planes P at elements i, i + 1 (i even)
template <int K>
__device__ __forceinline__ void rl_plane2(RlPlanes<K> &P, int i, float v0, float v1) {
    unsigned h0, m0, l0, h1, m1, l1;
    rl_split3(v0, h0, m0, l0);
    rl_split3(v1, h1, m1, l1);
    *reinterpret_cast<unsigned *>(&P.v[0][i]) = h0 | (h1 << 16);
    *reinterpret_cast<unsigned *>(&P.v[1][i]) = m0 | (m1 << 16);
    *reinterpret_cast<unsigned *>(&P.v[2][i]) = l0 | (l1 << 16);
}

// ---------------------------------------------------------------------------
// attention helpers
// ---------------------------------------------------------------------------
// online-softmax fold of one key/value position into the lane's query head
// (qwen_causal_attention_heads, qwen_asr_kernels.c:1073-1089)
__device__ __forceinline__ void rl_fold1(const float (&q)[8], float4 k0, float4 k1, float4 v0, float4 v1, float scale,
                                         float &m, float &l, float (&o)[8]) {
    const float kv[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float d = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) d = fmaf(q[j], kv[j], d);
    d = group_sum<16>(d);
    const float sc = d * scale;
    const float mn = fmaxf(m, sc);
    const float corr = __expf(m - mn), pw = __expf(sc - mn);
    l = fmaf(l, corr, pw);
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = fmaf(o[j], corr, pw * vv[j]);
    m = mn;
}

// NB positions at once: independent scores, one max / rescale per batch.
template <int NB>
__device__ __forceinline__ void rl_fold_n(const float (&q)[8], const float4 (&k)[NB][2], const float4 (&v)[NB][2],
                                          const bool (&in)[NB], float scale, float &m, float &l, float (&o)[8]) {
    float sc[NB];
#pragma unroll
    for (int i = 0; i < NB; i++) {
        const float kv[8] = {k[i][0].x, k[i][0].y, k[i][0].z, k[i][0].w, k[i][1].x, k[i][1].y, k[i][1].z, k[i][1].w};
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) d = fmaf(q[j], kv[j], d);
        sc[i] = d;
    }
#pragma unroll
    for (int i = 0; i < NB; i++) sc[i] = group_sum<16>(sc[i]);
    float mn = m;
#pragma unroll
    for (int i = 0; i < NB; i++) {
        sc[i] = in[i] ? sc[i] * scale : -INFINITY;
        mn = fmaxf(mn, sc[i]);
    }
    const float corr = (mn == m) ? 1.0f : __expf(m - mn);
    float p[NB], ps = 0.0f;
#pragma unroll
    for (int i = 0; i < NB; i++) {
        p[i] = in[i] ? __expf(sc[i] - mn) : 0.0f;
        ps += p[i];
    }
    l = fmaf(l, corr, ps);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float acc = o[j] * corr;
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const float vj = j < 4 ? (&v[i][0].x)[j] : (&v[i][1].x)[j - 4];
            acc = fmaf(p[i], vj, acc);
        }
        o[j] = acc;
    }
    m = mn;
}

// The split of positions [0, pos] team rank q works on; cached positions
// [s0, cend) are in LDS, position pos (this step's k/v) belongs to the last
// split.
struct RlSplit {
    int nsplit, s0, s1, cend;
    bool active, last;
    __device__ __forceinline__ RlSplit(int pos, int q) {
        const int seq = pos + 1;
        int chunk = (seq + QK_RL_TEAM - 1) / QK_RL_TEAM;
        if (chunk < QK_RL_MIN_CHUNK) chunk = QK_RL_MIN_CHUNK;
        nsplit = (seq + chunk - 1) / chunk;
        active = q < nsplit;
        s0 = q * chunk;
        s1 = min(s0 + chunk, seq);
        last = active && s1 == seq;
        cend = last ? pos : s1;
        if (!active) cend = s0;
    }
};

// ---------------------------------------------------------------------------
// Shared state of a block
// ---------------------------------------------------------------------------
struct RlShared {
    float xs[RL_H];                 // residual (identical in every block of a team)
    float xn[RL_H];                 // final-normed row (LM head)
    RlPlanes<RL_H> xp;              // planes of the normed input
    RlPlanes<256> ap;               // planes of the group's merged attention output
    RlPlanes<RL_HG> hp;             // planes of the group's SwiGLU outputs
    float nin[RL_H], npost[RL_H];   // norm weights of the layer (from the load phase)
    float fnw[RL_H];                // final norm weights
    float nqk[256];                 // q norm | k norm
    float rope[256];                // cos | sin at the layer's position
    float qkv[512];                 // the group's raw q|q|k|v
    union {
        struct {
            float sm_m[RL_NG][2], sm_l[RL_NG][2];
            float sm_o[RL_NG][2][128];
        };
        float red[RL_NW][48];       // per-wave product partials
    };
    float pw[RL_NW][6 * QK_RL_TEAM];  // per wave: (m, l, o[4]) of every split for the wave's 4 merge dims
    float cand[2 * 256];            // LM-head candidates
    float ssq[RL_NW];
    float wv[RL_NW];
    int wi[RL_NW];
    int g, r, abort_, tok;
};

// K|V rows of this block's split: row j = position s0 + j, K in [0, 128), V in [128, 256)
typedef float RlKv[QK_RL_KVP][256];

__device__ __forceinline__ unsigned rl_tag(const qk_relay_args &a, int s, int l, int h) {
    return a.epoch + 1u + (unsigned)s * (QK_RL_TPL * ((unsigned)a.layers + 1u)) + (unsigned)l * QK_RL_TPL + (unsigned)h;
}

// Issue layer l's operands for position pos: this wave's weight tiles into
// registers; by LDS DMA the block's cached K/V rows, the norm weights and the
// RoPE row.  Nothing waits here.
__device__ __forceinline__ void rl_load_layer(const qk_relay_args &a, RlShared &S, RlKv &kv, RlW &w, int l, int pos,
                                              int g, int q, int wave, int lane) {
    const char *wb = a.wt + (long)l * QK_RL_LAYER_BYTES +
                     (long)(((g * QK_RL_TEAM + q) * RL_NW + wave) * QK_RL_TILES) * QK_RL_TILE_BYTES;
    rl_load_w(w, wb, lane);
    const RlSplit sp(pos, q);
    const float *kb = a.k_cache + ((long)l * RL_XCD + g) * (long)a.cap * 128;
    const float *vb = a.v_cache + ((long)l * RL_XCD + g) * (long)a.cap * 128;
    const int nc = sp.cend - sp.s0;
    for (int j = wave; j < nc; j += RL_NW) {
        const int p = sp.s0 + j;
        const float *src = lane < 32 ? kb + (long)p * 128 + lane * 4 : vb + (long)p * 128 + (lane - 32) * 4;
        __builtin_amdgcn_global_load_lds(src, &kv[j][0], 16, 0, 0);
    }
    const char *lb = a.layer0 + (long)l * a.layer_stride;
    __builtin_amdgcn_global_load_lds((const float *)(lb + a.off_nin) + wave * 256 + lane * 4, &S.nin[wave * 256], 16,
                                     0, 0);
    __builtin_amdgcn_global_load_lds((const float *)(lb + a.off_npost) + wave * 256 + lane * 4, &S.npost[wave * 256],
                                     16, 0, 0);
    if (wave == 0) {
        const float *src = lane < 32 ? (const float *)(lb + a.off_nq) + lane * 4 : (const float *)(lb + a.off_nk) + (lane - 32) * 4;
        __builtin_amdgcn_global_load_lds(src, &S.nqk[0], 16, 0, 0);
    } else if (wave == 1) {
        const float *src = lane < 32 ? a.rope_cos + (long)pos * 128 + lane * 4 : a.rope_sin + (long)pos * 128 + (lane - 32) * 4;
        __builtin_amdgcn_global_load_lds(src, &S.rope[0], 16, 0, 0);
    }
}

// S.xs slice q (64 words) = base + (P_0 + ... + P_7) over the 8 XCDs' split-K
// partials at part + g' * 1024 + 64 q (tag tp; the base from bsrc (tag tb)
// when given, else the block's own S.xs), republished at xl (tag tx); then
// the XCD's whole residual gathered into S.xs with per-wave sums of squares in
// S.ssq and, when w is given, the planes of x o w in S.xp (the next product's
// operand; its rows take the 1/rms factor in their epilogue, rl_rinv).  Wave
// w gathers elements [256 w, 256 w + 256), the norm-weight range its own
// load-phase DMA filled.  Order of the sum: x + (P_0 + ... + P_7), as x += o
// in qwen_asr_decoder.c:458, :468.
template <bool SYNC = true>
__device__ __forceinline__ bool rl_residual(const qk_relay_args &a, RlShared &S, const u64 *part, unsigned tp,
                                            const u64 *bsrc, unsigned tb, u64 *xl, unsigned tx, const float *w, int q,
                                            int wave, int lane, u64 *tr1, u64 *tr2) {
    // wave 0 polls the base rows (the other team's, when bsrc is given; else
    // the block's own) and all 8 slices of its rows, sums them in slice order
    // in registers and republishes at once, while the other waves go straight
    // to the gather: no barrier on the way (C1 2771 -> 2831 tok/s against the
    // four waves polling two slices each into LDS).  For its own base, wave 0
    // reads the rows before it publishes them, and a wave whose gather range
    // holds them overwrites them only after seeing that publication.
    bool ok = true;
    if (wave == 0) {
        float o = 0.0f, base = 0.0f;
        if (bsrc)   // XCD-local, published with the slices: first
            ok = rl_poll<1>(
                a, bsrc, [&](int i) { return RL_SO * q + i; }, 0, RL_SO, tb, [&](int, float v) { base = v; }, lane);
        if (ok)
            ok = rl_poll<RL_XCD>(
                a, part, [&](int i) { return (i >> 6) * RL_H + RL_SO * q + (i & 63); }, 0, RL_XCD * RL_SO, tp,
                [&](int i, float v) { o = (i >> 6) == 0 ? v : o + v; }, lane);
        if (!bsrc) base = S.xs[RL_SO * q + lane];
        if (ok) rl_put_local(xl + RL_SO * q + lane, base + o, tx);
        if (tr1) *tr1 = wall_clock64();
    }
    float v[4];
    if (ok) ok = rl_poll_vec<4>(a, xl, 256 * wave, tx, v, lane);
    float ss = 0.0f;
    if (ok) {
        const int i = 256 * wave + 4 * lane;
        *reinterpret_cast<float4 *>(&S.xs[i]) = make_float4(v[0], v[1], v[2], v[3]);
        ss = fmaf(v[0], v[0], ss);
        ss = fmaf(v[1], v[1], ss);
        ss = fmaf(v[2], v[2], ss);
        ss = fmaf(v[3], v[3], ss);
        if (w) {
            const float4 wv = *reinterpret_cast<const float4 *>(&w[i]);
            rl_plane2(S.xp, i, v[0] * wv.x, v[1] * wv.y);
            rl_plane2(S.xp, i + 2, v[2] * wv.z, v[3] * wv.w);
        }
    }
    ss = wave_sum(ss);
    if (lane == 0) S.ssq[wave] = ss;
    if (!ok) S.abort_ = 1;
    if constexpr (!SYNC) {
        // the caller's next product reads only this wave's own range; its
        // barrier after the product publishes S.ssq and S.abort_
        if (tr2) *tr2 = wall_clock64();
        return ok;
    }
    rl_sync();
    if (S.abort_) return false;
    if (tr2) *tr2 = wall_clock64();
    return true;
}

// 1 / rms of S.xs from the per-wave sums of squares (qwen_rms_norm,
// qwen_asr_kernels.c:750-809): a product over the planes of x o w times this
// is the product over rms_norm(x) * w.
__device__ __forceinline__ float rl_rinv(const qk_relay_args &a, const RlShared &S) {
    float ss = S.ssq[0];
#pragma unroll
    for (int i = 1; i < RL_NW; i++) ss += S.ssq[i];
    return rsqrt_norm(ss / (float)RL_H + a.eps);
}

// rms_norm(S.xs) * w (qwen_rms_norm, qwen_asr_kernels.c:750-809) from the
// per-wave sums of squares; planes P of the result (and the fp32 row at xn
// when given).  Wave w converts elements [256 w, 256 w + 256).
__device__ __forceinline__ void rl_norm(const qk_relay_args &a, RlShared &S, const float *w, RlPlanes<RL_H> *P,
                                        float *xn, int wave, int lane) {
    float ss = S.ssq[0];
#pragma unroll
    for (int i = 1; i < RL_NW; i++) ss += S.ssq[i];
    const float rinv = rsqrt_norm(ss / (float)RL_H + a.eps);
    const int i = 256 * wave + 4 * lane;
    const float4 x = *reinterpret_cast<const float4 *>(&S.xs[i]);
    const float4 wv = *reinterpret_cast<const float4 *>(&w[i]);
    const float v0 = (x.x * wv.x) * rinv, v1 = (x.y * wv.y) * rinv, v2 = (x.z * wv.z) * rinv, v3 = (x.w * wv.w) * rinv;
    if (xn) *reinterpret_cast<float4 *>(&xn[i]) = make_float4(v0, v1, v2, v3);
    if (P) {
        rl_plane2(*P, i, v0, v1);
        rl_plane2(*P, i + 2, v2, v3);
    }
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(RL_NW * 64, 1) void rl_decode(qk_relay_args a) {
    __shared__ __attribute__((aligned(16))) RlShared S;
    __shared__ __attribute__((aligned(16))) RlKv kv;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, tid = threadIdx.x;
    const int b = blockIdx.x, L = a.layers;

    // ---- launch check-in: every block on XCD g < 8 with rank < 32 ----
    if (tid == 0) {
        const int xcc = __builtin_amdgcn_s_getreg((15 << 11) | 20) & 15;   // HW_REG_XCC_ID
        const unsigned rank = __hip_atomic_fetch_add(&a.cnt[xcc], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool good = xcc < RL_XCD && rank < 2u * QK_RL_TEAM;
        S.g = xcc & 7;
        S.r = (int)(rank & 31u);
        S.abort_ = 0;
        __hip_atomic_store(&a.xv[b * QK_RL_LINE], ((u64)a.epoch << 32) | (good ? 1u : 0u), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    rl_sync();
    {
        bool good = true;
        const bool ok = rl_poll<1, true>(
            a, a.xv, [&](int i) { return (64 * wave + i) * QK_RL_LINE; }, 0, 64, a.epoch,
            [&](int, float v) { good = good && (__float_as_uint(v) & 1u); }, lane);
        if (!ok) S.abort_ = 1;
        if (ok && !__all(good)) {
            if (lane == 0) rl_raise(a.err, QK_PX_ERR_LAYOUT);
            S.abort_ = 1;
        }
    }
    rl_sync();
    if (S.abort_) return;
    const int g = __builtin_amdgcn_readfirstlane(S.g), r = __builtin_amdgcn_readfirstlane(S.r);
    const int team = r >> 4, q = r & 15;
    const long WG = RL_XCD;
    u64 *trb = a.trace ? a.trace + (long)b * QK_RL_TRACE : nullptr;

    // this block's Q|K|V rows in the group's 512: queries of heads 2g, 2g+1 (ranks 0-7), k (8-11), v (12-15)
    const int qrow = 32 * q;
    // the zero plane of every activation operand (A rows 3..15 of the products)
    for (int i = tid; i < RL_H; i += RL_NW * 64) S.xp.v[3][i] = 0;
    for (int i = tid; i < 256; i += RL_NW * 64) S.ap.v[3][i] = 0;
    for (int i = tid; i < RL_HG; i += RL_NW * 64) S.hp.v[3][i] = 0;

    RlW w;
    if (team < L) rl_load_layer(a, S, kv, w, team, a.pos0, g, q, wave, lane);
    // LM-head rows of this block
    // groups of LMR rows dealt round-robin to the blocks (block b: groups b,
    // b + 256, ...; wave w: the block's groups w, w + 4, ...), so at any
    // moment the grid streams one contiguous window of the table (C1: 2723 ->
    // 2778 tok/s against one contiguous range per block)
    constexpr int LMR = 4;
    const int lmg = (a.vocab + LMR - 1) / LMR;
    const int lmn = b < lmg ? (lmg - b + 255) / 256 : 0;
    const int lm1 = a.vocab;
    auto lrow = [&](int k, int j) { return (b + 256 * k) * LMR + j; };

    for (int s = 0; s < a.n_steps; s++) {
        const int pos = a.pos0 + s;
        const bool tracing = trb && s == a.trace_step && tid == 0;
        auto mark = [&](int i) {
            if (tracing) trb[i] = wall_clock64();
        };
        for (int l = team; l < L; l += 2) {
            const int t = team;
            auto T = [&](int h) { return rl_tag(a, s, l, h); };
            // ---- input residual ----
            mark(RL_TM * l + 0);
            if (l == 0) {
                // step input: emb[tok] (tok_embed_bf16_to_f32, qwen_asr.c:353-360) or the staged row
                const int i = 256 * wave + 4 * lane;
                float4 x;
                if (s == 0 && a.first_tok < 0) {
                    x = *reinterpret_cast<const float4 *>(a.x_in + i);
                } else {
                    const int tok = (s == 0) ? a.first_tok : S.tok;
                    const uint2 u = *reinterpret_cast<const uint2 *>(a.emb + (long)tok * RL_H + i);
                    x = make_float4(bf16_lo(u.x), bf16_hi(u.x), bf16_lo(u.y), bf16_hi(u.y));
                }
                *reinterpret_cast<float4 *>(&S.xs[i]) = x;
                float ss = fmaf(x.x, x.x, x.y * x.y);
                ss = fmaf(x.z, x.z, ss);
                ss = fmaf(x.w, x.w, ss);
                ss = wave_sum(ss);
                if (lane == 0) S.ssq[wave] = ss;
                rl_wait_vm();   // this layer's operands have landed (this wave's DMA filled nin[256 wave ..])
                const float4 nw = *reinterpret_cast<const float4 *>(&S.nin[i]);
                rl_plane2(S.xp, i, x.x * nw.x, x.y * nw.y);
                rl_plane2(S.xp, i + 2, x.z * nw.z, x.w * nw.w);
                rl_sync();
                mark(RL_TM * l + 1);
                mark(RL_TM * l + 2);
            } else {
                const unsigned tp = rl_tag(a, s, l - 1, 6);
                rl_residual<false>(a, S, a.xd + ((1 - t) * WG) * RL_H, tp, a.xs + ((1 - t) * WG + g) * RL_H, tp,
                                   a.xlb + (t * WG + g) * RL_H, T(7), S.nin, q, wave, lane,
                                   tracing ? trb + RL_TM * l + 1 : nullptr, tracing ? trb + RL_TM * l + 2 : nullptr);
                rl_wait_vm();
            }
            mark(RL_TM * l + 3);

            // ---- Q: 32 rows of the group's Q|K|V (qwen_linear_nobias_bf16_qkv, qwen_asr_kernels.c:434-460) ----
            {
                // wave w: row tiles 0, 1 over k tiles [8 w, 8 w + 8): the range of x
                // this wave gathered itself, so no barrier between gather and product
                f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
                bf16x8 af[8];
#pragma unroll
                for (int j = 0; j < 8; j++) af[j] = rl_afrag(S.xp, 8 * wave + j, lane);
                __builtin_amdgcn_sched_barrier(0);   // every fragment read in flight before the products
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    c0 = rl_mfma(af[j], w.q[j], c0);
                    c1 = rl_mfma(af[j], w.q[8 + j], c1);
                }
                if (lane < 16) {
                    S.red[wave][lane] = rl_rowsum(c0);
                    S.red[wave][16 + lane] = rl_rowsum(c1);
                }
            }
            rl_sync();
            if (S.abort_) return;
            if (wave == 0 && lane < 32) {
                const float y = (((S.red[0][lane] + S.red[1][lane]) + S.red[2][lane]) + S.red[3][lane]) * rl_rinv(a, S);
                rl_put_local(a.xq + (t * WG + g) * 512 + qrow + lane, y, T(0));
            }
            mark(RL_TM * l + 4);
            {
                const bool ok = rl_poll<2>(
                    a, a.xq + (t * WG + g) * 512, [&](int i) { return i; }, 128 * wave, 128 * wave + 128, T(0),
                    [&](int i, float v) { S.qkv[i] = v; }, lane);
                if (!ok) S.abort_ = 1;
            }
            rl_sync();
            if (S.abort_) return;
            mark(RL_TM * l + 5);

            // ---- A: q/k norm + RoPE + K/V append + attention split (qwen_asr_decoder.c:439-455) ----
            const RlSplit sp(pos, q);
            float *kcl = a.k_cache + ((long)l * RL_XCD + g) * (long)a.cap * 128;
            float *vcl = a.v_cache + ((long)l * RL_XCD + g) * (long)a.cap * 128;
            mark(RL_TM * l + 6);
            // causal attention of the group's two query heads over this block's
            // positions (qwen_causal_attention_heads, qwen_asr_kernels.c:1050-1097):
            // 32-lane group gid (two per wave) folds positions s0 + gid + 8 j from
            // LDS; its lane row (lane / 16) & 1 holds query head 2g + that bit, and
            // lane c of the row owns dims 4c .. 4c+3 and 64+4c .. 64+4c+3, so a
            // row's 16-byte reads of one K or V row cover 256 contiguous bytes (the
            // group's two rows read the same bytes).  Every row normalises and
            // rotates its query head itself (no stage of its own):
            // rms_norm_per_head (qwen_asr_kernels.c:811-873) + apply_rope_neox
            // (:1182-1247); the RoPE pair (d, d + 64) sits in one lane.
            if (sp.active) {
                const int hq = (lane >> 4) & 1, gid = wave * 2 + (lane >> 5), gl = lane & 15, d0 = 4 * gl,
                          d1 = 64 + 4 * gl;
                const float4 c4 = *reinterpret_cast<const float4 *>(&S.rope[d0]);
                const float4 s4 = *reinterpret_cast<const float4 *>(&S.rope[128 + d0]);
                float qv[8];
                {
                    float4 lo = *reinterpret_cast<const float4 *>(&S.qkv[hq * 128 + d0]);
                    float4 hi = *reinterpret_cast<const float4 *>(&S.qkv[hq * 128 + d1]);
                    norm_rope_row16(lo, hi, *reinterpret_cast<const float4 *>(&S.nqk[d0]),
                                    *reinterpret_cast<const float4 *>(&S.nqk[d1]), c4, s4, a.eps);
                    qv[0] = lo.x; qv[1] = lo.y; qv[2] = lo.z; qv[3] = lo.w;
                    qv[4] = hi.x; qv[5] = hi.y; qv[6] = hi.z; qv[7] = hi.w;
                }
                float m = -INFINITY, ls = 0.f, o[8];
#pragma unroll
                for (int j = 0; j < 8; j++) o[j] = 0.f;
                const int nc = sp.cend - sp.s0;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    if (b > 0 && nc <= 2 * RL_NG * b) break;   // block-uniform: no position from here on
                    float4 kk[2][2], vv[2][2];
                    bool in[2];
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const int jj = gid + RL_NG * (2 * b + j);
                        in[j] = jj < nc;
                        const float *row = kv[in[j] ? jj : 0];
                        kk[j][0] = *reinterpret_cast<const float4 *>(row + d0);
                        kk[j][1] = *reinterpret_cast<const float4 *>(row + d1);
                        vv[j][0] = *reinterpret_cast<const float4 *>(row + 128 + d0);
                        vv[j][1] = *reinterpret_cast<const float4 *>(row + 128 + d1);
                    }
                    rl_fold_n<2>(qv, kk, vv, in, a.scale, m, ls, o);
                }
                if (sp.last && gid == 0) {   // position pos: this step's k/v, appended to the cache (qwen_asr_decoder.c:446-447)
                    float4 k0 = *reinterpret_cast<const float4 *>(&S.qkv[256 + d0]);
                    float4 k1 = *reinterpret_cast<const float4 *>(&S.qkv[256 + d1]);
                    norm_rope_row16(k0, k1, *reinterpret_cast<const float4 *>(&S.nqk[128 + d0]),
                                    *reinterpret_cast<const float4 *>(&S.nqk[128 + d1]), c4, s4, a.eps);
                    const float4 v0 = *reinterpret_cast<const float4 *>(&S.qkv[384 + d0]);
                    const float4 v1 = *reinterpret_cast<const float4 *>(&S.qkv[384 + d1]);
                    if (hq == 0) {
                        *reinterpret_cast<float4 *>(kcl + (long)pos * 128 + d0) = k0;
                        *reinterpret_cast<float4 *>(kcl + (long)pos * 128 + d1) = k1;
                        *reinterpret_cast<float4 *>(vcl + (long)pos * 128 + d0) = v0;
                        *reinterpret_cast<float4 *>(vcl + (long)pos * 128 + d1) = v1;
                    }
                    rl_fold1(qv, k0, k1, v0, v1, a.scale, m, ls, o);
                }
                if (gl == 0) {
                    S.sm_m[gid][hq] = m;
                    S.sm_l[gid][hq] = ls;
                }
                *reinterpret_cast<float4 *>(&S.sm_o[gid][hq][d0]) = make_float4(o[0], o[1], o[2], o[3]);
                *reinterpret_cast<float4 *>(&S.sm_o[gid][hq][d1]) = make_float4(o[4], o[5], o[6], o[7]);
            }
            rl_sync();
            mark(RL_TM * l + 7);
            if (sp.active && tid < 256) {
                const int h = tid >> 7, d = tid & 127;
                float M = -INFINITY;
#pragma unroll
                for (int i = 0; i < RL_NG; i++) M = fmaxf(M, S.sm_m[i][h]);
                float Lh = 0.0f, acc = 0.0f;
#pragma unroll
                for (int i = 0; i < RL_NG; i++) {
                    // M is finite (every group of a split below the last folds a
                    // position, and group 0 of the last split folds pos), so a
                    // group without positions (m = -inf) gets exp(-inf) = 0
                    const float e = __expf(S.sm_m[i][h] - M);
                    Lh = fmaf(S.sm_l[i][h], e, Lh);
                    acc = fmaf(S.sm_o[i][h][d], e, acc);
                }
                // the K/V row stored at pos is read by other blocks of this XCD
                // in later steps: the stores retire before this block publishes
                if (sp.last && wave == 0) rl_wait_vm();
                u64 *dst = a.xa + ((t * WG + g) * QK_RL_TEAM + q) * (long)QK_RL_PART + h * 130;
                rl_put_local(dst + 2 + d, acc, T(1));
                if (d == 0) {
                    rl_put_local(dst, M, T(1));
                    rl_put_local(dst + 1, Lh, T(1));
                }
            }
            mark(RL_TM * l + 8);

            // ---- M: rank q merges dims [16 q, 16 q + 16) of the group's 256 over every split ----
            {
                // wave w merges dims d0 .. d0 + 3 and polls just their words: no barrier
                const int h = q >> 3, d0 = 16 * (q & 7) + 4 * wave;
                const u64 *src = a.xa + ((t * WG + g) * QK_RL_TEAM) * (long)QK_RL_PART + h * 130;
                // word 6 i + k: split i's m (k 0), l (k 1), o[d0 + k - 2] (k 2..5)
                const int nw = 6 * sp.nsplit;
                const bool ok = rl_poll<2>(
                    a, src,
                    [&](int i) {
                        const int si = i / 6, k = i - 6 * si;
                        return si * QK_RL_PART + (k < 2 ? k : d0 + k);
                    },
                    0, nw, T(1), [&](int i, float v) { S.pw[wave][i] = v; }, lane);
                if (!ok) S.abort_ = 1;
                mark(RL_TM * l + 9);
                {
                    // 16 dims x 16 splits on the block's 256 lanes: lane (4 wave + lane / 16, lane % 16) holds
                    // split lane % 16 of dim d0 + 4 wave + lane / 16; max, sum and weighted sum over the 16-lane
                    // row (the online merge of qwen_causal_attention_heads' running max and sum,
                    // qwen_asr_kernels.c:1073-1094, taken over the splits at once)
                    const int dl = lane >> 4, si = lane & 15;
                    const bool in = si < sp.nsplit;
                    const float mv = in ? S.pw[wave][si * 6] : -INFINITY;
                    const float lv = in ? S.pw[wave][si * 6 + 1] : 0.0f;
                    const float ov = in ? S.pw[wave][si * 6 + 2 + dl] : 0.0f;
                    const float M = group_max<16>(mv);
                    const float e = __expf(mv - M);   // M finite: split 0 is always in
                    const float Lh = group_sum<16>(lv * e);
                    const float acc = group_sum<16>(ov * e);
                    // the reference scales by 1/sum (qwen_asr_kernels.c:1091-1094)
                    if (si == 0 && ok)
                        rl_put_local(a.xm + (t * WG + g) * 256 + h * 128 + d0 + dl, acc * __builtin_amdgcn_rcpf(Lh), T(2));
                }
                mark(RL_TM * l + 10);
                const bool ok2 = rl_poll<1>(
                    a, a.xm + (t * WG + g) * 256, [&](int i) { return i; }, 64 * wave, 64 * wave + 64, T(2),
                    [&](int i, float v) { rl_plane1(S.ap, i, v); }, lane);
                if (!ok2) S.abort_ = 1;
                rl_sync();
                if (S.abort_) return;
                mark(RL_TM * l + 11);
            }

            // ---- O: 64 rows of W_o over the group's 256 columns (qwen_asr_decoder.c:457) ----
            {
                // wave w: row tile w over all 8 k tiles
                f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
                bf16x8 af[8];
#pragma unroll
                for (int j = 0; j < 8; j++) af[j] = rl_afrag(S.ap, j, lane);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    c0 = rl_mfma(af[j], w.o[j], c0);
                    c1 = rl_mfma(af[j + 1], w.o[j + 1], c1);
                }
                if (lane < 16)
                    rl_put_global(a.xo + (t * WG + g) * RL_H + RL_SO * q + 16 * wave + lane, rl_rowsum(c0) + rl_rowsum(c1),
                                  T(3));
            }
            mark(RL_TM * l + 12);

            // ---- F: x' = x + O; rms_norm; 48 gate|up rows + SwiGLU (qwen_asr_decoder.c:458-466) ----
            {
                rl_residual<false>(a, S, a.xo + (t * WG) * RL_H, T(3), nullptr, 0u, a.xla + (t * WG + g) * RL_H, T(4),
                                   S.npost, q, wave, lane, tracing ? trb + RL_TM * l + 13 : nullptr,
                                   tracing ? trb + RL_TM * l + 14 : nullptr);
            }
            mark(RL_TM * l + 15);
            {
                // wave w: row tiles 0..2 over k tiles [8 w, 8 w + 8)
                f32x4 c[3] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
                bf16x8 af[8];
#pragma unroll
                for (int j = 0; j < 8; j++) af[j] = rl_afrag(S.xp, 8 * wave + j, lane);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 8; j++) {
#pragma unroll
                    for (int rt = 0; rt < 3; rt++) c[rt] = rl_mfma(af[j], w.f[8 * rt + j], c[rt]);
                }
                if (lane < 16) {
#pragma unroll
                    for (int rt = 0; rt < 3; rt++) S.red[wave][16 * rt + lane] = rl_rowsum(c[rt]);
                }
            }
            rl_sync();
            if (S.abort_) return;
            mark(RL_TM * l + 16);
            if (wave == 0 && lane < 48) {
                const float y = (((S.red[0][lane] + S.red[1][lane]) + S.red[2][lane]) + S.red[3][lane]) * rl_rinv(a, S);
                // rows 2i (gate), 2i+1 (up) sit in adjacent lanes (qwen_swiglu_multiply, qwen_asr_kernels.c:930-931)
                const float up = xor_lane<1>(y);
                if ((lane & 1) == 0)
                    rl_put_local(a.xh + (t * WG + g) * RL_HG + 24 * q + (lane >> 1), swiglu1(y, up), T(5));
            }
            mark(RL_TM * l + 17);
            {
                const bool ok = rl_poll<2>(
                    a, a.xh + (t * WG + g) * RL_HG, [&](int i) { return i; }, 96 * wave, 96 * wave + 96, T(5),
                    [&](int i, float v) { rl_plane1(S.hp, i, v); }, lane);
                if (!ok) S.abort_ = 1;
            }
            rl_sync();
            if (S.abort_) return;
            mark(RL_TM * l + 18);

            // ---- D: 64 rows of W_down over the group's 384 columns (qwen_asr_decoder.c:467) ----
            {
                // wave w: row tile w over all 12 k tiles
                f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
                bf16x8 af[12];
#pragma unroll
                for (int j = 0; j < 12; j++) af[j] = rl_afrag(S.hp, j, lane);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 12; j += 2) {
                    c0 = rl_mfma(af[j], w.d[j], c0);
                    c1 = rl_mfma(af[j + 1], w.d[j + 1], c1);
                }
                if (lane < 16) {
                    const int row = RL_SO * q + 16 * wave + lane;
                    rl_put_global(a.xd + (t * WG + g) * RL_H + row, rl_rowsum(c0) + rl_rowsum(c1), T(6));
                    rl_put_local(a.xs + (t * WG + g) * RL_H + row, S.xs[row], T(6));
                }
            }
            mark(RL_TM * l + 19);
            // ---- the team's next layer (the next step's first one after the last) ----
            if (l + 2 < L) {
                rl_load_layer(a, S, kv, w, l + 2, pos, g, q, wave, lane);
            } else if (s + 1 < a.n_steps && l + 1 < L) {
                // not the last layer: the LM head does not follow at once
                rl_load_layer(a, S, kv, w, t, pos + 1, g, q, wave, lane);
            }
            mark(RL_TM * l + 20);
        }

        // ---- LM: final residual (x += down partials of layer L-1), rms_norm (in place, :474) ----
        {
            const int tl = (L - 1) & 1;
            mark(RL_TM * L + 0);
            // final norm weights, and the first LM-head rows of each wave
            if (wave < 4) __builtin_amdgcn_global_load_lds(a.fnorm + wave * 256 + lane * 4, &S.fnw[wave * 256], 16, 0, 0);
            uint4 lmw[LMR][2];
#pragma unroll
            for (int j = 0; j < LMR; j++) {
                const int row = lrow(wave, j);
#pragma unroll
                for (int c = 0; c < 2; c++)
                    lmw[j][c] = ld_stream16(a.emb + (long)min(row, lm1 - 1) * RL_H + c * 512 + lane * 8);
            }
            const unsigned tp = rl_tag(a, s, L - 1, 6);
            // one barrier publishes the gathered residual, the sums of squares
            // and every wave's final-norm weight DMA
            rl_residual<false>(a, S, a.xd + (tl * WG) * RL_H, tp, a.xs + (tl * WG + g) * RL_H, tp,
                               a.xlb + (team * WG + g) * RL_H, rl_tag(a, s, L, 7), nullptr, q, wave, lane,
                               tracing ? trb + RL_TM * L + 1 : nullptr, tracing ? trb + RL_TM * L + 2 : nullptr);
            rl_wait_vm();
            rl_sync();
            if (S.abort_) return;
            rl_norm(a, S, S.fnw, nullptr, S.xn, wave, lane);
            rl_sync();
            if (g == 0 && r == 0 && a.hidden_out)
                for (int i = tid; i < RL_H; i += RL_NW * 64) a.hidden_out[i] = S.xn[i];

            // ---- argmax over this block's rows of the tied embedding (qwen_argmax_matvec_bf16, :518-543) ----
            float bv = -1e30f;
            int bi = 0x7fffffff;
            for (int k = wave; k < lmn; k += RL_NW) {
                uint4 nx[LMR][2];
                const bool more = k + RL_NW < lmn;
                if (more) {
#pragma unroll
                    for (int j = 0; j < LMR; j++) {
                        const int row = lrow(k + RL_NW, j);
#pragma unroll
                        for (int c = 0; c < 2; c++)
                            nx[j][c] = ld_stream16(a.emb + (long)min(row, lm1 - 1) * RL_H + c * 512 + lane * 8);
                    }
                }
                float acc[LMR];
#pragma unroll
                for (int j = 0; j < LMR; j++) acc[j] = 0.0f;
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    float xv[8];
                    const float4 p0 = *reinterpret_cast<const float4 *>(&S.xn[c * 512 + lane * 8]);
                    const float4 p1 = *reinterpret_cast<const float4 *>(&S.xn[c * 512 + lane * 8 + 4]);
                    xv[0] = p0.x; xv[1] = p0.y; xv[2] = p0.z; xv[3] = p0.w;
                    xv[4] = p1.x; xv[5] = p1.y; xv[6] = p1.z; xv[7] = p1.w;
#pragma unroll
                    for (int j = 0; j < LMR; j++) acc[j] = dot8_bf16(lmw[j][c], xv, acc[j]);
                }
                reduce_rows<LMR, 1>(acc, lane);   // lane groups of 16 hold row lane / 16
                const int row = lrow(k, lane / (64 / LMR));
                if (row < lm1) {
                    if (a.logits && (lane % (64 / LMR)) == 0) a.logits[row] = acc[0];
                    if (argmax_better(acc[0], row, bv, bi)) {
                        bv = acc[0];
                        bi = row;
                    }
                }
                if (more) {
#pragma unroll
                    for (int j = 0; j < LMR; j++)
#pragma unroll
                        for (int c = 0; c < 2; c++) lmw[j][c] = nx[j][c];
                }
            }
            wave_argmax(bv, bi);
            if (lane == 0) {
                S.wv[wave] = bv;
                S.wi[wave] = bi;
            }
            rl_sync();
            if (tid == 0) {
                float v = S.wv[0];
                int ix = S.wi[0];
                for (int ww = 1; ww < RL_NW; ww++)
                    if (argmax_better(S.wv[ww], S.wi[ww], v, ix)) {
                        v = S.wv[ww];
                        ix = S.wi[ww];
                    }
                const unsigned Tc = rl_tag(a, s, L, 0);
                rl_put_global(a.xc + (long)b * QK_RL_LINE, v, Tc);
                rl_put_global(a.xc + (long)b * QK_RL_LINE + 1, __int_as_float(ix), Tc);
            }
            mark(RL_TM * L + 3);
        }
        // the team whose last layer was L - 1 loads its next layer now
        if (s + 1 < a.n_steps && team < L && (team == ((L - 1) & 1)))
            rl_load_layer(a, S, kv, w, team, pos + 1, g, q, wave, lane);

        // ---- T: team 0 reduces the candidates (qwen_asr_kernels.c:534-541) ----
        if (team == 0) {
            const unsigned Tc = rl_tag(a, s, L, 0);
            const bool ok = rl_poll<2>(
                a, a.xc, [&](int i) { return (64 * wave + (i >> 1)) * QK_RL_LINE + (i & 1); }, 0, 128, Tc,
                [&](int i, float v) { S.cand[128 * wave + i] = v; }, lane);
            if (!ok) S.abort_ = 1;
            rl_sync();
            if (S.abort_) return;
            if (wave == 0) {
                float bv = -1e30f;
                int bi = 0x7fffffff;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int c = 64 * j + lane;
                    const float v = S.cand[2 * c];
                    const int ix = __float_as_int(S.cand[2 * c + 1]);
                    if (argmax_better(v, ix, bv, bi)) {
                        bv = v;
                        bi = ix;
                    }
                }
                wave_argmax(bv, bi);
                // nothing above the reference's -1e30 floor: it returns its start row
                const int tok = bi == 0x7fffffff ? 0 : bi;
                if (lane == 0) {
                    S.tok = tok;
                    if (g == 0 && r == 0) {
                        if (a.log) a.log[s] = tok;
                        if (a.tok_out) *a.tok_out = tok;
                        if (a.pos_out) *a.pos_out = pos + 1;
                    }
                }
            }
            rl_sync();
            mark(RL_TM * L + 4);
        }
    }
    rl_wait_vm();
}

// ---------------------------------------------------------------------------
// weight tiling
// ---------------------------------------------------------------------------
// One uint4 (8 bf16) per thread: tile i of wave w of team rank q on XCD g,
// lane l: row (tile row) + l % 16, columns (tile column) + 8 (l / 16) .. + 8.
__global__ __launch_bounds__(256) void rl_pack(uint4 *dst, const uint16_t *wqkv, const uint16_t *wo,
                                               const uint16_t *wgu, const uint16_t *wdown) {
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    const long total = QK_RL_LAYER_BYTES / 16;
    if (idx >= total) return;
    const int lane = (int)(idx & 63);
    long t = idx >> 6;
    const int i = (int)(t % QK_RL_TILES);
    t /= QK_RL_TILES;
    const int w = (int)(t % RL_NW);
    t /= RL_NW;
    const int q = (int)(t % QK_RL_TEAM);
    const int g = (int)(t / QK_RL_TEAM);
    const int rl = lane & 15, kl = 8 * (lane >> 4);
    const uint16_t *src;
    if (i < 16) {           // Q: row tile i >> 3, k tile 8 w + (i & 7)
        // group row 32 q: queries of heads 2g, 2g+1 (stacked rows 256 g ..), k (2048 + 128 g ..), v (3072 + 128 g ..)
        const int gr = 32 * q;
        const int row = gr < 256 ? 256 * g + gr : (gr < 384 ? 2048 + 128 * g + (gr - 256) : 3072 + 128 * g + (gr - 384));
        const int kt = 8 * w + (i & 7);
        src = wqkv + (long)(row + 16 * (i >> 3) + rl) * RL_H + 32 * kt + kl;
    } else if (i < 24) {    // O: rows 64 q + 16 w, columns 256 g + 32 kt
        const int kt = i - 16;
        src = wo + (long)(RL_SO * q + 16 * w + rl) * 2048 + 256 * g + 32 * kt + kl;
    } else if (i < 48) {    // F: interleaved gate|up rows 768 g + 48 q + 16 rt, k tile 8 w + j
        const int j = i - 24, rt = j >> 3, kt = 8 * w + (j & 7);
        src = wgu + (long)(2 * RL_HG * g + 48 * q + 16 * rt + rl) * RL_H + 32 * kt + kl;
    } else {                // D: rows 64 q + 16 w, columns 384 g + 32 kt
        const int kt = i - 48;
        src = wdown + (long)(RL_SO * q + 16 * w + rl) * RL_I + RL_HG * g + 32 * kt + kl;
    }
    dst[idx] = *reinterpret_cast<const uint4 *>(src);
}

extern "C" int qk_relay_pack(char *dst, const uint16_t *wqkv, const uint16_t *wo, const uint16_t *wgu,
                             const uint16_t *wdown, hipStream_t s) {
    if (!dst || !wqkv || !wo || !wgu || !wdown) return QWEN_HIP_EINVAL;
    const long total = QK_RL_LAYER_BYTES / 16;
    hipLaunchKernelGGL(rl_pack, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, reinterpret_cast<uint4 *>(dst),
                       wqkv, wo, wgu, wdown);
    return hipGetLastError() == hipSuccess ? 0 : QWEN_HIP_EDEVICE;
}

// One block per CU, every block resident at once: 256 CUs, and at most one
// block fits a CU (its LDS and registers), so the dispatcher spreads the grid
// one per CU.
extern "C" int qk_relay_supported(int hidden, int inter, int heads, int kv_heads, int device) {
    if (hidden != RL_H || inter != RL_I || heads != 16 || kv_heads != RL_XCD) return 0;
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
    if (cus != QK_PX_BLOCKS) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void *)rl_decode, RL_NW * 64, 0) != hipSuccess ||
        per != 1)
        return 0;
    return 1;
}

extern "C" int qk_relay_launch(const qk_relay_args *a, hipStream_t s) {
    if (!a || a->n_steps <= 0 || a->layers <= 0 || a->epoch == 0u || !a->wt) return QWEN_HIP_EINVAL;
    if (a->trace && RL_TM * a->layers + 5 > QK_RL_TRACE) return QWEN_HIP_EINVAL;
    if (a->first_tok < 0 && !a->x_in) return QWEN_HIP_EINVAL;
    if (a->first_tok >= a->vocab || a->pos0 < 0 || a->pos0 + a->n_steps > a->cap) return QWEN_HIP_EINVAL;
    if (a->pos0 + a->n_steps > QK_RL_MAX_SEQ) return QWEN_HIP_EINVAL;   // positions beyond the LDS split capacity
    qk_relay_args copy = *a;
    void *args[] = {&copy};
    if (hipLaunchKernel((const void *)rl_decode, dim3(QK_PX_BLOCKS), dim3(RL_NW * 64), args, 0, s) != hipSuccess)
        return QWEN_HIP_EDEVICE;
    return 0;
}
