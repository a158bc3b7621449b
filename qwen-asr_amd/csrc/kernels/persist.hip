// persist.hip - the greedy decode loop of the Qwen3 decoder as ONE persistent
// kernel on gfx950: qwen_decoder_forward (reference qwen_asr_decoder.c:388-476)
// repeated by the token loop (qwen_asr.c:729-759), n steps per launch.
//
// Why one kernel: a 0.6B decode step streams 1.2 GB of weights but is a chain
// of ~140 dependent all-to-all hand-overs (5 per layer).  As separate kernels
// each hand-over costs a launch plus a cold start of the next kernel; here the
// blocks stay resident, hand activations over through memory, and issue the
// next stage's weight loads before they wait, so HBM latency hides behind the
// hand-over.
//
// Work layout (MI355X: 8 XCDs x 32 CUs, one block per CU).  XCD g owns kv head
// g with its query heads 2g, 2g+1, 1/8 of the MLP intermediate rows, and the
// matching split-K column slices of the O and down projections.  Per layer
// only the two split-K partial sums (8 x hidden floats) cross XCDs; the other
// six hand-overs stay inside one XCD and go through its L2.
//
//   Q  rms_norm(x) . Wqkv rows of the group (16 rows per block)      -> local
//   A  q/k norm + RoPE + K/V append + attention over a position split -> local
//   M  block r merges 8 of the group's 256 attention dims over splits -> local
//   O  W_o[:, group cols] over the merged output (H/32 rows per block) -> cross
//   F  x += sum of O partials; rms_norm; gate|up rows + SwiGLU         -> local
//   D  W_down[:, group cols] (H/32 rows per block)                    -> cross
//   (next layer's Q adds the down partials to x), LM head + argmax    -> cross
//
// Exchange words are 64-bit: (tag << 32) | fp32 bits.  A reader polls the
// words it needs until each carries the expected tag, so every word is its
// own ready flag and no fence is needed.  XCD-local words are written with
// plain stores (they land in the XCD's shared L2) and read with agent-scope
// loads (sc1: they skip the CU-private L1).  Cross-XCD words use agent-scope
// stores (written through to the memory side) and agent-scope loads.  Tags
// are unique per hand-over within a launch and across launches (the host
// advances the epoch), so a stale word can never pass as fresh: at worst a
// wait times out, raises an error bit and every block leaves.
//
// Each block runs NCW compute waves and one sync wave.  Only the sync wave
// polls, so outstanding weight prefetches of the compute waves never hold up
// a poll (loads retire in order per wave).  Both roles walk the same barrier
// sequence; the block barrier does not wait on global loads.
//
// Every wait is bounded in wall-clock time: a poll that has not seen its words
// after a.wait_ticks ticks of the constant-rate clock (the host passes about
// one second) raises QK_PX_ERR_TIMEOUT, and every poll also gives up once
// another block raised an error, so all waves of the grid reach the end of the
// kernel whatever happens to the others (a block that is never scheduled, a
// producer that faulted).  The kernel is launched as an ordinary grid of one
// block per CU (each block's LDS does not leave room for a second one); the
// launch check-in verifies that every block is resident and that each XCD holds
// exactly 32 of them before any work starts.
#include "common.h"
#include "qk_kernels.h"
#include "qwen_asr_hip.h"

#include <math.h>

typedef unsigned long long u64;

#define PX_QD 2048                 // 16 query heads x 128
#define PX_KVD 1024                // 8 kv heads x 128

// ---------------------------------------------------------------------------
// exchange words
// ---------------------------------------------------------------------------
__device__ __forceinline__ u64 px_word(float v, unsigned tag) { return ((u64)tag << 32) | __float_as_uint(v); }

__device__ __forceinline__ void px_put_local(u64 *p, float v, unsigned tag) {
    __hip_atomic_store(p, px_word(v, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}

__device__ __forceinline__ void px_put_global(u64 *p, float v, unsigned tag) {
    __hip_atomic_store(p, px_word(v, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ u64 px_get(const u64 *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool px_aborted(unsigned *err) {
    return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}

__device__ __forceinline__ void px_raise(unsigned *err, unsigned bits) {
    __hip_atomic_fetch_or(err, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte streaming load at a wave-uniform base plus a 32-bit per-lane byte
// offset, so the load uses the scalar-base addressing form and a lane keeps one
// offset register per slab instead of a 64-bit address per load.
__device__ __forceinline__ uint4 px_ld16(const void *base, unsigned off) {
    return ld_stream16(reinterpret_cast<const uint16_t *>(reinterpret_cast<const char *>(base) + off));
}

__device__ __forceinline__ float4 px_ldf4(const void *base, unsigned off) {
    return *reinterpret_cast<const float4 *>(reinterpret_cast<const char *>(base) + off);
}

// Block barrier that leaves global loads in flight (weight prefetches cross
// it); this wave's LDS accesses are complete before it.
__device__ __forceinline__ void px_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// This lane's index, produced where it is used: the compiler cannot hoist the
// asm out of the layer loop, so offsets derived from it are recomputed in
// place (two VALU ops) instead of being kept live across the loop.  Under
// register pressure (1.7B) a kept offset was spilled, and its scratch reload
// waits for every load the wave has in flight: the D-stage publish then
// waited for the next layer's whole W_q slab.
__device__ __forceinline__ int px_lane_here() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// Sync wave: wait until the n words at addr(i), i < n, carry `tag`, then
// dst[i] = value.  PER words per lane in flight per pass.  False when the wait
// passed a.wait_ticks (QK_PX_ERR_TIMEOUT raised) or another block raised an
// error.  The clock is read while the pass's loads are in flight, so the
// bound costs no extra round trip.  CHECKIN: the bound is a.checkin_ticks.
template <int PER, bool CHECKIN = false, typename Addr>
__device__ bool px_poll(const qk_persist_args &a, Addr addr, int n, unsigned tag, float *dst, int lane,
                        float *ssq = nullptr) {
    const u64 t0 = wall_clock64();
    for (int base = 0; base < n; base += 64 * PER) {
        for (unsigned spin = 1;; spin++) {
            u64 w[PER];
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const int i = base + j * 64 + lane;
                w[j] = (i < n) ? px_get(addr(i)) : ((u64)tag << 32);
            }
            const u64 now = wall_clock64();
            bool ok = true;
#pragma unroll
            for (int j = 0; j < PER; j++) ok = ok && ((unsigned)(w[j] >> 32) == tag);
            if (__all(ok)) {
#pragma unroll
                for (int j = 0; j < PER; j++) {
                    const int i = base + j * 64 + lane;
                    if (i < n) {
                        const float v = __uint_as_float((unsigned)w[j]);
                        dst[i] = v;
                        if (ssq) *ssq = fmaf(v, v, *ssq);   // this lane's share of sum(x^2), in px_rmsnorm's order
                    }
                }
                break;
            }
            if (now - t0 > (CHECKIN ? a.checkin_ticks : a.wait_ticks)) {
                if (lane == 0) px_raise(a.err, QK_PX_ERR_TIMEOUT);
                return false;
            }
            if ((spin & 15u) == 0u && px_aborted(a.err)) return false;
        }
    }
    return true;
}

// SO rows (64 or 32) of 8 split-K partials each, the partial of XCD j at
// p + j * stride, polled like px_poll and summed in XCD order in registers.
// SO = 64: lane = row, 8 loads.  SO = 32: lane l polls XCDs 2 k + l / 32 of
// row l % 32 and one permlane32 swap hands each pair (even, odd) to both
// lanes of the row.  The row's sum lands in o of lane row (and row + 32).
template <int SO>
__device__ bool px_poll_rows(const qk_persist_args &a, const u64 *p, long stride, unsigned tag, int lane, float &o) {
    static_assert(SO == 64 || SO == 32, "one or two lanes per row");
    constexpr int NL = SO == 64 ? 8 : 4;
    const u64 *q = SO == 64 ? p + lane : p + (lane >> 5) * stride + (lane & 31);
    const long js = SO == 64 ? stride : 2 * stride;
    const u64 t0 = wall_clock64();
    for (unsigned spin = 1;; spin++) {
        u64 w[NL];
#pragma unroll
        for (int j = 0; j < NL; j++) w[j] = px_get(q + j * js);
        const u64 now = wall_clock64();
        bool ok = true;
#pragma unroll
        for (int j = 0; j < NL; j++) ok = ok && ((unsigned)(w[j] >> 32) == tag);
        if (__all(ok)) {
            if constexpr (SO == 64) {
                o = __uint_as_float((unsigned)w[0]);
#pragma unroll
                for (int j = 1; j < 8; j++) o += __uint_as_float((unsigned)w[j]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float ev = __uint_as_float((unsigned)w[j]), od = ev;
                    swap32(ev, od);   // ev: XCD 2 j's partial, od: XCD 2 j + 1's, in both lanes of the row
                    o = j == 0 ? ev + od : (o + ev) + od;
                }
            }
            return true;
        }
        if (now - t0 > a.wait_ticks) {
            if (lane == 0) px_raise(a.err, QK_PX_ERR_TIMEOUT);
            return false;
        }
        if ((spin & 15u) == 0u && px_aborted(a.err)) return false;
    }
}

// ---------------------------------------------------------------------------
// A slab of bf16 weight rows held in registers by the compute waves.  Lanes
// form groups of LW; a group covers 8*LW consecutive columns per 16-byte load
// (SEGS loads per row), a wave covers 64/LW rows per batch and BPW batches.
// Rows [0, R) of the slab start at W with row stride ld (elements).  Wave w
// owns batches [w*WB, w*WB + BPW) of the row range (WB > BPW: the slab is
// the first BPW batches of each wave's share, the rest held by another slab).
// ---------------------------------------------------------------------------
template <int LW, int SEGS, int BPW, int WB = BPW>
struct PxSlab {
    static constexpr int RPI = 64 / LW;
    uint4 w[BPW][SEGS];

    // wave must be wave-uniform (an SGPR): every per-batch offset then folds
    // into the scalar base and a lane needs one 32-bit offset for all loads.
    __device__ __forceinline__ void load(const uint16_t *W, int ld, int wave, int /*lane*/) {
        // recomputed at every call: otherwise the compiler keeps per-lane slab
        // offsets live across the layer loop and spills them
        const int ln = px_lane_here();
        const unsigned lo = (unsigned)((ln / LW) * ld + (ln % LW) * 8) * 2u;
#pragma unroll
        for (int b = 0; b < BPW; b++) {
            const uint16_t *wb = W + (long)((wave * WB + b) * RPI) * ld;
#pragma unroll
            for (int s = 0; s < SEGS; s++) w[b][s] = px_ld16(wb + s * 8 * LW, lo);
        }
    }

    // slab row of batch b for this lane
    __device__ __forceinline__ static int row(int wave, int b, int lane) { return (wave * WB + b) * RPI + lane / LW; }

    // y[b] = W[row] . x for the row of batch b, in every lane of the LW group
    __device__ __forceinline__ void dot(const float *x, float (&y)[BPW], int lane) const {
        const int cl = (lane % LW) * 8;
#pragma unroll
        for (int b = 0; b < BPW; b++) y[b] = 0.0f;
#pragma unroll
        for (int s = 0; s < SEGS; s++) {
            float xv[8];
            const float4 p0 = *reinterpret_cast<const float4 *>(x + s * 8 * LW + cl);
            const float4 p1 = *reinterpret_cast<const float4 *>(x + s * 8 * LW + cl + 4);
            xv[0] = p0.x; xv[1] = p0.y; xv[2] = p0.z; xv[3] = p0.w;
            xv[4] = p1.x; xv[5] = p1.y; xv[6] = p1.z; xv[7] = p1.w;
#pragma unroll
            for (int b = 0; b < BPW; b++) y[b] = dot8_bf16(w[b][s], xv, y[b]);
        }
#pragma unroll
        for (int b = 0; b < BPW; b++) y[b] = group_sum<LW>(y[b]);
    }
};

// K/V rows of one attention split in flight: 16 lanes own a position, 8 dims each
template <int AB>
struct PxKv {
    float4 k[AB][2], v[AB][2];
    // kb, vb: wave-uniform (layer, kv head) bases; lane owns dims [8*gl, 8*gl+8)
    // of position p0 + stride*j (positions >= end give zeros)
    __device__ __forceinline__ void load(const float *kb, const float *vb, int gl, int p0, int stride, int end) {
#pragma unroll
        for (int j = 0; j < AB; j++) {
            // every element is (re)defined so the compiler can drop the old batch
            const int p = p0 + stride * j;
            const bool in = p < end;
            const unsigned o = (unsigned)((in ? p : 0) * 128 + gl * 8) * 4u;
            const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            k[j][0] = in ? px_ldf4(kb, o) : z;
            k[j][1] = in ? px_ldf4(kb, o + 16u) : z;
            v[j][0] = in ? px_ldf4(vb, o) : z;
            v[j][1] = in ? px_ldf4(vb, o + 16u) : z;
        }
    }
    // the same rows, every load issued: positions >= end read position 0
    // (finite: the cache is zeroed when allocated) and must not be folded
    __device__ __forceinline__ void load_all(const float *kb, const float *vb, int gl, int p0, int stride, int end) {
#pragma unroll
        for (int j = 0; j < AB; j++) {
            const int p = p0 + stride * j;
            const unsigned o = (unsigned)((p < end ? p : 0) * 128 + gl * 8) * 4u;
            k[j][0] = px_ldf4(kb, o);
            k[j][1] = px_ldf4(kb, o + 16u);
            v[j][0] = px_ldf4(vb, o);
            v[j][1] = px_ldf4(vb, o + 16u);
        }
    }
};

// Issue the first K/V batch of a split straight into LDS (no registers held
// across the stages in between).  Lane (16-lane group, gl) loads dims
// [8gl, 8gl+8) of position p0 + stride*j; positions >= end, and every position
// of a block without a split, read position 0 (always valid memory) and are
// never folded.  Every block issues the same loads, which keeps the
// compiler's wait counting exact.  Each wave later reads back only what it
// loaded itself, after waiting for its loads.
template <int AB>
__device__ __forceinline__ void px_kv_dma(uint4 (&dst)[AB][4][64], const float *kb, const float *vb, int gl, int p0,
                                          int stride, int end, bool active) {
#pragma unroll
    for (int j = 0; j < AB; j++) {
        const int p = p0 + stride * j;
        const unsigned o = active ? (unsigned)((p < end ? p : 0) * 128 + gl * 8) * 4u : 0u;
        const char *kc = reinterpret_cast<const char *>(kb) + o;
        const char *vc = reinterpret_cast<const char *>(vb) + o;
        __builtin_amdgcn_global_load_lds(kc, &dst[j][0][0], 16, 0, 0);
        __builtin_amdgcn_global_load_lds(kc + 16, &dst[j][1][0], 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vc, &dst[j][2][0], 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vc + 16, &dst[j][3][0], 16, 0, 0);
    }
}

// Wait for every load and store this wave issued (vmcnt(0)); the builtin keeps
// the compiler's own wait bookkeeping in step.
__device__ __forceinline__ void px_wait_loads() { __builtin_amdgcn_s_waitcnt(0x0f70); }

__device__ __forceinline__ float4 px_u2f(uint4 u) {
    return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
}

// online-softmax fold of one key/value position into both query heads
// (qwen_causal_attention_heads, qwen_asr_kernels.c:1073-1089)
__device__ __forceinline__ void px_fold(const float (&q)[2][8], float4 k0, float4 k1, float4 v0, float4 v1, float scale,
                                        float (&m)[2], float (&l)[2], float (&o)[2][8]) {
    const float kv[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) d = fmaf(q[h][j], kv[j], d);
        d = group_sum<16>(d);
        const float sc = d * scale;
        const float mn = fmaxf(m[h], sc);
        const float corr = __expf(m[h] - mn), pw = __expf(sc - mn);
        l[h] = fmaf(l[h], corr, pw);
#pragma unroll
        for (int j = 0; j < 8; j++) o[h][j] = fmaf(o[h][j], corr, pw * vv[j]);
        m[h] = mn;
    }
}

// px_fold for NB positions at once: the NB scores of a head are independent
// dot products, then one max / rescale and an exp-weighted sum, so the online
// softmax pays one dependent update per batch instead of one per position.
// in[i] false: position i is skipped (its k/v may be anything finite).
template <int NB>
__device__ __forceinline__ void px_fold_n(const float (&q)[2][8], const float4 (&k)[NB][2], const float4 (&v)[NB][2],
                                          const bool (&in)[NB], float scale, float (&m)[2], float (&l)[2],
                                          float (&o)[2][8]) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float sc[NB];
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const float kv[8] = {k[i][0].x, k[i][0].y, k[i][0].z, k[i][0].w, k[i][1].x, k[i][1].y, k[i][1].z, k[i][1].w};
            float d = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) d = fmaf(q[h][j], kv[j], d);
            sc[i] = d;
        }
#pragma unroll
        for (int i = 0; i < NB; i++) sc[i] = group_sum<16>(sc[i]);
        float mn = m[h];
#pragma unroll
        for (int i = 0; i < NB; i++) {
            sc[i] = in[i] ? sc[i] * scale : -INFINITY;
            mn = fmaxf(mn, sc[i]);
        }
        // mn == m[h] covers the batch with no position in and the start (m = -inf)
        const float corr = (mn == m[h]) ? 1.0f : __expf(m[h] - mn);
        float p[NB], ps = 0.0f;
#pragma unroll
        for (int i = 0; i < NB; i++) {
            p[i] = in[i] ? __expf(sc[i] - mn) : 0.0f;
            ps += p[i];
        }
        l[h] = fmaf(l[h], corr, ps);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float acc = o[h][j] * corr;
#pragma unroll
            for (int i = 0; i < NB; i++) {
                const float vj = j < 4 ? (&v[i][0].x)[j] : (&v[i][1].x)[j - 4];
                acc = fmaf(p[i], vj, acc);
            }
            o[h][j] = acc;
        }
        m[h] = mn;
    }
}

// The split of positions [0, pos] a block of the group works on.
struct PxSplit {
    int nsplit, s0, s1, cend;
    bool active, last;
    __device__ __forceinline__ PxSplit(int pos, int r) {
        const int seq = pos + 1;
        int chunk = (seq + QK_PX_MAX_SPLIT - 1) / QK_PX_MAX_SPLIT;
        if (chunk < QK_PX_MIN_CHUNK) chunk = QK_PX_MIN_CHUNK;
        nsplit = (seq + chunk - 1) / chunk;
        active = r < nsplit;
        s0 = r * chunk;
        s1 = min(s0 + chunk, seq);
        last = active && s1 == seq;
        cend = last ? pos : s1;      // position pos itself comes from this step's k/v
    }
};

// ---------------------------------------------------------------------------
// Shared state of a block
// ---------------------------------------------------------------------------
template <int H, int I, int NCW>
struct PxShared {
    static constexpr int SO = H / QK_PX_LOC;    // O / down rows per block
    static constexpr int HG = I / QK_PX_XCD;    // SwiGLU outputs per XCD group
    static constexpr int NG = NCW * 4;          // 16-lane attention groups
    // 1.7B: the sync wave starts the q|k|v and SwiGLU polls without the
    // stage-entry barrier (those polls fill S.qkv / S.hs, which the compute
    // waves' dot still running then does not read): C3 1005 -> 1015 tok/s.
    // 0.6B keeps it (2128 -> 2121 without, C4 1157 -> 1148), and both keep the Q and F entries,
    // which also place the slab loads against the x-update polls (C3 1001
    // with those removed too)
    static constexpr bool EARLY_POLL = NCW != 4;
    float xs[H];                                // residual (kept identical in every block)
    float xn[H];                                // normed input of Q / F / LM head
    float nw[H];                                // norm weight of the pending RMSNorm (sync wave)
    float qkv[512];                             // raw q|q|k|v of the group
    float qr[2][128], kr[128], vr[128];         // normed + rotated q, k; v

    // attention scratch: the 16-lane groups' (max, sum, output) while the split
    // is folded (stage A), then the (m, l, 8 o words) of every split polled by
    // the sync wave for its share of the merge (stage O); the stages are
    // barrier-separated, so they share storage
    union {
        struct {
            float sm_m[NG][2], sm_l[NG][2];
            float sm_o[NG][2][128];
        };
        float part[QK_PX_MAX_SPLIT * 10];
    };
    float att[256];                             // merged attention output of the group
    float hs[HG];                               // SwiGLU outputs of the group
    float ysum[8 * SO];                         // split-K partial slices
    float wv[NCW];
    int wi[NCW];
    float cand[2 * QK_PX_BLOCKS];
    int g, r, abort_, tok;
};

// First K/V batch of each attention split, loaded straight into LDS: per
// compute wave, AB positions x (k[0:4], k[4:8], v[0:4], v[4:8]) x 64 lanes.
// A __shared__ object of its own: LDS reads of PxShared then provably do not
// alias the in-flight DMA, and the compiler does not wait for it ahead of them.
template <int NCW>
using PxKvLds = uint4[NCW][64 / (NCW * 4)][4][64];

template <int H>
__device__ __forceinline__ const char *px_layer(const qk_persist_args &a, int l) {
    return a.layer0 + (long)l * a.layer_stride;
}

// ---------------------------------------------------------------------------
// sync wave
// ---------------------------------------------------------------------------
template <int H, int I, int NCW>
__device__ bool px_x_update(const qk_persist_args &a, PxShared<H, I, NCW> &S, const u64 *yp, unsigned ty, u64 *xl,
                            unsigned tx, int lane, float &ssq, unsigned long long *tr_hop = nullptr) {
    constexpr int SO = PxShared<H, I, NCW>::SO;
    const int r = S.r;
    // this block's slice of the 8 split-K partials
    if constexpr (SO == 64 || SO == 32) {
        // summed in registers, XCD order
        float o;
        if (!px_poll_rows<SO>(a, yp + SO * r, H, ty, lane, o)) return false;
        if (tr_hop) *tr_hop = wall_clock64();
        if (lane < SO) px_put_local(xl + SO * r + lane, S.xs[SO * r + lane] + o, tx);   // x += o (qwen_asr_decoder.c:458, :468)
    } else {
        auto slice = [&](int i) { return yp + (long)(i / SO) * H + SO * r + (i % SO); };
        if (!px_poll<8 * SO / 64>(a, slice, 8 * SO, ty, S.ysum, lane)) return false;
        if (tr_hop) *tr_hop = wall_clock64();
        if (lane < SO) {
            float o = S.ysum[lane];
#pragma unroll
            for (int gg = 1; gg < QK_PX_XCD; gg++) o += S.ysum[gg * SO + lane];
            px_put_local(xl + SO * r + lane, S.xs[SO * r + lane] + o, tx);   // x += o (qwen_asr_decoder.c:458, :468)
        }
    }
    // the XCD's whole new residual
    auto whole = [&](int i) { return xl + i; };
    ssq = 0.0f;
    return px_poll<(H / 64 < 16 ? H / 64 : 16)>(a, whole, H, tx, S.xs, lane, &ssq);
}

// xn = rms_norm(xs) * w (qwen_rms_norm, qwen_asr_kernels.c:750-809); w was
// DMA'd into LDS by px_load_norm and has landed (the caller's polls waited
// for every load of this wave).
// ssq_lane >= 0: this lane's share of sum(x^2) already accumulated (by the
// poll that wrote xs, same elements in the same order); < 0: compute it here.
template <int H, int I, int NCW>
__device__ void px_rmsnorm(const qk_persist_args &a, PxShared<H, I, NCW> &S, const float *w, int lane,
                           float ssq_lane = -1.0f) {
    float ss = ssq_lane;
    if (ss < 0.0f) {
        ss = 0.0f;
#pragma unroll
        for (int j = 0; j < H / 64; j++) {
            const float v = S.xs[j * 64 + lane];
            ss = fmaf(v, v, ss);
        }
    }
    ss = wave_sum(ss);
    const float rinv = rsqrt_norm(ss / (float)H + a.eps);
    // elementwise, so any lane may take any element: four consecutive ones
    // per 16-byte access
#pragma unroll
    for (int j = 0; j < H / 256; j++) {
        const int i = 256 * j + 4 * lane;
        const float4 x = *reinterpret_cast<const float4 *>(&S.xs[i]);
        const float4 wv = *reinterpret_cast<const float4 *>(&w[i]);
        *reinterpret_cast<float4 *>(&S.xn[i]) =
            make_float4((x.x * wv.x) * rinv, (x.y * wv.y) * rinv, (x.z * wv.z) * rinv, (x.w * wv.w) * rinv);
    }
}

// Stage O's input, in two hand-overs: block r of the group merges 8 of the
// group's 256 attention output dims (head r / 16, dims 8 (r % 16) ..) over
// every split (m, l and its 8 o words per split) and publishes them; then the
// block reads all 256 merged dims into S.att.  The merge is the online merge
// of qwen_causal_attention_heads' running max and sum (qwen_asr_kernels.c:
// 1073-1094), taken over chunks of 8 splits.
template <int H, int I, int NCW>
__device__ bool px_merge_splits(const qk_persist_args &a, PxShared<H, I, NCW> &S, int pos, int g, int r, int par,
                                unsigned T, int lane) {
    const long WG = (long)QK_PX_XCD;
    const PxSplit sp(pos, 0);
    const int h = r >> 4, d0 = 8 * (r & 15);
    const u64 *src = a.xa + (par * WG + g) * (long)(QK_PX_MAX_SPLIT * QK_PX_PART) + h * 130;
    // word 10 i + k: split i's m (k 0), l (k 1), o[d0 + k - 2] (k 2..9)
    auto part = [&](int i) {
        const int sidx = i / 10, k = i - 10 * sidx;
        return src + (long)sidx * QK_PX_PART + (k < 2 ? k : d0 + k);
    };
    if (!px_poll<QK_PX_MAX_SPLIT * 10 / 64>(a, part, 10 * sp.nsplit, T + 1u, S.part, lane)) return false;
    u64 *xm = a.xm + (par * WG + g) * 256;
    {
        // lane (8 sg + dl) folds splits sg, sg + 8, ... of dim d0 + dl; then
        // the 8 split groups of a dim combine (xor 8 by DPP, xor 16 / 32 by the
        // permlane swaps).  M is finite from split 0 on, so exp(-inf - M) = 0
        // covers the lanes and splits without positions.
        const int dl = lane & 7, sg = lane >> 3;
        float M = -INFINITY, Lh = 0.0f, acc = 0.0f;
        for (int i = sg; i < sp.nsplit; i += 8) {
            const float *pp = S.part + i * 10;
            const float mv = pp[0], lv = pp[1], ov = pp[2 + dl];
            const float Mn = fmaxf(M, mv);
            const float sc = __expf(M - Mn), e = __expf(mv - Mn);
            Lh = fmaf(lv, e, Lh * sc);
            acc = fmaf(ov, e, acc * sc);
            M = Mn;
        }
        float Ma = fmaxf(M, xor_lane<8>(M));
        {
            float x = Ma, y = Ma;
            swap16(x, y);
            Ma = fmaxf(x, y);
            x = Ma;
            y = Ma;
            swap32(x, y);
            Ma = fmaxf(x, y);
        }
        const float sc = __expf(M - Ma);
        Lh *= sc;
        acc *= sc;
        Lh += xor_lane<8>(Lh);
        acc += xor_lane<8>(acc);
        {
            float x = Lh, y = Lh, u = acc, v = acc;
            swap16(x, y);
            swap16(u, v);
            Lh = x + y;
            acc = u + v;
            x = Lh;
            y = Lh;
            u = acc;
            v = acc;
            swap32(x, y);
            swap32(u, v);
            Lh = x + y;
            acc = u + v;
        }
        // the reference scales by 1/sum (qwen_asr_kernels.c:1091-1094); a
        // hardware reciprocal here
        if (lane < 8) px_put_local(xm + h * 128 + d0 + lane, acc * __builtin_amdgcn_rcpf(Lh), T + 7u);
    }
    auto whole = [&](int i) { return xm + i; };
    return px_poll<4>(a, whole, 256, T + 7u, S.att, lane);
}

// Start the DMA of a norm weight vector [H] into LDS (no registers held while
// the sync wave polls).
template <int H>
__device__ __forceinline__ void px_load_norm(const float *p, float *dst, int lane) {
#pragma unroll
    for (int j = 0; j < H / 256; j++)
        __builtin_amdgcn_global_load_lds(p + j * 256 + lane * 4, dst + j * 256, 16, 0, 0);
}

template <int H, int I, int NCW>
__device__ void px_sync_role(const qk_persist_args &a, PxShared<H, I, NCW> &S, int lane) {
    constexpr int HG = PxShared<H, I, NCW>::HG;
    constexpr bool EARLY_POLL = PxShared<H, I, NCW>::EARLY_POLL;
    const int L = a.layers, b = blockIdx.x;
    const long WG = (long)QK_PX_XCD;

    // ---- launch check-in: every block must sit on XCD g < 8 with rank < 32 ----
    px_sync();
    {
        float *dst = S.cand;   // scratch
        auto addr = [&](int i) { return a.xv + i; };
        bool ok = px_poll<4, true>(a, addr, QK_PX_BLOCKS, a.epoch, dst, lane);
        if (ok) {
            bool good = true;
            for (int i = lane; i < QK_PX_BLOCKS; i += 64) good = good && (__float_as_uint(dst[i]) & 1u);
            if (!__all(good)) {
                ok = false;
                if (lane == 0) px_raise(a.err, QK_PX_ERR_LAYOUT);
            }
        }
        if (lane == 0) S.abort_ = ok ? 0 : 1;
    }
    px_sync();
    if (S.abort_) return;
    const int g = __builtin_amdgcn_readfirstlane(S.g), r = __builtin_amdgcn_readfirstlane(S.r);

    for (int s = 0; s < a.n_steps; s++) {
        const int pos = a.pos0 + s;
        const unsigned tstep = a.epoch + 1u + (unsigned)s * (QK_PX_TPL * (unsigned)L + 1u);
        unsigned long long *tr = (a.trace && s == a.trace_step && lane == 0) ? a.trace + (long)b * QK_PX_TRACE : nullptr;
        auto mark = [&](int i) {
            if (tr) tr[i] = wall_clock64();
        };
        for (int l = 0; l < L; l++) {
            const unsigned T = tstep + QK_PX_TPL * (unsigned)l;
            const int par = l & 1;
            const char *lb = px_layer<H>(a, l);
            bool ok = true;
            float ssq = -1.0f;
            // ---- Q: input (embedding / x_in) or x += down partials; input norm ----
            px_load_norm<H>((const float *)(lb + a.off_nin), S.nw, lane);
            px_sync();
            mark(10 * l + 0);
            if (l == 0) {
                if (s == 0 && a.first_tok < 0) {
                    for (int i = lane; i < H; i += 64) S.xs[i] = a.x_in[i];
                } else {
                    // tok_embed_bf16_to_f32 (qwen_asr.c:353-360)
                    const int tok = (s == 0) ? a.first_tok : S.tok;
                    const uint16_t *e = a.emb + (long)tok * H;
                    for (int i = lane * 8; i < H; i += 512) {
                        const uint4 q = *reinterpret_cast<const uint4 *>(e + i);
                        S.xs[i + 0] = bf16_lo(q.x); S.xs[i + 1] = bf16_hi(q.x);
                        S.xs[i + 2] = bf16_lo(q.y); S.xs[i + 3] = bf16_hi(q.y);
                        S.xs[i + 4] = bf16_lo(q.z); S.xs[i + 5] = bf16_hi(q.z);
                        S.xs[i + 6] = bf16_lo(q.w); S.xs[i + 7] = bf16_hi(q.w);
                    }
                }
            } else {
                const int pp = (l - 1) & 1;
                ok = px_x_update<H, I, NCW>(a, S, a.xd + (pp * WG) * H, T - QK_PX_TPL + 5u, a.xlb + (pp * WG + g) * H,
                                            T - QK_PX_TPL + 6u, lane, ssq, tr ? tr + QK_PX_TRACE_XU + 2 * l : nullptr);
            }
            if (ok) {
                px_wait_loads();
                px_rmsnorm<H, I, NCW>(a, S, S.nw, lane, l == 0 ? -1.0f : ssq);
            }
            mark(10 * l + 1);
            if (lane == 0) S.abort_ = !ok;
            px_sync();
            if (S.abort_) return;

            // ---- A: the group's q|q|k|v ----
            if (!EARLY_POLL) px_sync();
            mark(10 * l + 2);
            {
                const u64 *src = a.xq + (par * WG + g) * 512;
                auto addr = [&](int i) { return src + i; };
                ok = px_poll<8>(a, addr, 512, T, S.qkv, lane);
            }
            mark(10 * l + 3);
            if (lane == 0) S.abort_ = !ok;
            px_sync();
            if (S.abort_) return;
            px_sync();   // after q/k norm + RoPE
            px_sync();   // after the position fold

            // ---- O: merge the group's split partials, then read the merged output ----
            px_sync();
            mark(10 * l + 4);
            ok = px_merge_splits<H, I, NCW>(a, S, pos, g, r, par, T, lane);
            mark(10 * l + 5);
            if (lane == 0) S.abort_ = !ok;
            px_sync();
            if (S.abort_) return;

            // ---- F: x += O partials; post-attention norm ----
            px_load_norm<H>((const float *)(lb + a.off_npost), S.nw, lane);
            px_sync();
            mark(10 * l + 6);
            ok = px_x_update<H, I, NCW>(a, S, a.xo + (par * WG) * H, T + 2u, a.xla + (par * WG + g) * H, T + 3u, lane,
                                        ssq, tr ? tr + QK_PX_TRACE_XU + 2 * l + 1 : nullptr);
            if (ok) {
                px_wait_loads();
                px_rmsnorm<H, I, NCW>(a, S, S.nw, lane, ssq);
            }
            mark(10 * l + 7);
            if (lane == 0) S.abort_ = !ok;
            px_sync();
            if (S.abort_) return;

            // ---- D: the group's SwiGLU outputs ----
            if (!EARLY_POLL) px_sync();
            mark(10 * l + 8);
            {
                const u64 *src = a.xh + (par * WG + g) * HG;
                auto addr = [&](int i) { return src + i; };
                ok = px_poll<(HG + 63) / 64>(a, addr, HG, T + 4u, S.hs, lane);
            }
            mark(10 * l + 9);
            if (lane == 0) S.abort_ = !ok;
            px_sync();
            if (S.abort_) return;
        }
        // ---- LM: x += last down partials; final norm (in place in the reference, :474) ----
        {
            const unsigned T = tstep + QK_PX_TPL * (unsigned)(L - 1);
            const int pp = (L - 1) & 1;
            px_load_norm<H>(a.fnorm, S.nw, lane);
            px_sync();
            mark(10 * L + 0);
            float ssq = -1.0f;
            bool ok = px_x_update<H, I, NCW>(a, S, a.xd + (pp * WG) * H, T + 5u, a.xlb + (pp * WG + g) * H, T + 6u, lane,
                                             ssq, tr ? tr + QK_PX_TRACE_XU + 2 * L : nullptr);
            if (ok) {
                px_wait_loads();
                px_rmsnorm<H, I, NCW>(a, S, S.nw, lane, ssq);
                if (b == 0 && a.hidden_out)
                    for (int i = lane; i < H; i += 64) a.hidden_out[i] = S.xn[i];
            }
            mark(10 * L + 1);
            if (lane == 0) S.abort_ = !ok;
            px_sync();
            if (S.abort_) return;
            px_sync();   // after the per-wave winners
        }
        // ---- T: argmax over the per-block candidates (qwen_asr_kernels.c:534-541) ----
        {
            const unsigned Tc = tstep + QK_PX_TPL * (unsigned)L;
            px_sync();
            mark(10 * L + 2);
            auto addr = [&](int i) { return a.xc + i; };
            bool ok = px_poll<8>(a, addr, 2 * QK_PX_BLOCKS, Tc, S.cand, lane);
            mark(10 * L + 3);
            if (ok) {
                float bv = -1e30f;
                int bi = 0x7fffffff;
                for (int i = lane; i < QK_PX_BLOCKS; i += 64) {
                    const float v = S.cand[i];
                    const int ix = __float_as_int(S.cand[QK_PX_BLOCKS + i]);
                    if (argmax_better(v, ix, bv, bi)) { bv = v; bi = ix; }
                }
                wave_argmax(bv, bi);
                // nothing above the reference's -1e30 floor: it returns its start row
                const int tok = bi == 0x7fffffff ? 0 : bi;
                if (lane == 0) {
                    S.tok = tok;
                    if (b == 0) {
                        if (a.log) a.log[s] = tok;
                        if (a.tok_out) *a.tok_out = tok;
                        if (a.pos_out) *a.pos_out = pos + 1;
                    }
                }
            }
            if (lane == 0) S.abort_ = !ok;
            px_sync();
            if (S.abort_) return;
        }
    }
}

// ---------------------------------------------------------------------------
// compute waves
//
// Weight slabs are issued stages before they are used so their HBM latency
// overlaps the hand-overs.  DEEP (0.6B) keeps two stages in flight:
//   end of D(l-1): K/V(l)     end of A: gate|up(l)
//   end of O: down(l), Q(l+1) end of F: O(l+1)
// the 1.7B slabs are 4x larger, so it issues each one stage ahead, between
// the two barriers that open the stage before the one that uses it (its
// stream then overlaps the sync wave's wait there, not the compute waves'):
//   Q(l): K/V(l), O(l)   end of A: gate|up(l) but FR rows per wave (half in
//   registers, FL rows by LDS DMA into the wave's K/V buffer)
//   F(l): the FR rows, used right after   D(l): down(l), Q(l+1)
// ---------------------------------------------------------------------------
template <int H, int I, int NCW>
__device__ void px_compute_role(const qk_persist_args &a, PxShared<H, I, NCW> &S, PxKvLds<NCW> &kvb, int wave,
                                int lane) {
    constexpr int SO = PxShared<H, I, NCW>::SO;
    constexpr int HG = PxShared<H, I, NCW>::HG;
    constexpr int NG = PxShared<H, I, NCW>::NG;
    constexpr int AB = 64 / NG;                         // K/V positions per 16-lane group in the LDS batch
    constexpr int SEGH = H / 512;
    constexpr int RF = 2 * I / QK_PX_BLOCKS;            // gate|up rows per block
    constexpr int LMR = NCW == 4 ? 4 : 2;               // LM-head rows per wave batch
    constexpr bool DEEP = NCW == 4;
    using SlabQ = PxSlab<64, SEGH, 16 / NCW>;
    using SlabO = PxSlab<32, 1, SO / 2 / NCW>;
    // gate|up: DEEP holds the block's rows in one slab.  1.7B: the first half
    // of each wave's rows in registers and FL rows in the wave's share of the
    // K/V LDS buffer (free between the fold and the next layer's K/V DMA),
    // both issued after attention; the FR rows left go to registers when
    // stage F opens
    constexpr int FB = RF / NCW, FB1 = DEEP ? FB : FB / 2, FB2 = FB - FB1;
    constexpr int KVW = (int)sizeof(PxKvLds<NCW>) / NCW;                     // LDS bytes per wave
    constexpr int FL = DEEP ? 0 : (FB2 < KVW / (2 * H) ? FB2 : KVW / (2 * H));
    constexpr int FR = FB2 - FL;
    using SlabF = PxSlab<64, SEGH, FB1, FB>;
    using SlabF2 = PxSlab<64, SEGH, (FR > 0 ? FR : 1), FB>;
    static_assert(DEEP || (FR >= 1 && FL >= 1), "1.7B gate|up split");
    using SlabD = PxSlab<16, HG / 128, SO / 4 / NCW>;
    static_assert(16 % NCW == 0 && (SO / 2) % NCW == 0 && RF % NCW == 0 && (SO / 4) % NCW == 0, "slab split");
    // the slabs tile their row ranges exactly (no bounds checks in PxSlab::load)
    static_assert(SlabQ::RPI * (16 / NCW) * NCW == 16 && SlabO::RPI * (SO / 2 / NCW) * NCW == SO, "tiling");
    static_assert(SlabF::RPI * (RF / NCW) * NCW == RF && SlabD::RPI * (SO / 4 / NCW) * NCW == SO, "tiling");
    static_assert((RF / NCW) % 2 == 0, "SwiGLU pairs must stay in one wave");
    static_assert(HG % 128 == 0 && AB >= 1, "shape");

    const int L = a.layers, b = blockIdx.x, tid = threadIdx.x;
    const long WG = (long)QK_PX_XCD;
    // LM head: groups of LMR rows dealt round-robin to the blocks (block b:
    // groups b, b + 256, ...), so at any moment the grid streams one window of
    // the table (C3 992.8 -> 1000.3 tok/s, C1 2114 -> 2134 against one
    // contiguous range per block)
    const int lmg = (a.vocab + LMR - 1) / LMR;
    const int lmn = b < lmg ? (lmg - b + QK_PX_BLOCKS - 1) / QK_PX_BLOCKS : 0;
    const int lm1 = a.vocab;
    auto lrow = [&](int k, int j) { return (b + QK_PX_BLOCKS * k) * LMR + j; };

    // launch check-in
    if (tid == 0) {
        const int xcc = __builtin_amdgcn_s_getreg((15 << 11) | 20) & 15;   // HW_REG_XCC_ID
        const unsigned rank = __hip_atomic_fetch_add(&a.cnt[xcc], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool good = xcc < QK_PX_XCD && rank < (unsigned)QK_PX_LOC;
        S.g = xcc & 7;
        S.r = (int)(rank & 31u);
        __hip_atomic_store(&a.xv[b], ((u64)a.epoch << 32) | (good ? 1u : 0u), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    px_sync();
    px_sync();
    if (S.abort_) return;
    const int g = __builtin_amdgcn_readfirstlane(S.g), r = __builtin_amdgcn_readfirstlane(S.r);

    // the block's slices of every layer
    const int qrow0 = r < 16 ? 256 * g + 16 * r
                             : (r < 24 ? PX_QD + 128 * g + 16 * (r - 16) : PX_QD + PX_KVD + 128 * g + 16 * (r - 24));
    auto Wq = [&](int l) { return (const uint16_t *)(px_layer<H>(a, l) + a.off_qkv) + (long)qrow0 * H; };
    auto Wo = [&](int l) { return (const uint16_t *)(px_layer<H>(a, l) + a.off_o) + (long)(SO * r) * PX_QD + 256 * g; };
    auto Wf = [&](int l) {
        return (const uint16_t *)(px_layer<H>(a, l) + a.off_gu) + (long)((2 * I / QK_PX_XCD) * g + RF * r) * H;
    };
    auto Wd = [&](int l) { return (const uint16_t *)(px_layer<H>(a, l) + a.off_down) + (long)(SO * r) * I + HG * g; };
    auto Kc = [&](int l) { return a.k_cache + ((long)l * QK_PX_XCD + g) * (long)a.cap * 128; };
    auto Vc = [&](int l) { return a.v_cache + ((long)l * QK_PX_XCD + g) * (long)a.cap * 128; };

    const int gid = wave * 4 + (lane >> 4), gl = lane & 15;
    const bool tracer = a.trace && tid == 0;
    SlabQ wq;
    SlabO wo;
    SlabF wf;
    SlabF2 wf2;
    SlabD wd;

    // first step's layer-0 operands
    {
        const PxSplit sp(a.pos0, r);
        wq.load(Wq(0), H, wave, lane);
        if (DEEP) px_kv_dma<AB>(kvb[wave], Kc(0), Vc(0), gl, sp.s0 + gid, NG, sp.cend, sp.active);
    }

    for (int s = 0; s < a.n_steps; s++) {
        const int pos = a.pos0 + s;
        const unsigned tstep = a.epoch + 1u + (unsigned)s * (QK_PX_TPL * (unsigned)L + 1u);
        const PxSplit sp(pos, r);
        unsigned long long *tr = (tracer && s == a.trace_step) ? a.trace + (long)b * QK_PX_TRACE + QK_PX_TRACE_CW : nullptr;
        for (int l = 0; l < L; l++) {
            const unsigned T = tstep + QK_PX_TPL * (unsigned)l;
            const int par = l & 1;
            const char *lb = px_layer<H>(a, l);
            float *kcl = Kc(l), *vcl = Vc(l);
            auto mark = [&](int i) {
                if (tr) tr[10 * l + i] = wall_clock64();
            };

            // ---- Q: the group's Q|K|V rows (qwen_linear_nobias_bf16_qkv, qwen_asr_kernels.c:434-460) ----
            px_sync();
            if (!DEEP) {   // streams while the sync wave waits for the residual
                wo.load(Wo(l), PX_QD, wave, lane);
                px_kv_dma<AB>(kvb[wave], Kc(l), Vc(l), gl, sp.s0 + gid, NG, sp.cend, sp.active);
            }
            px_sync();
            if (S.abort_) return;
            {
                float y[16 / NCW];
                wq.dot(S.xn, y, lane);
                mark(0);
                if (lane == 0) {
                    u64 *dst = a.xq + (par * WG + g) * 512 + 16 * r;
#pragma unroll
                    for (int i = 0; i < 16 / NCW; i++) px_put_local(dst + SlabQ::row(wave, i, 0), y[i], T);
                }
            }
            // 0.6B spreads its prefetches so no hand-over waits behind more than ~32 KB per CU:
            // W_o here, W_f after attention, W_d and the next W_q once the O / F hand-overs landed
            if (DEEP) wo.load(Wo(l), PX_QD, wave, lane);
            // operands of the norm/RoPE step
            float rc = 0.f, rs = 0.f, nw1 = 0.f, nw2 = 0.f;
            if (wave < 3) {
                rc = a.rope_cos[(long)pos * 128 + lane];
                rs = a.rope_sin[(long)pos * 128 + lane];
                const float *nwp = (const float *)(lb + (wave < 2 ? a.off_nq : a.off_nk));
                nw1 = nwp[lane];
                nw2 = nwp[lane + 64];
            }
            mark(1);

            // ---- A: q/k norm + RoPE + K/V append + attention split (qwen_asr_decoder.c:439-455) ----
            if (!PxShared<H, I, NCW>::EARLY_POLL) px_sync();
            px_sync();
            if (S.abort_) return;
            if (wave < 3) {
                const float *src = S.qkv + wave * 128;
                float x1 = src[lane], x2 = src[lane + 64];
                // rms_norm_per_head (qwen_asr_kernels.c:811-873) + apply_rope_neox (:1182-1247)
                const float ss = wave_sum(fmaf(x1, x1, x2 * x2));
                const float rinv = rsqrt_norm(ss / 128.0f + a.eps);
                const float p1 = (x1 * nw1) * rinv, p2 = (x2 * nw2) * rinv;
                x1 = fmaf(p1, rc, -(p2 * rs));
                x2 = fmaf(p2, rc, p1 * rs);
                float *dst = wave < 2 ? S.qr[wave] : S.kr;
                dst[lane] = x1;
                dst[lane + 64] = x2;
                if (wave == 2 && sp.last) {   // K store at pos (qwen_asr_decoder.c:446)
                    kcl[(long)pos * 128 + lane] = x1;
                    kcl[(long)pos * 128 + lane + 64] = x2;
                }
            } else if (wave == 3) {
                const float v1 = S.qkv[384 + lane], v2 = S.qkv[448 + lane];
                S.vr[lane] = v1;
                S.vr[lane + 64] = v2;
                if (sp.last) {                // V store at pos (:447)
                    vcl[(long)pos * 128 + lane] = v1;
                    vcl[(long)pos * 128 + lane + 64] = v2;
                }
            }
            mark(2);
            px_sync();
            // Causal attention of the group's two query heads over this block's
            // positions (qwen_causal_attention_heads, qwen_asr_kernels.c:1050-1097):
            // each 16-lane group folds every NG-th position into its online softmax,
            // then the NG groups merge in LDS.
            if (sp.active) {
                float q[2][8];
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int j = 0; j < 8; j++) q[h][j] = S.qr[h][gl * 8 + j];
                float m[2] = {-INFINITY, -INFINITY}, lsum[2] = {0.f, 0.f}, o[2][8];
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int j = 0; j < 8; j++) o[h][j] = 0.f;
                // the first AB positions of each group were DMA'd into LDS by this wave
                px_wait_loads();
                {
                    float4 kk[AB][2], vv[AB][2];
                    bool in[AB];
#pragma unroll
                    for (int j = 0; j < AB; j++) {
                        in[j] = sp.s0 + gid + NG * j < sp.cend;
                        kk[j][0] = px_u2f(kvb[wave][j][0][lane]);
                        kk[j][1] = px_u2f(kvb[wave][j][1][lane]);
                        vv[j][0] = px_u2f(kvb[wave][j][2][lane]);
                        vv[j][1] = px_u2f(kvb[wave][j][3][lane]);
                    }
                    px_fold_n<AB>(q, kk, vv, in, a.scale, m, lsum, o);
                }
                // longer splits continue in register batches.  0.6B: two per pass,
                // both batches' loads issued together, so the second one's memory
                // latency passes during the first one's fold (block-uniform loop;
                // a second batch wholly past the split is loaded from position 0,
                // which stays in L2, and skipped).  1.7B (fewer registers per
                // wave): one batch at a time.
                if (!DEEP) {
                    const int ln = px_lane_here(), lgl = ln & 15, lgid = wave * 4 + (ln >> 4);
                    for (int pb = sp.s0 + lgid + NG * AB; pb < sp.cend; pb += NG * AB) {
                        PxKv<AB> kv;
                        kv.load(kcl, vcl, lgl, pb, NG, sp.cend);
                        bool in[AB];
#pragma unroll
                        for (int j = 0; j < AB; j++) in[j] = pb + NG * j < sp.cend;
                        px_fold_n<AB>(q, kv.k, kv.v, in, a.scale, m, lsum, o);
                    }
                }
                for (int b0 = sp.s0 + NG * AB; DEEP && b0 < sp.cend; b0 += 2 * NG * AB) {
                    const int b1 = b0 + NG * AB;
                    PxKv<AB> k0, k1;
                    k0.load_all(kcl, vcl, gl, b0 + gid, NG, sp.cend);
                    k1.load_all(kcl, vcl, gl, b1 + gid, NG, sp.cend);
                    bool in0[AB], in1[AB];
#pragma unroll
                    for (int j = 0; j < AB; j++) {
                        in0[j] = b0 + gid + NG * j < sp.cend;
                        in1[j] = b1 + gid + NG * j < sp.cend;
                    }
                    px_fold_n<AB>(q, k0.k, k0.v, in0, a.scale, m, lsum, o);
                    if (b1 < sp.cend) px_fold_n<AB>(q, k1.k, k1.v, in1, a.scale, m, lsum, o);
                }
                if (sp.last && gid == 0) {   // position pos: this step's k/v
                    const float4 *kn = reinterpret_cast<const float4 *>(&S.kr[gl * 8]);
                    const float4 *vn = reinterpret_cast<const float4 *>(&S.vr[gl * 8]);
                    px_fold(q, kn[0], kn[1], vn[0], vn[1], a.scale, m, lsum, o);
                }
                mark(3);
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    if (gl == 0) { S.sm_m[gid][h] = m[h]; S.sm_l[gid][h] = lsum[h]; }
#pragma unroll
                    for (int j = 0; j < 8; j++) S.sm_o[gid][h][gl * 8 + j] = o[h][j];
                }
            }
            px_sync();
            if (sp.active && tid < 256) {
                const int h = tid >> 7, d = tid & 127;
                float M = -INFINITY;
#pragma unroll
                for (int i = 0; i < NG; i++) M = fmaxf(M, S.sm_m[i][h]);
                float Lh = 0.0f, acc = 0.0f;
#pragma unroll
                for (int i = 0; i < NG; i++) {
                    // M is finite (every group of a split below the last folds
                    // positions, group 0 of the last one folds pos): a group
                    // without positions (m = -inf) gets exp(-inf) = 0
                    const float e = __expf(S.sm_m[i][h] - M);
                    Lh = fmaf(S.sm_l[i][h], e, Lh);
                    acc = fmaf(S.sm_o[i][h][d], e, acc);
                }
                u64 *dst = a.xa + ((par * WG + g) * QK_PX_MAX_SPLIT + r) * (long)QK_PX_PART + h * 130;
                px_put_local(dst + 2 + d, acc, T + 1u);
                if (d == 0) {
                    px_put_local(dst, M, T + 1u);
                    px_put_local(dst + 1, Lh, T + 1u);
                }
            }
            // The K/V row stored at pos is read by other blocks of this XCD in
            // later steps; retire the stores before this wave writes anything
            // those blocks can depend on.
            if (sp.last && (wave == 2 || wave == 3)) px_wait_loads();
            mark(4);
            if constexpr (!DEEP) {
                // the fold's reads of this wave's K/V buffer are complete and its
                // K/V DMA has landed (an inactive block never waited for it)
                px_wait_loads();
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                uint4(*fl)[64] = reinterpret_cast<uint4(*)[64]>(&kvb[wave][0][0][0]);
                const uint16_t *wl = Wf(l) + (long)(wave * FB + FB1 + FR) * H + lane * 8;
#pragma unroll
                for (int b = 0; b < FL; b++)
#pragma unroll
                    for (int c = 0; c < SEGH; c++)
                        __builtin_amdgcn_global_load_lds(wl + (long)b * H + c * 512, &fl[b * SEGH + c][0], 16, 0, 0);
            }
            wf.load(Wf(l), H, wave, lane);

            // ---- O: this block's rows of W_o over the group's columns (merged attention output in S.att) ----
            px_sync();
            px_sync();
            if (S.abort_) return;
            if (DEEP) wd.load(Wd(l), I, wave, lane);
            mark(5);
            {
                float y[SO / 2 / NCW];
                wo.dot(S.att, y, lane);
                mark(6);
                if ((lane & 31) == 0) {
                    u64 *dst = a.xo + (par * WG + g) * H + SO * r;
                    const int ln = px_lane_here();
#pragma unroll
                    for (int i = 0; i < SO / 2 / NCW; i++) {
                        unsigned ro = (unsigned)SlabO::row(wave, i, ln);
                        asm volatile("" : "+v"(ro));   // no per-lane address kept across the loop
                        px_put_global(dst + ro, y[i], T + 2u);
                    }
                }
            }
            mark(7);

            // ---- F: gate|up rows of the group + SwiGLU (qwen_asr_decoder.c:463-466) ----
            px_sync();
            if (!DEEP) wf2.load(Wf(l) + (long)FB1 * H, H, wave, lane);   // FR rows
            px_sync();
            if (S.abort_) return;
            if (DEEP) wq.load(Wq(l + 1 < L ? l + 1 : 0), H, wave, lane);
            {
                float y[FB];
                if constexpr (DEEP) {
                    wf.dot(S.xn, y, lane);
                } else {
                    float y1[FB1], y2[FR], y3[FL];
                    wf.dot(S.xn, y1, lane);
                    wf2.dot(S.xn, y2, lane);
                    // the FL rows in LDS: PxSlab::dot's sums in the same order
                    px_wait_loads();
                    const uint4(*fl)[64] = reinterpret_cast<const uint4(*)[64]>(&kvb[wave][0][0][0]);
                    const int cl = lane * 8;
#pragma unroll
                    for (int b = 0; b < FL; b++) y3[b] = 0.0f;
#pragma unroll
                    for (int c = 0; c < SEGH; c++) {
                        float xv[8];
                        const float4 p0 = *reinterpret_cast<const float4 *>(S.xn + c * 512 + cl);
                        const float4 p1 = *reinterpret_cast<const float4 *>(S.xn + c * 512 + cl + 4);
                        xv[0] = p0.x; xv[1] = p0.y; xv[2] = p0.z; xv[3] = p0.w;
                        xv[4] = p1.x; xv[5] = p1.y; xv[6] = p1.z; xv[7] = p1.w;
#pragma unroll
                        for (int b = 0; b < FL; b++) y3[b] = dot8_bf16(fl[b * SEGH + c][lane], xv, y3[b]);
                    }
#pragma unroll
                    for (int b = 0; b < FL; b++) y3[b] = group_sum<64>(y3[b]);
#pragma unroll
                    for (int i = 0; i < FB; i++) y[i] = i < FB1 ? y1[i] : (i < FB1 + FR ? y2[i - FB1] : y3[i - FB1 - FR]);
                }
                mark(8);
                if (lane == 0) {
                    u64 *dst = a.xh + (par * WG + g) * HG + (RF / 2) * r;
#pragma unroll
                    for (int i = 0; i < RF / NCW; i += 2)
                        px_put_local(dst + SlabF::row(wave, i, 0) / 2, swiglu1(y[i], y[i + 1]), T + 4u);
                }
            }

            // ---- D: this block's rows of W_down over the group's columns (:467-468) ----
            if (!PxShared<H, I, NCW>::EARLY_POLL) px_sync();
            if (!DEEP) wd.load(Wd(l), I, wave, lane);
            px_sync();
            if (S.abort_) return;
            {
                float y[SO / 4 / NCW];
                wd.dot(S.hs, y, lane);
                mark(9);
                if ((lane & 15) == 0) {
                    u64 *dst = a.xd + (par * WG + g) * H + SO * r;
                    const int ln = px_lane_here();
#pragma unroll
                    for (int i = 0; i < SO / 4 / NCW; i++) {
                        unsigned ro = (unsigned)SlabD::row(wave, i, ln);
                        asm volatile("" : "+v"(ro));   // no per-lane address kept across the loop
                        px_put_global(dst + ro, y[i], T + 5u);
                    }
                }
            }
            // 1.7B: the next W_q is issued once the down partials are out, so the
            // D-stage hand-over queues behind W_down only (C3 1002.8 -> 1007.2 tok/s;
            // the x-update hand-over before Q then waits behind W_q instead)
            if (!DEEP) wq.load(Wq(l + 1 < L ? l + 1 : 0), H, wave, lane);
            {   // the next layer's operands (after the last layer: layer 0 of the next step)
                const int ln = l + 1 < L ? l + 1 : 0;
                const PxSplit sn(l + 1 < L ? pos : pos + 1, r);
                if (DEEP) px_kv_dma<AB>(kvb[wave], Kc(ln), Vc(ln), gl, sn.s0 + gid, NG, sn.cend, sn.active);
            }
        }
        // the first LM-head rows, issued before the final hand-over
        uint4 lmw[LMR][SEGH];
#pragma unroll
        for (int j = 0; j < LMR; j++) {
            const int row = lrow(wave, j);
#pragma unroll
            for (int c = 0; c < SEGH; c++)
                lmw[j][c] = px_ld16(a.emb + (long)min(row, lm1 - 1) * H + c * 512, (unsigned)lane * 16u);
        }

        // ---- LM head: argmax over this block's rows of the tied embedding (qwen_argmax_matvec_bf16, :518-543) ----
        px_sync();
        px_sync();
        if (S.abort_) return;
        {
            float bv = -1e30f;
            int bi = 0x7fffffff;
            for (int k = wave; k < lmn; k += NCW) {
                uint4 nx[LMR][SEGH];
                const bool more = k + NCW < lmn;
                if (more) {
#pragma unroll
                    for (int j = 0; j < LMR; j++) {
                        const int row = lrow(k + NCW, j);
#pragma unroll
                        for (int c = 0; c < SEGH; c++)
                            nx[j][c] = px_ld16(a.emb + (long)min(row, lm1 - 1) * H + c * 512, (unsigned)lane * 16u);
                    }
                }
                float acc[LMR];
#pragma unroll
                for (int j = 0; j < LMR; j++) acc[j] = 0.0f;
#pragma unroll
                for (int c = 0; c < SEGH; c++) {
                    float xv[8];
                    const float4 p0 = *reinterpret_cast<const float4 *>(&S.xn[c * 512 + lane * 8]);
                    const float4 p1 = *reinterpret_cast<const float4 *>(&S.xn[c * 512 + lane * 8 + 4]);
                    xv[0] = p0.x; xv[1] = p0.y; xv[2] = p0.z; xv[3] = p0.w;
                    xv[4] = p1.x; xv[5] = p1.y; xv[6] = p1.z; xv[7] = p1.w;
#pragma unroll
                    for (int j = 0; j < LMR; j++) acc[j] = dot8_bf16(lmw[j][c], xv, acc[j]);
                }
                reduce_rows<LMR, 1>(acc, lane);   // lane groups of 64/LMR hold row lane / (64/LMR)
                const int row = lrow(k, lane / (64 / LMR));
                if (row < lm1) {
                    if (a.logits && (lane % (64 / LMR)) == 0) a.logits[row] = acc[0];
                    if (argmax_better(acc[0], row, bv, bi)) { bv = acc[0]; bi = row; }
                }
                if (more) {
#pragma unroll
                    for (int j = 0; j < LMR; j++)
#pragma unroll
                        for (int c = 0; c < SEGH; c++) lmw[j][c] = nx[j][c];
                }
            }
            wave_argmax(bv, bi);
            if (lane == 0) { S.wv[wave] = bv; S.wi[wave] = bi; }
        }
        px_sync();
        if (tid == 0) {
            float bv = S.wv[0];
            int bi = S.wi[0];
            for (int w = 1; w < NCW; w++)
                if (argmax_better(S.wv[w], S.wi[w], bv, bi)) { bv = S.wv[w]; bi = S.wi[w]; }
            const unsigned Tc = tstep + QK_PX_TPL * (unsigned)L;
            px_put_global(a.xc + b, bv, Tc);
            px_put_global(a.xc + QK_PX_BLOCKS + b, __int_as_float(bi), Tc);
        }
        // ---- T: the sync wave reduces the candidates ----
        px_sync();
        px_sync();
        if (S.abort_) return;
    }
}

template <int H, int I, int NCW>
__global__ __launch_bounds__((NCW + 1) * 64, 1) void px_decode(qk_persist_args a) {
    __shared__ __attribute__((aligned(16))) PxShared<H, I, NCW> S;
    __shared__ __attribute__((aligned(16))) PxKvLds<NCW> kvb;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (wave == NCW) px_sync_role<H, I, NCW>(a, S, lane);
    else px_compute_role<H, I, NCW>(a, S, kvb, wave, lane);
}

// 0.6B: hidden 1024, intermediate 3072, 4 compute waves; 1.7B: 2048 / 6144, 8.
#define PX_K06 px_decode<1024, 3072, 4>
#define PX_K17 px_decode<2048, 6144, 8>

static const void *px_kernel(int hidden, int inter, int *threads) {
    if (hidden == 1024 && inter == 3072) { *threads = 5 * 64; return (const void *)PX_K06; }
    if (hidden == 2048 && inter == 6144) { *threads = 9 * 64; return (const void *)PX_K17; }
    return nullptr;
}

// The grid is one block per CU and every block must be resident at once: the
// device must have exactly 256 CUs and a block must fit on a CU, and at most one
// may (the LDS of a block is more than half a CU's), so the dispatcher spreads
// the grid one block per CU.
extern "C" int qk_persist_supported(int hidden, int inter, int heads, int kv_heads, int device) {
    int threads = 0;
    const void *k = px_kernel(hidden, inter, &threads);
    if (!k || heads != 16 || kv_heads != QK_PX_XCD) return 0;
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
    if (cus != QK_PX_BLOCKS) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k, threads, 0) != hipSuccess || per != 1) return 0;
    return 1;
}

extern "C" int qk_persist_launch(const qk_persist_args *a, int hidden, int inter, hipStream_t s) {
    int threads = 0;
    const void *k = px_kernel(hidden, inter, &threads);
    if (!a || !k || a->n_steps <= 0 || a->layers <= 0 || a->epoch == 0u) return QWEN_HIP_EINVAL;
    if (a->trace && (10 * a->layers + 4 > QK_PX_TRACE_CW || QK_PX_TRACE_CW + 10 * a->layers > QK_PX_TRACE_XU ||
                     QK_PX_TRACE_XU + 2 * a->layers + 1 > QK_PX_TRACE))
        return QWEN_HIP_EINVAL;
    if (a->first_tok < 0 && !a->x_in) return QWEN_HIP_EINVAL;
    if (a->first_tok >= a->vocab || a->pos0 < 0 || a->pos0 + a->n_steps > a->cap) return QWEN_HIP_EINVAL;
    qk_persist_args copy = *a;
    void *args[] = {&copy};
    // An ordinary launch on the caller's stream: residency of the whole grid is
    // checked by the kernel's own check-in, under the same bounded wait as
    // every other hand-over.
    if (hipLaunchKernel(k, dim3(QK_PX_BLOCKS), dim3(threads), args, 0, s) != hipSuccess) return QWEN_HIP_EDEVICE;
    return 0;
}
