"""Launch planners of the prefill kernels (host code, no GPU needed):
qk_gemm_plan_for (tile shape, kernel, split-K slices of the projection GEMMs) and
qk_attn_prefill_plan (key chunk per block of the prefill attention).  Their
invariants are what the kernels rely on: slices cover K exactly once in whole
64-deep k tiles, at most 16 of them (the partial-sum consumers' bound); key
chunks are whole 32-key tiles, cover the longest query tile, and no block
walks more than max(256, a sixth of it) keys, except that with four or more
query tiles and up to 2048 keys a split covers a quarter of the longest range
at least, a single query tile (a short continuation prefill) splits its keys
64 at a time at least, and a prefill with at least two (64-query tile, kv
head) blocks per CU is not split at all."""
import ctypes as C

import pytest


class GemmPlan(C.Structure):
    _fields_ = [("bm", C.c_int), ("nsplit", C.c_int), ("kc", C.c_int), ("bn", C.c_int), ("nst", C.c_int)]


SHAPES = [(M, N, K) for M in (1, 17, 31, 32, 33, 64, 65, 401, 512, 513, 1515, 8191)
          for N in (1000, 1024, 2048, 4096, 6144, 12288) for K in (520, 1024, 2048, 3072, 6144)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_plan_invariants(qa, M, N, K):
    p = GemmPlan()
    qa.lib().qk_gemm_plan_for(M, N, K, C.byref(p))
    def fills(bm):   # bm x 256 tiles alone fill the CUs, last round >= 85 % used
        wt = -(-M // bm) * (N // 256)
        return M > 512 and N % 256 == 0 and K % 32 == 0 and wt >= 256 and wt * 100 >= -(-wt // 256) * 256 * 85
    ring = N % 128 == 0 and K % 32 == 0
    if fills(256):                                                     # wide tiles, never split
        assert (p.bm, p.bn, p.nsplit, p.nst) == (256, 256, 1, 0)
    elif fills(128):
        assert (p.bm, p.bn, p.nsplit, p.nst) == (128, 256, 1, 0)
    elif ring and M > 512:                                             # LDS ring, 128 x 128 on 3 stages
        assert (p.bm, p.bn, p.nst) == (128, 128, 3)
    elif ring:                                                         # LDS ring, 4 stages
        assert (p.bn, p.nst) == (128, 4) and p.bm == (32 if M <= 32 else 64)
    else:                                                              # register-staged
        assert p.bn == 128 and p.nst == 0 and p.bm == (32 if M <= 32 else 64 if M <= 512 else 128)
    assert p.kc > 0 and p.kc % 64 == 0
    assert 1 <= p.nsplit <= 16
    assert p.kc * p.nsplit >= K and p.kc * (p.nsplit - 1) < K       # every slice non-empty, K covered once
    tiles = -(-M // p.bm) * -(-N // p.bn)
    if p.nst == 3:
        # 128 x 128 tiles: two splits per 4096 of K (an even count)
        want = min(2 * -(-K // 4096), 16, -(-K // 64))
        assert p.kc == -(-(-(-K // 64)) // want) * 64
    elif p.nst:
        # about 224 blocks, and k walks of 2048 or more in two halves at least
        # (within the 16-split cap and whole 64-deep k tiles)
        want = min(max(-(-224 // tiles), 2 if K >= 2048 else 1), 16, -(-K // 64))
        assert p.kc == -(-(-(-K // 64)) // want) * 64                 # whole k tiles, want slices at most
    elif tiles >= 256:
        assert p.nsplit == 1                                           # the grid alone fills the chip


@pytest.mark.parametrize("epi", [2, 3])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_plan_swiglu_rope(qa, M, N, K, epi):
    """A SwiGLU product (epilogue 2) and the Q|K|V product with the RoPE
    epilogue (3) split K only to fill the chip: SwiGLU's split partials (twice
    its output) need a reduce pass, and the RoPE epilogue runs on one split;
    above 512 rows on the LDS ring a SwiGLU product takes the 128 x 128 tiles
    on 3 stages of the STORE products and the Q|K|V + RoPE product the 64 x
    128 tiles on 4 stages; otherwise they are planned like any other product."""
    lib = qa.lib()
    p, q = GemmPlan(), GemmPlan()
    lib.qk_gemm_plan_for(M, N, K, C.byref(p))
    lib.qk_gemm_plan_epi(M, N, K, epi, C.byref(q))
    if epi == 3 and p.nst and M > 512:
        assert (q.bm, q.bn, q.nst) == (64, 128, 4)
    else:
        assert (q.bm, q.bn, q.nst) == (p.bm, p.bn, p.nst)
    assert q.kc * q.nsplit >= K and q.kc * (q.nsplit - 1) < K and q.kc % 64 == 0
    if p.nst:
        tiles = -(-M // q.bm) * (N // q.bn)
        want = min(-(-224 // tiles), 16, -(-K // 64))
        assert q.kc == -(-(-(-K // 64)) // want) * 64
    else:
        assert (q.nsplit, q.kc) == (p.nsplit, p.kc)
    # the fused Q|K|V + RoPE kernel takes exactly the one-split 64 x 128 ring plans
    assert lib.qk_gemm_rope_fusable(C.byref(q)) == int((q.nst, q.bm, q.bn, q.nsplit) == (4, 64, 128, 1))


def kmax_of(seq_q, seq_k, q_offset):
    nq = -(-seq_q // 64)
    return max(min(seq_k, q_offset + min(seq_q, (t + 1) * 64)) for t in range(nq))


@pytest.mark.parametrize("seq_q,seq_k,q_offset", [(1, 1, 0), (31, 1000, 969), (64, 64, 0), (401, 401, 0),
                                                  (1515, 1515, 0), (6400, 6400, 0), (8191, 8191, 0),
                                                  (26, 1024, 998), (100, 5000, 4900), (2048, 4096, 2048)])
def test_attention_plan_invariants(qa, seq_q, seq_k, q_offset):
    lib = qa.lib()
    lib.qk_attn_prefill_plan.restype = C.c_size_t
    lib.qk_attn_prefill_plan.argtypes = [C.c_int] * 5 + [C.POINTER(C.c_int)] * 2
    chunk, nsplit = C.c_int(), C.c_int()
    part = lib.qk_attn_prefill_plan(seq_q, seq_k, q_offset, 16, 8, C.byref(chunk), C.byref(nsplit))
    kmax = kmax_of(seq_q, seq_k, q_offset)
    assert chunk.value > 0 and chunk.value % 32 == 0
    assert nsplit.value >= 1 and chunk.value * nsplit.value >= kmax and chunk.value * (nsplit.value - 1) < kmax
    cap = max(256, -(-(-(-kmax // 6)) // 32) * 32)
    q4 = (kmax // 4 + 16) // 32 * 32                 # a quarter of the range, nearest 32
    nq = -(-seq_q // 64)
    assert chunk.value <= max(cap, q4, -(-kmax // 32) * 32)
    if nq >= 4 and kmax <= 2048:                      # several query tiles: quarter-range splits at least
        assert chunk.value >= min(q4, -(-kmax // 32) * 32)
    if nq * 8 >= 512:
        assert nsplit.value == 1
    if nq == 1:                                       # one query tile: 64-key splits at least
        assert chunk.value >= min(64, -(-kmax // 32) * 32)
    # partial buffer: (o[128], m, l) per split, query and head, only when split
    assert part == (nsplit.value * seq_q * 16 * 130 if nsplit.value > 1 else 0)


class RopeArgs(C.Structure):
    _fields_ = [("qkv", C.c_void_p), ("nsum", C.c_int), ("pstride", C.c_long), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p), ("eps", C.c_float), ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
                ("k_cache", C.c_void_p), ("v_cache", C.c_void_p), ("cap", C.c_int), ("pos_dev", C.c_void_p),
                ("start", C.c_int), ("S", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int), ("q_out", C.c_void_p)]


@pytest.mark.parametrize("field", ["qkv", "q_norm", "rope_cos", "k_cache", "q_out"])
def test_rope_launches_refuse_unaligned_pointers(qa, field):
    """The q/k norm + RoPE kernels move 16-byte vectors: a pointer off a
    16-byte boundary, or split partials a non-multiple of 4 floats apart, is
    refused with QWEN_HIP_EINVAL before anything is launched (host-side
    checks; the addresses are never dereferenced)."""
    lib = qa.lib()
    lib.qk_rope_append_launch.argtypes = [C.c_void_p, C.c_void_p]
    lib.qk_gemm_rope_launch.argtypes = [C.c_void_p] * 3 + [C.c_int] * 2 + [C.c_void_p] * 3
    base = 1 << 20
    good = {f: base + (i << 16) for i, f in enumerate(["qkv", "q_norm", "k_norm", "rope_cos", "rope_sin", "k_cache",
                                                       "v_cache", "q_out"])}

    def args(**over):
        v = dict(good, **over)
        return RopeArgs(v["qkv"], 1, 0, v["q_norm"], v["k_norm"], 1e-6, v["rope_cos"], v["rope_sin"], v["k_cache"],
                        v["v_cache"], 64, None, 0, 64, 16, 8, v["q_out"])
    bad = args(**{field: good[field] + 4})
    assert lib.qk_rope_append_launch(C.byref(bad), None) == -1
    split = args()
    split.nsum, split.pstride = 2, 64 * 4096 + 2
    assert lib.qk_rope_append_launch(C.byref(split), None) == -1
    if field != "qkv":               # the fused kernel reads the product from its own tiles
        p = GemmPlan(64, 1, 1024, 128, 4)
        assert lib.qk_gemm_rope_launch(base, base, base, 64, 1024, C.byref(p), C.byref(bad), None) == -1


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_linear_op_workspace(qa, M, N, K):
    """The op-level linear (qwen_hip_linear_nobias_bf16 and its no-alloc
    variant) splits K only where its output tiles number fewer than 256 and
    the width is even: its workspace is the bf16 hi/lo halves of x (4*M*K
    bytes, rounded up to 256) plus, for such small grids only, the split-K
    partials.  A 1024-row product into 4096 columns therefore fits the
    no-alloc entry point's 32 MiB array (4 MiB of x halves, no partials)."""
    lib = qa.lib()
    lib.qk_linear_ws_bytes.restype = C.c_size_t
    p = GemmPlan()
    lib.qk_gemm_plan_for(M, N, K, C.byref(p))
    tiles = -(-M // p.bm) * -(-N // p.bn)
    halves = -(-4 * M * K // 256) * 256
    need = lib.qk_linear_ws_bytes(M, K, N)
    if tiles >= 256 or N % 2 or p.nsplit == 1:
        assert need == halves
    else:
        assert need == halves + 4 * p.nsplit * M * N


def test_linear_op_workspace_advice_case(qa):
    lib = qa.lib()
    lib.qk_linear_ws_bytes.restype = C.c_size_t
    assert lib.qk_linear_ws_bytes(1024, 1024, 4096) == 4 * 1024 * 1024      # x halves only
    assert lib.qk_linear_ws_bytes(1024, 1024, 4096) <= lib.qwen_hip_linear_noalloc_max_bytes()
