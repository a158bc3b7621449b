"""Op-level parity: each qwen_asr_kernels.h operator of the HIP library,
called through the C ABI on device memory, against the CPU oracle on the same
seeded inputs.  Tolerances are stated per test; fp32 accumulation order
differs between the GPU and CPU, so GEMV checks use the rounding bound
4*K*2^-24*sum|w*x| (and the bf16 hi/lo GEMM adds 2^-16*sum|w*x|)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    return t.cpu().numpy()


def ptr(t):
    return t.data_ptr()


# the GEMV sweep (rows x cols), plus the true 1.7B 2048x2048
SWEEP = [(2048, 1024), (1024, 2048), (6144, 1024), (1024, 3072), (151936, 1024), (4096, 2048),
         (2048, 4096), (12288, 2048), (2048, 6144), (151936, 2048), (2048, 2048)]


@pytest.mark.parametrize("rows,cols", SWEEP)
def test_gemv_sweep(P, qa, gpu, rows, cols):
    W = P.synth_bf16(rows * cols, 0, 9000 + rows + cols).reshape(rows, cols)
    x = P.synth_uniform(cols, 0, 9100 + cols)
    dW, dx = dev(gpu, W.view(np.int16)), dev(gpu, x)
    dy = gpu.empty(rows, dtype=gpu.float32, device="cuda")
    qa.check(qa.lib().qwen_hip_linear_nobias_bf16(ptr(dy), ptr(dx), ptr(dW), 1, cols, rows, None), "gemv")
    gpu.cuda.synchronize()
    y = host(dy)
    yo = np.empty(rows, np.float32)
    P.orc_lib().orc_linear_bf16(yo, x, W, 1, cols, rows)
    Wf = P.bf16_to_f32(W)
    absum = np.abs(Wf) @ np.abs(x)
    bound = 8 * cols * 2.0 ** -24 * absum + 1e-12
    assert np.all(np.abs(y - yo) <= bound), float(np.max(np.abs(y - yo) / bound))


@pytest.mark.parametrize("hidden,qd,kvd", [(1024, 2048, 1024), (2048, 2048, 1024)])
def test_linear_qkv(P, qa, gpu, hidden, qd, kvd):
    """qwen_hip_linear_nobias_bf16_qkv (qwen_asr_kernels.h:45-49): the three
    seq = 1 products of one input row, each against the reference's own
    qwen_linear_nobias_bf16 (oracle/_ref) and the oracle, at the GEMV rounding
    bound."""
    Ws = [P.synth_bf16(n * hidden, 2, 9400 + i).reshape(n, hidden) for i, n in enumerate((qd, kvd, kvd))]
    x = P.synth_uniform(hidden, 2, 9450 + hidden)
    dW = [dev(gpu, W.view(np.int16)) for W in Ws]
    dx = dev(gpu, x)
    dq = gpu.empty(qd, dtype=gpu.float32, device="cuda")
    dk = gpu.empty(kvd, dtype=gpu.float32, device="cuda")
    dv = gpu.empty(kvd, dtype=gpu.float32, device="cuda")
    qa.check(qa.lib().qwen_hip_linear_nobias_bf16_qkv(ptr(dq), ptr(dk), ptr(dv), ptr(dx), ptr(dW[0]), ptr(dW[1]),
                                                      ptr(dW[2]), hidden, qd, kvd, None), "qkv")
    gpu.cuda.synchronize()
    ref = P.ref_lib() if P.ref_available() else None
    for W, d in zip(Ws, (dq, dk, dv)):
        y, n = host(d), W.shape[0]
        yo = np.empty(n, np.float32)
        P.orc_lib().orc_linear_bf16(yo, x, W, 1, hidden, n)
        bound = 8 * hidden * 2.0 ** -24 * (np.abs(P.bf16_to_f32(W)) @ np.abs(x)) + 1e-12
        assert np.all(np.abs(y - yo) <= bound)
        if ref is not None:
            yr = np.empty(n, np.float32)
            ref.qwen_linear_nobias_bf16(yr, x, np.ascontiguousarray(W), 1, hidden, n)
            assert np.all(np.abs(y - yr) <= bound)


# covers every tiling of qk_gemm_plan_for: 32 / 64 / 128-row blocks, split-K
# with its reduce pass (and the odd-N case that cannot split), one split
@pytest.mark.parametrize("M,N,K", [(2, 64, 256), (31, 4096, 1024), (64, 1024, 2048), (401, 6144, 1024),
                                   (130, 2048, 6144), (7, 100, 200), (33, 101, 64), (1000, 1024, 1024),
                                   (2100, 4096, 256), (30, 1024, 3072)])
def test_gemm_hilo(P, qa, gpu, M, N, K):
    W = P.synth_bf16(N * K, 1, 9200 + N).reshape(N, K)
    x = P.synth_f32(M * K, 1, 9300 + M).reshape(M, K)
    dW, dx = dev(gpu, W.view(np.int16)), dev(gpu, x)
    dy = gpu.empty((M, N), dtype=gpu.float32, device="cuda")
    qa.check(qa.lib().qwen_hip_linear_nobias_bf16(ptr(dy), ptr(dx), ptr(dW), M, K, N, None), "gemm")
    gpu.cuda.synchronize()
    y = host(dy)
    yo = np.empty((M, N), np.float32)
    P.orc_lib().orc_linear_bf16(yo, x, W, M, K, N)
    absum = np.abs(x) @ np.abs(P.bf16_to_f32(W)).T
    bound = (2.0 ** -16 + 8 * K * 2.0 ** -24) * absum + 1e-12
    assert np.all(np.abs(y - yo) <= bound), float(np.max(np.abs(y - yo) / bound))


class GemmPlan(C.Structure):
    _fields_ = [("bm", C.c_int), ("nsplit", C.c_int), ("kc", C.c_int), ("bn", C.c_int), ("nst", C.c_int)]


# the three epilogues of the prefill GEMM on every tile shape and kernel it
# plans: 256 x 256 and 128 x 256 (wide direct-to-LDS rings; M not a multiple
# of the tile, k walks shorter than the ring), 64 x 128 and 32 x 128 on the
# 4-stage ring (one split, and split with the partials summed by the reduce
# pass with the epilogue), 128 x 128 on the 3-stage ring above 512 rows (four
# 1536-deep splits of K 6144), register-staged 64 x 128 and split 128 x 128
# (N not a multiple of 128, K not of 32)
@pytest.mark.parametrize("M,N,K,bm,bn,nst", [(1000, 16384, 64, 256, 256, 0), (4000, 4096, 96, 256, 256, 0),
                                             (4000, 2048, 96, 128, 256, 0), (2000, 4096, 32, 128, 256, 0),
                                             (401, 6144, 1024, 64, 128, 4), (401, 1024, 2048, 64, 128, 4),
                                             (700, 1024, 6144, 128, 128, 3),
                                             (31, 4096, 1024, 32, 128, 4), (100, 1000, 512, 64, 128, 0),
                                             (1515, 1000, 520, 128, 128, 0)])
@pytest.mark.parametrize("epi", [0, 1, 2])
def test_gemm_epilogues(P, qa, gpu, M, N, K, bm, bn, nst, epi):
    lib = qa.lib()
    p = GemmPlan()
    lib.qk_gemm_plan_for(M, N, K, C.byref(p))
    assert (p.bm, p.bn, p.nst) == (bm, bn, nst), (p.bm, p.bn, p.nst, p.nsplit)
    check_gemm(P, qa, gpu, M, N, K, p, epi)


# the 128 x 128 tiles on the 3-stage ring that a SwiGLU or STORE product above
# 512 rows is planned on, with each epilogue, in one split (N 4096: 384 tiles) and in two
# (N 2048: 192 tiles; STORE partials, then the reduce pass with the epilogue);
# a partial last row tile (1515 = 11 x 128 + 107)
@pytest.mark.parametrize("N,ns", [(4096, 1), (2048, 2)])
@pytest.mark.parametrize("epi", [0, 1, 2])
def test_gemm_ring128(P, qa, gpu, N, ns, epi):
    M, K = 1515, 1024
    p = GemmPlan()
    qa.lib().qk_gemm_plan_epi(M, N, K, 2, C.byref(p))
    assert (p.bm, p.bn, p.nst, p.nsplit) == (128, 128, 3, ns)
    check_gemm(P, qa, gpu, M, N, K, p, epi)


def check_gemm(P, qa, gpu, M, N, K, p, epi):
    """Run qk_gemm_launch with plan p and epilogue epi (split plans: STORE
    partials, then the reduce pass with the epilogue) against an fp64 product
    of the same bf16 hi/lo operands, within the fp32 accumulation bound."""
    lib = qa.lib()
    W = P.synth_bf16(N * K, 2, 9400 + N).reshape(N, K)
    x = P.synth_f32(M * K, 2, 9500 + M).reshape(M, K)
    hi = P.f32_to_bf16(x)
    lo = P.f32_to_bf16(x - P.bf16_to_f32(hi))
    prod = (P.bf16_to_f32(hi).astype(np.float64) + P.bf16_to_f32(lo)) @ P.bf16_to_f32(W).astype(np.float64).T
    absum = np.abs(x).astype(np.float64) @ np.abs(P.bf16_to_f32(W)).astype(np.float64).T
    bound = 4 * K * 2.0 ** -24 * absum + 1e-12
    y0 = P.synth_f32(M * N, 2, 9600 + M).reshape(M, N)
    dh, dl, dW = dev(gpu, hi.view(np.int16)), dev(gpu, lo.view(np.int16)), dev(gpu, W.view(np.int16))
    lib.qk_gemm_launch.argtypes = [C.c_void_p] * 3 + [C.c_int] * 3 + [C.c_void_p, C.c_int] + [C.c_void_p] * 4
    lib.qk_gemm_reduce_launch.argtypes = [C.c_void_p] + [C.c_int] * 4 + [C.c_void_p] * 4
    split = p.nsplit > 1
    dy = dev(gpu, y0) if epi == 1 else gpu.zeros((M, N), dtype=gpu.float32, device="cuda")
    oh = gpu.zeros((M, N // 2), dtype=gpu.int16, device="cuda")
    ol = gpu.zeros((M, N // 2), dtype=gpu.int16, device="cuda")
    outs = (None, ptr(oh), ptr(ol)) if epi == 2 else (ptr(dy), None, None)
    if split:
        part = gpu.empty((p.nsplit, M, N), dtype=gpu.float32, device="cuda")
        qa.check(lib.qk_gemm_launch(ptr(dh), ptr(dl), ptr(dW), M, N, K, C.byref(p), 0, ptr(part), None, None,
                                    None), "gemm")
        qa.check(lib.qk_gemm_reduce_launch(ptr(part), p.nsplit, M, N, epi, *outs, None), "reduce")
    else:
        qa.check(lib.qk_gemm_launch(ptr(dh), ptr(dl), ptr(dW), M, N, K, C.byref(p), epi, *outs, None), "gemm")
    gpu.cuda.synchronize()
    if epi == 2:
        g, u = prod[:, 0::2], prod[:, 1::2]
        exp = g / (1.0 + np.exp(-g)) * u
        got = P.bf16_to_f32(host(oh).view(np.uint16)).astype(np.float64) + P.bf16_to_f32(host(ol).view(np.uint16))
        # product errors through silu(g) u (|d/dg| <= 1.1 |u|, |silu(g)| <= |g| + 0.3), plus
        # the hi + lo carry of the result (~2^-17 relative)
        tol = 1e-5 * np.abs(exp) + 1.2 * (np.abs(u) * bound[:, 0::2] + (np.abs(g) + 0.3) * bound[:, 1::2]) + 1e-9
        assert np.all(np.abs(got - exp) <= tol), float(np.max(np.abs(got - exp) / tol))
    else:
        exp = prod + (y0 if epi == 1 else 0.0)
        got = host(dy).astype(np.float64)
        tol = bound + (2.0 ** -23 * np.abs(exp) if epi == 1 else 0.0)
        assert np.all(np.abs(got - exp) <= tol), float(np.max(np.abs(got - exp) / tol))


class RopeArgs(C.Structure):
    _fields_ = [("qkv", C.c_void_p), ("nsum", C.c_int), ("pstride", C.c_long), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p), ("eps", C.c_float), ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
                ("k_cache", C.c_void_p), ("v_cache", C.c_void_p), ("cap", C.c_int), ("pos_dev", C.c_void_p),
                ("start", C.c_int), ("S", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int), ("q_out", C.c_void_p)]


# the Q|K|V GEMM with rope_append's work as its epilogue: bit for bit the
# GEMM (STORE) followed by rope_append, on a full and a partial last row tile,
# at a nonzero start position, for the 0.6B and 1.7B widths
@pytest.mark.parametrize("M,K,start", [(401, 1024, 37), (130, 2048, 0), (64, 1024, 900)])
def test_gemm_rope_epilogue(P, qa, gpu, M, K, start):
    lib = qa.lib()
    H, KVH, hd, cap = 16, 8, 128, 1024
    N = (H + 2 * KVH) * hd
    p = GemmPlan()
    lib.qk_gemm_plan_epi(M, N, K, 3, C.byref(p))
    # the plan fuses where the tiles fill the chip without a split (C1's 401
    # rows, 7 x 32 tiles); the kernel takes any M with one split
    assert lib.qk_gemm_rope_fusable(C.byref(p)) == (1 if M >= 385 else 0), (p.bm, p.bn, p.nst, p.nsplit)
    p = GemmPlan(64, 1, K, 128, 4)
    r = np.random.default_rng(M + K)
    W = P.synth_bf16(N * K, 3, 9700 + K).reshape(N, K)
    x = P.synth_f32(M * K, 3, 9800 + M).reshape(M, K)
    hi = P.f32_to_bf16(x)
    lo = P.f32_to_bf16(x - P.bf16_to_f32(hi))
    qn = (1 + 0.1 * r.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * r.standard_normal(hd)).astype(np.float32)
    cs = np.empty((cap, hd), np.float32)
    sn = np.empty((cap, hd), np.float32)
    P.orc_lib().orc_rope_table(cs, sn, cap, hd, 1e6)
    dh, dl, dW = dev(gpu, hi.view(np.int16)), dev(gpu, lo.view(np.int16)), dev(gpu, W.view(np.int16))
    dqn, dkn, dcs, dsn = dev(gpu, qn), dev(gpu, kn), dev(gpu, cs), dev(gpu, sn)
    outs = []
    for fused in (False, True):
        kc = gpu.full((KVH, cap, hd), 7.0, dtype=gpu.float32, device="cuda")
        vc = gpu.full((KVH, cap, hd), 7.0, dtype=gpu.float32, device="cuda")
        qo = gpu.full((M, H * hd), 7.0, dtype=gpu.float32, device="cuda")
        qkv = gpu.empty((M, N), dtype=gpu.float32, device="cuda")
        ra = RopeArgs(ptr(qkv), 1, M * N, ptr(dqn), ptr(dkn), 1e-6, ptr(dcs), ptr(dsn), ptr(kc), ptr(vc), cap, None,
                      start, M, H, KVH, ptr(qo))
        if fused:
            lib.qk_gemm_rope_launch.argtypes = [C.c_void_p] * 3 + [C.c_int] * 2 + [C.c_void_p] * 3
            qa.check(lib.qk_gemm_rope_launch(ptr(dh), ptr(dl), ptr(dW), M, K, C.byref(p), C.byref(ra), None), "fused")
        else:
            lib.qk_gemm_launch.argtypes = [C.c_void_p] * 3 + [C.c_int] * 3 + [C.c_void_p, C.c_int] + [C.c_void_p] * 4
            lib.qk_rope_append_launch.argtypes = [C.c_void_p, C.c_void_p]
            qa.check(lib.qk_gemm_launch(ptr(dh), ptr(dl), ptr(dW), M, N, K, C.byref(p), 0, ptr(qkv), None, None,
                                        None), "gemm")
            qa.check(lib.qk_rope_append_launch(C.byref(ra), None), "rope_append")
        gpu.cuda.synchronize()
        outs.append((host(kc), host(vc), host(qo)))
    for a, b, what in zip(outs[0], outs[1], ("k cache", "v cache", "q")):
        assert np.array_equal(a, b), what
    # the rows outside [start, start + M) are untouched
    assert np.all(outs[1][0][:, :start] == 7.0) and np.all(outs[1][0][:, start + M:] == 7.0)


# the prefill RMSNorm that completes the residual: x += part[0] + ... (split
# order), then hi/lo of rms_norm(x) * w; a wave per row above 1024 rows
# (16-byte pieces), a block per row below; every split count the planner uses
@pytest.mark.parametrize("S", [401, 1025])
@pytest.mark.parametrize("D", [1024, 2048])
@pytest.mark.parametrize("nsum", [0, 1, 2, 3])
def test_rmsnorm_split(P, qa, gpu, S, D, nsum):
    lib = qa.lib()
    lib.qk_rmsnorm_split_launch.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_long, C.c_void_p, C.c_int, C.c_int,
                                            C.c_float, C.c_void_p, C.c_void_p, C.c_void_p]
    r = np.random.default_rng(S + D + nsum)
    x = r.standard_normal((S, D)).astype(np.float32)
    part = r.standard_normal((max(nsum, 1), S, D)).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    dx, dp, dw = dev(gpu, x), dev(gpu, part), dev(gpu, w)
    hi = gpu.zeros((S, D), dtype=gpu.int16, device="cuda")
    lo = gpu.zeros((S, D), dtype=gpu.int16, device="cuda")
    qa.check(lib.qk_rmsnorm_split_launch(ptr(dx), ptr(dp) if nsum else None, nsum, S * D, ptr(dw), S, D, 1e-6,
                                         ptr(hi), ptr(lo), None), "rmsnorm_split")
    gpu.cuda.synchronize()
    v = x.copy()
    if nsum:
        ps = part[0].copy()
        for k in range(1, nsum):
            ps += part[k]
        v += ps
    assert np.array_equal(host(dx), v)                       # the same fp32 sums in the same order
    v64 = v.astype(np.float64)
    exp = v64 * w * (1.0 / np.sqrt((v64 * v64).mean(axis=1, keepdims=True) + 1e-6))
    got = P.bf16_to_f32(host(hi).view(np.uint16)).astype(np.float64) + P.bf16_to_f32(host(lo).view(np.uint16))
    # hi + lo carries ~2^-17 relative; rinv's sum is in another order (fp32)
    assert np.all(np.abs(got - exp) <= 1e-5 * np.abs(exp) + 1e-6), float(np.max(np.abs(got - exp)))


def test_elementwise_ops(P, qa, gpu):
    lib, orc = qa.lib(), P.orc_lib()
    r = np.random.default_rng(0)
    S, D, nh, hd = 5, 1024, 16, 128
    x = r.standard_normal((S, D)).astype(np.float32) * 2
    w = (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    # rms_norm, out-of-place and in place
    dx, dw = dev(gpu, x), dev(gpu, w)
    do = gpu.empty_like(dx)
    qa.check(lib.qwen_hip_rms_norm(ptr(do), ptr(dx), ptr(dw), S, D, 1e-6, None))
    qa.check(lib.qwen_hip_rms_norm(ptr(dx), ptr(dx), ptr(dw), S, D, 1e-6, None))
    exp = np.empty_like(x)
    orc.orc_rms_norm(exp, x, w, S, D, 1e-6)
    gpu.cuda.synchronize()
    np.testing.assert_allclose(host(do), exp, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(host(dx), exp, rtol=1e-5, atol=1e-6)
    # per-head norm + rope
    q = r.standard_normal((S, nh * hd)).astype(np.float32)
    wh = (1 + 0.1 * r.standard_normal(hd)).astype(np.float32)
    c = np.empty((9000, hd), np.float32)
    s = np.empty((9000, hd), np.float32)
    orc.orc_rope_table(c, s, 9000, hd, 1e6)
    pos = np.array([0, 5, 400, 4000, 8999])
    cs, ss = np.ascontiguousarray(c[pos]), np.ascontiguousarray(s[pos])
    # keep every device tensor referenced until the kernels ran: a temporary
    # freed after data_ptr() lets the caching allocator hand its block out again
    dq, dwh, dcs, dss = dev(gpu, q), dev(gpu, wh), dev(gpu, cs), dev(gpu, ss)
    qa.check(lib.qwen_hip_rms_norm_per_head(ptr(dq), ptr(dwh), S, nh, hd, 1e-6, None))
    qa.check(lib.qwen_hip_apply_rope_neox(ptr(dq), ptr(dcs), ptr(dss), S, nh, hd, None))
    e = q.copy()
    orc.orc_rms_norm_per_head(e, wh, S, nh, hd, 1e-6)
    orc.orc_apply_rope(e, cs, ss, S, nh, hd)
    gpu.cuda.synchronize()
    np.testing.assert_allclose(host(dq), e, rtol=1e-5, atol=2e-6)
    # swiglu, out-of-place and in place; add
    gu = r.standard_normal((3, 2 * 3072)).astype(np.float32) * 3
    dgu = dev(gpu, gu)
    dout = gpu.empty((3, 3072), dtype=gpu.float32, device="cuda")
    qa.check(lib.qwen_hip_swiglu_multiply(ptr(dout), ptr(dgu), 3, 3072, None))
    qa.check(lib.qwen_hip_swiglu_multiply(ptr(dgu), ptr(dgu), 3, 3072, None))
    eo = np.empty((3, 3072), np.float32)
    orc.orc_swiglu(eo, gu, 3, 3072)
    gpu.cuda.synchronize()
    np.testing.assert_allclose(host(dout), eo, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(host(dgu).reshape(-1)[:3 * 3072].reshape(3, 3072), eo, rtol=1e-5, atol=1e-6)
    a, b = r.standard_normal(1000).astype(np.float32), r.standard_normal(1000).astype(np.float32)
    da, db = dev(gpu, a), dev(gpu, b)
    qa.check(lib.qwen_hip_add_inplace(ptr(da), ptr(db), 1000, None))
    gpu.cuda.synchronize()
    assert np.array_equal(host(da), a + b)


@pytest.mark.parametrize("sq,sk,q_off", [(1, 1, 0), (1, 529, 528), (1, 3000, 2999), (1, 100, 40),
                                         (7, 7, 0), (64, 100, 36), (130, 130, 0), (33, 300, 200),
                                         (30, 1000, 970), (401, 401, 0), (600, 650, 40), (1100, 3000, 1900)])
def test_causal_attention(P, qa, gpu, sq, sk, q_off):
    nh, nkv, hd = 16, 8, 128
    r = np.random.default_rng(sq * 1000 + sk)
    Q = r.standard_normal((sq, nh * hd)).astype(np.float32)
    K = r.standard_normal((sk, nkv * hd)).astype(np.float32)
    V = r.standard_normal((sk, nkv * hd)).astype(np.float32)
    scale = 1.0 / np.sqrt(128.0)
    dout = gpu.empty((sq, nh * hd), dtype=gpu.float32, device="cuda")
    dQ, dK, dV = dev(gpu, Q), dev(gpu, K), dev(gpu, V)
    qa.check(qa.lib().qwen_hip_causal_attention(ptr(dout), ptr(dQ), ptr(dK), ptr(dV),
                                                sq, sk, nh, nkv, hd, scale, q_off, None), "attention")
    gpu.cuda.synchronize()
    exp = np.empty((sq, nh * hd), np.float32)
    P.orc_lib().orc_causal_attention(exp, Q, K, V, sq, sk, nh, nkv, hd, scale, q_off)
    np.testing.assert_allclose(host(dout), exp, atol=3e-5, rtol=1e-4)


@pytest.mark.parametrize("sq,sk", [(3000, 3000), (6400, 6400), (4096, 5000)])
def test_causal_attention_long_walk(P, qa, gpu, sq, sk):
    """Long prefills.  3000 query rows (47 query tiles x 8 kv heads, fewer than
    two blocks per CU): the plan caps a block's walk at a sixth of the longest
    query tile, so blocks walk 512 keys and the merge combines six splits.
    6400 rows (800 blocks of 64 queries): no split, so the kernel runs 8-wave
    blocks of 128 queries (400 of them) and the last query tiles walk all
    6400 keys in one block (the path the 8k-row prefill takes).  4096 rows
    after 904 cached keys (query i sees keys j <= 904 + i): the 8-wave blocks
    with a query offset, as a long continuation prefill runs them.  Checked
    against a float64 causal softmax attention computed with torch on the
    same device (the CPU oracle is too slow at this size)."""
    q_off = sk - sq
    nh, nkv, hd = 16, 8, 128
    chunk, nsplit = C.c_int(), C.c_int()
    qa.lib().qk_attn_prefill_plan(sq, sk, q_off, nh, nkv, C.byref(chunk), C.byref(nsplit))
    if sq == 3000:
        assert chunk.value == 512 and nsplit.value == 6, (chunk.value, nsplit.value)
    else:
        assert chunk.value >= sk and nsplit.value == 1, (chunk.value, nsplit.value)
    g = gpu.Generator(device="cuda").manual_seed(11)
    Q = gpu.randn((sq, nh * hd), generator=g, device="cuda", dtype=gpu.float32)
    K = gpu.randn((sk, nkv * hd), generator=g, device="cuda", dtype=gpu.float32)
    V = gpu.randn((sk, nkv * hd), generator=g, device="cuda", dtype=gpu.float32)
    scale = 1.0 / np.sqrt(128.0)
    out = gpu.empty((sq, nh * hd), dtype=gpu.float32, device="cuda")
    qa.check(qa.lib().qwen_hip_causal_attention(ptr(out), ptr(Q), ptr(K), ptr(V), sq, sk, nh, nkv, hd,
                                                scale, q_off, None), "attention")
    gpu.cuda.synchronize()
    mask = gpu.triu(gpu.ones((sq, sk), dtype=gpu.bool, device="cuda"), diagonal=1 + q_off)
    worst = 0.0
    for h in range(0, nh, 3):
        q = Q[:, h * hd:(h + 1) * hd].double()
        k = K[:, (h // 2) * hd:(h // 2 + 1) * hd].double().contiguous()
        v = V[:, (h // 2) * hd:(h // 2 + 1) * hd].double().contiguous()
        sc = (q @ k.t().contiguous()) * scale
        sc.masked_fill_(mask, float("-inf"))
        ref = gpu.softmax(sc, dim=-1) @ v
        got = out[:, h * hd:(h + 1) * hd].double()
        err = (got - ref).abs() - (3e-5 + 1e-4 * ref.abs())
        worst = max(worst, float(err.max()))
        del sc, ref
    assert worst <= 0.0, worst


@pytest.mark.parametrize("shards", [2, 8])
def test_vocab_sharded_argmax(P, qa, gpu, shards):
    """The LM head as it would shard over GPUs: each shard runs the argmax op
    on its contiguous vocabulary slice, the (logit, global index) pairs are
    combined by larger logit, then lower index; the result equals the argmax
    over the whole vocabulary, also with exact ties placed in different
    shards.  Logits of the slice winners come from the GEMV op on the slice."""
    K, N = 1024, 151936
    W = P.synth_bf16(N * K, 4, 1).reshape(N, K)
    x = P.synth_uniform(K, 4, 2)
    W2 = W.copy()
    full = P.orc_lib().orc_argmax_matvec_bf16(x, W, K, N, None)
    W2[3] = W[full]
    W2[N - 1] = W[full]
    dx = dev(gpu, x)
    for Wt, want in ((W, full), (W2, 3)):
        dW = dev(gpu, Wt.view(np.int16))
        esz = dW.element_size()
        best = None
        for i in range(shards):
            r0, r1 = N * i // shards, N * (i + 1) // shards
            wp = ptr(dW) + r0 * K * esz
            loc = qa.check(qa.lib().qwen_hip_argmax_matvec_bf16(ptr(dx), wp, K, r1 - r0, None))
            dy = gpu.empty(r1 - r0, dtype=gpu.float32, device="cuda")
            qa.check(qa.lib().qwen_hip_linear_nobias_bf16(ptr(dy), ptr(dx), wp, 1, K, r1 - r0, None), "gemv")
            gpu.cuda.synchronize()
            cand = (float(host(dy)[loc]), r0 + loc)
            if best is None or cand[0] > best[0] or (cand[0] == best[0] and cand[1] < best[1]):
                best = cand
        assert best[1] == want, (best, want)
        assert qa.lib().qwen_hip_argmax_matvec_bf16(ptr(dx), ptr(dW), K, N, None) == want


def test_argmax_matvec(P, qa, gpu):
    K, N = 1024, 151936
    W = P.synth_bf16(N * K, 4, 1).reshape(N, K)
    x = P.synth_uniform(K, 4, 2)
    dW, dx = dev(gpu, W.view(np.int16)), dev(gpu, x)
    got = qa.check(qa.lib().qwen_hip_argmax_matvec_bf16(ptr(dx), ptr(dW), K, N, None))
    exp = P.orc_lib().orc_argmax_matvec_bf16(x, W, K, N, None)
    assert got == exp
    # exact ties resolve to the lowest row, across blocks
    W2 = W.copy()
    W2[3] = W[exp]
    W2[N - 1] = W[exp]
    dW2 = dev(gpu, W2.view(np.int16))
    got2 = qa.lib().qwen_hip_argmax_matvec_bf16(ptr(dx), ptr(dW2), K, N, None)
    assert got2 == 3
