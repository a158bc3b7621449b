"""Pins the CPU oracle (oracle/qwen_oracle.c) before anything is checked
against it:
  * op by op against the reference's own operators compiled from
    /root/reference (oracle/_ref), when that build is present;
  * against fp64 closed forms and invariants that fix the math independently
    (RMSNorm, RoPE rotation/norm preservation/identity at position 0, SwiGLU,
    softmax attention with causal mask and GQA head map, argmax tie rule,
    GEMV error bound);
  * against the committed golden fixtures written by the reference decoder.
Each closed-form check is chosen so a plausible mistake fails it; the
"teeth" tests plant such mistakes in a copy of the oracle's result and show
the check rejects them.
"""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def rng(seed):
    return np.random.default_rng(seed)


def need_ref(P):
    if not P.ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent when it was last built)")
    return P.ref_lib()


# ---------------------------------------------------------------- fp64 forms
def rms64(x, w, eps):
    x = x.astype(np.float64)
    return x * w / np.sqrt((x * x).mean(-1, keepdims=True) + eps)


def rope64(x, cos, sin):
    x = x.astype(np.float64)
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    c, s = cos[..., :half], sin[..., :half]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)


def attn64(Q, K, V, nh, nkv, hd, scale, q_offset):
    sq, sk = Q.shape[0], K.shape[0]
    out = np.zeros((sq, nh * hd))
    for h in range(nh):
        kvh = h // (nh // nkv)
        for i in range(sq):
            kend = min(q_offset + i + 1, sk)
            q = Q[i, h * hd:(h + 1) * hd].astype(np.float64)
            k = K[:kend, kvh * hd:(kvh + 1) * hd].astype(np.float64)
            v = V[:kend, kvh * hd:(kvh + 1) * hd].astype(np.float64)
            s = k @ q * scale
            p = np.exp(s - s.max())
            out[i, h * hd:(h + 1) * hd] = p @ v / p.sum()
    return out


# ---------------------------------------------------------------- synth
def test_synth_is_deterministic_and_shared(P, qa):
    a = P.synth_bf16(1 << 21, 0, 1234)
    b = P.synth_bf16(1 << 21, 0, 1234)
    assert np.array_equal(a, b)
    # the product library carries the same generator
    c = np.empty_like(a)
    qa.lib().qwen_synth_normal_bf16(c.ctypes.data, c.size, 0, 1234, 0.0, 0.02, 0)
    assert np.array_equal(a, c)
    f = P.bf16_to_f32(a).astype(np.float64)
    assert abs(f.mean()) < 1e-4 and abs(f.std() - 0.02) < 2e-4
    u = P.synth_uniform(100000, 3, 9)
    assert u.min() >= -1 and u.max() < 1 and abs(u.mean()) < 0.01
    t = P.synth_tokens(10000, 0, 5, 151643)
    assert t.min() >= 0 and t.max() < 151643 and len(np.unique(t)) > 9000


def test_synth_checksums_are_pinned(P):
    # golden fixtures record the checksums of the weights they were made with
    g = np.load(os.path.join(GOLD, "c1_short.npz"))
    emb = P.synth_bf16(P.CFG_06B.vocab * P.CFG_06B.hidden, 0, P.SYNTH_EMBED)
    assert P.checksum_u16(emb) == int(g["emb_checksum"])


def test_bf16_rounding_is_rne(P):
    x = rng(0).standard_normal(100000).astype(np.float32)
    x = np.concatenate([x, np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 0.0, -0.0], np.float32)])
    lib = P.orc_lib()
    got = np.array([lib.qwen_f32_to_bf16_rne(float(v)) for v in x[-2000:]], np.uint16)
    # independent formulation: nearest of the two bf16 neighbours, ties to even mantissa
    u = x[-2000:].view(np.uint32)
    lo = (u >> 16).astype(np.uint64)
    rem = (u & 0xFFFF).astype(np.uint64)
    up = (rem > 0x8000) | ((rem == 0x8000) & (lo & 1 == 1))
    ref = (lo + up).astype(np.uint16)
    assert np.array_equal(got, ref)
    assert np.array_equal(P.f32_to_bf16(x[-2000:]), ref)


# ---------------------------------------------------------------- ops
def test_rms_norm(P):
    lib = P.orc_lib()
    x = rng(1).standard_normal((5, 1024)).astype(np.float32) * 3
    w = (1 + 0.1 * rng(2).standard_normal(1024)).astype(np.float32)
    out = np.empty_like(x)
    lib.orc_rms_norm(out, x, w, 5, 1024, 1e-6)
    np.testing.assert_allclose(out, rms64(x, w, 1e-6), rtol=2e-6, atol=1e-6)
    ref = need_ref(P) if P.ref_available() else None
    if ref is not None:
        o2 = np.empty_like(x)
        ref.qwen_rms_norm(o2, x, w, 5, 1024, 1e-6)
        np.testing.assert_allclose(out, o2, rtol=1e-6, atol=1e-7)


def test_rms_norm_per_head(P):
    lib = P.orc_lib()
    x = rng(3).standard_normal((3, 16 * 128)).astype(np.float32)
    w = (1 + 0.1 * rng(4).standard_normal(128)).astype(np.float32)
    a = x.copy()
    lib.orc_rms_norm_per_head(a, w, 3, 16, 128, 1e-6)
    exp = rms64(x.reshape(3, 16, 128), w, 1e-6).reshape(3, -1)
    np.testing.assert_allclose(a, exp, rtol=2e-6, atol=1e-6)
    if P.ref_available():
        b = x.copy()
        need_ref(P).qwen_rms_norm_per_head(b, w, 3, 16, 128, 1e-6)
        np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)


def test_rope_table_and_rotation(P):
    lib = P.orc_lib()
    n, hd, theta = 9000, 128, 1e6
    c = np.empty((n, hd), np.float32)
    s = np.empty((n, hd), np.float32)
    lib.orc_rope_table(c, s, n, hd, theta)
    # the table is cos/sin of the fp32 angle (float)p * inv[d]; check in fp64 of that angle
    # powf(theta, 2d/hd) as the correctly rounded fp32 of the fp64 power; 1/x in fp32
    pw = np.power(np.float64(theta), (np.arange(0, hd, 2, dtype=np.float32) / np.float32(hd)).astype(np.float64))
    inv = np.float32(1.0) / pw.astype(np.float32)
    ang = (np.arange(n, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32).astype(np.float64)
    np.testing.assert_allclose(c[:, :64], np.cos(ang), atol=2e-6)
    np.testing.assert_allclose(s[:, :64], np.sin(ang), atol=2e-6)
    assert np.array_equal(c[:, :64], c[:, 64:]) and np.array_equal(s[:, :64], s[:, 64:])
    # position 0 is the identity; rotation preserves each (d, d+64) pair norm
    x = rng(5).standard_normal((4, 3 * hd)).astype(np.float32)
    pos = np.array([0, 1, 777, 8999])
    y = x.copy()
    lib.orc_apply_rope(y, np.ascontiguousarray(c[pos]), np.ascontiguousarray(s[pos]), 4, 3, hd)
    assert np.array_equal(y[0], x[0])
    xr, yr = x.reshape(4, 3, 2, 64), y.reshape(4, 3, 2, 64)
    np.testing.assert_allclose((yr ** 2).sum(2), (xr ** 2).sum(2), rtol=1e-5)
    np.testing.assert_allclose(y.reshape(4, 3, hd), rope64(x.reshape(4, 3, hd), c[pos][:, None], s[pos][:, None]),
                               atol=1e-5)
    if P.ref_available():
        ref = need_ref(P)
        c2 = np.empty((len(pos), hd), np.float32)
        s2 = np.empty((len(pos), hd), np.float32)
        ref.qwen_compute_rope_neox(c2, s2, pos.astype(np.int32), len(pos), hd, theta)
        # the reference is built with -ffast-math, whose powf may differ by an
        # ulp of the inverse frequency: the angle error grows with position
        tol = 2e-6 + 1e-7 * pos[:, None]
        assert np.all(np.abs(c2 - c[pos]) <= tol) and np.all(np.abs(s2 - s[pos]) <= tol)
        z = x.copy()
        ref.qwen_apply_rope_neox(z, np.ascontiguousarray(c[pos]), np.ascontiguousarray(s[pos]), 4, 3, hd)
        np.testing.assert_allclose(y, z, atol=1e-6)


def test_swiglu(P):
    lib = P.orc_lib()
    gu = rng(6).standard_normal((3, 2 * 512)).astype(np.float32) * 4
    out = np.empty((3, 512), np.float32)
    lib.orc_swiglu(out, gu, 3, 512)
    g, u = gu[:, 0::2].astype(np.float64), gu[:, 1::2].astype(np.float64)
    np.testing.assert_allclose(out, g / (1 + np.exp(-g)) * u, rtol=2e-6, atol=1e-6)
    if P.ref_available():
        o2 = np.empty_like(out)
        need_ref(P).qwen_swiglu_multiply(o2, gu, 3, 512)
        np.testing.assert_allclose(out, o2, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("seq,K,N", [(1, 1024, 333), (1, 2048, 64), (3, 3072, 40), (2, 100, 7)])
def test_linear_bf16(P, seq, K, N):
    lib = P.orc_lib()
    W = P.synth_bf16(N * K, 1, 77).reshape(N, K)
    x = P.synth_uniform(seq * K, 1, 78).reshape(seq, K)
    y = np.empty((seq, N), np.float32)
    lib.orc_linear_bf16(y, x, W, seq, K, N)
    Wf = P.bf16_to_f32(W).astype(np.float64)
    exact = x.astype(np.float64) @ Wf.T
    bound = 4 * K * 2.0 ** -24 * (np.abs(x.astype(np.float64)) @ np.abs(Wf).T) + 1e-30
    assert np.all(np.abs(y - exact) <= bound)
    if P.ref_available():
        y2 = np.empty_like(y)
        need_ref(P).qwen_linear_nobias_bf16(y2, x, W, seq, K, N)
        assert np.all(np.abs(y2 - exact) <= bound)
        np.testing.assert_allclose(y, y2, rtol=0, atol=float(bound.max()))


def test_argmax_matvec_and_ties(P):
    lib = P.orc_lib()
    K, N = 1024, 5000
    W = P.synth_bf16(N * K, 2, 5).reshape(N, K)
    x = P.synth_uniform(K, 2, 6)
    lg = P.bf16_to_f32(W).astype(np.float64) @ x
    got = lib.orc_argmax_matvec_bf16(x, W, K, N, None)
    assert got == int(np.argmax(lg))
    # duplicate the winning row below and above: the lowest index must win
    W2 = W.copy()
    W2[17] = W[got]
    W2[N - 3] = W[got]
    assert lib.orc_argmax_matvec_bf16(x, W2, K, N, None) == min(17, got)
    if P.ref_available():
        ref = need_ref(P)
        assert ref.qwen_argmax_matvec_bf16(x, W, K, N) == got
        assert ref.qwen_argmax_matvec_bf16(x, W2, K, N) == min(17, got)


@pytest.mark.parametrize("sq,sk,q_off", [(1, 1, 0), (1, 37, 36), (5, 20, 15), (6, 6, 0), (3, 50, 10)])
def test_causal_attention(P, sq, sk, q_off):
    lib = P.orc_lib()
    nh, nkv, hd = 4, 2, 128
    r = rng(10 + sq + sk)
    Q = r.standard_normal((sq, nh * hd)).astype(np.float32)
    K = r.standard_normal((sk, nkv * hd)).astype(np.float32)
    V = r.standard_normal((sk, nkv * hd)).astype(np.float32)
    scale = np.float32(1 / np.sqrt(128))
    out = np.empty((sq, nh * hd), np.float32)
    lib.orc_causal_attention(out, Q, K, V, sq, sk, nh, nkv, hd, scale, q_off)
    np.testing.assert_allclose(out, attn64(Q, K, V, nh, nkv, hd, float(scale), q_off), atol=2e-5)
    if sk == 1:
        # a single visible key returns its value row exactly (GQA: heads 0,1 -> kv 0)
        np.testing.assert_allclose(out[0, :128], V[0, :128], atol=1e-6)
        np.testing.assert_allclose(out[0, 256:384], V[0, 128:], atol=1e-6)
    if P.ref_available():
        o2 = np.empty_like(out)
        need_ref(P).qwen_causal_attention(o2, Q, K, V, sq, sk, nh, nkv, hd, scale, q_off)
        np.testing.assert_allclose(out, o2, atol=2e-6)


def test_checks_have_teeth(P):
    """Plant plausible mistakes in copies of oracle results: each must fail
    the closed-form check the real result passes."""
    lib = P.orc_lib()
    nh, nkv, hd, sq, sk = 4, 2, 128, 3, 12
    r = rng(99)
    Q = r.standard_normal((sq, nh * hd)).astype(np.float32)
    K = r.standard_normal((sk, nkv * hd)).astype(np.float32)
    V = r.standard_normal((sk, nkv * hd)).astype(np.float32)
    exact = attn64(Q, K, V, nh, nkv, hd, 1 / np.sqrt(128), 9)
    wrong_map = np.zeros_like(exact)
    for h in range(nh):            # h % nkv instead of h // (nh / nkv)
        wrong_map[:, h * hd:(h + 1) * hd] = attn64(Q[:, h * hd:(h + 1) * hd], K[:, (h % nkv) * hd:(h % nkv + 1) * hd],
                                                   V[:, (h % nkv) * hd:(h % nkv + 1) * hd], 1, 1, hd, 1 / np.sqrt(128), 9)
    no_mask = attn64(Q, K, V, nh, nkv, hd, 1 / np.sqrt(128), 100)
    for bad in (wrong_map, no_mask):
        assert np.abs(bad - exact).max() > 1e-2
    x = r.standard_normal((2, 256)).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(256)).astype(np.float32)
    good = rms64(x, w, 1e-6)
    assert np.abs(rms64(x, np.ones_like(w), 1e-6) - good).max() > 1e-2      # dropped norm weight
    cs = np.cos(np.linspace(0, 3, 128))[None]
    sn = np.sin(np.linspace(0, 3, 128))[None]
    y = rope64(x[:, :128], cs, sn)
    assert np.abs(rope64(x[:, :128], cs, -sn) - y).max() > 1e-2               # sign of the rotation


# ---------------------------------------------------------------- decoder
def test_oracle_matches_reference_golden_tiny(P):
    g = np.load(os.path.join(GOLD, "tiny_teacher.npz"))
    m = P.SynthModel(P.CFG_TINY, seed=0, norm_std=0.1)
    rows, _ = P.prompt_rows(m, 20, 6)
    assert np.array_equal(rows, g["rows"])
    o = P.Oracle(m)
    o.prefill(rows[:-1])
    inp = [rows[-1]] + [o.embed(t) for t in g["teach"]]
    for i, x in enumerate(inp):
        t, lg, hd = o.forward(x, True, True)
        np.testing.assert_allclose(lg, g["logits"][i], atol=2e-5, rtol=1e-5)
        np.testing.assert_allclose(hd, g["hidden"][i], atol=2e-5, rtol=1e-5)
        assert t == g["tokens"][i]
    assert o.kv_len() == int(g["kv_len"])


@pytest.mark.parametrize("name,cfg_name,n_audio,n_ids", [("c1_short", "CFG_06B", 40, 12), ("c3_short", "CFG_17B", 30, 16)])
def test_oracle_matches_reference_golden_full_shape(P, name, cfg_name, n_audio, n_ids):
    g = np.load(os.path.join(GOLD, f"{name}.npz"))
    m = P.SynthModel(getattr(P, cfg_name), seed=0)
    assert P.checksum_u16(m.emb) == int(g["emb_checksum"])
    assert P.checksum_u16(m.layers[0][P.WQ]) == int(g["wq0_checksum"])
    rows, ids = P.prompt_rows(m, n_audio, n_ids)
    assert np.array_equal(ids, g["ids"])
    o = P.Oracle(m)
    o.prefill(rows[:-1])
    x = rows[-1]
    for i, ref_tok in enumerate(g["tokens"]):
        t, lg, _ = o.forward(x, True)
        np.testing.assert_allclose(lg[g["top_idx"][i]], g["top_val"][i], atol=1e-4)
        if t != ref_tok:
            assert g["margin"][i] < 1e-3, f"step {i}: oracle {t} vs reference {ref_tok}"
            break
        x = o.embed(t)


@pytest.mark.parametrize("name,cfg_name", [("c1_full", "CFG_06B"), ("c3_short", "CFG_17B")])
def test_oracle_matches_reference_full_logits(P, name, cfg_name):
    """Every vocabulary row's logit of the reference's first forwards
    (tests/golden/*_logits.npz) against the oracle's."""
    g = np.load(os.path.join(GOLD, f"{name}_logits.npz"))
    m = P.SynthModel(getattr(P, cfg_name), seed=0)
    assert P.checksum_u16(m.emb) == int(g["emb_checksum"])
    rows, ids = P.prompt_rows(m, int(g["n_audio"]), int(g["n_ids"]))
    assert np.array_equal(ids, g["ids"])
    o = P.Oracle(m)
    o.prefill(rows[:-1])
    x = rows[-1]
    for i, ref in enumerate(g["logits"]):
        t, lg, _ = o.forward(x, True)
        np.testing.assert_allclose(lg, ref, atol=1e-4, rtol=0)
        assert t == g["tokens"][i]
        x = o.embed(t)


def test_oracle_prefill_split_and_rollback(P):
    """prefill(n) == prefill(k) + prefill(n-k); forwards row by row == prefill;
    truncating the KV and re-prefilling reproduces the same logits."""
    m = P.SynthModel(P.CFG_TINY, seed=3, norm_std=0.1)
    rows, _ = P.prompt_rows(m, 30, 6, seed=3)
    a, b, c = P.Oracle(m), P.Oracle(m), P.Oracle(m)
    a.prefill(rows[:-1])
    b.prefill(rows[:11]); b.prefill(rows[11:-1])
    for r in rows[:-1]:
        c.forward(r)
    la = a.forward(rows[-1], True)[1]
    lb = b.forward(rows[-1], True)[1]
    lc = c.forward(rows[-1], True)[1]
    np.testing.assert_allclose(lb, la, atol=1e-5)
    np.testing.assert_allclose(lc, la, atol=1e-4)
    a.set_kv_len(20)
    a.prefill(rows[20:-1])
    np.testing.assert_allclose(a.forward(rows[-1], True)[1], la, atol=1e-6)


EOS_CFG = (1024, 2, 16, 8, 128, 3072, 151936)


def eos_model(P):
    """Two layers of the 0.6B shape with the full vocabulary, <|im_end|>'s
    embedding row scaled by 3: greedy decoding from the seed-3 prompt below
    emits <|im_end|> as its 5th token (top-2 margins >= 0.1 on the way)."""
    m = P.SynthModel(P.Config(*EOS_CFG), seed=3)
    m.emb[P.TOKEN_IM_END] = P.f32_to_bf16(P.bf16_to_f32(m.emb[P.TOKEN_IM_END]) * 3.0)
    return m


def test_greedy_loop_restatement(P):
    """greedy_until_eos (qwen_asr.c:729-759) on the oracle and on the
    reference's own decoder (oracle/_ref): the same kept tokens, stop at the
    first EOS without keeping or forwarding it, the KV holds exactly the
    forwarded tokens, and a max_tokens cap keeps exactly that many."""
    need_ref(P)
    m = eos_model(P)
    rows, _ = P.prompt_rows(m, 40, 8, seed=3)
    runs = []
    for dec in (P.Oracle(m), P.RefModel(m, threads=4)):
        dec.prefill(rows[:-1])
        t, _, _ = dec.forward(rows[-1])
        kept, last = P.greedy_until_eos(dec, t, 30)
        runs.append((kept, last, dec.kv_len()))
        assert dec.kv_len() == rows.shape[0] + len(kept)      # last row + every kept token forwarded once
        dec.set_kv_len(rows.shape[0])
        capped, _ = P.greedy_until_eos(dec, t, 2)
        assert capped == kept[:2] and dec.kv_len() == rows.shape[0] + 2
        dec.close()
    assert runs[0] == runs[1]
    assert runs[0][0] == [118997, 144330, 76550, 77354] and runs[0][1] == P.TOKEN_IM_END


def test_stream_restatement(P):
    """RefStream (qwen_asr.c:1748-1829): the reused prefix is the longest run of
    bitwise-equal leading prefill rows, the KV after a chunk holds its prefill
    rows + the last row + the kept tokens, and chunks with reuse give the same
    tokens as the same chunks prefilled from scratch (the oracle's prefill is
    split-invariant bit for bit)."""
    m = eos_model(P)
    head, _ = P.prompt_rows(m, 0, 8, seed=3)
    audio = [P.synth_f32(12 * 1024, 3, P.synth_audio_id(c)).reshape(12, 1024) for c in range(4)]
    tail = np.stack([m.embed(t) for t in (151644, 77091, 198)])
    chunks = [np.concatenate([head] + audio[:c + 1] + [tail]) for c in range(4)]
    chunks.append(np.concatenate([head] + audio[2:4] + [tail]))       # oldest audio evicted
    reuse = P.RefStream(P.Oracle(m))
    for i, rows in enumerate(chunks):
        kept, reused = reuse.chunk(rows, 6)
        want = 0 if i == 0 else (8 if i == 4 else 8 + 12 * i)
        assert reused == want, (i, reused)
        assert reuse.dec.kv_len() == rows.shape[0] + len(kept)
        fresh = P.RefStream(P.Oracle(m))
        assert fresh.chunk(rows, 6) == (kept, 0)
