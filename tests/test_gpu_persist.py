"""The persistent decode engine (engine 2: every layer, the LM head and the
greedy feedback of all steps of one call in a single persistent kernel)
against the graph engine (engine 0) on the reference's shapes.

Both engines compute in fp32 from the same bf16 weights and fp32 K/V cache;
they differ only in summation order (the persistent engine splits the O and
down projections by column group and reduces the split-K partials in a fixed
order), so teacher-forced logits agree to ~1e-5 and greedy tokens agree
except where the top-2 margin is a near-tie.  The absolute bar against the
reference decoder is checked by the golden tests in test_gpu_decoder.py,
which run under both engines.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ENGINE_GRAPH, ENGINE_PERSIST = 0, 2
AGREE = 2e-3      # |logit(engine 2) - logit(engine 0)|; the reference bar is 2e-2 + 1e-2 |ref|
TIE = 1e-3


@pytest.fixture(scope="module")
def dec06(qa, gpu):
    cfg = qa.preset(0)
    d = qa.Decoder(cfg, 0, 6000)
    d.load_synthetic(0, 0.02, 0.0)
    rows, _, _ = qa.prompt_rows(cfg, 390, 12)
    yield d, rows
    d.close()


def teacher_run(d, engine, base, first_row, teach):
    """forward(first_row) then forward_token over `teach`; logits + hidden of each step."""
    d.set_kv_len(base)
    d.set_engine(engine)
    d.set_keep_logits(True)
    toks, logits, hidden = [], [], []
    for i in range(len(teach) + 1):
        t = d.forward(first_row) if i == 0 else d.forward_token(int(teach[i - 1]))
        toks.append(t)
        logits.append(d.read_logits())
        hidden.append(d.read_hidden())
    d.set_keep_logits(False)
    return np.array(toks), np.array(logits), np.array(hidden)


def first_divergence(a, b, logits):
    """index of the first differing token; asserts it is a near-tie."""
    for i, (x, y) in enumerate(zip(a, b)):
        if x != y:
            s = np.sort(logits[i])
            assert s[-1] - s[-2] < TIE, f"step {i}: {x} vs {y} with top-2 margin {s[-1] - s[-2]:.2e}"
            return i
    return len(a)


def test_persistent_is_default_on_mi355x(qa, dec06):
    d, _ = dec06
    d.set_engine(ENGINE_PERSIST)
    assert d.engine() == ENGINE_PERSIST


def test_persistent_vs_graph_teacher_forced_06b(qa, dec06):
    d, rows = dec06
    d.set_kv_len(0)
    d.set_engine(ENGINE_GRAPH)
    d.prefill(rows[:-1])
    base = d.kv_len()
    teach = [int(t) for t in np.random.default_rng(3).integers(0, 151643, 20)]
    tg, lg, hg = teacher_run(d, ENGINE_GRAPH, base, rows[-1], teach)
    tp, lp, hp = teacher_run(d, ENGINE_PERSIST, base, rows[-1], teach)
    assert d.engine() == ENGINE_PERSIST, "persistent run fell back"
    err = float(np.abs(lp - lg).max())
    herr = float(np.abs(hp - hg).max())
    print(f"0.6B teacher-forced, {len(teach) + 1} steps from position {base}: max |dlogit| {err:.2e}, "
          f"max |dhidden| {herr:.2e}")
    assert err < AGREE, err
    assert herr < 1e-3, herr
    for i in range(len(tp)):
        if tp[i] != tg[i]:
            s = np.sort(lg[i])
            assert s[-1] - s[-2] < TIE, (i, tp[i], tg[i])


def test_persistent_generate_equals_single_steps(qa, dec06):
    """one launch of n steps == n launches of one step (bitwise: fixed reduction orders)"""
    d, rows = dec06
    d.set_engine(ENGINE_PERSIST)
    d.set_kv_len(0)
    d.prefill(rows[:-1])
    base = d.kv_len()
    first = d.forward(rows[-1])
    gen = d.generate(first, 24)
    assert d.kv_len() == base + 25
    d.set_kv_len(base + 1)
    t, steps = first, []
    for _ in range(24):
        t = d.forward_token(t)
        steps.append(t)
    assert list(gen) == steps
    # rollback by 7 positions and regenerate: the same continuation
    d.set_kv_len(base + 1 + 17)
    again = d.generate(int(gen[16]), 7)
    assert list(again) == list(gen[17:])
    assert d.engine() == ENGINE_PERSIST


def test_persistent_generate_vs_graph(qa, dec06):
    d, rows = dec06
    out = {}
    for eng in (ENGINE_GRAPH, ENGINE_PERSIST):
        d.set_engine(eng)
        d.set_kv_len(0)
        d.prefill(rows[:-1])
        first = d.forward(rows[-1])
        out[eng] = [first] + list(d.generate(first, 40))
    if out[0] != out[2]:
        # find the step and check it is a near-tie on the graph engine's logits
        i = next(k for k in range(len(out[0])) if out[0][k] != out[2][k])
        d.set_engine(ENGINE_GRAPH)
        d.set_kv_len(0)
        d.prefill(rows[:-1])
        d.set_keep_logits(True)
        t = d.forward(rows[-1])
        for k in range(i):
            t = d.forward_token(out[0][k])
        lg = d.read_logits()
        d.set_keep_logits(False)
        s = np.sort(lg)
        assert s[-1] - s[-2] < TIE, f"generate diverged at step {i} without a near-tie"
    print(f"40-step greedy continuation identical: {out[0] == out[2]}")


@pytest.mark.parametrize("n_ctx", [2500, 4200])
def test_persistent_long_context(qa, dec06, n_ctx):
    """more than 64 positions per split (register batches after the LDS one)
    and more than 2048 keys (the graph engine's long-step variant)"""
    d, _ = dec06
    cfg = qa.preset(0)
    rows, _, _ = qa.prompt_rows(cfg, n_ctx - 4, 4, seed=7)
    d.set_engine(ENGINE_GRAPH)
    d.set_kv_len(0)
    d.prefill(rows[:-1])
    base = d.kv_len()
    teach = [11, 151000, 4242, 77]
    _, lg, _ = teacher_run(d, ENGINE_GRAPH, base, rows[-1], teach)
    _, lp, _ = teacher_run(d, ENGINE_PERSIST, base, rows[-1], teach)
    err = float(np.abs(lp - lg).max())
    print(f"0.6B at {n_ctx} positions: max |dlogit| {err:.2e}")
    assert err < AGREE, err


def test_persistent_vs_graph_17b(qa, gpu):
    cfg = qa.preset(1)
    d = qa.Decoder(cfg, 0, 2048)
    d.load_synthetic(0, 0.02, 0.0)
    assert d.engine() == ENGINE_PERSIST
    rows, _, _ = qa.prompt_rows(cfg, 500, 8)
    d.set_engine(ENGINE_GRAPH)
    d.prefill(rows[:-1])
    base = d.kv_len()
    teach = [int(t) for t in np.random.default_rng(5).integers(0, 151643, 8)]
    _, lg, hg = teacher_run(d, ENGINE_GRAPH, base, rows[-1], teach)
    _, lp, hp = teacher_run(d, ENGINE_PERSIST, base, rows[-1], teach)
    err = float(np.abs(lp - lg).max())
    print(f"1.7B teacher-forced: max |dlogit| {err:.2e}")
    assert err < AGREE, err
    assert d.engine() == ENGINE_PERSIST
    d.set_kv_len(base)
    first = d.forward(rows[-1])
    gen = d.generate(first, 12)
    d.set_kv_len(base + 1)
    t, steps = first, []
    for _ in range(12):
        t = d.forward_token(t)
        steps.append(t)
    assert list(gen) == steps
    d.close()


def test_relay_kernel_selection(qa, dec06):
    """The relay kernel runs persistent launches whose positions stay below
    RELAY_MAX_POS, the split kernel the others and every launch after
    set_relay(0)."""
    d, rows = dec06
    d.set_engine(ENGINE_PERSIST)
    d.set_kv_len(0)
    d.prefill(rows[:-1])
    base = d.kv_len()
    first = d.forward(rows[-1])
    assert d.last_kernel() == qa.KERNEL_RELAY
    d.set_relay(False)
    d.forward_token(first)
    assert d.last_kernel() == qa.KERNEL_SPLIT
    d.set_relay(True)
    d.set_kv_len(base + 1)
    extra, _, _ = qa.prompt_rows(qa.preset(0), qa.RELAY_MAX_POS - 3 - (base + 1), 0, seed=11)
    d.prefill(extra)
    assert d.kv_len() == qa.RELAY_MAX_POS - 3
    d.generate(first, 3)                     # positions 1021..1023: still relay
    assert d.last_kernel() == qa.KERNEL_RELAY
    d.set_kv_len(qa.RELAY_MAX_POS - 2)
    d.generate(first, 3)                     # position 1024 is past the relay kernel's LDS splits
    assert d.last_kernel() == qa.KERNEL_SPLIT
    assert d.fallbacks() == 0


def test_relay_vs_split_teacher_forced_06b(qa, dec06):
    """The two persistent kernels on the same teacher-forced steps: the same
    arithmetic (bf16 weights, fp32 sums; the relay kernel's matrix-core
    products take each fp32 activation as three exact bf16 terms), different
    summation orders."""
    d, rows = dec06
    d.set_engine(ENGINE_PERSIST)
    d.set_kv_len(0)
    d.prefill(rows[:-1])
    base = d.kv_len()
    teach = [int(t) for t in np.random.default_rng(9).integers(0, 151643, 20)]
    d.set_relay(False)
    ts, ls, hs = teacher_run(d, ENGINE_PERSIST, base, rows[-1], teach)
    assert d.last_kernel() == qa.KERNEL_SPLIT
    d.set_relay(True)
    tr, lr, hr = teacher_run(d, ENGINE_PERSIST, base, rows[-1], teach)
    assert d.last_kernel() == qa.KERNEL_RELAY
    err, herr = float(np.abs(lr - ls).max()), float(np.abs(hr - hs).max())
    print(f"relay vs split, {len(teach) + 1} teacher-forced steps: max |dlogit| {err:.2e}, max |dhidden| {herr:.2e}")
    assert err < AGREE and herr < 1e-3, (err, herr)
    first_divergence(ts, tr, ls)


def test_relay_split_boundaries(qa, dec06):
    """The relay kernel against the split kernel on teacher-forced steps
    across the relay's split layout changes: short contexts (fewer than 16
    splits, fold groups without positions, a last split that holds only the
    new position: positions 16, 32, ...), 241 keys (every block of a team
    folds from here), 256 -> 257 and 512 -> 513 keys (16 -> 17 and 32 -> 33
    positions per split: a second LDS batch of the fold)."""
    d, rows = dec06
    d.set_engine(ENGINE_PERSIST)
    d.set_fallback(False)
    try:
        d.set_kv_len(0)
        d.prefill(rows[:2])
        d.generate(d.forward(rows[2]), 530)   # K/V of positions 0..532 in the cache
        rng = np.random.default_rng(11)
        for p0, n in ((505, 12), (236, 24), (3, 36)):   # set_kv_len only rolls back: highest window first
            teach = [int(t) for t in rng.integers(0, 151643, n)]
            res = {}
            for relay in (False, True):
                d.set_relay(relay)
                d.set_kv_len(p0)
                d.set_keep_logits(True)
                toks, logits = [], []
                for t in teach:
                    toks.append(d.forward_token(t))
                    logits.append(d.read_logits())
                d.set_keep_logits(False)
                assert d.last_kernel() == (qa.KERNEL_RELAY if relay else qa.KERNEL_SPLIT)
                res[relay] = (np.array(toks), np.array(logits))
            err = float(np.abs(res[True][1] - res[False][1]).max())
            print(f"positions {p0}..{p0 + n - 1}: relay vs split max |dlogit| {err:.2e}")
            assert err < AGREE, (p0, err)
            first_divergence(res[False][0], res[True][0], res[False][1])
        assert d.fallbacks() == 0
    finally:
        d.set_relay(True)
        d.set_fallback(True)


@pytest.mark.parametrize("relay", [False, True])
def test_generate_equals_single_steps_both_kernels(qa, dec06, relay):
    """one launch of n steps == n launches of one step, bit for bit, on each
    persistent kernel; and the two kernels' greedy continuations agree"""
    d, rows = dec06
    d.set_engine(ENGINE_PERSIST)
    d.set_relay(relay)
    try:
        d.set_kv_len(0)
        d.prefill(rows[:-1])
        base = d.kv_len()
        first = d.forward(rows[-1])
        gen = d.generate(first, 32)
        assert d.last_kernel() == (qa.KERNEL_RELAY if relay else qa.KERNEL_SPLIT)
        d.set_kv_len(base + 1)
        t, steps = first, []
        for _ in range(32):
            t = d.forward_token(t)
            steps.append(t)
        assert list(gen) == steps
    finally:
        d.set_relay(True)


@pytest.mark.parametrize("layers", [1, 2, 3])
def test_relay_short_models(qa, gpu, layers):
    """Layer counts where one team has no layer (1) or the teams hold unequal
    counts (3): every block still joins the LM head and the token feedback;
    against the split kernel, teacher-forced and free-running."""
    cfg = qa.preset(0)
    cfg.layers = layers
    d = qa.Decoder(cfg, 0, 512)
    d.set_fallback(False)
    d.load_synthetic(3, 0.02, 0.0)
    rows, _, _ = qa.prompt_rows(cfg, 60, 4, seed=layers)
    d.prefill(rows[:-1])
    base = d.kv_len()
    teach = [int(t) for t in np.random.default_rng(layers).integers(0, 151643, 6)]
    d.set_relay(False)
    ts, ls, _ = teacher_run(d, ENGINE_PERSIST, base, rows[-1], teach)
    d.set_relay(True)
    tr, lr, _ = teacher_run(d, ENGINE_PERSIST, base, rows[-1], teach)
    assert d.last_kernel() == qa.KERNEL_RELAY
    err = float(np.abs(lr - ls).max())
    assert err < AGREE, err
    first_divergence(ts, tr, ls)
    out = {}
    for relay in (False, True):
        d.set_relay(relay)
        d.set_kv_len(base + 1)
        out[relay] = list(d.generate(int(ts[0]), 24))
    assert out[False] == out[True], f"{layers} layers: free runs differ"
    assert d.fallbacks() == 0
    d.close()


def test_relay_trace_layout(qa, dec06):
    """read_trace after a relay launch: 704 words per block in the relay
    layout; each block stamped its own team's layers and the LM head."""
    d, rows = dec06
    d.set_engine(ENGINE_PERSIST)
    d.set_kv_len(0)
    d.prefill(rows[:-1])
    first = d.forward(rows[-1])
    d.set_trace(2)
    try:
        d.generate(first, 4)
    finally:
        d.set_trace(-1)
    assert d.last_kernel() == qa.KERNEL_RELAY
    tr = d.read_trace().astype(np.int64)
    L, TM = 28, 24
    assert tr.shape == (256, 704)
    team0 = tr[:, 0] > 0                  # layer 0's first stamp: team 0 blocks
    team1 = tr[:, TM] > 0                 # layer 1's
    assert team0.sum() == 128 and team1.sum() == 128 and not np.any(team0 & team1)
    for l in range(L):
        own = team0 if l % 2 == 0 else team1
        assert np.all(tr[own, TM * l + 19] > 0) and np.all(tr[~own, TM * l + 19] == 0), l
        assert np.all(tr[own, TM * l + 19] >= tr[own, TM * l + 4])     # down stored after Q stored
    assert np.all(tr[:, TM * L + 3] > 0)                               # every block's LM candidate
    assert np.all(tr[team0, TM * L + 4] > 0) and np.all(tr[team1, TM * L + 4] == 0)


def test_engine_errors(qa, gpu):
    """set_engine range check; the persistent engine is refused for shapes it
    does not cover (the tiny test model) and the decoder stays usable."""
    cfg = qa.HipConfig(256, 2, 4, 2, 128, 512, 1000, 1e-6, 1e6)
    d = qa.Decoder(cfg, 0, 64)
    assert d.engine() == ENGINE_GRAPH
    with pytest.raises(RuntimeError):
        d.set_engine(ENGINE_PERSIST)
    with pytest.raises(RuntimeError):
        d.set_engine(3)
    assert d.engine() == ENGINE_GRAPH
    d.close()


def test_streaming_rollback_pattern(qa, dec06):
    """The streaming op pattern (qwen_asr.c:1748-1829): per chunk roll the KV
    back by the last 5 decoded tokens, prefill their embeddings + 26 new audio
    rows, decode; when the window would pass its cap, keep the 9-row head and
    re-prefill recent audio.  The persistent engine is teacher-forced with the
    graph engine's tokens and their logits compared step by step."""
    d, _ = dec06
    cfg = qa.preset(0)
    emb = qa.synth_bf16(cfg.vocab * cfg.hidden, 0, qa.SYNTH_EMBED).reshape(cfg.vocab, cfg.hidden)
    head, _, _ = qa.prompt_rows(cfg, 0, 9, emb=emb)
    audio = [qa.prompt_rows(cfg, 26, 0, audio_chunk=c, emb=emb)[0] for c in range(5)]
    cap, n_dec = 160, 10

    def stream(engine, forced=None):
        d.set_engine(engine)
        d.set_keep_logits(True)
        d.set_kv_len(0)
        d.prefill(head)
        toks, logits, prev, resets = [], [], [], 0
        for c in range(len(audio)):
            if prev:
                d.set_kv_len(d.kv_len() - 5)
            if d.kv_len() + 5 + 26 + n_dec > cap:
                d.set_kv_len(9)
                d.prefill(np.concatenate(audio[max(0, c - 2):c]))
                resets += 1
            rows = audio[c]
            if prev:
                rows = np.concatenate([qa.bf16_to_f32(emb[prev[-5:]]).reshape(-1, cfg.hidden), rows])
            d.prefill(rows[:-1])
            chunk = []
            for i in range(n_dec):
                if i == 0:
                    t = d.forward(rows[-1])
                else:
                    t = d.forward_token(forced[c][i - 1] if forced else chunk[-1])
                chunk.append(t)
                logits.append(d.read_logits())
            toks.append(chunk)
            prev = forced[c] if forced else chunk
        d.set_keep_logits(False)
        return toks, np.array(logits), resets

    tg, lg, resets = stream(ENGINE_GRAPH)
    tp, lp, _ = stream(ENGINE_PERSIST, forced=tg)
    assert resets >= 1, "the window reset path was not exercised"
    assert d.engine() == ENGINE_PERSIST
    err = float(np.abs(lp - lg).max())
    print(f"streaming, {len(audio)} chunks x {n_dec} steps, {resets} window reset(s): max |dlogit| {err:.2e}")
    assert err < AGREE, err
    flat_g = [t for c in tg for t in c]
    flat_p = [t for c in tp for t in c]
    for i, (a, b) in enumerate(zip(flat_g, flat_p)):
        if a != b:
            s = np.sort(lg[i])
            assert s[-1] - s[-2] < TIE, (i, a, b)


@pytest.mark.parametrize("relay", [True, False])
def test_wait_bound_gives_up(qa, dec06, relay):
    """Every wait inside either persistent kernel is bounded in wall-clock time.
    With a zero limit every wait that its first poll does not satisfy gives
    up: the launch still ends (every block leaves), and with the fallback off
    the call fails with QWEN_HIP_EDEVICE and leaves kv_len as it was; with the
    fallback on the same call is redone by the graph engine, counted, and
    gives the graph engine's tokens; with the limit restored the persistent
    engine is usable again and reproduces its own earlier tokens."""
    d, rows = dec06
    try:
        d.set_engine(ENGINE_PERSIST)
        d.set_relay(relay)
        d.set_kv_len(0)
        d.prefill(rows[:-1])
        base = d.kv_len()
        first = d.forward(rows[-1])
        ref = list(d.generate(first, 6))
        assert d.last_kernel() == (qa.KERNEL_RELAY if relay else qa.KERNEL_SPLIT)
        n0 = d.fallbacks()
        d.set_kv_len(base + 1)
        d.set_fallback(False)
        d.set_wait_limit(0.0)
        with pytest.raises(RuntimeError, match="EDEVICE.*timed out"):
            d.generate(first, 6)
        assert d.kv_len() == base + 1
        assert d.engine() == ENGINE_PERSIST and d.fallbacks() == n0
        d.set_fallback(True)
        got = list(d.generate(first, 6))
        assert d.fallbacks() == n0 + 1 and d.engine() == ENGINE_GRAPH
        assert d.kv_len() == base + 7
        d.set_kv_len(base + 1)
        assert list(d.generate(first, 6)) == got, "the fallback's tokens are the graph engine's"
        d.set_wait_limit(1.0)
        d.set_engine(ENGINE_PERSIST)
        d.set_kv_len(base + 1)
        assert list(d.generate(first, 6)) == ref
        assert d.last_kernel() == (qa.KERNEL_RELAY if relay else qa.KERNEL_SPLIT)
        assert d.fallbacks() == n0 + 1
    finally:
        d.set_wait_limit(1.0)
        d.set_fallback(True)
        d.set_engine(ENGINE_PERSIST)
        d.set_relay(True)


@pytest.mark.parametrize("relay", [True, False])
def test_tag_space_restart(qa, dec06, relay):
    """Hand-over tags come from a 32-bit epoch that each launch advances by the
    tags it uses; a launch that would pass 0xFFFFFF00 first zeroes the exchange
    words and restarts at 1.  A launch that ends exactly at the limit (its
    last tags the highest ever used), the restart after it, and single-step
    launches across a restart all give the same tokens as at a low epoch."""
    d, rows = dec06
    top = 0xFFFFFF00
    try:
        d.set_engine(ENGINE_PERSIST)
        d.set_relay(relay)
        d.set_kv_len(0)
        d.prefill(rows[:-1])
        base = d.kv_len()
        first = d.forward(rows[-1])
        e0 = d.tag_epoch()
        ref = list(d.generate(first, 8))
        need = d.tag_epoch() - e0
        assert d.last_kernel() == (qa.KERNEL_RELAY if relay else qa.KERNEL_SPLIT)
        assert 0 < need < 1 << 20
        # a launch whose tags end exactly at the limit: no restart
        d.set_tag_epoch(top - need)
        d.set_kv_len(base + 1)
        assert list(d.generate(first, 8)) == ref
        assert d.tag_epoch() == top
        # the next launch restarts the tag space first
        d.set_kv_len(base + 1)
        assert list(d.generate(first, 8)) == ref
        assert d.tag_epoch() == 1 + need
        # one step per launch, restarting after the second launch
        d.set_kv_len(base + 1)
        e1 = d.tag_epoch()
        t = d.forward_token(first)
        one = d.tag_epoch() - e1
        d.set_tag_epoch(top - 2 * one)
        d.set_kv_len(base + 1)
        t, steps = first, []
        for _ in range(8):
            t = d.forward_token(t)
            steps.append(t)
        assert steps == ref
        assert d.tag_epoch() == 1 + 6 * one
        assert d.engine() == ENGINE_PERSIST
    finally:
        d.set_relay(True)
        d.set_engine(ENGINE_PERSIST)


def test_generate_beside_busy_stream(qa, dec06):
    """A persistent launch queued while another stream keeps the CUs busy
    (64 fp32 4096 x 4096 products): its blocks become resident as the other
    kernels' blocks retire (measured: no fallback, ~5 ms), and a grid that
    could not would give up at the launch check-in, bounded by 20 ms rather
    than the 1 s wait limit.  Either way the call returns well within a
    second with the right tokens."""
    import time
    import torch
    d, rows = dec06
    try:
        d.set_engine(ENGINE_PERSIST)
        d.set_kv_len(0)
        d.prefill(rows[:-1])
        base = d.kv_len()
        first = d.forward(rows[-1])
        ref = list(d.generate(first, 8))
        n0 = d.fallbacks()
        a = torch.randn(4096, 4096, device="cuda")
        side = torch.cuda.Stream()
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            for _ in range(64):
                a = torch.matmul(a, a) * 1e-3
        d.set_kv_len(base + 1)
        t0 = time.perf_counter()
        got = list(d.generate(first, 8))
        dt = time.perf_counter() - t0
        torch.cuda.synchronize()
        fell = d.fallbacks() - n0
        print(f"generate beside a busy stream: {dt * 1e3:.1f} ms, fallbacks {fell}, engine {d.engine()}")
        assert dt < 0.9, dt
        assert torch.isfinite(a).all()
        if fell:   # redone by the graph engine: its tokens (equal to the persistent ones but for near-ties)
            d.set_engine(ENGINE_GRAPH)
            d.set_kv_len(base + 1)
            ref = list(d.generate(first, 8))
        assert got == ref
    finally:
        d.set_engine(ENGINE_PERSIST)


def test_lm_head_exact_ties(qa, gpu):
    """Exact logit ties resolve to the lowest vocabulary row on every engine,
    as the reference's strict `>` scan and in-order combine do
    (qwen_asr_kernels_avx.c:223-226, qwen_asr_kernels.c:534-541).  Rows whose
    only nonzero weight is 64 at the largest element k of the final normed
    row all score exactly 64 * xn[k] (every other product adds an exact
    zero), far above the rest.  The tied rows sit in one 4-row group, in
    neighbouring groups, and in far-apart groups of different blocks."""
    cfg = qa.preset(0)
    cfg.layers = 2
    d = qa.Decoder(cfg, 0, 128)
    d.set_fallback(False)
    d.load_synthetic(5, 0.02, 0.0)
    base_emb = qa.synth_bf16(cfg.vocab * cfg.hidden, 5, qa.SYNTH_EMBED).reshape(cfg.vocab, cfg.hidden)
    ones = np.ones(cfg.hidden, np.float32)
    d.load_embeddings(base_emb, ones)
    rows, _, _ = qa.prompt_rows(cfg, 30, 4, seed=5, emb=base_emb)
    d.set_engine(ENGINE_GRAPH)
    d.prefill(rows[:-1])
    base = d.kv_len()
    d.set_keep_logits(True)
    d.forward(rows[-1])
    xn = d.read_hidden()
    k = int(np.argmax(xn))
    assert xn[k] > 0.5
    try:
        for tied in ((151930, 7), (1031, 1027), (40002, 40001), (150000, 70000, 99999)):
            emb = base_emb.copy()
            for r in tied:
                emb[r] = 0
                emb[r, k] = 0x4280          # bf16 64.0
            d.load_embeddings(emb, ones)
            for engine, relay in ((ENGINE_GRAPH, True), (ENGINE_PERSIST, True), (ENGINE_PERSIST, False)):
                d.set_engine(engine)
                d.set_relay(relay)
                d.set_kv_len(base)
                t = d.forward(rows[-1])
                lg = d.read_logits()
                assert lg[tied[0]] == lg[tied[1]], (tied, engine, relay)
                assert t == min(tied), (tied, engine, relay, t)
                if engine == ENGINE_PERSIST:
                    assert d.last_kernel() == (qa.KERNEL_RELAY if relay else qa.KERNEL_SPLIT)
    finally:
        d.set_relay(True)
        d.close()
