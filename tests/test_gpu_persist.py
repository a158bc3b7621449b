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


def test_wait_bound_gives_up(qa, dec06):
    """Every wait inside the persistent kernel is bounded in wall-clock time.
    With a zero limit every wait that its first poll does not satisfy gives
    up: the launch still ends (every block leaves), and with the fallback off
    the call fails with QWEN_HIP_EDEVICE and leaves kv_len as it was; with the
    fallback on the same call is redone by the graph engine, counted, and
    gives the graph engine's tokens; with the limit restored the persistent
    engine is usable again and reproduces its own earlier tokens."""
    d, rows = dec06
    try:
        d.set_engine(ENGINE_PERSIST)
        d.set_kv_len(0)
        d.prefill(rows[:-1])
        base = d.kv_len()
        first = d.forward(rows[-1])
        ref = list(d.generate(first, 6))
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
        assert d.fallbacks() == n0 + 1
    finally:
        d.set_wait_limit(1.0)
        d.set_fallback(True)
        d.set_engine(ENGINE_PERSIST)
