"""Parity of the HIP token loop with the CPU oracle on the configurations the
golden trajectories do not reach, through the C ABI, on both decode engines
(0: graph of fused kernels, 2: persistent kernel):

* C4 long context: an 8191-row prefill, then decode steps at positions
  8191-8193, 8450 (after extending the cache) and 8703 (after a rollback and
  re-prefill), where attention over the cache dominates
  (qwen_asr_decoder.c:449-455 over pos+1 keys);
* C5 streaming op list: per chunk roll back the last 5 tokens, prefill their
  embeddings + 26 audio rows, 24 steps, with window resets (qwen_asr.c:1748-1829);
* 1.7B: a 1515-row prefill (C3's) and decode steps after it;
* EOS: generate(stop_on_eos) and the streaming driver's chunk loop against
  the reference's loops (qwen_asr.c:729-759, :1802-1814) on a model whose
  <|im_end|> wins at known steps.

The models keep the reference's layer shapes and vocabulary but only two
layers, so the oracle's fp32 CPU run stays within seconds.  Bar (BASELINE
north star): logits within 2e-2 + 1e-2 |ref| over the whole vocabulary,
greedy tokens identical except where the oracle's top-2 margin is below
1e-3.  Steps are teacher-forced with the oracle's tokens, so a near-tie
cannot hide later steps.
"""
import numpy as np
import pytest

from test_oracle import EOS_CFG, eos_model

pytestmark = pytest.mark.gpu

ATOL, RTOL, TIE = 2e-2, 1e-2, 1e-3
CFG06_2L = (1024, 2, 16, 8, 128, 3072, 151936)
CFG17_2L = (2048, 2, 16, 8, 128, 6144, 151936)
ORACLE_THREADS = 16


def check_step(lg, lo, tok, otok, what):
    err = float(np.abs(lg - lo).max())
    assert np.all(np.abs(lg - lo) <= ATOL + RTOL * np.abs(lo)), f"{what}: max |dlogit| {err:.3e}"
    if tok != otok:
        s = np.sort(lo)
        assert s[-1] - s[-2] < TIE, f"{what}: token {tok} vs oracle {otok}, margin {s[-1] - s[-2]:.2e}"
    return err


def gpu_decoder(qa, m, cap, engine):
    d = qa.Decoder(qa.config_from(m.cfg), 0, cap)
    d.load_model(m)
    d.set_fallback(False)
    d.set_engine(engine)
    d.set_keep_logits(True)
    return d


# ----------------------------------------------------------------- C4
C4_ROWS = 8192                 # 8191 prefilled + the last one forwarded
C4_EXT, C4_BACK, C4_EXT2 = 256, 5, 258


@pytest.fixture(scope="module")
def c4(P, gpu):
    """The oracle's run of the C4 op sequence, once for both engines."""
    m = P.SynthModel(P.Config(*CFG06_2L), seed=4)
    rows = P.synth_f32(C4_ROWS * 1024, 4, P.synth_audio_id(40)).reshape(C4_ROWS, 1024)
    ext = P.synth_f32((C4_EXT + C4_EXT2) * 1024, 4, P.synth_audio_id(41)).reshape(-1, 1024)
    teach = [int(t) for t in P.synth_tokens(4, 4, P.synth_tokens_id(40))]
    o = P.Oracle(m, threads=ORACLE_THREADS)
    o.prefill(rows[:-1])
    steps = []
    t, lo, _ = o.forward(rows[-1], True)
    steps.append(("pos 8191", t, lo))
    for i in range(2):
        t, lo, _ = o.forward(o.embed(teach[i]), True)
        steps.append((f"pos {8192 + i}", t, lo))
    o.prefill(ext[:C4_EXT])
    assert o.kv_len() == 8450
    t, lo, _ = o.forward(o.embed(teach[2]), True)
    steps.append(("pos 8450", t, lo))
    o.set_kv_len(o.kv_len() - C4_BACK - 1)
    o.prefill(ext[C4_EXT:C4_EXT + C4_EXT2])
    assert o.kv_len() == 8703
    t, lo, _ = o.forward(o.embed(teach[3]), True)
    steps.append(("pos 8703", t, lo))
    o.close()
    return m, rows, ext, teach, steps


@pytest.mark.parametrize("engine", [0, 2])
def test_c4_long_context_vs_oracle(qa, c4, engine):
    m, rows, ext, teach, steps = c4
    d = gpu_decoder(qa, m, 9216, engine)
    d.prefill(rows[:-1])
    got = [(d.forward(rows[-1]), d.read_logits())]
    for i in range(2):
        got.append((d.forward_token(teach[i]), d.read_logits()))
    d.prefill(ext[:C4_EXT])
    got.append((d.forward_token(teach[2]), d.read_logits()))
    d.set_kv_len(d.kv_len() - C4_BACK - 1)
    d.prefill(ext[C4_EXT:C4_EXT + C4_EXT2])
    assert d.kv_len() == 8703
    got.append((d.forward_token(teach[3]), d.read_logits()))
    assert d.engine() == engine and d.fallbacks() == 0
    worst = max(check_step(lg, lo, t, ot, f"engine {engine} {what}")
                for (t, lg), (what, ot, lo) in zip(got, steps))
    print(f"C4 engine {engine}: 8191-row prefill, steps at 8191-8193 / 8450 / 8703: max |dlogit| {worst:.2e}")
    d.close()


# ----------------------------------------------------------------- C5
# C5 at its real window: the cache capped at 1024 positions, 24 chunks.  Each
# chunk adds 49 positions (roll back 5, prefill 30, 24 forwards); a 21-row head
# makes the cache reach 21 + 25 + 24 + 19 x 49 = 1001 positions before the
# first window reset (a 9-row head would peak at 989)
C5_HEAD, C5_AUDIO, C5_BACK, C5_STEPS, C5_CHUNKS, C5_CAP, C5_KEEP = 21, 26, 5, 24, 24, 1024, 3


def c5_ops(P, m):
    head, _ = P.prompt_rows(m, 0, C5_HEAD, seed=5)
    audio = [P.synth_f32(C5_AUDIO * 1024, 5, P.synth_audio_id(50 + c)).reshape(C5_AUDIO, 1024)
             for c in range(C5_CHUNKS)]
    return head, audio


def run_c5(dec, embed, head, audio, forced=None, peak=None):
    """The C5 op list on a decoder (GPU or oracle).  forced: per chunk the
    tokens to feed (teacher forcing); None: the decoder's own greedy tokens.
    Returns per step (token, logits) and the number of window resets."""
    out, prev, resets = [], [], 0
    dec.set_kv_len(0)
    dec.prefill(head)
    for c in range(len(audio)):
        if prev:
            dec.set_kv_len(dec.kv_len() - C5_BACK)
        if dec.kv_len() + C5_BACK + C5_AUDIO + C5_STEPS > C5_CAP:
            dec.set_kv_len(C5_HEAD)
            dec.prefill(np.concatenate(audio[max(0, c - C5_KEEP):c]))
            resets += 1
        rows = audio[c]
        if prev:
            rows = np.concatenate([np.stack([embed(t) for t in prev[-C5_BACK:]]), rows])
        dec.prefill(rows[:-1])
        chunk = []
        for i in range(C5_STEPS):
            feed = rows[-1] if i == 0 else embed(forced[c][i - 1] if forced else chunk[-1][0])
            chunk.append(dec.step(feed))
        if peak is not None:
            peak.append(dec.kv_len())
        out.append(chunk)
        prev = forced[c] if forced else [t for t, _ in chunk]
    return out, resets


class _OracleSteps:
    def __init__(self, o):
        self.o = o

    def __getattr__(self, k):
        return getattr(self.o, k)

    def step(self, row):
        t, lo, _ = self.o.forward(row, True)
        return int(t), lo


class _GpuSteps:
    def __init__(self, d):
        self.d = d

    def __getattr__(self, k):
        return getattr(self.d, k)

    def step(self, row):
        t = self.d.forward(row)
        return int(t), self.d.read_logits()


@pytest.fixture(scope="module")
def c5(P, gpu):
    m = P.SynthModel(P.Config(*CFG06_2L), seed=5)
    head, audio = c5_ops(P, m)
    o = _OracleSteps(P.Oracle(m, threads=ORACLE_THREADS))
    peak = []
    ref, resets = run_c5(o, m.embed, head, audio, peak=peak)
    o.close()
    assert resets >= 1, "the window reset path was not exercised"
    assert max(peak) > 1000, f"the cache never passed 1000 positions (peak {max(peak)})"
    return m, head, audio, ref


@pytest.mark.parametrize("path", ["graph", "split", "relay"])
def test_c5_streaming_oplist_vs_oracle(qa, c5, path):
    """All three decode paths: the graph engine, the split persistent kernel and
    the relay persistent kernel (which serves every C5 launch: the positions
    stay below 1024)."""
    m, head, audio, ref = c5
    engine = 0 if path == "graph" else 2
    d = _GpuSteps(gpu_decoder(qa, m, C5_CAP + 64, engine))
    if engine == 2:
        d.set_relay(path == "relay")
    forced = [[t for t, _ in chunk] for chunk in ref]
    got, resets = run_c5(d, m.embed, head, audio, forced)
    assert resets >= 1 and d.engine() == engine and d.fallbacks() == 0
    if engine == 2:
        assert d.last_kernel() == (2 if path == "relay" else 1)
    worst = 0.0
    for c, (gc, rc) in enumerate(zip(got, ref)):
        for i, ((t, lg), (ot, lo)) in enumerate(zip(gc, rc)):
            worst = max(worst, check_step(lg, lo, t, ot, f"{path} chunk {c} step {i}"))
    print(f"C5 {path}: {len(audio)} chunks x {C5_STEPS} steps, {resets} window reset(s), cap {C5_CAP}: "
          f"max |dlogit| {worst:.2e}")
    d.close()


# ----------------------------------------------------------------- 1.7B, C3 prefill length
C3_ROWS = 1516


@pytest.fixture(scope="module")
def c3(P, gpu):
    m = P.SynthModel(P.Config(*CFG17_2L), seed=6)
    rows, _ = P.prompt_rows(m, C3_ROWS - 16, 16, seed=6)
    teach = [int(t) for t in P.synth_tokens(3, 6, P.synth_tokens_id(60))]
    o = P.Oracle(m, threads=ORACLE_THREADS)
    o.prefill(rows[:-1])
    steps = [o.forward(rows[-1], True)[:2]]
    for t in teach:
        steps.append(o.forward(o.embed(t), True)[:2])
    o.close()
    return m, rows, teach, steps


@pytest.mark.parametrize("engine", [0, 2])
def test_17b_c3_prefill_vs_oracle(qa, c3, engine):
    m, rows, teach, steps = c3
    d = gpu_decoder(qa, m, 2048, engine)
    d.prefill(rows[:-1])
    got = [(d.forward(rows[-1]), d.read_logits())]
    for t in teach:
        got.append((d.forward_token(t), d.read_logits()))
    assert d.engine() == engine and d.fallbacks() == 0
    worst = max(check_step(lg, lo, t, ot, f"1.7B engine {engine} step {i}")
                for i, ((t, lg), (ot, lo)) in enumerate(zip(got, steps)))
    print(f"1.7B (2 layers) engine {engine}: 1515-row prefill + {len(teach) + 1} steps: max |dlogit| {worst:.2e}")
    d.close()


# ----------------------------------------------------------------- EOS
@pytest.fixture(scope="module")
def eos(P, gpu):
    return eos_model(P)


@pytest.mark.parametrize("engine", [0, 2])
def test_generate_stops_at_eos(P, qa, eos, engine):
    """generate(stop_on_eos) keeps the tokens up to and including the first
    <|im_end|> and leaves the KV as the reference loop does: the last row and
    every kept text token forwarded once, the EOS itself never forwarded."""
    rows, _ = P.prompt_rows(eos, 40, 8, seed=3)
    o = P.Oracle(eos, threads=ORACLE_THREADS)
    o.prefill(rows[:-1])
    t, _, _ = o.forward(rows[-1])
    kept, last = P.greedy_until_eos(o, t, 30)
    assert last == P.TOKEN_IM_END and len(kept) == 4
    d = gpu_decoder(qa, eos, 256, engine)
    d.prefill(rows[:-1])
    t1 = d.forward(rows[-1])
    assert t1 == kept[0]
    gen = list(d.generate(t1, 30, stop_on_eos=True))
    assert gen == kept[1:] + [P.TOKEN_IM_END]
    assert d.kv_len() == o.kv_len() == rows.shape[0] + len(kept)
    # without the stop the same steps run on (the KV then holds all of them)
    d.set_kv_len(rows.shape[0])
    gen2 = list(d.generate(t1, 6))
    assert gen2[:4] == gen and d.kv_len() == rows.shape[0] + 6
    assert d.engine() == engine and d.fallbacks() == 0
    d.close()
    o.close()


@pytest.mark.parametrize("engine", [0, 2])
def test_stream_chunks_vs_reference_loop(P, qa, eos, engine):
    """The streaming driver (qwen_hip_stream_chunk) against the reference's
    chunk loop restated on the oracle (RefStream): per chunk the reused
    prefix, the kept tokens (chunks end at <|im_end|> or at max_new) and the
    KV length; the chunk inputs grow, carry earlier tokens and drop their
    oldest audio once there are five windows."""
    m = eos
    head, _ = P.prompt_rows(m, 0, 8, seed=3)
    audio = [P.synth_f32(12 * 1024, 3, P.synth_audio_id(c)).reshape(12, 1024) for c in range(8)]
    tail = np.stack([m.embed(t) for t in (151644, 77091, 198)])
    ref = P.RefStream(P.Oracle(m, threads=ORACLE_THREADS))
    d = gpu_decoder(qa, m, 512, engine)
    st = qa.Stream(d)
    carried, ends = [], set()
    for c in range(len(audio)):
        parts = [head] + audio[max(0, c - 4):c + 1] + [tail]
        if carried:
            parts.append(np.stack([m.embed(t) for t in carried]))
        rows = np.ascontiguousarray(np.concatenate(parts), np.float32)
        want, want_reused = ref.chunk(rows, 8)
        got, reused = st.chunk(rows, 8)
        assert reused == want_reused, (c, reused, want_reused)
        assert list(got) == want, (c, list(got), want)
        assert d.kv_len() == ref.dec.kv_len() == rows.shape[0] + len(want)
        ends.add("eos" if len(want) < 8 else "max_new")
        carried = want[:max(0, len(want) - 2)]
    assert ends == {"eos", "max_new"}, ends
    assert d.engine() == engine and d.fallbacks() == 0
    st.close()
    d.close()
