"""TEST INFRASTRUCTURE: ctypes access to the CPU checkers.

* ``Oracle``  - the C restatement in ``oracle/qwen_oracle.c`` (liborc.so).
* ``RefModel`` - the reference's own decoder compiled from /root/reference
  into ``oracle/_ref`` (ref_harness.c drives qwen_decoder_prefill /
  qwen_decoder_forward, reference qwen_asr_decoder.c:262, :388).
* ``SynthModel`` - host copies of the seeded synthetic weights, drawn with the
  same C generator (qwen-asr_amd/csrc/host/synth.c) the product uses.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker / CPU baseline.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


@dataclass(frozen=True)
class Config:
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    eps: float = 1e-6
    theta: float = 1e6

    @property
    def q_dim(self):
        return self.heads * self.head_dim

    @property
    def kv_dim(self):
        return self.kv_heads * self.head_dim

    def args(self):
        return (self.hidden, self.layers, self.heads, self.kv_heads, self.head_dim,
                self.intermediate, self.vocab, C.c_float(self.eps), C.c_float(self.theta))


# Reference shapes (qwen_asr.c:153-186) and the small shape the tests use.
CFG_06B = Config(1024, 28, 16, 8, 128, 3072, 151936)
CFG_17B = Config(2048, 28, 16, 8, 128, 6144, 151936)
CFG_TINY = Config(256, 2, 4, 2, 128, 512, 1000)

# Tensor ids, as include/qwen_synth.h.
SYNTH_EMBED, SYNTH_FINAL_NORM = 1, 2
WQ, WK, WV, WO, GATE, UP, DOWN, QNORM, KNORM, INNORM, POSTNORM = range(11)


def synth_layer_id(layer, field):
    return 1000 + 32 * layer + field


def synth_audio_id(chunk):
    return 500000 + chunk


def synth_tokens_id(s):
    return 600000 + s


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load(path):
    if not os.path.exists(path):
        build()
    return C.CDLL(path)


_orc = None


def orc_lib():
    global _orc
    if _orc is None:
        lib = _load(os.path.join(HERE, "liborc.so"))
        lib.qwen_synth_normal_bf16.argtypes = [_u16p, C.c_size_t, C.c_uint64, C.c_uint64, C.c_double, C.c_double, C.c_int]
        lib.qwen_synth_normal_f32.argtypes = [_f32p, C.c_size_t, C.c_uint64, C.c_uint64, C.c_double, C.c_double, C.c_int]
        lib.qwen_synth_uniform_f32.argtypes = [_f32p, C.c_size_t, C.c_uint64, C.c_uint64, C.c_double, C.c_double, C.c_int]
        lib.qwen_synth_tokens.argtypes = [_i32p, C.c_size_t, C.c_uint64, C.c_uint64, C.c_int]
        lib.qwen_checksum_u16.argtypes = [_u16p, C.c_size_t]
        lib.qwen_checksum_u16.restype = C.c_uint64
        lib.qwen_f32_to_bf16_rne.argtypes = [C.c_float]
        lib.qwen_f32_to_bf16_rne.restype = C.c_uint16
        lib.orc_create.restype = C.c_void_p
        lib.orc_create.argtypes = [C.c_int] * 7 + [C.c_float, C.c_float]
        lib.orc_set_layer.argtypes = [C.c_void_p, C.c_int] + [_u16p] * 7 + [_f32p] * 4
        lib.orc_set_embeddings.argtypes = [C.c_void_p, _u16p, _f32p]
        lib.orc_prefill.argtypes = [C.c_void_p, _f32p, C.c_int]
        lib.orc_forward.argtypes = [C.c_void_p, _f32p, C.c_void_p, C.c_void_p]
        lib.orc_embed_token.argtypes = [C.c_void_p, C.c_int, _f32p]
        lib.orc_kv_len.argtypes = [C.c_void_p]
        lib.orc_set_kv_len.argtypes = [C.c_void_p, C.c_int]
        lib.orc_destroy.argtypes = [C.c_void_p]
        lib.orc_set_threads.argtypes = [C.c_int]
        lib.orc_rms_norm.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_float]
        lib.orc_rms_norm_per_head.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_float]
        lib.orc_rope_table.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_float]
        lib.orc_apply_rope.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        lib.orc_linear_bf16.argtypes = [_f32p, _f32p, _u16p, C.c_int, C.c_int, C.c_int]
        lib.orc_causal_attention.argtypes = [_f32p, _f32p, _f32p, _f32p] + [C.c_int] * 5 + [C.c_float, C.c_int]
        lib.orc_swiglu.argtypes = [_f32p, _f32p, C.c_int, C.c_int]
        lib.orc_argmax_matvec_bf16.argtypes = [_f32p, _u16p, C.c_int, C.c_int, C.c_void_p]
        lib.orc_argmax_matvec_bf16.restype = C.c_int
        lib.orc_dot_bf16.argtypes = [_u16p, _f32p, C.c_int]
        lib.orc_dot_bf16.restype = C.c_float
        lib.orc_stream_triad.argtypes = [C.c_long, C.c_int]
        lib.orc_stream_triad.restype = C.c_double
        _orc = lib
    return _orc


def host_info():
    """CPU model, logical CPUs and the ISA level the compiled reference runs at."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    isa = "x86-64-v4 (AVX-512F/BW)" if _cpu_has_avx512() else "x86-64-v3 (AVX2+FMA)"
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "isa": isa}


def stream_gbs(threads, n=1 << 26, reps=5):
    """STREAM-style triad bandwidth of this host on `threads` OpenMP threads (GB/s)."""
    lib = orc_lib()
    lib.orc_set_threads(threads)
    return float(lib.orc_stream_triad(n, reps))


def _cpu_has_avx512():
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
        return " avx512f" in flags and " avx512bw" in flags
    except OSError:
        return False


_ref = None


def ref_path():
    name = "libqwen_ref_v4.so" if _cpu_has_avx512() else "libqwen_ref_v3.so"
    return os.path.join(HERE, "_ref", name)


def ref_available():
    return os.path.exists(ref_path())


def ref_lib():
    """The compiled reference (None when oracle/_ref was never built)."""
    global _ref
    if _ref is None:
        p = ref_path()
        if not os.path.exists(p):
            return None
        lib = C.CDLL(p)
        lib.ref_create.restype = C.c_void_p
        lib.ref_create.argtypes = [C.c_int] * 7 + [C.c_float, C.c_float]
        lib.ref_set_layer.argtypes = [C.c_void_p, C.c_int] + [_u16p] * 7 + [_f32p] * 4
        lib.ref_set_embeddings.argtypes = [C.c_void_p, _u16p, _f32p]
        lib.ref_set_threads.argtypes = [C.c_int]
        lib.ref_prefill.argtypes = [C.c_void_p, _f32p, C.c_int]
        lib.ref_forward.argtypes = [C.c_void_p, _f32p, C.c_void_p, C.c_void_p]
        lib.ref_embed_token.argtypes = [C.c_void_p, C.c_int, _f32p]
        lib.ref_kv_len.argtypes = [C.c_void_p]
        lib.ref_set_kv_len.argtypes = [C.c_void_p, C.c_int]
        lib.ref_kv_max.argtypes = [C.c_void_p]
        lib.ref_bf16_widen.argtypes = [C.c_void_p, C.c_void_p, C.c_long]
        lib.ref_bf16_widen.restype = None
        lib.ref_generate.argtypes = [C.c_void_p, C.c_int, C.c_int, _i32p]
        lib.ref_generate.restype = C.c_double
        lib.ref_time_prefill.argtypes = [C.c_void_p, _f32p, C.c_int]
        lib.ref_time_prefill.restype = C.c_double
        lib.ref_destroy.argtypes = [C.c_void_p]
        # the reference op layer itself (qwen_asr_kernels.h)
        lib.qwen_rms_norm.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_float]
        lib.qwen_rms_norm_per_head.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_float]
        lib.qwen_apply_rope_neox.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        lib.qwen_linear_nobias_bf16.argtypes = [_f32p, _f32p, _u16p, C.c_int, C.c_int, C.c_int]
        lib.qwen_causal_attention.argtypes = [_f32p, _f32p, _f32p, _f32p] + [C.c_int] * 5 + [C.c_float, C.c_int]
        lib.qwen_swiglu_multiply.argtypes = [_f32p, _f32p, C.c_int, C.c_int]
        lib.qwen_argmax_matvec_bf16.argtypes = [_f32p, _u16p, C.c_int, C.c_int]
        lib.qwen_argmax_matvec_bf16.restype = C.c_int
        lib.qwen_compute_rope_neox.argtypes = [_f32p, _f32p, _i32p, C.c_int, C.c_int, C.c_float]
        _ref = lib
    return _ref


# ---------------------------------------------------------------------------
# synthetic inputs (same generator as the product)
# ---------------------------------------------------------------------------
def synth_bf16(n, seed, tid, std=0.02, mean=0.0):
    out = np.empty(n, np.uint16)
    orc_lib().qwen_synth_normal_bf16(out, n, seed, tid, mean, std, 0)
    return out


def synth_f32(n, seed, tid, std=1.0, mean=0.0):
    out = np.empty(n, np.float32)
    orc_lib().qwen_synth_normal_f32(out, n, seed, tid, mean, std, 0)
    return out


def synth_uniform(n, seed, tid, lo=-1.0, hi=1.0):
    out = np.empty(n, np.float32)
    orc_lib().qwen_synth_uniform_f32(out, n, seed, tid, lo, hi, 0)
    return out


def synth_tokens(n, seed, tid, n_ids=151643):
    out = np.empty(n, np.int32)
    orc_lib().qwen_synth_tokens(out, n, seed, tid, n_ids)
    return out


def checksum_u16(a):
    a = np.ascontiguousarray(a, np.uint16).ravel()
    return int(orc_lib().qwen_checksum_u16(a, a.size))


def bf16_to_f32(a):
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a):
    a = np.ascontiguousarray(a, np.float32)
    b = a.view(np.uint32).astype(np.uint64)
    b = b + 0x7FFF + ((b >> 16) & 1)
    return (b >> 16).astype(np.uint16)


class SynthModel:
    """Host copies of the seeded synthetic decoder (weights N(0, std) bf16,
    norms 1 + norm_std*N(0,1) fp32; norm_std = 0 gives all-ones norms)."""

    def __init__(self, cfg: Config, seed=0, weight_std=0.02, norm_std=0.0):
        self.cfg, self.seed = cfg, seed
        c = cfg
        self.layers = []
        for l in range(c.layers):
            L = {}
            shapes = {WQ: (c.q_dim, c.hidden), WK: (c.kv_dim, c.hidden), WV: (c.kv_dim, c.hidden),
                      WO: (c.hidden, c.q_dim), GATE: (c.intermediate, c.hidden),
                      UP: (c.intermediate, c.hidden), DOWN: (c.hidden, c.intermediate)}
            for f, shp in shapes.items():
                L[f] = synth_bf16(shp[0] * shp[1], seed, synth_layer_id(l, f), weight_std).reshape(shp)
            for f, n in ((QNORM, c.head_dim), (KNORM, c.head_dim), (INNORM, c.hidden), (POSTNORM, c.hidden)):
                L[f] = self._norm(n, synth_layer_id(l, f), norm_std)
            self.layers.append(L)
        self.emb = synth_bf16(c.vocab * c.hidden, seed, SYNTH_EMBED, weight_std).reshape(c.vocab, c.hidden)
        self.final_norm = self._norm(c.hidden, SYNTH_FINAL_NORM, norm_std)

    def _norm(self, n, tid, norm_std):
        if norm_std == 0.0:
            return np.ones(n, np.float32)
        return synth_f32(n, self.seed, tid, norm_std, 1.0)

    def embed(self, token):
        return bf16_to_f32(self.emb[token])

    def layer_args(self, l):
        L = self.layers[l]
        return [L[f] for f in (WQ, WK, WV, WO, GATE, UP, DOWN, QNORM, KNORM, INNORM, POSTNORM)]


class _Decoder:
    _create = _set_layer = _set_emb = _prefill = _forward = _embed = _kvlen = _setkv = _destroy = None

    def _init(self, lib, model: SynthModel, prefix):
        self.lib, self.model, self.cfg = lib, model, model.cfg
        g = lambda n: getattr(lib, prefix + n)
        self.h = g("create")(*self.cfg.args())
        if not self.h:
            raise RuntimeError("create failed")
        for l in range(self.cfg.layers):
            g("set_layer")(self.h, l, *model.layer_args(l))
        g("set_embeddings")(self.h, model.emb.reshape(-1), model.final_norm)
        self._p = prefix

    def prefill(self, rows):
        rows = np.ascontiguousarray(rows, np.float32).reshape(-1)
        n = rows.size // self.cfg.hidden
        if n:
            getattr(self.lib, self._p + "prefill")(self.h, rows, n)

    def forward(self, row, want_logits=False, want_hidden=False):
        row = np.ascontiguousarray(row, np.float32)
        hid = np.empty(self.cfg.hidden, np.float32) if want_hidden else None
        lg = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        tok = getattr(self.lib, self._p + "forward")(
            self.h, row, hid.ctypes.data if hid is not None else None,
            lg.ctypes.data if lg is not None else None)
        return tok, lg, hid

    def embed(self, token):
        out = np.empty(self.cfg.hidden, np.float32)
        getattr(self.lib, self._p + "embed_token")(self.h, int(token), out)
        return out

    def kv_len(self):
        return getattr(self.lib, self._p + "kv_len")(self.h)

    def set_kv_len(self, n):
        getattr(self.lib, self._p + "set_kv_len")(self.h, int(n))

    def close(self):
        if self.h:
            getattr(self.lib, self._p + "destroy")(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Oracle(_Decoder):
    """The C restatement (qwen_oracle.c)."""

    def __init__(self, model: SynthModel, threads=0):
        lib = orc_lib()
        if threads:
            lib.orc_set_threads(threads)
        self._init(lib, model, "orc_")


class RefModel(_Decoder):
    """The reference decoder compiled from its own sources (oracle/_ref)."""

    def __init__(self, model: SynthModel, threads=1):
        lib = ref_lib()
        if lib is None:
            raise RuntimeError("oracle/_ref not built")
        lib.ref_set_threads(threads)
        self._init(lib, model, "ref_")

    def generate(self, first_token, n_steps):
        out = np.empty(n_steps, np.int32)
        secs = self.lib.ref_generate(self.h, int(first_token), int(n_steps), out)
        return out, secs

    def extend_kv(self, n, row):
        """Raise the KV length to n without prefilling, for timing decode steps
        at a long context: the rows past the prefilled ones hold zeros (the
        attention's cost depends on the length, not the values).  The length
        is first stepped to the cache's capacity so that each growth of the
        next forward (qwen_asr_decoder.c:403-406, :133-160) copies only rows
        inside the old cache; `row` is that forward's input."""
        while self.lib.ref_kv_max(self.h) <= n:
            self.set_kv_len(self.lib.ref_kv_max(self.h))
            self.forward(row)
        self.set_kv_len(n)

    def time_prefill(self, rows):
        rows = np.ascontiguousarray(rows, np.float32).reshape(-1)
        return self.lib.ref_time_prefill(self.h, rows, rows.size // self.cfg.hidden)


# ---------------------------------------------------------------------------
# the reference's callers of the decoder (restated for the tests)
# ---------------------------------------------------------------------------
TOKEN_ENDOFTEXT, TOKEN_IM_END = 151643, 151645


def greedy_until_eos(dec, token, max_tokens):
    """The reference's greedy loop after the first token (qwen_asr.c:729-759,
    and the chunk loop :1802-1814): while fewer than max_tokens tokens were
    generated, stop at <|endoftext|> / <|im_end|>, otherwise keep the token
    and forward its embedding.  `dec` (Oracle or RefModel) has just produced
    `token`.  Returns (kept tokens, the token the last forward produced)."""
    kept, n = [], 0
    while n < max_tokens:
        n += 1
        if token in (TOKEN_ENDOFTEXT, TOKEN_IM_END):
            break
        kept.append(int(token))
        token, _, _ = dec.forward(dec.embed(token))
    return kept, token


class RefStream:
    """The decoder half of the reference's streaming transcriber
    (qwen_asr.c:1748-1829) on a CPU decoder: per chunk, keep the KV of the
    longest prefix of the prefill rows (all rows but the last) that is
    bitwise equal to the previous chunk's (memcmp, :1752-1761), prefill the
    rest (:1764-1770), forward the last row (:1773-1774), then the greedy
    loop up to max_new tokens (:1802-1814)."""

    def __init__(self, dec):
        self.dec, self.prev = dec, None

    def chunk(self, rows, max_new):
        rows = np.ascontiguousarray(rows, np.float32)
        n = rows.shape[0] - 1
        reused = 0
        if self.prev is not None:
            cmp = min(n, self.prev.shape[0])
            while reused < cmp and self.prev[reused].tobytes() == rows[reused].tobytes():
                reused += 1
        self.dec.set_kv_len(reused)
        if n > reused:
            self.dec.prefill(rows[reused:n])
        token, _, _ = self.dec.forward(rows[n])
        self.prev = rows[:n].copy()
        kept, _ = greedy_until_eos(self.dec, token, max_new)
        return kept, reused


# ---------------------------------------------------------------------------
# workload inputs
# ---------------------------------------------------------------------------
def prompt_rows(model: SynthModel, n_audio, n_ids, seed=0, audio_chunk=0, token_set=0, embed=None):
    """ids[:n_ids//2] || n_audio audio rows N(0,1) || ids[n_ids//2:], the
    prefix/audio/suffix template of qwen_asr.c:339-347 with synthetic ids."""
    c = model.cfg
    ids = synth_tokens(n_ids, seed, synth_tokens_id(token_set), min(151643, c.vocab))
    audio = synth_f32(n_audio * c.hidden, seed, synth_audio_id(audio_chunk)).reshape(n_audio, c.hidden)
    emb = embed or model.embed
    head = [emb(t) for t in ids[: n_ids // 2]]
    tail = [emb(t) for t in ids[n_ids // 2:]]
    rows = np.concatenate([np.array(head, np.float32).reshape(-1, c.hidden), audio,
                           np.array(tail, np.float32).reshape(-1, c.hidden)], axis=0)
    return np.ascontiguousarray(rows, np.float32), ids


# ---------------------------------------------------------------------------
# Audio encoder (reference qwen_asr_encoder.c) -- synthetic weights and the
# compiled reference's forward pass.
# ---------------------------------------------------------------------------
ENC_FIELDS = ("wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "ln1_w", "ln1_b",
              "fc1_w", "fc1_b", "fc2_w", "fc2_b", "ln2_w", "ln2_b")
STEM_FIELDS = ("conv1_w", "conv1_b", "conv2_w", "conv2_b", "conv3_w", "conv3_b", "conv_out_w",
               "ln_post_w", "ln_post_b", "proj1_w", "proj1_b", "proj2_w", "proj2_b")


def synth_enc_id(layer, field):
    return 700000 + 32 * layer + field


def synth_mel_id(s):
    return 750000 + s


class SynthEncoder:
    """The seeded synthetic encoder of qwen_hip_encoder_load_synthetic, as host
    fp32 arrays: bf16 N(0, wstd) matrices widened (conv1 N(0, 10 wstd)), fp32
    biases N(0, wstd), LayerNorm weights N(1, 0.1) and biases N(0, 0.02)."""

    def __init__(self, cfg, seed=0, wstd=0.02):
        d, f, o = cfg.d_model, cfg.ffn_dim, cfg.output_dim
        mat = lambda n, tid, std: bf16_to_f32(synth_bf16(n, seed, tid, std)).astype(np.float32)
        vec = lambda n, tid, mean, std: synth_f32(n, seed, tid, std, mean)
        self.cfg = cfg
        self.layers = []
        for l in range(cfg.layers):
            i = lambda k: synth_enc_id(l, k)
            self.layers.append([
                mat(d * d, i(0), wstd).reshape(d, d), vec(d, i(1), 0, wstd),
                mat(d * d, i(2), wstd).reshape(d, d), vec(d, i(3), 0, wstd),
                mat(d * d, i(4), wstd).reshape(d, d), vec(d, i(5), 0, wstd),
                mat(d * d, i(6), wstd).reshape(d, d), vec(d, i(7), 0, wstd),
                vec(d, i(8), 1.0, 0.1), vec(d, i(9), 0, 0.02),
                mat(f * d, i(10), wstd).reshape(f, d), vec(f, i(11), 0, wstd),
                mat(d * f, i(12), wstd).reshape(d, f), vec(d, i(13), 0, wstd),
                vec(d, i(14), 1.0, 0.1), vec(d, i(15), 0, 0.02)])
        s = lambda k: synth_enc_id(30, k)
        self.stem = [mat(480 * 9, s(0), wstd * 10), vec(480, s(1), 0, wstd),
                     mat(480 * 4320, s(2), wstd), vec(480, s(3), 0, wstd),
                     mat(480 * 4320, s(4), wstd), vec(480, s(5), 0, wstd),
                     mat(d * 7680, s(6), wstd).reshape(d, 7680), vec(d, s(7), 1.0, 0.1), vec(d, s(8), 0, 0.02),
                     mat(d * d, s(9), wstd).reshape(d, d), vec(d, s(10), 0, wstd),
                     mat(o * d, s(11), wstd).reshape(o, d), vec(o, s(12), 0, wstd)]


def synth_mel(frames, seed=0, s=0):
    return synth_f32(128 * frames, seed, synth_mel_id(s)).reshape(128, frames)


class RefEncoder:
    """qwen_encoder_forward of the reference (oracle/_ref), on a SynthEncoder's arrays."""

    def __init__(self, model: SynthEncoder, threads=0):
        lib = ref_lib()
        if lib is None:
            raise RuntimeError("oracle/_ref is not built")
        if threads:
            lib.ref_set_threads.argtypes = [C.c_int]
            lib.ref_set_threads(threads)
        lib.ref_enc_create.restype = C.c_void_p
        lib.ref_enc_create.argtypes = [C.c_int] * 8
        lib.ref_enc_set_layer.argtypes = [C.c_void_p, C.c_int] + [_f32p] * 16
        lib.ref_enc_set_stem.argtypes = [C.c_void_p] + [_f32p] * 13
        lib.ref_enc_forward.argtypes = [C.c_void_p, _f32p, C.c_int, _f32p, C.c_long]
        lib.ref_enc_time.argtypes = [C.c_void_p, _f32p, C.c_int, _f32p, C.c_long]
        lib.ref_enc_time.restype = C.c_double
        lib.ref_enc_destroy.argtypes = [C.c_void_p]
        self.lib, self.model, c = lib, model, model.cfg
        self.h = lib.ref_enc_create(c.d_model, c.layers, c.heads, c.head_dim, c.ffn_dim, c.output_dim,
                                    c.chunk_size, c.n_window_infer)
        self._keep = []
        for l, arrs in enumerate(model.layers):
            arrs = [np.ascontiguousarray(a, np.float32) for a in arrs]
            self._keep += arrs
            assert lib.ref_enc_set_layer(self.h, l, *arrs) == 0
        arrs = [np.ascontiguousarray(a, np.float32) for a in model.stem]
        self._keep += arrs
        lib.ref_enc_set_stem(self.h, *arrs)

    def forward(self, mel, tokens):
        mel = np.ascontiguousarray(mel, np.float32)
        out = np.empty((tokens, self.model.cfg.output_dim), np.float32)
        T = self.lib.ref_enc_forward(self.h, mel, mel.shape[1], out, out.size)
        assert T == tokens, (T, tokens)
        return out

    def time(self, mel, tokens):
        mel = np.ascontiguousarray(mel, np.float32)
        out = np.empty((tokens, self.model.cfg.output_dim), np.float32)
        return self.lib.ref_enc_time(self.h, mel, mel.shape[1], out, out.size)

    def __del__(self):
        try:
            self.lib.ref_enc_destroy(self.h)
        except Exception:
            pass
