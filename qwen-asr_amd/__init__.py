"""qwen-asr_amd: the Qwen3-ASR decoder token loop on MI355X (gfx950).

The product is the C-ABI library ``libqwen_asr_hip.so`` (declared in
``include/qwen_asr_hip.h``): hand-written HIP kernels plus C host code.  This
module is only a thin ctypes view of that ABI for tests, ``bench.py`` and
``__graft_entry__``; it has no compute of its own and no fallback: if the
library is missing, loading fails loudly.

The directory name is not a Python identifier, so import it with
``importlib.import_module("qwen-asr_amd")``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqwen_asr_hip.so")

QWEN_HIP_TOKEN_ENDOFTEXT = 151643
QWEN_HIP_TOKEN_IM_END = 151645
ERRORS = {0: "OK", -1: "EINVAL", -2: "ENOMEM", -3: "EDEVICE", -4: "ESTATE"}
KERNEL_SPLIT, KERNEL_RELAY, RELAY_MAX_POS = 1, 2, 1024   # QWEN_HIP_KERNEL_*, QWEN_HIP_RELAY_MAX_POS


class HipConfig(C.Structure):
    _fields_ = [("hidden", C.c_int), ("layers", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int),
                ("head_dim", C.c_int), ("intermediate", C.c_int), ("vocab", C.c_int),
                ("rms_eps", C.c_float), ("rope_theta", C.c_float)]


class LayerWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("wq", "wk", "wv", "wo", "gate", "up", "down",
                                          "q_norm", "k_norm", "input_norm", "post_attn_norm")]


def build(jobs=8):
    """Compile the library in-tree (hipcc for gfx950 + gcc)."""
    subprocess.run(["make", "-s", "-C", HERE, f"-j{jobs}"], check=True)


_lib = None

# (name, restype, argtypes) of every exported entry point of include/qwen_asr_hip.h
_vp, _i, _f, _d, _u64 = C.c_void_p, C.c_int, C.c_float, C.c_double, C.c_uint64
SIGNATURES = [
    ("qwen_hip_config_preset", None, [_vp, _i]),
    ("qwen_hip_decoder_create", _vp, [_vp, _i, _i]),
    ("qwen_hip_decoder_destroy", None, [_vp]),
    ("qwen_hip_decoder_load_layer", _i, [_vp, _i, _vp]),
    ("qwen_hip_decoder_load_embeddings", _i, [_vp, _vp, _vp]),
    ("qwen_hip_decoder_load_synthetic", _i, [_vp, _u64, _d, _d]),
    ("qwen_hip_decoder_prefill", _i, [_vp, _vp, _i]),
    ("qwen_hip_decoder_prefill_device", _i, [_vp, _vp, _i]),
    ("qwen_hip_decoder_forward", _i, [_vp, _vp]),
    ("qwen_hip_decoder_forward_token", _i, [_vp, _i]),
    ("qwen_hip_decoder_generate", _i, [_vp, _i, _i, _vp, _i]),
    ("qwen_hip_decoder_kv_len", _i, [_vp]),
    ("qwen_hip_decoder_set_kv_len", _i, [_vp, _i]),
    ("qwen_hip_decoder_set_keep_logits", _i, [_vp, _i]),
    ("qwen_hip_decoder_read_hidden", _i, [_vp, _vp]),
    ("qwen_hip_decoder_read_logits", _i, [_vp, _vp]),
    ("qwen_hip_decoder_set_engine", _i, [_vp, _i]),
    ("qwen_hip_decoder_engine", _i, [_vp]),
    ("qwen_hip_decoder_set_fallback", _i, [_vp, _i]),
    ("qwen_hip_decoder_fallbacks", _i, [_vp]),
    ("qwen_hip_decoder_set_wait_limit", _i, [_vp, _d]),
    ("qwen_hip_decoder_set_tag_epoch", _i, [_vp, C.c_uint]),
    ("qwen_hip_decoder_tag_epoch", C.c_uint, [_vp]),
    ("qwen_hip_decoder_set_trace", _i, [_vp, _i]),
    ("qwen_hip_decoder_read_trace", _i, [_vp, _vp, C.c_size_t]),
    ("qwen_hip_decoder_set_relay", _i, [_vp, _i]),
    ("qwen_hip_decoder_last_kernel", _i, [_vp]),
    ("qwen_hip_decoder_stream", _vp, [_vp]),
    ("qwen_hip_decoder_step_bytes", _d, [_vp, _i]),
    ("qwen_hip_last_error", C.c_char_p, []),
    ("qwen_hip_decoder_config", _vp, [_vp]),
    ("qwen_hip_checkpoint_open", _vp, [C.c_char_p]),
    ("qwen_hip_checkpoint_close", None, [_vp]),
    ("qwen_hip_checkpoint_count", _i, [_vp]),
    ("qwen_hip_checkpoint_tensor", _i, [_vp, C.c_char_p, _vp, _vp, _vp, _vp]),
    ("qwen_hip_checkpoint_config", _i, [_vp, _vp]),
    ("qwen_hip_decoder_load_checkpoint", _i, [_vp, _vp]),
    ("qwen_hip_decoder_create_from_checkpoint", _vp, [C.c_char_p, _i, _i]),
    ("qwen_hip_stream_create", _vp, [_vp]),
    ("qwen_hip_stream_destroy", None, [_vp]),
    ("qwen_hip_stream_reset", None, [_vp]),
    ("qwen_hip_stream_chunk", _i, [_vp, _vp, _i, _i, _vp, _vp]),
    ("qwen_hip_stream_stats", _i, [_vp, _vp, _vp]),
    ("qwen_hip_enc_config_preset", None, [_vp, _i]),
    ("qwen_hip_encoder_create", _vp, [_vp, _i]),
    ("qwen_hip_encoder_destroy", None, [_vp]),
    ("qwen_hip_encoder_load_layer", _i, [_vp, _i, _vp]),
    ("qwen_hip_encoder_load_stem", _i, [_vp, _vp]),
    ("qwen_hip_encoder_load_synthetic", _i, [_vp, _u64, _d]),
    ("qwen_hip_encoder_tokens", _i, [_vp, _i]),
    ("qwen_hip_encoder_forward", _i, [_vp, _vp, _i, _vp]),
    ("qwen_hip_encoder_forward_device", _i, [_vp, _vp, _i, _vp]),
    ("qwen_hip_encoder_stream", _vp, [_vp]),
    ("qwen_hip_encoder_config", _vp, [_vp]),
    ("qwen_hip_checkpoint_enc_config", _i, [_vp, _vp]),
    ("qwen_hip_encoder_load_checkpoint", _i, [_vp, _vp]),
    ("qwen_hip_encoder_create_from_checkpoint", _vp, [C.c_char_p, _i]),
    ("qwen_hip_vocab_load", _vp, [C.c_char_p]),
    ("qwen_hip_vocab_free", None, [_vp]),
    ("qwen_hip_vocab_size", _i, [_vp]),
    ("qwen_hip_vocab_piece", C.c_char_p, [_vp, _i]),
    ("qwen_hip_vocab_transcript", C.c_long, [_vp, _vp, _i, _i, C.c_char_p, C.c_size_t]),
    ("qwen_hip_add_inplace", _i, [_vp, _vp, _i, _vp]),
    ("qwen_hip_rms_norm", _i, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    ("qwen_hip_rms_norm_per_head", _i, [_vp, _vp, _i, _i, _i, _f, _vp]),
    ("qwen_hip_apply_rope_neox", _i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    ("qwen_hip_swiglu_multiply", _i, [_vp, _vp, _i, _i, _vp]),
    ("qwen_hip_linear_nobias_bf16", _i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    ("qwen_hip_linear_nobias_bf16_qkv", _i, [_vp] * 7 + [_i, _i, _i, _vp]),
    ("qwen_hip_linear_nobias_bf16_noalloc", _i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    ("qwen_hip_linear_noalloc_max_bytes", C.c_size_t, []),
    ("qwen_hip_causal_attention", _i, [_vp] * 4 + [_i] * 5 + [_f, _i, _vp]),
    ("qwen_hip_argmax_matvec_bf16", _i, [_vp, _vp, _i, _i, _vp]),
    ("qwen_synth_key", _u64, [_u64, _u64]),
    ("qwen_f32_to_bf16_rne", C.c_uint16, [_f]),
    ("qwen_synth_normal_bf16", None, [_vp, C.c_size_t, _u64, _u64, _d, _d, _i]),
    ("qwen_synth_normal_f32", None, [_vp, C.c_size_t, _u64, _u64, _d, _d, _i]),
    ("qwen_synth_uniform_f32", None, [_vp, C.c_size_t, _u64, _u64, _d, _d, _i]),
    ("qwen_synth_tokens", None, [_vp, C.c_size_t, _u64, _u64, _i]),
    ("qwen_checksum_u16", _u64, [_vp, C.c_size_t]),
]


def lib():
    """Load libqwen_asr_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (no CPU fallback exists)")
        L = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error():
    return lib().qwen_hip_last_error().decode(errors="replace")


def check(rc, what=""):
    if rc < 0:
        raise RuntimeError(f"{what}: {ERRORS.get(rc, rc)}: {last_error()}")
    return rc


def preset(model_b=0):
    c = HipConfig()
    lib().qwen_hip_config_preset(C.byref(c), model_b)
    return c


def config_from(cfg):
    """HipConfig from any object with hidden/layers/heads/kv_heads/head_dim/intermediate/vocab/eps/theta."""
    return HipConfig(cfg.hidden, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.intermediate,
                     cfg.vocab, cfg.eps, cfg.theta)


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------------------
# seeded synthetic inputs (csrc/host/synth.c; tensor ids of include/qwen_synth.h)
# ---------------------------------------------------------------------------
SYNTH_EMBED = 1


def synth_bf16(n, seed, tensor_id, std=0.02):
    out = np.empty(n, np.uint16)
    lib().qwen_synth_normal_bf16(_ptr(out), n, seed, tensor_id, 0.0, std, 0)
    return out


def synth_f32(n, seed, tensor_id, std=1.0, mean=0.0):
    out = np.empty(n, np.float32)
    lib().qwen_synth_normal_f32(_ptr(out), n, seed, tensor_id, mean, std, 0)
    return out


def synth_uniform(n, seed, tensor_id, lo=-1.0, hi=1.0):
    out = np.empty(n, np.float32)
    lib().qwen_synth_uniform_f32(_ptr(out), n, seed, tensor_id, lo, hi, 0)
    return out


def synth_tokens(n, seed, tensor_id, n_ids=151643):
    out = np.empty(n, np.int32)
    lib().qwen_synth_tokens(_ptr(out), n, seed, tensor_id, n_ids)
    return out


def synth_mel(frames, seed=0, s=0):
    """seeded N(0,1) log-mel [128][frames] (tensor id 750000 + s)"""
    return synth_f32(128 * frames, seed, 750000 + s).reshape(128, frames)


def bf16_to_f32(a):
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)


def prompt_rows(cfg, n_audio, n_ids, seed=0, audio_chunk=0, token_set=0, emb=None):
    """The benchmark input rows: ids[:n/2] || n_audio rows N(0,1) || ids[n/2:]
    (the prefix/audio/suffix template of the reference, qwen_asr.c:339-347,
    with synthetic ids).  emb: the [vocab][hidden] bf16 table, regenerated
    from the seed when not given."""
    ids = synth_tokens(n_ids, seed, 600000 + token_set, min(151643, cfg.vocab))
    if emb is None:
        emb = synth_bf16(cfg.vocab * cfg.hidden, seed, SYNTH_EMBED).reshape(cfg.vocab, cfg.hidden)
    audio = synth_f32(n_audio * cfg.hidden, seed, 500000 + audio_chunk).reshape(n_audio, cfg.hidden)
    head = bf16_to_f32(emb[ids[: n_ids // 2]]).reshape(-1, cfg.hidden)
    tail = bf16_to_f32(emb[ids[n_ids // 2:]]).reshape(-1, cfg.hidden)
    return np.ascontiguousarray(np.concatenate([head, audio, tail]), np.float32), ids, emb


ST_F32, ST_F16, ST_BF16, ST_OTHER = 0, 1, 2, -1


class EncConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("d_model", "layers", "heads", "head_dim", "ffn_dim", "output_dim",
                                       "chunk_size", "n_window_infer")]


class EncLayerWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "ln1_w", "ln1_b",
                                          "fc1_w", "fc1_b", "fc2_w", "fc2_b", "ln2_w", "ln2_b")]


class EncStemWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("conv1_w", "conv1_b", "conv2_w", "conv2_b", "conv3_w", "conv3_b",
                                          "conv_out_w", "ln_post_w", "ln_post_b", "proj1_w", "proj1_b",
                                          "proj2_w", "proj2_b")]


def enc_preset(model_b):
    cfg = EncConfig()
    lib().qwen_hip_enc_config_preset(C.byref(cfg), int(model_b))
    return cfg


class Encoder:
    """The audio encoder on one GPU (mel [128][frames] -> rows [tokens][output_dim])."""

    def __init__(self, cfg: EncConfig, device=0):
        self.cfg = cfg
        self.h = lib().qwen_hip_encoder_create(C.byref(cfg), device)
        if not self.h:
            raise RuntimeError(f"qwen_hip_encoder_create: {last_error()}")

    @classmethod
    def from_checkpoint(cls, model_dir, device=0):
        h = lib().qwen_hip_encoder_create_from_checkpoint(os.fsencode(model_dir), device)
        if not h:
            raise RuntimeError(f"qwen_hip_encoder_create_from_checkpoint: {last_error()}")
        self = cls.__new__(cls)
        self.h = h
        c = EncConfig.from_address(lib().qwen_hip_encoder_config(h))
        self.cfg = EncConfig(*[getattr(c, f) for f, _ in EncConfig._fields_])
        return self

    def load_synthetic(self, seed=0, wstd=0.02):
        check(lib().qwen_hip_encoder_load_synthetic(self.h, seed, wstd), "encoder_load_synthetic")

    def load_layer(self, l, arrays):
        """arrays: the 16 fp32 arrays of EncLayerWeights in field order"""
        arrs = [np.ascontiguousarray(a, np.float32) for a in arrays]
        w = EncLayerWeights(*[a.ctypes.data for a in arrs])
        check(lib().qwen_hip_encoder_load_layer(self.h, l, C.byref(w)), f"encoder_load_layer {l}")

    def load_stem(self, arrays):
        arrs = [np.ascontiguousarray(a, np.float32) for a in arrays]
        w = EncStemWeights(*[a.ctypes.data for a in arrs])
        check(lib().qwen_hip_encoder_load_stem(self.h, C.byref(w)), "encoder_load_stem")

    def tokens(self, frames):
        return lib().qwen_hip_encoder_tokens(C.byref(self.cfg), int(frames))

    def forward(self, mel):
        mel = np.ascontiguousarray(mel, np.float32)
        frames = mel.shape[1]
        out = np.empty((max(self.tokens(frames), 0), self.cfg.output_dim), np.float32)
        T = lib().qwen_hip_encoder_forward(self.h, _ptr(mel), frames, _ptr(out))
        check(T if T < 0 else 0, "encoder_forward")
        return out[:T]

    def forward_device(self, d_mel_ptr, frames):
        """(tokens, device pointer of the [tokens][output_dim] rows)"""
        p = C.c_void_p()
        T = lib().qwen_hip_encoder_forward_device(self.h, C.c_void_p(d_mel_ptr), int(frames), C.byref(p))
        check(T if T < 0 else 0, "encoder_forward_device")
        return T, p.value

    def stream(self):
        return lib().qwen_hip_encoder_stream(self.h)

    def close(self):
        if getattr(self, "h", None):
            lib().qwen_hip_encoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Vocab:
    """vocab.json for token -> text (host only)."""

    def __init__(self, path):
        self.h = lib().qwen_hip_vocab_load(os.fsencode(path))
        if not self.h:
            raise RuntimeError(f"qwen_hip_vocab_load: {last_error()}")

    def __len__(self):
        return lib().qwen_hip_vocab_size(self.h)

    def piece(self, token):
        return lib().qwen_hip_vocab_piece(self.h, int(token))

    def transcript(self, tokens, past_asr_text=False):
        """bytes of the text the reference's loop assembles from `tokens`"""
        t = np.ascontiguousarray(tokens, np.int32)
        n = lib().qwen_hip_vocab_transcript(self.h, _ptr(t), t.size, int(past_asr_text), None, 0)
        check(n if n < 0 else 0, "vocab_transcript")
        buf = C.create_string_buffer(n + 1)
        lib().qwen_hip_vocab_transcript(self.h, _ptr(t), t.size, int(past_asr_text), buf, n + 1)
        return buf.raw[:n]

    def close(self):
        if getattr(self, "h", None):
            lib().qwen_hip_vocab_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Checkpoint:
    """A safetensors checkpoint directory mapped read-only (host only, no GPU)."""

    def __init__(self, model_dir):
        self.h = lib().qwen_hip_checkpoint_open(os.fsencode(model_dir))
        if not self.h:
            raise RuntimeError(f"qwen_hip_checkpoint_open: {last_error()}")

    def __len__(self):
        return lib().qwen_hip_checkpoint_count(self.h)

    def config(self):
        cfg = HipConfig()
        check(lib().qwen_hip_checkpoint_config(self.h, C.byref(cfg)), "checkpoint_config")
        return cfg

    def enc_config(self):
        cfg = EncConfig()
        check(lib().qwen_hip_checkpoint_enc_config(self.h, C.byref(cfg)), "checkpoint_enc_config")
        return cfg

    def tensor(self, name):
        """(dtype code, shape, raw bytes) of one tensor; None when absent."""
        dt, nd, shape, ptr = C.c_int(), C.c_int(), (C.c_longlong * 8)(), C.c_void_p()
        if lib().qwen_hip_checkpoint_tensor(self.h, name.encode(), C.byref(dt), C.byref(nd), shape,
                                            C.byref(ptr)) != 0:
            return None
        shp = tuple(int(shape[i]) for i in range(nd.value))
        n = int(np.prod(shp)) if shp else 1
        size = {ST_F32: 4, ST_F16: 2, ST_BF16: 2}.get(dt.value, 0) * n
        return dt.value, shp, C.string_at(ptr.value, size) if size else b""

    def close(self):
        if getattr(self, "h", None):
            lib().qwen_hip_checkpoint_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Decoder:
    """One decoder context on one GPU (the decoder-level ABI)."""

    def __init__(self, cfg: HipConfig, device=0, kv_capacity=1024):
        self.cfg = cfg
        self.h = lib().qwen_hip_decoder_create(C.byref(cfg), device, kv_capacity)
        if not self.h:
            raise RuntimeError(f"qwen_hip_decoder_create: {last_error()}")

    @classmethod
    def from_checkpoint(cls, model_dir, device=0, kv_capacity=1024):
        """Create a decoder with the shape and weights of a safetensors checkpoint."""
        h = lib().qwen_hip_decoder_create_from_checkpoint(os.fsencode(model_dir), device, kv_capacity)
        if not h:
            raise RuntimeError(f"qwen_hip_decoder_create_from_checkpoint: {last_error()}")
        self = cls.__new__(cls)
        self.h = h
        self.cfg = HipConfig.from_address(lib().qwen_hip_decoder_config(h))
        self.cfg = HipConfig(*[getattr(self.cfg, f) for f, _ in HipConfig._fields_])
        return self

    def load_checkpoint(self, ckpt: "Checkpoint"):
        check(lib().qwen_hip_decoder_load_checkpoint(self.h, ckpt.h), "load_checkpoint")

    # weights -------------------------------------------------------------
    def load_synthetic(self, seed=0, weight_std=0.02, norm_std=0.0):
        check(lib().qwen_hip_decoder_load_synthetic(self.h, seed, weight_std, norm_std), "load_synthetic")

    def load_layer(self, l, wq, wk, wv, wo, gate, up, down, q_norm, k_norm, input_norm, post_attn_norm):
        arrs = [np.ascontiguousarray(a) for a in (wq, wk, wv, wo, gate, up, down)]
        arrs += [np.ascontiguousarray(a, np.float32) for a in (q_norm, k_norm, input_norm, post_attn_norm)]
        w = LayerWeights(*[a.ctypes.data for a in arrs])
        check(lib().qwen_hip_decoder_load_layer(self.h, l, C.byref(w)), f"load_layer {l}")

    def load_embeddings(self, emb, final_norm):
        emb = np.ascontiguousarray(emb, np.uint16)
        fn = np.ascontiguousarray(final_norm, np.float32)
        check(lib().qwen_hip_decoder_load_embeddings(self.h, _ptr(emb), _ptr(fn)), "load_embeddings")

    def load_model(self, model):
        """Upload a host model object exposing layer_args(l), emb, final_norm."""
        for l in range(self.cfg.layers):
            self.load_layer(l, *model.layer_args(l))
        self.load_embeddings(model.emb, model.final_norm)

    # token loop ----------------------------------------------------------
    def prefill(self, rows):
        rows = np.ascontiguousarray(rows, np.float32)
        n = rows.size // self.cfg.hidden
        check(lib().qwen_hip_decoder_prefill(self.h, _ptr(rows), n), "prefill")

    def prefill_device(self, ptr, n):
        check(lib().qwen_hip_decoder_prefill_device(self.h, C.c_void_p(ptr), n), "prefill_device")

    def forward(self, row):
        row = np.ascontiguousarray(row, np.float32)
        return lib().qwen_hip_decoder_forward(self.h, _ptr(row))

    def forward_token(self, token):
        return lib().qwen_hip_decoder_forward_token(self.h, int(token))

    def generate(self, first_token, n_steps, stop_on_eos=False):
        out = np.empty(max(n_steps, 1), np.int32)
        k = check(lib().qwen_hip_decoder_generate(self.h, int(first_token), int(n_steps), _ptr(out),
                                                  1 if stop_on_eos else 0), "generate")
        return out[:k]

    def kv_len(self):
        return lib().qwen_hip_decoder_kv_len(self.h)

    def set_kv_len(self, n):
        check(lib().qwen_hip_decoder_set_kv_len(self.h, int(n)), "set_kv_len")

    def set_keep_logits(self, on):
        check(lib().qwen_hip_decoder_set_keep_logits(self.h, 1 if on else 0), "set_keep_logits")

    def set_engine(self, engine):
        check(lib().qwen_hip_decoder_set_engine(self.h, int(engine)), "set_engine")

    def engine(self):
        """Active decode engine: 0 graph, 1 eager, 2 persistent."""
        return lib().qwen_hip_decoder_engine(self.h)

    def set_fallback(self, on):
        """on: a failed persistent launch is redone by the graph engine (and counted);
        off: the call fails with QWEN_HIP_EDEVICE."""
        check(lib().qwen_hip_decoder_set_fallback(self.h, 1 if on else 0), "set_fallback")

    def fallbacks(self):
        """How many persistent launches failed and were redone by the graph engine."""
        return check(lib().qwen_hip_decoder_fallbacks(self.h), "fallbacks")

    def set_wait_limit(self, seconds):
        check(lib().qwen_hip_decoder_set_wait_limit(self.h, float(seconds)), "set_wait_limit")

    def set_tag_epoch(self, epoch):
        """Zero the persistent engine's exchange words and set the tag epoch."""
        check(lib().qwen_hip_decoder_set_tag_epoch(self.h, int(epoch)), "set_tag_epoch")

    def tag_epoch(self):
        return int(lib().qwen_hip_decoder_tag_epoch(self.h))

    def set_trace(self, step):
        check(lib().qwen_hip_decoder_set_trace(self.h, int(step)), "set_trace")

    def read_trace(self):
        """Wall-clock stamps (100 MHz) of the traced step: [256 blocks][704] in the
        layout of the kernel that ran (see last_kernel and the header)."""
        out = np.zeros((256, 704), np.uint64)
        words = check(lib().qwen_hip_decoder_read_trace(self.h, _ptr(out), out.size), "read_trace")
        return out.reshape(-1)[:256 * words].reshape(256, words).copy()

    def set_relay(self, on):
        """on (default where available): persistent launches whose positions stay
        below RELAY_MAX_POS run the relay kernel; off: always the split kernel."""
        check(lib().qwen_hip_decoder_set_relay(self.h, 1 if on else 0), "set_relay")

    def last_kernel(self):
        """Kernel of the last persistent launch: KERNEL_SPLIT (1), KERNEL_RELAY (2), 0 before any."""
        return check(lib().qwen_hip_decoder_last_kernel(self.h), "last_kernel")

    def read_hidden(self):
        out = np.empty(self.cfg.hidden, np.float32)
        check(lib().qwen_hip_decoder_read_hidden(self.h, _ptr(out)), "read_hidden")
        return out

    def read_logits(self):
        out = np.empty(self.cfg.vocab, np.float32)
        check(lib().qwen_hip_decoder_read_logits(self.h, _ptr(out)), "read_logits")
        return out

    def stream(self):
        return lib().qwen_hip_decoder_stream(self.h)

    def step_bytes(self, kv_len):
        return lib().qwen_hip_decoder_step_bytes(self.h, int(kv_len))

    def close(self):
        if getattr(self, "h", None):
            lib().qwen_hip_decoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass



class Stream:
    """The streaming driver over one decoder (prefix KV reuse per chunk)."""

    def __init__(self, dec: Decoder):
        self.dec = dec
        self.h = lib().qwen_hip_stream_create(dec.h)
        if not self.h:
            raise RuntimeError(f"qwen_hip_stream_create: {last_error()}")

    def chunk(self, rows, max_new):
        """(tokens, reused rows) of one chunk's decoder input rows [n][hidden]."""
        rows = np.ascontiguousarray(rows, np.float32)
        n = rows.size // self.dec.cfg.hidden
        out = np.zeros(max(max_new, 1), np.int32)
        reused = C.c_int()
        k = lib().qwen_hip_stream_chunk(self.h, _ptr(rows), n, int(max_new), _ptr(out), C.byref(reused))
        check(k, "stream_chunk")
        return [int(t) for t in out[:k]], reused.value

    def reset(self):
        lib().qwen_hip_stream_reset(self.h)

    def stats(self):
        tot, reu = C.c_longlong(), C.c_longlong()
        check(lib().qwen_hip_stream_stats(self.h, C.byref(tot), C.byref(reu)), "stream_stats")
        return tot.value, reu.value

    def close(self):
        if getattr(self, "h", None):
            lib().qwen_hip_stream_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# Intervals of the relay kernel's per-layer trace (words 24 l + i, header
# layout): name, first stamp, last stamp.  Each is the median over the blocks of
# the team that computes the layer.
RELAY_STAGES = (
    ("input: wave 0's quarter of the residual gathered, planes written", 1, 3),
    ("Q product stored", 3, 4),
    ("hop Q -> attention (512 words)", 4, 5),
    ("attention: q/k norm + RoPE + fold", 5, 7),
    ("attention: merge of 8 groups, partials stored", 7, 8),
    ("hop split partials -> merge slices", 8, 9),
    ("merge over the splits, stored", 9, 10),
    ("hop merged dims -> every block (256 words)", 10, 11),
    ("O product stored", 11, 12),
    ("hop O partials: cross-XCD half in", 12, 13),
    ("post-attention: wave 0's quarter gathered, planes written", 13, 15),
    ("gate|up products reduced", 15, 16),
    ("SwiGLU stored", 16, 17),
    ("hop SwiGLU -> down (384 words)", 17, 18),
    ("down product stored", 18, 19),
)


def relay_stage_us(tr, layers):
    """Per-layer stage times (microseconds) of one traced relay step: the median
    over layers 2 .. layers-3 of each stage's median over the computing team's
    blocks; plus the hand-over between layers (the last block's down store of
    layer l-1 to the median block's cross-XCD half of layer l's input), the
    layer period, and the LM head (rows of the median / slowest block).  tr is
    read_trace()'s [256][704] array of 100 MHz stamps."""
    tr = np.asarray(tr).astype(np.int64)
    TM = 24
    t = (tr - tr[tr > 0].min()) * 0.01
    out = {}
    ls = list(range(2, layers - 2))
    for name, a, b in RELAY_STAGES:
        v = [np.median(t[tr[:, TM * l] > 0, TM * l + b] - t[tr[:, TM * l] > 0, TM * l + a]) for l in ls]
        out[name] = round(float(np.mean(v)), 3)
    hx, per = [], []
    for l in ls:
        cb, pb, nb = tr[:, TM * l] > 0, tr[:, TM * (l - 1)] > 0, tr[:, TM * (l + 1)] > 0
        hx.append(np.median(t[cb, TM * l + 1]) - t[pb, TM * (l - 1) + 19].max())
        per.append(np.median(t[nb, TM * (l + 1) + 3]) - np.median(t[cb, TM * l + 3]))
    out["hop between layers: last down store -> cross-XCD half of the input in"] = round(float(np.mean(hx)), 3)
    out["layer period"] = round(float(np.mean(per)), 3)
    blk = tr[:, TM * layers] > 0
    lm = t[blk, TM * layers + 3] - t[blk, TM * layers + 2]
    out["LM head rows: median block"] = round(float(np.median(lm)), 3)
    out["LM head rows: slowest block"] = round(float(np.max(lm)), 3)
    tb = tr[:, TM * layers + 4] > 0
    out["token: last candidate -> median token"] = round(float(np.median(t[tb, TM * layers + 4]) - t[blk, TM * layers + 3].max()), 3)
    return out


def split_stage_us(tr, layers):
    """Per-layer stage times (microseconds) of one traced split-kernel step
    (the header's split trace layout): for each of the five stages (Q, A, O,
    F, D) the sync wave's wait for its input and the compute that follows
    (median over blocks, averaged over the layers), the LM head's wait and
    compute, the token wait, and the cross-XCD half of the two residual
    updates.  tr is read_trace()'s [256][704] array of 100 MHz stamps."""
    tr = np.asarray(tr).astype(np.int64)
    L = layers
    t = (tr - tr[:, 0].min()) * 0.01
    med = lambda x: float(np.median(x))
    out = {}
    for k, name in enumerate(("Q", "A", "O", "F", "D")):
        w = c = 0.0
        for l in range(L):
            ent, rdy = t[:, 10 * l + 2 * k], t[:, 10 * l + 2 * k + 1]
            nxt = t[:, 10 * l + 2 * k + 2] if (l < L - 1 or k < 4) else t[:, 10 * L]
            w += med(rdy - ent)
            c += med(nxt - rdy)
        out[f"stage {name}: wait"] = round(w / L, 3)
        out[f"stage {name}: compute"] = round(c / L, 3)
    out["LM head: wait"] = round(med(t[:, 10 * L + 1] - t[:, 10 * L]), 3)
    out["LM head: compute"] = round(med(t[:, 10 * L + 2] - t[:, 10 * L + 1]), 3)
    out["token: wait"] = round(med(t[:, 10 * L + 3] - t[:, 10 * L + 2]), 3)
    X = 640
    ls = range(2, L - 1)
    out["residual before Q: cross-XCD half"] = round(float(np.mean([med(t[:, X + 2 * l] - t[:, 10 * l]) for l in ls])), 3)
    out["residual before F: cross-XCD half"] = round(float(np.mean([med(t[:, X + 2 * l + 1] - t[:, 10 * l + 6]) for l in ls])), 3)
    out["layer period"] = round(float(np.mean([med(t[:, 10 * (l + 1)] - t[:, 10 * l]) for l in ls])), 3)
    return out
