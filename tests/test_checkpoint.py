"""Checkpoint reader (qwen_hip_checkpoint_*, host only) against the
reference's own safetensors reader compiled from its sources (oracle/_ref:
multi_safetensors_open / multi_safetensors_find / safetensors_data,
qwen_asr_safetensors.c:194-394) on the same files: every tensor's dtype,
shape and bytes must agree, for a single file and for shards."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

from ckpt_util import write_checkpoint


class SafeTensor(C.Structure):          # safetensor_t, qwen_asr_safetensors.h:25-32
    _fields_ = [("name", C.c_char * 256), ("dtype", C.c_int), ("ndim", C.c_int), ("shape", C.c_int64 * 8),
                ("data_offset", C.c_size_t), ("data_size", C.c_size_t)]


def ref_reader(P):
    ref = P.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    ref.multi_safetensors_open.restype = C.c_void_p
    ref.multi_safetensors_open.argtypes = [C.c_char_p]
    ref.multi_safetensors_close.argtypes = [C.c_void_p]
    ref.multi_safetensors_find.restype = C.POINTER(SafeTensor)
    ref.multi_safetensors_find.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p)]
    ref.safetensors_data.restype = C.c_void_p
    ref.safetensors_data.argtypes = [C.c_void_p, C.POINTER(SafeTensor)]
    return ref


@pytest.fixture(scope="module")
def tiny_model(P):
    return P.SynthModel(P.CFG_TINY, seed=4, norm_std=0.1)


@pytest.mark.parametrize("shards,norm_bf16", [(1, False), (3, True)])
def test_reader_matches_reference_reader(P, qa, tmp_path, tiny_model, shards, norm_bf16):
    names = write_checkpoint(tiny_model, str(tmp_path), shards=shards, norm_bf16=norm_bf16)
    ck = qa.Checkpoint(str(tmp_path))
    assert len(ck) == len(names)
    ref = ref_reader(P)
    ms = ref.multi_safetensors_open(str(tmp_path).encode())
    assert ms
    try:
        for n in names:
            sf = C.c_void_p()
            t = ref.multi_safetensors_find(ms, n.encode(), C.byref(sf))
            assert t, n
            t = t.contents
            dt, shape, data = ck.tensor(n)
            assert dt == t.dtype, n
            assert shape == tuple(t.shape[i] for i in range(t.ndim)), n
            assert data == C.string_at(ref.safetensors_data(sf, C.byref(t)), t.data_size), n
        assert ck.tensor("thinker.model.layers.9.mlp.up_proj.weight") is None
    finally:
        ref.multi_safetensors_close(ms)
    cfg = ck.config()
    c = P.CFG_TINY
    assert (cfg.hidden, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.intermediate, cfg.vocab) == \
           (c.hidden, c.layers, c.heads, c.kv_heads, c.head_dim, c.intermediate, c.vocab)
    assert abs(cfg.rms_eps - 1e-6) < 1e-12 and cfg.rope_theta == 1e6
    ck.close()


def test_reader_weights_are_the_models(P, qa, tmp_path, tiny_model):
    """the bytes handed to the upload are the model's arrays (BF16 raw bits,
    norms widened exactly from BF16)"""
    write_checkpoint(tiny_model, str(tmp_path), norm_bf16=True)
    ck = qa.Checkpoint(str(tmp_path))
    dt, shape, data = ck.tensor("thinker.model.layers.1.mlp.down_proj.weight")
    assert dt == qa.ST_BF16
    assert np.array_equal(np.frombuffer(data, np.uint16).reshape(shape), tiny_model.layers[1][P.DOWN])
    dt, shape, data = ck.tensor("thinker.model.layers.0.input_layernorm.weight")
    assert dt == qa.ST_BF16 and shape == (P.CFG_TINY.hidden,)
    want = P.bf16_to_f32(np.array([qa.lib().qwen_f32_to_bf16_rne(float(v)) for v in tiny_model.layers[0][P.INNORM]],
                                  np.uint16))
    got = P.bf16_to_f32(np.frombuffer(data, np.uint16))
    assert np.array_equal(got, want)


def test_reader_rejects_bad_files(qa, tmp_path):
    with pytest.raises(RuntimeError, match="no model.safetensors"):
        qa.Checkpoint(str(tmp_path))
    bad = tmp_path / "model.safetensors"
    bad.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(RuntimeError, match="header length"):
        qa.Checkpoint(str(tmp_path))
    hdr = b'{"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 64]}}'
    bad.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 16)
    with pytest.raises(RuntimeError, match="bad byte range"):
        qa.Checkpoint(str(tmp_path))
    hdr = b'{"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]'
    bad.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 16)
    with pytest.raises(RuntimeError, match="malformed"):
        qa.Checkpoint(str(tmp_path))
    hdr = b'{"__metadata__": {"k": "v,}"}, "a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}'
    bad.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 16)
    ck = qa.Checkpoint(str(tmp_path))
    assert len(ck) == 1 and ck.tensor("a")[1] == (4,)
    with pytest.raises(RuntimeError, match="embed_tokens"):
        ck.config()


def test_encoder_config_from_tensor_shapes(P, qa, tmp_path):
    """qwen_hip_checkpoint_enc_config: d_model from conv_out rows, ffn from fc1
    rows, output_dim from proj2 rows, layers counted, 64-wide heads (the
    encoder part of the reference's detect_config); a checkpoint without an
    audio tower is refused with a message."""
    from safetensors.torch import save_file
    from ckpt_util import enc_tensors
    cfg = qa.EncConfig(128, 3, 2, 64, 256, 96, 100, 800)
    t = enc_tensors(P.SynthEncoder(cfg, seed=2))
    save_file(t, str(tmp_path / "model.safetensors"))
    got = qa.Checkpoint(str(tmp_path)).enc_config()
    assert [getattr(got, f) for f, _ in qa.EncConfig._fields_] == [128, 3, 2, 64, 256, 96, 100, 800]
    del t["thinker.audio_tower.proj2.weight"]
    save_file(t, str(tmp_path / "model.safetensors"))
    with pytest.raises(RuntimeError, match="no audio encoder"):
        qa.Checkpoint(str(tmp_path)).enc_config()
