"""The audio encoder (qwen_hip_encoder_*) against the reference's encoder
(qwen_encoder_forward, qwen_asr_encoder.c:171-372): the committed fixtures
tests/golden/enc_*.npz hold the compiled reference's output on seeded
weights and mel (tests/golden/make_enc_golden.py; test_encoder_oracle.py
re-derives one of them on the CPU).

Both compute in fp32 (the products of the fp32 matrix cores are exact fp32
products); sums run in another order, tanhf / expf of two libms differ by
ulps, and 2 layers of LayerNorm / attention / GELU amplify that: the bar is
|gpu - ref| <= 1e-4 + 1e-3 |ref| elementwise.
"""
import ctypes as C
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ATOL, RTOL = 1e-4, 1e-3


def fixture(name):
    return np.load(os.path.join(GOLD, name + ".npz"))


def build(qa, P, g):
    cfg = qa.EncConfig(*[int(v) for v in g["cfg"]])
    m = P.SynthEncoder(cfg, seed=int(g["seed"]))
    from golden.make_enc_golden import weight_checksum
    assert abs(weight_checksum(m) - float(g["weight_sum"])) <= 1e-9 * abs(float(g["weight_sum"]))
    mel = P.synth_mel(int(g["frames"]), int(g["seed"]), int(g["mel_set"]))
    assert float(np.float64(mel).sum()) == float(g["mel_sum"])
    return cfg, m, mel


def load(qa, cfg, m):
    e = qa.Encoder(cfg, 0)
    for l, arrs in enumerate(m.layers):
        e.load_layer(l, arrs)
    e.load_stem(m.stem)
    return e


@pytest.mark.parametrize("name", ["enc_tiny", "enc_06b2"])
def test_encoder_matches_reference(P, qa, gpu, name):
    g = fixture(name)
    cfg, m, mel = build(qa, P, g)
    e = load(qa, cfg, m)
    out = e.forward(mel)
    ref = g["out"]
    assert out.shape == ref.shape
    err = np.abs(out - ref)
    print(f"{name}: {out.shape[0]} tokens, max |d| {err.max():.2e}, max rel {float((err / (np.abs(ref) + 1e-6)).max()):.2e}")
    assert np.all(err <= ATOL + RTOL * np.abs(ref)), float((err - RTOL * np.abs(ref)).max())
    e.close()


def d2h(ptr, shape):
    """copy a device buffer (raw pointer) to a new host array"""
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    out = np.empty(shape, np.float32)
    assert hip.hipMemcpy(out.ctypes.data, C.c_void_p(ptr), out.nbytes, 2) == 0   # hipMemcpyDeviceToHost
    return out


def test_encoder_synthetic_loader_and_device_path(P, qa, gpu):
    """load_synthetic (C recipe) == the same weights through load_layer/load_stem,
    bit for bit; forward_device == forward; repeated calls with other lengths
    (buffers regrown, partial chunks of every size class)"""
    cfg = qa.EncConfig(128, 2, 2, 64, 256, 96, 100, 200)
    m = P.SynthEncoder(cfg, seed=5)
    a = load(qa, cfg, m)
    b = qa.Encoder(cfg, 0)
    b.load_synthetic(5, 0.02)
    for frames in (320, 99, 1, 400):
        mel = P.synth_mel(frames, 5, 3)
        oa = a.forward(mel)
        ob = b.forward(mel)
        assert oa.shape[0] == a.tokens(frames)
        assert np.array_equal(oa, ob), frames
        dm = gpu.from_numpy(np.ascontiguousarray(mel)).to("cuda")
        gpu.cuda.synchronize()
        T, p = b.forward_device(dm.data_ptr(), frames)
        assert np.array_equal(d2h(p, (T, cfg.output_dim)), ob), frames
    a.close()
    b.close()


def test_encoder_rows_feed_the_decoder(P, qa, gpu):
    """encoder output (0.6B widths: 1024 = the decoder's hidden) straight into
    the decoder's device prefill gives what the host path gives"""
    cfg = qa.enc_preset(0)
    cfg.layers = 2
    e = qa.Encoder(cfg, 0)
    e.load_synthetic(0, 0.02)
    mel = P.synth_mel(300, 0, 4)
    rows = e.forward(mel)
    dm = gpu.from_numpy(np.ascontiguousarray(mel)).to("cuda")
    gpu.cuda.synchronize()
    T, p = e.forward_device(dm.data_ptr(), 300)
    dcfg = qa.preset(0)
    d = qa.Decoder(dcfg, 0, 512)
    d.load_synthetic(0, 0.02, 0.0)
    d.set_engine(0)
    d.prefill(rows[:-1])
    t_host = d.forward(rows[-1])
    d.set_kv_len(0)
    d.prefill_device(p, T - 1)
    t_dev = d.forward(rows[-1])
    assert T == rows.shape[0] and t_dev == t_host
    d.close()
    e.close()


def test_encoder_from_checkpoint(P, qa, gpu, tmp_path):
    """thinker.audio_tower.* read from a safetensors checkpoint (BF16 matrices,
    F32 vectors, two shards): shape taken from the tensors, chunk 100 and
    attention window 800 frames as the reference fixes them (qwen_asr.c:182-184),
    output bit-identical to the same weights loaded by hand with that config"""
    import ckpt_util
    from safetensors.torch import save_file
    g = fixture("enc_tiny")
    cfg, m, mel = build(qa, P, g)
    t = ckpt_util.enc_tensors(m)
    names = sorted(t)
    half = len(names) // 2
    save_file({n: t[n] for n in names[:half]}, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file({n: t[n] for n in names[half:]}, str(tmp_path / "model-00002-of-00002.safetensors"))
    e = qa.Encoder.from_checkpoint(str(tmp_path), 0)
    cfg.n_window_infer = 800
    for f, _ in qa.EncConfig._fields_:
        assert getattr(e.cfg, f) == getattr(cfg, f), f
    out = e.forward(mel)
    ref_h = load(qa, cfg, m)
    np.testing.assert_array_equal(out, ref_h.forward(mel))
    e.close()
    ref_h.close()


def test_encoder_error_conventions(P, qa, gpu):
    """Invalid shapes, calls before the weights are in, empty input and a
    layer index out of range fail with a code and a message; the encoder
    stays usable afterwards."""
    bad = qa.EncConfig(128, 2, 3, 64, 256, 96, 100, 200)          # heads * 64 != d_model
    assert not qa.lib().qwen_hip_encoder_create(C.byref(bad), 0)
    assert "encoder configuration" in qa.last_error()
    cfg = qa.EncConfig(128, 2, 2, 64, 256, 96, 100, 200)
    e = qa.Encoder(cfg, 0)
    mel = P.synth_mel(120, 1, 0)
    with pytest.raises(RuntimeError, match="not loaded"):
        e.forward(mel)
    m = P.SynthEncoder(cfg, seed=1)
    e.load_stem(m.stem)
    with pytest.raises(RuntimeError, match="layer 0 not loaded"):
        e.forward(mel)
    with pytest.raises(RuntimeError):
        e.load_layer(cfg.layers, m.layers[0])
    assert "outside" in qa.last_error()
    for l, arrs in enumerate(m.layers):
        e.load_layer(l, arrs)
    with pytest.raises(RuntimeError, match="bad argument"):
        e.forward(np.zeros((128, 0), np.float32))
    ref = load(qa, cfg, m).forward(mel)
    np.testing.assert_array_equal(e.forward(mel), ref)
    e.close()


def test_encoder_fp32_weights_take_the_fp32_gemm(P, qa, gpu):
    """A weight matrix whose values are not all bf16 values (possible through
    the fp32 load API) keeps fp32 and runs on the fp32 GEMM, next to
    bf16-valued ones on the bf16 GEMM; the mix matches the reference encoder
    (oracle/_ref) on the same weights."""
    if not P.ref_available():
        pytest.skip("oracle/_ref not built")
    cfg = qa.EncConfig(128, 2, 2, 64, 256, 96, 100, 200)
    m = P.SynthEncoder(cfg, seed=9)
    rng = np.random.default_rng(9)
    wo = m.layers[1][6]
    m.layers[1][6] = (wo * (1.0 + 1e-3 * rng.standard_normal(wo.shape))).astype(np.float32)   # off the bf16 grid
    assert np.any(m.layers[1][6].view(np.uint32) & 0xFFFF)
    mel = P.synth_mel(250, 9, 1)
    e = load(qa, cfg, m)
    out = e.forward(mel)
    ref = P.RefEncoder(m).forward(mel, e.tokens(250))
    err = np.abs(out - ref)
    assert np.all(err <= ATOL + RTOL * np.abs(ref)), float(err.max())
    e.close()
