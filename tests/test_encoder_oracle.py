"""The tiny encoder fixture (tests/golden/enc_tiny.npz) re-derived from the
reference's encoder compiled from its sources (oracle/_ref), and the token
count rule (qwen_asr_encoder.c:193-214) against closed forms."""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_enc_tokens_rule(qa):
    cfg = qa.enc_preset(0)
    tok = lambda f: qa.lib().qwen_hip_encoder_tokens(qa.C.byref(cfg), f)
    assert tok(100) == 13 and tok(200) == 26 and tok(1) == 1 and tok(101) == 14
    assert tok(163) == 13 + 8          # 63 frames: 32 -> 16 -> 8
    assert tok(3000) == 30 * 13


@pytest.mark.slow
def test_tiny_fixture_reproduces(P, qa):
    if not P.ref_available():
        pytest.skip("oracle/_ref not built")
    g = np.load(os.path.join(GOLD, "enc_tiny.npz"))
    cfg = qa.EncConfig(*[int(v) for v in g["cfg"]])
    m = P.SynthEncoder(cfg, seed=int(g["seed"]))
    mel = P.synth_mel(int(g["frames"]), int(g["seed"]), int(g["mel_set"]))
    out = P.RefEncoder(m).forward(mel, g["out"].shape[0])
    assert np.array_equal(out, g["out"])
