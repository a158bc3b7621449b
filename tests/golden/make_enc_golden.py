"""Write the encoder golden fixtures with the reference's own encoder
(qwen_encoder_forward, qwen_asr_encoder.c:171-372, compiled from its sources
into oracle/_ref by oracle/Makefile).  Inputs are regenerated from seeds
(pyoracle.SynthEncoder / synth_mel); the fixtures hold the configuration,
seeds, a weight checksum and the reference output.

    python tests/golden/make_enc_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import pyoracle as P  # noqa: E402

CASES = {
    # tiny model: partial last chunk (250 frames = 100 + 100 + 50) and 26-token windows
    "enc_tiny": dict(cfg=(128, 2, 2, 64, 256, 96, 100, 200), seed=1, frames=250, mel_set=1),
    # 0.6B widths (d_model 896, 14 heads, ffn 3584, output 1024), 2 layers, 2 chunks
    "enc_06b2": dict(cfg=(896, 2, 14, 64, 3584, 1024, 100, 800), seed=2, frames=163, mel_set=2),
}


class Cfg:
    def __init__(self, t):
        (self.d_model, self.layers, self.heads, self.head_dim, self.ffn_dim, self.output_dim,
         self.chunk_size, self.n_window_infer) = t


def tokens(cfg, frames):
    co = lambda w: (w + 2 - 3) // 2 + 1
    n = (frames + cfg.chunk_size - 1) // cfg.chunk_size
    last = frames - (n - 1) * cfg.chunk_size
    return (n - 1) * co(co(co(cfg.chunk_size))) + co(co(co(last)))


def weight_checksum(m):
    h = 0.0
    for arrs in m.layers + [m.stem]:
        for a in arrs:
            h += float(np.float64(a).sum()) + float(np.abs(np.float64(a)).sum())
    return h


def main():
    for name, c in CASES.items():
        cfg = Cfg(c["cfg"])
        m = P.SynthEncoder(cfg, seed=c["seed"])
        mel = P.synth_mel(c["frames"], c["seed"], c["mel_set"])
        T = tokens(cfg, c["frames"])
        out = P.RefEncoder(m).forward(mel, T)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), cfg=np.array(c["cfg"], np.int32),
                            seed=c["seed"], frames=c["frames"], mel_set=c["mel_set"], out=out,
                            weight_sum=weight_checksum(m), mel_sum=float(np.float64(mel).sum()))
        print(name, T, "tokens, |out| max", float(np.abs(out).max()))


if __name__ == "__main__":
    main()
