"""Write the golden fixtures of tests/golden/ from the reference's own decoder.

The reference has no tests or vectors for its decoder (its only harness,
asr_regression.py, needs real checkpoints), so the fixtures here are produced
by running the reference's C decoder, compiled unmodified from
/root/reference into oracle/_ref (see oracle/Makefile and
oracle/ref_harness.c), on seeded synthetic weights, with one thread (so every
row goes through the same 4-row AVX-512 matvec path of
qwen_asr_kernels_avx.c:25-97).

Run in the development container (the reference sources are not on the GPU
box; the committed .npz files are):
    python tests/golden/make_golden.py [names...]
"""
import json
import os
import platform
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import pyoracle as P  # noqa: E402


def top_k(lg, k=8):
    idx = np.argsort(-lg, kind="stable")[:k]
    return idx.astype(np.int32), lg[idx].astype(np.float32)


def meta(extra):
    cpu = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    d = {"reference_lib": os.path.basename(P.ref_path()), "cpu": cpu, "machine": platform.machine(),
         "threads": 1, "flags": "-O3 -ffast-math (x86-64-v4 or v3), no BLAS"}
    d.update(extra)
    return d


def tiny_teacher():
    """CFG_TINY, non-unit norms: prefill, then 13 forwards fed a fixed token
    sequence (teacher forcing), full logits and hidden state per step."""
    m = P.SynthModel(P.CFG_TINY, seed=0, norm_std=0.1)
    rows, ids = P.prompt_rows(m, 20, 6)
    teach = P.synth_tokens(12, 0, P.synth_tokens_id(7), P.CFG_TINY.vocab)
    r = P.RefModel(m, threads=1)
    r.prefill(rows[:-1])
    logits, hidden, toks = [], [], []
    inp = [rows[-1]] + [r.embed(t) for t in teach]
    for x in inp:
        t, lg, hd = r.forward(x, True, True)
        logits.append(lg); hidden.append(hd); toks.append(t)
    np.savez_compressed(os.path.join(HERE, "tiny_teacher.npz"), rows=rows, teach=teach,
                        logits=np.array(logits), hidden=np.array(hidden), tokens=np.array(toks, np.int32),
                        kv_len=np.int32(r.kv_len()))
    return meta({"config": "tiny", "n_prompt_rows": int(rows.shape[0]), "steps": len(inp)})


def free_run(name, cfg, n_audio, n_ids, n_forwards):
    """Reference step convention (qwen_asr.c:705-710): prefill all rows but
    the last, forward the last, then greedy forwards on each new token."""
    t0 = time.time()
    m = P.SynthModel(cfg, seed=0)
    rows, ids = P.prompt_rows(m, n_audio, n_ids)
    r = P.RefModel(m, threads=1)
    tp = time.time()
    r.prefill(rows[:-1])
    tp = time.time() - tp
    x = rows[-1]
    toks, ti, tv, margin = [], [], [], []
    for i in range(n_forwards):
        t, lg, _ = r.forward(x, True)
        i8, v8 = top_k(lg)
        assert i8[0] == t or lg[i8[0]] == lg[t]
        toks.append(t); ti.append(i8); tv.append(v8); margin.append(v8[0] - v8[1])
        x = r.embed(t)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), ids=ids, tokens=np.array(toks, np.int32),
                        top_idx=np.array(ti), top_val=np.array(tv), margin=np.array(margin, np.float32),
                        emb_checksum=np.uint64(P.checksum_u16(m.emb)),
                        wq0_checksum=np.uint64(P.checksum_u16(m.layers[0][P.WQ])),
                        n_audio=np.int32(n_audio), n_ids=np.int32(n_ids), kv_len=np.int32(r.kv_len()))
    return meta({"config": name, "hidden": cfg.hidden, "prefill_rows": int(rows.shape[0] - 1),
                 "forwards": n_forwards, "prefill_s": round(tp, 2), "total_s": round(time.time() - t0, 1)})


def logits_run(name, cfg, n_audio, n_ids, n_forwards, prefill_threads=1):
    """Full fp32 logits (every vocabulary row) of the first n_forwards greedy
    forwards of fixture `name`'s run, written to {name}_logits.npz beside the
    top-8 fixture (same model, rows and step convention as free_run).  The
    prefill may use more threads: its linears run the reference's
    single-threaded loop and its attention splits by head, so the thread count
    changes no result there; the forwards run on one thread."""
    t0 = time.time()
    m = P.SynthModel(cfg, seed=0)
    rows, ids = P.prompt_rows(m, n_audio, n_ids)
    r = P.RefModel(m, threads=prefill_threads)
    r.prefill(rows[:-1])
    r.lib.ref_set_threads(1)
    x = rows[-1]
    toks, logits = [], []
    for i in range(n_forwards):
        t, lg, _ = r.forward(x, True)
        toks.append(t); logits.append(lg.astype(np.float32))
        x = r.embed(t)
    np.savez_compressed(os.path.join(HERE, f"{name}_logits.npz"), ids=ids, tokens=np.array(toks, np.int32),
                        logits=np.array(logits), emb_checksum=np.uint64(P.checksum_u16(m.emb)),
                        n_audio=np.int32(n_audio), n_ids=np.int32(n_ids))
    return meta({"config": f"{name}_logits", "hidden": cfg.hidden, "prefill_rows": int(rows.shape[0] - 1),
                 "forwards": n_forwards, "prefill_threads": prefill_threads, "total_s": round(time.time() - t0, 1)})


FIXTURES = {
    "tiny_teacher": tiny_teacher,
    "c1_short": lambda: free_run("c1_short", P.CFG_06B, 40, 12, 17),
    "c1_full": lambda: free_run("c1_full", P.CFG_06B, 390, 12, 128),
    "c3_short": lambda: free_run("c3_short", P.CFG_17B, 30, 16, 9),
    "c1_full_logits": lambda: logits_run("c1_full", P.CFG_06B, 390, 12, 4),
    "c3_short_logits": lambda: logits_run("c3_short", P.CFG_17B, 30, 16, 4),
    # C4's shape at full depth: 8191 prefill rows, then forwards at positions 8191-8193
    "c4_long_logits": lambda: logits_run("c4_long", P.CFG_06B, 8192, 0, 3, prefill_threads=8),
}


def main(names):
    names = names or list(FIXTURES)
    path = os.path.join(HERE, "fixtures.json")
    info = json.load(open(path)) if os.path.exists(path) else {}
    for n in names:
        print("generating", n, flush=True)
        info[n] = FIXTURES[n]()
        print(" ", info[n], flush=True)
    with open(path, "w") as f:
        json.dump(info, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main(sys.argv[1:])
