#!/usr/bin/env python3
"""Benchmark of the Qwen3 decoder token loop on one MI355X.

Metric: decode tok/s at batch 1 + achieved fraction of the
HBM roofline; prefill tok/s reported alongside.  Workload (default, configs[0]
= C1): Qwen3-ASR-0.6B decoder, random-init bf16 weights N(0, 0.02) with
all-ones norms (seed 0), 390 synthetic audio rows N(0,1) + 12 random prompt
ids; prefill 401 rows, forward the last row, then greedy decode.  A "step" is
one greedy decode forward (one token); K timed steps start at the C1
positions (402 ..), fed back on the device (qwen_hip_decoder_generate).

Roofline: the decode step is the unit launched per token; its algorithmic
bytes (bf16 weights + LM head + fp32 norms + fp32 K/V read + K/V write, from
qwen_hip_decoder_step_bytes) divided by the step's GPU time, measured with
HIP events on the decoder's own stream around the timed steps.

CPU baseline: the reference decoder compiled from its sources (oracle/_ref,
-O3 -ffast-math, no BLAS) on a bounded sample of the same workload, timed on
this host's cores.
"""
import argparse
import csv
import glob
import importlib
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

WORKLOADS = {
    "c1": dict(model_b=0, n_audio=390, n_ids=12,
               desc="C1 Qwen3-ASR-0.6B decoder token loop: 390 audio rows + 12 ids, prefill 401, greedy decode"),
    "c2": dict(model_b=0, n_audio=0, n_ids=0,
               desc="C2 bf16-weight GEMV sweep with fp32 x (op-level qwen_hip_linear_nobias_bf16, seq 1), "
                    "cold weights (rotation over >= 1 GiB of copies)"),
    "c3": dict(model_b=1, n_audio=1500, n_ids=16, steps=256,
               desc="C3 Qwen3-ASR-1.7B decoder: 1500 audio rows + 16 ids, prefill 1515, greedy decode"),
    "c4": dict(model_b=0, n_audio=8192, n_ids=0, steps=512,
               desc="C4 0.6B long context: prefill 8191 audio rows, greedy decode over up to 8.7k positions"),
    "enc": dict(model_b=0, n_audio=0, n_ids=0, steps=20,
                desc="Qwen3-ASR-0.6B audio encoder: 30 s of synthetic mel (3000 frames, 30 chunks -> 390 "
                     "tokens), conv stem + 18 layers + projection, fp32"),
    "c5": dict(model_b=0, n_audio=26, n_ids=9,
               desc="C5 0.6B streaming: 60 chunks x (roll back 5 tokens, prefill 5 token + 26 audio rows, "
                    "24 greedy forwards), KV window capped at 1024 positions"),
}
C5_CHUNKS, C5_AUDIO, C5_ROLLBACK, C5_STEPS, C5_CAP, C5_HEAD, C5_KEEP = 60, 26, 5, 24, 1024, 9, 3
HBM_PEAK_GBS = 8000.0
# CPU baseline: prefills longer than the first figure are sampled to the
# second (the reference's non-BLAS prefill runs ~60 rows/s on 0.6B and ~8.5
# rows/s on 1.7B with 16 threads, so a sample stays within ~30 s)
CPU_PREFILL_BOUND = {False: (1536, 1024), True: (256, 256)}   # keyed by "1.7B model"
PREFILL_REPS = 5


def log(*a):
    print(*a, file=sys.stderr, flush=True)


GRAPH_KERNELS = ("gemv_kernel", "attn_decode_fused", "attn_merge", "argmax_finish")
PMC_STEPS = 16


def pmc_pass(counter, workload, timeout=150, extra=None):
    """One child run of this script under rocprofv3 --pmc <counter>: a short
    decode of PMC_STEPS steps (plus a 256 MiB calibration copy kernel).
    Returns (KiB per decode step, calibration factor), or None.  Persistent
    engine: the counter of the last persistent-kernel dispatch (rl_decode or
    px_decode: the timed launch of PMC_STEPS steps) / PMC_STEPS.  Graph engine:
    the step's kernels summed, per argmax_finish."""
    exe = shutil.which("rocprofv3")
    if not exe:
        return None
    out = tempfile.mkdtemp(prefix="qk_pmc_")
    cmd = [exe, "--pmc", counter, "-d", out, "-o", "run", "--output-format", "csv", "--",
           sys.executable, os.path.abspath(__file__), "--no-cpu", "--no-traffic", "--no-extra", "--no-stages",
           "--steps", str(PMC_STEPS),
           "--warmup", "2", "--calib-copy-mb", "256", "--workload", workload] + list(extra or [])
    env = dict(os.environ, TMPDIR="/tmp")
    errlog = os.path.join(out, "child.err")
    try:
        with open(errlog, "w") as ef:
            # own process group, so a time-out ends the profiler and the program under it
            p = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL, stderr=ef,
                                 start_new_session=True)
            try:
                rc = p.wait(timeout=timeout)
            except subprocess.TimeoutExpired:
                os.killpg(p.pid, 9)
                p.wait()
                rc = "timeout"
        files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
        if rc != 0 or not files:
            tail = open(errlog, errors="replace").read().splitlines()[-6:]
            log(f"[gpu] rocprofv3 --pmc {counter} pass: exit {rc}, {len(files)} counter files; stderr tail:")
            for line in tail:
                log("    " + line)
        if not files:
            return None
        per_dispatch, names, cal = {}, {}, None
        for r in csv.DictReader(open(files[0])):
            name, v = r["Kernel_Name"], float(r["Counter_Value"])
            did = int(r.get("Dispatch_Id", len(per_dispatch)))
            if "AUnaryFunctor" in name:
                cal = v if cal is None else cal + v
                continue
            per_dispatch[did] = per_dispatch.get(did, 0.0) + v
            names[did] = name
        if not cal:
            return None
        factor = 256 * 1024 / cal
        px = sorted(d for d, n in names.items() if "px_decode" in n or "rl_decode" in n)
        if px:
            return per_dispatch[px[-1]] / PMC_STEPS * factor, factor
        total = sum(v for d, v in per_dispatch.items() if any(k in names[d] for k in GRAPH_KERNELS))
        steps = sum(1 for n in names.values() if "argmax_finish" in n)
        if not steps:
            return None
        return total / steps * factor, factor
    except (subprocess.SubprocessError, OSError, KeyError, ValueError):
        return None
    finally:
        shutil.rmtree(out, ignore_errors=True)


def kernel_trace_pass(args_list, timeout=300):
    """One child run of this script under rocprofv3 --kernel-trace; returns the
    (kernel name, duration in us) of every dispatch in dispatch order, or None."""
    exe = shutil.which("rocprofv3")
    if not exe:
        return None
    out = tempfile.mkdtemp(prefix="qk_kt_")
    cmd = [exe, "--kernel-trace", "-d", out, "-o", "run", "--output-format", "csv", "--",
           sys.executable, os.path.abspath(__file__)] + list(args_list)
    try:
        with open(os.path.join(out, "child.err"), "w") as ef:
            p = subprocess.Popen(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), stdout=subprocess.DEVNULL,
                                 stderr=ef, start_new_session=True)
            try:
                rc = p.wait(timeout=timeout)
            except subprocess.TimeoutExpired:
                os.killpg(p.pid, 9)
                p.wait()
                rc = "timeout"
        files = glob.glob(os.path.join(out, "**", "*kernel_trace.csv"), recursive=True)
        if rc != 0 or not files:
            log(f"[gpu] rocprofv3 --kernel-trace pass: exit {rc}, {len(files)} trace files")
            return None
        rows = [(int(r["Dispatch_Id"]), r["Kernel_Name"],
                 (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3) for r in csv.DictReader(open(files[0]))]
        return [(n, d) for _, n, d in sorted(rows)]
    except (subprocess.SubprocessError, OSError, KeyError, ValueError):
        return None
    finally:
        shutil.rmtree(out, ignore_errors=True)


C2_TRACE_REPS = 40
C2_SHAPES = [(2048, 1024), (1024, 2048), (6144, 1024), (1024, 3072), (151936, 1024), (4096, 2048),
             (2048, 4096), (12288, 2048), (2048, 6144), (151936, 2048), (2048, 2048)]


def c2_copies(wbytes):
    return max(4, -(-(1 << 30) // wbytes))


def run_gemv_sweep(qa, threads, with_cpu, trace_reps=0):
    """C2: y = W x for each (rows, cols), W bf16 N(0, 0.02), x U[-1, 1].  GPU:
    the op-level GEMV (qwen_hip_linear_nobias_bf16 at seq 1, the reference's
    qwen_linear_nobias_bf16 decode path, qwen_asr_kernels.c:462-466), timed
    with HIP events over launches that rotate through >= 4 copies of W
    spanning >= 1 GiB, so each launch streams its weights from HBM, not from
    the 256 MB last-level cache.  Bytes per launch 2RC + 4C + 4R.  CPU: the
    reference's own qwen_linear_nobias_bf16 (oracle/_ref) on `threads`
    threads, same W and x."""
    import numpy as np
    import torch
    out = []
    ref = None
    if with_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pyoracle as P
        ref = P.ref_lib() if P.ref_available() else None
        if ref is not None:
            ref.ref_set_threads(threads)
    for R, Cc in C2_SHAPES:
        W = qa.synth_bf16(R * Cc, 0, 9000 + R + Cc).reshape(R, Cc)
        x = qa.synth_uniform(Cc, 0, 9100 + Cc)
        wbytes = 2 * R * Cc
        copies = c2_copies(wbytes)
        dW0 = torch.from_numpy(W.view(np.int16)).to("cuda")
        dWs = [dW0] + [dW0.clone() for _ in range(copies - 1)]
        dx = torch.from_numpy(x).to("cuda")
        dy = torch.empty(R, dtype=torch.float32, device="cuda")
        lib = qa.lib()
        call = lambda w: lib.qwen_hip_linear_nobias_bf16(dy.data_ptr(), dx.data_ptr(), w.data_ptr(), 1, Cc, R, None)
        for i in range(copies):
            qa.check(call(dWs[i]), "gemv")
        reps = trace_reps or max(copies * 4, min(400, int(4e9 // wbytes)))
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(reps):
            call(dWs[i % copies])
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        nbytes = wbytes + 4 * Cc + 4 * R
        gbs = nbytes / (us * 1e-6) / 1e9
        row = {"rows": R, "cols": Cc, "bytes": nbytes, "us": round(us, 3), "gb_s": round(gbs, 1),
               "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": copies}
        if ref is not None:
            yc = np.empty(R, np.float32)
            Wc = np.ascontiguousarray(W)
            ref.qwen_linear_nobias_bf16(yc, x, Wc, 1, Cc, R)      # warm (thread pool, pages)
            n, t0 = 0, time.perf_counter()
            while n < 3 or time.perf_counter() - t0 < 0.5:
                ref.qwen_linear_nobias_bf16(yc, x, Wc, 1, Cc, R)
                n += 1
            cpu_s = (time.perf_counter() - t0) / n
            row["cpu_gb_s"] = round(nbytes / cpu_s / 1e9, 2)
            row["cpu_us"] = round(cpu_s * 1e6, 1)
            yg = dy.cpu().numpy()
            row["max_rel_diff_vs_ref"] = float(np.max(np.abs(yg - yc)) / (np.max(np.abs(yc)) + 1e-30))
        log(f"[gpu] gemv {R}x{Cc}: {us:.2f} us, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)"
            + (f"; cpu {row['cpu_gb_s']} GB/s" if "cpu_gb_s" in row else ""))
        out.append(row)
        del dWs, dW0
        torch.cuda.empty_cache()
    return out


def run_lm_shard(qa):
    """One GPU's share of a vocabulary-sharded LM head: the logit GEMV
    (qwen_hip_linear_nobias_bf16, seq 1) over 1/N of the 151936 rows at the
    real hidden sizes, cold weights (rotation over >= 1 GiB of copies), timed
    with HIP events.  (The argmax op synchronises the host per call; the
    persistent engine fuses the argmax into this pass.)  The exchange of the
    N (logit, index) pairs is not part of a one-GPU run."""
    import numpy as np
    import torch
    out = []
    for K in (1024, 2048):
        for n in (1, 8):
            R = -(-151936 // n)
            W = qa.synth_bf16(R * K, 0, 9200 + K + n).reshape(R, K)
            x = qa.synth_uniform(K, 0, 9300 + K)
            wbytes = 2 * R * K
            copies = max(4, -(-(1 << 30) // wbytes))
            dW0 = torch.from_numpy(W.view(np.int16)).to("cuda")
            dWs = [dW0] + [dW0.clone() for _ in range(copies - 1)]
            dx = torch.from_numpy(x).to("cuda")
            dy = torch.empty(R, dtype=torch.float32, device="cuda")
            lib = qa.lib()
            call = lambda w: lib.qwen_hip_linear_nobias_bf16(dy.data_ptr(), dx.data_ptr(), w.data_ptr(), 1, K, R, None)
            for i in range(copies):
                call(dWs[i])
            reps = max(copies * 4, 64)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(reps):
                call(dWs[i % copies])
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            gbs = (wbytes + 4 * K + 4 * R) / (us * 1e-6) / 1e9
            log(f"[gpu] LM-head logits, 1/{n} of the vocabulary ({R} x {K}): {us:.2f} us, {gbs:.0f} GB/s")
            out.append({"shards": n, "rows": R, "cols": K, "us": round(us, 3), "gb_s": round(gbs, 1)})
            del dWs, dW0
            torch.cuda.empty_cache()
    return out


def run_streaming(qa, d, cfg, chunks):
    """The C5 op pattern (the reference's streaming KV reuse, qwen_asr.c:1748-1829):
    a 9-row template head, then per chunk: roll the KV back by the last 5
    decoded tokens (set_kv_len), prefill their embeddings + the chunk's 26
    audio rows, forward the last row and generate 23 more tokens greedily.
    When the next chunk would pass 1024 positions, keep the template head and
    re-prefill the audio of the last 3 chunks.  Returns (tokens of every
    chunk, seconds per chunk)."""
    import numpy as np
    import torch
    emb = qa.synth_bf16(cfg.vocab * cfg.hidden, 0, qa.SYNTH_EMBED).reshape(cfg.vocab, cfg.hidden)
    head, _, _ = qa.prompt_rows(cfg, 0, C5_HEAD, emb=emb)
    audio = [qa.prompt_rows(cfg, C5_AUDIO, 0, audio_chunk=c, emb=emb)[0] for c in range(chunks)]
    e = lambda t: qa.bf16_to_f32(emb[np.asarray(t)]).reshape(-1, cfg.hidden)
    d.set_kv_len(0)
    d.prefill(head)
    out, times, prev = [], [], []
    for c in range(chunks):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        if prev:
            d.set_kv_len(d.kv_len() - C5_ROLLBACK)
        if d.kv_len() + C5_ROLLBACK + C5_AUDIO + C5_STEPS > C5_CAP:
            d.set_kv_len(C5_HEAD)
            d.prefill(np.concatenate(audio[max(0, c - C5_KEEP):c]))
        rows = np.concatenate([e(prev[-C5_ROLLBACK:]), audio[c]]) if prev else audio[c]
        d.prefill(rows[:-1])
        first = d.forward(rows[-1])
        toks = [first] + list(d.generate(first, C5_STEPS - 1))
        times.append(time.perf_counter() - t0)
        out.append(toks)
        prev = toks
    return out, times


ENC_FRAMES, ENC_CPU_FRAMES = 3000, 200
BF16_MFMA_PEAK_TFS = 2500.0        # dense bf16 matrix-core peak (the encoder's GEMMs and attention run there)


def prefill_rates(cfg, rows, seconds):
    """Whole-prefill arithmetic rate from the timed median: the reference's
    fp32 work (projections 2 * weights-per-layer * layers flop per row, causal
    attention 4 * hd * heads * layers * sum(pos + 1)) and the bf16 MFMA work
    the kernels execute for it (two products per projection term: hi and lo
    activation halves; three per attention term), against the dense bf16
    peak.  Includes everything in the prefill (norms, RoPE, launches)."""
    hd, H, I, L = cfg.head_dim, cfg.hidden, cfg.intermediate, cfg.layers
    per_layer_w = H * (cfg.heads * hd + 2 * cfg.kv_heads * hd) + cfg.heads * hd * H + 3 * H * I
    proj = 2.0 * per_layer_w * L * rows
    attn = 4.0 * hd * cfg.heads * L * rows * (rows + 1) / 2
    mfma = 2.0 * proj + 3.0 * attn
    return {"rows": rows, "ms": round(seconds * 1e3, 3), "fp32_equiv_tflops": round((proj + attn) / seconds / 1e12, 2),
            "mfma_tflops": round(mfma / seconds / 1e12, 2),
            "mfma_frac": round(mfma / seconds / 1e12 / BF16_MFMA_PEAK_TFS, 4),
            "arithmetic": "projections: each fp32 activation carried as bf16 hi + lo (|x - hi - lo| <= 2^-17 |x|) "
                          "against the bf16-exact weights, 2 bf16 MFMA products per term, fp32 accumulation; "
                          "attention: Q, K, V, P split the same way, hi.hi + hi.lo + lo.hi (3 products per term, "
                          "~2^-16 relative per product); softmax statistics and outputs fp32; the reference runs "
                          "fp32 SGEMM (2^-24)",
            "note": "whole prefill (projections x2 hi/lo and attention x3 bf16 MFMA work) over the median wall time"}


def enc_flops(c, frames):
    """Algorithmic flops of one encoder forward (2 per multiply-add): conv
    stem as GEMMs (conv1 K = 9), conv_out, per layer the Q/K/V/O, FFN and
    windowed attention products, ln_post projections.  Full chunks only."""
    cw = c.chunk_size
    conv = lambda w: (w + 2 - 3) // 2 + 1
    w1, w2, w3 = conv(cw), conv(conv(cw)), conv(conv(conv(cw)))
    chunks = frames // cw
    T = chunks * w3
    d, f, o = c.d_model, c.ffn_dim, c.output_dim
    fl = 2 * 480 * 9 * chunks * 64 * w1 + 2 * 480 * 4320 * chunks * (32 * w2 + 16 * w3)
    fl += 2 * T * d * 7680
    win = w3 * (c.n_window_infer // cw)
    att = sum(min(win, T - s) ** 2 for s in range(0, T, win)) * 4 * d
    fl += c.layers * (2 * T * (4 * d * d + 2 * d * f) + att)
    fl += 2 * T * d * (d + o)
    return fl, T


def run_encoder(qa, args, wl):
    """Encoder workload: one step = one forward of 30 s of mel resident in HBM
    (qwen_hip_encoder_forward_device), timed with HIP events on the encoder's
    stream; CPU baseline = the reference encoder (oracle/_ref) on 2 s of the
    same mel with the same weights."""
    import numpy as np
    import torch
    c = qa.enc_preset(wl["model_b"])
    K, W = args.steps or wl["steps"], args.warmup
    e = qa.Encoder(c, 0)
    t0 = time.time()
    e.load_synthetic(0, 0.02)
    mel_h = qa.synth_mel(ENC_FRAMES, 0, 0)
    mel = torch.from_numpy(mel_h).cuda()
    log(f"[gpu] enc: weights generated+uploaded in {time.time() - t0:.1f}s; {ENC_FRAMES} mel frames")
    for _ in range(W):
        T, _ = e.forward_device(mel.data_ptr(), ENC_FRAMES)
    s = torch.cuda.ExternalStream(e.stream())
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(s)
    for _ in range(K):
        T, _ = e.forward_device(mel.data_ptr(), ENC_FRAMES)
    ev1.record(s)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    fl, T_ = enc_flops(c, ENC_FRAMES)
    assert T == T_, (T, T_)
    audio_s = ENC_FRAMES / 100.0
    tfs = fl / (gpu_ms / K * 1e-3) / 1e12
    log(f"[gpu] enc: {K} forwards, {gpu_ms / K:.3f} ms GPU per forward ({wall / K * 1e3:.3f} ms wall), "
        f"{fl / 1e9:.1f} GFLOP -> {tfs:.1f} TFLOP/s")
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pyoracle as P
        if P.ref_available():
            threads = min(os.cpu_count() or 1, 16)
            t0 = time.time()
            m = P.SynthEncoder(c, seed=0)
            r = P.RefEncoder(m, threads=threads)
            log(f"[cpu] encoder weights generated in {time.time() - t0:.1f}s; {ENC_CPU_FRAMES} frames on "
                f"{threads} threads")
            n_tok = e.tokens(ENC_CPU_FRAMES)
            tc = r.time(mel_h[:, :ENC_CPU_FRAMES], n_tok)
            log(f"[cpu] reference encoder: {tc:.2f}s for {ENC_CPU_FRAMES / 100:.0f} s of audio")
            cpu = {"value": round(ENC_CPU_FRAMES / 100.0 / tc, 4), "unit": "audio-s/s", "cores": threads,
                   "kind": "reference",
                   "sample": f"reference encoder (oracle/_ref, no BLAS) on the first {ENC_CPU_FRAMES} frames "
                             f"({ENC_CPU_FRAMES // 100} s) of the same mel, same weights"}
    print(json.dumps({
        "metric": "encoder audio seconds per second (0.6B, 30 s input)",
        "value": round(audio_s / (gpu_ms / K * 1e-3), 2), "unit": "audio-s/s", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": round(gpu_ms / K, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": wl["desc"], "tokens": T, "weights": "synthetic N(0,0.02), seed 0"},
        "roofline": {"bound": "mfma", "achieved": round(tfs, 2), "peak": BF16_MFMA_PEAK_TFS, "unit": "TFLOP/s",
                     "frac": round(tfs / BF16_MFMA_PEAK_TFS, 4), "traffic": None,
                     "kernel": "encoder forward (all launches; enc_gemm_hl dominant)",
                     "note": "achieved counts the reference's fp32 flops; the GEMMs issue two bf16 MFMAs per "
                             "product (fp32 activation split hi + lo, bf16 weights exact), conv1 runs on fp32 MFMA",
                     "flops_per_launch": fl, "launch_us": round(gpu_ms / K * 1e3, 2)},
        "wall_ms_per_step": round(wall / K * 1e3, 4), "cpu_baseline": cpu}), flush=True)


CPU_1T_STEPS = 8
REF_BLAS = ("none: the reference's BLAS build (Makefile:47-48, cblas_sgemm in qwen_asr_kernels.c:181-202) "
            "needs cblas.h and an OpenBLAS library, which this image does not have; the reference is built "
            "from its sources without USE_BLAS, so its prefill runs the non-BLAS loop "
            "(qwen_asr_kernels.c:211-222) and its decode (seq 1, never BLAS) is unaffected")


def cpu_prefill_blas(P, r, m, pre, threads):
    """The reference's BLAS-build prefill (make blas: USE_BLAS, cblas_sgemm,
    Makefile:47-48), composed on this host because that build needs cblas.h,
    which the image lacks: qwen_decoder_prefill's operator sequence
    (qwen_asr_decoder.c:262-359) over the same rows, with the reference's own
    compiled operators (oracle/_ref: rms_norm, per-head norm, RoPE, causal
    attention, SwiGLU, residual adds) and, for each qwen_linear_nobias_bf16,
    what its BLAS path does (qwen_asr_kernels.c:196-202, :320-330): widen the
    bf16 weight to fp32 (the reference's loop, one thread) and one sgemm,
    here OpenBLAS (numpy's bundled scipy-openblas: the library family the
    reference's Linux BLAS build links) on `threads` threads.  Returns the
    seconds per part; None if a piece is missing."""
    import ctypes as C
    import numpy as np
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:
        return None
    lib, c = r.lib, m.cfg
    fp = C.POINTER(C.c_float)
    f = lambda a: a.ctypes.data_as(fp)
    for n_, at in (("qwen_rms_norm", [fp, fp, fp, C.c_int, C.c_int, C.c_float]),
                   ("qwen_rms_norm_per_head", [fp, fp, C.c_int, C.c_int, C.c_int, C.c_float]),
                   ("qwen_apply_rope_neox", [fp, fp, fp, C.c_int, C.c_int, C.c_int]),
                   ("qwen_causal_attention", [fp, fp, fp, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                              C.c_float, C.c_int]),
                   ("qwen_swiglu_multiply", [fp, fp, C.c_int, C.c_int]),
                   ("qwen_add_inplace", [fp, fp, C.c_int])):
        getattr(lib, n_).argtypes = at
        getattr(lib, n_).restype = None
    S, D, H, KV, HD, I = pre.shape[0], c.hidden, c.heads, c.kv_heads, c.head_dim, c.intermediate
    qd, kvd = H * HD, KV * HD
    x = np.ascontiguousarray(pre, np.float32).copy()
    xn, q, k, v = (np.empty((S, n), np.float32) for n in (D, qd, kvd, kvd))
    att, proj, gu, gate, ffn = (np.empty((S, n), np.float32) for n in (qd, D, 2 * I, I, D))
    inv = 1.0 / np.power(c.theta, np.arange(0, HD, 2, dtype=np.float64) / HD)
    ang = np.arange(S, dtype=np.float64)[:, None] * inv[None]
    cs = np.ascontiguousarray(np.concatenate([np.cos(ang)] * 2, 1), np.float32)
    sn = np.ascontiguousarray(np.concatenate([np.sin(ang)] * 2, 1), np.float32)
    wide = np.empty(max(2 * I * D, qd * D, D * I), np.float32)
    t = {"widen": 0.0, "sgemm": 0.0, "other": 0.0}

    def linear(y, xin, w16):
        out_dim, in_dim = w16.shape
        n = out_dim * in_dim
        t0 = time.perf_counter()
        lib.ref_bf16_widen(wide.ctypes.data, w16.ctypes.data, n)
        t1 = time.perf_counter()
        np.matmul(xin, wide[:n].reshape(out_dim, in_dim).T, out=y)
        t["widen"] += t1 - t0
        t["sgemm"] += time.perf_counter() - t1

    def op(fn, *a):
        t0 = time.perf_counter()
        fn(*a)
        t["other"] += time.perf_counter() - t0

    with threadpool_limits(threads, user_api="blas"):
        for l in range(c.layers):
            L = m.layers[l]
            gu16 = np.empty((2 * I, D), np.uint16)          # the loader's gate/up interleave (:95-107)
            gu16[0::2], gu16[1::2] = L[P.GATE], L[P.UP]
            op(lib.qwen_rms_norm, f(xn), f(x), f(L[P.INNORM]), S, D, c.eps)
            linear(q, xn, L[P.WQ])
            linear(k, xn, L[P.WK])
            linear(v, xn, L[P.WV])
            op(lib.qwen_rms_norm_per_head, f(q), f(L[P.QNORM]), S, H, HD, c.eps)
            op(lib.qwen_rms_norm_per_head, f(k), f(L[P.KNORM]), S, KV, HD, c.eps)
            op(lib.qwen_apply_rope_neox, f(q), f(cs), f(sn), S, H, HD)
            op(lib.qwen_apply_rope_neox, f(k), f(cs), f(sn), S, KV, HD)
            op(lib.qwen_causal_attention, f(att), f(q), f(k), f(v), S, S, H, KV, HD, 1.0 / np.sqrt(HD), 0)
            linear(proj, att, L[P.WO])
            op(lib.qwen_add_inplace, f(x), f(proj), S * D)
            op(lib.qwen_rms_norm, f(xn), f(x), f(L[P.POSTNORM]), S, D, c.eps)
            linear(gu, xn, gu16)
            op(lib.qwen_swiglu_multiply, f(gate), f(gu), S, I)
            linear(ffn, gate, L[P.DOWN])
            op(lib.qwen_add_inplace, f(x), f(ffn), S * D)
    return t


def cpu_baseline(wl, rows, first_token, threads, decode_steps):
    """Reference decoder (oracle/_ref) on this host: prefill of the same rows
    and `decode_steps` greedy forwards from the same first token on `threads`
    threads, then CPU_1T_STEPS forwards on one thread from the same position;
    with the host's CPU model, ISA level and STREAM-style triad bandwidth."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as P
    if not P.ref_available():
        return None
    cfg = P.CFG_17B if wl["model_b"] else P.CFG_06B
    t0 = time.time()
    m = P.SynthModel(cfg, seed=0)
    r = P.RefModel(m, threads=threads)
    # a long prefill (C4: 8191 rows of 0.6B, C3: 1515 rows of 1.7B) would take
    # the reference's non-BLAS loop minutes: the sample then prefills the
    # first rows only (CPU_PREFILL_BOUND)
    n = rows.shape[0] - 1
    max_rows, sample_rows = CPU_PREFILL_BOUND[bool(wl["model_b"])]
    sampled = n > max_rows
    pre = rows[:sample_rows] if sampled else rows[:-1]
    last = rows[sample_rows] if sampled else rows[-1]
    log(f"[cpu] weights generated in {time.time() - t0:.1f}s; prefill {pre.shape[0]} rows on {threads} threads")
    tp = r.time_prefill(pre)
    tok, _, _ = r.forward(last)
    base = r.kv_len()
    toks, td = r.generate(first_token, decode_steps)
    r.set_kv_len(base)
    r.lib.ref_set_threads(1)
    toks1, td1 = r.generate(first_token, CPU_1T_STEPS)
    r.lib.ref_set_threads(threads)
    at_gpu = None
    if sampled:
        # the same number of decode steps at the GPU's positions (n + 1 ..): the
        # cache is extended with zero rows, so the attention walks the GPU's
        # context length (its cost depends on the length only); tokens not compared
        r.extend_kv(n + 1, last)
        _, tdg = r.generate(first_token, decode_steps)
        at_gpu = decode_steps / tdg
        log(f"[cpu] {decode_steps} decode steps at positions {n + 1}+: {tdg:.2f}s ({at_gpu:.2f} tok/s)")
    blas = cpu_prefill_blas(P, r, m, pre, threads)
    host = P.host_info()
    bw = P.stream_gbs(threads)
    bw1 = P.stream_gbs(1)
    log(f"[cpu] prefill {tp:.1f}s, {decode_steps} decode steps {td:.2f}s (first token {tok}); 1 thread: "
        f"{CPU_1T_STEPS} steps {td1:.2f}s; triad {bw:.1f} GB/s ({threads} thr), {bw1:.1f} GB/s (1 thr); {host}")
    pb = None
    if blas:
        tb = sum(blas.values())
        log(f"[cpu] BLAS-path prefill estimate {pre.shape[0]} rows: {tb:.2f}s "
            + ", ".join(f"{k} {v:.2f}s" for k, v in blas.items()))
        pb = {"tok_s": round(pre.shape[0] / tb, 2), "rows": int(pre.shape[0]), "cores": threads,
              "kind": "composed",
              "seconds": {k: round(v, 3) for k, v in blas.items()},
              "what": "the reference's BLAS-build prefill (make blas) composed from its parts: qwen_decoder_prefill's "
                      "operator sequence (qwen_asr_decoder.c:262-359) with the reference's own compiled operators "
                      "(oracle/_ref) for norms, RoPE, attention, SwiGLU and adds, and per linear its BLAS path "
                      "(qwen_asr_kernels.c:196-202, :320-330): the reference's bf16 -> fp32 widening on one thread, "
                      "then one OpenBLAS sgemm (numpy's bundled scipy-openblas) on the same threads; the build itself "
                      "needs cblas.h, which the image lacks"}
    dec_value = at_gpu if sampled else decode_steps / td
    return {"value": round(dec_value, 3), "unit": "tok/s", "cores": threads, "kind": "reference",
            "at_sample_context": round(decode_steps / td, 3) if sampled else None,
            "prefill_tok_s": round(pre.shape[0] / tp, 2),
            "prefill_blas": pb,
            "one_thread": {"value": round(CPU_1T_STEPS / td1, 3), "unit": "tok/s", "cores": 1,
                           "steps": CPU_1T_STEPS,
                           "same_tokens": bool(list(toks1[:len(toks)]) == list(toks[:len(toks1)]))},
            "cpu_model": host["cpu_model"], "logical_cpus": host["logical_cpus"], "isa": host["isa"],
            "host_triad_gb_s": {str(threads): round(bw, 1), "1": round(bw1, 1)},
            "blas": REF_BLAS,
            "sample": (f"reference decoder (oracle/_ref, no BLAS) on the same weights/rows: prefill "
                       f"{pre.shape[0]} rows" + (f" (the first {pre.shape[0]} of the {n}: a bounded sample), "
                                                  f"{decode_steps} greedy decode steps after it (at_sample_context), "
                                                  f"then {decode_steps} more at the GPU's positions {n + 1}+ with the "
                                                  f"KV cache extended by zero rows (value; tokens not compared)"
                                                  if sampled else
                                                  f", then {decode_steps} greedy decode steps; decode tok/s over "
                                                  f"those steps")),
            "first_token_matches_gpu": None if sampled else bool(tok == first_token)}


KERNEL_NAMES = {1: "px_decode (split persistent kernel: every CU streams its share of every layer)",
                2: "rl_decode (relay persistent kernel: two teams of 16 CUs per XCD take the layers in turn, "
                   "one computing from register-held weights while the other streams the next layer)"}


def launch_fields(engine, K, step_bytes, gpu_ms, kernel=0):
    """What one launch of the dominant kernel is: the persistent engine runs the
    K timed steps in one rl_decode / px_decode dispatch; the graph engine
    replays one graph (per-layer GEMV/attention kernels + LM head argmax) per
    step."""
    if engine == 2:
        return {"kernel": f"{KERNEL_NAMES.get(kernel, 'persistent kernel')}, one block per CU: {K} greedy decode "
                          f"steps per launch",
                "steps_per_launch": K, "bytes_per_launch": round(sum(step_bytes)),
                "launch_us": round(gpu_ms * 1e3, 3), "step_us": round(gpu_ms * 1e3 / K, 3)}
    return {"kernel": "decode step graph (one token: all layers + LM head argmax)", "steps_per_launch": 1,
            "bytes_per_launch": round(sum(step_bytes) / K), "launch_us": round(gpu_ms * 1e3 / K, 3),
            "step_us": round(gpu_ms * 1e3 / K, 3)}


C3_LINE_STEPS = 64


def run_c3_decode(qa, K=C3_LINE_STEPS, W=8):
    """The 1.7B decode carried in the default (C1) line: the C3 shape (1500 audio
    rows + 16 ids, prefill 1515 rows, forward the last row), then K timed
    greedy steps from position 1516 in one persistent launch; HIP events on
    the decoder's stream.  No CPU leg and no counter passes (those are in
    --workload c3)."""
    import numpy as np
    import torch
    wl = WORKLOADS["c3"]
    cfg = qa.preset(wl["model_b"])
    n_rows = wl["n_audio"] + wl["n_ids"]
    d = qa.Decoder(cfg, 0, n_rows + K + W + 64)
    d.set_fallback(False)
    t0 = time.time()
    d.load_synthetic(0, 0.02, 0.0)
    rows, _, _ = qa.prompt_rows(cfg, wl["n_audio"], wl["n_ids"])
    d.prefill(rows[:-1])
    first = d.forward(rows[-1])
    base = d.kv_len()
    d.generate(first, W)
    d.set_kv_len(base)
    stream = torch.cuda.ExternalStream(d.stream())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    tw0 = time.perf_counter()
    toks = d.generate(first, K)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - tw0
    gpu_ms = e0.elapsed_time(e1)
    step_bytes = [d.step_bytes(base + i) for i in range(K)]
    achieved = float(np.mean(step_bytes)) / (gpu_ms * 1e-3 / K) / 1e9
    kernel = d.last_kernel() if d.engine() == 2 else 0
    d.close()
    log(f"[gpu] c3 decode in the line: {K} steps {K / wall:.1f} tok/s ({gpu_ms * 1e3 / K:.1f} us/step, "
        f"{achieved / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s); setup {time.time() - t0:.1f}s")
    return {"workload": "C3 Qwen3-ASR-1.7B decoder: prefill 1515 rows (1500 audio + 16 ids), forward, then greedy decode",
            "steps": K, "decode_positions": [base, base + K - 1], "value": round(K / wall, 3), "unit": "tok/s",
            "step_us": round(gpu_ms * 1e3 / K, 3),
            "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4),
                         **launch_fields(2 if kernel else 0, K, step_bytes, gpu_ms, kernel)},
            "tokens_head": [int(first)] + [int(t) for t in toks[:7]]}


C4_LINE_STEPS = 64


def run_c4_decode(qa, K=C4_LINE_STEPS, W=8, reps=3):
    """The 0.6B long-context decode carried in the default (C1) line: the C4
    shape (prefill 8191 audio rows, forward the last row), then K timed greedy
    steps from position 8192 in one persistent launch (the split kernel: the
    relay kernel covers launches below position 1024); HIP events on the
    decoder's stream.  The prefill time is the median of `reps` timed passes
    after an untimed one.  No CPU leg and no counter passes (those are in
    --workload c4)."""
    import numpy as np
    import torch
    wl = WORKLOADS["c4"]
    cfg = qa.preset(wl["model_b"])
    n_rows = wl["n_audio"] + wl["n_ids"]
    d = qa.Decoder(cfg, 0, n_rows + K + W + 64)
    d.set_fallback(False)
    t0 = time.time()
    d.load_synthetic(0, 0.02, 0.0)
    rows, _, _ = qa.prompt_rows(cfg, wl["n_audio"], wl["n_ids"])
    d.prefill(rows[:-1])
    times = []
    for _ in range(reps):
        d.set_kv_len(0)
        torch.cuda.synchronize()
        tp0 = time.perf_counter()
        d.prefill(rows[:-1])
        torch.cuda.synchronize()
        times.append(time.perf_counter() - tp0)
    prefill_s = sorted(times)[len(times) // 2]
    first = d.forward(rows[-1])
    base = d.kv_len()
    d.generate(first, W)
    d.set_kv_len(base)
    stream = torch.cuda.ExternalStream(d.stream())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    tw0 = time.perf_counter()
    toks = d.generate(first, K)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - tw0
    gpu_ms = e0.elapsed_time(e1)
    step_bytes = [d.step_bytes(base + i) for i in range(K)]
    achieved = float(np.mean(step_bytes)) / (gpu_ms * 1e-3 / K) / 1e9
    kernel = d.last_kernel() if d.engine() == 2 else 0
    d.close()
    log(f"[gpu] c4 in the line: prefill {n_rows - 1} rows {prefill_s * 1e3:.2f} ms; decode {K} steps "
        f"{K / wall:.1f} tok/s ({gpu_ms * 1e3 / K:.1f} us/step, {achieved / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s); "
        f"setup {time.time() - t0:.1f}s")
    return {"workload": "C4 Qwen3-ASR-0.6B long context: prefill 8191 audio rows, forward, then greedy decode",
            "steps": K, "decode_positions": [base, base + K - 1], "value": round(K / wall, 3), "unit": "tok/s",
            "step_us": round(gpu_ms * 1e3 / K, 3),
            "prefill_ms": round(prefill_s * 1e3, 3), "prefill_tok_s": round((n_rows - 1) / prefill_s, 2),
            "prefill": prefill_rates(cfg, n_rows - 1, prefill_s),
            "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4),
                         **launch_fields(2 if kernel else 0, K, step_bytes, gpu_ms, kernel)},
            "tokens_head": [int(first)] + [int(t) for t in toks[:7]]}


def run_c5_line(qa):
    """The C5 streaming pattern carried in the default (C1) line: 2 warm-up
    chunks, then C5_CHUNKS timed chunks (run_streaming; each chunk's wall time
    includes its rollback, prefill, forward and greedy loop)."""
    cfg = qa.preset(WORKLOADS["c5"]["model_b"])
    d = qa.Decoder(cfg, 0, C5_CAP + 64)
    d.set_fallback(False)
    d.load_synthetic(0, 0.02, 0.0)
    run_streaming(qa, d, cfg, 2)
    toks, times = run_streaming(qa, d, cfg, C5_CHUNKS)
    d.close()
    total = sum(times)
    log(f"[gpu] c5 in the line: {C5_CHUNKS} chunks, {total / C5_CHUNKS * 1e3:.3f} ms per chunk "
        f"(max {max(times) * 1e3:.3f})")
    return {"workload": WORKLOADS["c5"]["desc"], "chunks": C5_CHUNKS,
            "value": round(C5_CHUNKS * C5_STEPS / total, 3), "unit": "generated tok/s",
            "chunk_ms": {"mean": round(total / C5_CHUNKS * 1e3, 4), "max": round(max(times) * 1e3, 4)},
            "tokens_head": [int(t) for t in toks[0][:8]]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed decode steps (default: the workload's count, C1 128, C3 256, C4 512)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="c1")
    ap.add_argument("--engine", type=int, default=None,
                    help="0 graph of fused kernels, 1 eager, 2 persistent kernel (default where supported)")
    ap.add_argument("--kernel", choices=("auto", "split", "relay"), default="auto",
                    help="persistent kernel: relay where available and the positions fit (default), or force one")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", "--no-c3", dest="no_extra", action="store_true",
                    help="default (C1) line: skip the C3 (1.7B decode), C4 (long context) and C5 (streaming) blocks")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 --pmc child runs")
    ap.add_argument("--c2-trace-reps", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--no-stages", action="store_true",
                    help="skip the relay kernel's stage-trace launch (the counter passes read the last launch)")
    ap.add_argument("--cpu-steps", type=int, default=48)
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="before timing, run one copy kernel (torch.mul by 1) over this many MiB: a "
                         "known-size kernel that calibrates rocprofv3 read/write byte counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (independent utterances would run "
              "one decoder context per GPU with no exchange). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    qa = importlib.import_module("qwen-asr_amd")
    wl = WORKLOADS[args.workload]
    cfg = qa.preset(wl["model_b"])
    if args.workload == "c2":
        threads = min(os.cpu_count() or 1, 16)
        if args.c2_trace_reps:          # the kernel-trace child: timed launches only
            run_gemv_sweep(qa, threads, False, args.c2_trace_reps)
            return
        rows = run_gemv_sweep(qa, threads, not args.no_cpu)
        kt = None if args.no_traffic else kernel_trace_pass(
            ["--workload", "c2", "--no-cpu", "--no-traffic", "--c2-trace-reps", str(C2_TRACE_REPS)])
        if kt:
            # each shape: its warm-up launch per weight copy, then the timed launches
            gv = [d for n, d in kt if n.startswith(("void gemv_kernel", "void gemv_ks"))]
            i = 0
            for r in rows:
                i += c2_copies(2 * r["rows"] * r["cols"])
                durs = sorted(gv[i:i + C2_TRACE_REPS])
                i += C2_TRACE_REPS
                if len(durs) == C2_TRACE_REPS:
                    kus = durs[len(durs) // 2]
                    r["kernel_us"] = round(kus, 3)
                    r["kernel_gb_s"] = round(r["bytes"] / (kus * 1e-6) / 1e9, 1)
                    r["kernel_frac"] = round(r["kernel_gb_s"] / HBM_PEAK_GBS, 4)
                    log(f"[gpu] gemv {r['rows']}x{r['cols']}: kernel {kus:.2f} us ({r['kernel_gb_s']:.0f} GB/s, "
                        f"{r['kernel_frac'] * 100:.1f}% of 8 TB/s)")
        tot_b = sum(r["bytes"] for r in rows)
        tot_us = sum(r["us"] for r in rows)
        big = max(rows, key=lambda r: r["bytes"])
        cpu = None
        if "cpu_gb_s" in rows[0]:
            cpu_us = sum(r["cpu_us"] for r in rows)
            cpu = {"value": round(tot_b / (cpu_us * 1e-6) / 1e9, 2), "unit": "GB/s", "cores": threads,
                   "kind": "reference",
                   "sample": "the reference's qwen_linear_nobias_bf16 (oracle/_ref, seq 1 threaded matvec) on "
                             "each shape, >= 0.5 s per shape; value = all shapes' bytes / summed time"}
        shard = run_lm_shard(qa)
        print(json.dumps({
            "metric": "bf16 GEMV GB/s (C2 sweep)", "value": round(tot_b / (tot_us * 1e-6) / 1e9, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": len(rows), "warmup": 1,
            "ms_per_step": round(tot_us / len(rows) / 1e3, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
            "config": {"workload": wl["desc"]},
            "roofline": {"bound": "hbm", "achieved": big["gb_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": big["frac"], "traffic": None,
                         "kernel": f"gemv {big['rows']}x{big['cols']} (largest shape)"},
            "per_shape": rows,
            "per_shape_note": "us / gb_s / frac: HIP events over back-to-back eager launches (launch gaps "
                              "included); kernel_us / kernel_gb_s / kernel_frac: the median rocprofv3 kernel-trace "
                              f"duration of {C2_TRACE_REPS} launches per shape in a child run (cold weights, the "
                              "kernel alone)",
            "lm_head_shard_share": shard, "cpu_baseline": cpu}), flush=True)
        return
    if args.workload == "enc":
        run_encoder(qa, args, wl)
        return
    if args.workload == "c5":
        d = qa.Decoder(cfg, 0, C5_CAP + 64)
        if args.engine is not None:
            d.set_engine(args.engine)
        d.set_fallback(False)      # a failed persistent launch fails the run instead of being redone
        d.load_synthetic(0, 0.02, 0.0)
        run_streaming(qa, d, cfg, 2)                      # warm-up
        toks, times = run_streaming(qa, d, cfg, C5_CHUNKS)
        total = sum(times)
        value = C5_CHUNKS * C5_STEPS / total
        log(f"[gpu] c5: {C5_CHUNKS} chunks in {total * 1e3:.1f} ms ({total / C5_CHUNKS * 1e3:.3f} ms per chunk, "
            f"{value:.1f} generated tok/s)")
        print(json.dumps({
            "metric": "streaming chunk latency (C5) and generated tok/s", "value": round(value, 3),
            "unit": "tok/s", "n_gpus": 1, "steps": C5_CHUNKS, "warmup": 2,
            "ms_per_step": round(total / C5_CHUNKS * 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
            "config": {"workload": wl["desc"], "engine": {0: "graph", 1: "eager", 2: "persistent"}.get(d.engine())},
            "chunk_ms": {"mean": round(total / C5_CHUNKS * 1e3, 4), "max": round(max(times) * 1e3, 4)},
            "tokens_head": [int(t) for t in toks[0][:8]]}), flush=True)
        d.close()
        return
    n_rows = wl["n_audio"] + wl["n_ids"]
    K, W = args.steps or wl.get("steps", 128), args.warmup
    d = qa.Decoder(cfg, 0, n_rows + K + W + 1024)
    if args.engine is not None:
        d.set_engine(args.engine)
    if args.kernel != "auto":
        d.set_relay(args.kernel == "relay")
    d.set_fallback(False)          # a failed persistent launch fails the run instead of being redone
    t0 = time.time()
    d.load_synthetic(0, 0.02, 0.0)
    rows, ids, emb = qa.prompt_rows(cfg, wl["n_audio"], wl["n_ids"])
    log(f"[gpu] {args.workload}: weights generated+uploaded in {time.time() - t0:.1f}s; {n_rows} input rows")
    stream = torch.cuda.ExternalStream(d.stream())
    if args.calib_copy_mb:
        # source written first, then 1 GiB of other writes so the source is no
        # longer in the 256 MB last-level cache when the copy reads it
        src = torch.ones(args.calib_copy_mb << 18, dtype=torch.float32, device="cuda")
        evict = torch.full((1 << 28,), 2.0, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.mul(src, 1.0, out=dst)   # an elementwise kernel: reads and writes exactly N MiB
        torch.cuda.synchronize()
        del src, dst, evict

    # prefill: one untimed pass, then the median of PREFILL_REPS timed passes
    d.prefill(rows[:-1])
    times = []
    for _ in range(PREFILL_REPS):
        d.set_kv_len(0)
        torch.cuda.synchronize()
        tp0 = time.perf_counter()
        d.prefill(rows[:-1])
        torch.cuda.synchronize()
        times.append(time.perf_counter() - tp0)
    prefill_s = sorted(times)[len(times) // 2]
    first = d.forward(rows[-1])
    base = d.kv_len()
    log(f"[gpu] prefill {n_rows - 1} rows in {prefill_s * 1e3:.2f} ms (median of {PREFILL_REPS}); first token {first}")

    d.generate(first, W)
    d.set_kv_len(base)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    tw0 = time.perf_counter()
    toks = d.generate(first, K)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - tw0
    gpu_ms = e0.elapsed_time(e1)
    value = K / wall
    step_bytes = [d.step_bytes(base + i) for i in range(K)]
    avg_bytes = float(np.mean(step_bytes))
    achieved = avg_bytes / (gpu_ms * 1e-3 / K) / 1e9
    log(f"[gpu] decode {K} steps: wall {wall * 1e3:.2f} ms ({value:.1f} tok/s), events {gpu_ms:.2f} ms; "
        f"{avg_bytes / 1e9:.4f} GB/step -> {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")

    traffic = None
    traffic_note = None
    engine = d.engine()
    kernel = d.last_kernel() if engine == 2 else 0
    stages = None
    if kernel in (qa.KERNEL_RELAY, qa.KERNEL_SPLIT) and not args.no_stages:
        # the kernel's own stage stamps for one step (step 6 of a 10-step launch
        # from the same position; outside the timed region)
        d.set_kv_len(base)
        d.set_trace(6)
        d.generate(first, 10)
        d.set_trace(-1)
        if kernel == qa.KERNEL_RELAY:
            stages = qa.relay_stage_us(d.read_trace(), cfg.layers)
            log(f"[gpu] relay stages (us per layer): period {stages['layer period']}, "
                f"LM rows {stages['LM head rows: median block']} / {stages['LM head rows: slowest block']}")
        else:
            stages = qa.split_stage_us(d.read_trace(), cfg.layers)
            log(f"[gpu] split stages (us per layer): period {stages['layer period']}, "
                + ", ".join(f"{k} {v}" for k, v in stages.items() if k.startswith("stage")))
    if not args.no_traffic:
        extra = ["--kernel", args.kernel]
        fr = pmc_pass("FETCH_SIZE", args.workload, extra=extra)
        wr = pmc_pass("WRITE_SIZE", args.workload, extra=extra)
        if fr and wr:
            per_step = (fr[0] + wr[0]) * 1024
            per_launch = K if engine == 2 else 1
            traffic = round(per_step * per_launch)
            traffic_note = (f"per launch = {per_launch} x the per-step HBM bytes measured over {PMC_STEPS} decode "
                            f"steps at positions {n_rows}-{n_rows + PMC_STEPS + 1}: FETCH_SIZE x {fr[1]:.4f} + "
                            f"WRITE_SIZE x {wr[1]:.4f} (factors from a 256 MiB copy kernel)")
            log(f"[gpu] traffic per step {per_step / 1e6:.1f} MB ({per_step / avg_bytes:.3f} x algorithmic)")
        else:
            log("[gpu] rocprofv3 traffic passes unavailable: traffic null")

    cpu = None
    if not args.no_cpu:
        threads = min(os.cpu_count() or 1, 16)
        cpu = cpu_baseline(wl, rows, first, threads, args.cpu_steps)

    d.close()
    extra = args.workload == "c1" and not args.no_extra
    c3 = run_c3_decode(qa) if extra else None
    c4 = run_c4_decode(qa) if extra else None
    c5 = run_c5_line(qa) if extra else None

    out = {
        "metric": "decode tok/s at batch 1 (0.6B, 1.7B) + % of peak HBM GB/s; prefill tok/s",
        "value": round(value, 3), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(wall * 1e3 / K, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": wl["desc"], "batch": 1, "weights": "bf16 N(0,0.02) seed 0, norms 1.0",
                   "activations": "fp32, fp32 accumulation", "kv_cache": "fp32",
                   "prefill_rows": n_rows - 1, "decode_positions": [base, base + K - 1],
                   "engine": {0: "graph", 1: "eager", 2: "persistent"}.get(engine, engine),
                   "kernel": {0: None, 1: "split", 2: "relay"}.get(kernel)},
        "prefill_tok_s": round((n_rows - 1) / prefill_s, 2),
        "prefill": prefill_rates(cfg, n_rows - 1, prefill_s),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_note": traffic_note,
                     **launch_fields(engine, K, step_bytes, gpu_ms, kernel)},
        "cpu_baseline": cpu,
        "tokens_head": [int(first)] + [int(t) for t in toks[:7]],
    }
    if stages:
        out["roofline"]["stage_trace_us"] = stages
        out["roofline"]["stage_trace_note"] = (
            f"the kernel's wall-clock stamps (100 MHz) for one step at position {base + 6}: per-layer stages as "
            "the median over blocks, averaged over layers (qwen_asr_amd." +
            ("relay_stage_us" if kernel == qa.KERNEL_RELAY else "split_stage_us") + ")")
    if c3:
        out["c3_decode"] = c3
    if c4:
        out["c4_long_context"] = c4
    if c5:
        out["c5_streaming"] = c5
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
