"""Benchmark of the HIP backend on BASELINE configuration 1: Qwen2.5-1.5B-shaped integer decode.

One step = one sslm_decode_step over a batch of sequences through all 28 layers and the LM head
(greedy token out), with every weight, KV block and stream state resident in HBM.  Prints one
JSON line.  Alongside it, the same run measures:
  * the int8 prefill GEMM rate of a 512-token chunk (BASELINE configuration 2's prefill),
  * single-sequence decode,
  * the reference's own CPU path (oracle/_ref, compiled from the reference sources) on a bounded
    sample of the same workload, whose tokens must equal the GPU's.
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch B]
"""
import argparse
import ctypes
import json
import os
import platform
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from superslm_amd.sslm import Model, SslmLib  # noqa: E402
from superslm_amd.sslm_artifact import CONFIGS, build_synthetic  # noqa: E402

METRIC = "int8 prefill GEMM TOPS + decode tok/s (1.5B shape), bit-exact vs CPU, % roofline"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
CLASSES = 5


def profile(lib, on):
    L = lib.lib
    L.sslm_hip_profile_enable.argtypes = [ctypes.c_int]
    L.sslm_hip_profile_read.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int]
    if on:
        L.sslm_hip_profile_reset()
    L.sslm_hip_profile_enable(1 if on else 0)


def profile_read(lib):
    ms = (ctypes.c_double * CLASSES)()
    la = (ctypes.c_int64 * CLASSES)()
    by = (ctypes.c_int64 * CLASSES)()
    op = (ctypes.c_int64 * CLASSES)()
    lib.lib.sslm_hip_profile_read(ms, la, by, op, CLASSES)
    return list(ms), list(la), list(by), list(op)


def cpu_model():
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=32)
    ap.add_argument("--cpu-seqs", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(sequences shard across GPUs with no exchange; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    cfg = CONFIGS["qwen1.5b"]
    t0 = time.time()
    sm = build_synthetic(cfg, seed=1515)
    image = sm.to_array()
    gen_s = time.time() - t0
    print(f"[bench] synthetic 1.5B artifact {image.nbytes / 1e9:.2f} GB in {gen_s:.1f}s", file=sys.stderr, flush=True)

    hip = SslmLib(os.path.join(ROOT, "superslm_amd", "libsslm_hip.so"))
    model = Model(hip, image)
    B = args.batch
    pool = model.pool(B + 1)
    rng = np.random.default_rng(99)
    prompts = [rng.integers(0, cfg.vocab, size=args.prompt) for _ in range(B)]
    seqs = [pool.seq() for _ in range(B)]
    for s, p in zip(seqs, prompts):
        s.prefill(p)
    print("[bench] prefilled", B, "sequences", file=sys.stderr, flush=True)

    # decode: warmup (the first step only computes logits for the prefilled rows)
    first_tokens = model.decode_step(seqs, cfg.layers)
    second_tokens = model.decode_step(seqs, cfg.layers)
    for _ in range(max(0, args.warmup - 2)):
        model.decode_step(seqs, cfg.layers)
    hip.lib.sslm_hip_synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.decode_step(seqs, cfg.layers)
    hip.lib.sslm_hip_synchronize()
    dt = time.perf_counter() - t0
    tok_s = B * args.steps / dt
    ms_step = dt * 1000.0 / args.steps
    print(f"[bench] decode B={B}: {ms_step:.3f} ms/step, {tok_s:.1f} tok/s", file=sys.stderr, flush=True)

    # profiled pass (events around every launch) for the roofline figures
    profile(hip, True)
    for _ in range(args.steps):
        model.decode_step(seqs, cfg.layers)
    ms, la, by, op = profile_read(hip)
    profile(hip, False)
    gemv_gbs = by[0] / (ms[0] * 1e-3) / 1e9 if ms[0] else 0.0
    head_gbs = by[1] / (ms[1] * 1e-3) / 1e9 if ms[1] else 0.0
    dec_bytes = by[0] + by[1]
    dec_ms = ms[0] + ms[1]
    all_gbs = dec_bytes / (dec_ms * 1e-3) / 1e9 if dec_ms else 0.0
    step_prof = {"gemv_ms": ms[0] / args.steps, "head_ms": ms[1] / args.steps, "attention_ms": ms[2] / args.steps,
                 "row_ms": ms[3] / args.steps, "launches_per_step": sum(la) / args.steps}

    # single-sequence decode (M = 1)
    one = seqs[:1]
    for _ in range(2):
        model.decode_step(one, cfg.layers)
    t0 = time.perf_counter()
    n1 = max(4, args.steps // 2)
    for _ in range(n1):
        model.decode_step(one, cfg.layers)
    m1_tok_s = n1 / (time.perf_counter() - t0)

    # prefill: one 512-token chunk (BASELINE configuration 2's chunk), GEMM rate from the profile
    pseq = pool.seq()
    chunk = rng.integers(0, cfg.vocab, size=512)
    pseq.prefill(chunk[:8])  # warm
    pseq.release()
    pseq = pool.seq()
    profile(hip, True)
    t0 = time.perf_counter()
    pseq.prefill(chunk)
    pre_s = time.perf_counter() - t0
    pms, pla, pby, pop = profile_read(hip)
    profile(hip, False)
    prefill_tops = pop[0] / (pms[0] * 1e-3) / 1e12 if pms[0] else 0.0
    prefill_tok_s = 512 / pre_s
    print(f"[bench] prefill 512: {pre_s * 1e3:.1f} ms, GEMM {prefill_tops:.1f} TOPS", file=sys.stderr, flush=True)

    # CPU baseline: the reference compiled from its sources, same artifact, bounded sample
    cpu = None
    bit_exact = None
    ref_so = os.path.join(ROOT, "oracle", "_ref", "libsuperslm_ref.so")
    if not args.no_cpu and os.path.exists(ref_so):
        ref = SslmLib(ref_so)
        t0 = time.time()
        rmodel = Model(ref, image)
        rpool = rmodel.pool(args.cpu_seqs)
        rseqs = [rpool.seq() for _ in range(args.cpu_seqs)]
        for s, p in zip(rseqs, prompts):
            s.prefill(p)
        r_first = rmodel.decode_step(rseqs, cfg.layers)  # logits of the prefilled rows
        t1 = time.perf_counter()
        r_second = rmodel.decode_step(rseqs, cfg.layers)  # one full decode step per sequence
        cpu_dt = time.perf_counter() - t1
        bit_exact = (r_first == first_tokens[:args.cpu_seqs]) and (r_second == second_tokens[:args.cpu_seqs])
        cpu = {"value": round(args.cpu_seqs / cpu_dt, 3), "unit": "tok/s", "cores": 1, "kind": "reference",
               "sample": f"{args.cpu_seqs} sequences x 1 decode step (28 layers + LM head) after a "
                         f"{args.prompt}-token prefill, same artifact; host {cpu_model()}, nproc {os.cpu_count()}"}
        print(f"[bench] CPU reference: {cpu['value']} tok/s, tokens equal: {bit_exact} "
              f"({time.time() - t0:.1f}s)", file=sys.stderr, flush=True)

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"config1: Qwen2.5-1.5B-shape integer decode, {B} sequences, 28 layers + "
                               f"LM head per step, seeded random int8 weights", "batch": B,
                   "prompt_tokens": args.prompt, "hidden": cfg.hidden, "layers": cfg.layers,
                   "intermediate": cfg.inter, "vocab": cfg.vocab},
        "roofline": {"bound": "hbm", "achieved": round(all_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(all_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "decode GEMV (projection GEMVs + LM head), algorithmic bytes / kernel time"},
        "cpu_baseline": cpu,
        "bit_exact_vs_cpu": bit_exact,
        "decode_m1_tok_s": round(m1_tok_s, 2),
        "decode_gemv_gbs": round(gemv_gbs, 1),
        "lm_head_gbs": round(head_gbs, 1),
        "step_profile_ms": {k: round(v, 4) for k, v in step_prof.items()},
        "prefill_512_tok_s": round(prefill_tok_s, 1),
        "prefill_gemm_tops": round(prefill_tops, 2),
        "prefill_gemm_mfma_frac": round(prefill_tops / INT8_PEAK_TOPS, 4),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
