"""Benchmark of the HIP backend on BASELINE configuration 1: Qwen2.5-1.5B-shaped integer decode.

One step = one sslm_decode_step over a batch of 16 sequences through all 28 layers and the LM
head (greedy token out), with every weight, KV block and stream state resident in HBM.  Prints
one JSON line whose value is the decode rate.  Alongside it, the same run measures:
  * roofline: the decode GEMVs of a step (every layer's projections with its own weights, then
    the LM head) back to back between two HIP events -- algorithmic bytes over time against
    8 TB/s; HBM traffic per launch from rocprofv3 PMC runs when profiles/decode_gemv_traffic.json
    holds them; and the whole step against its HBM floor,
  * prefill_roofline: the 112 projection GEMMs of a 512-token chunk the same way, against the
    5.0 POPS dense int8 MFMA peak, and the 512-token prefill rate (configuration 2's chunk),
  * single-sequence decode, configuration 0 (GEMM + requant), configuration 3 (LoRA r16 on q, v)
    and configuration 4 (7B shape, 32 x 2048-token prefill, then decode),
  * cpu_baseline: the reference compiled from its own sources (oracle/_ref) on this host's cores
    -- one sequence on one core and P sequences on P cores -- whose tokens must equal the GPU's.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch B] [--phase all|decode|prefill|config4]
       python bench.py --traffic-from FETCH.csv WRITE.csv   (summarise two rocprofv3 --pmc runs)
"""
import argparse
import csv
import ctypes
import json
import os
import platform
import subprocess
import sys
import time
from collections import defaultdict

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from superslm_amd.sslm import Model, SslmLib  # noqa: E402
from superslm_amd.sslm_artifact import CONFIGS, build_synthetic  # noqa: E402

METRIC = "int8 prefill GEMM TOPS + decode tok/s (1.5B shape), bit-exact vs CPU, % roofline"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
CLASSES = 5
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_gemv_traffic.json")
CALIBRATION_BYTES = 256 << 20  # device-to-device copy whose PMC counts scale FETCH/WRITE_SIZE


def profile(lib, on):
    L = lib.lib
    L.sslm_hip_profile_enable.argtypes = [ctypes.c_int]
    if on:
        L.sslm_hip_profile_reset()
    L.sslm_hip_profile_enable(1 if on else 0)


def profile_read(lib):
    ms = (ctypes.c_double * CLASSES)()
    la = (ctypes.c_int64 * CLASSES)()
    by = (ctypes.c_int64 * CLASSES)()
    op = (ctypes.c_int64 * CLASSES)()
    lib.lib.sslm_hip_profile_read.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int]
    lib.lib.sslm_hip_profile_read(ms, la, by, op, CLASSES)
    return list(ms), list(la), list(by), list(op)


def profile_shapes(lib):
    """[(cls, M, N, K, ms, launches, bytes, ops)] per GEMM launch shape."""
    L = lib.lib
    L.sslm_hip_profile_shapes.restype = ctypes.c_int
    L.sslm_hip_profile_shapes.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int]
    cap = 256
    keys = (ctypes.c_int64 * cap)()
    ms = (ctypes.c_double * cap)()
    la = (ctypes.c_int64 * cap)()
    by = (ctypes.c_int64 * cap)()
    op = (ctypes.c_int64 * cap)()
    n = min(cap, L.sslm_hip_profile_shapes(keys, ms, la, by, op, cap))
    out = []
    for i in range(n):
        k = keys[i]
        out.append((k >> 56, (k >> 40) & 0xFFFF, (k >> 20) & 0xFFFFF, k & 0xFFFFF, ms[i], la[i], by[i], op[i]))
    return out


def cpu_model():
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor()


def copy_calibration(hip):
    """A plain device-to-device copy of CALIBRATION_BYTES (rocprof sees __amd_rocclr_copyBuffer)."""
    from superslm_amd.device import Device
    dev = Device(hip)
    a = dev.zeros((CALIBRATION_BYTES,), np.int8)
    b = dev.zeros((CALIBRATION_BYTES,), np.int8)
    for _ in range(3):
        dev.copy_device(b, a)
    hip.lib.sslm_hip_synchronize()


def traffic_from(fetch_csv, write_csv):
    """HBM bytes per decode-GEMV launch from two rocprofv3 --pmc runs of
    `bench.py --phase decode --pmc-steps --calibrate` (decode steps only, so the dispatches are the
    step's own mix): FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each scaled by what the counter
    reads for the calibration copy of known size, averaged per (kernel, grid) and over every
    M <= 16 GEMV dispatch (k_gemv_pk<1, ...>, k_gemv_sk<1, ...> and the LM head's k_gemv_head<1, ...>;
    the prompts' prefill runs M = 32 instances, k_gemv_pk<2, ...> and k_gemv_sk<2, ...>)."""
    def per_dispatch(path, counter):
        vals, meta = defaultdict(float), {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] != counter:
                continue
            d = r["Dispatch_Id"]
            vals[d] += float(r["Counter_Value"])
            meta[d] = (r["Kernel_Name"], int(r["Grid_Size"]) // int(r["Workgroup_Size"]))
        groups = defaultdict(list)
        for d, v in vals.items():
            groups[meta[d]].append(v)
        return groups
    fetch = per_dispatch(fetch_csv, "FETCH_SIZE")
    write = per_dispatch(write_csv, "WRITE_SIZE")
    copy_key = next(k for k in fetch if "copyBuffer" in k[0])
    f_scale = CALIBRATION_BYTES / (max(fetch[copy_key]) * 1024.0)
    w_scale = CALIBRATION_BYTES / (max(write[copy_key]) * 1024.0)
    kernels = []
    for (name, blocks), fv in sorted(fetch.items(), key=lambda kv: kv[0][1]):
        if "k_gemv_pk<1," not in name and "k_gemv_sk<1," not in name and "k_gemv_head<1," not in name:
            continue
        f = np.mean(fv) * 1024.0 * f_scale
        w = np.mean(write.get((name, blocks), [0.0])) * 1024.0 * w_scale
        kernels.append({"kernel": name, "blocks": blocks, "dispatches": len(fv), "fetch_bytes": round(f),
                        "write_bytes": round(w)})
    total_d = sum(k["dispatches"] for k in kernels)
    total_b = sum((k["fetch_bytes"] + k["write_bytes"]) * k["dispatches"] for k in kernels)
    out = {"calibration": {"copy_bytes": CALIBRATION_BYTES, "fetch_scale": f_scale, "write_scale": w_scale},
           "kernels": kernels, "mean_traffic_bytes_per_launch": round(total_b / max(1, total_d)),
           "dispatches": total_d,
           "command": "rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) --output-format csv -- "
                      "python3 bench.py --phase decode --pmc-steps --steps 3 --warmup 2 --no-cpu --calibrate"}
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    json.dump(out, open(TRAFFIC_FILE, "w"), indent=1)
    print(json.dumps(out, indent=1))


def extras(hip, model, pool, cfg, sm, rng, args, line):
    """BASELINE configurations 0 and 3 beside the headline: the standalone GEMM + requant
    (sslm_hip_gemm_requant, M 32 x K 896 x N 4864) and the 16-sequence decode with a rank-16
    LoRA adapter on q and v."""
    from superslm_amd.device import Device
    from superslm_amd.sslm_artifact import build_adapter
    out = {}
    # configuration 0
    L = hip.lib
    L.sslm_hip_gemm_requant.restype = ctypes.c_int
    L.sslm_hip_gemm_requant.argtypes = ([ctypes.c_void_p] * 3 + [ctypes.c_int32] * 3 + [ctypes.c_int64] * 4 +
                                        [ctypes.c_void_p] * 3)
    M0, K0, N0 = 32, 896, 4864
    g = np.random.default_rng(20260101)
    a = g.integers(-127, 128, size=(M0, K0), dtype=np.int8)
    w = g.integers(-127, 128, size=(N0, K0), dtype=np.int8)
    fold = np.zeros((N0, 3), dtype=np.int32)
    fold[:, 1] = g.integers(1 << 30, 1 << 31, size=N0, dtype=np.int64).astype(np.int32)
    fold[:, 2] = g.integers(8, 21, size=N0, dtype=np.int32)
    dev = Device(hip)
    da, dw, df = dev.upload(a), dev.upload(w), dev.upload(fold)
    codes, me, st = dev.zeros((M0, N0), np.int8), dev.zeros((M0, 2), np.int64), dev.zeros((M0,), np.int32)
    args0 = (da.ptr, dw.ptr, df.ptr, M0, N0, K0, 1 << 30, -37, 1518500250, -45, codes.ptr, me.ptr, st.ptr)
    for _ in range(3):
        assert L.sslm_hip_gemm_requant(*args0) == 0
    n0 = 50
    profile(hip, True)
    t0 = time.perf_counter()
    for _ in range(n0):
        L.sslm_hip_gemm_requant(*args0)
    wall = (time.perf_counter() - t0) / n0
    ms, la, by, op = profile_read(hip)
    profile(hip, False)
    gemm_us, funnel_us = ms[0] * 1e3 / n0, ms[3] * 1e3 / n0
    c0_bytes = N0 * K0 + M0 * K0 + M0 * N0 + 12 * N0  # the algorithmic bytes of the fused op
    out["config0_gemm_requant"] = {
        "shape": "M 32 x K 896 x N 4864", "gemm_us": round(gemm_us, 3), "funnel_us": round(funnel_us, 3),
        "kernels_us": round(gemm_us + funnel_us, 3), "call_us_incl_sync": round(wall * 1e6, 2),
        "gbs": round(c0_bytes / ((gemm_us + funnel_us) * 1e-6) / 1e9, 1),
        "tops": round(2.0 * M0 * N0 * K0 / ((gemm_us + funnel_us) * 1e-6) / 1e12, 2)}
    print(f"[bench] config0: GEMM {gemm_us:.2f} us + funnel {funnel_us:.2f} us", file=sys.stderr, flush=True)
    # configuration 3: LoRA rank 16 on q and v, every sequence of the batch adapted
    blob = build_adapter(sm, rank=16, targets=("q_proj", "v_proj"), seed=3)
    ad = model.adapter(blob)
    B = args.batch
    seqs = [pool.seq() for _ in range(B)]
    c3_prompts = [rng.integers(0, cfg.vocab, size=args.prompt) for _ in range(B)]
    for s, p in zip(seqs, c3_prompts):
        s.set_adapter(ad)
        s.prefill(p)
    c3_tokens = []  # sequence 0's first calls, checked against the CPU reference with the same adapter
    for _ in range(3):
        c3_tokens.append(model.decode_step(seqs, cfg.layers)[0])
    hip.lib.sslm_hip_synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.decode_step(seqs, cfg.layers)
    hip.lib.sslm_hip_synchronize()
    dt = time.perf_counter() - t0
    out["config3_lora_decode_tok_s"] = round(B * args.steps / dt, 2)
    out["_config3_check"] = (blob, c3_prompts[0], c3_tokens)
    print(f"[bench] config3 (LoRA r16 q,v): {out['config3_lora_decode_tok_s']} tok/s", file=sys.stderr, flush=True)
    for s in seqs:
        s.release()
    ad.release()
    return out


def vendor_gemm_reference():
    """AMD's own int8 GEMMs (hipBLASLt best candidate, rocBLAS gemm_ex) on the chunk's four projection
    shapes with raw int32 output, each over 28 rotating weight copies (./bench_vendor_gemm, built by
    __graft_entry__.build() from bench_vendor_gemm.cpp; a child process with its own HIP state).
    A reference point for the prefill GEMM roofline; None when the program is not built."""
    exe = os.path.join(ROOT, "bench_vendor_gemm")
    if not os.path.exists(exe):
        return None
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        print(f"[bench] bench_vendor_gemm failed: {r.stderr[-500:]}", file=sys.stderr, flush=True)
        return None
    out = json.loads(r.stdout.strip().splitlines()[-1])
    out["what"] = ("hipBLASLt (best of its heuristic candidates) and rocBLAS int8 x int8 -> int32 GEMMs on the "
                   "512-token chunk's q|k|v, o, gate|up and down shapes, 28 rotating weight copies each; plain "
                   "GEMMs, no fold / funnel epilogue; pass_tops_best = one layer's 2MNK over the faster "
                   "library's per-layer sum")
    print(f"[bench] vendor int8 GEMM reference: {out['pass_tops_best']} TOPS per layer pass", file=sys.stderr, flush=True)
    return out


def gemv_class_passes(hip, model, M):
    """Per projection class: the GEMV pass (all layers' launches of one class back to back) and the
    same launches as plain streaming reads of their weights, at M tokens; fractions of 8 TB/s."""
    L_ = hip.lib
    L_.sslm_hip_bench_decode_gemv.restype = ctypes.c_int32
    L_.sslm_hip_bench_decode_gemv.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32] + \
        [ctypes.c_void_p] * 3 + [ctypes.c_int32]
    L_.sslm_hip_bench_read_floor.restype = ctypes.c_int32
    L_.sslm_hip_bench_read_floor.argtypes = L_.sslm_hip_bench_decode_gemv.argtypes
    out = {}
    res = []
    for fn in (L_.sslm_hip_bench_decode_gemv, L_.sslm_hip_bench_read_floor):
        us, by, n = (ctypes.c_double * 6)(), (ctypes.c_int64 * 6)(), (ctypes.c_int64 * 6)()
        if fn(model.handle, M, 5, us, by, n, 6) != 1:
            raise RuntimeError("GEMV class pass failed")
        res.append((us, by, n))
    (gu, gb, gn), (ru, rb, rn) = res
    for c, name in enumerate(("q|k|v", "o", "gate|up", "down", "lm_head"), start=1):
        out[name] = {"us_per_launch": round(gu[c] / gn[c], 2), "MB_per_launch": round(gb[c] / gn[c] / 1e6, 2),
                     "frac": round(gb[c] / (gu[c] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "read_us_per_launch": round(ru[c] / rn[c], 2),
                     "read_frac": round(rb[c] / (ru[c] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    out["pass"] = {"frac": round(gb[0] / (gu[0] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                   "read_frac": round(rb[0] / (ru[0] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                   "us": round(gu[0], 1), "read_us": round(ru[0], 1)}
    return out


def config4(hip, args):
    """BASELINE configuration 4 at one GPU's share: the 7B shape (H 3584, I 18944, 28 layers,
    28 / 4 heads, context cap 4608), 32 sequences each prefilled with a 2048-token prompt in one
    2048-token chunk, then 256 greedy decode steps over all 32 (contexts 2051 .. 2306; the
    first three are untimed warm steps, the next 253 timed).  No CPU leg (the
    reference needs minutes per token at this shape); its parity is pinned by
    tests/test_gpu_workloads.py."""
    cfg = CONFIGS["qwen7b"]
    t0 = time.time()
    sm = build_synthetic(cfg, seed=7007)
    image = sm.to_array()
    print(f"[bench] synthetic 7B artifact {image.nbytes / 1e9:.2f} GB in {time.time() - t0:.1f}s",
          file=sys.stderr, flush=True)
    model = Model(hip, image)
    B, ctx = 32, 2048
    pool = model.pool(B + 1)
    rng = np.random.default_rng(4)
    seqs = [pool.seq() for _ in range(B)]
    prompts = [rng.integers(0, cfg.vocab, size=ctx) for _ in range(B)]
    warm = pool.seq()
    warm.prefill(prompts[0], chunk_budget=ctx)  # the 2048-token span shape, seen once
    warm.release()
    hip.lib.sslm_hip_synchronize()
    t0 = time.perf_counter()
    for s, p in zip(seqs, prompts):
        assert s.prefill(p, chunk_budget=ctx) == ctx
    hip.lib.sslm_hip_synchronize()
    pre_s = time.perf_counter() - t0
    print(f"[bench] config4 prefill {B} x {ctx}: {pre_s:.2f} s, {B * ctx / pre_s:.0f} tok/s", file=sys.stderr, flush=True)
    # attention kernel time of the first decode steps (rows of 2,049-2,050 positions) under the
    # HIP-event profiler; they are the warm steps of the timed run below
    profile(hip, True)
    for _ in range(3):
        model.decode_step(seqs, cfg.layers)
    hip.lib.sslm_hip_synchronize()
    ms0, la0, _, _ = profile_read(hip)
    profile(hip, False)
    steps = 253
    t0 = time.perf_counter()
    for _ in range(steps):
        model.decode_step(seqs, cfg.layers)
    hip.lib.sslm_hip_synchronize()
    dt = time.perf_counter() - t0
    out = {"config4_7b": {"workload": "Qwen2.5-7B shape, 32 sequences x 2048-token prompt (one chunk each), then "
                                      "256 greedy decode steps (3 warm + 253 timed, contexts 2051-2306)",
                          "prefill_tok_s": round(B * ctx / pre_s, 1), "decode_tok_s": round(B * steps / dt, 1),
                          "decode_ms_per_step": round(dt * 1e3 / steps, 3), "decode_steps": steps}}
    print(f"[bench] config4 decode: {out['config4_7b']['decode_tok_s']} tok/s", file=sys.stderr, flush=True)
    # per-class kernel time of a few more steps under the runtime's HIP-event profiler (graphs off
    # while it runs; contexts 2308-2315)
    n_prof = 8
    profile(hip, True)
    for _ in range(n_prof):
        model.decode_step(seqs, cfg.layers)
    hip.lib.sslm_hip_synchronize()
    ms, la, by, op = profile_read(hip)
    profile(hip, False)
    per_layer = lambda c: round(ms[c] * 1e3 / (n_prof * cfg.layers), 2)
    kv_bytes = B * cfg.kv_heads * 2 * cfg.head_dim * 2310  # one layer's K and V rows at ~2310 positions
    attn_us = per_layer(2)
    out["config4_7b"]["decode_us_per_layer"] = {"attention": attn_us, "gemm": per_layer(0), "rows": per_layer(3),
                                                "lm_head_per_step": round(ms[1] * 1e3 / n_prof, 2)}
    # (one attention launch per layer; the first call after a prefill only takes logits)
    out["config4_7b"]["decode_attention_us_per_layer_first_steps"] = round(ms0[2] * 1e3 / max(1, la0[2]), 2)
    out["config4_7b"]["decode_attention_kv_gbs"] = round(kv_bytes / (attn_us * 1e-6) / 1e9, 1)
    print(f"[bench] config4 decode per layer: attention {attn_us} us", file=sys.stderr, flush=True)
    out["config4_7b"]["decode_gemv_by_class"] = gemv_class_passes(hip, model, B)
    for s in seqs:
        s.release()
    pool.close()
    model.close()
    return out


TIERS = {0: "SSE2", 1: "AVX2", 2: "AVX-512"}


def cpu_baseline(image, cfg, prompts, gpu_calls, calls, lora_check=None):
    """The reference compiled from its own sources (oracle/_ref) on this host's cores, same
    artifact and prompts: (i) one sequence on one core, (ii) P sequences on P cores (one thread
    per sequence; the reference's forward is single-threaded per sequence), each prefilled with
    its prompt and then decoded for `calls` calls.  Tokens must equal the GPU's first calls."""
    from concurrent.futures import ThreadPoolExecutor
    ref_so = os.path.join(ROOT, "oracle", "_ref", "libsuperslm_ref.so")
    ref = SslmLib(ref_so)
    ref.lib.ref_dot_row_tier.restype = ctypes.c_int
    tier = TIERS.get(ref.lib.ref_dot_row_tier(), "?")
    ncpu = os.cpu_count() or 1
    P = max(1, min(16, ncpu, len(prompts)))
    rmodel = Model(ref, image)
    L = cfg.layers

    def run(k):
        pool = rmodel.pool(k)
        seqs = [pool.seq() for _ in range(k)]
        with ThreadPoolExecutor(k) as ex:
            list(ex.map(lambda sp: sp[0].prefill(sp[1]), zip(seqs, prompts[:k])))
            t0 = time.perf_counter()
            toks = list(ex.map(lambda s: [rmodel.decode_step([s], L)[0] for _ in range(calls)], seqs))
            dt = time.perf_counter() - t0
        for s in seqs:
            s.release()
        pool.close()
        return toks, dt

    t_all = time.time()
    one_toks, one_dt = run(1)
    p_toks, p_dt = run(P)
    exact = all(p_toks[i] == [c[i] for c in gpu_calls[:calls]] for i in range(P)) and one_toks[0] == p_toks[0]
    lora_exact = None
    if lora_check is not None:  # configuration 3: the same adapter blob, prompt and calls on the reference
        blob, prompt, gpu_toks = lora_check
        rad = rmodel.adapter(blob)
        pool = rmodel.pool(1)
        rs = pool.seq()
        rs.set_adapter(rad)
        rs.prefill(prompt)
        lora_exact = [rmodel.decode_step([rs], L)[0] for _ in range(len(gpu_toks))] == list(gpu_toks)
        rs.release()
        pool.close()
        rad.release()
    rmodel.close()
    out = {"value": round(P * calls / p_dt, 3), "unit": "tok/s", "cores": P, "kind": "reference",
           "sample": f"{P} sequences on {P} threads x {calls} decode calls (28 layers + LM head) after "
                     f"{len(prompts[0])}-token prompts, same artifact; host {cpu_model()}, nproc {ncpu}, "
                     f"reference matmul tier {tier}",
           "one_core_tok_s": round(calls / one_dt, 3), "matmul_tier": tier, "nproc": ncpu,
           "cpu_model": cpu_model()}
    print(f"[bench] CPU reference ({tier}): 1 core {out['one_core_tok_s']} tok/s, {P} cores {out['value']} tok/s, "
          f"tokens equal: {exact} ({time.time() - t_all:.1f}s)", file=sys.stderr, flush=True)
    if lora_exact is not None:
        out["config3_lora_tokens_equal"] = lora_exact
    return out, exact


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=32)
    ap.add_argument("--cpu-calls", type=int, default=32, help="decode calls per sequence in the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-config4", action="store_true")
    ap.add_argument("--phase", choices=["all", "decode", "prefill", "config4"], default="all")
    ap.add_argument("--calibrate", action="store_true", help="add the PMC calibration copy")
    ap.add_argument("--pmc-steps", action="store_true",
                    help="for --pmc runs: decode steps only (--phase decode), or one chunk and one pass of its "
                         "GEMMs (--phase prefill)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    args = ap.parse_args()
    if args.traffic_from:
        traffic_from(*args.traffic_from)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(decode sequences shard across GPUs with no exchange: each GPU runs its own pool)", file=sys.stderr)
        sys.exit(2)

    hip = SslmLib(os.path.join(ROOT, "superslm_amd", "libsslm_hip.so"))
    if args.phase == "config4":
        print(json.dumps(config4(hip, args)))
        return
    cfg = CONFIGS["qwen1.5b"]
    t0 = time.time()
    sm = build_synthetic(cfg, seed=1515)
    image = sm.to_array()
    print(f"[bench] synthetic 1.5B artifact {image.nbytes / 1e9:.2f} GB in {time.time() - t0:.1f}s",
          file=sys.stderr, flush=True)
    if args.calibrate:
        copy_calibration(hip)
    model = Model(hip, image)
    B = args.batch
    pool = model.pool(2 * B + 1)  # decode batch, prefill chunk, configuration-3 batch
    rng = np.random.default_rng(99)
    prompts = [rng.integers(0, cfg.vocab, size=args.prompt) for _ in range(B)]
    line = None
    gpu_calls = []
    seqs = []
    if args.phase in ("all", "decode"):
        seqs = [pool.seq() for _ in range(B)]
        for s, p in zip(seqs, prompts):
            s.prefill(p)
        print("[bench] prefilled", B, "sequences", file=sys.stderr, flush=True)
        # warmup: the first call only computes the logits of the prefilled rows
        for _ in range(max(2, args.warmup)):
            gpu_calls.append(model.decode_step(seqs, cfg.layers))
        hip.lib.sslm_hip_synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            gpu_calls.append(model.decode_step(seqs, cfg.layers))
        hip.lib.sslm_hip_synchronize()
        dt = time.perf_counter() - t0
        tok_s = B * args.steps / dt
        ms_step = dt * 1000.0 / args.steps
        print(f"[bench] decode B={B}: {ms_step:.3f} ms/step, {tok_s:.1f} tok/s", file=sys.stderr, flush=True)
        if args.pmc_steps:
            return
        # tokens of the calls the CPU baseline compares against
        while len(gpu_calls) < args.cpu_calls:
            gpu_calls.append(model.decode_step(seqs, cfg.layers))

        # profiled pass of the same steps: events around every launch, per class (where the
        # step's time goes; per-launch events add their own overhead to each figure)
        n_prof = max(4, args.steps // 2)
        profile(hip, True)
        for _ in range(n_prof):
            model.decode_step(seqs, cfg.layers)
        ms, la, by, op = profile_read(hip)
        profile(hip, False)
        step_prof = {"gemv_ms": ms[0] / n_prof, "head_ms": ms[1] / n_prof,
                     "attention_ms": ms[2] / n_prof, "row_ms": ms[3] / n_prof,
                     "launches_per_step": sum(la) / n_prof}
        # the dominant kernel: every GEMV launch of a step (28 layers' q|k|v, o, gate|up, down with
        # their own weights, then the LM head) back to back between two HIP events
        L_ = hip.lib
        L_.sslm_hip_bench_decode_gemv.restype = ctypes.c_int32
        L_.sslm_hip_bench_decode_gemv.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32] + \
            [ctypes.c_void_p] * 3 + [ctypes.c_int32]
        g_us, g_bytes, g_n = (ctypes.c_double * 6)(), (ctypes.c_int64 * 6)(), (ctypes.c_int64 * 6)()
        if L_.sslm_hip_bench_decode_gemv(model.handle, B, 10, g_us, g_bytes, g_n, 6) != 1:
            raise RuntimeError("sslm_hip_bench_decode_gemv failed")
        achieved = g_bytes[0] / (g_us[0] * 1e-6) / 1e9
        # the same passes per projection class (all layers' launches of one class back to back)
        by_class = {}
        for c, name in enumerate(("q|k|v", "o", "gate|up", "down", "lm_head"), start=1):
            gbs = g_bytes[c] / (g_us[c] * 1e-6) / 1e9
            by_class[name] = {"us_per_launch": round(g_us[c] / g_n[c], 2), "bytes_per_launch": g_bytes[c] // g_n[c],
                              "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        # reference point: the same launch sequence with every GEMV replaced by a plain streaming
        # read of its (packed) weight buffer -- the HBM rate this launch structure reaches at all
        L_.sslm_hip_bench_read_floor.restype = ctypes.c_int32
        L_.sslm_hip_bench_read_floor.argtypes = L_.sslm_hip_bench_decode_gemv.argtypes
        r_us, r_bytes, r_n = (ctypes.c_double * 6)(), (ctypes.c_int64 * 6)(), (ctypes.c_int64 * 6)()
        if L_.sslm_hip_bench_read_floor(model.handle, B, 10, r_us, r_bytes, r_n, 6) != 1:
            raise RuntimeError("sslm_hip_bench_read_floor failed")
        read_floor = {"frac": round(r_bytes[0] / (r_us[0] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                      "us_per_pass": round(r_us[0], 2), "gemv_us_per_pass": round(g_us[0], 2),
                      "by_class": {name: {"us_per_launch": round(r_us[c] / r_n[c], 2),
                                          "frac": round(r_bytes[c] / (r_us[c] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
                                   for c, name in enumerate(("q|k|v", "o", "gate|up", "down", "lm_head"), start=1)},
                      "what": "the same 113 launches, bytes and order with each GEMV replaced by a plain "
                              "streaming read of its weight buffer (k_stream_read): the HBM fraction a "
                              "launch sequence of this shape reaches at all"}
        traffic = None
        if os.path.exists(TRAFFIC_FILE):
            traffic = json.load(open(TRAFFIC_FILE)).get("mean_traffic_bytes_per_launch")
        floor_bytes = g_bytes[0]

        # single-sequence decode (M = 1)
        one = seqs[:1]
        for _ in range(2):
            model.decode_step(one, cfg.layers)
        t0 = time.perf_counter()
        n1 = max(4, args.steps // 2)
        for _ in range(n1):
            model.decode_step(one, cfg.layers)
        m1_tok_s = n1 / (time.perf_counter() - t0)
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
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                         "kernel": "decode GEMV on the packed weight copy (k_gemv_pk for q|k|v, o and gate|up with "
                                   "their epilogues, k_gemv_sk split-K planes for down, k_gemv_head for the LM head): "
                                   "the 113 GEMV launches of one step at M = 16 (28 layers' "
                                   "q|k|v, o, gate|up, down with their own weights, then the LM head) back to back "
                                   "between two HIP events on the library's stream, so every weight byte streams "
                                   "from HBM as in a step: algorithmic bytes per pass / pass time (launch gaps "
                                   "included); traffic = mean HBM bytes per launch (rocprofv3 FETCH_SIZE + "
                                   "WRITE_SIZE, copy-calibrated)",
                         "bytes_per_launch": g_bytes[0] // max(1, g_n[0]),
                         "us_per_launch": round(g_us[0] / max(1, g_n[0]), 3),
                         "launches_per_pass": g_n[0],
                         "by_class": by_class,
                         "read_floor": read_floor},
            "decode_step_hbm_floor_ms": round(floor_bytes / (HBM_PEAK_GBS * 1e9) * 1e3, 4),
            "decode_step_hbm_frac": round(floor_bytes / (HBM_PEAK_GBS * 1e9) / (ms_step * 1e-3), 4),
            "cpu_baseline": None,
            "bit_exact_vs_cpu": None,
            "decode_m1_tok_s": round(m1_tok_s, 2),
            "step_profile_ms": {k: round(v, 4) for k, v in step_prof.items()},
        }

    if args.phase == "prefill" and args.pmc_steps:
        # counter runs: one 512-token chunk, then one pass of the chunk's 112 projection GEMMs
        pseq = pool.seq()
        pseq.prefill(rng.integers(0, cfg.vocab, size=512))
        pseq.release()
        L_ = hip.lib
        L_.sslm_hip_bench_prefill_gemm.restype = ctypes.c_int32
        L_.sslm_hip_bench_prefill_gemm.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32] + [ctypes.c_void_p] * 3
        p_us, p_ops, p_n = (ctypes.c_double * 1)(), (ctypes.c_int64 * 1)(), (ctypes.c_int64 * 1)()
        L_.sslm_hip_bench_prefill_gemm(model.handle, 512, 1, p_us, p_ops, p_n)
        return
    if args.phase in ("all", "prefill"):
        # prefill: one 512-token chunk (BASELINE configuration 2's chunk)
        chunk = rng.integers(0, cfg.vocab, size=512)
        for n in (8, 512, 512):  # warm: small shapes, then the 512-token span twice (its graph)
            pseq = pool.seq()
            pseq.prefill(chunk[:n])
            pseq.release()
        pseq = pool.seq()
        profile(hip, True)  # one profiled chunk: per-launch events, graphs off
        pseq.prefill(chunk)
        pms, pla, pby, pop = profile_read(hip)
        profile(hip, False)
        pseq.release()
        times = []  # then the median of 5 unprofiled chunks (graph replay), each into a fresh sequence
        for _ in range(5):
            pseq = pool.seq()
            t0 = time.perf_counter()
            pseq.prefill(chunk)
            times.append(time.perf_counter() - t0)
            pseq.release()
        pre_s = float(np.median(times))
        L_ = hip.lib
        L_.sslm_hip_bench_prefill_gemm.restype = ctypes.c_int32
        L_.sslm_hip_bench_prefill_gemm.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32] + [ctypes.c_void_p] * 3
        p_us, p_ops, p_n = (ctypes.c_double * 1)(), (ctypes.c_int64 * 1)(), (ctypes.c_int64 * 1)()
        if L_.sslm_hip_bench_prefill_gemm(model.handle, 512, 5, p_us, p_ops, p_n) != 1:
            raise RuntimeError("sslm_hip_bench_prefill_gemm failed")
        prefill_tops = p_ops[0] / (p_us[0] * 1e-6) / 1e12
        print(f"[bench] prefill 512: {pre_s * 1e3:.2f} ms, GEMM {prefill_tops:.1f} TOPS", file=sys.stderr, flush=True)
        pre = {"prefill_512_tok_s": round(512 / pre_s, 1), "prefill_512_ms": round(pre_s * 1e3, 3),
               "prefill_roofline": {"bound": "mfma", "achieved": round(prefill_tops, 1), "peak": INT8_PEAK_TOPS,
                                    "unit": "TOPS", "frac": round(prefill_tops / INT8_PEAK_TOPS, 4),
                                    "kernel": "prefill GEMM (k_gemm_wide for gate|up, k_gemm_mfma split-K for down, k_gemm_narrow for q|k|v and o): the 112 projection GEMMs of one "
                                              "512-token chunk (28 layers' q|k|v, o, gate|up, down, the layer loop's "
                                              "launch shapes) back to back between two HIP events: sum of 2*M*N*K "
                                              "/ pass time; peak = MI355X dense int8 MFMA",
                                    "us_per_pass": round(p_us[0], 2), "launches_per_pass": p_n[0]},
               "prefill_profile_ms": {"gemm_ms": round(pms[0], 3), "attention_ms": round(pms[2], 3),
                                      "row_ms": round(pms[3], 3), "launches": int(sum(pla))}}
        vendor = vendor_gemm_reference()
        if vendor:
            pre["prefill_roofline"]["vendor_reference"] = vendor
        if line is None:
            line = {"metric": METRIC, "value": round(prefill_tops, 2), "unit": "TOPS", "n_gpus": 1, "steps": 5,
                    "warmup": 2, "ms_per_step": round(pre_s * 1e3, 3), "higher_is_better": True,
                    "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
                    "config": {"workload": "config2 prefill: one 512-token chunk through 28 layers, 1.5B shape"}}
        line.update(pre)

    if args.phase == "all":
        line.update(extras(hip, model, pool, cfg, sm, rng, args, line))

    if args.phase in ("all", "decode") and not args.no_cpu and os.path.exists(
            os.path.join(ROOT, "oracle", "_ref", "libsuperslm_ref.so")):
        line["cpu_baseline"], line["bit_exact_vs_cpu"] = cpu_baseline(image, cfg, prompts, gpu_calls, args.cpu_calls,
                                                                      line.get("_config3_check"))
        if "config3_lora_tokens_equal" in line["cpu_baseline"]:
            line["config3_bit_exact_vs_cpu"] = line["cpu_baseline"].pop("config3_lora_tokens_equal")
    line.pop("_config3_check", None)
    for s in seqs:
        s.release()
    pool.close()
    model.close()
    del sm, image
    if args.phase == "all" and not args.no_config4:
        line.update(config4(hip, args))
    print(json.dumps(line))


if __name__ == "__main__":
    main()
