"""Regenerates workload_fixtures.json: the compiled reference's results on BASELINE configurations
1-4 at their real shapes (tests/baseline_workloads.py), as tokens and SHA-256 digests.

Needs oracle/_ref/libsuperslm_ref.so (built by `make -C oracle` where the reference sources
are); runs on the CPU only.  The 1.5B runs take a few minutes, the 7B run (--c4) about ten more
and ~20 GB of memory:
    python tests/golden/make_workload_fixtures.py [--c4] [--threads 8]
Existing entries are kept unless recomputed.
"""
import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))
OUT = os.path.join(HERE, "workload_fixtures.json")

import baseline_workloads as W  # noqa: E402
from oracle_bind import REF_SO  # noqa: E402
from superslm_amd.sslm import SslmLib  # noqa: E402


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--c4", action="store_true", help="also the 7B-shape run")
    ap.add_argument("--only", default="c1,c2,c3", help="comma-separated 1.5B workloads to run")
    ap.add_argument("--threads", type=int, default=8)
    args = ap.parse_args()
    ref = SslmLib(REF_SO)
    data = json.load(open(OUT)) if os.path.exists(OUT) else {}
    only = set(args.only.split(",")) if args.only else set()
    if only:
        sm = W.model_15b()
        data["artifact_15b"] = W.artifact_hash(sm)
        t0 = time.time()
        if "c1" in only:
            data["c1"] = W.run_c1(ref, sm, batched=False, threads=args.threads)
            data["c1_solo"] = W.run_c1_solo(ref, sm)
            print(f"c1 done {time.time() - t0:.0f}s", flush=True)
        if "c2" in only:
            data["c2"] = W.run_c2(ref, sm, [W.C2_PROMPT], sm.config.layers)
            print(f"c2 done {time.time() - t0:.0f}s", flush=True)
        if "c3" in only:
            data["c3"] = W.run_c3(ref, sm, sm.config.layers)
            print(f"c3 done {time.time() - t0:.0f}s", flush=True)
    if args.c4:
        sm7 = W.model_7b()
        data["artifact_7b"] = W.artifact_hash(sm7)
        t0 = time.time()
        data["c4"] = W.run_c4(ref, sm7, sm7.config.layers, W.C4_PROMPT)
        print(f"c4 done {time.time() - t0:.0f}s", flush=True)
    data["_source"] = "oracle/_ref/libsuperslm_ref.so (the reference compiled from its own sources) on " \
                      "tests/baseline_workloads.py"
    with open(OUT, "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
