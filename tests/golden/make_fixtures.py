"""Regenerates reference_fixtures.json: the golden vectors of the reference's own unit tests
for the integer forward path, as data.

Needs the reference tree (default /root/reference) and g++; run it where both exist:
    python tests/golden/make_fixtures.py [--ref /root/reference]
dump_reference_fixtures.cpp includes the reference's fixture headers by path and prints
their cases; this script compiles it into a temporary directory, runs it and writes the JSON
beside itself.  The reference is Apache-2.0 (its LICENSE / NOTICE); the vectors keep that
attribution in the "_source" entry.
"""
import argparse
import json
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "reference_fixtures.json")

HEADERS = [
    "tests/sslm_intmath_fixtures.h", "tests/sslm_s3_1_wide_intmath_fixtures.h",
    "tests/sslm_iexp_domain_fixtures.h", "tests/sslm_s3_1_c30_iexp_domain_sweep_fixtures.h",
    "tests/sslm_s3_2_fixtures.h", "tests/sslm_s3_3_fixtures.h",
    "tests/sslm_s3_3_rope_application_site_fixtures.h", "tests/sslm_matmul_fixtures.h",
    "tests/matmul_golden_pin.h", "tests/silu_lut_golden_table.h",
]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    args = ap.parse_args()
    with tempfile.TemporaryDirectory() as tmp:
        exe = os.path.join(tmp, "dump")
        subprocess.run(["g++", "-std=c++20", "-O0", "-w", "-I", os.path.join(args.ref, "tests"), "-I",
                        os.path.join(args.ref, "include"), os.path.join(HERE, "dump_reference_fixtures.cpp"),
                        "-o", exe], check=True)
        data = json.loads(subprocess.run([exe], check=True, capture_output=True, text=True).stdout)
    data["_source"] = {"project": "SuperSLM reference unit-test fixtures", "license": "Apache-2.0",
                       "headers": HEADERS}
    with open(OUT, "w") as f:
        json.dump(data, f, separators=(",", ":"), sort_keys=True)
        f.write("\n")
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(data) - 1} tables)")


if __name__ == "__main__":
    main()
