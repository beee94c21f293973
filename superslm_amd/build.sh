#!/bin/bash
# Builds libsslm_hip.so in place (gfx950).  Usage: superslm_amd/build.sh
set -euo pipefail
cd "$(dirname "$0")"
FLAGS="-O3 -std=c++17 -fPIC --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops"
mkdir -p _build
hipcc $FLAGS -c csrc/kernels.hip -o _build/kernels.o 2>&1 | grep -v "packed-fp32-ops" || true
hipcc $FLAGS -c csrc/runtime.cpp -o _build/runtime.o 2>&1 | grep -v "packed-fp32-ops" || true
hipcc $FLAGS -c csrc/artifact.cpp -o _build/artifact.o 2>&1 | grep -v "packed-fp32-ops" || true
hipcc $FLAGS -c csrc/noalloc.hip -o _build/noalloc.o 2>&1 | grep -v "packed-fp32-ops" || true
hipcc -shared -fPIC --offload-arch=gfx950 _build/kernels.o _build/runtime.o _build/artifact.o _build/noalloc.o -lcrypto -o libsslm_hip.so
