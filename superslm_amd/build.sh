#!/bin/bash
# Builds libsslm_hip.so in place (gfx950).  Usage: superslm_amd/build.sh
# Any compile or link failure exits non-zero; objects are rebuilt from scratch every time so a
# stale object can never be linked into the library.
set -euo pipefail
cd "$(dirname "$0")"
FLAGS="-O3 -std=c++17 -fPIC --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops"
rm -rf _build
mkdir -p _build
compile() {
  local src=$1 obj=$2 log
  log=$(mktemp)
  if ! hipcc $FLAGS -c "$src" -o "$obj" >"$log" 2>&1; then
    cat "$log" >&2
    rm -f "$log"
    echo "build.sh: compiling $src failed" >&2
    exit 1
  fi
  # The host pass warns that it does not know the packed-fp32 feature: harmless, filtered out.
  grep -v "packed-fp32-ops" "$log" >&2 || true
  rm -f "$log"
}
compile csrc/kernels.hip _build/kernels.o &
P1=$!
compile csrc/runtime.cpp _build/runtime.o &
P2=$!
compile csrc/artifact.cpp _build/artifact.o &
P3=$!
compile csrc/noalloc.hip _build/noalloc.o &
P4=$!
FAIL=0
for p in $P1 $P2 $P3 $P4; do wait $p || FAIL=1; done
if [ $FAIL -ne 0 ]; then
  rm -f libsslm_hip.so
  exit 1
fi
hipcc -shared -fPIC --offload-arch=gfx950 _build/kernels.o _build/runtime.o _build/artifact.o \
  _build/noalloc.o -lcrypto -o libsslm_hip.so.tmp
mv libsslm_hip.so.tmp libsslm_hip.so
