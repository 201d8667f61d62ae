#!/bin/bash
# Sanitizer builds for the CPU tests (no GPU): the library's host code (every
# source compiled host-only) linked with the C-ABI probe, and the C oracle
# linked with its probe, both under AddressSanitizer and
# UndefinedBehaviorSanitizer. Usage: build.sh OUTDIR
set -euo pipefail
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
OUT=$1
mkdir -p "$OUT"
HIPCC=${HIPCC:-/opt/rocm/bin/hipcc}
SAN="-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -Xarch_host -fno-sanitize-recover=all"
pids=()
for src in abi.cpp matvec.hip moe.hip moe_i8.hip moe_tiles.hip router.hip plan.hip gemm_q8.hip rht.hip layer.hip block.hip encode.hip; do
  $HIPCC -x hip -O1 -g -fPIC -std=c++17 --offload-arch=gfx950 $SAN -Xclang -target-feature -Xclang -packed-fp32-ops \
    -Wno-unused-command-line-argument -c "$ROOT/keep_amd/csrc/$src" -o "$OUT/${src%.*}.lib.o" &
  pids+=($!)
done
for p in "${pids[@]}"; do wait "$p"; done
$HIPCC -O1 -g -std=c++17 --offload-host-only $SAN -I "$ROOT/include" -c "$HERE/abi_probe.cpp" \
  -o "$OUT/abi_probe.o"
$HIPCC --offload-arch=gfx950 $SAN "$OUT/abi_probe.o" "$OUT"/*.lib.o -o "$OUT/abi_probe"
gcc -O1 -g -std=c11 -fopenmp -fsanitize=address,undefined -fno-sanitize-recover=all "$HERE/oracle_probe.c" \
  "$ROOT/oracle/cpu_ref.c" -o "$OUT/oracle_probe" -lm
