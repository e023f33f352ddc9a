#!/bin/bash
# The host ABI checks under AddressSanitizer + UBSan: the library's sources
# compiled for the host only (no device code; -Xarch_host applies the
# sanitizers to host code; relocatable device code, so the link step makes
# the empty device image the host-only objects refer to), linked with
# host_abi_check.c.  Usage:
#   tests/sanitize/build.sh OUT_DIR    -> OUT_DIR/host_abi_check
set -e
HERE="$(cd "$(dirname "$0")" && pwd)"
ROOT="$(cd "$HERE/../.." && pwd)"
OUT="${1:?output directory}"
HIPCC="${HIPCC:-/opt/rocm/bin/hipcc}"
mkdir -p "$OUT"
SAN="-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -fno-omit-frame-pointer -fno-sanitize-recover=all"
INC="-I $ROOT/include -I $ROOT/spider-web-moe_amd/csrc"
pids=()
for f in "$ROOT"/spider-web-moe_amd/csrc/*.hip; do
  $HIPCC -x hip --offload-host-only -fgpu-rdc -O1 -g -std=c++17 -fPIC $SAN $INC -c "$f" -o "$OUT/$(basename "$f").o" &
  pids+=($!)
done
for p in "${pids[@]}"; do wait "$p"; done
$HIPCC -x c -O1 -g $SAN $INC -c "$HERE/host_abi_check.c" -o "$OUT/host_abi_check.o"
$HIPCC -fgpu-rdc --hip-link --offload-arch=gfx950 $SAN "$OUT"/*.o -o "$OUT/host_abi_check"
