#!/bin/bash
# Build oracle/_ref/ref_verify: the reference's own runner sources
# (src/runner/buffers.cpp, cpu_ref.cpp, gpu_ref.cpp), compiled where they lie
# under the reference tree, plus oracle/ref_harness.cpp, linked against this
# build's libfmha_native_amd.so.  Test infrastructure only; outputs go to
# oracle/_ref/ (git-ignored) and nothing is copied out of the reference.
#
# Flags follow the reference's CMake Release build (CMakeLists.txt:1-40):
# cpu_ref.cpp as host C++ with -O3 -fopenmp, buffers.cpp and gpu_ref.cpp as
# HIP, here for gfx950 (-w: the reference's own warnings are not ours to fix).
#
#   oracle/build_ref.sh [REFERENCE_ROOT]     (default /root/reference)
# Exits 0 without building when the reference tree is absent.
set -euo pipefail
HERE="$(cd "$(dirname "$0")" && pwd)"
ROOT="$(dirname "$HERE")"
REF="${1:-${FMHA_REFERENCE:-/root/reference}}"
if [ ! -f "$REF/src/runner/cpu_ref.cpp" ]; then
    echo "build_ref: no reference tree at $REF; oracle/_ref not built"
    exit 0
fi
LIB="$ROOT/fmha_native_amd/libfmha_native_amd.so"
if [ ! -f "$LIB" ]; then
    echo "build_ref: $LIB missing (build the package first)" >&2
    exit 1
fi
OUT="$HERE/_ref"
mkdir -p "$OUT"
TMP="$(mktemp -d)"
trap 'rm -rf "$TMP"' EXIT
HIPCC="${HIPCC:-/opt/rocm/bin/hipcc}"
HIPFLAGS=(--offload-arch=gfx950 -O3 -DNDEBUG -std=c++17 -fPIC
          -Xclang -target-feature -Xclang -packed-fp32-ops -I"$REF/src")

g++ -O3 -DNDEBUG -std=c++17 -fopenmp -fPIC -w -D__HIP_PLATFORM_AMD__ -I/opt/rocm/include -I"$REF/src" \
    -c "$REF/src/runner/cpu_ref.cpp" -o "$TMP/cpu_ref.o" &
"$HIPCC" "${HIPFLAGS[@]}" -w -c "$REF/src/runner/buffers.cpp" -o "$TMP/buffers.o" 2>&1 | grep -v "not a recognized feature" || true &
"$HIPCC" "${HIPFLAGS[@]}" -w -c "$REF/src/runner/gpu_ref.cpp" -o "$TMP/gpu_ref.o" 2>&1 | grep -v "not a recognized feature" || true &
"$HIPCC" "${HIPFLAGS[@]}" -fopenmp -I"$ROOT/include" -c "$HERE/ref_harness.cpp" -o "$TMP/ref_harness.o" 2>&1 \
    | grep -v "not a recognized feature" || true &
wait
for o in cpu_ref buffers gpu_ref ref_harness; do
    [ -f "$TMP/$o.o" ] || { echo "build_ref: compiling $o failed" >&2; exit 1; }
done
"$HIPCC" --offload-arch=gfx950 -fopenmp "$TMP/ref_harness.o" "$TMP/cpu_ref.o" "$TMP/buffers.o" "$TMP/gpu_ref.o" \
    -L"$ROOT/fmha_native_amd" -lfmha_native_amd -Wl,-rpath,'$ORIGIN/../../fmha_native_amd' \
    -o "$OUT/ref_verify.tmp"
mv "$OUT/ref_verify.tmp" "$OUT/ref_verify"
echo "build_ref: built $OUT/ref_verify"
