#!/usr/bin/env bash
# Host-side AddressSanitizer + UndefinedBehaviorSanitizer qualification (CPU only).
#
# Builds, under _build/sanitize/:
#   libloom_infer_hip.so  - every translation unit of the product library with
#                           the host pass instrumented (-Xarch_host -fsanitize=...;
#                           device code is compiled as usual, and not run here)
#   libloom_oracle.so     - the C oracle, instrumented, with the same clang
# then runs the CPU test suite (-m "not gpu": the C-ABI host contract layer,
# plan-free spec and metadata validation, the oracle against its golden
# vectors) against both builds with the clang ASan runtime preloaded.
# Any sanitizer report aborts the run (halt_on_error), so a clean exit is a
# clean qualification.
set -euo pipefail
root="$(cd "$(dirname "$0")/.." && pwd)"
out="$root/_build/sanitize"
mkdir -p "$out/obj"
LLVM=/opt/rocm/llvm
HIPCC="${HIPCC:-/opt/rocm/bin/hipcc}"
SAN=(-fsanitize=address,undefined -fno-sanitize-recover=undefined -fno-omit-frame-pointer)
HOSTSAN=()
for f in "${SAN[@]}"; do HOSTSAN+=(-Xarch_host "$f"); done
csrc="$root/loom-kernels_amd/csrc"
FLAGS=(--offload-arch=gfx950 -O1 -g -std=c++17 -fPIC -Wall -Wno-unused-function -Wno-unused-value
       -Wno-unused-result -Xclang -target-feature -Xclang -packed-fp32-ops
       -I"$root/include" -I"$csrc")
pids=()
for s in contract.cpp runtime.cpp paged_decode.hip paged_prefill.hip rope_append.hip; do
  "$HIPCC" -x hip "${FLAGS[@]}" "${HOSTSAN[@]}" -c "$csrc/$s" -o "$out/obj/${s%.*}.o" \
      2> >(grep -v "packed-fp32-ops' is not a recognized feature" >&2) &
  pids+=($!)
done
for p in "${pids[@]}"; do wait "$p"; done
"$HIPCC" --offload-arch=gfx950 -shared -fPIC "${HOSTSAN[@]}" -shared-libsan "$out"/obj/*.o \
    -o "$out/libloom_infer_hip.so"
"$LLVM/bin/clang" -std=c11 -O1 -g -ffp-contract=off -fno-fast-math -fPIC -shared -Wall -Wextra \
    "${SAN[@]}" -shared-libsan "$root/oracle/loom_oracle.c" -o "$out/libloom_oracle.so" -lm

[ "${1:-}" = "--build-only" ] && exit 0
rt="$("$LLVM/bin/clang" -print-file-name=libclang_rt.asan-x86_64.so)"
[ -f "$rt" ] || rt="$(ls "$LLVM"/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -n1)"
# detect_leaks=0: CPython and torch keep allocations alive until exit by design.
export ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1:protect_shadow_gap=0"
export UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1"
export LOOM_INFER_HIP_LIB="$out/libloom_infer_hip.so"
export LOOM_ORACLE_LIB="$out/libloom_oracle.so"
cd "$root"
LD_PRELOAD="$rt" python -m pytest tests -q -m "not gpu" -p no:cacheprovider "$@"
