#!/usr/bin/env bash
# Builds libloom_infer_hip.so (gfx950 only) in-tree:
#   loom-kernels_amd/lib/libloom_infer_hip.so
#   loom-kernels_amd/lib/capi_bench  (C-ABI eager benchmark, links the library)
# Every HIP translation unit is compiled with packed FP32 ops disabled.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
root="$(cd "$here/.." && pwd)"
out="$here/lib"
obj="$here/lib/obj"
mkdir -p "$obj"
HIPCC="${HIPCC:-/opt/rocm/bin/hipcc}"
FLAGS=(--offload-arch=gfx950 -O3 -std=c++17 -fPIC -Wall -Wno-unused-function -Wno-unused-value -Wno-unused-result
       -Xclang -target-feature -Xclang -packed-fp32-ops
       -I"$root/include" -I"$here/csrc")
srcs=(contract.cpp runtime.cpp paged_decode.hip paged_prefill.hip rope_append.hip)
pids=()
for s in "${srcs[@]}"; do
  "$HIPCC" -x hip "${FLAGS[@]}" -c "$here/csrc/$s" -o "$obj/${s%.*}.o" \
      2> >(grep -v "packed-fp32-ops' is not a recognized feature" >&2) &
  pids+=($!)
done
for p in "${pids[@]}"; do wait "$p"; done
"$HIPCC" --offload-arch=gfx950 -shared -fPIC "$obj"/*.o -o "$out/libloom_infer_hip.so.tmp"
mv "$out/libloom_infer_hip.so.tmp" "$out/libloom_infer_hip.so"
# provenance of this build for the benchmark's evidence records (the GPU box
# has no git metadata): source commit, worktree state, library hash
commit=$(git -C "$root" rev-parse HEAD 2>/dev/null || echo unknown)
dirty=$( [ -n "$(git -C "$root" status --porcelain -- loom-kernels_amd include 2>/dev/null)" ] && echo true || echo false)
sha=$(sha256sum "$out/libloom_infer_hip.so" | cut -d' ' -f1)
printf '{"commit": "%s", "dirty": %s, "library_sha256": "%s", "abi_version": "1", "built_utc": "%s"}\n' \
    "$commit" "$dirty" "$sha" "$(date -u +%Y-%m-%dT%H:%M:%SZ)" > "$out/BUILD_INFO.json"
# the C-ABI eager benchmark (bench.py runs it as a child process)
"$HIPCC" --offload-arch=gfx950 -O2 -std=c++17 -Wall -I"$root/include" "$here/csrc/capi_bench.cpp" \
    -L"$out" -lloom_infer_hip -Wl,-rpath,'$ORIGIN' -o "$out/capi_bench.tmp"
mv "$out/capi_bench.tmp" "$out/capi_bench"
