#!/usr/bin/env bash
# Builds the device test programs under tests/checks/ (not part of the
# library):
#   tests/checks/bin/bf16_rounding_check  (exhaustive BF16 output-rounding check)
# They include the library's device helpers, with the library's HIP flags.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
root="$(cd "$here/../.." && pwd)"
HIPCC="${HIPCC:-/opt/rocm/bin/hipcc}"
mkdir -p "$here/bin"
"$HIPCC" -x hip --offload-arch=gfx950 -O3 -std=c++17 -Wall -Wno-unused-function -Wno-unused-result -Wno-unused-value \
    -Xclang -target-feature -Xclang -packed-fp32-ops \
    -I"$root/include" -I"$root/loom-kernels_amd/csrc" \
    "$here/bf16_rounding_check.hip" -o "$here/bin/bf16_rounding_check.tmp" \
    2> >(grep -v "packed-fp32-ops' is not a recognized feature" >&2)
mv "$here/bin/bf16_rounding_check.tmp" "$here/bin/bf16_rounding_check"
