#!/usr/bin/env bash
# Builds the CPU oracle (test infrastructure) as oracle/libloom_oracle.so.
# -ffp-contract=off keeps every product rounded separately, as in the Rust
# reference; no fast-math so the C library exp/log/pow/sin/cos are used.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
gcc -std=c11 -O2 -ffp-contract=off -fno-fast-math -fPIC -shared -Wall -Wextra \
    "$here/loom_oracle.c" -o "$here/libloom_oracle.so" -lm
