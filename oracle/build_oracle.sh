#!/bin/sh
# Builds the CPU oracle (test infrastructure) into oracle/liboracle.so.
# -ffp-contract=off and no -ffast-math: binary32 IEEE arithmetic in source order.
set -e
here="$(cd "$(dirname "$0")" && pwd)"
gcc -O2 -std=c11 -fPIC -shared -fopenmp -ffp-contract=off -fno-fast-math \
    -Wall -Wextra -Wno-unused-parameter \
    -o "$here/liboracle.so" "$here/gsv_oracle.c" -lm
