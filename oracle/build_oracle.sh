#!/bin/sh
# Builds the CPU oracle (test infrastructure): oracle/liboracle.so in binary32
# and its binary64 twin oracle/liboracle64.so, from the same source.
# -ffp-contract=off and no -ffast-math: IEEE arithmetic in source order.
set -e
here="$(cd "$(dirname "$0")" && pwd)"
flags="-O2 -std=c11 -fPIC -shared -fopenmp -ffp-contract=off -fno-fast-math -Wall -Wextra -Wno-unused-parameter"
gcc $flags -o "$here/liboracle.so" "$here/gsv_oracle.c" -lm
gcc $flags -DORC_BINARY64 -o "$here/liboracle64.so" "$here/gsv_oracle.c" -lm
