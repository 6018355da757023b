#!/bin/sh
# Builds the CPU oracle (test infrastructure) into oracle/libhq_oracle.so.
# -ffp-contract=off: every multiply and add rounds separately, as MLX's
# op-by-op CPU path does. x86-64-v3 (AVX2/FMA) so the same .so runs on the
# GPU box's host CPU.
set -e
cd "$(dirname "$0")"
gcc -O3 -march=x86-64-v3 -fopenmp -ffp-contract=off -fPIC -shared -std=c99 \
    -Wall -Wextra -o libhq_oracle.so.tmp hq_oracle.c -lm
mv libhq_oracle.so.tmp libhq_oracle.so
