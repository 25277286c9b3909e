#!/bin/sh
# Builds the CPU oracle (test infrastructure only) into oracle/liboracle.so.
# -ffp-contract=off keeps F32 element math un-fused so that the k-means
# distance sums are bit-reproducible against the device kernels.
set -e
here="$(cd "$(dirname "$0")" && pwd)"
g++ -O3 -march=x86-64-v3 -fopenmp -ffp-contract=off -fPIC -shared -std=c++17 \
    -Wall -Wno-unused-function \
    "$here/oracle.cpp" -o "$here/liboracle.so"
