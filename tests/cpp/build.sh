#!/bin/sh
# Builds the C++ host-API test program (test infrastructure) against the
# in-tree library: tests/cpp/_build/test_host_api.
set -e
here="$(cd "$(dirname "$0")" && pwd)"
root="$(cd "$here/../.." && pwd)"
mkdir -p "$here/_build"
g++ -O1 -std=c++17 -Wall -D__HIP_PLATFORM_AMD__ -I/opt/rocm/include -I"$root/include" \
    "$here/test_host_api.cpp" -o "$here/_build/test_host_api" \
    -L"$root/tensor-adapt_amd" -ltadapt -Wl,-rpath,'$ORIGIN/../../../tensor-adapt_amd' \
    -L/opt/rocm/lib -lamdhip64 -Wl,-rpath,/opt/rocm/lib
