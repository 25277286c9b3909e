#!/bin/sh
# Builds oracle/_ref/libref_host.so from the reference's own host-only
# sources (cosine_schedule.hpp, dataset.cpp) where they lie under
# /root/reference, plus oracle/ref_host_shim.cpp.  Test infrastructure only;
# skipped (exit 0) when the reference tree is absent.
set -e
here="$(cd "$(dirname "$0")" && pwd)"
ref="${TA_REFERENCE_DIR:-/root/reference}"
if [ ! -f "$ref/src/data/dataset.cpp" ]; then
    echo "build_ref: $ref not present, skipping" >&2
    exit 0
fi
mkdir -p "$here/_ref"
g++ -O2 -std=c++20 -fPIC -shared -I"$ref/include" \
    "$here/ref_host_shim.cpp" "$ref/src/data/dataset.cpp" -o "$here/_ref/libref_host.so"
