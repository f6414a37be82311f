#!/bin/sh
# Build oracle/_ref/libjaxrandom_ref.so from the reference's jaxrandom.cuh
# (pure host C++, native/jaxrandom.cuh:32-34) where it lies under
# /root/reference, plus this directory's driver.  Checker only.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
REF=${BC2N_REFERENCE:-/root/reference}
mkdir -p "$HERE/_ref"
g++ -O2 -std=c++17 -shared -fPIC -I "$REF/native" \
    "$HERE/ref_jaxrandom_driver.cpp" -o "$HERE/_ref/libjaxrandom_ref.so"
