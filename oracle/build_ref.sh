#!/usr/bin/env bash
# Builds oracle/_ref/libref.so: the reference's own run.cpp (plus tokenizer.cpp,
# whose symbols run.cpp's CLI code references) compiled from where the sources
# lie under /root/reference, with the flags of the reference's `make runomp`
# (hipcc -O3 -fopenmp, FMA available), around oracle/ref_harness.cpp.
# Nothing from the reference is copied; the output goes to oracle/_ref/ only.
# TEST INFRASTRUCTURE ONLY (pins the oracle; never part of the product).
set -euo pipefail
REF=${GKV_REFERENCE:-/root/reference}
HERE="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
if [ ! -f "$REF/run.cpp" ]; then
  echo "build_ref: $REF/run.cpp not found; skipping the reference build" >&2
  exit 0
fi
mkdir -p "$HERE/_ref"
# -DTESTING drops run.cpp's main(); x86-64-v3 has the FMA instructions that the
# reference's -march=native build contracts into.
hipcc --std=c++17 -O3 -fopenmp -march=x86-64-v3 -DTESTING -fPIC -shared \
  --offload-arch=gfx950 -w -I"$REF" \
  "$HERE/ref_harness.cpp" "$REF/tokenizer.cpp" -o "$HERE/_ref/libref.so.tmp"
mv "$HERE/_ref/libref.so.tmp" "$HERE/_ref/libref.so"
echo "build_ref: wrote $HERE/_ref/libref.so"
# The int8-V rule lives in the reference's attention test (host code); its
# file is compiled where it lies, around oracle/ref_q8_harness.cpp.
if [ -f "$REF/getp-csrc/tests/attn_test.cpp" ]; then
  hipcc --std=c++17 -O3 -fPIC -shared --offload-arch=gfx950 -w -I"$REF/getp-csrc" \
    "$HERE/ref_q8_harness.cpp" -o "$HERE/_ref/libref_q8.so.tmp"
  mv "$HERE/_ref/libref_q8.so.tmp" "$HERE/_ref/libref_q8.so"
  echo "build_ref: wrote $HERE/_ref/libref_q8.so"
fi

