#!/bin/bash
# Build the reference CPU decode kernels (inference/cpu/cpu_inference.c) from the file where it
# lies under the reference checkout, into oracle/_ref/ (git-ignored; the .so travels to the GPU
# box with the tree). TEST / BASELINE INFRASTRUCTURE ONLY.
#
# The reference hard-codes `#define HEADDIM 32` (cpu_inference.c:27) and a -D flag cannot
# override a #define in the source, so the source is streamed through sed, which rewrites that
# one line to 64 (the Mamba-2 1.3B head dimension), and straight into gcc's stdin. No copy of the
# reference source is written anywhere. ref_shim.c is appended to the same translation unit so
# the file-static step functions can be called from tests.
#
# Flags: the reference's own build line is `gcc -O3 -march=native -fopenmp -shared -fPIC`
# (cpu_inference.c:11-13). -march=native would tune for this container's CPU, not the GPU box's,
# so the ISA is named explicitly: x86-64-v4 (AVX-512 F/BW/DQ/VL) plus VNNI, which the reference's
# intrinsics need. Callers must check the host supports avx512f/avx512bw/avx512_vnni first.
set -euo pipefail
REF="${DFSSM_REFERENCE:-/root/reference}"
SRC="$REF/inference/cpu/cpu_inference.c"
HERE="$(cd "$(dirname "$0")" && pwd)"
OUT="$HERE/_ref"
if [ ! -f "$SRC" ]; then
  echo "build_ref.sh: $SRC not found; reference build skipped" >&2
  exit 0
fi
n=$(grep -c '^#define HEADDIM[[:space:]]*32[[:space:]]*$' "$SRC" || true)
if [ "$n" != "1" ]; then
  echo "build_ref.sh: expected exactly one '#define HEADDIM 32' line in $SRC, found $n" >&2
  exit 1
fi
mkdir -p "$OUT"
for HD in 64 32; do
  { sed -e "s/^#define HEADDIM[[:space:]]*32[[:space:]]*\$/#define HEADDIM $HD/" "$SRC"; cat "$HERE/ref_shim.c"; } \
    | gcc -x c -O3 -march=x86-64-v4 -mavx512vnni -fopenmp -shared -fPIC -w -o "$OUT/libcpu_inference_h$HD.so.tmp" - -lm
  mv "$OUT/libcpu_inference_h$HD.so.tmp" "$OUT/libcpu_inference_h$HD.so"
done
echo "built $OUT/libcpu_inference_h64.so $OUT/libcpu_inference_h32.so"
