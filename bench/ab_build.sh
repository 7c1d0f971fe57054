#!/bin/bash
# ab_build.sh COMMIT OUTDIR -- builds the product library of git COMMIT into OUTDIR/libgpt2amd.so and
# this tree's timing harness (bench/bench.hip, compiled against this tree's headers) linked to it into
# OUTDIR/libgpt2bench.so, for bench/ab.py's lib=OUTDIR variants.  Build here (hipcc cross-compiles
# gfx950), then run ab.py on the GPU box; OUTDIR must lie inside the repository to travel there.
set -euo pipefail
ROOT=$(cd "$(dirname "$0")/.." && pwd)
COMMIT=$1
mkdir -p "$2"
OUT=$(cd "$2" && pwd)
SRC=$(mktemp -d)
trap 'rm -rf "$SRC"' EXIT
git -C "$ROOT" archive "$COMMIT" bare-metal-gpt2_amd/csrc include | tar -x -C "$SRC"
# the commit's own bench.hip lived in csrc/ before the harness moved to bench/: leave it out
sed -i 's/ bench\.hip//' "$SRC/bare-metal-gpt2_amd/csrc/Makefile"
make -s -C "$SRC/bare-metal-gpt2_amd/csrc" -j8 OUT="$OUT/libgpt2amd.so"
/opt/rocm/bin/hipcc -O3 -std=c++17 -fPIC --offload-arch=gfx950 -Wno-unused-value -Wno-unused-result -I"$ROOT/include" -I"$ROOT/bare-metal-gpt2_amd/csrc" \
    -Xclang -target-feature -Xclang -packed-fp32-ops -shared -o "$OUT/libgpt2bench.so" "$ROOT/bench/bench.hip" \
    -L"$OUT" -lgpt2amd -Wl,-rpath,'$ORIGIN' 2>&1 | grep -v "packed-fp32-ops' is not a recognized feature" || true
test -f "$OUT/libgpt2amd.so" && test -f "$OUT/libgpt2bench.so"
echo "built $OUT (libgpt2amd.so of $COMMIT, libgpt2bench.so of this tree)"
