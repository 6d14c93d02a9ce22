#!/usr/bin/env bash
# check_handwritten.sh -- every GPU version must be hand-written: no GEMM or
# ML library and no CUDA-compatibility layer in the kernel sources.
# ROCm counterpart of the reference's scripts/check_handwritten.sh:14-34
# (which greps for cutlass|cute|cublas|cudnn outside v0, skipping comments).
# Exit 0 = clean, 1 = violation, 2 = bad path.
set -uo pipefail
ROOT="${1:-$(cd "$(dirname "${BASH_SOURCE[0]}")/.." && pwd)}"
SRC="$ROOT/csrc"
[ -d "$SRC" ] || { echo "no source directory $SRC"; exit 2; }
FILES=$(find "$SRC" "$ROOT/../include" -type f \( -name '*.hip' -o -name '*.hpp' -o -name '*.cpp' -o -name '*.h' \) 2>/dev/null)
PAT='rocblas|hipblas|hipblaslt|composable_kernel|ck_tile|include[^/]*[<"]ck/|rocwmma|triton|miopen|cuda_runtime|cuda_fp16|cublas|cutlass|cute/|cudnn|__HIP_PLATFORM_NVIDIA__'
bad=0
for f in $FILES; do
  hits=$(grep -nEi "$PAT" "$f" 2>/dev/null | grep -vE ':[[:space:]]*(//|\*|/\*)' || true)
  if [ -n "$hits" ]; then
    echo "violation (library or compatibility layer): ${f#$ROOT/}"
    echo "$hits" | sed 's/^/    /'
    bad=1
  fi
done
if [ "$bad" = 0 ]; then
  echo "ok: no GEMM library / compatibility layer in $(echo "$FILES" | grep -c .) kernel and ABI files"
else
  exit 1
fi
