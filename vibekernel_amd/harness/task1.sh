#!/usr/bin/env bash
# task1.sh -- build / run / profile the task1 harness binaries.
# Command surface of the reference's driver (documented in
# CLAUDE_For_KernelAgent.md:37-43 and :76 of the reference):
#   ./task1.sh run     --float f16 --ver N [-- binary args]   build + run + logs/
#   ./task1.sh build   --float f16 --ver N
#   ./task1.sh profile --float f16 --ver N [-- binary args]   rocprofv3 kernel trace (+ --pmc "...")
#   ./task1.sh clean | clean-logs
# Logs: logs/task1_<dtype>_v<N>_<timestamp>.log in the reference's format.
set -euo pipefail
HERE="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
cd "$HERE"
CMD="${1:-run}"; shift || true
FLOAT=f16; VER=0; PMC=""; EXTRA=()
while [ $# -gt 0 ]; do
  case "$1" in
    --float) FLOAT="$2"; shift 2;;
    --ver) VER="$2"; shift 2;;
    --pmc) PMC="$2"; shift 2;;
    --) shift; EXTRA=("$@"); break;;
    *) echo "unknown option $1" >&2; exit 2;;
  esac
done
case "$FLOAT" in f16|float16) DT=float16;; f32|float32) DT=float32;; *) echo "--float f16|f32" >&2; exit 2;; esac
BIN="$HERE/bin/task1_${DT}_v${VER}"
build() {
  make -C "$HERE/../csrc" -j8 >/dev/null
  make -C "$HERE" -j8 "bin/task1_${DT}_v${VER}" "../lib/libvk_v0.so" >/dev/null
}
case "$CMD" in
  build) build; echo "built $BIN";;
  run)
    build
    mkdir -p logs
    TS=$(date -u +%Y%m%d_%H%M%S)
    LOG="logs/task1_${DT}_v${VER}_${TS}.log"
    {
      echo "Run started at: $(date -u)"
      echo "FLOAT_TYPE: ${DT}"
      echo "VERSION: ${VER}"
      echo "======================================"
      "$BIN" "${EXTRA[@]}"
      echo "======================================"
      echo "Run completed at: $(date -u)"
      echo "Log saved to: ${LOG}"
    } 2>&1 | tee "$LOG"
    ;;
  profile)
    build
    mkdir -p logs/profiles
    TS=$(date -u +%Y%m%d_%H%M%S)
    OUT="logs/profiles/task1_${DT}_v${VER}_${TS}"
    if [ -n "$PMC" ]; then
      timeout -s KILL 120 rocprofv3 --pmc $PMC --output-format csv -d "$OUT" -o pmc -- "$BIN" -t 1 "${EXTRA[@]}"
    else
      rocprofv3 --kernel-trace --stats --output-format csv -d "$OUT" -o trace -- "$BIN" "${EXTRA[@]}"
    fi
    echo "profile written to $OUT"
    ;;
  clean) make -C "$HERE" clean >/dev/null; echo "cleaned";;
  clean-logs) rm -rf logs; echo "logs removed";;
  *) echo "usage: $0 run|build|profile|clean|clean-logs --float f16|f32 --ver N [-- args]" >&2; exit 2;;
esac
