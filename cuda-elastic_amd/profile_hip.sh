#!/usr/bin/env bash
# Profiling driver of the MI355X llama2c build: the subcommands of the
# reference's llama2c/profile_cuda.sh with ROCm tools (rocprofv3 in place of
# nsys/ncu). Output goes to $OUT_DIR (default ./profiles-hip).
#
#   profile_hip.sh build
#   profile_hip.sh run    [harness args...]          one llama2c_hip invocation
#   profile_hip.sh trace  [harness args...]          rocprofv3 --kernel-trace --stats
#   profile_hip.sh counters OP B S R                 FETCH_SIZE and WRITE_SIZE passes of
#                                                    l2c_kernel_bench OP B S R 5 (one pass each)
#   profile_hip.sh sweep | sweep-fill                graph-vs-direct sweeps (python -m l2c.sweep)
#   profile_hip.sh speedup SWEEP.csv                 derived speedup CSV
#   profile_hip.sh decoder [decoder args...]         rocprofv3 trace of llama2c_decoder_hip
set -euo pipefail

HERE="$(cd -- "$(dirname -- "${BASH_SOURCE[0]}")" && pwd)"
OUT_DIR="${OUT_DIR:-$PWD/profiles-hip}"
STAMP="$(date +%Y%m%d-%H%M%S)"
BIN="$HERE/bin/llama2c_hip"
require() { command -v "$1" >/dev/null || { printf 'error: %s is not installed or not in PATH\n' "$1" >&2; exit 127; }; }
ensure_built() { [[ -x "$BIN" ]] || make -C "$HERE" -j8; }
usage() { sed -n '2,13p' "${BASH_SOURCE[0]}" | sed 's/^# \{0,1\}//'; }

case "${1:-}" in
  build) make -C "$HERE" -j8 ;;
  run) ensure_built; "$BIN" "${@:2}" ;;
  trace)
    require rocprofv3; ensure_built; mkdir -p "$OUT_DIR"
    # Kernel trace and statistics only: counters run in their own passes.
    rocprofv3 --kernel-trace --stats -d "$OUT_DIR/trace-$STAMP" -o trace --output-format csv -- "$BIN" "${@:2}" ;;
  counters)
    require rocprofv3; ensure_built; mkdir -p "$OUT_DIR"
    [[ $# -eq 5 ]] || { printf 'usage: %s counters OP BATCH SIZE ROWS\n' "$0" >&2; exit 2; }
    for counter in FETCH_SIZE WRITE_SIZE; do
      timeout -s KILL 90 rocprofv3 --pmc "$counter" -d "$OUT_DIR/pmc-$2-$counter-$STAMP" -o pmc \
        --output-format csv -- "$HERE/bin/l2c_kernel_bench" "$2" "$3" "$4" "$5" 5
    done ;;
  sweep|sweep-fill)
    ensure_built
    PYTHONPATH="$HERE${PYTHONPATH:+:$PYTHONPATH}" python3 -m l2c.sweep "$1" --out "$OUT_DIR" \
      --trials "${SWEEP_TRIALS:-3}" --warmup-ms "${SWEEP_WARMUP_MS:-100}" \
      ${SWEEP_CONFIGS:+--configs "$SWEEP_CONFIGS"} ${SWEEP_LAUNCHES:+--launches "$SWEEP_LAUNCHES"} \
      ${SWEEP_MATMUL:+--matmul "$SWEEP_MATMUL"} ;;
  speedup) PYTHONPATH="$HERE${PYTHONPATH:+:$PYTHONPATH}" python3 -m l2c.sweep speedup "$2" ;;
  decoder)
    require rocprofv3; ensure_built; mkdir -p "$OUT_DIR"
    rocprofv3 --kernel-trace --stats -d "$OUT_DIR/decoder-$STAMP" -o decoder --output-format csv -- \
      "$HERE/bin/llama2c_decoder_hip" "${@:2}" ;;
  *) usage >&2; exit 2 ;;
esac
