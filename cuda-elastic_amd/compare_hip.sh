#!/usr/bin/env bash
# Runs the graph-mode and direct-mode harness, the fused single launch and the
# naive product on identical inputs, each writing --dump, and compares the
# dumps within the oracle tolerances with l2c_compare (the check flow of the
# reference's llama2c/compare_sota.sh:41-71). Every run also validates its own
# output against the CPU oracle and must exit 0.
#
# Environment:
#   SHAPES   default "1024 16384 8192|64 1000 300|33 1001 77"
#   INPUTS   default "deterministic random=1 random=2 random=3"
#   COPIES   default "nocopy" (also try "copy")
#   LAUNCHES default 3, WARMUP_MS default 1 (a check, not a measurement)
#   DUMP_DIR default a fresh temporary directory, removed afterwards
set -euo pipefail

HERE="$(cd -- "$(dirname -- "${BASH_SOURCE[0]}")" && pwd)"
HARNESS="${HARNESS:-$HERE/bin/llama2c_hip}"
COMPARE="${COMPARE:-$HERE/bin/l2c_compare}"
SHAPES="${SHAPES:-1024 16384 8192|64 1000 300|33 1001 77}"
INPUTS="${INPUTS:-deterministic random=1 random=2 random=3}"
COPIES="${COPIES:-nocopy}"
LAUNCHES="${LAUNCHES:-3}"
WARMUP_MS="${WARMUP_MS:-1}"

make -C "$HERE" --no-print-directory >/dev/null

if [[ -n "${DUMP_DIR:-}" ]]; then
  mkdir -p "$DUMP_DIR"
  out="$DUMP_DIR"
else
  out="$(mktemp -d "${TMPDIR:-/tmp}/l2c-compare.XXXXXX")"
  trap 'rm -rf "$out"' EXIT
fi

run() {  # run <label> <mode> <variant> <batch> <size> <rows> <copies> <inputs> <dump>
  local label="$1" mode="$2" variant="$3" batch="$4" size="$5" rows="$6" copies="$7" inputs="$8" dump="$9"
  local line
  if ! line="$("$HARNESS" "$mode" "$LAUNCHES" "$batch" "$size" "$rows" 1 "$WARMUP_MS" \
               "$copies" "$variant" "$inputs" "--dump=$dump" 2>&1)"; then
    printf '  %s: FAILED (exit code or validation)\n%s\n' "$label" "$line"
    return 1
  fi
  printf '  %-15s %s\n' "$label" "$(printf '%s\n' "$line" | tr ' ' '\n' |
    grep -E '^(mode|matmul|gpu_ms_per_iter|valid)=' | paste -sd' ')"
}

failures=0
IFS='|' read -r -a shape_list <<< "$SHAPES"
for shape in "${shape_list[@]}"; do
  read -r batch size rows <<< "$shape"
  for copies in $COPIES; do
    for inputs in $INPUTS; do
      printf '== batch=%s size=%s rows=%s %s %s\n' "$batch" "$size" "$rows" "$copies" "$inputs"
      ok=1
      run graph graph coalesced "$batch" "$size" "$rows" "$copies" "$inputs" "$out/graph.bin" || ok=0
      run direct direct coalesced "$batch" "$size" "$rows" "$copies" "$inputs" "$out/direct.bin" || ok=0
      run fused graph fused "$batch" "$size" "$rows" "$copies" "$inputs" "$out/fused.bin" || ok=0
      run naive direct naive "$batch" "$size" "$rows" "$copies" "$inputs" "$out/naive.bin" || ok=0
      if ((ok)); then
        "$COMPARE" "$out/graph.bin" "$out/direct.bin" "$out/fused.bin" "$out/naive.bin" || ok=0
      fi
      ((ok)) || failures=$((failures + 1))
      rm -f "$out"/*.bin
    done
  done
done
if ((failures)); then
  printf 'compare_hip: %d configuration(s) FAILED\n' "$failures"
  exit 1
fi
printf 'compare_hip: all configurations match\n'
