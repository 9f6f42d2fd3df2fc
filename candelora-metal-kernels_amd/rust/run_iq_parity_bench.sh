#!/usr/bin/env bash
# CPU-vs-GPU parity tests and the latency bench of the IQ matmul, for either
# backend of the crate: run_iq_parity_bench.sh [--backend metal|hip] [options]
#
# Counterpart of the crate's run_iq_parity_bench.sh with `--backend` added:
# `metal` runs the cpu_vs_metal_parity_* tests and the bench under
# `--features metal`; `hip` runs the cpu_vs_hip_parity_* tests
# (src/hip/parity_tests.rs) and the bench under `--features rocm`.  The other
# options and their defaults are the crate's.  Run from the crate root.  Not
# run in this repository (no Rust toolchain in its image).
set -euo pipefail

cd "$(dirname "${BASH_SOURCE[0]}")"

backend=metal
variants="iq2-xxs,iq2-xs,iq2-s,iq3-s"
m=1
out_dim=4096
in_dim=4096
warmup_runs=5
runs=20
dtype=f16
mode=off
do_parity=1
do_bench=1

usage() {
  sed -n '2,10p' "${BASH_SOURCE[0]}" | sed 's/^# \{0,1\}//'
  cat <<'EOF'

Options:
  --backend <metal|hip>     GPU backend (default: metal)
  --variants <csv>          iq2-xxs,iq2-xs,iq2-s,iq3-s (default: all four)
  --m <n>                   Batch rows for the bench (default: 1)
  --out-dim <n>             Output dimension (default: 4096)
  --in-dim <n>              Input dimension (default: 4096)
  --warmup-runs <n>         Warmup runs for the bench (default: 5)
  --runs <n>                Measured runs for the bench (default: 20)
  --dtype <f16|bf16|f32>    x dtype for the bench (default: f16)
  --activation-quant-mode <off|w8a8>
                            Mode for parity and bench (default: off)
  --skip-parity             Skip the parity tests
  --skip-bench              Skip the bench
  --help                    Show this help
EOF
}

need_value() {
  if [[ $# -lt 2 ]]; then
    echo "missing value for $1" >&2
    exit 1
  fi
}

while [[ $# -gt 0 ]]; do
  case "$1" in
    --backend) need_value "$@"; backend="$2"; shift 2 ;;
    --variants) need_value "$@"; variants="$2"; shift 2 ;;
    --m) need_value "$@"; m="$2"; shift 2 ;;
    --out-dim) need_value "$@"; out_dim="$2"; shift 2 ;;
    --in-dim) need_value "$@"; in_dim="$2"; shift 2 ;;
    --warmup-runs) need_value "$@"; warmup_runs="$2"; shift 2 ;;
    --runs) need_value "$@"; runs="$2"; shift 2 ;;
    --dtype) need_value "$@"; dtype="$2"; shift 2 ;;
    --activation-quant-mode) need_value "$@"; mode="$2"; shift 2 ;;
    --skip-parity) do_parity=0; shift ;;
    --skip-bench) do_bench=0; shift ;;
    --help|-h) usage; exit 0 ;;
    *) echo "Unknown option: $1" >&2; usage >&2; exit 1 ;;
  esac
done

case "${backend}" in
  metal) feature=metal; gpu_name=metal ;;
  hip) feature=rocm; gpu_name=hip ;;
  *) echo "invalid --backend: ${backend} (expected metal|hip)" >&2; exit 1 ;;
esac

mode="$(echo "${mode}" | tr '[:upper:]' '[:lower:]' | xargs)"
case "${mode}" in
  off) test_infix="" ;;
  w8a8) test_infix="w8a8_" ;;
  *) echo "invalid --activation-quant-mode: ${mode} (expected off|w8a8)" >&2; exit 1 ;;
esac

# normalised variant list; each name maps to its test suffix (iq2-xxs -> iq2_xxs)
normalised=()
IFS=',' read -r -a requested <<< "${variants}"
for raw in "${requested[@]}"; do
  v="$(echo "${raw}" | tr '[:upper:]' '[:lower:]' | xargs)"
  [[ -z "${v}" ]] && continue
  case "${v}" in
    iq2-xxs|iq2-xs|iq2-s|iq3-s) normalised+=("${v}") ;;
    *) echo "invalid variant in --variants: ${v}" >&2; exit 1 ;;
  esac
done
if [[ ${#normalised[@]} -eq 0 ]]; then
  echo "--variants resolved to empty list" >&2
  exit 1
fi
variant_csv="$(IFS=','; echo "${normalised[*]}")"

if [[ "${do_parity}" -eq 1 ]]; then
  echo "[iq-kernel] backend=${backend}: parity tests (mode=${mode})"
  for v in "${normalised[@]}"; do
    test_name="cpu_vs_${gpu_name}_parity_${test_infix}${v//-/_}"
    echo "[iq-kernel] parity ${v} (${test_name})"
    cargo test -q --features "${feature}" "${test_name}"
  done
fi

if [[ "${do_bench}" -eq 1 ]]; then
  echo "[iq-kernel] backend=${backend}: microbench"
  cargo run --release --features "${feature}" --example iq2_matmul_bench -- \
    --backend "${backend}" --variants "${variant_csv}" --m "${m}" --out-dim "${out_dim}" \
    --in-dim "${in_dim}" --warmup-runs "${warmup_runs}" --runs "${runs}" --dtype "${dtype}" \
    --activation-quant-mode "${mode}"
fi
