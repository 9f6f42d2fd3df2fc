#!/usr/bin/env bash
# Backend selection for run_iq_parity_bench.sh: source this file after the
# script's argument parsing, with BACKEND set from `--backend metal|hip`
# (default metal).  It maps the backend to the cargo feature and runs the
# parity tests and the bench example under that feature, with the same
# variables the script already defines (test_name, VARIANTS_NORM, M, OUT_DIM,
# IN_DIM, WARMUP_RUNS, RUNS, DTYPE, ACTIVATION_QUANT_MODE).  Not run here.
BACKEND="${BACKEND:-metal}"
case "${BACKEND}" in
  metal) FEATURE=metal ;;
  hip) FEATURE=rocm ;;
  *) echo "unknown --backend ${BACKEND}: expected metal or hip" >&2; exit 2 ;;
esac

run_backend_parity() {
  cargo test -q --features "${FEATURE}" "$1"
}

run_backend_bench() {
  cargo run --release --features "${FEATURE}" --example iq2_matmul_bench -- \
    --backend "${BACKEND}" --variants "${VARIANTS_NORM}" --m "${M}" --out-dim "${OUT_DIM}" \
    --in-dim "${IN_DIM}" --warmup-runs "${WARMUP_RUNS}" --runs "${RUNS}" --dtype "${DTYPE}" \
    --activation-quant-mode "${ACTIVATION_QUANT_MODE}"
}
