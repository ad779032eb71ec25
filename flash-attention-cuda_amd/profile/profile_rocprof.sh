#!/usr/bin/env bash
#
# rocprofv3 capture of the hot-path kernels on an MI355X, then the report.
#
#   bash flash-attention-cuda_amd/profile/profile_rocprof.sh [OUT_DIR [WORKLOAD ...]]
#   bash flash-attention-cuda_amd/profile/profile_rocprof.sh --extract-only OUT_DIR
#
# Default OUT_DIR: the raw-output folder set below (raw rocprofv3 CSVs, not committed).
# Default workloads: every one of profile_workload.py, copy_1g included (it
# calibrates the HBM byte counters), then bench.py's prefill and decode runs
# under the kernel trace. Writes OUT_DIR/report.md, OUT_DIR/report.json and
# OUT_DIR/split/ (one file per workload, named <workload>__<kernel>.md, plus
# bench_traces.md and occupancy.md: the files committed under profiles/).
#
# Per workload, four separate rocprofv3 runs (counters are never combined
# with tracing, and each --pmc pass stays inside one pass's counter limits:
# 5 SQ counters and 1 GRBM counter for the derived metrics, 3 and 2 TCC
# counters for FETCH_SIZE and WRITE_SIZE):
#   trace  --kernel-trace --stats
#   fetch  --pmc FETCH_SIZE
#   write  --pmc WRITE_SIZE
#   sq     --pmc MfmaUtil MfmaFlopsF16 LdsBankConflict OccupancyPercent
# Every run has its own time limit; the script stops at the first failure.
#
# The reference's counterpart is bench/profile_ncu.sh (Nsight Compute
# capture + bench/ncu_extract.py).

set -uo pipefail

HERE="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
REPO="$(cd "${HERE}/../.." && pwd)"
PYTHON="${PYTHON:-python3}"
ROCPROF="${ROCPROF:-rocprofv3}"

EXTRACT_ONLY=0
if [[ "${1:-}" == "--extract-only" ]]; then
  EXTRACT_ONLY=1
  shift
fi
OUT="${1:-gpurun_out/rocprof}"
shift || true
BENCH=0
if [[ $# -gt 0 ]]; then
  WORKLOADS=("$@")
else
  WORKLOADS=(copy_1g prefill_c3 prefill_c2_causal prefill_c2_full decode_c4 decode_c5 decode_gqa_c5
             prefill_c3_d128 decode_c5_d128)
  BENCH=1
fi
mkdir -p "${OUT}"
export TMPDIR="${TMPDIR:-/tmp}"

run() {  # run <dir> <seconds> <rocprofv3 options...> -- <program and arguments...>
  local dir="$1" limit="$2"
  shift 2
  local opts=()
  while [[ $# -gt 0 && "$1" != "--" ]]; do
    opts+=("$1")
    shift
  done
  shift
  echo ">>> [$(date +%T)] ${dir}"
  timeout -s KILL "${limit}" "${ROCPROF}" "${opts[@]}" --output-format csv -d "${dir}" -o run \
    -- "$@" > "${dir}.log" 2>&1
  local rc=$?
  if [[ ${rc} -ne 0 ]]; then
    echo "error: rocprofv3 run ${dir} ended with status ${rc}; see ${dir}.log" >&2
    tail -5 "${dir}.log" >&2
    exit "${rc}"
  fi
}

if [[ ${EXTRACT_ONLY} -eq 0 ]]; then
  if ! command -v "${ROCPROF}" > /dev/null 2>&1; then
    echo "error: ${ROCPROF} not found (ROCm's rocprofv3; set ROCPROF=/path/to/rocprofv3)" >&2
    exit 1
  fi
  for w in "${WORKLOADS[@]}"; do
    mkdir -p "${OUT}/${w}"
    W=("${PYTHON}" "${HERE}/profile_workload.py" "${w}")
    run "${OUT}/${w}/trace" 300 --kernel-trace --stats -- "${W[@]}"
    run "${OUT}/${w}/fetch" 180 --pmc FETCH_SIZE -- "${W[@]}"
    run "${OUT}/${w}/write" 180 --pmc WRITE_SIZE -- "${W[@]}"
    if [[ "${w}" != copy_1g ]]; then
      run "${OUT}/${w}/sq" 180 --pmc MfmaUtil MfmaFlopsF16 LdsBankConflict OccupancyPercent \
        -- "${W[@]}"
    fi
  done
  if [[ ${BENCH} -eq 1 ]]; then
    # bench.py's own contract runs under the kernel trace: the report sets the
    # trace average of the roofline kernel beside bench.py's live HIP-event
    # figure from the same run.
    for part in prefill decode; do
      mkdir -p "${OUT}/bench_${part}"
      run "${OUT}/bench_${part}/trace" 300 --kernel-trace --stats -- "${PYTHON}" -u \
        "${REPO}/bench.py" --only "${part}" --no-cpu --no-configs --steps 50 --warmup 5
    done
  fi
  echo ">>> [$(date +%T)] occupancy report"
  timeout -k 10 120 "${PYTHON}" "${HERE}/profile_workload.py" occupancy "${OUT}/occupancy.json" || exit $?
fi

"${PYTHON}" "${HERE}/rocprof_extract.py" --root "${OUT}" --out "${OUT}/report.md" \
  --json "${OUT}/report.json" --split-dir "${OUT}/split" \
  --command "bash flash-attention-cuda_amd/profile/profile_rocprof.sh ${OUT} ${WORKLOADS[*]}"
