#!/bin/bash
# rocprofv3 evidence for one CVMM workload on one MI355X.  The reference
# profiles its kernels with Nsight Compute (profile_forward.sh,
# profile_backward.sh); this is the rocprofv3 equivalent:
#   1. the bench.py line of the workload;
#   2. rocprofv3 --kernel-trace --stats of the same command (per-kernel times);
#   3. three counter passes over a short run of the same command, one counter
#      group each (rocprofv3 does not split counters over passes):
#        fetch: FETCH_SIZE
#        write: WRITE_SIZE, TCC_HIT_sum, TCC_MISS_sum
#        sq:    MFMA busy cycles and ops, LDS bank conflicts and instructions,
#               CU busy cycles, waves, GRBM_GUI_ACTIVE
#   `profile.sh copy` instead runs the plain 256 MiB device copy the
#   summaries scale FETCH_SIZE / WRITE_SIZE by (bytes moved / counter value).
# usage:  bash profile.sh WORKLOAD [OUTDIR]
#   WORKLOAD: a bench.py --workload name, `ffn` (the FFN stack) or `copy`
#   then:   python bench.py --summarize OUTDIR/WORKLOAD [--copy-dir OUTDIR/copy]
#           python bench.py --summarize OUTDIR/WORKLOAD --copy-dir OUTDIR/copy --traffic CLASS
#             (CLASS: gemm_fwd, gemm_bwd_x, wgrad, or step for the whole step's fabric bytes)
set -o pipefail
W=${1:?usage: profile.sh WORKLOAD [OUTDIR]}
ROOT=$(cd "$(dirname "$0")" && pwd)
OUT=${2:-$ROOT/gpurun_out/prof}/$W
export TMPDIR=/tmp
mkdir -p "$OUT"
cd "$ROOT" || exit 1
step() { echo "[profile.sh] $W: $*"; }

if [ "$W" = copy ]; then
  for c in FETCH_SIZE WRITE_SIZE; do
    step "copy calibration, $c"
    timeout -s KILL 120 rocprofv3 --pmc $c --output-format csv -d "$OUT/$c" -o run -- \
      python3 bench.py --only copy --steps 5 > "$OUT/$c.log" 2>&1 || exit $?
  done
  exit 0
fi

# ffn: the bench line times the fused and the composed stack; the trace and
# the counter runs take the fused stack (the bench line's value) alone
if [ "$W" = ffn ]; then ARGS="--ffn --ffn-variant fused"; LINE="--ffn"; else ARGS="--workload $W"; LINE=$ARGS; fi
# the tiny fp32 step is host-bound: its steps are timed as HIP graph replays
if [ "$W" = tiny_fp32 ]; then ARGS="$ARGS --graph"; LINE="$LINE --graph"; fi
step "bench line"
timeout -k 10 300 python3 bench.py $LINE --no-cpu-baseline > "$OUT/bench.json" 2> "$OUT/bench.err" || exit $?
step "kernel trace"
timeout -k 10 300 rocprofv3 --kernel-trace --stats --output-format csv -d "$OUT/trace" -o run -- \
  python3 bench.py $ARGS --no-cpu-baseline --steps 20 --kernel-iters 10 > "$OUT/trace.log" 2>&1 || exit $?
SHORT="python3 bench.py $ARGS --no-cpu-baseline --steps 3 --warmup 2 --kernel-iters 2"
step "counters: fetch"
timeout -s KILL 240 rocprofv3 --pmc FETCH_SIZE --output-format csv -d "$OUT/fetch" -o run -- \
  $SHORT > "$OUT/fetch.log" 2>&1 || exit $?
step "counters: write"
timeout -s KILL 240 rocprofv3 --pmc WRITE_SIZE TCC_HIT_sum TCC_MISS_sum --output-format csv -d "$OUT/write" -o run -- \
  $SHORT > "$OUT/write.log" 2>&1 || exit $?
step "counters: sq"
timeout -s KILL 240 rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_INSTS_VALU_MFMA_MOPS_F32 \
  SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS SQ_BUSY_CU_CYCLES SQ_WAVES GRBM_GUI_ACTIVE \
  --output-format csv -d "$OUT/sq" -o run -- $SHORT > "$OUT/sq.log" 2>&1 || exit $?
step "done"
