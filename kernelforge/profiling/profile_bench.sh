#!/bin/bash
# Regenerate the files of profiles/ on one MI355X, from the repository root:
#
#   bash kernelforge/profiling/profile_bench.sh [OUT]      (OUT: gpurun_out/prof)
#
# Five rocprofv3 passes over `bench.py --marks` (kernel trace with --stats,
# FETCH_SIZE, WRITE_SIZE, busy/MFMA cycles, LDS counters), each pass in a
# process of its own and under a time limit, then the summariser
# (kernelforge.profiling.bench_profiles). The summaries land in OUT/out; copy
# them to profiles/. Each records the commands that made it and the library's
# source digest, which bench.py checks before it prints the figures.
set -o pipefail
P="${1:-gpurun_out/prof}"
mkdir -p "$P" && rm -rf "$P"/trace "$P"/fetch "$P"/write "$P"/busy "$P"/lds "$P"/out "$P"/marks_*.json
export TMPDIR=/tmp
B="python -u bench.py --no-cpu-baseline --no-sustained"
TRACE_CMD="rocprofv3 --kernel-trace --stats --output-format csv -d $P/trace -o bench -- $B --steps 50 --warmup 10 --marks $P/marks_trace.json"
FETCH_CMD="rocprofv3 --pmc FETCH_SIZE --output-format csv -d $P/fetch -o fetch -- $B --steps 2 --warmup 1 --marks $P/marks_fetch.json"
WRITE_CMD="rocprofv3 --pmc WRITE_SIZE --output-format csv -d $P/write -o write -- $B --steps 2 --warmup 1 --marks $P/marks_write.json"
BUSY_CMD="rocprofv3 --pmc GRBM_GUI_ACTIVE SQ_BUSY_CU_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_VALU_MFMA_MOPS_BF16 --output-format csv -d $P/busy -o busy -- $B --steps 2 --warmup 1 --marks $P/marks_busy.json"
LDS_CMD="rocprofv3 --pmc SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE --output-format csv -d $P/lds -o lds -- $B --steps 2 --warmup 1 --marks $P/marks_lds.json"
run() { local name=$1 limit=$2; shift 2; echo "step: $name"; timeout -s KILL $limit "$@" > $P/$name.log 2>&1 || { echo "$name failed"; tail -5 $P/$name.log; exit 11; }; }
run trace 600 $TRACE_CMD
run fetch 300 $FETCH_CMD
run write 300 $WRITE_CMD
run busy 300 $BUSY_CMD
run lds 300 $LDS_CMD
f() { find $P/$1 -name "*$2" | head -1; }
echo "step: summarise"
S="python -m kernelforge.profiling.bench_profiles"
$S --marks $P/marks_trace.json --trace "$(f trace kernel_trace.csv)" --stats "$(f trace kernel_stats.csv)" --trace-command "$TRACE_CMD" --out $P/out || exit 14
$S --marks $P/marks_fetch.json --fetch "$(f fetch counter_collection.csv)" --write "$(f write counter_collection.csv)" \
   --traffic-command "$FETCH_CMD" --traffic-command "$WRITE_CMD" --out $P/out || exit 15
$S --marks $P/marks_busy.json --pmc "$(f busy counter_collection.csv)" --pmc "$(f lds counter_collection.csv)" \
   --pmc-command "$BUSY_CMD" --pmc-command "$LDS_CMD" --out $P/out || exit 16
cat $P/out/*.md
echo PROFILES_DONE
