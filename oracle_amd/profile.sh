#!/bin/bash
# Profiles one bench.py workload with rocprofv3 and writes short text summaries:
#   OUT/<workload>_kernel_stats.txt   rocprofv3 --kernel-trace --stats of the bench command
#   OUT/<workload>_traffic.json       HBM bytes per dispatch of KERNEL (FETCH_SIZE, WRITE_SIZE),
#                                     each scaled against a device-to-device copy of known size
#
#   OUT/<workload>_counters.json      with a fourth argument "mfma": MFMA and LDS counters of
#                                     KERNEL (two counter passes) and the MFMA-busy fraction
#
#   bash oracle_amd/profile.sh WORKLOAD KERNEL_SUBSTRING [OUT] [mfma] [TAG]  (OUT defaults to prof_out;
#   TAG is appended to the output names, e.g. _int8 for a run with OQ_GEMM_INT8=1 exported)
#
# Every rocprofv3 run has a time limit of its own; counters are collected one per run, with no
# trace domain beside them.
set -euo pipefail
WL=$1
KERN=$2
OUT=${3:-prof_out}
TAG=${5:-}
ROOT=$(cd "$(dirname "$0")/.." && pwd)
cd /tmp && export TMPDIR=/tmp
cd "$ROOT"
mkdir -p "$OUT"
RAW="$OUT/raw_$WL$TAG"
COPY_BYTES=28311552
SECONDARY=""
[ "$WL" = "q4k_gemv" ] && SECONDARY="--no-secondary"
# workloads that are a bench workload with options
BWL=$WL
case "$WL" in
    attention_decode_f16) BWL="attention_decode --kv f16" ;;
    attention_block_4_tokens) BWL="attention_block --tokens 4" ;;
    deltanet_block_4_tokens) BWL="deltanet_block --tokens 4" ;;
    attention_block_2_tokens) BWL="attention_block --tokens 2" ;;
    deltanet_block_2_tokens) BWL="deltanet_block --tokens 2" ;;
esac

# the headline workload is traced in the shape the default run times it (20 steps after 5 warmup
# steps, every secondary workload after it); the others in 200 steps after 20
if [ "$WL" = "q4k_gemv" ]; then
    TRACE_CMD="rocprofv3 --kernel-trace --stats --output-format csv -d $RAW/trace -o run -- python3 bench.py --workload $WL --steps 20 --warmup 5 --no-cpu"
else
    TRACE_CMD="rocprofv3 --kernel-trace --stats --output-format csv -d $RAW/trace -o run -- python3 bench.py --workload $BWL --steps 200 --warmup 20 --no-cpu $SECONDARY"
fi
echo "trace: $TRACE_CMD"
timeout -k 10 300 $TRACE_CMD > "$RAW.trace.log" 2>&1
for C in FETCH_SIZE WRITE_SIZE; do
    echo "pmc $C"
    timeout -s KILL 60 rocprofv3 --pmc $C --output-format csv -d "$RAW/$C" -o run -- \
        python3 bench.py --workload $BWL --steps 20 --warmup 2 --no-cpu $SECONDARY > "$RAW.$C.log" 2>&1
    timeout -s KILL 60 rocprofv3 --pmc $C --output-format csv -d "$RAW/copy_$C" -o run -- \
        python3 bench.py --workload copy_calibration --steps 20 > "$RAW.copy_$C.log" 2>&1
done

{
    echo "# rocprofv3 kernel statistics, workload $WL$TAG"
    [ -n "$TAG" ] && echo "# launch options: $(env | grep '^OQ_' | tr '\n' ' ')"
    echo "# recipe: bash oracle_amd/profile.sh $WL '$KERN' <out> ${4:-} $TAG"
    echo "# command: (cd \$REPO && ${TRACE_CMD//$OUT/<out>})   (<out>: the OUT argument)"
    echo "# bench line of that run:"
    grep '^{' "$RAW.trace.log" | tail -1 | sed 's/^/#   /'
    python3 -m oracle_amd.profsum stats "$RAW/trace"
} > "$OUT/${WL}${TAG}_kernel_stats.txt"
# the blocks' launches are summarised one by one (each kernel and grid of the step)
PER=""
case "$WL" in deltanet_block*|attention_block*) PER="--per-kernel" ;; esac
python3 -m oracle_amd.profsum traffic --kernel "$KERN" --fetch "$RAW/FETCH_SIZE" --write "$RAW/WRITE_SIZE" \
    --copy-fetch "$RAW/copy_FETCH_SIZE" --copy-write "$RAW/copy_WRITE_SIZE" --copy-bytes $COPY_BYTES $PER \
    > "$OUT/${WL}${TAG}_traffic.json"
echo "wrote $OUT/${WL}${TAG}_kernel_stats.txt $OUT/${WL}${TAG}_traffic.json"
if [ "$WL" = "q4k_gemv" ]; then
    # the same timed steps with no host launch between them (bench.py --graph): a kernel trace
    # delays each eager launch by several microseconds, so the GPU idles between the traced
    # dispatches above; in a graph they run back to back, as in the untraced run
    GRAPH_CMD="rocprofv3 --kernel-trace --stats --output-format csv -d $RAW/graph -o run -- python3 bench.py --workload $WL --steps 20 --warmup 5 --no-cpu --no-secondary --graph"
    echo "trace: $GRAPH_CMD"
    timeout -k 10 300 $GRAPH_CMD > "$RAW.graph.log" 2>&1
    {
        echo "# rocprofv3 kernel statistics, workload $WL, timed steps as one HIP graph launch"
        echo "# recipe: bash oracle_amd/profile.sh $WL '$KERN' <out>"
        echo "# command: (cd \$REPO && ${GRAPH_CMD//$OUT/<out>})   (<out>: the OUT argument)"
        echo "# bench line of that run:"
        grep '^{' "$RAW.graph.log" | tail -1 | sed 's/^/#   /'
        python3 -m oracle_amd.profsum stats "$RAW/graph"
        echo "# the timed graph launch's dispatches of the matching kernel (the last K of them):"
        python3 -m oracle_amd.profsum dispatches --kernel "$KERN" --last 20 "$RAW/graph"
    } > "$OUT/${WL}_graph_kernel_stats.txt"
    echo "wrote $OUT/${WL}_graph_kernel_stats.txt"
fi
if [ "${4:-}" = "mfma" ]; then
    P1="SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_VALU_MFMA_MOPS_I8 GRBM_GUI_ACTIVE SQ_INSTS_MFMA SQ_INSTS_VALU SQ_WAVE_CYCLES"
    P2="SQ_LDS_BANK_CONFLICT SQ_ACTIVE_INST_LDS SQ_WAIT_INST_LDS SQ_LDS_DATA_FIFO_FULL SQ_LDS_CMD_FIFO_FULL SQ_WAIT_ANY SQ_ACTIVE_INST_VALU SQ_VALU_MFMA_COEXEC_CYCLES"
    for PASS in 1 2; do
        if [ $PASS = 1 ]; then C=$P1; else C=$P2; fi
        echo "pmc pass $PASS"
        timeout -s KILL 90 rocprofv3 --pmc $C --output-format csv -d "$RAW/mfma$PASS" -o run -- \
            python3 bench.py --workload $BWL --steps 10 --warmup 2 --no-cpu $SECONDARY > "$RAW.mfma$PASS.log" 2>&1
    done
    python3 -m oracle_amd.profsum counters --kernel "$KERN" "$RAW/mfma1" "$RAW/mfma2" > "$OUT/${WL}${TAG}_counters.json"
    echo "wrote $OUT/${WL}${TAG}_counters.json"
fi
