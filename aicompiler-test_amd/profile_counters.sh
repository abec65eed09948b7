#!/bin/bash
# Counter passes over one bench.py workload on an MI355X, then the per-kernel
# traffic and MFMA tables (aicompiler-test_amd/profiling.py).
#
#   bash aicompiler-test_amd/profile_counters.sh extra OUT   # C1-C4 kernels
#   bash aicompiler-test_amd/profile_counters.sh c5 OUT      # 7B decode steps, B = 1 and 16
#   bash aicompiler-test_amd/profile_counters.sh stalls OUT  # issue / stall counters, C1-C4 kernels
#
# Every pass is its own rocprofv3 run (a kernel trace, then FETCH_SIZE,
# WRITE_SIZE, the EA read-request sizes, TCC hit/miss and MfmaUtil with the
# f16 MFMA operation count), each within the per-block counter limits and
# under its own time limit.  Results: OUT/traffic.md, OUT/traffic.json,
# OUT/mfma.json; the databases stay in OUT/db/<pass>/run_results.db.
set -euo pipefail
workload=$1
out=$(realpath -m "$2")
root=$(cd "$(dirname "$0")/.." && pwd)
# Algorithmic bytes per launch (weights + activations read and written once)
# of the kernels each workload is measured on, as name[@grid]=bytes.
case "$workload" in
  extra)
    args=(--extra-only)
    algo=("gemv_dot_kernel@262144x1x1=33579008"                      # C1 4096 x 4096
          "read_probe_kernel=33554432"                                # C1's read floor, 32 MiB
          "gather_probe_kernel=147775488"                             # C4 K/V bytes alone
          "attn_mfma_kernel<4, 1, 4>=148046676"                       # C4 paged GQA
          "attn_mfma_kernel<1, 0, 4>=67125248"                        # C3 L = 4095 (+1)
          "packed_gemm_kernel [Li2ELi2EDF16_=180596736"               # C2 B=8 gate/up
          "packed_gemm_kernel [Li1ELi2Ef=90484736"                    # C2 B=8 down
          "mfma_rows_kernel [Li2ELi1ELi1EDF16_=180596736"
          "mfma_rows_kernel [Li1ELi1ELi2Ef=90484736") ;;
  c5)
    args=(--c5-only --decode-tokens 8)
    # Batch 1 runs the norm-folded GEMVs (row + gamma read in the prologue)
    # and the residual epilogues (residual read, sum written); batch 16 the
    # packed GEMMs with the norm folded (gamma in the weights) or the
    # residual added in the epilogue.
    algo=("gemv_norm_kernel [Li2ELi1ELi2EDF16_Li2ELb0E@313344x1x1=180393472"  # B=1 norm + gate/up + SiLU*Mul
          "gemv_norm_kernel [Li1ELi2ELi2EDF16_Li2ELb1E@393216x1x1=100704256"  # B=1 norm + q.k.v + RoPE + append
          "gemv_norm_kernel [Li1ELi1ELi6EDF16_Li3ELb0E=90215936"       # B=1 down + residual (persistent dot)
          "gemv_dot_kernel [Li1ELi1ELi2ELi4ELi2EDF16_Li3ELb0E]@262144x1x1=33579008"  # B=1 o + residual
          "packed_gemm_kernel [Li2ELi2EDF16_Lb1ELb1ELb0ELi1E@176128x1x1=180838400"  # B=16 norm + gate/up
          "packed_gemm_kernel [Li1ELi2EDF16_Lb1ELb0ELb1ELi1E@196608x1x1=101187584"  # B=16 norm + q.k.v
          # B=16 o + residual (33947648) and down + residual (90791936): with
          # packed input both are this kernel at this grid, one table row
          # over both launches, so the row's bytes are their mean
          "packed_gemm_kernel [Li1ELi2EDF16_Lb1ELb1ELb0ELi2E@262144x1x1=62369792") ;;
  stalls)
    args=(--extra-only)
    algo=() ;;
  *) echo "workload must be extra, c5 or stalls" >&2; exit 2 ;;
esac
algo_args=()
for a in "${algo[@]}"; do algo_args+=(--algorithmic "$a"); done
mkdir -p "$out/db"
export TMPDIR=/tmp
cd /tmp
run() {  # run NAME [rocprofv3 options...]
  local name=$1; shift
  echo "[profile] $workload: $name" >&2
  timeout -s KILL 300 rocprofv3 "$@" -d "$out/db/$name" -o run -- \
    python3 "$root/bench.py" "${args[@]}" > "$out/db/$name.log" 2>&1
}
run trace --kernel-trace
if [ "$workload" = stalls ]; then
  # each pass within the per-block limits (8 SQ, 4 TCP, 2 TA); the derived
  # accumulators (VmemLatency, MeanOccupancyPerCU) get passes of their own
  run sq --pmc SQ_WAVES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY \
    SQ_ACTIVE_INST_VMEM SQ_INSTS_VMEM_RD SQ_INSTS_VALU
  run sq2 --pmc SQ_WAVES SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_INSTS_LDS SQ_INSTS_SMEM \
    SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_BUSY_CU_CYCLES
  run tcp --pmc TCP_TCC_READ_REQ_LATENCY_sum TCP_TCC_READ_REQ_sum \
    TCP_UTCL1_TRANSLATION_MISS_sum TCP_UTCL1_TRANSLATION_HIT_sum TA_TA_BUSY_sum \
    TA_ADDR_STALLED_BY_TC_CYCLES_sum
  run lat --pmc VmemLatency
  run occ --pmc MeanOccupancyPerCU
  dbs=()
  for pass in sq sq2 tcp lat occ; do dbs+=(--db "$out/db/$pass/run_results.db"); done
  python3 "$root/aicompiler-test_amd/profiling.py" stalls "${dbs[@]}" \
    --trace "$out/db/trace/run_results.db" --kernel attn_mfma_kernel \
    --kernel gather_probe_kernel --kernel gemv_dot_kernel --kernel read_probe_kernel \
    --kernel copy_kernel \
    --command "bash aicompiler-test_amd/profile_counters.sh stalls OUT" \
    --workload "bench.py --extra-only: C1 GEMV, C2 B=8, C3, C4 and the C4 gather probe" \
    --json "$out/stalls.json" > /dev/null
  echo "[profile] $workload: done" >&2
  exit 0
fi
run fetch --pmc FETCH_SIZE
run write --pmc WRITE_SIZE
run rdreq --pmc TCC_EA0_RDREQ_32B_sum TCC_EA0_RDREQ_64B_sum TCC_EA0_RDREQ_128B_sum
run hit --pmc TCC_HIT_sum TCC_MISS_sum
cmd="bash aicompiler-test_amd/profile_counters.sh $workload OUT"
python3 "$root/aicompiler-test_amd/profiling.py" table --fetch "$out/db/fetch/run_results.db" \
  --write "$out/db/write/run_results.db" --rdreq "$out/db/rdreq/run_results.db" \
  --trace "$out/db/trace/run_results.db" --hit "$out/db/hit/run_results.db" \
  --copy-bytes 268435456 --min-calls 2 "${algo_args[@]}" \
  --title "Per-kernel HBM traffic: bench.py ${args[*]}" --command "$cmd" \
  --md "$out/traffic.md" --json "$out/traffic.json" > /dev/null
run mfma --pmc MfmaUtil SQ_INSTS_VALU_MFMA_MOPS_F16
python3 "$root/aicompiler-test_amd/profiling.py" mfma --db "$out/db/mfma/run_results.db" \
  --trace "$out/db/trace/run_results.db" --command "$cmd" --json "$out/mfma.json" > /dev/null
echo "[profile] $workload: done" >&2
