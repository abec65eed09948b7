#!/bin/bash
# Counter passes over one bench.py workload on an MI355X, then the per-kernel
# traffic and MFMA tables (aicompiler-test_amd/profiling.py).
#
#   bash aicompiler-test_amd/profile_counters.sh extra OUT   # C1-C4 kernels
#   bash aicompiler-test_amd/profile_counters.sh c5 OUT      # 7B decode steps, B = 1 and 16
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
          "attn_mfma_kernel<4, 1, 4>=148046676"                       # C4 paged GQA
          "attn_mfma_kernel<1, 0, 4>=67125248"                        # C3 L = 4095 (+1)
          "packed_gemm_kernel [Li2ELi2EDF16_=180596736"               # C2 B=8 gate/up
          "packed_gemm_kernel [Li1ELi2Ef=90484736"                    # C2 B=8 down
          "mfma_rows_kernel [Li2ELi1ELi1EDF16_=180596736"
          "mfma_rows_kernel [Li1ELi1ELi2Ef=90484736") ;;
  c5)
    args=(--c5-only --decode-tokens 8)
    algo=("gemv_dot_kernel@2818048x1x1=180385280"                     # B=1 gate/up + SiLU*Mul
          "gemv_dot_kernel@1572864x1x1=100696064"                     # B=1 q.k.v + RoPE
          "gemv_dot_kernel@524288x1x1=90207744"                       # B=1 down
          "gemv_dot_kernel@262144x1x1=33570816"                       # B=1 o
          "packed_gemm_kernel [Li2ELi2EDF16_Lb1ELb1ELb0E]@176128x1x1=180838400"  # B=16 gate/up
          "packed_gemm_kernel [Li1ELi2EDF16_Lb1ELb0ELb1E]@98304x1x1=101187584"   # B=16 q.k.v
          "packed_gemm_kernel [Li1ELi2EDF16_Lb1ELb0ELb0E]@262144x1x1=90660864"   # B=16 down
          "packed_gemm_kernel [Li1ELi2EDF16_Lb0ELb0ELb0E]@262144x1x1=33816576") ;; # B=16 o
  *) echo "workload must be extra or c5" >&2; exit 2 ;;
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
