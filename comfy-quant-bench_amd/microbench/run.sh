#!/bin/bash
# Runs every microbenchmark once (each finishes in well under a second of GPU time).
cd "$(dirname "$0")"
for b in mfma_peak lds_read_bw mfma_fma_coissue_small mfma_fma_coissue_random mfma_valu_operands mfma_valu_roles \
         mfma_lds_reads read_30mb lds_transpose stream_rq operand_delivery; do
  echo "== $b"
  timeout -k 5 120 ./$b || exit $?
done
