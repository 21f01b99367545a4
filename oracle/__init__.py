"""CPU oracle for the MoBA hot path -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import, call, link or execute anything in this directory, and
only as the checker. The product (`moba-triton_amd/`) never imports it: every
product entry point runs the HIP library or raises.

Contents:

* `naive.py`   -- torch restatement of the reference oracle
                  (`src/moba/naive.py`, `src/moba/gqa.py`,
                  `src/moba/kernels/routing.py:467-624`) plus the sparse
                  gather form used for long sequences and the textbook merge
                  (`tests/test_moba_kernel.py:117-139`).
* `moba_oracle.c` -- plain-C restatement of pooling, the gate (streaming
                  top-k, exact scores) and the CSC transpose, for bit-exact
                  checks at sizes where a dense [S, num_blocks] score matrix
                  would not fit.
* `Makefile`   -- builds `moba_oracle.c` into `oracle/_build/`.

Score rounding, stated once. The reference ranks `bf16(einsum(q, kbar))`
(`src/moba/naive.py:109`) where the einsum accumulates in float32 in an order
chosen by the BLAS underneath; no order is part of the reference's contract
(cuBLAS on GPU, oneDNN on CPU, each different). This oracle fixes the order
out of the result: a score is the exact dot product rounded once to float32
and then to the input dtype. Products of bf16/fp16/fp32 values are exact in
float64 and the 64-128-term sums are exact for any input whose exponents span
fewer than ~30 binades, so "float64 sum, then round" *is* the correctly
rounded value. The GPU kernels compute the same quantity. Parity of this
definition against the reference's own float32 einsum is pinned by the golden
fixtures in `tests/golden/` (see `tests/test_oracle_golden.py`): every
disagreement there is a score whose float32 accumulation error crossed a bf16
rounding boundary.
"""
