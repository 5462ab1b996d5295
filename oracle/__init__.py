"""CPU oracle of the sparse-attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithms the HIP kernels implement, so
that tests can check the GPU results. It is a checker, never a product path: only the
tests under tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it,
and nothing in sparseattnfunctions_amd/ does.

  attention.py  dense attention with the kron-expanded block mask, fp64 / fp32 (torch CPU)
  estimator.py  sampled block scores of the adaptive estimator (fp64)
  pattern.py    frame-pattern attention and the head-routing judges (fp64)
  pooling.py    dense / causal attention with its 2-D max-pooled attention map (fp64)
  sta.py        sliding-tile token order and token-level mask
  sa_oracle.c   bit-exact integer/fp32 parts (block pooling, block scores, top-k lists,
                local window, token-merge matching), built into liboracle.so by the
                Makefile here and loaded through oracle/native.py
"""
