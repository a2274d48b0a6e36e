"""CPU oracle for asmllm's quantized matvec path.

TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the reported CPU
baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import this package; the product (asmllm_amd) never does.

  * liboracle.so (oracle.c): op-for-op C restatement of the reference's
    kernels, threadpool, quantizers, GEMM recipe and decode ops;
  * ops_ref.py: numpy restatement of tests/reference/ops.py;
  * golden.py: the reference's golden-input recipe (tools/reference_gen.py).
"""
