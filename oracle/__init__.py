"""TEST INFRASTRUCTURE ONLY: the CPU parity oracle.

Restatements of the reference's algorithms for the compiled GPU path of lariaus/lokinfer, used only by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker. The product
(lokinfer_amd) never imports this package.

  oracle.kernels   numpy float64 restatements of every GPU kernel op (each cites the reference file:line)
  oracle.mnist     ctypes binding of oracle/mnist_ref.c (bit-exact restatement of the NEON GEMM's fma order)
  oracle.gpt2      GPT-2 124M decode via transformers.GPT2LMHeadModel built locally with seeded weights
  oracle.kokoro    PyTorch Kokoro-82M-shaped forward (the reference model graph's semantics)

Parity pinning of each function is listed in tests/test_oracle.py; functions without an independent check
are marked "parity unpinned" in their docstring.
"""
