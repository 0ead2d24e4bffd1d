"""TEST INFRASTRUCTURE — CPU oracle of the decider hot path.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker: the product
(``fastdecisions_amd``) never imports, links or runs it.

Contents (each function cites the reference file:line it restates):
  fd_oracle.c  packed conv + SiLU and fused add + RMSNorm in fp32 (C, bit-level)
  cpu.py       ctypes wrappers of fd_oracle.c; fp64 numpy GQA attention;
               the decision readout (masked softmax + argmax)
  build.py     gcc recipe for liboracle_fd.so (-ffp-contract=off)

Parity pins (tests/test_oracle.py): golden fixtures in tests/golden/, torch's
own F.conv1d / scaled_dot_product_attention / eager RMSNorm on CPU, fp64
closed forms and brute force, special cases.  No reference code is imported
or run: the reference is Python + Triton and cannot run without a CUDA device.
"""
