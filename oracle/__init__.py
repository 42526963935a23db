"""Test infrastructure only: CPU restatements of leat's quantized-weight path.

Nothing in the product (`leat_amd`) imports, calls, links or executes anything here. Only the
tests, `__graft_entry__.smoke()` and bench.py's `cpu_baseline` leg use this package, and only
as the checker (or, for the CPU baseline, as the timed restatement of leat's `LEAT_KERNELS=ref`
path), never as the thing measured on the GPU.

- `leat_oracle.py`: NumPy restatement of the GGML block formats, the q8 activation quantizer,
  the f64 reference product, exact int32 group sums, GLU, routing and the expert mixture.
- `ggml_loops.py`: a second, loop-structured restatement of the dequantizers (ggml's C loop
  order), used to cross-check the vectorised one on small inputs.
- `leat_ref.c` (+ `Makefile`): C/OpenMP restatement of the `LEAT_KERNELS=ref` semantics
  (dequantize in ggml's op order, fp32 activations, fp32 accumulation), built as
  `oracle/libleatref.so`; the timed CPU baseline.
"""
