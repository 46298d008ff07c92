"""CPU oracle for TileQuant's mixed INT8/BF16 64x64-tile linear path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker (or the timed CPU baseline).  The product package ``tilequant_amd``
never imports it, and it is never a fallback for the HIP path.

Contents:

* ``oracle.numerics`` -- numpy restatement of the closed forms (activation
  per-64-column-tile absmax scales and codes, weight tile scales and codes,
  exact INT32 tile products, the float64 tile GEMM with an error bound).
* ``oracle.packing`` -- numpy restatement of the load-time packer's tile
  bookkeeping (id order, CSR row pointers, row-stacking of packs) and of the
  MFMA operand-major tile re-layout used by the HIP kernels.
* ``oracle.masks`` -- the Decision/ tile-map archive format and the top-k
  mask rule.
* ``oracle.torch_ref`` -- the reference's CPU quantization branch as torch
  ops (quant_utils.py:61-74, 103-115) and its whole-tensor helpers
  (:17-37, 138-148): checker, and the quantization leg of the CPU baseline.
* ``oracle.native`` -- ctypes wrapper of ``tq_oracle.c`` (same closed forms in
  C, OpenMP over row tiles) for the larger cases and the CPU baseline.

Parity pinning (what checks each function):

* whole-tensor quantization (``numerics.tensor_quant``): exhaustive sweeps of
  every bf16 / fp16 value of a range against the reference's torch expressions
  on CPU tensors (``torch_ref.tensor_quant``), with exact half-integer
  quotients; a planted mistake (the quotient not rounded to the input dtype)
  must fail.
* activation/weight closed forms: exhaustive sweeps over bf16 values against
  torch-CPU ops (the reference's own CPU branch, quant_utils.py:61-74,
  103-115), numpy-vs-C agreement, and the invariant that a tile's absmax
  element maps to +-127 whenever its scale is a normal number.
* INT32 tile products: brute-force integer matmul (numpy int64) and the C
  loop agree; linearity and sign-flip invariants.
* tile GEMM fp32/fp64 sums: numpy float64 vs C float64, a dense
  dequantised-matmul closed form, and hand-built cases with known answers.
* packing bookkeeping: invariants (T8+T16 = n_tr*n_tc, sorted ids,
  row_ptr[-1] = T) and hand-built cases.
* top-k mask rule: the reference's released Decision/ maps (golden fixtures
  under tests/golden/).
"""
