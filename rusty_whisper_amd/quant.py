"""The reference's quantized-weight API (src/quant.rs) on the MI355X.

Re-exports the C++ mirror (host/rw_quant.hpp, via the _rw_quant binding):

  QK, block_bytes   src/quant.rs:17, 43-52
  QTensor           src/quant.rs:495-640   (shape, dtype, raw, row_f32, to_dense)
  Weight            src/quant.rs:643-675   (Weight.Dense / Weight.Quant)
  matmul_t_q        src/quant.rs:754-1051
  matmul_t          src/tensor.rs:194-238  (the dense f32 tier, bit-identical)
  linear_w          src/quant.rs:1054-1063
  Panic             raised where the reference panics, with its message

numpy float32 arrays play the role of the reference's Tensor.
"""
from ._rw_quant import QK, Panic, QTensor, Weight, block_bytes, linear_w, matmul_t, matmul_t_q  # noqa: F401
