// rw_quant.hpp -- C++ mirror of rusty_whisper's quantized-weight API
// (src/quant.rs), running on the MI355X through the C ABI of rw_rocm.h.
//
// Same names, argument meanings and failure conditions as the reference:
//   QK, block_bytes            src/quant.rs:17, 43-52
//   Tensor                     src/tensor.rs:7-41
//   QTensor                    src/quant.rs:495-640 (new, row_f32, to_dense)
//   Weight                     src/quant.rs:643-675
//   matmul_t_q                 src/quant.rs:754-1051
//   matmul_t                   src/tensor.rs:194-238 (the dense f32 tier)
//   linear_w                   src/quant.rs:1054-1063
// Where the reference panics (assert!/panic!), this mirror throws rw::Panic
// with the same message.  A QTensor uploads its blocks to the device once, on
// first use, guarded like the reference's OnceLock caches; concurrent callers
// may share one QTensor.
#pragma once

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <string>
#include <variant>
#include <vector>

#include "rw_rocm.h"

namespace rw {

constexpr size_t QK = 32;

// The reference's panic!/assert! at the same call sites.
struct Panic : std::logic_error {
  explicit Panic(const std::string &what, int code = 0) : std::logic_error(what), code(code) {}
  int code;  // RW_E* status when the failure came from the device library
};

// src/quant.rs:43-52
std::optional<size_t> block_bytes(int dtype);

// src/tensor.rs:7-41: row-major f32, element (r, c) at r * cols + c
struct Tensor {
  std::vector<size_t> shape;
  std::vector<float> data;

  static Tensor zeros(const std::vector<size_t> &shape);
  static Tensor from_vec(const std::vector<size_t> &shape, std::vector<float> data);
  size_t rows() const { return shape.at(0); }
  size_t cols() const { return shape.at(shape.size() - 1); }
};

// src/quant.rs:495-640: a [rows, cols] matrix kept in ggml blocks.
class QTensor {
 public:
  QTensor(std::vector<size_t> shape, int dtype, std::vector<uint8_t> raw);
  ~QTensor();
  QTensor(const QTensor &) = delete;
  QTensor &operator=(const QTensor &) = delete;
  QTensor(QTensor &&other) noexcept;

  std::vector<size_t> shape;
  int dtype;
  std::vector<uint8_t> raw;

  // Dequantize row i into out (shape[1] floats); src/quant.rs:566-570
  void row_f32(size_t i, float *out) const;
  // The whole matrix as f32; src/quant.rs:572-576
  Tensor to_dense() const;
  // The resident device copy, uploaded on first use (throws Panic on failure)
  const rw_weight *device() const;

 private:
  mutable std::once_flag once_;
  mutable rw_weight *dev_ = nullptr;
  mutable int status_ = 0;
  mutable std::string error_;
};

// src/quant.rs:643-675
class Weight {
 public:
  static Weight Dense(Tensor t);
  static Weight Quant(QTensor q);
  const std::vector<size_t> &shape() const;
  bool is_quant() const { return v_.index() == 1; }
  // the dense tensor; panics for a quantized weight (src/quant.rs:658-663)
  const Tensor &dense() const;
  const QTensor &quant() const;
  // embedding gather (src/quant.rs:666-674)
  void row_f32(size_t i, float *out) const;

 private:
  explicit Weight(std::variant<Tensor, QTensor> v) : v_(std::move(v)) {}
  std::variant<Tensor, QTensor> v_;
};

// C = A[m,k] x B^T with B quantized [n,k]; src/quant.rs:754-1051
Tensor matmul_t_q(const Tensor &a, const QTensor &b);

// C = A[m,k] x B^T with B dense f32 [n,k]; src/tensor.rs:194-238, on the
// device, bit-identical to the reference (tensor::dot's order and roundings)
Tensor matmul_t(const Tensor &a, const Tensor &b);

// y = x W^T + b; src/quant.rs:1054-1063.  Both arms run on the device: Quant
// through matmul_t_q, Dense through matmul_t; the bias is added as add_bias
// does (src/tensor.rs:262-272).
Tensor linear_w(const Tensor &x, const Weight &w, const std::vector<float> *b);

}  // namespace rw
