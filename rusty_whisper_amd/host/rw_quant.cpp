// rw_quant.cpp -- the C++ mirror of src/quant.rs over librw_rocm.so.
#include "rw_quant.hpp"

#include <utility>

namespace rw {

static std::string last_error() {
  char buf[1024];
  rw_rocm_last_error(buf, sizeof buf);
  return buf;
}

static void check(int rc, const char *what) {
  if (rc < 0) throw Panic(std::string(what) + ": " + last_error(), rc);
}

std::optional<size_t> block_bytes(int dtype) {
  switch (dtype) {
    case RW_Q4_0: return 18;
    case RW_Q4_1: return 20;
    case RW_Q5_0: return 22;
    case RW_Q5_1: return 24;
    case RW_Q8_0: return 34;
    default: return std::nullopt;
  }
}

static size_t product(const std::vector<size_t> &shape) {
  size_t n = 1;
  for (size_t s : shape) n *= s;
  return n;
}

Tensor Tensor::zeros(const std::vector<size_t> &shape) { return Tensor{shape, std::vector<float>(product(shape))}; }

Tensor Tensor::from_vec(const std::vector<size_t> &shape, std::vector<float> data) {
  if (product(shape) != data.size()) throw Panic("shape/data mismatch");  // tensor.rs:23-27
  return Tensor{shape, std::move(data)};
}

QTensor::QTensor(std::vector<size_t> shape_, int dtype_, std::vector<uint8_t> raw_)
    : shape(std::move(shape_)), dtype(dtype_), raw(std::move(raw_)) {}

QTensor::QTensor(QTensor &&o) noexcept : shape(std::move(o.shape)), dtype(o.dtype), raw(std::move(o.raw)) {
  // a moved-from tensor that was already uploaded hands over its device copy
  dev_ = o.dev_;
  status_ = o.status_;
  error_ = std::move(o.error_);
  if (dev_) std::call_once(once_, [] {});
  o.dev_ = nullptr;
}

QTensor::~QTensor() {
  if (dev_) rw_rocm_weight_free(dev_);
}

const rw_weight *QTensor::device() const {
  std::call_once(once_, [this] {
    if (shape.size() != 2) {
      status_ = RW_EINVAL;
      error_ = "a quantized weight must be 2-D";
      return;
    }
    rw_weight *w = nullptr;
    status_ = rw_rocm_weight_upload(dtype, shape[0], shape[1], raw.data(), raw.size(), &w);
    if (status_ < 0)
      error_ = last_error();
    else
      dev_ = w;
  });
  if (status_ < 0) throw Panic("QTensor upload: " + error_, status_);
  return dev_;
}

void QTensor::row_f32(size_t i, float *out) const {
  if (i >= shape.at(0)) throw Panic("row index out of range");
  check(rw_rocm_dequant_rows(device(), i, 1, out), "row_f32");
}

Tensor QTensor::to_dense() const {
  Tensor t = Tensor::zeros(shape);
  check(rw_rocm_dequant_rows(device(), 0, shape.at(0), t.data.data()), "to_dense");
  return t;
}

Weight Weight::Dense(Tensor t) { return Weight(std::variant<Tensor, QTensor>(std::in_place_index<0>, std::move(t))); }

Weight Weight::Quant(QTensor q) { return Weight(std::variant<Tensor, QTensor>(std::in_place_index<1>, std::move(q))); }

const std::vector<size_t> &Weight::shape() const {
  return v_.index() == 0 ? std::get<0>(v_).shape : std::get<1>(v_).shape;
}

const Tensor &Weight::dense() const {
  if (v_.index() != 0) throw Panic("expected dense weight, found quantized");
  return std::get<0>(v_);
}

const QTensor &Weight::quant() const {
  if (v_.index() != 1) throw Panic("expected quantized weight, found dense");
  return std::get<1>(v_);
}

void Weight::row_f32(size_t i, float *out) const {
  if (v_.index() == 0) {
    const Tensor &t = std::get<0>(v_);
    size_t k = t.cols();
    std::copy(t.data.begin() + i * k, t.data.begin() + (i + 1) * k, out);
  } else {
    std::get<1>(v_).row_f32(i, out);
  }
}

Tensor matmul_t_q(const Tensor &a, const QTensor &b) {
  size_t m = a.shape.at(0), k = a.shape.at(1);
  size_t n = b.shape.at(0), k2 = b.shape.at(1);
  if (k != k2)  // quant.rs:757
    throw Panic("matmul_t_q inner dims: " + std::to_string(k) + " vs " + std::to_string(k2));
  if (k % QK)  // quant.rs:758
    throw Panic("k must be a multiple of " + std::to_string(QK));
  Tensor out = Tensor::zeros({m, n});
  if (m == 0) return out;
  check(rw_rocm_matmul_t_q(b.device(), a.data.data(), m, k, nullptr, out.data.data()), "matmul_t_q");
  return out;
}

// tensor::matmul_t (src/tensor.rs:194-238) with linear_w's optional bias
static Tensor dense_product(const Tensor &a, const Tensor &b, const std::vector<float> *bias, const char *what) {
  if (a.shape.size() != 2 || b.shape.size() != 2) throw Panic("matmul_t takes 2-D tensors");
  size_t m = a.shape[0], k = a.shape[1], n = b.shape[0];
  if (k != b.shape[1])  // tensor.rs:200
    throw Panic("matmul_t inner dims: " + std::to_string(k) + " vs " + std::to_string(b.shape[1]));
  if (bias && bias->size() != n)  // tensor.rs:266 (add_bias asserts cols == bias.len())
    throw Panic("bias length " + std::to_string(bias->size()) + " != " + std::to_string(n));
  Tensor out = Tensor::zeros({m, n});
  if (m == 0) return out;
  check(rw_rocm_matmul_t_f32(a.data.data(), m, k, b.data.data(), n, bias ? bias->data() : nullptr,
                             out.data.data()),
        what);
  return out;
}

Tensor matmul_t(const Tensor &a, const Tensor &b) { return dense_product(a, b, nullptr, "matmul_t"); }

Tensor linear_w(const Tensor &x, const Weight &w, const std::vector<float> *b) {
  if (!w.is_quant()) return dense_product(x, w.dense(), b, "linear_w");
  const QTensor &q = w.quant();
  size_t m = x.shape.at(0), k = x.shape.at(1);
  size_t n = q.shape.at(0);
  if (k != q.shape.at(1))
    throw Panic("matmul_t_q inner dims: " + std::to_string(k) + " vs " + std::to_string(q.shape.at(1)));
  if (k % QK) throw Panic("k must be a multiple of " + std::to_string(QK));
  if (b && b->size() != n)  // tensor.rs:266 (add_bias asserts cols == bias.len())
    throw Panic("bias length " + std::to_string(b->size()) + " != " + std::to_string(n));
  Tensor out = Tensor::zeros({m, n});
  if (m == 0) return out;
  check(rw_rocm_matmul_t_q(q.device(), x.data.data(), m, k, b ? b->data() : nullptr, out.data.data()),
        "linear_w");
  return out;
}

}  // namespace rw
