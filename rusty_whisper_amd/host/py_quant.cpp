// py_quant.cpp -- pybind11 binding of the C++ mirror (module _rw_quant).
// numpy float32 arrays stand in for rw::Tensor in both directions.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "rw_quant.hpp"

namespace py = pybind11;

using F32 = py::array_t<float, py::array::c_style | py::array::forcecast>;
using U8 = py::array_t<uint8_t, py::array::c_style | py::array::forcecast>;

static rw::Tensor to_tensor(const F32 &a) {
  py::buffer_info b = a.request();
  std::vector<size_t> shape(b.shape.begin(), b.shape.end());
  const float *p = static_cast<const float *>(b.ptr);
  size_t n = 1;
  for (size_t s : shape) n *= s;
  return rw::Tensor{shape, std::vector<float>(p, p + n)};
}

static py::array_t<float> to_numpy(const rw::Tensor &t) {
  std::vector<py::ssize_t> shape(t.shape.begin(), t.shape.end());
  py::array_t<float> out(shape);
  if (!t.data.empty()) std::copy(t.data.begin(), t.data.end(), out.mutable_data());
  return out;
}

PYBIND11_MODULE(_rw_quant, m) {
  m.doc() = "C++ mirror of rusty_whisper src/quant.rs on the MI355X (librw_rocm.so)";
  m.attr("QK") = rw::QK;

  static py::exception<rw::Panic> panic(m, "Panic", PyExc_RuntimeError);
  py::register_exception_translator([](std::exception_ptr p) {
    try {
      if (p) std::rethrow_exception(p);
    } catch (const rw::Panic &e) {
      PyErr_SetObject(panic.ptr(), py::make_tuple(e.what(), e.code).ptr());
    }
  });

  m.def("block_bytes", &rw::block_bytes, py::arg("dtype"));

  py::class_<rw::QTensor>(m, "QTensor")
      .def(py::init([](std::vector<size_t> shape, int dtype, U8 raw) {
             py::buffer_info b = raw.request();
             const uint8_t *p = static_cast<const uint8_t *>(b.ptr);
             return new rw::QTensor(std::move(shape), dtype, std::vector<uint8_t>(p, p + b.size));
           }),
           py::arg("shape"), py::arg("dtype"), py::arg("raw"))
      .def_readonly("shape", &rw::QTensor::shape)
      .def_readonly("dtype", &rw::QTensor::dtype)
      .def_property_readonly("raw",
                             [](const rw::QTensor &q) {
                               return py::bytes(reinterpret_cast<const char *>(q.raw.data()), q.raw.size());
                             })
      .def("row_f32",
           [](const rw::QTensor &q, size_t i) {
             py::array_t<float> out(static_cast<py::ssize_t>(q.shape.at(1)));
             q.row_f32(i, out.mutable_data());
             return out;
           })
      .def("to_dense", [](const rw::QTensor &q) { return to_numpy(q.to_dense()); })
      .def("uploaded", [](const rw::QTensor &q) { return q.device() != nullptr; });

  py::class_<rw::Weight>(m, "Weight")
      .def_static("Dense", [](const F32 &t) { return rw::Weight::Dense(to_tensor(t)); })
      .def_static("Quant",
                  [](std::vector<size_t> shape, int dtype, U8 raw) {
                    py::buffer_info b = raw.request();
                    const uint8_t *p = static_cast<const uint8_t *>(b.ptr);
                    return rw::Weight::Quant(rw::QTensor(std::move(shape), dtype, std::vector<uint8_t>(p, p + b.size)));
                  })
      .def("shape", &rw::Weight::shape)
      .def("is_quant", &rw::Weight::is_quant)
      .def("dense", [](const rw::Weight &w) { return to_numpy(w.dense()); })
      .def("row_f32", [](const rw::Weight &w, size_t i) {
        py::array_t<float> out(static_cast<py::ssize_t>(w.shape().at(w.shape().size() - 1)));
        w.row_f32(i, out.mutable_data());
        return out;
      });

  // the device call runs without the GIL, so Python threads really overlap
  m.def(
      "matmul_t_q",
      [](const F32 &a, const rw::QTensor &b) {
        rw::Tensor x = to_tensor(a), y;
        {
          py::gil_scoped_release nogil;
          y = rw::matmul_t_q(x, b);
        }
        return to_numpy(y);
      },
      py::arg("a"), py::arg("b"));
  m.def(
      "matmul_t",
      [](const F32 &a, const F32 &b) {
        rw::Tensor x = to_tensor(a), w = to_tensor(b), y;
        {
          py::gil_scoped_release nogil;
          y = rw::matmul_t(x, w);
        }
        return to_numpy(y);
      },
      py::arg("a"), py::arg("b"));
  m.def(
      "linear_w",
      [](const F32 &x, const rw::Weight &w, std::optional<F32> b) {
        std::vector<float> bias;
        if (b) {
          py::buffer_info bi = b->request();
          const float *p = static_cast<const float *>(bi.ptr);
          bias.assign(p, p + bi.size);
        }
        rw::Tensor xt = to_tensor(x), y;
        {
          py::gil_scoped_release nogil;
          y = rw::linear_w(xt, w, b ? &bias : nullptr);
        }
        return to_numpy(y);
      },
      py::arg("x"), py::arg("w"), py::arg("b") = py::none());
}
