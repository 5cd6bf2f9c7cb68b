// pybind11 module `tinytorch_pybind`: the Node API of the reference bindings
// (reference src/bindings.cpp:54-150) rebuilt against the GPU backend.
//
// Same class, method names, argument names and defaults; a NULL from the C
// layer raises ValueError("tinytorch: invalid arguments or shape mismatch")
// and a wrong-length backward seed raises ValueError before any gradient is
// touched (reference src/bindings.cpp:22-30, 79-92).  value()/grad() return
// fresh NumPy copies of the device data, as the reference's do; with
// copy=False they return a view of the pinned host mirror instead.
// detach() re-enters a device-resident parameter into a new graph.  Additions of this backend:
// softmax_ce(labels), probs(), backward_device(seed_node), sgd_step(lr), the
// Optim class (SGD-momentum, Adam), the Dataset class (device-resident
// MNIST / CIFAR-10) and the module function available().
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstring>
#include <memory>
#include <vector>

#include "autograd.h"
#include "tensor.h"
#include "tt_data.h"
#include "tt_hip.h"

namespace py = pybind11;

namespace {

using Arr = py::array_t<float, py::array::c_style | py::array::forcecast>;

struct NodeRef {
  AGNode *p;
  explicit NodeRef(AGNode *n) : p(n) {}
  ~NodeRef() { if (p) ag_release(p); }
  NodeRef(const NodeRef &) = delete;
  NodeRef &operator=(const NodeRef &) = delete;
};

[[noreturn]] void bad() { throw py::value_error("tinytorch: invalid arguments or shape mismatch"); }

py::array_t<float> to_numpy(Tensor *t) {
  if (!t) return py::array_t<float>();
  const int nd = tt_ndim(t);
  std::vector<long> shp(nd);
  tt_shape(t, shp.data());
  std::vector<py::ssize_t> shape(shp.begin(), shp.end());
  const float *src = tt_data(t);
  if (!src) throw std::runtime_error("tinytorch: device to host copy failed");
  py::array_t<float> out(shape);
  std::memcpy(out.mutable_data(), src, sizeof(float) * (size_t)tt_numel(t));
  return out;
}

// Zero-copy form: a NumPy array over the tensor's pinned host mirror that
// keeps the tensor alive.  The mirror is refreshed in place by every later
// value()/grad()/tt_data() of the same tensor, and writes through the array
// reach the device before the tensor's next use (the host copy stays
// authoritative until then).
py::array_t<float> view_numpy(Tensor *t) {
  if (!t) return py::array_t<float>();
  const int nd = tt_ndim(t);
  std::vector<long> shp(nd);
  tt_shape(t, shp.data());
  std::vector<py::ssize_t> shape(shp.begin(), shp.end());
  float *src = tt_data(t);
  if (!src) throw std::runtime_error("tinytorch: device to host copy failed");
  tt_retain(t);
  py::capsule owner(t, [](void *p) { tt_release(static_cast<Tensor *>(p)); });
  return py::array_t<float>(shape, src, owner);
}

class PyNode {
 public:
  std::shared_ptr<NodeRef> ref;

  explicit PyNode(AGNode *n) {
    if (!n) bad();
    ref = std::make_shared<NodeRef>(n);
  }
  AGNode *get() const { return ref->p; }

  static PyNode leaf(Arr arr, bool requires_grad) {
    py::buffer_info info = arr.request();
    std::vector<long> shape(info.shape.begin(), info.shape.end());
    Tensor *t = tt_fromdata(static_cast<const float *>(info.ptr), shape.data(), (int)info.ndim);
    if (!t) bad();
    AGNode *n = ag_leaf(t, requires_grad ? 1 : 0);
    tt_release(t);  // the node holds its own reference
    return PyNode(n);
  }

  py::array_t<float> value(bool copy) const {
    return copy ? to_numpy(ag_value(get())) : view_numpy(ag_value(get()));
  }

  py::object grad(bool copy) const {
    Tensor *g = ag_grad(get());
    if (!g) return py::none();
    return copy ? to_numpy(g) : view_numpy(g);
  }

  // a new leaf around this node's value tensor (shared, not copied)
  PyNode detach(bool requires_grad) const {
    return PyNode(ag_leaf(ag_value(get()), requires_grad ? 1 : 0));
  }

  void backward(py::object seed) {
    if (seed.is_none()) {
      ag_backward(get());
      return;
    }
    Arr arr = seed.cast<Arr>();
    Tensor *v = ag_value(get());
    const long need = v ? tt_numel(v) : -1;
    if ((long)arr.size() != need) throw py::value_error("tinytorch: seed length mismatch");
    ag_backward_from(get(), arr.data(), (size_t)arr.size());
  }

  PyNode add(const PyNode &o) { return PyNode(ag_add(get(), o.get())); }
  PyNode mul(const PyNode &o) { return PyNode(ag_mul(get(), o.get())); }
  PyNode addscalar(float s) { return PyNode(ag_addscalar(get(), s)); }
  PyNode mulscalar(float s) { return PyNode(ag_mulscalar(get(), s)); }
  PyNode matmul(const PyNode &o) { return PyNode(ag_matmul(get(), o.get())); }
  PyNode relu() { return PyNode(ag_relu(get())); }
  PyNode softmax() { return PyNode(ag_softmax(get())); }
  PyNode padones() { return PyNode(ag_padones(get())); }
  PyNode reshape(std::vector<long> shape) {
    return PyNode(ag_reshape(get(), shape.data(), (int)shape.size()));
  }
  PyNode conv2d(const PyNode &w, py::object b, int sh, int sw, int ph, int pw) {
    AGNode *bp = b.is_none() ? nullptr : b.cast<PyNode &>().get();
    return PyNode(ag_conv2d(get(), w.get(), bp, sh, sw, ph, pw));
  }
  PyNode maxpool2d(int ph, int pw, int sh, int sw) { return PyNode(ag_maxpool2d(get(), ph, pw, sh, sw)); }
  PyNode avgpool2d(int ph, int pw, int sh, int sw) { return PyNode(ag_avgpool2d(get(), ph, pw, sh, sw)); }

  // ---- additions ----
  PyNode softmax_ce(py::array_t<int, py::array::c_style | py::array::forcecast> labels) {
    return PyNode(ag_softmax_ce(get(), labels.data(), (long)labels.size()));
  }
  py::object probs() const {
    Tensor *p = ag_softmax_ce_probs(get());
    if (!p) return py::none();
    return to_numpy(p);
  }
  void sgd_step(float lr) {
    if (ag_sgd_step(get(), lr) != 0) throw std::runtime_error("tinytorch: sgd step failed");
  }
};

// Optimizer with device-resident state; step() takes the parameter nodes in
// the same order every call (state slot i follows position i).
class PyOptim {
 public:
  std::shared_ptr<AGOptim> opt;
  explicit PyOptim(AGOptim *o) {
    if (!o) bad();
    opt.reset(o, ag_optim_release);
  }
  static PyOptim sgd_momentum(double lr, double momentum) {
    return PyOptim(ag_optim_sgd_momentum(lr, momentum));
  }
  static PyOptim adam(double lr, double b1, double b2, double eps) {
    return PyOptim(ag_optim_adam(lr, b1, b2, eps));
  }
  void step(const std::vector<PyNode> &params) {
    std::vector<AGNode *> ps;
    ps.reserve(params.size());
    for (const auto &p : params) ps.push_back(p.get());
    if (ag_optim_step(opt.get(), ps.data(), (int)ps.size()) != 0)
      throw py::value_error("tinytorch: optimizer step failed (parameter list or sizes changed?)");
  }
  long steps() const { return ag_optim_steps(opt.get()); }
  double lr() const { return ag_optim_lr(opt.get()); }
  void set_lr(double v) { ag_optim_set_lr(opt.get(), v); }
};

// Device-resident uint8 dataset; batch(idx) returns (leaf Node, labels).
class PyDataset {
 public:
  std::shared_ptr<TTDataset> d;
  std::vector<float> mean, stdv;
  PyDataset(TTDataset *p, std::vector<float> m, std::vector<float> s) : mean(m), stdv(s) {
    if (!p) throw py::value_error("tinytorch: dataset load failed (missing or malformed file?)");
    d.reset(p, tt_dataset_release);
    int c, h, w;
    tt_dataset_shape(p, &c, &h, &w);
    if ((int)mean.size() != c || (int)stdv.size() != c)
      throw py::value_error("tinytorch: mean/std need one value per channel");
  }
  static PyDataset mnist(const std::string &img, const std::string &lab, std::vector<float> m,
                         std::vector<float> s) {
    return PyDataset(tt_dataset_idx(img.c_str(), lab.c_str()), m, s);
  }
  static PyDataset cifar10(const std::vector<std::string> &paths, std::vector<float> m,
                           std::vector<float> s) {
    std::vector<const char *> ps;
    for (const auto &p : paths) ps.push_back(p.c_str());
    return PyDataset(tt_dataset_cifar10_bin(ps.data(), (int)ps.size()), m, s);
  }
  long len() const { return tt_dataset_len(d.get()); }
  py::tuple batch(py::array_t<long, py::array::c_style | py::array::forcecast> idx, bool flat,
                  bool requires_grad) {
    py::array_t<int32_t> lab(idx.size());
    Tensor *t = tt_dataset_batch(d.get(), idx.data(), (long)idx.size(), mean.data(), stdv.data(),
                                 flat ? 1 : 0, lab.mutable_data());
    if (!t) bad();
    AGNode *n = ag_leaf(t, requires_grad ? 1 : 0);
    tt_release(t);
    return py::make_tuple(PyNode(n), lab);
  }
};

}  // namespace

PYBIND11_MODULE(tinytorch_pybind, m) {
  m.doc() = "tinytorch autograd Node API on the MI355X (gfx950) backend";
  m.def("available", []() { return tth_available() == 1; });
  // waits for every queued kernel; raises when a launch (also one that an op
  // left pending) failed
  m.def("sync", []() {
    if (tth_sync() != 0) throw std::runtime_error("tinytorch: device work failed");
  });

  py::class_<PyNode>(m, "Node")
      .def_static("leaf", &PyNode::leaf, py::arg("arr"), py::arg("requires_grad") = true)
      .def("value", &PyNode::value, py::arg("copy") = true)
      .def("grad", &PyNode::grad, py::arg("copy") = true)
      .def("detach", &PyNode::detach, py::arg("requires_grad") = true)
      .def("backward", &PyNode::backward, py::arg("seed") = py::none())
      .def("add", &PyNode::add)
      .def("mul", &PyNode::mul)
      .def("addscalar", &PyNode::addscalar)
      .def("mulscalar", &PyNode::mulscalar)
      .def("matmul", &PyNode::matmul)
      .def("relu", &PyNode::relu)
      .def("softmax", &PyNode::softmax)
      .def("padones", &PyNode::padones)
      .def("reshape", &PyNode::reshape)
      .def("conv2d", &PyNode::conv2d, py::arg("w"), py::arg("b") = py::none(),
           py::arg("stride_h") = 1, py::arg("stride_w") = 1, py::arg("pad_h") = 0,
           py::arg("pad_w") = 0)
      .def("maxpool2d", &PyNode::maxpool2d, py::arg("pool_h") = 2, py::arg("pool_w") = 2,
           py::arg("stride_h") = 2, py::arg("stride_w") = 2)
      .def("avgpool2d", &PyNode::avgpool2d, py::arg("pool_h") = 2, py::arg("pool_w") = 2,
           py::arg("stride_h") = 2, py::arg("stride_w") = 2)
      .def("softmax_ce", &PyNode::softmax_ce, py::arg("labels"))
      .def("probs", &PyNode::probs)
      .def("sgd_step", &PyNode::sgd_step, py::arg("lr"))
      .def("__add__", &PyNode::add)
      .def("__mul__", &PyNode::mul);

  py::class_<PyDataset>(m, "Dataset")
      .def_static("mnist", &PyDataset::mnist, py::arg("images"), py::arg("labels"),
                  py::arg("mean") = std::vector<float>{0.1307f},
                  py::arg("std") = std::vector<float>{0.3081f})
      .def_static("cifar10", &PyDataset::cifar10, py::arg("paths"),
                  py::arg("mean") = std::vector<float>{0.4914f, 0.4822f, 0.4465f},
                  py::arg("std") = std::vector<float>{0.2023f, 0.1994f, 0.2010f})
      .def("__len__", &PyDataset::len)
      .def("batch", &PyDataset::batch, py::arg("idx"), py::arg("flat") = false,
           py::arg("requires_grad") = false);

  py::class_<PyOptim>(m, "Optim")
      .def_static("sgd_momentum", &PyOptim::sgd_momentum, py::arg("lr"), py::arg("momentum"))
      .def_static("adam", &PyOptim::adam, py::arg("lr") = 0.003, py::arg("beta1") = 0.9,
                  py::arg("beta2") = 0.999, py::arg("eps") = 1e-8)
      .def("step", &PyOptim::step, py::arg("params"))
      .def_property_readonly("t", &PyOptim::steps)
      .def_property("lr", &PyOptim::lr, &PyOptim::set_lr);
}
