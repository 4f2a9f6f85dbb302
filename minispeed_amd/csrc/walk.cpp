// Host-side pointer walk for the boundary's segment tables.
//
// At every boundary the engine needs the device address of each parameter's
// gradient (K1 / K3 read them) and of each parameter's storage (K3 writes the
// model copy there).  Done attribute by attribute from Python this costs
// ~0.3 us per tensor before K1 can launch; here it is one call per group.
//
// Both functions take the group's parameters and only look at tensor
// metadata.  They never raise for a bad tensor: they return the index of the
// first parameter that is not on the fast path (wrong dtype, size, device or
// layout), and the caller re-walks from there in Python, which raises the
// precise error or makes the contiguous copy.  Everything on the fast path is
// exactly what the Python walk would have accepted.

#include <torch/csrc/autograd/python_variable.h>
#include <torch/csrc/utils/pybind.h>
#include <pybind11/numpy.h>

#include <c10/core/Stream.h>

#include <cstdint>

namespace py = pybind11;

namespace {

at::Tensor unpack(PyObject* obj) {
  if (!THPVariable_Check(obj)) {
    throw py::type_error("expected a torch.Tensor / nn.Parameter");
  }
  return THPVariable_Unpack(obj);
}

bool on_fast_path(const at::Tensor& t, at::ScalarType dtype, int64_t numel, int64_t device_index) {
  return t.scalar_type() == dtype && t.numel() == numel && t.is_cuda() &&
         t.get_device() == device_index && t.is_contiguous();
}

// grad_pointers(params, numels, device_index, out) -> (bad, keep)
//   out[k]  : data_ptr of params[k].grad, 0 when it has none
//   keep[k] : params[k].grad (None when it has none), to hold the storage
//             until the kernels reading it are queued
//   bad     : -1, or the first k whose gradient needs the slow path (then
//             out and keep cover indices < bad only)
py::tuple grad_pointers(py::list params, py::array_t<int64_t, py::array::c_style> numels,
                        int64_t device_index, py::array_t<int64_t, py::array::c_style> out) {
  const Py_ssize_t n = PyList_GET_SIZE(params.ptr());
  if (numels.size() != n || out.size() < n) {
    throw py::value_error("numels / out must have one entry per parameter");
  }
  const int64_t* num = numels.data();
  int64_t* dst = out.mutable_data();
  py::list keep;
  if (n == 0) return py::make_tuple(-1, keep);
  const at::ScalarType dtype = unpack(PyList_GET_ITEM(params.ptr(), 0)).scalar_type();
  for (Py_ssize_t k = 0; k < n; ++k) {
    const at::Tensor p = unpack(PyList_GET_ITEM(params.ptr(), k));
    const at::Tensor& g = p.grad();
    if (!g.defined()) {
      dst[k] = 0;
      keep.append(py::none());
      continue;
    }
    if (!on_fast_path(g, dtype, num[k], device_index)) {
      return py::make_tuple(static_cast<int64_t>(k), keep);
    }
    dst[k] = reinterpret_cast<int64_t>(g.data_ptr());
    keep.append(py::reinterpret_steal<py::object>(THPVariable_Wrap(g)));
  }
  return py::make_tuple(-1, keep);
}

// model_pointers(params, device_index, out) -> bad
//   out[k] : data_ptr of params[k] (the cast target), all of the group dtype
//            (params[0]'s), contiguous and on the device
//   bad    : -1, or the first k that is not
int64_t model_pointers(py::list params, int64_t device_index,
                       py::array_t<int64_t, py::array::c_style> out) {
  const Py_ssize_t n = PyList_GET_SIZE(params.ptr());
  if (out.size() < n) throw py::value_error("out must have one entry per parameter");
  int64_t* dst = out.mutable_data();
  if (n == 0) return -1;
  const at::ScalarType dtype = unpack(PyList_GET_ITEM(params.ptr(), 0)).scalar_type();
  for (Py_ssize_t k = 0; k < n; ++k) {
    const at::Tensor p = unpack(PyList_GET_ITEM(params.ptr(), k));
    if (!(p.scalar_type() == dtype && p.is_cuda() && p.get_device() == device_index &&
          p.is_contiguous())) {
      return static_cast<int64_t>(k);
    }
    dst[k] = reinterpret_cast<int64_t>(p.data_ptr());
  }
  return -1;
}

// record_streams(tensors, device_type, device_index, stream_id) -> count
//   Tensor.record_stream(stream) for every device tensor of `tensors` (None
//   entries and host tensors are skipped): the caching allocator then hands
//   their memory out again only after the work queued on that stream by the
//   time they are freed.  One call instead of one Python call per tensor
//   (~0.3 us each) at every boundary.
int64_t record_streams(py::list tensors, int64_t device_type, int64_t device_index,
                       int64_t stream_id) {
  const c10::Stream stream(c10::Stream::UNSAFE,
                           c10::Device(static_cast<c10::DeviceType>(device_type),
                                       static_cast<c10::DeviceIndex>(device_index)),
                           static_cast<c10::StreamId>(stream_id));
  int64_t count = 0;
  const Py_ssize_t n = PyList_GET_SIZE(tensors.ptr());
  for (Py_ssize_t k = 0; k < n; ++k) {
    PyObject* obj = PyList_GET_ITEM(tensors.ptr(), k);
    if (obj == Py_None) continue;
    const at::Tensor t = unpack(obj);
    if (!t.is_cuda()) continue;
    t.record_stream(stream);
    ++count;
  }
  return count;
}

}  // namespace

PYBIND11_MODULE(_walk, m) {
  m.doc() = "device addresses of parameter gradients / storages for the boundary tables";
  m.def("grad_pointers", &grad_pointers);
  m.def("model_pointers", &model_pointers);
  m.def("record_streams", &record_streams);
}
