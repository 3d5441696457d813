// kaon_key.cpp -- the host side of a step's launch-cache check, as one native
// call (Python module _kaon_key, built by build_key.py).
//
// A step reuses a group's cached plans while nothing they were built from has
// changed: which params have a gradient, and the param and gradient storage,
// the gradient dtype, contiguity and layout.  Done in Python this takes five
// attribute or method calls per parameter (about 0.15 ms for the 512 tensors
// of a LoRA bag, more than the step's GPU time); here it is one pass over the
// list.
#include <torch/csrc/autograd/python_variable.h>
#include <torch/python.h>

#include <cstdint>
#include <cstring>
#include <string>

namespace py = pybind11;

namespace {

// One param's record in the key: two data pointers and three tag bytes.
constexpr size_t kRec = 2 * sizeof(uint64_t) + 3;

// group_key(params) -> (kept, key): `kept` lists the params whose .grad is set,
// in order; `key` holds, for each of them, the param's and the gradient's data
// pointers (0 for a sparse gradient) and the gradient's dtype, contiguity and
// sparsity.  Equal keys mean equal plans.  The list and the key are sized for
// every param up front and cut to the kept ones at the end; the gradient is
// read from the tensor's autograd slot directly (at::Tensor::grad() adds a
// non-leaf check, a third of the call's time for a bag of small tensors).
py::tuple group_key(py::handle params) {
  auto seq = py::reinterpret_steal<py::object>(PySequence_Fast(params.ptr(), "kaon_amd: params must be a sequence"));
  if (!seq) throw py::error_already_set();
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(seq.ptr());
  PyObject** items = PySequence_Fast_ITEMS(seq.ptr());
  auto kept = py::reinterpret_steal<py::list>(PyList_New(n));  // slots NULL until set
  if (!kept) throw py::error_already_set();
  std::string key((size_t)n * kRec, '\0');
  char* out = &key[0];
  Py_ssize_t nk = 0;
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* o = items[i];
    if (!THPVariable_Check(o)) throw py::type_error("kaon_amd: optimizer params must be tensors");
    const at::Tensor& p = THPVariable_Unpack(o);
    const at::Tensor& g = p.unsafeGetTensorImpl()->grad();
    if (!g.defined()) continue;
    Py_INCREF(o);
    PyList_SET_ITEM(kept.ptr(), nk++, o);
    const bool sparse = g.is_sparse();
    const uint64_t ptr[2] = {(uint64_t)(uintptr_t)p.data_ptr(), sparse ? 0u : (uint64_t)(uintptr_t)g.data_ptr()};
    const char tag[3] = {(char)g.scalar_type(), (char)(!sparse && g.is_contiguous()), (char)sparse};
    std::memcpy(out, ptr, sizeof ptr);
    std::memcpy(out + sizeof ptr, tag, sizeof tag);
    out += kRec;
  }
  key.resize((size_t)nk * kRec);
  // drop the unused (NULL) slots
  if (nk < n && PyList_SetSlice(kept.ptr(), nk, n, nullptr) != 0) throw py::error_already_set();
  return py::make_tuple(kept, py::bytes(key));
}

}  // namespace

PYBIND11_MODULE(_kaon_key, m) {
  m.doc() = "kaon_amd: the launch-cache key of a parameter group";
  m.def("group_key", &group_key, "(params) -> (params with a grad, key bytes)");
}
