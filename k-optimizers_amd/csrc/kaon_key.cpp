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
#include <string>

namespace py = pybind11;

namespace {

// group_key(params) -> (kept, key): `kept` lists the params whose .grad is set,
// in order; `key` holds, for each of them, the param's and the gradient's data
// pointers (0 for a sparse gradient) and the gradient's dtype, contiguity and
// sparsity.  Equal keys mean equal plans.
py::tuple group_key(py::handle params) {
  std::string key;
  py::list kept;
  for (py::handle h : params) {
    PyObject* o = h.ptr();
    if (!THPVariable_Check(o)) throw py::type_error("kaon_amd: optimizer params must be tensors");
    const at::Tensor& p = THPVariable_Unpack(o);
    const at::Tensor& g = p.grad();
    if (!g.defined()) continue;
    kept.append(h);
    const bool sparse = g.is_sparse();
    const uint64_t ptr[2] = {(uint64_t)(uintptr_t)p.data_ptr(), sparse ? 0u : (uint64_t)(uintptr_t)g.data_ptr()};
    const char tag[3] = {(char)g.scalar_type(), (char)(!sparse && g.is_contiguous()), (char)sparse};
    key.append(reinterpret_cast<const char*>(ptr), sizeof ptr);
    key.append(tag, sizeof tag);
  }
  return py::make_tuple(kept, py::bytes(key));
}

}  // namespace

PYBIND11_MODULE(_kaon_key, m) {
  m.doc() = "kaon_amd: the launch-cache key of a parameter group";
  m.def("group_key", &group_key, "(params) -> (params with a grad, key bytes)");
}
