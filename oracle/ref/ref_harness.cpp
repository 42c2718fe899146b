// Python binding of the reference's CPU ATen ops, for validating the oracle.
// TEST INFRASTRUCTURE ONLY.  Built by oracle/ref/build_ref.py from the
// reference's own grm/csrc/grm_cuda.cpp, compiled where it lies; outputs go
// to oracle/_ref/.  Binds the functions as plain Python functions (no
// TORCH_LIBRARY), so the module can be loaded next to grm_cuda_ext.  The GIL
// is released around each call, as the torch dispatcher does, because the
// reference's backward runs the autograd engine.
#include <torch/extension.h>

#include "grm_cuda.h"  // the reference's declarations (grm/csrc/grm_cuda.h)

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "reference CPU ops (grm/csrc/grm_cuda.cpp) for oracle validation";
  m.def("chunk_update_forward", &grm::chunk_update_forward, pybind11::call_guard<pybind11::gil_scoped_release>());
  m.def("chunk_update_backward", &grm::chunk_update_backward, pybind11::call_guard<pybind11::gil_scoped_release>());
  m.def("apply_query_forward", &grm::apply_query_forward, pybind11::call_guard<pybind11::gil_scoped_release>());
  m.def("apply_query_backward", &grm::apply_query_backward, pybind11::call_guard<pybind11::gil_scoped_release>());
  m.def("batched_memory_gather", &grm::batched_memory_gather, pybind11::call_guard<pybind11::gil_scoped_release>());
}
