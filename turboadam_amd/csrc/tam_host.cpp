// tam_host.cpp -- the per-parameter host work of a steady TurboAdam step, in
// C++ (a torch extension module, _tam_host).
//
// A steady step (turboadam_amd/optimizer.py, _FastStep) reuses the descriptor
// table of the previous step and rewrites only what changes: each row's
// gradient pointer and step number.  Before it may, it checks that the step is
// in fact steady: the same parameters have gradients, each parameter still
// has the storage its row points at, each new gradient object is a dense,
// contiguous tensor of its parameter's dtype on the step's device, and each
// row's state tensors are the objects the row was built from.  Doing this per
// row in Python costs about a microsecond per parameter; here it is a few
// dictionary lookups and pointer comparisons.
//
// steady_rows() returns False, with nothing written, when any check fails
// (the optimizer then takes its full path, which validates and raises where
// something is wrong); advance_steps() adds 1 to each state's step counter
// once the step has been launched.
#include <torch/extension.h>

#include <cstdint>
#include <cstring>

namespace py = pybind11;

namespace {

// Borrowed item of a dict by an interned key, or nullptr (no exception set).
PyObject* item(PyObject* d, PyObject* key) {
  if (!PyDict_Check(d)) return nullptr;
  return PyDict_GetItemWithError(d, key);
}

struct Keys {
  PyObject *grad, *compressed_v, *indices, *scales, *exp_avg_sq, *exp_avg, *compress_m, *m_mgr, *encoded,
      *sign_packed, *labels, *block_norms, *alpha, *ef_residual, *step;
  Keys() {
    grad = PyUnicode_InternFromString("grad");
    compressed_v = PyUnicode_InternFromString("compressed_v");
    indices = PyUnicode_InternFromString("indices");
    scales = PyUnicode_InternFromString("scales");
    exp_avg_sq = PyUnicode_InternFromString("exp_avg_sq");
    exp_avg = PyUnicode_InternFromString("exp_avg");
    compress_m = PyUnicode_InternFromString("_compress_m");
    m_mgr = PyUnicode_InternFromString("m_mgr");
    encoded = PyUnicode_InternFromString("_encoded");
    sign_packed = PyUnicode_InternFromString("sign_packed");
    labels = PyUnicode_InternFromString("labels");
    block_norms = PyUnicode_InternFromString("block_norms");
    alpha = PyUnicode_InternFromString("_alpha");
    ef_residual = PyUnicode_InternFromString("_ef_residual");
    step = PyUnicode_InternFromString("step");
  }
};

const Keys& keys() {
  static const Keys k;
  return k;
}

// Whether the state tensors of one row are, in order, the kept objects at
// kept[*pos ...] (the order of optimizer._row_tensors); advances *pos.
bool row_tensors_kept(PyObject* st, bool compress_v, PyObject* kept, Py_ssize_t n_kept, Py_ssize_t* pos) {
  const Keys& K = keys();
  PyObject* got[8];
  int n = 0;
  if (compress_v) {
    PyObject* cv = item(st, K.compressed_v);
    if (!cv) return false;
    got[n++] = item(cv, K.indices);
    got[n++] = item(cv, K.scales);
  } else {
    got[n++] = item(st, K.exp_avg_sq);
  }
  PyObject* cm = item(st, K.compress_m);
  if (!cm) return false;
  const int costate = PyObject_IsTrue(cm);
  if (costate < 0) return false;
  if (costate) {
    PyObject* mgr = item(st, K.m_mgr);
    if (!mgr) return false;
    // the manager's attributes from its instance dict (an attribute held
    // elsewhere is not found: the step is then not taken as steady)
    PyObject* md = PyObject_GenericGetDict(mgr, nullptr);  // new reference
    if (!md) return false;
    PyObject* enc = item(md, K.encoded);
    PyObject* a = item(md, K.alpha);
    PyObject* r = item(md, K.ef_residual);
    Py_DECREF(md);  // the manager keeps its dict and the objects alive
    if (!enc || !a || !r) return false;
    got[n++] = item(enc, K.sign_packed);
    got[n++] = item(enc, K.labels);
    got[n++] = item(enc, K.block_norms);
    got[n++] = item(enc, K.scales);
    got[n++] = a;  // identity only
    got[n++] = r;
  } else {
    got[n++] = item(st, K.exp_avg);
  }
  for (int i = 0; i < n; ++i) {
    if (!got[i] || *pos >= n_kept) return false;
    // None in the kept list stands for a missing error-feedback residual
    if (PyList_GET_ITEM(kept, *pos) != got[i]) return false;
    ++*pos;
  }
  return true;
}

// Whether every row's state tensors are the kept objects (lists: the rows'
// state dicts, their compress_v flags, the kept tensors flattened).
bool all_rows_kept(PyObject* S, PyObject* CV, PyObject* T) {
  if (!PyList_Check(S) || !PyList_Check(CV) || !PyList_Check(T) || PyList_GET_SIZE(S) != PyList_GET_SIZE(CV))
    return false;
  Py_ssize_t pos = 0;
  const Py_ssize_t n_kept = PyList_GET_SIZE(T);
  for (Py_ssize_t j = 0; j < PyList_GET_SIZE(S); ++j) {
    if (!row_tensors_kept(PyList_GET_ITEM(S, j), PyList_GET_ITEM(CV, j) == Py_True, T, n_kept, &pos)) {
      PyErr_Clear();
      return false;
    }
  }
  return pos == n_kept;
}

}  // namespace

// Whether the rows' state tensors of the kept _FastStep f are still the
// objects its descriptor rows were built from.
bool states_kept(py::handle f) {
  py::object states = f.attr("states"), tensors = f.attr("tensors"), row_cv = f.attr("plan").attr("row_cv");
  return all_rows_kept(states.ptr(), row_cv.ptr(), tensors.ptr());
}

// The per-row part of a steady step (optimizer.TurboAdam._fast_step), given
// the kept _FastStep f and the descriptor table's memory (table_addr, row
// stride, byte offsets of the uint64 gradient pointer and the uint32 step
// fields).  On success the gradient pointers and step numbers of every row
// are written and f.grads holds this step's gradient objects.
bool steady_rows(py::handle f, uint64_t table_addr, int64_t stride, int64_t grad_off, int64_t step_off) {
  if (PyErr_Occurred()) return false;
  const Keys& K = keys();
  bool ok = false;
  // every attribute of f read once (new references, released on return)
  py::object params = f.attr("params"), absent = f.attr("absent"), rows = f.attr("rows"),
             row_params = f.attr("row_params"), ptrs = f.attr("ptrs"), kept_grads = f.attr("grads"),
             pdtypes = f.attr("pcodes"), states = f.attr("states"), tensors = f.attr("tensors"),
             row_cv = f.attr("plan").attr("row_cv");
  const int64_t dev_index = f.attr("dev_index").cast<int64_t>();
  PyObject* P = params.ptr();
  PyObject* A = absent.ptr();
  PyObject* R = rows.ptr();
  PyObject* RP = row_params.ptr();
  PyObject* PT = ptrs.ptr();
  PyObject* KG = kept_grads.ptr();
  PyObject* PD = pdtypes.ptr();
  PyObject* S = states.ptr();
  PyObject* T = tensors.ptr();
  PyObject* CV = row_cv.ptr();
  if (!PyList_Check(P) || !PyList_Check(A) || !PyList_Check(R) || !PyList_Check(RP) || !PyList_Check(PT) ||
      !PyList_Check(KG) || !PyList_Check(PD) || !PyList_Check(S) || !PyList_Check(T) || !PyList_Check(CV))
    return false;
  const Py_ssize_t np_ = PyList_GET_SIZE(P), nr = PyList_GET_SIZE(R);
  if (PyList_GET_SIZE(A) != np_ || PyList_GET_SIZE(RP) != nr || PyList_GET_SIZE(PT) != nr ||
      PyList_GET_SIZE(KG) != nr || PyList_GET_SIZE(PD) != nr || PyList_GET_SIZE(S) != nr ||
      PyList_GET_SIZE(CV) != nr)
    return false;
  if (!all_rows_kept(S, CV, T)) return false;
  std::vector<PyObject*> gs((size_t)np_, nullptr);  // new references
  auto release = [&]() {
    for (PyObject* g : gs) Py_XDECREF(g);
  };
  // the same parameters have gradients
  for (Py_ssize_t i = 0; i < np_; ++i) {
    PyObject* g = PyObject_GetAttr(PyList_GET_ITEM(P, i), K.grad);
    if (!g) {
      PyErr_Clear();
      release();
      return false;
    }
    gs[(size_t)i] = g;
    if ((g == Py_None) != (PyList_GET_ITEM(A, i) == Py_True)) {
      release();
      return false;
    }
  }
  // per row: parameter dtype and storage, gradient object
  std::vector<uint64_t> gptr((size_t)nr);
  for (Py_ssize_t j = 0; j < nr; ++j) {
    const Py_ssize_t i = PyLong_AsSsize_t(PyList_GET_ITEM(R, j));
    if (i < 0 || i >= np_) {
      PyErr_Clear();
      release();
      return false;
    }
    PyObject* p = PyList_GET_ITEM(RP, j);
    if (!THPVariable_Check(p)) {
      release();
      return false;
    }
    const at::Tensor& pt = THPVariable_Unpack(p);
    // the row was built for this dtype (TAM_DTYPE_F32 / BF16 / F16) and storage
    const long code = PyLong_AsLong(PyList_GET_ITEM(PD, j));
    const at::ScalarType want = code == 0 ? at::kFloat : code == 1 ? at::kBFloat16 : at::kHalf;
    if (pt.scalar_type() != want ||
        (uint64_t)(uintptr_t)pt.data_ptr() != PyLong_AsUnsignedLongLong(PyList_GET_ITEM(PT, j))) {
      PyErr_Clear();
      release();
      return false;
    }
    PyObject* g = gs[(size_t)i];
    if (!THPVariable_Check(g)) {
      release();
      return false;
    }
    const at::Tensor& gt = THPVariable_Unpack(g);
    if (g != PyList_GET_ITEM(KG, j)) {  // a new gradient object: the checks of _grad_ptr
      if (gt.scalar_type() != pt.scalar_type() || gt.layout() != at::kStrided || !gt.is_contiguous() ||
          !gt.is_cuda() || gt.get_device() != dev_index) {
        release();
        return false;
      }
    }
    gptr[(size_t)j] = (uint64_t)(uintptr_t)gt.data_ptr();
  }
  // steady: write the rows' gradient pointers and step numbers
  char* base = (char*)(uintptr_t)table_addr;
  for (Py_ssize_t j = 0; j < nr; ++j) {
    PyObject* stp = item(PyList_GET_ITEM(S, j), K.step);
    const long long s = stp ? PyLong_AsLongLong(stp) : -1;
    if (!stp || s < 0) {
      PyErr_Clear();
      release();
      return false;
    }
    char* row = base + j * stride;
    std::memcpy(row + grad_off, &gptr[(size_t)j], 8);
    const uint32_t s1 = (uint32_t)(s + 1);
    std::memcpy(row + step_off, &s1, 4);
  }
  // f.grads holds this step's gradient objects (checked from now on by identity)
  for (Py_ssize_t j = 0; j < nr; ++j) {
    PyObject* g = gs[(size_t)PyLong_AsSsize_t(PyList_GET_ITEM(R, j))];
    Py_INCREF(g);
    PyList_SetItem(KG, j, g);  // steals the new reference
  }
  ok = true;
  release();
  return ok;
}

// state["step"] += 1 for each state dict (once the step has been launched).
void advance_steps(py::list states) {
  const Keys& K = keys();
  for (py::handle st : states) {
    PyObject* s = item(st.ptr(), K.step);
    if (!s) throw py::key_error("step");
    PyObject* one = PyLong_FromLong(1);
    PyObject* s1 = PyNumber_Add(s, one);
    Py_DECREF(one);
    if (!s1 || PyDict_SetItem(st.ptr(), K.step, s1) != 0) {
      Py_XDECREF(s1);
      throw py::error_already_set();
    }
    Py_DECREF(s1);
  }
}

PYBIND11_MODULE(_tam_host, m) {
  m.doc() = "Host side of a steady TurboAdam step (turboadam_amd.optimizer)";
  m.def("steady_rows", &steady_rows, py::arg("f"), py::arg("table_addr"), py::arg("stride"), py::arg("grad_off"),
        py::arg("step_off"));
  m.def("advance_steps", &advance_steps, py::arg("states"));
  m.def("states_kept", &states_kept, py::arg("f"));
}
