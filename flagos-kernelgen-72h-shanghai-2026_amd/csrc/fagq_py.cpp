// fagq_py.cpp - CPython binding of the operator's per-call path.
//
// The Python operator (ops.fused_add_rmsnorm_group_quant, the drop-in for
// src/task01_fused_add_rmsnorm_group_quant.py:1731-1741) spends most of a
// decode-sized call on the host: some 30 tensor attribute reads in Python and
// a 16-argument ctypes call cost about 5 us against a 3 us kernel.  This
// module does the same checks on the tensors' C++ metadata and calls
// fagq_launch (bf16 tensors) or fagq_launch_typed (fp16 activations or an
// fp32 residual stream; include/fagq.h) through function pointers handed
// over from the ctypes binding at import, so both bindings reach the one
// library.
//
//   launch(x, residual, gamma, residual_out, norm_out, x_q, x_scale, eps,
//          group_size, rounding, stream) -> int
//     rounding: -1 = the format's default (fp8 RNE, int8 truncation),
//               0 = RNE, 1 = truncation, anything else = invalid.
//     Returns fagq_launch's status, or kArgError when a tensor argument is
//     rejected here (the Python layer then raises its detailed error).
//     The caller passes the current stream of the tensors' device and has
//     made that device current.
//
// No device work happens here and nothing is allocated: the launch is
// fagq_launch's.
#include <Python.h>

#include <torch/csrc/autograd/python_variable.h>

#include <cstdint>

#include "fagq.h"

namespace {

constexpr int kArgError = 1000;

using LaunchFn = int (*)(const void*, const void*, const void*, void*, void*, void*, void*, int64_t,
                         int64_t, int64_t, float, int, int, int, int, void*);
using TypedLaunchFn = int (*)(const void*, const void*, const void*, void*, void*, void*, void*,
                              int64_t, int64_t, int64_t, float, int, int, int, int, int, int,
                              void*);
LaunchFn g_launch = nullptr;
TypedLaunchFn g_launch_typed = nullptr;

bool is_tensor(PyObject* o) { return THPVariable_Check(o); }

// A contiguous tensor of element type `st` and `shape` on CUDA device `dev`.
bool rows_ok(const at::Tensor& t, at::IntArrayRef shape, c10::DeviceIndex dev,
             at::ScalarType st) {
  return t.scalar_type() == st && t.sizes() == shape && t.is_cuda() && t.get_device() == dev &&
         t.is_contiguous();
}

// fagq_dtype code of an element type, -1 for others.
int dtype_code(at::ScalarType st) {
  switch (st) {
    case at::kBFloat16: return FAGQ_DT_BF16;
    case at::kHalf: return FAGQ_DT_F16;
    case at::kFloat: return FAGQ_DT_F32;
    default: return -1;
  }
}

PyObject* launch(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 11) {
    PyErr_SetString(PyExc_TypeError, "launch() takes 11 arguments");
    return nullptr;
  }
  if (!g_launch) {
    PyErr_SetString(PyExc_RuntimeError, "launch(): bind() has not been called");
    return nullptr;
  }
  for (int i : {0, 1, 2, 3, 5, 6})
    if (!is_tensor(args[i])) return PyLong_FromLong(kArgError);
  const bool has_norm = args[4] != Py_None;
  if (has_norm && !is_tensor(args[4])) return PyLong_FromLong(kArgError);
  // Numbers of other types (a float group size, say) go to the Python checks.
  if (!PyFloat_Check(args[7]) || !PyLong_Check(args[8]) || !PyLong_Check(args[9]) ||
      !PyLong_Check(args[10]))
    return PyLong_FromLong(kArgError);
  const double eps = PyFloat_AS_DOUBLE(args[7]);
  const long long G = PyLong_AsLongLong(args[8]);
  const long rounding = PyLong_AsLong(args[9]);
  void* stream = PyLong_AsVoidPtr(args[10]);
  if (PyErr_Occurred()) {
    PyErr_Clear();
    return PyLong_FromLong(kArgError);
  }

  const at::Tensor& x = THPVariable_Unpack(args[0]);
  const at::Tensor& residual = THPVariable_Unpack(args[1]);
  const at::Tensor& gamma = THPVariable_Unpack(args[2]);
  const at::Tensor& residual_out = THPVariable_Unpack(args[3]);
  const at::Tensor& x_q = THPVariable_Unpack(args[5]);
  const at::Tensor& x_scale = THPVariable_Unpack(args[6]);
  if (x.dim() != 2 || !x.is_cuda()) return PyLong_FromLong(kArgError);
  const c10::DeviceIndex dev = x.get_device();
  const auto shape = x.sizes();
  const int64_t M = shape[0], D = shape[1];
  const int64_t dshape[1] = {D};
  // x, gamma and norm_out share the activation type, residual and
  // residual_out the residual stream's; the library checks the pair.
  const at::ScalarType at_ = x.scalar_type(), rt = residual.scalar_type();
  const int act = dtype_code(at_), res = dtype_code(rt);
  if (act < 0 || res < 0) return PyLong_FromLong(kArgError);
  if (!rows_ok(x, shape, dev, at_) || !rows_ok(residual, shape, dev, rt) ||
      !rows_ok(residual_out, shape, dev, rt) ||
      !rows_ok(gamma, at::IntArrayRef(dshape, 1), dev, at_))
    return PyLong_FromLong(kArgError);
  if (has_norm && !rows_ok(THPVariable_Unpack(args[4]), shape, dev, at_))
    return PyLong_FromLong(kArgError);
  if (G <= 0 || D % G != 0) return PyLong_FromLong(kArgError);

  int qf;
  if (x_q.scalar_type() == at::kFloat8_e4m3fn)
    qf = FAGQ_Q_FP8_E4M3FN;
  else if (x_q.scalar_type() == at::kChar)
    qf = FAGQ_Q_INT8;
  else
    return PyLong_FromLong(kArgError);
  if (x_q.sizes() != shape || !x_q.is_cuda() || x_q.get_device() != dev || !x_q.is_contiguous())
    return PyLong_FromLong(kArgError);

  int sf;
  if (x_scale.scalar_type() == at::kFloat)
    sf = FAGQ_SCALE_F32;
  else if (x_scale.scalar_type() == at::kByte)
    sf = FAGQ_SCALE_UE8M0;
  else
    return PyLong_FromLong(kArgError);
  const int64_t groups = D / G;
  if (x_scale.dim() != 2 || x_scale.size(0) != M || x_scale.size(1) != groups ||
      !x_scale.is_cuda() || x_scale.get_device() != dev)
    return PyLong_FromLong(kArgError);
  int layout;
  if (x_scale.is_contiguous())
    layout = FAGQ_LAYOUT_ROW_MAJOR;
  else if (x_scale.stride(0) == 1 && x_scale.stride(1) == M)
    layout = FAGQ_LAYOUT_COL_MAJOR;
  else
    return PyLong_FromLong(kArgError);

  int rnd;
  if (rounding == -1)
    rnd = qf == FAGQ_Q_FP8_E4M3FN ? FAGQ_ROUND_RNE : FAGQ_ROUND_TRUNC;
  else if (rounding == 0)
    rnd = FAGQ_ROUND_RNE;
  else if (rounding == 1 && qf == FAGQ_Q_INT8)
    rnd = FAGQ_ROUND_TRUNC;
  else
    return PyLong_FromLong(kArgError);
  if (M == 0) return PyLong_FromLong(FAGQ_OK);

  void* norm = has_norm ? THPVariable_Unpack(args[4]).data_ptr() : nullptr;
  if (act == FAGQ_DT_BF16 && res == FAGQ_DT_BF16)
    return PyLong_FromLong(g_launch(x.data_ptr(), residual.data_ptr(), gamma.data_ptr(),
                                    residual_out.data_ptr(), norm, x_q.data_ptr(),
                                    x_scale.data_ptr(), M, D, G, (float)eps, qf, sf, layout, rnd,
                                    stream));
  if (!g_launch_typed) return PyLong_FromLong(kArgError);
  const int st = g_launch_typed(x.data_ptr(), residual.data_ptr(), gamma.data_ptr(),
                                residual_out.data_ptr(), norm, x_q.data_ptr(), x_scale.data_ptr(),
                                M, D, G, (float)eps, qf, sf, layout, rnd, act, res, stream);
  // An unsupported type pair goes to the Python checks, which word the error.
  return PyLong_FromLong(st == FAGQ_E_FORMAT ? kArgError : st);
}

// bind(address of fagq_launch, address of fagq_launch_typed) in the loaded
// libfagq.so.
PyObject* bind(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 2) {
    PyErr_SetString(PyExc_TypeError, "bind() takes 2 arguments");
    return nullptr;
  }
  void* p = PyLong_AsVoidPtr(args[0]);
  void* pt = PyLong_AsVoidPtr(args[1]);
  if (PyErr_Occurred()) return nullptr;
  if (!p || !pt) {
    PyErr_SetString(PyExc_ValueError, "bind(): null function address");
    return nullptr;
  }
  g_launch = reinterpret_cast<LaunchFn>(p);
  g_launch_typed = reinterpret_cast<TypedLaunchFn>(pt);
  Py_RETURN_NONE;
}

PyMethodDef kMethods[] = {
    {"launch", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(&launch)),
     METH_FASTCALL, "Checks the operator's tensors and calls fagq_launch; returns its status."},
    {"bind", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(&bind)),
     METH_FASTCALL, "Sets the addresses of fagq_launch and fagq_launch_typed."},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_fagq_py", "Per-call binding of fagq_launch.", -1,
                       kMethods, nullptr, nullptr, nullptr, nullptr};

}  // namespace

PyMODINIT_FUNC PyInit__fagq_py(void) {
  PyObject* m = PyModule_Create(&kModule);
  if (m && PyModule_AddIntConstant(m, "ARG_ERROR", kArgError) != 0) {
    Py_DECREF(m);
    return nullptr;
  }
  return m;
}
