/* Fast-call CPython binding of the library's most frequent entry points (GEMM, row
 * reductions, softmax): the same C ABI as the ctypes binding, without the per-argument ctypes
 * conversions.  Python integers are taken as int64 values or addresses (None is a null
 * pointer); each function returns the entry point's status code.  Optional: the Python package
 * falls back to ctypes when this module is absent.  Linked against libbiops.so in the same
 * directory. */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <string.h>

#include "../../include/biops.h"

static int as_i64(PyObject* o, int64_t* v) {
  *v = (int64_t)PyLong_AsLongLong(o);
  return !(*v == -1 && PyErr_Occurred());
}

static int as_ptr(PyObject* o, void** p) {
  if (o == Py_None) {
    *p = NULL;
    return 1;
  }
  *p = PyLong_AsVoidPtr(o);
  return !(*p == NULL && PyErr_Occurred());
}

/* Converts args[i] by kind: 'l' int64, 'p' pointer. */
static int parse(PyObject* const* args, Py_ssize_t nargs, const char* kinds, int64_t* iv, void** pv) {
  Py_ssize_t n = (Py_ssize_t)strlen(kinds);
  if (nargs != n) {
    PyErr_Format(PyExc_TypeError, "expected %zd arguments, got %zd", n, nargs);
    return 0;
  }
  for (Py_ssize_t i = 0; i < n; ++i) {
    if (kinds[i] == 'p' ? !as_ptr(args[i], &pv[i]) : !as_i64(args[i], &iv[i])) return 0;
  }
  return 1;
}

/* gemm(dtype, M, N, K, A, sAm, sAk, B, sBk, sBn, bias, C, sCm, sCn, stream) */
static PyObject* fast_gemm(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[15];
  void* pv[15];
  (void)self;
  if (!parse(args, nargs, "llllpllpllppllp", iv, pv)) return NULL;
  return PyLong_FromLong(biops_gemm((int)iv[0], iv[1], iv[2], iv[3], pv[4], iv[5], iv[6], pv[7], iv[8], iv[9],
                                    pv[10], pv[11], iv[12], iv[13], pv[14]));
}

/* reduce(op, dtype_in, dtype_out, M, N, K, in, sM, sN, sK, out, stream) */
static PyObject* fast_reduce(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[12];
  void* pv[12];
  (void)self;
  if (!parse(args, nargs, "llllllplllpp", iv, pv)) return NULL;
  return PyLong_FromLong(biops_reduce((int)iv[0], (int)iv[1], (int)iv[2], iv[3], iv[4], iv[5], pv[6], iv[7],
                                      iv[8], iv[9], pv[10], pv[11]));
}

/* softmax(dtype_in, dtype_out, rows, cols, in, ld_in, out, ld_out, is_log, stream) */
static PyObject* fast_softmax(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[10];
  void* pv[10];
  (void)self;
  if (!parse(args, nargs, "llllplpllp", iv, pv)) return NULL;
  return PyLong_FromLong(biops_softmax((int)iv[0], (int)iv[1], iv[2], iv[3], pv[4], iv[5], pv[6], iv[7],
                                       (int)iv[8], pv[9]));
}

static PyMethodDef kMethods[] = {
    {"gemm", (PyCFunction)(void (*)(void))fast_gemm, METH_FASTCALL, "biops_gemm"},
    {"reduce", (PyCFunction)(void (*)(void))fast_reduce, METH_FASTCALL, "biops_reduce"},
    {"softmax", (PyCFunction)(void (*)(void))fast_softmax, METH_FASTCALL, "biops_softmax"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_biops_fast", NULL, -1, kMethods,
                                     NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__biops_fast(void) { return PyModule_Create(&kModule); }
