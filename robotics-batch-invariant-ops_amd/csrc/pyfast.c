/* Fast-call CPython binding of the library's most frequent entry points (GEMM, padded GEMM, row
 * reductions, softmax, fused attention, the varlen planner and fused varlen attention), of
 * the host-to-device copy of the varlen work list and of the device-to-host copy of the MoE
 * index flag: the same C ABI as the ctypes binding,
 * without the per-argument ctypes conversions.  Python integers are taken as
 * int64 values or addresses (None is a null pointer), Python floats as float; each function
 * returns the entry point's result.  The GIL is released around every library call (only
 * plain C values cross it), as ctypes does, so a launch that waits for a hardware queue or the
 * varlen planner's host work never stalls the other Python threads.  Optional: the Python package
 * falls back to ctypes when this module is absent.  Linked against libbiops.so in the same
 * directory. */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <string.h>

#include "../../include/biops.h"

/* HIP runtime (libamdhip64, a dependency of libbiops.so): the asynchronous copy the varlen
 * wrapper uploads its work list with. */
extern int hipMemcpyAsync(void* dst, const void* src, size_t bytes, int kind, void* stream);
enum { kHipMemcpyHostToDevice = 1, kHipMemcpyDeviceToHost = 2 };

/* Runs `call` (an expression of type T) with the GIL released and stores it in `out`. */
#define WITHOUT_GIL(out, call) \
  do {                         \
    Py_BEGIN_ALLOW_THREADS     \
    out = (call);              \
    Py_END_ALLOW_THREADS       \
  } while (0)

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

static int as_f32(PyObject* o, float* v) {
  const double d = PyFloat_AsDouble(o);
  *v = (float)d;
  return !(d == -1.0 && PyErr_Occurred());
}

/* Converts args[i] by kind: 'l' int64 (iv), 'p' pointer (pv), 'f' float (fv). */
static int parse(PyObject* const* args, Py_ssize_t nargs, const char* kinds, int64_t* iv, void** pv, float* fv) {
  Py_ssize_t n = (Py_ssize_t)strlen(kinds);
  if (nargs != n) {
    PyErr_Format(PyExc_TypeError, "expected %zd arguments, got %zd", n, nargs);
    return 0;
  }
  for (Py_ssize_t i = 0; i < n; ++i) {
    int ok;
    if (kinds[i] == 'p') ok = as_ptr(args[i], &pv[i]);
    else if (kinds[i] == 'f') ok = as_f32(args[i], &fv[i]);
    else ok = as_i64(args[i], &iv[i]);
    if (!ok) return 0;
  }
  return 1;
}

/* gemm(dtype, M, N, K, A, sAm, sAk, B, sBk, sBn, bias, C, sCm, sCn, stream) */
static PyObject* fast_gemm(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[15];
  void* pv[15];
  (void)self;
  if (!parse(args, nargs, "llllpllpllppllp", iv, pv, NULL)) return NULL;
  int rc;
  WITHOUT_GIL(rc, biops_gemm((int)iv[0], iv[1], iv[2], iv[3], pv[4], iv[5], iv[6], pv[7], iv[8], iv[9],
                                    pv[10], pv[11], iv[12], iv[13], pv[14]));
  return PyLong_FromLong(rc);
}

/* gemm_padded(dtype, M, N, K, A, sAm, sAk, B, sBk, sBn, bias, C, sCm, sCn, workspace, bytes, stream) */
static PyObject* fast_gemm_padded(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[17];
  void* pv[17];
  (void)self;
  if (!parse(args, nargs, "llllpllpllppllplp", iv, pv, NULL)) return NULL;
  int rc;
  WITHOUT_GIL(rc, biops_gemm_padded((int)iv[0], iv[1], iv[2], iv[3], pv[4], iv[5], iv[6], pv[7], iv[8], iv[9],
                                    pv[10], pv[11], iv[12], iv[13], pv[14], iv[15], pv[16]));
  return PyLong_FromLong(rc);
}

/* reduce(op, dtype_in, dtype_out, M, N, K, in, sM, sN, sK, out, stream) */
static PyObject* fast_reduce(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[12];
  void* pv[12];
  (void)self;
  if (!parse(args, nargs, "llllllplllpp", iv, pv, NULL)) return NULL;
  int rc;
  WITHOUT_GIL(rc, biops_reduce((int)iv[0], (int)iv[1], (int)iv[2], iv[3], iv[4], iv[5], pv[6], iv[7],
                                      iv[8], iv[9], pv[10], pv[11]));
  return PyLong_FromLong(rc);
}

/* softmax(dtype_in, dtype_out, rows, cols, in, ld_in, out, ld_out, is_log, stream) */
static PyObject* fast_softmax(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[10];
  void* pv[10];
  (void)self;
  if (!parse(args, nargs, "llllplpllp", iv, pv, NULL)) return NULL;
  int rc;
  WITHOUT_GIL(rc, biops_softmax((int)iv[0], (int)iv[1], iv[2], iv[3], pv[4], iv[5], pv[6], iv[7],
                                       (int)iv[8], pv[9]));
  return PyLong_FromLong(rc);
}

/* varlen_plan(nseq, cu_q, cu_kv, hq, dv, dtype, plan) -> workspace bytes or < 0 */
static PyObject* fast_varlen_plan(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[7];
  void* pv[7];
  (void)self;
  if (!parse(args, nargs, "lpplllp", iv, pv, NULL)) return NULL;
  long long rc;
  WITHOUT_GIL(rc, biops_varlen_plan(iv[0], (const int64_t*)pv[1], (const int64_t*)pv[2], iv[3], iv[4],
                                               (int)iv[5], (int64_t*)pv[6]));
  return PyLong_FromLongLong(rc);
}

/* varlen_fused_order(plan, causal, order) -> entries or < 0 */
static PyObject* fast_varlen_fused_order(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[3];
  void* pv[3];
  (void)self;
  if (!parse(args, nargs, "plp", iv, pv, NULL)) return NULL;
  long long rc;
  WITHOUT_GIL(rc, biops_varlen_fused_order((const int64_t*)pv[0], (int)iv[1], (int64_t*)pv[2]));
  return PyLong_FromLongLong(rc);
}

/* varlen_sdpa_fused(dtype, hq, hkv, d, dv, q, sq_t, sq_h, k, sk_t, sk_h, v, sv_t, sv_h, out,
 *                   so_t, so_h, dplan, hplan, dorder, causal, scale, stream) */
static PyObject* fast_varlen_sdpa_fused(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[23];
  void* pv[23];
  float fv[23];
  (void)self;
  if (!parse(args, nargs, "lllllpllpllpllpllppplfp", iv, pv, fv)) return NULL;
  int rc;
  WITHOUT_GIL(rc, biops_varlen_sdpa_fused((int)iv[0], iv[1], iv[2], iv[3], iv[4], pv[5], iv[6], iv[7], pv[8],
                                                 iv[9], iv[10], pv[11], iv[12], iv[13], pv[14], iv[15], iv[16],
                                                 (const int64_t*)pv[17], (const int64_t*)pv[18],
                                                 (const int64_t*)pv[19], (int)iv[20], fv[21], pv[22]));
  return PyLong_FromLong(rc);
}

/* varlen_sdpa_fused_planned(dtype, hq, hkv, d, dv, q, sq_t, sq_h, k, sk_t, sk_h, v, sv_t, sv_h,
 *                           out, so_t, so_h, total_q, total_kv, nseq, cu_q, cu_kv, host_buf,
 *                           host_words, dev_buf, causal, scale, stream) */
static PyObject* fast_varlen_sdpa_fused_planned(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[28];
  void* pv[28];
  float fv[28];
  (void)self;
  if (!parse(args, nargs, "lllllpllpllpllplllllppplplfp", iv, pv, fv)) return NULL;
  int rc;
  WITHOUT_GIL(rc, biops_varlen_sdpa_fused_planned(
      (int)iv[0], iv[1], iv[2], iv[3], iv[4], pv[5], iv[6], iv[7], pv[8], iv[9], iv[10], pv[11], iv[12], iv[13],
      pv[14], iv[15], iv[16], iv[17], iv[18], iv[19], (const int64_t*)pv[20], (const int64_t*)pv[21],
      (int64_t*)pv[22], iv[23], (int64_t*)pv[24], (int)iv[25], fv[26], pv[27]));
  return PyLong_FromLong(rc);
}

/* sdpa_fused(dtype, batch, hq, hkv, lq, lk, d, dv, q, sqB, sqH, sqL, k, skB, skH, skL, v, svB,
 *            svH, svL, mask, mask_dtype, mB, mH, mI, mJ, causal, scale, out, stream) */
static PyObject* fast_sdpa_fused(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[30];
  void* pv[30];
  float fv[30];
  (void)self;
  if (!parse(args, nargs, "llllllllplllplllplllpllllllfpp", iv, pv, fv)) return NULL;
  int rc;
  WITHOUT_GIL(rc, biops_sdpa_fused((int)iv[0], iv[1], iv[2], iv[3], iv[4], iv[5], iv[6], iv[7], pv[8], iv[9],
                                          iv[10], iv[11], pv[12], iv[13], iv[14], iv[15], pv[16], iv[17], iv[18],
                                          iv[19], pv[20], (int)iv[21], iv[22], iv[23], iv[24], iv[25], (int)iv[26],
                                          fv[27], pv[28], pv[29]));
  return PyLong_FromLong(rc);
}

/* copy_h2d(dst, src, bytes, stream) -> hipError_t: hipMemcpyAsync host -> device on `stream` */
static PyObject* fast_copy_h2d(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[4];
  void* pv[4];
  (void)self;
  if (!parse(args, nargs, "pplp", iv, pv, NULL)) return NULL;
  if (iv[2] < 0) {
    PyErr_SetString(PyExc_ValueError, "negative copy size");
    return NULL;
  }
  int rc;
  WITHOUT_GIL(rc, hipMemcpyAsync(pv[0], pv[1], (size_t)iv[2], kHipMemcpyHostToDevice, pv[3]));
  return PyLong_FromLong(rc);
}

/* copy_d2h(dst, src, bytes, stream) -> hipError_t: hipMemcpyAsync device -> host on `stream`
 * (into pinned host memory, so the copy stays asynchronous) */
static PyObject* fast_copy_d2h(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  int64_t iv[4];
  void* pv[4];
  (void)self;
  if (!parse(args, nargs, "pplp", iv, pv, NULL)) return NULL;
  if (iv[2] < 0) {
    PyErr_SetString(PyExc_ValueError, "negative copy size");
    return NULL;
  }
  int rc;
  WITHOUT_GIL(rc, hipMemcpyAsync(pv[0], pv[1], (size_t)iv[2], kHipMemcpyDeviceToHost, pv[3]));
  return PyLong_FromLong(rc);
}

static PyMethodDef kMethods[] = {
    {"gemm", (PyCFunction)(void (*)(void))fast_gemm, METH_FASTCALL, "biops_gemm"},
    {"gemm_padded", (PyCFunction)(void (*)(void))fast_gemm_padded, METH_FASTCALL, "biops_gemm_padded"},
    {"reduce", (PyCFunction)(void (*)(void))fast_reduce, METH_FASTCALL, "biops_reduce"},
    {"softmax", (PyCFunction)(void (*)(void))fast_softmax, METH_FASTCALL, "biops_softmax"},
    {"sdpa_fused", (PyCFunction)(void (*)(void))fast_sdpa_fused, METH_FASTCALL, "biops_sdpa_fused"},
    {"varlen_plan", (PyCFunction)(void (*)(void))fast_varlen_plan, METH_FASTCALL, "biops_varlen_plan"},
    {"varlen_fused_order", (PyCFunction)(void (*)(void))fast_varlen_fused_order, METH_FASTCALL,
     "biops_varlen_fused_order"},
    {"varlen_sdpa_fused", (PyCFunction)(void (*)(void))fast_varlen_sdpa_fused, METH_FASTCALL,
     "biops_varlen_sdpa_fused"},
    {"varlen_sdpa_fused_planned", (PyCFunction)(void (*)(void))fast_varlen_sdpa_fused_planned, METH_FASTCALL,
     "biops_varlen_sdpa_fused_planned"},
    {"copy_h2d", (PyCFunction)(void (*)(void))fast_copy_h2d, METH_FASTCALL, "hipMemcpyAsync host to device"},
    {"copy_d2h", (PyCFunction)(void (*)(void))fast_copy_d2h, METH_FASTCALL, "hipMemcpyAsync device to host"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_biops_fast", NULL, -1, kMethods,
                                     NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__biops_fast(void) { return PyModule_Create(&kModule); }
