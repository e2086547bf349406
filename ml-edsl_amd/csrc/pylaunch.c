/* CPython binding of the two device launch entries (include/edsl_hip_device.h).
 *
 * Enqueuing a small layer costs ~2.7 us in the library (2.2-2.4 of them the
 * HIP launch itself); a ctypes call spends another ~1 us converting the 13
 * arguments. This module takes them through METH_FASTCALL instead, so a
 * 256^3 layer can be enqueued faster than it runs. Arguments are the C
 * entry's, in order: pointers as Python ints (None for a null bias), strides
 * and sizes as ints, alpha as a float, the stream as an int handle. It
 * returns the entry's status code; the error text stays with
 * edsl_hip_last_error. The GIL is released around the call, as ctypes does.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include "../../include/edsl_hip_device.h"

static int as_ptr(PyObject *o, void **out) {
  if (o == Py_None) {
    *out = NULL;
    return 0;
  }
  void *p = PyLong_AsVoidPtr(o);
  if (p == NULL && PyErr_Occurred()) return -1;
  *out = p;
  return 0;
}

static int as_i64(PyObject *o, int64_t *out) {
  long long v = PyLong_AsLongLong(o);
  if (v == -1 && PyErr_Occurred()) return -1;
  *out = (int64_t)v;
  return 0;
}

/* The operands common to both entries: X, ldx, W, ldw, bias, Y, ldy, M, N, K, epilogue. */
struct launch_args {
  void *x, *w, *bias, *y, *stream;
  int64_t ldx, ldw, ldy, m, n, k, epi;
};

static int parse_common(PyObject *const *a, struct launch_args *p) {
  return as_ptr(a[0], &p->x) || as_i64(a[1], &p->ldx) || as_ptr(a[2], &p->w) || as_i64(a[3], &p->ldw) ||
         as_ptr(a[4], &p->bias) || as_ptr(a[5], &p->y) || as_i64(a[6], &p->ldy) || as_i64(a[7], &p->m) ||
         as_i64(a[8], &p->n) || as_i64(a[9], &p->k) || as_i64(a[10], &p->epi);
}

/* dense_f32(X, ldx, W, ldw, bias, Y, ldy, M, N, K, epilogue, alpha, stream) -> int */
static PyObject *dense_f32(PyObject *self, PyObject *const *a, Py_ssize_t n) {
  (void)self;
  if (n != 13) {
    PyErr_SetString(PyExc_TypeError, "dense_f32 takes 13 arguments");
    return NULL;
  }
  struct launch_args p;
  if (parse_common(a, &p)) return NULL;
  const double alpha = PyFloat_AsDouble(a[11]);
  if (alpha == -1.0 && PyErr_Occurred()) return NULL;
  if (as_ptr(a[12], &p.stream)) return NULL;
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = edsl_hip_dense_f32_launch((const float *)p.x, p.ldx, (const float *)p.w, p.ldw, (const float *)p.bias,
                                 (float *)p.y, p.ldy, p.m, p.n, p.k, (int)p.epi, (float)alpha, p.stream);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

/* dense_i32(X, ldx, W, ldw, bias, Y, ldy, M, N, K, epilogue, stream) -> int */
static PyObject *dense_i32(PyObject *self, PyObject *const *a, Py_ssize_t n) {
  (void)self;
  if (n != 12) {
    PyErr_SetString(PyExc_TypeError, "dense_i32 takes 12 arguments");
    return NULL;
  }
  struct launch_args p;
  if (parse_common(a, &p) || as_ptr(a[11], &p.stream)) return NULL;
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = edsl_hip_dense_i32_launch((const int32_t *)p.x, p.ldx, (const int32_t *)p.w, p.ldw,
                                 (const int32_t *)p.bias, (int32_t *)p.y, p.ldy, p.m, p.n, p.k, (int)p.epi,
                                 p.stream);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

static PyMethodDef methods[] = {
    {"dense_f32", (PyCFunction)(void (*)(void))dense_f32, METH_FASTCALL,
     "edsl_hip_dense_f32_launch(X, ldx, W, ldw, bias, Y, ldy, M, N, K, epilogue, alpha, stream) -> status"},
    {"dense_i32", (PyCFunction)(void (*)(void))dense_i32, METH_FASTCALL,
     "edsl_hip_dense_i32_launch(X, ldx, W, ldw, bias, Y, ldy, M, N, K, epilogue, stream) -> status"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_launch",
                                    "METH_FASTCALL binding of the device launch entries.", -1, methods};

PyMODINIT_FUNC PyInit__launch(void) { return PyModule_Create(&module); }
