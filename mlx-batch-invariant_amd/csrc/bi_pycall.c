/* bi_pycall.c — a CPython binding of the three most frequently called C-ABI
 * entry points (bi_quantized_matmul, bi_matmul, bi_rms_norm) for eager callers.
 *
 * ctypes converts every argument through its argtypes on each call (about
 * 3 us for the 15 arguments of bi_quantized_matmul); here the arguments are
 * read with one PyLong_AsLongLong each. The entry points are reached through
 * addresses the Python layer passes in once (bind), taken from its ctypes
 * handle of libbi_kernels.so, so this module has no link-time dependency on
 * the kernel library and calls exactly the functions ctypes would. Arguments
 * keep the C ABI's order and meaning (include/bi_kernels.h); None stands for
 * a NULL pointer. The functions return the ABI's status code.
 *
 * The GIL is released for the library call, as ctypes does: the call can block
 * on host work (first-use code-object load, a full launch queue), and
 * bi_last_error is thread-local, so the message stays with the calling thread.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stddef.h>
#include <stdint.h>

typedef int (*qmm_fn)(const void*, int64_t, const uint32_t*, const void*, const void*, void*, int64_t, int64_t,
                      int64_t, int, int, int, void*, size_t, void*);
typedef int (*mm_fn)(const void*, int64_t, const void*, int64_t, void*, int64_t, int64_t, int64_t, int, void*,
                     size_t, void*);
typedef int (*rms_fn)(const void*, int64_t, const void*, void*, int64_t, int64_t, float, int, void*);

static qmm_fn g_qmm;
static mm_fn g_mm;
static rms_fn g_rms;

#define PTR(v) ((void*)(intptr_t)(v))

/* Reads n integer arguments (None -> 0) into v, skipping index `skip`. */
static int read_i64(PyObject* const* args, Py_ssize_t n, Py_ssize_t want, Py_ssize_t skip, int64_t* v,
                    const char* name) {
  if (n != want) {
    PyErr_Format(PyExc_TypeError, "%s: %zd arguments, expected %zd", name, n, want);
    return -1;
  }
  for (Py_ssize_t i = 0; i < n; ++i) {
    if (i == skip) continue;
    if (args[i] == Py_None) {
      v[i] = 0;
      continue;
    }
    v[i] = PyLong_AsLongLong(args[i]);
    if (v[i] == -1 && PyErr_Occurred()) return -1;
  }
  return 0;
}

static PyObject* py_bind(PyObject* self, PyObject* args) {
  unsigned long long q, m, r;
  (void)self;
  if (!PyArg_ParseTuple(args, "KKK", &q, &m, &r)) return NULL;
  if (!q || !m || !r) {
    PyErr_SetString(PyExc_ValueError, "bind: null entry point");
    return NULL;
  }
  g_qmm = (qmm_fn)(uintptr_t)q;
  g_mm = (mm_fn)(uintptr_t)m;
  g_rms = (rms_fn)(uintptr_t)r;
  Py_RETURN_NONE;
}

static PyObject* py_quantized_matmul(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  int64_t v[15];
  int rc;
  (void)self;
  if (!g_qmm) {
    PyErr_SetString(PyExc_RuntimeError, "quantized_matmul: entry points not bound");
    return NULL;
  }
  if (read_i64(args, n, 15, -1, v, "quantized_matmul")) return NULL;
  Py_BEGIN_ALLOW_THREADS
  rc = g_qmm(PTR(v[0]), v[1], (const uint32_t*)PTR(v[2]), PTR(v[3]), PTR(v[4]), PTR(v[5]), v[6], v[7], v[8],
             (int)v[9], (int)v[10], (int)v[11], PTR(v[12]), (size_t)v[13], PTR(v[14]));
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

static PyObject* py_matmul(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  int64_t v[12];
  int rc;
  (void)self;
  if (!g_mm) {
    PyErr_SetString(PyExc_RuntimeError, "matmul: entry points not bound");
    return NULL;
  }
  if (read_i64(args, n, 12, -1, v, "matmul")) return NULL;
  Py_BEGIN_ALLOW_THREADS
  rc = g_mm(PTR(v[0]), v[1], PTR(v[2]), v[3], PTR(v[4]), v[5], v[6], v[7], (int)v[8], PTR(v[9]), (size_t)v[10],
            PTR(v[11]));
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

static PyObject* py_rms_norm(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  int64_t v[9];
  double eps;
  int rc;
  (void)self;
  if (!g_rms) {
    PyErr_SetString(PyExc_RuntimeError, "rms_norm: entry points not bound");
    return NULL;
  }
  if (read_i64(args, n, 9, 6, v, "rms_norm")) return NULL;
  eps = PyFloat_AsDouble(args[6]);
  if (eps == -1.0 && PyErr_Occurred()) return NULL;
  Py_BEGIN_ALLOW_THREADS
  rc = g_rms(PTR(v[0]), v[1], PTR(v[2]), PTR(v[3]), v[4], v[5], (float)eps, (int)v[7], PTR(v[8]));
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

static PyMethodDef methods[] = {
    {"bind", py_bind, METH_VARARGS, "bind(qmm, matmul, rms_norm): addresses of the C-ABI entry points"},
    {"quantized_matmul", (PyCFunction)(void (*)(void))py_quantized_matmul, METH_FASTCALL,
     "bi_quantized_matmul with the C ABI's arguments"},
    {"matmul", (PyCFunction)(void (*)(void))py_matmul, METH_FASTCALL, "bi_matmul with the C ABI's arguments"},
    {"rms_norm", (PyCFunction)(void (*)(void))py_rms_norm, METH_FASTCALL, "bi_rms_norm with the C ABI's arguments"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_bi_pycall", NULL, -1, methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__bi_pycall(void) { return PyModule_Create(&module); }
