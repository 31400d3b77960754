/* pycall.c - CPython fast-call shim for the integer-argument entry points of
 * liblynnreal_amd.so.
 *
 * _pycall.call(address, *args) calls the C function at `address` with up to
 * MAX_ARGS integer arguments and returns its int status. Every argument is a
 * Python int or None (0, a null pointer). The entry points it is used for take
 * only pointers and integers, which the x86-64 System V convention passes in
 * integer registers and then 8-byte stack slots, the same way for int and
 * int64_t (the callee reads the low 32 bits of an int). Passing unused
 * trailing slots is harmless under that convention: the caller owns and pops
 * them. Entry points with float arguments stay on ctypes.
 *
 * This replaces ctypes' per-call argument conversion (about 4 us for the
 * GEMM's 24 arguments) with a METH_FASTCALL loop; it computes nothing itself.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>

#define MAX_ARGS 24

typedef int (*entry_fn)(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                        int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                        int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t);

static PyObject* pycall_call(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (nargs < 1 || nargs > MAX_ARGS + 1) {
    PyErr_Format(PyExc_TypeError, "call(address, *args) takes 1 to %d arguments, got %zd",
                 MAX_ARGS + 1, nargs);
    return NULL;
  }
  void* address = PyLong_AsVoidPtr(args[0]);
  if (address == NULL) {
    if (!PyErr_Occurred()) PyErr_SetString(PyExc_ValueError, "null function address");
    return NULL;
  }
  int64_t v[MAX_ARGS] = {0};
  for (Py_ssize_t i = 1; i < nargs; ++i) {
    PyObject* a = args[i];
    if (a == Py_None) continue;
    if (!PyLong_Check(a)) {
      PyErr_Format(PyExc_TypeError, "argument %zd must be an int or None, not %.80s", i,
                   Py_TYPE(a)->tp_name);
      return NULL;
    }
    /* Pointers above 2^63 do not occur in user space; unsigned values that
     * fit 64 bits are taken bit for bit. */
    long long x = PyLong_AsLongLong(a);
    if (x == -1 && PyErr_Occurred()) {
      PyErr_Clear();
      unsigned long long u = PyLong_AsUnsignedLongLong(a);
      if (u == (unsigned long long)-1 && PyErr_Occurred()) return NULL;
      x = (long long)u;
    }
    v[i - 1] = (int64_t)x;
  }
  const entry_fn fn = (entry_fn)address;
  const int status = fn(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7], v[8], v[9], v[10], v[11],
                        v[12], v[13], v[14], v[15], v[16], v[17], v[18], v[19], v[20], v[21], v[22],
                        v[23]);
  return PyLong_FromLong(status);
}

static PyMethodDef pycall_methods[] = {
    {"call", (PyCFunction)(void (*)(void))pycall_call, METH_FASTCALL,
     "call(address, *args) -> int: call an integer-argument C entry point"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef pycall_module = {PyModuleDef_HEAD_INIT, "_pycall",
                                           "Fast calls into liblynnreal_amd.so.", -1,
                                           pycall_methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__pycall(void) { return PyModule_Create(&pycall_module); }
