/* CPython entry for the per-call launch of a prepared decode.
 *
 * ctypes converts every argument through its argtypes on each call, about
 * 0.1 us per argument: ~1.5 us for the 13 arguments of kvssd_hip_fused_decode
 * (include/kvssd_hip.h), as much as the rest of a prepared decode's Python
 * work.  This module's one function takes the entry point's address and the
 * call's arguments as Python ints (METH_FASTCALL, no argument tuple) and calls
 * it with the GIL released, as ctypes does.  It holds no state and knows
 * nothing of the library beyond that signature; the library itself is loaded
 * and checked by kvssd._native.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <stddef.h>

/* kvssd_hip_fused_decode: desc, query, packed_k, packed_v, scales_k,
 * scales_v, valid_tokens, block_table, out, lse, workspace, workspace_bytes,
 * stream */
typedef int (*fused_decode_fn)(const void*, const void*, const void*, const void*, const void*, const void*,
                               const void*, const void*, void*, void*, void*, size_t, void*);

enum { kArgs = 14, kBytesArg = 12 };

/* The hash of the sources this module and the library were built from
 * (build.py passes it to both); also kept as a marked string, so that the
 * build script can read it from the file without importing the module. */
#ifndef KVSSD_BUILD_ID
#define KVSSD_BUILD_ID "unknown"
#endif
__attribute__((used)) static const char kBuildIdMarked[] = "kvssd-build-id:" KVSSD_BUILD_ID;

static int as_pointer(PyObject* o, void** p) {
  if (o == Py_None) {
    *p = NULL;
    return 0;
  }
  *p = PyLong_AsVoidPtr(o);
  return (*p == NULL && PyErr_Occurred()) ? -1 : 0;
}

static PyObject* fused_decode(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (nargs != kArgs) {
    PyErr_Format(PyExc_TypeError, "fused_decode takes %d arguments (%zd given)", kArgs, nargs);
    return NULL;
  }
  void* p[kArgs];
  for (int i = 0; i < kArgs; ++i)
    if (i != kBytesArg && as_pointer(args[i], &p[i]) != 0) return NULL;
  const size_t bytes = PyLong_AsSize_t(args[kBytesArg]);
  if (bytes == (size_t)-1 && PyErr_Occurred()) return NULL;
  if (p[0] == NULL) {
    PyErr_SetString(PyExc_ValueError, "fused_decode: NULL entry point");
    return NULL;
  }
  const fused_decode_fn fn = (fused_decode_fn)p[0];
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = fn(p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8], p[9], p[10], p[11], bytes, p[13]);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

static PyMethodDef methods[] = {
    {"fused_decode", (PyCFunction)(void (*)(void))fused_decode, METH_FASTCALL,
     "fused_decode(entry, desc, query, packed_k, packed_v, scales_k, scales_v, valid_tokens, block_table, out, "
     "lse, workspace, workspace_bytes, stream) -> int: call kvssd_hip_fused_decode at address entry (every "
     "pointer an int or None) and return its status"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_fastcall", NULL, -1, methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__fastcall(void) {
  PyObject* m = PyModule_Create(&module);
  /* the argument list above, for the loader's check */
  if (m != NULL && (PyModule_AddStringConstant(m, "SIGNATURE", "kvssd_hip_fused_decode/13") != 0 ||
                    PyModule_AddStringConstant(m, "BUILD_ID", kBuildIdMarked + sizeof("kvssd-build-id:") - 1) != 0)) {
    Py_DECREF(m);
    return NULL;
  }
  return m;
}
