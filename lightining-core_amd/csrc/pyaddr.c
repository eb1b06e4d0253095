/* pyaddr.c -- the Python binding's pointer marshalling.
 *
 * The ctypes binding hands numpy buffers to the C ABI as plain addresses.
 * numpy's own route (ndarray.ctypes.data_as) builds several Python objects per
 * array and costs microseconds; for the small one-shot calls that is a large
 * share of the call.  addr(obj) reads the address through the buffer protocol
 * instead (C-contiguous buffers only; None -> None).  Host code only: no HIP.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

static PyObject* lc_addr(PyObject* self, PyObject* obj) {
  (void)self;
  if (obj == Py_None) {
    Py_RETURN_NONE;
  }
  Py_buffer view;
  if (PyObject_GetBuffer(obj, &view, PyBUF_C_CONTIGUOUS) != 0) {
    return NULL;
  }
  /* The caller keeps obj alive for the duration of the C call. */
  PyObject* r = PyLong_FromVoidPtr(view.buf);
  PyBuffer_Release(&view);
  return r;
}

static PyMethodDef kMethods[] = {
    {"addr", lc_addr, METH_O, "Address of a C-contiguous buffer (None -> None)."},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_addr", NULL, -1, kMethods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__addr(void) { return PyModule_Create(&kModule); }
