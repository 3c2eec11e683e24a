/*
 * _trkcall: CPython fast-call binding of the per-call entry points of include/trk.h.
 *
 * trk_forward runs once per operator call, so its Python binding is on the latency path.
 * ctypes converts each argument through Python objects (~1 us for six); this module takes
 * the six integers through METH_FASTCALL and calls the C ABI directly. Every other libtrk
 * entry point (plans, packing, queries) keeps its ctypes binding.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include "trk.h"

static int as_ptr(PyObject *o, void **out) {
    *out = PyLong_AsVoidPtr(o);
    return !(*out == NULL && PyErr_Occurred());
}

/* forward(plan, packed, x, y, tokens, stream) -> status */
static PyObject *py_forward(PyObject *self, PyObject *const *args, Py_ssize_t n) {
    void *plan, *packed, *x, *y, *stream;
    (void)self;
    if (n != 6) {
        PyErr_SetString(PyExc_TypeError, "forward(plan, packed, x, y, tokens, stream)");
        return NULL;
    }
    if (!as_ptr(args[0], &plan) || !as_ptr(args[1], &packed) || !as_ptr(args[2], &x) ||
        !as_ptr(args[3], &y) || !as_ptr(args[5], &stream))
        return NULL;
    const long tokens = PyLong_AsLong(args[4]);
    if (tokens == -1 && PyErr_Occurred()) return NULL;
    return PyLong_FromLong(trk_forward((const trk_plan *)plan, packed, x, y, (int)tokens, stream));
}

/* forward_variant(plan, variant, packed, x, y, tokens, stream) -> status */
static PyObject *py_forward_variant(PyObject *self, PyObject *const *args, Py_ssize_t n) {
    void *plan, *packed, *x, *y, *stream;
    (void)self;
    if (n != 7) {
        PyErr_SetString(PyExc_TypeError, "forward_variant(plan, variant, packed, x, y, tokens, stream)");
        return NULL;
    }
    if (!as_ptr(args[0], &plan) || !as_ptr(args[2], &packed) || !as_ptr(args[3], &x) ||
        !as_ptr(args[4], &y) || !as_ptr(args[6], &stream))
        return NULL;
    const long variant = PyLong_AsLong(args[1]);
    const long tokens = PyLong_AsLong(args[5]);
    if (PyErr_Occurred()) return NULL;
    return PyLong_FromLong(trk_forward_variant((const trk_plan *)plan, (int)variant, packed, x, y,
                                               (int)tokens, stream));
}

/* forward_epilogue(plan, variant, packed, x, y, tokens, epilogue, aux, aux_dtype, stream)
 * -> status */
static PyObject *py_forward_epilogue(PyObject *self, PyObject *const *args, Py_ssize_t n) {
    void *plan, *packed, *x, *y, *aux, *stream;
    (void)self;
    if (n != 10) {
        PyErr_SetString(PyExc_TypeError, "forward_epilogue(plan, variant, packed, x, y, tokens, "
                                         "epilogue, aux, aux_dtype, stream)");
        return NULL;
    }
    if (!as_ptr(args[0], &plan) || !as_ptr(args[2], &packed) || !as_ptr(args[3], &x) ||
        !as_ptr(args[4], &y) || !as_ptr(args[7], &aux) || !as_ptr(args[9], &stream))
        return NULL;
    const long variant = PyLong_AsLong(args[1]);
    const long tokens = PyLong_AsLong(args[5]);
    const long epilogue = PyLong_AsLong(args[6]);
    const long aux_dtype = PyLong_AsLong(args[8]);
    if (PyErr_Occurred()) return NULL;
    return PyLong_FromLong(trk_forward_epilogue((const trk_plan *)plan, (int)variant, packed, x,
                                                y, (int)tokens, (int)epilogue, aux,
                                                (int)aux_dtype, stream));
}

static PyMethodDef methods[] = {
    {"forward", (PyCFunction)(void (*)(void))py_forward, METH_FASTCALL,
     "trk_forward(plan, packed, x, y, tokens, stream) -> status"},
    {"forward_variant", (PyCFunction)(void (*)(void))py_forward_variant, METH_FASTCALL,
     "trk_forward_variant(plan, variant, packed, x, y, tokens, stream) -> status"},
    {"forward_epilogue", (PyCFunction)(void (*)(void))py_forward_epilogue, METH_FASTCALL,
     "trk_forward_epilogue(plan, variant, packed, x, y, tokens, epilogue, aux, aux_dtype, "
     "stream) -> status"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_trkcall",
                                    "Fast-call binding of trk_forward", -1, methods};

PyMODINIT_FUNC PyInit__trkcall(void) { return PyModule_Create(&module); }
