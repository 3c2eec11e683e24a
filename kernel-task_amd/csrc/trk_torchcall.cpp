// _trktorch: the per-call path of PreparedTRKernel as one C++ call.
//
// A prepared operator call checks x, allocates y with torch's caching allocator on x's device
// and launches trk_forward on that device's current stream. Done from Python, the allocation
// alone goes through the Python dispatcher (about 1.1 us); here the whole call stays in C++,
// and y is allocated below the dispatcher (at::detail::empty_cuda: the caching allocator
// under a device guard). The type Op carries the call itself: PreparedTRKernel derives from
// it, so calling a prepared operator enters this C++ slot without a Python frame.
// Inputs this path does not take (another dtype or device, a wrong shape, non-contiguous or
// misaligned x, not a tensor) go to the Python checked path (Op calls the instance's
// _checked_call; forward() returns None to its caller), which raises the reference's
// ValueError or copies x.
//
// Built with g++ against torch's headers and libraries; it calls libtrk.so only through the
// C ABI of include/trk.h.
#include <Python.h>

#include <ATen/core/Tensor.h>
#include <ATen/hip/EmptyTensor.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/Exceptions.h>
#include <torch/csrc/autograd/python_variable.h>

#include <climits>
#include <cstdint>

#include "trk.h"

namespace {

// What one prepared operator binds: its plan, packed cores and the x it accepts.
struct Bound {
    const trk_plan *plan;
    const void *packed;
    int64_t in_features, out_features;
    c10::ScalarType dtype;
    int dtype_code;  // the same dtype as an enum trk_dtype
    c10::DeviceIndex device;
};

constexpr const char *kCapsule = "trk.bound";

void free_bound(PyObject *capsule) {
    delete static_cast<Bound *>(PyCapsule_GetPointer(capsule, kCapsule));
}

bool scalar_type_of(long code, c10::ScalarType *out) {
    switch (code) {
        case TRK_DTYPE_F16: *out = c10::ScalarType::Half; return true;
        case TRK_DTYPE_BF16: *out = c10::ScalarType::BFloat16; return true;
        case TRK_DTYPE_F32: *out = c10::ScalarType::Float; return true;
        default: return false;
    }
}

// bind(plan, packed, in_features, out_features, trk_dtype, device_index) -> capsule.
// The capsule does not own the plan or the packed buffer: the Python object that holds it
// keeps both alive.
PyObject *py_bind(PyObject *, PyObject *const *args, Py_ssize_t n) {
    if (n != 6) {
        PyErr_SetString(PyExc_TypeError,
                        "bind(plan, packed, in_features, out_features, dtype, device_index)");
        return nullptr;
    }
    auto *b = new Bound{};
    b->plan = static_cast<const trk_plan *>(PyLong_AsVoidPtr(args[0]));
    b->packed = PyLong_AsVoidPtr(args[1]);
    b->in_features = PyLong_AsLongLong(args[2]);
    b->out_features = PyLong_AsLongLong(args[3]);
    const long code = PyLong_AsLong(args[4]);
    b->device = static_cast<c10::DeviceIndex>(PyLong_AsLong(args[5]));
    if (PyErr_Occurred()) {
        delete b;
        return nullptr;
    }
    b->dtype_code = static_cast<int>(code);
    if (!b->plan || !b->packed || !scalar_type_of(code, &b->dtype)) {
        delete b;
        PyErr_SetString(PyExc_ValueError, "bind: null plan or packed buffer, or unknown dtype");
        return nullptr;
    }
    PyObject *capsule = PyCapsule_New(b, kCapsule, free_bound);
    if (!capsule) delete b;
    return capsule;
}

// y for x through bound b with an epilogue (enum trk_epilogue; aux read by TRK_EPI_ADD and
// TRK_EPI_SILU_MUL): a new reference to y, to None when x or aux needs the checked path, or
// null with a Python error set. y is fp32 for TRK_EPI_F32 and in the plan's dtype otherwise;
// aux is [T, out], the plan's dtype or fp32, contiguous, on x's device.
PyObject *forward_impl(const Bound *b, PyObject *xo, int epilogue, PyObject *auxo) {
    HANDLE_TH_ERRORS
    if (epilogue < TRK_EPI_STORE || epilogue > TRK_EPI_SILU_MUL) Py_RETURN_NONE;
    if (!THPVariable_Check(xo)) Py_RETURN_NONE;
    const at::Tensor &x = THPVariable_Unpack(xo);
    if (x.scalar_type() != b->dtype || !x.is_cuda() || x.get_device() != b->device ||
        x.dim() != 2 || x.size(1) != b->in_features || x.size(0) > INT_MAX ||
        !x.is_contiguous() || (reinterpret_cast<uintptr_t>(x.const_data_ptr()) & 15))
        Py_RETURN_NONE;
    const int64_t tokens = x.size(0);
    const void *aux_ptr = nullptr;
    int aux_dtype = TRK_DTYPE_F32;
    if (epilogue == TRK_EPI_ADD || epilogue == TRK_EPI_SILU_MUL) {
        if (!auxo || !THPVariable_Check(auxo)) Py_RETURN_NONE;
        const at::Tensor &aux = THPVariable_Unpack(auxo);
        const bool f32 = aux.scalar_type() == c10::ScalarType::Float;
        if ((!f32 && aux.scalar_type() != b->dtype) || !aux.is_cuda() ||
            aux.get_device() != b->device || aux.dim() != 2 || aux.size(0) != tokens ||
            aux.size(1) != b->out_features || !aux.is_contiguous())
            Py_RETURN_NONE;
        aux_ptr = aux.const_data_ptr();
        if (!f32) aux_dtype = b->dtype_code;
    }
    const int64_t shape[2] = {tokens, b->out_features};
    at::Tensor y = at::detail::empty_cuda(
        shape, epilogue == TRK_EPI_F32 ? c10::ScalarType::Float : b->dtype,
        c10::Device(c10::DeviceType::CUDA, b->device), std::nullopt);
    if (tokens > 0) {
        const hipStream_t stream = c10::hip::getCurrentHIPStream(b->device).stream();
        const int status =
            epilogue == TRK_EPI_STORE
                ? trk_forward(b->plan, b->packed, x.const_data_ptr(), y.mutable_data_ptr(),
                              static_cast<int>(tokens), stream)
                : trk_forward_epilogue(b->plan, -1, b->packed, x.const_data_ptr(),
                                       y.mutable_data_ptr(), static_cast<int>(tokens), epilogue,
                                       aux_ptr, aux_dtype, stream);
        if (status != TRK_OK) {
            PyErr_SetString(PyExc_RuntimeError, trk_last_error());
            return nullptr;
        }
    }
    return THPVariable_Wrap(std::move(y));
    END_HANDLE_TH_ERRORS
}

// forward(capsule, x[, epilogue, aux]) -> y, or None when x or aux needs the checked path.
PyObject *py_forward(PyObject *, PyObject *const *args, Py_ssize_t n) {
    if (n != 2 && n != 4) {
        PyErr_SetString(PyExc_TypeError, "forward(bound, x[, epilogue, aux])");
        return nullptr;
    }
    const auto *b = static_cast<const Bound *>(PyCapsule_GetPointer(args[0], kCapsule));
    if (!b) return nullptr;
    int epilogue = TRK_EPI_STORE;
    if (n == 4) {
        epilogue = static_cast<int>(PyLong_AsLong(args[2]));
        if (PyErr_Occurred()) return nullptr;
    }
    return forward_impl(b, args[1], epilogue, n == 4 ? args[3] : nullptr);
}

// Op: a callable whose call is y = forward(x) through the Bound it holds (set once by
// _bind_native with bind()'s arguments). A call with one positional argument takes the C++
// path; anything else, and every x that path does not take, goes to self._checked_call(...)
// with the same arguments. Python subclasses (PreparedTRKernel) inherit the call slot.
struct OpObject {
    PyObject_HEAD
    Bound b;
    int bound;  // 1 once _bind_native succeeded (the allocation zeroes the object)
};

PyObject *op_call(PyObject *self, PyObject *args, PyObject *kwargs) {
    auto *op = reinterpret_cast<OpObject *>(self);
    if (op->bound && PyTuple_GET_SIZE(args) == 1 && (!kwargs || PyDict_GET_SIZE(kwargs) == 0)) {
        PyObject *y = forward_impl(&op->b, PyTuple_GET_ITEM(args, 0), TRK_EPI_STORE, nullptr);
        if (y != Py_None) return y;  // the output, or null with the error set
        Py_DECREF(y);
    }
    PyObject *checked = PyObject_GetAttrString(self, "_checked_call");
    if (!checked) return nullptr;
    PyObject *r = PyObject_Call(checked, args, kwargs);
    Py_DECREF(checked);
    return r;
}

PyObject *op_bind(PyObject *self, PyObject *const *args, Py_ssize_t n) {
    PyObject *capsule = py_bind(nullptr, args, n);
    if (!capsule) return nullptr;
    auto *op = reinterpret_cast<OpObject *>(self);
    op->b = *static_cast<Bound *>(PyCapsule_GetPointer(capsule, kCapsule));
    op->bound = 1;
    Py_DECREF(capsule);
    Py_RETURN_NONE;
}

PyMethodDef op_methods[] = {
    {"_bind_native", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(op_bind)),
     METH_FASTCALL,
     "_bind_native(plan, packed, in_features, out_features, dtype, device): what a call runs"},
    {nullptr, nullptr, 0, nullptr},
};

PyTypeObject OpType = {PyVarObject_HEAD_INIT(nullptr, 0)};

PyMethodDef methods[] = {
    {"bind", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(py_bind)),
     METH_FASTCALL, "bind(plan, packed, in_features, out_features, dtype, device) -> capsule"},
    {"forward", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(py_forward)),
     METH_FASTCALL,
     "forward(bound, x[, epilogue, aux]) -> y, or None when x or aux needs the checked path"},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef module = {PyModuleDef_HEAD_INIT, "_trktorch",
                      "Per-call path of PreparedTRKernel (allocate y, launch trk_forward)", -1,
                      methods};

}  // namespace

PyMODINIT_FUNC PyInit__trktorch(void) {
    OpType.tp_name = "_trktorch.Op";
    OpType.tp_doc = "Callable running y = forward(x) in C++ (base of PreparedTRKernel)";
    OpType.tp_basicsize = sizeof(OpObject);
    OpType.tp_flags = Py_TPFLAGS_DEFAULT | Py_TPFLAGS_BASETYPE;
    OpType.tp_new = PyType_GenericNew;
    OpType.tp_call = op_call;
    OpType.tp_methods = op_methods;
    if (PyType_Ready(&OpType) < 0) return nullptr;
    PyObject *m = PyModule_Create(&module);
    if (!m) return nullptr;
    Py_INCREF(&OpType);
    if (PyModule_AddObject(m, "Op", reinterpret_cast<PyObject *>(&OpType)) < 0) {
        Py_DECREF(&OpType);
        Py_DECREF(m);
        return nullptr;
    }
    return m;
}
