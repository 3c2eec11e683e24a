// _trktorch: the per-call path of PreparedTRKernel as one C++ call.
//
// A prepared operator call checks x, allocates y with torch's caching allocator on x's device
// and launches trk_forward on that device's current stream. Done from Python, the allocation
// alone goes through the Python dispatcher (about 1.1 us); here the whole call stays in C++.
// Inputs this path does not take (another dtype or device, a wrong shape, non-contiguous or
// misaligned x, not a tensor) return None, and the Python caller takes its checked path,
// which raises the reference's ValueError or copies x.
//
// Built with g++ against torch's headers and libraries; it calls libtrk.so only through the
// C ABI of include/trk.h.
#include <Python.h>

#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
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

// forward(capsule, x[, epilogue, aux]) -> y, or None when x or aux needs the checked path.
// epilogue is an enum trk_epilogue (default TRK_EPI_STORE); y is fp32 for TRK_EPI_F32 and
// in the plan's dtype otherwise; aux ([T, out], the plan's dtype or fp32, contiguous, on x's
// device) is read by TRK_EPI_ADD and TRK_EPI_SILU_MUL.
PyObject *py_forward(PyObject *, PyObject *const *args, Py_ssize_t n) {
    HANDLE_TH_ERRORS
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
        if (epilogue < TRK_EPI_STORE || epilogue > TRK_EPI_SILU_MUL) Py_RETURN_NONE;
    }
    if (!THPVariable_Check(args[1])) Py_RETURN_NONE;
    const at::Tensor &x = THPVariable_Unpack(args[1]);
    if (x.scalar_type() != b->dtype || !x.is_cuda() || x.get_device() != b->device ||
        x.dim() != 2 || x.size(1) != b->in_features || x.size(0) > INT_MAX ||
        !x.is_contiguous() || (reinterpret_cast<uintptr_t>(x.const_data_ptr()) & 15))
        Py_RETURN_NONE;
    const int64_t tokens = x.size(0);
    const void *aux_ptr = nullptr;
    int aux_dtype = TRK_DTYPE_F32;
    if (epilogue == TRK_EPI_ADD || epilogue == TRK_EPI_SILU_MUL) {
        if (!THPVariable_Check(args[3])) Py_RETURN_NONE;
        const at::Tensor &aux = THPVariable_Unpack(args[3]);
        const bool f32 = aux.scalar_type() == c10::ScalarType::Float;
        if ((!f32 && aux.scalar_type() != b->dtype) || !aux.is_cuda() ||
            aux.get_device() != b->device || aux.dim() != 2 || aux.size(0) != tokens ||
            aux.size(1) != b->out_features || !aux.is_contiguous())
            Py_RETURN_NONE;
        aux_ptr = aux.const_data_ptr();
        if (!f32) aux_dtype = b->dtype_code;
    }
    at::Tensor y = at::empty({tokens, b->out_features},
                             epilogue == TRK_EPI_F32 ? x.options().dtype(c10::ScalarType::Float)
                                                     : x.options());
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

PyMODINIT_FUNC PyInit__trktorch(void) { return PyModule_Create(&module); }
