// Pointer tables for the library's Python mirror, built in one call: the trainer's list passes
// (hsn_amd/trainer.py) and the fused cell round's operands (hsn_amd/kernels/window.py).
//
// Each pass takes R lists of n tensors and hands the C entry points of include/hsn_trainer.h one
// array of n device pointers a list and the n element counts. Before that, every tensor must be a
// contiguous fp32 tensor on the first tensor's device, and the tensors at one index of the lists
// must hold as many elements. Made in the interpreter, those checks and tables cost a few
// attribute reads a tensor (about 0.3 ms for four lists of 198 tensors); here they are one pass
// over the tensors' metadata. Host code only: nothing is read from or launched on a device.
//
// The module `hsn_amd._tables` (CPython C API, linked against the installed PyTorch) exports
//   list_table(rows) -> bytearray | None
// rows: a sequence of R >= 1 sequences of n >= 1 tensors, every one as long as the first.
// Returns None when a tensor is not a contiguous fp32 tensor with storage on the first tensor's
// device or a column's element counts differ; otherwise R * n pointers (list after list), then
// the first list's n element counts, as 8-byte native integers. Anything that is not a sequence
// of sequences of tensors raises TypeError.
//   tensor_table(tensors, dtypes, shapes, device) -> bytearray | int
// tensors: a sequence of n tensors; dtypes and shapes: sequences of n torch dtypes and n tuples
// of ints; device: the device index every tensor must be on (-1: the CPU). Returns the index of
// the first tensor that is not contiguous, or whose dtype, shape or device differ from the given
// ones (the caller then names the mismatch), else the n data pointers as 8-byte integers. The
// cell round makes these checks of its twenty operands at every call.
#include <Python.h>

#include <torch/csrc/Dtype.h>
#include <torch/csrc/autograd/python_variable.h>

#include <cstdint>
#include <cstring>
#include <vector>

namespace {

struct Fast {  // a new reference from PySequence_Fast, released on scope exit
    PyObject* seq = nullptr;
    Fast() = default;
    Fast(const Fast&) = delete;
    Fast& operator=(const Fast&) = delete;
    ~Fast() { Py_XDECREF(seq); }
};

PyObject* list_table(PyObject*, PyObject* rows) {
    try {
        Fast outer;
        outer.seq = PySequence_Fast(rows, "list_table: rows must be a sequence of tensor lists");
        if (!outer.seq) return nullptr;
        const Py_ssize_t R = PySequence_Fast_GET_SIZE(outer.seq);
        if (R < 1) Py_RETURN_NONE;
        std::vector<Fast> lists(static_cast<size_t>(R));
        for (Py_ssize_t r = 0; r < R; ++r) {
            lists[r].seq = PySequence_Fast(PySequence_Fast_GET_ITEM(outer.seq, r),
                                           "list_table: every row must be a sequence of tensors");
            if (!lists[r].seq) return nullptr;
        }
        const Py_ssize_t n = PySequence_Fast_GET_SIZE(lists[0].seq);
        if (n < 1) Py_RETURN_NONE;
        for (Py_ssize_t r = 1; r < R; ++r)
            if (PySequence_Fast_GET_SIZE(lists[r].seq) != n) Py_RETURN_NONE;

        std::vector<int64_t> table(static_cast<size_t>((R + 1) * n));
        int64_t* const numels = table.data() + R * n;
        c10::Device device(c10::kCPU);
        for (Py_ssize_t r = 0; r < R; ++r) {
            PyObject** items = PySequence_Fast_ITEMS(lists[r].seq);
            for (Py_ssize_t j = 0; j < n; ++j) {
                if (!THPVariable_Check(items[j])) {
                    PyErr_SetString(PyExc_TypeError, "list_table: every item must be a tensor");
                    return nullptr;
                }
                const at::Tensor& t = THPVariable_Unpack(items[j]);
                if (r == 0 && j == 0) device = t.device();
                if (t.scalar_type() != at::kFloat || !t.has_storage() || !t.is_contiguous() ||
                    t.device() != device)
                    Py_RETURN_NONE;
                const int64_t count = t.numel();
                if (r == 0) numels[j] = count;
                else if (numels[j] != count) Py_RETURN_NONE;
                table[r * n + j] = static_cast<int64_t>(reinterpret_cast<uintptr_t>(t.data_ptr()));
            }
        }
        return PyByteArray_FromStringAndSize(reinterpret_cast<const char*>(table.data()),
                                             static_cast<Py_ssize_t>(table.size() * sizeof(int64_t)));
    } catch (const std::exception& e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
}

PyObject* tensor_table(PyObject*, PyObject* args) {
    PyObject *tensors, *dtypes, *shapes;
    long long device;
    if (!PyArg_ParseTuple(args, "OOOL", &tensors, &dtypes, &shapes, &device)) return nullptr;
    try {
        Fast ts, ds, ss;
        ts.seq = PySequence_Fast(tensors, "tensor_table: tensors must be a sequence");
        if (!ts.seq) return nullptr;
        ds.seq = PySequence_Fast(dtypes, "tensor_table: dtypes must be a sequence");
        if (!ds.seq) return nullptr;
        ss.seq = PySequence_Fast(shapes, "tensor_table: shapes must be a sequence");
        if (!ss.seq) return nullptr;
        const Py_ssize_t n = PySequence_Fast_GET_SIZE(ts.seq);
        if (PySequence_Fast_GET_SIZE(ds.seq) != n || PySequence_Fast_GET_SIZE(ss.seq) != n) {
            PyErr_SetString(PyExc_ValueError, "tensor_table: as many dtypes and shapes as tensors");
            return nullptr;
        }
        std::vector<int64_t> table(static_cast<size_t>(n));
        for (Py_ssize_t i = 0; i < n; ++i) {
            PyObject* item = PySequence_Fast_GET_ITEM(ts.seq, i);
            PyObject* dt = PySequence_Fast_GET_ITEM(ds.seq, i);
            if (!THPVariable_Check(item) || !THPDtype_Check(dt)) {
                PyErr_SetString(PyExc_TypeError, "tensor_table: tensors and torch dtypes expected");
                return nullptr;
            }
            const at::Tensor& t = THPVariable_Unpack(item);
            bool ok = t.scalar_type() == reinterpret_cast<THPDtype*>(dt)->scalar_type &&
                      t.has_storage() && t.is_contiguous() &&
                      (t.is_cuda() ? static_cast<long long>(t.get_device()) : -1LL) == device;
            if (ok) {
                Fast shape;
                shape.seq = PySequence_Fast(PySequence_Fast_GET_ITEM(ss.seq, i),
                                            "tensor_table: every shape must be a sequence of ints");
                if (!shape.seq) return nullptr;
                const Py_ssize_t dims = PySequence_Fast_GET_SIZE(shape.seq);
                ok = dims == t.dim();
                for (Py_ssize_t k = 0; ok && k < dims; ++k) {
                    const long long v = PyLong_AsLongLong(PySequence_Fast_GET_ITEM(shape.seq, k));
                    if (v == -1 && PyErr_Occurred()) return nullptr;
                    ok = v == t.size(k);
                }
            }
            if (!ok) return PyLong_FromSsize_t(i);
            table[i] = static_cast<int64_t>(reinterpret_cast<uintptr_t>(t.data_ptr()));
        }
        return PyByteArray_FromStringAndSize(reinterpret_cast<const char*>(table.data()),
                                             static_cast<Py_ssize_t>(table.size() * sizeof(int64_t)));
    } catch (const std::exception& e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
}

PyMethodDef kMethods[] = {
    {"list_table", list_table, METH_O,
     "list_table(rows) -> bytearray | None: the pointer tables and element counts of R lists of n "
     "contiguous fp32 tensors on one device (R * n pointers, then n counts, 8-byte integers)"},
    {"tensor_table", tensor_table, METH_VARARGS,
     "tensor_table(tensors, dtypes, shapes, device) -> bytearray | int: the data pointers of "
     "contiguous tensors of the given dtypes and shapes on one device, or the first mismatch's "
     "index"},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_tables",
                       "Pointer tables for the library's Python mirror (host code only).", -1,
                       kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__tables() { return PyModule_Create(&kModule); }
