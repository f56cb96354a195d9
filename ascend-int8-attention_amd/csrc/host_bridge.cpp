// CPython host bridge over the C ABI of libsharedkv_hip.so: the counterpart
// of the reference's pybind launch module (csrc/host/launch.cpp:98-115 and
// csrc/host/c8_launch.cpp:17-43 of the reference checkout).  Each call takes
// plain integers (argument-block address, work-groups, variant, HIP stream
// handle), releases the GIL around the launch as the reference does, and
// raises RuntimeError on a non-zero hipError_t.  It holds no torch types: the
// caller passes torch's current raw stream.
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <stdint.h>

#include "sharedkv_hip.h"

namespace {

constexpr long VARIANT_SPARSE = 20, VARIANT_DENSE = 21, VARIANT_SPARSE_SMALL = 22;   // c8_launch.cpp:14-17
constexpr long VARIANT_DENSE_PAIRED = 23;   // grouped plans, 256-key tiles: groups of two (launch_sharedkv_c8_dense_paired)
constexpr long VARIANT_DENSE_PACKED = 24;   // groups of four (launch_sharedkv_c8_dense_packed)
constexpr long VARIANT_PAIRED_NARROW = 25;  // grouped plans, 128-key tiles (launch_sharedkv_c8_dense_paired_narrow)
constexpr long VARIANT_PACKED_NARROW = 26;  // (launch_sharedkv_c8_dense_packed_narrow)

bool read_u64(PyObject *o, uint64_t *out)
{
    const unsigned long long v = PyLong_AsUnsignedLongLong(o);
    if (v == (unsigned long long)-1 && PyErr_Occurred()) return false;
    *out = (uint64_t)v;
    return true;
}

PyObject *raise_code(int code, const char *what)
{
    PyErr_Format(PyExc_RuntimeError, "%s failed with hipError_t %d", what, code);
    return nullptr;
}

// attention(address, blocks, variant, stream) -> None
PyObject *attention(PyObject *, PyObject *const *args, Py_ssize_t nargs)
{
    if (nargs != 4) {
        PyErr_SetString(PyExc_TypeError, "attention(address, blocks, variant, stream)");
        return nullptr;
    }
    uint64_t address, blocks, stream;
    if (!read_u64(args[0], &address) || !read_u64(args[1], &blocks) || !read_u64(args[3], &stream)) return nullptr;
    const long variant = PyLong_AsLong(args[2]);
    if (variant == -1 && PyErr_Occurred()) return nullptr;
    int (*launch)(uint32_t, void *, const SharedKVArgs *) =
        variant == VARIANT_SPARSE ? launch_sharedkv_c8_sparse
        : variant == VARIANT_DENSE ? launch_sharedkv_c8_dense
        : variant == VARIANT_SPARSE_SMALL ? launch_sharedkv_c8_sparse_small
        : variant == VARIANT_DENSE_PAIRED ? launch_sharedkv_c8_dense_paired
        : variant == VARIANT_DENSE_PACKED ? launch_sharedkv_c8_dense_packed
        : variant == VARIANT_PAIRED_NARROW ? launch_sharedkv_c8_dense_paired_narrow
        : variant == VARIANT_PACKED_NARROW ? launch_sharedkv_c8_dense_packed_narrow : nullptr;
    if (!launch) {
        PyErr_SetString(PyExc_ValueError, "Invalid C8 variant");   // c8_launch.cpp:17
        return nullptr;
    }
    if (!address || blocks > 0xffffffffull) {
        PyErr_SetString(PyExc_ValueError, "Invalid C8 argument block or work-group count");
        return nullptr;
    }
    int code;
    Py_BEGIN_ALLOW_THREADS
    code = launch((uint32_t)blocks, (void *)(uintptr_t)stream, (const SharedKVArgs *)(uintptr_t)address);
    Py_END_ALLOW_THREADS
    if (code) return raise_code(code, "sharedkv C8 attention");
    Py_RETURN_NONE;
}

// cache_write(address, blocks, stream) -> None
PyObject *cache_write(PyObject *, PyObject *const *args, Py_ssize_t nargs)
{
    if (nargs != 3) {
        PyErr_SetString(PyExc_TypeError, "cache_write(address, blocks, stream)");
        return nullptr;
    }
    uint64_t address, blocks, stream;
    if (!read_u64(args[0], &address) || !read_u64(args[1], &blocks) || !read_u64(args[2], &stream)) return nullptr;
    if (!address || blocks > 0xffffffffull) {
        PyErr_SetString(PyExc_ValueError, "Invalid cache-write argument block or work-group count");
        return nullptr;
    }
    int code;
    Py_BEGIN_ALLOW_THREADS
    code = launch_cache_write((uint32_t)blocks, (void *)(uintptr_t)stream, (const CacheWriteArgs *)(uintptr_t)address);
    Py_END_ALLOW_THREADS
    if (code) return raise_code(code, "sharedkv cache write");
    Py_RETURN_NONE;
}

PyMethodDef methods[] = {
    {"attention", (PyCFunction)(void (*)(void))attention, METH_FASTCALL,
     "attention(address, blocks, variant, stream): launch a C8 attention argument block on a HIP stream"},
    {"cache_write", (PyCFunction)(void (*)(void))cache_write, METH_FASTCALL,
     "cache_write(address, blocks, stream): launch an INT8 cache-write argument block on a HIP stream"},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef module = {PyModuleDef_HEAD_INIT, "_sharedkv_host",
                      "Launch bridge over libsharedkv_hip.so (GIL released around each launch).", -1, methods,
                      nullptr, nullptr, nullptr, nullptr};

}  // namespace

PyMODINIT_FUNC PyInit__sharedkv_host(void) { return PyModule_Create(&module); }
