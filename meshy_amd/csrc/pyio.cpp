// CPython extension module meshy_amd._pyio: the rollout wire's per-token columns
// from Python sequences of numbers, in one pass over the objects.
//
// The rollout keeps each sample's tokens, log-probs and masks as Python lists
// (rollout.py:118-153 turns them into one tensor per sample).  Flattening them
// into one jagged column is a walk over a few hundred thousand Python numbers:
// done here without the iterator protocol or a per-element dispatch.
//
//   seq_offsets(seqs, offsets) -> total or None
//       seqs: list of list/tuple; offsets: writable int64 buffer of len(seqs)+1,
//       filled with the running lengths.  None (buffer contents unspecified)
//       when an entry is not a list or tuple.
//   flatten_into(seqs, out, kind) -> bool
//       kind 'q': int64 from int / bool; kind 'f': float32 from float / int /
//       bool, rounded to nearest even.  out: writable buffer of exactly
//       offsets[-1] elements of that type.  False (out unspecified) when an
//       element has another type or an int does not fit; the caller then
//       converts the column with numpy, which gives numpy's own result or error.
//
// Both functions hold the GIL and call no Python code, so the sequences cannot
// change while they are read; a long column is converted by several threads.
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <algorithm>
#include <cstdint>
#include <thread>
#include <vector>

namespace {

// Items and length of a list or tuple; false for anything else.
inline bool seq_items(PyObject* s, PyObject*** items, Py_ssize_t* n) {
    if (PyList_Check(s)) {
        *items = reinterpret_cast<PyListObject*>(s)->ob_item;
        *n = PyList_GET_SIZE(s);
        return true;
    }
    if (PyTuple_Check(s)) {
        *items = reinterpret_cast<PyTupleObject*>(s)->ob_item;
        *n = PyTuple_GET_SIZE(s);
        return true;
    }
    return false;
}

inline bool as_int64(PyObject* x, int64_t* v) {
    if (PyLong_CheckExact(x)) {
        int overflow = 0;
        const long long r = PyLong_AsLongLongAndOverflow(x, &overflow);
        if (overflow) return false;  // numpy raises OverflowError for it
        *v = static_cast<int64_t>(r);
        return true;
    }
    if (PyBool_Check(x)) {
        *v = x == Py_True ? 1 : 0;
        return true;
    }
    return false;
}

inline bool as_float32(PyObject* x, float* v) {
    if (PyFloat_CheckExact(x)) {
        *v = static_cast<float>(PyFloat_AS_DOUBLE(x));
        return true;
    }
    if (PyLong_CheckExact(x)) {
        // An int converts through double, as numpy does; one too large for a
        // double is left to numpy (OverflowError).
        int overflow = 0;
        const long long r = PyLong_AsLongLongAndOverflow(x, &overflow);
        if (overflow) return false;
        *v = static_cast<float>(static_cast<double>(r));
        return true;
    }
    if (PyBool_Check(x)) {
        *v = x == Py_True ? 1.f : 0.f;
        return true;
    }
    return false;
}

PyObject* seq_offsets(PyObject*, PyObject* args) {
    PyObject* seqs = nullptr;
    Py_buffer off;
    if (!PyArg_ParseTuple(args, "Ow*", &seqs, &off)) return nullptr;
    PyObject** outer = nullptr;
    Py_ssize_t n = 0;
    if (!seq_items(seqs, &outer, &n)) {
        PyBuffer_Release(&off);
        Py_RETURN_NONE;
    }
    if (off.len != static_cast<Py_ssize_t>(sizeof(int64_t)) * (n + 1)) {
        PyBuffer_Release(&off);
        PyErr_SetString(PyExc_ValueError, "seq_offsets: offsets must hold len(seqs) + 1 int64 values");
        return nullptr;
    }
    int64_t* o = static_cast<int64_t*>(off.buf);
    int64_t acc = 0;
    o[0] = 0;
    for (Py_ssize_t i = 0; i < n; ++i) {
        PyObject** items = nullptr;
        Py_ssize_t len = 0;
        if (!seq_items(outer[i], &items, &len)) {
            PyBuffer_Release(&off);
            Py_RETURN_NONE;
        }
        acc += static_cast<int64_t>(len);
        o[i + 1] = acc;
    }
    PyBuffer_Release(&off);
    return PyLong_FromLongLong(acc);
}

// Converts samples [i0, i1) into dst (dst[0] is the first element of sample i0).
template <typename T, bool (*Conv)(PyObject*, T*)>
bool fill_range(PyObject** outer, Py_ssize_t i0, Py_ssize_t i1, T* dst) {
    Py_ssize_t k = 0;
    for (Py_ssize_t i = i0; i < i1; ++i) {
        PyObject** items = nullptr;
        Py_ssize_t len = 0;
        seq_items(outer[i], &items, &len);
        for (Py_ssize_t j = 0; j < len; ++j)
            if (!Conv(items[j], dst + k + j)) return false;
        k += len;
    }
    return true;
}

// Below this many elements one thread does the whole column.
constexpr Py_ssize_t kPerThread = 1 << 15;
constexpr unsigned kMaxThreads = 8;

// The whole column: sizes checked first, then the samples cut into runs of
// about equal element counts, one thread each.  Worker threads run only type
// checks, field reads and PyLong_AsLongLongAndOverflow on exact ints (which
// neither raises nor touches reference counts), while the calling thread holds
// the GIL, so no Python code can run or change the sequences meanwhile.
template <typename T, bool (*Conv)(PyObject*, T*)>
bool fill(PyObject** outer, Py_ssize_t n, T* dst, Py_ssize_t cap) {
    std::vector<Py_ssize_t> start(static_cast<size_t>(n) + 1);
    start[0] = 0;
    for (Py_ssize_t i = 0; i < n; ++i) {
        PyObject** items = nullptr;
        Py_ssize_t len = 0;
        if (!seq_items(outer[i], &items, &len) || len > cap - start[i]) return false;
        start[i + 1] = start[i] + len;
    }
    if (start[n] != cap) return false;
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const Py_ssize_t want = std::min<Py_ssize_t>(std::min(hw, kMaxThreads), cap / kPerThread);
    if (want <= 1 || n < 2) return fill_range<T, Conv>(outer, 0, n, dst);
    // Cut points: the first sample whose start reaches each share of the elements.
    std::vector<Py_ssize_t> cut(static_cast<size_t>(want) + 1);
    cut[0] = 0;
    cut[want] = n;
    for (Py_ssize_t t = 1; t < want; ++t) {
        const Py_ssize_t target = cap / want * t;
        cut[t] = std::lower_bound(start.begin(), start.end(), target) - start.begin();
        cut[t] = std::max(cut[t - 1], std::min(cut[t], n));
    }
    std::vector<char> ok(static_cast<size_t>(want), 0);
    std::vector<std::thread> pool;
    pool.reserve(static_cast<size_t>(want) - 1);
    Py_ssize_t started = 1;  // runs [1, started) have a thread of their own
    try {
        for (; started < want; ++started) {
            const Py_ssize_t t = started;
            pool.emplace_back([&, t] { ok[t] = fill_range<T, Conv>(outer, cut[t], cut[t + 1], dst + start[cut[t]]); });
        }
    } catch (...) {
        // No thread to be had: the calling thread converts the remaining runs.
    }
    ok[0] = fill_range<T, Conv>(outer, cut[0], cut[1], dst);
    for (Py_ssize_t t = started; t < want; ++t) ok[t] = fill_range<T, Conv>(outer, cut[t], cut[t + 1], dst + start[cut[t]]);
    for (std::thread& th : pool) th.join();
    return std::all_of(ok.begin(), ok.end(), [](char c) { return c != 0; });
}

PyObject* flatten_into(PyObject*, PyObject* args) {
    PyObject* seqs = nullptr;
    Py_buffer out;
    int kind = 0;
    if (!PyArg_ParseTuple(args, "Ow*C", &seqs, &out, &kind)) return nullptr;
    PyObject** outer = nullptr;
    Py_ssize_t n = 0;
    bool ok = false;
    if (kind != 'q' && kind != 'f') {
        PyBuffer_Release(&out);
        PyErr_SetString(PyExc_ValueError, "flatten_into: kind must be 'q' (int64) or 'f' (float32)");
        return nullptr;
    }
    const Py_ssize_t width = kind == 'q' ? 8 : 4;
    if (out.len % width != 0) {
        PyBuffer_Release(&out);
        PyErr_SetString(PyExc_ValueError, "flatten_into: buffer size is not a whole number of elements");
        return nullptr;
    }
    if (seq_items(seqs, &outer, &n)) {
        if (kind == 'q')
            ok = fill<int64_t, as_int64>(outer, n, static_cast<int64_t*>(out.buf), out.len / width);
        else
            ok = fill<float, as_float32>(outer, n, static_cast<float*>(out.buf), out.len / width);
    }
    PyBuffer_Release(&out);
    return PyBool_FromLong(ok);
}

PyMethodDef kMethods[] = {
    {"seq_offsets", seq_offsets, METH_VARARGS, "Running lengths of a list of lists/tuples, or None."},
    {"flatten_into", flatten_into, METH_VARARGS, "Flatten a list of number sequences into a buffer; False if unsupported."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_pyio", "Rollout wire helpers over Python objects.", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__pyio(void) { return PyModule_Create(&kModule); }
