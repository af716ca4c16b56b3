// meshy_amd._stage: the host side of staging per-sample tensors for the pack,
// as a CPython extension over libtorch's tensor type (host code only).
//
// build_micro_batch (meshy/backend/titan/batch.py:96-230) reads, for every
// sample of a micro, sample["tokens"], sample["mask_assistant"],
// sample["logprobs"], sample.get("advantage"), ... one attribute at a time.
// From Python each tensor attribute (data_ptr, dtype, shape, device,
// contiguity) costs ~80 ns, ~1 us per column; these passes read them from the
// at::Tensor behind each object in a few ns, so the staging of a step's 256
// samples is one call per concern instead of ~3000 attribute reads.  Any
// conversion of a column (a list, another dtype, a strided view) stays with
// the caller.
//
//   plan_tables(micros, n_samples)
//       -> (used, need_len, doc_sample, doc_len, seq_len, n_docs, n_tokens)
//       The samples the micros read, compacted in order of first use
//       (used[j] = sample index), the longest prefix any micro reads of each
//       (need_len), and per document its compact sample and length; per micro
//       its seq_len, document count and token count.  int64 (doc_sample
//       int32) little-endian bytes.
//   columns(samples, used, key)
//       -> bytes of n_used records {u64 ptr; i64 dim0; i64 row; i32 dtype; i32 flags}
//       sample[key] for each used sample (KeyError if absent): flags bit 0 a
//       tensor, bit 1 on the CPU, bit 2 contiguous; ptr its data, dim0 its
//       first dimension, row the elements per first-dimension index, dtype
//       the c10::ScalarType (-1 when not a tensor).
//   scalars(samples, used, key, default)
//       -> bytes of n_used float64: sample.get(key), a number or the first
//       element of a tensor, `default` when absent or None or empty.
//   gather(samples, used, need, key, dst, dtype, elem_size, row, gather_fn)
//       -> True after concatenating the first need[j] rows of each used
//       sample's column at dst (through the library's threaded gather), or
//       False, copying nothing, when some column is not a CPU contiguous
//       tensor of that dtype and row width.
//   stage_micros(samples, micros, packed, need_rollout_lp, dst, capacity, gather_fn
//                [, gather_i32_fn, narrow_min_tokens])
//       The whole staging of build_micro_batches in one pass, for the common
//       case: every used sample's tokens (all int64 or all int32), fp32 mask
//       and (with need_rollout_lp) fp32 log-probs are CPU contiguous tensors
//       long enough for the micros.  With gather_i32_fn (the library's
//       meshy_host_gather_i32) int64 tokens are staged as int32 when the
//       staging holds at least narrow_min_tokens tokens, which checks each;
//       a token outside int32 returns None.  Lays the regions out as the Python
//       staging does (256-byte aligned: tokens, mask, [logprobs],
//       adv_samples, s_off, seq, out_off, doc_len, doc_start, doc_sample,
//       pos_w), gathers the columns and writes every table at dst.  Returns
//       None when a column is of another kind or a micro overflows its
//       seq_len (the Python path handles and reports it), the byte size
//       needed when capacity is smaller (nothing written), else
//       (size, bounds, n_used, total, tokens_int64, n_docs_total, max_elems,
//       max_docs, seq, rows, out_off, doc_start, used, need) with bounds the
//       regions' [start, end) byte offsets in that order as int64 pairs (-1
//       for an absent region), the four tables as bytes, and the compact
//       sample map with each used sample's prefix length as plan_tables
//       gives them.
#include <Python.h>

#include <torch/csrc/autograd/python_variable.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <type_traits>
#include <vector>

namespace {

struct Record {
    uint64_t ptr;
    int64_t dim0;
    int64_t row;
    int32_t dtype;
    int32_t flags;
};
static_assert(sizeof(Record) == 32, "record layout");

template <class T>
PyObject* to_bytes(const std::vector<T>& v) {
    return PyBytes_FromStringAndSize(reinterpret_cast<const char*>(v.data()),
                                     static_cast<Py_ssize_t>(v.size() * sizeof(T)));
}

// A Python int as int64 (false with an exception set otherwise).
bool as_i64(PyObject* o, int64_t& out) {
    const long long v = PyLong_AsLongLong(o);
    if (v == -1 && PyErr_Occurred()) return false;
    out = v;
    return true;
}

// The used sample indices from a bytes object of int64.
bool used_of(PyObject* b, const int64_t*& p, Py_ssize_t& n) {
    if (!PyBytes_Check(b)) {
        PyErr_SetString(PyExc_TypeError, "used must be bytes of int64");
        return false;
    }
    p = reinterpret_cast<const int64_t*>(PyBytes_AS_STRING(b));
    n = PyBytes_GET_SIZE(b) / static_cast<Py_ssize_t>(sizeof(int64_t));
    return true;
}

PyObject* plan_tables(PyObject*, PyObject* args) {
    PyObject* micros;
    long long n_samples;
    if (!PyArg_ParseTuple(args, "OL", &micros, &n_samples)) return nullptr;
    PyObject* seq = PySequence_Fast(micros, "micros must be a sequence");
    if (!seq) return nullptr;
    const Py_ssize_t n_micro = PySequence_Fast_GET_SIZE(seq);
    std::vector<int64_t> remap(static_cast<size_t>(n_samples > 0 ? n_samples : 0), -1);
    std::vector<int64_t> used, need, doc_len, seq_len, n_docs, n_tokens;
    std::vector<int32_t> doc_sample;
    seq_len.reserve(n_micro);
    n_docs.reserve(n_micro);
    n_tokens.reserve(n_micro);
    bool ok = true;
    for (Py_ssize_t k = 0; ok && k < n_micro; ++k) {
        PyObject* m = PySequence_Fast_GET_ITEM(seq, k);
        PyObject* sl = PyObject_GetAttrString(m, "seq_len");
        PyObject* si = sl ? PyObject_GetAttrString(m, "sample_idx") : nullptr;
        PyObject* dl = si ? PyObject_GetAttrString(m, "doc_lens") : nullptr;
        PyObject* fsi = dl ? PySequence_Fast(si, "sample_idx must be a sequence") : nullptr;
        PyObject* fdl = fsi ? PySequence_Fast(dl, "doc_lens must be a sequence") : nullptr;
        int64_t s_len = 0;
        ok = fdl && as_i64(sl, s_len);
        if (ok && PySequence_Fast_GET_SIZE(fsi) != PySequence_Fast_GET_SIZE(fdl)) {
            PyErr_SetString(PyExc_ValueError, "a micro's sample_idx and doc_lens differ in length");
            ok = false;
        }
        int64_t tokens = 0;
        const Py_ssize_t nd = ok ? PySequence_Fast_GET_SIZE(fsi) : 0;
        for (Py_ssize_t j = 0; ok && j < nd; ++j) {
            int64_t idx = 0, L = 0;
            ok = as_i64(PySequence_Fast_GET_ITEM(fsi, j), idx) && as_i64(PySequence_Fast_GET_ITEM(fdl, j), L);
            if (!ok) break;
            if (idx < 0 || idx >= n_samples) {
                PyErr_Format(PyExc_IndexError, "micro %zd reads sample %lld of %lld", k, static_cast<long long>(idx),
                             n_samples);
                ok = false;
                break;
            }
            if (L < 0) {
                PyErr_Format(PyExc_ValueError, "micro %zd has a negative document length", k);
                ok = false;
                break;
            }
            int64_t& c = remap[static_cast<size_t>(idx)];
            if (c < 0) {
                c = static_cast<int64_t>(used.size());
                used.push_back(idx);
                need.push_back(L);
            } else if (L > need[static_cast<size_t>(c)]) {
                need[static_cast<size_t>(c)] = L;
            }
            doc_sample.push_back(static_cast<int32_t>(c));
            doc_len.push_back(L);
            tokens += L;
        }
        if (ok) {
            seq_len.push_back(s_len);
            n_docs.push_back(nd);
            n_tokens.push_back(tokens);
        }
        Py_XDECREF(fdl);
        Py_XDECREF(fsi);
        Py_XDECREF(dl);
        Py_XDECREF(si);
        Py_XDECREF(sl);
    }
    Py_DECREF(seq);
    if (!ok) return nullptr;
    return Py_BuildValue("(NNNNNNN)", to_bytes(used), to_bytes(need), to_bytes(doc_sample), to_bytes(doc_len),
                         to_bytes(seq_len), to_bytes(n_docs), to_bytes(n_tokens));
}

PyObject* columns(PyObject*, PyObject* args) {
    PyObject *samples, *used_b, *key;
    if (!PyArg_ParseTuple(args, "OOO", &samples, &used_b, &key)) return nullptr;
    const int64_t* used;
    Py_ssize_t n;
    if (!used_of(used_b, used, n)) return nullptr;
    PyObject* seq = PySequence_Fast(samples, "samples must be a sequence");
    if (!seq) return nullptr;
    const Py_ssize_t n_samples = PySequence_Fast_GET_SIZE(seq);
    std::vector<Record> out(static_cast<size_t>(n));
    bool ok = true;
    for (Py_ssize_t i = 0; ok && i < n; ++i) {
        if (used[i] < 0 || used[i] >= n_samples) {
            PyErr_SetString(PyExc_IndexError, "used sample index out of range");
            ok = false;
            break;
        }
        PyObject* s = PySequence_Fast_GET_ITEM(seq, used[i]);
        PyObject* v;
        if (PyDict_CheckExact(s)) {
            v = PyDict_GetItemWithError(s, key);
            if (!v) {
                if (!PyErr_Occurred()) PyErr_SetObject(PyExc_KeyError, key);
                ok = false;
                break;
            }
            Py_INCREF(v);
        } else {
            v = PyObject_GetItem(s, key);
            if (!v) {
                ok = false;
                break;
            }
        }
        Record r{0, 0, 0, -1, 0};
        if (THPVariable_Check(v)) {
            const at::Tensor& t = THPVariable_Unpack(v);
            r.flags = 1;
            if (t.device().is_cpu()) r.flags |= 2;
            if (t.is_contiguous()) r.flags |= 4;
            r.dtype = static_cast<int32_t>(t.scalar_type());
            if (t.dim() == 0) {
                r.dim0 = 1;
                r.row = 1;
            } else {
                r.dim0 = t.size(0);
                r.row = r.dim0 ? t.numel() / r.dim0 : 1;
                for (int64_t d = 1; d < t.dim() && !r.dim0; ++d) r.row *= t.size(d);
            }
            if ((r.flags & 6) == 6 && t.numel()) r.ptr = reinterpret_cast<uint64_t>(t.data_ptr());
        }
        Py_DECREF(v);
        out[static_cast<size_t>(i)] = r;
    }
    Py_DECREF(seq);
    if (!ok) return nullptr;
    return to_bytes(out);
}

// The first element of a CPU contiguous tensor of a common numeric type, read
// in place; anything else goes through item().
bool first_element(const at::Tensor& t, double& out) {
    if (!t.numel()) return false;
    if (t.device().is_cpu() && t.is_contiguous()) {
        const void* p = t.data_ptr();
        switch (t.scalar_type()) {
            case at::kFloat: out = *static_cast<const float*>(p); return true;
            case at::kDouble: out = *static_cast<const double*>(p); return true;
            case at::kLong: out = static_cast<double>(*static_cast<const int64_t*>(p)); return true;
            case at::kInt: out = static_cast<double>(*static_cast<const int32_t*>(p)); return true;
            case at::kBool: out = *static_cast<const bool*>(p) ? 1.0 : 0.0; return true;
            default: break;
        }
    }
    out = t.reshape(-1)[0].item<double>();
    return true;
}

PyObject* scalars(PyObject*, PyObject* args) {
    PyObject *samples, *used_b, *key;
    double dflt;
    if (!PyArg_ParseTuple(args, "OOOd", &samples, &used_b, &key, &dflt)) return nullptr;
    const int64_t* used;
    Py_ssize_t n;
    if (!used_of(used_b, used, n)) return nullptr;
    PyObject* seq = PySequence_Fast(samples, "samples must be a sequence");
    if (!seq) return nullptr;
    const Py_ssize_t n_samples = PySequence_Fast_GET_SIZE(seq);
    std::vector<double> out(static_cast<size_t>(n), dflt);
    bool ok = true;
    try {
        for (Py_ssize_t i = 0; ok && i < n; ++i) {
            if (used[i] < 0 || used[i] >= n_samples) {
                PyErr_SetString(PyExc_IndexError, "used sample index out of range");
                ok = false;
                break;
            }
            PyObject* s = PySequence_Fast_GET_ITEM(seq, used[i]);
            PyObject* v = nullptr;
            if (PyDict_CheckExact(s)) {
                v = PyDict_GetItemWithError(s, key);
                if (!v && PyErr_Occurred()) {
                    ok = false;
                    break;
                }
                Py_XINCREF(v);
            } else if (PyObject_HasAttrString(s, "get")) {
                v = PyObject_CallMethod(s, "get", "OO", key, Py_None);
                if (!v) {
                    ok = false;
                    break;
                }
            }
            if (!v || v == Py_None) {
                Py_XDECREF(v);
                continue;
            }
            double x = dflt;
            if (THPVariable_Check(v)) {
                if (!first_element(THPVariable_Unpack(v), x)) x = dflt;
            } else {
                x = PyFloat_AsDouble(v);
                if (x == -1.0 && PyErr_Occurred()) ok = false;
            }
            Py_DECREF(v);
            out[static_cast<size_t>(i)] = x;
        }
    } catch (const std::exception& e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        ok = false;
    }
    Py_DECREF(seq);
    if (!ok) return nullptr;
    return to_bytes(out);
}

// The library's meshy_host_gather (passed in by address, so this module needs
// no link to it).
typedef int (*GatherFn)(const void* const*, const int64_t*, int64_t, void*, int);
// The library's meshy_host_gather_i32.
typedef int (*GatherI32Fn)(const int64_t* const*, const int64_t*, int64_t, int32_t*, int, int32_t*);

// gather(samples, used, need, key, dst, dtype, elem_size, row, gather_fn)
//   Copies the first need[j] rows (row elements of elem_size bytes) of
//   samples[used[j]][key] for every j, back to back, to the host address dst,
//   when every column is a CPU contiguous tensor of c10::ScalarType dtype with
//   rows of `row` elements; returns True.  Otherwise copies nothing and returns
//   False (the caller converts).  A tensor column shorter than need[j] raises
//   ValueError.
PyObject* gather(PyObject*, PyObject* args) {
    PyObject *samples, *used_b, *need_b, *key;
    unsigned long long dst, fn;
    int dtype;
    long long elem_size, row;
    if (!PyArg_ParseTuple(args, "OOOOKiLLK", &samples, &used_b, &need_b, &key, &dst, &dtype, &elem_size, &row,
                          &fn))
        return nullptr;
    const int64_t *used, *need;
    Py_ssize_t n, n_need;
    if (!used_of(used_b, used, n) || !used_of(need_b, need, n_need)) return nullptr;
    if (n_need != n) {
        PyErr_SetString(PyExc_ValueError, "used and need differ in length");
        return nullptr;
    }
    PyObject* seq = PySequence_Fast(samples, "samples must be a sequence");
    if (!seq) return nullptr;
    const Py_ssize_t n_samples = PySequence_Fast_GET_SIZE(seq);
    std::vector<const void*> srcs(static_cast<size_t>(n));
    std::vector<int64_t> nbytes(static_cast<size_t>(n));
    bool ok = true, fast = true;
    int64_t total = 0;
    for (Py_ssize_t i = 0; ok && i < n; ++i) {
        if (used[i] < 0 || used[i] >= n_samples) {
            PyErr_SetString(PyExc_IndexError, "used sample index out of range");
            ok = false;
            break;
        }
        PyObject* s = PySequence_Fast_GET_ITEM(seq, used[i]);
        PyObject* v;
        if (PyDict_CheckExact(s)) {
            v = PyDict_GetItemWithError(s, key);
            if (!v) {
                if (!PyErr_Occurred()) PyErr_SetObject(PyExc_KeyError, key);
                ok = false;
                break;
            }
            Py_INCREF(v);
        } else {
            v = PyObject_GetItem(s, key);
            if (!v) {
                ok = false;
                break;
            }
        }
        const int64_t L = need[i];
        nbytes[static_cast<size_t>(i)] = L * row * elem_size;
        total += nbytes[static_cast<size_t>(i)];
        if (!THPVariable_Check(v)) {
            fast = false;
        } else {
            const at::Tensor& t = THPVariable_Unpack(v);
            const int64_t dim0 = t.dim() ? t.size(0) : 1;
            if (dim0 < L) {
                PyErr_Format(PyExc_ValueError, "column %R of sample %lld holds %lld rows, %lld are needed", key,
                             static_cast<long long>(used[i]), static_cast<long long>(dim0),
                             static_cast<long long>(L));
                ok = false;
            } else if (!t.device().is_cpu() || !t.is_contiguous() || static_cast<int>(t.scalar_type()) != dtype ||
                       (dim0 && t.numel() / dim0 != row) || (!dim0 && L)) {
                fast = false;
            } else {
                srcs[static_cast<size_t>(i)] = L ? t.data_ptr() : nullptr;
            }
        }
        Py_DECREF(v);
    }
    Py_DECREF(seq);
    if (!ok) return nullptr;
    if (!fast) Py_RETURN_FALSE;
    if (total > 0) {
        if (!dst || !fn) {
            PyErr_SetString(PyExc_ValueError, "gather: no destination or gather function");
            return nullptr;
        }
        // The columns stay alive (the samples hold them) while the copy runs.
        const int rc = reinterpret_cast<GatherFn>(fn)(srcs.data(), nbytes.data(), n, reinterpret_cast<void*>(dst), 0);
        if (rc != 0) {
            PyErr_Format(PyExc_RuntimeError, "meshy_host_gather failed (%d)", rc);
            return nullptr;
        }
    }
    Py_RETURN_TRUE;
}

// sample[key] (a dict's item, or __getitem__), a new reference; nullptr with
// an exception set when absent.
PyObject* item_of(PyObject* s, PyObject* key) {
    if (PyDict_CheckExact(s)) {
        PyObject* v = PyDict_GetItemWithError(s, key);
        if (!v) {
            if (!PyErr_Occurred()) PyErr_SetObject(PyExc_KeyError, key);
            return nullptr;
        }
        Py_INCREF(v);
        return v;
    }
    return PyObject_GetItem(s, key);
}

// sample.get(key) as a float64 (the `scalars` rules): `dflt` when absent,
// None or an empty tensor; false with an exception set on error.
bool scalar_of(PyObject* s, PyObject* key, double dflt, double& out) {
    out = dflt;
    PyObject* v = nullptr;
    if (PyDict_CheckExact(s)) {
        v = PyDict_GetItemWithError(s, key);
        if (!v) return !PyErr_Occurred();
        Py_INCREF(v);
    } else if (PyObject_HasAttrString(s, "get")) {
        v = PyObject_CallMethod(s, "get", "OO", key, Py_None);
        if (!v) return false;
    } else {
        return true;
    }
    bool ok = true;
    if (v != Py_None) {
        if (THPVariable_Check(v)) {
            double x;
            if (first_element(THPVariable_Unpack(v), x)) out = x;
        } else {
            const double x = PyFloat_AsDouble(v);
            if (x == -1.0 && PyErr_Occurred()) ok = false;
            else out = x;
        }
    }
    Py_DECREF(v);
    return ok;
}

// A CPU contiguous tensor column of `dtype` with one element per row and at
// least `need` rows: its data pointer (nullptr for need == 0), else false.
bool fast_column(PyObject* v, at::ScalarType dtype, int64_t need, const void*& ptr) {
    if (!THPVariable_Check(v)) return false;
    const at::Tensor& t = THPVariable_Unpack(v);
    if (!t.device().is_cpu() || !t.is_contiguous() || t.scalar_type() != dtype || t.dim() != 1) return false;
    if (t.size(0) < need) return false;
    ptr = need ? t.data_ptr() : nullptr;
    return true;
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

PyObject* stage_micros(PyObject*, PyObject* args) {
    PyObject *samples, *micros;
    int packed, need_lp;
    unsigned long long dst, capacity, fn, fn_i32 = 0;
    long long narrow_min = 0;
    if (!PyArg_ParseTuple(args, "OOppKKK|KL", &samples, &micros, &packed, &need_lp, &dst, &capacity, &fn, &fn_i32,
                          &narrow_min))
        return nullptr;
    PyObject* seq_samples = PySequence_Fast(samples, "samples must be a sequence");
    if (!seq_samples) return nullptr;
    const Py_ssize_t n_samples = PySequence_Fast_GET_SIZE(seq_samples);
    // The compact sample map and the document tables (as plan_tables).
    PyObject* tables = Py_BuildValue("(On)", micros, n_samples);
    PyObject* pt = tables ? plan_tables(nullptr, tables) : nullptr;
    Py_XDECREF(tables);
    if (!pt) {
        Py_DECREF(seq_samples);
        return nullptr;
    }
    auto vec_of = [&](int i, auto* type_tag) {
        using T = std::remove_pointer_t<decltype(type_tag)>;
        PyObject* b = PyTuple_GET_ITEM(pt, i);
        const T* p = reinterpret_cast<const T*>(PyBytes_AS_STRING(b));
        return std::vector<T>(p, p + PyBytes_GET_SIZE(b) / static_cast<Py_ssize_t>(sizeof(T)));
    };
    const std::vector<int64_t> used = vec_of(0, static_cast<int64_t*>(nullptr));
    const std::vector<int64_t> need = vec_of(1, static_cast<int64_t*>(nullptr));
    const std::vector<int32_t> doc_sample = vec_of(2, static_cast<int32_t*>(nullptr));
    const std::vector<int64_t> doc_len = vec_of(3, static_cast<int64_t*>(nullptr));
    const std::vector<int64_t> seq = vec_of(4, static_cast<int64_t*>(nullptr));
    const std::vector<int64_t> n_docs = vec_of(5, static_cast<int64_t*>(nullptr));
    const std::vector<int64_t> n_tok = vec_of(6, static_cast<int64_t*>(nullptr));
    Py_DECREF(pt);
    const int64_t n_s = static_cast<int64_t>(used.size());
    const int64_t n_micro = static_cast<int64_t>(seq.size());
    const int64_t nd_total = static_cast<int64_t>(doc_len.size());
    bool fast = true;
    for (int64_t k = 0; k < n_micro && fast; ++k) fast = !packed || n_tok[k] <= seq[k];
    // The columns: all tensors of the staged dtypes, long enough.
    std::vector<const void*> tok_p(n_s), mask_p(n_s), lp_p(need_lp ? n_s : 0);
    std::vector<double> adv(n_s), reward(n_s), posw(n_s);
    PyObject* k_tokens = PyUnicode_InternFromString("tokens");
    PyObject* k_mask = PyUnicode_InternFromString("mask_assistant");
    PyObject* k_lp = PyUnicode_InternFromString("logprobs");
    PyObject* k_adv = PyUnicode_InternFromString("advantage");
    PyObject* k_adv_tok = PyUnicode_InternFromString("advantage_tokens");
    PyObject* k_reward = PyUnicode_InternFromString("reward");
    PyObject* k_posw = PyUnicode_InternFromString("positive_lm_weight");
    bool ok = k_tokens && k_mask && k_lp && k_adv && k_adv_tok && k_reward && k_posw;
    int tok64 = -1;  // unknown until the first tensor
    try {
        for (int64_t j = 0; ok && fast && j < n_s; ++j) {
            PyObject* s = PySequence_Fast_GET_ITEM(seq_samples, used[j]);
            // Per-token advantages take the Python path.
            // Any error (a missing column, an odd sample type) also leaves
            // the micros to the Python staging, which reports it.
            fast = PyDict_CheckExact(s) ? !PyDict_GetItemWithError(s, k_adv_tok) && !PyErr_Occurred()
                                        : PySequence_Contains(s, k_adv_tok) == 0;
            PyObject* t = fast ? item_of(s, k_tokens) : nullptr;
            if (!t) {
                fast = false;
                break;
            }
            if (THPVariable_Check(t)) {
                const at::ScalarType st = THPVariable_Unpack(t).scalar_type();
                const int is64 = st == at::kLong ? 1 : (st == at::kInt ? 0 : -2);
                if (is64 < 0 || (tok64 >= 0 && tok64 != is64)) fast = false;
                else tok64 = is64;
            } else {
                fast = false;
            }
            fast = fast && fast_column(t, tok64 == 1 ? at::kLong : at::kInt, need[j], tok_p[j]);
            Py_DECREF(t);
            if (!fast) break;
            PyObject* m = item_of(s, k_mask);
            if (!m) {
                fast = false;
                break;
            }
            fast = fast_column(m, at::kFloat, need[j], mask_p[j]);
            Py_DECREF(m);
            if (fast && need_lp) {
                PyObject* l = item_of(s, k_lp);
                if (!l) {
                    fast = false;
                    break;
                }
                fast = fast_column(l, at::kFloat, need[j], lp_p[j]);
                Py_DECREF(l);
            }
            fast = fast && scalar_of(s, k_adv, 0.0, adv[j]) && scalar_of(s, k_reward, 0.0, reward[j]) &&
                   scalar_of(s, k_posw, 0.0, posw[j]);
        }
    } catch (const std::exception&) {
        fast = false;
    }
    if (ok && !fast) PyErr_Clear();
    Py_XDECREF(k_tokens);
    Py_XDECREF(k_mask);
    Py_XDECREF(k_lp);
    Py_XDECREF(k_adv);
    Py_XDECREF(k_adv_tok);
    Py_XDECREF(k_reward);
    Py_XDECREF(k_posw);
    Py_DECREF(seq_samples);
    if (!ok) return nullptr;
    if (!fast) Py_RETURN_NONE;
    if (tok64 < 0) tok64 = 1;  // no samples: an empty int64 region, as the Python staging
    // The layout (the Python staging's region order).
    int64_t total = 0;
    for (int64_t L : need) total += L;
    const bool narrow = tok64 == 1 && fn_i32 != 0 && total >= narrow_min;
    if (narrow) tok64 = 0;  // staged as int32
    const int64_t tok_sz = tok64 ? 8 : 4;
    const int64_t sizes[11] = {total * tok_sz,
                               total * 4,
                               need_lp ? total * 4 : -1,
                               std::max<int64_t>(n_s, 1) * 4,
                               (n_s + 1) * 8,
                               n_micro * 8,
                               (n_micro + 1) * 8,
                               std::max<int64_t>(nd_total, 1) * 8,
                               (n_micro + 1) * 4,
                               std::max<int64_t>(nd_total, 1) * 4,
                               std::max<int64_t>(nd_total, 1) * 4};
    int64_t offs[11];
    int64_t size = 0;
    for (int r = 0; r < 11; ++r) {
        offs[r] = size;
        if (sizes[r] >= 0) size += align256(sizes[r]);
    }
    if (static_cast<unsigned long long>(size) > capacity) return PyLong_FromLongLong(size);
    if (!dst || !fn) {
        PyErr_SetString(PyExc_ValueError, "stage_micros: no destination or gather function");
        return nullptr;
    }
    char* base = reinterpret_cast<char*>(dst);
    // The columns, through the library's threaded gather.
    std::vector<int64_t> nbytes(n_s);
    auto gather_col = [&](const std::vector<const void*>& src, int64_t elem, int64_t off) -> bool {
        for (int64_t j = 0; j < n_s; ++j) nbytes[j] = need[j] * elem;
        if (total == 0) return true;
        const int rc = reinterpret_cast<GatherFn>(fn)(src.data(), nbytes.data(), n_s, base + off, 0);
        if (rc != 0) PyErr_Format(PyExc_RuntimeError, "meshy_host_gather failed (%d)", rc);
        return rc == 0;
    };
    if (narrow) {
        for (int64_t j = 0; j < n_s; ++j) nbytes[j] = need[j];  // elements
        int32_t fits = 1;
        if (total > 0) {
            const int rc = reinterpret_cast<GatherI32Fn>(fn_i32)(reinterpret_cast<const int64_t* const*>(tok_p.data()),
                                                                 nbytes.data(), n_s,
                                                                 reinterpret_cast<int32_t*>(base + offs[0]), 0, &fits);
            if (rc != 0) {
                PyErr_Format(PyExc_RuntimeError, "meshy_host_gather_i32 failed (%d)", rc);
                return nullptr;
            }
        }
        if (!fits) Py_RETURN_NONE;  // a token outside int32: the Python staging keeps the int64s
    } else if (!gather_col(tok_p, tok_sz, offs[0])) {
        return nullptr;
    }
    if (!gather_col(mask_p, 4, offs[1]) || (need_lp && !gather_col(lp_p, 4, offs[2]))) return nullptr;
    // The tables.
    float* adv_s = reinterpret_cast<float*>(base + offs[3]);
    for (int64_t j = 0; j < n_s; ++j) adv_s[j] = static_cast<float>(adv[j]);
    int64_t* s_off = reinterpret_cast<int64_t*>(base + offs[4]);
    s_off[0] = 0;
    for (int64_t j = 0; j < n_s; ++j) s_off[j + 1] = s_off[j] + need[j];
    std::vector<int64_t> rows(n_micro), out_off(n_micro + 1);
    std::vector<int32_t> doc_start(n_micro + 1);
    int64_t max_elems = 0, max_docs = 0;
    out_off[0] = 0;
    doc_start[0] = 0;
    for (int64_t k = 0; k < n_micro; ++k) {
        rows[k] = packed ? 1 : std::max<int64_t>(n_docs[k], 1);
        const int64_t elems = seq[k] * rows[k];
        out_off[k + 1] = out_off[k] + elems;
        doc_start[k + 1] = doc_start[k] + static_cast<int32_t>(n_docs[k]);
        max_elems = std::max(max_elems, elems);
        max_docs = std::max(max_docs, n_docs[k]);
    }
    std::memcpy(base + offs[5], seq.data(), n_micro * 8);
    std::memcpy(base + offs[6], out_off.data(), (n_micro + 1) * 8);
    std::memcpy(base + offs[7], doc_len.data(), nd_total * 8);
    std::memcpy(base + offs[8], doc_start.data(), (n_micro + 1) * 4);
    std::memcpy(base + offs[9], doc_sample.data(), nd_total * 4);
    // Positive-LM weights only for rewards above 0.5 (batch.py:225-229).
    float* pos_w = reinterpret_cast<float*>(base + offs[10]);
    for (int64_t d = 0; d < nd_total; ++d) {
        const int64_t j = doc_sample[d];
        pos_w[d] = reward[j] > 0.5 ? static_cast<float>(posw[j]) : 0.f;
    }
    std::vector<int64_t> off_v(22, -1);  // [start, end) per region; -1 for no log-probs region
    for (int r = 0; r < 11; ++r) {
        if (sizes[r] < 0) continue;
        off_v[2 * r] = offs[r];
        off_v[2 * r + 1] = offs[r] + sizes[r];
    }
    return Py_BuildValue("(LNLLiLLLNNNNNN)", static_cast<long long>(size), to_bytes(off_v),
                         static_cast<long long>(n_s), static_cast<long long>(total), tok64,
                         static_cast<long long>(nd_total), static_cast<long long>(max_elems),
                         static_cast<long long>(max_docs), to_bytes(seq), to_bytes(rows), to_bytes(out_off),
                         to_bytes(doc_start), to_bytes(used), to_bytes(need));
}

PyMethodDef kMethods[] = {
    {"gather", gather, METH_VARARGS, "Concatenate one column of the used samples into a host buffer."},
    {"plan_tables", plan_tables, METH_VARARGS, "Compact sample map and document tables of a list of micros."},
    {"columns", columns, METH_VARARGS, "Pointer, shape and dtype records of one column of the used samples."},
    {"scalars", scalars, METH_VARARGS, "One scalar field of the used samples as float64."},
    {"stage_micros", stage_micros, METH_VARARGS, "The whole staging of a list of micros, for the common case."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_stage", "Host staging passes over per-sample tensors.", -1,
                       kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__stage() { return PyModule_Create(&kModule); }
