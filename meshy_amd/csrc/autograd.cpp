// meshy_amd._autograd: the autograd nodes of the three loss drop-ins, as a
// CPython extension over libtorch (host code only; the kernels are the C ABI
// of libmeshy_amd).
//
// A loss written as a Python torch.autograd.Function pays the Function
// machinery on both sides of every call: the context object, saving tensors,
// marking outputs, and on the way back the autograd engine's worker thread
// taking the GIL to run Python.  For the PPO loss that was ~60 us of host time
// around ~23 us of kernels.  Here each loss is one C++ call that allocates its
// outputs, launches the forward on torch's current stream and hangs a C++
// Node on the loss; the engine runs that Node's backward without Python.
//
//   ppo_inputs(args_bytes, keep) / distill_inputs(args_bytes, keep) -> capsule
//       A meshy_ppo_args / meshy_distill_args (the bytes of the ctypes
//       struct, checked against sizeof) and the tensors its pointers name,
//       held for as long as any call's backward may read them.
//   ppo_loss(new_lp, inputs) -> (loss, parts)
//       meshy_ppo_loss_fwd over the flat fp32 new_lp (the struct's new_lp and
//       grad_unit filled per call); loss is a 0-dim alias of the total-loss
//       sum carrying the backward, parts the MESHY_PPO_NOUT sums as 0-dim
//       views.  With grad enabled and new_lp requiring grad, the token mean
//       also has the forward write the unit gradient (the backward is one
//       scale) and the sequence mean keeps the per-document counts.
//   distill_loss(student, inputs) -> (loss, parts)
//       meshy_distill_loss_fwd / _bwd the same way (loss = parts[0]).
//   clipped_value_error(values, targets, old_values | None, clip | None) -> out
//       meshy_clipped_value_error over flat fp32 tensors; the backward reads
//       a broadcast (stride-0) gradient as one value.
//   set_error_type(cls)
//       The exception class raised for a HIP launch error in a forward
//       (negative codes raise ValueError, as the ctypes path does).
//
// Each Node checks, as autograd's saved tensors do, that the tensors it reads
// in the backward were not modified in place since the forward, and refuses a
// second backward once the engine has released them.
#include <Python.h>

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/Exceptions.h>
#include <torch/csrc/autograd/function.h>
#include <torch/csrc/autograd/functions/utils.h>
#include <torch/csrc/autograd/grad_mode.h>
#include <torch/csrc/autograd/python_variable.h>

#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "meshy_amd.h"

namespace {

using torch::autograd::variable_list;

PyObject* g_launch_error = nullptr;  // meshy_amd._lib.MeshyError once set

hipStream_t current_stream(const at::Tensor& t) {
    return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Python error for a failed C-ABI call in a forward (the GIL is held).
PyObject* raise_rc(int rc, const char* who) {
    const char* msg = meshy_last_error();
    if (rc < 0) {
        PyErr_SetString(PyExc_ValueError, (msg && *msg) ? msg : who);
    } else {
        PyErr_Format(g_launch_error ? g_launch_error : PyExc_RuntimeError, "%s: %s (hip error %d)", who,
                     msg ? msg : "", rc);
    }
    return nullptr;
}

// The same in a backward, which the engine runs without the GIL: a
// c10::ValueError reaches Python as ValueError, anything else as RuntimeError.
void throw_rc(int rc, const char* who) {
    const char* msg = meshy_last_error();
    std::string text = std::string(who) + ": " + ((msg && *msg) ? msg : "failed");
    if (rc < 0) TORCH_CHECK_VALUE(false, text);
    TORCH_CHECK(false, text, " (hip error ", rc, ")");
}

// A 0-dim tensor over element `index` of `buf`'s storage that is not a view
// of `buf`, so that it can carry its own grad_fn.
at::Tensor scalar_alias(const at::Tensor& buf, int64_t index) {
    auto impl = c10::make_intrusive<c10::TensorImpl>(c10::Storage(buf.storage()), buf.key_set(), buf.dtype());
    impl->set_storage_offset(buf.storage_offset() + index);
    impl->set_sizes_contiguous({});
    return at::Tensor(std::move(impl));
}

// A tensor a Node reads in its backward, with the version it had then.
struct Kept {
    at::Tensor t;
    int64_t version = 0;

    void keep(const at::Tensor& x) {
        t = x;
        version = x.defined() ? x._version() : 0;
    }
    const at::Tensor& get(const char* node) const {
        TORCH_CHECK(t.defined(), "Trying to backward through ", node,
                    " a second time; its saved tensors were freed after the first backward "
                    "(pass retain_graph=True to the first one)");
        TORCH_CHECK(t._version() == version, "one of the tensors ", node,
                    " reads in the backward was modified by an inplace operation after the forward "
                    "(version ", t._version(), ", expected ", version, ")");
        return t;
    }
};

template <class Args>
struct Inputs {
    Args args{};
    std::vector<at::Tensor> keep;  // what args points into
};

template <class Args>
const char* capsule_name();
template <>
const char* capsule_name<meshy_ppo_args>() { return "meshy_amd.ppo_inputs"; }
template <>
const char* capsule_name<meshy_distill_args>() { return "meshy_amd.distill_inputs"; }

template <class Args>
void capsule_free(PyObject* cap) {
    delete static_cast<std::shared_ptr<const Inputs<Args>>*>(PyCapsule_GetPointer(cap, capsule_name<Args>()));
}

template <class Args>
PyObject* make_inputs(PyObject* args) {
    HANDLE_TH_ERRORS
    Py_buffer raw;
    PyObject* keep;
    if (!PyArg_ParseTuple(args, "y*O", &raw, &keep)) return nullptr;
    if (static_cast<size_t>(raw.len) != sizeof(Args)) {
        PyErr_Format(PyExc_ValueError, "argument struct has %zd bytes, the library's has %zu", raw.len,
                     sizeof(Args));
        PyBuffer_Release(&raw);
        return nullptr;
    }
    auto in = std::make_shared<Inputs<Args>>();
    std::memcpy(&in->args, raw.buf, sizeof(Args));
    PyBuffer_Release(&raw);
    PyObject* seq = PySequence_Fast(keep, "keep must be a sequence of tensors or None");
    if (!seq) return nullptr;
    const Py_ssize_t n = PySequence_Fast_GET_SIZE(seq);
    for (Py_ssize_t i = 0; i < n; ++i) {
        PyObject* item = PySequence_Fast_GET_ITEM(seq, i);
        if (item == Py_None) continue;
        if (!THPVariable_Check(item)) {
            Py_DECREF(seq);
            PyErr_SetString(PyExc_TypeError, "keep must hold tensors or None");
            return nullptr;
        }
        in->keep.push_back(THPVariable_Unpack(item));
    }
    Py_DECREF(seq);
    auto* holder = new std::shared_ptr<const Inputs<Args>>(std::move(in));
    PyObject* cap = PyCapsule_New(holder, capsule_name<Args>(), capsule_free<Args>);
    if (!cap) delete holder;
    return cap;
    END_HANDLE_TH_ERRORS
}

template <class Args>
const std::shared_ptr<const Inputs<Args>>* unpack_inputs(PyObject* cap) {
    if (!PyCapsule_IsValid(cap, capsule_name<Args>())) {
        PyErr_Format(PyExc_TypeError, "inputs must be a %s capsule", capsule_name<Args>());
        return nullptr;
    }
    return static_cast<const std::shared_ptr<const Inputs<Args>>*>(PyCapsule_GetPointer(cap, capsule_name<Args>()));
}

bool unpack_tensor(PyObject* obj, const char* what, at::Tensor& out) {
    if (!THPVariable_Check(obj)) {
        PyErr_Format(PyExc_TypeError, "%s must be a tensor", what);
        return false;
    }
    out = THPVariable_Unpack(obj);
    return true;
}

// Flat fp32 device tensor on one device, as the kernels read it.
bool check_flat_f32(const at::Tensor& t, const char* what) {
    if (t.scalar_type() != at::kFloat || !t.is_contiguous() || !t.is_cuda()) {
        PyErr_Format(PyExc_ValueError, "%s must be a contiguous fp32 device tensor", what);
        return false;
    }
    return true;
}

PyObject* wrap_result(const at::Tensor& loss, const at::Tensor& out, int64_t nout) {
    PyObject* parts = PyTuple_New(nout);
    if (!parts) return nullptr;
    std::vector<at::Tensor> views = at::unbind(out.narrow(0, 0, nout), 0);
    for (int64_t i = 0; i < nout; ++i) PyTuple_SET_ITEM(parts, i, THPVariable_Wrap(views[i]));
    PyObject* l = THPVariable_Wrap(loss);
    if (!l) {
        Py_DECREF(parts);
        return nullptr;
    }
    PyObject* res = PyTuple_Pack(2, l, parts);
    Py_DECREF(l);
    Py_DECREF(parts);
    return res;
}

// ------------------------------------------------------------------ PPO

struct PpoLossBackward final : torch::autograd::Node {
    std::shared_ptr<const Inputs<meshy_ppo_args>> in;
    meshy_ppo_args a{};
    Kept new_lp;
    at::Tensor saved;  // the unit gradient (token mean) or the per-document counts

    variable_list apply(variable_list&& grads) override {
        if (!grads[0].defined()) return {at::Tensor()};
        const at::Tensor& lp = new_lp.get("the PPO loss");
        at::Tensor g = grads[0].reshape({1});
        if (g.scalar_type() != at::kFloat) g = g.to(at::kFloat);
        g = g.contiguous();
        at::Tensor grad = at::empty_like(lp);
        const float* seg_cnt = a.grad_unit ? nullptr : saved.data_ptr<float>();
        int rc = meshy_ppo_loss_bwd(&a, seg_cnt, g.data_ptr<float>(), grad.data_ptr<float>(), current_stream(lp));
        if (rc) throw_rc(rc, "meshy_ppo_loss_bwd");
        return {grad};
    }
    std::string name() const override { return "MeshyPpoLossBackward"; }
    void release_variables() override {
        new_lp.t.reset();
        saved.reset();
        in.reset();
    }
};

PyObject* ppo_loss(PyObject*, PyObject* args) {
    HANDLE_TH_ERRORS
    PyObject *py_lp, *cap;
    if (!PyArg_ParseTuple(args, "OO", &py_lp, &cap)) return nullptr;
    const auto* in = unpack_inputs<meshy_ppo_args>(cap);
    if (!in) return nullptr;
    at::Tensor lp;
    if (!unpack_tensor(py_lp, "new_lp", lp) || !check_flat_f32(lp, "new_lp")) return nullptr;
    c10::DeviceGuard guard(lp.device());
    meshy_ppo_args a = (*in)->args;
    if (lp.numel() != a.n_tokens) {
        PyErr_Format(PyExc_ValueError, "new_lp has %lld tokens, the inputs %lld", static_cast<long long>(lp.numel()),
                     static_cast<long long>(a.n_tokens));
        return nullptr;
    }
    const bool want_grad = torch::autograd::GradMode::is_enabled() && lp.requires_grad();
    const auto opts = lp.options();
    at::Tensor buf = at::empty({MESHY_PPO_NOUT}, opts);
    at::Tensor unit, seg_cnt;
    if (want_grad && a.per_token_loss) {
        unit = at::empty_like(lp);
    } else if (want_grad) {
        seg_cnt = at::empty({a.n_docs + 1}, opts);
    }
    a.new_lp = lp.data_ptr<float>();
    a.grad_unit = unit.defined() ? unit.data_ptr<float>() : nullptr;
    int rc = meshy_ppo_loss_fwd(&a, buf.data_ptr<float>(), seg_cnt.defined() ? seg_cnt.data_ptr<float>() : nullptr,
                                current_stream(lp));
    if (rc) return raise_rc(rc, "meshy_ppo_loss_fwd");
    at::Tensor loss = scalar_alias(buf, MESHY_PPO_TOTAL_LOSS);
    if (want_grad) {
        auto node = std::shared_ptr<PpoLossBackward>(new PpoLossBackward(), torch::autograd::deleteNode);
        node->set_next_edges(torch::autograd::collect_next_edges(lp));
        node->in = *in;
        node->a = a;
        node->new_lp.keep(lp);
        node->saved = unit.defined() ? unit : seg_cnt;
        torch::autograd::set_history(loss, node);
    }
    return wrap_result(loss, buf, MESHY_PPO_NOUT);
    END_HANDLE_TH_ERRORS
}

// ------------------------------------------------------------------ distillation

struct DistillLossBackward final : torch::autograd::Node {
    std::shared_ptr<const Inputs<meshy_distill_args>> in;
    meshy_distill_args a{};
    Kept student;
    at::Tensor seg_cnt;

    variable_list apply(variable_list&& grads) override {
        if (!grads[0].defined()) return {at::Tensor()};
        const at::Tensor& s = student.get("the distillation loss");
        at::Tensor g = grads[0].reshape({1});
        if (g.scalar_type() != at::kFloat) g = g.to(at::kFloat);
        g = g.contiguous();
        at::Tensor grad = at::empty_like(s);
        int rc = meshy_distill_loss_bwd(&a, seg_cnt.data_ptr<float>(), g.data_ptr<float>(), grad.data_ptr<float>(),
                                        current_stream(s));
        if (rc) throw_rc(rc, "meshy_distill_loss_bwd");
        return {grad};
    }
    std::string name() const override { return "MeshyDistillLossBackward"; }
    void release_variables() override {
        student.t.reset();
        seg_cnt.reset();
        in.reset();
    }
};

PyObject* distill_loss(PyObject*, PyObject* args) {
    HANDLE_TH_ERRORS
    PyObject *py_s, *cap;
    if (!PyArg_ParseTuple(args, "OO", &py_s, &cap)) return nullptr;
    const auto* in = unpack_inputs<meshy_distill_args>(cap);
    if (!in) return nullptr;
    at::Tensor s;
    if (!unpack_tensor(py_s, "student", s) || !check_flat_f32(s, "student")) return nullptr;
    c10::DeviceGuard guard(s.device());
    meshy_distill_args a = (*in)->args;
    if (s.numel() != a.n_tokens * (a.k + 1)) {
        PyErr_Format(PyExc_ValueError, "student has %lld values, the inputs expect %lld tokens x %lld",
                     static_cast<long long>(s.numel()), static_cast<long long>(a.n_tokens),
                     static_cast<long long>(a.k + 1));
        return nullptr;
    }
    // One allocation: the sums, then the per-document token counts the
    // backward reads.
    at::Tensor buf = at::empty({MESHY_DISTILL_NOUT + a.n_docs + 1}, s.options());
    at::Tensor seg_cnt = buf.narrow(0, MESHY_DISTILL_NOUT, a.n_docs + 1);
    a.student = s.data_ptr<float>();
    int rc = meshy_distill_loss_fwd(&a, buf.data_ptr<float>(), seg_cnt.data_ptr<float>(), current_stream(s));
    if (rc) return raise_rc(rc, "meshy_distill_loss_fwd");
    at::Tensor loss = scalar_alias(buf, MESHY_DISTILL_LOSS);
    if (torch::autograd::GradMode::is_enabled() && s.requires_grad()) {
        auto node = std::shared_ptr<DistillLossBackward>(new DistillLossBackward(), torch::autograd::deleteNode);
        node->set_next_edges(torch::autograd::collect_next_edges(s));
        node->in = *in;
        node->a = a;
        node->student.keep(s);
        node->seg_cnt = seg_cnt;
        torch::autograd::set_history(loss, node);
    }
    return wrap_result(loss, buf, MESHY_DISTILL_NOUT);
    END_HANDLE_TH_ERRORS
}

// ------------------------------------------------------------------ clipped value error

struct ClippedValueErrorBackward final : torch::autograd::Node {
    Kept v, t, o;
    int32_t has_clip = 0;
    float clip = 0.f;

    variable_list apply(variable_list&& grads) override {
        if (!grads[0].defined()) return {at::Tensor()};
        const char* node = "the clipped value error";
        const at::Tensor& vv = v.get(node);
        const at::Tensor& tt = t.get(node);
        const float* op = has_clip ? o.get(node).data_ptr<float>() : nullptr;
        at::Tensor g = grads[0];
        if (g.scalar_type() != at::kFloat) g = g.to(at::kFloat);
        // The gradient of a sum or a mean is one value broadcast (stride 0):
        // the kernel reads it as such instead of a materialised copy.
        int64_t stride = 1;
        if (g.dim() == 1 && g.numel() > 0 && g.stride(0) == 0) {
            stride = 0;
        } else {
            g = g.contiguous();
        }
        at::Tensor grad = at::empty_like(vv);
        int rc = meshy_clipped_value_error_bwd(vv.data_ptr<float>(), tt.data_ptr<float>(), op, has_clip, clip,
                                               vv.numel(), g.data_ptr<float>(), stride, grad.data_ptr<float>(),
                                               current_stream(vv));
        if (rc) throw_rc(rc, "meshy_clipped_value_error_bwd");
        return {grad};
    }
    std::string name() const override { return "MeshyClippedValueErrorBackward"; }
    void release_variables() override {
        v.t.reset();
        t.t.reset();
        o.t.reset();
    }
};

PyObject* clipped_value_error(PyObject*, PyObject* args) {
    HANDLE_TH_ERRORS
    PyObject *py_v, *py_t, *py_o, *py_clip;
    if (!PyArg_ParseTuple(args, "OOOO", &py_v, &py_t, &py_o, &py_clip)) return nullptr;
    at::Tensor v, t, o;
    if (!unpack_tensor(py_v, "values", v) || !check_flat_f32(v, "values")) return nullptr;
    if (!unpack_tensor(py_t, "targets", t) || !check_flat_f32(t, "targets")) return nullptr;
    const bool has_clip = py_clip != Py_None;
    float clip = 0.f;
    if (has_clip) {
        clip = static_cast<float>(PyFloat_AsDouble(py_clip));
        if (PyErr_Occurred()) return nullptr;
        if (!unpack_tensor(py_o, "old_values", o) || !check_flat_f32(o, "old_values")) return nullptr;
    }
    for (const at::Tensor* x : {&t, &o}) {
        if (x->defined() && x->numel() != v.numel()) {
            PyErr_Format(PyExc_ValueError, "values has %lld elements but %s has %lld",
                         static_cast<long long>(v.numel()), x == &t ? "targets" : "old_values",
                         static_cast<long long>(x->numel()));
            return nullptr;
        }
    }
    c10::DeviceGuard guard(v.device());
    at::Tensor out = at::empty_like(v);
    int rc = meshy_clipped_value_error(v.data_ptr<float>(), t.data_ptr<float>(),
                                       has_clip ? o.data_ptr<float>() : nullptr, has_clip, clip, v.numel(),
                                       out.data_ptr<float>(), current_stream(v));
    if (rc) return raise_rc(rc, "meshy_clipped_value_error");
    if (torch::autograd::GradMode::is_enabled() && v.requires_grad()) {
        auto node =
            std::shared_ptr<ClippedValueErrorBackward>(new ClippedValueErrorBackward(), torch::autograd::deleteNode);
        node->set_next_edges(torch::autograd::collect_next_edges(v));
        node->v.keep(v);
        node->t.keep(t);
        if (has_clip) node->o.keep(o);
        node->has_clip = has_clip;
        node->clip = clip;
        torch::autograd::set_history(out, node);
    }
    return THPVariable_Wrap(out);
    END_HANDLE_TH_ERRORS
}

PyObject* set_error_type(PyObject*, PyObject* cls) {
    Py_XINCREF(cls);
    Py_XSETREF(g_launch_error, cls);
    Py_RETURN_NONE;
}

PyObject* ppo_inputs(PyObject*, PyObject* args) { return make_inputs<meshy_ppo_args>(args); }
PyObject* distill_inputs(PyObject*, PyObject* args) { return make_inputs<meshy_distill_args>(args); }

PyMethodDef kMethods[] = {
    {"ppo_inputs", ppo_inputs, METH_VARARGS, "Capsule of a meshy_ppo_args and the tensors it points into."},
    {"distill_inputs", distill_inputs, METH_VARARGS,
     "Capsule of a meshy_distill_args and the tensors it points into."},
    {"ppo_loss", ppo_loss, METH_VARARGS, "PPO clip loss forward; the loss carries its backward."},
    {"distill_loss", distill_loss, METH_VARARGS, "Top-K distillation loss forward; the loss carries its backward."},
    {"clipped_value_error", clipped_value_error, METH_VARARGS,
     "Per-token (clipped) squared value error; the output carries its backward."},
    {"set_error_type", set_error_type, METH_O, "Exception class for HIP launch errors."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_autograd", "Autograd nodes of the loss drop-ins.", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__autograd() { return PyModule_Create(&kModule); }
