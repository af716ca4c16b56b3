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
//   ppo_inputs(...) / distill_inputs(...) -> capsule
//       The inputs of one micro-batch's loss, read once: a meshy_ppo_args /
//       meshy_distill_args over the batch's tensors (each on the GPU, flat,
//       converted only when its type or layout differs, sizes checked) with
//       its workspace, and those tensors, held for as long as any call's
//       backward may read them.  args_bytes(capsule) gives the struct.
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
#include <optional>
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
        // The gradient of a sum or a mean is one value broadcast (every
        // stride 0): the kernel reads it as such instead of a materialised copy.
        bool broadcast = g.numel() > 0;
        for (int64_t d = 0; d < g.dim() && broadcast; ++d) broadcast = g.size(d) <= 1 || g.stride(d) == 0;
        const int64_t stride = broadcast ? 0 : 1;
        if (!broadcast) g = g.contiguous();
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

// ------------------------------------------------------------------ inputs

// Reads the tensors of one loss's inputs as the kernels take them: each on
// the GPU, flat, of one element type, a copy only when its type or layout
// differs; every tensor read is held in `keep`.  Errors are Python
// ValueErrors with the messages of the Python-side checks.
class Reader {
  public:
    explicit Reader(std::vector<at::Tensor>& keep) : keep_(keep) {}

    // The tensor behind `obj`, which must be a GPU tensor (nullopt for None;
    // false with an exception set on error).
    bool tensor(PyObject* obj, const char* what, at::Tensor& out) {
        if (obj == Py_None) {
            out = at::Tensor();
            return true;
        }
        if (!unpack_tensor(obj, what, out)) return false;
        if (!out.is_cuda()) {
            PyErr_SetString(PyExc_ValueError,
                            "meshy_amd kernels run on the GPU; got a CPU tensor (move inputs to a HIP device)");
            return false;
        }
        if (device_ && out.device() != *device_) {
            PyErr_Format(PyExc_ValueError, "%s is on another device than the other inputs", what);
            return false;
        }
        if (!device_) device_ = out.device();
        return true;
    }

    // A flat pointer of `dtype` over `t` (nullptr for an undefined tensor).
    template <class T>
    const T* flat(const at::Tensor& t, at::ScalarType dtype) {
        if (!t.defined()) return nullptr;
        at::Tensor x = t;
        if (x.scalar_type() != dtype) x = x.to(dtype);
        if (!x.is_contiguous()) x = x.contiguous();
        keep_.push_back(x);
        return x.data_ptr<T>();
    }

    // A uint8 workspace of `bytes` (at least one) on the inputs' device.
    void* workspace(size_t bytes, size_t& size) {
        size = bytes > 0 ? bytes : 1;
        at::Tensor w = at::empty({static_cast<int64_t>(size)}, at::TensorOptions().dtype(at::kByte).device(*device_));
        keep_.push_back(w);
        return w.data_ptr();
    }

  private:
    std::vector<at::Tensor>& keep_;
    std::optional<at::Device> device_;
};

template <class Args>
PyObject* wrap_inputs(std::shared_ptr<Inputs<Args>>&& in) {
    auto* holder = new std::shared_ptr<const Inputs<Args>>(std::move(in));
    PyObject* cap = PyCapsule_New(holder, capsule_name<Args>(), capsule_free<Args>);
    if (!cap) delete holder;
    return cap;
}

using Named = std::pair<const char*, const at::Tensor*>;

bool bad_tokens(const char* fmt, const char* name, int64_t n_tokens, int64_t got) {
    PyErr_Format(PyExc_ValueError, fmt, static_cast<long long>(n_tokens), name, static_cast<long long>(got));
    return true;
}

// ppo_inputs(old_lp, mask, rollout_lp|None, entropy|None, advantages,
//            positive_lm_weights|None, doc_ids, seg_offsets, n_tokens, n_docs,
//            n_docs_global, n_tokens_global, clip_low, clip_high, tis_min,
//            tis_max, positive_lm_coef, use_tis, use_icepop, per_token_loss,
//            train_lp_is_old, cp_degree) -> capsule
// Advantages of more than one dimension are per token, else per document.
PyObject* ppo_inputs(PyObject*, PyObject* args) {
    HANDLE_TH_ERRORS
    PyObject *o_old, *o_mask, *o_roll, *o_ent, *o_adv, *o_pos, *o_ids, *o_off;
    long long n_tokens, n_docs, n_docs_global, n_tokens_global;
    double clip_low, clip_high, tis_min, tis_max, coef;
    int use_tis, use_icepop, per_token, train_is_old, cp;
    if (!PyArg_ParseTuple(args, "OOOOOOOOLLLLdddddppppi", &o_old, &o_mask, &o_roll, &o_ent, &o_adv, &o_pos, &o_ids,
                          &o_off, &n_tokens, &n_docs, &n_docs_global, &n_tokens_global, &clip_low, &clip_high,
                          &tis_min, &tis_max, &coef, &use_tis, &use_icepop, &per_token, &train_is_old, &cp))
        return nullptr;
    at::NoGradGuard no_grad;
    auto in = std::make_shared<Inputs<meshy_ppo_args>>();
    Reader rd(in->keep);
    at::Tensor old, mask, roll, ent, adv, pos, ids, off;
    if (!rd.tensor(o_old, "old_lp", old) || !rd.tensor(o_mask, "mask", mask) ||
        !rd.tensor(o_adv, "advantages", adv) || !rd.tensor(o_ids, "doc_ids", ids) ||
        !rd.tensor(o_roll, "rollout_logprobs", roll) || !rd.tensor(o_ent, "entropy", ent) ||
        !rd.tensor(o_pos, "positive_lm_weights", pos) || !rd.tensor(o_off, "seg_offsets", off))
        return nullptr;
    const bool adv_per_token = adv.dim() != 1;
    const char* tok_fmt = "new_lp has %lld tokens but %s has %lld";
    for (auto [name, t] : {Named{"old_lp", &old}, Named{"mask", &mask}, Named{"doc_ids", &ids},
                           Named{"rollout_logprobs", &roll}, Named{"entropy", &ent},
                           Named{"advantages", adv_per_token ? &adv : nullptr}}) {
        if (t && t->defined() && t->numel() != n_tokens && bad_tokens(tok_fmt, name, n_tokens, t->numel()))
            return nullptr;
    }
    for (auto [name, t] : {Named{"positive_lm_weights", &pos}, Named{"advantages", adv_per_token ? nullptr : &adv}}) {
        if (t && t->defined() && t->numel() < n_docs) {
            PyErr_Format(PyExc_ValueError, "%s has %lld entries for %lld documents", name,
                         static_cast<long long>(t->numel()), n_docs);
            return nullptr;
        }
    }
    if (off.scalar_type() != at::kLong || !off.is_contiguous() || off.numel() < n_docs + 2) {
        PyErr_SetString(PyExc_ValueError, "seg_offsets must be n_docs + 2 contiguous int64 values");
        return nullptr;
    }
    meshy_ppo_args& a = in->args;
    a.old_lp = rd.flat<float>(old, at::kFloat);
    a.mask = rd.flat<float>(mask, at::kFloat);
    a.rollout_lp = rd.flat<float>(roll, at::kFloat);
    a.entropy = rd.flat<float>(ent, at::kFloat);
    a.adv = rd.flat<float>(adv, at::kFloat);
    a.positive_lm_weights = rd.flat<float>(pos, at::kFloat);
    a.doc_ids = rd.flat<int64_t>(ids, at::kLong);
    a.seg_offsets = rd.flat<int64_t>(off, at::kLong);
    a.n_tokens = n_tokens;
    a.n_docs = n_docs;
    a.n_docs_global = n_docs_global;
    a.n_tokens_global = n_tokens_global;
    a.clip_low = static_cast<float>(clip_low);
    a.clip_high = static_cast<float>(clip_high);
    a.tis_min = static_cast<float>(tis_min);
    a.tis_max = static_cast<float>(tis_max);
    a.positive_lm_coef = static_cast<float>(coef);
    a.adv_per_token = adv_per_token;
    a.use_tis = use_tis;
    a.use_icepop = use_icepop;
    a.per_token_loss = per_token;
    a.train_lp_is_old = train_is_old;
    a.cp_degree = cp;
    a.workspace = rd.workspace(meshy_ppo_workspace_size(n_tokens, n_docs), a.workspace_bytes);
    return wrap_inputs(std::move(in));
    END_HANDLE_TH_ERRORS
}

// distill_inputs(teacher_lp, mask, rollout_lp|None, doc_ids, seg_offsets, k,
//                n_tokens, n_docs, n_docs_global, n_tokens_global,
//                lp_min_clamp|None, loss_max_clamp|None, per_token_loss) -> capsule
PyObject* distill_inputs(PyObject*, PyObject* args) {
    HANDLE_TH_ERRORS
    PyObject *o_teacher, *o_mask, *o_roll, *o_ids, *o_off, *o_lp_min, *o_loss_max;
    long long k, n_tokens, n_docs, n_docs_global, n_tokens_global;
    int per_token;
    if (!PyArg_ParseTuple(args, "OOOOOLLLLLOOp", &o_teacher, &o_mask, &o_roll, &o_ids, &o_off, &k, &n_tokens,
                          &n_docs, &n_docs_global, &n_tokens_global, &o_lp_min, &o_loss_max, &per_token))
        return nullptr;
    at::NoGradGuard no_grad;
    auto in = std::make_shared<Inputs<meshy_distill_args>>();
    Reader rd(in->keep);
    at::Tensor teacher, mask, roll, ids, off;
    if (!rd.tensor(o_teacher, "teacher_topk_logprobs", teacher) || !rd.tensor(o_mask, "mask", mask) ||
        !rd.tensor(o_ids, "doc_ids", ids) || !rd.tensor(o_roll, "rollout_logprobs", roll) ||
        !rd.tensor(o_off, "seg_offsets", off))
        return nullptr;
    const char* tok_fmt = "the student has %lld tokens but %s has %lld";
    if (teacher.numel() != n_tokens * k &&
        bad_tokens(tok_fmt, "teacher_topk_logprobs", n_tokens, k > 0 ? teacher.numel() / k : teacher.numel()))
        return nullptr;
    for (auto [name, t] : {Named{"mask", &mask}, Named{"doc_ids", &ids}, Named{"rollout_logprobs", &roll}}) {
        if (t->defined() && t->numel() != n_tokens && bad_tokens(tok_fmt, name, n_tokens, t->numel())) return nullptr;
    }
    if (off.scalar_type() != at::kLong || !off.is_contiguous() || off.numel() < n_docs + 2) {
        PyErr_SetString(PyExc_ValueError, "seg_offsets must be n_docs + 2 contiguous int64 values");
        return nullptr;
    }
    meshy_distill_args& a = in->args;
    a.teacher = rd.flat<float>(teacher, at::kFloat);
    a.mask = rd.flat<float>(mask, at::kFloat);
    a.rollout_lp = rd.flat<float>(roll, at::kFloat);
    a.doc_ids = rd.flat<int64_t>(ids, at::kLong);
    a.seg_offsets = rd.flat<int64_t>(off, at::kLong);
    a.n_tokens = n_tokens;
    a.n_docs = n_docs;
    a.k = k;
    a.n_docs_global = n_docs_global;
    a.n_tokens_global = n_tokens_global;
    a.has_lp_clamp = o_lp_min != Py_None;
    a.lp_min_clamp = a.has_lp_clamp ? static_cast<float>(PyFloat_AsDouble(o_lp_min)) : 0.f;
    a.has_loss_clamp = o_loss_max != Py_None;
    a.loss_max_clamp = a.has_loss_clamp ? static_cast<float>(PyFloat_AsDouble(o_loss_max)) : 0.f;
    if (PyErr_Occurred()) return nullptr;
    a.per_token_loss = per_token;
    a.workspace = rd.workspace(meshy_distill_workspace_size(n_tokens, n_docs), a.workspace_bytes);
    return wrap_inputs(std::move(in));
    END_HANDLE_TH_ERRORS
}

// args_bytes(capsule) -> the bytes of its argument struct (for callers that
// drive the C ABI themselves).
PyObject* args_bytes(PyObject*, PyObject* cap) {
    if (PyCapsule_IsValid(cap, capsule_name<meshy_ppo_args>())) {
        const auto* in = unpack_inputs<meshy_ppo_args>(cap);
        return PyBytes_FromStringAndSize(reinterpret_cast<const char*>(&(*in)->args), sizeof(meshy_ppo_args));
    }
    const auto* in = unpack_inputs<meshy_distill_args>(cap);
    if (!in) return nullptr;
    return PyBytes_FromStringAndSize(reinterpret_cast<const char*>(&(*in)->args), sizeof(meshy_distill_args));
}

PyMethodDef kMethods[] = {
    {"ppo_inputs", ppo_inputs, METH_VARARGS, "Capsule of the PPO loss's inputs (argument struct and tensors)."},
    {"distill_inputs", distill_inputs, METH_VARARGS,
     "Capsule of the distillation loss's inputs (argument struct and tensors)."},
    {"args_bytes", args_bytes, METH_O, "The bytes of an inputs capsule's argument struct."},
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
