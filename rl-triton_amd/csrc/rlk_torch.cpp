// rlk_torch.cpp -- the thin PyTorch-ROCm extension over the C ABI (include/rl_triton_amd.h).
//
// Python module rl_triton._rlk_torch.  One function per estimator takes the public API's
// arguments as they were passed.  When the call can go to the C ABI as it stands, the
// function allocates the outputs, launches on torch's current stream and returns them.
// That needs every tensor to be a contiguous tensor of the expected dtype (float32, or
// bfloat16 throughout) and shape on the current GPU, RL_TRITON_CORRECTNESS_WARNINGS unset,
// and, for rows long enough to need a look-back workspace, a stream that is not capturing
// a graph (captured calls get buffers of their own on the Python path).  Any other call
// returns None, and the Python implementation takes its general path: the reference's
// assertions and contiguous copies.  A call that is taken gives the results the general
// path would give, and a malformed call never reaches a kernel from here.
// The public functions themselves are Entry objects (below) over these functions.
//
// The point is host time.  At [4096, 128] a kernel runs ~4 us; the Python path costs ~10 us
// per call (argument checks in Python, ctypes conversion), this one ~3.5 us, most of it the
// HIP runtime's own launch.
#include <Python.h>

#include <ATen/ATen.h>
#include <ATen/hip/EmptyTensor.h>
#include <c10/hip/HIPFunctions.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/python_variable.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <type_traits>
#include <utility>

#include "rl_triton_amd.h"

namespace {

bool correctness_warnings() {
  const char* v = std::getenv("RL_TRITON_CORRECTNESS_WARNINGS");
  return v != nullptr && std::strcmp(v, "1") == 0;
}

// A call this path declines: the Python wrapper handles it.
PyObject* decline() { Py_RETURN_NONE; }

struct Call {
  c10::DeviceIndex dev = -1;
  int64_t E = 0, T = 0;
  at::ScalarType io = at::kFloat;  // the storage type of every float tensor of the call
  bool ok = true;

  bool bf16() const { return io == at::kBFloat16; }

  // The leading [E, T] float32 or bfloat16 tensor: fixes device, shape and storage type
  // for the rest.
  const at::Tensor* lead(PyObject* o) {
    if (!ok || !THPVariable_Check(o)) return fail();
    const at::Tensor& t = THPVariable_Unpack(o);
    io = t.scalar_type();
    if (!t.is_cuda() || t.dim() != 2 || (io != at::kFloat && io != at::kBFloat16) ||
        !t.is_contiguous())
      return fail();
    dev = t.get_device();
    E = t.size(0);
    T = t.size(1);
    if (dev != c10::hip::current_device()) return fail();
    return &t;
  }
  // A tensor of shape [E, T] (or [E] / [E, T, A]) on the same device, of the call's storage
  // type unless `st` names another.
  const at::Tensor* need(PyObject* o, int kind = 2, int64_t A = 0,
                         at::ScalarType st = at::ScalarType::Undefined) {
    if (st == at::ScalarType::Undefined) st = io;
    if (!ok || !THPVariable_Check(o)) return fail();
    const at::Tensor& t = THPVariable_Unpack(o);
    if (!t.is_cuda() || t.get_device() != dev || t.scalar_type() != st || !t.is_contiguous())
      return fail();
    const bool shape_ok = kind == 1   ? (t.dim() == 1 && t.size(0) == E)
                        : kind == 2   ? (t.dim() == 2 && t.size(0) == E && t.size(1) == T)
                                      : (t.dim() == 3 && t.size(0) == E && t.size(1) == T &&
                                         t.size(2) == A);
    if (!shape_ok) return fail();
    return &t;
  }
  const at::Tensor* opt(PyObject* o, int kind = 2) { return o == Py_None ? nullptr : need(o, kind); }
  float scalar(PyObject* o) {
    if (!ok) return 0.f;
    if (PyFloat_CheckExact(o)) return (float)PyFloat_AS_DOUBLE(o);
    if (PyLong_CheckExact(o) || PyFloat_Check(o)) {
      const double d = PyFloat_AsDouble(o);
      if (d == -1.0 && PyErr_Occurred()) {
        PyErr_Clear();
        fail();
        return 0.f;
      }
      return (float)d;
    }
    fail();
    return 0.f;
  }
  const at::Tensor* fail() {
    ok = false;
    return nullptr;
  }
  void* stream() const { return c10::hip::getCurrentHIPStream(dev).stream(); }
  // the output, allocated directly by the HIP backend (no operator dispatch)
  at::Tensor output(const at::Tensor& like) const {
    return at::Tensor(at::detail::empty_cuda({E, T}, like.scalar_type(), like.device(), std::nullopt));
  }
};

// Look-back workspaces of the calls this module launches, one per (device, stream):
// zero-filled when allocated (on that stream), grown by doubling, and left ready by every
// call for the next.  Calls on one stream are ordered, so one buffer serves them all, and
// the caching allocator keeps a replaced buffer until the stream's earlier work is done.
// (The Python path keeps workspaces of its own; a workspace is only ever shared by calls
// on one stream, whichever path they take.)  The GIL guards the map.  It is never
// destroyed: tensors must not be freed after the HIP allocator has gone at process exit.
std::map<std::pair<int, uintptr_t>, at::Tensor>& workspaces() {
  static auto* m = new std::map<std::pair<int, uintptr_t>, at::Tensor>();
  return *m;
}

// Long-row calls served by each cached workspace since it was last zero-filled.  Its status
// words carry a 30-bit count of the calls made on it, which wraps after 2^30 calls; a word
// left 2^30 calls earlier would then read as current.  So a workspace is zero-filled again
// (on its stream, before the call) once it has served g_ws_max_calls calls: the C ABI's
// RLK_WORKSPACE_MAX_CALLS, lowered only by tests (set_workspace_max_calls).
std::map<std::pair<int, uintptr_t>, uint64_t>& workspace_calls() {
  static auto* m = new std::map<std::pair<int, uintptr_t>, uint64_t>();
  return *m;
}
uint64_t g_ws_max_calls = RLK_WORKSPACE_MAX_CALLS;
uint64_t g_ws_clears = 0;

struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
  bool ok = true;  // false: decline (a graph capture is in progress on the stream)
};

Workspace workspace(const Call& c, const at::Tensor& like) {
  Workspace w;
  if (!c.ok) return w;
  const size_t need = rlk_workspace_bytes(c.E, c.T);
  if (need == 0) return w;
  hipStream_t s = static_cast<hipStream_t>(c.stream());
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    w.ok = false;
    return w;
  }
  const std::pair<int, uintptr_t> key{(int)c.dev, reinterpret_cast<uintptr_t>(s)};
  at::Tensor& buf = workspaces()[key];
  uint64_t& calls = workspace_calls()[key];
  if (!buf.defined() || (size_t)buf.numel() < need) {
    size_t size = buf.defined() ? std::max(need, 2 * (size_t)buf.numel()) : need;
    size = (size + 255) / 256 * 256;
    buf = at::zeros({(int64_t)size}, like.options().dtype(at::kByte));
    calls = 0;
  }
  if (calls >= g_ws_max_calls) {
    buf.zero_();  // a fill kernel on the current stream, before this call's launch
    ++g_ws_clears;
    calls = 0;
  }
  ++calls;
  w.ptr = buf.data_ptr();
  w.bytes = (size_t)buf.numel();
  return w;
}

// Typed data pointers (T = float or rlk_bf16) of an input (nullable) and of an output.
template <class T>
const T* in_ptr(const at::Tensor* t) {
  return t ? static_cast<const T*>(t->data_ptr()) : nullptr;
}
template <class T>
T* out_ptr(at::Tensor& t) {
  return static_cast<T*>(t.data_ptr());
}

// The entry point for storage type T: `f32` for float, its `_bf16` twin for rlk_bf16.
template <class T, class F32, class BF16>
constexpr auto pick(F32 f32, BF16 bf16) {
  if constexpr (std::is_same_v<T, float>) return f32;
  else return bf16;
}

// Runs `body` with a value of the call's storage type; body(x) picks the entry point and
// pointer types from decltype(x).
template <class Body>
int dispatch(const Call& c, Body body) {
  return c.bf16() ? body(rlk_bf16{}) : body(0.f);
}

// Calls this module has launched (a diagnostic for tests: which path served a call).
uint64_t g_launched = 0;

PyObject* finish(int status, const char* what, PyObject* result) {
  ++g_launched;
  if (status != RLK_OK) {
    Py_XDECREF(result);
    PyErr_Format(PyExc_RuntimeError, "%s failed: %s (status %d)", what, rlk_status_string(status),
                 status);
    return nullptr;
  }
  return result;
}

PyObject* pair(at::Tensor& a, at::Tensor& b) {
  PyObject* t = PyTuple_New(2);
  if (!t) return nullptr;
  PyTuple_SET_ITEM(t, 0, THPVariable_Wrap(std::move(a)));
  PyTuple_SET_ITEM(t, 1, THPVariable_Wrap(std::move(b)));
  return t;
}

// The call's tensors' host metadata, requested level by level before the checks read it.
// A caller's tensors whose metadata has gone cold (built long before the call, or untouched
// since) miss in the host caches at each step of PyObject -> TensorImpl -> StorageImpl, and
// the checks walk the tensors one after another.  Requesting every tensor's TensorImpl,
// then every StorageImpl, overlaps those misses across the call's tensors.  Measured on
// MI355X's host, the driver's 20-step GAE + V-trace loop on cold sets: 10.96 -> 10.34 us
// per step (mean of four fresh processes each, same box); warm calls unchanged.
void prefetch_tensors(PyObject* const* a, Py_ssize_t n) {
  const c10::TensorImpl* impl[16];
  int k = 0;
  for (Py_ssize_t i = 0; i < n && k < 16; ++i)  // tensors (not subclasses): a type compare
    if (THPVariable_CheckExact(a[i])) impl[k++] = THPVariable_Unpack(a[i]).unsafeGetTensorImpl();
  for (int j = 0; j < k; ++j)
    for (size_t off = 0; off < sizeof(c10::TensorImpl); off += 64)
      __builtin_prefetch(reinterpret_cast<const char*>(impl[j]) + off);
  for (int j = 0; j < k; ++j) {
    const c10::StorageImpl* st = impl[j]->unsafe_storage().unsafeGetStorageImpl();
    if (st != nullptr) {
      __builtin_prefetch(st);
      __builtin_prefetch(reinterpret_cast<const char*>(st) + 64);
    }
  }
}

bool nargs_is(Py_ssize_t n, Py_ssize_t want, const char* name) {
  if (n == want) return true;
  PyErr_Format(PyExc_TypeError, "%s expects %zd arguments, got %zd", name, want, n);
  return false;
}

// gae(rewards, values, terminateds, truncateds, gamma, lambda_, bootstrap_values, last_value,
//     mask)
PyObject* op_gae(PyObject* const* a, Py_ssize_t n) {
  if (!nargs_is(n, 9, "gae")) return nullptr;
  prefetch_tensors(a, n);
  if (correctness_warnings()) return decline();
  Call c;
  const at::Tensor* r = c.lead(a[0]);
  const at::Tensor* v = c.need(a[1]);
  const at::Tensor* te = c.need(a[2]);
  const at::Tensor* tr = c.opt(a[3]);
  const float gamma = c.scalar(a[4]), lam = c.scalar(a[5]);
  const bool has_bv = a[6] != Py_None, has_lv = a[7] != Py_None;
  if (has_bv && has_lv) return decline();  // the wrapper raises "not both"
  if (has_lv && tr) return decline();      // ... and "cannot be combined with truncateds"
  const at::Tensor* boot = has_lv ? c.need(a[7], 1) : c.opt(a[6]);
  const at::Tensor* mask = c.opt(a[8]);
  if (!c.ok) return decline();
  const int mode = has_lv ? RLK_BOOT_ROW : has_bv ? RLK_BOOT_FULL : RLK_BOOT_NONE;
  const Workspace ws = workspace(c, *r);
  if (!ws.ok) return decline();
  at::Tensor out = c.output(*r);
  const int st = dispatch(c, [&](auto z) {
    using T = decltype(z);
    if (mask)
      return pick<T>(rlk_gae_masked, rlk_gae_masked_bf16)(in_ptr<T>(r), in_ptr<T>(v),
        in_ptr<T>(te), in_ptr<T>(tr), in_ptr<T>(boot), mode, in_ptr<T>(mask), out_ptr<T>(out),
        c.E, c.T, gamma, lam, ws.ptr, ws.bytes, c.stream());
    return pick<T>(rlk_gae, rlk_gae_bf16)(in_ptr<T>(r), in_ptr<T>(v), in_ptr<T>(te), in_ptr<T>(tr),
      in_ptr<T>(boot), mode, out_ptr<T>(out), c.E, c.T, gamma, lam, ws.ptr, ws.bytes, c.stream());
  });
  return finish(st, mask ? "rlk_gae_masked" : "rlk_gae", THPVariable_Wrap(std::move(out)));
}

// gae_normalized(rewards, values, terminateds, truncateds, gamma, lambda_, bootstrap_values,
//                last_value, eps, mask) -> (advantages, returns)
PyObject* op_gae_normalized(PyObject* const* a, Py_ssize_t n) {
  if (!nargs_is(n, 10, "gae_normalized")) return nullptr;
  prefetch_tensors(a, n);
  if (correctness_warnings()) return decline();
  Call c;
  const at::Tensor* r = c.lead(a[0]);
  const at::Tensor* v = c.need(a[1]);
  const at::Tensor* te = c.need(a[2]);
  const at::Tensor* tr = c.opt(a[3]);
  const float gamma = c.scalar(a[4]), lam = c.scalar(a[5]), eps = c.scalar(a[8]);
  const bool has_bv = a[6] != Py_None, has_lv = a[7] != Py_None;
  if (has_bv && has_lv) return decline();
  if (has_lv && tr) return decline();
  const at::Tensor* boot = has_lv ? c.need(a[7], 1) : c.opt(a[6]);
  const at::Tensor* mask = c.opt(a[9]);
  if (!c.ok) return decline();
  const int mode = has_lv ? RLK_BOOT_ROW : has_bv ? RLK_BOOT_FULL : RLK_BOOT_NONE;
  const Workspace ws = workspace(c, *r);
  if (!ws.ok) return decline();
  at::Tensor adv = c.output(*r), ret = c.output(*r);
  const size_t pb = rlk_gae_normalized_partials_bytes(c.E, c.T);
  at::Tensor parts = at::empty({(int64_t)(pb > 0 ? pb : 8)}, r->options().dtype(at::kByte));
  const int st = dispatch(c, [&](auto z) {
    using T = decltype(z);
    if (mask)
      return pick<T>(rlk_gae_normalized_masked, rlk_gae_normalized_masked_bf16)(
        in_ptr<T>(r), in_ptr<T>(v), in_ptr<T>(te), in_ptr<T>(tr), in_ptr<T>(boot), mode,
        in_ptr<T>(mask), out_ptr<T>(adv), out_ptr<T>(ret), c.E, c.T, gamma, lam, eps, ws.ptr, ws.bytes,
        parts.data_ptr(), pb, c.stream());
    return pick<T>(rlk_gae_normalized, rlk_gae_normalized_bf16)(in_ptr<T>(r), in_ptr<T>(v),
      in_ptr<T>(te), in_ptr<T>(tr), in_ptr<T>(boot), mode, out_ptr<T>(adv), out_ptr<T>(ret),
      c.E, c.T, gamma, lam, eps, ws.ptr, ws.bytes, parts.data_ptr(), pb, c.stream());
  });
  return finish(st, mask ? "rlk_gae_normalized_masked" : "rlk_gae_normalized", pair(adv, ret));
}

// vtrace(log_pi_target, log_pi_behavior, values, rewards, terminateds, truncateds, gamma,
//        rho_bar, c_bar, bootstrap_values, last_value)
PyObject* op_vtrace(PyObject* const* a, Py_ssize_t n) {
  if (!nargs_is(n, 11, "vtrace")) return nullptr;
  prefetch_tensors(a, n);
  if (correctness_warnings()) return decline();
  Call c;
  const at::Tensor* r = c.lead(a[3]);
  const at::Tensor* lpt = c.need(a[0]);
  const at::Tensor* lpb = c.need(a[1]);
  const at::Tensor* v = c.need(a[2]);
  const at::Tensor* te = c.need(a[4]);
  const at::Tensor* tr = c.opt(a[5]);
  const float gamma = c.scalar(a[6]), rho_bar = c.scalar(a[7]), c_bar = c.scalar(a[8]);
  const bool has_bv = a[9] != Py_None, has_lv = a[10] != Py_None;
  if (has_bv && has_lv) return decline();
  const at::Tensor* boot = has_lv ? c.need(a[10], 1) : c.opt(a[9]);
  if (!c.ok) return decline();
  const int mode = has_lv ? RLK_BOOT_ROW : has_bv ? RLK_BOOT_FULL : RLK_BOOT_NONE;
  const Workspace ws = workspace(c, *r);
  if (!ws.ok) return decline();
  at::Tensor tg = c.output(*r), adv = c.output(*r);
  const int st = dispatch(c, [&](auto z) {
    using T = decltype(z);
    return pick<T>(rlk_vtrace, rlk_vtrace_bf16)(in_ptr<T>(lpt), in_ptr<T>(lpb), in_ptr<T>(v),
      in_ptr<T>(r), in_ptr<T>(te), in_ptr<T>(tr), in_ptr<T>(boot), mode, out_ptr<T>(tg),
      out_ptr<T>(adv), c.E, c.T, gamma, rho_bar, c_bar, ws.ptr, ws.bytes, c.stream());
  });
  return finish(st, "rlk_vtrace", pair(tg, adv));
}

// retrace(action_probs_target, action_probs_behavior, q_values, next_q_values_all, actions,
//         rewards, terminateds, truncateds, gamma, lambda_, c_bar, rho_bar)
PyObject* op_retrace(PyObject* const* a, Py_ssize_t n) {
  if (!nargs_is(n, 12, "retrace")) return nullptr;
  prefetch_tensors(a, n);
  if (correctness_warnings()) return decline();
  Call c;
  const at::Tensor* r = c.lead(a[5]);
  int64_t A = 0;
  if (c.ok && THPVariable_Check(a[0])) {
    const at::Tensor& pi = THPVariable_Unpack(a[0]);
    if (pi.dim() == 3) A = pi.size(2);
  }
  if (A <= 0 || A > (1 << 20)) return decline();
  const at::Tensor* pi = c.need(a[0], 3, A);
  const at::Tensor* mu = c.need(a[1]);
  const at::Tensor* q = c.need(a[2]);
  const at::Tensor* nq = c.need(a[3], 3, A);
  const at::Tensor* act = c.need(a[4], 2, 0, at::kLong);
  const at::Tensor* te = c.need(a[6]);
  const at::Tensor* tr = c.need(a[7]);
  const float gamma = c.scalar(a[8]), lam = c.scalar(a[9]), c_bar = c.scalar(a[10]),
              rho_bar = c.scalar(a[11]);
  if (!c.ok) return decline();
  const Workspace ws = workspace(c, *r);
  if (!ws.ok) return decline();
  at::Tensor tg = c.output(*r), adv = c.output(*r);
  const int st = dispatch(c, [&](auto z) {
    using T = decltype(z);
    return pick<T>(rlk_retrace, rlk_retrace_bf16)(in_ptr<T>(pi), in_ptr<T>(mu), in_ptr<T>(q),
      in_ptr<T>(nq), act->data_ptr<int64_t>(), in_ptr<T>(r), in_ptr<T>(te), in_ptr<T>(tr),
      out_ptr<T>(tg), out_ptr<T>(adv), c.E, c.T, A, gamma, lam, c_bar, rho_bar, ws.ptr, ws.bytes,
      c.stream());
  });
  return finish(st, "rlk_retrace", pair(tg, adv));
}

// lambda_returns(rewards, next_values, terminateds, truncateds, gamma, lambda_, bootstrap_values)
PyObject* op_lambda_returns(PyObject* const* a, Py_ssize_t n) {
  if (!nargs_is(n, 7, "lambda_returns")) return nullptr;
  prefetch_tensors(a, n);
  if (correctness_warnings()) return decline();
  Call c;
  const at::Tensor* r = c.lead(a[0]);
  const at::Tensor* nv = c.need(a[1]);
  const at::Tensor* te = c.need(a[2]);
  const at::Tensor* tr = c.opt(a[3]);
  const float gamma = c.scalar(a[4]), lam = c.scalar(a[5]);
  const at::Tensor* boot = c.opt(a[6]);
  if (!c.ok) return decline();
  const Workspace ws = workspace(c, *r);
  if (!ws.ok) return decline();
  at::Tensor out = c.output(*r);
  const int st = dispatch(c, [&](auto z) {
    using T = decltype(z);
    return pick<T>(rlk_lambda_returns, rlk_lambda_returns_bf16)(in_ptr<T>(r), in_ptr<T>(nv),
      in_ptr<T>(te), in_ptr<T>(tr), in_ptr<T>(boot), boot ? RLK_BOOT_FULL : RLK_BOOT_NONE,
      out_ptr<T>(out), c.E, c.T, gamma, lam, ws.ptr, ws.bytes, c.stream());
  });
  return finish(st, "rlk_lambda_returns", THPVariable_Wrap(std::move(out)));
}

// discounted_returns(rewards, terminateds, truncateds, gamma, bootstrap_values)
PyObject* op_discounted_returns(PyObject* const* a, Py_ssize_t n) {
  if (!nargs_is(n, 5, "discounted_returns")) return nullptr;
  prefetch_tensors(a, n);
  if (correctness_warnings()) return decline();
  Call c;
  const at::Tensor* r = c.lead(a[0]);
  const at::Tensor* te = c.need(a[1]);
  const at::Tensor* tr = c.opt(a[2]);
  const float gamma = c.scalar(a[3]);
  const at::Tensor* boot = c.opt(a[4]);
  if (!c.ok) return decline();
  const Workspace ws = workspace(c, *r);
  if (!ws.ok) return decline();
  at::Tensor out = c.output(*r);
  const int st = dispatch(c, [&](auto z) {
    using T = decltype(z);
    return pick<T>(rlk_discounted_returns, rlk_discounted_returns_bf16)(in_ptr<T>(r), in_ptr<T>(te),
      in_ptr<T>(tr), in_ptr<T>(boot), boot ? RLK_BOOT_FULL : RLK_BOOT_NONE, out_ptr<T>(out), c.E,
      c.T, gamma, ws.ptr, ws.bytes, c.stream());
  });
  return finish(st, "rlk_discounted_returns", THPVariable_Wrap(std::move(out)));
}

// eligibility_traces(gradients, dones, gamma, lambda_, seed_values)
PyObject* op_eligibility_traces(PyObject* const* a, Py_ssize_t n) {
  if (!nargs_is(n, 5, "eligibility_traces")) return nullptr;
  prefetch_tensors(a, n);
  if (correctness_warnings()) return decline();
  Call c;
  const at::Tensor* g = c.lead(a[0]);
  const at::Tensor* d = c.need(a[1]);
  const float gamma = c.scalar(a[2]), lam = c.scalar(a[3]);
  const at::Tensor* seed = c.opt(a[4], 1);
  if (!c.ok) return decline();
  const Workspace ws = workspace(c, *g);
  if (!ws.ok) return decline();
  at::Tensor out = c.output(*g);
  const int st = dispatch(c, [&](auto z) {
    using T = decltype(z);
    return pick<T>(rlk_eligibility_traces, rlk_eligibility_traces_bf16)(in_ptr<T>(g), in_ptr<T>(d),
      in_ptr<T>(seed), out_ptr<T>(out), c.E, c.T, gamma, lam, ws.ptr, ws.bytes, c.stream());
  });
  return finish(st, "rlk_eligibility_traces", THPVariable_Wrap(std::move(out)));
}

// prefix_sum(inputs, dones, seed_values, ends_at)   (ends_at: the boundary, already checked)
PyObject* op_prefix_sum(PyObject* const* a, Py_ssize_t n) {
  if (!nargs_is(n, 4, "prefix_sum")) return nullptr;
  prefetch_tensors(a, n);
  if (correctness_warnings()) return decline();
  Call c;
  const at::Tensor* x = c.lead(a[0]);
  const at::Tensor* d = c.need(a[1]);
  const at::Tensor* seed = c.opt(a[2], 1);
  if (!c.ok || !PyBool_Check(a[3])) return decline();
  const Workspace ws = workspace(c, *x);
  if (!ws.ok) return decline();
  at::Tensor out = c.output(*x);
  const int st = dispatch(c, [&](auto z) {
    using T = decltype(z);
    return pick<T>(rlk_prefix_sum, rlk_prefix_sum_bf16)(in_ptr<T>(x), in_ptr<T>(d), in_ptr<T>(seed),
      out_ptr<T>(out), c.E, c.T, a[3] == Py_True ? 1 : 0, ws.ptr, ws.bytes, c.stream());
  });
  return finish(st, "rlk_prefix_sum", THPVariable_Wrap(std::move(out)));
}

// affine_scan(u, v, carry, direction)
PyObject* op_affine_scan(PyObject* const* a, Py_ssize_t n) {
  if (!nargs_is(n, 4, "affine_scan")) return nullptr;
  prefetch_tensors(a, n);
  if (correctness_warnings()) return decline();
  Call c;
  const at::Tensor* u = c.lead(a[0]);
  const at::Tensor* v = c.need(a[1]);
  const at::Tensor* carry = c.opt(a[2], 1);
  const long dir = PyLong_CheckExact(a[3]) ? PyLong_AsLong(a[3]) : -1;
  if (!c.ok || (dir != RLK_BACKWARD && dir != RLK_FORWARD)) return decline();
  const Workspace ws = workspace(c, *u);
  if (!ws.ok) return decline();
  at::Tensor out = c.output(*u);
  const int st = dispatch(c, [&](auto z) {
    using T = decltype(z);
    return pick<T>(rlk_affine_scan, rlk_affine_scan_bf16)(in_ptr<T>(u), in_ptr<T>(v),
      in_ptr<T>(carry), out_ptr<T>(out), c.E, c.T, (int)dir, ws.ptr, ws.bytes, c.stream());
  });
  return finish(st, "rlk_affine_scan", THPVariable_Wrap(std::move(out)));
}

// C++ exceptions (an allocation that fails, say) must not cross into the interpreter: such
// a call is declined, and the Python path raises torch's own exception for it.
template <PyObject* (*F)(PyObject* const*, Py_ssize_t)>
PyObject* guarded(PyObject*, PyObject* const* a, Py_ssize_t n) {
  try {
    return F(a, n);
  } catch (...) {
    return decline();
  }
}

// ------------------------------------------------------------------------------------------
// The public functions themselves.  rl_triton.compute_* are instances of Entry: each binds
// its Python implementation's signature (positional or keyword arguments, defaults), takes
// the fast path, and hands every call the fast path does not take -- declined, malformed,
// unknown or repeated keywords -- to the Python implementation with its arguments exactly as
// given, so every check, message and result outside the fast path is the Python path's.
// This saves the Python frame (~0.8 us of host time per call); signatures, defaults and
// docstrings come from the Python functions (rl_triton/_native.py builds the entries).
// ------------------------------------------------------------------------------------------
using FastOp = PyObject* (*)(PyObject*, PyObject* const*, Py_ssize_t);

// prefix_sum's public argument is boundary="ends_at" | "starts_at"; its fast op takes a bool
PyObject* op_prefix_sum_api(PyObject* const* a, Py_ssize_t n) {
  if (n != 4 || !PyUnicode_Check(a[3])) return decline();
  PyObject* ends_at;
  if (PyUnicode_CompareWithASCIIString(a[3], "ends_at") == 0) ends_at = Py_True;
  else if (PyUnicode_CompareWithASCIIString(a[3], "starts_at") == 0) ends_at = Py_False;
  else return decline();  // the Python path raises its ValueError
  PyObject* b[4] = {a[0], a[1], a[2], ends_at};
  return op_prefix_sum(b, 4);
}

constexpr int kMaxParams = 16;

struct Entry {
  PyObject_HEAD
  vectorcallfunc vectorcall;
  PyObject* dict;
  PyObject* fallback;  // the Python implementation
  FastOp op;
  int nparams, npos;
  PyObject* names[kMaxParams];     // parameter names (str)
  PyObject* defaults[kMaxParams];  // nullptr: required
};

// Binds a call to the parameter list; false for anything the fast path should not interpret.
bool bind(const Entry* e, PyObject* const* args, Py_ssize_t nargs, PyObject* kwnames,
          PyObject** bound) {
  if (nargs > e->npos) return false;
  for (int i = 0; i < e->nparams; ++i) bound[i] = i < nargs ? args[i] : nullptr;
  const Py_ssize_t nkw = kwnames ? PyTuple_GET_SIZE(kwnames) : 0;
  for (Py_ssize_t j = 0; j < nkw; ++j) {
    PyObject* key = PyTuple_GET_ITEM(kwnames, j);
    int found = -1;
    for (int i = 0; i < e->nparams && found < 0; ++i)
      if (key == e->names[i]) found = i;  // keyword names are usually the interned literals
    for (int i = 0; i < e->nparams && found < 0; ++i) {
      const int c = PyUnicode_Compare(key, e->names[i]);
      if (c == -1 && PyErr_Occurred()) {
        PyErr_Clear();
        return false;
      }
      if (c == 0) found = i;
    }
    if (found < 0 || bound[found] != nullptr) return false;
    bound[found] = args[nargs + j];
  }
  for (int i = 0; i < e->nparams; ++i) {
    if (bound[i] == nullptr) {
      if (e->defaults[i] == nullptr) return false;
      bound[i] = e->defaults[i];
    }
  }
  return true;
}

PyObject* entry_call(PyObject* self, PyObject* const* args, size_t nargsf, PyObject* kwnames) {
  Entry* e = reinterpret_cast<Entry*>(self);
  const Py_ssize_t nargs = PyVectorcall_NARGS(nargsf);
  PyObject* bound[kMaxParams];
  if (bind(e, args, nargs, kwnames, bound)) {
    PyObject* r = e->op(nullptr, bound, e->nparams);
    if (r == nullptr || r != Py_None) return r;  // a result, or an error of the launch itself
    Py_DECREF(r);
  }
  return PyObject_Vectorcall(e->fallback, args, nargs, kwnames);
}

void entry_dealloc(PyObject* self) {
  Entry* e = reinterpret_cast<Entry*>(self);
  Py_CLEAR(e->dict);
  Py_CLEAR(e->fallback);
  for (int i = 0; i < e->nparams; ++i) {
    Py_CLEAR(e->names[i]);
    Py_CLEAR(e->defaults[i]);
  }
  Py_TYPE(self)->tp_free(self);
}

PyGetSetDef kEntryGetSet[] = {
    {"__dict__", PyObject_GenericGetDict, PyObject_GenericSetDict, nullptr, nullptr},
    {nullptr, nullptr, nullptr, nullptr, nullptr}};

PyTypeObject EntryType = {PyVarObject_HEAD_INIT(nullptr, 0)};

#define RLK_METHOD(name) \
  { #name, (PyCFunction)(void (*)(void))guarded<op_##name>, METH_FASTCALL, nullptr }

struct OpName {
  const char* name;
  FastOp op;
};
const OpName kOps[] = {
    {"gae", guarded<op_gae>},
    {"gae_normalized", guarded<op_gae_normalized>},
    {"vtrace", guarded<op_vtrace>},
    {"retrace", guarded<op_retrace>},
    {"lambda_returns", guarded<op_lambda_returns>},
    {"discounted_returns", guarded<op_discounted_returns>},
    {"eligibility_traces", guarded<op_eligibility_traces>},
    {"prefix_sum", guarded<op_prefix_sum_api>},
};

// entry(op, names, npos, defaults, required, fallback): a public function over fast op `op`
// (a name of kOps) with parameters `names` (the first `npos` positional), `defaults` aligned
// with them (the object `required` marks a parameter without one), falling back to `fallback`.
PyObject* make_entry(PyObject*, PyObject* args) {
  const char* opname;
  PyObject *names, *defaults, *required, *fallback;
  int npos;
  if (!PyArg_ParseTuple(args, "sO!iO!OO:entry", &opname, &PyTuple_Type, &names, &npos, &PyTuple_Type,
                        &defaults, &required, &fallback))
    return nullptr;
  FastOp op = nullptr;
  for (const OpName& o : kOps)
    if (std::strcmp(o.name, opname) == 0) op = o.op;
  const Py_ssize_t n = PyTuple_GET_SIZE(names);
  if (!op || n > kMaxParams || PyTuple_GET_SIZE(defaults) != n || npos < 0 || npos > n ||
      !PyCallable_Check(fallback)) {
    PyErr_SetString(PyExc_ValueError, "entry: bad arguments");
    return nullptr;
  }
  Entry* e = PyObject_New(Entry, &EntryType);
  if (!e) return nullptr;
  e->vectorcall = entry_call;
  e->dict = nullptr;
  e->op = op;
  e->nparams = (int)n;
  e->npos = npos;
  Py_INCREF(fallback);
  e->fallback = fallback;
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* nm = PyTuple_GET_ITEM(names, i);
    PyObject* d = PyTuple_GET_ITEM(defaults, i);
    Py_INCREF(nm);
    PyUnicode_InternInPlace(&nm);
    e->names[i] = nm;
    e->defaults[i] = d == required ? nullptr : (Py_INCREF(d), d);
  }
  return reinterpret_cast<PyObject*>(e);
}

PyObject* launched(PyObject*, PyObject*) { return PyLong_FromUnsignedLongLong(g_launched); }

// workspace_error(device) -> True if a workspace of this module on that device recorded a
// look-back wait that gave up (header word 3).  Reads the flags back: synchronises.
PyObject* workspace_error(PyObject*, PyObject* arg) {
  const long dev = PyLong_AsLong(arg);
  if (dev == -1 && PyErr_Occurred()) return nullptr;
  try {
    for (auto& kv : workspaces()) {
      if (kv.first.first != dev || !kv.second.defined()) continue;
      const at::Tensor flag = kv.second.narrow(0, 3 * 8, 8).to(at::kCPU);
      const uint8_t* b = flag.data_ptr<uint8_t>();
      for (int i = 0; i < 8; ++i)
        if (b[i] != 0) Py_RETURN_TRUE;
    }
  } catch (const std::exception& e) {
    PyErr_SetString(PyExc_RuntimeError, e.what());
    return nullptr;
  }
  Py_RETURN_FALSE;
}

// set_workspace_max_calls(n) -> the previous limit; n <= 0 restores
// RLK_WORKSPACE_MAX_CALLS.  For tests of the re-zeroing of cached workspaces.
PyObject* set_workspace_max_calls(PyObject*, PyObject* arg) {
  const long long n = PyLong_AsLongLong(arg);
  if (n == -1 && PyErr_Occurred()) return nullptr;
  const uint64_t prev = g_ws_max_calls;
  g_ws_max_calls = n <= 0 ? (uint64_t)RLK_WORKSPACE_MAX_CALLS : (uint64_t)n;
  return PyLong_FromUnsignedLongLong(prev);
}

PyObject* workspace_clears(PyObject*, PyObject*) { return PyLong_FromUnsignedLongLong(g_ws_clears); }

PyMethodDef kMethods[] = {
    {"entry", make_entry, METH_VARARGS, "entry(op, names, npos, defaults, required, fallback)"},
    {"set_workspace_max_calls", set_workspace_max_calls, METH_O,
     "set_workspace_max_calls(n) -> previous limit of long-row calls between zero-fills of a "
     "cached workspace (n <= 0: the default, RLK_WORKSPACE_MAX_CALLS)"},
    {"workspace_clears", workspace_clears, METH_NOARGS,
     "workspace_clears() -> cached workspaces zero-filled again at the call limit so far"},
    {"launched", launched, METH_NOARGS, "launched() -> calls the fast path has launched so far"},
    {"workspace_error", workspace_error, METH_O,
     "workspace_error(device) -> True if a look-back wait of this module's calls gave up"},
    RLK_METHOD(gae),
    RLK_METHOD(gae_normalized),
    RLK_METHOD(vtrace),
    RLK_METHOD(retrace),
    RLK_METHOD(lambda_returns),
    RLK_METHOD(discounted_returns),
    RLK_METHOD(eligibility_traces),
    RLK_METHOD(prefix_sum),
    RLK_METHOD(affine_scan),
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_rlk_torch",
                       "Tensor-level fast path of rl_triton over librl_triton_amd.so's C ABI.", -1,
                       kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__rlk_torch(void) {
  EntryType.tp_name = "rl_triton._rlk_torch.Entry";
  EntryType.tp_basicsize = sizeof(Entry);
  EntryType.tp_dealloc = entry_dealloc;
  EntryType.tp_vectorcall_offset = offsetof(Entry, vectorcall);
  EntryType.tp_call = PyVectorcall_Call;
  EntryType.tp_dictoffset = offsetof(Entry, dict);
  EntryType.tp_getset = kEntryGetSet;
  EntryType.tp_getattro = PyObject_GenericGetAttr;
  EntryType.tp_setattro = PyObject_GenericSetAttr;
  EntryType.tp_flags = Py_TPFLAGS_DEFAULT | Py_TPFLAGS_HAVE_VECTORCALL;
  EntryType.tp_doc = "A public rl_triton function: the C++ fast path over its Python implementation.";
  if (PyType_Ready(&EntryType) < 0) return nullptr;
  return PyModule_Create(&kModule);
}
