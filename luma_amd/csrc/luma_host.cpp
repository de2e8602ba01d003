// Host-side bookkeeping of LUMA.step for large parameter sets (the Python
// extension module luma_amd._luma_host).
//
// A step over the same parameters and gradient layout as the previous step
// re-uses its tensor table and only needs the current gradient and parameter
// pointers (the reference re-reads p.grad every step, optimizer.py:425-455).
// Reading p.grad, data_ptr() and the dtype of every parameter from Python
// costs about 1.2 us per tensor (24 ms for 20,000 tensors).  Here the same
// checks read the tensors' C++ objects directly.  Those objects lie scattered
// in host memory, so the walk is bound by memory latency: it runs in stages
// over arrays (parameter object -> TensorImpl -> autograd meta -> gradient
// TensorImpl -> data pointers) with software prefetch a few tensors ahead,
// and large sets are split over a few threads of a pool that lives as long as
// the process (made on first use, made again in a forked child).  The worker
// threads only read C++ objects while the calling thread holds the GIL, so
// nothing they read can change under them.  The module computes nothing of
// the step itself: the step runs in libluma_hip.so.
#include <ATen/core/Tensor.h>
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <torch/csrc/autograd/python_variable.h>

#include <unistd.h>

#include <algorithm>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace py = pybind11;

namespace {

// Gradient element type codes of the C ABI (LUMA_GRAD_*).
int grad_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return 0;
    case at::kBFloat16: return 1;
    case at::kHalf: return 2;
    default: return -1;
  }
}

constexpr int64_t kAhead = 8;             // prefetch distance, in tensors
constexpr int64_t kPerThread = 2048;      // parameters per thread, at least
constexpr int kMaxThreads = 8;            // the calling thread and up to 7 workers

// Workers that run part t of a job for t = 1 .. parts-1 while the calling
// thread runs part 0.  One job at a time (the callers hold the GIL).
class Pool {
 public:
  // The pool of this process; empty (run() then does every part on the
  // calling thread) when no thread could be started.
  static Pool &get() {
    static Pool *pool = nullptr;
    static pid_t owner = 0;
    if (!pool || owner != getpid()) {
      // a forked child inherits the memory but not the threads: it makes
      // its own pool (the parent's stays unused in the child)
      pool = new Pool(kMaxThreads - 1);
      owner = getpid();
    }
    return *pool;
  }

  void run(int parts, const std::function<void(int)> &fn) {
    const int use = std::min<int>(parts - 1, (int)threads_.size());
    {
      std::lock_guard<std::mutex> lock(mu_);
      fn_ = &fn;
      use_ = use;
      pending_ = use;
      ++gen_;
    }
    if (use > 0) wake_.notify_all();
    for (int t = use + 1; t < parts; ++t) fn(t);   // parts no worker took
    fn(0);
    std::unique_lock<std::mutex> lock(mu_);
    done_.wait(lock, [&] { return pending_ == 0; });
    fn_ = nullptr;
  }

 private:
  explicit Pool(int n) {
    for (int i = 0; i < n; ++i) {
      try {
        threads_.emplace_back([this, i] { loop(i + 1); });
      } catch (...) {
        break;
      }
    }
    for (std::thread &t : threads_) t.detach();
  }

  void loop(int part) {
    uint64_t seen = 0;
    for (;;) {
      const std::function<void(int)> *fn;
      {
        std::unique_lock<std::mutex> lock(mu_);
        wake_.wait(lock, [&] { return gen_ != seen; });
        seen = gen_;
        if (part > use_) continue;
        fn = fn_;
      }
      (*fn)(part);
      std::lock_guard<std::mutex> lock(mu_);
      if (--pending_ == 0) done_.notify_one();
    }
  }

  std::vector<std::thread> threads_;
  std::mutex mu_;
  std::condition_variable wake_, done_;
  const std::function<void(int)> *fn_ = nullptr;
  int use_ = 0, pending_ = 0;
  uint64_t gen_ = 0;
};

inline void prefetch(const void *p) { __builtin_prefetch(p, 0, 3); }

inline void prefetch_impl(const c10::TensorImpl *t) {
  const char *c = reinterpret_cast<const char *>(t);
  for (int off = 0; off < (int)sizeof(c10::TensorImpl); off += 64) prefetch(c + off);
}

// The Python types a planned parameter may have: torch.Tensor and
// torch.nn.Parameter (set at module import).
PyTypeObject *g_tensor_type = nullptr;
PyTypeObject *g_param_type = nullptr;

constexpr int kMaxCands = 8;   // cached pointer sets compared during a refresh

struct Plan {
  PyObject *const *params;   // planned parameter objects
  const uint8_t *has_grad;   // per parameter
  const int64_t *row_param;  // per row: index in params (increasing)
  const int32_t *grad_dtype; // per row
  const int64_t *layout_at;  // per row: offset in layout of [ndim, sizes..., strides...]
  const int64_t *layout;
  char *table;               // tensor table rows
  int64_t row_bytes, grad_off, param_off;
  int64_t device;
  int n_cands;               // cached (grad, param) pointer sets, one pair per row
  const uint64_t *cands[kMaxCands];
};

// Checks parameters [a, b) and the rows [ra, rb) that step them, writing
// the rows' pointers.  0: mismatch, 1: pointers unchanged, 2: some moved.
// *same: bit k cleared when a row's new pointers differ from cands[k]'s.
int check_range(const Plan &P, int64_t a, int64_t b, int64_t ra, int64_t rb,
                uint32_t *same) noexcept {
  try {
    const int64_t n = b - a;
    std::vector<const c10::TensorImpl *> pimpl(n), gimpl(n);
    std::vector<const c10::AutogradMetaInterface *> meta(n);
    for (int64_t i = 0; i < n; ++i) {
      if (i + kAhead < n) prefetch(P.params[a + i + kAhead]);
      PyObject *obj = P.params[a + i];
      if (Py_TYPE(obj) != g_tensor_type && Py_TYPE(obj) != g_param_type) return 0;
      pimpl[i] = THPVariable_Unpack(obj).unsafeGetTensorImpl();
    }
    for (int64_t i = 0; i < n; ++i) {
      if (i + kAhead < n) prefetch_impl(pimpl[i + kAhead]);
      meta[i] = pimpl[i]->autograd_meta();
    }
    for (int64_t i = 0; i < n; ++i) {
      if (i + kAhead < n && meta[i + kAhead]) {
        prefetch(meta[i + kAhead]);
        prefetch(reinterpret_cast<const char *>(meta[i + kAhead]) + 64);
      }
      const c10::TensorImpl *g = nullptr;
      if (meta[i]) {
        const at::Tensor &grad = meta[i]->grad();
        if (grad.defined()) g = grad.unsafeGetTensorImpl();
      }
      if ((g != nullptr) != (P.has_grad[a + i] != 0)) return 0;
      gimpl[i] = g;
    }
    bool changed = false;
    for (int64_t r = ra; r < rb; ++r) {
      if (r + kAhead < rb && gimpl[P.row_param[r + kAhead] - a])
        prefetch_impl(gimpl[P.row_param[r + kAhead] - a]);
      const int64_t j = P.row_param[r] - a;
      const c10::TensorImpl *p = pimpl[j], *g = gimpl[j];
      if (!g) return 0;
      // A tensor subclass (e.g. a DTensor) handles its own dispatch, and one
      // with a custom device or sizes policy answers is_cuda(), device(),
      // dim() and sizes() in Python, which needs the GIL that the calling
      // thread holds while the workers run: so the key set (a plain field)
      // is checked before anything else is asked of either tensor.
      if (g->key_set().has(c10::DispatchKey::Python) || p->key_set().has(c10::DispatchKey::Python) ||
          g->key_set().has(c10::DispatchKey::PythonTLSSnapshot) ||
          p->key_set().has(c10::DispatchKey::PythonTLSSnapshot))
        return 0;
      if (grad_code(g->dtype().toScalarType()) != P.grad_dtype[r]) return 0;
      if (p->dtype().toScalarType() != at::kFloat || !p->is_cuda() || !g->is_cuda() ||
          p->device().index() != P.device || g->device().index() != P.device)
        return 0;
      if (g->layout() != at::kStrided || p->layout() != at::kStrided || g->is_neg() ||
          p->is_neg())
        return 0;
      const int64_t *lay = P.layout + P.layout_at[r];
      const int64_t nd = lay[0];
      if (p->dim() != nd || g->dim() != nd) return 0;
      const c10::IntArrayRef ps = p->sizes(), pst = p->strides(), gs = g->sizes(),
                             gst = g->strides();
      for (int64_t d = 0; d < nd; ++d)
        if (ps[d] != lay[1 + d] || gs[d] != lay[1 + d] || pst[d] != lay[1 + nd + d] ||
            gst[d] != lay[1 + nd + d])
          return 0;
      if (!g->has_storage() || !p->has_storage()) return 0;
      const uint64_t ga = (uint64_t)(uintptr_t)g->data(), pa = (uint64_t)(uintptr_t)p->data();
      char *row = P.table + r * P.row_bytes;
      uint64_t *gp = reinterpret_cast<uint64_t *>(row + P.grad_off);
      uint64_t *pp = reinterpret_cast<uint64_t *>(row + P.param_off);
      changed |= (*gp != ga) | (*pp != pa);
      *gp = ga;
      *pp = pa;
      for (int k = 0; k < P.n_cands; ++k)
        if (((*same >> k) & 1u) && (P.cands[k][2 * r] != ga || P.cands[k][2 * r + 1] != pa))
          *same &= ~(1u << k);
    }
    return changed ? 2 : 1;
  } catch (...) {
    return 0;   // an unusual tensor: the caller rebuilds the table, which reports it
  }
}

}  // namespace

// Re-validates a planned step and writes the current pointers into its
// tensor table.
//   groups     -- the optimizer's param_groups (list of dicts with "params")
//   planned    -- the flat parameter list of the plan (same objects, same order)
//   has_grad   -- uint8 per planned parameter: 1 where it had a gradient
//   row_param  -- int64 per table row: index of the row's parameter in planned
//                 (increasing)
//   layout_at, layout -- per table row, [ndim, sizes..., strides...] of the
//                 planned parameter (its Q_m and gradient have the same)
//   gdtype     -- int32 per table row: the planned gradient dtype code
//   table      -- address of the tensor table (LumaTensor rows), its row
//                 size and the byte offsets of the grad and param fields
//   device     -- the planned CUDA device index
//   cands      -- optional: up to 8 (n_rows, 2) uint64 arrays of gradient and
//                 parameter pointers (pointer sets whose tables the caller
//                 keeps on the device)
// Returns 0 when anything differs from the plan (a parameter added, removed
// or replaced by another object, a gradient that appeared or disappeared, a
// gradient of another dtype, shape, layout or device, a tensor subclass, or
// a parameter whose storage was replaced by one of another dtype or layout);
// the table is then to be rebuilt, whatever this call wrote into it.
// Otherwise 1 when every pointer was already in the table, 2 when some moved,
// plus bit 2 + k when every row's new pointers equal cands[k]'s (compared
// while they are written, so the caller need not scan the table again).
template <typename T>
using carray = py::array_t<T, py::array::c_style | py::array::forcecast>;

int refresh(py::list groups, py::list planned, carray<uint8_t> has_grad,
            carray<int64_t> row_param, carray<int64_t> layout_at, carray<int64_t> layout,
            carray<int32_t> gdtype, uintptr_t table, int64_t row_bytes, int64_t grad_off,
            int64_t param_off, int64_t device, py::object cands) {
  const int64_t n_params = (int64_t)planned.size();
  const int64_t n_rows = row_param.shape(0);
  if (has_grad.ndim() != 1 || row_param.ndim() != 1 || layout_at.ndim() != 1 ||
      layout.ndim() != 1 || gdtype.ndim() != 1 || has_grad.shape(0) != n_params ||
      layout_at.shape(0) != n_rows || gdtype.shape(0) != n_rows)
    return 0;
  const int64_t *rp = row_param.data();
  const int64_t *lat = layout_at.data();
  const int64_t *lay = layout.data();
  const int64_t n_layout = layout.shape(0);
  for (int64_t r = 0; r < n_rows; ++r) {
    if (rp[r] < 0 || rp[r] >= n_params || (r > 0 && rp[r] <= rp[r - 1])) return 0;
    if (lat[r] < 0 || lat[r] >= n_layout || lay[lat[r]] < 0 ||
        lat[r] + 1 + 2 * lay[lat[r]] > n_layout)
      return 0;
  }
  // same parameter objects in the same order
  PyObject *const *pl = n_params ? &PyList_GET_ITEM(planned.ptr(), 0) : nullptr;
  int64_t k = 0;
  for (py::handle g : groups) {
    PyObject *params = PyDict_GetItemString(g.ptr(), "params");
    if (!params || !PyList_Check(params)) return 0;
    const Py_ssize_t n = PyList_GET_SIZE(params);
    if (k + n > n_params) return 0;
    for (Py_ssize_t i = 0; i < n; ++i)
      if (PyList_GET_ITEM(params, i) != pl[k + i]) return 0;
    k += n;
  }
  if (k != n_params || !g_tensor_type || !g_param_type) return 0;

  Plan P{pl, has_grad.data(), rp, gdtype.data(), lat, lay,
         reinterpret_cast<char *>(table), row_bytes, grad_off, param_off, device, 0, {}};
  // the candidate arrays (held here for the call's duration); one of another
  // shape is never a match and never read (its bit starts cleared)
  std::vector<carray<uint64_t>> held;
  uint32_t usable = 0;
  if (!cands.is_none()) {
    const py::list cl = cands.cast<py::list>();
    for (py::handle h : cl) {
      if (P.n_cands == kMaxCands) break;
      held.push_back(h.cast<carray<uint64_t>>());
      const carray<uint64_t> &c = held.back();
      const bool fits = c.ndim() == 2 && c.shape(0) == n_rows && c.shape(1) == 2;
      P.cands[P.n_cands] = fits ? c.data() : nullptr;
      if (fits) usable |= 1u << P.n_cands;
      ++P.n_cands;
    }
  }
  const int T = (int)std::min<int64_t>(kMaxThreads, std::max<int64_t>(1, n_params / kPerThread));
  std::vector<int> res(T, 1);
  std::vector<uint32_t> same(T, usable);
  const std::function<void(int)> part = [&](int t) {
    const int64_t a = n_params * t / T, b = n_params * (t + 1) / T;
    const int64_t ra = std::lower_bound(rp, rp + n_rows, a) - rp;
    const int64_t rb = std::lower_bound(rp, rp + n_rows, b) - rp;
    res[t] = check_range(P, a, b, ra, rb, &same[t]);
  };
  if (T == 1)
    part(0);
  else
    Pool::get().run(T, part);
  int out = 1;
  uint32_t match = usable;
  for (int t = 0; t < T; ++t) {
    if (res[t] == 0) return 0;
    if (res[t] == 2) out = 2;
    match &= same[t];
  }
  return out | (int)(match << 2);
}

// Whether the gradient and parameter pointers of the table's rows are those
// of cols (one (grad, param) pair per row; the table has at least as many
// rows).  Stops at the first difference: a table that matches no cached
// pointer set costs one row per cached set.
bool same_pointers(uintptr_t table, int64_t row_bytes, int64_t grad_off, int64_t param_off,
                   carray<uint64_t> cols) {
  if (cols.ndim() != 2 || cols.shape(1) != 2)
    throw py::value_error("same_pointers: cols must be an (n, 2) array");
  const int64_t n = cols.shape(0);
  const uint64_t *c = cols.data();
  const char *t = reinterpret_cast<const char *>(table);
  for (int64_t r = 0; r < n; ++r) {
    const char *row = t + r * row_bytes;
    uint64_t g, p;
    std::memcpy(&g, row + grad_off, sizeof g);
    std::memcpy(&p, row + param_off, sizeof p);
    if (g != c[2 * r] || p != c[2 * r + 1]) return false;
  }
  return true;
}

// state["step"] += 1 for every state dict of the list.  The dicts of one
// plan usually hold the same count object, so the sum is formed once per
// distinct object.  The dicts lie scattered in memory: each one, and then its
// key table, is prefetched a few dicts ahead.
void bump_steps(py::list states) {
  static PyObject *key = PyUnicode_InternFromString("step");
  py::object last_v, last_nv;
  py::object one = py::int_(1);
  for (Py_ssize_t i = 0; i < PyList_GET_SIZE(states.ptr()); ++i) {
    // (the size is read again each time: a count object's __add__ could
    // change the list)
    const Py_ssize_t n = PyList_GET_SIZE(states.ptr());
    if (i + 2 * kAhead < n) prefetch(PyList_GET_ITEM(states.ptr(), i + 2 * kAhead));
    if (i + kAhead < n) {
      PyObject *a = PyList_GET_ITEM(states.ptr(), i + kAhead);
      if (PyDict_CheckExact(a)) {
        const char *keys = reinterpret_cast<const char *>(((PyDictObject *)a)->ma_keys);
        prefetch(keys);
        prefetch(keys + 64);
      }
    }
    PyObject *d = PyList_GET_ITEM(states.ptr(), i);
    if (!PyDict_Check(d)) throw py::type_error("bump_steps: a state is not a dict");
    PyObject *v = PyDict_GetItemWithError(d, key);
    if (!v) {
      if (PyErr_Occurred()) throw py::error_already_set();
      throw py::key_error("step");
    }
    if (v != last_v.ptr()) {
      PyObject *nv = PyNumber_Add(v, one.ptr());
      if (!nv) throw py::error_already_set();
      last_v = py::reinterpret_borrow<py::object>(v);
      last_nv = py::reinterpret_steal<py::object>(nv);
    }
    if (PyDict_SetItem(d, key, last_nv.ptr()) != 0) throw py::error_already_set();
  }
}

PYBIND11_MODULE(_luma_host, m) {
  m.doc() = "Host-side bookkeeping of LUMA.step (pointer refresh of a planned step).";
  py::object torch = py::module_::import("torch");
  g_tensor_type = reinterpret_cast<PyTypeObject *>(torch.attr("Tensor").ptr());
  g_param_type = reinterpret_cast<PyTypeObject *>(torch.attr("nn").attr("Parameter").ptr());
  // the module holds them for its lifetime
  Py_INCREF(g_tensor_type);
  Py_INCREF(g_param_type);
  m.def("refresh", &refresh, py::arg("groups"), py::arg("planned"), py::arg("has_grad"),
        py::arg("row_param"), py::arg("layout_at"), py::arg("layout"), py::arg("gdtype"),
        py::arg("table"), py::arg("row_bytes"), py::arg("grad_off"), py::arg("param_off"),
        py::arg("device"), py::arg("cands") = py::none());
  m.def("same_pointers", &same_pointers);
  m.def("bump_steps", &bump_steps);
  // the torch whose headers this module was compiled against: it reads
  // TensorImpl fields in that version's inline layout
  m.attr("torch_version") = LUMA_TORCH_VERSION;
}
