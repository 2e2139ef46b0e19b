// CPython binding of the kernel library's C ABI: the reference's native entries
// `decode`, `store` and `flash` (cpu_attention/_mojo/src/_C.mojo:87-316 of
// ducviet00/cpu-attention), which read torch tensors in place, validate them and
// return None for anything they do not take.
//
// The rules are the ones the package's ctypes module applies
// (cpu_attention/_kernel.py, class Module), in the same order and with the same
// results; this file only moves them out of the interpreter.  A small call's
// host time is mostly argument handling: here each tensor's metadata is read
// from the C++ tensor directly, outputs come from the caching allocator without
// a Python frame, and the argument structs are plain C.  The entry points of
// libcpu_attention_hip.so are not linked: the Python side passes the addresses
// of the functions its ctypes handle loaded (init), so CPU_ATTENTION_LIB keeps
// naming the library that runs.
//
// Built by cpu-attention_amd/build.py with the host compiler against torch's
// headers; no device code.
#include <Python.h>

#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <ATen/ops/max.h>
#include <torch/csrc/Exceptions.h>
#include <torch/csrc/autograd/python_variable.h>

#include <cmath>

#include "cpu_attention_hip.h"

namespace {

struct Entries {
  int (*decode)(const ca_decode_args*, void*) = nullptr;
  int (*store)(const ca_store_args*, void*) = nullptr;
  int (*flash)(const ca_flash_args*, void*) = nullptr;
  int64_t (*decode_ws)(int64_t, int64_t, int64_t, int64_t, int64_t) = nullptr;
  int64_t (*flash_ws)(int64_t, int64_t, int64_t, int64_t, int64_t, int32_t) = nullptr;
  const char* (*status)(int) = nullptr;
};

Entries g_lib;
PyObject* g_plain[2] = {nullptr, nullptr};  // torch.Tensor, torch.nn.Parameter
PyObject* g_raw_stream = nullptr;            // device index -> raw hipStream_t (an int)
bool g_host_checks = true;

bool ready() {
  if (g_lib.decode) return true;
  PyErr_SetString(PyExc_RuntimeError, "cpu_attention: the native binding is not initialised");
  return false;
}

// `type(x) in (torch.Tensor, torch.nn.Parameter)`: subclasses are declined, as
// the reference's entries decline them.
bool plain(PyObject* o) {
  PyObject* t = reinterpret_cast<PyObject*>(Py_TYPE(o));
  return t == g_plain[0] || t == g_plain[1];
}

const at::Tensor& T(PyObject* o) { return THPVariable_Unpack(o); }

bool is_dtype(at::ScalarType s) { return s == at::kFloat || s == at::kBFloat16; }
bool is_hd(int64_t hd) { return hd == 32 || hd == 64 || hd == 128; }
int32_t dtype_code(at::ScalarType s) { return s == at::kBFloat16 ? CA_BF16 : CA_F32; }
int64_t esize(at::ScalarType s) { return s == at::kBFloat16 ? 2 : 4; }

// Stride of dim i, 0 for a dim of size 1 (never stepped over).
int64_t stride0(const at::Tensor& t, int64_t i) { return t.size(i) == 1 ? 0 : t.stride(i); }

// Heads and dims contiguous (any token stride).
bool rows_ok(const at::Tensor& t, int64_t hd) {
  return t.stride(-1) == 1 && (t.size(-2) == 1 || t.stride(-2) == hd);
}

// [blocks, heads, page, dim], contiguous, matching, page a multiple of 16
// (_C.mojo:74-80).
bool caches_ok(PyObject* kco, PyObject* vco, at::ScalarType dt, int64_t heads, int64_t hd) {
  if (!plain(kco) || !plain(vco)) return false;
  const at::Tensor& kc = T(kco);
  const at::Tensor& vc = T(vco);
  if (kc.dim() != 4 || vc.sizes() != kc.sizes()) return false;
  return kc.scalar_type() == dt && vc.scalar_type() == dt && kc.size(1) == heads && kc.size(3) == hd &&
         kc.size(2) > 0 && kc.size(2) % 16 == 0 && kc.is_contiguous() && vc.is_contiguous();
}

bool int_vector(PyObject* o, at::ScalarType dt, int64_t n) {
  if (!plain(o)) return false;
  const at::Tensor& t = T(o);
  return t.dim() == 1 && t.scalar_type() == dt && t.size(0) == n && t.is_contiguous();
}

bool on_gpu(const at::Device& dev, const at::Tensor& t) { return t.is_cuda() && t.device() == dev; }

// An index tensor on the kernels' device (CPU index tensors are copied over).
at::Tensor index_on(const at::Tensor& t, const at::Device& dev) {
  return t.device() == dev ? t : t.to(dev, /*non_blocking=*/true);
}

int64_t max_of(const at::Tensor& t) { return at::max(t).item<int64_t>(); }

// torch's current stream on `dev` as a raw handle; nullptr with a Python error set.
bool stream_of(const at::Device& dev, void** out) {
  PyObject* idx = PyLong_FromLong(dev.index());
  if (!idx) return false;
  PyObject* s = PyObject_CallOneArg(g_raw_stream, idx);
  Py_DECREF(idx);
  if (!s) return false;
  *out = PyLong_AsVoidPtr(s);
  Py_DECREF(s);
  return !PyErr_Occurred();
}

// The softmax scale: hd^-0.5 (computed in double, as the reference does) or float(scale).
bool scale_of(PyObject* scale, int64_t hd, float* out) {
  if (scale == Py_None) {
    *out = static_cast<float>(std::pow(static_cast<double>(hd), -0.5));
    return true;
  }
  PyObject* f = PyNumber_Float(scale);
  if (!f) return false;
  *out = static_cast<float>(PyFloat_AS_DOUBLE(f));
  Py_DECREF(f);
  return true;
}

PyObject* failed(int rc, const char* what) {
  PyErr_Format(PyExc_RuntimeError, "cpu_attention: %s failed on the GPU: %s", what, g_lib.status(rc));
  return nullptr;
}

}  // namespace

// init(entries, plain_types, raw_stream, host_checks): `entries` holds the
// addresses of ca_decode, ca_store, ca_flash, ca_decode_workspace_bytes,
// ca_flash_workspace_bytes and ca_status_string.
static PyObject* b_init(PyObject*, PyObject* const* args, Py_ssize_t n) {
  if (n != 4 || !PyTuple_Check(args[0]) || PyTuple_GET_SIZE(args[0]) != 6 || !PyTuple_Check(args[1]) ||
      PyTuple_GET_SIZE(args[1]) != 2 || !PyCallable_Check(args[2])) {
    PyErr_SetString(PyExc_TypeError, "init(entries[6], plain_types[2], raw_stream, host_checks)");
    return nullptr;
  }
  void* p[6];
  for (int i = 0; i < 6; ++i) {
    p[i] = PyLong_AsVoidPtr(PyTuple_GET_ITEM(args[0], i));
    if (PyErr_Occurred()) return nullptr;
    if (!p[i]) {
      PyErr_SetString(PyExc_ValueError, "init: a null entry point");
      return nullptr;
    }
  }
  g_lib.decode = reinterpret_cast<int (*)(const ca_decode_args*, void*)>(p[0]);
  g_lib.store = reinterpret_cast<int (*)(const ca_store_args*, void*)>(p[1]);
  g_lib.flash = reinterpret_cast<int (*)(const ca_flash_args*, void*)>(p[2]);
  g_lib.decode_ws = reinterpret_cast<int64_t (*)(int64_t, int64_t, int64_t, int64_t, int64_t)>(p[3]);
  g_lib.flash_ws = reinterpret_cast<int64_t (*)(int64_t, int64_t, int64_t, int64_t, int64_t, int32_t)>(p[4]);
  g_lib.status = reinterpret_cast<const char* (*)(int)>(p[5]);
  for (int i = 0; i < 2; ++i) {
    Py_XDECREF(g_plain[i]);
    g_plain[i] = PyTuple_GET_ITEM(args[1], i);
    Py_INCREF(g_plain[i]);
  }
  Py_XDECREF(g_raw_stream);
  g_raw_stream = args[2];
  Py_INCREF(g_raw_stream);
  g_host_checks = PyObject_IsTrue(args[3]) == 1;
  Py_RETURN_NONE;
}

static PyObject* b_set_host_checks(PyObject*, PyObject* arg) {
  const int v = PyObject_IsTrue(arg);
  if (v < 0) return nullptr;
  g_host_checks = v == 1;
  Py_RETURN_NONE;
}

// decode(rt, q, k_cache, v_cache, k, v, slots, lens, page_table, scale, dst[, n])
// (_C.mojo:87-171): paged decode of q [seqs, (1,) heads, dim]; with k/v the new
// tokens are stored first (at `slots`, lens then being the length after the
// store, or appended at lens; n > 1 new tokens per sequence, rows of k/v
// [seqs * n, heads, dim], are the prompt append).  Returns the output (dst when
// given), or None for anything the kernels do not take.
static PyObject* b_decode(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  HANDLE_TH_ERRORS
  if (nargs != 11 && nargs != 12) {
    PyErr_SetString(PyExc_TypeError, "decode takes 11 or 12 positional arguments");
    return nullptr;
  }
  if (!ready()) return nullptr;
  PyObject *qo = args[1], *kco = args[2], *vco = args[3], *ko = args[4], *vo = args[5], *slo = args[6],
           *lo = args[7], *pto = args[8], *scale = args[9], *dsto = args[10];
  int64_t n = 1;
  if (nargs == 12) {
    n = PyLong_AsLongLong(args[11]);
    if (n == -1 && PyErr_Occurred()) return nullptr;
  }
  if (!(plain(qo) && plain(pto) && THPVariable_Check(lo))) Py_RETURN_NONE;
  const at::Tensor& q = T(qo);
  const int64_t nd = q.dim();
  if ((nd != 3 && nd != 4) || (nd == 4 && q.size(1) != 1)) Py_RETURN_NONE;
  const int64_t b = q.size(0), heads = q.size(-2), hd = q.size(-1);
  const at::ScalarType dt = q.scalar_type();
  if (!is_dtype(dt) || !is_hd(hd) || !rows_ok(q, hd)) Py_RETURN_NONE;
  if (!caches_ok(kco, vco, dt, heads, hd)) Py_RETURN_NONE;
  const at::Tensor& kc = T(kco);
  const at::Tensor& vc = T(vco);
  const int64_t page = kc.size(2);
  const at::Tensor& pt = T(pto);
  if (pt.dim() != 2 || pt.scalar_type() != at::kInt || pt.size(0) != b || !pt.is_contiguous()) Py_RETURN_NONE;
  const int64_t width = pt.size(1);
  if (!int_vector(lo, at::kInt, b)) Py_RETURN_NONE;
  const bool store = ko != Py_None;
  if (store) {
    if (!(plain(ko) && plain(vo))) Py_RETURN_NONE;
    const at::Tensor& k = T(ko);
    const at::Tensor& v = T(vo);
    const bool shape_ok = n == 1 ? k.sizes() == q.sizes()
                                 : (k.dim() == 3 && k.size(0) == b * n && k.size(1) == heads && k.size(2) == hd);
    if (!shape_ok || v.sizes() != k.sizes() || v.strides() != k.strides()) Py_RETURN_NONE;
    if (k.scalar_type() != dt || v.scalar_type() != dt || !rows_ok(k, hd)) Py_RETURN_NONE;
  } else if (vo != Py_None) {
    Py_RETURN_NONE;
  }
  if (slo != Py_None && !(store && int_vector(slo, at::kLong, b))) Py_RETURN_NONE;
  const at::Device dev = q.device();
  if (!q.is_cuda() || !on_gpu(dev, kc) || !on_gpu(dev, vc)) Py_RETURN_NONE;
  if (store && !(on_gpu(dev, T(ko)) && on_gpu(dev, T(vo)))) Py_RETURN_NONE;
  if (dsto != Py_None) {
    if (!plain(dsto)) Py_RETURN_NONE;
    const at::Tensor& dst = T(dsto);
    if (dst.sizes() != q.sizes() || dst.scalar_type() != dt || !dst.is_contiguous() || !on_gpu(dev, dst))
      Py_RETURN_NONE;
  }
  const int64_t q_stride = stride0(q, 0);
  const int64_t kv_stride = store ? stride0(T(ko), 0) : 0;
  // 16-byte vectors: pointers and element strides (a multiple of 16 / esize)
  const uintptr_t qp = (uintptr_t)q.data_ptr(), kcp = (uintptr_t)kc.data_ptr(), vcp = (uintptr_t)vc.data_ptr();
  const uintptr_t knp = store ? (uintptr_t)T(ko).data_ptr() : 0, vnp = store ? (uintptr_t)T(vo).data_ptr() : 0;
  if ((qp | kcp | vcp | knp | vnp) % 16 || (q_stride | kv_stride) % (16 / esize(dt))) Py_RETURN_NONE;
  const int64_t nblocks = kc.size(0);
  // The data-dependent rules (_C.mojo:139-153), on the host.
  if (g_host_checks && b) {
    if (slo != Py_None && max_of(T(slo)) >= nblocks * page) Py_RETURN_NONE;
    if (max_of(T(lo)) + (store && slo == Py_None ? n : 0) > width * page) Py_RETURN_NONE;
  }
  float sc;
  if (!scale_of(scale, hd, &sc)) return nullptr;
  void* stream;
  if (!stream_of(dev, &stream)) return nullptr;
  const at::Tensor lens = index_on(T(lo), dev);
  const at::Tensor table = index_on(pt, dev);
  at::Tensor slots;
  if (slo != Py_None) slots = index_on(T(slo), dev);
  at::Tensor out = dsto != Py_None ? T(dsto) : at::empty(q.sizes(), at::TensorOptions().dtype(dt).device(dev));
  const int64_t ws_bytes = g_lib.decode_ws(b, heads, hd, page, width);
  at::Tensor ws;  // held past the launch
  if (ws_bytes) ws = at::empty({ws_bytes}, at::TensorOptions().dtype(at::kByte).device(dev));
  ca_decode_args a{};
  a.q = reinterpret_cast<const void*>(qp);
  a.q_stride = q_stride;
  a.k_cache = reinterpret_cast<void*>(kcp);
  a.v_cache = reinterpret_cast<void*>(vcp);
  a.k_new = reinterpret_cast<const void*>(knp);
  a.v_new = reinterpret_cast<const void*>(vnp);
  a.kv_stride = kv_stride;
  a.slots = slots.defined() ? slots.data_ptr<int64_t>() : nullptr;
  a.lens = lens.data_ptr<int32_t>();
  a.page_table = table.data_ptr<int32_t>();
  a.page_table_width = width;
  a.out = out.data_ptr();
  a.num_seqs = b;
  a.num_heads = heads;
  a.head_dim = hd;
  a.page_size = page;
  a.num_blocks = nblocks;
  a.scale = sc;
  a.dtype = dtype_code(dt);
  a.workspace = ws_bytes ? ws.data_ptr() : nullptr;
  a.workspace_bytes = ws_bytes;
  a.new_tokens = store ? n : 0;
  const int rc = g_lib.decode(&a, stream);
  if (rc == CA_DECLINED) Py_RETURN_NONE;
  if (rc != CA_OK) return failed(rc, "decode");
  return THPVariable_Wrap(std::move(out));
  END_HANDLE_TH_ERRORS
}

// store(rt, key, value, k_cache, v_cache, slots) (_C.mojo:174-213):
// reshape_and_cache.  True, or None for anything the kernel does not take.
static PyObject* b_store(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  HANDLE_TH_ERRORS
  if (nargs != 6) {
    PyErr_SetString(PyExc_TypeError, "store takes 6 positional arguments");
    return nullptr;
  }
  if (!ready()) return nullptr;
  PyObject *keyo = args[1], *valo = args[2], *kco = args[3], *vco = args[4], *slo = args[5];
  if (!(THPVariable_Check(keyo) && THPVariable_Check(valo) && THPVariable_Check(slo))) Py_RETURN_NONE;
  if (!(plain(keyo) && plain(valo))) Py_RETURN_NONE;
  const at::Tensor& key = T(keyo);
  const at::Tensor& val = T(valo);
  if (key.dim() != 3 || val.dim() != 3) Py_RETURN_NONE;
  const int64_t n = key.size(0), heads = key.size(1), hd = key.size(2);
  const at::ScalarType dt = key.scalar_type();
  if (!is_dtype(dt) || !is_hd(hd) || val.scalar_type() != dt || !rows_ok(key, hd)) Py_RETURN_NONE;
  if (val.sizes() != key.sizes() || val.strides() != key.strides()) Py_RETURN_NONE;
  if (!caches_ok(kco, vco, dt, heads, hd) || !int_vector(slo, at::kLong, n)) Py_RETURN_NONE;
  const at::Tensor& kc = T(kco);
  const at::Tensor& vc = T(vco);
  const at::Device dev = kc.device();
  if (!kc.is_cuda() || !on_gpu(dev, vc) || !on_gpu(dev, key) || !on_gpu(dev, val)) Py_RETURN_NONE;
  const int64_t tstride = stride0(key, 0);
  const uintptr_t kp = (uintptr_t)key.data_ptr(), vp = (uintptr_t)val.data_ptr();
  const uintptr_t kcp = (uintptr_t)kc.data_ptr(), vcp = (uintptr_t)vc.data_ptr();
  if ((kp | vp | kcp | vcp) % 16 || (tstride * esize(dt)) % 16) Py_RETURN_NONE;
  const int64_t page = kc.size(2), nblocks = kc.size(0);
  if (g_host_checks && n && max_of(T(slo)) >= nblocks * page) Py_RETURN_NONE;
  if (n == 0) Py_RETURN_TRUE;
  void* stream;
  if (!stream_of(dev, &stream)) return nullptr;
  const at::Tensor slots = index_on(T(slo), dev);
  ca_store_args a{};
  a.key = reinterpret_cast<const void*>(kp);
  a.value = reinterpret_cast<const void*>(vp);
  a.token_stride = tstride;
  a.k_cache = reinterpret_cast<void*>(kcp);
  a.v_cache = reinterpret_cast<void*>(vcp);
  a.slot_mapping = slots.data_ptr<int64_t>();
  a.num_tokens = n;
  a.num_heads = heads;
  a.head_dim = hd;
  a.page_size = page;
  a.num_blocks = nblocks;
  a.dtype = dtype_code(dt);
  const int rc = g_lib.store(&a, stream);
  if (rc == CA_DECLINED) Py_RETURN_NONE;
  if (rc != CA_OK) return failed(rc, "store");
  Py_RETURN_TRUE;
  END_HANDLE_TH_ERRORS
}

// flash(rt, q, k, v, scale, causal, ws, ws_bytes) (_C.mojo:232-316):
// flash_attn_func over q/k/v [batch, seq, heads, dim] (MHA, dims contiguous).
// Returns the output, the workspace bytes the call needs when ws_bytes is short
// (an int), or None.
static PyObject* b_flash(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  HANDLE_TH_ERRORS
  if (nargs != 8) {
    PyErr_SetString(PyExc_TypeError, "flash takes 8 positional arguments");
    return nullptr;
  }
  if (!ready()) return nullptr;
  PyObject *qo = args[1], *ko = args[2], *vo = args[3], *scale = args[4], *causal = args[5], *wso = args[6],
           *wsbo = args[7];
  if (!(plain(qo) && plain(ko) && plain(vo))) Py_RETURN_NONE;
  const at::Tensor& q = T(qo);
  const at::Tensor& k = T(ko);
  const at::Tensor& v = T(vo);
  if (q.dim() != 4 || k.dim() != 4 || v.sizes() != k.sizes()) Py_RETURN_NONE;
  const int64_t b = q.size(0), sq = q.size(1), heads = q.size(2), hd = q.size(3), sk = k.size(1);
  const at::ScalarType dt = q.scalar_type();
  if (!is_dtype(dt) || !is_hd(hd) || sq < 1 || sk < 1) Py_RETURN_NONE;
  if (k.size(0) != b || k.size(2) != heads || k.size(3) != hd || k.scalar_type() != dt || v.scalar_type() != dt)
    Py_RETURN_NONE;
  if (q.stride(3) != 1 || k.stride(3) != 1 || v.stride(3) != 1) Py_RETURN_NONE;
  if (causal != Py_True && causal != Py_False) Py_RETURN_NONE;
  const at::Device dev = q.device();
  if (!q.is_cuda() || k.device() != dev || v.device() != dev) Py_RETURN_NONE;
  int64_t qs[3], ks[3], vs[3];
  for (int i = 0; i < 3; ++i) {
    qs[i] = stride0(q, i);
    ks[i] = stride0(k, i);
    vs[i] = stride0(v, i);
  }
  // 16-byte vectors: pointers and element strides (a multiple of 16 / esize)
  const uintptr_t qp = (uintptr_t)q.data_ptr(), kp = (uintptr_t)k.data_ptr(), vp = (uintptr_t)v.data_ptr();
  const int64_t unit = 16 / esize(dt);
  if ((qp | kp | vp) % 16 ||
      (qs[0] | qs[1] | qs[2] | ks[0] | ks[1] | ks[2] | vs[0] | vs[1] | vs[2]) % unit)
    Py_RETURN_NONE;
  const int64_t need = g_lib.flash_ws(b, sq, sk, heads, hd, dtype_code(dt));
  const int64_t ws_bytes = PyLong_AsLongLong(wsbo);
  if (ws_bytes == -1 && PyErr_Occurred()) return nullptr;
  if (need > ws_bytes) return PyLong_FromLongLong(need);
  void* ws = nullptr;
  if (wso != Py_None) {
    ws = PyLong_AsVoidPtr(wso);
    if (PyErr_Occurred()) return nullptr;
  }
  float sc;
  if (!scale_of(scale, hd, &sc)) return nullptr;
  void* stream;
  if (!stream_of(dev, &stream)) return nullptr;
  at::Tensor out = at::empty(q.sizes(), at::TensorOptions().dtype(dt).device(dev));
  ca_flash_args a{};
  a.q = reinterpret_cast<const void*>(qp);
  a.k = reinterpret_cast<const void*>(kp);
  a.v = reinterpret_cast<const void*>(vp);
  a.out = out.data_ptr();
  a.batch = b;
  a.seq_q = sq;
  a.seq_k = sk;
  a.num_heads = heads;
  a.head_dim = hd;
  for (int i = 0; i < 3; ++i) {
    a.q_strides[i] = qs[i];
    a.k_strides[i] = ks[i];
    a.v_strides[i] = vs[i];
  }
  a.scale = sc;
  a.causal = causal == Py_True ? 1 : 0;
  a.dtype = dtype_code(dt);
  a.workspace = ws;
  a.workspace_bytes = ws_bytes;
  const int rc = g_lib.flash(&a, stream);
  if (rc == CA_DECLINED) Py_RETURN_NONE;
  if (rc != CA_OK) return failed(rc, "flash");
  return THPVariable_Wrap(std::move(out));
  END_HANDLE_TH_ERRORS
}

static PyMethodDef kMethods[] = {
    {"init", (PyCFunction)(void (*)(void))b_init, METH_FASTCALL, "Entry addresses, tensor types, stream query."},
    {"set_host_checks", b_set_host_checks, METH_O, "Check slots and lengths on the host."},
    {"decode", (PyCFunction)(void (*)(void))b_decode, METH_FASTCALL, "Paged decode (_C.mojo:87-171)."},
    {"store", (PyCFunction)(void (*)(void))b_store, METH_FASTCALL, "reshape_and_cache (_C.mojo:174-213)."},
    {"flash", (PyCFunction)(void (*)(void))b_flash, METH_FASTCALL, "Dense prefill (_C.mojo:232-316)."},
    {nullptr, nullptr, 0, nullptr}};

static PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_binding",
                              "Native argument handling for the kernel library's C ABI.", -1, kMethods};

PyMODINIT_FUNC PyInit__binding() { return PyModule_Create(&kModule); }
