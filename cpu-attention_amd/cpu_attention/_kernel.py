# The module surface here (module(), runtime(), workspace(), physical_cores(),
# llc_bytes(), DTYPES, HEAD_DIMS, and the decode/store/flash entries with their
# positional arguments and None/int returns) follows ducviet00/cpu-attention's
# cpu_attention/_kernel.py and native module, Apache License 2.0, so that engine
# code written against it runs unchanged (see NOTICE at the repository root); the
# implementation is this build's own.

"""Loads the gfx950 kernel library and exposes the reference's native entries.

The reference loads a Mojo CPython extension per CPU tier (cpu_attention/_kernel.py:52-84
of ducviet00/cpu-attention) whose entries ``decode``, ``store`` and ``flash``
(_mojo/src/_C.mojo:87-316) read torch tensors in place, validate them, and return
``None`` for anything they do not take.  This build keeps that module surface --
``module().decode/.store/.flash`` with the same positional arguments and the same
``None`` / ``int`` return conventions.  The entries read tensor metadata in
place, apply the same acceptance rules, allocate outputs from torch's caching
allocator on the tensors' GPU, and call the C ABI of ``libcpu_attention_hip.so``
(include/cpu_attention_hip.h) on torch's current HIP stream; the kernels run
asynchronously.  Two bindings implement them with the same rules and results:

- ``NativeModule`` (the default when ``_binding`` is built): the argument
  handling in a small C++ extension (csrc/ca_binding.cpp), as the reference's
  own native module does it; a few microseconds per call;
- ``Module``: the same in Python over ctypes, which is also the binding a
  maintainer of the reference would add on its side.  It serves when the
  extension is not built, or when ``CPU_ATTENTION_BINDING=ctypes``.

Data-dependent rules (a slot past the cache's end, a length beyond the page
table's capacity) need the index values.  By default they are checked on the
host exactly as the reference does, which reads the index tensors (a device
synchronisation when they live on the GPU).  ``set_host_checks(False)`` (or
``CPU_ATTENTION_HOST_CHECKS=0``) skips that read: the kernels never access memory
out of bounds either way (such tokens are not stored, such positions not read),
but no ValueError is raised.

Environment: ``CPU_ATTENTION_LIB`` names another build of the library;
``CPU_ATTENTION_BINDING=ctypes`` selects the ctypes binding.
"""

import ctypes
import functools
import os
import threading

import torch

DTYPES = {torch.float32: 0, torch.bfloat16: 1}
HEAD_DIMS = (32, 64, 128)
_DIR = os.path.dirname(os.path.abspath(__file__))
LIBRARY = "libcpu_attention_hip.so"
ABI_VERSION = 3
_ESIZE = {torch.float32: 4, torch.bfloat16: 2}
_PLAIN = (torch.Tensor, torch.nn.Parameter)

CA_OK, CA_DECLINED, CA_SCRATCH_EXCEEDED = 0, 1, 2


class StoreArgs(ctypes.Structure):
    """``ca_store_args`` (include/cpu_attention_hip.h)."""
    _fields_ = [
        ("key", ctypes.c_void_p), ("value", ctypes.c_void_p), ("token_stride", ctypes.c_int64),
        ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("slot_mapping", ctypes.c_void_p), ("num_tokens", ctypes.c_int64),
        ("num_heads", ctypes.c_int64), ("head_dim", ctypes.c_int64),
        ("page_size", ctypes.c_int64), ("num_blocks", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("reserved", ctypes.c_int32),
    ]


class DecodeArgs(ctypes.Structure):
    """``ca_decode_args`` (include/cpu_attention_hip.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("q_stride", ctypes.c_int64),
        ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("k_new", ctypes.c_void_p), ("v_new", ctypes.c_void_p), ("kv_stride", ctypes.c_int64),
        ("slots", ctypes.c_void_p), ("lens", ctypes.c_void_p), ("page_table", ctypes.c_void_p),
        ("page_table_width", ctypes.c_int64), ("out", ctypes.c_void_p),
        ("num_seqs", ctypes.c_int64), ("num_heads", ctypes.c_int64),
        ("head_dim", ctypes.c_int64), ("page_size", ctypes.c_int64),
        ("num_blocks", ctypes.c_int64), ("scale", ctypes.c_float), ("dtype", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
        ("new_tokens", ctypes.c_int64),
    ]


class FlashArgs(ctypes.Structure):
    """``ca_flash_args`` (include/cpu_attention_hip.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p), ("batch", ctypes.c_int64), ("seq_q", ctypes.c_int64),
        ("seq_k", ctypes.c_int64), ("num_heads", ctypes.c_int64), ("head_dim", ctypes.c_int64),
        ("q_strides", ctypes.c_int64 * 3), ("k_strides", ctypes.c_int64 * 3),
        ("v_strides", ctypes.c_int64 * 3), ("scale", ctypes.c_float), ("causal", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("reserved", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
    ]


EXPORTS = ("ca_store", "ca_decode", "ca_decode_noalloc", "ca_decode_workspace_bytes", "ca_flash",
           "ca_flash_workspace_bytes", "ca_abi_version", "ca_version", "ca_status_string")

_HOST_CHECKS = [os.environ.get("CPU_ATTENTION_HOST_CHECKS", "1") != "0"]


def set_host_checks(enabled):
    """Check slots and lengths against the cache on the host (the reference's
    ValueErrors; a device sync per call when they live on the GPU). Returns the
    previous setting."""
    old = _HOST_CHECKS[0]
    _HOST_CHECKS[0] = bool(enabled)
    if _MODULE is not None and isinstance(_MODULE, NativeModule):
        _MODULE.binding.set_host_checks(_HOST_CHECKS[0])
    return old


def host_checks():
    return _HOST_CHECKS[0]


def library_path():
    return os.environ.get("CPU_ATTENTION_LIB") or os.path.join(_DIR, LIBRARY)


def load_library(path=None):
    """The ctypes handle of the kernel library, with every entry's signature set."""
    lib = ctypes.CDLL(path or library_path())
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    lib.ca_store.argtypes = [ctypes.POINTER(StoreArgs), vp]
    lib.ca_store.restype = ctypes.c_int
    lib.ca_decode.argtypes = [ctypes.POINTER(DecodeArgs), vp]
    lib.ca_decode.restype = ctypes.c_int
    lib.ca_decode_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), vp]
    lib.ca_decode_noalloc.restype = ctypes.c_int
    lib.ca_decode_workspace_bytes.argtypes = [i64, i64, i64, i64, i64]
    lib.ca_decode_workspace_bytes.restype = i64
    lib.ca_flash.argtypes = [ctypes.POINTER(FlashArgs), vp]
    lib.ca_flash.restype = ctypes.c_int
    lib.ca_flash_workspace_bytes.argtypes = [i64, i64, i64, i64, i64, i32]
    lib.ca_flash_workspace_bytes.restype = i64
    lib.ca_abi_version.argtypes = []
    lib.ca_abi_version.restype = ctypes.c_int
    lib.ca_version.argtypes = []
    lib.ca_version.restype = ctypes.c_char_p
    lib.ca_status_string.argtypes = [ctypes.c_int]
    lib.ca_status_string.restype = ctypes.c_char_p
    if lib.ca_abi_version() != ABI_VERSION:
        raise RuntimeError(f"cpu_attention: {path or library_path()} has ABI "
                           f"{lib.ca_abi_version()}, this package needs {ABI_VERSION}")
    return lib


# ---------------------------------------------------------------------------
# tensor helpers
# ---------------------------------------------------------------------------
def _plain(x):
    return type(x) in _PLAIN


def _stride(t, i):
    """Stride of dim i, 0 for a dim of size 1 (never stepped over)."""
    return 0 if t.shape[i] == 1 else t.stride(i)


def _strides3(st, sh):
    """The first three of ``st`` (a tensor's strides), 0 where ``sh`` has size 1."""
    return (0 if sh[0] == 1 else st[0], 0 if sh[1] == 1 else st[1], 0 if sh[2] == 1 else st[2])


def _rows_ok(t, hd):
    """Heads and dims contiguous (any token stride: chunks of a fused projection)."""
    return t.stride(-1) == 1 and (t.shape[-2] == 1 or t.stride(-2) == hd)


def aligned(t, strides=()):
    """The kernels read 16-byte vectors: the data pointer and the given element
    strides must keep 16-byte alignment."""
    e = _ESIZE.get(t.dtype, 1)
    return t.data_ptr() % 16 == 0 and all((s * e) % 16 == 0 for s in strides)


def _on_gpu(device, *ts):
    return all(t.is_cuda and t.device == device for t in ts)


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device):
    """torch's current stream on ``device`` as a raw handle (the direct query when
    this torch has it: it skips building a Stream object on every call)."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def _caches_ok(kc, vc, dtype, heads, hd):
    """``[blocks, heads, page, dim]``, contiguous, matching, page a multiple of 16
    (the reference's _caches_ok, _C.mojo:74-80)."""
    if not (_plain(kc) and _plain(vc)) or kc.dim() != 4 or vc.shape != kc.shape:
        return False
    return (kc.dtype == dtype and vc.dtype == dtype and kc.shape[1] == heads
            and kc.shape[3] == hd and kc.shape[2] > 0 and kc.shape[2] % 16 == 0
            and kc.is_contiguous() and vc.is_contiguous())


def _int_vector(t, dtype, n):
    return _plain(t) and t.dim() == 1 and t.dtype == dtype and t.shape[0] == n and t.is_contiguous()


def _index_on(t, device):
    """An index tensor on the kernels' device (CPU index tensors are copied over)."""
    return t if t.device == device else t.to(device, non_blocking=True)


class Module:
    """The kernel module: the reference's ``decode``/``store``/``flash`` entries
    over the C ABI of the gfx950 library."""

    def __init__(self, lib):
        self.lib = lib
        # Workspace sizes are pure functions of the shapes: asked once per shape.
        self._dec_ws = {}
        self._flash_ws = {}

    def _raise(self, rc, what):
        msg = self.lib.ca_status_string(rc).decode()
        raise RuntimeError(f"cpu_attention: {what} failed on the GPU: {msg}")

    def tier(self):
        return "gfx950"

    def amx_available(self):
        return False

    def version(self):
        return self.lib.ca_version().decode()

    # -- decode ---------------------------------------------------------------
    def decode(self, rt, q, k_cache, v_cache, k, v, slots, lens, page_table, scale, dst):
        """Paged decode of q ``[seqs, (1,) heads, dim]`` (MHA); see _C.mojo:87-171.
        With k/v, each sequence's new token is stored first: at ``slots`` (then
        ``lens`` is the length after the store), or appended at ``lens`` (the
        length before). Writes ``dst`` when given, else a new tensor; returns it,
        or None for anything the kernels do not take."""
        return self._decode(q, k_cache, v_cache, k, v, slots, lens, page_table, scale, dst, 1)

    def append_decode(self, rt, q, k_cache, v_cache, k, v, lens, page_table, scale):
        """The prompt append of flash_attn_with_kvcache (flash_attn_interface.py:109-117)
        in one native call: token j of ``k``/``v`` ``[seqs, n, heads, dim]`` is stored
        at position ``lens + j`` of its sequence (through the page table, inside
        the store kernel), then q attends ``lens + n`` keys. Returns the output, or
        None for anything the kernels do not take (the caller then takes the
        reference's path, which raises the precise error)."""
        if not (isinstance(k, torch.Tensor) and isinstance(v, torch.Tensor)):
            return None
        if not (_plain(k) and _plain(v)) or k.dim() != 4 or v.shape != k.shape \
                or not isinstance(q, torch.Tensor) or q.shape[0] != k.shape[0] \
                or tuple(k.shape[2:]) != tuple(q.shape[-2:]):
            return None
        b, n = k.shape[0], k.shape[1]
        if n < 1:
            return None
        kr, vr = k.reshape(b * n, *k.shape[2:]), v.reshape(b * n, *v.shape[2:])
        if vr.stride() != kr.stride():
            return None
        return self._decode(q, k_cache, v_cache, kr, vr, None, lens, page_table, scale, None, n)

    def _decode(self, q, k_cache, v_cache, k, v, slots, lens, page_table, scale, dst, n):
        """decode() with ``n`` new tokens per sequence (k/v rows ``[seqs * n, heads,
        dim]`` when n > 1, appended at ``lens``)."""
        if not (_plain(q) and _plain(page_table) and isinstance(lens, torch.Tensor)):
            return None
        qsh = q.shape
        nd = len(qsh)
        if nd not in (3, 4) or (nd == 4 and qsh[1] != 1):
            return None
        b, heads, hd = qsh[0], qsh[-2], qsh[-1]
        dt = q.dtype
        if dt not in DTYPES or hd not in HEAD_DIMS or not _rows_ok(q, hd):
            return None
        if not _caches_ok(k_cache, v_cache, dt, heads, hd):
            return None
        page = k_cache.shape[2]
        if page_table.dim() != 2 or page_table.dtype != torch.int32 or page_table.shape[0] != b \
                or not page_table.is_contiguous():
            return None
        width = page_table.shape[1]
        if not _int_vector(lens, torch.int32, b):
            return None
        store = k is not None
        if store:
            rows = q.shape if n == 1 else (b * n, heads, hd)
            if not (_plain(k) and _plain(v) and k.shape == rows and v.shape == rows
                    and v.stride() == k.stride()):
                return None
            if k.dtype != q.dtype or v.dtype != q.dtype or not _rows_ok(k, hd):
                return None
        elif v is not None:
            return None
        if slots is not None and not (store and _int_vector(slots, torch.int64, b)):
            return None
        dev = q.device
        if not q.is_cuda or not _on_gpu(dev, k_cache, v_cache) or (store and not _on_gpu(dev, k, v)):
            return None
        if dst is not None and not (_plain(dst) and dst.shape == q.shape and dst.dtype == q.dtype
                                    and dst.is_contiguous() and _on_gpu(dev, dst)):
            return None
        q_stride = _stride(q, 0)
        kv_stride = _stride(k, 0) if store else 0
        # 16-byte vectors: pointers and element strides (a multiple of 16 / esize)
        qp, kcp, vcp = q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr()
        knp, vnp = (k.data_ptr(), v.data_ptr()) if store else (0, 0)
        if (qp | kcp | vcp | knp | vnp) % 16 or (q_stride | kv_stride) % (16 // _ESIZE[dt]):
            return None
        nblocks = k_cache.shape[0]
        # The data-dependent rules (_C.mojo:139-153), on the host.
        if _HOST_CHECKS[0] and b:
            if slots is not None and int(slots.max()) >= nblocks * page:
                return None
            if int(lens.max()) + (n if store and slots is None else 0) > width * page:
                return None
        lens = _index_on(lens, dev)
        page_table = _index_on(page_table, dev)
        if slots is not None:
            slots = _index_on(slots, dev)
        out = dst if dst is not None else torch.empty(qsh, dtype=dt, device=dev)
        key = (b, heads, hd, page, width)
        ws_bytes = self._dec_ws.get(key)
        if ws_bytes is None:
            ws_bytes = self._dec_ws[key] = self.lib.ca_decode_workspace_bytes(*key)
        wst = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None  # held past the launch
        ws = wst.data_ptr() if ws_bytes else None
        args = DecodeArgs(qp, q_stride, kcp, vcp, knp or None, vnp or None, kv_stride,
                          slots.data_ptr() if slots is not None else None, lens.data_ptr(),
                          page_table.data_ptr(), width, out.data_ptr(), b, heads, hd, page, nblocks,
                          float(hd) ** -0.5 if scale is None else float(scale), DTYPES[dt],
                          ws, ws_bytes, n if store else 0)
        rc = self.lib.ca_decode(ctypes.byref(args), _stream(dev))
        if rc == CA_DECLINED:
            return None
        if rc != CA_OK:
            self._raise(rc, "decode")
        return out

    # -- store ----------------------------------------------------------------
    def store(self, rt, key, value, k_cache, v_cache, slots):
        """``reshape_and_cache``: token i of key/value ``[tokens, heads, dim]`` goes
        to slot ``slots[i]`` (int64; negative skips it). True, or None
        (_C.mojo:174-213)."""
        if not (isinstance(key, torch.Tensor) and isinstance(value, torch.Tensor)
                and isinstance(slots, torch.Tensor)):
            return None
        if not (_plain(key) and _plain(value)) or key.dim() != 3 or value.dim() != 3:
            return None
        n, heads, hd = key.shape
        if key.dtype not in DTYPES or hd not in HEAD_DIMS or value.dtype != key.dtype \
                or not _rows_ok(key, hd):
            return None
        if value.shape != key.shape or value.stride() != key.stride():
            return None
        if not _caches_ok(k_cache, v_cache, key.dtype, heads, hd) \
                or not _int_vector(slots, torch.int64, n):
            return None
        dev = k_cache.device
        if not k_cache.is_cuda or not _on_gpu(dev, v_cache, key, value):
            return None
        tstride = _stride(key, 0)
        if not (aligned(key, (tstride,)) and aligned(value) and aligned(k_cache)
                and aligned(v_cache)):
            return None
        page, nblocks = k_cache.shape[2], k_cache.shape[0]
        if _HOST_CHECKS[0] and n and int(slots.max()) >= nblocks * page:
            return None
        if n == 0:
            return True
        slots = _index_on(slots, dev)
        args = StoreArgs(
            key=key.data_ptr(), value=value.data_ptr(), token_stride=tstride,
            k_cache=k_cache.data_ptr(), v_cache=v_cache.data_ptr(), slot_mapping=slots.data_ptr(),
            num_tokens=n, num_heads=heads, head_dim=hd, page_size=page, num_blocks=nblocks,
            dtype=DTYPES[key.dtype])
        rc = self.lib.ca_store(ctypes.byref(args), _stream(dev))
        if rc == CA_DECLINED:
            return None
        if rc != CA_OK:
            self._raise(rc, "store")
        return True

    # -- flash ----------------------------------------------------------------
    def flash_workspace_bytes(self, q, k):
        key = (q.shape[0], q.shape[1], k.shape[1], q.shape[2], q.shape[3], q.dtype)
        need = self._flash_ws.get(key)
        if need is None:
            need = self._flash_ws[key] = self._flash_ws_query(q, k)
        return need

    def _flash_ws_query(self, q, k):
        return self.lib.ca_flash_workspace_bytes(q.shape[0], q.shape[1], k.shape[1], q.shape[2],
                                                 q.shape[3], DTYPES.get(q.dtype, 0))

    def flash(self, rt, q, k, v, scale, causal, ws, ws_bytes):
        """flash_attn_func over q/k/v ``[batch, seq, heads, dim]`` (MHA, dims
        contiguous). Returns the output, the workspace bytes it needs when
        ``ws_bytes`` is short (an int), or None (_C.mojo:232-316).  Small calls
        are bound by this host work, so each tensor's shape and strides are read
        once."""
        if not (type(q) in _PLAIN and type(k) in _PLAIN and type(v) in _PLAIN):
            return None
        qsh, ksh = q.shape, k.shape
        if len(qsh) != 4 or len(ksh) != 4 or v.shape != ksh:
            return None
        b, sq, heads, hd = qsh
        sk = ksh[1]
        dt = q.dtype
        if dt not in DTYPES or hd not in HEAD_DIMS or sq < 1 or sk < 1:
            return None
        if ksh[0] != b or ksh[2] != heads or ksh[3] != hd or k.dtype != dt or v.dtype != dt:
            return None
        qst, kst, vst = q.stride(), k.stride(), v.stride()
        if qst[3] != 1 or kst[3] != 1 or vst[3] != 1:
            return None
        if not (causal is True or causal is False):
            return None
        dev = q.device
        if not q.is_cuda or k.device != dev or v.device != dev:
            return None
        qs, ks, vs = _strides3(qst, qsh), _strides3(kst, ksh), _strides3(vst, ksh)
        # 16-byte vectors: pointers and element strides (a multiple of 16 / esize)
        qp, kp, vp = q.data_ptr(), k.data_ptr(), v.data_ptr()
        unit = 16 // _ESIZE[dt]
        if (qp | kp | vp) % 16 or (qs[0] | qs[1] | qs[2] | ks[0] | ks[1] | ks[2] | vs[0] | vs[1] | vs[2]) % unit:
            return None
        key = (b, sq, sk, heads, hd, dt)
        need = self._flash_ws.get(key)
        if need is None:
            need = self._flash_ws[key] = self._flash_ws_query(q, k)
        if need > ws_bytes:
            return int(need)
        out = torch.empty(qsh, dtype=dt, device=dev)
        args = FlashArgs(qp, kp, vp, out.data_ptr(), b, sq, sk, heads, hd, qs, ks, vs,
                         float(hd) ** -0.5 if scale is None else float(scale), 1 if causal else 0,
                         DTYPES[dt], 0, ws or None, ws_bytes)
        rc = self.lib.ca_flash(ctypes.byref(args), _stream(dev))
        if rc == CA_DECLINED:
            return None
        if rc != CA_OK:
            self._raise(rc, "flash")
        return out


def _stream_of_index(index):
    return torch.cuda.current_stream(index).cuda_stream


class NativeModule(Module):
    """``Module`` with decode/store/flash's argument handling in the native
    extension ``_binding`` (csrc/ca_binding.cpp): the same rules in the same
    order, the same results.  The entries are the extension's functions
    themselves, so a call runs no Python code of this package."""

    ENTRIES = ("ca_decode", "ca_store", "ca_flash", "ca_decode_workspace_bytes",
               "ca_flash_workspace_bytes", "ca_status_string")

    def __init__(self, lib, binding):
        super().__init__(lib)
        addrs = tuple(ctypes.cast(getattr(lib, name), ctypes.c_void_p).value for name in self.ENTRIES)
        binding.init(addrs, _PLAIN, _RAW_STREAM or _stream_of_index, _HOST_CHECKS[0])
        self.binding = binding
        self.decode = binding.decode
        self.store = binding.store
        self.flash = binding.flash

    def _decode(self, q, k_cache, v_cache, k, v, slots, lens, page_table, scale, dst, n):
        return self.binding.decode(None, q, k_cache, v_cache, k, v, slots, lens, page_table, scale, dst, n)


def _native_binding():
    """The ``_binding`` extension, or None when it is not built or
    ``CPU_ATTENTION_BINDING=ctypes``.  A built extension that fails to load
    raises."""
    if os.environ.get("CPU_ATTENTION_BINDING", "native") == "ctypes":
        return None
    import importlib
    import importlib.util

    if importlib.util.find_spec(__package__ + "._binding") is None:
        return None
    return importlib.import_module(__package__ + "._binding")


_MODULE = None
_LOCK = threading.Lock()


def module():
    """The kernel module (RuntimeError when the library is not built)."""
    global _MODULE
    if _MODULE is None:
        with _LOCK:
            if _MODULE is None:
                path = library_path()
                if not os.path.exists(path):
                    raise RuntimeError("cpu_attention: the gfx950 kernel library is not built; run "
                                       "`python cpu-attention_amd/build.py`")
                lib = load_library(path)
                binding = _native_binding()
                _MODULE = NativeModule(lib, binding) if binding is not None else Module(lib)
    return _MODULE


def ctypes_module():
    """A ``Module`` (the ctypes binding) over the loaded library, whichever
    binding ``module()`` uses."""
    return Module(module().lib)


def runtime():
    """An opaque handle the entries take as their first argument (the reference
    passes its runtime-config address here, _kernel.py:167-207; the GPU build
    keeps no runtime state)."""
    module()
    return ABI_VERSION


@functools.lru_cache(maxsize=None)
def physical_cores():
    """Physical cores this process may run on: the CPUs of its affinity mask,
    counted once per set of hardware threads that share a core (the sysfs
    ``thread_siblings_list`` of each CPU).  Falls back to the CPU count."""
    try:
        cpus = sorted(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        cpus = list(range(os.cpu_count() or 1))
    cores = set()
    for cpu in cpus:
        try:
            with open(f"/sys/devices/system/cpu/cpu{cpu}/topology/thread_siblings_list") as f:
                cores.add(f.read().strip())
        except OSError:
            return len(cpus) or 1
    return len(cores) or len(cpus) or 1


@functools.lru_cache(maxsize=None)
def llc_bytes():
    """Size in bytes of the largest-level cache sysfs lists for CPU 0 (the last
    level), or 32 MiB when sysfs says nothing."""
    base = "/sys/devices/system/cpu/cpu0/cache"
    best = (0, 0)  # (level, bytes)
    try:
        names = [n for n in os.listdir(base) if n.startswith("index")]
    except OSError:
        names = []
    for name in names:
        try:
            with open(f"{base}/{name}/level") as f:
                level = int(f.read())
            with open(f"{base}/{name}/size") as f:
                text = f.read().strip().upper()
        except (OSError, ValueError):
            continue
        scale = {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}.get(text[-1:], 1)
        digits = text.rstrip("KMG")
        if digits.isdigit():
            best = max(best, (level, int(digits) * scale))
    return best[1] or 32 << 20


_WS = {}
_WS_LOCK = threading.Lock()


def workspace(nbytes=0):
    """A flash workspace for callers of ``module().flash`` that pass their own, as
    (address, bytes): one per (thread, device, current stream), grown to
    ``nbytes`` and never shrunk; (0, 0) until something asks for one.

    Keyed by stream because calls on two streams would otherwise write the same
    partials at once.  A buffer that is outgrown is kept (not returned to the
    allocator), since a captured graph may still name its address: the buffers
    of a (thread, device, stream) stay until ``release_workspace()`` drops them or
    the process ends, so a process that keeps creating threads or streams should
    release each one's buffers once nothing (no graph) uses them.  The package's
    own ``flash_attn_func`` does not use this: it allocates the scratch per call
    on the current stream."""
    if not torch.cuda.is_available():
        return 0, 0
    dev = torch.cuda.current_device()
    key = (threading.get_ident(), dev, _stream(torch.device("cuda", dev)))
    with _WS_LOCK:
        held = _WS.setdefault(key, [])
        if nbytes and (not held or held[-1].numel() < nbytes):
            size = max(nbytes, 2 * held[-1].numel()) if held else nbytes
            held.append(torch.empty(size, dtype=torch.uint8, device=f"cuda:{dev}"))
        if not held:
            return 0, 0
        return held[-1].data_ptr(), held[-1].numel()


def release_workspace(all_streams=False):
    """Drops the calling thread's ``workspace()`` buffers on the current device:
    those of the current stream, or of every stream with ``all_streams``.  The
    caller vouches that no pending call or captured graph still uses them (their
    memory goes back to torch's allocator).  Returns how many were dropped."""
    if not torch.cuda.is_available():
        return 0
    dev = torch.cuda.current_device()
    me = threading.get_ident()
    stream = _stream(torch.device("cuda", dev))
    with _WS_LOCK:
        keys = [k for k in _WS if k[0] == me and k[1] == dev and (all_streams or k[2] == stream)]
        return sum(len(_WS.pop(k)) for k in keys)
