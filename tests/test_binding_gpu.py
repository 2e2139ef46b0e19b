"""The two bindings of the kernel module give the same results (GPU).

``K.module()`` is the native binding (csrc/ca_binding.cpp) when it is built, and
``K.ctypes_module()`` the ctypes one (cpu_attention/_kernel.py, class Module).
Both apply the reference's acceptance rules (_C.mojo:87-316) before calling the
same C ABI.  Here every case runs through each binding on its own copy of the
caches.  Accepted calls must return bit-identical outputs and leave
bit-identical caches.  Declined calls must return None from both.  Calls that
raise must raise the same exception type.  The cases cover each rule: dtypes,
shapes, strides, alignment, devices, the engine path's slots, `dst`, the
prompt append, the host checks, and the few-rows prefill's workspace request.
"""

import pytest
import torch

from cpu_attention import _kernel as K

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module")
def bindings():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    native = K.module()
    if not isinstance(native, K.NativeModule):
        pytest.skip("native binding not built")
    return native, K.ctypes_module()


def _outcome(fn):
    """(kind, value): the result, or the exception type a call raised."""
    try:
        r = fn()
    except Exception as e:  # noqa: BLE001 -- compared across bindings
        return "raise", type(e)
    if r is None or r is True:
        return "const", r
    if isinstance(r, int):
        return "int", r
    torch.cuda.synchronize()
    return "tensor", r


def _same(a, b):
    assert a[0] == b[0], (a, b)
    if a[0] == "tensor":
        assert a[1].shape == b[1].shape and a[1].dtype == b[1].dtype
        assert torch.equal(a[1].view(torch.uint8) if a[1].dtype == torch.bfloat16 else a[1],
                           b[1].view(torch.uint8) if b[1].dtype == torch.bfloat16 else b[1])
    else:
        assert a[1] == b[1], (a, b)


def paged(dtype, n=3, h=4, e=64, page=16, width=6, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    nb = n * width + 2
    kc = torch.randn(nb, h, page, e, generator=g, device=DEV).to(dtype)
    vc = torch.randn(nb, h, page, e, generator=g, device=DEV).to(dtype)
    table = torch.randperm(n * width, device=DEV, generator=g).to(torch.int32).view(n, width)
    lens = torch.tensor([0, 37, width * page - 1][:n], dtype=torch.int32, device=DEV)
    q = torch.randn(n, 1, h, e, generator=g, device=DEV).to(dtype)
    k = torch.randn(n, 1, h, e, generator=g, device=DEV).to(dtype)
    v = torch.randn(n, 1, h, e, generator=g, device=DEV).to(dtype)
    return q, kc, vc, k, v, lens, table


def _run_decode(mods, case, *args):
    """Runs `case(mod, kc, vc)` per binding on fresh copies of the caches."""
    outs = []
    for mod in mods:
        kc, vc = args[0].clone(), args[1].clone()
        res = _outcome(lambda: case(mod, kc, vc))
        torch.cuda.synchronize()
        outs.append((res, kc, vc))
    (ra, kca, vca), (rb, kcb, vcb) = outs
    _same(ra, rb)
    assert torch.equal(kca.view(torch.uint8) if kca.dtype == torch.bfloat16 else kca,
                       kcb.view(torch.uint8) if kcb.dtype == torch.bfloat16 else kcb)
    assert torch.equal(vca.view(torch.uint8) if vca.dtype == torch.bfloat16 else vca,
                       vcb.view(torch.uint8) if vcb.dtype == torch.bfloat16 else vcb)
    return ra


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_cases(bindings, dtype):
    q, kc, vc, k, v, lens, table = paged(dtype)
    rt = K.runtime()
    n, width, page = q.shape[0], table.shape[1], kc.shape[2]
    slots = (table[:, 0].long() * page + 3).contiguous()
    cases = {
        "plain": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens, table, None, None),
        "q 3-D": lambda m, a, b: m.decode(rt, q[:, 0], a, b, None, None, None, lens, table, 0.3, None),
        "append": lambda m, a, b: m.decode(rt, q, a, b, k, v, None, lens.clamp(max=width * page - 2),
                                           table, None, None),
        "slots": lambda m, a, b: m.decode(rt, q, a, b, k, v, slots, lens.clamp(min=1), table, None, None),
        "dst": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens, table, None, torch.empty_like(q)),
        "cpu index tensors": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens.cpu(), table.cpu(),
                                                      None, None),
        "scale int": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens, table, 1, None),
        "scale str": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens, table, "0.25", None),
        "scale bad": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens, table, "x", None),
        # declines
        "int64 table": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens, table.long(), None, None),
        "short lens": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens[:2], table, None, None),
        "int64 lens": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens.long(), table, None, None),
        "k without v": lambda m, a, b: m.decode(rt, q, a, b, k, None, None, lens, table, None, None),
        "v without k": lambda m, a, b: m.decode(rt, q, a, b, None, v, None, lens, table, None, None),
        "slots without k": lambda m, a, b: m.decode(rt, q, a, b, None, None, slots, lens, table, None, None),
        "int32 slots": lambda m, a, b: m.decode(rt, q, a, b, k, v, slots.int(), lens, table, None, None),
        "q on cpu": lambda m, a, b: m.decode(rt, q.cpu(), a, b, None, None, None, lens, table, None, None),
        "k on cpu": lambda m, a, b: m.decode(rt, q, a, b, k.cpu(), v.cpu(), None, lens, table, None, None),
        "half": lambda m, a, b: m.decode(rt, q.half(), a, b, None, None, None, lens, table, None, None),
        "L=2": lambda m, a, b: m.decode(rt, torch.cat([q, q], 1), a, b, None, None, None, lens, table, None, None),
        "dst shape": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens, table, None, q[:1].clone()),
        "dst dtype": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens, table, None,
                                              torch.empty(q.shape, device=DEV, dtype=torch.float16)),
        "dst view": lambda m, a, b: m.decode(rt, q, a, b, None, None, None, lens, table, None,
                                             torch.empty(n, 1, q.shape[2], 2 * q.shape[3], device=DEV,
                                                         dtype=dtype)[..., :q.shape[3]]),
        "heads strided q": lambda m, a, b: m.decode(rt, torch.cat([q, q], 3)[..., :q.shape[3]], a, b, None, None,
                                                    None, lens, table, None, None),
        "misaligned q": lambda m, a, b: m.decode(rt, torch.cat([q.flatten(), q.flatten()[:1]])[1:].view(q.shape),
                                                 a, b, None, None, None, lens, table, None, None),
        "caches view": lambda m, a, b: m.decode(rt, q, a[:, :, :, :32], b[:, :, :, :32], None, None, None, lens,
                                                table, None, None),
        "caches subclass": lambda m, a, b: m.decode(rt, q, a.as_subclass(Sub), b, None, None, None, lens, table,
                                                    None, None),
        "lens past capacity": lambda m, a, b: m.decode(rt, q, a, b, k, v, None, lens + 1, table, None, None),
        "slot past cache": lambda m, a, b: m.decode(rt, q, a, b, k, v, slots + a.shape[0] * page, lens, table,
                                                    None, None),
    }
    seen = {}
    for name, case in cases.items():
        seen[name] = _run_decode(bindings, case, kc, vc)[0]
    for name in ("plain", "q 3-D", "append", "slots", "dst", "cpu index tensors", "scale int", "scale str"):
        assert seen[name] == "tensor", (name, seen[name])
    assert seen["scale bad"] == "raise"
    for name in ("int64 table", "short lens", "int64 lens", "k without v", "v without k", "slots without k",
                 "int32 slots", "q on cpu", "k on cpu", "half", "L=2", "dst shape", "dst dtype", "dst view",
                 "heads strided q", "misaligned q", "caches view", "caches subclass", "lens past capacity", "slot past cache"):
        assert seen[name] == "const", (name, seen[name])


class Sub(torch.Tensor):
    pass


def test_decode_without_host_checks(bindings):
    """With host checks off both bindings launch the out-of-range calls; the
    kernels skip what lies past the page table or the cache, identically."""
    q, kc, vc, k, v, lens, table = paged(torch.bfloat16, seed=1)
    rt, page = K.runtime(), kc.shape[2]
    slots = (table[:, 0].long() * page + 5).contiguous()
    old = K.set_host_checks(False)
    try:
        r = _run_decode(bindings, lambda m, a, b: m.decode(rt, q, a, b, k, v, None, lens + 1, table, None, None),
                        kc, vc)
        assert r[0] == "tensor"
        r = _run_decode(bindings, lambda m, a, b: m.decode(rt, q, a, b, k, v, slots + a.shape[0] * page, lens,
                                                           table, None, None), kc, vc)
        assert r[0] == "tensor"
    finally:
        K.set_host_checks(old)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prompt_append(bindings, dtype):
    q, kc, vc, _, _, lens, table = paged(dtype, seed=2)
    g = torch.Generator(device=DEV).manual_seed(3)
    kn = torch.randn(q.shape[0], 5, q.shape[2], q.shape[3], generator=g, device=DEV).to(dtype)
    vn = torch.randn_like(kn)
    lens = lens.clamp(max=table.shape[1] * kc.shape[2] - 5)
    rt = K.runtime()
    r = _run_decode(bindings, lambda m, a, b: m.append_decode(rt, q, a, b, kn, vn, lens, table, None), kc, vc)
    assert r[0] == "tensor"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_store_cases(bindings, dtype):
    _, kc, vc, _, _, _, table = paged(dtype, seed=4)
    g = torch.Generator(device=DEV).manual_seed(5)
    t, h, e, page = 40, kc.shape[1], kc.shape[3], kc.shape[2]
    key = torch.randn(t, h, e, generator=g, device=DEV).to(dtype)
    val = torch.randn(t, h, e, generator=g, device=DEV).to(dtype)
    slots = torch.randperm(kc.shape[0] * page, generator=g, device=DEV)[:t].contiguous()
    slots[::7] = -1
    fused = torch.randn(t, 3, h, e, generator=g, device=DEV).to(dtype)
    rt = K.runtime()
    cases = {
        "plain": lambda m, a, b: m.store(rt, key, val, a, b, slots),
        "one token": lambda m, a, b: m.store(rt, key[:1], val[:1], a, b, slots[1:2]),
        "no token": lambda m, a, b: m.store(rt, key[:0], val[:0], a, b, slots[:0]),
        "fused views": lambda m, a, b: m.store(rt, fused[:, 1], fused[:, 2], a, b, slots),
        "cpu slots": lambda m, a, b: m.store(rt, key, val, a, b, slots.cpu()),
        # declines
        "int32 slots": lambda m, a, b: m.store(rt, key, val, a, b, slots.int()),
        "strides differ": lambda m, a, b: m.store(rt, fused[:, 1], val, a, b, slots),
        "misaligned": lambda m, a, b: m.store(rt, torch.cat([key.flatten(), key.flatten()[:1]])[1:].view(key.shape),
                                              val, a, b, slots),
        "slot past cache": lambda m, a, b: m.store(rt, key, val, a, b, slots + a.shape[0] * page),
        "cpu key": lambda m, a, b: m.store(rt, key.cpu(), val.cpu(), a, b, slots),
        "not tensors": lambda m, a, b: m.store(rt, 1, 2, a, b, slots),
        "2-D key": lambda m, a, b: m.store(rt, key[:, 0], val[:, 0], a, b, slots),
    }
    seen = {name: _run_decode(bindings, case, kc, vc)[0:2] for name, case in cases.items()}
    for name in ("plain", "one token", "no token", "fused views", "cpu slots"):
        assert seen[name] == ("const", True), (name, seen[name])
    for name in ("int32 slots", "strides differ", "misaligned", "slot past cache", "cpu key", "not tensors",
                 "2-D key"):
        assert seen[name] == ("const", None), (name, seen[name])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_flash_cases(bindings, dtype):
    g = torch.Generator(device=DEV).manual_seed(6)
    qkv = torch.randn(2, 70, 3, 4, 64, generator=g, device=DEV).to(dtype)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    q1 = torch.randn(2, 1, 4, 64, generator=g, device=DEV).to(dtype)
    kl = torch.randn(2, 3000, 4, 64, generator=g, device=DEV).to(dtype)
    rt = K.runtime()
    native, ctypes_mod = bindings
    need = ctypes_mod.flash(rt, q1, kl, kl, None, False, 0, 0)
    ws = torch.empty(need if isinstance(need, int) else 0, dtype=torch.uint8, device=DEV)
    cases = {
        "fused causal": lambda m: m.flash(rt, q, k, v, None, True, 0, 0),
        "fused": lambda m: m.flash(rt, q, k, v, 0.2, False, 0, 0),
        "contiguous": lambda m: m.flash(rt, q.contiguous(), k.contiguous(), v.contiguous(), None, True, None, 0),
        "cross short ws": lambda m: m.flash(rt, q1, kl, kl, None, False, 0, 0),
        "cross with ws": lambda m: m.flash(rt, q1, kl, kl, None, False, ws.data_ptr(), ws.numel()),
        # declines and errors
        "causal int": lambda m: m.flash(rt, q, k, v, None, 1, 0, 0),
        "head dim 96": lambda m: m.flash(rt, q[..., :48], k[..., :48], v[..., :48], None, True, 0, 0),
        "dim strided": lambda m: m.flash(rt, qkv[:, :, 0, :, ::2], k[..., :32], v[..., :32], None, True, 0, 0),
        "gqa": lambda m: m.flash(rt, q, k[:, :, :2], v[:, :, :2], None, True, 0, 0),
        "cpu": lambda m: m.flash(rt, q.cpu(), k.cpu(), v.cpu(), None, True, 0, 0),
        "misaligned": lambda m: m.flash(rt, torch.cat([q.flatten(), q.flatten()[:1]])[1:].view(q.shape), k, v,
                                        None, True, 0, 0),
        "subclass": lambda m: m.flash(rt, q.as_subclass(Sub), k, v, None, True, 0, 0),
        "ws_bytes None": lambda m: m.flash(rt, q1, kl, kl, None, False, 0, None),
    }
    seen = {}
    for name, case in cases.items():
        a, b = _outcome(lambda: case(native)), _outcome(lambda: case(ctypes_mod))
        _same(a, b)
        seen[name] = a[0]
    for name in ("fused causal", "fused", "contiguous", "cross with ws"):
        assert seen[name] == "tensor", (name, seen[name])
    assert seen["cross short ws"] == ("int" if need else "tensor")
    for name in ("causal int", "head dim 96", "dim strided", "gqa", "cpu", "misaligned", "subclass"):
        assert seen[name] == "const", (name, seen[name])
    assert seen["ws_bytes None"] == "raise"
