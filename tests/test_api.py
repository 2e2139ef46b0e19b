"""What the kernels cannot do is rejected, never silently ignored (CPU only).

Mirrors the reference's tests/test_api.py: the same calls raise the same exception
types.  Each bad-argument case also checks the message, to show the precise
check fired (and not the GPU build's own device rule, which comes last), and a
well-formed call with CPU tensors is refused with the device message.
"""

import os
import subprocess
import sys

import pytest
import torch

import cpu_attention as C
from cpu_attention import _kernel as K
from conftest import PKG


def paged():
    q = torch.randn(2, 1, 4, 64)
    kc = torch.zeros(4, 4, 16, 64)
    return q, kc, kc.clone(), torch.arange(4, dtype=torch.int32).view(2, 2)


@pytest.mark.parametrize("kwargs", [
    dict(window_size=(8, 0)), dict(softcap=30.0), dict(return_softmax_lse=True),
    dict(attention_chunk=64), dict(rotary_cos=torch.ones(1)), dict(qv=torch.ones(1)),
    dict(alibi_slopes=torch.ones(4)), dict(rotary_sin=torch.ones(1)),
    dict(cache_leftpad=torch.ones(1)), dict(cu_seqlens_q=torch.ones(1)),
    dict(cu_seqlens_k_new=torch.ones(1)), dict(max_seqlen_q=4), dict(rotary_seqlens=torch.ones(1)),
    dict(q_descale=torch.ones(1)), dict(k_descale=torch.ones(1)), dict(v_descale=torch.ones(1)),
])
def test_kvcache_unsupported_options(kwargs):
    q, kc, vc, bt = paged()
    with pytest.raises(NotImplementedError):
        C.flash_attn_with_kvcache(q, kc, vc, cache_seqlens=4, page_table=bt, **kwargs)


def test_kvcache_tuning_hints_are_ignored_not_rejected():
    q, kc, vc, bt = paged()
    # the hints pass the option screen; CPU tensors then meet the device rule
    with pytest.raises(ValueError, match="ROCm GPU"):
        C.flash_attn_with_kvcache(q, kc, vc, cache_seqlens=4, page_table=bt, num_splits=3,
                                  pack_gqa=True, scheduler_metadata=object(), sm_margin=2,
                                  causal=True, rotary_interleaved=False)


def test_kvcache_one_query_token_only():
    q, kc, vc, bt = paged()
    with pytest.raises(NotImplementedError):
        C.flash_attn_with_kvcache(q.expand(2, 3, 4, 64), kc, vc, cache_seqlens=4,
                                  page_table=bt)


@pytest.mark.parametrize("bad,msg", [
    ("dtype", "share a dtype"), ("head_dim", "head_dim must be"), ("page", "multiple of 16"),
    ("heads", "disagree on heads"), ("no_table", "pass `page_table`"), ("both_tables", "not both"),
    ("no_seqlens", "is required"), ("lens_dtype", "cache_seqlens must be"),
    ("table_dtype", "page_table must be"), ("capacity", "exceed the page table"),
    ("kv_shape", "k/v must both be"), ("q_dim", "q must be"), ("cache_shape", "must be"),
    ("noncontig", "must be contiguous"),
])
def test_kvcache_bad_arguments(bad, msg):
    q, kc, vc, bt = paged()
    lens = 4
    extra = {}
    if bad == "dtype":
        q = q.half()
    elif bad == "head_dim":
        q, kc, vc = q[..., :48], kc[..., :48].contiguous(), vc[..., :48].contiguous()
    elif bad == "page":
        kc, vc = kc[:, :, :8].contiguous(), vc[:, :, :8].contiguous()
    elif bad == "heads":
        q = q[:, :, :3]
    elif bad == "no_table":
        bt = None
    elif bad == "both_tables":
        extra = dict(block_table=bt)
    elif bad == "no_seqlens":
        lens = None
    elif bad == "lens_dtype":
        lens = torch.full((2,), 4, dtype=torch.int64)
    elif bad == "table_dtype":
        bt = bt.long()
    elif bad == "capacity":
        lens = 33  # 2 pages of 16
    elif bad == "kv_shape":
        extra = dict(k=torch.randn(2, 1, 4, 64), v=torch.randn(2, 1, 4, 32))
    elif bad == "q_dim":
        q = q[:, 0]
    elif bad == "cache_shape":
        vc = vc[:3]
    elif bad == "noncontig":
        kc = kc.transpose(2, 3).contiguous().transpose(2, 3)
    with pytest.raises(ValueError, match=msg):
        C.flash_attn_with_kvcache(q, kc, vc, cache_seqlens=lens, page_table=bt, **extra)


@pytest.mark.parametrize("kv_heads", [2, 1])
def test_gqa_mqa_not_supported_yet(kv_heads):
    q, kc, vc, bt = paged()
    kc = torch.zeros(4, kv_heads, 16, 64)
    with pytest.raises(NotImplementedError):
        C.flash_attn_with_kvcache(q, kc, kc.clone(), cache_seqlens=4, page_table=bt)
    k = torch.randn(2, 8, kv_heads, 64)
    with pytest.raises(NotImplementedError):
        C.flash_attn_func(torch.randn(2, 8, 4, 64), k, k)


@pytest.mark.parametrize("bad,msg", [
    ("dtype", "share a dtype"), ("heads", "do not match the cache"),
    ("slots_dtype", "int64"), ("slots_len", "int64"), ("past_end", "past the end"),
    ("rank", "key/value must both be"), ("page", "multiple of 16"),
])
def test_reshape_and_cache_bad_arguments(bad, msg):
    k = torch.randn(5, 2, 64)
    kc = torch.zeros(2, 2, 16, 64)
    slots = torch.arange(5)
    if bad == "dtype":
        k = k.bfloat16()
    elif bad == "heads":
        k = torch.randn(5, 3, 64)
    elif bad == "slots_dtype":
        slots = slots.int()
    elif bad == "slots_len":
        slots = slots[:4]
    elif bad == "past_end":
        slots = slots + 30
    elif bad == "rank":
        k = k[None]
    elif bad == "page":
        kc = torch.zeros(2, 2, 8, 64)
    with pytest.raises(ValueError, match=msg):
        C.reshape_and_cache(k, k, kc, kc.clone(), slots)


@pytest.mark.parametrize("bad,msg", [
    ("dtype", "share a dtype"), ("head_dim", "head_dim must be"), ("heads", "matching q"),
    ("batch", "matching q"), ("rank", "must be \\[batch"), ("empty", "matching q"),
])
def test_flash_bad_arguments(bad, msg):
    q, k = torch.randn(2, 8, 4, 64), torch.randn(2, 8, 4, 64)
    if bad == "dtype":
        q, k = q.half(), k.half()
    elif bad == "head_dim":
        q, k = q[..., :48], k[..., :48]
    elif bad == "heads":
        q = q[:, :, :3]
    elif bad == "batch":
        k = k[:1]
    elif bad == "rank":
        q = q[0]
    elif bad == "empty":
        k = k[:, :0]
    with pytest.raises(ValueError, match=msg):
        C.flash_attn_func(q, k, k)


@pytest.mark.parametrize("fn", [C.flash_attn_varlen_func, C.flash_attn_qkvpacked_func,
                                C.flash_attn_kvpacked_func,
                                C.flash_attn_varlen_qkvpacked_func,
                                C.flash_attn_varlen_kvpacked_func])
def test_not_ported(fn):
    with pytest.raises(NotImplementedError):
        fn(*[torch.zeros(1)] * 7)


def test_cpu_tensors_meet_the_device_rule():
    """Well-formed calls on CPU tensors: the GPU build refuses them precisely."""
    q, kc, vc, bt = paged()
    with pytest.raises(ValueError, match="ROCm GPU"):
        C.flash_attn_with_kvcache(q, kc, vc, cache_seqlens=4, page_table=bt)
    with pytest.raises(ValueError, match="ROCm GPU"):
        C.flash_attn_func(torch.randn(1, 8, 2, 64), torch.randn(1, 8, 2, 64), torch.randn(1, 8, 2, 64))
    with pytest.raises(ValueError, match="ROCm GPU"):
        C.reshape_and_cache(torch.randn(3, 4, 64), torch.randn(3, 4, 64), kc, vc, torch.arange(3))


@pytest.mark.parametrize("binding", ["default", "ctypes"])
def test_native_entries_decline_with_none(binding):
    """The module entries keep the reference's None convention (_C.mojo:87-316),
    through either binding."""
    mod, rt = (K.module() if binding == "default" else K.ctypes_module()), K.runtime()
    q, kc, vc, bt = paged()
    lens = torch.full((2,), 4, dtype=torch.int32)
    assert mod.decode(rt, q, kc, vc, None, None, None, lens, bt, None, None) is None
    assert mod.decode(rt, q.half(), kc, vc, None, None, None, lens, bt, None, None) is None
    assert mod.store(rt, torch.randn(3, 4, 64), torch.randn(3, 4, 64), kc, vc, torch.arange(3)) is None
    x = torch.randn(1, 4, 2, 64)
    assert mod.flash(rt, x, x, x, None, 1, 0, 0) is None  # causal must be True/False
    assert mod.flash(rt, x, x, x, None, True, 0, 0) is None  # CPU tensors
    assert mod.tier() == "gfx950" and mod.amx_available() is False


def test_native_binding_is_the_default_when_built():
    """The C++ binding serves the entries once built; CPU_ATTENTION_BINDING=ctypes
    selects the ctypes one (checked in a fresh interpreter)."""
    import importlib.util
    built = importlib.util.find_spec("cpu_attention._binding") is not None
    assert isinstance(K.module(), K.NativeModule) == built
    if built:
        assert K.module().decode is K.module().binding.decode
    code = ("import sys; sys.path.insert(0, %r); from cpu_attention import _kernel as K; "
            "print(type(K.module()).__name__)" % PKG)
    env = dict(os.environ, CPU_ATTENTION_BINDING="ctypes")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, check=True)
    assert out.stdout.strip() == "Module"


def test_native_binding_argument_errors():
    """Wrong argument counts and scales raise as the ctypes binding's would."""
    mod = K.module()
    if not isinstance(mod, K.NativeModule):
        pytest.skip("native binding not built")
    with pytest.raises(TypeError):
        mod.decode(None, 1, 2)
    with pytest.raises(TypeError):
        mod.flash(None)
    with pytest.raises(TypeError):
        mod.store()


def test_host_info():
    assert K.physical_cores() >= 1
    assert K.llc_bytes() >= 1 << 10
    assert K.workspace() == (0, 0)
    old = K.set_host_checks(False)
    assert K.host_checks() is False
    K.set_host_checks(old)
