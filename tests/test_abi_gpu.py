"""C-ABI workspace rules on the GPU: a decode workspace sized once for the largest
batch of a page table serves a smaller batch whose preferred tiles would need more
(the entry takes 256-key tiles instead), and ca_flash declines a workspace that is
not 16-byte aligned for a call that uses one, without touching the output."""

import ctypes

import pytest
import torch

from cpu_attention import _kernel as K
from helpers import assert_close, attention, reference, stage, values
from test_zz_no_alloc import args_for, stream

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_workspace_sized_for_the_largest_batch(cuda, dtype):
    """H=32, E=128, 16-token pages, a page table of 2048 keys: 8 sequences (256
    rows) prefer 256-key tiles and need no workspace; 7 sequences prefer 64-key
    tiles, whose partials need some.  Sized for the 8, the 7 run on 256-key tiles;
    11 sequences need a workspace again, and one sized for them serves 7 too."""
    lib = K.module().lib
    h, d, page, width = 32, 128, 16, 128
    assert lib.ca_decode_workspace_bytes(8, h, d, page, width) == 0
    assert lib.ca_decode_workspace_bytes(7, h, d, page, width) > 0
    need11 = lib.ca_decode_workspace_bytes(11, h, d, page, width)
    assert need11 > lib.ca_decode_workspace_bytes(7, h, d, page, width)
    lens = [2030, 17, 1500, 512, 513, 2000, 64]
    print(f"decode workspace sizing dtype={dtype}", flush=True)
    q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed=21, device=cuda)
    table = torch.cat([bt, bt[:, -1:].expand(-1, width - bt.shape[1])], dim=1).contiguous()
    seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
    ref = reference(q, ks, vs, d ** -0.5)
    for ws in (None, torch.empty(need11, dtype=torch.uint8, device=cuda)):
        out = torch.full_like(q, float("nan"))
        rc = lib.ca_decode(ctypes.byref(args_for(q, kc, vc, seqlens, table, out, ws)), stream())
        assert rc == K.CA_OK, lib.ca_status_string(rc)
        torch.cuda.synchronize()
        assert_close(out, ref, dtype, paged=True)


def flash_args(q, k, v, out, ws, nbytes, causal):
    a = K.FlashArgs()
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.batch, a.seq_q, a.seq_k, a.num_heads, a.head_dim = q.shape[0], q.shape[1], k.shape[1], q.shape[2], q.shape[3]
    for name, t in (("q_strides", q), ("k_strides", k), ("v_strides", v)):
        arr = getattr(a, name)
        arr[0], arr[1], arr[2] = t.stride(0), t.stride(1), t.stride(2)
    a.scale, a.causal, a.dtype = q.shape[3] ** -0.5, int(causal), K.DTYPES[q.dtype]
    a.workspace, a.workspace_bytes = ws, nbytes
    return a


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("sq", [3, 64])
def test_flash_declines_a_misaligned_workspace(cuda, dtype, sq):
    """Calls whose keys are split over blocks (3 rows: the few-rows route; 64 rows
    over 4096 keys: the tiled kernel's split mode) write their partials with 16-byte
    stores: a workspace 4 bytes off alignment is declined and the output keeps its
    poison; the aligned one gives the oracle's result."""
    lib = K.module().lib
    b, sk, h, d = 1, 4096, 8, 128
    need = lib.ca_flash_workspace_bytes(b, sq, sk, h, d, K.DTYPES[dtype])
    assert need > 0
    g = torch.Generator().manual_seed(sq)
    q, k, v = (torch.randn(b, n, h, d, generator=g).to(dtype).to(cuda) for n in (sq, sk, sk))
    buf = torch.empty(need + 256, dtype=torch.uint8, device=cuda)
    base = buf.data_ptr()
    print(f"flash misaligned workspace dtype={dtype} sq={sq}", flush=True)
    out = torch.full_like(q, float("nan"))
    rc = lib.ca_flash(ctypes.byref(flash_args(q, k, v, out, base + 4, need, False)), stream())
    assert rc == K.CA_DECLINED
    torch.cuda.synchronize()
    assert bool(torch.isnan(out).all())
    rc = lib.ca_flash(ctypes.byref(flash_args(q, k, v, out, base, need, False)), stream())
    assert rc == K.CA_OK, lib.ca_status_string(rc)
    torch.cuda.synchronize()
    assert_close(out, attention(values(q), values(k), values(v), d ** -0.5, False), dtype, paged=False)
