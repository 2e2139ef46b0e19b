"""C-ABI workspace rules on the GPU: a decode workspace sized once for the largest
batch of a page table serves a smaller batch whose preferred tiles would need more
(the entry takes 256-key tiles instead), and ca_flash declines a workspace that is
not 16-byte aligned for a call that uses one, without touching the output; the
decode's in-kernel merge of small calls works from any workspace contents."""

import ctypes

import numpy as np

import pytest
import torch

from cpu_attention import _kernel as K
from helpers import assert_close, attention, reference, stage, values
from test_zz_no_alloc import args_for, stream

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_workspace_sized_for_the_largest_batch(cuda, dtype):
    """H=32, E=32, 16-token pages, a page table of 2048 keys: 8 sequences (256
    rows) prefer 256-key tiles and need no workspace; 7 sequences prefer 64-key
    tiles, whose partials need some.  Sized for the 8, the 7 run on 256-key tiles;
    41 sequences need a workspace again, and one sized for them serves 7 too."""
    lib = K.module().lib
    h, d, page, width = 32, 32, 16, 128
    assert lib.ca_decode_workspace_bytes(8, h, d, page, width) == 0
    assert lib.ca_decode_workspace_bytes(7, h, d, page, width) > 0
    need11 = lib.ca_decode_workspace_bytes(41, h, d, page, width)
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


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_merge_counters_in_any_workspace(cuda, dtype):
    """Calls of 64 to 512 rows of at most 4 blocks merge their split rows inside the
    decode kernel:
    each block counts itself in on a per-row counter in the workspace, tagged with
    the call, and the row's last block merges.  Whatever the workspace holds
    beforehand (zeros, all-ones bytes, random bytes, small integers, the previous
    call's counters), ten calls in a row give the same bits, within the oracle's
    gates; a second call shape on the same workspace (its slots and counters
    elsewhere) does too."""
    lib = K.module().lib
    h, d, page = 16, 128, 16
    lens = [2000, 17, 1500, 513, 1900, 64]  # 96 rows, 2016 keys of page table (4 blocks)
    print(f"decode merge counters dtype={dtype}", flush=True)
    q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed=31, device=cuda)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
    need = lib.ca_decode_workspace_bytes(len(lens), h, d, page, bt.shape[1])
    assert need > 0
    g = torch.Generator(device=cuda).manual_seed(5)
    small = (torch.arange(need // 4, dtype=torch.int32, device=cuda) % 1000 + 1).view(torch.uint8)
    fills = [torch.zeros(need, dtype=torch.uint8, device=cuda),
             torch.full((need,), 255, dtype=torch.uint8, device=cuda),
             torch.randint(0, 256, (need,), generator=g, dtype=torch.uint8, device=cuda),
             small]
    outs = []
    for ws in fills:
        for _ in range(10):
            out = torch.full_like(q, float("nan"))
            rc = lib.ca_decode(ctypes.byref(args_for(q, kc, vc, seqlens, bt, out, ws)), stream())
            assert rc == K.CA_OK, lib.ca_status_string(rc)
            outs.append(out)
    torch.cuda.synchronize()
    assert_close(outs[0], reference(q, ks, vs, d ** -0.5), dtype, paged=True)
    for o in outs[1:]:
        assert torch.equal(o.view(torch.uint8), outs[0].view(torch.uint8))
    lens2 = [1800, 700, 1100, 90]  # 64 rows, 4 blocks
    q2, kc2, vc2, bt2, ks2, vs2 = stage(lens2, h, d, page, dtype, seed=32, device=cuda)
    assert lib.ca_decode_workspace_bytes(len(lens2), h, d, page, bt2.shape[1]) <= need
    out2 = torch.full_like(q2, float("nan"))
    rc = lib.ca_decode(ctypes.byref(args_for(q2, kc2, vc2, torch.tensor(lens2, dtype=torch.int32, device=cuda), bt2,
                                             out2, fills[2])), stream())
    assert rc == K.CA_OK, lib.ca_status_string(rc)
    torch.cuda.synchronize()
    assert_close(out2, reference(q2, ks2, vs2, d ** -0.5), dtype, paged=True)


@pytest.mark.parametrize("nseq", [16, 17])
def test_decode_merge_row_limit(cuda, nseq):
    """H=32: 16 sequences (512 rows) merge inside the decode kernel, 17 (544 rows)
    go through the combine kernel; both match the oracle."""
    lib = K.module().lib
    h, d, page, dtype = 32, 64, 16, torch.bfloat16
    rng = np.random.default_rng(nseq)
    lens = rng.integers(17, 2000, size=nseq).tolist()  # page tables of at most 4 blocks
    print(f"decode merge row limit nseq={nseq}", flush=True)
    q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed=nseq, device=cuda)
    ws = torch.empty(lib.ca_decode_workspace_bytes(nseq, h, d, page, bt.shape[1]), dtype=torch.uint8, device=cuda)
    out = torch.full_like(q, float("nan"))
    rc = lib.ca_decode(ctypes.byref(args_for(q, kc, vc, torch.tensor(lens, dtype=torch.int32, device=cuda), bt, out,
                                             ws)), stream())
    assert rc == K.CA_OK, lib.ca_status_string(rc)
    torch.cuda.synchronize()
    assert_close(out, reference(q, ks, vs, d ** -0.5), dtype, paged=True)


@pytest.mark.parametrize("nseq,h,longest,merges", [(2, 32, 2000, True), (2, 32, 2100, False), (1, 32, 2000, False),
                                                    (1, 8, 30000, False)])
def test_decode_merge_block_limit(cuda, nseq, h, longest, merges):
    """The in-kernel merge takes calls of 64 to 512 rows whose page table holds at
    most 4 blocks (2048 keys of 64-key tiles); more blocks or fewer rows go through
    the combine kernel (many blocks of a row counting in at once serialise).  The
    workspace size shows the route (one 8-byte counter per row); both routes match
    the oracle."""
    lib = K.module().lib
    d, page, dtype = 64, 16, torch.bfloat16
    lens = [longest] + [longest // 3] * (nseq - 1)
    print(f"decode merge block limit nseq={nseq} h={h} longest={longest}", flush=True)
    q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed=41, device=cuda)
    need = lib.ca_decode_workspace_bytes(nseq, h, d, page, bt.shape[1])
    rows, blocks = nseq * h, -(-bt.shape[1] * page // 512)
    acc = (rows * blocks * d * 4 + 255) // 256 * 256 + rows * blocks * 8
    assert need == acc + (rows * 8 if merges else 0)
    ws = torch.empty(need, dtype=torch.uint8, device=cuda)
    out = torch.full_like(q, float("nan"))
    rc = lib.ca_decode(ctypes.byref(args_for(q, kc, vc, torch.tensor(lens, dtype=torch.int32, device=cuda), bt, out,
                                             ws)), stream())
    assert rc == K.CA_OK, lib.ca_status_string(rc)
    torch.cuda.synchronize()
    assert_close(out, reference(q, ks, vs, d ** -0.5), dtype, paged=True)
