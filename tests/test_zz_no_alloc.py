"""ca_decode_noalloc (the decode entry that allocates nothing; its split-K scratch
is a fixed per-GPU buffer inside the library) against ca_decode with a caller
workspace, through the C ABI: two calls in a row, the second with a smaller
batch and page table, each bit-equal to ca_decode's output and within the
decode gates of the float64 oracle; a call whose usual tile size needs more
scratch than the buffer holds, on 256-key tiles; calls on two streams without a
host synchronisation, ordered by the entry; a call past the buffer's size even
then is refused without touching the output."""

import ctypes

import numpy as np
import pytest
import torch

from cpu_attention import _kernel as K
from helpers import assert_close, reference, stage

pytestmark = pytest.mark.gpu


def args_for(q, kc, vc, lens, table, out, ws=None):
    b, h, d = q.shape[0], q.shape[2], q.shape[3]
    return K.DecodeArgs(
        q=q.data_ptr(), q_stride=q.stride(0), k_cache=kc.data_ptr(), v_cache=vc.data_ptr(),
        k_new=None, v_new=None, kv_stride=0, slots=None, lens=lens.data_ptr(),
        page_table=table.data_ptr(), page_table_width=table.shape[1], out=out.data_ptr(),
        num_seqs=b, num_heads=h, head_dim=d, page_size=kc.shape[2], num_blocks=kc.shape[0],
        scale=d ** -0.5, dtype=K.DTYPES[q.dtype],
        workspace=ws.data_ptr() if ws is not None else None,
        workspace_bytes=ws.numel() if ws is not None else 0, new_tokens=0)


def stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_matches_decode_on_two_calls(cuda, dtype):
    lib = K.module().lib
    h, d, page = 4, 128, 16
    # First call: rows up to 5000 keys (three blocks of 2048 keys, so the split-K
    # scratch and the combine kernel are in use); second: fewer rows and a
    # narrower page table, still past one block.
    for lens, seed in (([5000, 2100, 100, 4095], 1), ([3000, 17], 2)):
        print(f"noalloc dtype={dtype} lens={lens}", flush=True)
        q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed=seed, device=cuda)
        seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
        need = lib.ca_decode_workspace_bytes(len(lens), h, d, page, bt.shape[1])
        assert 0 < need <= 32 << 20
        ws = torch.empty(need, dtype=torch.uint8, device=cuda)
        ref_out = torch.empty_like(q)
        rc = lib.ca_decode(ctypes.byref(args_for(q, kc, vc, seqlens, bt, ref_out, ws)), stream())
        assert rc == K.CA_OK, lib.ca_status_string(rc)
        out = torch.full_like(q, float("nan"))
        rc = lib.ca_decode_noalloc(ctypes.byref(args_for(q, kc, vc, seqlens, bt, out)), stream())
        assert rc == K.CA_OK, lib.ca_status_string(rc)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.uint8), ref_out.view(torch.uint8))
        assert_close(out, reference(q, ks, vs, d ** -0.5), dtype, paged=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_takes_long_tiles_when_short_ones_do_not_fit(cuda, dtype):
    """A batch whose 64-key-tile partials need more than the 32 MiB buffer (1024
    rows, a page table of 40,960 keys) runs with 256-key tiles, whose partials fit,
    and matches the float64 oracle; rows past 2048 keys use the combine kernel."""
    lib = K.module().lib
    h, d, page, width = 32, 128, 16, 2560
    rng = np.random.default_rng(5)
    lens = [2047, 2048, 2049, 5000] + rng.integers(17, 300, size=28).tolist()
    print(f"noalloc long tiles dtype={dtype}", flush=True)
    assert lib.ca_decode_workspace_bytes(len(lens), h, d, page, width) > 32 << 20
    q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed=5, device=cuda)
    # widen the page table to `width`: the entries past each row's pages name the
    # helper's poisoned padding block, which the kernel never reads
    table = torch.cat([bt, bt[:, -1:].expand(-1, width - bt.shape[1])], dim=1).contiguous()
    seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
    out = torch.full_like(q, float("nan"))
    rc = lib.ca_decode_noalloc(ctypes.byref(args_for(q, kc, vc, seqlens, table, out)), stream())
    assert rc == K.CA_OK, lib.ca_status_string(rc)
    torch.cuda.synchronize()
    assert_close(out, reference(q, ks, vs, d ** -0.5), dtype, paged=True)


def test_noalloc_calls_on_two_streams_run_in_turn(cuda):
    """Calls that use the one scratch buffer, issued on two streams with no host
    synchronisation between them (two batches whose rows span several blocks,
    alternating), each give ca_decode's output: the entry makes every such call
    wait for the previous one's kernels, whichever stream it ran on."""
    lib = K.module().lib
    h, d, page = 8, 128, 16
    dtype = torch.bfloat16
    jobs = []
    for lens, seed in (([5000, 2100, 4095, 3000, 2500, 4000], 7), ([3000, 2300, 1700], 8)):
        q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed=seed, device=cuda)
        seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
        ws = torch.empty(lib.ca_decode_workspace_bytes(len(lens), h, d, page, bt.shape[1]),
                         dtype=torch.uint8, device=cuda)
        ref_out = torch.empty_like(q)
        rc = lib.ca_decode(ctypes.byref(args_for(q, kc, vc, seqlens, bt, ref_out, ws)), stream())
        assert rc == K.CA_OK, lib.ca_status_string(rc)
        jobs.append((q, kc, vc, seqlens, bt, ref_out))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = []
    print("noalloc on two streams", flush=True)
    for i in range(6):
        j = i % 2
        q, kc, vc, seqlens, bt, _ = jobs[j]
        out = torch.full_like(q, float("nan"))
        rc = lib.ca_decode_noalloc(ctypes.byref(args_for(q, kc, vc, seqlens, bt, out)), streams[j].cuda_stream)
        assert rc == K.CA_OK, lib.ca_status_string(rc)
        outs.append((j, out))
    torch.cuda.synchronize()
    for j, out in outs:
        assert torch.equal(out.view(torch.uint8), jobs[j][5].view(torch.uint8))


def test_noalloc_refuses_past_its_buffer(cuda):
    lib = K.module().lib
    n, h, d, page, width = 64, 32, 128, 16, 4033
    assert lib.ca_decode_workspace_bytes(n, h, d, page, width) > 32 << 20
    q = torch.randn(n, 1, h, d, device=cuda).bfloat16()
    kc = torch.zeros(2, h, page, d, device=cuda, dtype=torch.bfloat16)
    table = torch.zeros(n, width, dtype=torch.int32, device=cuda)
    lens = torch.ones(n, dtype=torch.int32, device=cuda)
    out = torch.full_like(q, 7.0)
    rc = lib.ca_decode_noalloc(ctypes.byref(args_for(q, kc, kc, lens, table, out)), stream())
    assert rc == K.CA_SCRATCH_EXCEEDED
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
