"""The C ABI library: it loads, exports every entry include/*.h declares, its ctypes
structures match the C header byte for byte, and it declines malformed calls
without touching a GPU (CPU only)."""

import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from cpu_attention import _kernel as K

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cpu_attention_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*[\w\s\*]+?\b(ca_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_entry():
    names = declared_functions()
    assert {"ca_store", "ca_decode", "ca_flash", "ca_version"} <= set(names)
    lib = ctypes.CDLL(K.library_path())
    for name in names:
        assert hasattr(lib, name), name
    assert set(K.EXPORTS) == set(names)


def test_version_and_status_strings():
    lib = K.load_library()
    assert lib.ca_abi_version() == K.ABI_VERSION == 3
    assert b"gfx950" in lib.ca_version()
    assert lib.ca_status_string(0) == b"ok"
    assert b"declined" in lib.ca_status_string(1)
    assert b"32 MiB" in lib.ca_status_string(K.CA_SCRATCH_EXCEEDED)
    assert lib.ca_status_string(-1 - 1)  # a HIP error code renders as text


_LAYOUT_C = r"""
#include <stddef.h>
#include <stdio.h>
#include "cpu_attention_hip.h"
#define F(T, f) printf("%s.%s %zu %zu\n", #T, #f, offsetof(T, f), sizeof(((T*)0)->f));
int main(void) {
  printf("ca_store_args %zu\n", sizeof(ca_store_args));
  printf("ca_decode_args %zu\n", sizeof(ca_decode_args));
  printf("ca_flash_args %zu\n", sizeof(ca_flash_args));
  FIELDS
  return 0;
}
"""


def test_ctypes_structures_match_the_header():
    structs = {"ca_store_args": K.StoreArgs, "ca_decode_args": K.DecodeArgs,
               "ca_flash_args": K.FlashArgs}
    fields = "\n".join(f"F({c}, {name})" for c, py in structs.items() for name, _ in py._fields_)
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "layout.c"), os.path.join(d, "layout")
        open(src, "w").write(_LAYOUT_C.replace("FIELDS", fields))
        subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), src, "-o", exe],
                       check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    for line in filter(None, out):
        parts = line.split()
        if len(parts) == 2:
            assert ctypes.sizeof(structs[parts[0]]) == int(parts[1]), line
        else:
            cname, field = parts[0].split(".")
            desc = getattr(structs[cname], field)
            assert (desc.offset, desc.size) == (int(parts[1]), int(parts[2])), line


def test_entries_decline_malformed_calls_without_a_gpu():
    lib = K.load_library()
    s = K.StoreArgs(num_tokens=4, num_heads=2, head_dim=48, page_size=16, dtype=0)
    assert lib.ca_store(ctypes.byref(s), None) == K.CA_DECLINED  # head_dim
    s.head_dim, s.page_size = 64, 24
    assert lib.ca_store(ctypes.byref(s), None) == K.CA_DECLINED  # page
    s.page_size = 16
    assert lib.ca_store(ctypes.byref(s), None) == K.CA_DECLINED  # null pointers
    s.num_tokens = 0
    assert lib.ca_store(ctypes.byref(s), None) == K.CA_OK  # nothing to do
    d = K.DecodeArgs(num_seqs=2, num_heads=2, head_dim=64, page_size=16, dtype=3)
    assert lib.ca_decode(ctypes.byref(d), None) == K.CA_DECLINED  # dtype
    d.dtype = 1
    assert lib.ca_decode(ctypes.byref(d), None) == K.CA_DECLINED  # null pointers
    # the no-allocation decode: a call whose split-K scratch exceeds the fixed buffer
    # even with 256-key tiles (32 blocks of 2048 keys per row, 2048 rows: 34 MB of
    # partials) is refused before anything is enqueued (no GPU needed to see it);
    # one 233 pages narrower fits with 256-key tiles, so it gets as far as the
    # pointer checks, although its usual 64-key tiles would need 126 MB
    d.dtype, d.page_table_width = 1, 4033
    d.num_seqs, d.num_heads, d.head_dim = 64, 32, 128
    assert lib.ca_decode_workspace_bytes(64, 32, 128, 16, 4033) > 32 << 20
    assert lib.ca_decode_noalloc(ctypes.byref(d), None) == K.CA_SCRATCH_EXCEEDED
    d.page_table_width = 3800
    assert lib.ca_decode_workspace_bytes(64, 32, 128, 16, 3800) > 32 << 20
    assert lib.ca_decode_noalloc(ctypes.byref(d), None) == K.CA_DECLINED  # null pointers
    assert lib.ca_decode_noalloc(None, None) == K.CA_DECLINED
    f = K.FlashArgs(batch=1, seq_q=0, seq_k=4, num_heads=1, head_dim=64, dtype=1)
    assert lib.ca_flash(ctypes.byref(f), None) == K.CA_DECLINED  # seq_q < 1
    f.seq_q = 4
    assert lib.ca_flash(ctypes.byref(f), None) == K.CA_DECLINED  # null pointers
    # decode: one (max, sum, P.V) partial per (row, block of 8 tiles), none when a row
    # fits one block.  Tiles are 64 keys (512 per block) unless the page table holds
    # more than 512 keys and every row fits one block of 256-key tiles (2048 keys),
    # there are 256 rows or more, K holds at most 80 Mi elements at the page table's
    # capacity, and a row is narrow (E * esize at most 128 bytes).  The query answers
    # for the larger of the bf16 and the fp32 call.
    def partials(rows, blocks, d, merges=None):
        # accumulators (256-byte aligned), (max, sum) pairs, and for calls of 64 to
        # 512 rows of at most 4 blocks one 8-byte merge counter per row
        if merges is None:
            merges = 64 <= rows <= 512 and blocks <= 4
        return ((rows * blocks * d * 4 + 255) // 256) * 256 + rows * blocks * 2 * 4 + (rows * 8 if merges else 0)
    assert lib.ca_decode_workspace_bytes(8, 32, 32, 32, 64) == 0          # 256-key tiles in either dtype
    assert lib.ca_decode_workspace_bytes(8, 32, 64, 32, 64) == partials(256, 4, 64)  # fp32 E=64: 64-key tiles
    assert lib.ca_decode_workspace_bytes(64, 32, 128, 32, 64) == partials(2048, 4, 128)
    assert lib.ca_decode_workspace_bytes(4, 32, 32, 32, 64) == partials(128, 4, 32)  # < 256 rows
    assert lib.ca_decode_workspace_bytes(8, 32, 32, 32, 65) == partials(256, 5, 32)  # > 2048 keys
    assert lib.ca_decode_workspace_bytes(1, 32, 128, 16, 32) == 0          # 512 keys: one block
    assert lib.ca_decode_workspace_bytes(128, 8, 32, 16, 32) == 0          # 512 keys, 1024 rows: one block
    assert lib.ca_decode_workspace_bytes(8, 32, 128, 16, 128) == partials(256, 4, 128)  # wide rows
    # the in-kernel merge's counters: 64 to 512 rows of at most 4 blocks
    assert lib.ca_decode_workspace_bytes(2, 32, 64, 16, 128) == partials(64, 4, 64)
    assert partials(64, 4, 64) == partials(64, 4, 64, merges=False) + 64 * 8
    assert lib.ca_decode_workspace_bytes(1, 32, 64, 16, 128) == partials(32, 4, 64, merges=False)  # 32 rows
    assert lib.ca_decode_workspace_bytes(2, 32, 64, 16, 129) == partials(64, 5, 64, merges=False)  # 5 blocks
    assert lib.ca_decode_workspace_bytes(1, 8, 128, 16, 2048) == partials(8, 64, 128, merges=False)
    # not monotonic in the batch: 8 sequences of H=32 E=32 over 2048 keys prefer
    # 256-key tiles (no partials), 7 prefer 64-key tiles (ca_decode then takes 256-key
    # tiles when its workspace holds only theirs), 41 exceed 80 Mi K elements
    assert lib.ca_decode_workspace_bytes(8, 32, 32, 16, 128) == 0
    assert lib.ca_decode_workspace_bytes(7, 32, 32, 16, 128) == partials(224, 4, 32)
    assert lib.ca_decode_workspace_bytes(41, 32, 32, 16, 128) == partials(1312, 4, 32)
    assert lib.ca_flash_workspace_bytes(1, 1, 1, 1, 64, 1) == 0


@pytest.mark.parametrize("dtype,d,chunk", [(1, 32, 64), (1, 64, 32), (1, 128, 16),
                                           (0, 32, 32), (0, 64, 16), (0, 128, 8)])
def test_flash_workspace_for_few_rows(dtype, d, chunk):
    """Few query rows (up to 4 in bf16; in fp32 up to 8, or 16 when batch x heads
    is 256 or more) go to blocks of 8 waves per
    (batch, head, row group: 1 row for single-row calls, else 4); chunks of 4 load
    steps (16-byte slices, 64 lanes).  Only when those blocks number fewer than 256
    are a row group's chunks split over more blocks (at most one chunk per wave and
    64 splits).  Single-row calls whose head count is a multiple of the heads one
    load instruction reads (64 lanes / (E * esize / 16)) may instead take blocks of
    one (batch, group of those heads), split the same way over chunks of 4 keys;
    the strides choose, so the query answers for the larger.  A split call needs
    (E + 2) floats per (batch, head, row, split); otherwise no workspace."""
    lib = K.load_library()

    def split(blocks, chunks):
        s = 1 if blocks >= 256 else -(-256 // blocks)
        return max(1, min(s, -(-chunks // 8), 64))

    def expect(b, sq, sk, h):
        if sq > (4 if dtype == 1 else 16 if b * h >= 256 else 8):
            return tiled(b, sq, sk, h, d, dtype)
        splits = split(b * h * -(-sq // (1 if sq == 1 else 4)), -(-sk // chunk))
        hp = 64 // (d * (2 if dtype == 1 else 4) // 16)
        if sq == 1 and h % hp == 0:
            splits = max(splits, split(b * h // hp, -(-sk // 4)))
        rows = b * h * sq
        return 0 if splits == 1 else rows * splits * (d + 2) * 4

    for b, sq, sk, h in ((1, 1, 100000, 1), (2, 16, 1000, 3), (3, 4, chunk + 1, 5), (8, 1, 2048, 32),
                         (8, 1, 2048, 33), (64, 1, 512, 32), (1, 3, 70000, 2)):
        assert lib.ca_flash_workspace_bytes(b, sq, sk, h, d, dtype) == expect(b, sq, sk, h)
    assert lib.ca_flash_workspace_bytes(1, 1, 100000, 1, d, dtype) == 64 * (d + 2) * 4
    assert lib.ca_flash_workspace_bytes(8, 1, 2048, 33, d, dtype) == 0  # 264 blocks fill the chip
    # 32 heads: the packed-heads blocks (8 x 32 / hp of them) split 2048 keys
    hp = 64 // (d * (2 if dtype == 1 else 4) // 16)
    s = min(-(-256 // (8 * 32 // hp)), 64)
    assert lib.ca_flash_workspace_bytes(8, 1, 2048, 32, d, dtype) == 256 * s * (d + 2) * 4
    assert lib.ca_flash_workspace_bytes(3, 4, 8 * chunk, 5, d, dtype) == 0  # one chunk per wave
    assert lib.ca_flash_workspace_bytes(3, 17, 5000, 5, d, dtype) == tiled(3, 17, 5000, 5, d, dtype)
    assert lib.ca_flash_workspace_bytes(1, 5, 50000, 1, d, dtype) > 0  # bf16: tiled split; fp32: few rows
    assert lib.ca_flash_workspace_bytes(3, 4, 5000, 5, 48, dtype) == 0  # head_dim


def tiled(b, sq, sk, h, d, dtype):
    """The tiled prefill's split mode: when its query blocks (b * h * ceil(sq /
    rows per block): 256 in bf16, 128 in fp32) number fewer than a target (256 in
    bf16, 512 in fp32), each one's keys are split over target / blocks blocks
    (rounded down in bf16: one round of the chip; up in fp32), at least 256 keys
    each (whole 64-key units) and at most 64 splits, which needs (E + 2) floats
    per (batch, head, row, split).  bf16 calls with fewer than twice as many keys
    as rows do not split from 128 query blocks under 4096 keys, nor from 64 under
    2048 keys, nor, if causal or from 16 query blocks, under 1024 keys.  The query answers for the larger
    of the causal and non-causal call."""
    blocks = b * h * -(-sq // (256 if dtype == 1 else 128))
    target = 256 if dtype == 1 else 512

    def splits(causal):
        if blocks >= target:
            return 1
        if dtype == 1 and sk < 2 * sq and ((blocks >= 128 and sk < 4096) or (blocks >= 64 and sk < 2048) or
                                           (sk < 1024 and (causal or blocks >= 16))):
            return 1
        per = target // blocks if dtype == 1 else -(-target // blocks)
        return min(per, -(-sk // 64) // 4, 64)

    s = max(splits(False), splits(True))
    return 0 if s < 2 else b * h * sq * s * (d + 2) * 4


@pytest.mark.parametrize("d", [32, 64, 128])
def test_flash_workspace_for_split_keys(d):
    lib = K.load_library()
    for b, sq, sk, h in ((1, 64, 4096, 32), (1, 17, 2100, 8), (2, 300, 1500, 4), (4, 4096, 4096, 32),
                         (1, 128, 128, 16), (1, 600, 255, 3), (1, 5, 100000, 1), (1, 100, 4096, 300),
                         (1, 4096, 4096, 4), (1, 2048, 2048, 12), (1, 1024, 1024, 8), (1, 512, 512, 16),
                         (1, 1500, 1500, 20), (1, 4096, 4096, 8), (1, 4096, 4096, 12), (1, 3000, 3000, 16)):
        assert lib.ca_flash_workspace_bytes(b, sq, sk, h, d, 1) == tiled(b, sq, sk, h, d, 1)
        if sq > 16:  # fp32 past the few-rows route
            assert lib.ca_flash_workspace_bytes(b, sq, sk, h, d, 0) == tiled(b, sq, sk, h, d, 0)
    assert lib.ca_flash_workspace_bytes(1, 64, 4096, 32, d, 1) == 32 * 64 * 8 * (d + 2) * 4  # 8 splits
    assert lib.ca_flash_workspace_bytes(1, 64, 4096, 32, d, 0) == 32 * 64 * 16 * (d + 2) * 4  # 16 splits
    for dtype in (0, 1):
        assert lib.ca_flash_workspace_bytes(4, 4096, 4096, 32, d, dtype) == 0  # cfg4: >= 2048 query blocks
        assert lib.ca_flash_workspace_bytes(1, 128, 128, 16, d, dtype) == 0  # cfg1: 128 keys
    # 300 query blocks fill the chip in bf16 (one block per CU) but not in fp32 (two
    # per CU): 2 splits
    assert lib.ca_flash_workspace_bytes(1, 100, 4096, 300, d, 1) == 0
    assert lib.ca_flash_workspace_bytes(1, 100, 4096, 300, d, 0) == 100 * 300 * 2 * (d + 2) * 4
    # 120 query blocks: 2 splits in bf16 (256 / 120 rounded down), 5 in fp32 (512 / 120 up)
    assert lib.ca_flash_workspace_bytes(1, 100, 4096, 120, d, 1) == 100 * 120 * 2 * (d + 2) * 4
    assert lib.ca_flash_workspace_bytes(1, 100, 4096, 120, d, 0) == 100 * 120 * 5 * (d + 2) * 4
    # bf16, keys under twice the rows: 64 query blocks or more do not split, fewer do
    assert lib.ca_flash_workspace_bytes(1, 1024, 1024, 16, d, 1) == 0
    assert lib.ca_flash_workspace_bytes(2, 700, 1200, 8, d, 1) == 2 * 8 * 700 * 4 * (d + 2) * 4
    # ... except 64 to 127 query blocks over 2048 keys or more: L=S=4096 H=4 (64
    # query blocks) 4 splits
    assert lib.ca_flash_workspace_bytes(1, 4096, 4096, 4, d, 1) == 4 * 4096 * 4 * (d + 2) * 4
    assert lib.ca_flash_workspace_bytes(1, 1500, 1500, 20, d, 1) == 0  # 120 query blocks under 2048 keys
    # 128 query blocks over 4096 keys: 2 splits (more than 128 round down to 1)
    assert lib.ca_flash_workspace_bytes(1, 4096, 4096, 8, d, 1) == 8 * 4096 * 2 * (d + 2) * 4
    assert lib.ca_flash_workspace_bytes(1, 4096, 4096, 12, d, 1) == 0
    # under 1024 keys: no split from 16 query blocks, causal or not
    assert lib.ca_flash_workspace_bytes(2, 600, 600, 8, d, 1) == 0
    assert lib.ca_flash_workspace_bytes(1, 768, 768, 4, d, 1) > 0  # 12 blocks split


def test_missing_library_is_a_loud_error(monkeypatch):
    monkeypatch.setenv("CPU_ATTENTION_LIB", "/nonexistent/libcpu_attention_hip.so")
    monkeypatch.setattr(K, "_MODULE", None)
    with pytest.raises(RuntimeError, match="not built"):
        K.module()
