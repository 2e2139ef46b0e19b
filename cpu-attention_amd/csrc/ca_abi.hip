// The extern "C" entries declared in include/cpu_attention_hip.h.  Each one checks
// what its kernels assume (the static half of the reference's native validation,
// cpu_attention/_mojo/src/_C.mojo:104-160, 190-205, 249-267, plus the 16-byte
// alignment the vector loads need) and returns CA_DECLINED without launching
// anything otherwise.
#include <stdio.h>

#include <atomic>

#include "ca_device.h"
#include "ca_internal.h"

using namespace ca;

namespace {

bool head_dim_ok(int64_t e) { return e == 32 || e == 64 || e == 128; }
bool dtype_ok(int32_t dt) { return dt == CA_F32 || dt == CA_BF16; }
int64_t esize(int32_t dt) { return dt == CA_BF16 ? 2 : 4; }
bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }
// An element stride whose byte size keeps 16-byte alignment.
bool stride16(int64_t stride, int32_t dt) { return (stride * esize(dt)) % 16 == 0; }
bool page_ok(int64_t page) { return page > 0 && page % 16 == 0; }

}  // namespace

extern "C" int ca_abi_version(void) { return CA_ABI_VERSION; }

extern "C" const char* ca_version(void) {
  return "cpu-attention gfx950 (MI355X) HIP kernels, ABI " "3";
}

extern "C" const char* ca_status_string(int status) {
  if (status == CA_OK) return "ok";
  if (status == CA_DECLINED) return "declined: arguments outside what the kernels take";
  if (status == CA_SCRATCH_EXCEEDED)
    return "ca_decode_noalloc: the call needs more split-K scratch than the fixed 32 MiB buffer "
           "(a page table of this capacity needs ca_decode with a caller workspace)";
  if (status < 0) return hipGetErrorString((hipError_t)(CA_HIP_ERROR - status));
  return "unknown status";
}

extern "C" int ca_store(const ca_store_args* a, void* stream) {
  if (!a || !dtype_ok(a->dtype) || !head_dim_ok(a->head_dim) || !page_ok(a->page_size))
    return CA_DECLINED;
  if (a->num_tokens < 0 || a->num_heads <= 0 || a->num_blocks < 0) return CA_DECLINED;
  if (a->num_tokens == 0) return CA_OK;
  if (!a->key || !a->value || !a->k_cache || !a->v_cache || !a->slot_mapping) return CA_DECLINED;
  if (!aligned16(a->key) || !aligned16(a->value) || !aligned16(a->k_cache) || !aligned16(a->v_cache))
    return CA_DECLINED;
  // One token is never stepped over, so its stride is not read (a [1, H, E]
  // view may carry any stride there, 0 included).
  const bool one = a->num_tokens == 1;
  if (!one && (!stride16(a->token_stride, a->dtype) || a->token_stride < a->num_heads * a->head_dim))
    return CA_DECLINED;
  const int64_t words = a->head_dim * esize(a->dtype) / 4;
  StoreParams p{};
  p.key = static_cast<const uint32_t*>(a->key);
  p.value = static_cast<const uint32_t*>(a->value);
  p.tok_stride_w = one ? 0 : a->token_stride * esize(a->dtype) / 4;
  p.kc = static_cast<uint32_t*>(a->k_cache);
  p.vc = static_cast<uint32_t*>(a->v_cache);
  p.slots = a->slot_mapping;
  p.ntok = a->num_tokens;
  p.per_seq = 1;
  p.heads = a->num_heads;
  p.page = a->page_size;
  p.nblocks = a->num_blocks;
  return store_launch(p, (int)words, static_cast<hipStream_t>(stream));
}

// Workspace layout: fp32 partial accumulators [slots, E], then (max, sum) pairs
// [slots, 2], one slot per (row, block of 8 tiles of the page table's capacity);
// for calls of kMergeMinRows to kMergeMaxRows rows of at most kMergeMaxBlocks
// blocks, then one 8-byte counter per row (the in-kernel merge).
static int64_t decode_acc_bytes(int64_t slots, int64_t head_dim) {
  return ((slots * head_dim * 4 + 255) / 256) * 256;
}

// slots = rows x blocks per row (0: every row fits one block).
static bool decode_merges(int64_t rows, int64_t slots) {
  return slots > 0 && rows >= kMergeMinRows && rows <= kMergeMaxRows && slots <= rows * kMergeMaxBlocks;
}

static int64_t decode_ws_bytes(int64_t rows, int64_t head_dim, int64_t page, int64_t width, int tile_keys) {
  const int64_t slots = decode_workspace_slots(rows, decode_tiles(width, page, tile_keys));
  return decode_acc_bytes(slots, head_dim) + slots * 2 * 4 + (decode_merges(rows, slots) ? rows * 8 : 0);
}

// The in-kernel merge's per-call tag: n * 0x9E3779B9 for the process's n-th call
// (an odd multiplier, so no tag repeats within 2^32 calls), skipping values
// within 2^24 of zero: never 0 (the value a counter holds between calls), nor the
// small integers of either sign that a reused workspace tends to hold in a
// counter's high word.
static uint32_t next_merge_tag() {
  static std::atomic<uint32_t> n{0};
  constexpr uint32_t kNear = 1u << 24;
  uint32_t t = 0;
  while (t < kNear || t > ~kNear) t = ++n * 0x9E3779B9u;
  return t;
}

extern "C" int64_t ca_decode_workspace_bytes(int64_t num_seqs, int64_t num_heads,
                                             int64_t head_dim, int64_t page_size,
                                             int64_t page_table_width) {
  if (num_seqs < 0 || num_heads < 0 || page_size <= 0 || page_table_width < 0) return -1;
  // The tile size depends on the element size, which the query does not name: it
  // answers for the larger of the bf16 and the fp32 call.
  const int64_t rows = num_seqs * num_heads;
  int64_t most = 0;
  for (int esize : {2, 4}) {
    const int64_t b = decode_ws_bytes(rows, head_dim, page_size, page_table_width,
                                      decode_tile_keys(rows, page_table_width, page_size, head_dim, esize));
    most = b > most ? b : most;
  }
  return most;
}

// ca_decode and ca_decode_noalloc.  The split-K scratch is the caller's workspace,
// or for noalloc the library's fixed buffer.  A call whose partials with the
// preferred tile size do not fit the scratch it has takes 256-key tiles (fewer
// partials per row) if those fit.  With one tile size the need grows with the
// rows, so a workspace sized by ca_decode_workspace_bytes for the largest batch
// holds every smaller batch of the same page table, whichever tile size the
// smaller batch would prefer.
static int decode_entry(const ca_decode_args* a, void* stream, bool noalloc) {
  if (!a || !dtype_ok(a->dtype) || !head_dim_ok(a->head_dim) || !page_ok(a->page_size))
    return CA_DECLINED;
  if (a->num_seqs < 0 || a->num_heads <= 0 || a->num_blocks < 0 || a->page_table_width < 0)
    return CA_DECLINED;
  if (a->num_seqs == 0) return CA_OK;
  // The tile size and the split-K scratch it needs depend on the shapes only; the
  // no-allocation entry refuses a call its buffer cannot hold before anything else.
  const int64_t rows = a->num_seqs * a->num_heads;
  const int64_t have = noalloc ? CA_DECODE_NOALLOC_SCRATCH_BYTES
                               : (a->workspace && aligned16(a->workspace) && a->workspace_bytes > 0
                                      ? a->workspace_bytes : 0);
  int tile_keys = decode_tile_keys(rows, a->page_table_width, a->page_size, a->head_dim, a->dtype == CA_BF16 ? 2 : 4);
  int64_t need = decode_ws_bytes(rows, a->head_dim, a->page_size, a->page_table_width, tile_keys);
  if (need > have && tile_keys != kDecodeLongTile) {
    const int64_t need_long = decode_ws_bytes(rows, a->head_dim, a->page_size, a->page_table_width, kDecodeLongTile);
    if (need_long <= have || noalloc) {
      tile_keys = kDecodeLongTile;
      need = need_long;
    }
  }
  if (noalloc && need > CA_DECODE_NOALLOC_SCRATCH_BYTES) return CA_SCRATCH_EXCEEDED;
  if (!a->q || !a->k_cache || !a->v_cache || !a->lens || !a->page_table || !a->out)
    return CA_DECLINED;
  if ((a->k_new == nullptr) != (a->v_new == nullptr)) return CA_DECLINED;
  if (a->slots && !a->k_new) return CA_DECLINED;
  if (a->new_tokens < 0 || a->new_tokens > (1 << 30) || (a->slots && a->new_tokens > 1)) return CA_DECLINED;
  const int64_t per_seq = a->new_tokens > 1 ? a->new_tokens : 1;
  if (!aligned16(a->q) || !aligned16(a->k_cache) || !aligned16(a->v_cache) ||
      !aligned16(a->out) || !stride16(a->q_stride, a->dtype))
    return CA_DECLINED;
  if (a->k_new && (!aligned16(a->k_new) || !aligned16(a->v_new) || !stride16(a->kv_stride, a->dtype)))
    return CA_DECLINED;
  void* workspace = a->workspace;
  int64_t workspace_bytes = a->workspace_bytes;
  int scratch_device = -1;  // noalloc: the device whose scratch this call uses
  if (noalloc) {
    workspace = nullptr;
    workspace_bytes = 0;
    if (need > 0) {
      const int r = decode_noalloc_scratch(&workspace, &scratch_device);
      if (r != CA_OK) return r;
      workspace_bytes = CA_DECODE_NOALLOC_SCRATCH_BYTES;
    }
  }
  if (need > 0 && (!workspace || !aligned16(workspace) || workspace_bytes < need)) return CA_DECLINED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t words = a->head_dim * esize(a->dtype) / 4;
  // The reference stores the new token, then attends (paged_attn.mojo:852-863).
  // For a small batch, one token appended at lens (the serving step) is folded
  // into the decode kernel: the wave whose tile holds position lens[s] writes it
  // to the cache and attends it, so one launch does both.  Larger batches,
  // several tokens, or a store at given slots (which need not be the position
  // the row attends) go through a store kernel first: the scatter kernel for one
  // token per sequence (each on a page of its own), the staging one for a prompt.
  const bool fused = a->k_new && !a->slots && per_seq == 1 &&
                     a->num_seqs * a->num_heads <= kFusedAppendMaxRows;
  auto launch = [&]() -> int {
    if (a->k_new && !fused) {
      StoreParams sp{};
      sp.key = static_cast<const uint32_t*>(a->k_new);
      sp.value = static_cast<const uint32_t*>(a->v_new);
      sp.tok_stride_w = a->kv_stride * esize(a->dtype) / 4;
      sp.kc = static_cast<uint32_t*>(a->k_cache);
      sp.vc = static_cast<uint32_t*>(a->v_cache);
      sp.slots = a->slots;
      sp.lens = a->lens;
      sp.page_table = a->page_table;
      sp.pt_width = a->page_table_width;
      sp.ntok = a->num_seqs * per_seq;
      sp.per_seq = per_seq;
      sp.heads = a->num_heads;
      sp.page = a->page_size;
      sp.nblocks = a->num_blocks;
      const int r = per_seq == 1 ? store_scatter_launch(sp, (int)words, st) : store_launch(sp, (int)words, st);
      if (r != CA_OK) return r;
    }

    DecodeParams p{};
    p.q = a->q;
    p.q_stride = a->q_stride;
    p.kc = static_cast<const uint32_t*>(a->k_cache);
    p.vc = a->v_cache;
    p.lens = a->lens;
    // Appending at lens: the row attends lens + 1 keys.  With slots, lens is
    // already the post-store length (_C.mojo:100-103, paged_attn.mojo:721-723).
    p.len_add = (a->k_new && !a->slots) ? (int32_t)per_seq : 0;
    p.page_table = a->page_table;
    p.pt_width = a->page_table_width;
    p.heads = a->num_heads;
    p.page = a->page_size;
    p.nblocks = a->num_blocks;
    p.nseqs = a->num_seqs;
    p.c = a->scale * kLog2e;
    p.tile_keys = tile_keys;
    p.tiles = (int)decode_tiles(a->page_table_width, a->page_size, tile_keys);
    p.slots = decode_workspace_slots(rows, p.tiles);
    const int64_t acc_bytes = decode_acc_bytes(p.slots, a->head_dim);
    p.part_acc = static_cast<float*>(workspace);
    p.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + acc_bytes);
    if (decode_merges(rows, p.slots)) {
      p.counters = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + acc_bytes + p.slots * 8);
      p.tag = next_merge_tag();
    }
    p.out = a->out;
    if (fused) {
      p.k_new = static_cast<const uint32_t*>(a->k_new);
      p.v_new = static_cast<const uint32_t*>(a->v_new);
      p.kv_stride_w = a->kv_stride * esize(a->dtype) / 4;
      p.kc_store = static_cast<uint32_t*>(a->k_cache);
      p.vc_store = static_cast<uint32_t*>(a->v_cache);
    }
    return decode_launch(p, (int)a->head_dim, a->dtype == CA_BF16, st);
  };
  // The no-allocation entry's calls that use its one scratch buffer run one after
  // another on the device, whichever streams they come on.
  if (scratch_device >= 0) return decode_noalloc_ordered(scratch_device, st, launch);
  return launch();
}


extern "C" int ca_decode(const ca_decode_args* a, void* stream) { return decode_entry(a, stream, false); }

extern "C" int ca_decode_noalloc(const ca_decode_args* a, void* stream) {
  static_assert(CA_DECODE_NOALLOC_SCRATCH_BYTES == (32ll << 20), "the status string names the size");
  return decode_entry(a, stream, true);
}

extern "C" int64_t ca_flash_workspace_bytes(int64_t batch, int64_t seq_q, int64_t seq_k, int64_t num_heads,
                                            int64_t head_dim, int32_t dtype) {
  if (!dtype_ok(dtype) || !head_dim_ok(head_dim) || batch < 0 || num_heads < 0 || seq_q < 1 || seq_k < 1)
    return 0;
  return flash_rows_workspace_bytes(batch, seq_q, seq_k, num_heads, (int)head_dim, dtype == CA_BF16);
}

extern "C" int ca_flash(const ca_flash_args* a, void* stream) {
  if (!a || !dtype_ok(a->dtype) || !head_dim_ok(a->head_dim)) return CA_DECLINED;
  if (a->batch < 0 || a->num_heads <= 0 || a->seq_q < 1 || a->seq_k < 1) return CA_DECLINED;
  if (a->batch == 0) return CA_OK;
  if (!a->q || !a->k || !a->v || !a->out) return CA_DECLINED;
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->out))
    return CA_DECLINED;
  for (int i = 0; i < 3; ++i)
    if (!stride16(a->q_strides[i], a->dtype) || !stride16(a->k_strides[i], a->dtype) ||
        !stride16(a->v_strides[i], a->dtype))
      return CA_DECLINED;
  FlashParams p{};
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.out = a->out;
  p.batch = a->batch;
  p.seq_q = a->seq_q;
  p.seq_k = a->seq_k;
  p.heads = a->num_heads;
  for (int i = 0; i < 3; ++i) {
    p.qs[i] = a->q_strides[i];
    p.ks[i] = a->k_strides[i];
    p.vs[i] = a->v_strides[i];
  }
  p.c = a->scale * kLog2e;
  p.causal = a->causal ? 1 : 0;
  if (a->workspace_bytes < 0) return CA_DECLINED;
  // The split kernels write their partials with 16-byte stores.
  if (a->workspace && !aligned16(a->workspace) && flash_call_splits(p, (int)a->head_dim, a->dtype == CA_BF16) > 1)
    return CA_DECLINED;
  flash_rows_workspace(p, a->workspace, a->workspace_bytes, (int)a->head_dim, a->dtype == CA_BF16);
  return flash_launch(p, (int)a->head_dim, a->dtype == CA_BF16, static_cast<hipStream_t>(stream));
}
