// Parameter blocks passed from the C-ABI entries (ca_abi.hip) to the kernel
// launchers (ca_store.hip, ca_decode.hip, ca_flash.hip).  Host-only plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <functional>

namespace ca {

struct StoreParams {
  const uint32_t* key;    // [T, H, W] 32-bit words, token stride tok_stride_w
  const uint32_t* value;
  int64_t tok_stride_w;
  uint32_t* kc;           // per (block, head): W word rows of P tokens (K transposed)
  uint32_t* vc;           // per (block, head): P rows of W words
  const int64_t* slots;   // slot mode: [T]; nullptr selects append mode
  const int32_t* lens;    // append mode: [T / per_seq] positions (the pre-store lengths)
  const int32_t* page_table;
  int64_t pt_width;
  int64_t ntok, heads, page, nblocks;
  int64_t per_seq;        // append mode: consecutive tokens per sequence
};

struct DecodeParams {
  const void* q;          // [N, H, E] rows, sequence stride q_stride (elements)
  int64_t q_stride;
  const uint32_t* kc;     // K cache as 32-bit words
  const void* vc;
  const int32_t* lens;
  int32_t len_add;        // tokens appended at lens that the row also attends
  const int32_t* page_table;
  int64_t pt_width;
  int64_t heads, page, nblocks, nseqs;
  float c;                // softmax scale * log2(e)
  int tiles;              // tiles per row at the page table's capacity
  int tile_keys;          // keys per tile: 256, or 64 for a batch too small to fill the GPU
  int64_t slots;          // partial slots the workspace holds
  float* part_acc;        // [slots, E]
  float* part_ml;         // [slots, 2]: running max (scaled log2 units), sum
  // In-kernel merge (calls of at most kMergeMaxRows rows; nullptr: the combine
  // kernel merges): one counter word per row after the partials, and the call's
  // tag (never 0) that marks a word as this call's.
  uint64_t* counters;
  uint32_t tag;
  void* out;              // [N, H, E] contiguous
  // The one-token append done inside the decode (nullptr: none): token s of
  // k_new/v_new ([N, H, W] word rows, sequence stride kv_stride_w) is written to
  // the cache at position lens[s] by the wave whose tile holds that position,
  // which also attends it.
  const uint32_t* k_new;
  const uint32_t* v_new;
  int64_t kv_stride_w;
  uint32_t* kc_store;     // the caches, writable (for the appended token)
  uint32_t* vc_store;
};

struct FlashParams {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int64_t batch, seq_q, seq_k, heads;
  int64_t qs[3], ks[3], vs[3];  // batch, token, head strides (elements)
  float c;                      // softmax scale * log2(e)
  int causal;
  // Split-K partials in the caller's workspace (few-rows route, and the bf16
  // tiled kernel's split mode).
  float* part_acc;              // [batch*heads*seq_q, splits, E]
  float* part_ml;               // [batch*heads*seq_q, splits, 2]: max (scaled log2 units), sum
  int64_t workspace_bytes;
};

// Calls with few query rows take the few-rows route (ca_rows.hip): up to 4 rows
// in bf16 (past that the tiled MFMA kernel is faster on MI355X); in fp32 up to 8,
// and up to 16 when batch x heads alone fills the chip (256 or more).  Below that
// the tiled kernel's split mode is faster for 9-16 rows (N=1 L=12 S=4096 H=32
// E=128: 115 -> 79 us; L=16 S=8192: 182 -> 141 us), above it it is not (N=8 L=9
// S=2048 H=32 E=64: 130 against 148 us).  kRowsPerWave rows per wave.
constexpr int64_t kRowsMaxL = 16;
constexpr int64_t kRowsMaxLFew = 8;
constexpr int kRowsPerWave = 4;
// fp32 calls of 13 to 16 rows: kRowsPerWaveMany rows per wave, so two waves
// instead of four read each key (bit-identical results).  Measured on MI355X,
// back-to-back: N=16 L=16 S=4096 H=32 E=128 1212 -> 968 us, E=64 causal 568 -> 450
// us, N=2 L=16 S=8192 H=128 E=64 551 -> 434 us, N=8 L=16 S=1024 H=32 E=128 167 -> 134
// us; at 12 rows (3 waves against 2) it lost (N=4 L=12 S=3000 H=64 E=128 340 -> 366
// us), at 9 it was even.
constexpr int kRowsPerWaveMany = 8;
constexpr int64_t kRowsManyMinL = 13;
__host__ __device__ inline bool rows_route(int64_t batch, int64_t seq_q, int64_t heads, bool bf16) {
  if (bf16) return seq_q <= 4;
  return seq_q <= kRowsMaxLFew || (seq_q <= kRowsMaxL && batch * heads >= 256);
}
// bf16 calls past the few-rows route whose keys number at most kSmallMaxKeys take
// flash_small_kernel (ca_small.hip): one wave per kSmallRows query rows, every key
// in registers, when the call's row blocks (at most kSmallMaxBlocks) all run at
// once (small_max_blocks).  Measured on MI355X against the tiled kernel (bf16,
// back-to-back calls):
// N=1 L=S=128 H=16 E=64 causal 8.5 -> 4.9 us, N=1 L=S=128 H=32 E=128 11.4 -> 6.3 us,
// N=4 (512 row blocks) 11.9 -> 8.3 us; even at 2048 row blocks (N=16) 26.5 -> 26.0
// us, and slower at 4096 (N=8 L=512 S=128: 29.4 -> 45.5 us), where the tiled
// kernel's 256-row passes reuse each key tile for more rows.
constexpr int64_t kSmallMaxKeys = 256;
constexpr int kSmallRows = 32;
constexpr int64_t kSmallMaxBlocks = 1024;
// LDS rows of the short-key kernel's staged V: E bf16 padded to small_rsv(E)
// 16-byte chunks.  The 32 lanes a transposed read serves together read 4 rows x
// two 32-byte segments; a stride of 4 or 12 chunks mod 16 puts the 4 rows 16
// banks apart.
__host__ __device__ constexpr int small_rsv(int E) { return E == 128 ? 20 : (E == 64 ? 12 : 4); }
// Row blocks that run at once: one wave per SIMD (4 one-wave blocks per CU) on
// 256 CUs, as far as each block's staged V rows (LDS, 160 KB per CU) allow: E = 64
// past 192 keys 3 per CU, E = 128 past 128 keys 3 or 2.  A call that needed a
// second round measured slower than the tiled kernel (N=4 L=S=256 H=32 E=64
// causal: 12.3 against 17.6 us).
constexpr int64_t kSmallCuLds = 160 * 1024;
__host__ __device__ inline int64_t small_max_blocks(int64_t seq_k, int E) {
  const int64_t lds = ((seq_k + 31) / 32) * 32 * small_rsv(E) * 16;
  const int64_t per_cu = kSmallCuLds / lds;
  const int64_t blocks = 256 * (per_cu < 4 ? per_cu : 4);
  return blocks < kSmallMaxBlocks ? blocks : kSmallMaxBlocks;
}
__host__ __device__ inline bool small_route(int64_t batch, int64_t seq_q, int64_t seq_k, int64_t heads, int E,
                                            bool bf16) {
  return bf16 && seq_k <= kSmallMaxKeys &&
         batch * heads * ((seq_q + kSmallRows - 1) / kSmallRows) <= small_max_blocks(seq_k, E);
}
constexpr int kRowsWaves = 8;                 // waves per block
constexpr int64_t kRowsTargetBlocks = 256;    // blocks that keep every CU streaming
constexpr int64_t kRowsMaxSplits = 64;

// The tiled prefill splits each query block's keys over several blocks when its
// query blocks (batch x heads x ceil(seq_q / rows per block): 256 rows in bf16,
// 128 in fp32) leave the chip's CUs short of blocks: about kTiledTargetBlocks
// blocks (twice that in fp32, whose kernel keeps two blocks on each CU), at least
// kTiledMinKeys keys per split, at most kTiledMaxSplits.  Such
// calls (few rows over long key ranges) would otherwise leave most CUs idle,
// with a block's serial walk over every key tile the whole call's time.  In bf16
// (one block per CU) the split count rounds down, so the split blocks fit one
// round of the chip: rounded up, some CUs ran two blocks each (N=1 L=S=1792 H=20
// E=128, 140 query blocks: 2 splits 77.1 us, none 48.8 us).  The fp32 kernel
// keeps two blocks on a CU, which share its MFMA pipes; there the count rounds
// up, and neither rounding wins everywhere: causal L=S=1280 H=16 (160 query
// blocks) 4 splits 109.1 us, 3 splits 136.6 us; L=100 S=4096 H=300 (300) 2 splits
// 428.2 us, unsplit 570.7 us; but L=640 S=2048 H=24 (120) 5 splits 187.2 us, 4
// splits 152.0 us.  bf16 calls with fewer than twice as many keys as rows do not split
// from 2 * kTiledMinItemsUnsplit query blocks under 2 * kTiledMinKeysLong keys (more
// query blocks than that round down to one split anyway), nor from
// kTiledMinItemsUnsplit under kTiledMinKeysLong keys, nor, if causal or from
// kTiledMinItemsShort query blocks, under kTiledMinKeysCausal keys: the
// partials (fp32 (E + 2) per row and split, written and read back) and, for causal
// calls, a triangle that is most of the work make the unsplit blocks finish sooner
// (N=1 L=S=1024 H=32 E=128 non-causal 39.7 -> 31.3 us, causal 41.1 -> 33.8 us;
// L=S=1500 H=20 E=64: 34.6 -> 31.5 us; causal L=S=512 H=16 E=64, 32 query blocks,
// 18.6 -> 16.6 us; non-causal N=2 L=S=600 H=8 E=64, 48 blocks, 20.5 -> 17.3 us;
// N=1 L=S=512 H=8 E=128, 16 blocks, 20.7 -> 20.0 us).  Non-causal calls of fewer
// blocks under 1024 keys still split (N=1 L=S=768 H=4 E=128, 12 blocks: 20.8 split
// against 25.3 us; N=1 L=S=1000 H=2 E=64, 8: 15.5 against 23.2 us).  With fewer
// query blocks, or 64 to 127 over longer keys, most
// CUs would sit idle unsplit (N=2 L=700 S=1200 H=8 E=64, 48 blocks: split 23.0 us,
// unsplit 26.1 us; N=1 L=S=4096 H=4 E=128, 64: non-causal 51.6 against 96.1 us,
// causal 47.0 against 97.2 us; L=S=2048 H=8 E=64 26.3 / 27.9 against 38.6 / 40.8
// us; causal L=S=2048 H=4 E=128, 32: 30.3 against 53.8 us; 128 query blocks over
// 4096 keys or more, 2 splits: L=S=4096 H=8 E=128 80.8 against 96.3 us, causal 74.2
// against 97.1 us, causal L=S=8192 H=4 115.8 against 184.5 us).  fp32 calls split (193
// -> 301 us unsplit at L=1280 causal).  A causal call never splits more than the
// non-causal call of the same shapes; the workspace query answers for both.
constexpr int64_t kTiledTargetBlocks = 256;
constexpr int64_t kTiledMinKeys = 256;
constexpr int64_t kTiledMaxSplits = 64;
constexpr int64_t kTiledMinItemsUnsplit = 64;
constexpr int64_t kTiledMinKeysCausal = 1024;
constexpr int64_t kTiledMinItemsShort = 16;
constexpr int64_t kTiledMinKeysLong = 2048;
__host__ __device__ inline int64_t tiled_splits(int64_t batch, int64_t seq_q, int64_t seq_k, int64_t heads,
                                                bool bf16, bool causal) {
  if (rows_route(batch, seq_q, heads, bf16)) return 1;
  const int64_t bm = bf16 ? 256 : 128;
  const int64_t items = batch * heads * ((seq_q + bm - 1) / bm);
  if (bf16 && seq_k < 2 * seq_q &&
      ((items >= 2 * kTiledMinItemsUnsplit && seq_k < 2 * kTiledMinKeysLong) ||
       (items >= kTiledMinItemsUnsplit && seq_k < kTiledMinKeysLong) ||
       (seq_k < kTiledMinKeysCausal && (causal || items >= kTiledMinItemsShort))))
    return 1;
  const int64_t target = bf16 ? kTiledTargetBlocks : 2 * kTiledTargetBlocks;
  if (items <= 0 || items >= target) return 1;
  int64_t s = bf16 ? target / items : (target + items - 1) / items;
  const int64_t by_keys = (seq_k + 63) / 64 / (kTiledMinKeys / 64);
  s = s < by_keys ? s : by_keys;
  s = s < kTiledMaxSplits ? s : kTiledMaxSplits;
  return s < 2 ? 1 : s;
}
// Workspace bytes of the split mode: (O[E], m, l) per row and split.
__host__ __device__ inline int64_t tiled_workspace_bytes(int64_t batch, int64_t seq_q, int64_t seq_k,
                                                         int64_t heads, int E, bool bf16, bool causal) {
  const int64_t s = tiled_splits(batch, seq_q, seq_k, heads, bf16, causal);
  return s > 1 ? batch * heads * seq_q * s * (E + 2) * 4 : 0;
}
// The same for a call whose causal flag the caller does not state: the larger.
__host__ __device__ inline int64_t tiled_workspace_bytes_any(int64_t batch, int64_t seq_q, int64_t seq_k,
                                                             int64_t heads, int E, bool bf16) {
  const int64_t a = tiled_workspace_bytes(batch, seq_q, seq_k, heads, E, bf16, false);
  const int64_t c = tiled_workspace_bytes(batch, seq_q, seq_k, heads, E, bf16, true);
  return a > c ? a : c;
}

// The decode kernel does a one-token append itself (rather than a store kernel
// launched before it) for batches of up to this many rows (sequences x heads).
// Measured on MI355X: a 128-row fp32 batch (8 x 16) runs 13% faster fused (one
// launch instead of two); a 4096-row bf16 batch (128 x 32) runs 2.5% slower,
// because the token's K words, 4 bytes in each of W lines (K is transposed in the
// page), are partial-line writes that then compete with the decode's reads.
constexpr int64_t kFusedAppendMaxRows = 1024;

// Split rows of calls with at most this many rows are merged by their last block
// inside the decode kernel instead of by the combine kernel.  Measured on MI355X
// (bf16 E=128 page 16 unless noted, back-to-back calls): 32 rows 9.91 -> 9.37 us,
// 64 rows 11.20 -> 10.38 us, 128 rows 17.89 -> 16.69 us (fp32 H=16 E=64 with an
// append: 18.24 -> 16.96 us), 512 rows 38.0 -> 37.4 us; 1024 rows even (86.2 ->
// 85.8 us; fp32 E=64 84.7 -> 85.6 us), 4096 rows (bf16 E=128 page 32) 189.3 ->
// 191.4 us.  It also needs at least kMergeMinRows rows and at most kMergeMaxBlocks
// blocks per row (of the page table's capacity): a row's blocks count themselves
// in on one counter with a compare-and-swap, and when many finish at once the
// retries serialise.  Against the combine kernel (bf16 E=128 page 16 unless
// noted, back-to-back, with a one-token append): N=1 H=8 at 32768 keys (64 blocks
// per row) 213.1 -> 31.7 us, N=1 H=32 at 32768 keys 157.7 -> 90.6 us, at 4096 (8
// blocks) 20.5 -> 15.5 us, at 3072 (6) 16.2 -> 13.6 us, at 2560 (5) 14.6 -> 12.6 us,
// at 2048 (4 blocks, 32 rows of one length) 12.8 -> 11.8 us, fp32 N=2 H=4 E=64 at
// 20000 keys 94.9 -> 23.2 us; the merge still wins at 4 blocks from 64 rows (fp32
// N=8 H=16 E=64 at 2048 keys 25.3 -> 24.7 us, cfg2 18.1 -> 17.3 us, N=16 H=32
// lengths up to 2047 without append 37.4 -> 36.7 us) and is even at 5 blocks
// over 64 rows (fp32 N=8 H=8 E=64 at 2560 keys 20.5 -> 20.4 us).
constexpr int64_t kMergeMaxRows = 512;
constexpr int64_t kMergeMinRows = 64;
constexpr int64_t kMergeMaxBlocks = 4;

int store_launch(const StoreParams& p, int words, hipStream_t stream);
// One token per sequence (p.per_seq == 1): one wave per (token, head), no staging.
int store_scatter_launch(const StoreParams& p, int words, hipStream_t stream);
constexpr int kDecodeLongTile = 256;  // keys per tile of the decode's long tiles
int decode_tile_keys(int64_t rows, int64_t pt_width, int64_t page, int64_t head_dim, int esize);
int64_t decode_tiles(int64_t pt_width, int64_t page, int tile_keys);
int64_t decode_workspace_slots(int64_t rows, int64_t tiles);
int decode_launch(const DecodeParams& p, int head_dim, int bf16, hipStream_t stream);
// ca_decode_noalloc's scratch on the current device (and that device's index),
// and the ordering of the calls that use it: see ca_noalloc.hip.
int decode_noalloc_scratch(void** ptr, int* device);
int decode_noalloc_ordered(int device, hipStream_t stream, const std::function<int()>& launch);
// How flash_launch runs a call: the kernel, its grid (gy = splits of the keys
// in the split modes), and whether the combine kernel merges `splits` partials
// per row afterwards.  kind is kPlanDeclined for a call the kernels cannot take.
enum { kPlanDeclined = 0, kPlanNone, kPlanRows, kPlanRowsHeads, kPlanBf16, kPlanF32, kPlanSmall };
struct FlashPlan {
  int kind;
  int rows_r;      // kPlanRows: query rows per wave group (1, kRowsPerWave or kRowsPerWaveMany)
  bool split;      // kPlanBf16 / kPlanF32: keys split over gy blocks
  bool pair;       // kPlanF32: causal query-block pairs
  int64_t gx, gy;  // grid
  int64_t splits;  // > 1: the combine kernel merges this many partials per row
  int64_t need;    // workspace bytes the partials take
};
FlashPlan flash_plan(const FlashParams& p, int head_dim, bool bf16);
int flash_launch(const FlashParams& p, int head_dim, int bf16, hipStream_t stream);
int64_t flash_rows_workspace_bytes(int64_t batch, int64_t seq_q, int64_t seq_k, int64_t heads, int head_dim,
                                   bool bf16);
// Splits of the keys the call's kernels use (1: no workspace); p's shapes and
// causal flag must be set.
int64_t flash_call_splits(const FlashParams& p, int head_dim, bool bf16);
void flash_rows_workspace(FlashParams& p, void* ws, int64_t bytes, int head_dim, bool bf16);
int flash_rows_launch(const FlashParams& p, const FlashPlan& plan, int head_dim, int bf16, hipStream_t stream);
// The few-rows route's part of flash_plan (p.seq_q within rows_route).
FlashPlan rows_plan(const FlashParams& p, int head_dim, bool bf16);
// The short-key route's plan (small_route) and launch.
FlashPlan small_plan(const FlashParams& p);
int flash_small_launch(const FlashParams& p, const FlashPlan& plan, int head_dim, hipStream_t stream);
// Merges each row's `splits` partials (p.part_acc / p.part_ml) into p.out.
int flash_combine_launch(const FlashParams& p, int head_dim, int bf16, int64_t splits, hipStream_t stream);

}  // namespace ca
