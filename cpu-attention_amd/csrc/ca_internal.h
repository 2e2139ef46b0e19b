// Parameter blocks passed from the C-ABI entries (ca_abi.hip) to the kernel
// launchers (ca_store.hip, ca_decode.hip, ca_flash.hip).  Host-only plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ca {

struct StoreParams {
  const uint32_t* key;    // [T, H, W] 32-bit words, token stride tok_stride_w
  const uint32_t* value;
  int64_t tok_stride_w;
  uint32_t* kc;           // per (block, head): W word rows of P tokens (K transposed)
  uint32_t* vc;           // per (block, head): P rows of W words
  const int64_t* slots;   // slot mode: [T]; nullptr selects append mode
  const int32_t* lens;    // append mode: [T] positions (the pre-store lengths)
  const int32_t* page_table;
  int64_t pt_width;
  int64_t ntok, heads, page, nblocks;
  int heads_per_block;
};

struct DecodeParams {
  const void* q;          // [N, H, E] rows, sequence stride q_stride (elements)
  int64_t q_stride;
  const uint32_t* kc;     // K cache as 32-bit words
  const void* vc;
  const int32_t* lens;
  int32_t len_add;        // 1 when the row also attends a token appended at lens
  const int32_t* page_table;
  int64_t pt_width;
  int64_t heads, page, nblocks, nseqs;
  float c;                // softmax scale * log2(e)
  int tiles;              // 256-key tiles per row at the page table's capacity
  int64_t slots;          // partial slots the workspace holds
  float* part_acc;        // [slots, E]
  float* part_ml;         // [slots, 2]: running max (scaled log2 units), sum
  void* out;              // [N, H, E] contiguous
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
};

int store_launch(const StoreParams& p, int words, hipStream_t stream);
int64_t decode_tiles(int64_t pt_width, int64_t page);
int64_t decode_workspace_slots(int64_t rows, int64_t tiles);
int decode_launch(const DecodeParams& p, int head_dim, int bf16, hipStream_t stream);
int flash_launch(const FlashParams& p, int head_dim, int bf16, hipStream_t stream);

}  // namespace ca
