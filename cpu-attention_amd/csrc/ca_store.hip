// reshape_and_cache and the decode-time append: a pure copy of K/V rows into the
// paged cache (the reference's PageLayout, cpu_attention/_mojo/src/paged_attn.mojo:58-130;
// store paths _store_kv :151-176, _store_block :180-204).
//
// The kernel works on 32-bit words, so one instantiation per row width serves both
// dtypes: a head's K or V row is W words (bf16: E/2 words, each a pair of adjacent
// dims; fp32: E words).  V rows are copied as they are (16-byte loads and stores).
// K is transposed inside the page (word (w, t) at w*P + t): a block stages 16
// tokens' K rows in LDS and writes word w of the 16 tokens from 16 neighbouring
// lanes, so tokens in consecutive slots of one page become one contiguous 64-byte
// run per word row.  Bytes are moved, never converted: the result is bit-exact.
#include "ca_device.h"
#include "ca_internal.h"

namespace ca {

constexpr int kStoreTok = 16;  // tokens per block

// Where token i goes: block index (or -1 to skip) and position in the page.
__device__ __forceinline__ void store_target(const StoreParams& p, int64_t i, int64_t& blk,
                                             int64_t& off) {
  blk = -1;
  off = 0;
  if (p.slots) {
    // reshape_and_cache / the engine path: negative slots are padding (vLLM
    // semantics, paged_attn.mojo:158-160); a slot past the cache is never written.
    int64_t s = p.slots[i];
    if (s >= 0 && s < p.nblocks * p.page) {
      blk = s / p.page;
      off = s - blk * p.page;
    }
  } else {
    // Append at the pre-store length through the page table (paged_attn.mojo:165-170):
    // token j of a sequence goes to position lens + j; a negative length stores
    // nothing, nor does a position past the page table.
    const int64_t seq = p.per_seq == 1 ? i : i / p.per_seq;
    const int64_t len = p.lens[seq];
    int64_t pos = len + (i - seq * p.per_seq);
    if (len >= 0) {
      int64_t pi = pos / p.page;
      if (pi < p.pt_width) {
        int64_t b = p.page_table[seq * p.pt_width + pi];
        if (b >= 0 && b < p.nblocks) {
          blk = b;
          off = pos - pi * p.page;
        }
      }
    }
  }
}

template <int W>
__global__ __launch_bounds__(256) void store_kernel(StoreParams p) {
  constexpr int LD = W + 1;  // padded LDS row: the transposed reads hit 16 distinct banks
  constexpr int Q4 = W / 4;  // 16-byte chunks per row
  __shared__ uint32_t kbuf[kStoreTok * LD];
  __shared__ int64_t s_blk[kStoreTok];
  __shared__ int64_t s_off[kStoreTok];

  const int tid = threadIdx.x;
  const int64_t i0 = (int64_t)blockIdx.x * kStoreTok;
  const int nt = (int)min<int64_t>(kStoreTok, p.ntok - i0);
  if (tid < kStoreTok) {
    int64_t blk = -1, off = 0;
    if (tid < nt) store_target(p, i0 + tid, blk, off);
    s_blk[tid] = blk;
    s_off[tid] = off;
  }
  __syncthreads();

  const int64_t h0 = (int64_t)blockIdx.y * p.heads_per_block;
  const int64_t h1 = min<int64_t>(p.heads, h0 + p.heads_per_block);
  const int64_t page_words = p.page * W;
  for (int64_t h = h0; h < h1; ++h) {
    // Stage K rows (coalesced 16-byte loads) and copy V rows straight through.
    for (int c = tid; c < kStoreTok * Q4; c += 256) {
      const int t = c / Q4, q4 = c - t * Q4;
      if (t < nt) {
        const int64_t src = (i0 + t) * p.tok_stride_w + h * W + 4 * q4;
        u32x4 kv = *reinterpret_cast<const u32x4*>(p.key + src);
        kbuf[t * LD + 4 * q4 + 0] = kv.x;
        kbuf[t * LD + 4 * q4 + 1] = kv.y;
        kbuf[t * LD + 4 * q4 + 2] = kv.z;
        kbuf[t * LD + 4 * q4 + 3] = kv.w;
        const int64_t blk = s_blk[t];
        if (blk >= 0) {
          u32x4 vv = *reinterpret_cast<const u32x4*>(p.value + src);
          const int64_t dst = ((blk * p.heads + h) * p.page + s_off[t]) * W + 4 * q4;
          *reinterpret_cast<u32x4*>(p.vc + dst) = vv;
        }
      }
    }
    __syncthreads();
    // K: word w of token t -> w*P + off_t; 16 neighbouring lanes take the 16 tokens.
    for (int idx = tid; idx < kStoreTok * W; idx += 256) {
      const int t = idx & (kStoreTok - 1), w = idx / kStoreTok;
      const int64_t blk = s_blk[t];
      if (t < nt && blk >= 0)
        p.kc[(blk * p.heads + h) * page_words + (int64_t)w * p.page + s_off[t]] = kbuf[t * LD + w];
    }
    __syncthreads();
  }
}

int store_launch(const StoreParams& sp, int W, hipStream_t stream) {
  if (sp.ntok == 0) return CA_OK;
  const int64_t gx = cdiv(sp.ntok, kStoreTok);
  if (gx > 0x7fffffff) return CA_DECLINED;
  // Enough blocks to fill the chip: split the heads over grid.y when tokens are few.
  int64_t gy = gx >= 2048 ? 1 : std::min<int64_t>(sp.heads, std::max<int64_t>(1, 2048 / gx));
  StoreParams p = sp;
  p.heads_per_block = (int)cdiv(sp.heads, gy);
  gy = cdiv(sp.heads, p.heads_per_block);
  dim3 grid((unsigned)gx, (unsigned)gy), block(256);
  switch (W) {
    case 16: hipLaunchKernelGGL(store_kernel<16>, grid, block, 0, stream, p); break;
    case 32: hipLaunchKernelGGL(store_kernel<32>, grid, block, 0, stream, p); break;
    case 64: hipLaunchKernelGGL(store_kernel<64>, grid, block, 0, stream, p); break;
    case 128: hipLaunchKernelGGL(store_kernel<128>, grid, block, 0, stream, p); break;
    default: return CA_DECLINED;
  }
  return ca_launch_status();
}

}  // namespace ca
