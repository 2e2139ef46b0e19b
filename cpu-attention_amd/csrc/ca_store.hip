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
// run per word row.  A block takes 16 tokens of 256/W heads (grid.y walks the
// heads) and issues all of its loads before any store, so every CU keeps many
// rows in flight.  Bytes are moved, never converted: the result is bit-exact.
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
  constexpr int LD = W + 1;                          // padded LDS row: transposed reads hit distinct banks
  constexpr int Q4 = W / 4;                          // 16-byte chunks per row
  constexpr int HB = 256 / W;                        // heads per block
  constexpr int NCH = kStoreTok * HB * Q4 / 256;     // chunks per thread (K and V each): 4
  static_assert(NCH * 256 == kStoreTok * HB * Q4, "block shape");
  __shared__ uint32_t kbuf[HB][kStoreTok * LD];
  __shared__ int64_t s_blk[kStoreTok];
  __shared__ int64_t s_off[kStoreTok];

  const int tid = threadIdx.x;
  // One-dimensional grid over (head group, token group), token groups fastest;
  // neighbouring token groups share an XCD, so the two blocks that write parts
  // of one page's 64-byte K word rows meet in one L2.
  const int64_t ngx = cdiv(p.ntok, kStoreTok);
  const int64_t lg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t gy = lg / ngx;
  const int64_t i0 = (lg - gy * ngx) * kStoreTok;
  const int nt = (int)min<int64_t>(kStoreTok, p.ntok - i0);
  const int64_t h0 = gy * HB;
  if (tid < kStoreTok) {
    int64_t blk = -1, off = 0;
    if (tid < nt) store_target(p, i0 + tid, blk, off);
    s_blk[tid] = blk;
    s_off[tid] = off;
  }
  // Every K and V load of the block in flight at once (coalesced 16-byte loads:
  // a token's rows of HB heads are contiguous); tokens that are not stored
  // (padding slots, positions past the page table) are not read.
  u32x4 kv[NCH], vv[NCH];
  int64_t dst[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int idx = tid + 256 * c;
    const int t = idx / (HB * Q4), rem = idx - t * (HB * Q4), hh = rem / Q4, q4 = rem - hh * Q4;
    dst[c] = -1;
    kv[c] = u32x4{0u, 0u, 0u, 0u};
    vv[c] = u32x4{0u, 0u, 0u, 0u};
    if (t < nt && h0 + hh < p.heads) {
      int64_t blk, off;
      store_target(p, i0 + t, blk, off);
      if (blk >= 0) {
        const int64_t src = (i0 + t) * p.tok_stride_w + (h0 + hh) * W + 4 * q4;
        // Each byte is read once and written once: non-temporal loads and V
        // stores keep them out of L2 (cfg5's staging 453 -> 438 us).  K's word
        // stores below stay plain: written non-temporally, their 64-byte runs
        // (half lines) took 1.6x as long.
        kv[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.key + src));
        vv[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.value + src));
        dst[c] = ((blk * p.heads + h0 + hh) * p.page + off) * W + 4 * q4;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int idx = tid + 256 * c;
    const int t = idx / (HB * Q4), rem = idx - t * (HB * Q4), hh = rem / Q4, q4 = rem - hh * Q4;
    if (dst[c] >= 0) {
      uint32_t* kr = &kbuf[hh][t * LD + 4 * q4];
      kr[0] = kv[c].x;
      kr[1] = kv[c].y;
      kr[2] = kv[c].z;
      kr[3] = kv[c].w;
      __builtin_nontemporal_store(vv[c], reinterpret_cast<u32x4*>(p.vc + dst[c]));
    }
  }
  __syncthreads();
  const int64_t page_words = p.page * W;
  // K: word w of token t -> w*P + off_t; 16 neighbouring lanes take the 16 tokens,
  // so consecutive slots of one page become one 64-byte run per word row.
  for (int idx = tid; idx < kStoreTok * W * HB; idx += 256) {
    const int t = idx & (kStoreTok - 1), r = idx / kStoreTok, hh = r / W, w = r - hh * W;
    const int64_t blk = s_blk[t];
    if (t < nt && blk >= 0 && h0 + hh < p.heads)
      p.kc[(blk * p.heads + h0 + hh) * page_words + (int64_t)w * p.page + s_off[t]] = kbuf[hh][t * LD + w];
  }
}

// One token per sequence (the decode-time append, and the engine path's store at
// a slot): every token lands on a page of its own, so store_kernel's staging, which
// merges consecutive slots of a page into 64-byte K word rows, has nothing to
// merge, and its 16-token blocks leave most of the chip idle on a small batch.
// Here one wave moves one (token, head): lane w moves K word w (one 4-byte store
// per word row of the page) and lanes below W/4 move the V row in 16-byte pieces.
// A block is 4 waves (4 heads of one token).
template <int W>
__global__ __launch_bounds__(256) void scatter_kernel(StoreParams p) {
  constexpr int KPL = (W + kWave - 1) / kWave;  // K words per lane
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t hg = cdiv(p.heads, 4);
  const int64_t i = blockIdx.x / hg;
  const int64_t h = (blockIdx.x - i * hg) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (i >= p.ntok || h >= p.heads) return;
  int64_t blk, off;
  store_target(p, i, blk, off);
  if (blk < 0) return;
  const int64_t src = i * p.tok_stride_w + h * W;
  const int64_t row0 = (blk * p.heads + h) * p.page;  // the (block, head)'s first row
  uint32_t kw[KPL];
  u32x4 vv = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int c = 0; c < KPL; ++c) {
    const int w = lane + kWave * c;
    kw[c] = w < W ? p.key[src + w] : 0u;
  }
  if (lane < W / 4) vv = *reinterpret_cast<const u32x4*>(p.value + src + 4 * lane);
#pragma unroll
  for (int c = 0; c < KPL; ++c) {
    const int w = lane + kWave * c;
    if (w < W) p.kc[row0 * W + (int64_t)w * p.page + off] = kw[c];
  }
  if (lane < W / 4) *reinterpret_cast<u32x4*>(p.vc + (row0 + off) * W + 4 * lane) = vv;
}

int store_scatter_launch(const StoreParams& sp, int W, hipStream_t stream) {
  if (sp.ntok == 0) return CA_OK;
  if (sp.per_seq != 1) return CA_DECLINED;
  const int64_t nb = sp.ntok * cdiv(sp.heads, 4);
  if (nb > 0x7fffffff) return CA_DECLINED;
  dim3 grid((unsigned)nb), block(256);
  switch (W) {
    case 16: hipLaunchKernelGGL(scatter_kernel<16>, grid, block, 0, stream, sp); break;
    case 32: hipLaunchKernelGGL(scatter_kernel<32>, grid, block, 0, stream, sp); break;
    case 64: hipLaunchKernelGGL(scatter_kernel<64>, grid, block, 0, stream, sp); break;
    case 128: hipLaunchKernelGGL(scatter_kernel<128>, grid, block, 0, stream, sp); break;
    default: return CA_DECLINED;
  }
  return ca_launch_status();
}

int store_launch(const StoreParams& sp, int W, hipStream_t stream) {
  if (sp.ntok == 0) return CA_OK;
  const int64_t nb = cdiv(sp.ntok, kStoreTok) * cdiv(sp.heads, 256 / W);
  if (nb > 0x7fffffff) return CA_DECLINED;
  dim3 grid((unsigned)nb), block(256);
  switch (W) {
    case 16: hipLaunchKernelGGL(store_kernel<16>, grid, block, 0, stream, sp); break;
    case 32: hipLaunchKernelGGL(store_kernel<32>, grid, block, 0, stream, sp); break;
    case 64: hipLaunchKernelGGL(store_kernel<64>, grid, block, 0, stream, sp); break;
    case 128: hipLaunchKernelGGL(store_kernel<128>, grid, block, 0, stream, sp); break;
    default: return CA_DECLINED;
  }
  return ca_launch_status();
}

}  // namespace ca
