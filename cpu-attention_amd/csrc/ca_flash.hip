// flash_attn_func forward on CDNA4 matrix cores.
//
// Semantics follow the reference's prefill driver (cpu_attention/_mojo/src/flash_attn.mojo:
// 127-183): causal is bottom-right aligned (row i sees keys j <= i + S - L), key
// tiles past the last visible key are never touched, the online softmax runs in
// base 2 with c = scale*log2(e), and a row that sees no key is exactly 0.
//
// bf16 (flash_bf16_p64_kernel, the default): 4 waves x 64 query rows per block,
// one wave per SIMD.  A wave's VALU work runs while its own independent MFMAs
// execute, so each wave issues one stream per key tile of 64: the P.V MFMAs of
// the previous tile, the S MFMAs of the next and the softmax of this one.  Key
// tiles go global -> LDS with direct buffer loads; K is read with ds_read_b128,
// V^T with ds_read_b64_tr_b16 from the row-major V tile.
//   S^T = K Q^T   32x32x16 MFMAs with keys as rows and queries as columns, so a
//                 lane ends up owning one query and 16 keys of each 32-key half;
//   softmax       per lane (its query) against a max fixed 64 log2 units above
//                 the first tile's; rows whose later logits outgrow the first
//                 tile's by more than about 123 are redone by a safe pass with a
//                 running max;
//   O^T += V^T P^T the probabilities are already in the B-operand layout of the
//                 MFMA (no LDS round trip); P is rounded to bf16 as the reference's
//                 bf16 policy does (flash_vec.mojo:255-259), fp32 accumulation.
// fp32 (flash_f32_kernel): 4 waves x 32 rows, K/V staged through registers into
// LDS, v_mfma_f32_32x32x2_f32, everything fp32.
#include <type_traits>

#include "ca_device.h"
#include "ca_internal.h"

namespace ca {

constexpr int kBM = 128;  // fp32: query rows per block (4 waves x 32)

// A raw buffer resource over [base, base + bytes): loads past `bytes` return 0.
// The per-tile K/V loads rebase the resource at each tile, so their per-lane
// offsets stay fixed across the loop (no address registers rewritten under
// in-flight loads) and rows past the last key come back as zeros.
// A tile that starts past the last key (the prefetch after the last tile) has a
// negative byte count: it becomes an empty window, where every load reads zero
// without touching memory.
__host__ __device__ inline int window_bytes(int64_t bytes) {
  return (int)(bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, window_bytes(bytes), 0x00020000);
}

__host__ __device__ inline int imin(int a, int b) { return a < b ? a : b; }
__host__ __device__ inline int imax(int a, int b) { return a > b ? a : b; }

struct BlockWork {
  int64_t b, h, q0;
};

__host__ __device__ inline BlockWork block_work(const FlashParams& p, int64_t bid) {
  const int64_t nqb = cdiv(p.seq_q, kBM);
  const int64_t nb = p.batch * p.heads * nqb;
  const int64_t lg = xcd_remap(bid, nb);
  const int64_t bh = lg / nqb;
  const int64_t qb = nqb - 1 - (lg - bh * nqb);  // the most expensive causal blocks first
  BlockWork w;
  w.b = bh / p.heads;
  w.h = bh - w.b * p.heads;
  w.q0 = qb * kBM;
  return w;
}

// ---------------------------------------------------------------------------
// bf16: key-tile geometry
// ---------------------------------------------------------------------------
// Key tiles of 64 go from global memory straight into LDS (buffer loads with LDS
// as the destination: no staging registers; rows past the block's key range
// fill with zeros), split over the block's 4 waves.
//
// LDS layouts: rows of E bf16 padded to RSK (K) or RSV (V) 16-byte chunks, so
// operand reads are conflict-free and every address is a per-lane base plus a
// constant.  The V^T MFMA operands come from ds_read_b64_tr_b16 on the row-major
// V tile: it gives lane j of a 16-lane group column j of a 4-row x 16-column
// block (4 keys of one dim).
template <int E>
struct FlashBf16Cfg {
  static constexpr int NWG = 4;            // waves that share a tile's loads
  static constexpr int BN = 64;            // keys per tile
  static constexpr int CPR = E / 8;        // 16-byte chunks per row
  // Padded row strides in chunks.  K: 16 lanes reading one 16-byte column of 16
  // consecutive rows hit 16 different 4-bank groups.  V: the 32 lanes that a
  // transposed read serves together read 4 rows x two 32-byte segments; a stride
  // of 4 or 12 chunks mod 16 puts the 4 rows 16 banks apart, so the 8 segments
  // cover the 64 banks once.
  static constexpr int RSK = CPR + 1;
  static constexpr int RSV = CPR == 16 ? 20 : (CPR == 8 ? 12 : 4);
  // Direct loads per thread and tile: the 4 waves load a tile, every load of a
  // wave fills 64 consecutive chunks, so a tile buffer is NL rounds of 4 x 64
  // chunks.  K and V tiles take the same NL (the larger), so every wave issues
  // the same number of loads per tile and one wait count serves all.
  static constexpr int NLK = (BN * RSK + 64 * NWG - 1) / (64 * NWG);
  static constexpr int NLV = (BN * RSV + 64 * NWG - 1) / (64 * NWG);
  static constexpr int NL = NLK > NLV ? NLK : NLV;
  static constexpr int TBUF = NL * 64 * NWG * 8;  // elements per tile buffer
};

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4v;
typedef __attribute__((address_space(3))) bf16x4v lds_bf16x4;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;

// One bf16 block's work: a (batch, head) and one or two query blocks.  Causal
// calls pair query block j with nqb-1-j, so every block walks about the same
// number of key tiles (the expensive one first); non-causal blocks take one.
struct PairWork {
  int64_t b, h, qb0, qb1;
  int n;
};

// Causal calls pair query blocks (qb, nqb-1-qb), so that every block has the
// same work, unless the unpaired query blocks number few enough to all run at
// once: then pairs would leave CUs idle.  bf16 (256-row blocks, one per CU):
// pairs past 256 query blocks.  fp32 (128-row blocks, two per CU; below 512 the
// split mode runs instead): pairs from 1024, or from 512 when the causal
// triangle is most of the work (fewer than twice as many keys as rows); with
// more keys the blocks' work is nearly even, and 512 blocks as 256 pairs would
// leave each CU one block instead of two.
constexpr int64_t kPairMinBlocks = 256;  // the chip's CUs
__host__ __device__ inline bool pair_blocks(const FlashParams& p, int64_t nqb, bool bf16) {
  const int64_t items = p.batch * p.heads * nqb;
  if (!p.causal) return false;
  if (bf16) return items > kPairMinBlocks;
  return items >= 4 * kPairMinBlocks || (items >= 2 * kPairMinBlocks && p.seq_k < 2 * p.seq_q);
}

__host__ __device__ inline PairWork pair_work(const FlashParams& p, int bm, bool bf16, int64_t bid) {
  const int64_t nqb = cdiv(p.seq_q, bm);
  const bool pair = pair_blocks(p, nqb, bf16);
  const int64_t per = pair ? (nqb + 1) / 2 : nqb;
  const int64_t lg = xcd_remap(bid, p.batch * p.heads * per);
  const int64_t bh = lg / per, j = lg - bh * per;
  PairWork w;
  w.b = bh / p.heads;
  w.h = bh - w.b * p.heads;
  w.qb0 = p.causal ? nqb - 1 - j : j;
  w.qb1 = j;
  w.n = (pair && w.qb0 != j) ? 2 : 1;
  return w;
}

// The bf16 tiled kernel's work for block (bx, by) of its grid: a causal pair or
// one query block (pair_work), or in the split mode (gy splits) query block bx %
// nqb of (batch, head) bx / nqb and split by of its keys.
__host__ __device__ inline PairWork bf16_block_work(const FlashParams& p, bool split, int64_t bx) {
  PairWork pw;
  if (split) {
    const int64_t nqb = cdiv(p.seq_q, 256);
    const int64_t bh = bx / nqb;
    pw.b = bh / p.heads;
    pw.h = bh - pw.b * p.heads;
    pw.qb0 = pw.qb1 = bx - bh * nqb;
    pw.n = 1;
  } else {
    pw = pair_work(p, 256, true, bx);
  }
  return pw;
}

// A pass's rows and keys: query block rows [q0, q0 + 256), keys [kbeg, kend) in
// nkt tiles of 64 (the split mode's share of them: whole tiles, empty past the
// pass's last key).
struct Bf16Geom {
  int q0, kbeg, kend, nkt;
};
__host__ __device__ inline Bf16Geom bf16_pass_geom(const FlashParams& p, const PairWork& pw, int pass, bool split,
                                                   int sp, int splits) {
  const int S = (int)p.seq_k, diag = (int)(p.seq_k - p.seq_q);
  Bf16Geom g;
  g.q0 = (int)(pass == 0 ? pw.qb0 : pw.qb1) * 256;
  g.kbeg = 0;
  g.kend = p.causal ? imin(S, g.q0 + 256 + diag) : S;
  if (split) {
    const int chunk = (int)cdiv(cdiv(p.seq_k, 64), splits) * 64;
    g.kbeg = imin(sp * chunk, imax(g.kend, 0));
    g.kend = imin(g.kbeg + chunk, g.kend);
  }
  g.nkt = g.kend > g.kbeg ? (g.kend - g.kbeg + 63) / 64 : 0;
  return g;
}
// Tiles of the pass's keys [kbeg, kend) that rows [r0, r0 + nrows) walk (S
// keys, diag = S - L); `clamp` cuts their keys at kend (the split mode's range;
// a whole pass's kend never cuts a row's).
__host__ __device__ inline int bf16_row_tiles(int S, int diag, int causal, int kbeg, int kend, int r0, int nrows,
                                              bool clamp) {
  int kend_w = causal ? imin(S, r0 + nrows + diag) : S;
  if (clamp) kend_w = imin(kend_w, kend);
  return kend_w > kbeg ? (kend_w - kbeg + 63) / 64 : 0;
}

// What one pass (a query block of one (batch, head)) needs, shared by the fast
// walk and the safe pass.
struct Bf16Pass {
  const uint16_t* q;  // row 0 of the (batch, head)
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;      // row 0 of the (batch, head); rows H*E apart
  int L, S, diag, q0, kend;
  int qs1, ks1, vs1, heads;
  float c;
  int causal;
};

// Fixed per-thread byte offsets of the direct loads of a tile: load i of wave w
// of a group fills LDS chunk P = (4i + w)*64 + lane, i.e. row P / RS, column
// P % RS.  Pad columns and chunks past the tile's rows get an offset past any
// window, so they read as zeros without touching memory.
template <int E, int RS, int NL>
__host__ __device__ inline void tile_offsets(int wv4, int lane, int stride, int (&off)[NL]) {
  constexpr int CPR = E / 8, BN = FlashBf16Cfg<E>::BN, NWG = FlashBf16Cfg<E>::NWG;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int P = (NWG * i + wv4) * 64 + lane, r = P / RS, col = P % RS;
    off[i] = (r < BN && col < CPR) ? (r * stride + 8 * col) * 2 : (int)0x80000000;
  }
}

// The byte window of a key tile whose first row is followed by `rows` rows of
// the pass's key range (row stride stride2 bytes): a full tile gets 2^31 - 1
// bytes (its 64 rows lie inside the range; the launcher bounds 64 rows of the
// stride below 2^31 bytes), a partial one is cut after its last row, one past
// the range is empty.
template <int E>
__host__ __device__ inline int tile_window(int rows, int stride2) {
  return rows >= FlashBf16Cfg<E>::BN ? 0x7fffffff : (rows <= 0 ? 0 : (rows - 1) * stride2 + E * 2);
}

// One wave's share of the successive K tiles or V tiles of a pass: rows [k0, k0 + BN) of the source per tile, cut at the pass's key
// range (rows past it read as zeros, a tile past it touches no memory), into
// `nbuf` rotating tile buffers.  Every field is wave-uniform and advances by an
// add per tile, so a tile's loads cost a few scalar instructions.
// The loads are issued from inline assembly: the compiler does not track them,
// so it inserts no wait for them before unrelated LDS reads (it cannot tell the
// buffers apart); loads_landed_barrier() waits for them explicitly.
typedef __attribute__((ext_vector_type(4))) int i32x4;
template <int E>
struct TileStream {
  static constexpr int BN = FlashBf16Cfg<E>::BN, NL = FlashBf16Cfg<E>::NL, NWG = FlashBf16Cfg<E>::NWG;
  static constexpr uint32_t BUF_BYTES = FlashBf16Cfg<E>::TBUF * 2;
  uint64_t addr;   // first row of the next tile
  uint32_t step;   // bytes from one tile's first row to the next (< 2^31: the launcher checks)
  int rows;        // rows of the key range from the next tile's first row on
  int stride2;     // row stride in bytes
  uint32_t lds;    // this wave's LDS byte address in the next tile's buffer
  uint32_t lds0, lds_last;

  __device__ __forceinline__ void init(const uint16_t* src, int stride, int kend, const uint16_t* buf0, int nbuf,
                                       int first, int wv4) {
    addr = reinterpret_cast<uint64_t>(src);
    stride2 = 2 * stride;
    step = (uint32_t)(BN * stride2);
    rows = kend;
    lds0 = (uint32_t)reinterpret_cast<uintptr_t>((const lds_void*)buf0) + wv4 * 1024;
    lds_last = lds0 + (nbuf - 1) * BUF_BYTES;
    lds = lds0 + first * BUF_BYTES;
  }

  // Loads of one tile through a window of `bytes` from `addr` (0: all zeros).
  __device__ __forceinline__ void issue_window(int bytes, const int (&off)[NL]) {
    const i32x4 rs = {__builtin_amdgcn_readfirstlane((int)(uint32_t)addr),
                      __builtin_amdgcn_readfirstlane((int)((addr >> 32) & 0xffff)),
                      __builtin_amdgcn_readfirstlane(bytes), 0x00020000};
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds);
#pragma unroll
    for (int i = 0; i < NL; ++i)
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                   :
                   : "s"(base + i * NWG * 1024), "v"(off[i]), "s"(rs)
                   : "memory");
    lds = lds == lds_last ? lds0 : lds + BUF_BYTES;
  }

  // The next tile of the key range.  A window of 2^31 - 1 bytes covers any tile
  // (the launcher bounds BN rows of the stride below 2^31 bytes).
  __device__ __forceinline__ void issue(const int (&off)[NL]) {
    issue_window(tile_window<E>(rows, stride2), off);
    addr += step;
    rows -= BN;
  }

  // A tile of zeros (no memory touched); the stream's position does not move.
  __device__ __forceinline__ void issue_zeros(const int (&off)[NL]) { issue_window(0, off); }
};

// Waits until at most N of this wave's memory loads are outstanding (loads
// complete in issue order), then the block barrier.
template <int N>
__device__ __forceinline__ void loads_landed_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
  __syncthreads();
}
__device__ __forceinline__ void loads_done_barrier() { loads_landed_barrier<0>(); }

// K operand of the S MFMA: dims 16s + 8hf..+7 of key row `row`.
template <int E>
__device__ __forceinline__ bf16x8 k_operand(const uint16_t* kb, int row, int s, int hf) {
  return *reinterpret_cast<const bf16x8*>(kb + (row * FlashBf16Cfg<E>::RSK + 2 * s + hf) * 8);
}

// V^T operand of the P.V MFMA for keys 16cc.. and dims 32d..: lane (dim li, half
// hf) gets keys 16cc + 4hf + 0..3 and 16cc + 8 + 4hf + 0..3 (the order in which
// the probabilities sit in the B operand).
template <int E>
__device__ __forceinline__ bf16x8 v_operand(const uint16_t* vb, int lane, int cc, int d) {
  constexpr int RSV = FlashBf16Cfg<E>::RSV;
  const int j = lane & 15, dh = (lane >> 4) & 1, hf = lane >> 5;
  const uint16_t* base = vb + (4 * hf + (j >> 2)) * RSV * 8 + 16 * dh + 4 * (j & 3);
  bf16x4v a[2];
#pragma unroll
  for (int q = 0; q < 2; ++q)
    a[q] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(base + (16 * cc + 8 * q) * RSV * 8 + 32 * d));
  return bf16x8{a[0][0], a[0][1], a[0][2], a[0][3], a[1][0], a[1][1], a[1][2], a[1][3]};
}

// -inf for keys past the row's limit (an arithmetic mask: a compare per element
// would take a scalar mask register each).
__device__ __forceinline__ float mask_key(float v, int vis, int key) {
  int msk;
  asm("v_ashrrev_i32 %0, 31, %1" : "=v"(msk) : "v"(vis - key));
  return v + __int_as_float(msk & (int)0xff800000u);
}

// State and key-tile step of the safe pass (one column block): 32 query rows of
// one (batch, head), lane (query li, half hf), with a running max.
template <int E>
struct Bf16Rows {
  static constexpr int BN = FlashBf16Cfg<E>::BN, NS = E / 16, ND = E / 32;
  bf16x8 qr[NS];  // Q rows as B operands: dims 16s + 8hf..+7
  f32x16 o[ND];   // O^T accumulators: dims 32d + 8(r/4) + 4hf + r%4
  float m, l;
  int li, hf, lane, r0;

  __device__ __forceinline__ void load_q(const Bf16Pass& a) {
    issue_q(a, r0);
    reset();
  }

  // The Q loads of the 32 rows from `row0` alone (the accumulators may still
  // hold the previous pass, whose rows r0 names).
  __device__ __forceinline__ void issue_q(const Bf16Pass& a, int row0) {
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(a.q + (int64_t)row0 * a.qs1, ((int64_t)(a.L - 1 - row0) * a.qs1 + E) * 2);
#pragma unroll
    for (int s = 0; s < NS; ++s)
      qr[s] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, (li * a.qs1 + 16 * s + 8 * hf) * 2, 0, 0));
  }

  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int d = 0; d < ND; ++d) o[d] = f32x16{};
    m = -INFINITY;
    l = 0.f;
  }

  // Keys of tile t this lane's row may see: key 32kt + 8(r/4) + 4hf + r%4 of the
  // tile is visible when 32kt + 8(r/4) + r%4 <= the returned limit.
  __device__ __forceinline__ int vis_of(const Bf16Pass& a, int kbeg, int t) const {
    const int k0 = kbeg + t * BN;
    int lim = a.S - 1 - k0;
    if (a.causal) lim = min(lim, r0 + li + a.diag - k0);
    return max(-1, min(lim, BN)) - 4 * hf;
  }

  // S^T = K Q^T for the tile: keys as rows, queries as columns, so a lane ends
  // up with one query and 16 keys of each 32-key half (two independent chains).
  __device__ __forceinline__ void logits(const uint16_t* kb, f32x16 (&st)[2]) const {
    f32x16 a0 = f32x16{}, a1 = f32x16{};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      a0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_operand<E>(kb, li, s, hf), qr[s], a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_operand<E>(kb, 32 + li, s, hf), qr[s], a1, 0, 0, 0);
    }
    st[0] = a0;
    st[1] = a1;
  }

  // Row max of the tile in scaled log2 units, as the reference takes it (tile
  // max of the visible raw logits times c).
  __device__ __forceinline__ float tile_max(const f32x16 (&st)[2], int vis, float c) const {
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, mask_key(st[kt][r], vis, 32 * kt + 8 * (r >> 2) + (r & 3)));
    return fmaxf(mx, __shfl_xor(mx, 32)) * c;
  }

  // p = 2^(s*c - m), rounded to bf16 for P.V as the reference's bf16 policy does
  // (flash_vec.mojo:255-259; l sums the unrounded p).  The 8 probabilities a lane
  // holds per 16 keys are exactly the B operand of the P.V MFMA.  Returns this
  // lane's sum of p over the tile (it bounds every p of the lane).
  template <bool MASK>
  __device__ __forceinline__ float softmax(const f32x16 (&st)[2], int vis, float c, bf16x8 (&pb)[4]) {
    const float nmu = m == -INFINITY ? 0.f : -m;
    float ls = 0.f;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      uint32_t w[4];
#pragma unroll
      for (int jj = 0; jj < 8; jj += 2) {
        const int kt = cc >> 1, r = 8 * (cc & 1) + jj;
        float v0 = st[kt][r], v1 = st[kt][r + 1];
        if (MASK) {
          v0 = mask_key(v0, vis, 32 * kt + 8 * (r >> 2) + (r & 3));
          v1 = mask_key(v1, vis, 32 * kt + 8 * ((r + 1) >> 2) + ((r + 1) & 3));
        }
        const float e0 = __builtin_amdgcn_exp2f(fmaf(v0, c, nmu));
        const float e1 = __builtin_amdgcn_exp2f(fmaf(v1, c, nmu));
        ls += e0 + e1;
        w[jj / 2] = pack_bf16x2(e0, e1);
      }
      pb[cc] = __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
    }
    l += ls;
    return ls;
  }

  // O^T += V^T P^T.
  __device__ __forceinline__ void pv(const uint16_t* vb, const bf16x8 (&pb)[4]) {
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
#pragma unroll
      for (int d = 0; d < ND; ++d)
        o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v_operand<E>(vb, lane, cc, d), pb[cc], o[d], 0, 0, 0);
  }

  // The rows' partial for the combine (keys split over blocks): O^T unnormalised,
  // the running max (scaled log2 units) and l, at slot slot0 + row * splits of
  // the workspace.  A row that saw no key leaves m = -inf, l = 0, O = 0.
  __device__ __forceinline__ void store_partial(const Bf16Pass& a, float* pacc, float* pml, int64_t slot0,
                                                int splits) const {
    const float lt = l + __shfl_xor(l, 32);
    const int row = r0 + li;
    if (row < a.L) {
      const int64_t slot = slot0 + (int64_t)row * splits;
      float* orow = pacc + slot * E;
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f32x4*>(orow + 32 * d + 8 * q + 4 * hf) =
              f32x4{o[d][4 * q], o[d][4 * q + 1], o[d][4 * q + 2], o[d][4 * q + 3]};
      if (hf == 0) {
        pml[2 * slot] = m;
        pml[2 * slot + 1] = lt;
      }
    }
  }

  // out = acc / l; a row with no visible key is 0.
  __device__ __forceinline__ void store(const Bf16Pass& a) const {
    const float lt = l + __shfl_xor(l, 32);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int row = r0 + li;
    if (row < a.L) {
      uint16_t* orow = a.out + (int64_t)row * a.heads * E;
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          u32x2 w = {pack_bf16x2(o[d][4 * q] * inv, o[d][4 * q + 1] * inv),
                     pack_bf16x2(o[d][4 * q + 2] * inv, o[d][4 * q + 3] * inv)};
          *reinterpret_cast<u32x2*>(orow + 32 * d + 8 * q + 4 * hf) = w;
        }
    }
  }
};

// ---------------------------------------------------------------------------
// bf16, 64 query rows per wave, softmax overlapped with the MFMAs
// ---------------------------------------------------------------------------
// Block = 4 waves x 64 query rows (256-row query blocks), one wave per SIMD with the whole register file: Q and the
// O accumulators live in AGPRs (only MFMAs read them), S, P and the operands in
// VGPRs.  A wave's VALU work runs while its own MFMAs execute (measured on
// gfx950: 4 MFMAs and 64 independent VALU ops per iteration take as long as the
// VALU ops alone), so iteration t of the tile walk issues one interleaved stream
//   the P.V MFMAs of tile t-1 and the S MFMAs of tile t+1 (64 at E = 128), and
//   the softmax of tile t (one score per MFMA at E = 128),
// with the S of consecutive tiles in two register sets.  Each K operand read
// from LDS feeds the S MFMAs of both 32-row column blocks, and each V^T operand
// both P.V MFMAs: half the LDS operand bytes per MFMA of the 32-row layout.
// The MFMAs are inline assembly (for the AGPR operands), so the compiler does
// not know their result latency: where a VALU read of an MFMA result follows
// closely, mfma_guard() supplies the wait states.
template <int E>
struct FlashP64Cfg {
  static constexpr int NW = 4;        // waves per block
  static constexpr int BM = 64 * NW;  // query rows per block
  static constexpr int BN = FlashBf16Cfg<E>::BN;
  static constexpr int NL = FlashBf16Cfg<E>::NL;  // direct loads per wave and tile (K or V)
  static constexpr int TBUF = FlashBf16Cfg<E>::TBUF;
  static constexpr int NBUFK = 4;  // K tiles: K(t+3) goes out while S(t+1) reads K(t+1)
  static constexpr int NBUFV = 3;  // V tiles: V(t+1) goes out while P.V reads V(t-1)
  static constexpr int LDS_BYTES = (NBUFK + NBUFV) * TBUF * 2;
  static_assert(NW == FlashBf16Cfg<E>::NWG, "the tile loads are split over NWG waves");
  static_assert(LDS_BYTES + 1024 <= 160 * 1024, "tile buffers fit the LDS with room for the block's own");
};

// 64 query rows of one (batch, head) as two 32-row column blocks cb: lane (query
// li, half hf) of block cb holds row r0 + 32 cb + li.
template <int E>
struct P64Rows {
  static constexpr int BN = FlashP64Cfg<E>::BN, NS = E / 16, ND = E / 32;
  static constexpr int NPV = 4 * ND;  // V^T operands of a tile: keys 16cc.., dims 32d..
  static constexpr int NSK = 2 * NS;  // K operands of a tile: keys 32kt.., dims 16s..
  static constexpr int LA = 6;        // operand reads run LA operands ahead of their MFMAs
  bf16x8 qr[2][NS];    // Q^T of column block cb as B operands (AGPRs)
  f32x16 o[2][ND];     // O^T accumulators (AGPRs): dims 32d + 8(r/4) + 4hf + r%4
  f32x16 st[2][2][2];  // S^T of two consecutive tiles: [tile parity][cb][kt]
  bf16x8 pb[2][4];     // P^T of the latest softmax: [cb][16-key group cc]
  float m[2], nmu[2], l[2];
  int li, hf, lane, r0;
  int klo, vlo;  // this lane's byte offsets of its K and V^T operand reads in a tile buffer

  __device__ __forceinline__ void init(int lane_) {
    lane = lane_;
    li = lane & 31;
    hf = lane >> 5;
    // K operand: row li (+ 32 kt), 16-byte chunk hf (+ 2 s), rows RSK chunks apart.
    klo = (li * FlashBf16Cfg<E>::RSK + hf) * 16;
    // V^T operand (as v_operand): lane (j, dh, hf) reads the 4-element run of
    // row 4 hf + j / 4 at column 16 dh + 4 (j % 4).
    const int j = lane & 15, dh = (lane >> 4) & 1;
    vlo = ((4 * hf + (j >> 2)) * FlashBf16Cfg<E>::RSV * 8 + 16 * dh + 4 * (j & 3)) * 2;
  }

  // The Q loads of both column blocks (VGPRs; moved to AGPRs by q_home).
  __device__ __forceinline__ void issue_q(const Bf16Pass& a) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int rb = r0 + 32 * cb;
      const __amdgpu_buffer_rsrc_t rs = tile_rsrc(a.q + (int64_t)rb * a.qs1, ((int64_t)(a.L - 1 - rb) * a.qs1 + E) * 2);
#pragma unroll
      for (int s = 0; s < NS; ++s)
        qr[cb][s] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, (li * a.qs1 + 16 * s + 8 * hf) * 2, 0, 0));
    }
  }

  // Q to the AGPRs, O = 0 (written by MFMAs, so the accumulators are born in
  // AGPRs; volatile, so each block gets its own MFMA rather than a copy of one
  // block's zeros), and the softmax state reset.  settle() must follow.  The
  // compiler may write the zero operand just before (it does not know the asm
  // is an MFMA, which reads a VGPR that VALU code wrote only 2 wait states later),
  // hence the s_nop.
  __device__ __forceinline__ void q_home() {
    const bf16x8 z = bf16x8{};
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
      for (int s = 0; s < NS; ++s) asm("" : "+a"(qr[cb][s]));
#pragma unroll
      for (int d = 0; d < ND; ++d)
        asm volatile("s_nop 2\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %1, 0" : "=a"(o[cb][d]) : "v"(z));
      m[cb] = -INFINITY;
      nmu[cb] = 0.f;
      l[cb] = 0.f;
    }
  }

  // LDS byte address of buf + off, opaque to the compiler's reassociation.
  __device__ __forceinline__ static uint32_t lds_base(const uint16_t* buf, int off) {
    uint32_t a = (uint32_t)reinterpret_cast<uintptr_t>((const lds_void*)buf) + off;
    asm volatile("" : "+v"(a));
    return a;
  }

  // At least 11 wait states (an 8-pass MFMA) before a VALU read of an MFMA result.
  __device__ __forceinline__ static void mfma_guard() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }

  // The wait states after MFMAs that wrote O, then the accumulators marked as
  // redefined here.  The MFMAs are inline assembly, so the compiler does not know
  // their results land late: a copy it makes of O on its own (to merge two
  // control-flow paths, say) could otherwise read the registers too early.
  __device__ __forceinline__ void settle() {
    mfma_guard();
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int d = 0; d < ND; ++d) asm volatile("" : "+a"(o[cb][d]));
  }

  // Keys of tile t (from key kbeg on) row (cb, li) may see: key 32kt + 8(r/4) +
  // 4hf + r%4 of the tile is visible when 32kt + 8(r/4) + r%4 <= the returned
  // limit.  The lane id is recomputed here (this runs only on masked tiles), so
  // that no register holds a lane constant for it across the walk.
  __device__ __forceinline__ int vis_of(const Bf16Pass& a, int kbeg, int t, int cb) const {
    int lid;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lid));
    const int k0 = kbeg + t * BN;
    int lim = a.S - 1 - k0;
    if (a.causal) lim = min(lim, r0 + 32 * cb + (lid & 31) + a.diag - k0);
    return max(-1, min(lim, BN)) - 4 * (lid >> 5);
  }

  // The MFMAs and the pins below are volatile so that they keep their order and
  // their slot in the stream (the compiler would otherwise move pure arithmetic
  // freely across the slots).
  __device__ __forceinline__ void mfma_pv(int cb, int d, const bf16x8& vop, const bf16x8& p) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(o[cb][d]) : "v"(vop), "v"(p));
  }

  template <int PAR>
  __device__ __forceinline__ void mfma_s(int cb, int kt, int s, const bf16x8& kop) {
    if (s == 0)
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(st[PAR][cb][kt]) : "v"(kop), "a"(qr[cb][s]));
    else
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(st[PAR][cb][kt]) : "v"(kop), "a"(qr[cb][s]));
  }

  // -inf for the keys of st[PAR] past each row's limit (tile t), in place: one
  // fixed assembly block per logit with a single temporary (the compiler would
  // interleave the elements and run out of registers on this rare path).
  template <int PAR>
  __device__ __forceinline__ void apply_mask(const Bf16Pass& a, int kbeg, int t) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int vis = vis_of(a, kbeg, t, cb);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          int tmp;
          asm volatile(
              "v_subrev_u32 %1, %3, %2\n\tv_ashrrev_i32 %1, 31, %1\n\t"
              "v_and_b32 %1, 0xff800000, %1\n\tv_add_f32 %0, %0, %1"
              : "+v"(st[PAR][cb][kt][r]), "=&v"(tmp)
              : "v"(vis), "i"(32 * kt + 8 * (r >> 2) + (r & 3)));
        }
    }
  }

  // Fixes each row's max at kMaxLift above tile 0's (every row that sees any key
  // sees key 0), in scaled log2 units as the reference takes it.  The softmax is
  // the same for any max; the lift only moves the window of logits the fixed max
  // serves exactly.  p of tile 0's largest logit is 2^-64, so p stays a normal
  // fp32 (and bf16) for logits down to 62 below it: smaller ones weigh less than
  // 2^-62 against that key and may flush to 0.  Upwards, a lane's sum of p over a
  // tile stays within the walk's 2^64 headroom for logits up to about 123 above
  // tile 0's max (64 without the lift); only rows whose logits outgrow that go
  // through the safe pass.
  static constexpr float kMaxLift = 64.f;
  __device__ __forceinline__ void fix_max(float c) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[0][cb][kt][r]);
      m[cb] = fmaxf(mx, __shfl_xor(mx, 32)) * c + kMaxLift;
      nmu[cb] = m[cb] == -INFINITY ? 0.f : -m[cb];
    }
  }

  // Iteration t of the walk, as one stream in which every MFMA shares its issue
  // slot with VALU work:
  //   PV:   O^T += V^T P^T for tile t-1 (V^T from vb, P^T from pb);
  //   SN:   S^T = K Q^T for tile t+1 (K from kb) into st[PAR ^ 1];
  //   SOFT: the softmax of tile t from st[PAR] (masked beforehand where the
  //         tile needs it) into new P^T, rounded to bf16 as the reference's
  //         bf16 policy does (flash_vec.mojo:255-259; l sums the unrounded p).
  // `loads` (this wave's share of the next tiles' loads) goes out after the
  // first operand reads.  Returns false when a row's sum of p over the tile
  // exceeds the fast walk's headroom (or is NaN).
  template <int PAR, bool PV, bool SN, bool SOFT, typename F>
  __device__ __forceinline__ bool step(const uint16_t* vb, const uint16_t* kb, float c, F&& loads) {
    // A lane's p summed over a tile <= 2^64.  p taken against a max that a later
    // logit exceeds is still exact in floating point (no precision is lost to a
    // large exponent); the bound only keeps the sums finite: l stays below 2^71
    // over any 4096 keys, so O = sum p V cannot overflow fp32 unless |V| > 2^57.
    constexpr float kHeadSum = 18446744073709551616.f;
    constexpr int NPVo = PV ? NPV : 0, NOP = NPVo + (SN ? NSK : 0), NM = 2 * NOP;
    constexpr int NSLOT = NM > 0 ? NM : 1, NSC = SOFT ? 64 : 0;
    static_assert(NSC % NSLOT == 0, "scores spread evenly over the MFMA slots");
    // Operand addresses: one per-lane base per buffer, constant offsets.
    // The bases are opaque to the compiler (it would otherwise fold the constant
    // offsets into per-operand base registers, kept live across the loop, and
    // add the buffer's offset to each of them).
    const uint32_t vbase = lds_base(vb, vlo), kbase = lds_base(kb, klo);
    auto read_v = [&](uint32_t base, int q) __attribute__((always_inline)) {
      const int cc = q / ND, d = q % ND;
      bf16x4v h[2];
#pragma unroll
      for (int u = 0; u < 2; ++u)
        h[u] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4*)(uintptr_t)(base + ((16 * cc + 8 * u) * FlashBf16Cfg<E>::RSV * 8 + 32 * d) * 2));
      return bf16x8{h[0][0], h[0][1], h[0][2], h[0][3], h[1][0], h[1][1], h[1][2], h[1][3]};
    };
    auto read = [&](int q) __attribute__((always_inline)) {
      if (q < NPVo) return read_v(vbase, q);
      const int j = q - NPVo, kt = j & 1, sq = j >> 1;
      return *(lds_bf16x8*)(uintptr_t)(kbase + (32 * kt * FlashBf16Cfg<E>::RSK + 2 * sq) * 16);
    };
    bf16x8 op[NOP > 0 ? NOP : 1];
#pragma unroll
    for (int q = 0; q < (NOP < LA ? NOP : LA); ++q) op[q] = read(q);
    loads();
    __builtin_amdgcn_sched_barrier(0);
    // Score x (in the order of the P^T groups (cc, cb), so that the P^T of a
    // group is complete early; the P.V MFMAs read the previous P^T) goes through
    // three stages in consecutive slots: the exponent (slot of x), exp2 (next
    // slot), the row sum and the bf16 pair (the one after), so that no stage
    // waits in its slot for the result of the stage before it.
    constexpr int PER = NSC / NSLOT;
    float ls[2] = {0.f, 0.f};
    float sv[64], ev[64];
    uint32_t pw[2][4][4];
    auto coords = [](int x, int& cb, int& cc, int& kt, int& r, int& jj) __attribute__((always_inline)) {
      const int g = x >> 3;
      jj = x & 7;
      cb = g & 1;
      cc = g >> 1;
      kt = cc >> 1;
      r = 8 * (cc & 1) + jj;
    };
#pragma unroll
    for (int i = 0; i < NSLOT + (SOFT ? 2 : 0); ++i) {
      // The slot's VALU work goes first: it overlaps the previous slot's MFMA
      // and gives the operand read of this slot's MFMA more time.
      // Each stage is one fixed-order assembly block (volatile: the blocks keep
      // their slots).  Spacing kept by the stage order: an exp2 result is read
      // two slots later, an exponent one slot later, and the register an exp2
      // reads is not rewritten by the instruction right after it.
      if (i >= 2) {  // stage 3 for the scores of slot i - 2: row sums, bf16 pairs
#pragma unroll
        for (int x = (i - 2) * PER; x < (i - 1) * PER; ++x) {
          int cb, cc, kt, r, jj;
          coords(x, cb, cc, kt, r, jj);
          if (jj & 1)
            asm volatile("v_add_f32 %0, %0, %2\n\tv_cvt_pk_bf16_f32 %1, %3, %2"
                         : "+v"(ls[cb]), "=&v"(pw[cb][cc][jj >> 1])
                         : "v"(ev[x]), "v"(ev[x - 1]));
          else
            asm volatile("v_add_f32 %0, %0, %1" : "+v"(ls[cb]) : "v"(ev[x]));
        }
      }
      if (i < NSLOT) {  // stage 1 for the scores of slot i: exponents s*c - m
#pragma unroll
        for (int x = i * PER; x < (i + 1) * PER; ++x) {
          int cb, cc, kt, r, jj;
          coords(x, cb, cc, kt, r, jj);
          asm volatile("v_fma_f32 %0, %1, %2, %3" : "=&v"(sv[x]) : "v"(st[PAR][cb][kt][r]), "s"(c), "v"(nmu[cb]));
        }
      }
      if (i >= 1 && i <= NSLOT) {  // stage 2 for the scores of slot i - 1: exp2
#pragma unroll
        for (int x = (i - 1) * PER; x < i * PER; ++x) asm volatile("v_exp_f32 %0, %1" : "=&v"(ev[x]) : "v"(sv[x]));
      }
      if ((i & 1) == 0 && i / 2 + LA < NOP) op[i / 2 + LA] = read(i / 2 + LA);
      if (i < NM) {
        const int q = i >> 1, cb = i & 1;
        if (q < NPVo) {
          mfma_pv(cb, q % ND, op[q], pb[cb][q / ND]);
        } else {
          const int j = q - NPVo;
          mfma_s<PAR ^ 1>(cb, j & 1, j >> 1, op[q]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!SOFT) return true;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
        pb[cb][cc] = __builtin_bit_cast(bf16x8, u32x4{pw[cb][cc][0], pw[cb][cc][1], pw[cb][cc][2], pw[cb][cc][3]});
    l[0] += ls[0];
    l[1] += ls[1];
    return ls[0] <= kHeadSum && ls[1] <= kHeadSum;
  }

  // Bytes of LDS that store_staged needs per wave: 32 rows of E bf16, padded.
  static constexpr int kStageRow = 2 * E + 16;
  static constexpr int kStageBytes = 32 * kStageRow;

  // out = acc / l, staged through this wave's `stage` area of LDS one column
  // block at a time: in the O^T layout a lane holds 4-dim runs of one row, so
  // direct stores would touch 32 rows per instruction; staged, each store
  // instruction writes whole rows (64 / (E/8) rows of E/8 16-byte chunks).  The
  // area is private to the wave, whose LDS accesses run in order.  A row with no
  // visible key is 0.
  __device__ __forceinline__ void store_staged(const Bf16Pass& a, char* stage) {
    constexpr int CPR = E / 8, RPI = 64 / CPR;  // 16-byte chunks per row, rows per store
    mfma_guard();
    const int ch = lane % CPR, rr0 = lane / CPR;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const float lt = l[cb] + __shfl_xor(l[cb], 32);
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      char* rowp = stage + li * kStageRow;
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          u32x2 v = {pack_bf16x2(o[cb][d][4 * q] * inv, o[cb][d][4 * q + 1] * inv),
                     pack_bf16x2(o[cb][d][4 * q + 2] * inv, o[cb][d][4 * q + 3] * inv)};
          *reinterpret_cast<u32x2*>(rowp + (32 * d + 8 * q + 4 * hf) * 2) = v;
        }
#pragma unroll
      for (int k = 0; k < 32 / RPI; ++k) {
        const int rr = rr0 + RPI * k, row = r0 + 32 * cb + rr;
        const u32x4 v = *reinterpret_cast<const u32x4*>(stage + rr * kStageRow + ch * 16);
        // Non-temporal: the output is not read again here, and keeping it out of
        // L2 leaves the lines to the K/V tiles other blocks re-read (cfg4 541 ->
        // 534 us, N=16 L=S=1024 222 -> 212 us, bit-identical).
        if (row < a.L)
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(a.out + (int64_t)row * a.heads * E + ch * 8));
      }
    }
  }

  // Bytes of LDS that store_partials needs per wave: 32 rows of E floats, padded.
  static constexpr int kPartRow = 4 * E + 16;
  static constexpr int kPartBytes = 32 * kPartRow;

  // The rows' partial for the combine (keys split over blocks): O^T unnormalised
  // (fp32), the fixed max m (scaled log2 units) and l, at slot slot0 + row *
  // splits of the workspace, staged through this wave's `stage` area as
  // store_staged stages the output (each store instruction writes 256 / E whole
  // rows).  A row that saw no key leaves m = -inf, l = 0, O = 0.
  __device__ __forceinline__ void store_partials(const Bf16Pass& a, char* stage, float* pacc, float* pml,
                                                 int64_t slot0, int splits) {
    constexpr int CPR = E / 4, RPI = 64 / CPR;  // 16-byte chunks per row, rows per store
    mfma_guard();
    const int ch = lane % CPR, rr0 = lane / CPR;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const float lt = l[cb] + __shfl_xor(l[cb], 32);
      const int rowl = r0 + 32 * cb + li;
      if (hf == 0 && rowl < a.L) {
        const int64_t slot = slot0 + (int64_t)rowl * splits;
        pml[2 * slot] = m[cb];
        pml[2 * slot + 1] = lt;
      }
      char* rowp = stage + li * kPartRow;
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f32x4*>(rowp + (32 * d + 8 * q + 4 * hf) * 4) =
              f32x4{o[cb][d][4 * q], o[cb][d][4 * q + 1], o[cb][d][4 * q + 2], o[cb][d][4 * q + 3]};
#pragma unroll
      for (int k = 0; k < 32 / RPI; ++k) {
        const int rr = rr0 + RPI * k, row = r0 + 32 * cb + rr;
        const f32x4 v = *reinterpret_cast<const f32x4*>(stage + rr * kPartRow + ch * 16);
        if (row < a.L) *reinterpret_cast<f32x4*>(pacc + (slot0 + (int64_t)row * splits) * E + ch * 4) = v;
      }
    }
  }
};

// The safe pass of the 64-row kernel: both column blocks of every wave walk the
// pass with a lazily refreshed running max (as bf16_safe_pass), one tile buffer
// each for K and V, loaded by all 4 waves.  Waves with `active` false compute and
// store nothing but take part in the loads and barriers.
// The split mode's pass: its keys start at kbeg, and its rows' partials go to
// slots slot0 + row * splits of the workspace.
struct SplitOut {
  float* pacc;
  float* pml;
  int64_t slot0;
  int splits;
  int kbeg;
};

template <int E, bool SPLIT>
__device__ __forceinline__ void bf16_safe_pass_body(const Bf16Pass& a, bool active, const SplitOut* so) {
  using C = FlashP64Cfg<E>;
  constexpr int BN = C::BN, ND = E / 32, NL = C::NL;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* Ks = smem;
  uint16_t* Vs = smem + C::NBUFK * C::TBUF;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  int koff[NL], voff[NL];
  tile_offsets<E, FlashBf16Cfg<E>::RSK>(wv, lane, a.ks1, koff);
  tile_offsets<E, FlashBf16Cfg<E>::RSV>(wv, lane, a.vs1, voff);
  // The pass's keys [kbeg, a.kend): all it sees, or the block's split of them.
  int kbeg = 0;
  if constexpr (SPLIT) kbeg = so->kbeg;
  TileStream<E> tk, tv;
  tk.init(a.k + (int64_t)kbeg * a.ks1, a.ks1, a.kend - kbeg, Ks, 1, 0, wv);
  tv.init(a.v + (int64_t)kbeg * a.vs1, a.vs1, a.kend - kbeg, Vs, 1, 0, wv);
  const int nkt = a.kend > kbeg ? (a.kend - kbeg + BN - 1) / BN : 0;
  Bf16Rows<E> w[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    w[cb].lane = lane;
    w[cb].li = lane & 31;
    w[cb].hf = lane >> 5;
    w[cb].r0 = a.q0 + 64 * wv + 32 * cb;
    w[cb].load_q(a);
  }
  __syncthreads();  // the fast walk is done with the tile buffers
  for (int t = 0; t < nkt; ++t) {
    tk.issue(koff);
    tv.issue(voff);
    loads_done_barrier();
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int nkt_w = active ? bf16_row_tiles(a.S, a.diag, a.causal, kbeg, a.kend, w[cb].r0, 32, true) : 0;
      if (t < nkt_w) {
        f32x16 st[2];
        w[cb].logits(Ks, st);
        const int vis = w[cb].vis_of(a, kbeg, t);
        const float mt = w[cb].tile_max(st, vis, a.c);
        if (__any(mt > w[cb].m + 8.f)) {
          const float mn = fmaxf(w[cb].m, mt);
          const float alpha = __builtin_amdgcn_exp2f(w[cb].m - (mn == -INFINITY ? 0.f : mn));
          w[cb].l *= alpha;
#pragma unroll
          for (int d = 0; d < ND; ++d) w[cb].o[d] *= alpha;
          w[cb].m = mn;
        }
        bf16x8 pb[4];
        w[cb].template softmax<true>(st, vis, a.c, pb);
        w[cb].pv(Vs, pb);
      }
    }
    __syncthreads();  // every wave is done with the tiles before they are refilled
  }
  if (active) {
    if constexpr (SPLIT) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) w[cb].store_partial(a, so->pacc, so->pml, so->slot0, so->splits);
    } else {
      w[0].store(a);
      w[1].store(a);
    }
  }
}

// The safe pass out of line: for the output, or for the split mode's partials
// (the slots are passed in: a called function cannot read the kernel's
// arguments itself).
template <int E>
__device__ __noinline__ void bf16_safe_pass_p64(const Bf16Pass& a, bool active) {
  bf16_safe_pass_body<E, false>(a, active, nullptr);
}
template <int E>
__device__ __noinline__ void bf16_safe_pass_p64(const Bf16Pass& a, bool active, const SplitOut& so) {
  bf16_safe_pass_body<E, true>(a, active, &so);
}

// SPLIT: the keys of each query block are split over gridDim.y blocks (calls whose
// query blocks leave most CUs idle); each block walks its range of whole key
// tiles and leaves (O, m, l) partials per row in the workspace for the combine
// kernel.  Otherwise a block takes a causal pair or a query block and writes the
// output.
template <int E, bool SPLIT>
__global__ __launch_bounds__(256, 1) void flash_bf16_p64_kernel(FlashParams p) {
  using C = FlashP64Cfg<E>;
  constexpr int BM = C::BM, BN = C::BN, NL = C::NL;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* Ks = smem;                       // K tile buffers [NBUFK]
  uint16_t* Vs = smem + C::NBUFK * C::TBUF;  // V tile buffers [NBUFV]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  static_assert(BM == 256 && BN == 64, "bf16_block_work and bf16_pass_geom assume 256-row blocks of 64-key tiles");
  const PairWork pw = bf16_block_work(p, SPLIT, blockIdx.x);
  const int sp = SPLIT ? (int)blockIdx.y : 0, splits = SPLIT ? (int)gridDim.y : 1;
  // Positions and token strides fit 32 bits (the launcher declines otherwise).
  Bf16Pass a;
  a.L = (int)p.seq_q;
  a.S = (int)p.seq_k;
  a.diag = a.S - a.L;
  a.qs1 = (int)p.qs[1];
  a.ks1 = (int)p.ks[1];
  a.vs1 = (int)p.vs[1];
  a.heads = (int)p.heads;
  a.c = p.c;
  a.causal = p.causal;
  a.q = reinterpret_cast<const uint16_t*>(p.q) + pw.b * p.qs[0] + pw.h * p.qs[2];
  a.k = reinterpret_cast<const uint16_t*>(p.k) + pw.b * p.ks[0] + pw.h * p.ks[2];
  a.v = reinterpret_cast<const uint16_t*>(p.v) + pw.b * p.vs[0] + pw.h * p.vs[2];
  a.out = reinterpret_cast<uint16_t*>(p.out) + (pw.b * p.seq_q * p.heads + pw.h) * E;
  const int S = a.S, diag = a.diag;
  int koff[NL], voff[NL];
  tile_offsets<E, FlashBf16Cfg<E>::RSK>(wv, lane, a.ks1, koff);
  tile_offsets<E, FlashBf16Cfg<E>::RSV>(wv, lane, a.vs1, voff);

  P64Rows<E> w;
  w.init(lane);
  auto kbuf = [&](int t) { return Ks + (t % C::NBUFK) * C::TBUF; };
  auto vbuf = [&](int t) { return Vs + (t % C::NBUFV) * C::TBUF; };

  for (int pass = 0; pass < pw.n; ++pass) {
    // The pass's keys [kbeg, kend_b): all it sees, or this block's split of them
    // (whole tiles; a split past the pass's last key is empty).
    const Bf16Geom g = bf16_pass_geom(p, pw, pass, SPLIT, sp, splits);
    const int q0 = g.q0, kbeg = g.kbeg, kend_b = g.kend, nkt = g.nkt;
    w.r0 = q0 + 64 * wv;
    const int nkt_w = bf16_row_tiles(S, diag, p.causal, kbeg, kend_b, w.r0, 64, SPLIT);
    a.q0 = q0;
    a.kend = kend_b;

    if (pass > 0) __syncthreads();  // every wave is done with the previous pass's tiles
    w.issue_q(a);
    // The walk.  K(j) lives in buffer j % 4 and is read by iteration j - 1 (the
    // S of tile j; K(0) by the pass's first S, before iteration 0); V(j) lives
    // in buffer j % 3 and is read by iteration j + 1 (the P.V of tile j).
    // Iteration t issues K(t+3) (into the buffer of K(t-1), last read at t-2)
    // and V(t+1) (into that of V(t-2), last read at t-1), and ends with a block
    // barrier after each wave has waited for all but those loads, so K(t+2) and
    // V(t) have landed when iteration t+1 starts.  Every buffer a load refills
    // was last read before a barrier that the load comes after, whichever wave
    // issues it, and every tile is read only after a barrier that follows its
    // landing.
    TileStream<E> tk, tv;
    tk.init(a.k + (int64_t)kbeg * a.ks1, a.ks1, kend_b - kbeg, Ks, C::NBUFK, 0, wv);
    tv.init(a.v + (int64_t)kbeg * a.vs1, a.vs1, kend_b - kbeg, Vs, C::NBUFV, 0, wv);
    if (nkt > 0) {
      tk.issue(koff);
      tk.issue(koff);
      tk.issue(koff);
      tv.issue(voff);
    }
    w.q_home();
    w.settle();
    bool bad = false;
    if (nkt > 0) {
      loads_landed_barrier<2 * NL>();  // K(0) and K(1) have landed
      auto loads = [&]() __attribute__((always_inline)) {
        tk.issue(koff);
        tv.issue(voff);
      };
      // A tile needs the key limits when a row of the wave ends inside it.
      auto masked = [&](int t) __attribute__((always_inline)) {
        const int k0 = kbeg + t * BN;
        return k0 + BN > S || (p.causal && k0 + BN - 1 > w.r0 + diag);
      };
      int t = 0;
      if (nkt_w > 0) {
        // Tile 0: its S, the row max fixed 64 above its own (never refreshed:
        // the sum of a lane's p over a tile stays below 2^64 unless a later
        // logit exceeds tile 0's max by about 123 in log2 units, which `bad`
        // records for the safe pass), then the softmax of tile 0 beside the S of
        // tile 1.
        w.template step<1, false, true, false>(Vs, kbuf(0), a.c, [] {});
        P64Rows<E>::mfma_guard();
        w.template apply_mask<0>(a, kbeg, 0);
        w.fix_max(a.c);
        bad |= !w.template step<0, false, true, true>(Vs, kbuf(1), a.c, loads);
        loads_landed_barrier<2 * NL>();
        // Tiles 1 .. nkt_w - 1: the P.V of the previous tile, the softmax of
        // this one and the S of the next (past the wave's last tile that S is
        // of a tile it does not use).
        auto body = [&](auto par_tag, int tt) __attribute__((always_inline)) {
          constexpr int PAR = decltype(par_tag)::value;
          if (masked(tt)) w.template apply_mask<PAR>(a, kbeg, tt);
          bad |= !w.template step<PAR, true, true, true>(vbuf(tt + C::NBUFV - 1), kbuf(tt + 1), a.c, loads);
          loads_landed_barrier<2 * NL>();
        };
        for (t = 1; t + 1 < nkt_w; t += 2) {
          body(std::integral_constant<int, 1>{}, t);
          body(std::integral_constant<int, 0>{}, t + 1);
        }
        if (t < nkt_w) {
          body(std::integral_constant<int, 1>{}, t);
          ++t;
        }
        // t == nkt_w: the P.V of the last tile.
        w.template step<0, true, false, false>(vbuf(t + C::NBUFV - 1), Ks, a.c, loads);
        loads_landed_barrier<2 * NL>();
        ++t;
      }
      // Tiles of the block past this wave's rows: loads and barriers only.
      for (; t <= nkt; ++t) {
        loads();
        loads_landed_barrier<2 * NL>();
      }
      __builtin_amdgcn_s_waitcnt(0x0f70);  // the loads past the range (zeros) have landed
    }
    // After the barrier every wave's tile loads have landed and nobody reads the
    // tiles any more: the tile buffers can stage the output.
    bad = __any(bad);
    const bool any_bad = __syncthreads_or(bad);
    static_assert(C::NW * P64Rows<E>::kStageBytes <= C::LDS_BYTES, "the staging areas fit the tile buffers");
    static_assert(C::NW * P64Rows<E>::kPartBytes <= C::LDS_BYTES, "the partials' staging fits the tile buffers");
    if constexpr (SPLIT) {
      const int64_t slot0 = (pw.b * p.heads + pw.h) * p.seq_q * splits + sp;
      if (!bad)
        w.store_partials(a, reinterpret_cast<char*>(smem) + wv * P64Rows<E>::kPartBytes, p.part_acc, p.part_ml,
                         slot0, splits);
      if (any_bad) {
        const SplitOut so{p.part_acc, p.part_ml, slot0, splits, kbeg};
        const Bf16Pass pa = a;
        bf16_safe_pass_p64<E>(pa, bad, so);
      }
    } else {
      if (!bad) w.store_staged(a, reinterpret_cast<char*>(smem) + wv * P64Rows<E>::kStageBytes);
      if (any_bad) {
        // The call takes its arguments through the stack: a copy made only here
        // keeps `a` itself in registers, so the fast path writes no scratch.
        const Bf16Pass pa = a;
        bf16_safe_pass_p64<E>(pa, bad);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp32
// ---------------------------------------------------------------------------
template <int E>
struct FlashF32Cfg {
  static constexpr int BN = 32;
  static constexpr int KS = E + 2;   // K row stride (floats): conflict-free 8-byte reads
  static constexpr int VS = E;
  static constexpr int CH = BN * E / 4 / 256;  // 16-byte chunks per thread (K and V each)
  static constexpr int LDS_K = BN * KS;
  static constexpr int LDS_V = BN * VS;
  static constexpr int LDS_BYTES = 2 * (LDS_K + LDS_V) * 4;
};

// The fp32 kernel's keys for the query block at row q0: [kbeg, kend) in nkt
// tiles of 32, all the block sees or its split sp of splits (whole tiles).
struct F32Keys {
  int64_t kbeg, kend;
  int nkt;
};
__host__ __device__ inline F32Keys f32_keys(const FlashParams& p, int64_t q0, bool split, int sp, int splits) {
  const int64_t S = p.seq_k, diag = p.seq_k - p.seq_q, BN = 32;
  F32Keys k;
  k.kbeg = 0;
  k.kend = p.causal ? (S < q0 + kBM + diag ? S : q0 + kBM + diag) : S;
  if (split) {
    const int64_t chunk = cdiv(cdiv(S, BN), splits) * BN;
    const int64_t lo = k.kend > 0 ? k.kend : 0;
    k.kbeg = sp * chunk < lo ? sp * chunk : lo;
    k.kend = k.kbeg + chunk < k.kend ? k.kbeg + chunk : k.kend;
  }
  k.nkt = k.kend > k.kbeg ? (int)cdiv(k.kend - k.kbeg, BN) : 0;
  return k;
}
// Byte offset of thread tid's 16-byte chunk i of a 32-key tile (rows `stride`
// floats apart), and the window from the tile at key k0 to the tensor's last key.
template <int E>
__host__ __device__ inline int f32_tile_offset(int tid, int i, int64_t stride) {
  const int c = tid + 256 * i;
  const int r = c / (E / 4), c4 = c % (E / 4);
  return (int)((r * stride + 4 * c4) * 4);
}
template <int E>
__host__ __device__ inline int64_t f32_tile_bytes(int64_t S, int64_t k0, int64_t stride) {
  return ((S - 1 - k0) * stride + E) * 4;
}

// SPLIT: blockIdx.y is one of gridDim.y splits of the key range, each a run of
// whole tiles; the block writes unnormalised (O, max, sum) partials of its rows
// for the combine kernel instead of the output.
//
// PAIR (causal calls of many query blocks, pair_blocks()): the block runs the pair
// (qb, nqb-1-qb) one pass after the other, so every block does the same work;
// otherwise one query block, the most expensive causal blocks first.
template <int E, bool SPLIT, bool PAIR>
__global__ __launch_bounds__(256, 2) void flash_f32_kernel(FlashParams p) {
  static_assert(!(SPLIT && PAIR), "split calls are not paired");
  using C = FlashF32Cfg<E>;
  constexpr int BN = C::BN, KS = C::KS, VS = C::VS;
  extern __shared__ __attribute__((aligned(16))) float smemf[];
  float* Ks = smemf;                 // [2][BN][KS]
  float* Vs = smemf + 2 * C::LDS_K;  // [2][BN][VS]

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int li = lane & 31, hf = lane >> 5;
  PairWork pw{};
  if constexpr (PAIR) pw = pair_work(p, kBM, false, blockIdx.x);
#pragma unroll 1
  for (int pass = 0; pass < (PAIR ? pw.n : 1); ++pass) {
  if (PAIR && pass > 0) __syncthreads();  // the first pass's tile buffers are free again
  const BlockWork bw = PAIR ? BlockWork{pw.b, pw.h, (pass ? pw.qb1 : pw.qb0) * kBM} : block_work(p, blockIdx.x);
  const int64_t L = p.seq_q, S = p.seq_k, diag = S - L;
  const float* qg = reinterpret_cast<const float*>(p.q) + bw.b * p.qs[0] + bw.h * p.qs[2];
  const float* kg = reinterpret_cast<const float*>(p.k) + bw.b * p.ks[0] + bw.h * p.ks[2];
  const float* vg = reinterpret_cast<const float*>(p.v) + bw.b * p.vs[0] + bw.h * p.vs[2];

  const int64_t row = bw.q0 + 32 * wv + li;
  const int sp = SPLIT ? (int)blockIdx.y : 0, splits = SPLIT ? (int)gridDim.y : 1;
  const F32Keys kr_ = f32_keys(p, bw.q0, SPLIT, sp, splits);
  const int64_t kbeg = kr_.kbeg;
  // The partial slot of (row, split): O at part_acc[slot * E], (max, sum) at part_ml[2 * slot].
  const int64_t slot = ((bw.b * p.heads + bw.h) * L + row) * splits + sp;
  const int nkt = kr_.nkt;
  if (nkt == 0) {  // every row of the block sees no key of this range: exactly 0
    if (SPLIT && row < L) {
      float* pa = p.part_acc + slot * E;
#pragma unroll
      for (int d = 0; d < E / 2; d += 4) *reinterpret_cast<f32x4*>(pa + (E / 2) * hf + d) = f32x4{0, 0, 0, 0};
      if (hf == 0) {
        p.part_ml[2 * slot] = -INFINITY;
        p.part_ml[2 * slot + 1] = 0.f;
      }
    } else if (row < L) {
      float* og = reinterpret_cast<float*>(p.out) + ((bw.b * L + row) * p.heads + bw.h) * E;
#pragma unroll
      for (int d = 0; d < E / 2; d += 4) *reinterpret_cast<f32x4*>(og + (E / 2) * hf + d) = f32x4{0, 0, 0, 0};
    }
    continue;
  }

  // Q: lane (query li, half hf) holds dims 4t+2hf and 4t+2hf+1.
  float qr[E / 2];
#pragma unroll
  for (int t = 0; t < E / 4; ++t) {
    u32x2 v = {0, 0};
    if (row < L) v = *reinterpret_cast<const u32x2*>(qg + row * p.qs[1] + 4 * t + 2 * hf);
    qr[2 * t] = __uint_as_float(v.x);
    qr[2 * t + 1] = __uint_as_float(v.y);
  }

  const int64_t r0w = bw.q0 + 32 * wv;
  const int64_t kend_w = p.causal ? min<int64_t>(S, r0w + 32 + diag) : S;

  // Global -> register staging through buffer loads rebased at each tile (fixed
  // per-lane offsets; rows past S read as zeros).
  u32x4 kreg[C::CH], vreg[C::CH];
  int koff[C::CH], voff[C::CH];
#pragma unroll
  for (int i = 0; i < C::CH; ++i) {
    koff[i] = f32_tile_offset<E>(tid, i, p.ks[1]);
    voff[i] = f32_tile_offset<E>(tid, i, p.vs[1]);
  }
  auto load_tile = [&](int t) {
    const int64_t k0 = kbeg + (int64_t)t * BN;
    const int64_t kbytes = f32_tile_bytes<E>(S, k0, p.ks[1]), vbytes = f32_tile_bytes<E>(S, k0, p.vs[1]);
    const __amdgpu_buffer_rsrc_t kr = tile_rsrc(kg + k0 * p.ks[1], kbytes);
    const __amdgpu_buffer_rsrc_t vr = tile_rsrc(vg + k0 * p.vs[1], vbytes);
#pragma unroll
    for (int i = 0; i < C::CH; ++i) {
      kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, koff[i], 0, 0);
      vreg[i] = __builtin_amdgcn_raw_buffer_load_b128(vr, voff[i], 0, 0);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < C::CH; ++i) {
      const int c = tid + 256 * i;
      const int r = c / (E / 4), c4 = c % (E / 4);
      float* kd = Ks + buf * C::LDS_K + r * KS + 4 * c4;
      *reinterpret_cast<u32x2*>(kd) = u32x2{kreg[i].x, kreg[i].y};
      *reinterpret_cast<u32x2*>(kd + 2) = u32x2{kreg[i].z, kreg[i].w};
      *reinterpret_cast<u32x4*>(Vs + buf * C::LDS_V + r * VS + 4 * c4) = vreg[i];
    }
  };

  f32x16 oacc[E / 32];
#pragma unroll
  for (int d = 0; d < E / 32; ++d) oacc[d] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;
  const float c = p.c;

  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int t = 0; t < nkt; ++t) {
    const int buf = t & 1;
    load_tile(t + 1);  // past the last tile: never used (range-checked zeros past S)
    const int64_t k0 = kbeg + (int64_t)t * BN;
    if (k0 < kend_w) {
      const float* kb = Ks + buf * C::LDS_K;
      const float* vb = Vs + buf * C::LDS_V;
      f32x16 st = f32x16{};
#pragma unroll
      for (int t4 = 0; t4 < E / 4; ++t4) {
        const u32x2 a = *reinterpret_cast<const u32x2*>(kb + li * KS + 4 * t4 + 2 * hf);
        st = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), qr[2 * t4], st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), qr[2 * t4 + 1], st, 0, 0, 0);
      }
      const bool need_mask = (k0 + BN > S) || (p.causal && k0 + BN - 1 > r0w + diag);
      const int64_t lim = r0w + li + diag;
      float x[16];
      float mt = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = st[r] * c;
        if (need_mask) {
          const int64_t j = k0 + 8 * (r >> 2) + 4 * hf + (r & 3);
          if (j >= S || (p.causal && j > lim)) v = -INFINITY;
        }
        x[r] = v;
        mt = fmaxf(mt, v);
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32));
      const float m_new = fmaxf(m_run, mt);
      const float mu = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - mu);
      m_run = m_new;
      float ls = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        x[r] = __builtin_amdgcn_exp2f(x[r] - mu);
        ls += x[r];
      }
      l_run = l_run * alpha + ls;
#pragma unroll
      for (int d = 0; d < E / 32; ++d) oacc[d] *= alpha;
      // O^T += V^T P^T, two keys per step: step r takes key 8(r/4)+4hf+r%4.
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * hf + (r & 3);
#pragma unroll
        for (int d = 0; d < E / 32; ++d)
          oacc[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(vb[key * VS + 32 * d + li], x[r], oacc[d], 0, 0, 0);
      }
    }
    store_tile(buf ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if constexpr (SPLIT) {
    if (row < L) {
      float* pa = p.part_acc + slot * E;
#pragma unroll
      for (int d = 0; d < E / 32; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4*>(pa + 32 * d + 8 * g + 4 * hf) =
              f32x4{oacc[d][4 * g], oacc[d][4 * g + 1], oacc[d][4 * g + 2], oacc[d][4 * g + 3]};
      if (hf == 0) {
        p.part_ml[2 * slot] = m_run;
        p.part_ml[2 * slot + 1] = l_tot;
      }
    }
    continue;
  }
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row < L) {
    float* og = reinterpret_cast<float*>(p.out) + ((bw.b * L + row) * p.heads + bw.h) * E;
#pragma unroll
    for (int d = 0; d < E / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4*>(og + 32 * d + 8 * g + 4 * hf) =
            f32x4{oacc[d][4 * g] * inv, oacc[d][4 * g + 1] * inv, oacc[d][4 * g + 2] * inv,
                  oacc[d][4 * g + 3] * inv};
  }
  }  // passes
}

template <typename K>
static int launch_lds(K kernel, int64_t nb, int threads, int lds, const FlashParams& p, hipStream_t stream,
                      int64_t ny = 1) {
  if (nb > 0x7fffffff || ny > 0xffff) return CA_DECLINED;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return CA_HIP_ERROR - (int)e;
  }
  hipLaunchKernelGGL(kernel, dim3((unsigned)nb, (unsigned)ny), dim3(threads), lds, stream, p);
  return ca_launch_status();
}

FlashPlan flash_plan(const FlashParams& p, int E, bool bf16) {
  FlashPlan plan{};
  if (p.batch * p.heads * p.seq_q == 0) {
    plan.kind = kPlanNone;
    return plan;
  }
  if (E != 32 && E != 64 && E != 128) return plan;
  // The tile loads address a tile's rows with 32-bit byte offsets from its first
  // row: 64 rows of the token stride must fit (larger strides are declined and
  // the caller copies the tensor).
  const int64_t esz = bf16 ? 2 : 4;
  int64_t ts = p.ks[1] > p.vs[1] ? p.ks[1] : p.vs[1];
  if (p.qs[1] > ts) ts = p.qs[1];
  if (p.qs[1] < 0 || p.ks[1] < 0 || p.vs[1] < 0 || 64 * (ts + E) * esz >= ((int64_t)1 << 31)) return plan;
  // Row and key positions are 32-bit inside the kernels.
  if (p.seq_q >= ((int64_t)1 << 30) || p.seq_k >= ((int64_t)1 << 30)) return plan;
  if (rows_route(p.batch, p.seq_q, p.heads, bf16)) return rows_plan(p, E, bf16);
  // The short-key kernel addresses K and V rows by 32-bit byte offsets from the
  // (batch, head) base: seq_k rows of the token stride must fit (64 do, above).
  if (small_route(p.batch, p.seq_q, p.seq_k, p.heads, E, bf16) && p.seq_k * (ts + E) * esz < ((int64_t)1 << 32))
    return small_plan(p);
  // Split mode: one block per (batch, head, query block) and split of its keys,
  // then the combine of each row's partials into the output.  Otherwise one
  // block per (batch, head) and query-block pair (causal) or query block.
  plan.kind = bf16 ? kPlanBf16 : kPlanF32;
  plan.splits = tiled_splits(p.batch, p.seq_q, p.seq_k, p.heads, bf16, p.causal != 0);
  plan.need = tiled_workspace_bytes(p.batch, p.seq_q, p.seq_k, p.heads, E, bf16, p.causal != 0);
  plan.split = plan.splits > 1;
  plan.gy = plan.splits;
  const int64_t nqb = cdiv(p.seq_q, bf16 ? 256 : kBM);
  plan.pair = !plan.split && pair_blocks(p, nqb, bf16);
  plan.gx = p.batch * p.heads * (plan.pair ? (nqb + 1) / 2 : nqb);
  if (plan.gx > 0x7fffffff || plan.gy > 0xffff) plan.kind = kPlanDeclined;
  return plan;
}

int flash_launch(const FlashParams& p, int E, int bf16, hipStream_t stream) {
  const FlashPlan plan = flash_plan(p, E, bf16 != 0);
  if (plan.kind == kPlanNone) return CA_OK;
  if (plan.kind == kPlanDeclined) return CA_DECLINED;
  if (plan.need > 0 && (p.part_acc == nullptr || p.part_ml == nullptr || p.workspace_bytes < plan.need))
    return CA_DECLINED;
  if (plan.kind == kPlanRows || plan.kind == kPlanRowsHeads) return flash_rows_launch(p, plan, E, bf16, stream);
  if (plan.kind == kPlanSmall) return flash_small_launch(p, plan, E, stream);
  const int64_t nb = plan.gx, splits = plan.splits;
  if (bf16) {
    if (plan.split) {
      int st = CA_DECLINED;
      switch (E) {
        case 32: st = launch_lds(flash_bf16_p64_kernel<32, true>, nb, 64 * FlashP64Cfg<32>::NW, FlashP64Cfg<32>::LDS_BYTES, p, stream, splits); break;
        case 64: st = launch_lds(flash_bf16_p64_kernel<64, true>, nb, 64 * FlashP64Cfg<64>::NW, FlashP64Cfg<64>::LDS_BYTES, p, stream, splits); break;
        case 128: st = launch_lds(flash_bf16_p64_kernel<128, true>, nb, 64 * FlashP64Cfg<128>::NW, FlashP64Cfg<128>::LDS_BYTES, p, stream, splits); break;
      }
      if (st != CA_OK) return st;
      return flash_combine_launch(p, E, bf16, splits, stream);
    }
    switch (E) {
      case 32: return launch_lds(flash_bf16_p64_kernel<32, false>, nb, 64 * FlashP64Cfg<32>::NW, FlashP64Cfg<32>::LDS_BYTES, p, stream);
      case 64: return launch_lds(flash_bf16_p64_kernel<64, false>, nb, 64 * FlashP64Cfg<64>::NW, FlashP64Cfg<64>::LDS_BYTES, p, stream);
      case 128: return launch_lds(flash_bf16_p64_kernel<128, false>, nb, 64 * FlashP64Cfg<128>::NW, FlashP64Cfg<128>::LDS_BYTES, p, stream);
    }
  } else {
    if (plan.split) {
      int st = CA_DECLINED;
      switch (E) {
        case 32: st = launch_lds(flash_f32_kernel<32, true, false>, nb, 256, FlashF32Cfg<32>::LDS_BYTES, p, stream, splits); break;
        case 64: st = launch_lds(flash_f32_kernel<64, true, false>, nb, 256, FlashF32Cfg<64>::LDS_BYTES, p, stream, splits); break;
        case 128: st = launch_lds(flash_f32_kernel<128, true, false>, nb, 256, FlashF32Cfg<128>::LDS_BYTES, p, stream, splits); break;
      }
      if (st != CA_OK) return st;
      return flash_combine_launch(p, E, bf16, splits, stream);
    }
    if (plan.pair) {
      switch (E) {
        case 32: return launch_lds(flash_f32_kernel<32, false, true>, nb, 256, FlashF32Cfg<32>::LDS_BYTES, p, stream);
        case 64: return launch_lds(flash_f32_kernel<64, false, true>, nb, 256, FlashF32Cfg<64>::LDS_BYTES, p, stream);
        case 128: return launch_lds(flash_f32_kernel<128, false, true>, nb, 256, FlashF32Cfg<128>::LDS_BYTES, p, stream);
      }
      return CA_DECLINED;
    }
    switch (E) {
      case 32: return launch_lds(flash_f32_kernel<32, false, false>, nb, 256, FlashF32Cfg<32>::LDS_BYTES, p, stream);
      case 64: return launch_lds(flash_f32_kernel<64, false, false>, nb, 256, FlashF32Cfg<64>::LDS_BYTES, p, stream);
      case 128: return launch_lds(flash_f32_kernel<128, false, false>, nb, 256, FlashF32Cfg<128>::LDS_BYTES, p, stream);
    }
  }
  return CA_DECLINED;
}

}  // namespace ca
