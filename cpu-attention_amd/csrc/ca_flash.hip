// flash_attn_func forward on CDNA4 matrix cores.
//
// Semantics follow the reference's prefill driver (cpu_attention/_mojo/src/flash_attn.mojo:
// 127-183): causal is bottom-right aligned (row i sees keys j <= i + S - L), key
// tiles past the last visible key are never touched, the online softmax runs in
// base 2 with c = scale*log2(e), and a row that sees no key is exactly 0.
//
// Block = 4 waves x 32 query rows.  Each wave keeps its Q rows in registers and
// walks the key range in tiles staged through LDS (double-buffered; the next tile's
// buffer loads are in flight while the current one is consumed, one barrier per
// tile).  The loop body is branch-free around the loads: a conditional prefetch
// made the compiler wait for it before the first MFMA of every tile.
//
//   S^T = K Q^T   32x32 MFMA tiles with keys as rows and queries as columns, so a
//                 lane ends up owning one query and 16 keys of each tile;
//   softmax       per lane (its query), with one cross-half exchange for the row max;
//   O^T += V^T P^T the probabilities are already in the B-operand layout of the next
//                 MFMA (no LDS round trip); V^T comes from LDS, where it is stored
//                 transposed with bits 2 and 3 of the key index swapped so each lane's
//                 8 keys are one 16-byte read.
//
// bf16: v_mfma_f32_32x32x16_bf16, P rounded to bf16 for P.V (as the reference's
// bf16 policy does, flash_vec.mojo:255-259), fp32 accumulation.
// fp32: v_mfma_f32_32x32x2_f32, everything fp32.
#include "ca_device.h"
#include "ca_internal.h"

namespace ca {

constexpr int kBM = 128;  // query rows per block (4 waves x 32)

// A raw buffer resource over [base, base + bytes): loads past `bytes` return 0.
// The per-tile K/V loads rebase the resource at each tile, so their per-lane
// offsets stay fixed across the loop (no address registers rewritten under
// in-flight loads) and rows past the last key come back as zeros.
// A tile that starts past the last key (the prefetch after the last tile) has a
// negative byte count: it becomes an empty window, where every load reads zero
// without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int64_t bytes) {
  const int64_t n = bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

// Hardware dispatches workgroup i to XCD i % 8.  Remap so each XCD walks a
// contiguous range of (batch*head, query block) work: one head's K/V stays in
// that XCD's L2 while its query blocks run.
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t nb) {
  const int64_t x = bid & 7, slot = bid >> 3;
  const int64_t per = nb >> 3, rem = nb & 7;
  return x * per + (x < rem ? x : rem) + slot;
}

struct BlockWork {
  int64_t b, h, q0;
};

__device__ __forceinline__ BlockWork block_work(const FlashParams& p) {
  const int64_t nqb = cdiv(p.seq_q, kBM);
  const int64_t nb = p.batch * p.heads * nqb;
  const int64_t lg = xcd_remap(blockIdx.x, nb);
  const int64_t bh = lg / nqb;
  const int64_t qb = nqb - 1 - (lg - bh * nqb);  // the most expensive causal blocks first
  BlockWork w;
  w.b = bh / p.heads;
  w.h = bh - w.b * p.heads;
  w.q0 = qb * kBM;
  return w;
}

// ---------------------------------------------------------------------------
// bf16
// ---------------------------------------------------------------------------
template <int E>
struct FlashBf16Cfg {
  static constexpr int BN = 64;          // keys per tile
  static constexpr int KS = E + 8;       // K row stride in LDS (elements): conflict-free reads
  static constexpr int VS = BN + 8;      // V^T row stride
  static constexpr int KCH = BN * E / 8 / 256;  // 16-byte K chunks per thread
  static constexpr int VBLK = (BN / 4) * (E / 8);  // 4-key x 8-dim V blocks per tile
  static constexpr int LDS_K = BN * KS;  // elements per K buffer
  static constexpr int LDS_V = E * VS;
  static constexpr int LDS_BYTES = 2 * (LDS_K + LDS_V) * 2;
};

// Position of key k (0..63) in a V^T row: bits 2 and 3 swapped.
__device__ __forceinline__ int vt_pos(int k) {
  return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
}

template <int E>
__global__ __launch_bounds__(256, 2) void flash_bf16_kernel(FlashParams p) {
  using C = FlashBf16Cfg<E>;
  constexpr int BN = C::BN, KS = C::KS, VS = C::VS;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* Ks = smem;                  // [2][BN][KS]
  uint16_t* Vt = smem + 2 * C::LDS_K;   // [2][E][VS]

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int li = lane & 31, hf = lane >> 5;
  const BlockWork bw = block_work(p);
  const int64_t L = p.seq_q, S = p.seq_k, diag = S - L;
  const uint16_t* qg = reinterpret_cast<const uint16_t*>(p.q) + bw.b * p.qs[0] + bw.h * p.qs[2];
  const uint16_t* kg = reinterpret_cast<const uint16_t*>(p.k) + bw.b * p.ks[0] + bw.h * p.ks[2];
  const uint16_t* vg = reinterpret_cast<const uint16_t*>(p.v) + bw.b * p.vs[0] + bw.h * p.vs[2];

  const int64_t row = bw.q0 + 32 * wv + li;
  const int64_t kend_blk = p.causal ? min<int64_t>(S, bw.q0 + kBM + diag) : S;
  const int nkt = kend_blk > 0 ? (int)cdiv(kend_blk, BN) : 0;
  if (nkt == 0) {  // every row of the block sees no key: exactly 0
    if (row < L) {
      uint16_t* og = reinterpret_cast<uint16_t*>(p.out) + ((bw.b * L + row) * p.heads + bw.h) * E;
#pragma unroll
      for (int d = 0; d < E / 2; d += 8) *reinterpret_cast<u32x4*>(og + (E / 2) * hf + d) = u32x4{0, 0, 0, 0};
    }
    return;
  }

  // Q rows of this wave as B operands: lane (query li, half hf) holds dims 16s+8hf..+7.
  bf16x8 qr[E / 16];
#pragma unroll
  for (int s = 0; s < E / 16; ++s) {
    u32x4 v = {0, 0, 0, 0};
    if (row < L) v = *reinterpret_cast<const u32x4*>(qg + row * p.qs[1] + 16 * s + 8 * hf);
    qr[s] = __builtin_bit_cast(bf16x8, v);
  }

  const int64_t r0w = bw.q0 + 32 * wv;  // first row of this wave
  const int64_t kend_w = p.causal ? min<int64_t>(S, r0w + 32 + diag) : S;

  // Global -> register staging of one K/V tile through buffer loads: fixed per-lane
  // byte offsets, the resource rebased at the tile; rows past S read as zeros.
  u32x4 kreg[C::KCH];
  u32x4 vreg[4];
  int koff[C::KCH], voff[4];
#pragma unroll
  for (int i = 0; i < C::KCH; ++i) {
    const int c = tid + 256 * i;
    koff[i] = (int)(((c / (E / 8)) * p.ks[1] + 8 * (c % (E / 8))) * 2);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) voff[r] = (int)(((4 * (tid & 15) + r) * p.vs[1] + 8 * (tid >> 4)) * 2);
  auto load_tile = [&](int t) {
    const int64_t k0 = (int64_t)t * BN;
    const int64_t kbytes = ((S - 1 - k0) * p.ks[1] + E) * 2, vbytes = ((S - 1 - k0) * p.vs[1] + E) * 2;
    const __amdgpu_buffer_rsrc_t kr = tile_rsrc(kg + k0 * p.ks[1], kbytes);
    const __amdgpu_buffer_rsrc_t vr = tile_rsrc(vg + k0 * p.vs[1], vbytes);
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, koff[i], 0, 0);
    if (C::VBLK >= 256 || tid < C::VBLK) {
#pragma unroll
      for (int r = 0; r < 4; ++r) vreg[r] = __builtin_amdgcn_raw_buffer_load_b128(vr, voff[r], 0, 0);
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* kb = Ks + buf * C::LDS_K;
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) {
      const int c = tid + 256 * i;
      const int r = c / (E / 8), c8 = c % (E / 8);
      *reinterpret_cast<u32x4*>(kb + r * KS + 8 * c8) = kreg[i];
    }
    if (C::VBLK >= 256 || tid < C::VBLK) {
      const int kgp = tid & 15, dc = tid >> 4;
      uint16_t* vb = Vt + buf * C::LDS_V + (8 * dc) * VS + vt_pos(4 * kgp);
      const uint32_t w0[4] = {vreg[0].x, vreg[0].y, vreg[0].z, vreg[0].w};
      const uint32_t w1[4] = {vreg[1].x, vreg[1].y, vreg[1].z, vreg[1].w};
      const uint32_t w2[4] = {vreg[2].x, vreg[2].y, vreg[2].z, vreg[2].w};
      const uint32_t w3[4] = {vreg[3].x, vreg[3].y, vreg[3].z, vreg[3].w};
#pragma unroll
      for (int d2 = 0; d2 < 4; ++d2) {
        // dims 2*d2 (low halves) and 2*d2+1 (high halves) of keys 0..3
        u32x2 lo = {(w0[d2] & 0xffffu) | (w1[d2] << 16), (w2[d2] & 0xffffu) | (w3[d2] << 16)};
        u32x2 hi = {(w0[d2] >> 16) | (w1[d2] & 0xffff0000u), (w2[d2] >> 16) | (w3[d2] & 0xffff0000u)};
        *reinterpret_cast<u32x2*>(vb + (2 * d2) * VS) = lo;
        *reinterpret_cast<u32x2*>(vb + (2 * d2 + 1) * VS) = hi;
      }
    }
  };

  f32x16 oacc[E / 32];
#pragma unroll
  for (int d = 0; d < E / 32; ++d) oacc[d] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;
  const float c = p.c;

  if (nkt > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();
  for (int t = 0; t < nkt; ++t) {
    const int buf = t & 1;
    load_tile(t + 1);  // past the last tile: range-checked zeros, never used
    const int64_t k0 = (int64_t)t * BN;
    if (k0 < kend_w) {
      const uint16_t* kb = Ks + buf * C::LDS_K;
      const uint16_t* vb = Vt + buf * C::LDS_V;
      // S^T tiles: keys 0-31 and 32-63 of the tile.  All 2*E/16 A operands are read
      // from LDS first, then the two accumulator chains are interleaved.
      bf16x8 ka[2][E / 16];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int s = 0; s < E / 16; ++s)
          ka[kt][s] = *reinterpret_cast<const bf16x8*>(kb + (32 * kt + li) * KS + 16 * s + 8 * hf);
      f32x16 st[2] = {f32x16{}, f32x16{}};
#pragma unroll
      for (int s = 0; s < E / 16; ++s)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
          st[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[kt][s], qr[s], st[kt], 0, 0, 0);
      // Online softmax for query row r0w+li over the 32 keys this lane holds: raw
      // logits (masked keys -inf), row max in scaled log2 units as the reference
      // takes it (tile max of the raw logits times c), p = 2^(s*c - m) with the
      // scale folded into one FMA.  The running max is refreshed lazily: only when
      // some row's tile max exceeds it by more than 8 (p stays below 2^8), which
      // skips the accumulator rescale on most tiles; acc/l cancels it exactly.
      const bool need_mask = (k0 + BN > S) || (p.causal && k0 + BN - 1 > r0w + diag);
      float mt = -INFINITY;
      if (need_mask) {
        const int64_t lim = r0w + li + diag;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t j = k0 + 32 * kt + 8 * (r >> 2) + 4 * hf + (r & 3);
            if (j >= S || (p.causal && j > lim)) st[kt][r] = -INFINITY;
          }
      }
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, st[kt][r]);
      mt = fmaxf(mt, __shfl_xor(mt, 32)) * c;
      if (__any(mt > m_run + 8.f)) {
        const float m_new = fmaxf(m_run, mt);
        const float alpha = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.f : m_new));
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < E / 32; ++d) oacc[d] *= alpha;
        m_run = m_new;
      }
      const float mu = m_run == -INFINITY ? 0.f : m_run;
      float ls = 0.f;
      bf16x8 pb[4];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        uint32_t w[4];
#pragma unroll
        for (int jj = 0; jj < 8; jj += 2) {
          const float e0 = __builtin_amdgcn_exp2f(fmaf(st[cc >> 1][8 * (cc & 1) + jj], c, -mu));
          const float e1 = __builtin_amdgcn_exp2f(fmaf(st[cc >> 1][8 * (cc & 1) + jj + 1], c, -mu));
          ls += e0 + e1;
          w[jj / 2] = pack_bf16x2(e0, e1);
        }
        pb[cc] = __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
      }
      l_run += ls;
      // O^T += V^T P^T: all V^T operands read first, then E/32 independent chains.
      bf16x8 va[4][E / 32];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
#pragma unroll
        for (int d = 0; d < E / 32; ++d)
          va[cc][d] = *reinterpret_cast<const bf16x8*>(vb + (32 * d + li) * VS + 16 * cc + 8 * hf);
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
#pragma unroll
        for (int d = 0; d < E / 32; ++d)
          oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[cc][d], pb[cc], oacc[d], 0, 0, 0);
    }
    store_tile(buf ^ 1);  // past the last tile: zeros into the idle buffer
    __syncthreads();
  }

  // Epilogue: out = acc / l; a row with no visible key is 0.
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row < L) {
    uint16_t* og = reinterpret_cast<uint16_t*>(p.out) + ((bw.b * L + row) * p.heads + bw.h) * E;
#pragma unroll
    for (int d = 0; d < E / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 w = {pack_bf16x2(oacc[d][4 * g] * inv, oacc[d][4 * g + 1] * inv),
                   pack_bf16x2(oacc[d][4 * g + 2] * inv, oacc[d][4 * g + 3] * inv)};
        *reinterpret_cast<u32x2*>(og + 32 * d + 8 * g + 4 * hf) = w;
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

template <int E>
__global__ __launch_bounds__(256, 2) void flash_f32_kernel(FlashParams p) {
  using C = FlashF32Cfg<E>;
  constexpr int BN = C::BN, KS = C::KS, VS = C::VS;
  extern __shared__ __attribute__((aligned(16))) float smemf[];
  float* Ks = smemf;                 // [2][BN][KS]
  float* Vs = smemf + 2 * C::LDS_K;  // [2][BN][VS]

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int li = lane & 31, hf = lane >> 5;
  const BlockWork bw = block_work(p);
  const int64_t L = p.seq_q, S = p.seq_k, diag = S - L;
  const float* qg = reinterpret_cast<const float*>(p.q) + bw.b * p.qs[0] + bw.h * p.qs[2];
  const float* kg = reinterpret_cast<const float*>(p.k) + bw.b * p.ks[0] + bw.h * p.ks[2];
  const float* vg = reinterpret_cast<const float*>(p.v) + bw.b * p.vs[0] + bw.h * p.vs[2];

  const int64_t row = bw.q0 + 32 * wv + li;
  const int64_t kend_blk = p.causal ? min<int64_t>(S, bw.q0 + kBM + diag) : S;
  const int nkt = kend_blk > 0 ? (int)cdiv(kend_blk, BN) : 0;
  if (nkt == 0) {  // every row of the block sees no key: exactly 0
    if (row < L) {
      float* og = reinterpret_cast<float*>(p.out) + ((bw.b * L + row) * p.heads + bw.h) * E;
#pragma unroll
      for (int d = 0; d < E / 2; d += 4) *reinterpret_cast<f32x4*>(og + (E / 2) * hf + d) = f32x4{0, 0, 0, 0};
    }
    return;
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
    const int c = tid + 256 * i;
    const int r = c / (E / 4), c4 = c % (E / 4);
    koff[i] = (int)((r * p.ks[1] + 4 * c4) * 4);
    voff[i] = (int)((r * p.vs[1] + 4 * c4) * 4);
  }
  auto load_tile = [&](int t) {
    const int64_t k0 = (int64_t)t * BN;
    const int64_t kbytes = ((S - 1 - k0) * p.ks[1] + E) * 4, vbytes = ((S - 1 - k0) * p.vs[1] + E) * 4;
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
    load_tile(t + 1);  // past the last tile: range-checked zeros, never used
    const int64_t k0 = (int64_t)t * BN;
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
}

template <typename K>
static int launch_lds(K kernel, int64_t nb, int lds, const FlashParams& p, hipStream_t stream) {
  if (nb > 0x7fffffff) return CA_DECLINED;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return CA_HIP_ERROR - (int)e;
  }
  hipLaunchKernelGGL(kernel, dim3((unsigned)nb), dim3(256), lds, stream, p);
  return ca_launch_status();
}

int flash_launch(const FlashParams& p, int E, int bf16, hipStream_t stream) {
  const int64_t nb = p.batch * p.heads * cdiv(p.seq_q, kBM);
  if (nb == 0) return CA_OK;
  // The tile loads address a tile's rows with 32-bit byte offsets from its first
  // row: 64 rows of the token stride must fit (larger strides are declined and
  // the caller copies the tensor).
  const int64_t esz = bf16 ? 2 : 4;
  const int64_t ts = p.ks[1] > p.vs[1] ? p.ks[1] : p.vs[1];
  if (ts < 0 || 64 * (ts + E) * esz >= ((int64_t)1 << 31)) return CA_DECLINED;
  if (bf16) {
    switch (E) {
      case 32: return launch_lds(flash_bf16_kernel<32>, nb, FlashBf16Cfg<32>::LDS_BYTES, p, stream);
      case 64: return launch_lds(flash_bf16_kernel<64>, nb, FlashBf16Cfg<64>::LDS_BYTES, p, stream);
      case 128: return launch_lds(flash_bf16_kernel<128>, nb, FlashBf16Cfg<128>::LDS_BYTES, p, stream);
    }
  } else {
    switch (E) {
      case 32: return launch_lds(flash_f32_kernel<32>, nb, FlashF32Cfg<32>::LDS_BYTES, p, stream);
      case 64: return launch_lds(flash_f32_kernel<64>, nb, FlashF32Cfg<64>::LDS_BYTES, p, stream);
      case 128: return launch_lds(flash_f32_kernel<128>, nb, FlashF32Cfg<128>::LDS_BYTES, p, stream);
    }
  }
  return CA_DECLINED;
}

}  // namespace ca
