// flash_attn_func for calls with few query rows (rows_route(): up to 4 rows in
// bf16; in fp32 up to 8, or 16 with 256 or more (batch, head) pairs): split-K
// over key chunks.
//
// With few rows the matrix cores have almost nothing to do; the call is bound by
// reading K and V once (about one FLOP per byte).  The reference routes such
// calls to its vector policy (cpu_attention/_mojo/src/_C.mojo:216-229); the
// numerics here are that policy's (flash_vec.mojo:216-356): logits q.k in fp32
// from exact bf16 products, base-2 online softmax with c = scale*log2(e) and the
// max in scaled log2 units, P rounded to bf16 for P.V on bf16 inputs (fp32 P on
// fp32 inputs) against exactly widened V, l summed from the unrounded p, and a
// row that sees no key is exactly 0.  Causal is bottom-right aligned (query i
// sees keys j <= i + seq_k - seq_q, flash_attn.mojo:143-170).
//
// Work split.  A block of 8 waves takes one (batch, head, group of R query rows)
// (R = 1 for single-row calls, else 4) and walks that group's key chunks: wave w
// takes chunks w, w + 8, ..., with the next chunks' loads in flight (a ring of 3
// chunk buffers for R = 1, 2 otherwise) while it folds the current one into a
// per-lane online softmax.  Lanes cut each K/V row into 16-byte slices: G lanes
// per key, 64/G keys per load instruction, so every load instruction reads whole
// rows; a lane's partial dot product is summed over its G lanes with DPP moves.
// The waves' states merge in LDS at the end, and the block writes the rows.  Only
// when the row groups are too few to fill the chip are a group's chunks also
// split over several blocks; those leave partials (max, sum, P.V) in the caller's
// workspace for the combine kernel.
#include "ca_device.h"
#include "ca_internal.h"

namespace ca {

template <int E, bool BF, int R_>
struct RowsShape {
  static constexpr int ES = BF ? 2 : 4;    // element bytes
  static constexpr int DPL = 16 / ES;      // elements per lane slice
  static constexpr int G = E / DPL;        // lanes per key
  static constexpr int KPI = kWave / G;    // keys per load instruction
  static constexpr int NSTEP = 4;          // load instructions per chunk (K and V each)
  static constexpr int CH = NSTEP * KPI;   // keys per chunk
  static constexpr int R = R_;             // query rows per wave
  static constexpr int NBUF = R == 1 ? 3 : 2;  // chunks in flight per wave
};

constexpr int kRowsLoadSteps = 4;  // RowsShape::NSTEP

__host__ __device__ inline int64_t rows_chunk_keys(int E, bool bf16) {
  const int dpl = bf16 ? 8 : 4;
  return (int64_t)kRowsLoadSteps * (kWave / (E / dpl));
}

// Query rows per wave: one for single-row calls (the deepest load ring fits),
// kRowsPerWaveMany from kRowsManyMinL rows (fp32 only: bf16 calls of more than 4
// rows take the tiled kernel), else kRowsPerWave.
__host__ __device__ inline int rows_per_wave(int64_t seq_q) {
  return seq_q == 1 ? 1 : (seq_q >= kRowsManyMinL ? kRowsPerWaveMany : kRowsPerWave);
}

// Keys row i may see: [0, kend).
__host__ __device__ inline int64_t rows_kend(const FlashParams& p, int64_t i) {
  if (!p.causal) return p.seq_k;
  const int64_t e = i + 1 + p.seq_k - p.seq_q;
  return e < 0 ? 0 : (e < p.seq_k ? e : p.seq_k);
}

// Block (bx of gx, split of gy) of the per-head kernel with R rows per group:
// (batch b, head h), rows [i0, i0 + nr), whose widest key range is kend_g keys in
// nch chunks of ch.  With one split, neighbouring (batch, head) pairs share an
// XCD (E = 32 bf16 rows are half a 128-byte line; the other half is the next
// head's).
struct RowsWork {
  int64_t b, h, i0, kend_g, nch;
  int nr;
};
__host__ __device__ inline RowsWork rows_work(const FlashParams& p, int R, int ch, int64_t bx, int64_t gx, int64_t gy) {
  const int64_t ngroups = cdiv(p.seq_q, R);
  const int64_t lb = gy == 1 ? xcd_remap(bx, gx) : bx;
  const int64_t bh = lb / ngroups, rg = lb - bh * ngroups;
  RowsWork w;
  w.b = bh / p.heads;
  w.h = bh - w.b * p.heads;
  w.i0 = rg * R;
  w.nr = (int)(p.seq_q - w.i0 < R ? p.seq_q - w.i0 : R);
  w.kend_g = rows_kend(p, w.i0 + w.nr - 1);
  w.nch = cdiv(w.kend_g, ch);
  return w;
}

// Sum over aligned groups of G lanes; every lane of a group ends with the same
// bits (each step adds two equal-order operands, and fp32 addition commutes).
template <int G>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (G >= 2)
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));  // quad_perm 1,0,3,2
  if constexpr (G >= 4)
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));  // quad_perm 2,3,0,1
  if constexpr (G >= 8)
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false));  // row_half_mirror
  if constexpr (G >= 16)
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xf, 0xf, false));  // row_mirror
  if constexpr (G >= 32) x += __shfl_xor(x, 16);
  return x;
}

// Partial dot product of a 16-byte K slice with the matching q slice.
template <bool BF>
__device__ __forceinline__ float slice_dot(const u32x4& k, const u32x4& q) {
  if constexpr (BF) {
    float a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k.x), as_bf16x2(q.x), 0.f, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k.y), as_bf16x2(q.y), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k.z), as_bf16x2(q.z), a, false);
    return __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k.w), as_bf16x2(q.w), a, false);
  } else {
    float a = __uint_as_float(k.x) * __uint_as_float(q.x);
    a = fmaf(__uint_as_float(k.y), __uint_as_float(q.y), a);
    a = fmaf(__uint_as_float(k.z), __uint_as_float(q.z), a);
    return fmaf(__uint_as_float(k.w), __uint_as_float(q.w), a);
  }
}

// acc += p * v over one 16-byte V slice (V widened exactly).
template <bool BF>
__device__ __forceinline__ void slice_pv(float* acc, float p, const u32x4& v) {
  if constexpr (BF) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = fmaf(p, bf16_lo(w[i]), acc[2 * i]);
      acc[2 * i + 1] = fmaf(p, bf16_hi(w[i]), acc[2 * i + 1]);
    }
  } else {
    acc[0] = fmaf(p, __uint_as_float(v.x), acc[0]);
    acc[1] = fmaf(p, __uint_as_float(v.y), acc[1]);
    acc[2] = fmaf(p, __uint_as_float(v.z), acc[2]);
    acc[3] = fmaf(p, __uint_as_float(v.w), acc[3]);
  }
}

// Online-softmax state of one lane for one query row over the keys it has
// folded: m (scaled log2 units), l and acc (its slice of P.V).  Lanes of one key
// group see the same keys, so they hold the same m and l.
template <int DPL>
struct RowAcc {
  float m, l, acc[DPL];
};

// Merges state o into st (either may be empty: m = -inf, l = 0, acc = 0).
template <int DPL>
__device__ __forceinline__ void merge_state(RowAcc<DPL>& st, float om, float ol, const float (&oacc)[DPL]) {
  const float mn = fmaxf(st.m, om);
  if (mn == -INFINITY) return;
  const float a = __builtin_amdgcn_exp2f(st.m - mn), b = __builtin_amdgcn_exp2f(om - mn);
  st.l = st.l * a + ol * b;
#pragma unroll
  for (int d = 0; d < DPL; ++d) st.acc[d] = st.acc[d] * a + oacc[d] * b;
  st.m = mn;
}

template <int E, bool BF>
__device__ __forceinline__ void load_chunk(const char* kb, const char* vb, const FlashParams& p, int64_t j0,
                                           int64_t kend_g, int kl, int sl, u32x4 (&kk)[RowsShape<E, BF, 1>::NSTEP],
                                           u32x4 (&vv)[RowsShape<E, BF, 1>::NSTEP]) {
  using S = RowsShape<E, BF, 1>;
#pragma unroll
  for (int s = 0; s < S::NSTEP; ++s) {
    const int64_t j = j0 + s * S::KPI + kl;
    kk[s] = u32x4{0u, 0u, 0u, 0u};
    vv[s] = u32x4{0u, 0u, 0u, 0u};
    if (j < kend_g) {
      kk[s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kb + (j * p.ks[1] + sl * S::DPL) * S::ES));
      vv[s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vb + (j * p.vs[1] + sl * S::DPL) * S::ES));
    }
  }
}

// Folds one chunk (keys j0 ..) into a row's per-lane state: the lane's running
// max moves at most once per chunk, and no value crosses key groups.
template <int E, bool BF>
__device__ __forceinline__ void fold_chunk(const FlashParams& p, const u32x4 (&kk)[RowsShape<E, BF, 1>::NSTEP],
                                           const u32x4 (&vv)[RowsShape<E, BF, 1>::NSTEP], const u32x4& q, int64_t j0,
                                           int64_t kend, int kl, RowAcc<RowsShape<E, BF, 1>::DPL>& st) {
  using S = RowsShape<E, BF, 1>;
  constexpr int NSTEP = S::NSTEP, DPL = S::DPL;
  // Scaled logits (log2 units); keys past the row's range are -inf.
  float lg[NSTEP];
  float mx = st.m;
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const float d = group_sum<S::G>(slice_dot<BF>(kk[s], q));
    lg[s] = (j0 + s * S::KPI + kl < kend) ? d * p.c : -INFINITY;
    mx = fmaxf(mx, lg[s]);
  }
  if (mx == -INFINITY) return;  // nothing visible to this lane yet
  if (mx > st.m) {
    const float alpha = __builtin_amdgcn_exp2f(st.m - mx);  // 0 while m is -inf
    st.l *= alpha;
#pragma unroll
    for (int d = 0; d < DPL; ++d) st.acc[d] *= alpha;
    st.m = mx;
  }
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const float e = __builtin_amdgcn_exp2f(lg[s] - mx);
    st.l += e;
    const float pe = BF ? __uint_as_float(pack_bf16x2(e, 0.f) << 16) : e;
    slice_pv<BF>(st.acc, pe, vv[s]);
  }
}

// One split's partial of a row: P.V sums, max (scaled log2 units) and sum.
template <int E, int DPC>
__device__ __forceinline__ void rows_put_partial(const FlashParams& p, int64_t slot, const float (&acc)[DPC], float mx,
                                                 float l, int lane) {
  if (lane < E / DPC) {
#pragma unroll
    for (int d = 0; d < DPC; ++d) p.part_acc[slot * E + lane * DPC + d] = acc[d];
  }
  if (lane == 0) {
    p.part_ml[2 * slot] = mx;
    p.part_ml[2 * slot + 1] = l;
  }
}

// Writes row `row` (= (batch*heads + head)*seq_q + query) of the output: acc * inv.
template <int E, int DPC, bool BF>
__device__ __forceinline__ void rows_put_out(const FlashParams& p, int64_t row, const float (&acc)[DPC], float inv,
                                             int lane) {
  if (lane >= E / DPC) return;
  const int64_t bh = row / p.seq_q, i = row - bh * p.seq_q;
  const int64_t b = bh / p.heads, h = bh - b * p.heads;
  const int64_t oidx = ((b * p.seq_q + i) * p.heads + h) * E + lane * DPC;
  if constexpr (BF) {
    uint16_t* o = static_cast<uint16_t*>(p.out) + oidx;
#pragma unroll
    for (int d = 0; d < DPC; ++d) o[d] = (uint16_t)pack_bf16x2(acc[d] * inv, 0.f);
  } else {
    float* o = static_cast<float*>(p.out) + oidx;
#pragma unroll
    for (int d = 0; d < DPC; ++d) o[d] = acc[d] * inv;
  }
}

// One wave merges row `row`'s partials of all splits (at most 64) and writes the
// row: lane t loads split t's max and sum and computes its weight; the P.V
// partials come C splits at a time, every load of a round issued before any is
// used (the merge is latency-bound), each weighted by its lane's weight.
static_assert(kRowsMaxSplits <= kWave && kTiledMaxSplits <= kWave, "rows_merge_row takes a lane per split");
template <int E, bool BF>
__device__ __forceinline__ void rows_merge_row(const FlashParams& p, int64_t row, int splits, int lane) {
  constexpr int DPC = E >= 64 ? E / 64 : 1;
  constexpr int ACTIVE = E / DPC;
  constexpr int C = 16;
  const float* ml = p.part_ml + row * splits * 2;
  float mt = -INFINITY, lt = 0.f;
  if (lane < splits) {
    mt = ml[2 * lane];
    lt = ml[2 * lane + 1];
  }
  const float mx = wave_max(mt);
  float acc[DPC];
#pragma unroll
  for (int d = 0; d < DPC; ++d) acc[d] = 0.f;
  float inv = 0.f;
  if (mx != -INFINITY) {
    const float wgt = __builtin_amdgcn_exp2f(mt - mx);  // 0 for a split that saw nothing, and past the splits
    const float l = wave_sum(wgt * lt);
    const bool dims = lane < ACTIVE;
    const float* pa = p.part_acc + row * splits * E + (dims ? lane * DPC : 0);
    for (int t0 = 0; t0 < splits; t0 += C) {
      float at[C][DPC];
#pragma unroll
      for (int c = 0; c < C; ++c) {
#pragma unroll
        for (int d = 0; d < DPC; ++d)
          at[c][d] = t0 + c < splits && dims ? pa[(int64_t)(t0 + c) * E + d] : 0.f;
      }
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), t0 + c));
#pragma unroll
        for (int d = 0; d < DPC; ++d) acc[d] = fmaf(w, at[c][d], acc[d]);
      }
    }
    inv = l > 0.f ? 1.f / l : 0.f;
  }
  rows_put_out<E, DPC, BF>(p, row, acc, inv, lane);
}

// Block = kRowsWaves waves on one (batch, head, row group) and one split of its
// chunks: wave w walks chunks sp*W + w, + W*splits, ..., with the next chunk's
// loads in flight while it folds the current one.  The waves' states merge in
// LDS; a call with one split writes the rows, otherwise the block leaves a
// partial per row and split in the workspace.
template <int E, bool BF, int R_>
__global__ __launch_bounds__(64 * kRowsWaves) void flash_rows_kernel(FlashParams p) {
  using S = RowsShape<E, BF, R_>;
  constexpr int DPL = S::DPL, G = S::G, CH = S::CH, R = S::R, W = kRowsWaves, NSTEP = S::NSTEP, NBUF = S::NBUF;
  // The row counts the routes use and the tests cover (16 rows per wave gave wrong
  // results when tried, so the kernel admits only these).
  static_assert(R == 1 || R == kRowsPerWave || R == kRowsPerWaveMany, "rows per wave");
  constexpr int PS = E + 2;  // floats per partial: acc[E], m, l
  __shared__ float part[W][R][PS];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const RowsWork rw = rows_work(p, R, CH, blockIdx.x, gridDim.x, gridDim.y);
  const int64_t b = rw.b, h = rw.h, bh = b * p.heads + h, i0 = rw.i0;
  const int nr = rw.nr;
  const int64_t kend_g = rw.kend_g;  // the group's widest key range
  const int64_t nch = rw.nch;
  const int64_t splits = gridDim.y, sp = blockIdx.y;
  const int sl = lane % G;  // this lane's slice of a row
  const int kl = lane / G;  // this lane's key within a load instruction

  const char* qb = static_cast<const char*>(p.q) + (b * p.qs[0] + h * p.qs[2]) * S::ES;
  const char* kb = static_cast<const char*>(p.k) + (b * p.ks[0] + h * p.ks[2]) * S::ES;
  const char* vb = static_cast<const char*>(p.v) + (b * p.vs[0] + h * p.vs[2]) * S::ES;

  u32x4 qv[R];
  int64_t kend[R];
  RowAcc<DPL> st[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    qv[r] = u32x4{0u, 0u, 0u, 0u};
    if (r < nr) qv[r] = *reinterpret_cast<const u32x4*>(qb + ((i0 + r) * p.qs[1] + sl * DPL) * S::ES);
    kend[r] = r < nr ? rows_kend(p, i0 + r) : 0;
    st[r].m = -INFINITY;
    st[r].l = 0.f;
#pragma unroll
    for (int d = 0; d < DPL; ++d) st[r].acc[d] = 0.f;
  }

  const int64_t stride = (int64_t)W * splits;
  int64_t c = sp * W + wv;
  // A ring of NBUF chunk buffers: NBUF - 1 chunks' loads are in flight while one
  // is folded (static indices: the ring is unrolled).
  if (c < nch) {
    u32x4 kr[NBUF][NSTEP], vr[NBUF][NSTEP];
#pragma unroll
    for (int i = 0; i + 1 < NBUF; ++i)
      if (c + i * stride < nch) load_chunk<E, BF>(kb, vb, p, (c + i * stride) * CH, kend_g, kl, sl, kr[i], vr[i]);
    bool more = true;
    while (more) {
#pragma unroll
      for (int i = 0; i < NBUF; ++i) {
        if (more) {
          const int64_t cp = c + (NBUF - 1) * stride;
          if (cp < nch) load_chunk<E, BF>(kb, vb, p, cp * CH, kend_g, kl, sl, kr[(i + NBUF - 1) % NBUF], vr[(i + NBUF - 1) % NBUF]);
#pragma unroll
          for (int r = 0; r < R; ++r)
            if (r < nr) fold_chunk<E, BF>(p, kr[i], vr[i], qv[r], c * CH, kend[r], kl, st[r]);
          c += stride;
          more = c < nch;
        }
      }
    }
  }

  // This wave's totals per row: merge the lane states over the key groups (lanes
  // with the same slice hold the same dims).
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r >= nr) break;
#pragma unroll
    for (int o = G; o < kWave; o <<= 1) {
      float oacc[DPL];
#pragma unroll
      for (int d = 0; d < DPL; ++d) oacc[d] = __shfl_xor(st[r].acc[d], o);
      merge_state<DPL>(st[r], __shfl_xor(st[r].m, o), __shfl_xor(st[r].l, o), oacc);
    }
    if (lane < G) {
#pragma unroll
      for (int d = 0; d < DPL; ++d) part[wv][r][sl * DPL + d] = st[r].acc[d];
      if (lane == 0) {
        part[wv][r][E] = st[r].m;
        part[wv][r][E + 1] = st[r].l;
      }
    }
  }
  __syncthreads();

  // Merge the waves: wave r takes row r.
  constexpr int DPC = E >= 64 ? E / 64 : 1;
  constexpr int ACTIVE = E / DPC;
  if (wv < nr) {
    const int r = wv;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) mx = fmaxf(mx, part[w][r][E]);
    float l = 0.f, acc[DPC];
#pragma unroll
    for (int d = 0; d < DPC; ++d) acc[d] = 0.f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float wgt = __builtin_amdgcn_exp2f(part[w][r][E] - mx);  // 0 for a wave that saw nothing
        l = fmaf(wgt, part[w][r][E + 1], l);
        if (lane < ACTIVE) {
#pragma unroll
          for (int d = 0; d < DPC; ++d) acc[d] = fmaf(wgt, part[w][r][lane * DPC + d], acc[d]);
        }
      }
    }
    const int64_t row = bh * p.seq_q + i0 + r;
    if (splits == 1)
      rows_put_out<E, DPC, BF>(p, row, acc, l > 0.f ? 1.f / l : 0.f, lane);
    else
      rows_put_partial<E, DPC>(p, row * splits + sp, acc, mx, l, lane);
  }
}

// Single-row calls whose heads lie side by side (head stride E in q, k and v, as
// in a [batch, seq, heads, E] tensor or a fused projection) and short key ranges:
// a wave instruction reads one key's HP = 64/G consecutive heads, 1 KB in one
// run, instead of KPI keys of one head, KPI runs of E*esize bytes a token stride
// apart, and the keys of a (batch, head group) are split over several blocks, so
// many rows with few keys still give every wave a few chunks to stream (the
// per-head route gives such a row one block of 8 waves with one chunk each).
// Block = kRowsWaves waves on (batch, group of HP heads, split of the
// keys); lane (hl, sl) holds head h0 + hl, slice sl; wave w takes chunks of
// NSTEP keys sp*W + w, + W*splits, ..., with NBUF chunks in flight.  The numerics
// are flash_rows_kernel's.
template <int E, bool BF>
struct HeadsShape {
  static constexpr int ES = BF ? 2 : 4;    // element bytes
  static constexpr int DPL = 16 / ES;      // elements per lane slice
  static constexpr int G = E / DPL;        // lanes per head
  static constexpr int HP = kWave / G;     // heads per load instruction
  static constexpr int NSTEP = 4;          // keys per chunk (one load instruction each for K and V)
  static constexpr int NBUF = 3;           // chunks in flight per wave (4 and 2 measured slower)
};

__host__ __device__ inline int rows_heads_per_load(int E, bool bf16) { return kWave / (E / (bf16 ? 8 : 4)); }

// Splits of each (batch, head group)'s keys across blocks.
__host__ __device__ inline int64_t rows_heads_splits(int64_t batch, int64_t seq_k, int64_t heads, int E, bool bf16) {
  const int64_t blocks = batch * (heads / rows_heads_per_load(E, bf16));
  const int64_t chunk_rounds = cdiv(cdiv(seq_k, 4), kRowsWaves);
  int64_t s = blocks >= kRowsTargetBlocks ? 1 : cdiv(kRowsTargetBlocks, blocks);
  s = s < chunk_rounds ? s : chunk_rounds;
  s = s < kRowsMaxSplits ? s : kRowsMaxSplits;
  return s < 1 ? 1 : s;
}

// The call takes flash_rows_heads_kernel: one query row, packed heads and a head
// count the loads divide, at any key count.  Measured on MI355X (bf16, back-to-back
// calls) against the per-head route: N=64 H=32 E=32, 512 keys, 44.8 -> 29.8 us;
// N=8 H=32 E=32, 2048 keys 20.5 -> 18.4 us, 4096 keys 38.0 -> 25.8 us, 8192 keys
// 74.1 -> 45.1 us; E=64 2048 keys 29.2 -> 26.6 us; E=128 8192 keys 174.7 -> 170.6 us.
__host__ __device__ inline bool rows_heads_shapes(int64_t seq_q, int64_t heads, int E, bool bf16) {
  return seq_q == 1 && heads % rows_heads_per_load(E, bf16) == 0;
}
__host__ __device__ inline bool rows_heads_route(const FlashParams& p, int E, bool bf16) {
  return rows_heads_shapes(p.seq_q, p.heads, E, bf16) && p.qs[2] == E && p.ks[2] == E && p.vs[2] == E;
}

// Block (bx of gx, split of gy) of the packed-heads kernel: batch b, heads
// [h0, h0 + hp).
struct HeadsWork {
  int64_t b, h0;
};
__host__ __device__ inline HeadsWork heads_work(const FlashParams& p, int hp, int64_t bx, int64_t gx, int64_t gy) {
  const int64_t ng = p.heads / hp;
  const int64_t lb = gy == 1 ? xcd_remap(bx, gx) : bx;
  HeadsWork w;
  w.b = lb / ng;
  w.h0 = (lb - w.b * ng) * hp;
  return w;
}

template <int E, bool BF>
__global__ __launch_bounds__(64 * kRowsWaves) void flash_rows_heads_kernel(FlashParams p) {
  using S = HeadsShape<E, BF>;
  constexpr int DPL = S::DPL, G = S::G, HP = S::HP, W = kRowsWaves, NSTEP = S::NSTEP, NBUF = S::NBUF;
  constexpr int PS = E + 2;  // floats per partial: acc[E], m, l
  __shared__ float part[W][HP][PS];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const HeadsWork hw = heads_work(p, HP, blockIdx.x, gridDim.x, gridDim.y);
  const int64_t b = hw.b, h0 = hw.h0;
  const int64_t splits = gridDim.y, sp = blockIdx.y;
  const int sl = lane % G;   // this lane's slice of a head row
  const int hl = lane / G;   // this lane's head within the group
  const int64_t S_ = p.seq_k;
  const int64_t nch = cdiv(S_, NSTEP);

  const char* qb = static_cast<const char*>(p.q) + (b * p.qs[0] + (h0 + hl) * E + sl * DPL) * S::ES;
  const char* kb = static_cast<const char*>(p.k) + (b * p.ks[0] + (h0 + hl) * E + sl * DPL) * S::ES;
  const char* vb = static_cast<const char*>(p.v) + (b * p.vs[0] + (h0 + hl) * E + sl * DPL) * S::ES;
  const u32x4 q = *reinterpret_cast<const u32x4*>(qb);
  RowAcc<DPL> st;
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int d = 0; d < DPL; ++d) st.acc[d] = 0.f;

  auto load = [&](int64_t c, u32x4 (&kk)[NSTEP], u32x4 (&vv)[NSTEP]) __attribute__((always_inline)) {
#pragma unroll
    for (int s2 = 0; s2 < NSTEP; ++s2) {
      const int64_t j = c * NSTEP + s2;
      kk[s2] = u32x4{0u, 0u, 0u, 0u};
      vv[s2] = u32x4{0u, 0u, 0u, 0u};
      if (j < S_) {
        kk[s2] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kb + j * p.ks[1] * S::ES));
        vv[s2] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vb + j * p.vs[1] * S::ES));
      }
    }
  };
  auto fold = [&](int64_t c, const u32x4 (&kk)[NSTEP], const u32x4 (&vv)[NSTEP]) __attribute__((always_inline)) {
    float lg[NSTEP];
    float mx = st.m;
#pragma unroll
    for (int s2 = 0; s2 < NSTEP; ++s2) {
      const float d = group_sum<G>(slice_dot<BF>(kk[s2], q));
      lg[s2] = c * NSTEP + s2 < S_ ? d * p.c : -INFINITY;
      mx = fmaxf(mx, lg[s2]);
    }
    if (mx == -INFINITY) return;
    if (mx > st.m) {
      const float alpha = __builtin_amdgcn_exp2f(st.m - mx);  // 0 while m is -inf
      st.l *= alpha;
#pragma unroll
      for (int d = 0; d < DPL; ++d) st.acc[d] *= alpha;
      st.m = mx;
    }
#pragma unroll
    for (int s2 = 0; s2 < NSTEP; ++s2) {
      const float e = __builtin_amdgcn_exp2f(lg[s2] - mx);
      st.l += e;
      const float pe = BF ? __uint_as_float(pack_bf16x2(e, 0.f) << 16) : e;
      slice_pv<BF>(st.acc, pe, vv[s2]);
    }
  };

  const int64_t stride = (int64_t)W * splits;
  int64_t c = sp * W + wv;
  if (c < nch) {
    u32x4 kr[NBUF][NSTEP], vr[NBUF][NSTEP];
#pragma unroll
    for (int i = 0; i + 1 < NBUF; ++i)
      if (c + i * stride < nch) load(c + i * stride, kr[i], vr[i]);
    bool more = true;
    while (more) {
#pragma unroll
      for (int i = 0; i < NBUF; ++i) {
        if (more) {
          const int64_t cp = c + (NBUF - 1) * stride;
          if (cp < nch) load(cp, kr[(i + NBUF - 1) % NBUF], vr[(i + NBUF - 1) % NBUF]);
          fold(c, kr[i], vr[i]);
          c += stride;
          more = c < nch;
        }
      }
    }
  }
#pragma unroll
  for (int d = 0; d < DPL; ++d) part[wv][hl][sl * DPL + d] = st.acc[d];
  if (sl == 0) {
    part[wv][hl][E] = st.m;
    part[wv][hl][E + 1] = st.l;
  }
  __syncthreads();

  // Merge the waves: wave w takes heads w, w + W, ... of the group.
  constexpr int DPC = E >= 64 ? E / 64 : 1;
  constexpr int ACTIVE = E / DPC;
  for (int hh = wv; hh < HP; hh += W) {
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) mx = fmaxf(mx, part[w][hh][E]);
    float l = 0.f, acc[DPC];
#pragma unroll
    for (int d = 0; d < DPC; ++d) acc[d] = 0.f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float wgt = __builtin_amdgcn_exp2f(part[w][hh][E] - mx);  // 0 for a wave that saw nothing
        l = fmaf(wgt, part[w][hh][E + 1], l);
        if (lane < ACTIVE) {
#pragma unroll
          for (int d = 0; d < DPC; ++d) acc[d] = fmaf(wgt, part[w][hh][lane * DPC + d], acc[d]);
        }
      }
    }
    const int64_t row = b * p.heads + h0 + hh;  // seq_q == 1
    if (splits == 1)
      rows_put_out<E, DPC, BF>(p, row, acc, l > 0.f ? 1.f / l : 0.f, lane);
    else
      rows_put_partial<E, DPC>(p, row * splits + sp, acc, mx, l, lane);
  }
}

// One wave per (batch, head, query) row: merges the row's partials of all splits
// (the few-rows kernels' and the tiled kernel's split modes).
template <int E, bool BF>
__global__ __launch_bounds__(256) void flash_rows_combine_kernel(FlashParams p, int splits) {
  const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= p.batch * p.heads * p.seq_q) return;
  rows_merge_row<E, BF>(p, row, splits, threadIdx.x & 63);
}

// Splits of each row group's chunks across blocks: one unless the row groups
// alone leave the chip short of blocks, and never more than the chunks allow.
__host__ __device__ inline int64_t rows_splits(int64_t batch, int64_t seq_q, int64_t seq_k, int64_t heads, int E,
                                               bool bf16) {
  const int64_t blocks = batch * heads * cdiv(seq_q, rows_per_wave(seq_q));
  const int64_t chunk_rounds = cdiv(cdiv(seq_k, rows_chunk_keys(E, bf16)), kRowsWaves);
  int64_t s = blocks >= kRowsTargetBlocks ? 1 : cdiv(kRowsTargetBlocks, blocks);
  s = s < chunk_rounds ? s : chunk_rounds;
  s = s < kRowsMaxSplits ? s : kRowsMaxSplits;
  return s < 1 ? 1 : s;
}

// Splits of the call's route (the strides choose between the two kernels).
static int64_t rows_call_splits(const FlashParams& p, int E, bool bf16) {
  return rows_heads_route(p, E, bf16) ? rows_heads_splits(p.batch, p.seq_k, p.heads, E, bf16)
                                      : rows_splits(p.batch, p.seq_q, p.seq_k, p.heads, E, bf16);
}

// Bytes of the few-rows route's workspace at `splits`: the partials, E + 2 floats
// each.
__host__ __device__ inline int64_t rows_ws_bytes(int64_t rows, int64_t splits, int E) {
  return splits > 1 ? rows * splits * (E + 2) * 4 : 0;
}

// The workspace a call of these shapes may need: its strides are not known
// here, so the larger of the two routes' partials; past the few-rows route, the
// tiled kernel's split mode, causal or not.
int64_t flash_rows_workspace_bytes(int64_t batch, int64_t seq_q, int64_t seq_k, int64_t heads, int E,
                                   bool bf16) {
  if (!rows_route(batch, seq_q, heads, bf16)) return tiled_workspace_bytes_any(batch, seq_q, seq_k, heads, E, bf16);
  int64_t splits = rows_splits(batch, seq_q, seq_k, heads, E, bf16);
  if (rows_heads_shapes(seq_q, heads, E, bf16)) {
    const int64_t hs = rows_heads_splits(batch, seq_k, heads, E, bf16);
    splits = splits > hs ? splits : hs;
  }
  return rows_ws_bytes(batch * heads * seq_q, splits, E);
}

int64_t flash_call_splits(const FlashParams& p, int E, bool bf16) {
  return rows_route(p.batch, p.seq_q, p.heads, bf16) ? rows_call_splits(p, E, bf16)
                                                     : tiled_splits(p.batch, p.seq_q, p.seq_k, p.heads, bf16, p.causal != 0);
}

void flash_rows_workspace(FlashParams& p, void* ws, int64_t bytes, int E, bool bf16) {
  const int64_t splits = flash_call_splits(p, E, bf16);
  p.part_acc = static_cast<float*>(ws);
  p.part_ml = ws ? reinterpret_cast<float*>(static_cast<char*>(ws) + p.batch * p.heads * p.seq_q * splits * E * 4)
                 : nullptr;
  p.workspace_bytes = bytes;
}

template <int E, bool BF>
static int rows_launch_t(const FlashParams& p, const FlashPlan& plan, hipStream_t stream) {
  const int R = plan.rows_r;
  const int64_t gx = plan.gx, splits = plan.gy;
  if (plan.kind == kPlanRowsHeads)
    hipLaunchKernelGGL((flash_rows_heads_kernel<E, BF>), dim3((unsigned)gx, (unsigned)splits), dim3(64 * kRowsWaves),
                       0, stream, p);
  else if (R == 1)
    hipLaunchKernelGGL((flash_rows_kernel<E, BF, 1>), dim3((unsigned)gx, (unsigned)splits), dim3(64 * kRowsWaves),
                       0, stream, p);
  else if (R == kRowsPerWaveMany)
    hipLaunchKernelGGL((flash_rows_kernel<E, BF, kRowsPerWaveMany>), dim3((unsigned)gx, (unsigned)splits),
                       dim3(64 * kRowsWaves), 0, stream, p);
  else
    hipLaunchKernelGGL((flash_rows_kernel<E, BF, kRowsPerWave>), dim3((unsigned)gx, (unsigned)splits),
                       dim3(64 * kRowsWaves), 0, stream, p);
  int st = ca_launch_status();
  if (st != CA_OK || splits == 1) return st;
  const int64_t rows = p.batch * p.heads * p.seq_q;
  hipLaunchKernelGGL((flash_rows_combine_kernel<E, BF>), dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, stream, p,
                     (int)splits);
  return ca_launch_status();
}

int flash_combine_launch(const FlashParams& p, int E, int bf16, int64_t splits, hipStream_t stream) {
  const int64_t rows = p.batch * p.heads * p.seq_q;
  if (cdiv(rows, 4) > 0x7fffffff || splits > kWave) return CA_DECLINED;
  const dim3 grid((unsigned)cdiv(rows, 4));
  if (bf16) {
    switch (E) {
      case 32: hipLaunchKernelGGL((flash_rows_combine_kernel<32, true>), grid, dim3(256), 0, stream, p, (int)splits); break;
      case 64: hipLaunchKernelGGL((flash_rows_combine_kernel<64, true>), grid, dim3(256), 0, stream, p, (int)splits); break;
      case 128: hipLaunchKernelGGL((flash_rows_combine_kernel<128, true>), grid, dim3(256), 0, stream, p, (int)splits); break;
      default: return CA_DECLINED;
    }
  } else {
    switch (E) {
      case 32: hipLaunchKernelGGL((flash_rows_combine_kernel<32, false>), grid, dim3(256), 0, stream, p, (int)splits); break;
      case 64: hipLaunchKernelGGL((flash_rows_combine_kernel<64, false>), grid, dim3(256), 0, stream, p, (int)splits); break;
      case 128: hipLaunchKernelGGL((flash_rows_combine_kernel<128, false>), grid, dim3(256), 0, stream, p, (int)splits); break;
      default: return CA_DECLINED;
    }
  }
  return ca_launch_status();
}

FlashPlan rows_plan(const FlashParams& p, int E, bool bf16) {
  FlashPlan plan{};
  const bool heads = rows_heads_route(p, E, bf16);
  plan.kind = heads ? kPlanRowsHeads : kPlanRows;
  plan.rows_r = rows_per_wave(p.seq_q);
  plan.gx = heads ? p.batch * (p.heads / rows_heads_per_load(E, bf16)) : p.batch * p.heads * cdiv(p.seq_q, plan.rows_r);
  plan.gy = plan.splits = rows_call_splits(p, E, bf16);
  plan.need = rows_ws_bytes(p.batch * p.heads * p.seq_q, plan.splits, E);
  if (plan.gx > 0x7fffffff || plan.gy > 0xffff) plan.kind = kPlanDeclined;
  return plan;
}

int flash_rows_launch(const FlashParams& p, const FlashPlan& plan, int E, int bf16, hipStream_t stream) {
  if (bf16) {
    switch (E) {
      case 32: return rows_launch_t<32, true>(p, plan, stream);
      case 64: return rows_launch_t<64, true>(p, plan, stream);
      case 128: return rows_launch_t<128, true>(p, plan, stream);
    }
  } else {
    switch (E) {
      case 32: return rows_launch_t<32, false>(p, plan, stream);
      case 64: return rows_launch_t<64, false>(p, plan, stream);
      case 128: return rows_launch_t<128, false>(p, plan, stream);
    }
  }
  return CA_DECLINED;
}

}  // namespace ca
