// Paged decode on CDNA4: split-K over 64- or 256-key tiles plus a combine pass.
//
// Follows the reference's decode (cpu_attention/_mojo/src/paged_attn.mojo:714-782):
// logits q.k, base-2 online softmax with c = scale*log2(e) and the running max in
// scaled log2 units, fp32 P against fp32-widened V, out = acc * (1/l), and a row
// that saw no key is exactly 0 (_store_row :297-319).  Keys past the length are
// never read (0 * NaN would poison the row, :686-687), nor are page-table entries
// past the last page in use.
//
// Work split.  One wave per tile of one row (sequence, head): grid.x walks the
// rows, grid.y the tile groups (8 tiles per 512-thread block: 512 keys of 64-key
// tiles, 2048 of 256-key tiles) up to the page table's capacity, so every row's
// first tiles are dispatched first.  decode_tile_keys (below) picks the tile size
// from the call's shapes.  Waves whose tile is past the row's length exit at once
// (a block barrier waits only for the waves still running).  The waves of a block
// merge their partial (max, sum, P.V) states in LDS: a row that fits one block is
// written by it, with no workspace traffic.  Longer rows leave one partial per
// block in the workspace, and the combine kernel merges those.  The host needs no
// lengths and nothing synchronises.  (A stream-K split into equal slices per
// resident wave was measured slower: 347 us against 189 us on a 1.1 GB batch.)
//
// Layout use (the reference's PageLayout, :58-130): a 16-key unit never straddles a
// page (P % 16 == 0), so a tile is up to 16 units, each one contiguous run inside one
// (block, head):
//   Q.K  lane l owns keys 4l..4l+3 of a 256-key tile; one 16-byte load per K word
//        row (w*P + t .. t+3) gives those 4 keys' word w, so the dot product needs
//        no cross-lane reduction.  A 64-key tile gives each key quad to 4 lanes
//        that take every 4th word and sum their partial products at the end.
//        bf16 words are dim pairs: v_dot2_f32_bf16 with the matching q pair
//        (exact products, fp32 accumulation).
//   P.V  lane groups of E/8 (bf16) or E/4 (fp32) lanes read whole V rows with
//        16-byte loads; each wave instruction reads rows of G different units
//        (pages), p comes from LDS.
// K and V are read with non-temporal loads: each byte is used once.  (Measured on
// MI355X: temporal loads for K and V made the bench's 1.1 GB batch 13% slower.
// Temporal K loads in a call that appends a token made back-to-back calls on one
// cache faster, since part of the cache then stays in the 256 MB MALL from one call
// to the next, but made a call after a cache flush 11% slower: 4096 rows,
// 287 against 258 us.  A model's other layers pass through the caches between two
// steps of one layer, so the flushed case is the one kept.)
#include "ca_device.h"
#include "ca_internal.h"

namespace ca {

constexpr int kTile = kDecodeLongTile;  // keys per long tile
constexpr int kShortTile = 64;           // keys per short tile
constexpr int kUnit = 16;                // keys per unit (one page run)
constexpr int kDecWaves = 8;             // tiles (waves) per block
static_assert(kTile == 256, "long tiles: one key quad per lane");

// out[idx .. idx+N) = v * inv in the output dtype (bf16: round to nearest even).
template <int N, bool BF>
__device__ __forceinline__ void store_out(void* out, int64_t idx, const float* v, float inv) {
  if constexpr (BF && N % 2 == 0) {
    uint32_t* o = reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(out) + idx);
#pragma unroll
    for (int i = 0; i < N; i += 2) o[i / 2] = pack_bf16x2(v[i] * inv, v[i + 1] * inv);
  } else if constexpr (BF) {
    uint16_t* o = reinterpret_cast<uint16_t*>(out) + idx;
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = (uint16_t)pack_bf16x2(v[i] * inv, 0.f);
  } else {
    float* o = reinterpret_cast<float*>(out) + idx;
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = v[i] * inv;
  }
}

__device__ __forceinline__ int64_t row_len(const DecodeParams& p, int64_t seq) {
  const int64_t cap = p.pt_width * p.page;
  const int64_t len = (int64_t)p.lens[seq] + p.len_add;
  return len < 0 ? 0 : (len < cap ? len : cap);
}

template <int E, bool BF>
struct DecodeShape {
  static constexpr int ES = BF ? 2 : 4;    // element bytes
  static constexpr int W = E * ES / 4;     // K words per key (per head)
  static constexpr int DPL = 16 / ES;      // V elements per 16-byte load
  static constexpr int LPR = E / DPL;      // lanes per V row
  static constexpr int G = kWave / LPR;    // V rows per wave load
  static constexpr int UNROLL = 16;
  static_assert(W % UNROLL == 0 && kUnit % G == 0, "tile shape");
};

// Online-softmax state of one wave for one row: m (scaled log2 units, uniform),
// l (per-lane partial sum), acc (per-lane partial P.V of dims dl*DPL.., summed over
// the lane groups at the end).
template <int E, bool BF>
struct RowState {
  float m, l;
  float acc[DecodeShape<E, BF>::DPL];
  __device__ void init() {
    m = -INFINITY;
    l = 0.f;
#pragma unroll
    for (int i = 0; i < DecodeShape<E, BF>::DPL; ++i) acc[i] = 0.f;
  }
};

// Keys [t0, t0 + ntok) of row (seq, h): 0 < ntok <= TK, t0 % 16 == 0, t0 + ntok <= len.
// Folds them into st.  p_lds is this wave's TK-float scratch.  newj >= 0 (wave-
// uniform) names the key of the tile that is the token appended by this call: the
// wave copies it from p.k_new / p.v_new into the cache.
//
// TK = 256: lane l owns the key quad l (keys 4l..4l+3) and all W words of it.
// TK = 64: the 16 key quads of the tile are shared by SPLIT = 4 lanes each: lane l
// takes quad l % 16 and words l / 16, l / 16 + 4, ..., and the four partial dot
// products are summed across the lanes afterwards.
template <int E, bool BF, bool APPEND, int TK>
__device__ __forceinline__ void decode_tile(const DecodeParams& p, int64_t seq, int64_t h,
                                            int64_t t0, int ntok, int newj, float* p_lds,
                                            RowState<E, BF>& st) {
  using D = DecodeShape<E, BF>;
  constexpr int W = D::W, DPL = D::DPL, LPR = D::LPR, G = D::G, ES = D::ES, UNROLL = D::UNROLL;
  constexpr int NU = TK / kUnit;           // units per tile
  constexpr int NQ = TK / 4;               // key quads per tile
  constexpr int SPLIT = kWave / NQ;        // lanes per key quad
  constexpr int WPL = W / SPLIT;           // K words per lane
  constexpr int QU = WPL < UNROLL ? WPL : UNROLL;  // K loads per batch
  static_assert((TK == kTile || TK == kShortTile) && W % SPLIT == 0 && WPL % QU == 0, "tile shape");
  const int lane = threadIdx.x & 63;
  const int quad = lane % NQ, phase = lane / NQ;

  // Unit table: lane u < NU resolves unit u's page once (word index of its K run,
  // element index of its V rows); -1 marks a unit past the tile or a page-table
  // entry that names no block.
  int64_t kb = -1, vb = -1;
  if (lane < NU && kUnit * lane < ntok) {
    const int64_t tu = t0 + kUnit * lane;
    const int64_t pi = tu / p.page, off = tu - pi * p.page;
    const int64_t blk = p.page_table[seq * p.pt_width + pi];
    if (blk >= 0 && blk < p.nblocks) {
      const int64_t base = (blk * p.heads + h) * p.page;
      kb = base * W + off;
      vb = (base + off) * E;
    }
  }

  // ---- the token appended by this call, at tile key newj.  Its words are read
  // here (beside the page-table reads above, so the latencies overlap).  Right
  // after the Q.K loop it goes to the cache: its K words land in lines the loop
  // has just brought into L2 (4-byte writes into lines that are not resident
  // would each cost the DRAM a read-modify-write), and its V row ahead of the
  // P.V loads that read it back (a workgroup-scope release and acquire orders the
  // two for the wave's lanes; on gfx950 the CU keeps them in order and the fence
  // costs nothing).  Its logit, computed from the registers, replaces what the
  // lane owning the key read from the slot.
  // Nothing is stored or substituted when the key's page names no block.
  constexpr int KNW = (W + kWave - 1) / kWave;  // K words of the new key per lane
  uint32_t knw[KNW], qnw[KNW];
  u32x4 vrow;
  int64_t kbn = -1;
  if (APPEND && newj >= 0) {
    const uint32_t* knew = p.k_new + seq * p.kv_stride_w + h * W;
    const uint32_t* vnew = p.v_new + seq * p.kv_stride_w + h * W;
    const uint32_t* qwd = reinterpret_cast<const uint32_t*>(p.q) + (seq * p.q_stride + h * E) * ES / 4;
#pragma unroll
    for (int i = 0; i < KNW; ++i) {
      const int w = lane + kWave * i;
      knw[i] = w < W ? knew[w] : 0u;
      qnw[i] = w < W ? qwd[w] : 0u;
    }
    vrow = lane < W / 4 ? *reinterpret_cast<const u32x4*>(vnew + 4 * lane) : u32x4{0u, 0u, 0u, 0u};
  }

  // ---- Q.K: keys 4*quad .. 4*quad+3 of the tile, words phase, phase + SPLIT, ...
  float s[4];
  {
    const int64_t kbu = __shfl(kb, quad >> 2);
    const int key0 = 4 * quad;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (kbu >= 0 && key0 < ntok) {
      const uint32_t* kp = p.kc + kbu + 4 * (quad & 3) + (int64_t)phase * p.page;
      if constexpr (BF) {
        const uint32_t* qw = reinterpret_cast<const uint32_t*>(
            reinterpret_cast<const uint16_t*>(p.q) + seq * p.q_stride + h * E) + phase;
        for (int w0 = 0; w0 < WPL; w0 += QU) {
          u32x4 k4[QU];
#pragma unroll
          for (int i = 0; i < QU; ++i)
            k4[i] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(kp + (int64_t)(w0 + i) * SPLIT * p.page));
#pragma unroll
          for (int i = 0; i < QU; ++i) {
            const bf16x2 qv = as_bf16x2(qw[(w0 + i) * SPLIT]);
            a0 = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k4[i].x), qv, a0, false);
            a1 = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k4[i].y), qv, a1, false);
            a2 = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k4[i].z), qv, a2, false);
            a3 = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k4[i].w), qv, a3, false);
          }
        }
      } else {
        // Four partial sums per key (words w mod 4): 32-term chains instead of one
        // 128-term chain keep the fp32 logits well inside the 1e-6 decode gate.
        const float* qf = reinterpret_cast<const float*>(p.q) + seq * p.q_stride + h * E + phase;
        float c0[4] = {0.f, 0.f, 0.f, 0.f}, c1[4] = {0.f, 0.f, 0.f, 0.f};
        float c2[4] = {0.f, 0.f, 0.f, 0.f}, c3[4] = {0.f, 0.f, 0.f, 0.f};
        for (int w0 = 0; w0 < WPL; w0 += QU) {
          u32x4 k4[QU];
#pragma unroll
          for (int i = 0; i < QU; ++i)
            k4[i] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(kp + (int64_t)(w0 + i) * SPLIT * p.page));
#pragma unroll
          for (int i = 0; i < QU; ++i) {
            const float qv = qf[(w0 + i) * SPLIT];
            c0[i & 3] = fmaf(__uint_as_float(k4[i].x), qv, c0[i & 3]);
            c1[i & 3] = fmaf(__uint_as_float(k4[i].y), qv, c1[i & 3]);
            c2[i & 3] = fmaf(__uint_as_float(k4[i].z), qv, c2[i & 3]);
            c3[i & 3] = fmaf(__uint_as_float(k4[i].w), qv, c3[i & 3]);
          }
        }
        a0 = (c0[0] + c0[1]) + (c0[2] + c0[3]);
        a1 = (c1[0] + c1[1]) + (c1[2] + c1[3]);
        a2 = (c2[0] + c2[1]) + (c2[2] + c2[3]);
        a3 = (c3[0] + c3[1]) + (c3[2] + c3[3]);
      }
    }
    if constexpr (SPLIT > 1) {
      // The SPLIT lanes of a quad (lanes quad, quad + NQ, ...) sum their partial
      // products; every one of them ends with the same four logits.
#pragma unroll
      for (int o = NQ; o < kWave; o <<= 1) {
        a0 += __shfl_xor(a0, o);
        a1 += __shfl_xor(a1, o);
        a2 += __shfl_xor(a2, o);
        a3 += __shfl_xor(a3, o);
      }
    }
    // Raw logits (masked keys -inf); the scale is folded into the exponent below.
    const bool ok = kbu >= 0;
    s[0] = (ok && key0 + 0 < ntok) ? a0 : -INFINITY;
    s[1] = (ok && key0 + 1 < ntok) ? a1 : -INFINITY;
    s[2] = (ok && key0 + 2 < ntok) ? a2 : -INFINITY;
    s[3] = (ok && key0 + 3 < ntok) ? a3 : -INFINITY;
  }
  if (APPEND && newj >= 0) {
    kbn = __shfl(kb, newj >> 4);
    const int64_t vbn = __shfl(vb, newj >> 4);
    if (kbn >= 0) {
      const int x = newj & (kUnit - 1);
#pragma unroll
      for (int i = 0; i < KNW; ++i) {
        const int w = lane + kWave * i;
        if (w < W) p.kc_store[kbn + (int64_t)w * p.page + x] = knw[i];
      }
      if (lane < W / 4)
        *reinterpret_cast<u32x4*>(p.vc_store + (vbn + (int64_t)x * E) * ES / 4 + 4 * lane) = vrow;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < KNW; ++i) {
      if constexpr (BF)
        part = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(knw[i]), as_bf16x2(qnw[i]), part, false);
      else
        part = fmaf(__uint_as_float(knw[i]), __uint_as_float(qnw[i]), part);
    }
    const float logit = wave_sum(part);
    if (kbn >= 0 && quad == (newj >> 2)) {
      const int j = newj & 3;
      s[0] = j == 0 ? logit : s[0];
      s[1] = j == 1 ? logit : s[1];
      s[2] = j == 2 ? logit : s[2];
      s[3] = j == 3 ? logit : s[3];
    }
  }

  // ---- online softmax: tile max in scaled log2 units, alpha = 2^(m_old - m_new)
  // (0 on the first tile), p = 2^(logit*c - m): one rounding inside the exponent
  // (the reference's _rescale / _exp_row, paged_attn.mojo:271-277, 643-676).
  const float mraw = wave_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
  const float m_new = fmaxf(st.m, mraw * p.c);
  const float mu = m_new == -INFINITY ? 0.f : m_new;  // nothing readable yet
  const float alpha = __builtin_amdgcn_exp2f(st.m - mu);
  st.m = m_new;
  float pr[4];
  float ls = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    pr[j] = __builtin_amdgcn_exp2f(fmaf(s[j], p.c, -mu));
    ls += pr[j];
  }
  st.l = fmaf(st.l, alpha, phase == 0 ? ls : 0.f);  // one lane per quad counts it
#pragma unroll
  for (int i = 0; i < DPL; ++i) st.acc[i] *= alpha;
  wave_lds_sync();  // the previous tile's P.V reads are done
  if (phase == 0) *reinterpret_cast<f32x4*>(&p_lds[4 * quad]) = f32x4{pr[0], pr[1], pr[2], pr[3]};
  wave_lds_sync();

  // ---- P.V: lane group g (of G), lane dl of the group dims dl*DPL..
  // 256-key tiles: group g takes units g*UPG .. g*UPG+UPG-1; load j of a lane reads
  // row j / UPG of unit g*UPG + j % UPG, so one wave instruction spans G units and a
  // batch of 16 loads spans every unit of the group: the reads fan out over many
  // pages at once, which streams far better than walking one page row by row.
  // 64-key tiles (4 units, G of 4 to 16 groups): load j of group g reads key
  // g + G*j, so one wave instruction reads G consecutive rows of one unit (the unit
  // is the same for every lane, since G divides 16) and a batch spans all 4 units.
  constexpr bool BY_UNIT = NU >= G;
  constexpr int UPG = BY_UNIT ? NU / G : 1;  // units per group (BY_UNIT)
  constexpr int NV = BY_UNIT ? UPG : NU;     // unit bases a lane holds
  constexpr int R = TK / G;                  // rows per lane
  constexpr int B = R < 16 ? R : 16;         // loads in flight
  const int g = lane / LPR, dl = lane - g * LPR;
  int64_t vbu[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) vbu[k] = __shfl(vb, BY_UNIT ? g * UPG + k : k);
  // Load j: its key in the tile, and which of the lane's unit bases holds it.
  auto key_of = [&](int j) { return BY_UNIT ? kUnit * (g * UPG + j % UPG) + j / UPG : g + G * j; };
  auto base_of = [&](int j) { return BY_UNIT ? j % UPG : G * j / kUnit; };
  const char* vbase = reinterpret_cast<const char*>(p.vc) + dl * 16;
  // fp32: odd loads of a batch go to a second set of sums, added at the end, so a
  // lane's chain over its up to 64 keys of a long tile is two chains of half the
  // length.  One chain took a row of 81 keys to 1.11e-6 against the reference's
  // 1e-6 fp32 decode gate; two take it to 6.9e-7, at no measured cost (eight Q.K
  // chains instead of four cost up to 18% on 256-key tiles and were not kept).
  float acc2[BF ? 1 : DPL];
#pragma unroll
  for (int i = 0; i < (BF ? 1 : DPL); ++i) acc2[i] = 0.f;
#pragma unroll
  for (int b0 = 0; b0 < R; b0 += B) {
    if (key_of(b0) >= ntok) break;  // the batch's first key (its smallest) is past the tile
    u32x4 v4[B];
    bool ok[B];
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int j = b0 + i, key = key_of(j), k = base_of(j);
      ok[i] = vbu[k] >= 0 && key < ntok;
      if (ok[i])
        v4[i] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(vbase + (vbu[k] + (int64_t)(key & (kUnit - 1)) * E) * ES));
    }
#pragma unroll
    for (int i = 0; i < B; ++i) {
      if (ok[i]) {
        const float pj = p_lds[key_of(b0 + i)];
        const u32x4 v = v4[i];
        if constexpr (BF) {
          st.acc[0] = fmaf(pj, bf16_lo(v.x), st.acc[0]);
          st.acc[1] = fmaf(pj, bf16_hi(v.x), st.acc[1]);
          st.acc[2] = fmaf(pj, bf16_lo(v.y), st.acc[2]);
          st.acc[3] = fmaf(pj, bf16_hi(v.y), st.acc[3]);
          st.acc[4] = fmaf(pj, bf16_lo(v.z), st.acc[4]);
          st.acc[5] = fmaf(pj, bf16_hi(v.z), st.acc[5]);
          st.acc[6] = fmaf(pj, bf16_lo(v.w), st.acc[6]);
          st.acc[7] = fmaf(pj, bf16_hi(v.w), st.acc[7]);
        } else {
          float* a = (i & 1) ? acc2 : st.acc;
          a[0] = fmaf(pj, __uint_as_float(v.x), a[0]);
          a[1] = fmaf(pj, __uint_as_float(v.y), a[1]);
          a[2] = fmaf(pj, __uint_as_float(v.z), a[2]);
          a[3] = fmaf(pj, __uint_as_float(v.w), a[3]);
        }
      }
    }
  }
  if constexpr (!BF) {
#pragma unroll
    for (int i = 0; i < DPL; ++i) st.acc[i] += acc2[i];
  }
}

// Reduces a wave's lane partials into part[E + 2] in LDS: acc over the lane
// groups (lanes with the same dims), l over the wave, and the wave's max.
template <int E, bool BF>
__device__ __forceinline__ void wave_partial(RowState<E, BF>& st, float* part) {
  using D = DecodeShape<E, BF>;
  constexpr int DPL = D::DPL, LPR = D::LPR;
  const int lane = threadIdx.x & 63;
  const float l = wave_sum(st.l);
#pragma unroll
  for (int o = LPR; o < kWave; o <<= 1)
#pragma unroll
    for (int i = 0; i < DPL; ++i) st.acc[i] += __shfl_xor(st.acc[i], o);
  if (lane < LPR) {
#pragma unroll
    for (int i = 0; i < DPL; ++i) part[lane * DPL + i] = st.acc[i];
    if (lane == 0) {
      part[E] = st.m;
      part[E + 1] = l;
    }
  }
}

// Merges n partial states (m_t, l_t, acc_t) with weights 2^(m_t - M): lane-wise
// dims lane*DPC.., returns the merged sum; acc gets the merged P.V.
template <int E, int DPC, typename Get>
__device__ __forceinline__ float merge_states(int n, Get&& get, float& mx, float (&acc)[DPC]) {
  const int lane = threadIdx.x & 63;
  mx = -INFINITY;
  for (int t = 0; t < n; ++t) mx = fmaxf(mx, get(t, -1));
#pragma unroll
  for (int i = 0; i < DPC; ++i) acc[i] = 0.f;
  float l = 0.f;
  if (mx == -INFINITY) return 0.f;  // nothing readable
  for (int t = 0; t < n; ++t) {
    const float wgt = __builtin_amdgcn_exp2f(get(t, -1) - mx);
    l = fmaf(wgt, get(t, -2), l);
    if (lane * DPC < E) {
#pragma unroll
      for (int i = 0; i < DPC; ++i) acc[i] = fmaf(wgt, get(t, lane * DPC + i), acc[i]);
    }
  }
  return l;
}

// Counts one more block of a row in: the counter word holds the call's tag (high
// 32 bits) and the blocks counted so far (low 32).  A word with another tag (a
// fresh workspace's contents, or 0, which the row's last block leaves behind and
// no call uses as its tag) counts as none.  Returns the count including this
// block.  Each failed compare-and-swap means another block's succeeded, so the
// loop ends after at most one try per block of the row.
__device__ __forceinline__ int merge_count_in(uint64_t* ctr, uint32_t tag) {
  uint64_t cur = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    const uint64_t want = (uint32_t)(cur >> 32) == tag ? cur + 1 : ((uint64_t)tag << 32) | 1u;
    if (__hip_atomic_compare_exchange_strong(ctr, &cur, want, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT))
      return (int)(uint32_t)want;
  }
}

// One wave per TK-key tile of each row, 8 tiles per block merged in LDS.
// APPEND: the call's one-token append is done here (p.k_new).
template <int E, bool BF, bool COHERENT>
__device__ __forceinline__ void merge_partials(const DecodeParams& p, int64_t row, int n, int lane);

template <int E, bool BF, bool APPEND, int TK>
__global__ __launch_bounds__(64 * kDecWaves) __attribute__((amdgpu_waves_per_eu(4)))
void decode_tiles_kernel(DecodeParams p) {
  __shared__ __attribute__((aligned(16))) float p_lds[kDecWaves][TK];
  __shared__ float part[kDecWaves][E + 2];
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = blockIdx.x;
  const int64_t s = row / p.heads, h = row - s * p.heads;
  const int64_t tile = (int64_t)blockIdx.y * kDecWaves + wv;
  const int64_t len = row_len(p, s);
  const int64_t t0 = tile * TK;
  // Waves past the row's end exit (whole waves: the barrier below waits for the
  // others only), except the first wave of the row, which writes a row with no
  // key as exactly 0.
  if (t0 >= len && tile != 0) return;
  RowState<E, BF> st;
  st.init();
  // The appended token (lens[s] is the length before it) sits in this wave's
  // tile when its position is one the row attends.
  int newj = -1;
  if (APPEND) {
    const int64_t pos = p.lens[s];
    if (pos >= t0 && pos < t0 + TK && pos < len) newj = (int)(pos - t0);
  }
  if (t0 < len) decode_tile<E, BF, APPEND, TK>(p, s, h, t0, (int)min<int64_t>(TK, len - t0), newj, p_lds[wv], st);
  wave_partial<E, BF>(st, part[wv]);
  __syncthreads();
  if (wv != 0) return;
  constexpr int DPC = E >= 64 ? E / 64 : 1;
  const int lane = threadIdx.x & 63;
  const int n = (int)max<int64_t>(1, min<int64_t>(kDecWaves, cdiv(len, TK) - (int64_t)blockIdx.y * kDecWaves));
  float mx, acc[DPC];
  const float l = merge_states<E, DPC>(n, [&](int t, int i) {
    return part[t][i == -1 ? E : (i == -2 ? E + 1 : i)];
  }, mx, acc);
  if (blockIdx.y == 0 && len <= kDecWaves * TK) {
    if (lane * DPC < E) store_out<DPC, BF>(p.out, row * E + lane * DPC, acc, l > 0.f ? 1.f / l : 0.f);
  } else if (!p.counters) {
    const int64_t slot = row * cdiv(p.tiles, kDecWaves) + blockIdx.y;
    if (lane * DPC < E) {
#pragma unroll
      for (int i = 0; i < DPC; ++i) p.part_acc[slot * E + lane * DPC + i] = acc[i];
    }
    if (lane == 0) {
      p.part_ml[2 * slot] = mx;
      p.part_ml[2 * slot + 1] = l;
    }
  } else {
    // In-kernel merge: the partial is written with agent-scope atomic stores,
    // which the hardware makes visible device-wide (they write through the
    // XCD's L2) by the time the wave's store counter reaches zero; only then does
    // the block count itself in on the row's counter.  The block that completes
    // the count has seen every other block's count, hence every other partial,
    // and reads them with agent-scope atomic loads: no L2 write-back or
    // invalidation, which agent-scope fences would do for the whole L2.
    const int64_t slot = row * cdiv(p.tiles, kDecWaves) + blockIdx.y;
    if (lane * DPC < E) {
#pragma unroll
      for (int i = 0; i < DPC; ++i)
        __hip_atomic_store(p.part_acc + slot * E + lane * DPC + i, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane == 0) {
      __hip_atomic_store(p.part_ml + 2 * slot, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.part_ml + 2 * slot + 1, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const int nrow = (int)cdiv(len, (int64_t)kDecWaves * TK);
    int arrived = 0;
    if (lane == 0) arrived = merge_count_in(p.counters + row, p.tag);
    arrived = __builtin_amdgcn_readfirstlane(arrived);
    if (arrived != nrow) return;
    asm volatile("" ::: "memory");
    if (lane == 0) __hip_atomic_store(p.counters + row, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    merge_partials<E, BF, true>(p, row, nrow, lane);
  }
}

// One wave per row longer than one block: merges the blocks' partials.  The
// partials are read C at a time, every load of a round issued before any is used
// (the kernel is latency-bound: a row has a few KB of partials); rounds merge
// online.  A row of at most C blocks merges in one round, with the same
// arithmetic as a single pass (weights 2^(m_t - M) against the row's max M).
// A partial-slot float: a plain load, or (COHERENT) a relaxed agent-scope atomic
// load, which reads the value the device-wide coherence point holds (the in-kernel
// merge reads partials other blocks, perhaps on other XCDs, wrote this launch).
template <bool COHERENT>
__device__ __forceinline__ float slot_load(float* q) {
  if constexpr (COHERENT) return __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *q;
}

// Merges row `row`'s n block partials (slots row * nb .. + n - 1) and writes the
// row's output: one wave, lane l taking dims l * DPC ...
template <int E, bool BF, bool COHERENT>
__device__ __forceinline__ void merge_partials(const DecodeParams& p, int64_t row, int n, int lane) {
  constexpr int DPC = E >= 64 ? E / 64 : 1;
  constexpr int C = 8;
  const int64_t nb = cdiv(p.tiles, kDecWaves);
  const bool dims = lane * DPC < E;
  float* ml = p.part_ml + row * nb * 2;
  float* pa = p.part_acc + row * nb * E + (dims ? lane * DPC : 0);
  float m = -INFINITY, l = 0.f, acc[DPC];
#pragma unroll
  for (int i = 0; i < DPC; ++i) acc[i] = 0.f;
  for (int t0 = 0; t0 < n; t0 += C) {
    float mt[C], lt[C], at[C][DPC];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const bool in = t0 + c < n;
      mt[c] = in ? slot_load<COHERENT>(ml + 2 * (t0 + c)) : -INFINITY;
      lt[c] = in ? slot_load<COHERENT>(ml + 2 * (t0 + c) + 1) : 0.f;
#pragma unroll
      for (int i = 0; i < DPC; ++i) at[c][i] = in && dims ? slot_load<COHERENT>(pa + (int64_t)(t0 + c) * E + i) : 0.f;
    }
    float mc = m;
#pragma unroll
    for (int c = 0; c < C; ++c) mc = fmaxf(mc, mt[c]);
    if (mc == -INFINITY) continue;  // nothing readable yet
    const float sc = __builtin_amdgcn_exp2f(m - mc);  // 0 on the first readable round
    l *= sc;
#pragma unroll
    for (int i = 0; i < DPC; ++i) acc[i] *= sc;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float w = __builtin_amdgcn_exp2f(mt[c] - mc);
      l = fmaf(w, lt[c], l);
#pragma unroll
      for (int i = 0; i < DPC; ++i) acc[i] = fmaf(w, at[c][i], acc[i]);
    }
    m = mc;
  }
  if (dims) store_out<DPC, BF>(p.out, row * E + lane * DPC, acc, l > 0.f ? 1.f / l : 0.f);
}

template <int E, bool BF>
__global__ __launch_bounds__(256) void decode_tiles_combine_kernel(DecodeParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= p.nseqs * p.heads) return;
  const int64_t len = row_len(p, row / p.heads);
  const int64_t span = (int64_t)kDecWaves * p.tile_keys;  // keys per block
  if (len <= span) return;  // written by its block
  merge_partials<E, BF, false>(p, row, (int)cdiv(len, span), lane);
}

// Tile size of a call.  64-key tiles give a row four times the waves of 256-key
// tiles, each with a quarter of the serial load batches (one K batch, one V batch),
// so more loads are in flight per CU; measured on MI355X with flushed caches they
// win from batch-1 decode (N=1 H=32 E=128, 4096 keys: 41 -> 23 us) up to the
// largest batches (N=64 H=32 E=128, lengths 17..2047: 196 -> 185 us; N=64 H=16
// E=128 fp32: 276 -> 208 us).  They lose where every row fits one 256-key block
// (2048 keys, so no combine pass), those blocks already give every CU one (256
// rows or more), the call is small, and its rows are narrow (E * esize at most 128
// bytes: a 256-key tile's K and V within 64 KB): there the merge the 64-key tiles
// need costs more than they save (bf16 N=8 H=32 E=64 P=32, lengths 17..2047: 14.5
// -> 16.2 us; E=32: 9.3 -> 12.5 us).  Wider rows load too much per wave for one
// 256-key tile: bf16 E=128 N=8 H=32 at 2048 keys 53.4 -> 44.5 us, N=16 H=32 at 1024
// keys 53.1 -> 45.2 us, fp32 E=64 N=64 H=8 at 2048 keys 100.9 -> 86.4 us, fp32
// E=128 N=16 H=16 at lengths up to 1500 85.2 -> 73.3 us.  A page table of at most
// 512 keys takes 64-key tiles whatever the rows: one block of them covers a row, so
// nothing is merged, and a row gets 8 waves instead of 2 (fp32 N=128 H=8 E=128 at 512
// keys 180.2 -> 103.2 us, bf16 55.5 -> 46.4 us; bf16 N=64 H=32 E=64 59.9 -> 48.7 us;
// bf16 N=256 H=8 E=64 at 128 keys 22.2 -> 18.6 us).  The rule depends on shapes and
// the element size only (not on lengths), so the workspace size does too.
int decode_tile_keys(int64_t rows, int64_t pt_width, int64_t page, int64_t head_dim, int esize) {
  const int64_t cap = pt_width * page;
  if (cap <= (int64_t)kDecWaves * kShortTile) return kShortTile;
  const bool one_block = cap <= (int64_t)kDecWaves * kTile;
  const bool fills = rows >= 256;
  const bool small = rows * cap * head_dim <= (80ll << 20);  // K elements at capacity
  const bool narrow = head_dim * esize <= 128;
  return one_block && fills && small && narrow ? kTile : kShortTile;
}

int64_t decode_tiles(int64_t pt_width, int64_t page, int tile_keys) { return cdiv(pt_width * page, tile_keys); }

// Partial slots the workspace must hold: one per (row, block of 8 tiles) when
// rows can outgrow one block, none otherwise.
int64_t decode_workspace_slots(int64_t rows, int64_t tiles) {
  return tiles > kDecWaves ? rows * cdiv(tiles, kDecWaves) : 0;
}

template <int E, bool BF, bool APPEND, int TK>
static void decode_tiles_launch(const DecodeParams& p, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((decode_tiles_kernel<E, BF, APPEND, TK>), grid, dim3(64 * kDecWaves), 0, stream, p);
}

template <int E, bool BF>
static int decode_launch_t(const DecodeParams& p, hipStream_t stream) {
  const int64_t rows = p.nseqs * p.heads;
  const int64_t gy = cdiv(p.tiles, kDecWaves);
  if (rows > 0x7fffffff || gy > 65535 || decode_workspace_slots(rows, p.tiles) > p.slots ||
      (p.tile_keys != kTile && p.tile_keys != kShortTile))
    return CA_DECLINED;
  const dim3 grid((unsigned)rows, (unsigned)gy);
  const bool append = p.k_new != nullptr;
  if (p.tile_keys == kShortTile)
    append ? decode_tiles_launch<E, BF, true, kShortTile>(p, grid, stream)
           : decode_tiles_launch<E, BF, false, kShortTile>(p, grid, stream);
  else
    append ? decode_tiles_launch<E, BF, true, kTile>(p, grid, stream)
           : decode_tiles_launch<E, BF, false, kTile>(p, grid, stream);
  int st = ca_launch_status();
  if (st != CA_OK || gy == 1 || p.counters) return st;
  hipLaunchKernelGGL((decode_tiles_combine_kernel<E, BF>), dim3((unsigned)cdiv(rows, 4)), dim3(256),
                     0, stream, p);
  return ca_launch_status();
}

int decode_launch(const DecodeParams& p, int E, int bf16, hipStream_t stream) {
  if (p.nseqs == 0) return CA_OK;
  if (bf16) {
    switch (E) {
      case 32: return decode_launch_t<32, true>(p, stream);
      case 64: return decode_launch_t<64, true>(p, stream);
      case 128: return decode_launch_t<128, true>(p, stream);
    }
  } else {
    switch (E) {
      case 32: return decode_launch_t<32, false>(p, stream);
      case 64: return decode_launch_t<64, false>(p, stream);
      case 128: return decode_launch_t<128, false>(p, stream);
    }
  }
  return CA_DECLINED;
}

}  // namespace ca
