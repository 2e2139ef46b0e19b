// Paged decode, split-K: one wave scores one 256-key tile of one (sequence, head)
// and leaves a partial (max, sum, P@V) that a combine pass merges.
//
// Follows the reference's decode (cpu_attention/_mojo/src/paged_attn.mojo:714-782):
// logits q.k, base-2 online softmax with c = scale*log2(e) and the running max in
// scaled log2 units, fp32 P against fp32-widened V, out = acc * (1/l), and a row
// that saw no key is exactly 0 (_store_row :297-319).  Keys past the length are
// never read (0 * NaN would poison the row, :686-687), nor are page-table entries
// past the last page in use.
//
// Layout use (the reference's PageLayout, :58-130): a 16-key unit never straddles a
// page (P % 16 == 0), so a tile is 16 units, each one contiguous run inside one
// (block, head):
//   Q.K  lane l owns keys 4l..4l+3 of the tile; one 16-byte load per K word row
//        (w*P + t .. t+3) gives those 4 keys' word w, so the dot product needs no
//        cross-lane reduction.  bf16 words are dim pairs: v_dot2_f32_bf16 with the
//        matching q pair (exact products, fp32 accumulation).
//   P.V  lane groups of E/8 (bf16) or E/4 (fp32) lanes read whole V rows with
//        16-byte loads, G rows per wave instruction; p comes from LDS.
#include "ca_device.h"
#include "ca_internal.h"

namespace ca {

constexpr int kTile = 256;  // keys per wave tile
constexpr int kUnit = 16;   // keys per unit (one page run)

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

__device__ __forceinline__ int64_t readlane64(int64_t x, int lane) {
  const int lo = __builtin_amdgcn_readlane((int)(x & 0xffffffff), lane);
  const int hi = __builtin_amdgcn_readlane((int)(x >> 32), lane);
  return (int64_t)(uint32_t)lo | ((int64_t)hi << 32);
}

template <int E, bool BF>
__global__ __launch_bounds__(256) void decode_partial_kernel(DecodeParams p) {
  constexpr int ES = BF ? 2 : 4;    // element bytes
  constexpr int W = E * ES / 4;     // K words per key (per head)
  constexpr int DPL = 16 / ES;      // V elements per 16-byte load
  constexpr int LPR = E / DPL;      // lanes per V row
  constexpr int G = kWave / LPR;    // V rows per wave load
  constexpr int UNROLL = 16;
  static_assert(W % UNROLL == 0 && kUnit % G == 0, "tile shape");
  __shared__ __attribute__((aligned(16))) float p_lds[4][kTile];

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t pair = blockIdx.x;
  const int64_t seq = pair / p.heads, h = pair - seq * p.heads;
  const int tile = blockIdx.y * 4 + wv;
  const int64_t cap = p.pt_width * p.page;
  int64_t len = (int64_t)p.lens[seq] + p.len_add;
  len = len < cap ? len : cap;
  const int64_t t0 = (int64_t)tile * kTile;
  if (len <= 0 || t0 >= len) return;
  const int ntok = (int)min<int64_t>(kTile, len - t0);

  // Unit table: lane u < 16 resolves unit u's page once (word index of its K run,
  // element index of its V rows); -1 marks a unit past the length or a page-table
  // entry that names no block.
  int64_t kb = -1, vb = -1;
  if (lane < kTile / kUnit) {
    const int64_t tu = t0 + kUnit * lane;
    if (tu < len) {
      const int64_t pi = tu / p.page, off = tu - pi * p.page;
      const int64_t blk = p.page_table[seq * p.pt_width + pi];
      if (blk >= 0 && blk < p.nblocks) {
        const int64_t base = (blk * p.heads + h) * p.page;
        kb = base * W + off;
        vb = (base + off) * E;
      }
    }
  }

  // ---- Q.K: keys 4*lane .. 4*lane+3 of the tile.
  float s[4];
  {
    const int u = lane >> 2;
    const int64_t kbu = __shfl(kb, u);
    const int64_t key0 = t0 + 4 * lane;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (kbu >= 0 && key0 < len) {
      const uint32_t* kp = p.kc + kbu + 4 * (lane & 3);
      if constexpr (BF) {
        const uint32_t* qw = reinterpret_cast<const uint32_t*>(
            reinterpret_cast<const uint16_t*>(p.q) + seq * p.q_stride + h * E);
        for (int w0 = 0; w0 < W; w0 += UNROLL) {
          u32x4 k4[UNROLL];
#pragma unroll
          for (int i = 0; i < UNROLL; ++i)
            k4[i] = *reinterpret_cast<const u32x4*>(kp + (int64_t)(w0 + i) * p.page);
#pragma unroll
          for (int i = 0; i < UNROLL; ++i) {
            const bf16x2 qv = as_bf16x2(qw[w0 + i]);
            a0 = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k4[i].x), qv, a0, false);
            a1 = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k4[i].y), qv, a1, false);
            a2 = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k4[i].z), qv, a2, false);
            a3 = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(k4[i].w), qv, a3, false);
          }
        }
      } else {
        // Four partial sums per key (words w mod 4): 32-term chains instead of one
        // 128-term chain keep the fp32 logits well inside the 1e-6 decode gate.
        const float* qf = reinterpret_cast<const float*>(p.q) + seq * p.q_stride + h * E;
        float c0[4] = {0.f, 0.f, 0.f, 0.f}, c1[4] = {0.f, 0.f, 0.f, 0.f};
        float c2[4] = {0.f, 0.f, 0.f, 0.f}, c3[4] = {0.f, 0.f, 0.f, 0.f};
        for (int w0 = 0; w0 < W; w0 += UNROLL) {
          u32x4 k4[UNROLL];
#pragma unroll
          for (int i = 0; i < UNROLL; ++i)
            k4[i] = *reinterpret_cast<const u32x4*>(kp + (int64_t)(w0 + i) * p.page);
#pragma unroll
          for (int i = 0; i < UNROLL; ++i) {
            const float qv = qf[w0 + i];
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
    // Raw logits (masked keys -inf); the scale is folded into the exponent below.
    const bool ok = kbu >= 0;
    s[0] = (ok && key0 + 0 < len) ? a0 : -INFINITY;
    s[1] = (ok && key0 + 1 < len) ? a1 : -INFINITY;
    s[2] = (ok && key0 + 2 < len) ? a2 : -INFINITY;
    s[3] = (ok && key0 + 3 < len) ? a3 : -INFINITY;
  }

  // ---- softmax over the tile: m = max(logit)*c in scaled log2 units and
  // p = 2^(logit*c - m), one rounding inside the exponent (the reference's
  // fma(logit, c, -m), flash_vec.mojo:255-259; paged_attn.mojo:643-676).
  const float mraw = wave_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
  const float m = mraw * p.c;
  const float mu = mraw == -INFINITY ? 0.f : m;  // a tile with no readable key
  float pr[4], lsum = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    pr[j] = __builtin_amdgcn_exp2f(fmaf(s[j], p.c, -mu));
    lsum += pr[j];
  }
  lsum = wave_sum(lsum);
  *reinterpret_cast<f32x4*>(&p_lds[wv][4 * lane]) = f32x4{pr[0], pr[1], pr[2], pr[3]};
  wave_lds_sync();

  // ---- P.V: lane (g, dl) takes dims dl*DPL.. of keys g, g+G, ... of each unit.
  const int g = lane / LPR, dl = lane - g * LPR;
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
  const char* vbase = reinterpret_cast<const char*>(p.vc) + dl * 16;
  const int nunits = (ntok + kUnit - 1) / kUnit;
  constexpr int LPU = kUnit / G;                  // V loads per unit per lane
  constexpr int UG = LPU >= 16 ? 1 : 16 / LPU;    // units per batch: 16 loads in flight
  for (int u0 = 0; u0 < nunits; u0 += UG) {
    u32x4 v4[UG][LPU];
    bool ok[UG][LPU];
#pragma unroll
    for (int uu = 0; uu < UG; ++uu) {
      const int u = u0 + uu;  // < 16: UG divides the 16 units of a tile
      const int64_t vbu = readlane64(vb, u);
#pragma unroll
      for (int jj = 0; jj < LPU; ++jj) {
        const int x = jj * G + g;
        ok[uu][jj] = vbu >= 0 && kUnit * u + x < ntok;
        if (ok[uu][jj])
          v4[uu][jj] = *reinterpret_cast<const u32x4*>(vbase + (vbu + (int64_t)x * E) * ES);
      }
    }
#pragma unroll
    for (int uu = 0; uu < UG; ++uu) {
#pragma unroll
      for (int jj = 0; jj < LPU; ++jj) {
        if (ok[uu][jj]) {
          const float pj = p_lds[wv][kUnit * (u0 + uu) + jj * G + g];
          const u32x4 v = v4[uu][jj];
          if constexpr (BF) {
            acc[0] = fmaf(pj, bf16_lo(v.x), acc[0]);
            acc[1] = fmaf(pj, bf16_hi(v.x), acc[1]);
            acc[2] = fmaf(pj, bf16_lo(v.y), acc[2]);
            acc[3] = fmaf(pj, bf16_hi(v.y), acc[3]);
            acc[4] = fmaf(pj, bf16_lo(v.z), acc[4]);
            acc[5] = fmaf(pj, bf16_hi(v.z), acc[5]);
            acc[6] = fmaf(pj, bf16_lo(v.w), acc[6]);
            acc[7] = fmaf(pj, bf16_hi(v.w), acc[7]);
          } else {
            acc[0] = fmaf(pj, __uint_as_float(v.x), acc[0]);
            acc[1] = fmaf(pj, __uint_as_float(v.y), acc[1]);
            acc[2] = fmaf(pj, __uint_as_float(v.z), acc[2]);
            acc[3] = fmaf(pj, __uint_as_float(v.w), acc[3]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int o = LPR; o < kWave; o <<= 1)
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] += __shfl_xor(acc[i], o);

  if (g == 0) {
    if (len <= kTile) {
      // The only tile of this row: write the output here (the combine skips it).
      store_out<DPL, BF>(p.out, pair * E + dl * DPL, acc, lsum > 0.f ? 1.f / lsum : 0.f);
    } else {
      float* pa = p.part_acc + (pair * p.tiles + tile) * E + dl * DPL;
#pragma unroll
      for (int i = 0; i < DPL; i += 4)
        *reinterpret_cast<f32x4*>(pa + i) = f32x4{acc[i], acc[i + 1], acc[i + 2], acc[i + 3]};
      if (lane == 0) {
        p.part_ml[(pair * p.tiles + tile) * 2 + 0] = m;
        p.part_ml[(pair * p.tiles + tile) * 2 + 1] = lsum;
      }
    }
  }
}

// One wave per (sequence, head): merge the tiles' partials into the output.
template <int E, bool BF>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeParams p) {
  constexpr int DPC = E >= 64 ? E / 64 : 1;  // dims per lane
  constexpr int ACTIVE = E / DPC;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t pair = (int64_t)blockIdx.x * 4 + wv;
  if (pair >= p.nseqs * p.heads) return;
  const int64_t seq = pair / p.heads;
  const int64_t cap = p.pt_width * p.page;
  int64_t len = (int64_t)p.lens[seq] + p.len_add;
  len = len < cap ? len : cap;
  float acc[DPC];
#pragma unroll
  for (int i = 0; i < DPC; ++i) acc[i] = 0.f;
  if (len > 0 && len <= kTile) return;  // written by the tile itself
  float inv = 0.f;
  if (len > 0) {
    const int nt = (int)((len + kTile - 1) / kTile);
    const float* ml = p.part_ml + pair * p.tiles * 2;
    float mx = -INFINITY;
    for (int t = lane; t < nt; t += kWave) mx = fmaxf(mx, ml[2 * t]);
    mx = wave_max(mx);
    if (mx != -INFINITY) {
      float l = 0.f;
      const float* pa = p.part_acc + pair * p.tiles * E + lane * DPC;
      for (int t = 0; t < nt; ++t) {
        const float wgt = __builtin_amdgcn_exp2f(ml[2 * t] - mx);
        l = fmaf(wgt, ml[2 * t + 1], l);
        if (lane < ACTIVE) {
#pragma unroll
          for (int i = 0; i < DPC; ++i) acc[i] = fmaf(wgt, pa[(int64_t)t * E + i], acc[i]);
        }
      }
      inv = l > 0.f ? 1.f / l : 0.f;
    }
  }
  if (lane < ACTIVE) store_out<DPC, BF>(p.out, pair * E + lane * DPC, acc, inv);
}

int64_t decode_tiles(int64_t pt_width, int64_t page) { return cdiv(pt_width * page, kTile); }

template <int E, bool BF>
static int decode_launch_t(const DecodeParams& p, hipStream_t stream) {
  const int64_t pairs = p.nseqs * p.heads;
  const int64_t gy = cdiv(p.tiles, 4);
  if (pairs > 0x7fffffff || gy > 65535) return CA_DECLINED;
  // grid.x = (sequence, head), grid.y = tile group: every row's first tiles are
  // dispatched first, the (mostly empty) tail tiles of short rows last.
  hipLaunchKernelGGL((decode_partial_kernel<E, BF>), dim3((unsigned)pairs, (unsigned)gy),
                     dim3(256), 0, stream, p);
  int st = ca_launch_status();
  if (st != CA_OK) return st;
  hipLaunchKernelGGL((decode_combine_kernel<E, BF>), dim3((unsigned)cdiv(pairs, 4)), dim3(256),
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
