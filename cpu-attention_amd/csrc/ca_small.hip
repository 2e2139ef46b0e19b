// Dense bf16 prefill over short key ranges (at most kSmallMaxKeys = 256 keys): the
// reference's flash_attn_func (flash_attn.mojo:127-183) for calls such as a short
// prompt, where every key fits in registers.  The tiled kernel would spend such a
// call on its per-pass pipeline (first-tile waits, the first softmax, the last
// P.V, the staged store) around one or two key tiles; here each query row's
// logits are all computed before its softmax, so the row max is exact and there
// is one dependent memory round trip before the MFMAs.
//
// One wave (= one block) per (batch, head, 32 query rows).  With the 32x32x16
// bf16 MFMA (lane l supplies row l % 32 and the 8 k-indices 8 * (l / 32) .. +7 of
// each operand; accumulator register r of lane l holds row 8 * (r / 4) +
// 4 * (l / 32) + r % 4, column l % 32):
//   S^T = K Q^T per 32-key block: A = 32 keys' dims straight from K rows, B = the
//        wave's 32 query rows' dims from Q rows (16-byte loads);
//   each lane then holds 16 keys of one query row per block: the softmax needs
//        one exchange with the lane 32 away;
//   O^T = V^T P^T per 16 keys: B = P^T is the lane's own 8 probabilities of the
//        step (a permutation of the step's keys, the same for both operands), A =
//        V^T read from the V rows staged in the wave's LDS with ds_read_b64_tr_b16
//        (lane j of a 16-lane group gets column j of a 4-row x 16-column block:
//        4 keys of one dim), two reads per operand.
// No barrier: the block is one wave.  Numerics are the reference's bf16 policy: fp32 logits,
// p = 2^(s*c - max) with l summing the unrounded p, P rounded to bf16 for P.V,
// the output rounded once; a row that sees no key is 0.
#include "ca_device.h"
#include "ca_internal.h"

namespace ca {

// Block bx of gx: batch b, head h, query rows [r0, r0 + kSmallRows).  Row blocks
// of one head are consecutive on an XCD, so they meet its K and V in one L2.
struct SmallWork {
  int64_t b, h;
  int r0;
};
__host__ __device__ inline SmallWork small_work(const FlashParams& p, int64_t bx, int64_t gx) {
  const int64_t nrb = cdiv(p.seq_q, kSmallRows);
  const int64_t lb = xcd_remap(bx, gx);
  const int64_t bh = lb / nrb;
  SmallWork w;
  w.b = bh / p.heads;
  w.h = bh - w.b * p.heads;
  w.r0 = (int)((lb - bh * nrb) * kSmallRows);
  return w;
}

// Keys query row i sees: [0, small_kend).  Causal is bottom-right aligned:
// key j is visible to row i when j <= i + seq_k - seq_q.
__host__ __device__ inline int small_kend(const FlashParams& p, int64_t i) {
  if (!p.causal) return (int)p.seq_k;
  const int64_t e = i + 1 + p.seq_k - p.seq_q;
  return (int)(e < 0 ? 0 : (e > p.seq_k ? p.seq_k : e));
}

// Row of a 32x32 accumulator block held by register r of a lane in half hf.
__host__ __device__ inline int small_acc_row(int r, int hf) { return 8 * (r >> 2) + 4 * hf + (r & 3); }

// Key (within a 32-key block) of k-index 8 * hf + t of the block's P.V step u: the
// key whose probability the lane holds in register 8 * u + t of the block's S^T.
__host__ __device__ inline int small_pv_key(int u, int hf, int t) { return small_acc_row(8 * u + t, hf); }

// The key row a load of key `key` reads: keys past the last read the last.
__host__ __device__ inline int small_clamp_key(int key, int S) { return key < S ? key : S - 1; }


typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 small_bf16x4;
typedef __attribute__((address_space(3))) small_bf16x4 small_lds_bf16x4;

// V^T operand of the P.V MFMA for keys 16 cc .. and dims 32 d ..: lane (dim j +
// 16 dh, half hf) gets keys 16 cc + 4 hf + 0..3 and 16 cc + 8 + 4 hf + 0..3, the
// keys small_pv_key gives for the lane's half.
template <int E>
__device__ __forceinline__ bf16x8 small_v_operand(const uint16_t* vs, int lane, int cc, int d) {
  constexpr int RS = small_rsv(E) * 8;  // elements per LDS row
  const int j = lane & 15, dh = (lane >> 4) & 1, hf = lane >> 5;
  const uint16_t* base = vs + (4 * hf + (j >> 2)) * RS + 16 * dh + 4 * (j & 3);
  small_bf16x4 a[2];
#pragma unroll
  for (int q = 0; q < 2; ++q)
    a[q] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((small_lds_bf16x4*)(base + (16 * cc + 8 * q) * RS + 32 * d));
  return bf16x8{a[0][0], a[0][1], a[0][2], a[0][3], a[1][0], a[1][1], a[1][2], a[1][3]};
}

template <int E, int NKB>
__global__ __launch_bounds__(64) void flash_small_kernel(FlashParams p) {
  constexpr int NKS = E / 16;  // 16-dim steps of S
  constexpr int NDB = E / 32;  // 32-dim blocks of O
  const int lane = threadIdx.x, n = lane & 31, hf = lane >> 5;
  const SmallWork w = small_work(p, blockIdx.x, gridDim.x);
  const int L = (int)p.seq_q, S = (int)p.seq_k;
  const uint16_t* qp = static_cast<const uint16_t*>(p.q) + w.b * p.qs[0] + w.h * p.qs[2];
  const uint16_t* kp = static_cast<const uint16_t*>(p.k) + w.b * p.ks[0] + w.h * p.ks[2];
  const uint16_t* vp = static_cast<const uint16_t*>(p.v) + w.b * p.vs[0] + w.h * p.vs[2];
  const int row = w.r0 + n;  // the query row of this lane's accumulator column
  const bool live = row < L;

  // Every load is unconditional, so the wave issues all of them before its
  // first wait: rows past the tensor's read its last row instead (row L - 1 for
  // Q, whose results are never stored; key S - 1 for K, whose logits are masked,
  // and for V, whose values are replaced by zeros).  K and V rows are addressed
  // by 32-bit byte offsets from the (batch, head) base: the plan keeps seq_k
  // token strides under 2^32 bytes.
  // Q^T operand: row `row`, dims 16 ks + 8 hf .. +7.
  const int64_t qrow = live ? row : L - 1;
  bf16x8 qo[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks)
    qo[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(qp + qrow * p.qs[1] + 16 * ks + 8 * hf));
  // S^T per 32-key block: A = K row 32 kb + n.
  f32x16 s[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    const uint32_t koff = (uint32_t)small_clamp_key(32 * kb + n, S) * (uint32_t)p.ks[1] * 2u;
    u32x4 ko[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      ko[ks] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(kp) + koff + (16 * ks + 8 * hf) * 2);
    f32x16 acc = {};
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ko[ks]), qo[ks], acc, 0, 0, 0);
    s[kb] = acc;
  }
  // V rows 0 .. 32 NKB - 1 into the wave's LDS (zero past the keys), 16 bytes per
  // lane and load: chunk c of the rows is row c / CPR, column chunk c % CPR.
  constexpr int CPR = E / 8, RS = small_rsv(E) * 8, NVL = NKB * 32 * CPR / 64;
  __shared__ __attribute__((aligned(16))) uint16_t vs[NKB * 32 * RS];
  {
    u32x4 vr[NVL];
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
      const int c = lane + 64 * i, key = c / CPR, col = c % CPR;
      const uint32_t voff = (uint32_t)small_clamp_key(key, S) * (uint32_t)p.vs[1] * 2u + col * 16;
      vr[i] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(vp) + voff);
    }
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
      const int c = lane + 64 * i, key = c / CPR, col = c % CPR;
      *reinterpret_cast<u32x4*>(vs + key * RS + col * 8) = key < S ? vr[i] : u32x4{0u, 0u, 0u, 0u};
    }
  }

  // Softmax of the row (base 2, scaled logits), masked to the row's keys.
  const int kend = live ? small_kend(p, row) : 0;
  float m = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float x = 32 * kb + small_acc_row(r, hf) < kend ? s[kb][r] * p.c : -INFINITY;
      s[kb][r] = x;
      m = fmaxf(m, x);
    }
  m = fmaxf(m, __shfl_xor(m, 32));
  const float mm = m == -INFINITY ? 0.f : m;  // a row with no key: every p is 0
  float l = 0.f;
  bf16x8 pk[NKB][2];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      uint32_t wd[4];
#pragma unroll
      for (int t = 0; t < 8; t += 2) {
        const float e0 = __builtin_amdgcn_exp2f(s[kb][8 * u + t] - mm);
        const float e1 = __builtin_amdgcn_exp2f(s[kb][8 * u + t + 1] - mm);
        l += e0 + e1;
        wd[t / 2] = pack_bf16x2(e0, e1);
      }
      pk[kb][u] = __builtin_bit_cast(bf16x8, u32x4{wd[0], wd[1], wd[2], wd[3]});
    }
  l += __shfl_xor(l, 32);

  // O^T = V^T P^T, then out = O / l (rows < L only).
  wave_lds_sync();  // the staged V rows before the transposed reads
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* out = static_cast<uint16_t*>(p.out) + ((w.b * L + row) * p.heads + w.h) * (int64_t)E;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    f32x16 o = {};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        o = __builtin_amdgcn_mfma_f32_32x32x16_bf16(small_v_operand<E>(vs, lane, 2 * kb + u, db), pk[kb][u], o, 0, 0,
                                                    0);
    if (live) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<u32x2*>(out + 32 * db + small_acc_row(4 * i, hf)) =
            u32x2{pack_bf16x2(o[4 * i] * inv, o[4 * i + 1] * inv), pack_bf16x2(o[4 * i + 2] * inv, o[4 * i + 3] * inv)};
    }
  }
}

template <int E>
static int small_launch_t(const FlashParams& p, const FlashPlan& plan, hipStream_t stream) {
  const dim3 grid((unsigned)plan.gx), block(64);
  switch (cdiv(p.seq_k, 32)) {
    case 1: hipLaunchKernelGGL((flash_small_kernel<E, 1>), grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((flash_small_kernel<E, 2>), grid, block, 0, stream, p); break;
    case 3: hipLaunchKernelGGL((flash_small_kernel<E, 3>), grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL((flash_small_kernel<E, 4>), grid, block, 0, stream, p); break;
    case 5: hipLaunchKernelGGL((flash_small_kernel<E, 5>), grid, block, 0, stream, p); break;
    case 6: hipLaunchKernelGGL((flash_small_kernel<E, 6>), grid, block, 0, stream, p); break;
    case 7: hipLaunchKernelGGL((flash_small_kernel<E, 7>), grid, block, 0, stream, p); break;
    case 8: hipLaunchKernelGGL((flash_small_kernel<E, 8>), grid, block, 0, stream, p); break;
    default: return CA_DECLINED;
  }
  return ca_launch_status();
}

FlashPlan small_plan(const FlashParams& p) {
  FlashPlan plan{};
  plan.kind = kPlanSmall;
  plan.gx = p.batch * p.heads * cdiv(p.seq_q, kSmallRows);
  plan.gy = plan.splits = 1;
  if (plan.gx > 0x7fffffff) plan.kind = kPlanDeclined;
  return plan;
}

int flash_small_launch(const FlashParams& p, const FlashPlan& plan, int E, hipStream_t stream) {
  switch (E) {
    case 32: return small_launch_t<32>(p, plan, stream);
    case 64: return small_launch_t<64>(p, plan, stream);
    case 128: return small_launch_t<128>(p, plan, stream);
  }
  return CA_DECLINED;
}

}  // namespace ca
