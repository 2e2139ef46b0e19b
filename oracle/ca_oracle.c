/*
 * ca_oracle.c -- TEST INFRASTRUCTURE / CPU BASELINE, NOT PRODUCT CODE.
 *
 * An fp32 C port of ducviet00/cpu-attention's CPU algorithms, used only by tests/
 * (cross-checked against the float64 oracle) and by bench.py's cpu_baseline leg
 * (timed on the GPU box's host cores).  The GPU path never calls it.
 *
 *   oracle_store   reshape_and_cache: PageLayout store_token / store_v
 *                  (cpu_attention/_mojo/src/paged_attn.mojo:72-113), slot semantics
 *                  of _store_kv (:151-176): negative slots skip.
 *   oracle_decode  paged decode per (sequence, head): key steps of KT keys, logits
 *                  q.k, running max in scaled log2 units with c = scale*log2(e),
 *                  alpha = 2^(m - m_new) (0 on the first step), p = 2^(x*c - m),
 *                  fp32 P against widened V, out = acc * (1/l), 0 when l <= 0
 *                  (_attend :714-782, _store_row :297-319).  libm exp2f stands in
 *                  for the reference's exp2 polynomial (isa.mojo:77-155).
 *   oracle_flash   prefill: bottom-right causal (row i sees keys j <= i + S - L),
 *                  key tiles, online softmax as above, bf16 P rounded to bf16 before
 *                  P.V (flash_vec.mojo:255-259), zero rows for rows with no key
 *                  (flash_attn.mojo:127-183).  K is packed transposed per
 *                  (batch, head) first, as the reference's split order packs slabs
 *                  (flash_attn.mojo:208-212).  Q K^T and P V run as AVX2/FMA register
 *                  tiles of 4 rows x 16 columns (AVX-512: 32, where the host has it) and
 *                  exp2 as a vector polynomial, as
 *                  the reference's vector policy vectorises its tiles (a baseline
 *                  should not be slowed by scalar code).  head_dim: a multiple of 16.
 *
 * Parallelised with OpenMP over independent work items; `threads` <= 0 uses the
 * OpenMP default.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define LOG2E 1.4426950408889634f
#define KT 256   /* keys per decode step */
#define FKT 64   /* keys per prefill tile */
#define FRQ 32   /* query rows per prefill work item */

static inline float bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f2bf(float f) {
  uint32_t u;
  if (isnan(f)) return 0x7fc0;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float ld(const void* p, int64_t i, int bf) {
  return bf ? bf2f(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

static inline void st(void* p, int64_t i, float x, int bf) {
  if (bf)
    ((uint16_t*)p)[i] = f2bf(x);
  else
    ((float*)p)[i] = x;
}

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
}

void oracle_store(const uint32_t* key, const uint32_t* value, int64_t tok_stride_w, uint32_t* kc,
                  uint32_t* vc, const int64_t* slots, int64_t ntok, int64_t heads, int64_t words,
                  int64_t page, int64_t nblocks, int threads) {
  set_threads(threads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < ntok; ++i) {
    const int64_t s = slots[i];
    if (s < 0 || s >= nblocks * page) continue;
    const int64_t blk = s / page, off = s % page;
    for (int64_t h = 0; h < heads; ++h) {
      const uint32_t* ks = key + i * tok_stride_w + h * words;
      const uint32_t* vs = value + i * tok_stride_w + h * words;
      uint32_t* kb = kc + (blk * heads + h) * page * words;
      uint32_t* vb = vc + ((blk * heads + h) * page + off) * words;
      for (int64_t w = 0; w < words; ++w) kb[w * page + off] = ks[w];
      memcpy(vb, vs, (size_t)words * 4);
    }
  }
}

void oracle_decode(int bf, const void* q, int64_t q_stride, const void* kc, const void* vc,
                   const int32_t* lens, const int32_t* page_table, int64_t width, int64_t nseqs,
                   int64_t heads, int64_t hd, int64_t page, float scale, void* out, int threads) {
  set_threads(threads);
  const float c = scale * LOG2E;
  const int64_t items = nseqs * heads;
#pragma omp parallel
  {
    float* logits = (float*)malloc(sizeof(float) * KT);
    float* acc = (float*)malloc(sizeof(float) * (size_t)hd);
    float* qv = (float*)malloc(sizeof(float) * (size_t)hd);
#pragma omp for schedule(dynamic, 1)
    for (int64_t it = 0; it < items; ++it) {
      const int64_t s = it / heads, h = it % heads;
      const int64_t len = lens[s] < width * page ? lens[s] : width * page;
      for (int64_t d = 0; d < hd; ++d) qv[d] = ld(q, s * q_stride + h * hd + d, bf);
      for (int64_t d = 0; d < hd; ++d) acc[d] = 0.f;
      float m = -INFINITY, l = 0.f;
      for (int64_t k0 = 0; k0 < len; k0 += KT) {
        const int64_t nk = len - k0 < KT ? len - k0 : KT;
        float mx = -INFINITY;
        /* Q.K over the step's page runs: K is [d][t] inside a block. */
        for (int64_t j = 0; j < nk;) {
          const int64_t t = k0 + j, off = t % page;
          const int64_t run = (page - off) < (nk - j) ? (page - off) : (nk - j);
          const int64_t blk = page_table[s * width + t / page];
          const int64_t base = (blk * heads + h) * page * hd;
          float* lg = logits + j;
          for (int64_t r = 0; r < run; ++r) lg[r] = 0.f;
          if (bf) {
            const uint32_t* kw = (const uint32_t*)kc + base / 2;
            for (int64_t d2 = 0; d2 < hd / 2; ++d2) {
              const float q0 = qv[2 * d2], q1 = qv[2 * d2 + 1];
              const uint32_t* row = kw + d2 * page + off;
              for (int64_t r = 0; r < run; ++r) {
                const uint32_t w = row[r];
                const uint32_t lo = w << 16, hi = w & 0xffff0000u;
                float flo, fhi;
                memcpy(&flo, &lo, 4);
                memcpy(&fhi, &hi, 4);
                lg[r] += q0 * flo + q1 * fhi;
              }
            }
          } else {
            const float* kf = (const float*)kc + base;
            for (int64_t d = 0; d < hd; ++d) {
              const float qd = qv[d];
              const float* row = kf + d * page + off;
              for (int64_t r = 0; r < run; ++r) lg[r] += qd * row[r];
            }
          }
          j += run;
        }
        for (int64_t j = 0; j < nk; ++j) mx = logits[j] > mx ? logits[j] : mx;
        const float m_new = k0 == 0 ? mx * c : fmaxf(m, mx * c);
        const float alpha = k0 == 0 ? 0.f : exp2f(m - m_new);
        m = m_new;
        float sum = 0.f;
        for (int64_t j = 0; j < nk; ++j) {
          logits[j] = exp2f(logits[j] * c - m);
          sum += logits[j];
        }
        l = l * alpha + sum;
        for (int64_t d = 0; d < hd; ++d) acc[d] *= alpha;
        for (int64_t j = 0; j < nk; ++j) {
          const int64_t t = k0 + j;
          const int64_t blk = page_table[s * width + t / page];
          const int64_t row = ((blk * heads + h) * page + t % page) * hd;
          const float p = logits[j];
          if (bf) {
            const uint16_t* vr = (const uint16_t*)vc + row;
            for (int64_t d = 0; d < hd; ++d) acc[d] += p * bf2f(vr[d]);
          } else {
            const float* vr = (const float*)vc + row;
            for (int64_t d = 0; d < hd; ++d) acc[d] += p * vr[d];
          }
        }
      }
      const float inv = l > 0.f ? 1.f / l : 0.f;
      for (int64_t d = 0; d < hd; ++d) st(out, (s * heads + h) * hd + d, l > 0.f ? acc[d] * inv : 0.f, bf);
    }
    free(logits);
    free(acc);
    free(qv);
  }
}

/* Vector helpers of the prefill port (AVX2 + FMA, the x86-64-v3 baseline). */
typedef __m256 v8;

/* 2^x for a vector: x = n + f with n = round(x), |f| <= 1/2, and 2^f = e^(f ln 2)
 * by the degree-6 Taylor polynomial of e^y (|y| <= 0.347: relative error below
 * 1.2e-7), scaled by 2^n through the exponent bits.  x below -126 (-inf
 * included) gives 0; the reference's own exp2 is a polynomial too
 * (isa.mojo:77-155). */
static inline v8 exp2v(v8 x) {
  const v8 lo = _mm256_set1_ps(-126.f);
  const v8 xc = _mm256_min_ps(_mm256_max_ps(x, lo), _mm256_set1_ps(127.f));
  const v8 n = _mm256_round_ps(xc, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  const v8 y = _mm256_mul_ps(_mm256_sub_ps(xc, n), _mm256_set1_ps(0.69314718055994531f));
  v8 e = _mm256_set1_ps(1.f / 720.f);
  e = _mm256_fmadd_ps(e, y, _mm256_set1_ps(1.f / 120.f));
  e = _mm256_fmadd_ps(e, y, _mm256_set1_ps(1.f / 24.f));
  e = _mm256_fmadd_ps(e, y, _mm256_set1_ps(1.f / 6.f));
  e = _mm256_fmadd_ps(e, y, _mm256_set1_ps(0.5f));
  e = _mm256_fmadd_ps(e, y, _mm256_set1_ps(1.f));
  e = _mm256_fmadd_ps(e, y, _mm256_set1_ps(1.f));
  const __m256i bits = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(n), _mm256_set1_epi32(127)), 23);
  const v8 r = _mm256_mul_ps(e, _mm256_castsi256_ps(bits));
  return _mm256_and_ps(r, _mm256_cmp_ps(x, lo, _CMP_GE_OQ));
}

/* Round to bf16 and back (round to nearest even; the probabilities are finite). */
static inline v8 bf16_round(v8 x) {
  const __m256i u = _mm256_castps_si256(x);
  const __m256i bias = _mm256_add_epi32(_mm256_set1_epi32(0x7fff), _mm256_and_si256(_mm256_srli_epi32(u, 16),
                                                                                     _mm256_set1_epi32(1)));
  return _mm256_castsi256_ps(_mm256_and_si256(_mm256_add_epi32(u, bias), _mm256_set1_epi32((int)0xffff0000u)));
}

static inline float hmax(v8 x) {
  __m128 m = _mm_max_ps(_mm256_castps256_ps128(x), _mm256_extractf128_ps(x, 1));
  m = _mm_max_ps(m, _mm_movehl_ps(m, m));
  m = _mm_max_ss(m, _mm_shuffle_ps(m, m, 1));
  return _mm_cvtss_f32(m);
}

static inline float hsum(v8 x) {
  __m128 m = _mm_add_ps(_mm256_castps256_ps128(x), _mm256_extractf128_ps(x, 1));
  m = _mm_add_ps(m, _mm_movehl_ps(m, m));
  m = _mm_add_ss(m, _mm_shuffle_ps(m, m, 1));
  return _mm_cvtss_f32(m);
}

/* S[4 rows][16 keys] = Q[4][hd] . K^T[hd][16]: kt points at key column 0 of the
 * 16, rows of K^T `ldk` floats apart. */
static inline void s_tile_4x16(const float* qb, int64_t hd, const float* kt, int64_t ldk, float* s, int64_t lds) {
  v8 a00 = _mm256_setzero_ps(), a01 = a00, a10 = a00, a11 = a00, a20 = a00, a21 = a00, a30 = a00, a31 = a00;
  for (int64_t d = 0; d < hd; ++d) {
    const v8 k0 = _mm256_loadu_ps(kt + d * ldk), k1 = _mm256_loadu_ps(kt + d * ldk + 8);
    const v8 q0 = _mm256_broadcast_ss(qb + d), q1 = _mm256_broadcast_ss(qb + hd + d);
    const v8 q2 = _mm256_broadcast_ss(qb + 2 * hd + d), q3 = _mm256_broadcast_ss(qb + 3 * hd + d);
    a00 = _mm256_fmadd_ps(q0, k0, a00);
    a01 = _mm256_fmadd_ps(q0, k1, a01);
    a10 = _mm256_fmadd_ps(q1, k0, a10);
    a11 = _mm256_fmadd_ps(q1, k1, a11);
    a20 = _mm256_fmadd_ps(q2, k0, a20);
    a21 = _mm256_fmadd_ps(q2, k1, a21);
    a30 = _mm256_fmadd_ps(q3, k0, a30);
    a31 = _mm256_fmadd_ps(q3, k1, a31);
  }
  _mm256_storeu_ps(s, a00);
  _mm256_storeu_ps(s + 8, a01);
  _mm256_storeu_ps(s + lds, a10);
  _mm256_storeu_ps(s + lds + 8, a11);
  _mm256_storeu_ps(s + 2 * lds, a20);
  _mm256_storeu_ps(s + 2 * lds + 8, a21);
  _mm256_storeu_ps(s + 3 * lds, a30);
  _mm256_storeu_ps(s + 3 * lds + 8, a31);
}

/* acc[4 rows][16 dims] += P[4][nk] . V[nk][16]: p rows `ldp` apart, v rows `hd`
 * apart from dim column 0 of the 16, acc rows `hd` apart. */
static inline void pv_tile_4x16(const float* p, int64_t ldp, int64_t nk, const float* v, int64_t hd, float* acc) {
  v8 a00 = _mm256_loadu_ps(acc), a01 = _mm256_loadu_ps(acc + 8);
  v8 a10 = _mm256_loadu_ps(acc + hd), a11 = _mm256_loadu_ps(acc + hd + 8);
  v8 a20 = _mm256_loadu_ps(acc + 2 * hd), a21 = _mm256_loadu_ps(acc + 2 * hd + 8);
  v8 a30 = _mm256_loadu_ps(acc + 3 * hd), a31 = _mm256_loadu_ps(acc + 3 * hd + 8);
  for (int64_t j = 0; j < nk; ++j) {
    const v8 v0 = _mm256_loadu_ps(v + j * hd), v1 = _mm256_loadu_ps(v + j * hd + 8);
    const v8 p0 = _mm256_broadcast_ss(p + j), p1 = _mm256_broadcast_ss(p + ldp + j);
    const v8 p2 = _mm256_broadcast_ss(p + 2 * ldp + j), p3 = _mm256_broadcast_ss(p + 3 * ldp + j);
    a00 = _mm256_fmadd_ps(p0, v0, a00);
    a01 = _mm256_fmadd_ps(p0, v1, a01);
    a10 = _mm256_fmadd_ps(p1, v0, a10);
    a11 = _mm256_fmadd_ps(p1, v1, a11);
    a20 = _mm256_fmadd_ps(p2, v0, a20);
    a21 = _mm256_fmadd_ps(p2, v1, a21);
    a30 = _mm256_fmadd_ps(p3, v0, a30);
    a31 = _mm256_fmadd_ps(p3, v1, a31);
  }
  _mm256_storeu_ps(acc, a00);
  _mm256_storeu_ps(acc + 8, a01);
  _mm256_storeu_ps(acc + hd, a10);
  _mm256_storeu_ps(acc + hd + 8, a11);
  _mm256_storeu_ps(acc + 2 * hd, a20);
  _mm256_storeu_ps(acc + 2 * hd + 8, a21);
  _mm256_storeu_ps(acc + 3 * hd, a30);
  _mm256_storeu_ps(acc + 3 * hd + 8, a31);
}

/* The same two products with AVX-512 registers (4 rows x 32 columns), for hosts
 * that have it (chosen at run time). */
__attribute__((target("avx512f"))) static void s_block_512(const float* qb, int64_t hd, const float* kt,
                                                            int64_t ldk, float* s) {
  for (int64_t r = 0; r < FRQ; r += 4)
    for (int64_t j = 0; j < FKT; j += 32) {
      const float* q = qb + r * hd;
      const float* k = kt + j;
      __m512 a00 = _mm512_setzero_ps(), a01 = a00, a10 = a00, a11 = a00, a20 = a00, a21 = a00, a30 = a00, a31 = a00;
      for (int64_t d = 0; d < hd; ++d) {
        const __m512 k0 = _mm512_loadu_ps(k + d * ldk), k1 = _mm512_loadu_ps(k + d * ldk + 16);
        const __m512 q0 = _mm512_set1_ps(q[d]), q1 = _mm512_set1_ps(q[hd + d]);
        const __m512 q2 = _mm512_set1_ps(q[2 * hd + d]), q3 = _mm512_set1_ps(q[3 * hd + d]);
        a00 = _mm512_fmadd_ps(q0, k0, a00);
        a01 = _mm512_fmadd_ps(q0, k1, a01);
        a10 = _mm512_fmadd_ps(q1, k0, a10);
        a11 = _mm512_fmadd_ps(q1, k1, a11);
        a20 = _mm512_fmadd_ps(q2, k0, a20);
        a21 = _mm512_fmadd_ps(q2, k1, a21);
        a30 = _mm512_fmadd_ps(q3, k0, a30);
        a31 = _mm512_fmadd_ps(q3, k1, a31);
      }
      float* o = s + r * FKT + j;
      _mm512_storeu_ps(o, a00);
      _mm512_storeu_ps(o + 16, a01);
      _mm512_storeu_ps(o + FKT, a10);
      _mm512_storeu_ps(o + FKT + 16, a11);
      _mm512_storeu_ps(o + 2 * FKT, a20);
      _mm512_storeu_ps(o + 2 * FKT + 16, a21);
      _mm512_storeu_ps(o + 3 * FKT, a30);
      _mm512_storeu_ps(o + 3 * FKT + 16, a31);
    }
}

__attribute__((target("avx512f"))) static void pv_block_512(const float* p, int64_t nk, const float* v,
                                                             int64_t hd, float* acc) {
  for (int64_t r = 0; r < FRQ; r += 4)
    for (int64_t d = 0; d < hd; d += 32) {
      const float* pr = p + r * FKT;
      float* a = acc + r * hd + d;
      __m512 a00 = _mm512_loadu_ps(a), a01 = _mm512_loadu_ps(a + 16);
      __m512 a10 = _mm512_loadu_ps(a + hd), a11 = _mm512_loadu_ps(a + hd + 16);
      __m512 a20 = _mm512_loadu_ps(a + 2 * hd), a21 = _mm512_loadu_ps(a + 2 * hd + 16);
      __m512 a30 = _mm512_loadu_ps(a + 3 * hd), a31 = _mm512_loadu_ps(a + 3 * hd + 16);
      for (int64_t j = 0; j < nk; ++j) {
        const __m512 v0 = _mm512_loadu_ps(v + j * hd + d), v1 = _mm512_loadu_ps(v + j * hd + d + 16);
        const __m512 p0 = _mm512_set1_ps(pr[j]), p1 = _mm512_set1_ps(pr[FKT + j]);
        const __m512 p2 = _mm512_set1_ps(pr[2 * FKT + j]), p3 = _mm512_set1_ps(pr[3 * FKT + j]);
        a00 = _mm512_fmadd_ps(p0, v0, a00);
        a01 = _mm512_fmadd_ps(p0, v1, a01);
        a10 = _mm512_fmadd_ps(p1, v0, a10);
        a11 = _mm512_fmadd_ps(p1, v1, a11);
        a20 = _mm512_fmadd_ps(p2, v0, a20);
        a21 = _mm512_fmadd_ps(p2, v1, a21);
        a30 = _mm512_fmadd_ps(p3, v0, a30);
        a31 = _mm512_fmadd_ps(p3, v1, a31);
      }
      _mm512_storeu_ps(a, a00);
      _mm512_storeu_ps(a + 16, a01);
      _mm512_storeu_ps(a + hd, a10);
      _mm512_storeu_ps(a + hd + 16, a11);
      _mm512_storeu_ps(a + 2 * hd, a20);
      _mm512_storeu_ps(a + 2 * hd + 16, a21);
      _mm512_storeu_ps(a + 3 * hd, a30);
      _mm512_storeu_ps(a + 3 * hd + 16, a31);
    }
}

/* Prefill.  Per (batch, head): K^T [hd][Sp] and V [Sp][hd] packed in fp32 with the
 * key count padded to whole tiles (zeros).  A work item is FRQ query rows: per
 * key tile of FKT keys, S = Q K^T for the block (4x16 register tiles), then per
 * row the masked tile max in scaled log2 units, alpha = 2^(m - m_new), p =
 * 2^(s*c - m_new) (its sum into l unrounded, p itself rounded to bf16 on bf16
 * inputs), acc *= alpha, and acc += P V (4x16 register tiles).  A tile a row
 * sees no key of leaves that row alone. */
void oracle_flash(int bf, const void* q, const void* k, const void* v, void* out, int64_t batch,
                  int64_t seq_q, int64_t seq_k, int64_t heads, int64_t hd, const int64_t* qs,
                  const int64_t* ks, const int64_t* vs, float scale, int causal, int threads) {
  set_threads(threads);
  const float c = scale * LOG2E;
  const int64_t bh = batch * heads;
  const int64_t sp = (seq_k + FKT - 1) / FKT * FKT;
  float* kt = (float*)aligned_alloc(64, sizeof(float) * (size_t)(bh * hd * sp + 16));
  float* vv = (float*)aligned_alloc(64, sizeof(float) * (size_t)(bh * hd * sp + 16));
  const int64_t ntile = sp / FKT;
#pragma omp parallel for schedule(static)
  for (int64_t it = 0; it < bh * ntile; ++it) {
    const int64_t i = it / ntile, j0 = (it % ntile) * FKT;
    const int64_t b = i / heads, h = i % heads;
    float* ktb = kt + i * hd * sp;
    float* vb = vv + i * hd * sp;
    for (int64_t j = j0; j < j0 + FKT; ++j)
      for (int64_t d = 0; d < hd; ++d) {
        const int in = j < seq_k;
        ktb[d * sp + j] = in ? ld(k, b * ks[0] + j * ks[1] + h * ks[2] + d, bf) : 0.f;
        vb[j * hd + d] = in ? ld(v, b * vs[0] + j * vs[1] + h * vs[2] + d, bf) : 0.f;
      }
  }
  const int64_t nqb = (seq_q + FRQ - 1) / FRQ;
  const int64_t diag = seq_k - seq_q;
  /* CA_ORACLE_AVX2=1 keeps the AVX2 tiles (so tests cover both on any host). */
  const char* narrow = getenv("CA_ORACLE_AVX2");
  const int wide = hd % 32 == 0 && __builtin_cpu_supports("avx512f") && !(narrow && narrow[0] == '1');
#pragma omp parallel
  {
    float* sc = (float*)aligned_alloc(64, sizeof(float) * FRQ * FKT);
    float* acc = (float*)aligned_alloc(64, sizeof(float) * FRQ * (size_t)hd);
    float* qb = (float*)aligned_alloc(64, sizeof(float) * FRQ * (size_t)hd);
    float m[FRQ], l[FRQ];
#pragma omp for schedule(dynamic, 1)
    for (int64_t it = 0; it < bh * nqb; ++it) {
      const int64_t i = it / nqb, q0 = (it % nqb) * FRQ;
      const int64_t b = i / heads, h = i % heads;
      const int64_t nr = seq_q - q0 < FRQ ? seq_q - q0 : FRQ;
      const float* ktb = kt + i * hd * sp;
      const float* vb = vv + i * hd * sp;
      for (int64_t r = 0; r < FRQ; ++r) {
        for (int64_t d = 0; d < hd; ++d)
          qb[r * hd + d] = r < nr ? ld(q, b * qs[0] + (q0 + r) * qs[1] + h * qs[2] + d, bf) : 0.f;
        m[r] = -INFINITY;
        l[r] = 0.f;
      }
      memset(acc, 0, sizeof(float) * FRQ * (size_t)hd);
      const int64_t kend = causal ? (q0 + nr + diag < seq_k ? q0 + nr + diag : seq_k) : seq_k;
      for (int64_t k0 = 0; k0 < kend; k0 += FKT) {
        const int64_t nk = kend - k0 < FKT ? kend - k0 : FKT;
        if (wide)
          s_block_512(qb, hd, ktb + k0, sp, sc);
        else
          for (int64_t r = 0; r < FRQ; r += 4)
            for (int64_t j = 0; j < FKT; j += 16) s_tile_4x16(qb + r * hd, hd, ktb + k0 + j, sp, sc + r * FKT + j, FKT);
        for (int64_t r = 0; r < nr; ++r) {
          float* srow = sc + r * FKT;
          /* keys this row sees in the tile: [0, vis) */
          int64_t vis = nk;
          if (causal) {
            const int64_t lim = q0 + r + diag - k0 + 1;
            vis = lim < vis ? (lim < 0 ? 0 : lim) : vis;
          }
          if (vis == 0) { /* nothing visible in this tile */
            memset(srow, 0, sizeof(float) * FKT);
            continue;
          }
          v8 mx = _mm256_set1_ps(-INFINITY);
          for (int64_t j = 0; j < FKT; j += 8) {
            const v8 key = _mm256_add_ps(_mm256_set1_ps((float)j), _mm256_setr_ps(0, 1, 2, 3, 4, 5, 6, 7));
            const v8 in = _mm256_cmp_ps(key, _mm256_set1_ps((float)vis), _CMP_LT_OQ);
            const v8 x = _mm256_blendv_ps(_mm256_set1_ps(-INFINITY), _mm256_mul_ps(_mm256_loadu_ps(srow + j),
                                                                                  _mm256_set1_ps(c)), in);
            _mm256_storeu_ps(srow + j, x);
            mx = _mm256_max_ps(mx, x);
          }
          const float m_new = fmaxf(m[r], hmax(mx));
          const float alpha = exp2f(m[r] - m_new);
          m[r] = m_new;
          v8 sum = _mm256_setzero_ps();
          for (int64_t j = 0; j < FKT; j += 8) {
            const v8 p = exp2v(_mm256_sub_ps(_mm256_loadu_ps(srow + j), _mm256_set1_ps(m_new)));
            sum = _mm256_add_ps(sum, p);
            _mm256_storeu_ps(srow + j, bf ? bf16_round(p) : p);
          }
          l[r] = l[r] * alpha + hsum(sum);
          float* ar = acc + r * hd;
          const v8 av = _mm256_set1_ps(alpha);
          for (int64_t d = 0; d < hd; d += 8) _mm256_storeu_ps(ar + d, _mm256_mul_ps(_mm256_loadu_ps(ar + d), av));
        }
        for (int64_t r = nr; r < FRQ; ++r) memset(sc + r * FKT, 0, sizeof(float) * FKT);
        if (wide)
          pv_block_512(sc, nk, vb + k0 * hd, hd, acc);
        else
          for (int64_t r = 0; r < FRQ; r += 4)
            for (int64_t d = 0; d < hd; d += 16) pv_tile_4x16(sc + r * FKT, FKT, nk, vb + k0 * hd + d, hd, acc + r * hd + d);
      }
      for (int64_t r = 0; r < nr; ++r) {
        const float inv = l[r] > 0.f ? 1.f / l[r] : 0.f;
        for (int64_t d = 0; d < hd; ++d)
          st(out, ((b * seq_q + q0 + r) * heads + h) * hd + d, l[r] > 0.f ? acc[r * hd + d] * inv : 0.f, bf);
      }
    }
    free(sc);
    free(acc);
    free(qb);
  }
  free(kt);
  free(vv);
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
