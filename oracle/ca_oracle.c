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
 *                  (flash_attn.mojo:208-212).
 *
 * Parallelised with OpenMP over independent work items; `threads` <= 0 uses the
 * OpenMP default.
 */
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

void oracle_flash(int bf, const void* q, const void* k, const void* v, void* out, int64_t batch,
                  int64_t seq_q, int64_t seq_k, int64_t heads, int64_t hd, const int64_t* qs,
                  const int64_t* ks, const int64_t* vs, float scale, int causal, int threads) {
  set_threads(threads);
  const float c = scale * LOG2E;
  const int64_t bh = batch * heads;
  /* Pack: K^T [hd][S] and V [S][hd] in fp32 per (batch, head). */
  float* kt = (float*)malloc(sizeof(float) * (size_t)(bh * hd * seq_k));
  float* vv = (float*)malloc(sizeof(float) * (size_t)(bh * hd * seq_k));
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < bh; ++i) {
    const int64_t b = i / heads, h = i % heads;
    float* ktb = kt + i * hd * seq_k;
    float* vb = vv + i * hd * seq_k;
    for (int64_t j = 0; j < seq_k; ++j)
      for (int64_t d = 0; d < hd; ++d) {
        ktb[d * seq_k + j] = ld(k, b * ks[0] + j * ks[1] + h * ks[2] + d, bf);
        vb[j * hd + d] = ld(v, b * vs[0] + j * vs[1] + h * vs[2] + d, bf);
      }
  }
  const int64_t nqb = (seq_q + FRQ - 1) / FRQ;
  const int64_t diag = seq_k - seq_q;
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * FRQ * FKT);
    float* acc = (float*)malloc(sizeof(float) * FRQ * (size_t)hd);
    float* qb = (float*)malloc(sizeof(float) * FRQ * (size_t)hd);
    float m[FRQ], l[FRQ];
#pragma omp for schedule(dynamic, 1)
    for (int64_t it = 0; it < bh * nqb; ++it) {
      const int64_t i = it / nqb, q0 = (it % nqb) * FRQ;
      const int64_t b = i / heads, h = i % heads;
      const int64_t nr = seq_q - q0 < FRQ ? seq_q - q0 : FRQ;
      const float* ktb = kt + i * hd * seq_k;
      const float* vb = vv + i * hd * seq_k;
      for (int64_t r = 0; r < nr; ++r) {
        for (int64_t d = 0; d < hd; ++d) qb[r * hd + d] = ld(q, b * qs[0] + (q0 + r) * qs[1] + h * qs[2] + d, bf);
        m[r] = -INFINITY;
        l[r] = 0.f;
      }
      memset(acc, 0, sizeof(float) * FRQ * (size_t)hd);
      const int64_t kend = causal ? (q0 + nr + diag < seq_k ? q0 + nr + diag : seq_k) : seq_k;
      for (int64_t k0 = 0; k0 < kend; k0 += FKT) {
        const int64_t nk = kend - k0 < FKT ? kend - k0 : FKT;
        for (int64_t r = 0; r < nr; ++r) {
          float* srow = sc + r * FKT;
          for (int64_t j = 0; j < nk; ++j) srow[j] = 0.f;
          for (int64_t d = 0; d < hd; ++d) {
            const float qd = qb[r * hd + d];
            const float* kr = ktb + d * seq_k + k0;
            for (int64_t j = 0; j < nk; ++j) srow[j] += qd * kr[j];
          }
          const int64_t lim = q0 + r + diag; /* last visible key of this row */
          float mx = -INFINITY;
          for (int64_t j = 0; j < nk; ++j) {
            if (causal && k0 + j > lim) srow[j] = -INFINITY;
            else srow[j] *= c;
            mx = srow[j] > mx ? srow[j] : mx;
          }
          if (mx == -INFINITY) continue; /* nothing visible in this tile */
          const float m_new = fmaxf(m[r], mx);
          const float alpha = exp2f(m[r] - m_new);
          m[r] = m_new;
          float sum = 0.f;
          for (int64_t j = 0; j < nk; ++j) {
            float p = exp2f(srow[j] - m_new);
            sum += p;
            srow[j] = bf ? bf2f(f2bf(p)) : p;
          }
          l[r] = l[r] * alpha + sum;
          float* ar = acc + r * hd;
          for (int64_t d = 0; d < hd; ++d) ar[d] *= alpha;
          for (int64_t j = 0; j < nk; ++j) {
            const float p = srow[j];
            const float* vr = vb + (k0 + j) * hd;
            for (int64_t d = 0; d < hd; ++d) ar[d] += p * vr[d];
          }
        }
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
