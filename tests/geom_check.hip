// Host-side address check of the flash kernels (test infrastructure; compiled on
// the host only, `hipcc --cuda-host-only`, and run by tests/test_geometry.py).
//
// It includes the kernel sources and replays, for each call shape it reads from
// stdin, the launcher's own plan (flash_plan: route, grid, splits) and the index
// arithmetic the kernels themselves call (bf16_block_work / pair_work /
// block_work / rows_work / heads_work / small_work, bf16_pass_geom, bf16_row_tiles, f32_keys,
// tile_window, window_bytes, tile_offsets, f32_tile_offset, f32_tile_bytes,
// rows_kend).  For every block, split, pass, wave, tile, load and lane it forms
// each global access the kernel would make (the bytes a buffer window lets
// through, or a guarded plain load) and asserts that it lies inside one row of
// the right tensor for the block's (batch, head), that key rows lie inside the
// pass's key range, that output rows and workspace slots exist, and that every
// direct-to-LDS tile load stays inside its tile buffer.
//
// Input lines: E bf16 causal batch seq_q seq_k heads qs0 qs1 qs2 ks0 ks1 ks2 vs0 vs1 vs2
// (element strides).  Output: "ok <shapes> <accesses>" or the first failure.
// --plant: widens every partial key tile's window by one row (a plausible
// mistake), so a test can check that the replay catches it.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../cpu-attention_amd/csrc/ca_flash.hip"
#include "../cpu-attention_amd/csrc/ca_rows.hip"
#include "../cpu-attention_amd/csrc/ca_small.hip"

#include <vector>

using namespace ca;

static bool g_plant = false;
static long long g_checks = 0;
static char g_fail[512];

#define FAIL(...)                                            \
  do {                                                       \
    if (!g_fail[0]) snprintf(g_fail, sizeof g_fail, __VA_ARGS__); \
    return false;                                            \
  } while (0)

// A [batch, tokens, heads, E] tensor by element strides; byte offsets are
// relative to its base.
struct Ten {
  int64_t s0, s1, s2, T;
  int E, esz;
  // Byte range [off, off + len) lies inside row t of (b, h) for some t < tmax,
  // within the row's E elements.
  bool inside(int64_t b, int64_t h, int64_t off, int len, int64_t tmax, int64_t* t_out = nullptr) const {
    const int64_t rel = off - (b * s0 + h * s2) * esz;
    if (rel < 0) return false;
    const int64_t rs = s1 * esz;
    const int64_t t = rs > 0 ? rel / rs : 0, within = rs > 0 ? rel - t * rs : rel;
    if (t_out) *t_out = t;
    return t < tmax && t < T && within + len <= (int64_t)E * esz;
  }
};

// One key tile (rows of the pass's range [kbeg, kend)) of one bf16 tile stream.
template <int E, int RS>
static bool bf16_tile(const Ten& t, int64_t b, int64_t h, int stride, int kbeg, int kend, int i, int wv,
                      const char* what) {
  using C = FlashBf16Cfg<E>;
  constexpr int NL = C::NL;
  int off[NL];
  tile_offsets<E, RS, NL>(wv, 0, stride, off);  // lane 0 first: the loop below redoes it per lane
  const int rows = (kend - kbeg) - 64 * i;
  int bytes = tile_window<E>(rows, 2 * stride);
  if (g_plant && rows > 0 && rows < 64) bytes += 2 * stride;
  const int64_t base = ((int64_t)kbeg + 64 * i) * stride * 2;  // from the (b, h) start
  for (int lane = 0; lane < 64; ++lane) {
    tile_offsets<E, RS, NL>(wv, lane, stride, off);
    for (int j = 0; j < NL; ++j) {
      // LDS: load j of wave wv fills chunk (4j + wv) * 64 + lane of the tile buffer
      if (((C::NWG * j + wv) * 64 + lane + 1) * 16 > C::TBUF * 2) FAIL("%s: LDS chunk past the tile buffer", what);
      const uint32_t o = (uint32_t)off[j];
      if ((uint64_t)o + 16 > (uint64_t)(uint32_t)bytes) continue;  // outside the window: zeros, no access
      ++g_checks;
      int64_t row;
      if (!t.inside(b, h, (b * t.s0 + h * t.s2) * t.esz + base + o, 16, t.T, &row))
        FAIL("%s: tile %d load %d lane %d (b %lld h %lld) outside the tensor", what, i, j, lane, (long long)b,
             (long long)h);
      if (row < kbeg || row >= kend)
        FAIL("%s: tile %d reads key %lld outside the pass's range [%d, %d)", what, i, (long long)row, kbeg, kend);
    }
  }
  return true;
}

template <int E>
static bool check_bf16(const FlashParams& p, const FlashPlan& plan, const Ten& q, const Ten& k, const Ten& v) {
  const int L = (int)p.seq_q, S = (int)p.seq_k, diag = S - L;
  constexpr int NS = E / 16;
  for (int64_t bx = 0; bx < plan.gx; ++bx)
    for (int64_t by = 0; by < plan.gy; ++by) {
      const PairWork pw = bf16_block_work(p, plan.split, bx);
      if (pw.b < 0 || pw.b >= p.batch || pw.h < 0 || pw.h >= p.heads) FAIL("bf16 block %lld: bad (b, h)", (long long)bx);
      const int64_t nqb = cdiv(p.seq_q, 256);
      if (pw.n < 1 || pw.n > 2 || pw.qb0 < 0 || pw.qb0 >= nqb || pw.qb1 < 0 || pw.qb1 >= nqb)
        FAIL("bf16 block %lld: bad query blocks", (long long)bx);
      for (int pass = 0; pass < pw.n; ++pass) {
        const Bf16Geom g = bf16_pass_geom(p, pw, pass, plan.split, (int)by, (int)plan.gy);
        if (g.nkt > 0 && (g.kbeg < 0 || g.kbeg >= g.kend || g.kend > S)) FAIL("bf16: key range [%d, %d)", g.kbeg, g.kend);
        if (g.nkt > 0 && (g.kend - g.kbeg + 63) / 64 != g.nkt) FAIL("bf16: tile count");
        for (int wv = 0; wv < 4; ++wv) {
          const int r0 = g.q0 + 64 * wv;
          const int nw = bf16_row_tiles(S, diag, p.causal, g.kbeg, g.kend, r0, 64, plan.split);
          if (nw > g.nkt) FAIL("bf16: wave walks %d of %d tiles", nw, g.nkt);
          for (int cb = 0; cb < 2; ++cb) {  // Q rows of both column blocks (fast walk and safe pass)
            const int rb = r0 + 32 * cb;
            const int bytes = window_bytes(((int64_t)(L - 1 - rb) * (int)p.qs[1] + E) * 2);
            for (int li = 0; li < 32; ++li)
              for (int hf = 0; hf < 2; ++hf)
                for (int s = 0; s < NS; ++s) {
                  const int off = (li * (int)p.qs[1] + 16 * s + 8 * hf) * 2;
                  if ((int64_t)off + 16 > bytes) continue;
                  ++g_checks;
                  if (!q.inside(pw.b, pw.h, (pw.b * q.s0 + pw.h * q.s2) * 2 + (int64_t)rb * p.qs[1] * 2 + off, 16, L))
                    FAIL("bf16: Q row %d outside the tensor", rb + li);
                }
            for (int rr = 0; rr < 32; ++rr) {  // output rows (store_staged, store_partials): row < L only
              const int64_t row = rb + rr;
              if (row >= L) continue;
              if (plan.split) {
                const int64_t slot = ((pw.b * p.heads + pw.h) * p.seq_q + row) * plan.splits + by;
                if (slot >= p.batch * p.heads * p.seq_q * plan.splits) FAIL("bf16: partial slot");
              }
            }
          }
          if (g.nkt == 0) continue;  // no tile loads at all
          // Every wave issues its share of K(0) .. K(nkt + 3) and V(0) .. V(nkt + 1)
          // (the fast walk); the safe pass reloads tiles 0 .. nkt - 1 of the same range.
          for (int i = 0; i < g.nkt + 4; ++i)
            if (!bf16_tile<E, FlashBf16Cfg<E>::RSK>(k, pw.b, pw.h, (int)p.ks[1], g.kbeg, g.kend, i, wv, "bf16 K"))
              return false;
          for (int i = 0; i < g.nkt + 2; ++i)
            if (!bf16_tile<E, FlashBf16Cfg<E>::RSV>(v, pw.b, pw.h, (int)p.vs[1], g.kbeg, g.kend, i, wv, "bf16 V"))
              return false;
        }
      }
    }
  return true;
}

template <int E>
static bool check_f32(const FlashParams& p, const FlashPlan& plan, const Ten& q, const Ten& k, const Ten& v) {
  constexpr int CH = FlashF32Cfg<E>::CH;
  const int64_t L = p.seq_q, S = p.seq_k;
  for (int64_t bx = 0; bx < plan.gx; ++bx)
    for (int64_t by = 0; by < plan.gy; ++by) {
      PairWork pw{};
      if (plan.pair) pw = pair_work(p, kBM, false, bx);
      for (int pass = 0; pass < (plan.pair ? pw.n : 1); ++pass) {
        const BlockWork bw = plan.pair ? BlockWork{pw.b, pw.h, (pass ? pw.qb1 : pw.qb0) * kBM} : block_work(p, bx);
        if (bw.b < 0 || bw.b >= p.batch || bw.h < 0 || bw.h >= p.heads || bw.q0 < 0 || bw.q0 >= L)
          FAIL("f32 block %lld: bad work", (long long)bx);
        const F32Keys kr = f32_keys(p, bw.q0, plan.split, (int)by, (int)plan.gy);
        if (kr.nkt > 0 && (kr.kbeg < 0 || kr.kbeg >= kr.kend || kr.kend > S)) FAIL("f32: key range");
        for (int wv = 0; wv < 4; ++wv)
          for (int li = 0; li < 32; ++li) {
            const int64_t row = bw.q0 + 32 * wv + li;
            if (row < L && plan.split &&
                ((bw.b * p.heads + bw.h) * L + row) * plan.splits + by >= p.batch * p.heads * L * plan.splits)
              FAIL("f32: partial slot");
          }
        if (kr.nkt == 0) continue;
        for (int t = 0; t <= kr.nkt; ++t) {  // load_tile(0) .. load_tile(nkt)
          const int64_t k0 = kr.kbeg + (int64_t)t * 32;
          for (int which = 0; which < 2; ++which) {
            const Ten& tn = which ? v : k;
            const int64_t stride = which ? p.vs[1] : p.ks[1];
            int bytes = window_bytes(f32_tile_bytes<E>(S, k0, stride));
            for (int tid = 0; tid < 256; ++tid)
              for (int i = 0; i < CH; ++i) {
                const int off = f32_tile_offset<E>(tid, i, stride);
                if ((int64_t)off + 16 > bytes) continue;
                ++g_checks;
                if (!tn.inside(bw.b, bw.h, (bw.b * tn.s0 + bw.h * tn.s2) * 4 + k0 * stride * 4 + off, 16, S))
                  FAIL("f32: tile at key %lld thread %d chunk %d outside the tensor", (long long)k0, tid, i);
              }
          }
        }
      }
    }
  return true;
}

// A split call's partials: they fit the workspace the plan asks for, and the grid
// writes every (row, split) slot exactly once, so the combine kernel merges no
// slot that a block left unwritten.
static bool check_slots(const FlashPlan& plan, int E, int64_t rows, const std::vector<int>& written) {
  if (plan.splits <= 1) return true;
  if (plan.need < rows * plan.splits * (E + 2) * 4) FAIL("partials outside the workspace");
  for (int64_t f = 0; f < (int64_t)written.size(); ++f) {
    ++g_checks;
    if (written[f] != 1)
      FAIL("partial of row %lld split %lld written %d times", (long long)(f / plan.splits),
           (long long)(f % plan.splits), written[f]);
  }
  return true;
}

template <int E, bool BF>
static bool check_rows(const FlashParams& p, const FlashPlan& plan, const Ten& q, const Ten& k, const Ten& v) {
  const int esz = BF ? 2 : 4;
  const int64_t rows = p.batch * p.heads * p.seq_q;
  // times each (row, split) partial slot is written
  std::vector<int> written(plan.splits > 1 ? rows * plan.splits : 0, 0);
  if (plan.kind == kPlanRowsHeads) {
    constexpr int HP = HeadsShape<E, BF>::HP, G = HeadsShape<E, BF>::G, DPL = HeadsShape<E, BF>::DPL;
    for (int64_t bx = 0; bx < plan.gx; ++bx)
      for (int64_t by = 0; by < plan.gy; ++by) {
        const HeadsWork hw = heads_work(p, HP, bx, plan.gx, plan.gy);
        if (hw.b < 0 || hw.b >= p.batch || hw.h0 < 0 || hw.h0 + HP > p.heads) FAIL("heads block: bad work");
        for (int lane = 0; lane < 64; ++lane) {
          const int64_t h = hw.h0 + lane / G, e0 = (lane % G) * DPL;
          // q row 0 and keys j < S of head h: the slice [e0, e0 + DPL) of each row
          ++g_checks;
          if (e0 + DPL > E || !q.inside(hw.b, h, (hw.b * q.s0 + h * q.s2 + e0) * esz, 16, p.seq_q)) FAIL("heads: q");
          if (!k.inside(hw.b, h, (hw.b * k.s0 + h * k.s2 + (p.seq_k - 1) * k.s1 + e0) * esz, 16, p.seq_k))
            FAIL("heads: last key");
        }
        // partial slots and merged rows: rows b*heads + h0 + hh, hh < HP
        if (plan.splits > 1) {
          for (int hh = 0; hh < HP; ++hh) {
            const int64_t slot = (hw.b * p.heads + hw.h0 + hh) * plan.splits + by;
            if (slot >= rows * plan.splits) FAIL("heads: partial slot");
            ++written[slot];
          }
        }
      }
    return check_slots(plan, E, rows, written);
  }
  const int R = plan.rows_r;
  constexpr int CH = RowsShape<E, BF, 1>::CH, G = RowsShape<E, BF, 1>::G, DPL = RowsShape<E, BF, 1>::DPL;
  for (int64_t bx = 0; bx < plan.gx; ++bx)
    for (int64_t by = 0; by < plan.gy; ++by) {
      const RowsWork rw = rows_work(p, R, CH, bx, plan.gx, plan.gy);
      if (rw.b < 0 || rw.b >= p.batch || rw.h < 0 || rw.h >= p.heads || rw.i0 < 0 || rw.i0 >= p.seq_q || rw.nr < 1 ||
          rw.nr > R)
        FAIL("rows block %lld: bad work", (long long)bx);
      if (rw.kend_g < 0 || rw.kend_g > p.seq_k) FAIL("rows: key range");
      for (int r = 0; r < rw.nr; ++r) {
        const int64_t i = rw.i0 + r;
        if (rows_kend(p, i) > rw.kend_g) FAIL("rows: a row's keys past the group's");
        for (int sl = 0; sl < G; ++sl) {
          ++g_checks;
          if (!q.inside(rw.b, rw.h, (rw.b * q.s0 + rw.h * q.s2 + i * q.s1 + sl * DPL) * esz, 16, p.seq_q))
            FAIL("rows: q row %lld", (long long)i);
        }
        if (plan.splits > 1) {
          const int64_t slot = ((rw.b * p.heads + rw.h) * p.seq_q + i) * plan.splits + by;
          if (slot >= rows * plan.splits) FAIL("rows: partial slot");
          ++written[slot];
        }
      }
      // the last key any lane loads (guarded by j < kend_g)
      if (rw.kend_g > 0) {
        ++g_checks;
        if (!k.inside(rw.b, rw.h, (rw.b * k.s0 + rw.h * k.s2 + (rw.kend_g - 1) * k.s1) * esz, 16 * G, p.seq_k))
          FAIL("rows: last key");
      }
    }
  return check_slots(plan, E, rows, written);
}

// flash_small_kernel: one wave per (batch, head, 32 query rows); every block's
// work must be a distinct row block, and every guarded load and output store
// must lie inside its tensor.
template <int E>
static bool check_small(const FlashParams& p, const FlashPlan& plan, const Ten& q, const Ten& k, const Ten& v) {
  const int L = (int)p.seq_q, S = (int)p.seq_k, NKB = (int)cdiv(S, 32);
  if (NKB < 1 || 32 * NKB > kSmallMaxKeys + 31) FAIL("small: %d key blocks", NKB);
  const int64_t nrb = cdiv(L, kSmallRows);
  if (plan.gx != p.batch * p.heads * nrb || plan.gy != 1) FAIL("small: grid");
  std::vector<char> seen((size_t)plan.gx, 0);
  const int64_t out_elems = p.batch * p.seq_q * p.heads * E;
  for (int64_t bx = 0; bx < plan.gx; ++bx) {
    const SmallWork w = small_work(p, bx, plan.gx);
    if (w.b < 0 || w.b >= p.batch || w.h < 0 || w.h >= p.heads || w.r0 < 0 || w.r0 >= L || w.r0 % kSmallRows)
      FAIL("small block %lld: bad work", (long long)bx);
    const int64_t id = (w.b * p.heads + w.h) * nrb + w.r0 / kSmallRows;
    if (seen[(size_t)id]++) FAIL("small: row block given to two blocks");
    for (int lane = 0; lane < 64; ++lane) {
      const int n = lane & 31, hf = lane >> 5, row = w.r0 + n;
      const int64_t qrow = row < L ? row : L - 1;  // every lane loads; past L the last row
      for (int ks = 0; ks < E / 16; ++ks) {
        ++g_checks;
        if (!q.inside(w.b, w.h, (w.b * q.s0 + w.h * q.s2 + qrow * q.s1 + 16 * ks + 8 * hf) * 2, 16, L))
          FAIL("small: Q row %lld", (long long)qrow);
      }
      if (row < L) {
        if (small_kend(p, row) > S) FAIL("small: row %d sees keys past S", row);
        for (int db = 0; db < E / 32; ++db)
          for (int i = 0; i < 4; ++i) {
            const int64_t o = ((w.b * L + row) * p.heads + w.h) * (int64_t)E + 32 * db + small_acc_row(4 * i, hf);
            ++g_checks;
            if (o < 0 || o + 4 > out_elems || (o % E) + 4 > E) FAIL("small: output row %d", row);
          }
      }
      // K and V: 32-bit byte offsets from the (b, h) base, keys clamped to S - 1
      for (int kb = 0; kb < NKB; ++kb) {
        const int64_t kkey = small_clamp_key(32 * kb + n, S);
        for (int ks = 0; ks < E / 16; ++ks) {
          const uint64_t off64 = (uint64_t)kkey * (uint64_t)p.ks[1] * 2u + (16 * ks + 8 * hf) * 2;
          const uint32_t off32 = (uint32_t)kkey * (uint32_t)p.ks[1] * 2u + (16 * ks + 8 * hf) * 2;
          if (off64 != off32) FAIL("small: K offset past 32 bits");
          ++g_checks;
          if (!k.inside(w.b, w.h, (w.b * k.s0 + w.h * k.s2) * 2 + (int64_t)off32, 16, S))
            FAIL("small: K row %lld", (long long)kkey);
        }
      }
      // V rows staged in LDS: 16-byte chunk c = lane + 64 i is row c / CPR (clamped
      // for the load), column chunk c % CPR; the LDS write must lie in the array
      constexpr int CPR = E / 8, RS = small_rsv(E) * 8;
      const int nvl = NKB * 32 * CPR / 64;
      for (int i = 0; i < nvl; ++i) {
        const int c = lane + 64 * i, key = c / CPR, col = c % CPR;
        const int64_t vk = small_clamp_key(key, S);
        const uint64_t off64 = (uint64_t)vk * (uint64_t)p.vs[1] * 2u + col * 16;
        const uint32_t off32 = (uint32_t)vk * (uint32_t)p.vs[1] * 2u + col * 16;
        if (off64 != off32) FAIL("small: V offset past 32 bits");
        ++g_checks;
        if (!v.inside(w.b, w.h, (w.b * v.s0 + w.h * v.s2) * 2 + (int64_t)off32, 16, S))
          FAIL("small: V row %lld", (long long)vk);
        if (key * RS + col * 8 + 8 > NKB * 32 * RS) FAIL("small: LDS write past the staged rows");
      }
      // the transposed reads: rows 16 cc + 8 q + 4 hf + j / 4, columns 32 d + 16 dh + 4 (j % 4) .. +3
      const int j = lane & 15, dh = (lane >> 4) & 1;
      for (int cc = 0; cc < 2 * NKB; ++cc)
        for (int q = 0; q < 2; ++q)
          for (int d = 0; d < E / 32; ++d) {
            const int r = 16 * cc + 8 * q + 4 * hf + (j >> 2), col = 32 * d + 16 * dh + 4 * (j & 3);
            if (r >= NKB * 32 || col + 4 > E) FAIL("small: transposed read outside the staged rows");
          }
    }
  }
  // the P.V steps' keys: each of a 16-key step's keys once, across the two halves
  for (int u = 0; u < 2; ++u) {
    int mask = 0;
    for (int hf = 0; hf < 2; ++hf)
      for (int t = 0; t < 8; ++t) mask |= 1 << (small_pv_key(u, hf, t) - 16 * u);
    if (mask != 0xffff) FAIL("small: P.V step %d does not cover its 16 keys once", u);
  }
  return true;
}

template <int E>
static bool check_e(const FlashParams& p, bool bf16, const Ten& q, const Ten& k, const Ten& v) {
  const FlashPlan plan = flash_plan(p, E, bf16);
  switch (plan.kind) {
    case kPlanNone:
    case kPlanDeclined:
      return true;
    case kPlanBf16:
      return check_bf16<E>(p, plan, q, k, v);
    case kPlanF32:
      return check_f32<E>(p, plan, q, k, v);
    case kPlanSmall:
      return check_small<E>(p, plan, q, k, v);
    default:
      return bf16 ? check_rows<E, true>(p, plan, q, k, v) : check_rows<E, false>(p, plan, q, k, v);
  }
}

int main(int argc, char** argv) {
  for (int i = 1; i < argc; ++i)
    if (!strcmp(argv[i], "--plant")) g_plant = true;
  long long shapes = 0;
  long long E, bf, causal, batch, sq, sk, h, qs[3], ks[3], vs[3];
  while (scanf("%lld %lld %lld %lld %lld %lld %lld %lld %lld %lld %lld %lld %lld %lld %lld %lld", &E, &bf, &causal,
               &batch, &sq, &sk, &h, &qs[0], &qs[1], &qs[2], &ks[0], &ks[1], &ks[2], &vs[0], &vs[1], &vs[2]) == 16) {
    FlashParams p{};
    p.batch = batch;
    p.seq_q = sq;
    p.seq_k = sk;
    p.heads = h;
    for (int j = 0; j < 3; ++j) {
      p.qs[j] = qs[j];
      p.ks[j] = ks[j];
      p.vs[j] = vs[j];
    }
    p.causal = (int)causal;
    const int esz = bf ? 2 : 4;
    const Ten q{qs[0], qs[1], qs[2], sq, (int)E, esz}, k{ks[0], ks[1], ks[2], sk, (int)E, esz},
        v{vs[0], vs[1], vs[2], sk, (int)E, esz};
    bool ok = E == 32 ? check_e<32>(p, bf != 0, q, k, v)
                      : E == 64 ? check_e<64>(p, bf != 0, q, k, v) : check_e<128>(p, bf != 0, q, k, v);
    ++shapes;
    if (!ok) {
      printf("FAIL E=%lld bf16=%lld causal=%lld N=%lld L=%lld S=%lld H=%lld: %s\n", E, bf, causal, batch, sq, sk, h,
             g_fail);
      return 1;
    }
  }
  printf("ok %lld %lld\n", shapes, g_checks);
  return 0;
}
