// Exact block top-k by (ordered BF16 score desc, ID asc) from a sampled cut.
//
// 1. Sample: 4096 items (all of them when n <= 4096, else the items at
//    floor(j n / 4096)) are histogrammed in LDS (12-bit bins, then the low 4
//    bits of the chosen bin) to find a score `cut` that about
//    k + 4 sqrt(k) + 8 items are expected to reach (exactly the k-th best
//    score when the sample is the whole input).
// 2. Candidates: one pass over all n scores appends (score, position) of
//    every item scoring >= cut to an LDS list (one atomic per wave).  IDs are
//    read later, only for items tied at the k-th score.
// 3. If the list holds fewer than k items (the sample over-estimated the
//    cut) or overflows, the caller runs the full exact selection instead.
//    Otherwise the top k of the input are exactly the top k of the list
//    (every other item scores below cut <= every candidate), found by a
//    histogram over the candidates' scores and, for ties at the k-th score,
//    a rank of the tied IDs.
// The result is therefore identical to a full selection; only the time
// depends on the sample.
#pragma once

#include <cstddef>

#include "skv_select.h"

namespace skv {

constexpr int FS_SAMPLE = 4096;
constexpr int FS_PER = FS_SAMPLE / SEL_BLOCK;  // sample items per thread
constexpr int CAND_CAP = 4096;
constexpr int FS_TIE_RANK = SEL_BLOCK;  // ties ranked by direct comparison up to this count
constexpr int FS_OCT = 4;  // score octets per lane per pass (a 32-bit candidate mask)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// Packed 16-bit test of both halves of w against cut (cm1 = cut - 1 in each
// half): bit 0 = (low half >= cut), bit 16 = (high half >= cut).
__device__ __forceinline__ uint32_t ge_cut2(uint32_t w, u16x2 cm1) {
  const u16x2 d = __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, w), cm1);
  const u16x2 one = {1, 1};
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(d, one));
}

struct FastScratch {
  union {
    uint32_t hist[4096];
    KthScratch k;
  };
  alignas(16) uint64_t cand[CAND_CAP];  // ord << 40 | position
  uint32_t hist4[16];
  alignas(16) uint32_t tie[FS_TIE_RANK];  // read as uint4 by count_below
  int ncand;
  int maxo;
  int ntie;
  int sel[4];
  int scan[SEL_WAVES + 1];
};
static_assert(offsetof(FastScratch, cand) % 16 == 0, "cand is read 16 bytes at a time");
static_assert(offsetof(FastScratch, tie) % 16 == 0, "tie is read 16 bytes at a time");

// Candidate key: ordered score (bits 40..55) | position (bits 0..19); a key
// tied at the k-th score also carries its ID (bits 20..39, flag bit 56).
constexpr uint64_t CAND_HAS_ID = 1ull << 56;
__device__ __forceinline__ uint32_t cand_ord(uint64_t c) { return (uint32_t)(c >> 40) & 0xffffu; }
__device__ __forceinline__ int cand_pos(uint64_t c) { return (int)(c & 0xfffffu); }

// Number of the n entries of a smaller than x; a is a 16-byte aligned LDS
// array.  Four 16-byte reads are in flight per step (a dependent read per
// entry would leave the loop bound by LDS latency).
__device__ __forceinline__ int count_below(const uint32_t* a, int n, uint32_t x) {
  const uint4* a4 = reinterpret_cast<const uint4*>(a);
  const int n4 = n >> 2;
  int r0 = 0, r1 = 0, r2 = 0, r3 = 0, j = 0;
  auto c4 = [x](uint4 w) { return (int)(w.x < x) + (int)(w.y < x) + (int)(w.z < x) + (int)(w.w < x); };
  for (; j + 4 <= n4; j += 4) {
    const uint4 w0 = a4[j], w1 = a4[j + 1], w2 = a4[j + 2], w3 = a4[j + 3];
    r0 += c4(w0);
    r1 += c4(w1);
    r2 += c4(w2);
    r3 += c4(w3);
  }
  for (; j < n4; ++j) r0 += c4(a4[j]);
  for (int i = 4 * n4; i < n; ++i) r1 += a[i] < x;
  return (r0 + r1) + (r2 + r3);
}

// Number of the n 64-bit entries of a (16-byte aligned LDS) larger than x.
__device__ __forceinline__ int count_above64(const uint64_t* a, int n, uint64_t x) {
  const uint4* a4 = reinterpret_cast<const uint4*>(a);
  const int n2 = n >> 1;
  int r0 = 0, r1 = 0, j = 0;
  auto c2 = [x](uint4 w) {
    const uint64_t lo = ((uint64_t)w.y << 32) | w.x, hi = ((uint64_t)w.w << 32) | w.z;
    return (int)(lo > x) + (int)(hi > x);
  };
  for (; j + 4 <= n2; j += 4) {
    const uint4 w0 = a4[j], w1 = a4[j + 1], w2 = a4[j + 2], w3 = a4[j + 3];
    r0 += c2(w0) + c2(w1);
    r1 += c2(w2) + c2(w3);
  }
  for (; j < n2; ++j) r0 += c2(a4[j]);
  if (n & 1) r1 += a[n - 1] > x;
  return r0 + r1;
}

struct FastResult {
  Selection sel;  // members: the candidates passing fs_member
  int ncand;      // candidates in FastScratch::cand
  bool ok;        // false: use the full selection
};

// Membership of candidate key c; id(position) is read only for a candidate
// tied at the cut score when not every tie is a member.
template <typename IdFn>
__device__ __forceinline__ bool fs_member(const FastResult& r, uint64_t c, IdFn id) {
  const uint32_t o = cand_ord(c);
  if (o == 0) return false;
  if (r.sel.all || o > r.sel.v) return true;
  if (o < r.sel.v) return false;
  if (r.sel.idcut == 0xffffffffu) return true;
  const uint32_t cid = (c & CAND_HAS_ID) ? (uint32_t)(c >> 20) & 0xfffffu : id(cand_pos(c));
  return cid <= r.sel.idcut;
}

// Score sources: at(i) = ordered score of item i; oct(o) = the 8 ordered
// scores of items 8o .. 8o+7 as packed 16-bit pairs.
struct RowScores {  // a 16-byte aligned row, readable to a multiple of 8 items
  static constexpr int PRE = 8;  // octets per thread fast_select loads at entry
  const uint16_t* __restrict__ row;
  __device__ uint32_t at(int i) const { return row[i]; }
  __device__ uint4 oct(int o) const { return reinterpret_cast<const uint4*>(row)[o]; }
};

struct MaskedScores {  // score[i] where gate[i] >= thr, else 0 (excluded)
  static constexpr int PRE = 4;
  const uint16_t* __restrict__ score;
  const uint16_t* __restrict__ gate;
  uint32_t thr;
  __device__ uint32_t at(int i) const {
    const uint32_t gv = gate[i], sv = score[i];  // both loads issued together
    return gv >= thr ? sv : 0u;
  }
  __device__ uint4 oct(int o) const {
    return pick4(reinterpret_cast<const uint4*>(score)[o], reinterpret_cast<const uint4*>(gate)[o],
                 thr);
  }
  // the 8 packed scores of s4 whose packed gates in g4 reach thr
  __device__ static uint4 pick4(uint4 s4, uint4 g4, uint32_t thr) {
    const uint32_t t16 = thr << 16;
    auto pick = [&](uint32_t sw, uint32_t gw) {
      return ((gw << 16) >= t16 ? (sw & 0xffffu) : 0u) | (gw >= t16 ? (sw & 0xffff0000u) : 0u);
    };
    return make_uint4(pick(s4.x, g4.x), pick(s4.y, g4.y), pick(s4.z, g4.z), pick(s4.w, g4.w));
  }
};


// Descending scan of a 4096-bin histogram (each thread owns 8 bins): the bin
// holding the rank-th largest value and the count in higher bins, in
// s.sel[0..1]; sel[0] = -1 if the histogram holds fewer than rank values.
// s.sel[2] = total count.
__device__ __forceinline__ void fs_rank_bin(FastScratch& s, int rank) {
  constexpr int BPT = 4096 / SEL_BLOCK;  // bins per thread, scanned downwards
  static_assert(BPT % 4 == 0, "bins per thread must fill 16-byte reads");
  const int lo = 4096 - BPT * ((int)threadIdx.x + 1);
  int cv[BPT];
#pragma unroll
  for (int q = 0; q < BPT / 4; ++q) {
    const uint4 a = *reinterpret_cast<const uint4*>(&s.hist[lo + 4 * q]);
    cv[BPT - 1 - 4 * q] = (int)a.x;
    cv[BPT - 2 - 4 * q] = (int)a.y;
    cv[BPT - 3 - 4 * q] = (int)a.z;
    cv[BPT - 4 - 4 * q] = (int)a.w;
  }
  int c = 0;
#pragma unroll
  for (int j = 0; j < BPT; ++j) c += cv[j];
  int total;
  const int exc = block_excl_scan(c, s.scan, &total);
  if (exc < rank && rank <= exc + c) {
    int acc = exc, bin = lo + BPT - 1;
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      if (acc + cv[j] >= rank) { bin = lo + BPT - 1 - j; break; }
      acc += cv[j];
    }
    s.sel[0] = bin;
    s.sel[1] = acc;
  }
  if (threadIdx.x == 0) {
    s.sel[2] = total;
    if (total < rank) s.sel[0] = -1;
  }
}

// Digit (0..15) of the rank-th largest value in s.hist4: s.sel[0] = digit,
// s.sel[1] += count in higher digits, s.sel[3] = count at the digit.
__device__ __forceinline__ void fs_rank_digit(FastScratch& s, int rank, int acc) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int cnt = lane < 16 ? (int)s.hist4[15 - lane] : 0;
    const int inc = acc + wave_incl_scan(cnt);
    if (lane < 16 && inc - cnt < rank && rank <= inc) {
      s.sel[0] = 15 - lane;
      s.sel[1] = inc - cnt;
      s.sel[3] = cnt;
    }
  }
}

// src: the n ordered scores (0 = excluded; see RowScores / MaskedScores).
// id(i): the item's ID (< 2^20), read only for candidates.  VALUE_ONLY: only
// sel.v (the k-th best score) is wanted: no IDs, no tie resolution.
// force_miss places the cut at the best sampled score (a test of the
// fallback: fewer than k candidates unless k ties share it).
// sample(u, i): the score of sample u (item i = fs_sample_item(n, u));
// fast_select without it reads src.at(i).
__device__ __forceinline__ int fs_sample_item(int n, int u) {
  const int j = (int)threadIdx.x + u * SEL_BLOCK;
  return n <= FS_SAMPLE ? j : (int)(((uint64_t)j * (uint64_t)n) >> 12);
}

// Phase 1 of the sampled selection: from this thread's FS_PER sample scores
// sv (0 = excluded), the cut that about k + 4 sqrt(k) + 8 of n items reach
// (the rank-th best sample, rank scaled to the sample); also resets the
// candidate list.  Returns cut >= 1 (1: every valid item).
__device__ __forceinline__ uint32_t fs_cut(const uint32_t (&sv)[FS_PER], int n, int k,
                                           bool force_miss, FastScratch& s, int ts) {
  const bool full = n <= FS_SAMPLE;
  for (int i = threadIdx.x; i < 4096; i += SEL_BLOCK) s.hist[i] = 0;
  if (threadIdx.x < 16) s.hist4[threadIdx.x] = 0;
  if (threadIdx.x == 0) {
    s.ncand = 0;
    s.maxo = 0;
    s.ntie = 0;
    s.sel[0] = -1;
    s.sel[1] = 0;
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < FS_PER; ++u)
    if (sv[u]) atomicAdd(&s.hist[sv[u] >> 4], 1u);
  __syncthreads();
  SKV_TS(ts, 1);
  int rank = k;
  if (!full) {
    const float e = (float)k * (float)FS_SAMPLE / (float)n;
    rank = (int)ceilf(e + 4.f * sqrtf(e) + 8.f);
  }
  if (force_miss) rank = 1;
  fs_rank_bin(s, rank);
  __syncthreads();
  const int b1 = s.sel[0];
  uint32_t cut = 1;  // every valid item
  if (b1 >= 0) {
    const int acc1 = s.sel[1];
#pragma unroll
    for (int u = 0; u < FS_PER; ++u)
      if (sv[u] && (int)(sv[u] >> 4) == b1) atomicAdd(&s.hist4[sv[u] & 15], 1u);
    __syncthreads();
    fs_rank_digit(s, rank, acc1);
    __syncthreads();
    cut = ((uint32_t)b1 << 4) | (uint32_t)s.sel[0];
  }
  __syncthreads();
  SKV_TS(ts, 2);
  return cut;
}

// Phases 3 on: the exact top-k among the candidates s.cand[0 .. s.ncand)
// (every item scoring >= cut; s.maxo their best score).
template <bool VALUE_ONLY, typename IdFn>
__device__ FastResult fs_finish(int k, IdFn id, FastScratch& s, uint32_t cut, int ts) {
  FastResult res;
  res.ok = true;
  res.ncand = 0;
  res.sel.idcut = 0xffffffffu;
  res.sel.all = false;
  res.sel.above = 0;
  SKV_TS(ts, 3);
  const int nc = s.ncand;
  res.ncand = nc;
  if (nc > CAND_CAP || (cut > 1 && nc < k)) {
    res.ok = false;
    return res;
  }
  if (cut == 1 && nc <= k) {  // fewer valid items than k: all are members
    res.sel.all = true;
    res.sel.v = 0;
    res.sel.above = nc;
    return res;
  }
  SKV_TS(ts, 4);
  // ---- 3. exact k-th score among the candidates (nc >= k here)
  const uint32_t maxo = (uint32_t)s.maxo;
  int shift = 0;
  while (((maxo - cut) >> shift) >= 4096u) ++shift;
  for (int i = threadIdx.x; i < 4096; i += SEL_BLOCK) s.hist[i] = 0;
  if (threadIdx.x < 16) s.hist4[threadIdx.x] = 0;
  __syncthreads();
  for (int c = threadIdx.x; c < nc; c += SEL_BLOCK)
    atomicAdd(&s.hist[(cand_ord(s.cand[c]) - cut) >> shift], 1u);
  __syncthreads();
  fs_rank_bin(s, k);
  __syncthreads();
  const int b2 = s.sel[0];
  int above = s.sel[1];
  // the IDs of the candidates in the k-th score's bin (the only possible
  // ties), loaded now so that they arrive while the score itself is found
  constexpr int CPT = CAND_CAP / SEL_BLOCK;  // candidates per thread
  uint32_t pid[CPT];
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const int c = (int)threadIdx.x + u * SEL_BLOCK;
    pid[u] = 0u;
    if (!VALUE_ONLY && c < nc) {
      const uint64_t key = s.cand[c];
      if ((int)((cand_ord(key) - cut) >> shift) == b2) pid[u] = id(cand_pos(key));
    }
  }
  uint32_t v;
  int ties;
  if (shift == 0) {
    v = cut + (uint32_t)b2;
    ties = (int)s.hist[b2];
  } else {
    const uint32_t lowmask = (1u << shift) - 1u;
    for (int c = threadIdx.x; c < nc; c += SEL_BLOCK) {
      const uint32_t d = cand_ord(s.cand[c]) - cut;
      if ((int)(d >> shift) == b2) atomicAdd(&s.hist4[d & lowmask], 1u);
    }
    __syncthreads();
    fs_rank_digit(s, k, above);
    __syncthreads();
    v = cut + (((uint32_t)b2 << shift) | (uint32_t)s.sel[0]);
    above = s.sel[1];
    ties = s.sel[3];
  }
  __syncthreads();
  res.sel.v = v;
  res.sel.above = above;
  SKV_TS(ts, 5);
  const int need = k - above;
  if (VALUE_ONLY || need >= ties) return res;  // every tie is a member

  // ---- ties at v: the `need` lowest IDs win (tied keys keep their ID for
  // fs_member)
  if (ties <= FS_TIE_RANK) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = (int)threadIdx.x + u * SEL_BLOCK;
      if (c >= nc) break;
      const uint64_t key = s.cand[c];
      if (cand_ord(key) == v) {
        s.tie[atomicAdd(&s.ntie, 1)] = pid[u];
        s.cand[c] = key | CAND_HAS_ID | ((uint64_t)pid[u] << 20);
      }
    }
    __syncthreads();
    if ((int)threadIdx.x < ties) {  // rank = number of smaller tied IDs
      const uint32_t x = s.tie[threadIdx.x];
      if (count_below(s.tie, ties, x) == need - 1) s.sel[2] = (int)x;
    }
    __syncthreads();
    res.sel.idcut = (uint32_t)s.sel[2];
    __syncthreads();
    return res;
  }
  auto val = [&](int c, uint64_t* out) {
    const uint64_t key = s.cand[c];
    if (cand_ord(key) != v) return false;
    *out = 0xfffffu - id(cand_pos(key));
    return true;
  };
  const uint64_t kth = block_kth<24>(nc, need, val, s.k);
  res.sel.idcut = 0xfffffu - (uint32_t)kth;
  return res;
}

template <bool VALUE_ONLY, typename Src, typename IdFn, typename SampleFn>
__device__ FastResult fast_select_s(const Src& src, int n, int k, IdFn id, FastScratch& s,
                                    bool force_miss, int ts, SampleFn sample) {
  // ---- 1. sample
  uint32_t sv[FS_PER];
#pragma unroll
  for (int u = 0; u < FS_PER; ++u) {
    const int i = fs_sample_item(n, u);
    sv[u] = i >= n ? 0u : sample(u, i);
  }
  // the candidate pass's first Src::PRE octets per thread, loaded now so that
  // they arrive while the cut is computed
  static_assert(Src::PRE % FS_OCT == 0, "prefetch whole passes");
  const int no = (n + 7) >> 3;
  uint4 pre[Src::PRE];
#pragma unroll
  for (int q = 0; q < Src::PRE; ++q) {
    const int o = (int)threadIdx.x + q * SEL_BLOCK;
    pre[q] = o < no ? src.oct(o) : make_uint4(0, 0, 0, 0);
  }
  const uint32_t cut = fs_cut(sv, n, k, force_miss, s, ts);

  // ---- 2. candidate positions: packed compares into a per-lane bit mask
  // (cut >= 1, so excluded items never pass), then one LDS append per set bit
  {
    const int lane = threadIdx.x & 63;
    const int base0 = threadIdx.x & ~63;
    const u16x2 cm1 = {(uint16_t)(cut - 1), (uint16_t)(cut - 1)};  // cut >= 1
    uint32_t mx = 0;
    auto pass = [&](const uint4 (&w)[FS_OCT], int base) {
      uint32_t mask = 0;
#pragma unroll
      for (int r = 0; r < FS_OCT; ++r) {
        // bit 2e: low half of word e >= cut; bit 2e + 1: high half
        const uint32_t m = ge_cut2(w[r].x, cm1) | (ge_cut2(w[r].y, cm1) << 2) |
                           (ge_cut2(w[r].z, cm1) << 4) | (ge_cut2(w[r].w, cm1) << 6);
        uint32_t m8 = (m & 0x55u) | ((m >> 15) & 0xaau);
        const int valid = n - 8 * (base + r * SEL_BLOCK + lane);
        if (valid < 8) m8 &= valid > 0 ? (1u << valid) - 1u : 0u;
        mask |= m8 << (8 * r);
      }
      const int cnt = __popc(mask);
      const int inc = wave_incl_scan(cnt);
      int wbase = 0;
      if (lane == 63) wbase = atomicAdd(&s.ncand, inc);
      wbase = __builtin_amdgcn_readlane(wbase, 63);
      int slot = wbase + inc - cnt;
#pragma unroll
      for (int r = 0; r < FS_OCT; ++r) {  // compile-time octet: no indexed arrays
        uint32_t m8 = (mask >> (8 * r)) & 0xffu;
        const u32x4 wv = {w[r].x, w[r].y, w[r].z, w[r].w};
        const int pos0 = 8 * (base + r * SEL_BLOCK + lane);
        while (m8) {
          const int e = __ffs(m8) - 1;
          m8 &= m8 - 1;
          const uint32_t word = wv[e >> 1];
          const uint32_t o = (e & 1) ? word >> 16 : word & 0xffffu;
          mx = max(mx, o);
          if (slot < CAND_CAP) s.cand[slot] = ((uint64_t)o << 40) | (uint64_t)(pos0 + e);
          ++slot;
        }
      }
    };
    // passes over the octets loaded at entry, then over the rest
#pragma unroll
    for (int p = 0; p < Src::PRE / FS_OCT; ++p) {
      const int base = base0 + p * FS_OCT * SEL_BLOCK;
      if (base >= no) break;  // wave-uniform
      const uint4 w[FS_OCT] = {pre[FS_OCT * p], pre[FS_OCT * p + 1], pre[FS_OCT * p + 2],
                               pre[FS_OCT * p + 3]};
      pass(w, base);
    }
    for (int base = base0 + Src::PRE * SEL_BLOCK; base < no; base += FS_OCT * SEL_BLOCK) {
      uint4 w[FS_OCT];
#pragma unroll
      for (int r = 0; r < FS_OCT; ++r) {
        const int o = base + r * SEL_BLOCK + lane;
        w[r] = o < no ? src.oct(o) : make_uint4(0, 0, 0, 0);
      }
      pass(w, base);
    }
    mx = (uint32_t)wave_max((int)mx);
    if (lane == 0) atomicMax(&s.maxo, (int)mx);
  }
  __syncthreads();
  return fs_finish<VALUE_ONLY>(k, id, s, cut, ts);
}

// 16-item tiles of a 16-byte aligned row of ordered scores.
struct RowTiles {
  const uint16_t* __restrict__ row;
  __device__ void tile(int t, uint4 (&w)[2]) const {
    const uint4* r4 = reinterpret_cast<const uint4*>(row) + 2 * t;
    w[0] = r4[0];
    w[1] = r4[1];
  }
};
// 16-item tiles of MaskedScores (score where gate >= thr, else excluded).
struct MaskedTiles {
  const uint16_t* __restrict__ score;
  const uint16_t* __restrict__ gate;
  uint32_t thr;
  __device__ void tile(int t, uint4 (&w)[2]) const {
    const uint4* s4 = reinterpret_cast<const uint4*>(score) + 2 * t;
    const uint4* g4 = reinterpret_cast<const uint4*>(gate) + 2 * t;
    const uint4 s0 = s4[0], s1 = s4[1], g0 = g4[0], g1 = g4[1];
    w[0] = MaskedScores::pick4(s0, g0, thr);
    w[1] = MaskedScores::pick4(s1, g1, thr);
  }
};

// Exact top-k of n (FS_SAMPLE < n <= 64 x SEL_BLOCK) ordered scores whose
// producer also wrote an upper bound of every 16-item tile (tmx, e.g. the
// tile's max): from this thread's fast_select sample sv the same cut as
// fast_select, then the candidate pass over the tiles whose bound reaches
// the cut only (their scores loaded then from src), one tile per thread and
// round.  The candidates are exactly fast_select's, so is the result.
template <typename TileSrc, typename IdFn>
__device__ FastResult tiled_select(const TileSrc& src, const uint16_t* __restrict__ tmx,
                                   const uint32_t (&sv)[FS_PER], int n, int k, IdFn id,
                                   FastScratch& s, bool force_miss, int ts) {
  // ---- 1. this thread's 4 tile bounds (loaded with the caller's sample)
  const int ntile = (n + 15) >> 4;
  const int t4 = 4 * (int)threadIdx.x;
  const uint2 tm = t4 < ntile ? *reinterpret_cast<const uint2*>(tmx + t4) : make_uint2(0, 0);
  const uint32_t cut = fs_cut(sv, n, k, force_miss, s, ts);
  // ---- 2. the tiles whose max reaches the cut, listed in s.hist (free
  // until fs_finish)
  const uint32_t tv[4] = {tm.x & 0xffffu, tm.x >> 16, tm.y & 0xffffu, tm.y >> 16};
  uint32_t hot = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) hot |= (uint32_t)(t4 + e < ntile && tv[e] >= cut) << e;
  int nhot;
  int at = block_excl_scan(__popc(hot), s.scan, &nhot);  // ends with a barrier
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if ((hot >> e) & 1u) s.hist[at++] = (uint32_t)(t4 + e);
  __syncthreads();
  SKV_TS(ts, 7);
  // ---- 3. candidates of the listed tiles (packed compares, one LDS append
  // per set bit, as fast_select's pass).  The tiles of every round (at most
  // TL_ROUNDS: the caller bounds the row to 4 x SEL_BLOCK tiles) are loaded
  // before the first is scanned, so the rounds share one memory latency;
  // the loads are branch-free (an unlisted slot reloads tile 0, unused).
  constexpr int TL_ROUNDS = 4;
  const int lane = threadIdx.x & 63;
  const u16x2 cm1 = {(uint16_t)(cut - 1), (uint16_t)(cut - 1)};  // cut >= 1
  uint32_t mx = 0;
  int tl[TL_ROUNDS];
  uint4 tw[TL_ROUNDS][2];
#pragma unroll
  for (int r = 0; r < TL_ROUNDS; ++r) {
    const int i = r * SEL_BLOCK + (int)threadIdx.x;
    tl[r] = i < nhot ? (int)s.hist[i] : -1;
  }
#pragma unroll
  for (int r = 0; r < TL_ROUNDS; ++r) src.tile(max(tl[r], 0), tw[r]);
#pragma unroll
  for (int r = 0; r < TL_ROUNDS; ++r) {
    if (r * SEL_BLOCK >= nhot) break;  // block-uniform
    const int tile = tl[r];
    uint32_t mask = 0;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t m = ge_cut2(tw[r][q].x, cm1) | (ge_cut2(tw[r][q].y, cm1) << 2) |
                         (ge_cut2(tw[r][q].z, cm1) << 4) | (ge_cut2(tw[r][q].w, cm1) << 6);
      mask |= ((m & 0x55u) | ((m >> 15) & 0xaau)) << (8 * q);
    }
    if (tile < 0) mask = 0;
    else if (n - 16 * tile < 16) mask &= (1u << (n - 16 * tile)) - 1u;
    const int cnt = __popc(mask);
    const int inc = wave_incl_scan(cnt);
    int wbase = 0;
    if (lane == 63) wbase = atomicAdd(&s.ncand, inc);
    wbase = __builtin_amdgcn_readlane(wbase, 63);
    int slot = wbase + inc - cnt;
#pragma unroll
    for (int q = 0; q < 2; ++q) {  // compile-time octet: no indexed arrays
      uint32_t m8 = (mask >> (8 * q)) & 0xffu;
      const u32x4 wv = {tw[r][q].x, tw[r][q].y, tw[r][q].z, tw[r][q].w};
      const int pos0 = 16 * tile + 8 * q;
      while (m8) {
        const int e = __ffs(m8) - 1;
        m8 &= m8 - 1;
        const uint32_t word = wv[e >> 1];
        const uint32_t o = (e & 1) ? word >> 16 : word & 0xffffu;
        mx = max(mx, o);
        if (slot < CAND_CAP) s.cand[slot] = ((uint64_t)o << 40) | (uint64_t)(pos0 + e);
        ++slot;
      }
    }
  }
  mx = (uint32_t)wave_max((int)mx);
  if (lane == 0) atomicMax(&s.maxo, (int)mx);
  __syncthreads();
  SKV_TS(ts, 8);
  return fs_finish<false>(k, id, s, cut, ts);
}

template <bool VALUE_ONLY = false, typename Src, typename IdFn>
__device__ FastResult fast_select(const Src& src, int n, int k, IdFn id, FastScratch& s,
                                  bool force_miss = false, int ts = -1) {
  return fast_select_s<VALUE_ONLY>(src, n, k, id, s, force_miss, ts,
                                   [&](int, int i) { return src.at(i); });
}

}  // namespace skv
