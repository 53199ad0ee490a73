// Exact block top-k by (ordered BF16 score desc, ID asc) of n <= 8 x SEL_BLOCK
// items held in registers: thread t holds the octet of items 8t .. 8t+7 as
// packed 16-bit ordered scores (0 = excluded or absent).
//
// Two histogram passes over the registers find the k-th best score v and the
// count of items above it: 4096 bins of the top 12 bits (LDS atomics), then
// 16 bins of the low 4 bits of the chosen bin.  No candidate list and no
// second read of memory.  Items tied at v are members in ID order:
//   POS_IDS (the ID is the item position): a block scan of the per-thread
//   tie counts ranks every tie directly;
//   otherwise the tied IDs are gathered into LDS and ranked by comparison
//   (up to FS_TIE_RANK ties; beyond that ok = false and the caller runs the
//   full selection).
#pragma once

#include "skv_fastsel.h"

namespace skv {

constexpr int OCT_ITEMS = 8 * SEL_BLOCK;  // largest n held one octet per thread

// Half e (0..7, a compile-time constant after unrolling) of an octet.
__device__ __forceinline__ uint32_t oct_half(const u32x4& wv, int e) {
  return (e & 1) ? wv[e >> 1] >> 16 : wv[e >> 1] & 0xffffu;
}

// This thread's octet of a 16-byte aligned row of n ordered scores, items
// beyond n cleared (the row may hold stale values there).
__device__ __forceinline__ uint4 load_oct(const uint16_t* __restrict__ row, int n) {
  const int t = threadIdx.x, valid = n - 8 * t;
  if (valid <= 0) return make_uint4(0, 0, 0, 0);
  const uint4 w = reinterpret_cast<const uint4*>(row)[t];
  if (valid >= 8) return w;
  auto cut = [&](uint32_t x, int q) {  // halves of word q kept: valid - 2q
    const int keep = valid - 2 * q;
    return keep >= 2 ? x : keep == 1 ? (x & 0xffffu) : 0u;
  };
  return make_uint4(cut(w.x, 0), cut(w.y, 1), cut(w.z, 2), cut(w.w, 3));
}

// Items tied at the k-th score where only `need` of the `ties` (<= FS_TIE_RANK)
// are members: the need lowest IDs win.  eq: this thread's tied items as
// member bits; pos(b): the position of bit b; s.ntie must be 0.  The tie
// positions are compacted into LDS, their IDs read with one load per tie and
// ranked by comparison.  Returns this thread's winning bits.
template <typename PosFn, typename IdFn>
__device__ __forceinline__ uint64_t rank_ties(uint64_t eq, int ties, int need, PosFn pos,
                                              IdFn id, FastScratch& s) {
  const int t = threadIdx.x;
  uint32_t* tpos = reinterpret_cast<uint32_t*>(s.cand);  // [FS_TIE_RANK] positions
  uint8_t* win = reinterpret_cast<uint8_t*>(tpos + FS_TIE_RANK);  // [FS_TIE_RANK]
  const int c = __popcll(eq);
  const int exc = c ? atomicAdd(&s.ntie, c) : 0;  // s.ntie is 0 on entry
  {
    uint64_t rest = eq;
    for (int j = exc; rest; ++j) {
      tpos[j] = (uint32_t)pos(__ffsll((long long)rest) - 1);
      rest &= rest - 1;
    }
  }
  __syncthreads();
  if (t < ties) s.tie[t] = id((int)tpos[t]);
  __syncthreads();
  if (t < ties) {  // rank = number of smaller tied IDs (IDs are distinct)
    const uint32_t x = s.tie[t];
    win[t] = count_below(s.tie, ties, x) < need;
  }
  __syncthreads();
  uint64_t m = 0, rest = eq;
  for (int j = exc; rest; ++j) {
    const uint64_t low = rest & (0ull - rest);
    if (win[j]) m |= low;
    rest &= rest - 1;
  }
  __syncthreads();  // the scratch may be reused on return
  return m;
}

struct OctResult {
  Selection sel;  // v (k-th best score), above (count scoring > v), all
  uint32_t mine;  // member bits of this thread's items (bit 8o + e = item e of octet o)
  bool ok;        // false: too many ties at v to rank here (use the full path)
};

// NO octets per thread: octet o of thread t holds items 8 (t + o SEL_BLOCK) ..
// +7 (NO = 2: the row's first 8 SEL_BLOCK items, then the rest, in the same
// layout).  POS_IDS ranks ties by a block scan in thread order, which is
// position order only for one octet per thread.
template <int NO, bool VALUE_ONLY, bool POS_IDS, typename IdFn>
__device__ __forceinline__ OctResult octn_select(const uint4 (&w)[NO], int k, IdFn id,
                                                 FastScratch& s, int ts = -1) {
  static_assert(NO >= 1 && NO <= 4 && !(POS_IDS && NO > 1), "octets per thread");
  OctResult res;
  res.ok = true;
  res.mine = 0;
  res.sel.v = 0;
  res.sel.idcut = 0xffffffffu;
  res.sel.above = 0;
  res.sel.all = false;
  u32x4 wv[NO];
#pragma unroll
  for (int o = 0; o < NO; ++o) wv[o] = u32x4{w[o].x, w[o].y, w[o].z, w[o].w};
  for (int i = threadIdx.x; i < 4096; i += SEL_BLOCK) s.hist[i] = 0;
  if (threadIdx.x < 16) s.hist4[threadIdx.x] = 0;
  if (threadIdx.x == 0) {
    s.ntie = 0;
    s.sel[0] = -1;
    s.sel[1] = 0;
  }
  __syncthreads();
  uint32_t valid = 0;
#pragma unroll
  for (int o = 0; o < NO; ++o)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t x = oct_half(wv[o], e);
      if (x) {
        atomicAdd(&s.hist[x >> 4], 1u);
        valid |= 1u << (8 * o + e);
      }
    }
  __syncthreads();
  SKV_TS(ts, 1);
  fs_rank_bin(s, k);
  __syncthreads();
  SKV_TS(ts, 2);
  const int b1 = s.sel[0];
  const int acc1 = s.sel[1];
  const int total = s.sel[2];
  if (b1 < 0) {  // fewer than k valid items: all of them are members
    __syncthreads();  // the scratch may be reused on return
    res.sel.all = true;
    res.sel.above = total;
    res.mine = valid;
    return res;
  }
#pragma unroll
  for (int o = 0; o < NO; ++o)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t x = oct_half(wv[o], e);
      if (x && (int)(x >> 4) == b1) atomicAdd(&s.hist4[x & 15], 1u);
    }
  __syncthreads();
  fs_rank_digit(s, k, acc1);
  __syncthreads();
  SKV_TS(ts, 3);
  const uint32_t v = ((uint32_t)b1 << 4) | (uint32_t)s.sel[0];
  const int above = s.sel[1];
  const int ties = s.sel[3];
  __syncthreads();  // the scratch may be reused on return
  res.sel.v = v;
  res.sel.above = above;
  if (VALUE_ONLY) return res;
  uint32_t gt = 0, eq = 0;
#pragma unroll
  for (int o = 0; o < NO; ++o)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t x = oct_half(wv[o], e);
      gt |= (uint32_t)(x > v) << (8 * o + e);
      eq |= (uint32_t)(x == v) << (8 * o + e);
    }
  const int need = k - above;  // 1 <= need <= ties
  if (need >= ties) {
    res.mine = gt | eq;
    return res;
  }
  if (POS_IDS) {  // ties in position order: thread order, then bit order
    const int c = __popc(eq);
    int nt;
    const int exc = block_excl_scan(c, s.scan, &nt);  // ends with a barrier
    const int take = min(max(need - exc, 0), c);  // this thread's lowest `take` ties
    uint32_t m = 0, rest = eq;
    for (int j = 0; j < take; ++j) {
      m |= rest & (0u - rest);
      rest &= rest - 1;
    }
    res.mine = gt | m;
    return res;
  }
  if (ties > FS_TIE_RANK) {
    res.ok = false;
    return res;
  }
  res.mine = gt | (uint32_t)rank_ties(
                       eq, ties, need,
                       [](int b) { return 8 * ((int)threadIdx.x + (b >> 3) * SEL_BLOCK) + (b & 7); },
                       id, s);
  return res;
}

template <bool VALUE_ONLY, bool POS_IDS, typename IdFn>
__device__ __forceinline__ OctResult oct_select(const uint4 w, int k, IdFn id, FastScratch& s,
                                                int ts = -1) {
  const uint4 w1[1] = {w};
  return octn_select<1, VALUE_ONLY, POS_IDS>(w1, k, id, s, ts);
}

}  // namespace skv
