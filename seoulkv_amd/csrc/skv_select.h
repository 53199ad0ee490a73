// Block-level top-k selection by (ordered BF16 score desc, ID asc).
//
// The block first copies the n 16-bit ordered scores into LDS (one coalesced
// pass over memory).  A 4096-bin histogram of the top 12 bits (one shared
// LDS histogram: BF16 scores of a pool span only a few binades, so coarser
// per-wave bins would put most lanes of a wave on one address) and a 16-bin
// pass over the low 4 bits then find the score v of the k-th best item and
// the count of items strictly above it.
// Items scoring exactly v are ties; the lowest IDs among them win: when all
// ties are needed nothing more is read, otherwise the tie IDs are gathered
// into LDS and a radix select over (0xfffff - id) finds the cut.  Ordered
// score 0 marks an excluded item (a real BF16 score never maps to 0).
#pragma once

#include "skv_device.h"

namespace skv {

constexpr int SEL_BLOCK = 1024;
constexpr int SEL_WAVES = SEL_BLOCK / WAVE;
constexpr int TIE_CAP = 2048;

struct KthScratch {
  uint32_t hist[SEL_WAVES][256];
  int sel[2];
};

struct SelectScratch {
  union {
    KthScratch k;          // 256-bin radix passes (ties, fallbacks)
    uint32_t hist12[4096]; // first pass of block_select
  };
  uint32_t tie_key[TIE_CAP];
  uint32_t hist4[16];
  int sel[2];
  int ntie;
  int scan[SEL_WAVES + 1];
};

// Selection outcome: member(i) <=> ord > v || (ord == v && id <= idcut),
// among items with ord != 0; all == true means every valid item is a member.
struct Selection {
  uint32_t v;
  uint32_t idcut;
  int above;
  bool all;
  __device__ bool member(uint32_t ord, uint32_t id) const {
    if (ord == 0) return false;
    if (all) return true;
    return ord > v || (ord == v && id <= idcut);
  }
};

// Locate the digit of the rank-th largest value in a 256-bin histogram (in
// s.hist[0]): returns the digit and the count of values in higher bins, or -1
// when fewer than rank values exist.  Executed by wave 0; result in s.sel.
__device__ __forceinline__ void kth_digit(KthScratch& s, int rank) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int base = 255 - 4 * lane;
    const int c4 = s.hist[0][base] + s.hist[0][base - 1] + s.hist[0][base - 2] +
                   s.hist[0][base - 3];
    const int inc = wave_incl_scan(c4);
    const int exc = inc - c4;
    if (exc < rank && rank <= inc) {
      int acc = exc, digit = base;
      for (int j = 0; j < 4; ++j) {
        const int cnt = s.hist[0][base - j];
        if (acc + cnt >= rank) { digit = base - j; break; }
        acc += cnt;
      }
      s.sel[0] = digit;
      s.sel[1] = acc;
    }
    if (lane == 63 && inc < rank) {
      s.sel[0] = -1;
      s.sel[1] = inc;
    }
  }
}

__device__ __forceinline__ void clear_hist(KthScratch& s) {
  for (int i = threadIdx.x; i < SEL_WAVES * 256; i += blockDim.x) (&s.hist[0][0])[i] = 0;
}

__device__ __forceinline__ void reduce_hist(KthScratch& s) {
  if (threadIdx.x < 256) {
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < SEL_WAVES; ++w) t += s.hist[w][threadIdx.x];
    s.hist[0][threadIdx.x] = t;
  }
}

// k-th largest of val(i) over n items (multiplicities counted), 8-bit radix
// passes over BITS bits reading val from memory each pass.  Returns 0 when
// fewer than k valid values exist.
template <int BITS, typename ValFn>
__device__ uint64_t block_kth(int n, int k, ValFn val, KthScratch& s) {
  const int wave = threadIdx.x >> 6;
  uint64_t prefix = 0;
  int remaining = k;
  for (int shift = BITS - 8; shift >= 0; shift -= 8) {
    clear_hist(s);
    __syncthreads();
    const int hs = shift + 8;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      uint64_t v;
      if (!val(i, &v)) continue;
      if (hs < BITS && (v >> hs) != (prefix >> hs)) continue;
      atomicAdd(&s.hist[wave][(v >> shift) & 255], 1u);
    }
    __syncthreads();
    reduce_hist(s);
    __syncthreads();
    kth_digit(s, remaining);
    __syncthreads();
    const int digit = s.sel[0], acc = s.sel[1];
    __syncthreads();
    if (digit < 0) return 0;
    remaining -= acc;
    prefix |= (uint64_t)digit << shift;
  }
  return prefix;
}

// Copy n 16-bit scores src[0..n) (16-byte aligned) into LDS, 8 per 16-byte
// load and store, 4 loads in flight per thread; xf maps each raw value.  The
// LDS copy is zero-padded to a whole number of octets (8 scores).
template <typename Fn>
__device__ __forceinline__ void load_lds_scores(uint16_t* so, const uint16_t* __restrict__ src,
                                                int n, Fn xf) {
  const int nv = n >> 3, no = (n + 7) >> 3;
  const uint4* s4 = reinterpret_cast<const uint4*>(src);
  uint4* d4 = reinterpret_cast<uint4*>(so);
  for (int base = threadIdx.x; base < nv; base += 4 * blockDim.x) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = base + u * blockDim.x;
      v[u] = i < nv ? s4[i] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = base + u * blockDim.x;
      if (i >= nv) continue;
      uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = xf(w[e] & 0xffffu) | (xf(w[e] >> 16) << 16);
      d4[i] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  if (nv < no && threadIdx.x < 8) {  // tail octet, zero-padded
    const int i = 8 * nv + threadIdx.x;
    so[i] = i < n ? (uint16_t)xf(src[i]) : 0;
  }
}

// Apply fn(item, score) to every LDS score, one 16-byte octet per read with
// two octets in flight per thread.
template <typename Fn>
__device__ __forceinline__ void for_scores(const uint16_t* so, int n, Fn fn) {
  const int no = (n + 7) >> 3;
  const uint4* s4 = reinterpret_cast<const uint4*>(so);
  for (int o = threadIdx.x; o < no; o += 2 * blockDim.x) {
    const int o2 = o + blockDim.x;
    const uint4 a = s4[o];
    const uint4 b = o2 < no ? s4[o2] : make_uint4(0, 0, 0, 0);
    const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) fn(8 * o + e, (wa[e >> 1] >> (16 * (e & 1))) & 0xffffu);
    if (o2 < no) {
#pragma unroll
      for (int e = 0; e < 8; ++e) fn(8 * o2 + e, (wb[e >> 1] >> (16 * (e & 1))) & 0xffffu);
    }
  }
}

// Select the k best of the n LDS-resident ordered scores so[] (0 = excluded),
// ties at the cut resolved by the lowest id(i).
template <typename IdFn>
__device__ Selection block_select(const uint16_t* so, int n, int k, IdFn id, SelectScratch& s) {
  Selection res;
  res.idcut = 0xffffffffu;
  res.all = false;
  // pass A: 4096 bins over the top 12 bits
  for (int i = threadIdx.x; i < 4096; i += blockDim.x) s.hist12[i] = 0;
  if (threadIdx.x < 16) s.hist4[threadIdx.x] = 0;
  if (threadIdx.x == 0) s.ntie = 0;
  __syncthreads();
  for_scores(so, n, [&](int, uint32_t o) {
    if (o) atomicAdd(&s.hist12[o >> 4], 1u);
  });
  __syncthreads();
  {  // thread t owns bins 4095 - PER t .. 4096 - PER (t + 1) (descending)
    constexpr int PER = 4096 / SEL_BLOCK;
    const int top = 4095 - PER * (int)threadIdx.x;
    int c = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) c += s.hist12[top - j];
    int total;
    const int exc = block_excl_scan(c, s.scan, &total);
    if (exc < k && k <= exc + c) {
      int acc = exc, bin = top;
      for (int j = 0; j < PER; ++j) {
        const int cnt = s.hist12[top - j];
        if (acc + cnt >= k) { bin = top - j; break; }
        acc += cnt;
      }
      s.sel[0] = bin;
      s.sel[1] = acc;
    }
    if (threadIdx.x == 0 && total < k) {
      s.sel[0] = -1;
      s.sel[1] = total;
    }
  }
  __syncthreads();
  const int b1 = s.sel[0], acc1 = s.sel[1];
  __syncthreads();
  if (b1 < 0) {
    res.all = true;
    res.v = 0;
    res.above = acc1;
    return res;
  }
  // pass B: the low 4 bits within bin b1
  for_scores(so, n, [&](int, uint32_t o) {
    if ((int)(o >> 4) == b1) atomicAdd(&s.hist4[o & 15], 1u);
  });
  __syncthreads();
  int d0 = 0, acc0 = 0, ties = 0;
  {
    const int need1 = k - acc1;
    int acc = 0;
    for (int d = 15; d >= 0; --d) {
      const int cnt = s.hist4[d];
      if (acc + cnt >= need1) { d0 = d; ties = cnt; break; }
      acc += cnt;
    }
    acc0 = acc;
  }
  res.v = ((uint32_t)b1 << 4) | (uint32_t)d0;
  res.above = acc1 + acc0;
  const int need = k - res.above;
  if (need >= ties) return res;  // every tie is a member
  // gather the tie IDs; keep the `need` smallest
  const uint32_t v = res.v;
  for_scores(so, n, [&](int i, uint32_t o) {
    if (o == v) {
      const int slot = atomicAdd(&s.ntie, 1);
      if (slot < TIE_CAP) s.tie_key[slot] = 0xfffffu - id(i);
    }
  });
  __syncthreads();
  const int nt = s.ntie;
  __syncthreads();
  uint64_t kth;
  if (nt <= TIE_CAP) {
    auto val = [&](int i, uint64_t* out) { *out = s.tie_key[i]; return true; };
    kth = block_kth<24>(nt, need, val, s.k);
  } else {
    auto val = [&](int i, uint64_t* out) {
      if (so[i] != v) return false;
      *out = 0xfffffu - id(i);
      return true;
    };
    kth = block_kth<24>(n, need, val, s.k);
  }
  res.idcut = 0xfffffu - (uint32_t)kth;
  return res;
}

// Membership bitmap of a selection over LDS-resident scores: word w covers
// items 64w .. 64w+63.  Lane l of a wave tests one octet (8 items); the
// 8-bit masks of 8 consecutive lanes form one word.
template <typename IdFn>
__device__ __forceinline__ void write_members(const uint16_t* so, int n, const Selection& sel,
                                              IdFn id, uint64_t* bm) {
  const int lane = threadIdx.x & 63;
  const int no = (n + 7) >> 3;
  const uint4* s4 = reinterpret_cast<const uint4*>(so);
  for (int base = threadIdx.x & ~63; base < no; base += blockDim.x) {
    const int o = base + lane;
    uint32_t m8 = 0;
    if (o < no) {
      const uint4 q = s4[o];
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t sc = (w[e >> 1] >> (16 * (e & 1))) & 0xffffu;
        bool m = false;
        if (sc && (sel.all || sc > sel.v)) m = true;
        else if (sc && sc == sel.v) m = id(8 * o + e) <= sel.idcut;
        m8 |= (uint32_t)m << e;
      }
    }
    uint64_t word = (uint64_t)m8 << (8 * (lane & 7));
    word |= __shfl_xor(word, 1, WAVE);
    word |= __shfl_xor(word, 2, WAVE);
    word |= __shfl_xor(word, 4, WAVE);
    if ((lane & 7) == 0 && o < no) bm[o >> 3] = word;
  }
}

}  // namespace skv
