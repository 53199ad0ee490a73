// SeoulKV4 sparse decode step for MI355X (gfx950).
//
// One decode step = query prep -> coarse 2-bit centroid intervals -> per-head
// P-th lower bound -> survivor masks -> fine 4-bit centroid scores -> per-head
// top-P + union -> spill-2 pool (mate-ownership dedup, encounter order) ->
// 2-bit key scores -> per-head top-1600 + union U1 -> 4-bit scores -> per-head
// top-256 + union U2 -> 8-bit scores -> per-head top-100 -> sparse FP8 SDPA.
// Reference stages: see the table in skv_step.h.
//
// Selection keys are (ordered BF16 score, lowest ID first); all score dots
// are exact integers on the int8 matrix cores (see skv_device.h).

#include "skv_device.h"
#include "skv_step.h"

namespace skv {

// ============================================================ query prep
// One block per KV group, 1024 threads: thread t owns head t/256, dim t%256.
__global__ __launch_bounds__(1024) void k_qprep(StepArgs a) {
  const int g = blockIdx.x;
  const int t = threadIdx.x, h = t >> 8, d = t & 255;
  const int lane = t & 63, wave = t >> 6;  // 4 waves per head
  __shared__ int s_X[QV_COUNT][H][D];
  __shared__ int s_red[16];
  __shared__ long long s_red64[16];

  const uint32_t qb = a.q[(g * H + h) * D + d];
  const float qf = bf16_f32(qb);
  const float ks = a.kscale[g * D + d];
  const float prod = __fmul_rn(qf, ks);
  uint32_t vb[QV_COUNT];
  vb[QV_RAW] = qb;
  vb[QV_Q15] = bf16_rne(__fmul_rn(prod, 0.015625f));    // q s / 64
  vb[QV_QS] = bf16_rne(__fmul_rn(prod, 0.00390625f));   // q s / 256

  for (int v = 0; v < QV_COUNT; ++v) {
    const uint32_t b = vb[v];
    const int expf = (b >> 7) & 0xff, mant = b & 0x7f;
    const int sig = expf ? (mant | 0x80) : mant;
    const int ex = expf ? expf - 134 : -133;
    int m = wave_max(sig ? ex : -(1 << 20));
    if (lane == 0) s_red[wave] = m;
    __syncthreads();
    int exmax = max(max(s_red[h * 4 + 0], s_red[h * 4 + 1]), max(s_red[h * 4 + 2], s_red[h * 4 + 3]));
    __syncthreads();
    if (exmax == -(1 << 20)) exmax = 0;
    const int shift = ex - exmax + FX_HEADROOM;
    int mag = shift >= 0 ? (sig << shift) : (shift <= -9 ? 0 : (sig >> -shift));
    const int X = (b & 0x8000u) ? -mag : mag;
    s_X[v][h][d] = X;
    a.qop[g * QV_COUNT + v].X[h][d] = X;
    // S_h and (RAW) the squared norm, exact in int64.
    long long sx = wave_sum64((long long)X);
    long long sq = wave_sum64((long long)X * X);
    if (lane == 0) s_red64[wave] = sx;
    __syncthreads();
    if (d == 0) {
      long long S = s_red64[h * 4] + s_red64[h * 4 + 1] + s_red64[h * 4 + 2] + s_red64[h * 4 + 3];
      a.qop[g * QV_COUNT + v].sum[h] = S;
      a.qop[g * QV_COUNT + v].fx[h] = exmax - FX_HEADROOM;
    }
    __syncthreads();
    if (v == QV_RAW) {
      if (lane == 0) s_red64[wave] = sq;
      __syncthreads();
      if (d == 0) {
        unsigned long long N = (unsigned long long)(s_red64[h * 4] + s_red64[h * 4 + 1] +
                                                    s_red64[h * 4 + 2] + s_red64[h * 4 + 3]);
        float norm = sqrt_rne_scaled(N, exmax - FX_HEADROOM);
        a.qop[g * QV_COUNT + QV_RAW].norm[h] = __fmul_rn(norm, a.lam[g]);
      }
      __syncthreads();
    }
  }
  __syncthreads();
  // B images: bimg[kc][lane][m] bytes = limb (col%4) of X_{col/4}[dim],
  // col = lane%16, dim = (lane/16)*64 + kc*16 + 4m + byte.
  for (int w = t; w < QV_COUNT * 4 * WAVE * 4; w += blockDim.x) {
    const int v = w / (4 * WAVE * 4);
    const int r = w % (4 * WAVE * 4);
    const int kc = r / (WAVE * 4), l = (r / 4) % WAVE, m = r % 4;
    const int col = l & 15, hh = col >> 2, limb = col & 3;
    uint32_t word = 0;
    for (int byte = 0; byte < 4; ++byte) {
      const int dim = (l >> 4) * 64 + kc * 16 + 4 * m + byte;
      const int X = s_X[v][hh][dim];
      const int l0 = (int)(int8_t)(X & 0xff);
      const int x1 = (X - l0) >> 8;
      const int l1 = (int)(int8_t)(x1 & 0xff);
      const int l2 = (x1 - l1) >> 8;
      const int limbv = limb == 0 ? l0 : limb == 1 ? l1 : limb == 2 ? l2 : 0;
      word |= (uint32_t)(limbv & 0xff) << (8 * byte);
    }
    a.qop[g * QV_COUNT + v].bimg[kc][l][m] = word;
  }
}

// Load the 16-register B operand of variant v for this lane.
__device__ __forceinline__ void load_b(const QOperand* q, uint32_t b[4][4]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    uint4 w = *reinterpret_cast<const uint4*>(&q->bimg[kc][lane][0]);
    b[kc][0] = w.x; b[kc][1] = w.y; b[kc][2] = w.z; b[kc][3] = w.w;
  }
}

// ============================================================ coarse
// Wave tile: 16 centroids x 4 heads.  lower/upper = bf16(value -/+ margin),
// value = RNE(sum q (2u - 3) ) * scale/4, margin = ||q|| lambda bf16(resid).
__global__ __launch_bounds__(256) void k_coarse(StepArgs a) {
  const int g = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int tile = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nc = a.nc;
  if (tile * 16 >= nc) return;
  const QOperand* q = &a.qop[g * QV_COUNT + QV_RAW];
  uint32_t b[4][4];
  load_b(q, b);
  const int row = lane & 15, kb = lane >> 4;
  const int c_in = tile * 16 + row;
  uint4 w = make_uint4(0, 0, 0, 0);
  if (c_in < nc)
    w = *reinterpret_cast<const uint4*>(a.cen_up + ((size_t)g * nc + c_in) * 64 + kb * 16);
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
  v4i acc = {0, 0, 0, 0};
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    uint32_t av[4];
    expand2(words[kc], av);
    acc = mfma_i8(av, b[kc], acc);
  }
  int64_t dot[4];
  combine_limbs(acc, dot);
  if ((lane & 3) == 0) {
    const int h = (lane & 15) >> 2;
    const int64_t S = q->sum[h];
    const int fx = q->fx[h];
    const float norm = q->norm[h];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = tile * 16 + 4 * kb + r;
      if (c >= nc) continue;
      const int64_t Dv = 2 * dot[r] - 3 * S;
      const float val = scaled_f32(Dv, fx);
      const float value = __fmul_rn(val, a.scale4[(size_t)g * (nc / 32) + c / 32]);
      const float margin = __fmul_rn(norm, a.resid[(size_t)g * nc + c]);
      const size_t o = ((size_t)g * H + h) * nc + c;
      a.lower[o] = (uint16_t)bf16_rne(__fsub_rn(value, margin));
      a.upper[o] = (uint16_t)bf16_rne(__fadd_rn(value, margin));
    }
  }
}

// ============================================================ selection helpers
// Find, over values val(i) in [0, 2^bits) (given by functor), the digit path
// of the k-th largest value counting multiplicities.  Items with
// valid(i) == false are ignored.  Radix 8 per pass.  Returns the k-th largest
// value and (in *above) how many valid items are strictly greater.
template <int BITS, typename ValFn>
__device__ uint64_t block_kth(int n, int k, ValFn val, uint32_t* hist, int* scratch,
                              int* above_out) {
  uint64_t prefix = 0;
  int remaining = k, above = 0;
  for (int shift = BITS - 8; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    const int hs = shift + 8;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      uint64_t v;
      if (!val(i, &v)) continue;
      if (hs < BITS && (v >> hs) != (prefix >> hs)) continue;
      atomicAdd(&hist[(v >> shift) & 255], 1u);
    }
    __syncthreads();
    // Thread 0..255: suffix counts over bins; locate the digit.
    if (threadIdx.x < 64) {
      // each of 64 lanes owns 4 bins (lane 0: 252..255 high end)
      const int lane = threadIdx.x;
      const int base = 255 - 4 * lane;  // bins base, base-1, base-2, base-3
      int c4 = hist[base] + hist[base - 1] + hist[base - 2] + hist[base - 3];
      int inc = wave_incl_scan(c4);
      int exc = inc - c4;
      // the lane whose range contains the remaining-th item
      if (exc < remaining && remaining <= inc) {
        int acc = exc;
        int digit = base;
        for (int j = 0; j < 4; ++j) {
          int cnt = hist[base - j];
          if (acc + cnt >= remaining) { digit = base - j; break; }
          acc += cnt;
        }
        scratch[0] = digit;
        scratch[1] = acc;  // count strictly above the digit, within prefix
      }
      if (lane == 63 && inc < remaining) {  // fewer than k items: take all
        scratch[0] = -1;
        scratch[1] = inc;
      }
    }
    __syncthreads();
    const int digit = scratch[0];
    const int acc = scratch[1];
    __syncthreads();
    if (digit < 0) {  // n_valid < k within this prefix: no k-th element
      *above_out = above + acc;
      return 0;
    }
    above += acc;
    remaining -= acc;
    prefix |= (uint64_t)digit << shift;
  }
  *above_out = above;
  return prefix;
}

// ============================================================ thresholds
__global__ __launch_bounds__(1024) void k_thresh(StepArgs a) {
  const int g = blockIdx.x / H, h = blockIdx.x % H;
  __shared__ uint32_t hist[256];
  __shared__ int scratch[4];
  const uint16_t* lo = a.lower + ((size_t)g * H + h) * a.nc;
  int above;
  auto val = [&](int i, uint64_t* v) { *v = ordered16(lo[i]); return true; };
  uint64_t kth = block_kth<16>(a.nc, a.P[g], val, hist, scratch, &above);
  if (threadIdx.x == 0) a.thr[g * H + h] = (uint32_t)kth;
}

// ============================================================ survivors
// Survivor c iff some head h has ordered(upper_h(c)) >= threshold_h.  The
// list is ascending (each thread owns a contiguous centroid range).
__global__ __launch_bounds__(1024) void k_survivors(StepArgs a) {
  const int g = blockIdx.x, nc = a.nc;
  __shared__ int scratch[40];
  const int per = (nc + blockDim.x - 1) / blockDim.x;
  const int c0 = threadIdx.x * per, c1 = min(nc, c0 + per);
  uint32_t thr[H];
  for (int h = 0; h < H; ++h) thr[h] = a.thr[g * H + h];
  auto mask_of = [&](int c) {
    uint32_t m = 0;
    for (int h = 0; h < H; ++h)
      m |= (uint32_t)(ordered16(a.upper[((size_t)g * H + h) * nc + c]) >= thr[h]) << h;
    return m;
  };
  int cnt = 0;
  for (int c = c0; c < c1; ++c) {
    const uint32_t m = mask_of(c);
    a.masks[(size_t)g * nc + c] = (uint8_t)m;
    cnt += m != 0;
  }
  int total;
  int pos = block_excl_scan(cnt, scratch, &total);
  for (int c = c0; c < c1; ++c)
    if (a.masks[(size_t)g * nc + c]) a.surv[(size_t)g * nc + pos++] = c;
  if (threadIdx.x == 0) a.status[g * 8 + ST_SURV] = total;
}

// ============================================================ fine
// 4-bit centroid score of survivors: bf16(RNE(sum q (2 code4 - 15)) * gfs).
// fine_ord[g][h][i] = ordered score if survivor i is eligible for head h, else 0.
__global__ __launch_bounds__(256) void k_fine(StepArgs a) {
  const int g = blockIdx.y, nc = a.nc;
  const int lane = threadIdx.x & 63;
  const int n = a.status[g * 8 + ST_SURV];
  const QOperand* q = &a.qop[g * QV_COUNT + QV_RAW];
  uint32_t b[4][4];
  bool loaded = false;
  for (int tile = blockIdx.x * 4 + (threadIdx.x >> 6); tile * 16 < n; tile += gridDim.x * 4) {
    if (!loaded) { load_b(q, b); loaded = true; }
    const int row = lane & 15, kb = lane >> 4;
    const int i_in = tile * 16 + row;
    uint4 wu = make_uint4(0, 0, 0, 0), wl = wu;
    if (i_in < n) {
      const int c = a.surv[(size_t)g * nc + i_in];
      wu = *reinterpret_cast<const uint4*>(a.cen_up + ((size_t)g * nc + c) * 64 + kb * 16);
      wl = *reinterpret_cast<const uint4*>(a.cen_lo + ((size_t)g * nc + c) * 64 + kb * 16);
    }
    const uint32_t up[4] = {wu.x, wu.y, wu.z, wu.w};
    const uint32_t lo[4] = {wl.x, wl.y, wl.z, wl.w};
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      uint32_t eu[4], el[4], av[4];
      expand2(up[kc], eu);
      expand2(lo[kc], el);
#pragma unroll
      for (int m = 0; m < 4; ++m) av[m] = (eu[m] << 2) | el[m];
      acc = mfma_i8(av, b[kc], acc);
    }
    int64_t dot[4];
    combine_limbs(acc, dot);
    if ((lane & 3) == 0) {
      const int h = (lane & 15) >> 2;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = tile * 16 + 4 * kb + r;
        if (i >= n) continue;
        const int c = a.surv[(size_t)g * nc + i];
        const int64_t Dv = 2 * dot[r] - 15 * q->sum[h];
        const float val = scaled_f32(Dv, q->fx[h]);
        const uint32_t bits = bf16_rne(__fmul_rn(val, a.gfs[(size_t)g * (nc / 32) + c / 32]));
        const bool ok = (a.masks[(size_t)g * nc + c] >> h) & 1;
        a.fine_ord[((size_t)g * H + h) * nc + i] = ok ? (uint16_t)ordered16(bits) : 0;
        if (a.debug) a.fine_bits[((size_t)g * H + h) * nc + c] = ok ? (uint16_t)bits : 0xffff;
      }
    }
  }
}

// ============================================================ select + pool
// Per group: each head's top-P eligible survivors by (score desc, id asc);
// selected = union, ascending; pool = postings of selected clusters in
// order, keeping a token iff its mate cluster is larger or unselected.
__global__ __launch_bounds__(1024) void k_select_pool(StepArgs a) {
  const int g = blockIdx.x, nc = a.nc;
  extern __shared__ uint32_t dyn[];
  uint32_t* selbits = dyn;                 // nc / 32 words
  __shared__ uint32_t hist[256];
  __shared__ int scratch[40];
  __shared__ uint64_t kth[H];
  const int n = a.status[g * 8 + ST_SURV];
  const int* surv = a.surv + (size_t)g * nc;
  for (int h = 0; h < H; ++h) {
    const uint16_t* f = a.fine_ord + ((size_t)g * H + h) * nc;
    auto val = [&](int i, uint64_t* v) {
      const uint32_t o = f[i];
      *v = ((uint64_t)o << 16) | (0xffffu - (uint32_t)surv[i]);
      return o != 0;
    };
    int above;
    uint64_t k = block_kth<32>(n, a.P[g], val, hist, scratch, &above);
    if (threadIdx.x == 0) kth[h] = k;
    __syncthreads();
  }
  for (int w = threadIdx.x; w < nc / 32; w += blockDim.x) selbits[w] = 0;
  __syncthreads();
  // Selected survivors; survivors are ascending so the list is ascending.
  const int per = (n + blockDim.x - 1) / blockDim.x;
  const int i0 = threadIdx.x * per, i1 = min(n, i0 + per);
  auto selected = [&](int i) {
    const uint32_t c = surv[i];
    bool s = false;
    for (int h = 0; h < H; ++h) {
      const uint32_t o = a.fine_ord[((size_t)g * H + h) * nc + i];
      const uint64_t key = ((uint64_t)o << 16) | (0xffffu - c);
      s |= o != 0 && key >= kth[h];
    }
    return s;
  };
  int cnt = 0;
  for (int i = i0; i < i1; ++i) cnt += selected(i);
  int total;
  int pos = block_excl_scan(cnt, scratch, &total);
  int* sel = a.sel + (size_t)g * nc;
  for (int i = i0; i < i1; ++i)
    if (selected(i)) {
      const int c = surv[i];
      sel[pos++] = c;
      atomicOr(&selbits[c >> 5], 1u << (c & 31));
    }
  __syncthreads();
  const int nsel = total;
  // Pool emission: owned postings of selected clusters, encounter order.
  const int* off = a.csr_off + (size_t)g * (nc + 1);
  const int* tok = a.post_tok + (size_t)g * a.np_max;
  const int* mate = a.post_mate + (size_t)g * a.np_max;
  const int per_c = (nsel + blockDim.x - 1) / blockDim.x;
  const int s0 = threadIdx.x * per_c, s1 = min(nsel, s0 + per_c);
  auto owned = [&](int j, uint32_t c) {
    const uint32_t m = (uint32_t)mate[j];
    return m > c || !((selbits[m >> 5] >> (m & 31)) & 1u);
  };
  int own = 0, scanned = 0;
  for (int s = s0; s < s1; ++s) {
    const uint32_t c = sel[s];
    for (int j = off[c]; j < off[c + 1]; ++j) own += owned(j, c);
    scanned += off[c + 1] - off[c];
  }
  int pool_n;
  int p = block_excl_scan(own, scratch, &pool_n);
  int scanned_total;
  block_excl_scan(scanned, scratch, &scanned_total);
  int* ptok = a.pool_tok + (size_t)g * a.cap;
  int* ppost = a.pool_post + (size_t)g * a.cap;
  const int limit = min(pool_n, a.cap);
  for (int s = s0; s < s1; ++s) {
    const uint32_t c = sel[s];
    for (int j = off[c]; j < off[c + 1]; ++j)
      if (owned(j, c)) {
        if (p < limit) { ptok[p] = tok[j]; ppost[p] = j; }
        ++p;
      }
  }
  if (threadIdx.x == 0) {
    int err = 0;
    if (a.pool_capacity > 0 && pool_n > a.pool_capacity) err = 4;
    else if (pool_n < a.pool_min) err = 5;
    a.status[g * 8 + ST_POOL] = limit;
    a.status[g * 8 + ST_ERR] = err;
    a.status[g * 8 + ST_SEL] = nsel;
    a.status[g * 8 + ST_SCANNED] = scanned_total;
  }
}

// ============================================================ key scores
// 2-bit pool scores: bf16(16 * RNE(sum q15 (2 p2 - 3))), p2 from the
// posting's cluster-block prefix row.
__global__ __launch_bounds__(256) void k_score2(StepArgs a) {
  const int g = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int n = a.status[g * 8 + ST_POOL];
  const QOperand* q = &a.qop[g * QV_COUNT + QV_Q15];
  uint32_t b[4][4];
  bool loaded = false;
  const int row = lane & 15, kb = lane >> 4;
  for (int tile = blockIdx.x * 4 + (threadIdx.x >> 6); tile * 16 < n; tile += gridDim.x * 4) {
    if (!loaded) { load_b(q, b); loaded = true; }
    const int i_in = tile * 16 + row;
    uint4 w = make_uint4(0, 0, 0, 0);
    if (i_in < n) {
      const int j = a.pool_post[(size_t)g * a.cap + i_in];
      w = *reinterpret_cast<const uint4*>(a.post_p2 + ((size_t)g * a.np_max + j) * 64 + kb * 16);
    }
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      uint32_t av[4];
      expand2(words[kc], av);
      acc = mfma_i8(av, b[kc], acc);
    }
    int64_t dot[4];
    combine_limbs(acc, dot);
    if ((lane & 3) == 0) {
      const int h = (lane & 15) >> 2;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = tile * 16 + 4 * kb + r;
        if (i >= n) continue;
        const int64_t Dv = 2 * dot[r] - 3 * q->sum[h];
        a.s2[((size_t)g * H + h) * a.cap + i] =
            (uint16_t)ordered16(bf16_rne(scaled_f32(Dv, q->fx[h] + 4)));
      }
    }
  }
}

// Code4 (p2 << 2 | r2) A operand words of key token t for chunk kc.
__device__ __forceinline__ void load_code4(const uint8_t* rec, int kb, uint32_t out[4][4]) {
  const uint4 p = *reinterpret_cast<const uint4*>(rec + kb * 16);
  const uint4 r = *reinterpret_cast<const uint4*>(rec + 64 + kb * 16);
  const uint32_t pw[4] = {p.x, p.y, p.z, p.w}, rw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    uint32_t ep[4], er[4];
    expand2(pw[kc], ep);
    expand2(rw[kc], er);
#pragma unroll
    for (int m = 0; m < 4; ++m) out[kc][m] = (ep[m] << 2) | er[m];
  }
}

// 4-bit U1 scores: bf16(16 * RNE(sum qs (2 code4 - 15))).
__global__ __launch_bounds__(256) void k_score4(StepArgs a) {
  const int g = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int n = a.status[g * 8 + ST_U1];
  const QOperand* q = &a.qop[g * QV_COUNT + QV_QS];
  const int row = lane & 15, kb = lane >> 4;
  uint32_t b[4][4];
  bool loaded = false;
  for (int tile = blockIdx.x * 4 + (threadIdx.x >> 6); tile * 16 < n; tile += gridDim.x * 4) {
    if (!loaded) { load_b(q, b); loaded = true; }
    const int i_in = tile * 16 + row;
    uint32_t av[4][4] = {};
    if (i_in < n) {
      const int t = a.u1_tok[(size_t)g * U1_MAX + i_in];
      load_code4(a.keyrec + ((size_t)g * a.T + t) * 256, kb, av);
    }
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) acc = mfma_i8(av[kc], b[kc], acc);
    int64_t dot[4];
    combine_limbs(acc, dot);
    if ((lane & 3) == 0) {
      const int h = (lane & 15) >> 2;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = tile * 16 + 4 * kb + r;
        if (i >= n) continue;
        const int64_t Dv = 2 * dot[r] - 15 * q->sum[h];
        a.s4[((size_t)g * H + h) * U1_MAX + i] =
            (uint16_t)ordered16(bf16_rne(scaled_f32(Dv, q->fx[h] + 4)));
      }
    }
  }
}

// 8-bit U2 scores: bf16(RNE(sum qs (2 code8 - 255))), code8 = 16 code4 + r4.
__global__ __launch_bounds__(256) void k_score8(StepArgs a) {
  const int g = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int n = a.status[g * 8 + ST_U2];
  const QOperand* q = &a.qop[g * QV_COUNT + QV_QS];
  const int row = lane & 15, kb = lane >> 4;
  uint32_t b[4][4];
  bool loaded = false;
  for (int tile = blockIdx.x * 4 + (threadIdx.x >> 6); tile * 16 < n; tile += gridDim.x * 4) {
    if (!loaded) { load_b(q, b); loaded = true; }
    const int i_in = tile * 16 + row;
    uint32_t hi[4][4] = {}, lo[4][4] = {};
    if (i_in < n) {
      const int t = a.u2_tok[(size_t)g * U2_MAX + i_in];
      const uint8_t* rec = a.keyrec + ((size_t)g * a.T + t) * 256;
      load_code4(rec, kb, hi);
      const uint4 r0 = *reinterpret_cast<const uint4*>(rec + 128 + kb * 32);
      const uint4 r1 = *reinterpret_cast<const uint4*>(rec + 128 + kb * 32 + 16);
      const uint32_t rw[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        expand4(rw[2 * kc], &lo[kc][0]);
        expand4(rw[2 * kc + 1], &lo[kc][2]);
      }
    }
    v4i acc_hi = {0, 0, 0, 0}, acc_lo = {0, 0, 0, 0};
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      acc_hi = mfma_i8(hi[kc], b[kc], acc_hi);
      acc_lo = mfma_i8(lo[kc], b[kc], acc_lo);
    }
    int64_t dh[4], dl[4];
    combine_limbs(acc_hi, dh);
    combine_limbs(acc_lo, dl);
    if ((lane & 3) == 0) {
      const int h = (lane & 15) >> 2;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = tile * 16 + 4 * kb + r;
        if (i >= n) continue;
        const int64_t Dv = 2 * (16 * dh[r] + dl[r]) - 255 * q->sum[h];
        a.s8[((size_t)g * H + h) * U2_MAX + i] =
            (uint16_t)ordered16(bf16_rne(scaled_f32(Dv, q->fx[h])));
      }
    }
  }
}

// ============================================================ token top-k
// Per (group, head): members = top-k by (ordered score desc, token asc) of
// n items; writes a membership bitmap (one bit per item).
__global__ __launch_bounds__(1024) void k_topk_members(TopkArgs t) {
  const int g = blockIdx.x / H, h = blockIdx.x % H;
  __shared__ uint32_t hist[256];
  __shared__ int scratch[40];
  const int n = *t.count_ptr(g);
  const uint16_t* s = t.scores + ((size_t)g * H + h) * t.stride;
  const int* tok = t.tokens + (size_t)g * t.stride;
  auto val = [&](int i, uint64_t* v) {
    *v = ((uint64_t)s[i] << 20) | (0xfffffu - (uint32_t)tok[i]);
    return true;
  };
  int above;
  const uint64_t kth = block_kth<40>(n, t.k, val, hist, scratch, &above);
  const bool take_all = n <= t.k;
  uint64_t* bm = t.bitmap + ((size_t)g * H + h) * t.words;
  const uint32_t kord = (uint32_t)(kth >> 20);
  for (int base = threadIdx.x & ~63; base < t.words * 64; base += blockDim.x) {
    const int i = base + (threadIdx.x & 63);
    bool m = false;
    if (i < n) {
      const uint32_t o = s[i];
      m = take_all || o > kord ||
          (o == kord && (((uint64_t)o << 20) | (0xfffffu - (uint32_t)tok[i])) >= kth);
    }
    const uint64_t ball = __ballot(m);
    if ((threadIdx.x & 63) == 0) bm[base >> 6] = ball;
  }
}

// Union of the four heads' members in item order -> compact token list.
__global__ __launch_bounds__(1024) void k_union(UnionArgs u) {
  const int g = blockIdx.x;
  __shared__ int scratch[40];
  const int n = *u.count_in(g);
  const int words = (n + 63) / 64;
  const uint64_t* bm = u.bitmap + (size_t)g * H * u.words;
  const int per = (words + blockDim.x - 1) / blockDim.x;
  const int w0 = threadIdx.x * per, w1 = min(words, w0 + per);
  int cnt = 0;
  for (int w = w0; w < w1; ++w)
    cnt += __popcll(bm[w] | bm[u.words + w] | bm[2 * u.words + w] | bm[3 * u.words + w]);
  int total;
  int pos = block_excl_scan(cnt, scratch, &total);
  const int* in = u.tokens_in + (size_t)g * u.stride_in;
  int* out = u.tokens_out + (size_t)g * u.stride_out;
  for (int w = w0; w < w1; ++w) {
    uint64_t m = bm[w] | bm[u.words + w] | bm[2 * u.words + w] | bm[3 * u.words + w];
    while (m) {
      const int bit = __ffsll((unsigned long long)m) - 1;
      m &= m - 1;
      if (pos < u.stride_out) out[pos] = in[w * 64 + bit];
      ++pos;
    }
  }
  if (threadIdx.x == 0) *u.count_out(g) = min(total, u.stride_out);
}

// ============================================================ final top-100
// Per (group, head): sort the U2 items by key (bitonic, 1024 slots) and keep
// the best 100 token IDs in order.
__global__ __launch_bounds__(256) void k_top100(StepArgs a) {
  const int g = blockIdx.x / H, h = blockIdx.x % H;
  __shared__ uint64_t keys[U2_MAX];
  const int n = a.status[g * 8 + ST_U2];
  const uint16_t* s = a.s8 + ((size_t)g * H + h) * U2_MAX;
  const int* tok = a.u2_tok + (size_t)g * U2_MAX;
  for (int i = threadIdx.x; i < U2_MAX; i += blockDim.x)
    keys[i] = i < n ? (((uint64_t)s[i] << 20) | (0xfffffu - (uint32_t)tok[i])) : 0;
  __syncthreads();
  for (int size = 2; size <= U2_MAX; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < U2_MAX; i += blockDim.x) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;  // overall descending
          const uint64_t x = keys[i], y = keys[j];
          if ((x < y) == desc) { keys[i] = y; keys[j] = x; }
        }
      }
      __syncthreads();
    }
  }
  for (int r = threadIdx.x; r < TOPK; r += blockDim.x) {
    const uint64_t k = keys[r];
    a.top[(g * H + h) * TOPK + r] = (r < n) ? (int)(0xfffffu - (uint32_t)(k & 0xfffffu)) : -1;
  }
}

// ============================================================ sparse SDPA
// One block per query head; 4 waves split the S + L + 100 keys; lane l owns
// dims 4l..4l+3.  Online softmax in FP32, scale 1/16, FP8 e4m3 records.
__device__ __forceinline__ void fp8x4_to_f32(uint32_t w, float f[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) f[i] = fp8_e4m3_to_f32((w >> (8 * i)) & 0xffu);
}

__global__ __launch_bounds__(256) void k_sdpa(StepArgs a) {
  const int j = blockIdx.x, g = j / H, h = j % H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __shared__ float s_m[4], s_l[4];
  __shared__ float s_o[4][D];
  float q[4];
  {
    const uint2 qw = *reinterpret_cast<const uint2*>(a.q + j * D + 4 * lane);
    q[0] = bf16_f32(qw.x & 0xffff); q[1] = bf16_f32(qw.x >> 16);
    q[2] = bf16_f32(qw.y & 0xffff); q[3] = bf16_f32(qw.y >> 16);
  }
  const int S = a.sink, L = a.local, total = S + L + TOPK;
  float m = -INFINITY, l = 0.f, o[4] = {0.f, 0.f, 0.f, 0.f};
  const uint8_t* kv = a.kv8 + (size_t)g * a.T * 512;
  for (int i = wave; i < total; i += 4) {
    int t;
    if (i < S) t = i;
    else if (i < S + L) t = a.T - L + (i - S);
    else t = a.top[(g * H + h) * TOPK + (i - S - L)];
    if (t < 0) continue;
    const uint8_t* rec = kv + (size_t)t * 512;
    const uint32_t kw = *reinterpret_cast<const uint32_t*>(rec + 256 + 4 * lane);
    const uint32_t vw = *reinterpret_cast<const uint32_t*>(rec + 4 * lane);
    float kf[4], vf[4];
    fp8x4_to_f32(kw, kf);
    fp8x4_to_f32(vw, vf);
    float part = q[0] * kf[0] + q[1] * kf[1] + q[2] * kf[2] + q[3] * kf[3];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off, WAVE);
    const float logit = part * 0.0625f;
    const float mn = fmaxf(m, logit);
    const float scale = __expf(m - mn);
    const float p = __expf(logit - mn);
    l = l * scale + p;
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = o[d] * scale + p * vf[d];
    m = mn;
  }
  if (lane == 0) { s_m[wave] = m; s_l[wave] = l; }
#pragma unroll
  for (int d = 0; d < 4; ++d) s_o[wave][4 * lane + d] = o[d];
  __syncthreads();
  // combine the 4 waves: thread t owns dim t
  const int d = threadIdx.x;
  float M = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
  float lsum = 0.f, acc = 0.f;
  for (int w = 0; w < 4; ++w) {
    if (s_m[w] == -INFINITY) continue;
    const float sc = __expf(s_m[w] - M);
    lsum += s_l[w] * sc;
    acc += s_o[w][d] * sc;
  }
  a.out[j * D + d] = (uint16_t)bf16_rne(acc / lsum);
}

// ============================================================ launcher
void launch_step(const StepArgs& a, const StepWork& w, hipStream_t st) {
  const int groups_tiles = (a.nc + 63) / 64;
  hipLaunchKernelGGL(k_qprep, dim3(G), dim3(1024), 0, st, a);
  hipLaunchKernelGGL(k_coarse, dim3(groups_tiles, G), dim3(256), 0, st, a);
  hipLaunchKernelGGL(k_thresh, dim3(G * H), dim3(1024), 0, st, a);
  hipLaunchKernelGGL(k_survivors, dim3(G), dim3(1024), 0, st, a);
  hipLaunchKernelGGL(k_fine, dim3(min(groups_tiles, 256), G), dim3(256), 0, st, a);
  hipLaunchKernelGGL(k_select_pool, dim3(G), dim3(1024), (size_t)(a.nc / 32) * 4, st, a);
  hipLaunchKernelGGL(k_score2, dim3(w.score_blocks, G), dim3(256), 0, st, a);
  hipLaunchKernelGGL(k_topk_members, dim3(G * H), dim3(1024), 0, st, w.top_u1);
  hipLaunchKernelGGL(k_union, dim3(G), dim3(1024), 0, st, w.union_u1);
  hipLaunchKernelGGL(k_score4, dim3(U1_MAX / 64, G), dim3(256), 0, st, a);
  hipLaunchKernelGGL(k_topk_members, dim3(G * H), dim3(1024), 0, st, w.top_u2);
  hipLaunchKernelGGL(k_union, dim3(G), dim3(1024), 0, st, w.union_u2);
  hipLaunchKernelGGL(k_score8, dim3(U2_MAX / 64, G), dim3(256), 0, st, a);
  hipLaunchKernelGGL(k_top100, dim3(G * H), dim3(256), 0, st, a);
  hipLaunchKernelGGL(k_sdpa, dim3(G * H), dim3(256), 0, st, a);
}

}  // namespace skv
