// SeoulKV4 sparse decode step for MI355X (gfx950).
//
// One decode step, per KV group g (4 query heads each):
//   front       query operands (q, q15 = bf16(q s / 64), qs = bf16(q s / 256)
//               -> fixed-point int8 limb images, ||q|| lambda), then for every
//               centroid the 2-bit interval [lower, upper] and the 4-bit fine
//               score of each head
//   select      per head: the P-th largest lower bound, then the top-P fine
//               scores among centroids whose upper bound reaches it ->
//               selected bitmap (union); extra blocks: sink/local attention
//               and the q15 / qs operands
//   pool        survivor masks; postings owned under the spill-2 mate rule;
//               selected list + pool tokens in encounter order (one pass,
//               decoupled look-back over the centroid ranges) and the 2-bit
//               scores of the pool keys
//   top1600     per head: top-1600 of the pool -> membership bitmap
//   union_score U1 = union over heads in pool order + 4-bit and 8-bit scores
//               of U1
//   top256      per head: top-256 of U1 -> membership bitmap
//   top100      per head: best-first top-100 token IDs of U2 (the union of
//               the heads' top-256, read as a mask over U1) by 8-bit score,
//               then FP8 attention over them merged with the sink/local
//               attention slices
// Reference stages: see the table in skv_step.h.
//
// Selection keys are (ordered BF16 score, lowest ID first); all score dots
// are exact integers on the int8 matrix cores (see skv_device.h).

#include <algorithm>

#include "skv_device.h"
#include "skv_fastsel.h"
#include "skv_octsel.h"
#include "skv_select.h"
#include "skv_step.h"

namespace skv {

#ifdef SKV_TRACE  // the tables of skv_trace.h
__device__ unsigned long long g_skv_trace[32][16];
__device__ unsigned long long g_skv_trace_blk[12][4096][4];
#endif

// ============================================================ query prep
// Fixed-point operand of query variant v for KV group g, computed by the
// first 4 waves of a block (wave h forms head h; lane l owns dims 4l ..
// 4l+3): the integers X, their sum, the scale exponent, ||q|| lambda (raw
// variant) and the int8 limb B image, written to *out (LDS or global
// memory).  Sum of squares: X^2 < 2^44 is split into 22-bit halves so that
// both wave sums stay below 2^30 (exact in int32).
__device__ void prep_head(const StepArgs& a, int g, int v, QOperand* out, int h, int lane,
                          uint2 qw, bool own);

// This lane's 4 BF16 query elements of head h of group g (dims 4 lane ..).
__device__ __forceinline__ uint2 load_qw(const StepArgs& a, int g, int h, int lane) {
  return *reinterpret_cast<const uint2*>(a.q + (g * H + h) * D + 4 * lane);
}

// Waves 0..3 form one head each from qw, their lanes' query words; the
// operand is complete after the barrier.  Later waves repeat head H - 1 and
// write nothing: every thread uses its query word, so the compiler keeps
// the caller's query load where the caller issued it (first).
__device__ void prep_operand(const StepArgs& a, int g, int v, QOperand* out, uint2 qw) {
  const int lane = threadIdx.x & 63, h = threadIdx.x >> 6;
  prep_head(a, g, v, out, min(h, H - 1), lane, qw, h < H);
  __syncthreads();
}

// One wave per head: the integers X, their sum, the scale exponent and
// ||q|| lambda (raw variant) of query head 4g + h.
__device__ void prep_head(const StepArgs& a, int g, int v, QOperand* out, int h, int lane,
                          uint2 qw, bool own) {
  const uint32_t qb[4] = {qw.x & 0xffffu, qw.x >> 16, qw.y & 0xffffu, qw.y >> 16};
  uint32_t bits[4];
  if (v != QV_RAW) {
    const float4 ks = *reinterpret_cast<const float4*>(a.kscale + g * D + 4 * lane);
    const float kv[4] = {ks.x, ks.y, ks.z, ks.w};
    const float mul = v == QV_Q15 ? 0.015625f : 0.00390625f;
#pragma unroll
    for (int i = 0; i < 4; ++i) bits[i] = bf16_rne(__fmul_rn(__fmul_rn(bf16_f32(qb[i]), kv[i]), mul));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) bits[i] = qb[i];
  }
  int sig[4], ex[4], emax = -(1 << 20);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int expf = (bits[i] >> 7) & 0xff, mant = bits[i] & 0x7f;
    sig[i] = expf ? (mant | 0x80) : mant;
    ex[i] = expf ? expf - 134 : -133;
    if (sig[i]) emax = max(emax, ex[i]);
  }
  int exmax = wave_max(emax);
  if (exmax == -(1 << 20)) exmax = 0;
  int X[4], sx = 0, sq_lo = 0, sq_hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int shift = ex[i] - exmax + FX_HEADROOM;
    const int mag = shift >= 0 ? (sig[i] << shift) : (shift <= -9 ? 0 : (sig[i] >> -shift));
    X[i] = (bits[i] & 0x8000u) ? -mag : mag;
    sx += X[i];
    const uint64_t x2 = (uint64_t)((int64_t)X[i] * X[i]);
    sq_lo += (int)(x2 & 0x3fffffu);
    sq_hi += (int)(x2 >> 22);
  }
  if (own) *reinterpret_cast<int4*>(&out->X[h][4 * lane]) = make_int4(X[0], X[1], X[2], X[3]);
  // B image: word (kc, lane l, m) holds bytes limb (col % 4) of X_{col/4}[dim]
  // for col = l % 16, dim = (l / 16) * 64 + kc * 16 + 4 byte + m (a lane's
  // 16-dim chunk transposed 4 x 4, to match the A words of expand2t and
  // expand4t: the MFMA pairs A and B bytes by position, so one permutation
  // of both keeps every dot).  This lane's dims 4 lane + i are byte
  // lane % 4 of words (kc = lane / 4 % 4, l = lane / 16 * 16 + 4h + limb,
  // m = i); X = l0 + 2^8 l1 + 2^16 l2 in signed bytes (|X| < 2^22), limb 3 = 0.
  if (own) {
    uint8_t* img = reinterpret_cast<uint8_t*>(&out->bimg[(lane >> 2) & 3][(lane >> 4) * 16 + 4 * h][0]) +
                   (lane & 3);
  #pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int l0 = (int)(int8_t)(X[i] & 0xff);
      const int x1 = (X[i] - l0) >> 8;
      const int l1 = (int)(int8_t)(x1 & 0xff);
      const int l2 = (x1 - l1) >> 8;
      img[0 * 16 + 4 * i] = (uint8_t)l0;  // word (kc, l + limb, m = i): 16 bytes per l
      img[1 * 16 + 4 * i] = (uint8_t)l1;
      img[2 * 16 + 4 * i] = (uint8_t)l2;
      img[3 * 16 + 4 * i] = 0;
    }
  }
  sx = wave_sum(sx);
  sq_lo = wave_sum(sq_lo);
  sq_hi = wave_sum(sq_hi);
  if (own && lane == 0) {
    out->fx[h] = exmax - FX_HEADROOM;
    out->sum[h] = sx;
    if (v == QV_RAW) {
      const unsigned long long N = ((unsigned long long)sq_hi << 22) + (unsigned long long)sq_lo;
      out->norm[h] = __fmul_rn(sqrt_rne_scaled(N, exmax - FX_HEADROOM), a.lam[g]);
    } else {
      out->norm[h] = 0.f;
    }
  }
}

// Load the 16-register B operand of a query variant for this lane.
__device__ __forceinline__ void load_b(const QOperand* q, uint32_t b[4][4]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    const uint4 w = *reinterpret_cast<const uint4*>(&q->bimg[kc][lane][0]);
    b[kc][0] = w.x; b[kc][1] = w.y; b[kc][2] = w.z; b[kc][3] = w.w;
  }
}

// ============================================================ sparse SDPA
// Attention of query head j = 4g + h over its KV group's FP8 [V || K] records
// for the keys [sink | local | top-100] (softmax over all of them, scale 1/16).
// The sink/local part depends only on Q: extra blocks of the k_select launch
// compute it as 128-key slices (partial max, sum, unnormalised output), and
// k_top100 attends the head's 100 selected keys and merges everything.
constexpr int SDPA_WAVE_KEYS = 16;
constexpr int DENSE_BLOCK_KEYS = (SEL_BLOCK / WAVE) * SDPA_WAVE_KEYS;
static_assert(U2_MAX <= OCT_ITEMS && U1_MAX <= OCT_ITEMS, "unions fit the register selection");
static_assert(DENSE_BLOCK_KEYS == DENSE_SLICE_KEYS && SEL_BLOCK / WAVE == ATTN_WAVES,
              "attention slices follow the selection block size");

__device__ __forceinline__ void load_q4(const StepArgs& a, int j, float q[4]) {
  const int lane = threadIdx.x & 63;
  const uint2 qw = *reinterpret_cast<const uint2*>(a.q + j * D + 4 * lane);
  q[0] = bf16_f32(qw.x & 0xffff); q[1] = bf16_f32(qw.x >> 16);
  q[2] = bf16_f32(qw.y & 0xffff); q[3] = bf16_f32(qw.y >> 16);
}

// One wave over up to KPW keys: lane b < KPW holds the token of key b in tk
// (-1: none); lane l owns dims 4l..4l+3.  attend_load issues every record
// load; attend_math (after any independent work) returns the wave's max
// logit m, softmax sum l and unnormalised output o.
template <int KPW>
struct AttnLoads {
  int t[KPW];
  uint32_t kw[KPW], vw[KPW];
};

template <int KPW>
__device__ __forceinline__ AttnLoads<KPW> attend_load(const uint8_t* __restrict__ kv, int tk) {
  const int lane = threadIdx.x & 63;
  AttnLoads<KPW> L;
#pragma unroll
  for (int b = 0; b < KPW; ++b) {
    L.t[b] = __builtin_amdgcn_readlane(tk, b);
    const uint8_t* rec = kv + (size_t)max(L.t[b], 0) * 512;
    L.kw[b] = *reinterpret_cast<const uint32_t*>(rec + 256 + 4 * lane);
    L.vw[b] = *reinterpret_cast<const uint32_t*>(rec + 4 * lane);
  }
  return L;
}

template <int KPW>
__device__ __forceinline__ void attend_math(const AttnLoads<KPW>& L, const float q[4], float& m,
                                            float& l, float o[4]) {
  float logit[KPW];
#pragma unroll
  for (int b = 0; b < KPW; ++b) {
    float kf[4];
    fp8x4_to_f32(L.kw[b], kf);
    logit[b] = q[0] * kf[0] + q[1] * kf[1] + q[2] * kf[2] + q[3] * kf[3];
  }
#pragma unroll
  for (int b = 0; b < KPW; ++b) logit[b] = wave_sum_f(logit[b]);
  m = -INFINITY;
#pragma unroll
  for (int b = 0; b < KPW; ++b)
    if (L.t[b] >= 0) m = fmaxf(m, logit[b] * 0.0625f);
  l = 0.f;
  o[0] = o[1] = o[2] = o[3] = 0.f;
#pragma unroll
  for (int b = 0; b < KPW; ++b) {
    if (L.t[b] < 0) continue;
    const float p = __expf(logit[b] * 0.0625f - m);
    float vf[4];
    fp8x4_to_f32(L.vw[b], vf);
    l += p;
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] += p * vf[d];
  }
}

struct AttnScratch {
  float m[SEL_BLOCK / WAVE], l[SEL_BLOCK / WAVE];
  float o[SEL_BLOCK / WAVE][D];
};
static_assert(sizeof(AttnScratch) == ATTN_SCRATCH_BYTES, "attention scratch size");

// Publish a wave partial to LDS; after a barrier, merge_waves gives thread
// d < 256 the block's (max, sum, output[d]).
__device__ __forceinline__ void stash_wave(AttnScratch& s, float m, float l, const float o[4]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    s.m[wave] = m;
    s.l[wave] = l;
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) s.o[wave][4 * lane + d] = o[d];
}

__device__ __forceinline__ void merge_waves(const AttnScratch& s, int d, float& M, float& L,
                                            float& O) {
  constexpr int NW = SEL_BLOCK / WAVE;
  // every LDS read issued before the first use (no per-wave branch); a wave
  // without keys has m = -inf, l = o = 0 and weight exp(-inf) = 0
  float mw[NW], lw[NW], ow[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    mw[w] = s.m[w];
    lw[w] = s.l[w];
    ow[w] = s.o[w][d];
  }
  M = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w) M = fmaxf(M, mw[w]);
  L = 0.f;
  O = 0.f;
  if (M == -INFINITY) return;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float sc = __expf(mw[w] - M);
    L += lw[w] * sc;
    O += ow[w] * sc;
  }
}

// Record base and per-lane record index of token tk (-1: none) of group g:
// contiguous records index tokens from the group's first record, paged ones
// index the pool through the page table.
template <bool PAGED>
__device__ __forceinline__ const uint8_t* kv_base(const StepArgs& a, int g) {
  return PAGED ? a.kv8 : a.kv8 + (size_t)g * a.kv_rows * 512;
}
template <bool PAGED>
__device__ __forceinline__ int kv_lane_row(const StepArgs& a, int g, int tk) {
  if (!PAGED || tk < 0) return tk;
  return (int)kv_row_paged(a.kv_table, a.kv_shift, g, tk);
}

// Dense slice r of query head j: keys r*256 .. r*256+255 of [sink | local].
template <bool PAGED>
__device__ void dense_attend(const StepArgs& a, int blk, AttnScratch& s) {
  const int j = blk / a.dense_slices, r = blk % a.dense_slices, g = j / H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ndense = a.sink + a.local;
  float q[4];
  load_q4(a, j, q);
  int tk = -1;
  const int i = r * DENSE_BLOCK_KEYS + wave * SDPA_WAVE_KEYS + lane;
  if (lane < SDPA_WAVE_KEYS && i < ndense) tk = i < a.sink ? i : a.T - a.local + (i - a.sink);
  float m, l, o[4];
  // the slice's record gather (trace builds time it: issue, then arrival)
  const AttnLoads<SDPA_WAVE_KEYS> L =
      attend_load<SDPA_WAVE_KEYS>(kv_base<PAGED>(a, g), kv_lane_row<PAGED>(a, g, tk));
  SKV_TSB(5, 1);
  SKV_WAIT(L.kw[SDPA_WAVE_KEYS - 1] ^ L.vw[SDPA_WAVE_KEYS - 1]);
  SKV_TSW(5, 2);
  attend_math<SDPA_WAVE_KEYS>(L, q, m, l, o);
  stash_wave(s, m, l, o);
  __syncthreads();
  if (threadIdx.x < D) {
    float M, L, O;
    merge_waves(s, threadIdx.x, M, L, O);
    float* part = a.dense_part + ((size_t)j * a.dense_slices + r) * (D + 2);
    part[threadIdx.x] = O;
    if (threadIdx.x == 0) {
      part[D] = M;
      part[D + 1] = L;
    }
  }
}

// ============================================================ front
constexpr int FR_BLOCK = 512;   // front: one 16-centroid tile per wave
constexpr int FR_WAVES = FR_BLOCK / WAVE;
static_assert(FR_WAVES >= H, "front: wave w < H forms query head w");
static_assert(APPEND_FUSE * 512 <= FR_BLOCK * 16, "front block 0 packs a folded append");
constexpr int FR_CENTROIDS = 16 * FR_WAVES;
constexpr int FR_MAX_BLOCKS = 128;  // front blocks per group (each loops over its tiles)

// One wave tile = 16 centroids x 4 heads.  Every block first forms the raw
// query operand of its group in LDS (its centroid-plane loads are already in
// flight), then per centroid and head:
//   coarse  lower/upper = bf16(value -/+ margin), value = RNE(sum q (2u - 3))
//           * scale/4, margin = ||q|| lambda bf16(resid)  (ordered, all heads)
//   fine    bf16(RNE(sum q (2 code4 - 15)) * group_fine_scale)  (ordered;
//           eligibility is applied by the selection kernel)
// Block 0 of each group also publishes the raw operand and clears the
// group's per-step state (the q15 / qs operands of the later kernels are
// formed by extra blocks of the selection launch).
// Loads of one 16-centroid tile for one wave: the two planes (lane row
// l % 16, dims (l / 16) * 16 ..), the residual norm of the lane's output
// centroid l % 16 and the tile's 32-centroid block factors.
struct FrTile {
  uint4 wu, wl;
  float rs, sc4, gf;
};

// Per-lane conversion constants of the front (lane l converts head l / 16):
// value = (2 dq - 3 S) 2^fx, fine = (2 dq - 15 S) 2^fx.
struct FrConv {
  LimbScale ls;
  double cc, cf;
  float norm;
  __device__ FrConv(const QOperand& sq, int h)
      : ls(sq.fx[h], 1),
        cc(LimbScale::offset(-3 * sq.sum[h], sq.fx[h])),
        cf(LimbScale::offset(-15 * sq.sum[h], sq.fx[h])),
        norm(sq.norm[h]) {}
};

// Branch-free (a tile past the end reloads the last one, unused), so the
// compiler can wait for earlier loads while these are in flight.
__device__ __forceinline__ FrTile fr_load(const StepArgs& a, int g, int tile, int lane) {
  const int nc = a.nc, row = lane & 15, kb = lane >> 4;
  const int tt = min(tile, nc / 16 - 1);
  FrTile t;
  const size_t rowoff = ((size_t)g * nc + tt * 16 + row) * 64 + kb * 16;
  t.wu = *reinterpret_cast<const uint4*>(a.cen_up + rowoff);
  t.wl = *reinterpret_cast<const uint4*>(a.cen_lo + rowoff);
  t.rs = a.resid[(size_t)g * nc + tt * 16 + row];
  t.sc4 = a.scale4[(size_t)g * (nc / 32) + (tt >> 1)];
  t.gf = a.gfs[(size_t)g * (nc / 32) + (tt >> 1)];
  return t;
}

// Coarse bounds and fine scores of one tile's 16 centroids x 4 heads.  The
// query image is the matrix core's row operand (head x limb) and the tile's
// centroids its columns, so lane l holds the limb sums of centroid l % 16
// for head l / 16 and converts them itself.
__device__ __forceinline__ void fr_score(const StepArgs& a, int g, int tile, int lane, const FrTile& t,
                                         const uint32_t (&b)[4][4], const FrConv& cv) {
  const int nc = a.nc;
  const uint32_t up[4] = {t.wu.x, t.wu.y, t.wu.z, t.wu.w};
  const uint32_t lo[4] = {t.wl.x, t.wl.y, t.wl.z, t.wl.w};
  // the 4-bit code is 4 upper + lower, so its dot is 4 (upper dot) + (lower
  // dot), exact in each int32 limb (|sum| <= 256 * 128 * 15)
  v4i acc_c = {0, 0, 0, 0}, acc_l = {0, 0, 0, 0};
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    uint32_t eu[4], el[4];
    expand2t(up[kc], eu);
    expand2t(lo[kc], el);
    acc_c = mfma_i8(b[kc], eu, acc_c);
    acc_l = mfma_i8(b[kc], el, acc_l);
  }
  const v4i acc_f = acc_c * 4 + acc_l;
  const int h = lane >> 4, r = lane & 15;
  const float value = __fmul_rn(cv.ls(acc_c[0], acc_c[1], acc_c[2], cv.cc), t.sc4);
  const float margin = __fmul_rn(cv.norm, t.rs);
  const size_t o = ((size_t)g * H + h) * nc + tile * 16 + r;
  const uint32_t lo16 = ordered16(bf16_rne(__fsub_rn(value, margin)));
  a.lower[o] = (uint16_t)lo16;
  a.upper[o] = (uint16_t)ordered16(bf16_rne(__fadd_rn(value, margin)));
  const uint32_t fb = bf16_rne(__fmul_rn(cv.ls(acc_f[0], acc_f[1], acc_f[2], cv.cf), t.gf));
  const uint32_t fo = ordered16(fb);
  a.fine_ord[o] = (uint16_t)fo;
  if (a.debug) a.fine_bits[o] = (uint16_t)fb;
  // tile maxima: read by the one-octet select instance only (centroid
  // lists past the register instances, or the selection-path test modes)
  if (a.tmax_lo && (a.exact_select != 0 || a.nc > 4 * OCT_ITEMS)) {
    // 8-centroid tile maxima: within each quad, then the two quads of each
    // half row (half-row mirror); the fine-score maximum of the whole row
    uint32_t lmax = lo16, fmax = fo;
    lmax = max(lmax, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lmax, 0xB1, 0xf, 0xf, false));
    lmax = max(lmax, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lmax, 0x4E, 0xf, 0xf, false));
    lmax = max(lmax, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lmax, 0x141, 0xf, 0xf, false));
    if ((r & 7) == 0)
      a.tmax_lo[((size_t)g * H + h) * (nc / 8) + tile * 2 + (r >> 3)] = (uint16_t)lmax;
    fmax = max(fmax, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)fmax, 0xB1, 0xf, 0xf, false));
    fmax = max(fmax, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)fmax, 0x4E, 0xf, 0xf, false));
    fmax = max(fmax, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)fmax, 0x141, 0xf, 0xf, false));
    fmax = max(fmax, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)fmax, 0x128, 0xf, 0xf, false));
    if (r == 0) a.tmax_fi[((size_t)g * H + h) * (nc / 16) + tile] = (uint16_t)fmax;
  }
}

// Block (x, g) forms group g's fixed-point query operand once, then its
// waves score 16-centroid tiles x*FR_WAVES + wave and, when LOOP (more tiles
// than one pass of the grid covers), every FR_WAVES * gridDim.x tiles after
// it, with the next tile's loads in flight while one is scored.
// APPEND (the step folds a host append, a.app_n > 0): block 0 of each group
// also packs the appended tokens' FP8 records.
template <bool LOOP, bool APPEND>
__global__ __launch_bounds__(FR_BLOCK) void k_front(const uint16_t* __restrict__ q, StepArgs a) {
  SKV_TSB(4, 0);
  SKV_TS(0, 0);
  const int g = blockIdx.y, nc = a.nc;
  const int lane = threadIdx.x & 63;
  const int ntiles = nc / 16;
  const int step = FR_WAVES * (int)gridDim.x;
  int tile = blockIdx.x * FR_WAVES + (threadIdx.x >> 6);
  // the query first: forming its operand then waits for it alone while the
  // plane loads are still in flight (waves 0 .. H-1 form heads 0 .. H-1)
  const uint2 qw = *reinterpret_cast<const uint2*>(
      q + (g * H + min((int)(threadIdx.x >> 6), H - 1)) * D + 4 * lane);
  __builtin_amdgcn_sched_barrier(0);  // keep the query load ahead of the tile's
  FrTile cur = fr_load(a, g, tile, lane);
  // a folded host append: block 0 of the group packs 16 bytes of the new
  // tokens' records per thread (record byte 16 t: token t / 32, V for the
  // first 256 bytes, then K); the BF16 source is loaded now and converted
  // after the tiles are scored.  Every thread issues the two loads (from
  // the query when it packs nothing): a conditional load would make the
  // compiler wait for it where the branches join, here.
  const int app_i = (int)threadIdx.x >> 5, app_w = ((int)threadIdx.x & 31) * 16;
  const bool app = APPEND && blockIdx.x == 0 && app_i < a.app_n;
  uint4 app_s0 = make_uint4(0, 0, 0, 0), app_s1 = app_s0;
  const size_t app_off = (app_w < D ? (size_t)G * a.app_n * D : 0) +
                         ((size_t)g * a.app_n + app_i) * D + (app_w < D ? app_w : app_w - D);
  if (APPEND) {
    const uint4* app_p = reinterpret_cast<const uint4*>(app ? a.app_src + app_off : q);
    app_s0 = app_p[0];
    app_s1 = app_p[1];
  }
  __shared__ __align__(16) QOperand sq;
  prep_operand(a, g, QV_RAW, &sq, qw);
  SKV_TS(0, 1);
  if (tile < ntiles) {
    uint32_t b[4][4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const uint4 w = *reinterpret_cast<const uint4*>(&sq.bimg[kc][lane][0]);
      b[kc][0] = w.x; b[kc][1] = w.y; b[kc][2] = w.z; b[kc][3] = w.w;
    }
    const FrConv cv(sq, lane >> 4);
    if (!LOOP) {
      fr_score(a, g, tile, lane, cur, b, cv);
    } else {
      for (;;) {
        const int next = tile + step;
        const FrTile nxt = fr_load(a, g, next, lane);
        fr_score(a, g, tile, lane, cur, b, cv);
        if (next >= ntiles) break;
        cur = nxt;
        tile = next;
      }
    }
  }
  SKV_TS(0, 2);
  if (blockIdx.x == 0) {  // per-step state of the group (read by later kernels)
    uint32_t* bm = a.selbm + (size_t)g * (nc / 32);
    for (int i = threadIdx.x; i < nc / 32; i += FR_BLOCK) bm[i] = 0;
    if (threadIdx.x == 0) {
      a.status[g * ST_WORDS + ST_FULLSEL] = 0;
      a.status[g * ST_WORDS + ST_ERR] = 0;
    }
  }
  if (blockIdx.x == 0) {  // publish the raw operand (a copy of sq)
    const uint32_t* src = reinterpret_cast<const uint32_t*>(&sq);
    uint32_t* dst = reinterpret_cast<uint32_t*>(&a.qop[g * QV_COUNT + QV_RAW]);
    for (int i = threadIdx.x; i < (int)(sizeof(QOperand) / 4); i += FR_BLOCK) dst[i] = src[i];
  }
  if (APPEND && app) {  // the folded append's records (read from the next kernel on)
    const int row = a.app_row + app_i;
    uint8_t* rec = const_cast<uint8_t*>(a.kv8) +
                   (a.kv_table ? (size_t)kv_row_paged(a.kv_table, a.kv_shift, g, row)
                               : (size_t)g * a.kv_rows + row) * 512;
    const uint4 w0 = app_s0, w1 = app_s1;
    *reinterpret_cast<uint4*>(rec + app_w) =
        make_uint4(bf16x4_to_fp8(make_uint2(w0.x, w0.y)), bf16x4_to_fp8(make_uint2(w0.z, w0.w)),
                   bf16x4_to_fp8(make_uint2(w1.x, w1.y)), bf16x4_to_fp8(make_uint2(w1.z, w1.w)));
  }
  SKV_TSE(4);
}

__device__ __forceinline__ uint32_t same16(uint32_t o) { return o; }

// ============================================================ centroid selection
// Per (group, head): the P-th largest lower bound thr, then the P centroids
// with the best (fine score, lowest ID) among those whose upper bound reaches
// thr; members set their bit in the group's selected-cluster bitmap.  Blocks
// beyond the 16 (group, head) pairs compute the sink/local attention slices.
__device__ __forceinline__ void load_lds_masked(uint16_t* so, const uint16_t* __restrict__ score,
                                                const uint16_t* __restrict__ gate, uint32_t thr,
                                                int n) {
  const MaskedScores src{score, gate, thr};
  uint4* d4 = reinterpret_cast<uint4*>(so);
  for (int o = threadIdx.x; o < (n >> 3); o += blockDim.x) d4[o] = src.oct(o);
}

// Both selections of one (group, head) with its nc <= OCT_ITEMS centroids
// held in registers, one octet of lower, upper and fine scores per thread.
__device__ void select_in_registers(const StepArgs& a, const uint16_t* lower,
                                    const uint16_t* upper, const uint16_t* fine, int nc, int g,
                                    int h, FastScratch& fs) {
  const int t = threadIdx.x;
  const size_t row = ((size_t)g * H + h) * nc;
  const uint4 wl = load_oct(lower + row, nc);
  const uint4 wu = load_oct(upper + row, nc);
  const uint4 wf = load_oct(fine + row, nc);
  auto cid = [](int i) { return (uint32_t)i; };
  const OctResult r1 = oct_select<true, true>(wl, a.P[g], cid, fs, 2);
  const uint32_t thr = r1.sel.all ? 0u : r1.sel.v;
  if (t == 0) a.thr[g * H + h] = thr;
  SKV_TS(2, 6);
  // fine scores of the eligible centroids (upper >= thr), others excluded
  const uint4 wm = MaskedScores::pick4(wf, wu, thr);
  const OctResult r2 = oct_select<false, true>(wm, a.P[g], cid, fs, 4);
  // items 8t .. 8t+7 are byte t & 3 of bitmap word t >> 2: merge 4 lanes
  uint32_t m = r2.mine << (8 * (t & 3));
  m |= __shfl_xor(m, 1);
  m |= __shfl_xor(m, 2);
  if ((t & 3) == 0 && m) atomicOr(&a.selbm[(size_t)g * (nc / 32) + (t >> 2)], m);
  SKV_TS(2, 15);
}

// The same for nc <= NO x 8 x SEL_BLOCK centroids held as NO octets per
// thread (octet o of thread t: centroids 8 (t + o SEL_BLOCK) ..): all three
// rows are loaded at once, the threshold and the fine selection each run in
// registers, so the longer lists need no tile maxima and no second load
// round.  The fine selection ranks ties by centroid ID as IDs (octet order is
// not position order); with more ties at its P-th score than that ranking
// holds it returns false (the threshold is written) and the caller runs the
// fine selection another way.
template <int NO>
__device__ __forceinline__ bool select_in_registers_n(const StepArgs& a, const uint16_t* lower,
                                                      const uint16_t* upper, const uint16_t* fine,
                                                      int nc, int g, int h, FastScratch& fs,
                                                      uint32_t* thr_out) {
  const int t = threadIdx.x;
  const size_t row = ((size_t)g * H + h) * nc;
  // the lower bounds first: the threshold waits for them alone (the waits
  // count loads in issue order), the rest arrive during its selection
  uint4 wl[NO], wu[NO], wf[NO];
#pragma unroll
  for (int o = 0; o < NO; ++o) wl[o] = load_oct(lower + row + o * OCT_ITEMS, nc - o * OCT_ITEMS);
#pragma unroll
  for (int o = 0; o < NO; ++o) {
    wu[o] = load_oct(upper + row + o * OCT_ITEMS, nc - o * OCT_ITEMS);
    wf[o] = load_oct(fine + row + o * OCT_ITEMS, nc - o * OCT_ITEMS);
  }
  auto cid = [](int i) { return (uint32_t)i; };
  const OctResult r1 = octn_select<NO, true, false>(wl, a.P[g], cid, fs, 2);
  const uint32_t thr = r1.sel.all ? 0u : r1.sel.v;
  if (t == 0) a.thr[g * H + h] = thr;
  *thr_out = thr;
  SKV_TS(2, 6);
  uint4 wm[NO];
#pragma unroll
  for (int o = 0; o < NO; ++o) wm[o] = MaskedScores::pick4(wf[o], wu[o], thr);
  const OctResult r2 = octn_select<NO, false, false>(wm, a.P[g], cid, fs, 4);
  if (!r2.ok) return false;  // block-uniform
  // items 8u .. 8u+7 (u = t + o SEL_BLOCK) are byte u & 3 of bitmap word u >> 2
#pragma unroll
  for (int o = 0; o < NO; ++o) {
    uint32_t m = ((r2.mine >> (8 * o)) & 0xffu) << (8 * (t & 3));
    m |= __shfl_xor(m, 1);
    m |= __shfl_xor(m, 2);
    if ((t & 3) == 0 && m) atomicOr(&a.selbm[(size_t)g * (nc / 32) + ((t + o * SEL_BLOCK) >> 2)], m);
  }
  SKV_TS(2, 15);
  return true;
}

// The leading arguments repeat the fields of a that the selection blocks'
// first loads need (preloaded into scalar registers at dispatch).  PAGED: the
// sink/local records are read through the page table.  NO > 1: the instance
// for nc in (8 x SEL_BLOCK, NO x 8 x SEL_BLOCK], selecting in registers
// (select_in_registers_n); NO = 1 for every other nc.
template <bool PAGED, int NO>
__global__ __launch_bounds__(SEL_BLOCK) void k_select(const uint16_t* lower, const uint16_t* upper,
                                                      const uint16_t* fine, int nc_arg,
                                                      int exact_select, int dense_slices,
                                                      StepArgs a) {
  SKV_TSB(5, 0);
  SKV_TS(2, 0);
  extern __shared__ __align__(16) unsigned char dyn[];
  const int n_dense = G * H * dense_slices;
  if ((int)blockIdx.x >= G * H + n_dense) {  // the q15 / qs operands of the later scorers
    const int i = blockIdx.x - G * H - n_dense, g = i / 2, v = QV_Q15 + i % 2;
    const int hq = min((int)(threadIdx.x >> 6), H - 1);
    // formed in LDS (the image is written byte by byte), then copied out
    QOperand& lq = *reinterpret_cast<QOperand*>(dyn);
    prep_operand(a, g, v, &lq, load_qw(a, g, hq, threadIdx.x & 63));
    const uint32_t* src = reinterpret_cast<const uint32_t*>(&lq);
    uint32_t* dst = reinterpret_cast<uint32_t*>(&a.qop[g * QV_COUNT + v]);
    for (int i = threadIdx.x; i < (int)(sizeof(QOperand) / 4); i += blockDim.x) dst[i] = src[i];
    SKV_TSE(5);
    return;
  }
  if (blockIdx.x >= G * H) {  // sink/local attention slices (depend only on Q)
    dense_attend<PAGED>(a, blockIdx.x - G * H, *reinterpret_cast<AttnScratch*>(dyn));
    SKV_TSE(5);
    return;
  }
  const int g = blockIdx.x / H, h = blockIdx.x % H, nc = nc_arg;
  if (NO == 1 && exact_select == 0 && nc <= OCT_ITEMS) {
    select_in_registers(a, lower, upper, fine, nc, g, h, *reinterpret_cast<FastScratch*>(dyn));
    SKV_TSE(5);
    return;
  }
  __shared__ SelectScratch s;
  if constexpr (NO > 1) {  // launched for exact_select == 0 and nc <= NO x OCT_ITEMS only
    uint32_t thr;
    if (!select_in_registers_n<NO>(a, lower, upper, fine, nc, g, h,
                                   *reinterpret_cast<FastScratch*>(dyn), &thr)) {
      // more ties at the P-th fine score than the register ranking holds:
      // the full selection over the LDS copy of the eligible fine scores
      const size_t row = ((size_t)g * H + h) * nc;
      uint16_t* so = reinterpret_cast<uint16_t*>(dyn);
      load_lds_masked(so, fine + row, upper + row, thr, nc);
      __syncthreads();
      const Selection sel = block_select(so, nc, a.P[g], [](int i) { return (uint32_t)i; }, s);
      uint32_t* selbm = a.selbm + (size_t)g * (nc / 32);
      for_scores(so, nc, [&](int c, uint32_t o) {
        if (sel.member(o, (uint32_t)c)) atomicOr(&selbm[c >> 5], 1u << (c & 31));
      });
    }
    SKV_TSE(5);
    return;
  }
  __shared__ uint32_t s_thr;
  const size_t row = ((size_t)g * H + h) * nc;
  const uint16_t* lo = a.lower + row;  // ordered; never 0 (the "excluded" mark)
  const uint16_t* up = a.upper + row;
  const uint16_t* fi = a.fine_ord + row;
  const bool force = a.exact_select == 2;
  auto cid = [](int i) { return (uint32_t)i; };
  // the fine selection's sample (gate and score), loaded now, masked later
  uint32_t pg[FS_PER], pf[FS_PER];
#pragma unroll
  for (int u = 0; u < FS_PER; ++u) {
    const int i = min(fs_sample_item(nc, u), nc - 1);
    pg[u] = up[i];
    pf[u] = fi[i];
  }
  // ---- threshold: the P-th largest lower bound (its value)
  bool done = false;
  if (a.exact_select == 0 && a.tmax_lo) {
    // From the 8-centroid tile maxima: x, the P-th largest of them, is at
    // most the P-th largest lower bound (P tiles hold a bound >= x), so every
    // bound at or above that value lies in a tile whose max is >= x.  Those
    // tiles (at most one octet per thread) are gathered and the exact value
    // selected among them in registers.
    FastScratch& fs = *reinterpret_cast<FastScratch*>(dyn);
    const int nt8 = nc / 8;
    const uint4 wt = load_oct(a.tmax_lo + ((size_t)g * H + h) * nt8, nt8);
    const OctResult rt = oct_select<true, false>(wt, a.P[g], cid, fs);
    const uint32_t x = rt.sel.all ? 1u : rt.sel.v;
    const u32x4 wtv = {wt.x, wt.y, wt.z, wt.w};
    uint32_t fl = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) fl |= (uint32_t)(oct_half(wtv, e) >= x) << e;
    int ntiles;
    int j = block_excl_scan(__popc(fl), fs.scan, &ntiles);  // ends with a barrier
    if (ntiles <= SEL_BLOCK) {
      int* tl = reinterpret_cast<int*>(fs.cand);
      for (uint32_t rest = fl; rest; rest &= rest - 1) tl[j++] = 8 * (int)threadIdx.x + __ffs(rest) - 1;
      __syncthreads();
      uint4 wg = make_uint4(0, 0, 0, 0);
      if ((int)threadIdx.x < ntiles) wg = reinterpret_cast<const uint4*>(lo)[tl[threadIdx.x]];
      const OctResult rg = oct_select<true, false>(wg, a.P[g], cid, fs);
      if (threadIdx.x == 0) s_thr = rg.sel.all ? 0u : rg.sel.v;
      done = true;
    }
  }
  if (!done && a.exact_select != 1) {
    FastScratch& fs = *reinterpret_cast<FastScratch*>(dyn);
    const FastResult r = fast_select<true>(RowScores{lo}, nc, a.P[g], cid, fs, force, 2);
    if (r.ok) {
      if (threadIdx.x == 0) s_thr = r.sel.all ? 0u : r.sel.v;
      done = true;
    } else {
      __syncthreads();
      if (threadIdx.x == 0) atomicOr(&a.status[g * ST_WORDS + ST_FULLSEL], FS_THRESH);
    }
  }
  if (!done) {
    uint16_t* so = reinterpret_cast<uint16_t*>(dyn);
    load_lds_scores(so, lo, nc, same16);
    __syncthreads();
    const Selection sel = block_select(so, nc, a.P[g], cid, s);
    if (threadIdx.x == 0) s_thr = sel.all ? 0u : sel.v;
  }
  __syncthreads();
  const uint32_t thr = s_thr;
  if (threadIdx.x == 0) a.thr[g * H + h] = thr;
  SKV_TS(2, 6);
  // ---- fine select among the eligible centroids
  uint32_t* selbm = a.selbm + (size_t)g * (nc / 32);
  done = false;
  if (a.exact_select != 1) {
    FastScratch& fs = *reinterpret_cast<FastScratch*>(dyn);
    FastResult r{};
    r.ok = false;
    if (a.tmax_fi && nc / 16 <= 4 * SEL_BLOCK) {
      // only the 16-centroid tiles whose max fine score reaches the cut can
      // hold a candidate: their scores and gates are loaded, no others
      uint32_t sv[FS_PER];
#pragma unroll
      for (int u = 0; u < FS_PER; ++u) sv[u] = pg[u] >= thr ? pf[u] : 0u;
      r = tiled_select(MaskedTiles{fi, up, thr}, a.tmax_fi + ((size_t)g * H + h) * (nc / 16), sv, nc,
                       a.P[g], cid, fs, force, 4);
      __syncthreads();
    }
    if (!r.ok)
      r = fast_select_s<false>(MaskedScores{fi, up, thr}, nc, a.P[g], cid, fs, force, 4,
                               [&](int u, int) { return pg[u] >= thr ? pf[u] : 0u; });
    if (r.ok) {
      for (int c = threadIdx.x; c < r.ncand; c += SEL_BLOCK) {
        const uint64_t key = fs.cand[c];
        if (fs_member(r, key, cid)) {
          const int cc = cand_pos(key);
          atomicOr(&selbm[cc >> 5], 1u << (cc & 31));
        }
      }
      done = true;
    } else {
      __syncthreads();
      if (threadIdx.x == 0) atomicOr(&a.status[g * ST_WORDS + ST_FULLSEL], FS_FINE);
    }
  }
  if (!done) {
    uint16_t* so = reinterpret_cast<uint16_t*>(dyn);
    load_lds_masked(so, fi, up, thr, nc);
    __syncthreads();
    const Selection sel = block_select(so, nc, a.P[g], cid, s);
    for_scores(so, nc, [&](int c, uint32_t o) {
      if (sel.member(o, (uint32_t)c)) atomicOr(&selbm[c >> 5], 1u << (c & 31));
    });
  }
  SKV_TS(2, 15);
  SKV_TSE(5);
}

// ============================================================ pool
// Posting j of cluster c is owned iff its mate cluster is larger (or absent)
// or not selected: the first occurrence in encounter order keeps the token.
__device__ __forceinline__ bool owned(const uint32_t* selbm, uint32_t mate, uint32_t c) {
  return mate > c || !((selbm[mate >> 5] >> (mate & 31)) & 1u);
}

constexpr int PL_BLOCK = 1024;  // pool: one block per CU; waves 1.. hold a posting per thread and page
constexpr int PL_WAVES = PL_BLOCK / WAVE;
constexpr int PL_RANGE_MAX = PL_BLOCK;  // centroids per pool block: one per thread
// The range scan packs (postings << PL_SEL_BITS) | selected into one unsigned
// word: a range selects at most PL_RANGE_MAX clusters, and its postings are
// fewer than 2^(32 - PL_SEL_BITS) = 2^21 (a group holds < 2^21 postings:
// spill 2 over at most 2^20 tokens, checked by skv_create).
constexpr int PL_SEL_BITS = 11;
constexpr unsigned PL_SEL_MASK = (1u << PL_SEL_BITS) - 1u;
static_assert(PL_RANGE_MAX <= (int)PL_SEL_MASK, "a range's selected count fits its scan field");
constexpr int PL_PAGE = PL_BLOCK - WAVE;     // postings per page (waves 1..)
constexpr int PL_BM_WORDS = 65536 / 32;      // selected-cluster bitmap words held in LDS (any nc)
// 16-key tiles of s2 the first two pages' owned postings overlap (at most)
constexpr int PL_TM_TILES = (2 * PL_PAGE + 15) / 16 + 1;

// Range records for the look-back, one 64-bit word written and read whole:
// state (bits 62..63) | launch epoch (57..61) | coarse survivors (40..56) |
// selected clusters (23..39) | owned postings (0..22).  Sums of record values
// add field by field (a group holds < 2^23 pool keys and <= 65536 clusters).
// A record of the previous launch (other epoch) reads as not yet published,
// so nothing is cleared between launches; the records carry every count the
// scan needs, so no memory fence orders other data before them.
constexpr unsigned long long LB_A = 1ull << 62;  // the range's own counts
constexpr unsigned long long LB_P = 2ull << 62;  // counts of all ranges up to this one
constexpr int LB_SEL = 23, LB_SURV = 40, LB_EPOCH = 57;
constexpr unsigned long long LB_VAL = (1ull << LB_EPOCH) - 1;
constexpr unsigned LB_EPOCHS = 32;
constexpr int LB_SPIN_MAX = 1 << 22;  // polls before a wait is abandoned (SKV_EPOOL_WAIT)
constexpr int LB_WIN = 4;             // 64-range windows read per poll
__device__ __forceinline__ int lb_field(unsigned long long v, int shift, int bits) {
  return (int)((v >> shift) & ((1ull << bits) - 1));
}

// 2-bit pool scores (reference codegen/stage15.py:886-995):
// s2 = bf16(16 RNE(sum q15 (2 p2 - 3))) of a key from its 64-byte prefix row
// (the posting-ordered copy), 16 keys per int8 matrix-core tile.  A wave
// scores the 64 postings its lanes hold, 4 tiles: s2_rows loads tile u's
// rows (lane (kb, row) reads bytes 16 kb .. 16 kb + 15 of the row of the
// posting held by lane 16 u + row; j < 0, absent: row 0 is read instead,
// and its score is never emitted).  The loads are unconditional, so all
// four are in flight together (a conditional load makes the compiler wait
// for it where the branches join).  s2_score
// multiplies the query image (rows: head x limb) by the keys (columns), so
// lane l receives the 4 limb sums of key l % 16 for head l / 16 in its 4
// accumulator registers (no exchange between lanes), and returns in sc[u]
// that key's ordered score; ls is head l / 16's scale.
__device__ __forceinline__ void s2_rows(const uint8_t* __restrict__ rows, int j, uint4 (&w)[4]) {
  const int lane = threadIdx.x & 63, row = lane & 15, kb = lane >> 4;
  int jj[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) jj[u] = max(__shfl(j, 16 * u + row), 0);
#pragma unroll
  for (int u = 0; u < 4; ++u)
    w[u] = *reinterpret_cast<const uint4*>(rows + (size_t)jj[u] * 64 + kb * 16);
}

__device__ __forceinline__ void s2_score(const uint4 (&w)[4], const uint32_t (&bq)[4][4],
                                         const LimbScale& ls, double c, uint32_t (&sc)[4]) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t words[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      uint32_t av[4];
      expand2t(words[kc], av);
      acc = mfma_i8(bq[kc], av, acc);
    }
    sc[u] = ordered16(bf16_rne(ls(acc[0], acc[1], acc[2], c)));  // (2 dq - 3 sum q15) 2^fx
  }
}

// Stores the scores of s2_score for the owned postings: own = the wave's
// ballot of owned postings (bit p: the posting lane p holds), wbase = the
// segment rank of its first owned posting; rank r lands at pool position
// base + r.  With tm, each score also raises tm[head][tile - t0], the LDS
// maximum of its 16-key tile (pool position / 16).
__device__ __forceinline__ void s2_emit(const uint32_t (&sc)[4], uint64_t own, int wbase, int base,
                                        uint16_t* s2, int cap, uint32_t* tm, int t0) {
  const int lane = threadIdx.x & 63, hq = lane >> 4;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int p = 16 * u + (lane & 15);
    if ((own >> p) & 1ull) {
      const int pos = base + wbase + __popcll(own & ((1ull << p) - 1ull));
      if (pos < cap) s2[(size_t)hq * cap + pos] = (uint16_t)sc[u];
      if (tm) atomicMax(&tm[hq * PL_TM_TILES + (pos >> 4) - t0], sc[u]);
    }
  }
}

// Maxima of the 16-key tiles of s2 ([H][tstride] words) that the pool
// positions [A, A + L) overlap.  With tm (the LDS maxima of s2_emit,
// tm[head][tile - A / 16]) a tile inside the segment gets its exact
// maximum, and so does its last tile when the segment ends the pool
// (end_exact: positions beyond hold no key); any other tile gets 0xffff.
// Such a tile is shared with another block, which writes 0xffff to it as
// well: an upper bound, all the top-1600's tile skip needs.
__device__ void s2_tile_max(int A, int L, bool end_exact, const uint32_t* tm, uint16_t* tmax,
                            int tstride) {
  if (L <= 0) return;
  const int t_lo = A >> 4, nt = ((A + L - 1) >> 4) - t_lo + 1;
  for (int x = threadIdx.x; x < nt * H; x += blockDim.x) {
    const int h = x / nt, i = x - h * nt, tile = t_lo + i, s0 = 16 * tile;
    const bool exact = tm && s0 >= A && (s0 + 16 <= A + L || end_exact);
    if (tile < tstride) tmax[(size_t)h * tstride + tile] = (uint16_t)(exact ? tm[h * PL_TM_TILES + i] : 0xffffu);
  }
}

__device__ __forceinline__ unsigned long long lb_load(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void lb_store(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The pool of one KV group in encounter order: selected clusters ascending,
// CSR order within a cluster, each token kept at its first occurrence, and
// the 2-bit scores of its keys.  Block b = range b of pool_range centroids
// (a multiple of 32).  Each range publishes its counts, then sums its
// predecessors' counts (decoupled look-back: a predecessor that already
// published its inclusive prefix ends the walk) and writes its owned
// postings at their pool positions, one posting per thread.  The prefix
// rows of the range's postings are loaded before the look-back and scored
// while wave 0 walks it, so the scores are ready with the positions.
// The leading arguments repeat the fields of a that the prologue loads need
// (preloaded into scalar registers at dispatch).
__global__ __launch_bounds__(PL_BLOCK) void k_pool(const uint32_t* selbm, const int* csr_off,
                                                   const uint16_t* upper, const uint32_t* thr,
                                                   const QOperand* qop,
                                                   const unsigned* pool_epoch, int nc_arg,
                                                   int pool_range, StepArgs a) {
  SKV_TSB(0, 0);
  SKV_TS(5, 0);
  const int g = blockIdx.y, nc = nc_arg, nb = gridDim.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, t = threadIdx.x;
  extern __shared__ uint32_t s_bm[];
  __shared__ int s_off[2 * PL_BLOCK], s_cum[PL_RANGE_MAX + 1], s_cl[PL_RANGE_MAX];
  __shared__ int s_scan[PL_WAVES + 1], s_surv;
  __shared__ unsigned long long s_excl;
  __shared__ uint32_t s_tm[H * PL_TM_TILES];  // tile maxima of the first two pages' keys
  // range b = block b: workgroups are dispatched in index order within each
  // XCD, so the lowest unfinished range always gets a slot and every wait
  // below ends.  The launch epoch tags this launch's records.
  const int b = blockIdx.x, c0 = b * pool_range;
  const int ncr = min(pool_range, nc - c0);  // centroids of the range (a multiple of 32)
  // every load of the prologue is issued before the first wait: the group's
  // selected-cluster bitmap (<= 2048 words), the range's CSR offsets
  // (<= 513), and its centroids' upper bounds and the thresholds
  const unsigned epoch = pool_epoch[g];
  const unsigned long long tag = (unsigned long long)(epoch % LB_EPOCHS) << LB_EPOCH;
  constexpr int BM_PER = PL_BM_WORDS / PL_BLOCK;
  const int nbw = nc / 32;
  const uint32_t* bm = selbm + (size_t)g * nbw;
  const int* off = csr_off + (size_t)g * (nc + 1) + c0;
  uint32_t bmw[BM_PER];
#pragma unroll
  for (int u = 0; u < BM_PER; ++u) bmw[u] = bm[min(t + u * PL_BLOCK, nbw - 1)];
  const int off0 = off[min(t, ncr)], off1 = off[min(t + PL_BLOCK, ncr)];
  const int cu = c0 + min(t, ncr - 1);
  uint32_t upv[H], thv[H];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    upv[h] = upper[((size_t)g * H + h) * nc + cu];
    thv[h] = thr[g * H + h];
  }
  // the 2-bit scorer's query operand (B image of 16 q15, its sum and scale)
  const QOperand* q15 = &qop[g * QV_COUNT + QV_Q15];
  uint32_t bq[4][4];
  load_b(q15, bq);
  // lane l's head l / 16: s2 = (2 dq - 3 sum q15) 2^(fx + 4)
  const LimbScale ls(q15->fx[lane >> 4] + 4, 1);
  const double lc = LimbScale::offset(-3 * q15->sum[lane >> 4], q15->fx[lane >> 4] + 4);
  // every slot stored (the bitmap's LDS copy is PL_BM_WORDS long; slots past
  // nbw repeat the last word and are never read): a conditional store would
  // let the compiler sink the bitmap load into it and wait there for every
  // load issued before
#pragma unroll
  for (int u = 0; u < BM_PER; ++u) s_bm[t + u * PL_BLOCK] = bmw[u];
  s_off[t] = off0;  // (unconditional, as s_bm: slots past ncr hold off[ncr], never read)
  s_off[t + PL_BLOCK] = off1;
  if (t == 0) {
    s_surv = 0;
  }
  if (t < H * PL_TM_TILES) s_tm[t] = 0;
  // survivor head masks (upper_h >= thr_h) of the range's centroids
  uint32_t m = 0;
  if (t < ncr) {
#pragma unroll
    for (int h = 0; h < H; ++h) m |= (uint32_t)(upv[h] >= thv[h]) << h;
    a.masks[(size_t)g * nc + c0 + t] = (uint8_t)m;
  }
  __syncthreads();
  {
    const int alive = __popcll(__ballot(m != 0));
    if (lane == 0 && alive) atomicAdd(&s_surv, alive);
  }
  // the range's selected clusters in order and their posting offsets: one
  // scan of (postings << PL_SEL_BITS | selected) over the range's centroids
  const bool is_sel = t < ncr && ((s_bm[(c0 + t) >> 5] >> (t & 31)) & 1u);
  const unsigned size = is_sel ? (unsigned)(s_off[t + 1] - s_off[t]) : 0u;
  unsigned tot;
  const unsigned ex = block_excl_scan_t<unsigned>((size << PL_SEL_BITS) | (is_sel ? 1u : 0u),
                                                  reinterpret_cast<unsigned*>(s_scan), &tot);
  const int nsel = (int)(tot & PL_SEL_MASK);
  if (is_sel) {
    const int r = (int)(ex & PL_SEL_MASK);
    s_cl[r] = t;
    s_cum[r] = (int)(ex >> PL_SEL_BITS);
  }
  if (t == 0) s_cum[nsel] = (int)(tot >> PL_SEL_BITS);
  __syncthreads();
  const int S = s_cum[nsel];  // postings of the selected clusters
  if (t == 0) a.pool_scan[g * a.pool_blocks + b] = S;  // summed by the U1 scorer (diagnostic)
  const int* __restrict__ mate = a.post_mate + (size_t)g * a.np_max;
  const int* __restrict__ ptok = a.post_tok + (size_t)g * a.np_max;
  // posting i of the range's selected lists -> posting index j (its cluster
  // in cl), and whether the range owns it
  auto locate = [&](int i, int& cl) {
    int lo = 0, hi = nsel;  // s_cum[lo] <= i < s_cum[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_cum[mid] <= i) lo = mid;
      else hi = mid;
    }
    cl = s_cl[lo];
    return s_off[cl] + (i - s_cum[lo]);
  };
  auto posting = [&](int i, int& j) {
    int cl;
    j = locate(i, cl);
    return owned(s_bm, (uint32_t)mate[j], (uint32_t)(c0 + cl));
  };
  // ---- count: postings go to waves 1.. (PL_PAGE per page; wave 0 walks
  // the look-back while they are scored).  The first two pages stay in
  // registers for the emit (their mate, token and prefix-row loads issued
  // together); later pages are re-walked.
  const int pi = (int)threadIdx.x - WAVE;  // this thread's posting of a page (wave 0: none)
  const bool h0 = pi >= 0 && pi < S, h1 = pi >= 0 && pi + PL_PAGE < S;
  int cl0 = 0, cl1 = 0;
  const int j0 = h0 ? locate(pi, cl0) : -1;
  const int j1 = h1 ? locate(pi + PL_PAGE, cl1) : -1;
  const int m0 = h0 ? mate[j0] : -1, m1 = h1 ? mate[j1] : -1;
  const int t0 = h0 ? ptok[j0] : 0, t1 = h1 ? ptok[j1] : 0;
  const bool o0 = h0 && owned(s_bm, (uint32_t)m0, (uint32_t)(c0 + cl0));
  const bool o1 = h1 && owned(s_bm, (uint32_t)m1, (uint32_t)(c0 + cl1));
  // prefix rows of the first two pages' owned postings, issued once the
  // mates are in; the rows (64 B per key) are the kernel's bulk traffic and
  // arrive during the scans and the look-back
  const uint8_t* __restrict__ rows = a.post_p2 + (size_t)g * a.np_max * 64;
  // (every wave, both pages: straight-line loads stay in flight together;
  // wave 0 and a missing second page read row 0, never scored)
  uint4 rw0[4], rw1[4];
  s2_rows(rows, o0 ? j0 : -1, rw0);
  s2_rows(rows, o1 ? j1 : -1, rw1);
  // one scan for both pages: page 1 in the high half (a page owns < 2^16)
  int both;
  const int exb = block_excl_scan((o1 ? 1 << 16 : 0) | (o0 ? 1 : 0), s_scan, &both);
  const int ex0 = exb & 0xffff, ex1 = exb >> 16;
  const int page0_total = both & 0xffff, page1_total = both >> 16;
  int owned_total = page0_total + page1_total;
  for (int base = 2 * PL_PAGE; base < S; base += PL_PAGE) {
    int j = 0;
    const bool o = pi >= 0 && base + pi < S && posting(base + pi, j);
    int tot;
    (void)block_excl_scan(o ? 1 : 0, s_scan, &tot);
    owned_total += tot;
  }
  // ---- publish, then look back for the counts of the earlier ranges
  unsigned long long* flags = a.pool_flags + (size_t)g * nb;
  const unsigned long long agg = ((unsigned long long)s_surv << LB_SURV) |
                                 ((unsigned long long)nsel << LB_SEL) | (unsigned)owned_total;
  if (wave == 0) {
    if (lane == 0) {
      lb_store(&flags[b], (b == 0 ? LB_P : LB_A) | tag | agg);
      SKV_TSB(0, 2);
    }
    // up to LB_WIN * 64 predecessors per poll: entry (k, lane) is range
    // i - 64 k - lane, k-major in distance
    unsigned long long excl = 0;
    int spins = 0;
    for (int i = b - 1; i >= 0;) {
      unsigned long long v[LB_WIN];
      bool cur[LB_WIN];
      uint64_t pm[LB_WIN], xm[LB_WIN];
#pragma unroll
      for (int k = 0; k < LB_WIN; ++k) {
        const int idx = i - 64 * k - lane;
        v[k] = idx >= 0 ? lb_load(&flags[idx]) : (LB_P | tag);
      }
#pragma unroll
      for (int k = 0; k < LB_WIN; ++k) {
        cur[k] = (v[k] & ~LB_VAL & ~(3ull << 62)) == tag;  // published in this launch
        pm[k] = __ballot(cur[k] && (v[k] >> 62) == 2);
        xm[k] = __ballot(!cur[k] || (v[k] >> 62) == 0);
      }
      // the nearest inclusive prefix ends the walk; every nearer entry is needed
      int kp = LB_WIN, lp = 63;
#pragma unroll
      for (int k = LB_WIN - 1; k >= 0; --k)
        if (pm[k]) {
          kp = k;
          lp = __ffsll((long long)pm[k]) - 1;
        }
      bool wait = false;
#pragma unroll
      for (int k = 0; k < LB_WIN; ++k) {
        const uint64_t need = k < kp ? ~0ull : k == kp ? (lp == 63 ? ~0ull : ((1ull << (lp + 1)) - 1ull)) : 0ull;
        wait = wait || (xm[k] & need) != 0;
      }
      if (wait) {  // a needed range has not published yet
        if (++spins > LB_SPIN_MAX) {
          if (lane == 0) a.status[g * ST_WORDS + ST_ERR] = SKV_EPOOL_WAIT;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        continue;
      }
      int o = 0, sl = 0, sv = 0;
#pragma unroll
      for (int k = 0; k < LB_WIN; ++k) {
        const bool take = k < kp || (k == kp && lane <= lp);
        if (take) {
          o += lb_field(v[k], 0, LB_SEL);
          sl += lb_field(v[k], LB_SEL, LB_SURV - LB_SEL);
          sv += lb_field(v[k], LB_SURV, LB_EPOCH - LB_SURV);
        }
      }
      o = wave_sum(o);
      sl = wave_sum(sl);
      sv = wave_sum(sv);
      excl += ((unsigned long long)sv << LB_SURV) | ((unsigned long long)sl << LB_SEL) | (unsigned)o;
      if (kp < LB_WIN) break;
      i -= 64 * LB_WIN;
    }
    if (lane == 0) {
      if (b > 0) lb_store(&flags[b], LB_P | tag | (excl + agg));
      s_excl = excl;
      // every range has published, so every block has read the epoch
      if (b == nb - 1) a.pool_epoch[g] = epoch + 1;
      SKV_TSV(10, 0, spins);
      SKV_TSV(10, 1, b);
      SKV_TSV(10, 2, S);
    }
  }
  // 2-bit scores of the first two pages (waves 1.. while wave 0 looks back)
  uint32_t sc0[4] = {0, 0, 0, 0}, sc1[4] = {0, 0, 0, 0};
  if (wave > 0 && (wave - 1) * WAVE < S) s2_score(rw0, bq, ls, lc, sc0);  // wave-uniform
  if (wave > 0 && PL_PAGE + (wave - 1) * WAVE < S) s2_score(rw1, bq, ls, lc, sc1);
  __syncthreads();
  SKV_TSB(0, 1);
  const unsigned long long excl = s_excl;
  const int pos0 = lb_field(excl, 0, LB_SEL), sel0 = lb_field(excl, LB_SEL, LB_SURV - LB_SEL);
  const int surv0 = lb_field(excl, LB_SURV, LB_EPOCH - LB_SURV);
  // ---- emit: the selected list and the owned postings at their positions
  for (int r = t; r < nsel; r += PL_BLOCK) a.sel[(size_t)g * nc + sel0 + r] = c0 + s_cl[r];
  int* pool = a.pool_tok + (size_t)g * a.cap;
  uint16_t* s2 = a.s2 + (size_t)g * H * a.cap;
  uint16_t* tmax = a.s2_tmax + (size_t)g * H * (a.cap / 16);
  if (o0 && pos0 + ex0 < a.cap) pool[pos0 + ex0] = t0;
  if (o1 && pos0 + page0_total + ex1 < a.cap) pool[pos0 + page0_total + ex1] = t1;
  s2_emit(sc0, __ballot(o0), __builtin_amdgcn_readfirstlane(ex0), pos0, s2, a.cap, s_tm, pos0 >> 4);
  if (S > PL_PAGE)
    s2_emit(sc1, __ballot(o1), page0_total + __builtin_amdgcn_readfirstlane(ex1), pos0, s2, a.cap,
            s_tm, pos0 >> 4);
  const int p01 = page0_total + page1_total;
  int carry = p01;
  for (int base = 2 * PL_PAGE; base < S; base += PL_PAGE) {  // ranges over two pages
    int j = -1;
    const bool o = pi >= 0 && base + pi < S && posting(base + pi, j);
    uint4 rw[4];
    if (wave > 0) s2_rows(rows, o ? j : -1, rw);
    int tot;
    const int ex = block_excl_scan(o ? 1 : 0, s_scan, &tot);
    const int p = pos0 + carry + ex;
    if (o && p < a.cap) pool[p] = ptok[j];
    uint32_t sc[4] = {0, 0, 0, 0};
    if (wave > 0 && base + (wave - 1) * WAVE < S) s2_score(rw, bq, ls, lc, sc);
    s2_emit(sc, __ballot(o), __builtin_amdgcn_readfirstlane(ex), pos0 + carry, s2, a.cap, nullptr,
            0);
    s2_tile_max(pos0 + carry, tot, false, nullptr, tmax, a.cap / 16);  // bounds only
    carry += tot;
  }
  // tile maxima of the first two pages' segment (from the LDS maxima)
  __syncthreads();
  s2_tile_max(pos0, p01, b == nb - 1 && S <= 2 * PL_PAGE, s_tm, tmax, a.cap / 16);
  // ---- the last range writes the group's totals
  if (b == nb - 1 && threadIdx.x == 0) {
    {
      const int sv = surv0 + s_surv;
      const int to = pos0 + owned_total, ts = sel0 + nsel;
      int err = a.status[g * ST_WORDS + ST_ERR];
      if (err == 0) {
        if (a.pool_capacity > 0 && to > a.pool_capacity) err = 4;
        else if (to < a.pool_min) err = 5;
      }
      a.status[g * ST_WORDS + ST_POOL] = min(to, a.cap);
      a.status[g * ST_WORDS + ST_ERR] = err;
      a.status[g * ST_WORDS + ST_SEL] = ts;
      a.status[g * ST_WORDS + ST_SURV] = sv;
    }
  }
  SKV_TSE(0);
}

// ============================================================ token top-k
// Member bits of this thread's octet (bit e = item 8t + e) -> 64-bit bitmap
// words: octet t is byte t & 7 of word t >> 3, merged over 8 lanes.
__device__ __forceinline__ void write_member_words(uint32_t mine, int n, uint64_t* bm) {
  const int u = threadIdx.x, words = (n + 63) / 64;
  const uint32_t m = mine << (8 * (u & 3));
  uint32_t lo = (u & 4) ? 0u : m, hi = (u & 4) ? m : 0u;
  lo |= __shfl_xor(lo, 1);
  hi |= __shfl_xor(hi, 1);
  lo |= __shfl_xor(lo, 2);
  hi |= __shfl_xor(hi, 2);
  lo |= __shfl_xor(lo, 4);
  hi |= __shfl_xor(hi, 4);
  if ((u & 7) == 0 && (u >> 3) < words) bm[u >> 3] = ((uint64_t)hi << 32) | lo;
}


// Dynamic LDS of k_topk: the sampled-cut scratch and the member bitmap
// (TOPK_LDS_WORDS words), or the LDS-resident scores of the full selection.
size_t topk_dynamic_lds(int lds_items) {
  return std::max(sizeof(FastScratch) + (size_t)TOPK_LDS_WORDS * 8, (size_t)lds_items * 2);
}

// Per (group, head): members = top-k by (ordered score, lowest token) of the
// n items; writes the membership bitmap.  LDS-resident when n <= lds_items,
// otherwise 8-bit radix passes over the full 40-bit keys in memory.
// The leading arguments repeat the fields of t that the first loads need
// (preloaded into scalar registers at dispatch, so those loads do not wait
// for the argument block).
// OCT2: rows of up to 2 x OCT_ITEMS items are selected in registers too (two
// octets per thread), which a top-1600 over pools of 8K-16K keys gains from;
// the extra path costs the other selections some speed when it is compiled
// into their instance, so the runtime launches it only while the pools are
// that small (TopkArgs::regs2).  Both instances select the same members.
template <bool OCT2>
__global__ __launch_bounds__(SEL_BLOCK) void k_topk(const int* count_word, const uint16_t* scores,
                                                    int stride, int exact_select,
                                                    const uint16_t* tile_max, int words,
                                                    TopkArgs t) {
  SKV_TSB((t.count_slot == ST_POOL ? 6 : 7), 0);
  const int ts = t.count_slot == ST_POOL ? 7 : 10;
  SKV_TS(ts, 0);
  const int g = blockIdx.x / H, h = blockIdx.x % H;
  __shared__ SelectScratch s;
  extern __shared__ __align__(16) unsigned char dyn[];
  const int n = count_word[g * ST_WORDS];
  const uint16_t* sc = scores + ((size_t)g * H + h) * stride;
  const int* tok = t.tokens + (size_t)g * t.stride;
  uint64_t* bm = t.bitmap + ((size_t)g * H + h) * words;
  auto id = [tok](int i) { return (uint32_t)tok[i]; };
  if (exact_select == 0 && n <= OCT_ITEMS) {  // the scores fit in registers
    const OctResult r = oct_select<false, false>(load_oct(sc, n), t.k, id,
                                                 *reinterpret_cast<FastScratch*>(dyn), ts);
    if (r.ok) {
      write_member_words(r.mine, n, bm);
      SKV_TS(ts, 15);
      SKV_TSE((t.count_slot == ST_POOL ? 6 : 7));
      return;
    }
  } else if (OCT2 && exact_select == 0 && n <= 2 * OCT_ITEMS) {  // two octets per thread
    const uint4 w2[2] = {load_oct(sc, n), load_oct(sc + OCT_ITEMS, n - OCT_ITEMS)};
    const OctResult r = octn_select<2, false, false>(w2, t.k, id,
                                                     *reinterpret_cast<FastScratch*>(dyn), ts);
    if (r.ok) {
      write_member_words(r.mine & 0xffu, OCT_ITEMS, bm);
      write_member_words(r.mine >> 8, n - OCT_ITEMS, bm + OCT_ITEMS / 64);
      SKV_TS(ts, 15);
      SKV_TSE((t.count_slot == ST_POOL ? 6 : 7));
      return;
    }
  }
  if (exact_select != 1) {
    FastScratch& fs = *reinterpret_cast<FastScratch*>(dyn);
    // the member bitmap: in LDS beside the scratch (cleared before the
    // selection) when it fits, else in place
    const int words = (n + 63) / 64;
    const bool local = words <= TOPK_LDS_WORDS;
    uint64_t* mb = local ? reinterpret_cast<uint64_t*>(dyn + sizeof(FastScratch)) : bm;
    if (local)
      for (int w = threadIdx.x; w < words; w += SEL_BLOCK) mb[w] = 0;
    FastResult r{};
    r.ok = false;
    if (tile_max && exact_select != 1 && n > OCT_ITEMS && (n + 15) / 16 <= 4 * SEL_BLOCK) {
      // the producer wrote the max of every 16-item tile: only the tiles
      // reaching the cut are read for candidates
      uint32_t sv[FS_PER];
#pragma unroll
      for (int u = 0; u < FS_PER; ++u) sv[u] = sc[fs_sample_item(n, u)];
      r = tiled_select(RowTiles{sc}, tile_max + ((size_t)g * H + h) * t.tile_stride, sv, n, t.k,
                       id, fs, exact_select == 2, ts);
      __syncthreads();
    }
    if (!r.ok) r = fast_select(RowScores{sc}, n, t.k, id, fs, exact_select == 2, ts);
    if (r.ok) {
      SKV_TS(ts, 6);
      if (!local) {
        for (int w = threadIdx.x; w < words; w += SEL_BLOCK) mb[w] = 0;
        __syncthreads();
      }
      for (int c = threadIdx.x; c < r.ncand; c += SEL_BLOCK) {
        const uint64_t key = fs.cand[c];
        if (fs_member(r, key, id)) {
          const int p = cand_pos(key);
          atomicOr(reinterpret_cast<unsigned long long*>(&mb[p >> 6]), 1ull << (p & 63));
        }
      }
      if (local) {
        __syncthreads();
        for (int w = threadIdx.x; w < words; w += SEL_BLOCK) bm[w] = mb[w];
      }
      SKV_TS(ts, 15);
      SKV_TSE((t.count_slot == ST_POOL ? 6 : 7));
      return;
    }
    __syncthreads();
    if (threadIdx.x == 0) atomicOr(&t.status[g * ST_WORDS + ST_FULLSEL], t.fullsel_bit);
  }
  uint16_t* so = reinterpret_cast<uint16_t*>(dyn);
  if (n <= t.lds_items) {
    load_lds_scores(so, sc, n, same16);
    __syncthreads();
    const Selection sel = block_select(so, n, t.k, id, s);
    write_members(so, n, sel, id, bm);
    SKV_TSE((t.count_slot == ST_POOL ? 6 : 7));
    return;
  }
  auto val = [sc, tok](int i, uint64_t* v) {
    *v = ((uint64_t)sc[i] << 20) | (0xfffffu - (uint32_t)tok[i]);
    return true;
  };
  const uint64_t kth = n <= t.k ? 0 : block_kth<40>(n, t.k, val, s.k);
  const int lane = threadIdx.x & 63;
  for (int base = threadIdx.x & ~63; base < n; base += SEL_BLOCK) {
    const int i = base + lane;
    uint64_t v = 0;
    const bool m = i < n && val(i, &v) && v >= kth;
    const uint64_t ball = __ballot(m);
    if (lane == 0) bm[base >> 6] = ball;
  }
  SKV_TSE((t.count_slot == ST_POOL ? 6 : 7));
}

// ============================================================ key scores
// Code4 (p2 << 2 | r2) A-operand words of one key record for all 4 chunks.
__device__ __forceinline__ void load_code4(const uint8_t* rec, int kb, uint32_t out[4][4]) {
  const uint4 p = *reinterpret_cast<const uint4*>(rec + kb * 16);
  const uint4 r = *reinterpret_cast<const uint4*>(rec + 64 + kb * 16);
  const uint32_t pw[4] = {p.x, p.y, p.z, p.w}, rw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    uint32_t ep[4], er[4];
    expand2t(pw[kc], ep);
    expand2t(rw[kc], er);
#pragma unroll
    for (int m = 0; m < 4; ++m) out[kc][m] = (ep[m] << 2) | er[m];
  }
}

// ============================================================ union + scores
// U1: the union of the four heads' top-1600 member bitmaps over the pool,
// compacted in pool order, with every member's 4-bit and 8-bit scores.  The
// 8-bit dot is 16 x (the 4-bit code dot) + (the residual-4 dot), so one pass
// over a key's record gives both; the top-256 ranks the 4-bit scores and the
// top-100 the 8-bit scores of the top-256 union (U2), read from this list by
// U1 position.  Block b of a group owns a contiguous span of bitmap words:
// it counts the members in all earlier words (its output base), lists its
// own members in LDS, copies their tokens to the output list and scores
// them 16 keys per MFMA tile.  64 blocks of 1024 threads per group, one per
// CU across the 4 groups, each listing up to 16 words per pass (config 2:
// one pass).
constexpr int US_BLOCK = 1024;
constexpr int US_GRID = 64;  // blocks per group over the pool

// The leading arguments are the pool size word, the top-1600 member bitmaps,
// the pool's token list, bitmap words per head and the token list's stride
// per group: the fields the first loads need, preloaded into scalar
// registers at dispatch.
__global__ __launch_bounds__(US_BLOCK) void k_union_score(const int* count_word,
                                                          const uint64_t* bm_in,
                                                          const int* tok_base, int W,
                                                          int tok_stride, StepArgs a) {
  constexpr int US_CHUNK = US_BLOCK / 64;  // bitmap words listed per pass (1 item per thread)
  SKV_TSB(3, 0);
  const int ts = 8;
  SKV_TS(ts, 0);
  const int g = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_in = count_word[g * ST_WORDS];
  const int words_in = (n_in + 63) / 64;
  const uint64_t* __restrict__ bm = bm_in + (size_t)g * H * W;
  const int* __restrict__ tok_in = tok_base + (size_t)g * tok_stride;
  int* __restrict__ tok_out = a.u1_tok + (size_t)g * U1_MAX;
  if (blockIdx.x == 0 && wave == 0) {  // diagnostic: postings the pool ranges walked
    const int nb = (a.nc + a.pool_range - 1) / a.pool_range;
    int sc = 0;
    for (int i = lane; i < nb; i += WAVE) sc += a.pool_scan[g * a.pool_blocks + i];
    sc = wave_sum(sc);
    if (lane == 0) a.status[g * ST_WORDS + ST_SCANNED] = sc;
  }
  if (n_in == 0) {
    if (blockIdx.x == 0 && threadIdx.x == 0) a.status[g * ST_WORDS + ST_U1] = 0;
    SKV_TSE(3);
    return;
  }
  const int span = max(US_CHUNK, (words_in + (int)gridDim.x - 1) / (int)gridDim.x);
  const int w_lo = blockIdx.x * span;
  if (w_lo >= words_in) {
    SKV_TSE(3);
    return;
  }
  const int w_hi = min(words_in, w_lo + span);

  __shared__ int s_red[US_BLOCK / WAVE + 1];
  __shared__ uint64_t s_word[US_CHUNK];
  __shared__ int s_wbase[US_CHUNK + 1];
  __shared__ int s_tok[US_CHUNK * 64];
  auto word = [&](int w) { return bm[w] | bm[W + w] | bm[2 * W + w] | bm[3 * W + w]; };

  // issued together: the member counts of words [0, w_lo) (4 words, 16
  // loads in flight per thread), the first chunk's words (one bitmap word per
  // thread < 4 US_CHUNK) and its input tokens (one per thread)
  const int nw0 = min(US_CHUNK, w_hi - w_lo);
  uint64_t hw = 0;
  if ((int)threadIdx.x < H * nw0) hw = bm[(threadIdx.x / nw0) * W + w_lo + threadIdx.x % nw0];
  const int tok0 = (int)threadIdx.x < 64 * nw0 ? tok_in[64 * w_lo + threadIdx.x] : 0;
  int cnt = 0;
  for (int w = threadIdx.x; w < w_lo; w += 4 * US_BLOCK) {
    uint64_t m[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int ww = w + u * US_BLOCK;
      m[u] = ww < w_lo ? word(ww) : 0ull;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) cnt += __popcll(m[u]);
  }
  if (threadIdx.x < US_CHUNK) s_word[threadIdx.x] = 0;
  cnt = wave_sum(cnt);
  if (lane == 0) s_red[wave] = cnt;
  __syncthreads();
  if (hw) atomicOr(reinterpret_cast<unsigned long long*>(&s_word[threadIdx.x % nw0]), hw);
  int base = 0;
#pragma unroll
  for (int i = 0; i < US_BLOCK / WAVE; ++i) base += s_red[i];
  SKV_TS(ts, 1);

  const QOperand* q = &a.qop[g * QV_COUNT + QV_QS];
  uint32_t b[4][4];
  load_b(q, b);
  const int row = lane & 15, kb = lane >> 4;
  // lane l converts key l % 16 of a tile for head l / 16:
  // 4-bit (2 dq - 15 S) 2^(fx + 4), 8-bit (2 dq - 255 S) 2^fx
  const int hq = lane >> 4;
  const LimbScale ls4(q->fx[hq] + 4, 1), ls8(q->fx[hq], 1);
  const double lc4 = LimbScale::offset(-15 * q->sum[hq], q->fx[hq] + 4);
  const double lc8 = LimbScale::offset(-255 * q->sum[hq], q->fx[hq]);
  for (int c0 = w_lo; c0 < w_hi; c0 += US_CHUNK) {
    const int nw = min(US_CHUNK, w_hi - c0);
    const bool first = c0 == w_lo;
    if (!first) {  // later chunks (long inputs): the union words now
      __syncthreads();
      if (threadIdx.x < US_CHUNK) s_word[threadIdx.x] = (int)threadIdx.x < nw ? word(c0 + threadIdx.x) : 0ull;
    }
    __syncthreads();
    if (threadIdx.x < 64) {  // wave 0: the member base of each word
      const uint64_t m = lane < US_CHUNK ? s_word[lane] : 0ull;
      const int pc = __popcll(m);
      const int inc = wave_incl_scan(pc);
      if (lane < US_CHUNK) s_wbase[lane] = inc - pc;
      if (lane == US_CHUNK - 1) s_wbase[US_CHUNK] = inc;
    }
    __syncthreads();
    const int nloc = s_wbase[US_CHUNK];
    // list the chunk's members: thread t tests bit t % 64 of word t / 64
    {
      const int j = threadIdx.x >> 6, bit = threadIdx.x & 63;
      const uint64_t m = s_word[j];
      if ((m >> bit) & 1ull) {
        const int r = s_wbase[j] + __popcll(m & ((1ull << bit) - 1));
        const int t = first ? tok0 : tok_in[64 * (c0 + j) + bit];
        s_tok[r] = t;
        if (base + r < U1_MAX) tok_out[base + r] = t;
      }
    }
    __syncthreads();
    // scores of the listed members, one 16-key tile per wave at a time
    for (int tile = wave; tile * 16 < nloc; tile += US_BLOCK / WAVE) {
      const int i_in = tile * 16 + row;
      uint32_t hi[4][4] = {}, lo[4][4] = {};
      if (i_in < nloc) {
        const uint8_t* rec = a.keyrec + ((size_t)g * a.rec_rows + s_tok[i_in]) * 256;
        load_code4(rec, kb, hi);
        const uint4 r0 = *reinterpret_cast<const uint4*>(rec + 128 + kb * 32);
        const uint4 r1 = *reinterpret_cast<const uint4*>(rec + 128 + kb * 32 + 16);
        const uint32_t rw[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) expand4t(rw[2 * kc], rw[2 * kc + 1], lo[kc]);
      }
      v4i acc = {0, 0, 0, 0}, acc_lo = {0, 0, 0, 0};
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        acc = mfma_i8(b[kc], hi[kc], acc);
        acc_lo = mfma_i8(b[kc], lo[kc], acc_lo);
      }
      // 8-bit dot = 16 x (code4 dot) + (residual-4 dot), limb by limb
      // (|16 hi + lo| < 2^23 per limb)
      const v4i acc8 = acc * 16 + acc_lo;
      const int i = tile * 16 + row, o = base + i;
      if (i < nloc && o < U1_MAX) {
        const size_t at = ((size_t)g * H + hq) * U1_MAX + o;
        a.s4[at] = (uint16_t)ordered16(bf16_rne(ls4(acc[0], acc[1], acc[2], lc4)));
        a.s8[at] = (uint16_t)ordered16(bf16_rne(ls8(acc8[0], acc8[1], acc8[2], lc8)));
      }
    }
    base += nloc;
    __syncthreads();
  }
  if (w_hi == words_in && threadIdx.x == 0) a.status[g * ST_WORDS + ST_U1] = min(base, U1_MAX);
  SKV_TS(ts, 15);
  SKV_TSE(3);
}

// ============================================================ final top-100
// Per (group, head): the 100 best of U2 (the union of the four heads'
// top-256 over U1) by 8-bit score, written best first (the rank of a member
// is the number of members with a larger (score, -token) key), then the
// head's attention over them merged with its sink/local slices.  U2 is not
// listed: the block reads the U1-indexed 8-bit scores and keeps those whose
// U1 position is set in any head's top-256 bitmap, so the members come out
// in U1 order, which is U2's list order.
constexpr int TOP_KPW = (TOPK + ATTN_WAVES - 1) / ATTN_WAVES;  // selected keys per wave
constexpr int DENSE_PREF = 2;  // sink/local partials prefetched per merge thread

// Bits 8o .. 8o + 7 of the union of 4 bitmap rows of W words (octet o).
__device__ __forceinline__ uint32_t union_octet(const uint64_t* __restrict__ bm, int W, int o) {
  const int w = o >> 3;
  const uint64_t u = bm[w] | bm[W + w] | bm[2 * W + w] | bm[3 * W + w];
  return (uint32_t)(u >> (8 * (o & 7))) & 0xffu;
}

// The packed scores of octet w whose bit in `bits` is set; the rest 0.
__device__ __forceinline__ uint4 keep_octet(uint4 w, uint32_t bits) {
  auto keep = [bits](uint32_t word, int q) {
    const uint32_t b = bits >> (2 * q);
    return word & (((b & 1u) ? 0xffffu : 0u) | ((b & 2u) ? 0xffff0000u : 0u));
  };
  return make_uint4(keep(w.x, 0), keep(w.y, 1), keep(w.z, 2), keep(w.w, 3));
}

// 8-bit scores of U2 members by U1 position (0 elsewhere): a fast_select source.
struct UnionScores {
  static constexpr int PRE = 4;
  const uint16_t* __restrict__ score;
  const uint64_t* __restrict__ bm;  // 4 rows of W words
  int W;
  __device__ uint32_t at(int i) const {
    const uint32_t sv = score[i];
    return (union_octet(bm, W, i >> 3) >> (i & 7)) & 1u ? sv : 0u;
  }
  __device__ uint4 oct(int o) const {
    return keep_octet(reinterpret_cast<const uint4*>(score)[o], union_octet(bm, W, o));
  }
};

// The leading arguments repeat the fields of a that the first loads need
// (preloaded into scalar registers at dispatch).  PAGED: the selected records
// are read through the page table.
template <bool PAGED>
__global__ __launch_bounds__(SEL_BLOCK) void k_top100(const int* status, const uint16_t* s8,
                                                      const int* u1_tok, const uint64_t* bm_u2,
                                                      int W, const uint16_t* q_in,
                                                      const float* dense_part, int dense_slices,
                                                      int exact_select, StepArgs a) {
  SKV_TSB(9, 0);
  SKV_TS(13, 0);
  const int g = blockIdx.x / H, h = blockIdx.x % H, j = g * H + h;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __shared__ SelectScratch s;
  __shared__ __align__(16) uint64_t s_key[TOPK];
  __shared__ __align__(16) uint32_t s_pos[TOPK];  // U1 positions (atomic-order paths)
  __shared__ int s_cnt;
  __shared__ int s_u2[SEL_WAVES];  // U2 members per wave's octets
  __shared__ AttnScratch att;
  const int n = status[g * ST_WORDS + ST_U1];
  const uint16_t* sc = s8 + (size_t)j * U1_MAX;
  const int* tok = u1_tok + (size_t)g * U1_MAX;
  const uint64_t* bmg = bm_u2 + (size_t)g * H * W;
  auto id = [tok](int i) { return (uint32_t)tok[i]; };
  extern __shared__ __align__(16) unsigned char dyn[];
  // this thread's octet of U1 positions: union bits (n <= U1_MAX <= 8 x SEL_BLOCK)
  const uint32_t ubits = 8 * (int)threadIdx.x < n ? union_octet(bmg, W, threadIdx.x) : 0u;
  {
    const int c = wave_sum(__popc(ubits));
    if (lane == 0) s_u2[wave] = c;  // read after a later barrier
  }
  // loads independent of the selection, issued first: the query and the
  // sink/local partials (consumed only by the final merge)
  float q[4];
  {
    const uint2 qw = *reinterpret_cast<const uint2*>(q_in + j * D + 4 * lane);
    q[0] = bf16_f32(qw.x & 0xffff); q[1] = bf16_f32(qw.x >> 16);
    q[2] = bf16_f32(qw.y & 0xffff); q[3] = bf16_f32(qw.y >> 16);
  }
  const int d = threadIdx.x & (D - 1);
  const float* parts = dense_part + (size_t)j * dense_slices * (D + 2);
  float pm[DENSE_PREF], pl[DENSE_PREF], po[DENSE_PREF];
#pragma unroll
  for (int r = 0; r < DENSE_PREF; ++r) {
    const bool has = r < dense_slices && (int)threadIdx.x < D;
    pm[r] = has ? parts[r * (D + 2) + D] : -INFINITY;
    pl[r] = has ? parts[r * (D + 2) + D + 1] : 0.f;
    po[r] = has ? parts[r * (D + 2) + d] : 0.f;
  }
  if (threadIdx.x == 0) s_cnt = 0;
  bool done = false, listed = false;  // listed: s_key is in U2 list order
  if (exact_select == 0) {  // n <= U1_MAX <= OCT_ITEMS: scores and IDs in registers
    const uint4 w = keep_octet(load_oct(sc, n), ubits);
    uint4 t0 = make_uint4(0, 0, 0, 0), t1 = t0;
    if (8 * (int)threadIdx.x < n) {  // rows hold U1_MAX (a multiple of 8) entries
      t0 = reinterpret_cast<const uint4*>(tok)[2 * threadIdx.x];
      t1 = reinterpret_cast<const uint4*>(tok)[2 * threadIdx.x + 1];
    }
    // the octet's tokens in LDS for the tie ranking (ordered before their
    // reads by the selection's first barrier)
    __shared__ __align__(16) uint32_t s_tok[U1_MAX];
    if (8 * (int)threadIdx.x < U1_MAX) {
      reinterpret_cast<uint4*>(s_tok)[2 * threadIdx.x] = t0;
      reinterpret_cast<uint4*>(s_tok)[2 * threadIdx.x + 1] = t1;
    }
    const OctResult r = oct_select<false, false>(
        w, TOPK, [&](int i) { return s_tok[i]; }, *reinterpret_cast<FastScratch*>(dyn), 13);
    if (r.ok) {
      SKV_TS(13, 6);
      // members in list order (deterministic, so the attention sums are too)
      int nm;
      const int base = block_excl_scan(__popc(r.mine), s.scan, &nm);
      const u32x4 wv = {w.x, w.y, w.z, w.w};
      const u32x4 ta = {t0.x, t0.y, t0.z, t0.w}, tb = {t1.x, t1.y, t1.z, t1.w};
      int slot = base;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (!((r.mine >> e) & 1u)) continue;
        const uint32_t t = e < 4 ? ta[e & 3] : tb[e & 3];
        if (slot < TOPK) s_key[slot] = ((uint64_t)oct_half(wv, e) << 20) | (0xfffffu - t);
        ++slot;
      }
      if (threadIdx.x == 0) s_cnt = nm;
      done = listed = true;
    }
  }
  const UnionScores src{sc, bmg, W};
  if (!done && exact_select != 1) {
    FastScratch& fs = *reinterpret_cast<FastScratch*>(dyn);
    const FastResult r = fast_select(src, n, TOPK, id, fs, exact_select == 2, 13);
    if (r.ok) {
      SKV_TS(13, 6);
      for (int c = threadIdx.x; c < r.ncand; c += SEL_BLOCK) {
        const uint64_t key = fs.cand[c];
        if (fs_member(r, key, id)) {
          const uint32_t t = id(cand_pos(key));
          const int slot = atomicAdd(&s_cnt, 1);
          if (slot < TOPK) {
            s_key[slot] = ((uint64_t)cand_ord(key) << 20) | (0xfffffu - t);
            s_pos[slot] = (uint32_t)cand_pos(key);
          }
        }
      }
      done = true;
    } else {
      __syncthreads();
      if (threadIdx.x == 0) atomicOr(&a.status[g * ST_WORDS + ST_FULLSEL], FS_TOP100);
    }
  }
  if (!done) {
    __shared__ __align__(16) uint16_t so[U1_MAX];
    if (8 * (int)threadIdx.x < n)  // n <= U1_MAX <= 8 x SEL_BLOCK: one octet per thread
      reinterpret_cast<uint4*>(so)[threadIdx.x] = keep_octet(load_oct(sc, n), ubits);
    __syncthreads();
    const Selection sel = block_select(so, n, TOPK, id, s);
    for_scores(so, n, [&](int i, uint32_t o) {
      if (!o || !(sel.all || o >= sel.v)) return;
      const uint32_t t = tok[i];
      if (sel.member(o, t)) {
        const int slot = atomicAdd(&s_cnt, 1);
        if (slot < TOPK) {
          s_key[slot] = ((uint64_t)o << 20) | (0xfffffu - t);
          s_pos[slot] = (uint32_t)i;
        }
      }
    });
  }
  __syncthreads();
  SKV_TS(13, 7);
  const int m = min(s_cnt, TOPK);
  if (!listed) {  // block-uniform
    // members listed in atomic order: put them in U1 (= U2 list) order, as the
    // register path lists them, so that the attention sums run in the same
    // order on every selection path (bit-identical, reproducible outputs)
    uint64_t key = 0;
    int rank = 0;
    if ((int)threadIdx.x < m) {
      key = s_key[threadIdx.x];
      rank = count_below(s_pos, m, s_pos[threadIdx.x]);  // positions are distinct
    }
    __syncthreads();
    if ((int)threadIdx.x < m) s_key[rank] = key;
    __syncthreads();
  }
  // attention over the members: wave w takes list entries w + 16 b; the
  // record loads are issued before the output list is ranked
  int tk = -1;
  if (lane < TOP_KPW) {
    const int i = wave + ATTN_WAVES * lane;
    if (i < m) tk = (int)(0xfffffu - (uint32_t)(s_key[i] & 0xfffffu));
  }
  const AttnLoads<TOP_KPW> L =
      attend_load<TOP_KPW>(kv_base<PAGED>(a, g), kv_lane_row<PAGED>(a, g, tk));
  SKV_TSB(9, 1);  // trace builds: the top-100 record gather is issued
  // the output list, best first (member keys are distinct)
  int* out = a.top + j * TOPK;
  if ((int)threadIdx.x < m) {
    const uint64_t key = s_key[threadIdx.x];
    out[count_above64(s_key, m, key)] = (int)(0xfffffu - (uint32_t)(key & 0xfffffu));
  } else if ((int)threadIdx.x < TOPK) {
    out[threadIdx.x] = -1;
  }
  SKV_TS(13, 8);
  SKV_WAIT(L.kw[TOP_KPW - 1] ^ L.vw[TOP_KPW - 1]);  // trace builds: ... and has arrived
  SKV_TSW(9, 2);
  float mw, lw, ow[4];
  attend_math<TOP_KPW>(L, q, mw, lw, ow);
  stash_wave(att, mw, lw, ow);
  __syncthreads();
  SKV_TS(13, 9);
  if (h == 0 && threadIdx.x == 0) {  // |U2|
    int u2 = 0;
#pragma unroll
    for (int i = 0; i < SEL_WAVES; ++i) u2 += s_u2[i];
    a.status[g * ST_WORDS + ST_U2] = u2;
  }
  // merge with the sink/local slices
  if (threadIdx.x < D) {
    float M, Ls, O;
    merge_waves(att, d, M, Ls, O);
    float Mt = M;
#pragma unroll
    for (int r = 0; r < DENSE_PREF; ++r) Mt = fmaxf(Mt, pm[r]);
    for (int r = DENSE_PREF; r < dense_slices; ++r) Mt = fmaxf(Mt, parts[r * (D + 2) + D]);
    float Lt = 0.f, Ot = 0.f;
    if (M != -INFINITY) {
      const float sc0 = __expf(M - Mt);
      Lt = Ls * sc0;
      Ot = O * sc0;
    }
#pragma unroll
    for (int r = 0; r < DENSE_PREF; ++r) {
      if (pm[r] == -INFINITY) continue;
      const float f = __expf(pm[r] - Mt);
      Lt += pl[r] * f;
      Ot += po[r] * f;
    }
    for (int r = DENSE_PREF; r < dense_slices; ++r) {
      const float mr = parts[r * (D + 2) + D];
      if (mr == -INFINITY) continue;
      const float f = __expf(mr - Mt);
      Lt += parts[r * (D + 2) + D + 1] * f;
      Ot += parts[r * (D + 2) + d] * f;
    }
    const uint16_t ob = (uint16_t)bf16_rne(Ot / Lt);
    a.out[j * D + d] = ob;
    a.out_tiles[((size_t)(g * 32 + h) * H + h) * D + d] = ob;
  }
  SKV_TS(13, 15);
  SKV_TSE(9);
}

// ============================================================ launcher
const char* const kKernelNames[N_STEP_KERNELS] = {
    "front", "select", "pool", "top1600", "union_score", "top256", "top100_sdpa"};

// The select instance for the centroid count: rows of up to 2 or 4 x
// OCT_ITEMS centroids selected in registers, every other count by the
// one-octet instance (its register path, tile maxima or sampled cuts).
using SelectFn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*, int, int, int,
                          StepArgs);
static SelectFn select_kernel(const StepArgs& a) {
  const int no = a.exact_select != 0 || a.nc <= OCT_ITEMS ? 1
                 : a.nc <= 2 * OCT_ITEMS                  ? 2
                 : a.nc <= 4 * OCT_ITEMS                  ? 4
                                                          : 1;
  if (a.kv_table) return no == 2 ? k_select<true, 2> : no == 4 ? k_select<true, 4> : k_select<true, 1>;
  return no == 2 ? k_select<false, 2> : no == 4 ? k_select<false, 4> : k_select<false, 1>;
}

static void launch_topk(const TopkArgs& t, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL(t.regs2 ? k_topk<true> : k_topk<false>, dim3(G * H), dim3(SEL_BLOCK), lds,
                     st, t.status + t.count_slot,
                     t.scores, t.stride, t.exact_select, t.tile_max, t.words, t);
}

// Launch every kernel of one decode step on stream st.  If ev is non-NULL
// (N_STEP_KERNELS + 1 events), ev[i] is recorded before kernel i and
// ev[N_STEP_KERNELS] after the last one.
void launch_kernel(const StepArgs& a, const StepWork& w, hipStream_t st, int k) {
  const int tiles_blocks = std::min((a.nc + FR_CENTROIDS - 1) / FR_CENTROIDS, FR_MAX_BLOCKS);
  const size_t bm_lds = (size_t)PL_BM_WORDS * 4;
  switch (k) {
    case 0: {
      const bool loop = tiles_blocks * FR_CENTROIDS < a.nc, app = a.app_n > 0;
      const auto fn = loop ? (app ? k_front<true, true> : k_front<true, false>)
                           : (app ? k_front<false, true> : k_front<false, false>);
      hipLaunchKernelGGL(fn, dim3(tiles_blocks, G), dim3(FR_BLOCK), 0, st, a.q, a);
      break;
    }
    case 1:
      hipLaunchKernelGGL(select_kernel(a),
                         dim3(G * H * (1 + a.dense_slices) + 2 * G), dim3(SEL_BLOCK),
                         w.select_lds, st, (const uint16_t*)a.lower, (const uint16_t*)a.upper,
                         (const uint16_t*)a.fine_ord, a.nc, a.exact_select, a.dense_slices, a);
      break;
    case 2:
      hipLaunchKernelGGL(k_pool, dim3((a.nc + a.pool_range - 1) / a.pool_range, G), dim3(PL_BLOCK),
                         bm_lds, st, (const uint32_t*)a.selbm, (const int*)a.csr_off,
                         (const uint16_t*)a.upper, (const uint32_t*)a.thr, (const QOperand*)a.qop,
                         (const unsigned*)a.pool_epoch, a.nc, a.pool_range, a);
      break;
    case 3:
      launch_topk(w.top_u1, w.top_u1_lds, st);
      break;
    case 4:
      hipLaunchKernelGGL(k_union_score, dim3(US_GRID, G), dim3(US_BLOCK), 0, st,
                         (const int*)a.status + ST_POOL, (const uint64_t*)a.bm_u1,
                         (const int*)a.pool_tok, a.words_u1, a.cap, a);
      break;
    case 5:
      launch_topk(w.top_u2, w.top_u2_lds, st);
      break;
    case 6:
      hipLaunchKernelGGL(a.kv_table ? k_top100<true> : k_top100<false>, dim3(G * H),
                         dim3(SEL_BLOCK), sizeof(FastScratch), st,
                         (const int*)a.status, (const uint16_t*)a.s8, (const int*)a.u1_tok,
                         (const uint64_t*)a.bm_u2, a.words_u2, a.q, (const float*)a.dense_part,
                         a.dense_slices, a.exact_select, a);
      break;
    default:
      break;
  }
}

hipError_t step_kernel_lds(const StepArgs& a, const StepWork& w, int k, size_t* static_bytes,
                           size_t* dynamic_bytes) {
  const void* fn = nullptr;
  size_t dyn = 0;
  switch (k) {
    case 0: fn = reinterpret_cast<const void*>(&k_front<true, true>); break;
    case 1:
      fn = reinterpret_cast<const void*>(select_kernel(a));
      dyn = w.select_lds;
      break;
    case 2: fn = reinterpret_cast<const void*>(&k_pool); dyn = (size_t)PL_BM_WORDS * 4; break;
    case 3: fn = reinterpret_cast<const void*>(&k_topk<true>); dyn = w.top_u1_lds; break;
    case 4: fn = reinterpret_cast<const void*>(&k_union_score); break;
    case 5: fn = reinterpret_cast<const void*>(&k_topk<false>); dyn = w.top_u2_lds; break;
    case 6:
      fn = a.kv_table ? reinterpret_cast<const void*>(&k_top100<true>)
                      : reinterpret_cast<const void*>(&k_top100<false>);
      dyn = sizeof(FastScratch);
      break;
    default: return hipErrorInvalidValue;
  }
  hipFuncAttributes attr;
  const hipError_t e = hipFuncGetAttributes(&attr, fn);
  if (e != hipSuccess) return e;
  size_t st = attr.sharedSizeBytes;
  if (k == 1) {  // the one-octet instance too (the selection-path test modes launch it)
    hipFuncAttributes a1;
    const hipError_t e1 = hipFuncGetAttributes(
        &a1, a.kv_table ? reinterpret_cast<const void*>(&k_select<true, 1>)
                        : reinterpret_cast<const void*>(&k_select<false, 1>));
    if (e1 != hipSuccess) return e1;
    st = std::max(st, (size_t)a1.sharedSizeBytes);
  }
  if (k == 3) {  // both top-k instances
    hipFuncAttributes attr2;
    const hipError_t e2 = hipFuncGetAttributes(&attr2, reinterpret_cast<const void*>(&k_topk<false>));
    if (e2 != hipSuccess) return e2;
    st = std::max(st, (size_t)attr2.sharedSizeBytes);
  }
  if (k == 0) {  // every front variant
    for (const void* f : {reinterpret_cast<const void*>(&k_front<true, false>),
                          reinterpret_cast<const void*>(&k_front<false, true>),
                          reinterpret_cast<const void*>(&k_front<false, false>)}) {
      hipFuncAttributes attr2;
      const hipError_t e2 = hipFuncGetAttributes(&attr2, f);
      if (e2 != hipSuccess) return e2;
      st = std::max(st, (size_t)attr2.sharedSizeBytes);
    }
  }
  *static_bytes = st;
  *dynamic_bytes = dyn;
  return hipSuccess;
}

void launch_step(const StepArgs& a, const StepWork& w, hipStream_t st, hipEvent_t* ev) {
  for (int k = 0; k < N_STEP_KERNELS; ++k) {
    if (ev) (void)hipEventRecord(ev[k], st);
    launch_kernel(a, w, st, k);
  }
  if (ev) (void)hipEventRecord(ev[N_STEP_KERNELS], st);
}

}  // namespace skv

#ifdef SKV_TRACE
extern "C" int skv_trace_read(unsigned long long* out) {
  return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(skv::g_skv_trace), sizeof(skv::g_skv_trace));
}
extern "C" int skv_trace_blocks(unsigned long long* out) {
  return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(skv::g_skv_trace_blk),
                                  sizeof(skv::g_skv_trace_blk));
}
#endif
