// Device helpers shared by the SeoulKV4 gfx950 kernels.
//
// Score arithmetic (exact, order independent):
//   a BF16 query vector x[256] is held as integers X[d] = trunc(x[d] * 2^-fx)
//   with |X| < 2^22 (fx = exmax - 14, exmax the largest element exponent); a
//   key score is D = sum_d X[d] * c[d] for the integer key code c, computed
//   exactly, rounded once to FP32 (RNE) after scaling by 2^(fx + e), then the
//   stage's FP32 operations (RNE, no contraction), then BF16 (RNE).
//   X is split into three signed 8-bit limbs so the dot runs on the int8
//   matrix cores: D = L0 + 256 L1 + 65536 L2, each limb dot exact in int32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "skv_trace.h"

namespace skv {

constexpr int G = 4;          // KV heads (index cells)
constexpr int H = 4;          // query heads per KV head
constexpr int D = 256;        // head dimension
constexpr int TOPK = 100;
constexpr int M15 = 1600;     // ranks of the Stage-1.5 frontier entering the union
constexpr int M16 = 256;      // Stage-1.6 survivors per head
constexpr int U1_MAX = H * M15;
constexpr int U2_MAX = H * M16;
constexpr int FX_HEADROOM = 14;
constexpr int WAVE = 64;

// Record index of token tok of KV group g in paged FP8 [V || K] records (the
// record is at pool + 512 * index): token tok lies at slot tok mod 2^shift of
// logical page tok >> shift, and a physical page holds the G groups' slots
// one group after another.  Contiguous records are simply g * rows + tok.
__host__ __device__ __forceinline__ uint32_t kv_row_paged(const int* table, int shift, int g,
                                                          int tok) {
  return (((uint32_t)table[tok >> shift] * G + (uint32_t)g) << shift) |
         ((uint32_t)tok & ((1u << shift) - 1u));
}

// Query operand variants.
enum { QV_RAW = 0, QV_Q15 = 1, QV_QS = 2, QV_COUNT = 3 };

// Per (group, variant) query operand block, written by the query-prep kernel.
struct QOperand {
  // int8 matrix-core operand image: [chunk kc][lane][16 bytes]; lane l holds
  // row l%16 (head (l%16)/4, limb (l%16)%4, limb 3 = 0) for dims
  // (l/16)*64 + kc*16 + [0,16).
  uint32_t bimg[4][WAVE][4];
  int64_t sum[H];   // S_h = sum_d X_h[d]
  int32_t fx[H];    // scale exponent of X_h
  float norm[H];    // ||q_h|| * lambda (RAW variant only)
  int32_t X[H][D];  // the fixed-point integers (diagnostics / tests)
};

__host__ __device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }

__device__ __forceinline__ uint32_t ordered16(uint32_t b) {
  return (b & 0x8000u) ? (~b & 0xffffu) : (b ^ 0x8000u);
}

__device__ __forceinline__ uint32_t bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t nan = ((u >> 16) | 0x40u) & 0xffffu, r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (u & 0x7fffffffu) > 0x7f800000u ? nan : r;  // a select, no branch
}

__device__ __forceinline__ float bf16_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Four FP8 e4m3 values -> FP32 with the gfx950 converter (OCP e4m3fn; exact).
__device__ __forceinline__ void fp8x4_to_f32(uint32_t w, float f[4]) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  f[0] = lo[0]; f[1] = lo[1]; f[2] = hi[0]; f[3] = hi[1];
}

// RNE_f32(Dv * 2^e) for |Dv| < 2^53.
__device__ __forceinline__ float scaled_f32(int64_t Dv, int e) {
  return __double2float_rn(ldexp((double)Dv, e));
}

// scaled_f32(2^m dq + off, e) for the dot dq = x0 + 2^8 x1 + 2^16 x2 of a
// matrix core's limb sums (|x_i| < 2^24, |off| < 2^40) without 64-bit
// integer arithmetic: x2 2^(e+m+16) + x1 2^(e+m+8) + x0 2^(e+m) + off 2^e
// in double FMAs, every partial sum exact (a multiple of 2^e under 2^53 of
// them), so the one rounding is the final conversion, as in scaled_f32.
struct LimbScale {
  double p0, p1, p2;  // 2^(e+m), 2^(e+m+8), 2^(e+m+16)
  __device__ LimbScale(int e, int m)
      : p0(ldexp(1.0, e + m)), p1(ldexp(1.0, e + m + 8)), p2(ldexp(1.0, e + m + 16)) {}
  // the offset term off 2^e
  __device__ static double offset(int64_t off, int e) { return ldexp((double)off, e); }
  __device__ float operator()(int x0, int x1, int x2, double c) const {
    return __double2float_rn(
        __fma_rn((double)x2, p2, __fma_rn((double)x1, p1, __fma_rn((double)x0, p0, c))));
  }
};

// RNE_f32(sqrt(N) * 2^fx) by integer arithmetic: the root of N << 2k
// (largest k keeping it below 2^62) carries >= 26 significant bits, a sticky
// bit records an inexact root, and 24 bits are kept with round-half-even.
__host__ __device__ inline float sqrt_rne_scaled(unsigned long long N, int fx) {
  if (N == 0) return 0.f;
  const int bits = 64 - __builtin_clzll(N);
  const int k = (62 - bits) / 2;
  const unsigned long long M = N << (2 * k);
  unsigned long long s = (unsigned long long)sqrt((double)M);
  while (s * s > M) --s;
  while ((s + 1) * (s + 1) <= M) ++s;
  const bool sticky = s * s != M;
  const int sb = 64 - __builtin_clzll(s);
  const int drop = sb - 24;
  unsigned long long qv = s >> drop;
  const unsigned long long rem = s & ((1ull << drop) - 1), half = 1ull << (drop - 1);
  if (rem > half || (rem == half && (sticky || (qv & 1)))) ++qv;
  return (float)ldexp((double)qv, drop - k + fx);
}

// FP8 e4m3fn (OCP: bias 7, no infinities, S.1111.111 = NaN) -> FP32, exact.
__host__ __device__ inline float fp8_e4m3_to_f32(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  if (e == 0) {
    const float v = (float)m * 0.001953125f;  // m * 2^-9
    return sign ? -v : v;
  }
  if (e == 15 && m == 7) return u2f(0x7fc00000u | sign);
  return u2f(sign | ((e + 120u) << 23) | (m << 20));
}

// FP32 -> FP8 e4m3fn, round to nearest even; magnitudes above 464 (the
// midpoint past 448) and NaN/Inf become NaN (0x7f | sign), as torch's
// float8_e4m3fn cast does.
__host__ __device__ inline uint32_t f32_to_fp8_e4m3(float f) {
  uint32_t u = f2u(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  u &= 0x7fffffffu;
  if (u > 0x7f800000u || u == 0x7f800000u) return sign | 0x7fu;
  if (u < 0x3c800000u) {  // below 2^-6: subnormal grid of 2^-9
    const float scaled = u2f(u) * 512.0f;  // exact
    uint32_t m = (uint32_t)scaled;
    const float frac = scaled - (float)m;
    if (frac > 0.5f || (frac == 0.5f && (m & 1u))) ++m;
    return sign | m;  // m == 8 is the smallest normal (0x08)
  }
  const uint32_t r = u + 0x7ffffu + ((u >> 20) & 1u);
  const int e = (int)(r >> 23) - 127 + 7;
  const uint32_t m = (r >> 20) & 7u;
  if (e > 15 || (e == 15 && m == 7)) return sign | 0x7fu;
  return sign | ((uint32_t)e << 3) | m;
}

// Four BF16 values (packed in w) -> four FP8 e4m3fn bytes (torch's cast).
// The gfx950 converter (v_cvt_pk_fp8_f32, round to nearest even) gives
// torch's byte for every finite and infinite BF16 input (checked on all
// 65536 patterns); a NaN input becomes torch's NaN byte (sign | 0x7f).
__device__ __forceinline__ uint32_t bf16x4_to_fp8(uint2 w) {
  const float f0 = bf16_f32(w.x & 0xffffu), f1 = bf16_f32(w.x >> 16);
  const float f2 = bf16_f32(w.y & 0xffffu), f3 = bf16_f32(w.y >> 16);
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(f0, f1, 0, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(f2, f3, r, true);
  uint32_t out = (uint32_t)r;
  // BF16 NaN: exponent all ones, mantissa nonzero (rare: one test per lane)
  const uint32_t nan_lo = ((w.x & 0x7fffu) > 0x7f80u) | (((w.x >> 16) & 0x7fffu) > 0x7f80u) << 1 |
                          ((w.y & 0x7fffu) > 0x7f80u) << 2 | (((w.y >> 16) & 0x7fffu) > 0x7f80u) << 3;
  if (nan_lo) {
    const uint32_t hv[4] = {w.x & 0xffffu, w.x >> 16, w.y & 0xffffu, w.y >> 16};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if ((nan_lo >> e) & 1u)
        out = (out & ~(0xffu << (8 * e))) | ((((hv[e] >> 8) & 0x80u) | 0x7fu) << (8 * e));
  }
  return out;
}

// ---------------------------------------------------------------- wave ops
// Cross-lane scans and reductions on the DPP data paths (row shifts within
// 16-lane rows, then row broadcasts 15 and 31 across rows), the wave64 scan
// pattern of AMD's GCN cross-lane operations guide.  Every lane of the wave
// must be active.  update_dpp(old, v, ctrl, row_mask, bank_mask, zero_fill)
// returns v moved by ctrl; lanes without a source take old (or 0).
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

// Wave total, uniform across lanes.
__device__ __forceinline__ int wave_sum(int v) {
  return __builtin_amdgcn_readlane(wave_incl_scan(v), 63);
}

// Float wave total (tree order fixed by the DPP pattern), uniform across lanes.
#define SKV_DPP_ADDF(v, ctrl, rows, zero) \
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, rows, 0xf, zero))
__device__ __forceinline__ float wave_sum_f(float v) {
  SKV_DPP_ADDF(v, 0x111, 0xf, true);   // row_shr:1
  SKV_DPP_ADDF(v, 0x112, 0xf, true);   // row_shr:2
  SKV_DPP_ADDF(v, 0x114, 0xf, true);   // row_shr:4
  SKV_DPP_ADDF(v, 0x118, 0xf, true);   // row_shr:8
  SKV_DPP_ADDF(v, 0x142, 0xa, false);  // row_bcast:15
  SKV_DPP_ADDF(v, 0x143, 0xc, false);  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
#undef SKV_DPP_ADDF

__device__ __forceinline__ int wave_max(int v) {
  constexpr int LO = (int)0x80000000;
  v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0x111, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0x112, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0x114, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0x118, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0x142, 0xa, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0x143, 0xc, 0xf, false));
  return __builtin_amdgcn_readlane(v, 63);
}

// Unsigned inclusive wave scan (sums modulo 2^32, the same DPP pattern).
__device__ __forceinline__ unsigned wave_incl_scan_u(unsigned v) {
  v +=(unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true);
  v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true);
  v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, true);
  v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, true);
  v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);
  v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);
  return v;
}

// Exclusive block scan of one value per thread; returns the exclusive prefix
// and stores the block total in *total.  scratch: >= blockDim/64 + 1 words.
// T = int, or unsigned for packed fields whose sums may pass 2^31.
template <typename T>
__device__ __forceinline__ T block_excl_scan_t(T v, T* scratch, T* total) {
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const int nw = (blockDim.x + WAVE - 1) / WAVE;
  auto scan = [](T x) -> T {
    if constexpr (sizeof(T) == 4 && T(-1) > T(0)) return wave_incl_scan_u(x);
    else return wave_incl_scan(x);
  };
  T inc = scan(v);
  if (lane == WAVE - 1) scratch[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    T w = lane < nw ? scratch[lane] : T(0);
    T winc = scan(w);
    if (lane < nw) scratch[lane] = winc - w;
    if (lane == nw - 1) scratch[nw] = winc;
  }
  __syncthreads();
  T res = inc - v + scratch[wave];
  *total = scratch[nw];
  __syncthreads();
  return res;
}

__device__ __forceinline__ int block_excl_scan(int v, int* scratch, int* total) {
  return block_excl_scan_t<int>(v, scratch, total);
}

// ------------------------------------------------------- code expansion
// 16 little-endian 2-bit codes of w in the byte-transposed order of the
// query images: word j byte m = code 4m + j, i.e. bits 2j.. of every byte;
// one shift and one mask per word.
__device__ __forceinline__ void expand2t(uint32_t w, uint32_t out[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) out[j] = (w >> (2 * j)) & 0x03030303u;
}
// 16 little-endian 4-bit codes (8 in w0, 8 in w1) in the same order: word j
// = nibbles j, 4 + j of w0 and j, 4 + j of w1 (codes j, 4 + j, 8 + j,
// 12 + j); one byte permute gathers the two masked halves.
__device__ __forceinline__ void expand4t(uint32_t w0, uint32_t w1, uint32_t out[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t a = (w0 >> (4 * j)) & 0x000f000fu, b = (w1 >> (4 * j)) & 0x000f000fu;
    out[j] = __builtin_amdgcn_perm(b, a, 0x06040200u);  // a.b0, a.b2, b.b0, b.b2
  }
}

typedef int v4i __attribute__((ext_vector_type(4)));

// One 16 x 16 x 64 int8 matrix-core step, C[m][n] += sum_k A[m][k] B[k][n]:
// lane l supplies row (A) / column (B) l % 16 over k = 16 (l / 16) .. + 15
// and receives C[4 (l / 16) + i][l % 16] in register i.  The scorers pass
// the query image as A (rows: head x limb) and 16 keys as B, so lane l gets
// the limb sums of key l % 16 for head l / 16.
__device__ __forceinline__ v4i mfma_i8(const uint32_t a[4], const uint32_t b[4], v4i c) {
  v4i av = {(int)a[0], (int)a[1], (int)a[2], (int)a[3]};
  v4i bv = {(int)b[0], (int)b[1], (int)b[2], (int)b[3]};
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, c, 0, 0, 0);
}


}  // namespace skv
