// Dense FP8 decode over every key of the cache (interface in skv_dense.h).
//
// k_dense: block (b, g) covers DN_WAVES x iters 16-key tiles of KV group g.
// Per tile, one wave scores its 16 keys for the group's 4 query heads with
// two FP8 matrix-core steps (16 x 16 x 128): the A operand is the K half of
// the records as stored, the B operand holds each head's BF16 query split
// into four FP8 terms (column 4h + s carries term s, weight 2^-4s), so the
// products are those of the BF16 query and the FP8 keys.  The V half is
// accumulated on the vector ALUs in FP32: lane (row kb, column c) owns keys
// 4kb..4kb+3 of every tile and dims 16c..16c+15 of all 4 heads, with its own
// online-softmax state per row; rows, waves and blocks are merged by the
// usual max/sum rescaling.  k_dense_merge folds the per-block partials of
// each query head into the BF16 output.
#include <mutex>

#include "../../include/seoulkv4_hip.h"
#include "skv_dense.h"
#include "skv_device.h"

namespace skv {

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));

constexpr float DN_LOG2E = 1.4426950408889634f;
// A row's running max moves only when a logit exceeds it by more than this
// (log2 units), so the accumulators are rescaled rarely; p <= 2^DN_TAU.
constexpr float DN_TAU = 8.f;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// the value held by lane 4h of this lane's 16-lane row (row_newbcast)
template <int HH>
__device__ __forceinline__ float head_bcast(float v) {
  return dpp_f<0x150 + 4 * HH>(v);
}

__device__ __forceinline__ uint32_t f32_fp8_byte(float x) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x, 0.f, 0, false) & 0xffu;
}
__device__ __forceinline__ float fp8_byte_f32(uint32_t b) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  const v2f f = __builtin_amdgcn_cvt_pk_f32_fp8((int)b, false);
  return f[0];
}

// B operand of the score step.  Lane l: column c = l % 16 = 4h + s, key
// block kb = l / 16; MFMA m covers dims m*128 + kb*32 + [0, 32).  Term s of
// head h is FP8(r_s) with r_0 = q_h * 2^E_h and r_{s+1} = (r_s - FP8(r_s)) * 16,
// where 2^E_h scales max|q_h| into [128, 256).  zc = 2^(-4s - E_h) * log2(e) / 16
// turns the column's dot product into its share of the logit in log2 units.
__device__ __forceinline__ void dense_query(const uint16_t* __restrict__ qg, int lane, v8i bq[2],
                                            float& zc) {
  const int col = lane & 15, h = col >> 2, s = col & 3, kb = lane >> 4;
  const uint16_t* qh = qg + h * D + kb * 32;
  uint32_t w[2][16];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 u = *reinterpret_cast<const uint4*>(qh + m * 128 + 8 * i);
      w[m][4 * i] = u.x; w[m][4 * i + 1] = u.y; w[m][4 * i + 2] = u.z; w[m][4 * i + 3] = u.w;
    }
  float mx = 0.f;
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 16; ++i)
      mx = fmaxf(mx, fmaxf(fabsf(bf16_f32(w[m][i] & 0xffffu)), fabsf(bf16_f32(w[m][i] >> 16))));
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  int E = 0;
  if (mx > 0.f) {
    int e;
    (void)frexpf(mx, &e);
    E = 8 - e;
  }
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    int packed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = 4 * i + j;
        const uint32_t bits = (k & 1) ? (w[m][k >> 1] >> 16) : (w[m][k >> 1] & 0xffffu);
        float x = ldexpf(bf16_f32(bits), E);
        uint32_t t = f32_fp8_byte(x);
#pragma unroll
        for (int r = 1; r < 4; ++r) {  // term r, kept by the lanes with s >= r
          x = (x - fp8_byte_f32(t)) * 16.f;
          const uint32_t u = f32_fp8_byte(x);
          t = r <= s ? u : t;
        }
        word |= t << (8 * j);
      }
      packed[i] = (int)word;
    }
    bq[m] = v8i{packed[0], packed[1], packed[2], packed[3], packed[4], packed[5], packed[6], packed[7]};
  }
  zc = ldexpf(DN_LOG2E / 16.f, -4 * s - E);
}

struct DnTile {
  uint4 k[4];  // A operand: K dims kb*32 + [0, 32) and 128 + kb*32 + [0, 32) of key row l % 16
  uint4 v[4];  // V dims 16c..16c+15 of keys 4kb + r
};

__device__ __forceinline__ DnTile dn_load(const uint8_t* __restrict__ kv, int T, int t0, int lane) {
  const int row = lane & 15, kb = lane >> 4;
  DnTile x;
  const uint8_t* kr = kv + (size_t)min(t0 + row, T - 1) * 512 + 256 + kb * 32;
  x.k[0] = *reinterpret_cast<const uint4*>(kr);
  x.k[1] = *reinterpret_cast<const uint4*>(kr + 16);
  x.k[2] = *reinterpret_cast<const uint4*>(kr + 128);
  x.k[3] = *reinterpret_cast<const uint4*>(kr + 144);
#pragma unroll
  for (int r = 0; r < 4; ++r)
    x.v[r] = *reinterpret_cast<const uint4*>(kv + (size_t)min(t0 + 4 * kb + r, T - 1) * 512 + 16 * row);
  return x;
}

// The same tile from paged records: tile points at the record of its first
// key t0; a page holds a power-of-two number (>= DN_TILE) of consecutive
// tokens, so the 16 keys of an aligned tile are consecutive records of one
// page; last = T - 1 - t0 clamps the rows past the context.
__device__ __forceinline__ DnTile dn_load_paged(const uint8_t* __restrict__ tile, int last,
                                                int lane) {
  const int row = lane & 15, kb = lane >> 4;
  DnTile x;
  const uint8_t* kr = tile + (size_t)min(row, last) * 512 + 256 + kb * 32;
  x.k[0] = *reinterpret_cast<const uint4*>(kr);
  x.k[1] = *reinterpret_cast<const uint4*>(kr + 16);
  x.k[2] = *reinterpret_cast<const uint4*>(kr + 128);
  x.k[3] = *reinterpret_cast<const uint4*>(kr + 144);
#pragma unroll
  for (int r = 0; r < 4; ++r)
    x.v[r] = *reinterpret_cast<const uint4*>(tile + (size_t)min(4 * kb + r, last) * 512 + 16 * row);
  return x;
}

__device__ __forceinline__ v8i as_v8i(uint4 a, uint4 b) {
  return v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

// One 16-key tile (keys t0 ..) of a wave: scores, online softmax, V sums.
__device__ __forceinline__ void dn_tile(const DnTile& x, int t0, int T, int kb, const v8i (&bq)[2],
                                        float zc, float (&o)[H][16], float& m, float& l) {
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(as_v8i(x.k[0], x.k[1]), bq[0], acc, 0,
                                                          0, 0, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(as_v8i(x.k[2], x.k[3]), bq[1], acc, 0,
                                                          0, 0, 0, 0, 0);
  // logits (log2 units) of keys t0 + 4kb + r for head col / 4: the four
  // split columns of a head are adjacent lanes
  float z[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = acc[r] * zc;
    v += dpp_f<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);  // quad_perm [2,3,0,1]
    z[r] = t0 + 4 * kb + r < T ? v : -INFINITY;
  }
  const float tm = fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3]));
  const bool grow = tm > m + DN_TAU;
  if (__ballot(grow)) {
    const float mn = grow ? tm : m;
    const float al = grow ? exp2f(m - mn) : 1.f;
    l *= al;
    m = mn;
    const float ah[H] = {head_bcast<0>(al), head_bcast<1>(al), head_bcast<2>(al), head_bcast<3>(al)};
#pragma unroll
    for (int h = 0; h < H; ++h)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[h][i] *= ah[h];
  }
  float p[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) p[r] = z[r] == -INFINITY ? 0.f : exp2f(z[r] - m);
  l += (p[0] + p[1]) + (p[2] + p[3]);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float vf[16];
    fp8x4_to_f32(x.v[r].x, vf);
    fp8x4_to_f32(x.v[r].y, vf + 4);
    fp8x4_to_f32(x.v[r].z, vf + 8);
    fp8x4_to_f32(x.v[r].w, vf + 12);
    const float ph[H] = {head_bcast<0>(p[r]), head_bcast<1>(p[r]), head_bcast<2>(p[r]),
                         head_bcast<3>(p[r])};
#pragma unroll
    for (int h = 0; h < H; ++h)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[h][i] = fmaf(ph[h], vf[i], o[h][i]);
  }
}

// PAGED: the records are read through the page table (a.table, a.shift).
template <bool PAGED>
__global__ __launch_bounds__(DN_BLOCK) void k_dense(DenseArgs a) {
  const int g = blockIdx.y, b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, kb = lane >> 4;
  const int T = a.T;
  const uint8_t* __restrict__ kv = a.kv8 + (size_t)g * a.rows * 512;
  __shared__ float s_o[DN_WAVES][H][D];
  __shared__ float s_m[DN_WAVES][H], s_l[DN_WAVES][H];

  // this wave's tiles: the block sweeps its DN_WAVES x iters tiles in order,
  // consecutive waves taking consecutive tiles
  const int ntiles = (T + DN_TILE - 1) / DN_TILE;
  const int first = b * DN_WAVES * a.iters + wave;
  const int n = first < ntiles ? min(a.iters, (ntiles - first + DN_WAVES - 1) / DN_WAVES) : 0;
  auto key0 = [&](int i) { return (first + DN_WAVES * i) * DN_TILE; };
  // paged: lane i (i + 64 in the second word) holds the record index of the
  // first key of the wave's tile i (a wave has at most DN_PAGED_MAX_TILES
  // tiles: T <= 2^20, checked at create); loaded before the query is split,
  // so the first tile loads need not wait for the table
  static_assert(DN_PAGED_MAX_TILES == 2 * WAVE, "two index words per lane");
  uint32_t prow[2] = {0u, 0u};
  if (PAGED) {
#pragma unroll
    for (int r = 0; r < 2; ++r)
      if (lane + 64 * r < n) prow[r] = kv_row_paged(a.table, a.shift, g, key0(lane + 64 * r));
  }

  v8i bq[2];
  float zc;
  dense_query(a.q + (size_t)g * H * D, lane, bq, zc);

  float o[H][16];
#pragma unroll
  for (int h = 0; h < H; ++h)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[h][i] = 0.f;
  float m = -INFINITY, l = 0.f;  // running max / sum of head col / 4 over this row's keys

  auto load = [&](int i) {
    if (PAGED) {
      const uint32_t r = __builtin_amdgcn_readlane(i < 64 ? prow[0] : prow[1], i & 63);
      return dn_load_paged(a.kv8 + (size_t)r * 512, T - 1 - key0(i), lane);
    }
    return dn_load(kv, T, key0(i), lane);
  };
  if (n > 0) {
    // three tiles in registers: two loads in flight while one is processed
    DnTile b0 = load(0), b1, b2;
    if (n > 1) b1 = load(1);
    for (int i = 0;; i += 3) {
      if (i + 2 < n) b2 = load(i + 2);
      dn_tile(b0, key0(i), T, kb, bq, zc, o, m, l);
      if (i + 1 >= n) break;
      if (i + 3 < n) b0 = load(i + 3);
      dn_tile(b1, key0(i + 1), T, kb, bq, zc, o, m, l);
      if (i + 2 >= n) break;
      if (i + 4 < n) b1 = load(i + 4);
      dn_tile(b2, key0(i + 2), T, kb, bq, zc, o, m, l);
      if (i + 3 >= n) break;
    }
  }

  // the wave's 4 rows -> one partial per head (every row ends with the sums)
  float M = fmaxf(m, __shfl_xor(m, 16));
  M = fmaxf(M, __shfl_xor(M, 32));
  const float f = m == -INFINITY ? 0.f : exp2f(m - M);
  float L = l * f;
  L += __shfl_xor(L, 16);
  L += __shfl_xor(L, 32);
  const float fh[H] = {head_bcast<0>(f), head_bcast<1>(f), head_bcast<2>(f), head_bcast<3>(f)};
#pragma unroll
  for (int h = 0; h < H; ++h)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float v = o[h][i] * fh[h];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      o[h][i] = v;
    }
  if (kb == 0) {
#pragma unroll
    for (int h = 0; h < H; ++h)
#pragma unroll
      for (int i = 0; i < 16; i += 4)
        *reinterpret_cast<float4*>(&s_o[wave][h][16 * col + i]) =
            make_float4(o[h][i], o[h][i + 1], o[h][i + 2], o[h][i + 3]);
    if ((col & 3) == 0) {
      s_m[wave][col >> 2] = M;
      s_l[wave][col >> 2] = L;
    }
  }
  __syncthreads();
  // the block's partial: waves merged in wave order
  for (int e = threadIdx.x; e < H * D; e += DN_BLOCK) {
    const int h = e / D, d = e % D;
    float Mb = -INFINITY;
#pragma unroll
    for (int w = 0; w < DN_WAVES; ++w) Mb = fmaxf(Mb, s_m[w][h]);
    float O = 0.f, Lb = 0.f;
#pragma unroll
    for (int w = 0; w < DN_WAVES; ++w) {
      const float fw = s_m[w][h] == -INFINITY ? 0.f : exp2f(s_m[w][h] - Mb);
      O = fmaf(fw, s_o[w][h][d], O);
      Lb = fmaf(fw, s_l[w][h], Lb);
    }
    float* dst = a.part + (((size_t)g * a.nb + b) * H + h) * (D + 2);
    dst[d] = O;
    if (d == 0) {
      dst[D] = Mb;
      dst[D + 1] = Lb;
    }
  }
}

// Query head j = blockIdx.x, dims 8 * blockIdx.y + [0, 8): thread (slice s,
// dim) loads partials s, s + 32, ... (at most DN_MERGE_PER, all in flight
// together), the block agrees on their max, and the slices are added in order.
constexpr int DN_MERGE_PER = (DN_TARGET_BLOCKS + 31) / 32;

__global__ __launch_bounds__(256) void k_dense_merge(DenseArgs a) {
  const int j = blockIdx.x, g = j / H, h = j % H;
  const int dl = threadIdx.x & 7, sl = threadIdx.x >> 3;
  const int d = blockIdx.y * 8 + dl;
  const size_t stride = (size_t)H * (D + 2);
  const float* __restrict__ base = a.part + ((size_t)g * a.nb * H + h) * (D + 2);
  __shared__ float s_max[256 / WAVE];
  __shared__ float s_o[32][8], s_l[32];
  float pm[DN_MERGE_PER], pl[DN_MERGE_PER], po[DN_MERGE_PER];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < DN_MERGE_PER; ++i) {
    const int b = sl + 32 * i;
    pm[i] = -INFINITY;
    pl[i] = po[i] = 0.f;
    if (b < a.nb) {
      const float* p = base + b * stride;
      pm[i] = p[D];
      pl[i] = p[D + 1];
      po[i] = p[d];
    }
    mx = fmaxf(mx, pm[i]);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = mx;
  __syncthreads();
  float M = s_max[0];
#pragma unroll
  for (int w = 1; w < 256 / WAVE; ++w) M = fmaxf(M, s_max[w]);
  float O = 0.f, L = 0.f;
#pragma unroll
  for (int i = 0; i < DN_MERGE_PER; ++i) {
    const float f = pm[i] == -INFINITY ? 0.f : exp2f(pm[i] - M);
    O = fmaf(f, po[i], O);
    L = fmaf(f, pl[i], L);
  }
  s_o[sl][dl] = O;
  if (dl == 0) s_l[sl] = L;
  __syncthreads();
  if (threadIdx.x < 8) {
    float Ot = 0.f, Lt = 0.f;
#pragma unroll
    for (int s = 0; s < 32; ++s) {
      Ot += s_o[s][dl];
      Lt += s_l[s];
    }
    a.out[j * D + d] = (uint16_t)bf16_rne(Ot / Lt);
  }
}

}  // namespace

void launch_dense(const DenseArgs& a, hipStream_t st, int k) {
  if (k == 0)
    hipLaunchKernelGGL(a.table ? k_dense<true> : k_dense<false>, dim3(a.nb, G), dim3(DN_BLOCK), 0,
                       st, a);
  else
    hipLaunchKernelGGL(k_dense_merge, dim3(G * H, DN_MERGE_SLICES), dim3(256), 0, st, a);
}

// ------------------------------------------------ allocation-free dense decode
// The partials of skv_dense_decode_static: one file-scope device array per
// GPU, [G][DN_TARGET_BLOCKS][H][D + 2] FP32 (1 MiB), enough for every context
// up to 2^20 keys (dense_shape never uses more than DN_TARGET_BLOCKS blocks
// per group).  Host code never names it in a launch: the device address comes
// from hipGetSymbolAddress, once per device, with that device current.
constexpr size_t DN_SCRATCH_FLOATS = (size_t)G * DN_TARGET_BLOCKS * H * (D + 2);
static __device__ __align__(256) float scratch[DN_SCRATCH_FLOATS];

namespace {

constexpr int DN_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[DN_MAX_DEVICES] = {};

// The calling thread's current device's copy of `scratch` (looked up on the
// first call on that device); NULL with *err set on failure.
float* device_scratch(int* device, hipError_t* err) {
  *err = hipGetDevice(device);
  if (*err != hipSuccess) return nullptr;
  if (*device < 0 || *device >= DN_MAX_DEVICES) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[*device]) {
    void* ptr = nullptr;
    *err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    g_scratch_ptr[*device] = static_cast<float*>(ptr);
  }
  return g_scratch_ptr[*device];
}

}  // namespace

}  // namespace skv

extern "C" int skv_dense_decode_static(const void* kv8, int rows, int T, const void* q_dev,
                                       void* out_dev, void* stream) {
  using namespace skv;
  if (!kv8 || !q_dev || !out_dev) return note_call_error(SKV_EINVAL, "NULL records, query or output");
  if (T < 1 || T > (1 << 20))
    return note_call_error(SKV_EINVAL, "context %d outside [1, 2^20] (the static partials hold "
                           "%d blocks per group)", T, DN_TARGET_BLOCKS);
  if (rows < T) return note_call_error(SKV_EINVAL, "rows %d < context %d", rows, T);
  int device = 0;
  hipError_t e = hipSuccess;
  float* part = device_scratch(&device, &e);
  if (!part)
    return note_call_error(SKV_EHIP, "device scratch lookup failed: %s", hipGetErrorString(e));
  // every operand must be device memory of the current device large enough
  // for what the kernels touch (a wrong size or a host pointer is refused
  // here rather than faulting in a kernel)
  const struct { const void* ptr; uint64_t bytes; const char* name; } operands[] = {
      {kv8, (uint64_t)G * rows * 512, "records"},
      {q_dev, 16 * D * 2, "query"},
      {out_dev, 16 * D * 2, "output"}};
  for (const auto& op : operands)
    if (const char* why = device_range_error(op.ptr, op.bytes, device))
      return note_call_error(SKV_EINVAL, "%s (%llu bytes) %s", op.name,
                             (unsigned long long)op.bytes, why);
  (void)hipGetLastError();  // a launch error below is this call's, not an earlier one's
  DenseArgs a{};
  a.kv8 = static_cast<const uint8_t*>(kv8);
  a.q = static_cast<const uint16_t*>(q_dev);
  a.T = T;
  a.rows = rows;
  dense_shape(T, a.iters, a.nb);
  if (a.nb > DN_TARGET_BLOCKS)  // never for T <= 2^20
    return note_call_error(SKV_EINVAL, "context %d needs %d partials per group", T, a.nb);
  a.part = part;
  a.out = static_cast<uint16_t*>(out_dev);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  launch_dense(a, st, 0);
  launch_dense(a, st, 1);
  e = hipGetLastError();
  if (e != hipSuccess) return note_call_error(SKV_EHIP, "dense launch failed: %s", hipGetErrorString(e));
  return SKV_OK;
}
