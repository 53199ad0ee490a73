// Phase timestamps of the decode-step kernels, for development builds only
// (-DSKV_TRACE, python -m seoulkv_amd.build --trace); every macro compiles to
// nothing otherwise, so the product library carries no trace code.
//
//   SKV_TS(k, i)      thread 0 of block (0, 0) stores the 100 MHz real-time
//                     counter at point i (< 16) of kernel slot k (< 32)
//   SKV_TSB(k, i)     every block's thread 0 stores it at point i (< 3) of
//                     block slot k (< 12; first 4096 blocks, x-major)
//   SKV_TSE(k)        point 3 of block slot k: the latest time any wave of
//                     the block reached it
//   SKV_TSV(k, i, v)  every block's lane 0 of the calling wave stores the
//                     value v (not a time) at point i of block slot k
//   SKV_TSW(k, i)     point i of block slot k: the latest time any wave of
//                     the block reached it (as SKV_TSE for point 3)
//   SKV_WAIT(x)       makes the calling wave wait for the loads that produce
//                     the 32-bit value x (trace builds: a phase ends when its
//                     data has arrived)
//
// The tables live in skv_kernels.hip; skv_trace_read / skv_trace_blocks (C
// ABI, trace builds only) copy them to the host.
#pragma once

#ifdef SKV_TRACE
namespace skv {
extern __device__ unsigned long long g_skv_trace[32][16];
extern __device__ unsigned long long g_skv_trace_blk[12][4096][4];
}  // namespace skv
#define SKV_TS(k, i)                                                           \
  do {                                                                         \
    if ((k) >= 0 && threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0)   \
      ::skv::g_skv_trace[(k)][(i)] = __builtin_amdgcn_s_memrealtime();         \
  } while (0)
#define SKV_TSB(k, i)                                                          \
  do {                                                                         \
    const unsigned _b = blockIdx.x + blockIdx.y * gridDim.x;                   \
    if (threadIdx.x == 0 && _b < 4096)                                         \
      ::skv::g_skv_trace_blk[(k)][_b][(i)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#define SKV_TSE(k)                                                             \
  do {                                                                         \
    const unsigned _b = blockIdx.x + blockIdx.y * gridDim.x;                   \
    if ((threadIdx.x & 63) == 0 && _b < 4096)                                  \
      atomicMax(&::skv::g_skv_trace_blk[(k)][_b][3], __builtin_amdgcn_s_memrealtime()); \
  } while (0)
#define SKV_TSV(k, i, v)                                                       \
  do {                                                                         \
    const unsigned _b = blockIdx.x + blockIdx.y * gridDim.x;                   \
    if ((threadIdx.x & 63) == 0 && _b < 4096)                                  \
      ::skv::g_skv_trace_blk[(k)][_b][(i)] = (unsigned long long)(v);          \
  } while (0)
#define SKV_TSW(k, i)                                                          \
  do {                                                                         \
    const unsigned _b = blockIdx.x + blockIdx.y * gridDim.x;                   \
    if ((threadIdx.x & 63) == 0 && _b < 4096)                                  \
      atomicMax(&::skv::g_skv_trace_blk[(k)][_b][(i)], __builtin_amdgcn_s_memrealtime()); \
  } while (0)
#define SKV_WAIT(x)                        \
  do {                                     \
    uint32_t _x = (x);                     \
    asm volatile("" : "+v"(_x));           \
  } while (0)
#else
#define SKV_TS(k, i) \
  do {               \
  } while (0)
#define SKV_TSB(k, i) \
  do {                \
  } while (0)
#define SKV_TSE(k) \
  do {             \
  } while (0)
#define SKV_TSV(k, i, v) \
  do {                   \
  } while (0)
#define SKV_TSW(k, i) \
  do {                \
  } while (0)
#define SKV_WAIT(x) \
  do {              \
  } while (0)
#endif
