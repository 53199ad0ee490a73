// C ABI of the SeoulKV4 MI355X decode path (see include/seoulkv4_hip.h).
//
// skv_create is the reference's _runtime.initialize (_runtime.py:36-177): it
// uploads the index once, derives the spill-2 mate table (reference
// posting_mates, _kernels/common/seoulkv4_cluster_blocks.py:10-32), and runs
// the prefill kernels on the device:
//   * key codec (reference _codecs/keys.py:16-26): per-coordinate max-abs
//     scale over all tokens, code8 = clamp(floor((k + s) / (2 s / 256)), 0, 255);
//   * token-major key records [T][256 B] = 2-bit prefix plane | 2-bit
//     residual plane | 4-bit residual plane (the three planes of
//     _codecs/keys.py:29-44, contiguous per token so Stage 1.6 reads one 128 B
//     line and Stage II the next);
//   * cluster-block prefixes [postings][64 B]: the prefix plane copied in CSR
//     order (reference pack_cluster_blocks, seoulkv4_cluster_blocks.py:55-104)
//     so Stage 1.5 reads each selected cluster contiguously;
//   * FP8 e4m3fn [V || K] records [T][512 B] (reference _runtime.py:76-92).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/seoulkv4_hip.h"
#include "skv_dense.h"
#include "skv_device.h"
#include "skv_fastsel.h"
#include "skv_octsel.h"
#include "skv_select.h"
#include "skv_step.h"

using namespace skv;

namespace {

thread_local std::string g_create_error;

// Bump allocator over one device allocation.  A plan runs twice: first with
// base == nullptr to size the allocation (take() then returns nullptr: no
// arithmetic on a null pointer), then over the allocation itself.
struct Arena {
  char* base = nullptr;
  size_t size = 0, used = 0;
  void* take(size_t bytes) {
    size_t at = (used + 255) & ~size_t(255);
    used = at + bytes;
    return base ? base + at : nullptr;
  }
};

constexpr int APPEND_CHUNK = 256;   // tokens per host-append staging round
constexpr int Q_RING = 16;          // query staging slots (host run-ahead, in steps)
constexpr int Q_MARK = 8;           // uploads per completion event of the staging ring

constexpr int DEV_OK_SLOTS = 8;
struct DevRange {
  uintptr_t lo, hi;
};

struct Handle {
  int device = 0;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  // pinned staging ring of skv_bind_query: slot i is reused once its
  // previous upload has left it, so the host runs up to Q_RING steps ahead
  // of the device.  An event recorded on the stream costs the device about
  // as much as the 8 KiB upload itself, so only the upload of every
  // Q_MARK-th slot (slot % Q_MARK == Q_MARK - 1) records one: event
  // q_marked[i / Q_MARK] covers slot i's upload and the uploads before it.
  hipEvent_t q_marked[Q_RING / Q_MARK] = {};
  uint16_t* q_host = nullptr;  // [Q_RING][q_slot]: query [16][D], then a staged append
  size_t q_slot = 16 * D;      // elements per slot: + K and V of APPEND_FUSE tokens when
                               // the handle can append
  unsigned q_next = 0;
  // A host append of at most APPEND_FUSE tokens waits in the next ring slot
  // (pend_host) until the next query upload carries it to pend_dev (the
  // device buffer after the query), and is packed by the next step's k_front
  // or, before any other reader of the records, by k_pack_kv8.
  int pend_n = 0, pend_row = 0;
  bool pend_host = false;
  uint16_t* pend_dev = nullptr;  // [2][G][pend_n][D] BF16 K then V
  // device allocations skv_append_device has accepted (see checked_device_range)
  DevRange dev_ok[DEV_OK_SLOTS] = {};
  int dev_ok_n = 0, dev_ok_next = 0;
  // device-query binding on a producer stream: the handle's steps so far
  // (readers of the query buffer) and the copy on the producer stream
  hipEvent_t steps_done = nullptr, q_ready = nullptr;
  void* static_mem = nullptr;
  void* work_mem = nullptr;
  size_t static_bytes = 0, work_bytes = 0;
  StepArgs a{};
  StepWork w{};
  DenseArgs dn{};  // dense FP8 decode over every key (comparison path)
  // cache append: tokens after the prefill context extend the local window
  int context0 = 0, append_capacity = 0;
  // pinned host staging of long host appends: two [2][G][chunk][256] BF16
  // slots used in turn, each reused once the pack kernel that reads it over
  // the bus (through append_host_dev, its device address) has finished
  uint16_t* append_host = nullptr;
  const uint16_t* append_host_dev = nullptr;
  hipEvent_t append_ev[2] = {};
  unsigned append_next = 0;
  int n_centroids = 0, np_max = 0;
  int top_u1_lds_items = 0, top_u2_lds_items = 0;  // LDS-resident sizes (select modes 0-2)
  bool dense_ran = false;
  bool bound = false, ran = false;
  std::vector<int> page_table;  // paged records: physical page of each logical page
  size_t lds_per_block = 0;
  // per-kernel event timing (skv_profile)
  bool profiling = false, prof_pending = false;
  hipEvent_t prof_ev[N_STEP_KERNELS + 1] = {};
  double prof_ms[N_STEP_KERNELS] = {};
  int prof_steps = 0;
  // opt-in: the step's kernels captured once into a graph, replayed by
  // skv_enqueue (consecutive graph launches leave ~8 us idle between them on
  // ROCm 7.2, more than the launch gaps of the eager path)
  bool use_graph = false;
  hipStream_t capture_stream = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  std::string error, meta;
};

std::string json_escape(const std::string& s);

// The handle's JSON metadata (context and local window as of the last append).
void build_meta(Handle* h) {
  const StepArgs& a = h->a;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, h->device) != hipSuccess) memset(&prop, 0, sizeof prop);
  char buf[1024];
  snprintf(buf, sizeof buf,
           "{\"device\": \"%s\", \"arch\": \"%s\", \"context\": %d, \"sink\": %d, \"local\": %d, "
           "\"n_centroids\": %d, \"nprobe\": [%d, %d, %d, %d], \"pool_buffer\": %d, "
           "\"pool_min\": %d, \"pool_capacity\": %d, \"postings_max\": %d, "
           "\"static_device_bytes\": %zu, \"workspace_device_bytes\": %zu, "
           "\"kernels_per_step\": %d, \"lds_per_block\": %zu, \"pool_lds_items\": %d, "
           "\"prefill_context\": %d, \"appended\": %d, \"append_capacity\": %d, "
           "\"kv_page_tokens\": %d, \"top1600_in_registers_to\": %d}",
           json_escape(prop.name).c_str(), json_escape(prop.gcnArchName).c_str(), a.T, a.sink,
           a.local, h->n_centroids, a.P[0], a.P[1], a.P[2], a.P[3], a.cap, a.pool_min,
           a.pool_capacity, h->np_max, h->static_bytes, h->work_bytes, N_STEP_KERNELS,
           h->lds_per_block, h->w.top_u1.lds_items, h->context0, a.T - h->context0,
           h->append_capacity, a.kv_table ? 1 << a.kv_shift : 0,
           h->w.top_u1.regs2 ? 2 * OCT_ITEMS : OCT_ITEMS);
  h->meta = buf;
}

// Drop the captured step (launch options changed).
void drop_graph(Handle* h) {
  if (h->graph_exec) (void)hipGraphExecDestroy(h->graph_exec);
  if (h->graph) (void)hipGraphDestroy(h->graph);
  h->graph_exec = nullptr;
  h->graph = nullptr;
}

int fail(Handle* h, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (h) h->error = buf; else g_create_error = buf;
  return code;
}

#define HIPCHK(h, call)                                                          \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess)                                                        \
      return fail((h), SKV_EHIP, "%s failed: %s", #call, hipGetErrorString(e_)); \
  } while (0)

// ------------------------------------------------------------- prefill kernels
__global__ void k_init_kscale(const uint16_t* k, int T, uint32_t* bits) {
  const int g = blockIdx.y, d = threadIdx.x;
  uint32_t m = 0;
  for (int t = blockIdx.x; t < T; t += gridDim.x) {
    const uint32_t b = k[((size_t)g * T + t) * D + d] & 0x7fffu;  // |k| as bf16
    m = max(m, b);
  }
  atomicMax(&bits[g * D + d], m << 16);  // positive floats order as integers
}

__global__ void k_init_kscale_final(const uint32_t* bits, float* kscale) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < G * D) kscale[i] = fmaxf(__uint_as_float(bits[i]), 1e-9f);
}

__device__ __forceinline__ uint32_t key_code8(float kf, float s) {
  const float step8 = __fmul_rn(2.0f, s) * 0.00390625f;  // (2 s) / 256, exact
  const float c = floorf(__fdiv_rn(__fadd_rn(kf, s), step8));
  return (uint32_t)fminf(fmaxf(c, 0.0f), 255.0f);
}

// One thread per (group, token, 4-dim byte): writes byte b of the prefix and
// residual-2 planes and bytes 2b, 2b+1 of the residual-4 plane.
__global__ void k_init_keyrec(const uint16_t* k, const float* kscale, int T, uint8_t* keyrec) {
  const size_t n = (size_t)G * T * 64;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const int b = (int)(i & 63);
    const size_t gt = i >> 6;
    const int g = (int)(gt / T);
    const uint16_t* row = k + gt * D;
    uint32_t c[4];
    for (int j = 0; j < 4; ++j) {
      const int d = 4 * b + j;
      c[j] = key_code8(bf16_f32(row[d]), kscale[g * D + d]);
    }
    uint8_t* rec = keyrec + gt * 256;
    uint32_t p2 = 0, r2 = 0;
    for (int j = 0; j < 4; ++j) {
      p2 |= ((c[j] >> 6) & 3u) << (2 * j);
      r2 |= ((c[j] >> 4) & 3u) << (2 * j);
    }
    rec[b] = (uint8_t)p2;
    rec[64 + b] = (uint8_t)r2;
    rec[128 + 2 * b] = (uint8_t)((c[0] & 15u) | ((c[1] & 15u) << 4));
    rec[128 + 2 * b + 1] = (uint8_t)((c[2] & 15u) | ((c[3] & 15u) << 4));
  }
}

// FP8 [V || K] records of n tokens: k, v [G][n][256] bf16 (rows of the
// group g that are src_stride tokens apart) -> records of tokens row0 ..
// row0+n-1 of each group: rows row0 + t of kv8's [G][rows] records, or with a
// page table, the paged record of token row0 + t.  One thread per (group,
// token, 4 dims).
__global__ void k_pack_kv8(const uint16_t* k, const uint16_t* v, int n, size_t src_stride,
                           int row0, int rows, uint8_t* kv8, const int* table, int shift) {
  const size_t total = (size_t)G * n * (D / 4);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % (D / 4));
    const size_t gt = i / (D / 4);
    const int g = (int)(gt / n), t = (int)(gt % n);
    const size_t src = ((size_t)g * src_stride + t) * D + 4 * c;
    const uint2 kw = *reinterpret_cast<const uint2*>(k + src);
    const uint2 vw = *reinterpret_cast<const uint2*>(v + src);
    uint8_t* rec = kv8 + (table ? (size_t)kv_row_paged(table, shift, g, row0 + t)
                                : (size_t)g * rows + row0 + t) * 512;
    *reinterpret_cast<uint32_t*>(rec + 4 * c) = bf16x4_to_fp8(vw);
    *reinterpret_cast<uint32_t*>(rec + 256 + 4 * c) = bf16x4_to_fp8(kw);
  }
}

// Cluster-block prefix rows: post_p2[g][j] = prefix plane of token values[j].
__global__ void k_init_postp2(const int* post_tok, const uint8_t* keyrec, int T, int np_max,
                              const int* np_count, uint8_t* post_p2) {
  const size_t n = (size_t)G * np_max * 4;  // 16 B chunks
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const int part = (int)(i & 3);
    const size_t gj = i >> 2;
    const int g = (int)(gj / np_max), j = (int)(gj % np_max);
    uint4 val = make_uint4(0, 0, 0, 0);
    if (j < np_count[g]) {
      const int t = post_tok[gj];
      val = *reinterpret_cast<const uint4*>(keyrec + ((size_t)g * T + t) * 256 + part * 16);
    }
    *reinterpret_cast<uint4*>(post_p2 + gj * 64 + part * 16) = val;
  }
}

// IEEE half -> float on the host (exact).
float half_bits_to_float(uint16_t b) {
  const uint32_t sign = (uint32_t)(b & 0x8000u) << 16;
  const uint32_t e = (b >> 10) & 31u, m = b & 1023u;
  uint32_t u;
  if (e == 0) {
    if (m == 0) {
      u = sign;
    } else {  // subnormal: m * 2^-24
      float v = (float)m * 5.9604644775390625e-08f;
      memcpy(&u, &v, 4);
      u |= sign;
    }
  } else if (e == 31) {
    u = sign | 0x7f800000u | (m << 13);
  } else {
    u = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

std::string json_escape(const std::string& s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    o += c;
  }
  return o;
}

}  // namespace

int skv::note_call_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_create_error = buf;
  return code;
}

// Whether ptr is device memory of `device` whose allocation holds `bytes`
// from ptr on (nullptr) or why not.  Runtime queries only: no allocation.
const char* skv::device_range_error(const void* ptr, uint64_t bytes, int device) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, ptr) != hipSuccess || attr.type != hipMemoryTypeDevice ||
      attr.device != device) {
    (void)hipGetLastError();  // clear the query's error state
    return "is not device memory of the handle's device";
  }
  void* base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(ptr)) != hipSuccess) {
    (void)hipGetLastError();
    return "has no device allocation at its address";
  }
  const uint64_t off = (uint64_t)((const char*)ptr - (const char*)base);
  if (off > size || bytes > size - off) return "extends past the end of its device allocation";
  return nullptr;
}

extern "C" {

const char* skv_version(void) { return "seoulkv4-hip gfx950 1"; }

const char* skv_last_error(void* handle) {
  if (!handle) return g_create_error.c_str();
  return static_cast<Handle*>(handle)->error.c_str();
}

void skv_destroy(void* handle) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return;
  if (h->stream) (void)hipStreamSynchronize(h->stream);
  for (hipEvent_t e : h->q_marked)
    if (e) (void)hipEventDestroy(e);
  if (h->steps_done) (void)hipEventDestroy(h->steps_done);
  if (h->q_ready) (void)hipEventDestroy(h->q_ready);
  for (hipEvent_t e : h->prof_ev)
    if (e) (void)hipEventDestroy(e);
  drop_graph(h);
  if (h->capture_stream) (void)hipStreamDestroy(h->capture_stream);
  if (h->q_host) (void)hipHostFree(h->q_host);
  if (h->append_host) (void)hipHostFree(h->append_host);
  for (hipEvent_t e : h->append_ev)
    if (e) (void)hipEventDestroy(e);
  if (h->static_mem) (void)hipFree(h->static_mem);
  if (h->work_mem) (void)hipFree(h->work_mem);
  if (h->own_stream && h->stream) (void)hipStreamDestroy(h->stream);
  delete h;
}


// skv_create / skv_create_paged; pages NULL: contiguous records in the
// handle's own memory.
static int create_impl(const skv_index_desc* ix, const uint16_t* k_bf16, const uint16_t* v_bf16,
                       const skv_kv_pages* pages, int device, void* stream, void** handle_out) {
  if (!handle_out) return fail(nullptr, SKV_EINVAL, "handle_out is NULL");
  *handle_out = nullptr;
  if (!ix || !k_bf16 || !v_bf16) return fail(nullptr, SKV_EINVAL, "NULL index or K/V");
  const int T = ix->context, nc = ix->n_centroids;
  if (T <= 0 || T > (1 << 20)) return fail(nullptr, SKV_EINVAL, "context %d outside (0, 2^20]", T);
  if (nc <= 0 || nc % 32 || nc > 65536)
    return fail(nullptr, SKV_EINVAL, "n_centroids %d must be a multiple of 32 in [32, 65536]", nc);
  if (ix->sink < 0 || ix->local < 0 || ix->sink + ix->local >= T)
    return fail(nullptr, SKV_EINVAL, "sink/local %d/%d do not fit context %d", ix->sink, ix->local, T);
  if (ix->append_capacity < 0 || ix->append_capacity > (1 << 20) - T)
    return fail(nullptr, SKV_EINVAL, "append capacity %d: context plus capacity above 2^20",
                ix->append_capacity);
  const int cap_app = ix->append_capacity;
  const int R = T - ix->sink - ix->local;
  int page_shift = 0, table_len = 0;
  if (pages) {
    const int pt = pages->page_tokens;
    if (!pages->pool || ((uintptr_t)pages->pool & 255))
      return fail(nullptr, SKV_EINVAL, "page pool is NULL or not 256-byte aligned");
    if (pt < 16 || pt > 65536 || (pt & (pt - 1)))
      return fail(nullptr, SKV_EINVAL, "page_tokens %d is not a power of two in [16, 65536]", pt);
    while ((1 << page_shift) < pt) ++page_shift;
    // n_pages is bounded before it is multiplied, so the product cannot wrap
    if (pages->n_pages < 1 || pages->n_pages > ((int64_t)1 << 31) / (G * (int64_t)pt))
      return fail(nullptr, SKV_EINVAL, "page pool of %lld pages: 1 to 2^31 records",
                  (long long)pages->n_pages);
    table_len = (T + cap_app + pt - 1) / pt;
    if (!pages->page_table || pages->table_len < table_len)
      return fail(nullptr, SKV_EINVAL, "page table of %d entries; context %d plus capacity %d "
                  "needs %d pages of %d tokens", pages->page_table ? pages->table_len : 0, T,
                  cap_app, table_len, pt);
    std::vector<int> sorted(pages->page_table, pages->page_table + table_len);
    std::sort(sorted.begin(), sorted.end());
    for (int i = 0; i < table_len; ++i) {
      if (sorted[i] < 0 || sorted[i] >= pages->n_pages)
        return fail(nullptr, SKV_EINVAL, "page table entry %d outside [0, %lld)", sorted[i],
                    (long long)pages->n_pages);
      if (i && sorted[i] == sorted[i - 1])
        return fail(nullptr, SKV_EINVAL, "page %d appears twice in the page table", sorted[i]);
    }
  }

  // ---- host-side validation and the spill-2 mate table
  std::vector<std::vector<int>> mates(G);
  std::vector<int> np(G);
  int np_max = 1;
  for (int g = 0; g < G; ++g) {
    const skv_cell_desc& c = ix->cells[g];
    if (!c.upper || !c.lower || !c.scale || !c.resid_f16 || !c.gfs_f16 || !c.offsets || !c.values)
      return fail(nullptr, SKV_EINVAL, "cell %d has a NULL array", g);
    if (c.nprobe < 1 || c.nprobe > nc)
      return fail(nullptr, SKV_EINVAL, "cell %d nprobe %d outside [1, %d]", g, c.nprobe, nc);
    if (c.offsets[0] != 0) return fail(nullptr, SKV_EINVAL, "cell %d CSR offsets[0] != 0", g);
    for (int i = 0; i < nc; ++i)
      if (c.offsets[i + 1] < c.offsets[i])
        return fail(nullptr, SKV_EINVAL, "cell %d CSR offsets not monotone", g);
    np[g] = c.offsets[nc];
    if (np[g] >= (1 << 21))  // the pool kernel's range scan holds posting counts in 21 bits
      return fail(nullptr, SKV_EINVAL, "cell %d holds %d postings (at most 2^21 - 1)", g, np[g]);
    np_max = std::max(np_max, np[g]);
    std::vector<int> first_post(T, -1), first_cluster(T, -1), seen(T, 0);
    std::vector<int>& m = mates[g];
    m.assign(np[g], -1);
    for (int cl = 0; cl < nc; ++cl)
      for (int j = c.offsets[cl]; j < c.offsets[cl + 1]; ++j) {
        const int t = c.values[j];
        if (t < 0 || t >= T) return fail(nullptr, SKV_EINVAL, "cell %d invalid CSR token ID %d", g, t);
        if (++seen[t] > 2)
          return fail(nullptr, SKV_EINVAL, "local ownership requires at most two memberships/token");
        if (first_post[t] < 0) {
          first_post[t] = j;
          first_cluster[t] = cl;
        } else {
          if (first_cluster[t] == cl)
            return fail(nullptr, SKV_EINVAL, "duplicate token inside one cluster");
          m[j] = first_cluster[t];
          m[first_post[t]] = cl;
        }
      }
  }

  Handle* h = new Handle();
  h->device = device;
  auto bail = [&](int code) {
    g_create_error = h->error;
    skv_destroy(h);
    return code;
  };
  if (hipSetDevice(device) != hipSuccess) {
    fail(h, SKV_EHIP, "hipSetDevice(%d) failed", device);
    return bail(SKV_EHIP);
  }
  if (pages) {  // device memory of this device holding all n_pages pages
    const uint64_t need = (uint64_t)pages->n_pages * G * pages->page_tokens * 512;
    if (const char* why = device_range_error(pages->pool, need, device)) {
      fail(h, SKV_EINVAL, "page pool of %lld pages (%llu bytes) %s", (long long)pages->n_pages,
           (unsigned long long)need, why);
      return bail(SKV_EINVAL);
    }
  }
  {
    int lds = 0;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device) !=
        hipSuccess || lds <= 0) {
      fail(h, SKV_EHIP, "cannot query the LDS size of device %d", device);
      return bail(SKV_EHIP);
    }
    h->lds_per_block = (size_t)lds;
  }
  if (stream) {
    h->stream = static_cast<hipStream_t>(stream);
  } else {
    if (hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess) {
      fail(h, SKV_EHIP, "hipStreamCreate failed");
      return bail(SKV_EHIP);
    }
    h->own_stream = true;
  }

  StepArgs& a = h->a;
  a.T = T;
  a.rec_rows = T;
  a.kv_rows = T + cap_app;
  h->context0 = T;
  h->append_capacity = cap_app;
  h->n_centroids = nc;
  h->np_max = np_max;
  a.sink = ix->sink;
  a.local = ix->local;
  a.nc = nc;
  a.np_max = np_max;
  a.cap = (std::max(R, 64) + 63) / 64 * 64;  // 16-byte aligned score rows
  a.pool_min = ix->pool_min;
  a.pool_capacity = ix->pool_capacity;
  a.debug = ix->debug;
  for (int g = 0; g < G; ++g) {
    a.P[g] = ix->cells[g].nprobe;
    a.lam[g] = ix->cells[g].lam;
  }
  const int words1 = (a.cap + 63) / 64, words2 = (U1_MAX + 63) / 64;
  a.words_u1 = words1;
  a.words_u2 = words2;
  a.pool_blocks = nc / 32;
  // at most 64 ranges per group (one pool block per CU over the 4 groups;
  // one look-back poll reaches every predecessor), at least 32 centroids
  // (one bitmap word) per range: small indexes still spread the pool's row
  // fetch over ~64 CUs per group
  a.pool_range = std::max(32, (nc / 64 + 31) / 32 * 32);
  a.dense_slices = (a.sink + a.local + DENSE_SLICE_KEYS - 1) / DENSE_SLICE_KEYS;
  const int max_slices = (a.sink + a.local + cap_app + DENSE_SLICE_KEYS - 1) / DENSE_SLICE_KEYS;
  h->dn.T = T;
  h->dn.rows = T + cap_app;
  dense_shape(T, h->dn.iters, h->dn.nb);
  if (h->dn.nb > DN_TARGET_BLOCKS) {  // the merge kernel holds at most this many partials
    fail(h, SKV_EINVAL, "dense decode shape: %d blocks per group", h->dn.nb);
    return bail(SKV_EINVAL);
  }
  {  // the paged dense kernel holds the record index of each wave's tiles in
     // two registers: at most DN_PAGED_MAX_TILES tiles per wave at the largest
     // context the handle can reach
    int it = 0, nb = 0;
    dense_shape(T + cap_app, it, nb);
    if (pages && it > DN_PAGED_MAX_TILES) {
      fail(h, SKV_EINVAL, "paged dense decode: %d tiles per wave (at most %d)", it,
           DN_PAGED_MAX_TILES);
      return bail(SKV_EINVAL);
    }
  }

  // ---- static arena
  Arena s;
  auto plan_static = [&](Arena& ar) {
    a.kscale = (float*)ar.take(G * D * 4);
    a.cen_up = (uint8_t*)ar.take((size_t)G * nc * 64);
    a.cen_lo = (uint8_t*)ar.take((size_t)G * nc * 64);
    a.scale4 = (float*)ar.take((size_t)G * (nc / 32) * 4);
    a.resid = (float*)ar.take((size_t)G * nc * 4);
    a.gfs = (float*)ar.take((size_t)G * (nc / 32) * 4);
    a.csr_off = (int*)ar.take((size_t)G * (nc + 1) * 4);
    a.post_tok = (int*)ar.take((size_t)G * np_max * 4);
    a.post_mate = (int*)ar.take((size_t)G * np_max * 4);
    a.post_p2 = (uint8_t*)ar.take((size_t)G * np_max * 64);
    a.keyrec = (uint8_t*)ar.take((size_t)G * T * 256);
    if (pages)  // the records live in the caller's pages
      a.kv_table = (int*)ar.take((size_t)table_len * 4);
    else
      a.kv8 = (uint8_t*)ar.take((size_t)G * (T + cap_app) * 512);
  };
  plan_static(s);
  h->static_bytes = s.used;
  if (hipMalloc(&h->static_mem, s.used) != hipSuccess) {
    fail(h, SKV_ENOMEM, "cannot allocate %zu bytes of static device memory", s.used);
    return bail(SKV_ENOMEM);
  }
  s.base = (char*)h->static_mem;
  s.used = 0;
  plan_static(s);
  if (pages) {
    a.kv8 = static_cast<const uint8_t*>(pages->pool);
    a.kv_shift = page_shift;
    h->page_table.assign(pages->page_table, pages->page_table + table_len);
    if (hipMemcpy(const_cast<int*>(a.kv_table), h->page_table.data(), (size_t)table_len * 4,
                  hipMemcpyHostToDevice) != hipSuccess) {
      fail(h, SKV_EHIP, "page table upload failed");
      return bail(SKV_EHIP);
    }
  }

  // ---- workspace arena
  Arena wk;
  auto plan_work = [&](Arena& ar) {
    // the query, then a folded append's BF16 K and V (one upload for both)
    a.q = (uint16_t*)ar.take((16 + (cap_app ? 2 * G * APPEND_FUSE : 0)) * D * 2);
    a.qop = (QOperand*)ar.take(sizeof(QOperand) * G * QV_COUNT);
    a.lower = (uint16_t*)ar.take((size_t)G * H * nc * 2);
    a.upper = (uint16_t*)ar.take((size_t)G * H * nc * 2);
    a.thr = (uint32_t*)ar.take(G * H * 4);
    a.masks = (uint8_t*)ar.take((size_t)G * nc);
    a.fine_ord = (uint16_t*)ar.take((size_t)G * H * nc * 2);
    a.fine_bits = (uint16_t*)ar.take((size_t)G * H * nc * 2);
    a.tmax_lo = nc > 8 * SEL_BLOCK ? (uint16_t*)ar.take((size_t)G * H * (nc / 8) * 2) : nullptr;
    a.tmax_fi = nc > 8 * SEL_BLOCK ? (uint16_t*)ar.take((size_t)G * H * (nc / 16) * 2) : nullptr;
    a.sel = (int*)ar.take((size_t)G * nc * 4);
    a.pool_flags = (unsigned long long*)ar.take((size_t)G * a.pool_blocks * 8);
    a.pool_scan = (int*)ar.take((size_t)G * a.pool_blocks * 4);
    a.pool_epoch = (unsigned*)ar.take((size_t)G * 4);
    a.pool_tok = (int*)ar.take((size_t)G * a.cap * 4);
    a.s2 = (uint16_t*)ar.take((size_t)G * H * a.cap * 2);
    a.s2_tmax = (uint16_t*)ar.take((size_t)G * H * (a.cap / 16) * 2);
    a.dense_part = (float*)ar.take((size_t)G * H * std::max(max_slices, 1) * (D + 2) * 4);
    a.selbm = (uint32_t*)ar.take((size_t)G * (nc / 32) * 4);  // cleared by k_front
    a.u1_tok = (int*)ar.take((size_t)G * U1_MAX * 4);
    a.s4 = (uint16_t*)ar.take((size_t)G * H * U1_MAX * 2);
    a.s8 = (uint16_t*)ar.take((size_t)G * H * U1_MAX * 2);
    a.top = (int*)ar.take(G * H * TOPK * 4);
    a.status = (int*)ar.take(G * ST_WORDS * 4);
    a.out = (uint16_t*)ar.take(16 * D * 2);
    a.out_tiles = (uint16_t*)ar.take((size_t)G * 32 * H * D * 2);
    a.bm_u1 = (uint64_t*)ar.take((size_t)G * H * words1 * 8);
    a.bm_u2 = (uint64_t*)ar.take((size_t)G * H * words2 * 8);
    h->dn.part = (float*)ar.take((size_t)G * DN_TARGET_BLOCKS * H * (D + 2) * 4);  // any T
    h->dn.out = (uint16_t*)ar.take(16 * D * 2);
  };
  plan_work(wk);
  h->work_bytes = wk.used;
  if (hipMalloc(&h->work_mem, wk.used) != hipSuccess) {
    fail(h, SKV_ENOMEM, "cannot allocate %zu bytes of device workspace", wk.used);
    return bail(SKV_ENOMEM);
  }
  wk.base = (char*)h->work_mem;
  wk.used = 0;
  plan_work(wk);
  h->dn.kv8 = a.kv8;
  h->dn.table = a.kv_table;
  h->dn.shift = a.kv_shift;
  h->dn.q = a.q;
  if (hipMemsetAsync(h->work_mem, 0, h->work_bytes, h->stream) != hipSuccess) {
    fail(h, SKV_EHIP, "workspace clear failed");
    return bail(SKV_EHIP);
  }

  // ---- index upload
  std::vector<float> scale4((size_t)G * (nc / 32)), resid((size_t)G * nc), gfs((size_t)G * (nc / 32));
  std::vector<uint8_t> up((size_t)G * nc * 64), lo((size_t)G * nc * 64);
  std::vector<int> off((size_t)G * (nc + 1)), ptok((size_t)G * np_max, 0), pmate((size_t)G * np_max, -1);
  for (int g = 0; g < G; ++g) {
    const skv_cell_desc& c = ix->cells[g];
    memcpy(&up[(size_t)g * nc * 64], c.upper, (size_t)nc * 64);
    memcpy(&lo[(size_t)g * nc * 64], c.lower, (size_t)nc * 64);
    for (int i = 0; i < nc; ++i) {
      // bf16(fp16 residual norm) as fp32, like the reference's .bfloat16()
      const float rf = half_bits_to_float(c.resid_f16[i]);
      uint32_t u;
      memcpy(&u, &rf, 4);
      u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
      memcpy(&resid[(size_t)g * nc + i], &u, 4);
    }
    for (int i = 0; i < nc / 32; ++i) {
      const float s0 = c.scale[i * 32];
      for (int j = 1; j < 32; ++j)
        if (c.scale[i * 32 + j] != s0) {
          fail(h, SKV_EINVAL, "cell %d scale is not shared within 32-centroid group %d", g, i);
          return bail(SKV_EINVAL);
        }
      scale4[(size_t)g * (nc / 32) + i] = s0 / 4.0f;
      gfs[(size_t)g * (nc / 32) + i] = half_bits_to_float(c.gfs_f16[i]);
    }
    memcpy(&off[(size_t)g * (nc + 1)], c.offsets, (size_t)(nc + 1) * 4);
    memcpy(&ptok[(size_t)g * np_max], c.values, (size_t)np[g] * 4);
    memcpy(&pmate[(size_t)g * np_max], mates[g].data(), (size_t)np[g] * 4);
  }
  auto up_copy = [&](const void* dst, const void* src, size_t bytes) {
    return hipMemcpy(const_cast<void*>(dst), src, bytes, hipMemcpyHostToDevice);
  };
  if (up_copy(a.cen_up, up.data(), up.size()) || up_copy(a.cen_lo, lo.data(), lo.size()) ||
      up_copy(a.scale4, scale4.data(), scale4.size() * 4) ||
      up_copy(a.resid, resid.data(), resid.size() * 4) ||
      up_copy(a.gfs, gfs.data(), gfs.size() * 4) ||
      up_copy(a.csr_off, off.data(), off.size() * 4) ||
      up_copy(a.post_tok, ptok.data(), ptok.size() * 4) ||
      up_copy(a.post_mate, pmate.data(), pmate.size() * 4)) {
    fail(h, SKV_EHIP, "index upload failed");
    return bail(SKV_EHIP);
  }

  // ---- prefill: key codec, key records, cluster-block prefixes, FP8 records
  {
    const size_t kv_bytes = (size_t)G * T * D * 2;
    uint16_t *dk = nullptr, *dv = nullptr;
    uint32_t* sbits = nullptr;
    int* dnp = nullptr;
    if (hipMalloc(&dk, kv_bytes) != hipSuccess || hipMalloc(&dv, kv_bytes) != hipSuccess ||
        hipMalloc(&sbits, G * D * 4) != hipSuccess || hipMalloc(&dnp, G * 4) != hipSuccess) {
      (void)hipFree(dk); (void)hipFree(dv); (void)hipFree(sbits); (void)hipFree(dnp);
      fail(h, SKV_ENOMEM, "cannot allocate prefill staging (%zu bytes)", 2 * kv_bytes);
      return bail(SKV_ENOMEM);
    }
    bool ok = hipMemcpy(dk, k_bf16, kv_bytes, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(dv, v_bf16, kv_bytes, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(dnp, np.data(), G * 4, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemset(sbits, 0, G * D * 4) == hipSuccess;
    if (ok) {
      hipLaunchKernelGGL(k_init_kscale, dim3(std::min(T, 4096), G), dim3(D), 0, h->stream, dk, T, sbits);
      hipLaunchKernelGGL(k_init_kscale_final, dim3((G * D + 255) / 256), dim3(256), 0, h->stream,
                         sbits, (float*)a.kscale);
      hipLaunchKernelGGL(k_init_keyrec, dim3(8192), dim3(256), 0, h->stream, dk, a.kscale, T,
                         (uint8_t*)a.keyrec);
      hipLaunchKernelGGL(k_pack_kv8, dim3(8192), dim3(256), 0, h->stream, dk, dv, T, (size_t)T, 0,
                         a.kv_rows, (uint8_t*)a.kv8, a.kv_table, a.kv_shift);
      hipLaunchKernelGGL(k_init_postp2, dim3(4096), dim3(256), 0, h->stream, a.post_tok, a.keyrec, T,
                         np_max, dnp, (uint8_t*)a.post_p2);
      ok = hipGetLastError() == hipSuccess && hipStreamSynchronize(h->stream) == hipSuccess;
    }
    (void)hipFree(dk); (void)hipFree(dv); (void)hipFree(sbits); (void)hipFree(dnp);
    if (!ok) {
      fail(h, SKV_EHIP, "prefill kernels failed");
      return bail(SKV_EHIP);
    }
  }

  // ---- step plumbing
  StepWork& w = h->w;
  // LDS-resident selection: 16-bit scores beside the selection scratch
  const size_t sel_static = sizeof(SelectScratch) + 1024;
  const int lds_items = (int)std::min<size_t>(
      65536, (h->lds_per_block - std::min(h->lds_per_block, sel_static)) / 2 / 8 * 8);
  if (nc > lds_items) {
    fail(h, SKV_EINVAL, "n_centroids %d exceeds the LDS selection capacity %d", nc, lds_items);
    return bail(SKV_EINVAL);
  }
  w.top_u1 = TopkArgs{a.s2, a.pool_tok, a.cap, M15, a.bm_u1, words1, a.status, ST_POOL,
                      std::min(lds_items, a.cap), 0, FS_TOP1600, a.s2_tmax, a.cap / 16, 0};
  w.top_u2 = TopkArgs{a.s4, a.u1_tok, U1_MAX, M16, a.bm_u2, words2, a.status, ST_U1, U1_MAX,
                      0, FS_TOP256, nullptr, 0, 0};
  h->top_u1_lds_items = w.top_u1.lds_items;
  h->top_u2_lds_items = w.top_u2.lds_items;
  // Dynamic LDS of the selection kernels: the sampled-cut scratch, or the
  // LDS-resident scores of the full selection, or the attention scratch of
  // the sink/local blocks, whichever is largest (they are never live together).
  const size_t fs_bytes = sizeof(FastScratch);
  w.select_lds = std::max({fs_bytes, (size_t)nc * 2, ATTN_SCRATCH_BYTES, sizeof(QOperand)});
  w.top_u1_lds = topk_dynamic_lds(w.top_u1.lds_items);
  w.top_u2_lds = topk_dynamic_lds(w.top_u2.lds_items);
  // every launch must fit the block's LDS (static + dynamic): checked here,
  // on the host, rather than left to a failed dispatch
  for (int k = 0; k < N_STEP_KERNELS; ++k) {
    size_t st = 0, dy = 0;
    if (step_kernel_lds(a, w, k, &st, &dy) != hipSuccess) {
      fail(h, SKV_EHIP, "cannot query kernel %s", kKernelNames[k]);
      return bail(SKV_EHIP);
    }
    if (st + dy > h->lds_per_block) {
      fail(h, SKV_EINVAL, "kernel %s needs %zu bytes of LDS per block, the device has %zu",
           kKernelNames[k], st + dy, h->lds_per_block);
      return bail(SKV_EINVAL);
    }
  }

  h->q_slot = (size_t)(16 + (cap_app ? 2 * G * APPEND_FUSE : 0)) * D;
  h->pend_dev = cap_app ? const_cast<uint16_t*>(a.q) + 16 * D : nullptr;
  bool ring_ok = hipHostMalloc((void**)&h->q_host, (size_t)Q_RING * h->q_slot * 2,
                               hipHostMallocDefault) == hipSuccess;
  if (cap_app && ring_ok) {
    const size_t slot = (size_t)2 * G * std::min(cap_app, APPEND_CHUNK) * D;
    ring_ok = hipHostMalloc((void**)&h->append_host, 2 * slot * 2, hipHostMallocDefault) ==
                  hipSuccess &&
              hipHostGetDevicePointer((void**)&h->append_host_dev, h->append_host, 0) ==
                  hipSuccess;
    for (hipEvent_t& e : h->append_ev)
      ring_ok = ring_ok && hipEventCreateWithFlags(&e, hipEventDisableTiming) == hipSuccess;
  }
  for (int i = 0; i < Q_RING / Q_MARK && ring_ok; ++i)
    ring_ok = hipEventCreateWithFlags(&h->q_marked[i], hipEventDisableTiming) == hipSuccess;
  if (!ring_ok ||
      hipEventCreateWithFlags(&h->steps_done, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&h->q_ready, hipEventDisableTiming) != hipSuccess) {
    fail(h, SKV_EHIP, "pinned query staging failed");
    return bail(SKV_EHIP);
  }
  // write every pinned staging page once now: the first CPU write into a
  // fresh pinned page faults (measured ~100 us per 256 KiB, against ~5 us
  // for a rewrite), a cost that would otherwise fall on the first binds and
  // appends
  memset(h->q_host, 0, (size_t)Q_RING * h->q_slot * 2);
  if (h->append_host)
    memset(h->append_host, 0, (size_t)2 * 2 * G * std::min(cap_app, APPEND_CHUNK) * D * 2);

  build_meta(h);
  *handle_out = h;
  return SKV_OK;
}

int skv_create(const skv_index_desc* ix, const uint16_t* k_bf16, const uint16_t* v_bf16,
               int device, void* stream, void** handle_out) {
  return create_impl(ix, k_bf16, v_bf16, nullptr, device, stream, handle_out);
}

int skv_create_paged(const skv_index_desc* ix, const uint16_t* k_bf16, const uint16_t* v_bf16,
                     const skv_kv_pages* pages, int device, void* stream, void** handle_out) {
  if (!pages) {
    if (handle_out) *handle_out = nullptr;
    return fail(nullptr, SKV_EINVAL, "NULL page descriptor");
  }
  return create_impl(ix, k_bf16, v_bf16, pages, device, stream, handle_out);
}

int skv_bind_query(void* handle, const uint16_t* q) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return SKV_ESTATE;
  if (!q) return fail(h, SKV_EINVAL, "NULL query");
  // The next ring slot.  Its previous upload (Q_RING binds ago) is covered
  // by the event of its mark group, last recorded between Q_RING and
  // Q_RING - Q_MARK + 1 binds ago (an event never recorded counts as done):
  // the host waits only when it is Q_RING - Q_MARK + 1 or more steps ahead.
  HIPCHK(h, hipSetDevice(h->device));
  const unsigned slot = h->q_next % Q_RING;
  uint16_t* stage = h->q_host + (size_t)slot * h->q_slot;
  HIPCHK(h, hipEventSynchronize(h->q_marked[slot / Q_MARK]));
  memcpy(stage, q, 16 * D * 2);
  // a staged append in this slot travels with the query: one upload
  const size_t bytes = (16 + (h->pend_host ? (size_t)2 * G * h->pend_n : 0)) * D * 2;
  HIPCHK(h, hipMemcpyAsync((void*)h->a.q, stage, bytes, hipMemcpyHostToDevice, h->stream));
  if (slot % Q_MARK == Q_MARK - 1) HIPCHK(h, hipEventRecord(h->q_marked[slot / Q_MARK], h->stream));
  ++h->q_next;
  h->pend_host = false;
  h->bound = true;
  return SKV_OK;
}

// A staged append still in its ring slot goes up on its own (no query bind
// came after it); the slot is used up as a bind would use it.
static int upload_pending(Handle* h) {
  if (!h->pend_host) return SKV_OK;
  const unsigned slot = h->q_next % Q_RING;
  const uint16_t* stage = h->q_host + (size_t)slot * h->q_slot + 16 * D;
  HIPCHK(h, hipMemcpyAsync(h->pend_dev, stage, (size_t)2 * G * h->pend_n * D * 2,
                           hipMemcpyHostToDevice, h->stream));
  if (slot % Q_MARK == Q_MARK - 1) HIPCHK(h, hipEventRecord(h->q_marked[slot / Q_MARK], h->stream));
  ++h->q_next;
  h->pend_host = false;
  return SKV_OK;
}

// Packs a pending append's records now (before a reader other than the next
// step: the dense decode, a record readback, kernel timing, graph capture,
// another append).
static int flush_pending(Handle* h) {
  if (h->pend_n == 0) return SKV_OK;
  if (const int rc = upload_pending(h)) return rc;
  const StepArgs& a = h->a;
  const int n = h->pend_n;
  hipLaunchKernelGGL(k_pack_kv8, dim3((G * n * (D / 4) + 255) / 256), dim3(256), 0, h->stream,
                     h->pend_dev, h->pend_dev + (size_t)G * n * D, n, (size_t)n, h->pend_row,
                     a.kv_rows, (uint8_t*)a.kv8, a.kv_table, a.kv_shift);
  HIPCHK(h, hipGetLastError());
  h->pend_n = 0;
  return SKV_OK;
}

int skv_bind_query_device(void* handle, const void* q_dev, void* producer_stream) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return SKV_ESTATE;
  if (!q_dev) return fail(h, SKV_EINVAL, "NULL device query");
  if (const int rc = upload_pending(h)) return rc;
  const hipStream_t ps = static_cast<hipStream_t>(producer_stream);
  if (ps == h->stream) {
    HIPCHK(h, hipMemcpyAsync((void*)h->a.q, q_dev, 16 * D * 2, hipMemcpyDeviceToDevice, h->stream));
  } else {
    // The copy is ordered on the producer's stream (NULL: the legacy default
    // stream), after the work that wrote q_dev and after the handle's steps
    // enqueued so far (they read the query buffer); the handle's stream then
    // waits for the copy.  q_dev stays the caller's until the producer
    // stream reaches the copy (stream-ordered lifetime).
    HIPCHK(h, hipEventRecord(h->steps_done, h->stream));
    HIPCHK(h, hipStreamWaitEvent(ps, h->steps_done, 0));
    HIPCHK(h, hipMemcpyAsync((void*)h->a.q, q_dev, 16 * D * 2, hipMemcpyDeviceToDevice, ps));
    HIPCHK(h, hipEventRecord(h->q_ready, ps));
    HIPCHK(h, hipStreamWaitEvent(h->stream, h->q_ready, 0));
  }
  h->bound = true;
  return SKV_OK;
}

int skv_enqueue(void* handle) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return SKV_ESTATE;
  if (!h->bound) return fail(h, SKV_ESTATE, "bind a query before enqueue");
  HIPCHK(h, hipSetDevice(h->device));
  // a pending host append: packed by this step's k_front (eager launches),
  // or now, before a captured step that takes no append arguments
  if (h->use_graph) {
    if (const int rc = flush_pending(h)) return rc;
  } else if (h->pend_n) {
    if (const int rc = upload_pending(h)) return rc;
    h->a.app_src = h->pend_dev;
    h->a.app_n = h->pend_n;
    h->a.app_row = h->pend_row;
    h->pend_n = 0;
  }
  if (h->profiling) {
    if (h->prof_pending) {  // fold the previous step's events in first
      HIPCHK(h, hipEventSynchronize(h->prof_ev[N_STEP_KERNELS]));
      for (int i = 0; i < N_STEP_KERNELS; ++i) {
        float ms = 0.f;
        HIPCHK(h, hipEventElapsedTime(&ms, h->prof_ev[i], h->prof_ev[i + 1]));
        h->prof_ms[i] += ms;
      }
      ++h->prof_steps;
    }
    launch_step(h->a, h->w, h->stream, h->prof_ev);
    h->prof_pending = true;
  } else if (h->use_graph) {
    if (!h->graph_exec) {  // capture the kernels once on a private stream
      if (!h->capture_stream)
        HIPCHK(h, hipStreamCreateWithFlags(&h->capture_stream, hipStreamNonBlocking));
      HIPCHK(h, hipStreamBeginCapture(h->capture_stream, hipStreamCaptureModeThreadLocal));
      launch_step(h->a, h->w, h->capture_stream, nullptr);
      HIPCHK(h, hipStreamEndCapture(h->capture_stream, &h->graph));
      HIPCHK(h, hipGraphInstantiate(&h->graph_exec, h->graph, nullptr, nullptr, 0));
    }
    HIPCHK(h, hipGraphLaunch(h->graph_exec, h->stream));
  } else {
    launch_step(h->a, h->w, h->stream, nullptr);
  }
  h->a.app_n = 0;  // later steps (and kernel timings) pack nothing
  h->a.app_src = nullptr;
  HIPCHK(h, hipGetLastError());
  h->ran = true;
  return SKV_OK;
}

int skv_graph_mode(void* handle, int enable) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return SKV_ESTATE;
  if (const int rc = flush_pending(h)) return rc;
  HIPCHK(h, hipStreamSynchronize(h->stream));
  h->use_graph = enable != 0;
  drop_graph(h);
  return SKV_OK;
}

int skv_profile(void* handle, int enable) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return SKV_ESTATE;
  HIPCHK(h, hipStreamSynchronize(h->stream));
  if (enable && !h->prof_ev[0])
    for (int i = 0; i <= N_STEP_KERNELS; ++i) HIPCHK(h, hipEventCreate(&h->prof_ev[i]));
  h->profiling = enable != 0;
  h->prof_pending = false;
  h->prof_steps = 0;
  for (double& v : h->prof_ms) v = 0.0;
  return SKV_OK;
}

int skv_time_kernel(void* handle, int kernel, int reps, float* mean_ms) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return SKV_ESTATE;
  if (kernel < 0 || kernel >= N_STEP_KERNELS || reps < 1 || !mean_ms)
    return fail(h, SKV_EINVAL, "kernel %d / reps %d out of range", kernel, reps);
  if (!h->ran) return fail(h, SKV_ESTATE, "no decode step has run");
  if (const int rc = flush_pending(h)) return rc;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  HIPCHK(h, hipEventCreate(&e0));
  HIPCHK(h, hipEventCreate(&e1));
  // the kernel's inputs are those of the last step; every step kernel is a
  // function of its inputs, so repeated launches recompute the same outputs
  HIPCHK(h, hipEventRecord(e0, h->stream));
  for (int r = 0; r < reps; ++r) launch_kernel(h->a, h->w, h->stream, kernel);
  HIPCHK(h, hipEventRecord(e1, h->stream));
  HIPCHK(h, hipEventSynchronize(e1));
  float ms = 0.f;
  HIPCHK(h, hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *mean_ms = ms / (float)reps;
  // a full step restores every downstream buffer (query prep clears state)
  launch_step(h->a, h->w, h->stream, nullptr);
  HIPCHK(h, hipStreamSynchronize(h->stream));
  return SKV_OK;
}

int skv_dense_decode(void* handle) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return SKV_ESTATE;
  if (!h->bound) return fail(h, SKV_ESTATE, "bind a query before the dense decode");
  HIPCHK(h, hipSetDevice(h->device));
  if (const int rc = flush_pending(h)) return rc;
  launch_dense(h->dn, h->stream, 0);
  launch_dense(h->dn, h->stream, 1);
  HIPCHK(h, hipGetLastError());
  h->dense_ran = true;
  return SKV_OK;
}

// Cache append: FP8 records of n new tokens at rows T .. T+n-1, then the
// context and the local window grow by n (the index, the key codec and the
// retrieval region are the prefill's).  k, v: [G][n][256] BF16, device
// pointers when on_device, else host memory staged APPEND_CHUNK tokens at a
// time.  Work already enqueued keeps the shape it was launched with.
// device_range_error for the K/V of skv_append_device, remembering the
// allocations it accepted: a range inside one of the last DEV_OK_SLOTS
// accepted allocations is not queried again (a decoder appends from the same
// buffers every step).
static const char* checked_device_range(Handle* h, const void* ptr, uint64_t bytes) {
  const uintptr_t lo = (uintptr_t)ptr;
  for (int i = 0; i < h->dev_ok_n; ++i)
    if (lo >= h->dev_ok[i].lo && lo < h->dev_ok[i].hi && bytes <= h->dev_ok[i].hi - lo)
      return nullptr;
  if (const char* why = device_range_error(ptr, bytes, h->device)) return why;
  void* base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(ptr)) == hipSuccess) {
    DevRange& r = h->dev_ok[h->dev_ok_next];
    r.lo = (uintptr_t)base;
    r.hi = (uintptr_t)base + size;
    h->dev_ok_next = (h->dev_ok_next + 1) % DEV_OK_SLOTS;
    h->dev_ok_n = std::min(h->dev_ok_n + 1, DEV_OK_SLOTS);
  } else {
    (void)hipGetLastError();
  }
  return nullptr;
}

static int append_tokens(Handle* h, const uint16_t* k, const uint16_t* v, int n, bool on_device) {
  if (!h) return SKV_ESTATE;
  if (!k || !v) return fail(h, SKV_EINVAL, "NULL K/V");
  if (on_device && (((uintptr_t)k | (uintptr_t)v) & 7))
    return fail(h, SKV_EINVAL, "device K/V must be 8-byte aligned");
  StepArgs& a = h->a;
  if (n < 1 || n > h->context0 + h->append_capacity - a.T)
    return fail(h, SKV_EINVAL, "append of %d tokens: %d of the capacity %d left", n,
                h->context0 + h->append_capacity - a.T, h->append_capacity);
  HIPCHK(h, hipSetDevice(h->device));
  if (const int rc = flush_pending(h)) return rc;  // appends pack in order
  if (!on_device && n <= APPEND_FUSE && !h->use_graph) {
    // staged in the next query ring slot; the next bind uploads it with the
    // query and the next step's k_front packs it
    const unsigned slot = h->q_next % Q_RING;
    uint16_t* stage = h->q_host + (size_t)slot * h->q_slot + 16 * D;
    HIPCHK(h, hipEventSynchronize(h->q_marked[slot / Q_MARK]));
    memcpy(stage, k, (size_t)G * n * D * 2);
    memcpy(stage + (size_t)G * n * D, v, (size_t)G * n * D * 2);
    h->pend_n = n;
    h->pend_row = a.T;
    h->pend_host = true;
  } else if (on_device) {
    const uint64_t bytes = (uint64_t)G * n * D * 2;
    for (const uint16_t* src : {k, v})
      if (const char* why = checked_device_range(h, src, bytes))
        return fail(h, SKV_EINVAL, "device %s of %d tokens (%llu bytes) %s", src == k ? "K" : "V",
                    n, (unsigned long long)bytes, why);
    hipLaunchKernelGGL(k_pack_kv8, dim3(std::min(1024, (G * n * (D / 4) + 255) / 256)), dim3(256),
                       0, h->stream, k, v, n, (size_t)n, a.T, a.kv_rows, (uint8_t*)a.kv8,
                       a.kv_table, a.kv_shift);
    HIPCHK(h, hipGetLastError());
  } else {
    // chunks of the caller's [G][n][D] arrays gathered into a pinned slot as
    // [K: G][c][D] then [V: G][c][D]; the pack kernel reads the slot over
    // the bus (no device staging buffer and no copy-engine transfer, whose
    // first use in a process took milliseconds), and the slot is reused once
    // that kernel has finished
    const int chunk = std::min(h->append_capacity, APPEND_CHUNK);
    for (int t0 = 0; t0 < n; t0 += chunk) {
      const int c = std::min(chunk, n - t0);
      const unsigned slot = h->append_next++ % 2;
      const size_t off = (size_t)slot * 2 * G * chunk * D;
      uint16_t* hk = h->append_host + off;
      uint16_t* hv = hk + (size_t)G * c * D;
      HIPCHK(h, hipEventSynchronize(h->append_ev[slot]));
      for (int g = 0; g < G; ++g) {
        memcpy(hk + (size_t)g * c * D, k + ((size_t)g * n + t0) * D, (size_t)c * D * 2);
        memcpy(hv + (size_t)g * c * D, v + ((size_t)g * n + t0) * D, (size_t)c * D * 2);
      }
      const uint16_t* dk = h->append_host_dev + off;
      hipLaunchKernelGGL(k_pack_kv8, dim3(std::min(1024, (G * c * (D / 4) + 255) / 256)),
                         dim3(256), 0, h->stream, dk, dk + (size_t)G * c * D, c, (size_t)c,
                         a.T + t0, a.kv_rows, (uint8_t*)a.kv8, a.kv_table, a.kv_shift);
      HIPCHK(h, hipGetLastError());
      HIPCHK(h, hipEventRecord(h->append_ev[slot], h->stream));
    }
  }
  a.T += n;
  a.local += n;
  a.dense_slices = (a.sink + a.local + DENSE_SLICE_KEYS - 1) / DENSE_SLICE_KEYS;
  h->dn.T = a.T;
  dense_shape(a.T, h->dn.iters, h->dn.nb);
  drop_graph(h);  // the step's launch shapes changed
  build_meta(h);
  return SKV_OK;
}

int skv_append(void* handle, const uint16_t* k_bf16, const uint16_t* v_bf16, int n) {
  return append_tokens(static_cast<Handle*>(handle), k_bf16, v_bf16, n, false);
}

int skv_append_device(void* handle, const void* k_dev, const void* v_dev, int n) {
  return append_tokens(static_cast<Handle*>(handle), static_cast<const uint16_t*>(k_dev),
                       static_cast<const uint16_t*>(v_dev), n, true);
}

int skv_dense_output_device(void* handle, void** dev_ptr) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !dev_ptr) return SKV_EINVAL;
  *dev_ptr = h->dn.out;
  return SKV_OK;
}

int skv_read_dense_output(void* handle, uint16_t* host_out) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !host_out) return SKV_EINVAL;
  if (!h->dense_ran) return fail(h, SKV_ESTATE, "no dense decode has run");
  HIPCHK(h, hipStreamSynchronize(h->stream));
  HIPCHK(h, hipMemcpy(host_out, h->dn.out, 16 * D * 2, hipMemcpyDeviceToHost));
  return SKV_OK;
}

int skv_time_dense(void* handle, int reps, float* mean_ms) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return SKV_ESTATE;
  if (reps < 1 || !mean_ms) return fail(h, SKV_EINVAL, "reps %d out of range", reps);
  if (!h->dense_ran) return fail(h, SKV_ESTATE, "no dense decode has run");
  hipEvent_t ev[4] = {};
  for (hipEvent_t& e : ev) HIPCHK(h, hipEventCreate(&e));
  // both kernels are functions of their inputs: repeats recompute the same
  // partials and output
  HIPCHK(h, hipEventRecord(ev[0], h->stream));
  for (int r = 0; r < reps; ++r) launch_dense(h->dn, h->stream, 0);
  HIPCHK(h, hipEventRecord(ev[1], h->stream));
  for (int r = 0; r < reps; ++r) launch_dense(h->dn, h->stream, 1);
  HIPCHK(h, hipEventRecord(ev[2], h->stream));
  for (int r = 0; r < reps; ++r) {
    launch_dense(h->dn, h->stream, 0);
    launch_dense(h->dn, h->stream, 1);
  }
  HIPCHK(h, hipEventRecord(ev[3], h->stream));
  HIPCHK(h, hipEventSynchronize(ev[3]));
  for (int i = 0; i < 3; ++i) {
    float ms = 0.f;
    HIPCHK(h, hipEventElapsedTime(&ms, ev[i], ev[i + 1]));
    mean_ms[i] = ms / (float)reps;
  }
  for (hipEvent_t e : ev) (void)hipEventDestroy(e);
  return SKV_OK;
}

int skv_select_mode(void* handle, int exact) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return SKV_ESTATE;
  HIPCHK(h, hipStreamSynchronize(h->stream));
  if (exact < 0 || exact > 3) return fail(h, SKV_EINVAL, "select mode %d not in 0..3", exact);
  // mode 3: the full selections, with the token top-k kernels' scores never
  // held in LDS (their in-memory radix passes run at every size)
  const int e = exact == 3 ? 1 : exact;
  h->a.exact_select = e;
  h->w.top_u1.exact_select = e;
  h->w.top_u2.exact_select = e;
  h->w.top_u1.lds_items = exact == 3 ? 0 : h->top_u1_lds_items;
  h->w.top_u2.lds_items = exact == 3 ? 0 : h->top_u2_lds_items;
  drop_graph(h);  // the kernels take the options by value
  return SKV_OK;
}

int skv_profile_read(void* handle, float* mean_ms, int n, int32_t* steps) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !mean_ms || n < N_STEP_KERNELS) return SKV_EINVAL;
  HIPCHK(h, hipStreamSynchronize(h->stream));
  if (h->profiling && h->prof_pending) {
    for (int i = 0; i < N_STEP_KERNELS; ++i) {
      float ms = 0.f;
      HIPCHK(h, hipEventElapsedTime(&ms, h->prof_ev[i], h->prof_ev[i + 1]));
      h->prof_ms[i] += ms;
    }
    ++h->prof_steps;
    h->prof_pending = false;
  }
  for (int i = 0; i < N_STEP_KERNELS; ++i)
    mean_ms[i] = h->prof_steps ? (float)(h->prof_ms[i] / h->prof_steps) : 0.f;
  if (steps) *steps = h->prof_steps;
  return SKV_OK;
}

int skv_kernel_count(void) { return N_STEP_KERNELS; }

const char* skv_kernel_name(int i) {
  return (i >= 0 && i < N_STEP_KERNELS) ? kKernelNames[i] : "";
}

int skv_sync(void* handle, int32_t* status) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return SKV_ESTATE;
  HIPCHK(h, hipStreamSynchronize(h->stream));
  if (status) {
    HIPCHK(h, hipMemcpy(status, h->a.status, G * ST_WORDS * 4, hipMemcpyDeviceToHost));
    // the top-1600 instance for the pool sizes just seen: pools of OCT_ITEMS
    // to 2 x OCT_ITEMS keys are selected in registers by the instance that
    // carries that path (a speed choice only: both select the same members)
    int pmax = 0;
    for (int g = 0; g < G; ++g) pmax = std::max(pmax, (int)status[g * ST_WORDS + ST_POOL]);
    const int regs2 = pmax > OCT_ITEMS && pmax <= 2 * OCT_ITEMS;
    if (regs2 != h->w.top_u1.regs2) {
      h->w.top_u1.regs2 = regs2;
      drop_graph(h);  // the captured step holds the other instance
      build_meta(h);
    }
  }
  return SKV_OK;
}

int skv_output_device(void* handle, void** dev_ptr) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !dev_ptr) return SKV_EINVAL;
  *dev_ptr = h->a.out;
  return SKV_OK;
}

int skv_output_tiles_device(void* handle, void** dev_ptr) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !dev_ptr) return SKV_EINVAL;
  *dev_ptr = h->a.out_tiles;
  return SKV_OK;
}

int skv_read_output(void* handle, uint16_t* host_out) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !host_out) return SKV_EINVAL;
  if (!h->ran) return fail(h, SKV_ESTATE, "no decode step has run");
  HIPCHK(h, hipStreamSynchronize(h->stream));
  HIPCHK(h, hipMemcpy(host_out, h->a.out, 16 * D * 2, hipMemcpyDeviceToHost));
  return SKV_OK;
}

int skv_debug_ids(void* handle, uint32_t* host_out) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !host_out) return SKV_EINVAL;
  if (!h->ran) return fail(h, SKV_ESTATE, "no decode step has run");
  HIPCHK(h, hipStreamSynchronize(h->stream));
  HIPCHK(h, hipMemcpy(host_out, h->a.top, G * H * TOPK * 4, hipMemcpyDeviceToHost));
  return SKV_OK;
}

int skv_read_stage(void* handle, int stage, int group, void* host_out, int64_t cap,
                   int64_t* count_out) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !host_out || group < 0 || group >= G || cap < 0) return SKV_EINVAL;
  if (stage == SKV_STAGE_KV8)
    if (const int rc = flush_pending(h)) return rc;  // a pending append's records
  HIPCHK(h, hipStreamSynchronize(h->stream));
  const StepArgs& a = h->a;
  int st[ST_WORDS];
  HIPCHK(h, hipMemcpy(st, a.status + group * ST_WORDS, sizeof st, hipMemcpyDeviceToHost));
  const int nc = a.nc;
  auto copy_rows = [&](const void* base, size_t row_stride, size_t elem, int64_t n, int rows) -> int {
    if ((int64_t)rows * n > cap) return fail(h, SKV_EINVAL, "stage buffer too small");
    for (int r = 0; r < rows; ++r) {
      hipError_t e = hipMemcpy((char*)host_out + (size_t)r * n * elem,
                               (const char*)base + r * row_stride * elem, (size_t)n * elem,
                               hipMemcpyDeviceToHost);
      if (e != hipSuccess) return fail(h, SKV_EHIP, "stage copy failed: %s", hipGetErrorString(e));
    }
    if (count_out) *count_out = n;
    return SKV_OK;
  };
  switch (stage) {
    case SKV_STAGE_LOWER:
    case SKV_STAGE_UPPER: {  // held as ordered BF16 on the device
      const int rc = copy_rows((stage == SKV_STAGE_LOWER ? a.lower : a.upper) +
                                   (size_t)group * H * nc, nc, 2, nc, H);
      if (rc != SKV_OK) return rc;
      uint16_t* o = static_cast<uint16_t*>(host_out);
      for (int64_t i = 0; i < (int64_t)H * nc; ++i)
        o[i] = (o[i] & 0x8000u) ? (uint16_t)(o[i] ^ 0x8000u) : (uint16_t)(~o[i] & 0xffffu);
      return SKV_OK;
    }
    case SKV_STAGE_THRESH:
      return copy_rows(a.thr + group * H, 0, 4, H, 1);
    case SKV_STAGE_MASKS:
      return copy_rows(a.masks + (size_t)group * nc, 0, 1, nc, 1);
    case SKV_STAGE_FINE: {  // BF16 fine scores; 0xffff where the head is ineligible
      if (!a.debug) return fail(h, SKV_ESTATE, "fine scores need debug=1");
      const int rc = copy_rows(a.fine_bits + (size_t)group * H * nc, nc, 2, nc, H);
      if (rc != SKV_OK) return rc;
      std::vector<uint8_t> m(nc);
      HIPCHK(h, hipMemcpy(m.data(), a.masks + (size_t)group * nc, nc, hipMemcpyDeviceToHost));
      uint16_t* o = static_cast<uint16_t*>(host_out);
      for (int hh = 0; hh < H; ++hh)
        for (int c = 0; c < nc; ++c)
          if (!((m[c] >> hh) & 1)) o[(size_t)hh * nc + c] = 0xffff;
      return SKV_OK;
    }
    case SKV_STAGE_SELECTED:
      return copy_rows(a.sel + (size_t)group * nc, 0, 4, st[ST_SEL], 1);
    case SKV_STAGE_POOL:
      return copy_rows(a.pool_tok + (size_t)group * a.cap, 0, 4, st[ST_POOL], 1);
    case SKV_STAGE_S2:
      return copy_rows(a.s2 + (size_t)group * H * a.cap, a.cap, 2, st[ST_POOL], H);
    case SKV_STAGE_U1:
      return copy_rows(a.u1_tok + (size_t)group * U1_MAX, 0, 4, st[ST_U1], 1);
    case SKV_STAGE_S4:
      return copy_rows(a.s4 + (size_t)group * H * U1_MAX, U1_MAX, 2, st[ST_U1], H);
    case SKV_STAGE_U2:
    case SKV_STAGE_S8: {
      // U2 is not listed on the device: its members are the U1 positions set
      // in any head's top-256 bitmap, in U1 order, and their 8-bit scores sit
      // at those positions of the U1-indexed score rows
      const int n1 = st[ST_U1], W = a.words_u2;
      std::vector<uint64_t> bm((size_t)H * W);
      HIPCHK(h, hipMemcpy(bm.data(), a.bm_u2 + (size_t)group * H * W, bm.size() * 8,
                          hipMemcpyDeviceToHost));
      std::vector<int> pos;
      for (int i = 0; i < n1; ++i) {
        const int w = i >> 6;
        if (((bm[w] | bm[W + w] | bm[2 * W + w] | bm[3 * W + w]) >> (i & 63)) & 1u) pos.push_back(i);
      }
      const int64_t n2 = (int64_t)pos.size();
      if (n2 != st[ST_U2])
        return fail(h, SKV_EINVAL, "U2 count word %d differs from the bitmaps' %lld", st[ST_U2],
                    (long long)n2);
      const bool toks = stage == SKV_STAGE_U2;
      if ((toks ? 1 : H) * n2 > cap) return fail(h, SKV_EINVAL, "stage buffer too small");
      if (toks) {
        std::vector<int> u1(std::max(n1, 1));
        HIPCHK(h, hipMemcpy(u1.data(), a.u1_tok + (size_t)group * U1_MAX, (size_t)n1 * 4,
                            hipMemcpyDeviceToHost));
        int* o = static_cast<int*>(host_out);
        for (int64_t k = 0; k < n2; ++k) o[k] = u1[pos[k]];
      } else {
        std::vector<uint16_t> row(std::max(n1, 1));
        uint16_t* o = static_cast<uint16_t*>(host_out);
        for (int hh = 0; hh < H; ++hh) {
          HIPCHK(h, hipMemcpy(row.data(), a.s8 + ((size_t)group * H + hh) * U1_MAX, (size_t)n1 * 2,
                              hipMemcpyDeviceToHost));
          for (int64_t k = 0; k < n2; ++k) o[hh * n2 + k] = row[pos[k]];
        }
      }
      if (count_out) *count_out = n2;
      return SKV_OK;
    }
    case SKV_STAGE_TOP:
      return copy_rows(a.top + group * H * TOPK, 0, 4, H * TOPK, 1);
    case SKV_STAGE_QPREP: {
      // [variant][head][X[256], fx, S lo, S hi, norm bits]
      if (cap < QV_COUNT * H * 260) return fail(h, SKV_EINVAL, "stage buffer too small");
      std::vector<QOperand> q(QV_COUNT);
      HIPCHK(h, hipMemcpy(q.data(), a.qop + group * QV_COUNT, sizeof(QOperand) * QV_COUNT,
                          hipMemcpyDeviceToHost));
      int32_t* o = (int32_t*)host_out;
      for (int v = 0; v < QV_COUNT; ++v)
        for (int hh = 0; hh < H; ++hh) {
          int32_t* r = o + (v * H + hh) * 260;
          memcpy(r, q[v].X[hh], D * 4);
          r[256] = q[v].fx[hh];
          r[257] = (int32_t)(uint32_t)((uint64_t)q[v].sum[hh] & 0xffffffffu);
          r[258] = (int32_t)(uint32_t)((uint64_t)q[v].sum[hh] >> 32);
          memcpy(&r[259], &q[v].norm[hh], 4);
        }
      if (count_out) *count_out = QV_COUNT * H * 260;
      return SKV_OK;
    }
    case SKV_STAGE_KEYREC: {
      if (cap < (int64_t)a.rec_rows * 256) return fail(h, SKV_EINVAL, "stage buffer too small");
      return copy_rows(a.keyrec + (size_t)group * a.rec_rows * 256, 0, 1,
                       (int64_t)a.rec_rows * 256, 1);
    }
    case SKV_STAGE_KV8:
      if (a.kv_table) {  // paged: the group's slots page by page, in token order
        if ((int64_t)a.T * 512 > cap) return fail(h, SKV_EINVAL, "stage buffer too small");
        const int pt = 1 << a.kv_shift;
        for (int t0 = 0; t0 < a.T; t0 += pt) {
          const size_t row = kv_row_paged(h->page_table.data(), a.kv_shift, group, t0);
          HIPCHK(h, hipMemcpy((char*)host_out + (size_t)t0 * 512, a.kv8 + row * 512,
                              (size_t)std::min(pt, a.T - t0) * 512, hipMemcpyDeviceToHost));
        }
        if (count_out) *count_out = (int64_t)a.T * 512;
        return SKV_OK;
      }
      return copy_rows(a.kv8 + (size_t)group * a.kv_rows * 512, 0, 1, (int64_t)a.T * 512, 1);
    case SKV_STAGE_KSCALE:
      return copy_rows(a.kscale + group * D, 0, 4, D, 1);
    default:
      return fail(h, SKV_EINVAL, "unknown stage %d", stage);
  }
}

const char* skv_metadata(void* handle) {
  Handle* h = static_cast<Handle*>(handle);
  return h ? h->meta.c_str() : "{}";
}

}  // extern "C"
