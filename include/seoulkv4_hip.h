/*
 * seoulkv4_hip.h - C ABI of the MI355X (gfx950) SeoulKV4 sparse decode path.
 *
 * This library replaces the reference's runtime seam
 *   src/seoulkv4/_runtime.py:36   initialize(ttnn, device, k, v, q, index, args)
 *   src/seoulkv4/_runtime.py:180  bind_query(state, q, args)
 *   src/seoulkv4/_runtime.py:189  enqueue(state)
 *   src/seoulkv4/_runtime.py:197  metadata(state)
 * plus the device reads done by the public API:
 *   src/seoulkv4/api.py:104       synchronize()
 *   src/seoulkv4/result.py:30     DecodeResult.to_torch()
 *   src/seoulkv4/api.py:119       debug_snapshot()
 *
 * Plain pointers and sizes only.  Host arrays are read during the call and not
 * retained.  Every function returns 0 on success or a SKV_E* code; after a
 * failure skv_last_error() describes it.  One handle serves one immutable
 * cache; calls on one handle must not overlap (reference docs/POC_API.md:15-17).
 */
#ifndef SEOULKV4_HIP_H
#define SEOULKV4_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SKV_GROUPS 4       /* KV heads ("cells") */
#define SKV_HEADS 4        /* query heads per KV head (GQA 4:1) */
#define SKV_DIM 256        /* head dimension */
#define SKV_TOPK 100       /* retrieval tokens per query head */

enum {
  SKV_OK = 0,
  SKV_EINVAL = 1,          /* bad argument or shape */
  SKV_EHIP = 2,            /* HIP runtime error */
  SKV_ENOMEM = 3,          /* device allocation failed */
  SKV_EPOOL_OVERFLOW = 4,  /* candidate pool above capacity (reference ingest err 4) */
  SKV_EPOOL_UNDERFLOW = 5, /* candidate pool below 2048 (reference ingest err 5) */
  SKV_ESTATE = 6,          /* call out of order / handle closed */
  SKV_EPOOL_WAIT = 7       /* device status only: the pool kernel abandoned a bounded
                              wait for an earlier centroid range (never expected) */
};

/* One index cell (KV head) as produced by SeoulKV4Index
 * (reference _codecs/index.py:294-312 field names). */
typedef struct {
  const uint8_t *upper;        /* [nc][64] 2-bit codes, bits 3..2 of the 4-bit code */
  const uint8_t *lower;        /* [nc][64] 2-bit codes, bits 1..0 */
  const float *scale;          /* [nc] fp32 group scale ("scale") */
  const uint16_t *resid_f16;   /* [nc] fp16 "coarse_residual_norm" */
  const uint16_t *gfs_f16;     /* [nc/32] fp16 "group_fine_scale" */
  const int32_t *offsets;      /* [nc+1] CSR offsets */
  const int32_t *values;       /* [offsets[nc]] CSR token IDs */
  int32_t nprobe;              /* P: probes per query head */
  float lam;                   /* coarse margin lambda */
} skv_cell_desc;

typedef struct {
  int32_t context;             /* T, tokens per KV head */
  int32_t sink;                /* S: tokens [0, S) always attended */
  int32_t local;               /* L: tokens [T-L, T) always attended */
  int32_t n_centroids;         /* nc per cell, multiple of 32, <= 65536 */
  int32_t pool_min;            /* pool lower bound (2048 in the reference) */
  int32_t pool_capacity;       /* pool upper bound; <= 0 means no bound */
  int32_t debug;               /* nonzero: keep stage outputs readable */
  skv_cell_desc cells[SKV_GROUPS];
  int32_t append_capacity;     /* tokens per KV head skv_append may add (0: static
                                  cache, the reference's only mode); context plus
                                  capacity <= 2^20 */
} skv_index_desc;

/* Reference _runtime.initialize (_runtime.py:36-177): uploads the index, runs
 * the key codec and packs FP8 [V||K] records on the device.
 * k_bf16, v_bf16: host [4][T][256] BF16 bit patterns.  device: HIP ordinal.
 * stream: hipStream_t to enqueue on (NULL = a stream owned by the handle). */
int skv_create(const skv_index_desc *index, const uint16_t *k_bf16,
               const uint16_t *v_bf16, int device, void *stream,
               void **handle_out);

/* Paged FP8 K/V records (the next step after the reference's contiguous
 * static cache; its README.md:66-69 leaves paged attention out).  The
 * records live in a caller-owned device pool of pages:
 *   pool = [n_pages][4 KV heads][page_tokens][512 B] FP8 [V || K],
 * and logical page p (tokens p*page_tokens ..) of this cache is physical
 * page page_table[p].  page_tokens is a power of two in [16, 65536];
 * page_table (host, read during the call) holds ceil((context +
 * append_capacity) / page_tokens) distinct entries in [0, n_pages); the pool
 * is at most 2^31 records (n_pages x 4 x page_tokens) and must be device
 * memory of the handle's device whose allocation holds all n_pages pages
 * from the pool address on (both checked: SKV_EINVAL otherwise).  The handle
 * writes only its own pages, so several handles (sequences) may share one
 * pool with disjoint tables; the pool must outlive the handle. */
typedef struct {
  void *pool;                  /* device pointer, 256-byte aligned */
  int64_t n_pages;             /* pages in the pool */
  int32_t page_tokens;         /* tokens per page */
  const int32_t *page_table;   /* host [table_len] physical page of each logical page */
  int32_t table_len;
} skv_kv_pages;

/* skv_create with the FP8 records in caller pages: the prefill records are
 * written into them, skv_append fills them further, and the decode step and
 * the dense decode read every record through the page table.  The key codes
 * of the index (its retrieval region, fixed at prefill) stay in the handle's
 * own memory.  Results are bit-identical to skv_create's contiguous layout. */
int skv_create_paged(const skv_index_desc *index, const uint16_t *k_bf16,
                     const uint16_t *v_bf16, const skv_kv_pages *pages,
                     int device, void *stream, void **handle_out);

/* Reference bind_query (_runtime.py:180-186): copies host Q [16][256] BF16
 * (query head j belongs to KV head j/4) to the device, asynchronously,
 * through a ring of 16 pinned staging slots: q_bf16 may be reused on return,
 * and the call blocks only when the host is 9 or more binds ahead of the
 * device. */
int skv_bind_query(void *handle, const uint16_t *q_bf16);

/* Device-resident variant: q_dev is a device pointer to [16][256] BF16,
 * written by work on producer_stream (a hipStream_t; NULL = the legacy default
 * stream).  The 8 KiB copy is enqueued on producer_stream after the handle's
 * steps enqueued so far (they read the query buffer), and the handle's stream
 * waits for it, so the next skv_enqueue sees this query.  q_dev must stay valid
 * until producer_stream reaches the copy (stream-ordered lifetime, as for a
 * tensor used on its own stream).  Pass the handle's own stream to copy there
 * without events. */
int skv_bind_query_device(void *handle, const void *q_dev, void *producer_stream);

/* Reference enqueue (_runtime.py:189-194): launches every stage of one decode
 * step on the handle's stream.  No host synchronisation, no readback. */
int skv_enqueue(void *handle);

/* Reference synchronize (api.py:104-107).  Waits for the stream and, if
 * status is non-NULL, stores the per-group device status words [4][8]:
 * 0 pool size, 1 error code (0, 4 pool above capacity, 5 pool below the
 * minimum, 7 pool kernel wait abandoned), 2 selected clusters, 3 coarse survivors, 4 |U1|, 5 |U2|,
 * 6 postings scanned, 7 full-selection bits (see skv_select_mode). */
int skv_sync(void *handle, int32_t *status);

/* Device pointer of the output [16][256] BF16 (valid until skv_destroy;
 * overwritten by the next skv_enqueue). */
int skv_output_device(void *handle, void **dev_ptr);

/* Device pointer of the same output in the reference's per-KV-head layout
 * (DecodeResult.device_tensors, result.py:25-28): [4][1][32][4][256] BF16,
 * query head 4g + h at [g][0][h][h], every other row zero.  Written by each
 * skv_enqueue with the compact output; valid until skv_destroy. */
int skv_output_tiles_device(void *handle, void **dev_ptr);

/* Reference DecodeResult.to_torch (result.py:30-38): sync + copy [16][256]. */
int skv_read_output(void *handle, uint16_t *host_out);

/* Reference debug_snapshot (api.py:119-126): sync + copy final token IDs
 * [4 groups][4 heads][100], best first. */
int skv_debug_ids(void *handle, uint32_t *host_out);

/* Cache append (the next step after the reference's static PoC cache, which
 * leaves cache append out: README.md:68-69).  Writes the FP8 [V || K]
 * records of n new tokens after the current context T and grows the context
 * and the local window by n: later steps attend [0, S) + [T0 - L, T) densely
 * plus the top-100 of the prefill index, whose key codec, CSR and retrieval
 * region [S, T0 - L) stay as built (T0 = the context at skv_create, L = its
 * local window).  k, v: [4][n][256] BF16, host memory (skv_append) or
 * device memory (skv_append_device, 8-byte aligned, of the handle's device,
 * each array inside one allocation).  skv_append copies k and v before it
 * returns.  Up to 16 host tokens wait in the pinned query staging slot of
 * the next skv_bind_query, travel with that query's upload and are packed
 * by the next step's first kernel (a decoder's per-token append costs the
 * step about 1 %); any other reader of the records (the dense decode, a
 * record readback, kernel timing, graph capture, another append) packs them
 * first.  Longer host appends are copied into pinned host slots of up to
 * 256 tokens, which the pack kernel reads over the bus.  skv_append_device
 * reads k and v on the handle's stream; the allocations it has accepted (the last 8) are remembered, and
 * arrays inside one of them are not queried again.  Enqueued on the
 * handle's stream; fails with SKV_EINVAL, the cache unchanged, when n < 1,
 * n exceeds the capacity left or a device array is not such memory. */
int skv_append(void *handle, const uint16_t *k_bf16, const uint16_t *v_bf16,
               int n);
int skv_append_device(void *handle, const void *k_dev, const void *v_dev,
                      int n);

/* Dense FP8 decode (a comparison path with no counterpart in the reference,
 * whose published comparison is TTNN's dense FlashDecode, README.md:7):
 * softmax attention of the bound query's 16 heads over all T keys, from the
 * same FP8 [V || K] records as the sparse step (scale 1/16, FP32
 * accumulation), into its own [16][256] BF16 output.  Enqueued on the
 * handle's stream; skv_read_dense_output syncs and copies. */
int skv_dense_decode(void *handle);
int skv_dense_output_device(void *handle, void **dev_ptr);
int skv_read_dense_output(void *handle, uint16_t *host_out);

/* Allocation-free dense FP8 decode.  No counterpart in the reference: this
 * entry point is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops or harnesses that forbid hipMalloc).  It
 * computes what skv_dense_decode computes, from caller buffers on the current
 * device: kv8 = [4][rows][512] FP8 e4m3fn [V (256 B) || K (256 B)] records,
 * of which rows 0 .. T-1 of each KV head are attended; q_dev = [16][256] BF16;
 * out_dev = [16][256] BF16.  stream: hipStream_t (NULL = default stream).
 * It calls no allocator: the per-block partials live in a file-scope device
 * array of 1 MiB (4 x 64 x 4 x 258 FP32) that each GPU holds until the
 * process ends, its address looked up on the first call on a device.  Every
 * call on one GPU shares that array: calls that overlap on one GPU (other
 * streams, other threads) race.  Requires 1 <= T <= 2^20, rows >= T, and
 * kv8 (4 x rows x 512 bytes), q_dev and out_dev (8 KiB each) in device
 * allocations of the current device that hold them, else SKV_EINVAL (runtime
 * pointer queries, no allocation); errors are read with
 * skv_last_error(NULL). */
int skv_dense_decode_static(const void *kv8, int rows, int T, const void *q_dev,
                            void *out_dev, void *stream);

/* Mean milliseconds per launch over `reps` back-to-back launches of
 * mean_ms[0] the dense partial kernel, mean_ms[1] its merge kernel and
 * mean_ms[2] both (one dense decode).  Needs one skv_dense_decode first. */
int skv_time_dense(void *handle, int reps, float *mean_ms);

/* Stage outputs for parity checks (sync + copy).  stage is one of SKV_STAGE_*;
 * copies at most cap elements for one KV group, stores the element count. */
enum {
  SKV_STAGE_LOWER = 1,     /* uint16 [4][nc] BF16 lower bounds */
  SKV_STAGE_UPPER = 2,     /* uint16 [4][nc] BF16 upper bounds */
  SKV_STAGE_THRESH = 3,    /* uint32 [4] ordered-BF16 thresholds */
  SKV_STAGE_MASKS = 4,     /* uint8  [nc] survivor head masks */
  SKV_STAGE_FINE = 5,      /* uint16 [4][nc] BF16 fine scores (0xffff if not scored) */
  SKV_STAGE_SELECTED = 6,  /* int32  [count] selected clusters, ascending */
  SKV_STAGE_POOL = 7,      /* int32  [count] pool tokens, encounter order */
  SKV_STAGE_S2 = 8,        /* uint16 [4][count] BF16 2-bit scores of the pool */
  SKV_STAGE_U1 = 9,        /* int32  [count] union of top-1600, pool order */
  SKV_STAGE_S4 = 10,       /* uint16 [4][count] BF16 4-bit scores of U1 */
  SKV_STAGE_U2 = 11,       /* int32  [count] union of top-256, U1 order */
  SKV_STAGE_S8 = 12,       /* uint16 [4][count] BF16 8-bit scores of U2 */
  SKV_STAGE_TOP = 13,      /* int32  [4][100] final IDs, best first */
  SKV_STAGE_QPREP = 14,    /* int32  [4][3][260] fixed-point query operands */
  SKV_STAGE_KEYREC = 15,   /* uint8  [T][256] key records: 2-bit prefix plane |
                              2-bit residual plane | 4-bit residual plane */
  SKV_STAGE_KV8 = 16,      /* uint8  [T][512] FP8 [V||K] records (group), in
                              token order (paged records gathered page by page) */
  SKV_STAGE_KSCALE = 17    /* float  [256] key codec scales (group) */
};
int skv_read_stage(void *handle, int stage, int group, void *host_out,
                   int64_t cap, int64_t *count_out);

/* Per-kernel timing (the reference's SKV4_* device markers,
 * codegen/profiling.py:4-64): while enabled, skv_enqueue records a HIP event
 * before every kernel of the step on the handle's stream.  skv_profile
 * (re)starts the accumulation; skv_profile_read syncs and returns the mean
 * milliseconds of each kernel over the profiled steps (n >= skv_kernel_count()). */
int skv_profile(void *handle, int enable);

/* Selection path (diagnostic; no counterpart in the reference, whose
 * TopK-XL trees always rank every item).  Each top-k of the step first tries
 * a cut estimated from a 4096-item sample and falls back to the full
 * selection when the sample misses; both give identical results.  exact = 1
 * always runs the full selection; exact = 2 (tests) makes every sampled cut
 * miss so the fallback runs; exact = 3 (tests) runs the full selections with
 * the token top-k scores never held in LDS, so their in-memory radix passes
 * run at every pool size; 0 restores the default.  Status word 7 of each group (see skv_sync)
 * records, one bit per stage (1 thresh, 2 fine select, 4 top-1600, 8 top-256,
 * 16 top-100), which selections of the last step took the full path. */
int skv_select_mode(void *handle, int exact);

/* Launch mode (no counterpart in the reference, whose programs are enqueued
 * by TT-Metal): enable = 1 captures the step's kernels into a HIP graph on
 * the next skv_enqueue and replays it with one host call per step; 0 (the
 * default) launches the step's kernels one by one.  The graph saves host time
 * but, measured on MI355X with ROCm 7.2, consecutive graph launches leave
 * ~8 us of device idle between them, so back-to-back steps run slower.
 * Per-kernel profiling (skv_profile) always launches one by one.  Results
 * are identical in both modes. */
int skv_graph_mode(void *handle, int enable);
int skv_profile_read(void *handle, float *mean_ms, int n, int32_t *steps);

/* Duration of step kernel `kernel` alone (diagnostic; the reference's
 * per-kernel device markers serve the same purpose): after at least one
 * step, launches that kernel `reps` times back to back on the handle's stream
 * between two HIP events and stores the mean milliseconds per launch, then
 * runs one full step so every buffer holds a consistent step again. */
int skv_time_kernel(void *handle, int kernel, int reps, float *mean_ms);
int skv_kernel_count(void);
const char *skv_kernel_name(int i);

/* Reference metadata (_runtime.py:197-454), as a JSON text. */
const char *skv_metadata(void *handle);

/* Releases every device buffer of the handle (reference close, api.py:128-137). */
void skv_destroy(void *handle);

/* Text of the last error of this handle (or of the last failed create when
 * handle is NULL).  Valid until the next call on the handle. */
const char *skv_last_error(void *handle);

/* Library build identification. */
const char *skv_version(void);

#ifdef __cplusplus
}
#endif
#endif /* SEOULKV4_HIP_H */
