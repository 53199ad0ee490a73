// Argument blocks of the decode-step kernels and their reference stages.
//
//   kernel           reference stage (src/seoulkv4/...)
//   k_front          _kernels/query_prepare/host.py:26-51 (q15, qs, ||q|| lambda);
//                    codegen/coarse_compute.py:61-119 (2-bit interval scores);
//                    codegen/fine_postscale_codegen.py:6-71 (4-bit fine scores)
//   k_select         _kernels/stage1_coarse/seoulkv4_coarse_select.py:297-310 (threshold);
//                    codegen/fine.py:1848-1861 (head masks),
//                    _kernels/stage1_fine/seoulkv4_fine_native_select.py:35-73 (top-P union)
//   k_pool           _kernels/stage1_coarse/seoulkv4_coarse_select.py:334-379 (survivor
//                    masks); codegen/stage15.py:275-345 (mate-ownership dedup,
//                    encounter-order pool); codegen/stage15.py:886-995 (2-bit scores)
//   k_top1600        codegen/stage15.py:1027-1180 (top-2048, first 1600 used)
//   k_union_score    codegen/stage15.py:1519-1597 (U1) +
//                    _kernels/stage16/seoulkv4_stage16_matrix.py:21-60 (4-bit scores) +
//                    _kernels/stage16/seoulkv4_union_matrix.py:58-139 (8-bit scores,
//                    here of every U1 key)
//   k_top256         codegen/refinement_fusion.py:263-266,402-455
//   k_top100         codegen/refinement_fusion.py:142-186 (U2, as a mask over U1) +
//                    codegen/refinement_fusion.py:296-300,495-531
//   k_select, k_top100  sparse SDPA: codegen/attention.py:35-201 (+ TTNN sparse_sdpa)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/seoulkv4_hip.h"
#include "skv_device.h"

namespace skv {

// status words per KV group
enum {
  ST_POOL = 0,     // pool size (clamped to the buffer)
  ST_ERR = 1,      // 0 ok, else an SKV_EPOOL_* code (include/seoulkv4_hip.h)
  ST_SEL = 2,      // selected clusters
  ST_SURV = 3,     // coarse survivors
  ST_U1 = 4,       // |U1|
  ST_U2 = 5,       // |U2|
  ST_SCANNED = 6,  // postings of the selected lists (summed by the U1 scorer)
  ST_FULLSEL = 7,  // selections that ran the full pass (bit per stage, FS_*)
  ST_WORDS = 8
};

// ST_FULLSEL bits: the sampled cut missed and the full selection ran
enum {
  FS_THRESH = 1,
  FS_FINE = 2,
  FS_TOP1600 = 4,
  FS_TOP256 = 8,
  FS_TOP100 = 16
};


struct StepArgs {
  // shapes
  int T, sink, local, nc, np_max, cap;  // T, local: current (grow with appended tokens)
  int rec_rows;             // key records per group (the prefill context)
  int kv_rows;              // FP8 records per group (prefill context + append capacity)
  int P[G];
  float lam[G];
  int pool_min, pool_capacity, debug;
  int exact_select;         // 1: always run the full selections (no sampled cut)
  int pool_blocks;          // nc / 32: 32-centroid bitmap words
  int pool_range;           // centroids per pool-kernel block (a multiple of 32, <= 1024)
  int words_u1, words_u2;   // bitmap words per (group, head)
  int dense_slices;         // DENSE_SLICE_KEYS-key sink/local attention slices per query head
  // static device data
  const uint16_t* q;        // [16][256] bf16 (bound query)
  const float* kscale;      // [G][256]
  const uint8_t* cen_up;    // [G][nc][64]
  const uint8_t* cen_lo;    // [G][nc][64]
  const float* scale4;      // [G][nc/32]
  const float* resid;       // [G][nc]
  const float* gfs;         // [G][nc/32]
  const int* csr_off;       // [G][nc+1]
  const int* post_tok;      // [G][np_max]
  const int* post_mate;     // [G][np_max] (-1: no mate)
  const uint8_t* post_p2;   // [G][np_max][64]
  const uint8_t* keyrec;    // [G][rec_rows][256]: p2 | r2 | r4 planes
  const uint8_t* kv8;       // [G][kv_rows][512]: fp8 V | fp8 K (rows < T valid); paged:
                            // the page pool [pages][G][1 << kv_shift][512]
  const int* kv_table;      // paged records: physical page of each logical page (else NULL)
  int kv_shift;             // paged records: log2 tokens per page
  // a small host append folded into this step: BF16 K [G][app_n][256] at
  // app_src, V right after it; k_front packs their FP8 records at rows
  // app_row .. app_row + app_n - 1 (app_n == 0: nothing pending)
  const uint16_t* app_src;
  int app_n, app_row;
  // per-step workspace
  QOperand* qop;            // [G][QV_COUNT]
  uint16_t* lower;          // [G][H][nc] ordered BF16
  uint16_t* upper;          // [G][H][nc] ordered BF16
  uint32_t* thr;            // [G][H]
  uint8_t* masks;           // [G][nc] survivor head masks
  uint16_t* fine_ord;       // [G][H][nc] ordered fine score of every centroid
  uint16_t* fine_bits;      // [G][H][nc] BF16 fine score (debug)
  uint16_t* tmax_lo;        // [G][H][nc/8] max ordered lower bound of each 8-centroid tile
  uint16_t* tmax_fi;        // [G][H][nc/16] max ordered fine score of each 16-centroid tile
                            // (both written when nc > 8 x SEL_BLOCK, else NULL)
  int* sel;                 // [G][nc] selected clusters, ascending
  unsigned long long* pool_flags;  // [G][pool_blocks] look-back records (epoch-tagged)
  int* pool_scan;           // [G][pool_blocks] postings of each pool range's selected lists
  unsigned* pool_epoch;     // [G] launches of the pool kernel (tags the look-back records)
  int* pool_tok;            // [G][cap]
  uint16_t* s2;             // [G][H][cap] ordered
  uint16_t* s2_tmax;        // [G][H][cap/16] upper bound (exact max, or 0xffff for a
                            // tile two pool blocks share) of every 16-key tile of s2
  uint64_t* bm_u1;          // [G][H][words_u1] top-1600 members
  uint64_t* bm_u2;          // [G][H][words_u2] top-256 members
  float* dense_part;        // [16][dense_slices][D + 2] sink/local partial (o, max, sum)
  uint32_t* selbm;          // [G][nc/32] selected-cluster bitmap (cleared each step)
  int* u1_tok;              // [G][U1_MAX]
  uint16_t* s4;             // [G][H][U1_MAX] ordered 4-bit scores of U1
  uint16_t* s8;             // [G][H][U1_MAX] ordered 8-bit scores of U1 (U2 members read)
  int* top;                 // [G][H][TOPK]
  int* status;              // [G][ST_WORDS]
  uint16_t* out;            // [16][256] bf16
  uint16_t* out_tiles;      // [G][32][H][D] bf16: query head 4g + h at [g][h][h] (the
                            // reference's tile-padded per-KV-head layout); the other
                            // rows stay zero (cleared once with the workspace)
};

struct TopkArgs {
  const uint16_t* scores;   // [G][H][stride] ordered
  const int* tokens;        // [G][stride]
  int stride;
  int k;
  uint64_t* bitmap;         // [G][H][words]
  int words;
  int* status;
  int count_slot;           // status word holding the item count
  int lds_items;            // scores held in LDS when count <= lds_items
  int exact_select;         // 1: skip the sampled cut
  int fullsel_bit;          // FS_* bit recorded when the full selection runs
  const uint16_t* tile_max; // [G][H][tile_stride] max of every 16-item tile (or NULL)
  int tile_stride;
  int regs2;                // launch choice: the instance that also selects rows of up to
                            // 2 x OCT_ITEMS items in registers (same members either way)
};


struct StepWork {
  TopkArgs top_u1, top_u2;
  size_t select_lds, top_u1_lds, top_u2_lds;  // dynamic LDS of the selection kernels
};

// Attention blocks: 1024 threads, 16 keys per wave; LDS bytes of their
// scratch (16 waves x (max, sum, o[256]) in FP32) and keys per sink/local
// slice.
constexpr int ATTN_WAVES = 16;
constexpr size_t ATTN_SCRATCH_BYTES = (size_t)ATTN_WAVES * (2 + D) * 4;
constexpr int DENSE_SLICE_KEYS = ATTN_WAVES * 16;

// Host appends of at most this many tokens are folded into the next step
// (staged with its query, packed by k_front): 16 tokens x 4 KV heads x 512
// B of BF16 K and V = 64 KiB per staging slot.
constexpr int APPEND_FUSE = 16;

// member-bitmap words the top-k kernel keeps in LDS beside its scratch
constexpr int TOPK_LDS_WORDS = 2048;

constexpr int N_STEP_KERNELS = 7;
extern const char* const kKernelNames[N_STEP_KERNELS];

// Dynamic LDS bytes of a top-k launch whose full selection holds lds_items
// scores in LDS.
size_t topk_dynamic_lds(int lds_items);

// Kernel k (0 .. N_STEP_KERNELS - 1, in step order) of one decode step.
void launch_kernel(const StepArgs& a, const StepWork& w, hipStream_t st, int k);
// Static and dynamic LDS bytes per block of step kernel k as launched.
hipError_t step_kernel_lds(const StepArgs& a, const StepWork& w, int k, size_t* static_bytes,
                           size_t* dynamic_bytes);
void launch_step(const StepArgs& a, const StepWork& w, hipStream_t st, hipEvent_t* ev);

}  // namespace skv
