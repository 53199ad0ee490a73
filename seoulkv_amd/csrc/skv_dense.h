// Dense FP8 decode: softmax attention of the 16 query heads over every key
// of the cache, from the same FP8 [V || K] records the sparse path attends.
// It has no kernel counterpart in the reference, which compares its sparse
// step with TTNN's dense FlashDecode (README.md:7); here it is the roofline
// comparison of the sparse step on the same hardware.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace skv {

constexpr int DN_WAVES = 8;                // waves per dense block
constexpr int DN_BLOCK = DN_WAVES * 64;
constexpr int DN_TILE = 16;                // keys per wave iteration (one MFMA row block)
constexpr int DN_TARGET_BLOCKS = 64;       // partials per KV group (upper bound): one block per CU
constexpr int DN_MERGE_SLICES = 32;        // 8-dim output slices per query head in the merge
constexpr int DN_PAGED_MAX_TILES = 128;    // tiles per wave whose record index a paged wave holds

struct DenseArgs {
  const uint8_t* kv8;   // [G][rows][512]: fp8 V | fp8 K; paged: the page pool
                        // [pages][G][1 << shift][512]
  const int* table;     // paged records: physical page of each logical page (else NULL)
  int shift;            // paged records: log2 tokens per page (>= log2 DN_TILE)
  const uint16_t* q;    // [16][256] bf16
  int T;                // keys attended (rows 0 .. T-1 of each group)
  int rows;             // records per group in kv8
  int iters;            // 16-key tiles per wave
  int nb;               // blocks (partials) per KV group
  float* part;          // [G][nb][H][D + 2]: unnormalised o, max (log2 units), sum
  uint16_t* out;        // [16][256] bf16
};

// 16-key tiles per wave and blocks per group for a context of T keys.
inline void dense_shape(int T, int& iters, int& nb) {
  const int tiles = (T + DN_TILE - 1) / DN_TILE;
  iters = (tiles + DN_TARGET_BLOCKS * DN_WAVES - 1) / (DN_TARGET_BLOCKS * DN_WAVES);
  if (iters < 1) iters = 1;
  nb = (tiles + iters * DN_WAVES - 1) / (iters * DN_WAVES);
  if (nb < 1) nb = 1;
}

// k = 0: the per-block partials; k = 1: the merge into the output.
void launch_dense(const DenseArgs& a, hipStream_t st, int k);

// Records the error text of a call without a handle (read back through
// skv_last_error(NULL)) and returns code.
int note_call_error(int code, const char* fmt, ...);

// NULL when ptr is device memory of `device` whose allocation holds `bytes`
// from ptr on, else the reason it is not (runtime queries; no allocation).
const char* device_range_error(const void* ptr, uint64_t bytes, int device);

}  // namespace skv
