/* Drives the host code of libseoulkv4_hip under AddressSanitizer and
 * UndefinedBehaviorSanitizer (tests/test_host_sanitizer.py builds both).
 *
 * Input: a case file written by the test (little-endian):
 *   int32 context, sink, local, n_centroids, append_capacity
 *   4 x { int32 nprobe; float lam; int32 n_postings;
 *         u8 upper[nc*64]; u8 lower[nc*64]; f32 scale[nc]; u16 resid[nc];
 *         u16 gfs[nc/32]; i32 offsets[nc+1]; i32 values[n_postings] }
 *   u16 k[4*context*256]; u16 v[4*context*256]; u16 q[16*256]  (BF16 bits)
 *
 * Host-only paths (any machine): skv_create on the valid descriptor
 * (validation + spill-2 mate table, then the device, which is absent on a
 * CPU-only machine: SKV_EHIP), every descriptor rejection, the page-table
 * checks of skv_create_paged, the size checks of skv_dense_decode_static and
 * the NULL-handle entry points.  With a GPU, skv_create succeeds and the
 * driver also runs the query staging ring (more binds than ring slots with
 * no host wait), host cache appends (single tokens, then more than one
 * staging chunk), the dense decode and destroy.  Exit status 0 when every
 * expectation holds; a sanitizer report aborts the process. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "seoulkv4_hip.h"

#define CHECK(cond, ...)                          \
  do {                                            \
    if (!(cond)) {                                \
      fprintf(stderr, "FAILED %s:%d: ", __FILE__, __LINE__); \
      fprintf(stderr, __VA_ARGS__);               \
      fprintf(stderr, "\n");                      \
      exit(2);                                    \
    }                                             \
  } while (0)

typedef struct {
  int32_t nprobe, np;
  float lam;
  uint8_t *upper, *lower;
  float *scale;
  uint16_t *resid, *gfs;
  int32_t *offsets, *values;
} cell_t;

static int32_t T, SINK, LOCAL, NC, APPEND;
static cell_t cells[4];
static uint16_t *K, *V, *Q;

static void *read_n(FILE *f, size_t bytes) {
  void *p = malloc(bytes ? bytes : 1);
  CHECK(p && fread(p, 1, bytes, f) == bytes, "short case file (%zu bytes)", bytes);
  return p;
}

static int32_t read_i32(FILE *f) {
  int32_t x;
  CHECK(fread(&x, 4, 1, f) == 1, "short case file");
  return x;
}

static void load_case(const char *path) {
  FILE *f = fopen(path, "rb");
  CHECK(f, "cannot open %s", path);
  T = read_i32(f);
  SINK = read_i32(f);
  LOCAL = read_i32(f);
  NC = read_i32(f);
  APPEND = read_i32(f);
  for (int g = 0; g < 4; ++g) {
    cell_t *c = &cells[g];
    c->nprobe = read_i32(f);
    CHECK(fread(&c->lam, 4, 1, f) == 1, "short case file");
    c->np = read_i32(f);
    c->upper = read_n(f, (size_t)NC * 64);
    c->lower = read_n(f, (size_t)NC * 64);
    c->scale = read_n(f, (size_t)NC * 4);
    c->resid = read_n(f, (size_t)NC * 2);
    c->gfs = read_n(f, (size_t)NC / 32 * 2);
    c->offsets = read_n(f, (size_t)(NC + 1) * 4);
    c->values = read_n(f, (size_t)c->np * 4);
  }
  K = read_n(f, (size_t)4 * T * 256 * 2);
  V = read_n(f, (size_t)4 * T * 256 * 2);
  Q = read_n(f, 16 * 256 * 2);
  fclose(f);
}

/* A descriptor over the case's arrays; `values` of cell g optionally replaced. */
static skv_index_desc desc_of(int g_values, int32_t *values) {
  skv_index_desc ix;
  memset(&ix, 0, sizeof ix);
  ix.context = T;
  ix.sink = SINK;
  ix.local = LOCAL;
  ix.n_centroids = NC;
  ix.pool_min = 0;
  ix.pool_capacity = 0;
  ix.debug = 1;
  ix.append_capacity = APPEND;
  for (int g = 0; g < 4; ++g) {
    skv_cell_desc *c = &ix.cells[g];
    c->upper = cells[g].upper;
    c->lower = cells[g].lower;
    c->scale = cells[g].scale;
    c->resid_f16 = cells[g].resid;
    c->gfs_f16 = cells[g].gfs;
    c->offsets = cells[g].offsets;
    c->values = g == g_values ? values : cells[g].values;
    c->nprobe = cells[g].nprobe;
    c->lam = cells[g].lam;
  }
  return ix;
}

static void expect_rejected(const skv_index_desc *ix, const char *text, const char *what) {
  void *h = (void *)1;
  const int code = skv_create(ix, K, V, 0, NULL, &h);
  const char *msg = skv_last_error(NULL);
  CHECK(code == SKV_EINVAL && h == NULL && strstr(msg, text), "%s: code %d, message '%s'", what,
        code, msg);
}

static void descriptor_rejections(void) {
  skv_index_desc ix;
  ix = desc_of(-1, NULL);
  ix.context = 0;
  expect_rejected(&ix, "context", "context 0");
  ix = desc_of(-1, NULL);
  ix.n_centroids = NC + 16;
  expect_rejected(&ix, "multiple of 32", "n_centroids");
  ix = desc_of(-1, NULL);
  ix.sink = T;
  expect_rejected(&ix, "sink/local", "sink");
  ix = desc_of(-1, NULL);
  ix.cells[2].nprobe = NC + 1;
  expect_rejected(&ix, "nprobe", "nprobe");
  ix = desc_of(-1, NULL);
  ix.cells[1].gfs_f16 = NULL;
  expect_rejected(&ix, "NULL", "NULL array");

  /* CSR faults, each on a private copy of one cell's arrays */
  const cell_t *c0 = &cells[0];
  int32_t *vals = malloc((size_t)c0->np * 4);
  int32_t *offs = malloc((size_t)(NC + 1) * 4);
  /* a token in a third list */
  memcpy(vals, c0->values, (size_t)c0->np * 4);
  int a = c0->offsets[0], b = c0->offsets[2], c = c0->offsets[4];
  CHECK(c0->offsets[1] > a && c0->offsets[3] > b && c0->offsets[5] > c, "empty lists in case");
  vals[b] = vals[a];
  vals[c] = vals[a];
  ix = desc_of(0, vals);
  expect_rejected(&ix, "two memberships", "third membership");
  /* a duplicate inside one list */
  memcpy(vals, c0->values, (size_t)c0->np * 4);
  CHECK(c0->offsets[7] - c0->offsets[6] >= 2, "short list in case");
  vals[c0->offsets[6] + 1] = vals[c0->offsets[6]];
  ix = desc_of(0, vals);
  {
    void *h = (void *)1;
    CHECK(skv_create(&ix, K, V, 0, NULL, &h) == SKV_EINVAL && h == NULL, "duplicate in a list");
  }
  /* token IDs out of range, both ends */
  memcpy(vals, c0->values, (size_t)c0->np * 4);
  vals[c0->np - 1] = T;
  ix = desc_of(0, vals);
  expect_rejected(&ix, "token ID", "token ID = context");
  vals[c0->np - 1] = -1;
  expect_rejected(&ix, "token ID", "negative token ID");
  /* offsets: first entry, monotonicity */
  memcpy(offs, c0->offsets, (size_t)(NC + 1) * 4);
  offs[0] = 1;
  ix = desc_of(-1, NULL);
  ix.cells[0].offsets = offs;
  expect_rejected(&ix, "offsets[0]", "offsets[0]");
  memcpy(offs, c0->offsets, (size_t)(NC + 1) * 4);
  offs[NC / 2] = offs[NC / 2 + 1] + 1;
  expect_rejected(&ix, "monotone", "offsets not monotone");
  free(vals);
  free(offs);
}

static void page_rejections(void) {
  const skv_index_desc ix = desc_of(-1, NULL);
  const int pt = 256;
  const int need = (T + APPEND + pt - 1) / pt;
  int32_t *table = malloc((size_t)need * 4);
  for (int i = 0; i < need; ++i) table[i] = need - 1 - i;
  static uint8_t fake_pool[4096] __attribute__((aligned(256)));
  struct {
    int64_t n_pages;
    int page_tokens, table_len, bad_entry, bad_value;
    const char *text;
  } cases[] = {
      {need, 8, need, -1, 0, "power of two"},
      {need, 384, need, -1, 0, "power of two"},
      {0, pt, need, -1, 0, "pages"},
      {(int64_t)1 << 58, pt, need, -1, 0, "2^31"},
      {INT64_MAX, pt, need, -1, 0, "2^31"},
      {need, pt, need - 1, -1, 0, "needs"},
      {need, pt, need, need - 1, need, "outside"},
      {need, pt, need, 0, -5, "outside"},
      {need, pt, need, need - 1, need - 1 - 0 /* = entry 0's page */, "twice"},
  };
  for (size_t i = 0; i < sizeof cases / sizeof cases[0]; ++i) {
    int32_t *tab = malloc((size_t)need * 4);
    memcpy(tab, table, (size_t)need * 4);
    if (cases[i].bad_entry >= 0) tab[cases[i].bad_entry] = cases[i].bad_value;
    skv_kv_pages pages = {fake_pool, cases[i].n_pages, cases[i].page_tokens, tab,
                          cases[i].table_len};
    void *h = (void *)1;
    const int code = skv_create_paged(&ix, K, V, &pages, 0, NULL, &h);
    const char *msg = skv_last_error(NULL);
    CHECK(code == SKV_EINVAL && h == NULL && strstr(msg, cases[i].text),
          "page case %zu: code %d, message '%s'", i, code, msg);
    free(tab);
  }
  /* a well-formed table over a pool that is not device memory: refused at
   * the device (no GPU: SKV_EHIP) or by the pool range check (SKV_EINVAL) */
  skv_kv_pages pages = {fake_pool, need, pt, table, need};
  void *h = (void *)1;
  const int code = skv_create_paged(&ix, K, V, &pages, 0, NULL, &h);
  CHECK((code == SKV_EHIP || code == SKV_EINVAL) && h == NULL, "host pool: code %d", code);
  free(table);
}

static void handle_free_calls(void) {
  uint8_t dummy[64];
  CHECK(skv_enqueue(NULL) == SKV_ESTATE, "enqueue(NULL)");
  CHECK(skv_sync(NULL, NULL) == SKV_ESTATE, "sync(NULL)");
  CHECK(skv_bind_query(NULL, Q) == SKV_ESTATE, "bind(NULL)");
  CHECK(skv_append(NULL, K, V, 1) == SKV_ESTATE, "append(NULL)");
  CHECK(skv_dense_decode_static(dummy, 10, 11, dummy, dummy, NULL) == SKV_EINVAL, "rows < T");
  CHECK(skv_dense_decode_static(dummy, 1 << 21, (1 << 20) + 1, dummy, dummy, NULL) == SKV_EINVAL,
        "T > 2^20");
  CHECK(skv_dense_decode_static(NULL, 8, 8, dummy, dummy, NULL) == SKV_EINVAL, "NULL records");
  skv_destroy(NULL);
}

/* With a device: the staging ring, host appends, the dense decode. */
static void device_lifecycle(void *h) {
  int32_t status[4 * 8];
  uint16_t out[16 * 256], first[16 * 256];
  CHECK(skv_bind_query(h, Q) == SKV_OK && skv_enqueue(h) == SKV_OK, "first step");
  CHECK(skv_sync(h, status) == SKV_OK, "sync: %s", skv_last_error(h));
  CHECK(skv_read_output(h, first) == SKV_OK, "read output");
  for (int i = 0; i < 40; ++i)  /* 40 binds through a 16-slot ring, no host wait */
    CHECK(skv_bind_query(h, Q) == SKV_OK && skv_enqueue(h) == SKV_OK, "step %d", i);
  CHECK(skv_sync(h, status) == SKV_OK && skv_read_output(h, out) == SKV_OK, "ring steps");
  CHECK(memcmp(out, first, sizeof out) == 0, "ring steps changed the output");
  if (APPEND >= 1100) {
    for (int i = 0; i < 20; ++i) {  /* single tokens, then more than one chunk */
      const uint16_t *k1 = K + (size_t)i * 256, *v1 = V + (size_t)i * 256;
      uint16_t kt[4 * 256], vt[4 * 256];
      for (int g = 0; g < 4; ++g) {
        memcpy(kt + g * 256, k1 + (size_t)g * T * 256, 512);
        memcpy(vt + g * 256, v1 + (size_t)g * T * 256, 512);
      }
      CHECK(skv_append(h, kt, vt, 1) == SKV_OK, "append 1: %s", skv_last_error(h));
      CHECK(skv_enqueue(h) == SKV_OK, "step after append");
    }
    const int n = 1050;  /* [4][n][256]: the first n tokens of each KV head */
    uint16_t *kn = malloc((size_t)4 * n * 512), *vn = malloc((size_t)4 * n * 512);
    for (int g = 0; g < 4; ++g) {
      memcpy(kn + (size_t)g * n * 256, K + (size_t)g * T * 256, (size_t)n * 512);
      memcpy(vn + (size_t)g * n * 256, V + (size_t)g * T * 256, (size_t)n * 512);
    }
    CHECK(skv_append(h, kn, vn, n) == SKV_OK, "append %d: %s", n, skv_last_error(h));
    CHECK(skv_append(h, kn, vn, APPEND) == SKV_EINVAL, "append past capacity");
    free(kn);
    free(vn);
    CHECK(skv_enqueue(h) == SKV_OK && skv_sync(h, status) == SKV_OK, "step after appends");
    for (int g = 0; g < 4; ++g) CHECK(status[g * 8 + 1] == 0, "status error %d", status[g * 8 + 1]);
  }
  CHECK(skv_dense_decode(h) == SKV_OK && skv_read_dense_output(h, out) == SKV_OK, "dense");
  const char *meta = skv_metadata(h);
  CHECK(meta && strlen(meta) > 10, "metadata");
  skv_destroy(h);
}

int main(int argc, char **argv) {
  CHECK(argc == 2, "usage: %s CASE", argv[0]);
  load_case(argv[1]);
  descriptor_rejections();
  page_rejections();
  handle_free_calls();
  const skv_index_desc ix = desc_of(-1, NULL);
  void *h = NULL;
  const int code = skv_create(&ix, K, V, 0, NULL, &h);
  if (code == SKV_OK) {
    device_lifecycle(h);
    printf("sanitizer driver ok (device lifecycle)\n");
  } else {
    /* validation and the mate table ran; the device is absent */
    CHECK(code == SKV_EHIP && h == NULL, "valid descriptor: code %d '%s'", code,
          skv_last_error(NULL));
    printf("sanitizer driver ok (host paths; no device: %s)\n", skv_last_error(NULL));
  }
  for (int g = 0; g < 4; ++g) {
    cell_t *c = &cells[g];
    free(c->upper); free(c->lower); free(c->scale); free(c->resid); free(c->gfs);
    free(c->offsets); free(c->values);
  }
  free(K); free(V); free(Q);
  return 0;
}
