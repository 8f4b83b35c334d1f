/*
 * CPU oracle for the submanifold sparse-convolution path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is a plain-C restatement of the reference algorithm. It is the checker that the HIP library is
 * compared against (tests/, __graft_entry__.smoke()) and the CPU baseline that bench.py times beside the GPU
 * (cpu_baseline leg). Nothing in the product library links, loads or calls it.
 *
 * Reference: suvadityamuk/trellis2-cuda
 *   hash key / hash / insert / probe ........ src/spconv.cu:13-21, 38-43
 *   27-offset neighbour map, mask, decode .... src/spconv.cu:22-36, 45-46
 *   stable sort of the decoded mask .......... src/spconv.cu:47-52 (cub::DeviceRadixSort::SortPairs, bits 0..32)
 *   per-block valid-offset lists ............. src/spconv.cu:56-75
 *   conv (gather semantics, weight layout) ... src/spconv.cu:91-134, src/sdec.cu:15-18
 *   SiLU, residual formulas .................. src/ops.cu:79-82, 105-113
 *   child subdivision (c2s) .................. src/sdec.cu:20-33, 45-57
 *
 * How each function is pinned (the reference commits no golden vectors for this path):
 *   orc_build_neighbors: nbr against a brute-force dictionary lookup, the symmetry nbr[i][v]=j <=> nbr[j][26-v]=i,
 *     gray against the nbr row, bin against the closed form (bin ^ bin>>1 == gray), sorted against Python's
 *     stable sorted() on bin.
 *   orc_valid: list/seg against numpy bitwise_or.reduceat + popcount on the sorted masks.
 *   orc_conv: against torch.nn.functional.conv3d on the dense grid the sparse set is scattered into (submanifold
 *     conv equals dense zero-padded conv sampled at the active sites), and against the centre-only GEMM.
 *   orc_subdivide: against a Python enumeration of kept children and the parent = child/2 invariant.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_EMPTY 0xffffffffu
#define ORC_HEMPTY (~0ull)

/* src/spconv.cu:13 -- first half of MurmurHash3's fmix64, truncated to 32 bits. */
static uint32_t orc_hash(uint64_t k) {
  k ^= k >> 33;
  k *= 0xff51afd7ed558ccdull;
  k ^= k >> 33;
  return (uint32_t)k;
}

/* src/spconv.cu:16,29 -- injective packing of (b,x,y,z) for a W x H x D grid. */
static uint64_t orc_key(int64_t b, int64_t x, int64_t y, int64_t z, int W, int H, int D) {
  return (((uint64_t)b * (uint64_t)W + (uint64_t)x) * (uint64_t)H + (uint64_t)y) * (uint64_t)D + (uint64_t)z;
}

/* Stable LSD radix sort of 32-bit keys with an index payload (4 byte-digit counting passes). */
static void orc_stable_argsort(const int32_t* key, int64_t n, int32_t* order) {
  int32_t* ka = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n ? n : 1));
  int32_t* kb = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n ? n : 1));
  int32_t* ia = order;
  int32_t* ib = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n ? n : 1));
  for (int64_t i = 0; i < n; i++) { ka[i] = key[i]; ia[i] = (int32_t)i; }
  for (int pass = 0; pass < 4; pass++) {
    int64_t cnt[257];
    memset(cnt, 0, sizeof(cnt));
    int sh = pass * 8;
    for (int64_t i = 0; i < n; i++) cnt[(((uint32_t)ka[i]) >> sh & 255u) + 1]++;
    for (int d = 0; d < 256; d++) cnt[d + 1] += cnt[d];
    for (int64_t i = 0; i < n; i++) {
      int64_t p = cnt[((uint32_t)ka[i]) >> sh & 255u]++;
      kb[p] = ka[i];
      ib[p] = ia[i];
    }
    int32_t* t = ka; ka = kb; kb = t;
    t = ia; ia = ib; ib = t;
  }
  /* four passes: the result is back in the caller's buffer */
  free(ka);
  free(kb);
  free(ib);
}

/*
 * src/spconv.cu:38-54 build_neighbors.  coords int32 [n,4] (b,x,y,z).  Outputs: nbr u32 [n,27], gray i32 [n],
 * bin i32 [n] (any of them may be NULL except where needed), sorted i32 [n].
 */
int orc_build_neighbors(const int32_t* coords, int64_t n, int W, int H, int D, uint32_t* nbr, int32_t* gray,
                        int32_t* bin, int32_t* sorted) {
  uint64_t cap = 1;
  while (cap < 2ull * (uint64_t)n) cap <<= 1;
  uint64_t mask = cap - 1;
  uint64_t* keys = (uint64_t*)malloc(sizeof(uint64_t) * cap);
  uint32_t* vals = (uint32_t*)malloc(sizeof(uint32_t) * cap);
  int32_t* binbuf = bin ? bin : (int32_t*)malloc(sizeof(int32_t) * (size_t)(n ? n : 1));
  if (!keys || !vals || !binbuf) return -1;
  memset(keys, 0xff, sizeof(uint64_t) * cap);
  for (int64_t i = 0; i < n; i++) { /* src/spconv.cu:14-21 */
    const int32_t* q = coords + 4 * i;
    uint64_t k = orc_key(q[0], q[1], q[2], q[3], W, H, D);
    for (uint64_t s = orc_hash(k) & mask;; s = (s + 1) & mask) {
      if (keys[s] == ORC_HEMPTY || keys[s] == k) { keys[s] = k; vals[s] = (uint32_t)i; break; }
    }
  }
  for (int64_t i = 0; i < n; i++) { /* src/spconv.cu:22-36 */
    const int32_t* q = coords + 4 * i;
    uint32_t g = 0;
    for (int v = 0; v < 27; v++) {
      int64_t x = (int64_t)q[1] + v / 9 - 1, y = (int64_t)q[2] + v / 3 % 3 - 1, z = (int64_t)q[3] + v % 3 - 1;
      uint32_t r = ORC_EMPTY;
      if (x >= 0 && x < W && y >= 0 && y < H && z >= 0 && z < D) {
        uint64_t k = orc_key(q[0], x, y, z, W, H, D);
        for (uint64_t s = orc_hash(k) & mask; keys[s] != ORC_HEMPTY; s = (s + 1) & mask)
          if (keys[s] == k) { r = vals[s]; break; }
      }
      if (nbr) nbr[i * 27 + v] = r;
      if (r != ORC_EMPTY) g |= 1u << v;
    }
    uint32_t b = g;
    for (int v = 1; v < 27; v++) b ^= g >> v;
    if (gray) gray[i] = (int32_t)g;
    binbuf[i] = (int32_t)b;
  }
  if (sorted) orc_stable_argsort(binbuf, n, sorted); /* src/spconv.cu:47-52 (stable, ascending, ties by row) */
  free(keys);
  free(vals);
  if (!bin) free(binbuf);
  return 0;
}

/*
 * src/spconv.cu:56-75 SpConvCache::valid(B1).  list must hold 27*ceil(n/B1) ints, seg ceil(n/B1)+1 ints.
 * Returns L = seg[nb], the used length of list.
 */
int64_t orc_valid(const int32_t* gray, const int32_t* sorted, int64_t n, int B1, int32_t* list, int32_t* seg) {
  int64_t nb = (n + B1 - 1) / B1;
  seg[0] = 0;
  int64_t L = 0;
  for (int64_t b = 0; b < nb; b++) {
    uint32_t o = 0;
    int64_t e = (b + 1) * B1 < n ? (b + 1) * B1 : n;
    for (int64_t i = b * B1; i < e; i++) o |= (uint32_t)gray[sorted[i]];
    for (int v = 0; v < 27; v++)
      if (o >> v & 1u) list[L++] = v;
    seg[b + 1] = (int32_t)L;
  }
  return L;
}

/* ------------------------------------------------------------------------------------------ conv */
typedef struct {
  const float *x, *wt, *b, *res;
  int act;
  const uint32_t* nbr;
  const int64_t* rows;
  int64_t r0, r1;
  int ci, co;
  float* out;
} orc_conv_job;

/* y[i,co] = act(sum_v sum_ci x[nbr[i,v],ci] * w[co,v,ci] + b[co]) [+ res[i,co]], EMPTY neighbours contribute 0.
 * Each output's fp32 sum runs over v ascending, then ci ascending (src/spconv.cu:18-19 chain order). */
static void* orc_conv_worker(void* p) {
  orc_conv_job* j = (orc_conv_job*)p;
  float* acc = (float*)malloc(sizeof(float) * (size_t)j->co);
  for (int64_t t = j->r0; t < j->r1; t++) {
    int64_t i = j->rows ? j->rows[t] : t;
    for (int c = 0; c < j->co; c++) acc[c] = 0.f;
    for (int v = 0; v < 27; v++) {
      uint32_t src = j->nbr[i * 27 + v];
      if (src == ORC_EMPTY) continue;
      const float* xr = j->x + (int64_t)src * j->ci;
      const float* wv = j->wt + (int64_t)v * j->ci * j->co;
      for (int c = 0; c < j->ci; c++) {
        float xv = xr[c];
        const float* wr = wv + (int64_t)c * j->co;
        for (int o = 0; o < j->co; o++) acc[o] += xv * wr[o];
      }
    }
    float* yr = j->out + t * j->co;
    for (int o = 0; o < j->co; o++) {
      float v = acc[o] + (j->b ? j->b[o] : 0.f);
      if (j->act == 1) v = v / (1.0f + expf(-v)); /* src/ops.cu:81 */
      if (j->res) v = v + j->res[i * j->co + o];
      yr[o] = v;
    }
  }
  free(acc);
  return NULL;
}

/*
 * x fp32 [n,ci], w fp32 [co,27,ci], b fp32 [co] or NULL, res fp32 [n,co] or NULL, act 0 = none / 1 = SiLU.
 * rows: optional list of nrows output rows to compute (NULL = all n rows, nrows = n); out is [nrows, co].
 */
int orc_conv(const float* x, const float* w, const float* b, const float* res, int act, const uint32_t* nbr,
             const int64_t* rows, int64_t nrows, int ci, int co, float* out, int nthreads) {
  float* wt = (float*)malloc(sizeof(float) * 27 * (size_t)ci * (size_t)co); /* [27][ci][co] */
  if (!wt) return -1;
  for (int o = 0; o < co; o++)
    for (int v = 0; v < 27; v++)
      for (int c = 0; c < ci; c++) wt[((int64_t)v * ci + c) * co + o] = w[((int64_t)o * 27 + v) * ci + c];
  if (nthreads < 1) nthreads = 1;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  orc_conv_job* jobs = (orc_conv_job*)malloc(sizeof(orc_conv_job) * (size_t)nthreads);
  for (int t = 0; t < nthreads; t++) {
    orc_conv_job j = {x, wt, b, res, act, nbr, rows, nrows * t / nthreads, nrows * (t + 1) / nthreads, ci, co, out};
    jobs[t] = j;
    pthread_create(&th[t], NULL, orc_conv_worker, &jobs[t]);
  }
  for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
  free(th);
  free(jobs);
  free(wt);
  return 0;
}

/* ------------------------------------------------------------------------------------------ c2s */
static int orc_f16_positive(uint16_t h) { return (h & 0x8000u) == 0 && h != 0 && (h & 0x7fffu) <= 0x7c00u; }

/*
 * src/sdec.cu:20-33,45-57.  Children of each parent whose fp16 logit is > 0, in (parent, slot) order, with
 * coords (b, 2x + (s&1), 2y + (s>>1&1), 2z + (s>>2&1)) and src = parent*8 + s.  out_coords/src may be NULL
 * to only count.  Returns the number of children.
 */
int64_t orc_subdivide(const int32_t* coords, const uint16_t* logits, int64_t n, int32_t* out_coords, int32_t* src) {
  int64_t m = 0;
  for (int64_t i = 0; i < n; i++)
    for (int s = 0; s < 8; s++) {
      if (!orc_f16_positive(logits[i * 8 + s])) continue;
      if (out_coords) {
        out_coords[4 * m + 0] = coords[4 * i + 0];
        out_coords[4 * m + 1] = coords[4 * i + 1] * 2 + (s & 1);
        out_coords[4 * m + 2] = coords[4 * i + 2] * 2 + (s >> 1 & 1);
        out_coords[4 * m + 3] = coords[4 * i + 3] * 2 + (s >> 2 & 1);
      }
      if (src) src[m] = (int32_t)(i * 8 + s);
      m++;
    }
  return m;
}
