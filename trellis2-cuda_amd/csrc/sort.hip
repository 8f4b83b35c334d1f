// Stable LSD radix argsort of 27-bit keys: 3 passes of 9-bit digits. It produces the reference's `sorted`
// permutation (src/spconv.cu:47-52: cub::DeviceRadixSort::SortPairs(bin -> iota), stable, bits 0..32; bin < 2^27
// so bits 27..31 are all zero and sorting 27 bits gives the same order).
//
// Per pass, over tiles of 4096 keys (4 wavefronts x 16 chunks x 64 lanes):
//   count   : per-tile digit histogram, written digit-major hist[d * ntiles + tile]
//   scan    : exclusive scan of hist -> global start of (digit, tile)
//   scatter : each wavefront ranks its 16 chunks in order; within a chunk, lanes holding the same digit find each
//             other with 9 ballots (one per digit bit) and take rank = popcount(peers below me). Wavefront counts
//             are then prefixed across the 4 wavefronts, so every key's destination preserves input order.
#include "scan.h"

namespace {
constexpr int RBITS = 9, NBUK = 1 << RBITS, RT = 256, RCH = 16, RTILE = RT * RCH;

__global__ void __launch_bounds__(RT) k_rs_count(const uint32_t* __restrict__ keys, i64 n, int shift,
                                                 uint32_t* __restrict__ hist, int ntiles) {
  __shared__ uint32_t cnt[NBUK];
  for (int d = threadIdx.x; d < NBUK; d += RT) cnt[d] = 0;
  __syncthreads();
  i64 base = (i64)blockIdx.x * RTILE;
#pragma unroll 4
  for (int j = 0; j < RCH; j++) {
    i64 i = base + j * RT + threadIdx.x;
    if (i < n) atomicAdd(&cnt[(keys[i] >> shift) & (NBUK - 1)], 1u);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < NBUK; d += RT) hist[(i64)d * ntiles + blockIdx.x] = cnt[d];
}

__global__ void __launch_bounds__(RT) k_rs_scatter(const uint32_t* __restrict__ kin, const int32_t* __restrict__ vin,
                                                   uint32_t* __restrict__ kout, int32_t* __restrict__ vout, i64 n,
                                                   int shift, const uint32_t* __restrict__ start, int ntiles) {
  __shared__ uint32_t cnt[RT / 64][NBUK];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int d = threadIdx.x; d < NBUK; d += RT)
    for (int w = 0; w < RT / 64; w++) cnt[w][d] = 0;
  __syncthreads();
  const uint64_t lt = (1ull << lane) - 1ull;
  const i64 seg = (i64)blockIdx.x * RTILE + (i64)wv * (RCH * 64);
  uint32_t key[RCH], rank[RCH];
  int32_t val[RCH];
#pragma unroll
  for (int c = 0; c < RCH; c++) {
    i64 i = seg + c * 64 + lane;
    bool ok = i < n;
    key[c] = ok ? kin[i] : 0u;
    val[c] = ok ? (vin ? vin[i] : (int32_t)i) : 0;
    uint32_t d = (key[c] >> shift) & (NBUK - 1);
    uint64_t peers = __ballot(ok);
#pragma unroll
    for (int b = 0; b < RBITS; b++) {
      uint64_t m = __ballot((d >> b) & 1u);
      peers &= ((d >> b) & 1u) ? m : ~m;
    }
    uint32_t r = (uint32_t)__popcll(peers & lt);
    uint32_t before = ok ? cnt[wv][d] : 0u;
    rank[c] = before + r;
    // the lowest lane of each peer group advances the wavefront's running count for that digit
    if (ok && r == 0) cnt[wv][d] = before + (uint32_t)__popcll(peers);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < NBUK; d += RT) {
    uint32_t run = start[(i64)d * ntiles + blockIdx.x];
#pragma unroll
    for (int w = 0; w < RT / 64; w++) {
      uint32_t t = cnt[w][d];
      cnt[w][d] = run;
      run += t;
    }
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < RCH; c++) {
    i64 i = seg + c * 64 + lane;
    if (i < n) {
      uint32_t d = (key[c] >> shift) & (NBUK - 1);
      uint32_t pos = cnt[wv][d] + rank[c];
      kout[pos] = key[c];
      vout[pos] = val[c];
    }
  }
}
}  // namespace

void stable_sort_pairs(const uint32_t* keys, const int32_t* vals, i64 n, int bits, int32_t* vals_out) {
  if (n <= 0) return;
  REQ(n < (1ll << 31), "sort size %lld", (long long)n);
  REQ(bits >= 1 && bits <= 32, "key bits %d", bits);
  const int passes = (bits + RBITS - 1) / RBITS;
  int ntiles = cdiv(n, RTILE);
  i64 nh = (i64)NBUK * ntiles;
  Tensor hist = empty({nh}, I32), kb0 = empty({n}, I32), kb1 = empty({n}, I32), vb0 = empty({n}, I32),
         vb1 = empty({n}, I32);
  hipStream_t s = stream();
  // ping-pong buffers; the last pass writes its values straight into vals_out
  const uint32_t* kin = keys;
  const int32_t* vin = vals;
  for (int p = 0; p < passes; p++) {
    const bool last = p + 1 == passes;
    uint32_t* kout = (p & 1) ? kb1.ptr<uint32_t>() : kb0.ptr<uint32_t>();
    int32_t* vout = last ? vals_out : ((p & 1) ? vb1.ptr<int32_t>() : vb0.ptr<int32_t>());
    int shift = p * RBITS;
    k_rs_count<<<ntiles, RT, 0, s>>>(kin, n, shift, hist.ptr<uint32_t>(), ntiles);
    excl_scan_u32(hist.ptr<uint32_t>(), hist.ptr<uint32_t>(), nh, nullptr);
    k_rs_scatter<<<ntiles, RT, 0, s>>>(kin, vin, kout, vout, n, shift, hist.ptr<uint32_t>(), ntiles);
    kin = kout;
    vin = vout;
  }
  CK(hipGetLastError());
}

void stable_argsort27(const uint32_t* keys, i64 n, int32_t* order) { stable_sort_pairs(keys, nullptr, n, 27, order); }
