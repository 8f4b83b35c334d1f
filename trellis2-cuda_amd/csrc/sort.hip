// Stable LSD radix argsort of 27-bit keys: 3 passes of 9-bit digits. It produces the reference's `sorted`
// permutation (src/spconv.cu:47-52: cub::DeviceRadixSort::SortPairs(bin -> iota), stable, bits 0..32; bin < 2^27
// so bits 27..31 are all zero and sorting 27 bits gives the same order).
//
// Up to 256 tiles of 2048 keys (512k keys, C3 and smaller): five launches for three passes (a zero fill, one
// histogram kernel for every pass's digit, one kernel per pass):
//   hist    : global digit histograms of all passes at once (LDS counts per tile, then global adds)
//   pass    : a workgroup takes the next tile ticket (an atomic counter, so tiles start in ticket order) and ranks
//             its keys: each wavefront ranks its 8 chunks of 64 keys in order; within a chunk, lanes holding the
//             same digit find each other with 9 ballots (one per digit bit) and take rank = popcount(peers below
//             me); wavefront counts are prefixed across the 4 wavefronts. Per digit the tile publishes its count,
//             looks back over the tiles before it, 16 per round (each publishes its count at once, then its
//             inclusive prefix, so the look-back stops at the first inclusive prefix it meets) and publishes its
//             own inclusive prefix. Destination = digit start (exclusive scan of the histogram) + tiles before +
//             wavefronts before + rank, so every key keeps its input order among equal digits.
// A look-back only waits on tiles with a smaller ticket, which are already running and publish their counts without
// waiting; the wait is bounded all the same (a tile that never published would read as empty: wrong order, no hang).
// Beyond 256 tiles the chain of published prefixes gets long (C4: 0.46 -> 0.49 ms build), so larger sorts run
// three kernels per pass over the same ranking (tiles of 4096 keys): per-tile digit counts (digit-major), an
// exclusive scan of them, and the scatter with those starts.
#include "scan.h"

namespace {
constexpr int RBITS = 9, NBUK = 1 << RBITS, RT = 256, MAXP = 4;
// look-back form: tiles of RT x RCH_LB keys (C2's 25k keys: 13 tiles, 0.085 -> 0.068 ms build against 4096-key
// tiles), LB tiles read per look-back round; count/scan/scatter form: tiles of RT x RCH_CS keys
constexpr int RCH_LB = 8, RTILE_LB = RT * RCH_LB, LB = 16, RCH_CS = 16, RTILE_CS = RT * RCH_CS;
constexpr uint64_t ST_AGG = 1ull << 32, ST_INC = 2ull << 32;
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr int kLookbackTiles = 256;

// Ranks a wavefront's RCH chunks of 64 keys (rows seg .. seg + RCH*64) by the digit at `shift`, in input order: lanes
// holding the same digit find each other with RBITS ballots and take rank = popcount(peers below me) plus the
// wavefront's running count for that digit (cw, in LDS, zeroed by the caller), which the lowest peer advances.
template <int RCH>
__device__ __forceinline__ void rank_chunks(const uint32_t* __restrict__ kin, const int32_t* __restrict__ vin, i64 n,
                                            int shift, i64 seg, int lane, uint32_t* cw, uint32_t (&key)[RCH],
                                            int32_t (&val)[RCH], uint32_t (&rank)[RCH]) {
  const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int c = 0; c < RCH; c++) {
    const i64 i = seg + c * 64 + lane;
    const bool ok = i < n;
    key[c] = ok ? kin[i] : 0u;
    val[c] = ok ? (vin ? vin[i] : (int32_t)i) : 0;
    const uint32_t d = (key[c] >> shift) & (NBUK - 1);
    uint64_t peers = __ballot(ok);
#pragma unroll
    for (int b = 0; b < RBITS; b++) {
      const uint64_t m = __ballot((d >> b) & 1u);
      peers &= ((d >> b) & 1u) ? m : ~m;
    }
    const uint32_t r = (uint32_t)__popcll(peers & lt);
    const uint32_t before = ok ? cw[d] : 0u;
    rank[c] = before + r;
    if (ok && r == 0) cw[d] = before + (uint32_t)__popcll(peers);
  }
}

__global__ void k_rs_zero(uint32_t* __restrict__ p, i64 n) {
  for (i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x) p[i] = 0;
}

__global__ void __launch_bounds__(RT) k_rs_hist(const uint32_t* __restrict__ keys, i64 n, int passes,
                                                uint32_t* __restrict__ hist) {
  __shared__ uint32_t cnt[MAXP][NBUK];
  for (int d = threadIdx.x; d < MAXP * NBUK; d += RT) (&cnt[0][0])[d] = 0;
  __syncthreads();
  const i64 base = (i64)blockIdx.x * RTILE_LB;
#pragma unroll 4
  for (int j = 0; j < RCH_LB; j++) {
    const i64 i = base + j * RT + threadIdx.x;
    if (i < n) {
      const uint32_t k = keys[i];
      for (int p = 0; p < passes; p++) atomicAdd(&cnt[p][(k >> (p * RBITS)) & (NBUK - 1)], 1u);
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < passes * NBUK; d += RT) {
    const uint32_t c = (&cnt[0][0])[d];
    if (c) atomicAdd(&hist[d], c);
  }
}

__global__ void __launch_bounds__(RT) k_rs_pass(const uint32_t* __restrict__ kin, const int32_t* __restrict__ vin,
                                                uint32_t* __restrict__ kout, int32_t* __restrict__ vout, i64 n,
                                                int shift, const uint32_t* __restrict__ hist, uint64_t* __restrict__ st,
                                                uint32_t* __restrict__ ticket) {
  __shared__ uint32_t cnt[RT / 64][NBUK];
  __shared__ uint32_t start[NBUK];
  __shared__ uint32_t wsum[RT / 64];
  __shared__ int tile_s;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (threadIdx.x == 0) tile_s = (int)atomicAdd(ticket, 1u);
  for (int d = threadIdx.x; d < NBUK; d += RT)
    for (int w = 0; w < RT / 64; w++) cnt[w][d] = 0;
  // digit starts: exclusive scan of this pass's histogram (thread t: digits 2t, 2t+1)
  const uint32_t h0 = hist[2 * threadIdx.x], h1 = hist[2 * threadIdx.x + 1];
  uint32_t inc = h0 + h1;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t t = (uint32_t)__shfl_up((int)inc, d, 64);
    if (lane >= d) inc += t;
  }
  if (lane == 63) wsum[wv] = inc;
  __syncthreads();
  uint32_t woff = 0;
  for (int w = 0; w < wv; w++) woff += wsum[w];
  const uint32_t ex = woff + inc - h0 - h1;
  start[2 * threadIdx.x] = ex;
  start[2 * threadIdx.x + 1] = ex + h0;
  const int tile = tile_s;

  const i64 seg = (i64)tile * RTILE_LB + (i64)wv * (RCH_LB * 64);
  uint32_t key[RCH_LB], rank[RCH_LB];
  int32_t val[RCH_LB];
  rank_chunks<RCH_LB>(kin, vin, n, shift, seg, lane, cnt[wv], key, val, rank);
  __syncthreads();
  for (int d = threadIdx.x; d < NBUK; d += RT) {
    uint32_t run = 0;
#pragma unroll
    for (int w = 0; w < RT / 64; w++) {
      const uint32_t t = cnt[w][d];
      cnt[w][d] = run;
      run += t;
    }
    uint64_t* my = st + (i64)tile * NBUK + d;
    uint32_t excl = 0;
    if (tile == 0) {
      __hip_atomic_store(my, ST_INC | run, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      __hip_atomic_store(my, ST_AGG | run, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // look back LB tiles per round (their words requested together); tiles before 0 read as an inclusive zero
      uint32_t spins = 0;
      for (int j = tile - 1; j >= 0;) {
        uint64_t w[LB];
#pragma unroll
        for (int k = 0; k < LB; k++)
          w[k] = j - k >= 0
                     ? __hip_atomic_load(st + (i64)(j - k) * NBUK + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : ST_INC;
        int k = 0;
        bool done = false;
        for (; k < LB; k++) {
          const uint32_t f = (uint32_t)(w[k] >> 32);
          if (f == 0) break;  // not published yet: the next round starts at this tile
          excl += (uint32_t)w[k];
          if (f == 2) {
            done = true;
            break;
          }
        }
        if (done) break;
        if (k == 0 && ++spins >= kSpinLimit) k = 1;  // never published: read as empty
        j -= k;
      }
      __hip_atomic_store(my, ST_INC | (excl + run), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    start[d] += excl;
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < RCH_LB; c++) {
    const i64 i = seg + c * 64 + lane;
    if (i < n) {
      const uint32_t d = (key[c] >> shift) & (NBUK - 1);
      const uint32_t pos = start[d] + cnt[wv][d] + rank[c];
      kout[pos] = key[c];
      vout[pos] = val[c];
    }
  }
}
__global__ void __launch_bounds__(RT) k_rs_count(const uint32_t* __restrict__ keys, i64 n, int shift,
                                                 uint32_t* __restrict__ hist, int ntiles) {
  __shared__ uint32_t cnt[NBUK];
  for (int d = threadIdx.x; d < NBUK; d += RT) cnt[d] = 0;
  __syncthreads();
  i64 base = (i64)blockIdx.x * RTILE_CS;
#pragma unroll 4
  for (int j = 0; j < RCH_CS; j++) {
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
  const i64 seg = (i64)blockIdx.x * RTILE_CS + (i64)wv * (RCH_CS * 64);
  uint32_t key[RCH_CS], rank[RCH_CS];
  int32_t val[RCH_CS];
  rank_chunks<RCH_CS>(kin, vin, n, shift, seg, lane, cnt[wv], key, val, rank);
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
  for (int c = 0; c < RCH_CS; c++) {
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
  hipStream_t s = stream();
  Tensor kb0 = empty({n}, I32), kb1 = empty({n}, I32), vb0 = empty({n}, I32), vb1 = empty({n}, I32);
  // ping-pong buffers; the last pass writes its values straight into vals_out
  const uint32_t* kin = keys;
  const int32_t* vin = vals;
  auto outs = [&](int p, uint32_t*& kout, int32_t*& vout) {
    kout = (p & 1) ? kb1.ptr<uint32_t>() : kb0.ptr<uint32_t>();
    vout = p + 1 == passes ? vals_out : ((p & 1) ? vb1.ptr<int32_t>() : vb0.ptr<int32_t>());
  };
  if (cdiv(n, RTILE_LB) <= kLookbackTiles) {
    const int ntiles = cdiv(n, RTILE_LB);
    // one zeroed block: histograms [passes][NBUK], tickets (64 words), look-back words [passes][ntiles][NBUK]
    const i64 hwords = (i64)passes * NBUK, twords = 64, swords = (i64)passes * ntiles * NBUK * 2;
    const i64 zw = hwords + twords + swords;
    Tensor scratch = empty({zw}, I32);
    uint32_t* hist = scratch.ptr<uint32_t>();
    uint32_t* tickets = hist + hwords;
    uint64_t* st = (uint64_t*)(tickets + twords);  // 8-byte aligned: hwords + twords is even
    k_rs_zero<<<(int)std::min<i64>(cdiv(zw, 256), 2048), 256, 0, s>>>(hist, zw);
    k_rs_hist<<<ntiles, RT, 0, s>>>(keys, n, passes, hist);
    for (int p = 0; p < passes; p++) {
      uint32_t* kout;
      int32_t* vout;
      outs(p, kout, vout);
      k_rs_pass<<<ntiles, RT, 0, s>>>(kin, vin, kout, vout, n, p * RBITS, hist + p * NBUK,
                                      st + (i64)p * ntiles * NBUK, tickets + p);
      kin = kout;
      vin = vout;
    }
  } else {
    const int ntiles = cdiv(n, RTILE_CS);
    const i64 nh = (i64)NBUK * ntiles;
    Tensor hist = empty({nh}, I32);
    for (int p = 0; p < passes; p++) {
      uint32_t* kout;
      int32_t* vout;
      outs(p, kout, vout);
      const int shift = p * RBITS;
      k_rs_count<<<ntiles, RT, 0, s>>>(kin, n, shift, hist.ptr<uint32_t>(), ntiles);
      excl_scan_u32(hist.ptr<uint32_t>(), hist.ptr<uint32_t>(), nh, nullptr);
      k_rs_scatter<<<ntiles, RT, 0, s>>>(kin, vin, kout, vout, n, shift, hist.ptr<uint32_t>(), ntiles);
      kin = kout;
      vin = vout;
    }
  }
  CK(hipGetLastError());
}

void stable_argsort27(const uint32_t* keys, i64 n, int32_t* order) { stable_sort_pairs(keys, nullptr, n, 27, order); }
