// Stable LSD radix argsort of 27-bit keys: 3 passes of 9-bit digits. It produces the reference's `sorted`
// permutation (src/spconv.cu:47-52: cub::DeviceRadixSort::SortPairs(bin -> iota), stable, bits 0..32; bin < 2^27
// so bits 27..31 are all zero and sorting 27 bits gives the same order).
//
// Three launches per pass over tiles of 256 x RCH keys (RCH = 4, 8 or 16, so there are at least ~900 tiles when
// the input allows it):
//   count      : per-tile digit counts, digit-major [512][ntiles] (the first one also zeroes the digit-sum slots;
//                a producer that already holds the keys may count the first pass itself, see SortWork)
//   digit scan : one workgroup per digit sums its row and publishes the sum; its start is the sum of the lower
//                digits' published sums (read back all at once); the row is scanned to exclusive tile starts.
//                One launch instead of a device-wide scan's three.
//   scatter    : each wavefront ranks its chunks of 64 keys in order; within a chunk, lanes holding the same digit
//                find each other with 9 ballots (one per digit bit) and take rank = popcount(peers below me);
//                wavefront counts are prefixed across the 4 wavefronts. Destination = tile start + wavefronts
//                before + rank, so every key keeps its input order among equal digits.
// Measured against a look-back (single-pass) form with tile tickets: the per-digit look-back chains cost more than
// the two extra launches at every size here (C3 build 0.128 -> 0.106 ms, C4 0.400 -> 0.382 ms).
#include "scan.h"

namespace {
constexpr int RBITS = 9, NBUK = 1 << RBITS, RT = 256;
constexpr uint64_t ST_SUM = 1ull << 32;  // published flag of a digit-sum slot
constexpr uint32_t kSpinLimit = 1u << 20;  // default bound of the digit-sum wait (SPCONV_SORT_SPIN_LIMIT)

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

// Per-tile digit counts. Workgroup 0 also zeroes `zero` (zn words: the digit-sum slots of every pass, before the
// first digit scan reads them), which saves the sort a launch.
template <int RCH>
__global__ void __launch_bounds__(RT) k_rs_count(const uint32_t* __restrict__ keys, i64 n, int shift,
                                                 uint32_t* __restrict__ hist, int ntiles, uint32_t* __restrict__ zero,
                                                 int zn, const uint32_t* __restrict__ ndev) {
  __shared__ uint32_t cnt[NBUK];
  if (ndev) {  // device-side key count: tiles past it are skipped (the digit scan reads only the tiles below it)
    n = min<i64>(n, *ndev);
    if (blockIdx.x > 0 && (i64)blockIdx.x * (RT * RCH) >= n) return;
  }
  if (zero && blockIdx.x == 0)
    for (int i = threadIdx.x; i < zn; i += RT) zero[i] = 0;
  for (int d = threadIdx.x; d < NBUK; d += RT) cnt[d] = 0;
  __syncthreads();
  i64 base = (i64)blockIdx.x * (RT * RCH);
#pragma unroll 4
  for (int j = 0; j < RCH; j++) {
    i64 i = base + j * RT + threadIdx.x;
    if (i < n) atomicAdd(&cnt[(keys[i] >> shift) & (NBUK - 1)], 1u);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < NBUK; d += RT) hist[(i64)d * ntiles + blockIdx.x] = cnt[d];
}

template <int RCH>
__global__ void __launch_bounds__(RT) k_rs_scatter(const uint32_t* __restrict__ kin, const int32_t* __restrict__ vin,
                                                   uint32_t* __restrict__ kout, int32_t* __restrict__ vout, i64 n,
                                                   int shift, const uint32_t* __restrict__ start, int ntiles,
                                                   const uint32_t* __restrict__ ndev) {
  __shared__ uint32_t cnt[RT / 64][NBUK];
  if (ndev) {
    n = min<i64>(n, *ndev);
    if (blockIdx.x > 0 && (i64)blockIdx.x * (RT * RCH) >= n) return;  // no keys in this tile
  }
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int d = threadIdx.x; d < NBUK; d += RT)
    for (int w = 0; w < RT / 64; w++) cnt[w][d] = 0;
  __syncthreads();
  const i64 seg = (i64)blockIdx.x * (RT * RCH) + (i64)wv * (RCH * 64);
  uint32_t key[RCH], rank[RCH];
  int32_t val[RCH];
  rank_chunks<RCH>(kin, vin, n, shift, seg, lane, cnt[wv], key, val, rank);
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
      if (kout) kout[pos] = key[c];  // the last pass writes only the values
      vout[pos] = val[c];
    }
  }
}

// Per-pass tile starts in one launch: workgroup d owns digit d. It sums its row of per-tile counts (digit-major,
// [NBUK][ntiles]) and publishes the sum (flag in the high word of a zeroed 64-bit slot); the digit's start is the
// sum of the lower digits' published sums, read back all at once (workgroups start in id order, so every lower
// digit's workgroup is already running and publishes without waiting). The wait is bounded: a sum not published
// within spin_limit polls is computed by the waiting workgroup from that digit's row of tile counts, so the
// result never depends on the schedule (the limit only trades waiting against re-reading). The row is then
// scanned to exclusive tile starts in `start` (not in place: the counts stay intact for such a fallback read).
__global__ void __launch_bounds__(RT) k_rs_digit_scan(const uint32_t* __restrict__ cnt,
                                                      uint32_t* __restrict__ start, uint64_t* __restrict__ dsum,
                                                      int ntiles, uint32_t spin_limit, const uint32_t* __restrict__ ndev,
                                                      int tile_keys) {
  __shared__ uint32_t red[RT / 64];
  const int d = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int stride = ntiles;  // rows keep the capacity stride
  const uint32_t* row = cnt + (i64)d * stride;
  uint32_t* orow = start + (i64)d * stride;
  if (ndev) ntiles = max(1, min(ntiles, (int)(((i64)*ndev + tile_keys - 1) / tile_keys)));  // tiles with keys
  auto wg_sum = [&](uint32_t v) __attribute__((always_inline)) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o, 64);
    if (lane == 0) red[wv] = v;
    __syncthreads();
    uint32_t all = 0;
#pragma unroll
    for (int w = 0; w < RT / 64; w++) all += red[w];
    __syncthreads();
    return all;
  };
  uint32_t mine = 0;
  for (int i = tid; i < ntiles; i += RT) mine += row[i];
  const uint32_t rsum = wg_sum(mine);
  if (tid == 0) __hip_atomic_store(dsum + d, ST_SUM | rsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t below = 0;
  for (int e = tid; e < d; e += RT) {
    uint64_t w = __hip_atomic_load(dsum + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (uint32_t spins = 0; (w >> 32) == 0 && spins < spin_limit; spins++)
      w = __hip_atomic_load(dsum + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((w >> 32) == 0) {
      // not published within the limit: sum digit e's row of tile counts here (they are complete: the count
      // kernel ran before this launch), so the start is exact whatever the workgroup schedule
      uint32_t s = 0;
      for (int i = 0; i < ntiles; i++) s += cnt[(i64)e * stride + i];
      w = s;
    }
    below += (uint32_t)w;
  }
  uint32_t carry = wg_sum(below);
  for (int b = 0; b < ntiles; b += RT) {
    const int i = b + tid;
    const uint32_t v = i < ntiles ? row[i] : 0u;
    uint32_t inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t t = (uint32_t)__shfl_up((int)inc, o, 64);
      if (lane >= o) inc += t;
    }
    if (lane == 63) red[wv] = inc;
    __syncthreads();
    uint32_t base = carry, all = 0;
#pragma unroll
    for (int w = 0; w < RT / 64; w++) {
      const uint32_t t = red[w];
      if (w < wv) base += t;
      all += t;
    }
    if (i < ntiles) orow[i] = base + inc - v;
    carry += all;
    __syncthreads();
  }
}
}  // namespace

SortWork sort_work(i64 n, int bits) {
  SortWork w;
  w.passes = (bits + RBITS - 1) / RBITS;
  // the largest tile that still leaves ~900 tiles (interleaved builds, one box: C3 0.390 M keys best at 4, C4 3.76 M
  // at 16 (8: +3%), C5's children 2.15 M at 8 (16: +1.2%))
  w.rch = n >= (i64)RT * 16 * 900 ? 16 : (n >= (i64)RT * 8 * 900 ? 8 : 4);
  w.ntiles = (int)std::max<i64>(cdiv(n, (i64)RT * w.rch), 1);
  w.zwords = (i64)w.passes * NBUK * 2 + (i64)NBUK * w.ntiles;
  // [digit-sum slots: passes x NBUK u64][first pass's counts: NBUK x ntiles][tile starts: NBUK x ntiles]; the
  // slot words are even in number, so the 64-bit slots and everything after them stay 8-byte aligned
  w.buf = empty({w.zwords + (i64)NBUK * w.ntiles}, I32);
  return w;
}

void stable_sort_pairs(const uint32_t* keys, const int32_t* vals, i64 n, int bits, int32_t* vals_out,
                       const uint32_t* ndev, SortWork* pre) {
  if (n <= 0) return;
  REQ(n < (1ll << 31), "sort size %lld", (long long)n);
  REQ(bits >= 1 && bits <= 32, "key bits %d", bits);
  hipStream_t s = stream();
  // SPCONV_SORT_SPIN_LIMIT overrides the digit-sum wait bound (0: every workgroup recomputes the lower digits' sums
  // itself; the tests use it to check that path)
  uint32_t spin_limit = kSpinLimit;
  if (const char* e = getenv("SPCONV_SORT_SPIN_LIMIT")) spin_limit = (uint32_t)strtoul(e, nullptr, 10);
  SortWork own;
  if (!pre) own = sort_work(n, bits);
  SortWork& w = pre ? *pre : own;
  REQ(w.passes == (bits + RBITS - 1) / RBITS && w.ntiles == (int)std::max<i64>(cdiv(n, (i64)RT * w.rch), 1),
      "sort workspace made for another size");
  const int passes = w.passes, rch = w.rch, ntiles = w.ntiles;
  Tensor kb0 = empty({n}, I32), kb1 = empty({n}, I32), vb0 = empty({n}, I32), vb1 = empty({n}, I32);
  // ping-pong buffers; the last pass writes only its values, straight into vals_out
  const uint32_t* kin = keys;
  const int32_t* vin = vals;
  auto outs = [&](int p, uint32_t*& kout, int32_t*& vout) {
    kout = p + 1 == passes ? nullptr : ((p & 1) ? kb1.ptr<uint32_t>() : kb0.ptr<uint32_t>());
    vout = p + 1 == passes ? vals_out : ((p & 1) ? vb1.ptr<int32_t>() : vb0.ptr<int32_t>());
  };
  const i64 swords = (i64)passes * NBUK * 2;
  uint64_t* dsum = (uint64_t*)w.buf.ptr<uint32_t>();
  uint32_t* h = w.buf.ptr<uint32_t>() + swords;
  uint32_t* st = h + (i64)NBUK * ntiles;
  for (int p = 0; p < passes; p++) {
    uint32_t* kout;
    int32_t* vout;
    outs(p, kout, vout);
    const int shift = p * RBITS;
    if (p > 0 || !pre) {  // a caller-made workspace arrives with the first pass counted and the slots zeroed
      uint32_t* z = p == 0 ? (uint32_t*)dsum : nullptr;  // the first count kernel zeroes every pass's digit sums
      const int zn = (int)swords;
      if (rch == 16) k_rs_count<16><<<ntiles, RT, 0, s>>>(kin, n, shift, h, ntiles, z, zn, ndev);
      else if (rch == 8) k_rs_count<8><<<ntiles, RT, 0, s>>>(kin, n, shift, h, ntiles, z, zn, ndev);
      else k_rs_count<4><<<ntiles, RT, 0, s>>>(kin, n, shift, h, ntiles, z, zn, ndev);
    }
    k_rs_digit_scan<<<NBUK, RT, 0, s>>>(h, st, dsum + p * NBUK, ntiles, spin_limit, ndev, RT * rch);
    if (rch == 16) k_rs_scatter<16><<<ntiles, RT, 0, s>>>(kin, vin, kout, vout, n, shift, st, ntiles, ndev);
    else if (rch == 8) k_rs_scatter<8><<<ntiles, RT, 0, s>>>(kin, vin, kout, vout, n, shift, st, ntiles, ndev);
    else k_rs_scatter<4><<<ntiles, RT, 0, s>>>(kin, vin, kout, vout, n, shift, st, ntiles, ndev);
    kin = kout;
    vin = vout;
  }
  CK(hipGetLastError());
}

void stable_argsort27(const uint32_t* keys, i64 n, int32_t* order, const uint32_t* ndev, SortWork* pre) {
  stable_sort_pairs(keys, nullptr, n, 27, order, ndev, pre);
}
