// Device-wide exclusive prefix sum of u32 (reduce -> scan of tile sums -> apply), the scan the kernel-map and
// subdivision paths need (the reference calls cub::DeviceScan::InclusiveSum at src/spconv.cu:69-70 and
// src/sdec.cu:50-51). Tiles are 4096 elements: 256 threads x 16 consecutive items per thread.
#include "scan.h"

namespace {
constexpr int ST = 256, SI = 16, STILE = ST * SI;

// Exclusive scan of one value per thread across a 256-thread workgroup; returns the workgroup total in *tot.
__device__ uint32_t wg_excl_scan(uint32_t v, uint32_t* lds, uint32_t* tot) {
  int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint32_t inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t t = __shfl_up(inc, d, 64);
    if (lane >= d) inc += t;
  }
  if (lane == 63) lds[wv] = inc;
  __syncthreads();
  uint32_t base = 0, all = 0;
#pragma unroll
  for (int w = 0; w < ST / 64; w++) {
    uint32_t s = lds[w];
    if (w < wv) base += s;
    all += s;
  }
  __syncthreads();
  *tot = all;
  return base + inc - v;
}

__global__ void __launch_bounds__(ST) k_scan_reduce(const uint32_t* __restrict__ in, i64 n, uint32_t* __restrict__ part) {
  __shared__ uint32_t lds[ST / 64];
  i64 base = (i64)blockIdx.x * STILE + (i64)threadIdx.x * SI;
  uint32_t s = 0;
#pragma unroll
  for (int j = 0; j < SI; j++)
    if (base + j < n) s += in[base + j];
  uint32_t tot;
  wg_excl_scan(s, lds, &tot);
  if (threadIdx.x == 0) part[blockIdx.x] = tot;
}

// Single workgroup: exclusive scan of the tile sums in place (any count, carried across 4096-element chunks).
__global__ void __launch_bounds__(ST) k_scan_parts(uint32_t* part, i64 nparts, uint32_t* total) {
  __shared__ uint32_t lds[ST / 64];
  uint32_t carry = 0;
  for (i64 c0 = 0; c0 < nparts; c0 += STILE) {
    i64 base = c0 + (i64)threadIdx.x * SI;
    uint32_t v[SI], s = 0;
#pragma unroll
    for (int j = 0; j < SI; j++) {
      v[j] = base + j < nparts ? part[base + j] : 0u;
      s += v[j];
    }
    uint32_t tot, pre = wg_excl_scan(s, lds, &tot) + carry;
#pragma unroll
    for (int j = 0; j < SI; j++) {
      if (base + j < nparts) part[base + j] = pre;
      pre += v[j];
    }
    carry += tot;
  }
  if (threadIdx.x == 0 && total) *total = carry;
}

__global__ void __launch_bounds__(ST) k_scan_apply(const uint32_t* __restrict__ in, uint32_t* __restrict__ out, i64 n,
                                                   const uint32_t* __restrict__ part) {
  __shared__ uint32_t lds[ST / 64];
  i64 base = (i64)blockIdx.x * STILE + (i64)threadIdx.x * SI;
  uint32_t v[SI], s = 0;
#pragma unroll
  for (int j = 0; j < SI; j++) {
    v[j] = base + j < n ? in[base + j] : 0u;
    s += v[j];
  }
  uint32_t tot, pre = wg_excl_scan(s, lds, &tot) + part[blockIdx.x];
#pragma unroll
  for (int j = 0; j < SI; j++) {
    if (base + j < n) out[base + j] = pre;
    pre += v[j];
  }
}
}  // namespace

i64 excl_scan_parts(i64 n) { return n <= 0 ? 0 : (n + STILE - 1) / STILE; }

void excl_scan_u32_ws(const uint32_t* in, uint32_t* out, i64 n, uint32_t* total_dev, uint32_t* part) {
  if (n <= 0) return;
  i64 nt = excl_scan_parts(n);
  hipStream_t s = stream();
  k_scan_reduce<<<(unsigned)nt, ST, 0, s>>>(in, n, part);
  k_scan_parts<<<1, ST, 0, s>>>(part, nt, total_dev);
  k_scan_apply<<<(unsigned)nt, ST, 0, s>>>(in, out, n, part);
  CK(hipGetLastError());
}

void excl_scan_u32(const uint32_t* in, uint32_t* out, i64 n, uint32_t* total_dev) {
  if (n <= 0) return;
  Tensor part = empty({excl_scan_parts(n)}, I32);
  excl_scan_u32_ws(in, out, n, total_dev, part.ptr<uint32_t>());
}
