// Voxel hash table + 27-offset kernel map + block schedules (reference src/spconv.cu:10-75).
//
// Hash table: open addressing with linear probing, capacity = next pow2 >= 2N (load factor <= 0.5, as the
// reference, src/spconv.cu:40). Each slot is 16 bytes {u64 key, u32 row, u32 pad} so a probe is one 128-bit load
// that returns the key and the row together (the reference keeps keys and values in two arrays, i.e. two random
// accesses per hit). Keys pack (b,x,y,z) as ((b*W+x)*H+y)*D+z, the reference's injective packing
// (src/spconv.cu:16,29); empty = all ones. The home slot (home_slot below) hashes the voxel's z-quad with
// MurmurHash3's 32-bit finalizer (fmix32, Austin Appleby, public domain). Inserts claim a slot with a 64-bit
// compare-and-swap on the key.
//
// Neighbour map: one thread per (voxel, offset) pair, 64 voxels x 27 offsets per 256-thread workgroup, so the
// [N,27] output is written as one contiguous, fully coalesced range per workgroup. The 27-bit mask is assembled
// with LDS atomic OR, then decoded (gray -> binary prefix xor) by one thread per voxel.
#include "scan.h"
#include "spconv.h"

namespace {
constexpr uint32_t EMPTY = 0xffffffffu;
constexpr uint64_t HEMPTY = ~0ull;

__device__ __forceinline__ uint64_t pack_key(int b, int x, int y, int z, int W, int H, int D) {
  return (((uint64_t)(uint32_t)b * (uint64_t)W + (uint64_t)x) * (uint64_t)H + (uint64_t)y) * (uint64_t)D + (uint64_t)z;
}

// Home slot of a voxel with packed key `key` and z coordinate z: the hash of its z-quad key (the key with z
// replaced by z>>2) picks a group of 4 slots (one 64-byte line) and z&3 the slot inside it, so the z-neighbours of a
// voxel mostly probe the same line. The quad key is folded to 32 bits and mixed with MurmurHash3's 32-bit
// finalizer (fmix32; two 32-bit multiplies instead of 64-bit ones). Insert and probe only have to agree.
__device__ __forceinline__ uint32_t home_slot(uint64_t key, int z, uint32_t mask) {
  const uint64_t kq = key - (uint64_t)(z - (z >> 2));
  uint32_t h = (uint32_t)kq ^ ((uint32_t)(kq >> 32) * 0x9e3779b1u);
  h ^= h >> 16;
  h *= 0x85ebca6bu;
  h ^= h >> 13;
  h *= 0xc2b2ae35u;
  h ^= h >> 16;
  return ((h << 2) | (uint32_t)(z & 3)) & mask;
}

__global__ void k_table_clear(ulonglong2* __restrict__ t, i64 cap) {
  i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < cap) t[i] = make_ulonglong2(HEMPTY, HEMPTY);
}

__global__ void __launch_bounds__(256) k_table_insert(const int4* __restrict__ c, i64 n, int W, int H, int D,
                                                      ulonglong2* __restrict__ t, uint32_t mask) {
  i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int4 q = c[i];
  uint64_t k = pack_key(q.x, q.y, q.z, q.w, W, H, D);
  for (uint32_t s = home_slot(k, q.w, mask);; s = (s + 1) & mask) {
    unsigned long long prev = atomicCAS((unsigned long long*)&t[s].x, (unsigned long long)HEMPTY, (unsigned long long)k);
    if (prev == HEMPTY || prev == k) {
      t[s].y = (unsigned long long)(uint32_t)i;
      return;
    }
  }
}

constexpr int NV = 64;  // voxels per workgroup in the neighbour kernel
__global__ void __launch_bounds__(256) k_neighbors(const int4* __restrict__ c, i64 n, int W, int H, int D,
                                                   const ulonglong2* __restrict__ t, uint32_t mask,
                                                   uint32_t* __restrict__ nbr, int32_t* __restrict__ gray,
                                                   uint32_t* __restrict__ bin) {
  __shared__ int4 cq[NV];
  __shared__ uint64_t ck[NV];
  __shared__ uint32_t gm[NV];
  i64 v0 = (i64)blockIdx.x * NV;
  int nv = (int)min<i64>(NV, n - v0);
  if (threadIdx.x < NV) {
    gm[threadIdx.x] = 0;
    if ((int)threadIdx.x < nv) {
      const int4 q = c[v0 + threadIdx.x];
      cq[threadIdx.x] = q;
      ck[threadIdx.x] = pack_key(q.x, q.y, q.z, q.w, W, H, D);
    }
  }
  __syncthreads();
  // neighbour keys are the centre key plus a per-offset stride: key(x+dx, y+dy, z+dz) = key + (dx*H + dy)*D + dz
  const int64_t sHD = (int64_t)H * D, sD = D;
  for (int p = threadIdx.x; p < nv * 27; p += 256) {
    int li = p / 27, v = p - li * 27;
    const int dx = v / 9 - 1, dy = v / 3 % 3 - 1, dz = v % 3 - 1;
    int4 q = cq[li];
    int x = q.y + dx, y = q.z + dy, z = q.w + dz;
    uint32_t r = EMPTY;
    if (x >= 0 && x < W && y >= 0 && y < H && z >= 0 && z < D) {
      const uint64_t k = ck[li] + (uint64_t)(dx * sHD + dy * sD + dz);
      for (uint32_t s = home_slot(k, z, mask);; s = (s + 1) & mask) {
        ulonglong2 e = t[s];
        if (e.x == k) {
          r = (uint32_t)e.y;
          break;
        }
        if (e.x == HEMPTY) break;
      }
    }
    nbr[v0 * 27 + p] = r;
    if (r != EMPTY) atomicOr(&gm[li], 1u << v);
  }
  __syncthreads();
  if ((int)threadIdx.x < nv) {
    uint32_t g = gm[threadIdx.x], b = g;
    b ^= b >> 1;
    b ^= b >> 2;
    b ^= b >> 4;
    b ^= b >> 8;
    b ^= b >> 16;
    gray[v0 + threadIdx.x] = (int32_t)g;
    bin[v0 + threadIdx.x] = b;
  }
}

// One wavefront per block of B1 consecutive rows of `order`: OR of the masks and its popcount.
__global__ void __launch_bounds__(256) k_block_or(const int32_t* __restrict__ gray, const int32_t* __restrict__ order,
                                                  i64 n, int B1, i64 nb, uint32_t* __restrict__ code,
                                                  uint32_t* __restrict__ cnt) {
  i64 b = (i64)blockIdx.x * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (b >= nb) return;
  uint32_t o = 0;
  i64 e = min<i64>(n, (b + 1) * (i64)B1);
  for (i64 i = b * (i64)B1 + lane; i < e; i += 64) o |= (uint32_t)gray[order ? order[i] : i];
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) o |= (uint32_t)__shfl_xor((int)o, d, 64);
  if (lane == 0) {
    code[b] = o;
    if (cnt) cnt[b] = (uint32_t)__popc(o);
  }
}

__global__ void k_block_list(const uint32_t* __restrict__ code, const uint32_t* __restrict__ seg, i64 nb,
                             int32_t* __restrict__ list) {
  i64 b = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nb) return;
  uint32_t c = code[b], s = seg[b];
  while (c) {
    list[s++] = __ffs(c) - 1;
    c &= c - 1;
  }
}

// ------------------------------------------------------------------------------------------ subdivision
__device__ __forceinline__ bool f16_positive(uint32_t h) { return (h & 0x8000u) == 0 && (h & 0x7fffu) != 0 && (h & 0x7fffu) <= 0x7c00u; }

__global__ void k_c2s_count(const uint4* __restrict__ lg, i64 n, uint32_t* __restrict__ cnt) {
  i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i > n) return;
  if (i == n) {  // trailing zero so the exclusive scan's last entry is the total
    cnt[n] = 0;
    return;
  }
  uint4 q = lg[i];
  uint32_t w[4] = {q.x, q.y, q.z, q.w}, c = 0;
#pragma unroll
  for (int s = 0; s < 8; s++) c += f16_positive((w[s >> 1] >> ((s & 1) * 16)) & 0xffffu);
  cnt[i] = c;
}

__global__ void k_c2s_emit(const uint4* __restrict__ lg, const int4* __restrict__ co, const uint32_t* __restrict__ off,
                           i64 n, int4* __restrict__ nco, int32_t* __restrict__ src) {
  i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint4 q = lg[i];
  uint32_t w[4] = {q.x, q.y, q.z, q.w}, r = off[i];
  int4 p = co[i];
#pragma unroll
  for (int s = 0; s < 8; s++)
    if (f16_positive((w[s >> 1] >> ((s & 1) * 16)) & 0xffffu)) {
      nco[r] = make_int4(p.x, p.y * 2 + (s & 1), p.z * 2 + (s >> 1 & 1), p.w * 2 + (s >> 2 & 1));
      src[r] = (int32_t)(i * 8 + s);
      r++;
    }
}
}  // namespace

SpConvCache build_neighbors(const Tensor& coords, int W, int H, int D) {
  REQ(coords.dt == I32 && coords.dim() == 2 && coords.size(1) == 4, "coords must be int32 [N,4]");
  REQ(W > 0 && H > 0 && D > 0, "grid %dx%dx%d", W, H, D);
  i64 n = coords.size(0);
  REQ(n < (1ll << 31) - 1, "too many voxels %lld", (long long)n);
  SpConvCache c;
  c.N = (int)n;
  c.nbr = empty({n, 27}, I32);
  c.gray = empty({n}, I32);
  c.sorted = empty({n}, I32);
  if (n == 0) return c;
  uint64_t cap = 1;
  while (cap < 2ull * (uint64_t)n) cap <<= 1;
  hipStream_t s = stream();
  Tensor table = empty({(i64)cap * 2}, I64), bin = empty({n}, I32);
  ulonglong2* t = (ulonglong2*)table.p;
  k_table_clear<<<cdiv((i64)cap, 256), 256, 0, s>>>(t, (i64)cap);
  k_table_insert<<<cdiv(n, 256), 256, 0, s>>>(coords.ptr<int4>(), n, W, H, D, t, (uint32_t)(cap - 1));
  k_neighbors<<<cdiv(n, NV), 256, 0, s>>>(coords.ptr<int4>(), n, W, H, D, t, (uint32_t)(cap - 1),
                                          c.nbr.ptr<uint32_t>(), c.gray.ptr<int32_t>(), bin.ptr<uint32_t>());
  CK(hipGetLastError());
  stable_argsort27(bin.ptr<uint32_t>(), n, c.sorted.ptr<int32_t>());
  return c;
}

const Tensor& SpConvCache::block_masks(int B1) {
  auto it = masks.find(B1);
  if (it != masks.end()) return it->second;
  REQ(B1 > 0, "B1=%d", B1);
  i64 nb = cdiv(N, B1);
  Tensor code = empty({std::max<i64>(nb, 1)}, I32);
  if (nb) {
    k_block_or<<<cdiv(nb, 4), 256, 0, stream()>>>(gray.ptr<int32_t>(), sorted.ptr<int32_t>(), N, B1, nb,
                                                  code.ptr<uint32_t>(), nullptr);
    CK(hipGetLastError());
  }
  return masks.emplace(B1, code).first->second;
}

__global__ void k_window_keys(const int32_t* __restrict__ sorted, i64 n, int shift, uint32_t* __restrict__ key) {
  i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) key[i] = (uint32_t)sorted[i] >> shift;
}

const Tensor& SpConvCache::window_order(int log2w) {
  auto it = worder.find(log2w);
  if (it != worder.end()) return it->second;
  REQ(log2w >= 0 && log2w < 31, "window 2^%d", log2w);
  Tensor o = empty({std::max<i64>(N, 1)}, I32);
  if (N) {
    // sorted is already stable by decoded mask; a stable pass by window index (row >> log2w) keeps that order
    // inside each window
    Tensor key = empty({N}, I32);
    k_window_keys<<<cdiv(N, 256), 256, 0, stream()>>>(sorted.ptr<int32_t>(), N, log2w, key.ptr<uint32_t>());
    int bits = 1;
    while (bits < 31 && ((i64)(N - 1) >> log2w) >> bits) bits++;
    stable_sort_pairs(key.ptr<uint32_t>(), sorted.ptr<int32_t>(), N, bits, o.ptr<int32_t>());
  }
  return worder.emplace(log2w, o).first->second;
}

// tbl[i][v] = nbr[order[i]][v], gs[i] = gray[order[i]]; rows past n are EMPTY with a zero mask. One thread per
// (row, offset) pair, so both the 108-byte source rows and the table are read and written contiguously.
__global__ void k_row_table(const uint32_t* __restrict__ nbr, const int32_t* __restrict__ gray,
                            const int32_t* __restrict__ order, i64 n, i64 npad, uint32_t* __restrict__ tbl,
                            int32_t* __restrict__ gs) {
  const i64 p = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= npad * 27) return;
  const i64 i = p / 27;
  const int v = (int)(p - i * 27);
  const int o = i < n ? order[i] : 0;
  tbl[p] = i < n ? nbr[(i64)o * 27 + v] : EMPTY;
  if (v == 0) gs[i] = i < n ? gray[o] : 0;
}

const SpConvCache::RowTable& SpConvCache::row_table(int log2w) {
  const int key = log2w < 0 ? -1 : log2w;
  auto it = rtab.find(key);
  if (it != rtab.end()) return it->second;
  RowTable r;
  r.order = key < 0 ? sorted : window_order(key);
  const i64 npad = std::max<i64>(cdiv(N, kRowTablePad), 1) * kRowTablePad;
  r.tbl = empty({npad, 27}, I32);
  r.gs = empty({npad}, I32);
  k_row_table<<<cdiv(npad * 27, 256), 256, 0, stream()>>>(nbr.ptr<uint32_t>(), gray.ptr<int32_t>(),
                                                          r.order.ptr<int32_t>(), N, npad, r.tbl.ptr<uint32_t>(),
                                                          r.gs.ptr<int32_t>());
  CK(hipGetLastError());
  return rtab.emplace(key, r).first->second;
}

const std::pair<Tensor, Tensor>& SpConvCache::valid(int B1) {
  auto it = vk.find(B1);
  if (it != vk.end()) return it->second;
  REQ(B1 > 0, "B1=%d", B1);
  i64 nb = cdiv(N, B1);
  Tensor code = empty({std::max<i64>(nb, 1)}, I32), seg = zeros({nb + 1}, I32);
  Tensor list = empty({std::max<i64>(27 * nb, 1)}, I32);
  if (nb) {
    hipStream_t s = stream();
    k_block_or<<<cdiv(nb, 4), 256, 0, s>>>(gray.ptr<int32_t>(), sorted.ptr<int32_t>(), N, B1, nb,
                                           code.ptr<uint32_t>(), seg.ptr<uint32_t>());
    excl_scan_u32(seg.ptr<uint32_t>(), seg.ptr<uint32_t>(), nb + 1, nullptr);  // seg[nb] was zeroed
    k_block_list<<<cdiv(nb, 256), 256, 0, s>>>(code.ptr<uint32_t>(), seg.ptr<uint32_t>(), nb, list.ptr<int32_t>());
    CK(hipGetLastError());
    masks.emplace(B1, code);
  }
  return vk.emplace(B1, std::make_pair(list, seg)).first->second;
}

Subdivision subdivide(const Tensor& coords, const Tensor& logits) {
  REQ(coords.dt == I32 && coords.dim() == 2 && coords.size(1) == 4, "coords must be int32 [N,4]");
  i64 n = coords.size(0);
  REQ(logits.dt == F16 && logits.numel() == n * 8, "logits must be fp16 [N,8]");
  Subdivision o;
  if (n == 0) {
    o.coords = empty({0, 4}, I32);
    o.src = empty({0}, I32);
    return o;
  }
  hipStream_t s = stream();
  Tensor off = empty({n + 1}, I32);
  k_c2s_count<<<cdiv(n + 1, 256), 256, 0, s>>>(logits.ptr<uint4>(), n, off.ptr<uint32_t>());
  excl_scan_u32(off.ptr<uint32_t>(), off.ptr<uint32_t>(), n + 1, nullptr);
  i64 m = (i64)to_host_vec<uint32_t>(off.slice0(n, n + 1))[0];  // host sync, as the reference (src/sdec.cu:52)
  o.coords = empty({m, 4}, I32);
  o.src = empty({m}, I32);
  if (m) {
    k_c2s_emit<<<cdiv(n, 256), 256, 0, s>>>(logits.ptr<uint4>(), coords.ptr<int4>(), off.ptr<uint32_t>(), n,
                                            o.coords.ptr<int4>(), o.src.ptr<int32_t>());
    CK(hipGetLastError());
  }
  return o;
}
