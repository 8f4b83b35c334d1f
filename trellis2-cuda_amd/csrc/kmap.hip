// Voxel hash table + 27-offset kernel map + block schedules (reference src/spconv.cu:10-75).
//
// The reference answers each of the 27 neighbour queries of a voxel with a probe of a voxel-keyed hash table
// (src/spconv.cu:13-36). Only the answers are observable (nbr rows, masks, the sorted order; bit-exact here), so
// the lookup structure is this build's own: a brick table. Space is cut into 4x4x4-voxel bricks; an
// open-addressed table (linear probing, capacity = next pow2 >= 2N, so it never fills even if every voxel is its
// own brick) maps the packed 64-bit brick key ((b*W4+x/4)*H4+y/4)*D4+z/4 to the brick's record of 64 rows.
// Slots are 16 bytes {u64 key, u32 id, pad}: one 128-bit load returns key and id together. Inserts claim a slot
// with a 64-bit compare-and-swap; the slot hash is MurmurHash3's 32-bit finalizer (fmix32, Austin Appleby, public
// domain) of the folded key.
//
// Neighbour map: one thread per voxel; its candidate bricks are probed once and kept in registers, its 27 rows
// read from the brick records, its mask assembled in registers and decoded (gray -> binary prefix xor), and the
// [N,27] rows of a 256-voxel workgroup written through LDS as one contiguous, fully coalesced range.
#include "scan.h"
#include "spconv.h"

namespace {
constexpr uint32_t EMPTY = 0xffffffffu;
constexpr uint64_t HEMPTY = ~0ull;

// Clears the live part of the table (mask + 1 slots; the mask is read from device memory when maskp is set) and
// zeroes the zn words at z (the sort's first-pass counts and digit-sum slots), grid-stride.
__global__ void k_table_clear(ulonglong2* __restrict__ t, uint32_t mask, const uint32_t* __restrict__ maskp,
                              uint32_t* __restrict__ z, i64 zn) {
  const i64 cap = (i64)(maskp ? *maskp : mask) + 1;
  for (i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x; i < cap; i += (i64)gridDim.x * blockDim.x)
    t[i] = make_ulonglong2(HEMPTY, HEMPTY);
  for (i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x; i < zn; i += (i64)gridDim.x * blockDim.x) z[i] = 0;
}

// ------------------------------------------------------------------------------------------ brick table
// Exact lookup structure for the neighbour query (only its answers are observable: nbr rows are bit-exact whatever
// the structure). Space is cut into bricks of 4x4x4 voxels; an open-addressed table keyed by the packed brick
// coordinate (b, x>>2, y>>2, z>>2) maps each occupied brick to a dense id, and bricks[id*64 + local] holds the
// row of every voxel in it (EMPTY elsewhere). The 27 neighbours of a voxel fall in 1-8 bricks (3.4 on average),
// so a voxel's probes touch a few table lines instead of one per neighbour column, and the rows it reads sit in
// a few 256-byte brick records shared with the voxels around it.
__device__ __forceinline__ uint64_t brick_key(int b, int x, int y, int z, int W4, int H4, int D4) {
  return (((uint64_t)(uint32_t)b * (uint64_t)W4 + (uint64_t)(x >> 2)) * (uint64_t)H4 + (uint64_t)(y >> 2)) *
             (uint64_t)D4 + (uint64_t)(z >> 2);
}
__device__ __forceinline__ int brick_local(int x, int y, int z) { return ((x & 3) << 4) | ((y & 3) << 2) | (z & 3); }
__device__ __forceinline__ uint32_t brick_home(uint64_t k, uint32_t mask) {
  uint32_t h = (uint32_t)k ^ ((uint32_t)(k >> 32) * 0x9e3779b1u);
  h ^= h >> 16;
  h *= 0x85ebca6bu;
  h ^= h >> 13;
  h *= 0xc2b2ae35u;
  h ^= h >> 16;
  return h & mask;
}
// Probe for brick key k: its id, or EMPTY when the brick holds no voxel.
__device__ __forceinline__ uint32_t brick_find(const ulonglong2* __restrict__ t, uint64_t k, uint32_t mask) {
  for (uint32_t s = brick_home(k, mask);; s = (s + 1) & mask) {
    const ulonglong2 e = t[s];
    if (e.x == k) return (uint32_t)e.y;
    if (e.x == HEMPTY) return EMPTY;
  }
}

// Table size without a host round trip: the number of runs of equal brick keys in input order bounds the number
// of occupied bricks (exactly, for spatially sorted input: C4 has 2.6 M voxels in 0.30 M bricks). Per-block run
// counts, then one block sums them and stores the mask of the smallest power-of-two table with at least twice
// that many slots (load <= 0.5), capped at the allocated capacity.
__global__ void __launch_bounds__(256) k_brick_runs(const int4* __restrict__ c, i64 n, int W4, int H4, int D4,
                                                    uint32_t* __restrict__ part, const uint32_t* __restrict__ ndev) {
  if (ndev) n = min<i64>(n, *ndev);  // device-side row count (rows past it are capacity)
  if ((i64)blockIdx.x * blockDim.x >= n) return;  // k_brick_mask reads only the blocks below n
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  int head = 0;
  if (i < n) {
    const int4 q = c[i];
    const uint64_t k = brick_key(q.x, q.y, q.z, q.w, W4, H4, D4);
    if (i == 0) {
      head = 1;
    } else {
      const int4 p = c[i - 1];
      head = brick_key(p.x, p.y, p.z, p.w, W4, H4, D4) != k;
    }
  }
  const int cnt = __syncthreads_count(head);
  if (threadIdx.x == 0) part[blockIdx.x] = (uint32_t)cnt;
}
__global__ void __launch_bounds__(1024) k_brick_mask(const uint32_t* __restrict__ part, i64 nb, uint64_t capmax,
                                                     uint32_t* __restrict__ maskp, const uint32_t* __restrict__ ndev,
                                                     int factor) {
  __shared__ uint64_t red[16];
  if (ndev) nb = min<i64>(nb, ((i64)*ndev + 255) / 256);  // the blocks k_brick_runs wrote
  uint64_t sum = 0;
  for (i64 b = threadIdx.x; b < nb; b += 1024) sum += part[b];
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) sum += (uint64_t)__shfl_xor((long long)sum, d, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sum;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t tot = 0;
    for (int w = 0; w < 16; w++) tot += red[w];
    uint64_t cap = 64;
    while (cap < (uint64_t)factor * tot && cap < capmax) cap <<= 1;
    *maskp = (uint32_t)(cap - 1);
  }
}

// Claims a slot for every occupied brick. A brick's id is the row of the voxel that inserted it (unique, so no
// shared counter), and the brick's 64-entry record is cleared by that voxel's wavefront.
__global__ void __launch_bounds__(256) k_brick_insert(const int4* __restrict__ c, i64 n, int W4, int H4, int D4,
                                                      ulonglong2* __restrict__ t, uint32_t mask0, const uint32_t* __restrict__ maskp,
                                                      uint4* __restrict__ bricks, const uint32_t* __restrict__ ndev) {
  if (ndev) n = min<i64>(n, *ndev);
  const uint32_t mask = maskp ? *maskp : mask0;
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t k = HEMPTY;
  if (i < n) {
    const int4 q = c[i];
    k = brick_key(q.x, q.y, q.z, q.w, W4, H4, D4);
  }
  // Voxels of one brick are usually adjacent rows (spatially sorted input): only the first lane of a run of equal
  // keys inserts, so a brick sees one compare-and-swap instead of one per voxel. (Other duplicates stay correct:
  // the compare-and-swap finds the key.)
  const int lane = threadIdx.x & 63;
  const uint64_t kprev = ((uint64_t)(uint32_t)__shfl_up((int)(uint32_t)(k >> 32), 1, 64) << 32) |
                         (uint32_t)__shfl_up((int)(uint32_t)k, 1, 64);
  bool won = false;
  if (i < n && (lane == 0 || kprev != k)) {
    for (uint32_t s = brick_home(k, mask);; s = (s + 1) & mask) {
      const unsigned long long prev =
          atomicCAS((unsigned long long*)&t[s].x, (unsigned long long)HEMPTY, (unsigned long long)k);
      if (prev == HEMPTY) {
        t[s].y = (unsigned long long)i;
        won = true;
        break;
      }
      if (prev == k) break;
    }
  }
  // the wavefront clears its inserters' records together, 16 lanes per 256-byte record and 4 records per store
  // (one lane storing its own record took 16 stores with a few lanes active: C4 insert 44.7 -> 33.4 us)
  uint64_t wmask = __ballot(won);
  const i64 wbase = i - lane;
  while (wmask) {
    int src[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      src[r] = wmask ? __builtin_ctzll(wmask) : -1;
      if (wmask) wmask &= wmask - 1;
    }
    const int r = lane >> 4;
    const int who = r == 0 ? src[0] : r == 1 ? src[1] : r == 2 ? src[2] : src[3];
    if (who >= 0) bricks[(wbase + who) * 16 + (lane & 15)] = make_uint4(EMPTY, EMPTY, EMPTY, EMPTY);
  }
}

__global__ void __launch_bounds__(256) k_brick_fill(const int4* __restrict__ c, i64 n, int W4, int H4, int D4,
                                                    const ulonglong2* __restrict__ t, uint32_t mask0, const uint32_t* __restrict__ maskp,
                                                    uint32_t* __restrict__ bricks, const uint32_t* __restrict__ ndev) {
  if (ndev) n = min<i64>(n, *ndev);
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t mask = maskp ? *maskp : mask0;
  const int4 q = c[i];
  const uint32_t id = brick_find(t, brick_key(q.x, q.y, q.z, q.w, W4, H4, D4), mask);
  bricks[(i64)id * 64 + brick_local(q.y, q.z, q.w)] = (uint32_t)i;
}

// One thread per voxel, 256 voxels per workgroup. The thread probes its own voxel's candidate bricks (own brick,
// and across each face the voxel sits on: 1-8, 3.4 on average), keeps the ids in registers, and then reads the
// 27 neighbour rows from the brick records with every per-offset quantity a compile-time constant except three
// face flags per axis; the mask is assembled in registers. The rows go through LDS so the [N,27] output is one
// contiguous, fully coalesced range per workgroup. Measured against one thread per (voxel, offset) pair with the
// candidate ids shared through LDS and the mask assembled by wavefront ballots: C4 220 -> 162 us, C3 32 -> 23 us
// (per-pair index arithmetic, LDS round trips and barriers were most of that kernel's time).
constexpr int NVV = 256;
__global__ void __launch_bounds__(NVV) k_neighbors_vox(const int4* __restrict__ c, i64 n, int W, int H, int D,
                                                       const ulonglong2* __restrict__ t,
                                                       uint32_t mask0, const uint32_t* __restrict__ maskp,
                                                       const uint32_t* __restrict__ bricks,
                                                       uint32_t* __restrict__ nbr, int32_t* __restrict__ gray,
                                                       uint32_t* __restrict__ bin, const uint32_t* __restrict__ ndev,
                                                       uint32_t* __restrict__ cnt0, int ntiles, int tile_keys) {
  __shared__ uint32_t rows[NVV * 27];
  __shared__ uint32_t dcnt[512];
  if (ndev) n = min<i64>(n, *ndev);
  const uint32_t mask = maskp ? *maskp : mask0;
  const i64 v0 = (i64)blockIdx.x * NVV;
  if (v0 >= n) return;  // a capacity block past the device-side count (uniform over the workgroup)
  const int nv = (int)min<i64>(NVV, n - v0);
  const int tid = threadIdx.x;
  const bool live = tid < nv;
  const int4 q = c[v0 + (live ? tid : 0)];
  dcnt[tid] = 0;
  dcnt[tid + NVV] = 0;
  __syncthreads();
  const int W4 = (W + 3) >> 2, H4 = (H + 3) >> 2, D4 = (D + 3) >> 2;
  const int ax = q.y & 3, ay = q.z & 3, az = q.w & 3;
  // per axis: the face the voxel sits on (-1 low, +1 high, 0 none)
  const int sx = ax == 0 ? -1 : (ax == 3 ? 1 : 0), sy = ay == 0 ? -1 : (ay == 3 ? 1 : 0),
            sz = az == 0 ? -1 : (az == 3 ? 1 : 0);
  uint64_t key[8];
  uint32_t slot[8], ids[8];
  bool pend[8];
#pragma unroll
  for (int cb = 0; cb < 8; cb++) {
    const int dx = (cb & 1) ? sx : 0, dy = (cb & 2) ? sy : 0, dz = (cb & 4) ? sz : 0;
    const int bx = (q.y >> 2) + dx, by = (q.z >> 2) + dy, bz = (q.w >> 2) + dz;
    const bool needed = ((cb & 1) == 0 || dx != 0) && ((cb & 2) == 0 || dy != 0) && ((cb & 4) == 0 || dz != 0);
    pend[cb] = live && needed && bx >= 0 && bx < W4 && by >= 0 && by < H4 && bz >= 0 && bz < D4;
    key[cb] = (((uint64_t)(uint32_t)q.x * W4 + bx) * H4 + by) * D4 + bz;
    slot[cb] = pend[cb] ? brick_home(key[cb], mask) : 0u;
    ids[cb] = EMPTY;
  }
  for (;;) {
    bool any = false;
#pragma unroll
    for (int cb = 0; cb < 8; cb++) any |= pend[cb];
    if (!any) break;
    ulonglong2 e[8];
#pragma unroll
    for (int cb = 0; cb < 8; cb++) e[cb] = pend[cb] ? t[slot[cb]] : make_ulonglong2(0, 0);
#pragma unroll
    for (int cb = 0; cb < 8; cb++) {
      if (!pend[cb]) continue;
      if (e[cb].x == key[cb]) {
        ids[cb] = (uint32_t)e[cb].y;
        pend[cb] = false;
      } else if (e[cb].x == HEMPTY) {
        pend[cb] = false;
      } else {
        slot[cb] = (slot[cb] + 1) & mask;
      }
    }
  }
  // offset v = 9 (dx+1) + 3 (dy+1) + (dz+1): the brick bit of an axis is set when the step crosses the face the
  // voxel sits on
  uint32_t r[27];
#pragma unroll
  for (int v = 0; v < 27; v++) {
    const int dx = v / 9 - 1, dy = v / 3 % 3 - 1, dz = v % 3 - 1;
    const int x = q.y + dx, y = q.z + dy, z = q.w + dz;
    const bool inb = live && x >= 0 && x < W && y >= 0 && y < H && z >= 0 && z < D;
    // candidate brick by three selects with constant register indices (a runtime index would go to scratch)
    const bool bx = dx != 0 && dx == sx, by = dy != 0 && dy == sy, bz = dz != 0 && dz == sz;
    const uint32_t a0 = bx ? ids[1] : ids[0], a1 = bx ? ids[3] : ids[2], a2 = bx ? ids[5] : ids[4],
                   a3 = bx ? ids[7] : ids[6];
    const uint32_t b0 = by ? a1 : a0, b1 = by ? a3 : a2;
    const uint32_t id = inb ? (bz ? b1 : b0) : EMPTY;
    const uint32_t* p = bricks + (id != EMPTY ? (i64)id * 64 + brick_local(x, y, z) : 0);
    r[v] = *p;  // entry 0 (a valid address) for misses
    r[v] = id != EMPTY ? r[v] : EMPTY;
  }
  uint32_t g = 0;
#pragma unroll
  for (int v = 0; v < 27; v++) {
    g |= r[v] != EMPTY ? (1u << v) : 0u;
    rows[tid * 27 + v] = r[v];
  }
  if (live) {
    uint32_t b = g;
    b ^= b >> 1;
    b ^= b >> 2;
    b ^= b >> 4;
    b ^= b >> 8;
    b ^= b >> 16;
    gray[v0 + tid] = (int32_t)g;
    bin[v0 + tid] = b;
    atomicAdd(&dcnt[b & 511u], 1u);
  }
  __syncthreads();
  // the sort's first pass counts its tiles' low 9-bit digits: this workgroup's voxels all lie in tile v0 / tile_keys
  const i64 tile = v0 / tile_keys;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int d = k * NVV + tid;
    if (dcnt[d]) atomicAdd(&cnt0[(i64)d * ntiles + tile], dcnt[d]);
  }
  const int tot = nv * 27;
  uint32_t* o = nbr + v0 * 27;
#pragma unroll
  for (int k = 0; k < 27; k++) {
    const int i = k * NVV + tid;
    // non-temporal: the 108-byte rows are not read again in this build, and kept in L2 they would evict the brick
    // records and table lines the neighbour queries read (C4 build 0.477 -> 0.421 ms, C5's children 0.330 -> 0.315)
    if (i < tot) __builtin_nontemporal_store(rows[i], &o[i]);
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

namespace {
// The build over rows [0, n) of coords; with ndev (device u32) the row count is read on the device and n is only a
// capacity bound: every launch is sized for n and its kernels stop at *ndev, so nothing here waits for the host.
// The cache's tensors then have n rows, of which the first *ndev are meaningful.
SpConvCache build_neighbors_impl(const int4* coords, i64 n, const uint32_t* ndev, int W, int H, int D,
                                 bool keep_hash) {
  REQ(W > 0 && H > 0 && D > 0, "grid %dx%dx%d", W, H, D);
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
  const int W4 = (W + 3) >> 2, H4 = (H + 3) >> 2, D4 = (D + 3) >> 2;
  // Large tables (>= 2^22 slots, 64 MB) use only their first 2^k >= 4 x (brick-key runs) slots, the mask computed
  // and kept in device memory: C4's clear and probes then touch 16 MB instead of 134 MB (build 0.48 -> 0.46 ms).
  // Smaller ones use all slots: the two extra launches cost more than they save (C3 0.155 -> 0.168 ms).
  Tensor maskt;
  uint32_t* maskp = nullptr;
  const uint32_t mask0 = (uint32_t)(cap - 1);
  if (cap >= (1ull << 22)) {
    const i64 nb = cdiv(n, 256);
    Tensor part = empty({nb}, I32);
    maskt = empty({1}, I32);
    maskp = maskt.ptr<uint32_t>();
    k_brick_runs<<<nb, 256, 0, s>>>(coords, n, W4, H4, D4, part.ptr<uint32_t>(), ndev);
    // slots >= 4 x the brick-key runs: shorter probe chains than at 2x (C4 build 0.483 -> 0.472 ms, C5 children
    // 0.361 -> 0.323 ms; 8x no better)
    k_brick_mask<<<1, 1024, 0, s>>>(part.ptr<uint32_t>(), nb, cap, maskp, ndev, 4);
  }
  // the sort's workspace: its first pass is counted by the neighbour kernel (slots and counts zeroed with the table)
  SortWork sw = sort_work(n, 27);
  REQ((sw.rch * 256) % NVV == 0, "sort tile of %d keys", sw.rch * 256);
  k_table_clear<<<(int)std::min<i64>(cdiv(std::max<i64>((i64)cap, sw.zwords), 256), 4096), 256, 0, s>>>(
      t, mask0, maskp, sw.buf.ptr<uint32_t>(), sw.zwords);
  // at most n occupied bricks: the table (capacity >= 2n) never fills. Brick records are indexed by the row of
  // the voxel that inserted the brick, so the record array has n slots (only occupied bricks' records are touched).
  Tensor bricks = empty({n * 64}, I32);
  k_brick_insert<<<cdiv(n, 256), 256, 0, s>>>(coords, n, W4, H4, D4, t, mask0, maskp, (uint4*)bricks.p, ndev);
  k_brick_fill<<<cdiv(n, 256), 256, 0, s>>>(coords, n, W4, H4, D4, t, mask0, maskp, bricks.ptr<uint32_t>(), ndev);
  k_neighbors_vox<<<cdiv(n, NVV), NVV, 0, s>>>(coords, n, W, H, D, t, mask0, maskp, bricks.ptr<uint32_t>(),
                                               c.nbr.ptr<uint32_t>(), c.gray.ptr<int32_t>(), bin.ptr<uint32_t>(),
                                               ndev, sw.counts(), sw.ntiles, sw.rch * 256);
  CK(hipGetLastError());
  stable_argsort27(bin.ptr<uint32_t>(), n, c.sorted.ptr<int32_t>(), ndev, &sw);
  c.W = W;
  c.H = H;
  c.D = D;
  if (keep_hash) {
    c.htable = table;
    c.hbricks = bricks;
    c.hmask = mask0;
    c.hmaskd = maskt;
  }
  return c;
}
}  // namespace

SpConvCache build_neighbors(const Tensor& coords, int W, int H, int D) {
  return build_neighbors(coords, W, H, D, false);
}

SpConvCache build_neighbors(const Tensor& coords, int W, int H, int D, bool keep_hash) {
  REQ(coords.dt == I32 && coords.dim() == 2 && coords.size(1) == 4, "coords must be int32 [N,4]");
  return build_neighbors_impl(coords.ptr<int4>(), coords.size(0), nullptr, W, H, D, keep_hash);
}

namespace {
__global__ void __launch_bounds__(256) k_lookup(const int4* __restrict__ q, i64 m, int W, int H, int D,
                                                const ulonglong2* __restrict__ t, uint32_t mask0,
                                                const uint32_t* __restrict__ maskp, const uint32_t* __restrict__ bricks,
                                                int32_t* __restrict__ out) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= m) return;
  const int4 c = q[i];
  int32_t r = -1;
  if (t && c.x >= 0 && c.y >= 0 && c.z >= 0 && c.w >= 0 && c.y < W && c.z < H && c.w < D) {  // t null: no voxels
    const uint32_t id = brick_find(t, brick_key(c.x, c.y, c.z, c.w, (W + 3) >> 2, (H + 3) >> 2, (D + 3) >> 2),
                                   maskp ? *maskp : mask0);
    if (id != EMPTY) r = (int32_t)bricks[(i64)id * 64 + brick_local(c.y, c.z, c.w)];  // EMPTY reads as -1
  }
  out[i] = r;
}

// neighbour column of the offset (dx, dy, dz) in {-1, 0, 1}^3: v = (dx+1)*9 + (dy+1)*3 + (dz+1)
__constant__ int8_t c_fdg_col[3][4] = {
    {13, 14, 17, 16},  // axis x: (0,0,0) (0,0,1) (0,1,1) (0,1,0)
    {13, 22, 23, 14},  // axis y: (0,0,0) (1,0,0) (1,0,1) (0,0,1)
    {13, 16, 25, 22},  // axis z: (0,0,0) (0,1,0) (1,1,0) (1,0,0)
};

__global__ void __launch_bounds__(256) k_fdg_quads(const uint32_t* __restrict__ nbr, const float* __restrict__ h,
                                                   i64 n, int4* __restrict__ quad, int32_t* __restrict__ ok) {
  const i64 e = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= 3 * n) return;
  const i64 i = e / 3;
  const int a = (int)(e % 3);
  bool g = h[i * 7 + 3 + a] > 0.f;
  int r[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    r[k] = (int)nbr[i * 27 + c_fdg_col[a][k]];
    g = g && r[k] >= 0;
  }
  ok[e] = g;
  if (g) quad[e] = make_int4(r[0], r[1], r[2], r[3]);
}

// Trilinear sample map (the bake's grid-sample neighbour map + weights): a point p (continuous voxel coordinates,
// voxel i spans [i, i+1) with its centre at i + 0.5) reads the 8 voxels around u = p - 0.5: corner v = dx*4 + dy*2 +
// dz of base floor(u), weight ((dx ? fx : 1-fx) * (dy ? fy : 1-fy)) * (dz ? fz : 1-fz), f = u - floor(u). Absent or
// off-grid corners: EMPTY with weight 0; with `normalize` the present weights are divided by their sum.
__global__ void __launch_bounds__(256) k_grid_sample_map(const float* __restrict__ grid, i64 L, int b, int W, int H,
                                                         int D, const ulonglong2* __restrict__ t, uint32_t mask0,
                                                         const uint32_t* __restrict__ maskp,
                                                         const uint32_t* __restrict__ bricks, bool normalize,
                                                         uint32_t* __restrict__ nb, float* __restrict__ wt) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= L) return;
  const float px = grid[i * 3], py = grid[i * 3 + 1], pz = grid[i * 3 + 2];
  uint32_t r[8];
  float w[8];
  const bool fin = isfinite(px) && isfinite(py) && isfinite(pz) && fabsf(px) < 1e9f && fabsf(py) < 1e9f &&
                   fabsf(pz) < 1e9f;
  const float ux = px - 0.5f, uy = py - 0.5f, uz = pz - 0.5f;
  const float bx = floorf(ux), by = floorf(uy), bz = floorf(uz);
  const float fx = ux - bx, fy = uy - by, fz = uz - bz;
  const int x0 = fin ? (int)bx : 0, y0 = fin ? (int)by : 0, z0 = fin ? (int)bz : 0;
  const uint32_t mask = maskp ? *maskp : mask0;
  float sum = 0.f;
#pragma unroll
  for (int v = 0; v < 8; v++) {
    const int dx = v >> 2, dy = (v >> 1) & 1, dz = v & 1;
    const int x = x0 + dx, y = y0 + dy, z = z0 + dz;
    uint32_t row = EMPTY;
    if (fin && t && b >= 0 && x >= 0 && y >= 0 && z >= 0 && x < W && y < H && z < D) {
      const uint32_t id = brick_find(t, brick_key(b, x, y, z, (W + 3) >> 2, (H + 3) >> 2, (D + 3) >> 2), mask);
      if (id != EMPTY) row = bricks[(i64)id * 64 + brick_local(x, y, z)];
    }
    r[v] = row;
    w[v] = row == EMPTY ? 0.f : ((dx ? fx : 1.f - fx) * (dy ? fy : 1.f - fy)) * (dz ? fz : 1.f - fz);
    sum += w[v];
  }
  if (normalize && sum > 0.f) {
#pragma unroll
    for (int v = 0; v < 8; v++) w[v] = w[v] / sum;
  }
#pragma unroll
  for (int v = 0; v < 8; v++) {
    nb[i * 8 + v] = r[v];
    wt[i * 8 + v] = w[v];
  }
}

// y[i, c] = sum over v = 0..7 of x[nb[i, v], c] * wt[i, v], fused multiply-adds in v order (EMPTY reads 0): the
// bake's weighted sum over the sample map (reference k_wsum, src/glb.cu:456-465).
__global__ void __launch_bounds__(256) k_grid_sample_sum(const float* __restrict__ x, int C,
                                                         const uint32_t* __restrict__ nb, const float* __restrict__ wt,
                                                         i64 L, float* __restrict__ y) {
  const i64 e = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= L * C) return;
  const i64 i = e / C;
  const int c = (int)(e - i * C);
  float acc = 0.f;
#pragma unroll
  for (int v = 0; v < 8; v++) {
    const uint32_t j = nb[i * 8 + v];
    acc = fmaf(j != EMPTY ? x[(i64)j * C + c] : 0.f, wt[i * 8 + v], acc);
  }
  y[e] = acc;
}
}  // namespace

void lookup(const SpConvCache& c, const Tensor& query, Tensor& rows) {
  REQ(query.dt == I32 && query.dim() == 2 && query.size(1) == 4, "query must be int32 [M,4]");
  REQ(rows.dt == I32 && rows.numel() == query.size(0), "rows must be int32 [M]");
  const i64 m = query.size(0);
  if (m == 0) return;
  REQ(c.N == 0 || c.htable.defined(), "the cache was built without keep_hash");
  k_lookup<<<cdiv(m, 256), 256, 0, stream()>>>(query.ptr<int4>(), m, c.W, c.H, c.D,
                                               c.N ? (const ulonglong2*)c.htable.p : nullptr, c.hmask,
                                               c.hmaskd.defined() ? c.hmaskd.ptr<uint32_t>() : nullptr,
                                               c.N ? c.hbricks.ptr<uint32_t>() : nullptr, rows.ptr<int32_t>());
  CK(hipGetLastError());
}

void grid_sample_map(const SpConvCache& c, const Tensor& grid, int batch, bool normalize, Tensor& nb, Tensor& wt) {
  REQ(grid.dt == F32 && grid.dim() == 2 && grid.size(1) == 3, "grid must be f32 [L,3]");
  const i64 L = grid.size(0);
  REQ(nb.numel() == L * 8 && wt.dt == F32 && wt.numel() == L * 8, "nb must be u32 [L,8], wt f32 [L,8]");
  if (L == 0) return;
  REQ(c.N == 0 || c.htable.defined(), "the cache was built without keep_hash");
  k_grid_sample_map<<<cdiv(L, 256), 256, 0, stream()>>>(
      grid.ptr<float>(), L, batch, c.W, c.H, c.D, c.N ? (const ulonglong2*)c.htable.p : nullptr, c.hmask,
      c.hmaskd.defined() ? c.hmaskd.ptr<uint32_t>() : nullptr, c.N ? c.hbricks.ptr<uint32_t>() : nullptr, normalize,
      nb.ptr<uint32_t>(), wt.ptr<float>());
  CK(hipGetLastError());
}

void grid_sample_sum(const Tensor& x, const Tensor& nb, const Tensor& wt, Tensor& y) {
  REQ(x.dt == F32 && x.dim() == 2, "x must be f32 [M,C]");
  const int C = (int)x.size(1);
  const i64 L = nb.numel() / 8;
  REQ(nb.numel() == L * 8 && wt.dt == F32 && wt.numel() == L * 8, "nb must be u32 [L,8], wt f32 [L,8]");
  REQ(y.dt == F32 && y.numel() == L * C, "y must be f32 [L,C]");
  if (L == 0 || C == 0) return;
  k_grid_sample_sum<<<cdiv(L * C, 256), 256, 0, stream()>>>(x.ptr<float>(), C, nb.ptr<uint32_t>(), wt.ptr<float>(), L,
                                                            y.ptr<float>());
  CK(hipGetLastError());
}

void fdg_quads(const SpConvCache& c, const Tensor& h, Tensor& quad, Tensor& ok) {
  const i64 n = c.N;
  REQ(h.dt == F32 && h.dim() == 2 && h.size(0) == n && h.size(1) == 7, "h must be f32 [N,7]");
  REQ(quad.dt == I32 && quad.numel() == 3 * n * 4 && ok.dt == I32 && ok.numel() == 3 * n,
      "quad must be int32 [3N,4], ok int32 [3N]");
  REQ((uintptr_t)quad.p % 16 == 0, "quad must be 16-byte aligned");
  if (n == 0) return;
  k_fdg_quads<<<cdiv(3 * n, 256), 256, 0, stream()>>>(c.nbr.ptr<uint32_t>(), h.ptr<float>(), n, quad.ptr<int4>(),
                                                      ok.ptr<int32_t>());
  CK(hipGetLastError());
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

// tbl[i][v] = nbr[order[i]][v], gs[i] = gray[order[i]]; rows past n are EMPTY with a zero mask. Seven lanes per
// row (nine rows per wavefront; grid = ceil(npad / 36) workgroups of four wavefronts): lane j moves bytes 16j .. 16j+16
// of the 108-byte row (12 for j = 6), so a load instruction covers nine rows' lines instead of one line per lane and
// the nine rows' output is one contiguous range (C5 children: 158 -> 145 us; the random row reads, ~2.4x their bytes
// in whole lines, hold it near the copy rate).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
typedef uint64_t u64x2_t __attribute__((ext_vector_type(2)));
__global__ void __launch_bounds__(256) k_row_table(const uint32_t* __restrict__ nbr, const int32_t* __restrict__ gray,
                                                   const int32_t* __restrict__ order, i64 nsrc, i64 n, i64 npad,
                                                   uint32_t* __restrict__ tbl, int32_t* __restrict__ gs) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane >= 63) return;
  const i64 i = ((i64)blockIdx.x * 4 + wv) * 9 + lane / 7;
  const int j = lane % 7;
  if (i >= npad) return;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(nbr), 0,
                                                                      (int)(nsrc * 108), 0x00020000);
  const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(tbl, 0, (int)(npad * 108), 0x00020000);
  const bool live = i < n;
  const int o = live ? order[i] : 0;
  const uint32_t src = live ? (uint32_t)o * 108u : 0xffff0000u, dst = (uint32_t)i * 108u;
  if (j < 6) {
    u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(rs, src + j * 16, 0, 0);
    if (!live) q = u32x4_t{EMPTY, EMPTY, EMPTY, EMPTY};
    __builtin_amdgcn_raw_buffer_store_b128(q, rd, dst + j * 16, 0, 0);
  } else {
    u32x3_t q = __builtin_amdgcn_raw_buffer_load_b96(rs, src + 96, 0, 0);
    if (!live) q = u32x3_t{EMPTY, EMPTY, EMPTY};
    __builtin_amdgcn_raw_buffer_store_b96(q, rd, dst + 96, 0, 0);
    gs[i] = live ? gray[o] : 0;
  }
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
  REQ(npad * 108 <= 0xfffe0000ll, "neighbour table of %lld rows too large", (long long)npad);
  k_row_table<<<cdiv(npad, 36), 256, 0, stream()>>>(nbr.ptr<uint32_t>(), gray.ptr<int32_t>(),
                                                    r.order.ptr<int32_t>(), N, N, npad, r.tbl.ptr<uint32_t>(),
                                                    r.gs.ptr<int32_t>());
  CK(hipGetLastError());
  return rtab.emplace(key, r).first->second;
}

// Per tile of B rows of a tile-order mask array (padded to a multiple of B): the number of offsets in the OR of
// its rows' masks. One workgroup of B threads per tile.
__global__ void __launch_bounds__(256) k_tile_cost(const int32_t* __restrict__ gs, int B, uint32_t* __restrict__ cost) {
  __shared__ uint32_t part[4];
  uint32_t m = (uint32_t)gs[(i64)blockIdx.x * B + threadIdx.x];
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) m |= (uint32_t)__shfl_xor((int)m, d, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t u = 0;
    for (int w = 0; w < (int)(blockDim.x + 63) / 64; w++) u |= part[w];
    cost[blockIdx.x] = (uint32_t)__popc(u);
  }
}

// Tile ids ordered by cost, largest first (counting sort over the 28 possible costs; ties keep tile order). One
// workgroup.
__global__ void __launch_bounds__(1024) k_tile_lpt(const uint32_t* __restrict__ cost, int nt, int32_t* __restrict__ order) {
  __shared__ uint32_t cnt[32], start[32];
  if (threadIdx.x < 32) cnt[threadIdx.x] = 0;
  __syncthreads();
  for (int t = threadIdx.x; t < nt; t += blockDim.x) atomicAdd(&cnt[27 - min(cost[t], 27u)], 1u);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (int c = 0; c < 32; c++) {
      start[c] = run;
      run += cnt[c];
    }
  }
  __syncthreads();
  // stable placement, one pass per chunk of 1024 tiles: a tile's rank among the chunk's tiles of its bucket is the
  // count of lower lanes of its wavefront holding the same bucket (5 ballots) plus the wavefronts before it
  __shared__ uint32_t wcnt[16][32];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint64_t lt = (1ull << lane) - 1ull;
  for (int base = 0; base < nt; base += 1024) {
    for (int e = threadIdx.x; e < 16 * 32; e += blockDim.x) wcnt[e >> 5][e & 31] = 0;
    __syncthreads();
    const int t = base + (int)threadIdx.x;
    const uint32_t k = t < nt ? 27 - min(cost[t], 27u) : 31u;
    uint64_t peers = ~0ull;
#pragma unroll
    for (int b = 0; b < 5; b++) {
      const uint64_t m = __ballot((k >> b) & 1u);
      peers &= ((k >> b) & 1u) ? m : ~m;
    }
    const uint32_t rank = (uint32_t)__popcll(peers & lt);
    if (rank == 0) wcnt[wv][k] = (uint32_t)__popcll(peers);
    __syncthreads();
    if (threadIdx.x < 32) {  // bucket b: exclusive offsets of the wavefronts, then advance the bucket start
      uint32_t run = start[threadIdx.x];
      for (int w = 0; w < 16; w++) {
        const uint32_t c = wcnt[w][threadIdx.x];
        wcnt[w][threadIdx.x] = run;
        run += c;
      }
      start[threadIdx.x] = run;
    }
    __syncthreads();
    if (t < nt) order[wcnt[wv][k] + rank] = t;
    __syncthreads();
  }
}

const Tensor& SpConvCache::tile_schedule(int log2w, int B) {
  const auto key = std::make_pair(log2w < 0 ? -1 : log2w, B);
  auto it = tsched.find(key);
  if (it != tsched.end()) return it->second;
  REQ(B > 0 && B <= 256 && B % 64 == 0 && kRowTablePad % B == 0, "tile rows %d", B);
  const RowTable& rt = row_table(log2w);
  const i64 nt = std::max<i64>(cdiv(N, B), 1);
  Tensor cost = empty({nt}, I32), order = empty({nt}, I32);
  k_tile_cost<<<(unsigned)nt, B, 0, stream()>>>(rt.gs.ptr<int32_t>(), B, cost.ptr<uint32_t>());
  k_tile_lpt<<<1, 1024, 0, stream()>>>(cost.ptr<uint32_t>(), (int)nt, order.ptr<int32_t>());
  CK(hipGetLastError());
  return tsched.emplace(key, order).first->second;
}

// mapped rows outside [0, m) become EMPTY, so the conv reads zeros for them
__global__ void k_map_table(const uint32_t* __restrict__ tbl, i64 entries, const int32_t* __restrict__ row_map,
                            int shift, uint32_t m, uint32_t* __restrict__ out) {
  const i64 e = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= entries) return;
  const uint32_t r = tbl[e];
  const uint32_t q = r == EMPTY ? EMPTY : (uint32_t)row_map[r] >> shift;
  out[e] = q < m ? q : EMPTY;
}

Tensor SpConvCache::mapped_table(int log2w, const Tensor& row_map, int shift, i64 m) {
  REQ(row_map.dt == I32 && row_map.numel() == N, "row_map must be int32 [%d]", N);
  REQ(shift >= 0 && shift < 31, "shift=%d", shift);
  const RowTable& rt = row_table(log2w);
  Tensor t = empty(rt.tbl.sh, I32);
  map_table_rows(rt.tbl, row_map, shift, m, t);
  return t;
}

void map_table_rows(const Tensor& tbl, const Tensor& row_map, int shift, i64 m, Tensor& out) {
  REQ(out.numel() == tbl.numel(), "mapped table size");
  const i64 entries = tbl.numel();
  k_map_table<<<cdiv(entries, 256), 256, 0, stream()>>>(tbl.ptr<uint32_t>(), entries, row_map.ptr<int32_t>(), shift,
                                                        (uint32_t)std::min<i64>(m, EMPTY), out.ptr<uint32_t>());
  CK(hipGetLastError());
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

// ------------------------------------------------------------------------------------------ subdivision + map, no sync
namespace {
// One pinned host word and an event per device: the child count is copied back while the map build runs.
struct CountReadback {
  uint32_t* host = nullptr;
  hipEvent_t ev = nullptr;
};
CountReadback& count_readback() {
  static CountReadback rb[64];
  int dev = 0;
  CK(hipGetDevice(&dev));
  REQ(dev >= 0 && dev < 64, "device %d", dev);
  CountReadback& r = rb[dev];
  if (!r.host) {
    CK(hipHostMalloc((void**)&r.host, sizeof(uint32_t), hipHostMallocDefault));
    CK(hipEventCreateWithFlags(&r.ev, hipEventDisableTiming));
  }
  return r;
}
}  // namespace

UpsampleLevel subdivide_build(const Tensor& coords, const Tensor& logits, int W, int H, int D, int32_t* coords_out,
                              int32_t* src_out) {
  REQ(coords.dt == I32 && coords.dim() == 2 && coords.size(1) == 4, "coords must be int32 [N,4]");
  const i64 n = coords.size(0);
  REQ(logits.dt == F16 && logits.numel() == n * 8, "logits must be fp16 [N,8]");
  REQ(8 * n < (1ll << 31) - 1, "too many parents %lld", (long long)n);
  UpsampleLevel o;
  if (n == 0) {
    o.coords = empty({0, 4}, I32);
    o.src = empty({0}, I32);
    o.cache = build_neighbors(o.coords, W, H, D);
    return o;
  }
  hipStream_t s = stream();
  const i64 cap = 8 * n;  // children at most
  Tensor cc = coords_out ? borrow(coords_out, {cap, 4}, I32) : empty({cap, 4}, I32);
  Tensor src = src_out ? borrow(src_out, {cap}, I32) : empty({cap}, I32);
  Tensor off = empty({n + 1}, I32);
  k_c2s_count<<<cdiv(n + 1, 256), 256, 0, s>>>(logits.ptr<uint4>(), n, off.ptr<uint32_t>());
  excl_scan_u32(off.ptr<uint32_t>(), off.ptr<uint32_t>(), n + 1, nullptr);
  const uint32_t* mdev = off.ptr<uint32_t>() + n;  // the child count, on the device
  CountReadback& rb = count_readback();
  CK(hipMemcpyAsync(rb.host, mdev, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  CK(hipEventRecord(rb.ev, s));
  k_c2s_emit<<<cdiv(n, 256), 256, 0, s>>>(logits.ptr<uint4>(), coords.ptr<int4>(), off.ptr<uint32_t>(), n,
                                          cc.ptr<int4>(), src.ptr<int32_t>());
  CK(hipGetLastError());
  // the children's map, sized for the capacity and stopped at the device-side count by every kernel
  SpConvCache c = build_neighbors_impl(cc.ptr<int4>(), cap, mdev, W, H, D, false);
  // every kernel of the build is queued: waiting for the count now leaves the GPU busy
  CK(hipEventSynchronize(rb.ev));
  const i64 m = *rb.host;
  REQ(m <= cap, "child count %lld above %lld", (long long)m, (long long)cap);
  c.N = (int)m;
  c.nbr = c.nbr.slice0(0, m);
  c.gray = c.gray.slice0(0, m);
  c.sorted = c.sorted.slice0(0, m);
  o.coords = cc.slice0(0, m);
  o.src = src.slice0(0, m);
  o.cache = std::move(c);
  return o;
}

// ------------------------------------------------------------------------------------------ subdivision, no allocation
// The allocation-free variant keeps its one scratch buffer -- the per-parent child counts, scanned in place into
// output offsets, plus the scan's tile sums -- in a file-scope device array. Every GPU holds its own copy of the
// array (at its own address) until the process ends; calls on one GPU share it, so calls that overlap on one GPU
// race. Every word a call reads is written earlier in the same call (the count kernel writes all n + 1 entries),
// so nothing needs clearing between calls.
namespace {
constexpr i64 kNoAllocMaxParents = i64(1) << 22;
constexpr i64 kNoAllocScratchWords = ((kNoAllocMaxParents + 1 + 63) / 64) * 64 + 2048;  // offsets + tile sums
__device__ __align__(256) uint32_t scratch[kNoAllocScratchWords];

__global__ void k_store_count(const uint32_t* __restrict__ total, i64* __restrict__ m) {
  if (threadIdx.x == 0 && blockIdx.x == 0) m[0] = total ? (i64)total[0] : 0;
}

// Device address of this GPU's copy of `scratch`; looked up once per device (the array's name is only a host-side
// stand-in, never a device address).
uint32_t* noalloc_scratch() {
  static uint32_t* ptr[64] = {};
  int dev = 0;
  CK(hipGetDevice(&dev));
  REQ(dev >= 0 && dev < 64, "device %d", dev);
  if (!ptr[dev]) {
    void* p = nullptr;
    CK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    REQ(p != nullptr, "scratch symbol has no device address");
    ptr[dev] = (uint32_t*)p;
  }
  return ptr[dev];
}
}  // namespace

i64 subdivide_noalloc_max_parents() { return kNoAllocMaxParents; }

void subdivide_noalloc(const int32_t* coords, const uint16_t* logits_f16, i64 n, int32_t* child_coords, int32_t* src,
                       i64* m_dev) {
  REQ(n >= 0 && n <= kNoAllocMaxParents, "subdivide_noalloc: %lld parents, at most %lld", (long long)n,
      (long long)kNoAllocMaxParents);
  REQ(m_dev, "m is null");
  uint32_t* ws = noalloc_scratch();
  hipStream_t s = stream();
  if (n == 0) {
    k_store_count<<<1, 64, 0, s>>>(nullptr, m_dev);
    CK(hipGetLastError());
    return;
  }
  REQ(coords && logits_f16 && child_coords && src, "null argument");
  uint32_t* off = ws;                                    // n + 1 offsets
  uint32_t* part = ws + ((n + 1 + 63) / 64) * 64;        // tile sums of the scan
  REQ((part - ws) + excl_scan_parts(n + 1) <= kNoAllocScratchWords, "scratch layout");
  k_c2s_count<<<cdiv(n + 1, 256), 256, 0, s>>>((const uint4*)logits_f16, n, off);
  excl_scan_u32_ws(off, off, n + 1, nullptr, part);
  k_store_count<<<1, 64, 0, s>>>(off + n, m_dev);
  k_c2s_emit<<<cdiv(n, 256), 256, 0, s>>>((const uint4*)logits_f16, (const int4*)coords, off, n, (int4*)child_coords,
                                          src);
  CK(hipGetLastError());
}

// ------------------------------------------------------------------------------------------ halo schedule
namespace {
constexpr int kHaloSlots = 1024;  // LDS hash slots per tile (>= 2 * kHaloMax)

__global__ void k_fill_i32(int32_t* __restrict__ p, i64 n, int32_t v) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// One workgroup per tile = B consecutive rows r0 .. r0+B of the input order, one thread per row. In one launch, with
// no host round trip, it
//  * orders the window: each row's rank among the window's rows by decoded mask (binary value of its gray code),
//    ties by row, which is the stable sort of the window (order[r0 + rank] = row; rows past n rank last);
//  * collects the tile's distinct neighbour rows: a row within D rows of the window (r0-D .. r0+B+D; 95% of the
//    (row, offset) entries on C4's shells for D = 512) marks a slot of a direct LDS flag array, any other goes into
//    an LDS open-addressed set (linear probing); a prefix count over both numbers the halo (flagged rows first,
//    ascending, then the set's slots) and gives every (row, offset) its index;
//  * stores the halo row ids (rows[t*UM + u], -1 past the count), the (offset, tile position) -> index table, the
//    16-position group masks and the count. A tile with more than UM distinct rows (or a full set) is a spill tile:
//    count -1, and it is appended to spill_list (spill_count entries, the order of appends is immaterial: each spill
//    tile is computed on its own by the gathering kernel).
// Only where a row sits in the conv's LDS copy depends on the halo numbering, never a sum.
template <int B, int UM, int D>
__global__ void __launch_bounds__(B) k_halo_build(const uint32_t* __restrict__ nbr, const int32_t* __restrict__ gray,
                                                  i64 n, int32_t* __restrict__ order, int32_t* __restrict__ rows,
                                                  int32_t* __restrict__ count, uint16_t* __restrict__ idx,
                                                  uint32_t* __restrict__ gm, int32_t* __restrict__ spill_list,
                                                  int32_t* __restrict__ spill_count) {
  constexpr int NWV = B / 64, SPT = kHaloSlots / B, R = B + 2 * D, RPT = R / B;
  static_assert(B % 64 == 0 && B <= 256 && UM < 65535 && R % B == 0, "halo tile shape");
  __shared__ uint32_t keys[kHaloSlots];
  __shared__ int pos[kHaloSlots];
  __shared__ int rpos[R];
  __shared__ __attribute__((aligned(16))) uint64_t keyL[B];
  __shared__ uint32_t maskL[B];
  __shared__ int wsum[2][NWV];
  __shared__ int bad;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const i64 t = blockIdx.x, r0 = t * B, r = r0 + tid;
  const bool live = r < n;
  // the thread's own 108-byte nbr row straight into registers: 6 x 16 + 12 bytes (4-byte aligned buffer loads; a
  // wavefront's loads cover one contiguous 6.9 KB range), EMPTY past n
  uint32_t nb[27];
  {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(nbr), 0,
                                                                        (int)(uint32_t)(n * 108), 0x00020000);
    const uint32_t o = live ? (uint32_t)r * 108u : 0xffff0000u;  // past the end: zeros
#pragma unroll
    for (int j = 0; j < 6; j++) {
      const u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(rs, o + j * 16, 0, 0);
      nb[4 * j] = q[0];
      nb[4 * j + 1] = q[1];
      nb[4 * j + 2] = q[2];
      nb[4 * j + 3] = q[3];
    }
    const u32x3_t q = __builtin_amdgcn_raw_buffer_load_b96(rs, o + 96, 0, 0);
    nb[24] = q[0];
    nb[25] = q[1];
    nb[26] = q[2];
  }
  for (int i = tid; i < kHaloSlots; i += B) keys[i] = EMPTY;
  for (int i = tid; i < R; i += B) rpos[i] = 0;
  if (tid == 0) bad = 0;
  const uint32_t g = live ? (uint32_t)gray[r] : 0u;
  uint32_t bn = g;
  bn ^= bn >> 1;
  bn ^= bn >> 2;
  bn ^= bn >> 4;
  bn ^= bn >> 8;
  bn ^= bn >> 16;
  if (!live) bn = 0xffffffffu;  // past the end: after every live row
  keyL[tid] = (uint64_t)bn << 8 | (uint32_t)tid;
  __syncthreads();
  // rank in the window: rows with a smaller decoded mask, or an equal one and a lower row (64-bit keys
  // (mask << 8 | row in window) are distinct, so the rank is one comparison per row)
  int rank = 0;
  const uint64_t mine = (uint64_t)bn << 8 | (uint32_t)tid;
#pragma unroll 16
  for (int j = 0; j < B; j += 2) {
    const u64x2_t q = *(const u64x2_t*)&keyL[j];
    rank += (q[0] < mine) + (q[1] < mine);
  }
  if (live) order[r0 + rank] = (int32_t)r;
  maskL[rank] = g;
  int16_t sl[27];  // >= 0: hash slot; -1: EMPTY; -2 - d: direct flag d
  const int lo = (int)r0 - D;
#pragma unroll
  for (int v = 0; v < 27; v++) {
    if (!live) nb[v] = EMPTY;
    sl[v] = -1;
    if (nb[v] == EMPTY) continue;
    const int d = (int)nb[v] - lo;
    if (d >= 0 && d < R) {
      rpos[d] = 1;
      sl[v] = (int16_t)(-2 - d);
      continue;
    }
    uint32_t h = (nb[v] * 0x9e3779b1u) >> 22;  // 10 bits: kHaloSlots = 1024
    for (int probe = 0; probe < kHaloSlots; probe++, h = (h + 1) & (kHaloSlots - 1)) {
      const uint32_t prev = atomicCAS(&keys[h], EMPTY, nb[v]);
      if (prev == EMPTY || prev == nb[v]) {
        sl[v] = (int16_t)h;
        break;
      }
    }
    if (sl[v] == -1) bad = 1;  // the set is full: the tile spills
  }
  __syncthreads();
  // number the flagged rows (RPT per thread), then the occupied set slots (SPT per thread): wave prefix by shuffles,
  // then the wave totals
  int fo = 0, ho = 0;
#pragma unroll
  for (int k = 0; k < RPT; k++) fo += rpos[tid * RPT + k];
#pragma unroll
  for (int k = 0; k < SPT; k++) ho += keys[tid * SPT + k] != EMPTY;
  int fi = fo, hi = ho;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int a = __shfl_up(fi, d, 64), b = __shfl_up(hi, d, 64);
    if (lane >= d) {
      fi += a;
      hi += b;
    }
  }
  if (lane == 63) {
    wsum[0][wv] = fi;
    wsum[1][wv] = hi;
  }
  __syncthreads();
  int fbase = fi - fo, hbase = hi - ho, UF = 0, UH = 0;
  for (int w = 0; w < NWV; w++) {
    if (w < wv) {
      fbase += wsum[0][w];
      hbase += wsum[1][w];
    }
    UF += wsum[0][w];
    UH += wsum[1][w];
  }
  const int U = UF + UH;
  hbase += UF;
  int32_t* trow = rows + t * UM;
#pragma unroll
  for (int k = 0; k < RPT; k++) {
    const int d = tid * RPT + k;
    if (rpos[d]) {
      if (fbase < UM) trow[fbase] = lo + d;
      rpos[d] = fbase++;
    }
  }
#pragma unroll
  for (int k = 0; k < SPT; k++) {
    const int sidx = tid * SPT + k;
    pos[sidx] = hbase;
    if (keys[sidx] != EMPTY) {
      if (hbase < UM) trow[hbase] = (int32_t)keys[sidx];
      hbase++;
    }
  }
  for (int u = U + tid; u < UM; u += B) trow[u] = -1;  // unused slots: the conv loads them unconditionally
  __syncthreads();  // numbering done
  // the (offset, tile position) -> index table: column `rank` of the tile's [27][B] block (positions past n hold
  // the zero row: their rows rank last)
  uint16_t* it = idx + t * 27 * B + rank;
#pragma unroll
  for (int v = 0; v < 27; v++) {
    int u = UM;  // EMPTY: the zero row
    if (sl[v] >= 0) u = pos[sl[v]];
    else if (sl[v] <= -2) u = rpos[-2 - sl[v]];
    it[v * B] = (uint16_t)min(u, UM);
  }
  // 16-position group masks (tile order)
  uint32_t mk = maskL[tid];
#pragma unroll
  for (int d = 1; d < 16; d <<= 1) mk |= (uint32_t)__shfl_xor((int)mk, d, 64);
  if ((tid & 15) == 0) gm[t * (B / 16) + tid / 16] = mk;
  if (tid == 0) {
    const bool spill = U > UM || bad;
    count[t] = spill ? -1 : U;  // a spill tile: served by the gathering kernel
    if (spill) spill_list[atomicAdd(spill_count, 1)] = (int32_t)t;
  }
}
}  // namespace

const SpConvCache::HaloTable& SpConvCache::halo_table(int B, int UM) {
  auto it = halo.find({B, UM});
  if (it != halo.end()) return it->second;
  HaloTable h;
  REQ((i64)N * 108 <= 0xfffe0000ll, "halo schedule: %d rows (at most %lld)", N, 0xfffe0000ll / 108);
  const i64 tiles = std::max<i64>(cdiv(N, B), 1);
  h.tiles = tiles;
  h.order = empty({std::max<i64>(N, 1)}, I32);  // B-row windows of the input order, gray-sorted inside
  h.rows = empty({tiles * UM}, I32);
  h.count = empty({tiles}, I32);
  h.idx = empty({tiles * 27 * B / 2}, I32);  // u16 entries
  h.gm = empty({tiles * (B / 16)}, I32);
  h.spill_list = empty({tiles}, I32);
  h.spill_count = empty({1}, I32);
  k_fill_i32<<<1, 64, 0, stream()>>>(h.spill_count.ptr<int32_t>(), 1, 0);
  auto go = [&](auto kern) {
    kern<<<(unsigned)tiles, B, 0, stream()>>>(nbr.ptr<uint32_t>(), gray.ptr<int32_t>(), N, h.order.ptr<int32_t>(),
                                              h.rows.ptr<int32_t>(), h.count.ptr<int32_t>(), (uint16_t*)h.idx.p,
                                              h.gm.ptr<uint32_t>(), h.spill_list.ptr<int32_t>(),
                                              h.spill_count.ptr<int32_t>());
  };
  if (B == 256 && UM == 512) go(k_halo_build<256, 512, 512>);
  else if (B == 128 && UM == 256) go(k_halo_build<128, 256, 256>);
  else REQ(false, "no halo builder for B=%d UM=%d", B, UM);
  CK(hipGetLastError());
  return halo.emplace(std::make_pair(B, UM), h).first->second;
}

int SpConvCache::HaloTable::host_spills() const {
  if (spills_host < 0) spills_host = to_host_vec<int32_t>(spill_count)[0];  // one host sync, on first request
  return spills_host;
}
