// Masked implicit-GEMM submanifold conv on CDNA4 MFMA (the operator of reference src/spconv.cu:77-175).
//
//   out[order[r], co] = epi( sum_{v in mask(blk(r))} sum_ci x[nbr[order[r], v], ci] * w[co, v, ci] )
//   epi(s) = act(s + b[co]) [+ residual[order[r], co]],   EMPTY neighbours contribute zeros
//
// A workgroup owns BM consecutive rows of the gray-sorted order (one schedule block, so one OR-mask) and BN output
// channels. Its K loop runs over the set bits v of the block's mask (ascending) x Ci in KC-channel stages:
//   * A stage: BM gathered feature rows x KC channels, 16-byte global loads (8 bf16) into registers, then LDS;
//   * B stage: w[co0:co0+BN, v, kc:kc+KC] (the reference [Co,27,Ci] layout is already "K contiguous"), same path;
//   * double-buffered LDS, the next stage's global loads are issued before the current stage's MFMAs;
//   * each wavefront computes a (BM/WGM) x (BN/WGN) sub-tile with v_mfma_f32_32x32x16_{bf16,f16}, fp32 accumulate.
// MFMA operand layout (gfx950, 32x32x16): lane l supplies row (l%32) of A and column (l%32) of B, 8 consecutive K
// values starting at (l/32)*8 of the 16-wide K step; the result tile gives lane l column (l%32) and rows
// (i/4)*8 + (l/32)*4 + i%4 for its 16 accumulators i.
// The next offset's neighbour indices are fetched one offset ahead so the gather never waits on the nbr load.
// Workgroups are mapped so each XCD (each L2) walks a contiguous range of tiles with both channel tiles of a row
// tile adjacent in time.
#include <utility>

#include "lnact.h"
#include "spconv.h"



namespace {
constexpr uint32_t EMPTY = 0xffffffffu;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16-byte load/store unit (native vector, not a struct)
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {  // round to nearest even, quiet NaN preserved
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

__device__ __forceinline__ float load_elem(const void* p, i64 i, int dt) {
  if (dt == F32) return ((const float*)p)[i];
  uint16_t h = ((const uint16_t*)p)[i];
  return dt == BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}
__device__ __forceinline__ void store_elem(void* p, i64 i, int dt, float v) {
  if (dt == F32) ((float*)p)[i] = v;
  else ((uint16_t*)p)[i] = dt == BF16 ? f32_to_bf16(v) : f32_to_f16(v);
}

template <bool F16>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

constexpr int kMaxCi = 8192;

// Cache policy of buffer accesses to data each launch touches once (the tile-order neighbour table and the halo
// index table, 16-bit residuals, outputs): non-temporal (gfx950 `nt`), so that streaming them does not evict the
// gathered feature rows and weights from L2 (same box: C4 0.619 -> 0.609 ms, C5 children 0.911 -> 0.905, C3
// 0.792 -> 0.787).
constexpr int kStreamed = 2;

// Offset used for an EMPTY neighbour: past the end of any gathered buffer (sizes are checked to stay below it),
// so the buffer load's range check returns zeros.
constexpr uint32_t kOutOfRange = 0xffff0000u;
constexpr uint64_t kMaxBufferBytes = 0xfffe0000ull;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  // word 3 = 0x00020000: 32-bit data format, the raw-buffer setting for gfx9-family (CDNA) parts
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}

// Logical tile of workgroup g when tiles are dealt to the XCDs in runs (workgroup ids go to the 8 XCDs in turn):
// each XCD takes run consecutive tiles of every 8 * run, in order; a last, partial block of rem < 8 * run tiles gives
// XCD x rem / 8 of them (one more for x < rem % 8). A bijection of [0, T); g >= T has no tile (-1).
__device__ __forceinline__ int xcd_run_tile(int g, int T, int run) {
  if (g >= T) return -1;
  const int bs = 8 * run, base = g / bs * bs, r = g - base, x = r % 8, k = r / 8, rem = min(bs, T - base);
  return base + x * (rem / 8) + min(x, rem % 8) + k;
}

// vmcnt-only s_waitcnt (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14])
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Workgroup barrier without the memory fence of __syncthreads(): that fence waits for every outstanding vector
// load (vmcnt(0)), including LDS-DMA prefetches meant to stay in flight. Callers order LDS data themselves
// (counted vmcnt waits); the empty asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void wg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// SiLU with the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp each). Large negative v gives
// exp -> inf, rcp -> 0 and a signed zero, as v / (1 + exp(-v)) does.
__device__ __forceinline__ float silu(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }
// fp16-compatible epilogue helpers: round to fp16 and back; SiLU with the IEEE quotient and the accurate exp
__device__ __forceinline__ float f16r(float v) { return (float)(_Float16)v; }
__device__ __forceinline__ float silu_ieee(float v) { return v / (1.0f + expf(-v)); }

struct ConvArgs {
  const uint16_t* x;
  const uint16_t* w;
  const float* bias;
  const void* res;
  void* out;
  const uint32_t* nbr;
  const int32_t* order;
  const uint32_t* tbl;  // neighbour table in tile order (SpConvCache::row_table), for the kernels that use it
  const int32_t* gs;    // neighbour masks in tile order
  const int32_t* gray;
  const uint32_t* code;
  const int32_t* hrows;    // halo schedule (SpConvCache::halo_table), for k_conv_halo
  const int32_t* hcount;
  const uint16_t* hidx;
  const uint32_t* hgm;
  const int32_t* tsched;  // row tiles in dispatch order (SpConvCache::tile_schedule), for k_conv_w256
  int kcontig;             // narrow kernel at Ci = 128: K step m reads bytes m*64 .. +64 of a row (k_pack_w_narrow natural order)
  // spill tiles of the halo schedule (k_conv_narrow): workgroup g computes tile tlist[g] if g < *tcount, with the
  // identity row order (tbl = nbr, gs = gray in input order) and exits otherwise
  const int32_t* tlist;
  const int32_t* tcount;
  const int32_t* rmap;  // gathered conv through the halo kernel: halo row h reads source row rmap[h] >> rshift
  int rshift, rmax;
  // skip residual (upsample block, halo kernel only): residual[i, c] = skip_x[src[i] >> 3, (src[i] & 7) * Cin/8 +
  // c / rep] with src = skip_src, Cin = skip_cin, rep = skip_rep (a power of two)
  const uint16_t* skip_x;
  const int32_t* skip_src;
  int skip_cin, skip_rep;
  uint32_t skip_bytes, skip_n;
  // pre-activation of the input rows (halo kernel only, ln_on): each halo row becomes act(LayerNorm(row) * ln_gamma
  // + ln_beta) before the K loop, ln_act = ACT_NONE / ACT_SILU, gamma / beta f32 [Ci] or null
  const float* ln_gamma;
  const float* ln_beta;
  float ln_eps;
  int ln_act, ln_on;
  int N, Ci, Co, res_dt, out_dt, act;
  int tiles_m, tiles_n, grid;
  uint32_t x_bytes, w_bytes, nbr_bytes, res_bytes, out_bytes, tbl_bytes;
  // Tail split of the 256-channel wide kernel (part != nullptr): XCD x owns tiles [xt0[x], xt0[x+1]); the first
  // xs of them run whole, each later one is split into xk[x] workgroups over its K stages, which write fp32
  // partial tiles [BM][256] from slot xpart0[x] on; k_split_reduce sums them and applies the epilogue.
  float* part;
  // tail-split schedule (part set): logical tiles numbered channel-tile-major (tile = tn * tiles_m + tm), so the
  // contiguous range an XCD walks stays on one 256-column weight slice instead of cycling through all of them
  // (C2, 768 -> 768: 32 MB of weights, past L2; 0.298 -> 0.287 ms)
  int tnmaj;
  int xt0[9], xk[8], xpart0[8], xs;
  // Tiles dealt to the XCDs in runs: each XCD takes xblk consecutive tiles of every 8*xblk, in order (k_conv_wide_dma's
  // longest-first schedule, k_conv_halo's windows). 0: one tile per XCD in turn (wide), one contiguous range per XCD
  // (halo).
  int xblk;
};

template <bool F16, int BM, int BN, int WGM, int WGN, int KC>
__global__ void __launch_bounds__(WGM* WGN * 64) k_conv(ConvArgs a) {
  constexpr int NT = WGM * WGN * 64;
  constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / 32, TN = WTN / 32;
  constexpr int PC = KC / 8;  // 16-byte pieces per row per stage
  constexpr int LD = KC + 8;  // LDS row stride in elements (16-byte pad against bank conflicts)
  constexpr int AL = BM * PC / NT, BL = BN * PC / NT;
  static_assert(TM >= 1 && TN >= 1 && AL * NT == BM * PC && BL * NT == BN * PC, "tile shape");
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LD];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LD];

  // XCD-contiguous tile walk: hardware round-robins workgroup ids over the 8 XCDs.
  const int g = blockIdx.x, per = a.grid / 8;
  const int logical = (g % 8) * per + g / 8;
  if (logical >= a.tiles_m * a.tiles_n) return;
  const int tm_ = logical / a.tiles_n, tn_ = logical % a.tiles_n;
  const int row0 = tm_ * BM, co0 = tn_ * BN;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, wm = wid % WGM, wn = wid / WGM;
  const int N = a.N, Ci = a.Ci, nkc = Ci / KC;

  int orow[AL];
#pragma unroll
  for (int j = 0; j < AL; j++) {
    int r = row0 + (tid + j * NT) / PC;
    orow[j] = r < N ? a.order[r] : -1;
  }
  uint32_t m = a.code[tm_];
  const int total = __popc(m) * nkc;
  auto fetch = [&](int v, uint32_t* s) {
#pragma unroll
    for (int j = 0; j < AL; j++) s[j] = orow[j] >= 0 ? a.nbr[(i64)orow[j] * 27 + v] : EMPTY;
  };
  int cv = m ? __ffs(m) - 1 : 0;
  m &= m - 1;
  int nv = m ? __ffs(m) - 1 : -1;
  if (m) m &= m - 1;
  uint32_t srcA[AL], srcN[AL];
  if (total) fetch(cv, srcA);
  if (nv >= 0) fetch(nv, srcN);
  int kc = 0;

  u32x4 ra[AL], rb[BL];
  auto gload = [&]() {
    const int k0 = kc * KC;
#pragma unroll
    for (int j = 0; j < AL; j++) {
      int pc = (tid + j * NT) % PC;
      ra[j] = srcA[j] == EMPTY ? u32x4{0, 0, 0, 0}
                               : *(const u32x4*)(a.x + (i64)srcA[j] * Ci + k0 + pc * 8);
    }
#pragma unroll
    for (int j = 0; j < BL; j++) {
      int q = tid + j * NT, r = q / PC, pc = q % PC;
      rb[j] = *(const u32x4*)(a.w + ((i64)(co0 + r) * 27 + cv) * Ci + k0 + pc * 8);
    }
  };
  auto advance = [&]() {
    if (++kc == nkc) {
      kc = 0;
      cv = nv;
#pragma unroll
      for (int j = 0; j < AL; j++) srcA[j] = srcN[j];
      nv = m ? __ffs(m) - 1 : -1;
      if (m) m &= m - 1;
      if (nv >= 0) fetch(nv, srcN);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < AL; j++) {
      int q = tid + j * NT;
      *(u32x4*)&As[buf][(q / PC) * LD + (q % PC) * 8] = ra[j];
    }
#pragma unroll
    for (int j = 0; j < BL; j++) {
      int q = tid + j * NT;
      *(u32x4*)&Bs[buf][(q / PC) * LD + (q % PC) * 8] = rb[j];
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = f32x16{};

  int buf = 0;
  if (total) {
    gload();
    advance();
    sstore(0);
  }
  __syncthreads();
  for (int it = 0; it < total; it++) {
    const bool more = it + 1 < total;
    if (more) {
      gload();
      advance();
    }
#pragma unroll
    for (int ks = 0; ks < KC / 16; ks++) {
      u32x4 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; i++)
        fa[i] = *(const u32x4*)&As[buf][(wm * WTM + i * 32 + (lane & 31)) * LD + ks * 16 + (lane >> 5) * 8];
#pragma unroll
      for (int j = 0; j < TN; j++)
        fb[j] = *(const u32x4*)&Bs[buf][(wn * WTN + j * 32 + (lane & 31)) * LD + ks * 16 + (lane >> 5) * 8];
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = mfma32<F16>(fa[i], fb[j], acc[i][j]);
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

  // epilogue: bias, activation, residual, one rounding to the output dtype, scatter through `order`
#pragma unroll
  for (int j = 0; j < TN; j++) {
    const int co = co0 + wn * WTN + j * 32 + (lane & 31);
    const float bv = a.bias ? a.bias[co] : 0.f;
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
      for (int e = 0; e < 16; e++) {
        int r = row0 + wm * WTM + i * 32 + (e / 4) * 8 + (lane >> 5) * 4 + (e % 4);
        if (r >= N) continue;
        i64 o = (i64)a.order[r] * a.Co + co;
        float v;
        if (a.act & EPI_F16_COMPAT) {
          v = f16r(f16r(acc[i][j][e]) + bv);
          if ((a.act & ~EPI_F16_COMPAT) == ACT_SILU) v = f16r(silu_ieee(v));
          if (a.res) v = f16r(v + load_elem(a.res, o, a.res_dt));
        } else {
          v = acc[i][j][e] + bv;
          if (a.act == ACT_SILU) v = silu(v);
          if (a.res) v += load_elem(a.res, o, a.res_dt);
        }
        store_elem(a.out, o, a.out_dt, v);
      }
    }
  }
}

// Compile-time unrolled loop: f(std::integral_constant<int, i>) for i in [0, N) (keeps register arrays indexed by
// constants, so they never fall back to scratch memory).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// two fp32 -> packed 16-bit, round to nearest even (bf16: one v_cvt_pk_bf16_f32)
template <bool BF>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (BF) return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
}

// Epilogue target of the tiled kernels: output and residual as buffer resources. Callers pass the element offset
// of 8 consecutive channels of one output row and whether the row exists; a missing row (past N) uses byte offset
// kOutOfRange, so its residual loads return zeros and its stores are dropped by the range check -- no branches.
struct Epi {
  __amdgpu_buffer_rsrc_t out, res;
  int out_dt, res_dt;  // res_dt < 0: no residual
  bool silu;
  bool compat;  // EPI_F16_COMPAT: the reference's fp16 rounding sequence (fp16 out, bias and residual)
};
__device__ __forceinline__ Epi make_epi(const ConvArgs& a) {
  Epi e;
  e.out = make_rsrc(a.out, a.out_bytes);
  e.res = make_rsrc(a.res, a.res_bytes);
  e.out_dt = a.out_dt;
  e.res_dt = a.res ? a.res_dt : -1;
  e.silu = (a.act & ~EPI_F16_COMPAT) == ACT_SILU;
  e.compat = (a.act & EPI_F16_COMPAT) != 0;
  return e;
}

// residual segment of 8 channels as raw bits: 8 x bf16/f16 in r[0], or 8 x f32 in r[0..1]
__device__ __forceinline__ void load_res8(const Epi& e, uint32_t o, bool ok, u32x4 (&r)[2]) {
  r[0] = r[1] = u32x4{0, 0, 0, 0};
  if (e.res_dt == F32) {
    const uint32_t b = ok ? o * 4u : kOutOfRange;
    r[0] = __builtin_amdgcn_raw_buffer_load_b128(e.res, b, 0, kStreamed);
    r[1] = __builtin_amdgcn_raw_buffer_load_b128(e.res, b + 16, 0, kStreamed);
  } else if (e.res_dt >= 0) {
    r[0] = __builtin_amdgcn_raw_buffer_load_b128(e.res, ok ? o * 2u : kOutOfRange, 0, kStreamed);
  }
}

// out[o .. o+8) = act(v + bias) [+ residual r], one rounding to the output dtype
__device__ __forceinline__ void store_row8(const Epi& e, uint32_t o, bool ok, float (&v)[8], const float (&bias8)[8],
                                           const u32x4 (&r)[2]) {
  if (e.compat) {  // f16(f16(acc) + b), then f16(silu), then f16(y + residual); every value is an fp16 from here
#pragma unroll
    for (int q = 0; q < 8; q++) {
      float y = f16r(f16r(v[q]) + bias8[q]);
      if (e.silu) y = f16r(silu_ieee(y));
      if (e.res_dt == F16) y = f16r(y + f16_to_f32((uint16_t)(r[0][q >> 1] >> ((q & 1) * 16))));
      v[q] = y;
    }
    u32x4 w;
#pragma unroll
    for (int q = 0; q < 4; q++) w[q] = pack2<false>(v[2 * q], v[2 * q + 1]);
    __builtin_amdgcn_raw_buffer_store_b128(w, e.out, ok ? o * 2u : kOutOfRange, 0, kStreamed);
    return;
  }
#pragma unroll
  for (int q = 0; q < 8; q++) v[q] += bias8[q];
  if (e.silu) {
#pragma unroll
    for (int q = 0; q < 8; q++) v[q] = silu(v[q]);
  }
  if (e.res_dt == F32) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      v[q] += __uint_as_float(r[0][q]);
      v[q + 4] += __uint_as_float(r[1][q]);
    }
  } else if (e.res_dt == BF16) {
#pragma unroll
    for (int q = 0; q < 8; q++) v[q] += __uint_as_float((q & 1) ? (r[0][q >> 1] & 0xffff0000u) : (r[0][q >> 1] << 16));
  } else if (e.res_dt == F16) {
#pragma unroll
    for (int q = 0; q < 8; q++) v[q] += f16_to_f32((uint16_t)(r[0][q >> 1] >> ((q & 1) * 16)));
  }
  if (e.out_dt == F32) {
    const uint32_t b = ok ? o * 4u : kOutOfRange;
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                                 __float_as_uint(v[3])}, e.out, b, 0, kStreamed);
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                                                 __float_as_uint(v[7])}, e.out, b + 16, 0, kStreamed);
  } else {
    u32x4 w;
    if (e.out_dt == BF16) {
#pragma unroll
      for (int q = 0; q < 4; q++) w[q] = pack2<true>(v[2 * q], v[2 * q + 1]);
    } else {
#pragma unroll
      for (int q = 0; q < 4; q++) w[q] = pack2<false>(v[2 * q], v[2 * q + 1]);
    }
    __builtin_amdgcn_raw_buffer_store_b128(w, e.out, ok ? o * 2u : kOutOfRange, 0, kStreamed);
  }
}

// Epilogue of one 32-row x 64-channel accumulator group, staged through LDS so every lane writes 16 contiguous
// bytes: out[order[r], co] = act(acc + b) [+ residual]. `ew` is this wavefront's private [32][72] fp32 area.
// Residual loads of one 32-row group (4 rows per lane slot p): RK 0 none, 1 fp32, 2 bf16/f16.
template <int RK, bool NEG = false>
__device__ __forceinline__ void load_group_res(const Epi& e, const int* tile_order, int rbase, int nrows, int Co,
                                               int col, int lane, u32x4 (&r)[4][2]) {
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const int rr = rbase + p * 8 + (lane >> 3);
    const uint32_t o = (uint32_t)tile_order[rr] * (uint32_t)Co + (uint32_t)col;
    const bool ok = rr < nrows && (!NEG || tile_order[rr] >= 0);
    r[p][0] = r[p][1] = u32x4{0, 0, 0, 0};
    if constexpr (RK == 1) {
      r[p][0] = __builtin_amdgcn_raw_buffer_load_b128(e.res, ok ? o * 4u : kOutOfRange, 0, kStreamed);
      r[p][1] = __builtin_amdgcn_raw_buffer_load_b128(e.res, ok ? o * 4u + 16u : kOutOfRange, 0, kStreamed);
    } else if constexpr (RK == 2) {
      r[p][0] = __builtin_amdgcn_raw_buffer_load_b128(e.res, ok ? o * 2u : kOutOfRange, 0, kStreamed);
    }
  }
}

// Epilogue of one 32-row x 64-channel accumulator group, staged through LDS so every lane writes 16 contiguous
// bytes: out[order[r], co] = act(acc + b) [+ residual r]. `ew` is this wavefront's private [32][72] fp32 area.
template <int TN, int TA = TN, int T0 = 0, bool NEG = false>
__device__ __forceinline__ void epilogue_group(const f32x16 (&acc)[TA], float* ew, const int* tile_order, int rbase,
                                               int nrows, int col, const float (&bias8)[8], const Epi& e, int Co,
                                               int lane, const u32x4 (&r)[4][2]) {
  constexpr int ES = 72;  // row stride in floats: 4 rows apart differ by 32 banks, so the scatter is conflict-free
  const int h = lane >> 5, l32 = lane & 31;
  const int c8 = (lane & 7) * 8;
#pragma unroll
  for (int t = 0; t < TN; t++)
#pragma unroll
    for (int i = 0; i < 16; i++) ew[((i >> 2) * 8 + h * 4 + (i & 3)) * ES + t * 32 + l32] = acc[T0 + t][i];
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const int rr = p * 8 + (lane >> 3);
    float v[8];
    *(f32x4*)&v[0] = *(const f32x4*)&ew[rr * ES + c8];
    *(f32x4*)&v[4] = *(const f32x4*)&ew[rr * ES + c8 + 4];
    const int orow = tile_order[rbase + rr];
    store_row8(e, (uint32_t)orow * (uint32_t)Co + (uint32_t)col, rbase + rr < nrows && (!NEG || orow >= 0), v, bias8, r[p]);
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

// All TM groups of a wavefront's 32*TM x 64 accumulator tile. Stores and loads share one in-order completion
// counter, so a residual load issued after a store cannot be waited for without also waiting for that store: the
// residuals of group i+1 are therefore requested before the stores of group i, and a tile without a residual
// issues no loads at all (its stores never hold the wavefront up).
// (TA: columns of the accumulator array; the tile's 64 channels are its columns T0 .. T0 + TN. NEG: rows whose
// tile_order entry is negative are absent)
template <int TM, int TN, int TA = TN, int T0 = 0, bool NEG = false>
__device__ __forceinline__ void epilogue_tile(const f32x16 (&acc)[TM][TA], float* ew, const int* tile_order,
                                              int nrows, int co_w, const float (&bias8)[8], const Epi& e, int Co,
                                              int lane) {
  const int col = co_w + (lane & 7) * 8;
  auto run = [&](auto RKc) __attribute__((always_inline)) {
    constexpr int RK = decltype(RKc)::value;
    u32x4 r[2][4][2];
    load_group_res<RK, NEG>(e, tile_order, 0, nrows, Co, col, lane, r[0]);
    static_for<TM>([&](auto I) __attribute__((always_inline)) {
      if constexpr (I + 1 < TM)
        load_group_res<RK, NEG>(e, tile_order, (I + 1) * 32, nrows, Co, col, lane, r[(I + 1) & 1]);
      epilogue_group<TN, TA, T0, NEG>(acc[I], ew, tile_order, I * 32, nrows, col, bias8, e, Co, lane, r[I & 1]);
    });
  };
  if (e.res_dt < 0) run(std::integral_constant<int, 0>{});
  else if (e.res_dt == F32) run(std::integral_constant<int, 1>{});
  else run(std::integral_constant<int, 2>{});
}

// Wide-channel kernel: BM sorted rows x BN = 64*NW channels, NW wavefronts; each wavefront owns all BM rows x its
// own 64 channels (BM/32 x 2 tiles of 32x32 fp32 accumulators).
//  * Traffic: per K stage (one offset v x 64 input channels) a workgroup reads BM gathered rows and BN weight rows
//    of 128 bytes, for 2*BM*BN*64 flops; BM = BN = 256 keeps this at 0.0078 byte/flop, which L2 can feed.
//  * Skipping: the K loop runs over the union of the tile's neighbour masks, but each 32-row group has its own
//    mask and skips its MFMAs for offsets none of its rows has, so padding work follows 32-row granularity.
//  * Software pipeline: stage s issues the gather loads of A(s+2) and the weight loads of B(s+1), runs the MFMAs of
//    stage s (A(s) from LDS, B(s) from registers), then writes A(s+1) -- loaded a full stage earlier -- into the
//    other LDS buffer and synchronises. The loop is unrolled by two so registers and buffers have fixed names.
//  * Only A is shared by the wavefronts, so only A goes through LDS; weights (L2-resident) stream straight into
//    MFMA operand registers. At tile start the offset list, the 32-row masks, the tile's output row indices and its
//    [BM x 27] neighbour indices are staged in LDS: the K loop has no dependent global loads. EMPTY neighbours
//    read past the end of the feature buffer, so every gather is an unconditional 16-byte load.
//  * LDS layout of a stage: row r occupies 128 contiguous bytes as eight 16-byte slots; channel piece p of row r is
//    stored in slot p ^ (r & 7) so the MFMA operand reads (32 rows, one piece) hit distinct banks.
//  * Within a 64-channel stage the K order is permuted (lane half h, step j -> piece h*4 + j) identically for A and
//    B, so each lane's four weight loads are one contiguous 64-byte run.
//  * Epilogue: per 32-row group, accumulators go through LDS and leave as 16-byte row segments (bias, SiLU,
//    residual fused, one rounding).
template <bool F16, int NW, int BM>
__global__ void __launch_bounds__(NW * 64) k_conv_wide(ConvArgs a) {
  constexpr int NT = NW * 64, KC = 64, PC = KC / 8;
  constexpr int TM = BM / 32, TN = 2, AL = BM * PC / NT;  // AL gather loads per lane per stage
  static_assert(AL * NT == BM * PC && TM <= 8, "tile shape");
  __shared__ __attribute__((aligned(16))) u32x4 As[2][BM * PC];
  __shared__ uint32_t srcT[BM * 27];
  __shared__ int ordT[BM];
  __shared__ uint32_t gmask[TM];
  __shared__ int vlist[32];

  const int g = blockIdx.x, per = a.grid / 8;
  const int logical = (g % 8) * per + g / 8;
  if (logical >= a.tiles_m * a.tiles_n) return;
  const int tm_ = logical / a.tiles_n, tn_ = logical % a.tiles_n;
  const int row0 = tm_ * BM, co0 = tn_ * (64 * NW);
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31, wn = tid >> 6;
  const int N = a.N, Ci = a.Ci, nkc = Ci / KC;

  // prologue: row indices, 32-row masks (OR of the rows' neighbour masks), offset list, neighbour table
  for (int r = tid; r < BM; r += NT) {
    const int row = row0 + r;
    const int o = row < N ? a.order[row] : 0;
    ordT[r] = o;
    uint32_t gm = row < N ? (uint32_t)a.gray[o] : 0u;
#pragma unroll
    for (int d = 1; d < 32; d <<= 1) gm |= (uint32_t)__shfl_xor((int)gm, d, 64);
    if ((r & 31) == 0) gmask[r >> 5] = gm;
  }
  __syncthreads();
  uint32_t mask = 0;
#pragma unroll
  for (int i = 0; i < TM; i++) mask |= gmask[i];
  const int nvv = __popc(mask), total = nvv * nkc;
  if (tid < 27 && ((mask >> tid) & 1u)) vlist[__popc(mask & ((1u << tid) - 1u))] = tid;
  const uint32_t row_bytes = (uint32_t)Ci * 2u;
  // one row per thread: its 27 neighbour indices are one contiguous 108-byte run, loaded as 27 independent loads
  for (int r = tid; r < BM; r += NT) {
    uint32_t src[27];
    const bool live = row0 + r < N;
    const uint32_t* nrow = a.nbr + (i64)ordT[r] * 27;
#pragma unroll
    for (int v = 0; v < 27; v++) src[v] = live ? nrow[v] : EMPTY;
#pragma unroll
    for (int v = 0; v < 27; v++) srcT[r * 27 + v] = src[v] == EMPTY ? kOutOfRange : src[v] * row_bytes;
  }
  uint32_t gms[TM];
#pragma unroll
  for (int i = 0; i < TM; i++) gms[i] = __builtin_amdgcn_readfirstlane(gmask[i]);
  __syncthreads();

  // this lane's gather pieces: LDS unit u = k*NT + tid -> row u/8, slot u%8, channel piece slot ^ (row & 7)
  int arow[AL], apiece[AL];
#pragma unroll
  for (int k = 0; k < AL; k++) {
    int u = k * NT + tid;
    arow[k] = u >> 3;
    apiece[k] = (u & 7) ^ ((arow[k] >> 1) & 7);
  }
  // buffer resources: 32-bit offsets, and gathers of EMPTY neighbours (offset kOutOfRange) return zeros
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes), rw = make_rsrc(a.w, a.w_bytes);
  // packed weights: the stage (v, kc) fragment of this wavefront's 64-channel slice is 8 KiB at
  // ((slice*27 + v)*nkc + kc) * 8 KiB, as [t][j][lane][16 bytes]
  const uint32_t wslice = (uint32_t)((co0 >> 6) + wn) * 27u * (uint32_t)nkc;
  const uint32_t wlane = (uint32_t)lane * 16u;

  // stage cursors (offset index, channel block); loads past the last stage re-read the last stage
  int avi = 0, akc = 0, bvi = 0, bkc = 0, cvi = 0, ckc = 0;
  auto next = [&](int& vi, int& kc) __attribute__((always_inline)) {
    const bool wrap = kc + 1 == nkc;
    kc = wrap ? 0 : kc + 1;
    vi += wrap ? 1 : 0;
  };
  auto load_a = [&](u32x4 (&ra)[AL]) __attribute__((always_inline)) {
    const bool live = avi < nvv;
    const int v = __builtin_amdgcn_readfirstlane(vlist[live ? avi : nvv - 1]);
    const int k0 = __builtin_amdgcn_readfirstlane((live ? akc : nkc - 1) * KC);
    uint32_t off[AL];
#pragma unroll
    for (int k = 0; k < AL; k++) off[k] = srcT[arow[k] * 27 + v];
#pragma unroll
    for (int k = 0; k < AL; k++)
      ra[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, off[k] + apiece[k] * 16, k0 * 2, 0);
    next(avi, akc);
  };
  auto store_a = [&](int buf, const u32x4 (&ra)[AL]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < AL; k++) As[buf][k * NT + tid] = ra[k];
  };
  auto load_b = [&](u32x4 (&rb)[TN][4]) __attribute__((always_inline)) {
    const bool live = bvi < nvv;
    const int v = __builtin_amdgcn_readfirstlane(vlist[live ? bvi : nvv - 1]);
    const int k0 = __builtin_amdgcn_readfirstlane((live ? bkc : nkc - 1) * KC);
    const int soff = __builtin_amdgcn_readfirstlane((int)((wslice + (uint32_t)(v * nkc) + (uint32_t)(k0 / KC)) * 8192u));
#pragma unroll
    for (int t = 0; t < TN; t++)
#pragma unroll
      for (int j = 0; j < 4; j++) rb[t][j] = __builtin_amdgcn_raw_buffer_load_b128(rw, wlane + (t * 4 + j) * 1024, soff, 0);
    next(bvi, bkc);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int t = 0; t < TN; t++) acc[i][t] = f32x16{};
  // One K stage, with the next stages' traffic interleaved between the MFMA groups so the vector-memory and LDS
  // queues drain while the matrix cores run: group i issues its share of the A(s+2) gathers and B(s+1) weight
  // loads, writes its share of A(s+1) (loaded a stage ago) into the other LDS buffer, prefetches the operands of
  // group i+1, then runs its MFMAs if any of its 32 rows has offset v.
  auto stage = [&](int buf, const u32x4 (&rbC)[TN][4], const u32x4 (&raW)[AL], u32x4 (&raL)[AL],
                   u32x4 (&rbN)[TN][4]) __attribute__((always_inline)) {
    const uint32_t vbit = 1u << __builtin_amdgcn_readfirstlane(vlist[cvi]);
    next(cvi, ckc);
    // A(s+2) addresses
    const bool alive = avi < nvv;
    const int va = __builtin_amdgcn_readfirstlane(vlist[alive ? avi : nvv - 1]);
    const int ka = __builtin_amdgcn_readfirstlane((alive ? akc : nkc - 1) * KC * 2);
    next(avi, akc);
    uint32_t off[AL];
#pragma unroll
    for (int k = 0; k < AL; k++) off[k] = srcT[arow[k] * 27 + va] + apiece[k] * 16;
    // B(s+1) base
    const bool blive = bvi < nvv;
    const int vb = __builtin_amdgcn_readfirstlane(vlist[blive ? bvi : nvv - 1]);
    const int kb = blive ? bkc : nkc - 1;
    const int soff = __builtin_amdgcn_readfirstlane((int)((wslice + (uint32_t)(vb * nkc + kb)) * 8192u));
    next(bvi, bkc);

    u32x4 fa[2][4];
    auto read_fa = [&](u32x4 (&f)[4], int i) __attribute__((always_inline)) {
      const int r = i * 32 + l32;
#pragma unroll
      for (int j = 0; j < 4; j++) f[j] = As[buf][r * PC + ((h * 4 + j) ^ ((r >> 1) & 7))];
    };
    read_fa(fa[0], 0);
    constexpr int AG = AL / TM, BG = TN * 4 / TM;  // loads per group
    static_assert(AG * TM == AL && BG * TM == TN * 4 && BG >= 1, "load split");
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
      for (int k = i * AG; k < (i + 1) * AG; k++) raL[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, off[k], ka, 0);
#pragma unroll
      for (int q = i * BG; q < (i + 1) * BG; q++)
        rbN[q / 4][q % 4] = __builtin_amdgcn_raw_buffer_load_b128(rw, wlane + q * 1024, soff, 0);
#pragma unroll
      for (int k = i * AG; k < (i + 1) * AG; k++) As[buf ^ 1][k * NT + tid] = raW[k];
      if (i + 1 < TM) read_fa(fa[(i + 1) & 1], i + 1);
      if (gms[i] & vbit) {
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
          for (int t = 0; t < TN; t++) acc[i][t] = mfma32<F16>(fa[i & 1][j], rbC[t][j], acc[i][t]);
      }
    }
    __syncthreads();
  };

  if (total > 0) {
    u32x4 ra0[AL], ra1[AL], rb0[TN][4], rb1[TN][4];
    load_a(ra0);  // A(0)
    load_b(rb0);  // B(0)
    load_a(ra1);  // A(1)
    store_a(0, ra0);
    __syncthreads();
    for (int s = 0; s < total; s += 2) {
      stage(0, rb0, ra1, ra0, rb1);  // MFMAs of stage s; writes A(s+1); loads A(s+2), B(s+1)
      if (s + 1 >= total) break;
      stage(1, rb1, ra0, ra1, rb0);  // stage s+1; writes A(s+2); loads A(s+3), B(s+2)
    }
  }

  // epilogue through this wavefront's share of the (now idle) A buffers
  float* ew = (float*)&As[0][0] + wn * (32 * 72);
  static_assert(NW * 32 * 72 * 4 <= 2 * BM * PC * 16, "epilogue staging fits in the A buffers");
  const int co_w = co0 + wn * 64;
  float bias8[8];
#pragma unroll
  for (int q = 0; q < 8; q++) bias8[q] = a.bias ? a.bias[co_w + (lane & 7) * 8 + q] : 0.f;
  const int nrows = N - row0;
  const Epi e = make_epi(a);
  epilogue_tile<TM, TN>(acc, ew, ordT, nrows, co_w, bias8, e, a.Co, lane);
}

typedef float f32x4v __attribute__((ext_vector_type(4)));
template <bool F16>
__device__ __forceinline__ f32x4v mfma16(u32x4 a, u32x4 b, f32x4v c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Weight repack for the narrow kernel: w [Co,27,Ci] -> per offset v, per 16-column tile t, per 32-channel step m,
// one 1 KiB block of 64 lanes x 16 bytes in v_mfma_f32_16x16x32 operand order: lane l holds column t*16 + (l & 15),
// input channels ((l >> 4)*S + m)*8 .. +8 (S = Ci/32 steps; lane quarter q owns channels q*8S .. q*8S + 8S).
// Grid (S, T, 27) of 64-thread blocks: block (m, t, v) writes destination block ((v*T + t)*S + m), so no thread
// divides (the 64-bit division of a flat index cost more than the copy).
// With contig set, step m holds channels m*32 + (l >> 4)*8 .. +8 instead (the operand order of a row read as S
// contiguous 64-byte pieces, one per step).
__global__ void __launch_bounds__(64) k_pack_w_narrow(const u32x4* __restrict__ w, u32x4* __restrict__ wp, int Co,
                                                      int Ci, int contig = 0) {
  const int S = Ci / 32, T = Co / 16, lane = threadIdx.x;
  const int m = blockIdx.x, t = blockIdx.y, v = blockIdx.z;
  const int co = t * 16 + (lane & 15), ch = (contig ? m * 4 + (lane >> 4) : (lane >> 4) * S + m) * 8;
  wp[(((i64)v * T + t) * S + m) * 64 + lane] = w[((i64)co * 27 + v) * Ci / 8 + ch / 8];
}

// Narrow-channel kernel (Co = 16*T <= 64, Ci = 32*S <= 128): the layers that are bound by HBM traffic (gathers,
// neighbour table, residual, output) rather than by the matrix cores.
//  * Workgroup = 4 wavefronts x 64 rows (256 rows of the row order); each wavefront owns its 64 rows x all Co
//    columns as 4 groups of 16 rows x T tiles of 16x16 fp32 accumulators (v_mfma_f32_16x16x32).
//  * Gathers go straight from global memory into MFMA operand registers: lane (row r, quarter q) of a 16-row group
//    loads channels q*8S .. q*8S+8S of the neighbour row (S contiguous 16-byte loads; a row's four lanes read one
//    contiguous Ci*2-byte run), through a buffer resource whose range check turns EMPTY into zeros.
//  * Weights: per offset, the [Co x Ci] slice (in MFMA operand order) is staged once per workgroup in LDS
//    (double-buffered, loaded while the previous offset computes) and shared by the 4 wavefronts.
//  * Skipping: each 16-row group has its own neighbour mask; groups without offset v issue neither gathers nor
//    MFMAs for it. Rows come in the order the caller chooses (null = identity); the spatial (Morton) order keeps
//    the gathers of neighbouring rows in L2.
//  * Epilogue: per 16-row group, accumulators go through LDS and leave as 16-byte segments of whole output rows.
//  * LITE (used at Ci = 128, G = 2): the gathers run one offset ahead instead of two, the weight fragments are read
//    from LDS per K step, and residuals are loaded in the epilogue instead of staged in LDS -- 158 VGPRs and 47 KB of
//    LDS, so three workgroups per CU instead of two. The gathers are served from the MALL and the loop waits on
//    them; a third workgroup hides more than the second offset of look-ahead did (C5 children 0.907 -> 0.856 ms;
//    two offsets ahead with the other savings, still two workgroups per CU: 0.923). Same sums, same bits.
// Copies rows [row0, row0+BM) of the tile-ordered neighbour table (27 u32 per row, contiguous) into LDS by DMA:
// 16 bytes per lane, so each wavefront instruction moves 1 KiB with no registers involved.
template <int BM, int NT>
__device__ __forceinline__ void dma_tile_table(const ConvArgs& a, int row0, uint32_t* srcT, int tid) {
  constexpr int TU = BM * 27 / 4;  // 16-byte units
  const __amdgpu_buffer_rsrc_t rt = make_rsrc(a.tbl, a.tbl_bytes);
  const uint32_t base = (uint32_t)row0 * 108u;
#pragma unroll
  for (int k = 0; k < (TU + NT - 1) / NT; k++) {
    const int u = k * NT + tid;
    if (u < TU)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (__attribute__((address_space(3))) void*)&srcT[(k * NT + (tid & ~63)) * 4],
                                               16, base + (uint32_t)u * 16u, 0, 0, kStreamed);
  }
}
// Byte offset of neighbour row n in a feature matrix with `rowbytes` bytes per row; EMPTY -> past the buffer end
__device__ __forceinline__ uint32_t nbr_offset(uint32_t n, uint32_t rowbytes) {
  return n == EMPTY ? kOutOfRange : n * rowbytes;
}

// 8 consecutive channels c8.. of the skip residual of one output row, as 8 x 16-bit in r (src < 0 or past the
// source rows: zeros). Channel c reads element c / rep of the parent's slot, so 8 channels need 8 / rep elements
// (one for rep >= 8): one 16-, 8-, 4- or 2-byte load, widened by repeating each element rep times.
__device__ __forceinline__ u32x4 load_skip8(const __amdgpu_buffer_rsrc_t& rs, const ConvArgs& a, int src, int c8,
                                            bool ok) {
  const uint32_t s = (uint32_t)src;
  const bool live = ok && s < a.skip_n * 8u;
  const uint32_t base = (s >> 3) * (uint32_t)a.skip_cin + (s & 7u) * (uint32_t)(a.skip_cin >> 3) +
                        (uint32_t)(c8 / a.skip_rep);
  const uint32_t off = live ? base * 2u : kOutOfRange;
  auto dup = [](uint32_t v16) { return (v16 & 0xffffu) | (v16 << 16); };
  if (a.skip_rep == 1) return __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
  if (a.skip_rep == 2) {
    typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
    const u32x2v q = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
    return u32x4{dup(q[0]), dup(q[0] >> 16), dup(q[1]), dup(q[1] >> 16)};
  }
  if (a.skip_rep == 4) {
    const uint32_t q = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
    return u32x4{dup(q), dup(q), dup(q >> 16), dup(q >> 16)};
  }
  const uint32_t q = dup(__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0));
  return u32x4{q, q, q, q};
}

template <bool F16, int S, int T, int G, bool LITE = false>
__global__ void __launch_bounds__(256, LITE ? 3 : 1) k_conv_narrow(ConvArgs a) {
  constexpr int NT = 256, BM = 4 * 16 * G, CI = 32 * S, CO = 16 * T, WB = T * S * 64;  // WB: 16B units per offset
  static_assert(WB % NT == 0, "weight slice split");
  __shared__ __attribute__((aligned(16))) u32x4 Bs[2][WB];
  constexpr int SR = 27;  // srcT row stride: the table's 27 neighbour indices per row
  __shared__ __attribute__((aligned(16))) uint32_t srcT[BM * SR];
  __shared__ int ordT[BM];
  __shared__ __attribute__((aligned(16))) u32x4 resL[LITE ? 1 : BM * CO * 2 / 16];
  __shared__ uint32_t gmask[BM / 16];
  __shared__ int vlist[32];

  const int g = blockIdx.x, per = a.grid / 8;
  int tile = (g % 8) * per + g / 8;
  if (a.tlist) {  // spill tiles of a halo schedule
    if (g >= __builtin_amdgcn_readfirstlane(*a.tcount)) return;
    tile = __builtin_amdgcn_readfirstlane(a.tlist[g]);
  }
  if (tile >= a.tiles_m) return;
  const int row0 = tile * BM;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, r16 = lane & 15, q4 = lane >> 4;
  const int N = a.N;

  // prologue: the tile's block of the neighbour table goes to LDS by DMA; rows, 16-row masks from the same order
  // (the table is padded to whole tiles, except nbr itself for spill tiles: rows past N read zeros there, which the
  // zero mask of those rows keeps out of every result)
  dma_tile_table<BM, NT>(a, row0, srcT, tid);
  if (tid < BM) {
    const int row = row0 + tid;
    const bool live = row < N;
    ordT[tid] = live ? (a.order ? a.order[row] : row) : 0;
    uint32_t gm = live ? a.gs[row] : 0u;
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) gm |= (uint32_t)__shfl_xor((int)gm, d, 64);
    if ((tid & 15) == 0) gmask[tid >> 4] = gm;
  }
  wait_vmcnt<0>();  // this lane's table DMA has landed (the barrier below covers the other lanes)
  __syncthreads();
  if (a.rmap) {  // gathered conv: the tile's neighbour rows become source rows row_map[r] >> shift (EMPTY past rmax)
    constexpr int NE = BM * SR, PER = (NE + NT - 1) / NT;
    uint32_t mv[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int e = k * NT + tid;
      const uint32_t r = e < NE ? srcT[e] : EMPTY;
      mv[k] = r != EMPTY ? (uint32_t)a.rmap[r] : EMPTY;
    }
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int e = k * NT + tid;
      const uint32_t q = mv[k] == EMPTY ? EMPTY : mv[k] >> a.rshift;
      if (e < NE) srcT[e] = q < (uint32_t)a.rmax ? q : EMPTY;
    }
    __syncthreads();
  }
  uint32_t mask = 0;
#pragma unroll
  for (int i = 0; i < BM / 16; i++) mask |= gmask[i];
  const int nvv = __popc(mask);
  if (tid < 27 && ((mask >> tid) & 1u)) vlist[__popc(mask & ((1u << tid) - 1u))] = tid;
  uint32_t gms[G];
#pragma unroll
  for (int i = 0; i < G; i++) gms[i] = __builtin_amdgcn_readfirstlane(gmask[wv * G + i]);

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes), rw = make_rsrc(a.w, a.w_bytes);
  f32x4v acc[G][T];
#pragma unroll
  for (int i = 0; i < G; i++)
#pragma unroll
    for (int t = 0; t < T; t++) acc[i][t] = f32x4v{0.f, 0.f, 0.f, 0.f};

  constexpr int BL = WB / NT;  // weight loads per thread per offset
  // gathers of offset list entry vi into ra (groups without that offset skip their loads)
  auto gather = [&](int vi, u32x4 (&ra)[G][S]) __attribute__((always_inline)) {
    const int v = __builtin_amdgcn_readfirstlane(vlist[vi]);
    uint32_t nb[G];  // all groups' neighbour rows first: one LDS round trip, not one per group
#pragma unroll
    for (int i = 0; i < G; i++) nb[i] = srcT[(wv * (16 * G) + i * 16 + r16) * SR + v];
#pragma unroll
    for (int i = 0; i < G; i++) {
      if ((gms[i] >> v) & 1u) {
        if constexpr (LITE) {
          // lanes of rows without this neighbour skip the load (exec-masked) instead of reading out of range: at
          // Ci = 128 half the rows of an active group lack its offset (C5 children: 0.854 -> 0.839 ms; at Ci = 64
          // no gain, 0.901 -> 0.905)
          const uint32_t off = nb[i] * (CI * 2) + q4 * (a.kcontig ? 16 : S * 16);
          const uint32_t mstep = a.kcontig ? 64 : 16;
          if (nb[i] != EMPTY) {
#pragma unroll
            for (int m = 0; m < S; m++) ra[i][m] = __builtin_amdgcn_raw_buffer_load_b128(rx, off + m * mstep, 0, 0);
          } else {
#pragma unroll
            for (int m = 0; m < S; m++) ra[i][m] = u32x4{0, 0, 0, 0};
          }
        } else {
          const uint32_t off = nbr_offset(nb[i], CI * 2) + q4 * (S * 16);
#pragma unroll
          for (int m = 0; m < S; m++) ra[i][m] = __builtin_amdgcn_raw_buffer_load_b128(rx, off + m * 16, 0, 0);
        }
      }
    }
  };
  // MFMAs of offset list entry vi (weights in Bs[buf]); the weights of entry vi+2 are requested into rbL, the
  // ones of entry vi+1 (requested an iteration earlier, in rbS) are stored into the other buffer, then barrier
  auto compute = [&](int vi, int buf, const u32x4 (&ra)[G][S], u32x4 (&rbL)[BL], const u32x4 (&rbS)[BL])
      __attribute__((always_inline)) {
    const int v = __builtin_amdgcn_readfirstlane(vlist[vi]);
    const int vn = __builtin_amdgcn_readfirstlane(vlist[vi + 2 < nvv ? vi + 2 : nvv - 1]);
#pragma unroll
    for (int k = 0; k < BL; k++) rbL[k] = __builtin_amdgcn_raw_buffer_load_b128(rw, (k * NT + tid) * 16, vn * WB * 16, 0);
    if constexpr (LITE) {  // weight fragments read per K step: T instead of T x S live at once
#pragma unroll
      for (int m = 0; m < S; m++) {
        u32x4 fb[T];
#pragma unroll
        for (int t = 0; t < T; t++) fb[t] = Bs[buf][(t * S + m) * 64 + lane];
#pragma unroll
        for (int i = 0; i < G; i++) {
          if ((gms[i] >> v) & 1u) {
#pragma unroll
            for (int t = 0; t < T; t++) acc[i][t] = mfma16<F16>(ra[i][m], fb[t], acc[i][t]);
          }
        }
      }
    } else {
    u32x4 fb[T][S];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int m = 0; m < S; m++) fb[t][m] = Bs[buf][(t * S + m) * 64 + lane];
#pragma unroll
    for (int i = 0; i < G; i++) {
      if ((gms[i] >> v) & 1u) {
#pragma unroll
        for (int m = 0; m < S; m++)
#pragma unroll
          for (int t = 0; t < T; t++) acc[i][t] = mfma16<F16>(ra[i][m], fb[t][m], acc[i][t]);
      }
    }
    }
#pragma unroll
    for (int k = 0; k < BL; k++) Bs[buf ^ 1][k * NT + tid] = rbS[k];
    __syncthreads();
  };
  constexpr int LPR = CO / 8;    // epilogue: lanes per output row (8 channels each)
  constexpr int RPP = 64 / LPR;   // epilogue: rows per pass
  const int c8 = (lane % LPR) * 8;
  // 16-bit residuals: the workgroup's [BM][CO] residual tile goes global -> LDS by DMA before the K loop (its
  // latency hides behind the loop; no registers held). Rows past N read out of range and land as zeros.
  constexpr int RU = BM * CO * 2 / 16, RK = RU / NT;  // 16-byte units, DMA loads per lane
  static_assert(RK * NT == RU, "residual tile split");
  const bool res16 = !LITE && a.res && a.res_dt != F32 && !a.skip_src;  // (skip residual: loaded in the epilogue)
  if (res16) {
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res, a.res_bytes);
#pragma unroll
    for (int k = 0; k < RK; k++) {
      const int u = (wv * RK + k) * 64 + lane, rrow = u / LPR, seg = u % LPR;
      const uint32_t off = row0 + rrow < N ? ((uint32_t)ordT[rrow] * CO + seg * 8) * 2u : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (__attribute__((address_space(3))) void*)&resL[(wv * RK + k) * 64],
                                               16, off, 0, 0, kStreamed);
    }
  }
  __syncthreads();  // vlist visible
  if (nvv > 0) {
    u32x4 rb[2][BL];
    {
      const int v0 = __builtin_amdgcn_readfirstlane(vlist[0]);
      const int v1 = __builtin_amdgcn_readfirstlane(vlist[nvv > 1 ? 1 : 0]);
#pragma unroll
      for (int k = 0; k < BL; k++) Bs[0][k * NT + tid] = __builtin_amdgcn_raw_buffer_load_b128(rw, (k * NT + tid) * 16, v0 * WB * 16, 0);
#pragma unroll
      for (int k = 0; k < BL; k++) rb[1][k] = __builtin_amdgcn_raw_buffer_load_b128(rw, (k * NT + tid) * 16, v1 * WB * 16, 0);
    }
    if constexpr (LITE) {  // gathers one entry ahead (two buffers)
      u32x4 ra[2][G][S];
      gather(0, ra[0]);
      __syncthreads();
      for (int vb = 0; vb < nvv; vb += 2) {
        static_for<2>([&](auto J) __attribute__((always_inline)) {
          constexpr int j = decltype(J)::value;
          const int vi = vb + j;
          if (vi < nvv) {
            if (vi + 1 < nvv) gather(vi + 1, ra[(j + 1) % 2]);
            compute(vi, j & 1, ra[j % 2], rb[j & 1], rb[(j + 1) & 1]);
          }
        });
      }
    } else {
    u32x4 ra[3][G][S];
    gather(0, ra[0]);
    if (nvv > 1) gather(1, ra[1]);
    __syncthreads();
    // software pipeline: gathers of entries vi+1 and vi+2 and the weights of entry vi+2 are in flight while entry vi
    // computes (gather buffers rotate by 3, weight buffers by 2: unrolled by 6 so every buffer has a fixed name)
    for (int vb = 0; vb < nvv; vb += 6) {
      static_for<6>([&](auto J) __attribute__((always_inline)) {
        constexpr int j = decltype(J)::value;
        const int vi = vb + j;
        if (vi < nvv) {
          if (vi + 2 < nvv) gather(vi + 2, ra[(j + 2) % 3]);
          compute(vi, j & 1, ra[j % 3], rb[j & 1], rb[(j + 1) & 1]);
        }
      });
    }
    }
  }

  // epilogue: per 16-row group through a per-wavefront [16][CO+4] fp32 area (aliases srcT, idle now)
  constexpr int ES = CO + 4;
  // staging: the neighbour table or the weight buffers, whichever holds 4 x [16][ES] floats (both idle now)
  constexpr bool kInSrcT = 4 * 16 * ES * 4 <= BM * 27 * 4;
  static_assert(kInSrcT || 4 * 16 * ES * 4 <= 2 * WB * 16, "epilogue staging fits");
  __syncthreads();  // every wavefront is done with the table and the weight buffers
  float* ew = (kInSrcT ? (float*)srcT : (float*)&Bs[0][0]) + wv * 16 * ES;
  float bias8[8];
#pragma unroll
  for (int q = 0; q < 8; q++) bias8[q] = a.bias ? a.bias[c8 + q] : 0.f;
  constexpr int NP = 16 / RPP;
  const Epi e = make_epi(a);
  u32x4 resv[G][NP][2];
  if (a.skip_src) {  // skip residual of the upsample block (spill tiles of the fused conv + skip)
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.skip_x, a.skip_bytes);
#pragma unroll
    for (int i = 0; i < G; i++)
#pragma unroll
      for (int p = 0; p < NP; p++) {
        const int lrow = wv * (16 * G) + i * 16 + p * RPP + lane / LPR;
        const bool ok = row0 + lrow < N;
        resv[i][p][0] = load_skip8(rs, a, ok ? a.skip_src[ordT[lrow]] : -1, c8, ok);
        resv[i][p][1] = u32x4{0, 0, 0, 0};
      }
  } else if (a.res && !res16) {  // fp32 residual: straight to registers, all requested before the first group
#pragma unroll
    for (int i = 0; i < G; i++)
#pragma unroll
      for (int p = 0; p < NP; p++) {
        const int lrow = wv * (16 * G) + i * 16 + p * RPP + lane / LPR;
        load_res8(e, (uint32_t)ordT[lrow] * CO + c8, row0 + lrow < N, resv[i][p]);
      }
  }
  if (res16) {
    wait_vmcnt<0>();
    __syncthreads();  // every wavefront's residual DMA has landed
  }
#pragma unroll
  for (int i = 0; i < G; i++) {
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int q = 0; q < 4; q++) ew[(q4 * 4 + q) * ES + t * 16 + r16] = acc[i][t][q];
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const int rr = p * RPP + lane / LPR;
      const int lrow = wv * (16 * G) + i * 16 + rr;
      float v8[8];
      *(f32x4*)&v8[0] = *(const f32x4*)&ew[rr * ES + c8];
      *(f32x4*)&v8[4] = *(const f32x4*)&ew[rr * ES + c8 + 4];
      if (res16) resv[i][p][0] = resL[lrow * LPR + lane % LPR];
      store_row8(e, (uint32_t)ordT[lrow] * CO + c8, row0 + lrow < N, v8, bias8, resv[i][p]);
    }
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
  }
}

// Halo kernel (Co = 64; Ci = 32*S, used at Ci = 64): a workgroup owns a window of B consecutive rows of the input (spatial)
// order, its rows gray-sorted inside the window (SpConvCache::halo_table: tight 16-row neighbour masks, 1.22x the
// active pairs on C4 against 1.81x unsorted). Before its K loop it copies, by DMA, every distinct neighbour row the
// tile reads (the tile's halo, ~1.4 rows per output row on shells instead of ~7 gathers) into LDS, plus the tile's
// (row, offset) -> halo index table; the K loop then reads its A operands from LDS with no barriers (each wavefront
// walks its own offsets) and its weights straight from L2 into registers, one offset ahead. Halo rows are stored
// with their 16-byte chunks XOR-swizzled by the halo index (hsw: conflict-light operand reads); index UM is a zero row
// that EMPTY neighbours point at. With a row map (gathered conv) the halo rows are read through it. Two
// workgroups per CU (LDS <= 80 KB each): one copies its halo while the other computes. Outputs and residuals are
// whole rows of the window, permuted inside it.
template <bool F16, int S, int B, int UM, int G, int T, int OCC>
__global__ void __launch_bounds__(256, OCC) k_conv_halo(ConvArgs a) {
  // wavefront (wr, wc) owns rows wr*16G .. +16G (G groups of 16) x output tiles wc*T .. +T (16 channels each)
  constexpr int CI = 32 * S, RU = CI / 8, CO = 64;  // RU: 16-byte units per feature row
  constexpr int WC = 4 / T;                         // wavefronts across the channels
  static_assert((B / (16 * G)) * WC == 4, "4 wavefronts cover B rows x 4 channel tiles");
  constexpr int IDXU = 27 * B * 2 / 16;        // 16-byte units of the index table
  constexpr int IDXP = (IDXU + 63) / 64 * 64;  // padded to whole wavefront DMA instructions (the tail reads zeros)
  __shared__ __attribute__((aligned(16))) u32x4 halo[(UM + 1) * RU];
  __shared__ __attribute__((aligned(16))) u32x4 idxL[IDXP];
  __shared__ uint32_t gmL[B / 16];
  static_assert((((UM + 1) * RU + IDXP) * 16 + B / 4) * OCC <= 163840, "OCC workgroups per CU");
  const int g = blockIdx.x, per = a.grid / 8;
  // tiles in runs of xblk consecutive windows per XCD (each XCD takes xblk of every 8 * xblk in order), so that the
  // eight XCDs work on nearby windows at any time; xblk = 0: each XCD walks one contiguous range
  const int tile = a.xblk > 0 ? xcd_run_tile(g, a.tiles_m, a.xblk) : (g % 8) * per + g / 8;
  if (tile < 0 || tile >= a.tiles_m) return;
  const int row0 = tile * B;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, r16 = lane & 15, q4 = lane >> 4;
  const int wr = wv / WC, wc = wv % WC;
  const int N = a.N;
  // halo row ids of this wavefront's DMA units, loaded together with the tile's row count instead of after it
  // (slots past the count hold -1, so no load depends on it): one memory round trip fewer before the DMA
  // (C4 prologue 9.7 -> 3.6 us per tile, kernel 0.77 -> 0.64 ms)
  constexpr int NINS = ((UM * RU + 63) / 64 + 3) / 4;  // DMA instructions per wavefront for a full halo
  const int32_t* hr = a.hrows + (size_t)tile * UM;
  int hrow[NINS];
#pragma unroll
  for (int k = 0; k < NINS; k++) {
    const int u = ((k * 4 + wv) * 64 + lane) / RU;
    hrow[k] = u < UM ? hr[u] : -1;
  }
  // 16-byte unit c of halo row u sits at position c ^ hsw(u) of the row. A 256-byte bank line holds 16 / RU rows,
  // so the swizzle takes the row bits above those: a unit's bank group is then a bijection of u mod 16, and the 16
  // lanes of an operand read (16 rows, one unit) spread over 16 bank groups instead of 8 (C4: LDS bank-conflict
  // cycles 7.3e7 -> 4.8e7 per launch)
  auto hsw = [](int u) __attribute__((always_inline)) { return RU < 16 ? (u / (16 / RU)) & (RU - 1) : u & (RU - 1); };
  const int U = __builtin_amdgcn_readfirstlane(a.hcount[tile]);
  if (U < 0) return;  // a spill tile (more distinct rows than UM): the gathering kernel computes its rows

  // prologue: index table and halo rows by DMA, the zero row and the group masks by plain stores
  {
    const __amdgpu_buffer_rsrc_t ri = make_rsrc(a.hidx + (size_t)tile * 27 * B, 27 * B * 2);
#pragma unroll
    for (int k = 0; k < (IDXP + 255) / 256; k++) {
      const int u = k * 256 + tid;
      if (k * 256 + wv * 64 < IDXP)  // wave-uniform: DMA destinations are per wavefront instruction
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ri, (__attribute__((address_space(3))) void*)&idxL[k * 256 + wv * 64],
                                                 16, (uint32_t)u * 16u, 0, 0, kStreamed);
    }
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
    const int nins = (U * RU + 63) / 64;  // wavefront instructions of 64 x 16 bytes (64 / RU halo rows each)
#pragma unroll
    for (int k = 0; k < NINS; k++) {
      const int j = k * 4 + wv;
      if (j >= nins) break;
      const int unit = j * 64 + lane, u = unit / RU, c = unit % RU;
      int h = hrow[k];
      if (a.rmap && h >= 0) {  // gathered conv: the halo row is row_map[h] >> shift of the source matrix
        const uint32_t q = (uint32_t)a.rmap[h] >> a.rshift;
        h = q < (uint32_t)a.rmax ? (int)q : -1;
      }
      const uint32_t off = h >= 0 ? (uint32_t)h * (CI * 2u) + (uint32_t)((c ^ hsw(u)) * 16) : kOutOfRange;
      // non-temporal: neighbouring tiles share only a fraction of their halo rows (C4: 0.608 -> 0.602 ms)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void*)&halo[j * 64], 16, off, 0,
                                               0, kStreamed);
    }
    if (tid < RU) halo[UM * RU + tid] = u32x4{0, 0, 0, 0};
    if (tid < B / 16) gmL[tid] = a.hgm[(size_t)tile * (B / 16) + tid];
  }
  wait_vmcnt<0>();
  if (a.ln_on) {
    // pre-activation of the halo rows in place: RU lanes per row, lane c holding the row's logical chunk c (stored
    // at c ^ hsw(u)), as gather_ln_act holds it, so the result is the same bits. Rows past the count are padding;
    // the zero row stays zero (an EMPTY neighbour), while a row whose source is out of range holds zeros and
    // becomes act(beta), as gather_ln_act makes it. Every lane takes part in the shuffles. Thread tid's unit
    // base + tid is the one its own lane DMA'd (instruction k * 4 + wv), and a row's units come from one DMA
    // instruction of the same wavefront, so this wavefront's wait above is enough: one barrier, after.
    for (int base = 0; base < U * RU; base += 256) {
      const int unit = base + tid, u = unit / RU, c = unit % RU;
      const bool live = u < U;
      u32x4* p = &halo[(live ? u : 0) * RU + (c ^ hsw(live ? u : 0))];
      const u32x4 q = live ? *p : u32x4{0, 0, 0, 0};
      float v[1][8];
#pragma unroll
      for (int j = 0; j < 8; j++) v[0][j] = lnact_h2f((uint16_t)(q[j >> 1] >> ((j & 1) * 16)), !F16);
      float mean, rstd;
      ln_stats<RU, 1>(v, CI, a.ln_eps, mean, rstd);
      float o[8];
      ln_out8(v[0], mean, rstd, a.ln_gamma ? a.ln_gamma + c * 8 : nullptr, a.ln_beta ? a.ln_beta + c * 8 : nullptr,
              a.ln_act == ACT_SILU, o);
      if (live)
        *p = u32x4{lnact_pack2(o[0], o[1], !F16), lnact_pack2(o[2], o[3], !F16), lnact_pack2(o[4], o[5], !F16),
                   lnact_pack2(o[6], o[7], !F16)};
    }
  }
  __syncthreads();

  // epilogue layout (16-byte row segments, LPR lanes per row) and the output rows, fetched now for later
  constexpr int ES = 16 * T + 4, LPR = 2 * T, RPP = 64 / LPR, NP = 16 / RPP;
  static_assert(NP >= 1, "a 16-row group spans whole epilogue passes");
  const int c8 = wc * 16 * T + (lane % LPR) * 8;
  int orow[G][NP];
#pragma unroll
  for (int i = 0; i < G; i++)
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const int pos = row0 + wr * 16 * G + i * 16 + p * RPP + lane / LPR;
      orow[i][p] = pos < N ? a.order[pos] : 0;
    }
  int ssrc[G][NP];  // skip residual: the output rows' c2s entries (row orow reads its parent slot)
  if (a.skip_src)
#pragma unroll
    for (int i = 0; i < G; i++)
#pragma unroll
      for (int p = 0; p < NP; p++) ssrc[i][p] = a.skip_src[orow[i][p]];
  uint32_t gms[G], wmask = 0;
#pragma unroll
  for (int i = 0; i < G; i++) {
    gms[i] = __builtin_amdgcn_readfirstlane(gmL[wr * G + i]);
    wmask |= gms[i];
  }
  f32x4v acc[G][T];
#pragma unroll
  for (int i = 0; i < G; i++)
#pragma unroll
    for (int t = 0; t < T; t++) acc[i][t] = f32x4v{0.f, 0.f, 0.f, 0.f};
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, a.w_bytes);
  const uint16_t* idx16 = (const uint16_t*)idxL;
  // The K loop walks stages (offset v, K chunk kc): KS 32-channel MFMA steps per stage, NKC chunks per offset (one
  // at Ci <= 64; two at Ci = 128, so a stage's operands stay within the register budget).
  constexpr int KS = S < 2 ? S : 2, NKC = S / KS;
  static_assert(NKC * KS == S, "K chunks");
  auto wload = [&](int v, int kc, u32x4 (&w)[T][KS]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int m = 0; m < KS; m++)
        w[t][m] = __builtin_amdgcn_raw_buffer_load_b128(
            rw, (uint32_t)(((v * 4 + wc * T + t) * S + kc * KS + m) * 64 + lane) * 16u, 0, 0);
  };
  // A operands of stage (v, kc) for every group (idle groups read the zero row: LDS reads are cheap, and reading
  // them unconditionally lets the reads of the next stage be issued before this stage's MFMAs). Lane quarter q4
  // takes channels (q4*S + m)*8 .. +8 in step m, the weight repack's order.
  auto aload = [&](int v, int kc, u32x4 (&av)[G][KS]) __attribute__((always_inline)) {
    int u[G];
#pragma unroll
    for (int i = 0; i < G; i++) u[i] = idx16[v * B + wr * 16 * G + i * 16 + r16];
#pragma unroll
    for (int i = 0; i < G; i++)
#pragma unroll
      for (int m = 0; m < KS; m++) av[i][m] = halo[u[i] * RU + ((q4 * S + kc * KS + m) ^ hsw(u[i]))];
  };
  auto compute = [&](int v, const u32x4 (&w)[T][KS], const u32x4 (&av)[G][KS]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < G; i++) {
      if ((gms[i] >> v) & 1u) {
#pragma unroll
        for (int m = 0; m < KS; m++)
#pragma unroll
          for (int t = 0; t < T; t++) acc[i][t] = mfma16<F16>(av[i][m], w[t][m], acc[i][t]);
      }
    }
  };
  // 16-bit residuals (or skip rows) of the first GE groups' output rows: requested together with the last stage's
  // weights (or after the loop when the wavefront has a single stage), so their round trip overlaps the last stages'
  // MFMAs instead of opening the epilogue; the other groups' residuals are requested at the epilogue's start, behind
  // the first group's stores. C4: 0.647 -> 0.630 ms (interleaved, one box; GE = 1, 2, 3 measured level, and all
  // four groups spill 14 registers). fp32 residuals (two registers per row segment) are loaded after the loop.
  const Epi e = make_epi(a);
  const bool res16 = a.skip_src || (e.res_dt >= 0 && e.res_dt != F32);
  constexpr int GE = 1;
  u32x4 rq[G][NP];
  bool res_issued = !res16;
  auto res_load = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < GE; i++)
#pragma unroll
      for (int p = 0; p < NP; p++) {
        const bool ok = row0 + wr * 16 * G + i * 16 + p * RPP + lane / LPR < N;
        const uint32_t o = (uint32_t)orow[i][p] * CO + c8;
        rq[i][p] = a.skip_src ? load_skip8(make_rsrc(a.skip_x, a.skip_bytes), a, ssrc[i][p], c8, ok)
                              : __builtin_amdgcn_raw_buffer_load_b128(e.res, ok ? o * 2u : kOutOfRange, 0, kStreamed);
      }
    res_issued = true;
  };
  // stages of this wavefront's offsets in ascending order; the weights (from L2) and A operands (from LDS) of the
  // next stage are requested while this one computes. The loads are unconditional -- the last stage reloads
  // itself -- so the compiler's wait counts stay exact.
  if (wmask) {
    uint32_t m = wmask;
    int v = __builtin_ctz(m), kc = 0;
    m &= m - 1;
    bool more = true;
    auto advance = [&](int& nv, int& nk) __attribute__((always_inline)) {
      if (kc + 1 < NKC) {
        nv = v;
        nk = kc + 1;
      } else if (m) {
        nv = __builtin_ctz(m);
        nk = 0;
        m &= m - 1;
      } else {
        nv = v;
        nk = kc;
        more = false;
      }
    };
    u32x4 wa[T][KS], wb[T][KS], aa[G][KS], ab[G][KS];
    wload(v, kc, wa);
    aload(v, kc, aa);
    for (;;) {
      int vn, kn;
      advance(vn, kn);
      wload(vn, kn, wb);
      aload(vn, kn, ab);
      if (!res_issued && more && !m && kn + 1 == NKC) res_load();
      compute(v, wa, aa);
      if (!more) break;
      v = vn;
      kc = kn;
      advance(vn, kn);
      wload(vn, kn, wa);
      aload(vn, kn, aa);
      if (!res_issued && more && !m && kn + 1 == NKC) res_load();
      compute(v, wb, ab);
      if (!more) break;
      v = vn;
      kc = kn;
    }
  }
  if (!res_issued) res_load();

  // epilogue: per 16-row group through a per-wavefront [16][16T+4] fp32 area in the (now idle) halo buffer; the
  // output rows (orow) were read before the K loop, the first group's residuals during it; the others' are requested now
  __syncthreads();  // every wavefront is done reading the halo
  float* ew = (float*)halo + wv * 16 * ES;
  float bias8[8];
#pragma unroll
  for (int q = 0; q < 8; q++) bias8[q] = a.bias ? a.bias[c8 + q] : 0.f;
  u32x4 resv[G][NP][2];
#pragma unroll
  for (int i = 0; i < G; i++)
#pragma unroll
    for (int p = 0; p < NP; p++) {
      if (res16 && i < GE) {
        resv[i][p][0] = rq[i][p];
        resv[i][p][1] = u32x4{0, 0, 0, 0};
      } else if (a.skip_src) {
        const bool ok = row0 + wr * 16 * G + i * 16 + p * RPP + lane / LPR < N;
        resv[i][p][0] = load_skip8(make_rsrc(a.skip_x, a.skip_bytes), a, ssrc[i][p], c8, ok);
        resv[i][p][1] = u32x4{0, 0, 0, 0};
      } else {
        const bool ok = row0 + wr * 16 * G + i * 16 + p * RPP + lane / LPR < N;
        load_res8(e, (uint32_t)orow[i][p] * CO + c8, ok, resv[i][p]);
      }
    }
#pragma unroll
  for (int i = 0; i < G; i++) {
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int q = 0; q < 4; q++) ew[(q4 * 4 + q) * ES + t * 16 + r16] = acc[i][t][q];
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const int rr = p * RPP + lane / LPR;
      const int pos = row0 + wr * 16 * G + i * 16 + rr;
      const int lc = (lane % LPR) * 8;  // column within this wavefront's channels
      float v8[8];
      *(f32x4*)&v8[0] = *(const f32x4*)&ew[rr * ES + lc];
      *(f32x4*)&v8[4] = *(const f32x4*)&ew[rr * ES + lc + 4];
      store_row8(e, (uint32_t)orow[i][p] * CO + c8, pos < N, v8, bias8, resv[i][p]);
    }
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
  }
}

// Halo shapes per input width (rows per tile, halo rows at most, groups and channel tiles per wavefront). Ci = 64
// by default; Ci = 128 on request (SPCONV_HALO128, see halo128_enabled for why it is not the default).
template <int S>
struct HaloShape;
template <>
struct HaloShape<2> {  // Ci = 64: 256-row windows, up to 512 halo rows (80 KB of LDS, two workgroups per CU)
  static constexpr int B = 256, UM = 512, G = 4, T = 4, OCC = 2;
};
template <>
struct HaloShape<4> {  // Ci = 128: 128-row windows, up to 256 halo rows of 256 bytes (73 KB, two workgroups per CU);
                       // wavefronts of 64 rows x 32 channels
  static constexpr int B = 128, UM = 256, G = 4, T = 2, OCC = 2;
};

template <bool F16, int S>
void launch_halo(ConvArgs a) {
  using H = HaloShape<S>;
  a.tiles_m = cdiv(a.N, H::B);
  a.tiles_n = 1;
  a.grid = (a.tiles_m + 7) / 8 * 8;
  // Runs of 16 windows per XCD instead of one contiguous range per XCD: C4 0.625 -> 0.616 ms (same bits; runs of
  // 4 / 8 / 32 / 64 measured 0.622 / 0.616 / 0.617 / 0.619, one window per XCD in turn 0.625; interleaved on two
  // boxes). The gathering kernel keeps its contiguous ranges: runs made C5's children slower (0.825 -> 0.835-0.854).
  a.xblk = 16;
  k_conv_halo<F16, S, H::B, H::UM, H::G, H::T, H::OCC><<<a.grid, 256, 0, stream()>>>(a);
}

template <bool F16, int S, int T>
void launch_narrow(ConvArgs a, hipStream_t st = stream()) {
  constexpr int G = S <= 2 ? 4 : 2;  // 16-row groups per wavefront: keeps two wavefronts per SIMD at Ci = 128
  a.tiles_m = cdiv(a.N, 4 * 16 * G);
  a.tiles_n = 1;
  a.grid = (a.tiles_m + 7) / 8 * 8;
  // Ci = 128: the three-workgroups-per-CU form (see k_conv_narrow)
  if constexpr (S == 4) k_conv_narrow<F16, S, T, G, true><<<a.grid, 256, 0, st>>>(a);
  else k_conv_narrow<F16, S, T, G><<<a.grid, 256, 0, st>>>(a);
}

// Wide-channel kernel, BM sorted rows x 256 channels per workgroup (4 wavefronts, each all BM rows x 64 channels =
// BM/32 x 2 tiles of 32x32 fp32 accumulators). BM = 128 is the one launched: two workgroups per CU, so one
// workgroup's prologue, barriers and epilogue overlap the other's MFMAs. Differences from k_conv_wide:
//  * The gathered A tile goes global -> LDS directly (buffer_load ... lds, 16 bytes per lane; EMPTY neighbours
//    read past the buffer end and land as zeros) into a 4-slot LDS ring, 3 stages ahead of the MFMAs: no
//    registers hold gathers in flight, and gather latency hides behind three stages of MFMA work. The slots are
//    four distinct LDS objects so the compiler can tell the DMA into one slot from the reads of another.
//  * Ring protocol per stage s: wait (counted vmcnt) for this lane's DMA of A(s), barrier (every wavefront's
//    part has landed and everyone is done with stage s-1), then refill the slot stage s-1 used with A(s+3).
//  * K-step-outer MFMA order: for each 16-wide K step j of the stage, the MFMAs of every 32-row group, then the
//    weights of stage s+1 for step j go into the registers step j just released. One weight register set (not two),
//    a stage of latency slack for every weight load, and BM/32 x 2 independent accumulator chains in flight.
template <bool F16, int BM>
__global__ void __launch_bounds__(256, BM == 128 ? 2 : 1) k_conv_wide_dma(ConvArgs a) {
  constexpr int NW = 4, NT = 256, KC = 64, PC = KC / 8;
  constexpr int TM = BM / 32, TN = 2, AL = BM * PC / NT;  // TM groups of 32 rows per wavefront
  static_assert(AL == TM, "one A DMA per 32-row group");
  static_assert(BM == 128 || BM == 256, "tile rows");
  __shared__ __attribute__((aligned(16))) u32x4 As0[BM * PC], As1[BM * PC], As2[BM * PC], As3[BM * PC];
  __shared__ uint32_t srcT[BM * 27];
  __shared__ int ordT[BM];
  __shared__ uint32_t gmask[BM / 32];
  __shared__ int vlist[32];

  const int g = blockIdx.x, per = a.grid / 8;
  int logical, split = 0, nsplit = 1, pslot = -1;
  if (a.part) {  // tail-split schedule: XCD x = g % 8 walks its own tiles, whole ones first, then the split pieces
    const int x = g % 8, u = g / 8, c = a.xt0[x + 1] - a.xt0[x], kx = a.xk[x];
    const int nfull = kx > 1 ? a.xs : c;
    if (u < nfull) {
      logical = a.xt0[x] + u;
    } else {
      const int q = u - nfull;
      if (nfull + q / kx >= c) return;
      logical = a.xt0[x] + nfull + q / kx;
      split = q % kx;
      nsplit = kx;
      pslot = a.xpart0[x] + q;
    }
  } else if (a.tsched) {
    // workgroups start in id order, dealt round-robin to the XCDs: row tiles longest first
    // (SpConvCache::tile_schedule), so every XCD gets an even share of long and short tiles and the launch ends on
    // short ones (the XCD-contiguous walk below leaves each XCD its densest tiles for last)
    // (in runs of xblk consecutive tiles per XCD: each XCD takes xblk of every 8 * xblk in order)
    logical = a.xblk > 0 ? xcd_run_tile(g, a.tiles_m * a.tiles_n, a.xblk) : g;
    if (logical < 0) return;
  } else {
    logical = (g % 8) * per + g / 8;
  }
  if (logical >= a.tiles_m * a.tiles_n) return;
  const bool tmaj = a.tnmaj;  // set only with the tail-split schedule (no tsched)
  const int tm_ = a.tsched && !a.part ? a.tsched[logical / a.tiles_n] : tmaj ? logical % a.tiles_m : logical / a.tiles_n;
  const int tn_ = tmaj ? logical / a.tiles_m : logical % a.tiles_n;
  const int row0 = tm_ * BM, co0 = tn_ * (64 * NW);
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), wn = wv;
  const int N = a.N, Ci = a.Ci, nkc = Ci / KC;

  // prologue: the tile's block of the neighbour table goes to LDS by DMA; rows and 32-row masks from the same order
  dma_tile_table<BM, NT>(a, row0, srcT, tid);
  if (tid < BM) {
    const int row = row0 + tid;
    ordT[tid] = row < N ? a.order[row] : 0;
    uint32_t gm = a.gs[row];  // padded rows have mask 0
#pragma unroll
    for (int d = 1; d < 32; d <<= 1) gm |= (uint32_t)__shfl_xor((int)gm, d, 64);
    if ((tid & 31) == 0) gmask[tid >> 5] = gm;
  }
  wait_vmcnt<0>();  // this lane's table DMA has landed (the barrier below covers the other lanes)
  __syncthreads();
  uint32_t mask = 0;
#pragma unroll
  for (int i = 0; i < BM / 32; i++) mask |= gmask[i];
  const int nvv = __popc(mask), all_stages = nvv * nkc;
  // K stages [s0, s0 + total) of this workgroup: all of them, or its share of a split tile
  const int s0 = (int)((long long)all_stages * split / nsplit);
  const int total = (int)((long long)all_stages * (split + 1) / nsplit) - s0;
  if (tid < 27 && ((mask >> tid) & 1u)) vlist[__popc(mask & ((1u << tid) - 1u))] = tid;
  uint32_t gms[TM];
#pragma unroll
  for (int i = 0; i < TM; i++) gms[i] = __builtin_amdgcn_readfirstlane(gmask[i]);
  __syncthreads();

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes), rw = make_rsrc(a.w, a.w_bytes);
  // DMA k of this lane fills LDS unit u = (wv*AL + k)*64 + lane: row u/8, slot u%8, channel piece
  // slot ^ ((row >> 1) & 7)
  uint32_t drow[AL], dpiece[AL];
#pragma unroll
  for (int k = 0; k < AL; k++) {
    const int u = (wv * AL + k) * 64 + lane;
    drow[k] = u >> 3;
    dpiece[k] = (u & 7) ^ ((u >> 4) & 7);
  }
  const uint32_t wslice = (uint32_t)((co0 >> 6) + wn) * 27u * (uint32_t)nkc;
  const uint32_t wlane = (uint32_t)lane * 16u;

  // K stages run channel block outer, offset inner: stage s = (kc = s / nvv, offset entry vi = s % nvv). A row chunk
  // gathered for one offset is then gathered again for the next offset's (one voxel over) neighbours one stage
  // later instead of nkc stages later, while it is still in L2: C3 0.837 -> 0.826 ms, C2 0.297 -> 0.293 (two
  // interleaved runs; each output's fp32 sum runs over (kc, v) in that order).
  int avi = s0 % nvv, akc = s0 / nvv, bvi = avi, bkc = akc, cvi = avi, ckc = akc;
  auto next = [&](int& vi, int& kc) __attribute__((always_inline)) {
    const bool wrap = vi + 1 == nvv;
    vi = wrap ? 0 : vi + 1;
    kc += wrap ? 1 : 0;
  };
  // DMA addresses of the next A stage (offset entry avi, channel block akc; clamped to the last stage)
  auto a_offsets = [&](uint32_t (&off)[AL], int& ka) __attribute__((always_inline)) {
    const bool live = avi < nvv && akc < nkc;
    const int va = __builtin_amdgcn_readfirstlane(vlist[live ? avi : nvv - 1]);
    ka = __builtin_amdgcn_readfirstlane((live ? akc : nkc - 1) * KC * 2);
    next(avi, akc);
#pragma unroll
    for (int k = 0; k < AL; k++) off[k] = nbr_offset(srcT[drow[k] * 27 + va], (uint32_t)(Ci * 2)) + dpiece[k] * 16;
  };
  auto dma = [&](u32x4* slot, int k, uint32_t off, int ka) __attribute__((always_inline)) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void*)&slot[(wv * AL + k) * 64],
                                             16, off, ka, 0, 0);
  };
  auto b_base = [&]() __attribute__((always_inline)) {
    const bool live = bvi < nvv && bkc < nkc;
    const int vb = __builtin_amdgcn_readfirstlane(vlist[live ? bvi : nvv - 1]);
    const int kb = live ? bkc : nkc - 1;
    next(bvi, bkc);
    return __builtin_amdgcn_readfirstlane((int)((wslice + (uint32_t)(vb * nkc + kb)) * 8192u));
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int t = 0; t < TN; t++) acc[i][t] = f32x16{};

  // one K stage: MFMAs from slot `cur` and the weights in rb (stage s); DMA A(s+3) into `fill`; rb refilled with
  // the weights of stage s+1, K step by K step
  auto stage = [&](const u32x4* cur, u32x4* fill, u32x4 (&rb)[TN][4]) __attribute__((always_inline)) {
    const uint32_t vbit = 1u << __builtin_amdgcn_readfirstlane(vlist[cvi]);
    next(cvi, ckc);
    uint32_t off[AL];
    int ka;
    a_offsets(off, ka);
    const int soff = b_base();
    u32x4 fa[2][TM];
    auto read_j = [&](u32x4 (&f)[TM], int j) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int r = i * 32 + l32;
        f[i] = cur[r * PC + ((h * 4 + j) ^ ((r >> 1) & 7))];
      }
    };
    read_j(fa[0], 0);
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int k = (j * AL) / 4; k < ((j + 1) * AL) / 4; k++) dma(fill, k, off[k], ka);
      if (j + 1 < 4) read_j(fa[(j + 1) & 1], j + 1);
      // raised wave priority over the MFMA burst: the sequencer keeps feeding this wave's matrix ops ahead of the
      // other workgroup's memory instructions (C3 0.922 -> 0.915 ms, C2 0.755 -> 0.751, same box; priority 1 over
      // the whole K loop instead was no better, C2 0.763; the halo kernel showed no change and does not do it)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < TM; i++)
        if (gms[i] & vbit) {
#pragma unroll
          for (int t = 0; t < TN; t++) acc[i][t] = mfma32<F16>(fa[j & 1][i], rb[t][j], acc[i][t]);
        }
      __builtin_amdgcn_s_setprio(0);
#pragma unroll
      for (int t = 0; t < TN; t++)
        rb[t][j] = __builtin_amdgcn_raw_buffer_load_b128(rw, wlane + (t * 4 + j) * 1024, soff, 0);
    }
  };
  // loads issued after this lane's last DMA of A(s) when stage s starts: prologue DMAs and B(0) for s < 3,
  // then (in steady state) the last K step's TN weight loads of stage s-3 plus two full stages of AL + 8
  constexpr int SL = AL + 8;
  auto wait_a = [&](int s) __attribute__((always_inline)) {
    if (s == 0) wait_vmcnt<2 * AL + 8>();
    else if (s == 1) wait_vmcnt<AL + 8 + SL>();
    else if (s == 2) wait_vmcnt<8 + 2 * SL>();
    else wait_vmcnt<TN + 2 * SL>();
  };

  if (total > 0) {
    u32x4 rb[TN][4];
    {
      uint32_t off[AL];
      int ka;
      a_offsets(off, ka);
#pragma unroll
      for (int k = 0; k < AL; k++) dma(As0, k, off[k], ka);
      a_offsets(off, ka);
#pragma unroll
      for (int k = 0; k < AL; k++) dma(As1, k, off[k], ka);
      a_offsets(off, ka);
#pragma unroll
      for (int k = 0; k < AL; k++) dma(As2, k, off[k], ka);
      const int soff = b_base();
#pragma unroll
      for (int q = 0; q < 8; q++) rb[q / 4][q % 4] = __builtin_amdgcn_raw_buffer_load_b128(rw, wlane + q * 1024, soff, 0);
    }
    for (int s = 0; s < total; s += 4) {
      wait_a(s);
      wg_barrier();
      stage(As0, As3, rb);
      if (s + 1 >= total) break;
      wait_a(s + 1);
      wg_barrier();
      stage(As1, As0, rb);
      if (s + 2 >= total) break;
      wait_a(s + 2);
      wg_barrier();
      stage(As2, As1, rb);
      if (s + 3 >= total) break;
      wait_a(s + 3);
      wg_barrier();
      stage(As3, As2, rb);
    }
  }
  wait_vmcnt<0>();
  if (pslot >= 0) {  // a piece of a split tile: its fp32 partial sums go to the workspace, the reduction does the rest
    float* pp = a.part + (size_t)pslot * (BM * 256);
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int t = 0; t < TN; t++)
#pragma unroll
        for (int q = 0; q < 16; q++)
          pp[(i * 32 + (q >> 2) * 8 + h * 4 + (q & 3)) * 256 + wn * 64 + t * 32 + l32] = acc[i][t][q];
    return;
  }
  __syncthreads();

  // epilogue through the (now idle) ring: one slot per wavefront
  float* ew = (float*)(wv == 0 ? &As0[0] : wv == 1 ? &As1[0] : wv == 2 ? &As2[0] : &As3[0]);
  static_assert(32 * 72 * 4 <= BM * PC * 16, "a wavefront's epilogue staging fits in a ring slot");
  const int co_w = co0 + wn * 64;
  float bias8[8];
#pragma unroll
  for (int q = 0; q < 8; q++) bias8[q] = a.bias ? a.bias[co_w + (lane & 7) * 8 + q] : 0.f;
  const int nrows = N - row0;
  const Epi e = make_epi(a);
  epilogue_tile<TM, TN>(acc, ew, ordT, nrows, co_w, bias8, e, a.Co, lane);
}

// 256 x 256 tile kernel with both operands in LDS (Co a multiple of 256, Ci a multiple of 32; opt-in with SPCONV_W8,
// an evaluated alternative to k_conv_wide_dma): one workgroup per CU of 8 wavefronts (two per SIMD), wavefront
// (wr, wc) owning rows wr*128 .. +128 x channels wc*64 .. +64 as 4 x 2 tiles of v_mfma_f32_32x32x16. A K stage is one
// offset x 32 input channels: the 256 gathered rows (64 bytes each) and the 256 weight columns (64 bytes each) both go
// global -> LDS by DMA into 3-slot rings (16 KB per slot and operand), two stages ahead, so each weight byte is
// fetched once per 256 rows instead of once per 128. Slot layout: row (column) q's 16-byte piece p sits in unit
// q*4 + (p ^ ((q >> 1) & 3)) (conflict-free fragment reads); the weight repack (k_pack_w8) stores the pieces in that
// order so the weight DMA is one contiguous 16 KB block per stage. Every wavefront waits for its own DMAs (counted
// vmcnt), then one barrier per stage publishes the slot and frees the one stage s+2 refills. Per-32-row-group skips
// as in k_conv_wide_dma. The rings are six distinct LDS objects (slots named per unrolled stage) so that the
// compiler can tell the DMA into one slot from the reads of another.
template <bool F16>
__global__ void __launch_bounds__(512, 1) k_conv_w8(ConvArgs a) {
  constexpr int BM = 256, NT = 512, KC = 32, PU = KC / 8, SU = BM * PU;  // SU: 16-byte units per slot
  constexpr int TM = 4, TN = 2;
  __shared__ __attribute__((aligned(16))) u32x4 A0[SU], A1[SU], A2[SU], B0[SU], B1[SU], B2[SU];
  __shared__ __attribute__((aligned(16))) uint32_t srcT[BM * 27];
  __shared__ int ordT[BM];
  __shared__ uint32_t gmask[BM / 32];
  __shared__ int vlist[32];

  const int tile = blockIdx.x;
  if (tile >= a.tiles_m * a.tiles_n) return;
  const int tm_ = a.tsched[tile / a.tiles_n], tn_ = tile % a.tiles_n;  // row tiles longest first
  const int row0 = tm_ * BM, co0 = tn_ * 256;
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), wr = wv >> 2, wc = wv & 3;
  const int N = a.N, Ci = a.Ci, nkc = Ci / KC;

  dma_tile_table<BM, NT>(a, row0, srcT, tid);
  if (tid < BM) {
    const int row = row0 + tid;
    ordT[tid] = row < N ? a.order[row] : 0;
    uint32_t gm = a.gs[row];  // padded rows have mask 0
#pragma unroll
    for (int d = 1; d < 32; d <<= 1) gm |= (uint32_t)__shfl_xor((int)gm, d, 64);
    if ((tid & 31) == 0) gmask[tid >> 5] = gm;
  }
  wait_vmcnt<0>();
  __syncthreads();
  uint32_t mask = 0;
#pragma unroll
  for (int i = 0; i < BM / 32; i++) mask |= gmask[i];
  const int nvv = __popc(mask), total = nvv * nkc;
  if (tid < 27 && ((mask >> tid) & 1u)) vlist[__popc(mask & ((1u << tid) - 1u))] = tid;
  uint32_t gms[TM];
#pragma unroll
  for (int i = 0; i < TM; i++) gms[i] = __builtin_amdgcn_readfirstlane(gmask[wr * TM + i]);
  __syncthreads();

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes), rw = make_rsrc(a.w, a.w_bytes);
  // this thread's DMA units (two A, two B per stage): unit u = k*NT + tid -> row/column u >> 2, slot u & 3, source
  // piece slot ^ ((row >> 1) & 3)
  uint32_t arow[2], apiece[2];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int u = k * NT + tid;
    arow[k] = (uint32_t)(u >> 2);
    apiece[k] = (uint32_t)((u & 3) ^ ((u >> 3) & 3));
  }
  auto issue = [&](int st, u32x4* As, u32x4* Bs) __attribute__((always_inline)) {
    const int vi = st / nkc, kc = st % nkc;
    const int v = __builtin_amdgcn_readfirstlane(vlist[vi]);
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const uint32_t off = nbr_offset(srcT[arow[k] * 27 + v], (uint32_t)(Ci * 2)) + apiece[k] * 16u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void*)&As[k * NT + wv * 64], 16,
                                               off, (uint32_t)(kc * KC * 2), 0, 0);
    }
    const uint32_t wbase = (uint32_t)(((tn_ * 27 + v) * nkc + kc) * SU) * 16u;
#pragma unroll
    for (int k = 0; k < 2; k++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (__attribute__((address_space(3))) void*)&Bs[k * NT + wv * 64], 16,
                                               (uint32_t)(k * NT + tid) * 16u, wbase, 0, 0);
  };
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int t = 0; t < TN; t++) acc[i][t] = f32x16{};
  auto compute = [&](int st, const u32x4* As, const u32x4* Bs) __attribute__((always_inline)) {
    const uint32_t vbit = 1u << __builtin_amdgcn_readfirstlane(vlist[st / nkc]);
#pragma unroll
    for (int j = 0; j < KC / 16; j++) {
      const int p = 2 * j + h;
      u32x4 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int r = wr * 128 + i * 32 + l32;
        fa[i] = As[r * PU + (p ^ ((r >> 1) & 3))];
      }
#pragma unroll
      for (int t = 0; t < TN; t++) {
        const int c = wc * 64 + t * 32 + l32;
        fb[t] = Bs[c * PU + (p ^ ((c >> 1) & 3))];
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
        if (gms[i] & vbit) {
#pragma unroll
          for (int t = 0; t < TN; t++) acc[i][t] = mfma32<F16>(fa[i], fb[t], acc[i][t]);
        }
    }
  };
  // stage s: wait for this thread's DMAs of stage s (the 4 of stage s+1 may stay in flight), barrier, refill the
  // slot stage s-1 used with stage s+2, compute stage s
  auto step = [&](int st, const u32x4* As, const u32x4* Bs, u32x4* Af, u32x4* Bf) __attribute__((always_inline)) {
    if (st + 1 < total) wait_vmcnt<4>();
    else wait_vmcnt<0>();
    wg_barrier();
    if (st + 2 < total) issue(st + 2, Af, Bf);
    compute(st, As, Bs);
  };
  if (total > 0) {
    issue(0, A0, B0);
    if (total > 1) issue(1, A1, B1);
    for (int st = 0; st < total; st += 3) {
      step(st, A0, B0, A2, B2);
      if (st + 1 >= total) break;
      step(st + 1, A1, B1, A0, B0);
      if (st + 2 >= total) break;
      step(st + 2, A2, B2, A1, B1);
    }
  }
  wait_vmcnt<0>();
  __syncthreads();
  // epilogue: a [32][72] fp32 staging area per wavefront in the idle rings (and the neighbour table for the last two)
  static_assert(32 * 72 * 4 <= SU * 16 && 2 * 32 * 72 * 4 <= BM * 27 * 4, "epilogue staging fits");
  float* ew = wv == 0 ? (float*)A0 : wv == 1 ? (float*)A1 : wv == 2 ? (float*)A2 : wv == 3 ? (float*)B0
            : wv == 4 ? (float*)B1 : wv == 5 ? (float*)B2 : (float*)srcT + (wv - 6) * 32 * 72;
  const int co_w = co0 + wc * 64;
  float bias8[8];
#pragma unroll
  for (int q = 0; q < 8; q++) bias8[q] = a.bias ? a.bias[co_w + (lane & 7) * 8 + q] : 0.f;
  const Epi e = make_epi(a);
  epilogue_tile<TM, TN>(acc, ew, ordT + wr * 128, N - row0 - wr * 128, co_w, bias8, e, a.Co, lane);
}

// Weight repack for k_conv_w8: per (column tile of 256, offset, 32-channel chunk) one contiguous block of 1024
// 16-byte units, unit u = column c (u >> 2) x slot (u & 3) holding channels ((u & 3) ^ ((c >> 1) & 3)) * 8 .. +8.
__global__ void __launch_bounds__(256) k_pack_w8(const u32x4* __restrict__ w, u32x4* __restrict__ wp, int Ci) {
  const int nkc = Ci / 32, kc = blockIdx.x, v = blockIdx.y, tn = blockIdx.z;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int u = k * 256 + threadIdx.x, c = u >> 2, piece = (u & 3) ^ ((c >> 1) & 3);
    const int co = tn * 256 + c;
    wp[(((i64)tn * 27 + v) * nkc + kc) * 1024 + u] = w[((i64)co * 27 + v) * (Ci / 8) + kc * 4 + piece];
  }
}

// 256 x 256 tile kernel (Co a multiple of 256, Ci a multiple of 64): one workgroup per CU, 4 wavefronts, each
// owning all 256 rows x its own 64 output channels (8 x 2 tiles of v_mfma_f32_32x32x16, 256 accumulator registers).
//  * Bytes per flop: a K stage (one offset x 64 input channels) reads 256 gathered rows and 256 weight columns of
//    128 bytes for 2*256*256*64 flops -- half the weight bytes per flop of a 128-row tile.
//  * Gathered rows go global -> LDS by DMA (buffer_load ... lds, 16 bytes per lane, 8 lanes per 128-byte row:
//    whole cache lines; a 64-byte piece per row costs the address path as much as a whole line) into a 4-slot
//    ring filled 3 stages ahead. Weights (distinct per wavefront) stream from L2 into operand registers one stage
//    ahead, K-step-outer: step j's registers are refilled right after step j's MFMAs.
//  * With one wavefront per SIMD every stall idles the matrix core, so the loop is software-pipelined across
//    stage boundaries: the barrier that publishes stage s+1's slot sits before stage s's last K step, whose MFMAs
//    then cover the latency of stage s+1's first fragment reads.
//  * The loop's memory operations (fragment and index reads, DMAs, weight loads) are inline assembly with explicit
//    counted waits: the compiler cannot tell the DMA into one ring slot from reads of another, and without that
//    it waits for every DMA in flight before each read. Every load's output is early-clobber: a destination that
//    shared a register with an address operand could be written by an earlier load's return before a later
//    instruction of the same statement (stalled at issue) has read its address.
//  * Slot layout: slot row q holds tile row q; its 16-byte piece p sits in unit p ^ ((q >> 1) & 7), so the fragment
//    reads (32 rows, one piece) are conflict-free. A lane's 8 DMAs fill rows wv*64 + k*8 + (lane >> 3), k = 0..7;
//    the offset-major index table stores row r at position pi(r) (pi transposes the 8 x 8 (k, m) blocks of each
//    64-row block), so those 8 rows' neighbour indices are two 16-byte LDS reads.
//  * No per-group MFMA skipping: the tile runs the union of its rows' offsets (EMPTY neighbours read past the
//    buffer end and land as zeros); scalar branches between the MFMAs cost about what the skipped work saves.
//  * Small row counts: a tile's K stages can be split over `ns` workgroups writing fp32 partial tiles, summed in
//    piece order by k_split_reduce256 (which applies the epilogue), so a grid of few tiles still fills the CUs.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int w256_pi(int q) { return (q & ~63) | ((q & 7) << 3) | ((q >> 3) & 7); }
template <int N>
__device__ __forceinline__ void asm_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void asm_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}
// Waits that also rewrite the registers the awaited loads fill ("+v"), in one volatile statement: the uses of those
// registers cannot be scheduled above the wait.
template <int N>
__device__ __forceinline__ void lgkm_tie8(u32x4 (&A)[8]) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(A[0]), "+v"(A[1]), "+v"(A[2]), "+v"(A[3]), "+v"(A[4]), "+v"(A[5]), "+v"(A[6]), "+v"(A[7])
               : "n"(N) : "memory");
}
// (lgkmcnt counts at most 15 outstanding operations: the loop never has more than 10 in flight.)
template <int N>
__device__ __forceinline__ void lgkm_tie10(u32x4 (&A)[8], u32x4 (&B)[2]) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%10)"
               : "+v"(A[0]), "+v"(A[1]), "+v"(A[2]), "+v"(A[3]), "+v"(A[4]), "+v"(A[5]), "+v"(A[6]), "+v"(A[7]),
                 "+v"(B[0]), "+v"(B[1])
               : "n"(N) : "memory");
}
// MFMA as volatile inline assembly: keeps its place among the loop's other (inline-assembly) instructions, so the
// fragment reads, DMAs and weight loads can be interleaved between the matrix instructions as written.
template <bool F16>
__device__ __forceinline__ void mfma_asm(f32x16& c, const u32x4& a, const u32x4& b) {
  if constexpr (F16) asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
template <int N>
__device__ __forceinline__ void vm_tie2(u32x4& a, u32x4& b) {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N) : "memory");
}

template <bool F16>
__global__ void __launch_bounds__(256, 1) k_conv_w256(ConvArgs a) {
  constexpr int BM = 256, KC = 64, SU = BM * 8;  // rows per tile, channels per stage, 16-byte units per slot
  __shared__ __attribute__((aligned(16))) u32x4 ring[4][SU];
  __shared__ __attribute__((aligned(16))) uint32_t srcT[27 * BM];  // offset-major: srcT[v*256 + pi(tile row)]
  __shared__ int ordP[BM];                                          // output row of tile row r (-1: none)
  __shared__ uint32_t gmask[BM / 64];

  // Workgroups start in id order, dealt round-robin to the XCDs; the row tiles are taken longest first
  // (SpConvCache::tile_schedule), each row tile's column tiles and K pieces adjacent, so every XCD gets an even
  // share of long and short tiles and the launch ends on short ones.
  const int unit = blockIdx.x;
  const int ns = a.xs > 0 ? a.xs : 1;  // K pieces per tile
  const int tile = unit / ns, piece = unit % ns;
  if (tile >= a.tiles_m * a.tiles_n) return;
  const int tm_ = a.tsched[tile / a.tiles_n], tn_ = tile % a.tiles_n;
  const int row0 = tm_ * BM;
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = a.N, Ci = a.Ci, nkc = Ci / KC;

  // prologue: this thread's tile row -> its 27 neighbour indices (offset-major), its output row at its slot row,
  // and the tile's union mask
  {
    const __amdgpu_buffer_rsrc_t rt = make_rsrc(a.tbl, a.tbl_bytes);
    const uint32_t base = (uint32_t)(row0 + tid) * 108u;  // the table is padded to a multiple of 256 rows
    uint32_t nb[27];
#pragma unroll
    for (int v = 0; v < 27; v++) nb[v] = __builtin_amdgcn_raw_buffer_load_b32(rt, base + v * 4, 0, 0);
    const int pr = w256_pi(tid);  // index-table position of tile row tid
#pragma unroll
    for (int v = 0; v < 27; v++) srcT[v * BM + pr] = nb[v];
    ordP[tid] = row0 + tid < N ? a.order[row0 + tid] : -1;
    uint32_t gm = a.gs[row0 + tid];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) gm |= (uint32_t)__shfl_xor((int)gm, d, 64);
    if (lane == 0) gmask[wv] = gm;
  }
  __syncthreads();
  const uint32_t mask = gmask[0] | gmask[1] | gmask[2] | gmask[3];
  const int all_stages = __popc(mask) * nkc;
  const int s0 = (int)((long long)all_stages * piece / ns);
  const int total = (int)((long long)all_stages * (piece + 1) / ns) - s0;

  f32x16 acc[8][2];
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int t = 0; t < 2; t++) acc[i][t] = f32x16{};

  if (total > 0) {
    // buffer descriptors as plain SGPR quads for the inline assembly (same fields as make_rsrc)
    auto rsrc4 = [](const void* p, uint32_t bytes) {
      const uint64_t b = (uint64_t)(uintptr_t)p;
      return i32x4{(int32_t)(uint32_t)b, (int32_t)(uint32_t)(b >> 32), (int32_t)bytes, 0x00020000};
    };
    const i32x4 rx = rsrc4(a.x, a.x_bytes), rw = rsrc4(a.w, a.w_bytes);
    const uint32_t rowbytes = (uint32_t)Ci * 2u;
    const uint32_t ring0 = (uint32_t)(size_t)(__attribute__((address_space(3))) u32x4*)&ring[0][0];
    const uint32_t srct0 = (uint32_t)(size_t)(__attribute__((address_space(3))) uint32_t*)&srcT[0];
    // DMA k of this lane: tile row wv*64 + (lane>>3)*8 + k into slot row q = (wv*8 + k)*8 + (lane>>3), piece
    // (lane & 7) ^ ((q >> 1) & 7)
    const uint32_t trow = (uint32_t)(wv * 64 + (lane >> 3) * 8);  // first of this lane's 8 tile rows
    uint32_t apiece[2];                                            // piece byte offset for even / odd k
#pragma unroll
    for (int k = 0; k < 2; k++) apiece[k] = (uint32_t)(((lane & 7) ^ ((k * 4 + (lane >> 4)) & 7)) * 16);
    const uint32_t dma_lds = ring0 + (uint32_t)(wv * 8 * 64) * 16u;  // + slot * 32 KB + k * 1 KB
    // A fragment (group i, K step j): slot row i*32 + l32, piece j*2 + h
    uint32_t alane[4];
#pragma unroll
    for (int j = 0; j < 4; j++) alane[j] = (uint32_t)(l32 * 128 + (((j * 2 + h) ^ ((l32 >> 1) & 7)) * 16));
    // weights: 4 KB block per (32-column block, offset, 64-channel chunk); this wavefront's two blocks
    const uint32_t wblk0 = (uint32_t)(tn_ * 8 + wv * 2) * 27u * (uint32_t)nkc;
    const uint32_t wblk_t = 27u * (uint32_t)nkc * 4096u;
    const uint32_t wlane = (uint32_t)lane * 16u;

    uint32_t skip_m = mask;
    for (int q = 0; q < s0 / nkc; q++) skip_m &= skip_m - 1u;
    const int vlast = 31 - __builtin_clz(mask | 1u);
    uint32_t dm = skip_m, bm = skip_m;  // offsets still to DMA (A) / to load (B)
    int dkc = s0 % nkc, bkc = s0 % nkc;
    auto advance = [&](uint32_t& m, int& kc, int& v, int& kcs) __attribute__((always_inline)) {
      const bool live = m != 0;  // past the last stage: the last one again (harmless loads, exact wait counts)
      v = __builtin_amdgcn_readfirstlane(live ? __builtin_ctz(m) : vlast);
      kcs = live ? kc : nkc - 1;
      const bool wrap = kc + 1 == nkc;
      kc = wrap ? 0 : kc + 1;
      if (wrap) m &= m - 1u;
    };
    // neighbour indices of this lane's 8 DMA rows for the next A stage, and that stage's channel-chunk offset
    u32x4 idx[2];
    int dka = 0;
    auto read_idx = [&]() __attribute__((always_inline)) {
      int v, kc;
      advance(dm, dkc, v, kc);
      dka = __builtin_amdgcn_readfirstlane(kc * KC * 2);
      const uint32_t ad = srct0 + ((uint32_t)v * BM + trow) * 4u;
      asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:16" : "=&v"(idx[0]), "=&v"(idx[1]) : "v"(ad) : "memory");
    };
    uint32_t off[8];
    int ka = 0;
    auto make_off = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int k = 0; k < 8; k++) off[k] = nbr_offset(idx[k >> 2][k & 3], rowbytes) + apiece[k & 1];
      ka = dka;
    };
    auto dma = [&](int slot, int k) __attribute__((always_inline)) {
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(dma_lds + (uint32_t)slot * (SU * 16) + (uint32_t)k * 1024u);
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                   :: "s"(m0), "v"(off[k]), "s"(rx), "s"(ka) : "memory", "m0");
    };
    u32x4 rb[2][4];  // weights of the stage being computed: column block t, K step j
    int bsoff = 0;
    auto b_next = [&]() __attribute__((always_inline)) {
      int v, kc;
      advance(bm, bkc, v, kc);
      bsoff = __builtin_amdgcn_readfirstlane((int)((wblk0 + (uint32_t)(v * nkc + kc)) * 4096u));
    };
    auto b_load = [&](int j) __attribute__((always_inline)) {
      asm volatile("buffer_load_dwordx4 %0, %2, %3, %4 offen\n\tbuffer_load_dwordx4 %1, %2, %3, %5 offen"
                   : "=&v"(rb[0][j]), "=&v"(rb[1][j])
                   : "v"(wlane + j * 1024), "s"(rw), "s"(bsoff), "s"(bsoff + (int)wblk_t) : "memory");
    };
    u32x4 fa[2][8];  // A fragments of a K step (double-buffered)
    auto read_a = [&](uint32_t slot_ad, int j, u32x4 (&A)[8]) __attribute__((always_inline)) {
      const uint32_t ad = slot_ad + alane[j];
#define SPC_READ_A(I) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(A[I]) : "v"(ad), "i"((I) * 4096) : "memory")
      SPC_READ_A(0);
      SPC_READ_A(1);
      SPC_READ_A(2);
      SPC_READ_A(3);
      SPC_READ_A(4);
      SPC_READ_A(5);
      SPC_READ_A(6);
      SPC_READ_A(7);
#undef SPC_READ_A
    };
    // One K step: the 16 MFMAs of step j (fragments A, weights rb[.][j]), with the next step's 8 fragment reads
    // (into An, from slot address nad, piece step jn) and the step's other memory work (work(p) after MFMA pair p)
    // spread between them, so each is issued while a matrix instruction runs. A read names A[I] as an input and
    // its output as early-clobber, so An[I] never shares registers with A[I]: an LDS return must not land in the
    // operands of a matrix instruction that may still be reading them.
    auto kstep = [&](const u32x4 (&A)[8], int j, u32x4 (&An)[8], uint32_t nad, int jn, auto&& work)
                     __attribute__((always_inline)) {
      const uint32_t ad = nad + alane[jn];
#define SPC_KSTEP_PAIR(I)                                                                                 \
      mfma_asm<F16>(acc[I][0], A[I], rb[0][j]);                                                          \
      mfma_asm<F16>(acc[I][1], A[I], rb[1][j]);                                                          \
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(An[I]) : "v"(ad), "i"((I) * 4096), "v"(A[I]) : "memory"); \
      work(I);
      SPC_KSTEP_PAIR(0)
      SPC_KSTEP_PAIR(1)
      SPC_KSTEP_PAIR(2)
      SPC_KSTEP_PAIR(3)
      SPC_KSTEP_PAIR(4)
      SPC_KSTEP_PAIR(5)
      SPC_KSTEP_PAIR(6)
      SPC_KSTEP_PAIR(7)
#undef SPC_KSTEP_PAIR
    };

    // prologue: A(0..2) by DMA, B(0), indices for A(3); then publish slot 0 and read stage 0's first fragments
#pragma unroll
    for (int p = 0; p < 3; p++) {
      read_idx();
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(idx[0]), "+v"(idx[1]) :: "memory");
      make_off();
#pragma unroll
      for (int k = 0; k < 8; k++) dma(p, k);
    }
    b_next();
#pragma unroll
    for (int j = 0; j < 4; j++) b_load(j);
    read_idx();
    asm_vmcnt<24>();  // A0 landed (A1, A2, B0 may be in flight)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(idx[0]), "+v"(idx[1]) :: "memory");
    make_off();
    wg_barrier();
    read_a(ring0, 0, fa[0]);

    // stage s (fragments of its K step 0 already requested): per K step j, wait for step j's fragments (requested a
    // whole K step earlier), request step j+1's, MFMAs, two DMAs of A(s+3) into slot (s+3)%4, B(s+1) step j. Before
    // the last step: wait for every read of slot s and the DMA of A(s+1), barrier, request stage s+1's step-0
    // fragments.
    // Stage 0 is peeled (FIRST): its weight waits count the prologue's loads, and a register-tied wait must not sit
    // on a branch (the compiler would copy the awaited registers before it).
    // Per stage s: K step j waits for its fragments (requested during step j-1) and weights, then runs kstep(), which
    // requests step j+1's fragments (step 3: stage s+1's step 0, from the next slot, after the barrier); the DMAs of
    // A(s+3) into slot (s+3)%4 go two per step, B(s+1) step j after step j's MFMAs.
    auto stage = [&](int s, auto FIRSTc) __attribute__((always_inline)) {
      constexpr bool FIRST = decltype(FIRSTc)::value;
      const uint32_t cur = ring0 + (uint32_t)(s & 3) * (SU * 16), nxt = ring0 + (uint32_t)((s + 1) & 3) * (SU * 16);
      const int fill = (s + 3) & 3;
      b_next();
      // B(s) step j was followed by 12 loads (stage 0: by 6 + 2j, the prologue's remaining B(0) loads and stage 0's)
      lgkm_tie8<0>(fa[0]);
      vm_tie2<FIRST ? 6 : 12>(rb[0][0], rb[1][0]);
      kstep(fa[0], 0, fa[1], cur, 1, [&](int p) __attribute__((always_inline)) {
        if (p == 3) dma(fill, 0);
        if (p == 5) dma(fill, 1);
        if (p == 7) b_load(0);
      });

      lgkm_tie8<0>(fa[1]);
      vm_tie2<FIRST ? 8 : 12>(rb[0][1], rb[1][1]);
      kstep(fa[1], 1, fa[0], cur, 2, [&](int p) __attribute__((always_inline)) {
        if (p == 1) read_idx();  // indices of A(s+4)
        if (p == 3) dma(fill, 2);
        if (p == 5) dma(fill, 3);
        if (p == 7) b_load(1);
      });

      lgkm_tie10<0>(fa[0], idx);  // step 2's fragments and the indices
      vm_tie2<FIRST ? 10 : 12>(rb[0][2], rb[1][2]);
      kstep(fa[0], 2, fa[1], cur, 3, [&](int p) __attribute__((always_inline)) {
        if (p == 3) dma(fill, 4);
        if (p == 5) dma(fill, 5);
        if (p == 7) b_load(2);
      });

      lgkm_tie8<0>(fa[1]);  // step 3's fragments: every read of slot s is done
      // A(s+1)'s last DMA was followed by 30 loads (stage 0: 28, stage 1: 36); no registers are tied here
      if (FIRST) asm_vmcnt<28>(); else if (s == 1) asm_vmcnt<36>(); else asm_vmcnt<30>();
      wg_barrier();
      vm_tie2<12>(rb[0][3], rb[1][3]);
      kstep(fa[1], 3, fa[0], nxt, 0, [&](int p) __attribute__((always_inline)) {
        if (p == 3) dma(fill, 6);
        if (p == 5) {
          dma(fill, 7);
          make_off();  // A(s+4)'s DMA offsets (after this stage's last DMAs read the previous ones)
        }
        if (p == 7) b_load(3);
      });
    };
    stage(0, std::true_type{});
#pragma nounroll
    for (int s = 1; s < total; s++) stage(s, std::false_type{});
    // The matrix instructions are inline assembly, so the compiler inserts no wait states between the last of them
    // and the accumulator reads below: the results are written at the end of an MFMA's passes, so wait out the
    // longest (a 32x32x16 MFMA is 8 passes of 4 cycles; 64 idle cycles cover it with margin).
    asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");
  }
  asm_vmcnt<0>();
  asm_lgkmcnt<0>();
  __syncthreads();
  if (a.part) {  // a K piece of a split tile: fp32 partial sums to the workspace, k_split_reduce256 does the rest
    float* pp = a.part + (size_t)unit * (BM * 256);
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int t = 0; t < 2; t++)
#pragma unroll
        for (int q = 0; q < 16; q++)
          pp[(i * 32 + (q >> 2) * 8 + h * 4 + (q & 3)) * 256 + wv * 64 + t * 32 + l32] = acc[i][t][q];
    return;
  }
  // epilogue through the idle ring: one slot per wavefront; slot rows map to output rows through ordP
  float* ew = (float*)&ring[wv][0];
  const int co_w = tn_ * 256 + wv * 64;
  float bias8[8];
#pragma unroll
  for (int q = 0; q < 8; q++) bias8[q] = a.bias ? a.bias[co_w + (lane & 7) * 8 + q] : 0.f;
  epilogue_tile<8, 2, 2, 0, true>(acc, ew, ordP, BM, co_w, bias8, make_epi(a), a.Co, lane);
}

// Sum of a split 256 x 256 tile's K pieces (in piece order), then the fused epilogue. One thread per (row, 8
// channels); 32 workgroups per tile.
__global__ void __launch_bounds__(256) k_split_reduce256(ConvArgs a) {
  const int tile = blockIdx.x / 32, ns = a.xs;
  const int e8 = (blockIdx.x % 32) * 256 + threadIdx.x, r = e8 / 32, c8 = (e8 % 32) * 8;
  const int tm_ = a.tsched[tile / a.tiles_n], tn_ = tile % a.tiles_n;
  const int row = tm_ * 256 + r, col = tn_ * 256 + c8;
  // pieces of this tile: units tile*ns .. tile*ns + ns (the kernel's unit numbering)
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < ns; j++) {
    const float* pp = a.part + ((size_t)(tile * ns + j) * 256 + r) * 256 + c8;
    const f32x4 lo = *(const f32x4*)pp, hi = *(const f32x4*)(pp + 4);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      v[q] += lo[q];
      v[q + 4] += hi[q];
    }
  }
  const bool ok = row < a.N;
  const Epi e = make_epi(a);
  float bias8[8];
#pragma unroll
  for (int q = 0; q < 8; q++) bias8[q] = a.bias ? a.bias[col + q] : 0.f;
  const uint32_t o = (uint32_t)(ok ? a.order[row] : 0) * (uint32_t)a.Co + (uint32_t)col;
  u32x4 rv[2];
  load_res8(e, o, ok, rv);
  store_row8(e, o, ok, v, bias8, rv);
}

// 128-row tiles, two workgroups per CU. Measured on C3 (1526 tiles of 256 rows): 256-row tiles with one workgroup
// per CU were 6% slower (prologue, barriers and epilogue exposed; 2x fewer weight loads per flop did not make up
// for it), as were 8 wavefronts of 128 rows x 64 channels on a 256-row tile (3% slower: weights loaded twice).
// Reduction of the split tiles: one thread per (row, 8 channels) of a split tile; sums its pieces' partials in
// piece order, then the fused epilogue (bias, act, residual, one rounding) of the unsplit kernel.
template <int BM>
__global__ void __launch_bounds__(256) k_split_reduce(ConvArgs a) {
  constexpr int UPT = BM * 256 / 8 / 256;  // workgroups per split tile
  int st = blockIdx.x / UPT;                 // split tile, counted over the XCDs in order
  const int e8 = (blockIdx.x % UPT) * 256 + threadIdx.x, r = e8 / 32, c8 = (e8 % 32) * 8;
  int x = 0, ntail = 0;
  for (; x < 8; x++) {
    ntail = a.xk[x] > 1 ? (a.xt0[x + 1] - a.xt0[x]) - a.xs : 0;
    if (st < ntail) break;
    st -= ntail;
  }
  if (x == 8) return;
  const int kx = a.xk[x], logical = a.xt0[x] + a.xs + st, pbase = a.xpart0[x] + st * kx;
  const int tm_ = a.tnmaj ? logical % a.tiles_m : logical / a.tiles_n;
  const int tn_ = a.tnmaj ? logical / a.tiles_m : logical % a.tiles_n;
  const int row = tm_ * BM + r, col = tn_ * 256 + c8;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < kx; j++) {
    const float* pp = a.part + ((size_t)(pbase + j) * BM + r) * 256 + c8;
    const f32x4 lo = *(const f32x4*)pp, hi = *(const f32x4*)(pp + 4);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      v[q] += lo[q];
      v[q + 4] += hi[q];
    }
  }
  const bool ok = row < a.N;
  const Epi e = make_epi(a);
  float bias8[8];
#pragma unroll
  for (int q = 0; q < 8; q++) bias8[q] = a.bias ? a.bias[col + q] : 0.f;
  const uint32_t o = (uint32_t)(ok ? a.order[row] : 0) * (uint32_t)a.Co + (uint32_t)col;
  u32x4 rv[2];
  load_res8(e, o, ok, rv);
  store_row8(e, o, ok, v, bias8, rv);
}

int device_cus() {
  static int n[64] = {};
  int dev = 0;
  CK(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) dev = 0;
  if (!n[dev]) CK(hipDeviceGetAttribute(&n[dev], hipDeviceAttributeMultiprocessorCount, dev));
  return n[dev];
}

// The tail split is off when SPCONV_NO_SPLIT is set (A/B runs and the tests that compare both schedules).
bool split_enabled() {
  const char* e = getenv("SPCONV_NO_SPLIT");
  return !(e && e[0] && e[0] != '0');
}

// Wave-quantization tail: with two workgroups per CU, an XCD (32 CUs, its own L2; workgroup ids are dealt to the
// 8 XCDs round-robin) runs 64 tiles at once. When an XCD's tiles number between 64 and 96 (C2: 594 tiles, 74-75
// per XCD), the last ones would run as a thin second round; instead each of them is split over k = 64 / tail
// (at most 8) workgroups along its K stages, so the second round is as wide as the first and k times shorter.
// Measured on C2: 0.81 ms with 198 row tiles against 0.59 ms with 170 (510 workgroups, one round).
template <bool F16>
void launch_wide_dma(ConvArgs a) {
  constexpr int BM = 128;
  a.tiles_m = cdiv(a.N, BM);
  a.tiles_n = a.Co / 256;
  const int tiles = a.tiles_m * a.tiles_n;
  a.grid = (tiles + 7) / 8 * 8;
  a.part = nullptr;
  const int slots = 2 * (device_cus() / 8);  // concurrent workgroups per XCD
  const int per = cdiv(tiles, 8);
  Tensor ws;
  if (split_enabled() && slots > 0 && per > slots && per - slots <= slots / 2) {
    int units = 0, pslots = 0;
    a.xs = slots;
    for (int x = 0; x < 8; x++) {
      a.xt0[x] = std::min(x * per, tiles);
      const int c = std::min(per, tiles - a.xt0[x]), tail = c - slots;
      a.xk[x] = tail > 0 ? std::min(8, slots / tail) : 1;
      a.xpart0[x] = pslots;
      if (a.xk[x] > 1) pslots += tail * a.xk[x];
      units = std::max(units, a.xk[x] > 1 ? slots + tail * a.xk[x] : c);
    }
    a.xt0[8] = tiles;
    if (pslots > 0) {
      ws = empty({(i64)pslots * BM * 256}, F32);
      a.part = ws.ptr<float>();
      a.grid = 8 * units;
    }
  } else if (split_enabled() && slots > 0 && 2 * per <= slots) {
    // too few tiles to fill half the slots (small N, e.g. C2's 85 x 3 tiles): every tile is split along its K
    // stages over k = min(8, slots / c) workgroups, so each XCD runs about `slots` pieces at once
    int units = 0, pslots = 0;
    a.xs = 0;
    for (int x = 0; x < 8; x++) {
      a.xt0[x] = std::min(x * per, tiles);
      const int c = std::min(per, tiles - a.xt0[x]);
      a.xk[x] = c > 0 ? std::min(8, slots / c) : 1;
      a.xpart0[x] = pslots;
      if (a.xk[x] > 1) pslots += c * a.xk[x];
      units = std::max(units, c * a.xk[x]);
    }
    a.xt0[8] = tiles;
    if (pslots > 0) {
      ws = empty({(i64)pslots * BM * 256}, F32);
      a.part = ws.ptr<float>();
      a.grid = 8 * units;
    }
  }
  if (a.part) a.tsched = nullptr;  // the tail split keeps the XCD-contiguous walk
  a.tnmaj = a.part != nullptr;
  // Longest-first tiles are dealt to the XCDs in runs of 16 consecutive ones instead of one by one: within a mask
  // the gray order is the input (Morton) order, so a run's gathers overlap in that XCD's L2. Same bits; C3 kernel
  // 0.800 -> 0.788 ms (three interleaved runs on two boxes; runs of 4 / 8 / 12 / 24 / 32 / 64 / 128 tiles measured
  // 0.795 / 0.793 / 0.792 / 0.793 / 0.792 / 0.798 / 0.815).
  a.xblk = 16;
  k_conv_wide_dma<F16, BM><<<a.grid, 256, 0, stream()>>>(a);
  if (a.part) {
    int ntail = 0;
    for (int x = 0; x < 8; x++)
      if (a.xk[x] > 1) ntail += (a.xt0[x + 1] - a.xt0[x]) - a.xs;
    k_split_reduce<BM><<<ntail * (BM * 256 / 8 / 256), 256, 0, stream()>>>(a);
  }
}

// Weight repack for k_conv_w256: w [Co,27,Ci] -> one 4 KB block per (32-column block cb, offset v, 64-channel
// chunk kc), inside it 4 K steps x 64 lanes x 16 bytes in v_mfma_f32_32x32x16 operand order: lane l of step j holds
// column cb*32 + (l & 31), input channels kc*64 + j*16 + (l >> 5)*8 .. +8.
// Grid (nkc, 27, Co/32) of 256-thread blocks: block (kc, v, cb), thread j*64 + lane.
__global__ void __launch_bounds__(256) k_pack_w256(const u32x4* __restrict__ w, u32x4* __restrict__ wp, int Ci) {
  const int nkc = Ci / 64, kc = blockIdx.x, v = blockIdx.y, cb = blockIdx.z;
  const int j = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int co = cb * 32 + (lane & 31), ch = kc * 64 + j * 16 + (lane >> 5) * 8;
  wp[(((i64)cb * 27 + v) * nkc + kc) * 256 + threadIdx.x] = w[((i64)co * 27 + v) * Ci / 8 + ch / 8];
}

// The 256 x 256 kernel (k_conv_w256) runs instead of the 128-row k_conv_wide_dma when SPCONV_W256 is set. Measured
// on C3 (same box, both with longest-first tile order): 0.947 ms against 0.918 -- it halves the weight bytes per
// flop, but one wavefront per SIMD exposes every per-stage wait, and without group skipping it runs the tile's
// union of offsets (1.18x the active pairs against 1.05x).
// The 8-wavefront both-operands-in-LDS kernel (k_conv_w8) runs when SPCONV_W8 is set (read per call).
bool w8_enabled() {
  const char* e = getenv("SPCONV_W8");
  return e && e[0] && e[0] != '0';
}
bool w256_enabled() {
  const char* e = getenv("SPCONV_W256");
  return e && e[0] && e[0] != '0';
}

// Tiles of 256 rows x 256 channels, one workgroup per CU. When the tiles fill the CUs poorly (small N, e.g. C2's
// 43 x 3 tiles on 256 CUs), each tile's K stages are split over ns workgroups whose fp32 partials
// k_split_reduce256 sums (ns from the cost model below).
template <bool F16>
void launch_w256(ConvArgs a) {
  a.tiles_m = cdiv(a.N, 256);
  a.tiles_n = a.Co / 256;
  const int tiles = a.tiles_m * a.tiles_n, cus = device_cus();
  // K pieces per tile: minimise rounds(ns) / ns x (a tile's time) + the partials' traffic (ns fp32 tiles written
  // and read back), with a tile's time estimated from ~20 offsets x Ci/32 stages of ~0.53 us
  int ns = 1;
  if (split_enabled() && tiles < 2 * cus) {
    const double t_tile = 20.0 * (a.Ci / 64) * 1.06e-6;
    double best = 1e30;
    for (int k = 1; k <= 8; k++) {
      const double rounds = (double)cdiv(tiles * k, cus);
      const double t = rounds / k * t_tile + (k > 1 ? 5e-6 + (double)k * tiles * 2 * 262144 / 4e12 : 0.0);
      if (t < best * 0.97) {
        best = t;
        ns = k;
      }
    }
  }
  a.xs = ns;
  Tensor ws;
  a.part = nullptr;
  if (ns > 1) {
    ws = empty({(i64)tiles * ns * 256 * 256}, F32);
    a.part = ws.ptr<float>();
  }
  a.grid = (tiles * ns + 7) / 8 * 8;
  k_conv_w256<F16><<<a.grid, 256, 0, stream()>>>(a);
  if (ns > 1) k_split_reduce256<<<tiles * 32, 256, 0, stream()>>>(a);
}

template <bool F16, int NW, int BM>
void launch_wide(ConvArgs a) {
  a.tiles_m = cdiv(a.N, BM);
  a.tiles_n = a.Co / (64 * NW);
  int tiles = a.tiles_m * a.tiles_n;
  a.grid = (tiles + 7) / 8 * 8;
  k_conv_wide<F16, NW, BM><<<a.grid, NW * 64, 0, stream()>>>(a);
}

// Weight repack for the wide kernel: w [Co,27,Ci] -> one 1 KiB block per (64-channel output slice, offset v,
// 64-channel input block kc, 32-column half t, step j), laid out as 64 lanes x 16 bytes in MFMA operand order:
// lane l holds column c = slice*64 + t*32 + (l & 31), input channels kc*64 + (l >> 5)*32 + j*8 .. +8.
// A wavefront then fetches a stage's weight fragment with fully coalesced 1 KiB loads.
// Grid (nkc*2, 27, Co/64) of 256-thread blocks: block (kc*2 + t, v, slice) writes the four 1 KiB blocks
// j = 0..3 of that (slice, v, kc, t), thread = j*64 + lane; no thread divides.
__global__ void __launch_bounds__(256) k_pack_w(const u32x4* __restrict__ w, u32x4* __restrict__ wp, int Co, int Ci) {
  const int nkc = Ci / 64, kc = blockIdx.x >> 1, t = blockIdx.x & 1, v = blockIdx.y, slice = blockIdx.z;
  const int j = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int co = slice * 64 + t * 32 + (lane & 31), ch = kc * 64 + (lane >> 5) * 32 + j * 8;
  wp[((((i64)slice * 27 + v) * nkc + kc) * 2 + t) * 256 + threadIdx.x] = w[((i64)co * 27 + v) * Ci / 8 + ch / 8];
}

__global__ void k_to_f32(const void* p, int dt, int n, float* o) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) o[i] = load_elem(p, i, dt);
}

template <bool F16, int BM, int BN, int WGM, int WGN, int KC>
void launch(ConvArgs a) {
  a.tiles_m = cdiv(a.N, BM);
  a.tiles_n = a.Co / BN;
  int tiles = a.tiles_m * a.tiles_n;
  a.grid = (tiles + 7) / 8 * 8;
  k_conv<F16, BM, BN, WGM, WGN, KC><<<a.grid, WGM * WGN * 64, 0, stream()>>>(a);
}

template <bool F16>
void dispatch(const SpConvCfg& cfg, ConvArgs a) {
  // The fp16-compatible epilogue (EPI_F16_COMPAT) runs in every kernel: store_row8 applies it.
  if (a.hrows) return a.Ci == 64 ? launch_halo<F16, 2>(a) : launch_halo<F16, 4>(a);
  if (a.Co == 64 && a.Ci <= 128) {
    switch (a.Ci / 32) {
      case 1: return launch_narrow<F16, 1, 4>(a);
      case 2: return launch_narrow<F16, 2, 4>(a);
      case 3: return launch_narrow<F16, 3, 4>(a);
      default: return launch_narrow<F16, 4, 4>(a);
    }
  }
  if (a.Co % 256 == 0 && a.Ci % 32 == 0 && w8_enabled()) {
    a.tiles_m = cdiv(a.N, 256);
    a.tiles_n = a.Co / 256;
    a.grid = a.tiles_m * a.tiles_n;
    k_conv_w8<F16><<<a.grid, 512, 0, stream()>>>(a);
    return;
  }
  // Fixed tiles per channel width (no autotune): BM = 128 sorted rows per tile.
  if (a.Co % 256 == 0 && a.Ci % 64 == 0 && w256_enabled()) return launch_w256<F16>(a);
  if (cfg.BK == 64 && a.Co % 256 == 0) return launch_wide_dma<F16>(a);
  if (cfg.BK == 64 && a.Co % 128 == 0) return launch_wide<F16, 2, 128>(a);
  if (a.Co % 128 == 0) {
    if (cfg.BK == 64) launch<F16, 128, 128, 2, 2, 64>(a);
    else launch<F16, 128, 128, 2, 2, 32>(a);
  } else {
    if (cfg.BK == 64) launch<F16, 128, 64, 4, 1, 64>(a);
    else launch<F16, 128, 64, 4, 1, 32>(a);
  }
}
}  // namespace

SpConvCfg spconv_cfg(int N, int Ci, int Co) {
  (void)N;
  (void)Co;
  return SpConvCfg{128, Ci % 64 == 0 ? 64 : 32, 1};
}

// The kernels that read their tiles' neighbour rows from the tile-order table (narrow, 256-channel wide) can read
// them through a row map instead; the others get the gathered rows materialized.
bool reads_row_table(const SpConvCfg& cfg, int Ci, int Co, int act) {
  (void)act;
  return (Co == 64 && Ci <= 128) || (cfg.BK == 64 && Co % 256 == 0);
}

__global__ void k_gather_rows(const u32x4* __restrict__ x, i64 m, int units, const int32_t* __restrict__ row_map,
                              int shift, i64 n, u32x4* __restrict__ out) {
  const i64 q = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= n * units) return;
  const i64 i = q / units;
  const uint32_t r = (uint32_t)row_map[i] >> shift;
  out[q] = r < (uint64_t)m ? x[(i64)r * units + (q - i * units)] : u32x4{0, 0, 0, 0};
}

// Conv-kernel timer (off unless kernel_timing(true)): while on, every conv call records a HIP event on the library
// stream right before its first conv kernel and right after its last (split-K reduction and spill-tile kernel
// included; weight repack, bias conversion and first-call schedules excluded), so a caller can time the kernels
// alone. Events are pooled and reused after kernel_timing(true) resets the list.
struct KernelTimer {
  bool on = false;
  std::vector<hipEvent_t> ev;
  size_t used = 0;
};
KernelTimer& ktimer() {
  static KernelTimer t;
  return t;
}
void ktimer_mark() {
  KernelTimer& t = ktimer();
  if (!t.on) return;
  if (t.used == t.ev.size()) {
    hipEvent_t e;
    CK(hipEventCreate(&e));
    t.ev.push_back(e);
  }
  CK(hipEventRecord(t.ev[t.used++], stream()));
}

// A second stream per device (default priority, like the library stream) with a fork and a join event, for the
// spill tiles' gathering kernel, which runs beside the halo kernel. Created on first use, kept until the process ends.
struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
SideStream& side_stream() {
  static SideStream ss[64];
  int dev = 0;
  CK(hipGetDevice(&dev));
  REQ(dev >= 0 && dev < 64, "device %d", dev);
  SideStream& r = ss[dev];
  if (!r.s) {
    CK(hipStreamCreateWithFlags(&r.s, hipStreamNonBlocking));
    CK(hipEventCreateWithFlags(&r.fork, hipEventDisableTiming));
    CK(hipEventCreateWithFlags(&r.join, hipEventDisableTiming));
  }
  return r;
}

// The halo kernel serves Ci = Co = 64 unless SPCONV_NO_HALO is set (then the gathering narrow kernel does).
bool halo_enabled() {
  static const bool on = [] {
    const char* e = getenv("SPCONV_NO_HALO");
    return !(e && e[0] && e[0] != '0');
  }();
  return on;
}
// Ci = 128 -> 64 takes the halo kernel only when SPCONV_HALO128 is set (read per call). Measured on C5's children
// (same box): 1.13 ms against 0.99 for the gathering kernel. The halo removes the gather misses, but a wavefront
// pair of 64 rows loads the whole 442 KB weight tensor from L2 (7.4 GB per launch, the per-CU load path's largest
// stream), and 128-row windows leave 16-row groups at 3.2x the active pairs (2.1x in 65536-row windows).
bool halo128_enabled() {
  const char* e = getenv("SPCONV_HALO128");
  return halo_enabled() && e && e[0] && e[0] != '0';
}

// x: the conv input [N,Ci], or with row_map the source rows [M,Ci] read through row_map >> shift
struct SkipRes {  // skip residual of the upsample block (see ConvArgs::skip_*)
  const Tensor* x;
  const Tensor* src;
};
struct PreLN {  // pre-activation of the input rows (see ConvArgs::ln_*); only with the halo kernel
  const Tensor* gamma;
  const Tensor* beta;
  float eps;
  int act;
};
void conv_impl(const Tensor& x, const Tensor* row_map, int shift, const Tensor& w, const Tensor* b,
               const Tensor* residual, int act, SpConvCache& c, Tensor& out, const SkipRes* skip = nullptr,
               const PreLN* ln = nullptr) {
  REQ(x.dim() == 2 && w.dim() == 3, "x must be [N,Ci], w [Co,27,Ci]");
  const int N = row_map ? c.N : (int)x.size(0), Ci = (int)x.size(1), Co = (int)w.size(0);
  const i64 M = x.size(0);
  REQ((x.dt == BF16 || x.dt == F16) && w.dt == x.dt, "x and w must both be bf16 or both fp16 (x %s, w %s)",
      dname(x.dt), dname(w.dt));
  REQ(w.size(1) == 27 && w.size(2) == Ci, "w must be [Co,27,%d]", Ci);
  REQ(Ci > 0 && Ci % 32 == 0 && Ci <= kMaxCi, "Ci=%d must be a multiple of 32 (at most %d)", Ci, kMaxCi);
  REQ(Co > 0 && Co % 64 == 0, "Co=%d must be a multiple of 64", Co);
  REQ(N == c.N, "x has %d rows, neighbour cache %d", N, c.N);
  const int act0 = act & ~EPI_F16_COMPAT;
  REQ(act0 == ACT_NONE || act0 == ACT_SILU, "act=%d", act);
  if (act & EPI_F16_COMPAT)
    REQ(x.dt == F16 && out.dt == F16 && (!b || b->dt == F16) && (!residual || residual->dt == F16),
        "the fp16-compatible epilogue needs fp16 x, w, out and an fp16 (or no) bias and residual");
  REQ(out.defined() && out.dim() == 2 && out.size(0) == N && out.size(1) == Co &&
          (out.dt == F32 || out.dt == F16 || out.dt == BF16),
      "out must be [N,Co] f32/f16/bf16");
  if (residual)
    REQ(residual->dim() == 2 && residual->size(0) == N && residual->size(1) == Co &&
            (residual->dt == F32 || residual->dt == F16 || residual->dt == BF16),
        "residual must be [N,Co] f32/f16/bf16");
  if (b) REQ(b->numel() == Co && (b->dt == F32 || b->dt == F16 || b->dt == BF16), "bias must be [Co] f32/f16/bf16");
  if (N == 0) return;
  SpConvCfg cfg = spconv_cfg(N, Ci, Co);
  Tensor bf;
  if (b) {
    if (b->dt == F32) bf = *b;
    else {
      bf = empty({Co}, F32);
      k_to_f32<<<cdiv(Co, 256), 256, 0, stream()>>>(b->p, b->dt, Co, bf.ptr<float>());
    }
  }
  ConvArgs a{};
  a.x = x.ptr<uint16_t>();
  a.w = w.ptr<uint16_t>();
  a.bias = b ? bf.ptr<float>() : nullptr;
  a.res = residual ? residual->p : nullptr;
  a.res_dt = residual ? residual->dt : F32;
  a.out = out.p;
  a.out_dt = out.dt;
  a.nbr = c.nbr.ptr<uint32_t>();
  a.order = c.sorted.ptr<int32_t>();
  a.gray = c.gray.ptr<int32_t>();
  REQ((uint64_t)M * Ci * 2 <= kMaxBufferBytes && (uint64_t)Co * 27 * Ci * 2 <= kMaxBufferBytes,
      "x or w larger than %llu bytes", (unsigned long long)kMaxBufferBytes);
  a.x_bytes = (uint32_t)((uint64_t)M * Ci * 2);
  REQ(((uint64_t)N + SpConvCache::kRowTablePad) * 108 <= kMaxBufferBytes, "neighbour table larger than %llu bytes",
      (unsigned long long)kMaxBufferBytes);
  a.nbr_bytes = (uint32_t)((uint64_t)N * 108);
  if (residual) {
    REQ((uint64_t)N * Co * dsize(residual->dt) <= kMaxBufferBytes, "residual larger than %llu bytes",
        (unsigned long long)kMaxBufferBytes);
    a.res_bytes = (uint32_t)((uint64_t)N * Co * dsize(residual->dt));
  }
  REQ((uint64_t)N * Co * dsize(out.dt) <= kMaxBufferBytes, "output larger than %llu bytes",
      (unsigned long long)kMaxBufferBytes);
  a.out_bytes = (uint32_t)((uint64_t)N * Co * dsize(out.dt));
  a.w_bytes = (uint32_t)((uint64_t)Co * 27 * Ci * 2);
  a.N = N;
  a.Ci = Ci;
  a.Co = Co;
  a.act = act;
  Tensor wpack, mtbl;
  REQ(!row_map || reads_row_table(cfg, Ci, Co, act), "row map with a kernel that reads nbr directly");
  const SpConvCache::HaloTable* ht = nullptr;
  if (Co == 64 && Ci == 64 && halo_enabled()) ht = &c.halo_table(HaloShape<2>::B, HaloShape<2>::UM);
  else if (Co == 64 && Ci == 128 && halo128_enabled()) ht = &c.halo_table(HaloShape<4>::B, HaloShape<4>::UM);
  if (ht) {  // halo kernel: narrow weight order, the tile's distinct neighbour rows copied to LDS once
    wpack = empty({(i64)Co * 27 * Ci}, x.dt);
    k_pack_w_narrow<<<dim3(Ci / 32, Co / 16, 27), 64, 0, stream()>>>((const u32x4*)w.p, (u32x4*)wpack.p, Co, Ci);
    a.w = wpack.ptr<uint16_t>();
    a.hrows = ht->rows.ptr<int32_t>();
    a.hcount = ht->count.ptr<int32_t>();
    a.hidx = (const uint16_t*)ht->idx.p;
    a.hgm = ht->gm.ptr<uint32_t>();
    a.order = ht->order.ptr<int32_t>();
    if (row_map) {
      a.rmap = row_map->ptr<int32_t>();
      a.rshift = shift;
      a.rmax = (int)std::min<i64>(M, INT32_MAX);
    }
    if (skip) {
      a.skip_x = skip->x->ptr<uint16_t>();
      a.skip_src = skip->src->ptr<int32_t>();
      a.skip_cin = (int)skip->x->size(1);
      a.skip_rep = Co / (a.skip_cin / 8);
      a.skip_n = (uint32_t)skip->x->size(0);
      a.skip_bytes = (uint32_t)skip->x->bytes();
      a.res = skip->x->p;  // the epilogue's residual type (16-bit); its rows come through load_skip8
      a.res_dt = skip->x->dt;
      a.res_bytes = a.skip_bytes;
    }
  } else if (Co == 64 && Ci <= 128) {  // narrow kernel: weights in 16x16x32 operand order, spatial row order
    wpack = empty({(i64)Co * 27 * Ci}, x.dt);
    // Ci = 128: each gather instruction reads one contiguous 64-byte piece of its 16 rows (16 half lines) instead of
    // four 16-byte pieces 64 bytes apart (32 lines, each half used): C5 children 0.857 -> 0.823 ms
    a.kcontig = Ci == 128;
    k_pack_w_narrow<<<dim3(Ci / 32, Co / 16, 27), 64, 0, stream()>>>((const u32x4*)w.p, (u32x4*)wpack.p, Co, Ci,
                                                                     a.kcontig);
    a.w = wpack.ptr<uint16_t>();
    const SpConvCache::RowTable& rt = c.row_table(16);
    a.order = rt.order.ptr<int32_t>();
    a.tbl = rt.tbl.ptr<uint32_t>();
    a.gs = rt.gs.ptr<int32_t>();
    a.tbl_bytes = (uint32_t)rt.tbl.bytes();
    if (row_map) {  // the kernel maps each tile's neighbour rows in its prologue (no mapped copy of the table)
      a.rmap = row_map->ptr<int32_t>();
      a.rshift = shift;
      a.rmax = (int)std::min<i64>(M, INT32_MAX);
    }
  } else if (Co % 256 == 0 && Ci % 32 == 0 && w8_enabled()) {  // 256 x 256 tiles, both operands through LDS
    wpack = empty({(i64)Co * 27 * Ci}, x.dt);
    k_pack_w8<<<dim3(Ci / 32, 27, Co / 256), 256, 0, stream()>>>((const u32x4*)w.p, (u32x4*)wpack.p, Ci);
    a.w = wpack.ptr<uint16_t>();
    const SpConvCache::RowTable& rt = c.row_table(-1);
    if (row_map) mtbl = c.mapped_table(-1, *row_map, shift, M);
    a.tbl = row_map ? mtbl.ptr<uint32_t>() : rt.tbl.ptr<uint32_t>();
    a.gs = rt.gs.ptr<int32_t>();
    a.tbl_bytes = (uint32_t)rt.tbl.bytes();
    a.tsched = c.tile_schedule(-1, 256).ptr<int32_t>();
  } else if (Co % 256 == 0 && Ci % 64 == 0 && w256_enabled()) {  // 256 x 256 tiles: 4 KB weight blocks
    wpack = empty({(i64)Co * 27 * Ci}, x.dt);
    k_pack_w256<<<dim3(Ci / 64, 27, Co / 32), 256, 0, stream()>>>((const u32x4*)w.p, (u32x4*)wpack.p, Ci);
    a.w = wpack.ptr<uint16_t>();
    const SpConvCache::RowTable& rt = c.row_table(-1);
    if (row_map) mtbl = c.mapped_table(-1, *row_map, shift, M);
    a.tbl = row_map ? mtbl.ptr<uint32_t>() : rt.tbl.ptr<uint32_t>();
    a.gs = rt.gs.ptr<int32_t>();
    a.tbl_bytes = (uint32_t)rt.tbl.bytes();
    a.tsched = c.tile_schedule(-1, 256).ptr<int32_t>();
  } else if (cfg.BK == 64 && Co % 128 == 0) {  // wide kernels read the 32x32x16-ordered weight copy
    wpack = empty({(i64)Co * 27 * Ci}, x.dt);
    k_pack_w<<<dim3(Ci / 64 * 2, 27, Co / 64), 256, 0, stream()>>>((const u32x4*)w.p, (u32x4*)wpack.p, Co, Ci);
    a.w = wpack.ptr<uint16_t>();
    if (Co % 256 == 0) {  // the 128 x 256 kernel reads its tiles' neighbour rows from the sorted-order table
      const SpConvCache::RowTable& rt = c.row_table(-1);
      if (row_map) mtbl = c.mapped_table(-1, *row_map, shift, M);
      a.tbl = row_map ? mtbl.ptr<uint32_t>() : rt.tbl.ptr<uint32_t>();
      a.gs = rt.gs.ptr<int32_t>();
      a.tbl_bytes = (uint32_t)rt.tbl.bytes();
      a.tsched = c.tile_schedule(-1, 128).ptr<int32_t>();
    }
  }
  REQ(!skip || ht, "the fused skip residual needs the halo kernel");
  REQ(!ln || (ht && ht->host_spills() == 0), "the fused pre-activation needs the halo kernel with no spill tiles");
  // the generic kernel reads the reference's per-block offset masks (valid(B1)'s OR masks); the others do not
  if (!ht && !(Co == 64 && Ci <= 128) && !(Co % 256 == 0 && Ci % 64 == 0 && w256_enabled()) &&
      !(Co % 256 == 0 && Ci % 32 == 0 && w8_enabled()) &&
      !(cfg.BK == 64 && Co % 128 == 0))
    a.code = c.block_masks(cfg.B1).ptr<uint32_t>();
  if (ln) {
    a.ln_on = 1;
    a.ln_gamma = ln->gamma ? ln->gamma->ptr<float>() : nullptr;
    a.ln_beta = ln->beta ? ln->beta->ptr<float>() : nullptr;
    a.ln_eps = ln->eps;
    a.ln_act = ln->act;
  }
  if (ht) {
    // The halo kernel skips the spill tiles (their count is known only on the device); the gathering kernel computes
    // them from the device list, with the identity row order inside each tile (tbl = nbr, gs = gray), on a second
    // stream beside the halo kernel (a few tiles of long latency; after it, it added ~36 us to C4's 0.64 ms). Its
    // grid covers every tile; workgroups past the spill count exit at once. Fork after everything both kernels read
    // is queued on the library stream, join before anything later on it.
    ConvArgs sa = a;
    sa.hrows = nullptr;
    sa.hcount = nullptr;
    sa.hidx = nullptr;
    sa.hgm = nullptr;
    sa.order = nullptr;
    sa.gs = c.gray.ptr<int32_t>();
    sa.tbl = c.nbr.ptr<uint32_t>();
    sa.tbl_bytes = a.nbr_bytes;
    sa.tlist = ht->spill_list.ptr<int32_t>();
    sa.tcount = ht->spill_count.ptr<int32_t>();
    ktimer_mark();
    SideStream& ss = side_stream();
    CK(hipEventRecord(ss.fork, stream()));
    CK(hipStreamWaitEvent(ss.s, ss.fork, 0));
    if (Ci == 64) x.dt == F16 ? launch_narrow<true, 2, 4>(sa, ss.s) : launch_narrow<false, 2, 4>(sa, ss.s);
    else x.dt == F16 ? launch_narrow<true, 4, 4>(sa, ss.s) : launch_narrow<false, 4, 4>(sa, ss.s);
    CK(hipGetLastError());
    CK(hipEventRecord(ss.join, ss.s));
    if (x.dt == F16) dispatch<true>(cfg, a);
    else dispatch<false>(cfg, a);
    CK(hipGetLastError());
    CK(hipStreamWaitEvent(stream(), ss.join, 0));
    ktimer_mark();
    return;
  }
  ktimer_mark();
  if (x.dt == F16) dispatch<true>(cfg, a);
  else dispatch<false>(cfg, a);
  CK(hipGetLastError());
  ktimer_mark();
}

void subm_conv_skip(const Tensor& x, const Tensor& w, const Tensor* b, int act, const Tensor& x_skip,
                    const Tensor& src, SpConvCache& c, Tensor& out) {
  REQ(x.dim() == 2 && w.dim() == 3 && x_skip.dim() == 2, "x [N,Ci], w [Co,27,Ci], x_skip [n,Cin]");
  const int Ci = (int)x.size(1), Co = (int)w.size(0), Cin = (int)x_skip.size(1);
  REQ(src.dt == I32 && src.numel() == c.N, "src must be int32 [%d]", c.N);
  REQ(x_skip.dt == out.dt && (out.dt == BF16 || out.dt == F16), "x_skip and out: one 16-bit dtype");
  REQ(Cin % 64 == 0 && Co % (Cin / 8) == 0, "Cin=%d Co=%d: need Cin %% 64 == 0 and Co a multiple of Cin/8", Cin, Co);
  const int rep = Co / (Cin / 8);
  REQ((rep & (rep - 1)) == 0, "Co / (Cin/8) = %d must be a power of two", rep);
  REQ((uint64_t)x_skip.bytes() <= kMaxBufferBytes && ((uintptr_t)x_skip.p % 16) == 0, "x_skip too large / unaligned");
  REQ(!(act & EPI_F16_COMPAT), "no fp16-compatible epilogue with the fused skip");
  // 64 -> 64: the halo kernel (and the gathering kernel for its spill tiles) adds the skip rows in the epilogue
  const bool fused = c.N > 0 && Ci == 64 && Co == 64 && halo_enabled();
  if (fused) {
    const SkipRes sk{&x_skip, &src};
    conv_impl(x, nullptr, 0, w, b, nullptr, act, c, out, &sk);
  } else {  // other shapes: the conv, then the skip add as its own pass
    conv_impl(x, nullptr, 0, w, b, nullptr, act, c, out);
    add_skip(out, x_skip, src);
  }
}

void subm_conv_fused(const Tensor& x, const Tensor& w, const Tensor* b, const Tensor* residual, int act,
                     SpConvCache& c, Tensor& out) {
  conv_impl(x, nullptr, 0, w, b, residual, act, c, out);
}

void subm_conv_gathered(const Tensor& x_src, const Tensor& row_map, int shift, const Tensor& w, const Tensor* b,
                        const Tensor* residual, int act, SpConvCache& c, Tensor& out) {
  REQ(x_src.dim() == 2 && w.dim() == 3, "x_src must be [M,Ci], w [Co,27,Ci]");
  REQ(row_map.dt == I32 && row_map.numel() == c.N, "row_map must be int32 [%d]", c.N);
  REQ(shift >= 0 && shift < 31, "shift=%d", shift);
  const int Ci = (int)x_src.size(1), Co = (int)w.size(0);
  REQ(Ci > 0 && Ci % 32 == 0 && Ci <= kMaxCi, "Ci=%d must be a multiple of 32 (at most %d)", Ci, kMaxCi);
  if (c.N == 0 || reads_row_table(spconv_cfg(c.N, Ci, Co), Ci, Co, act)) {
    conv_impl(x_src, &row_map, shift, w, b, residual, act, c, out);
    return;
  }
  Tensor xg = empty({(i64)c.N, Ci}, x_src.dt);
  const int units = Ci * 2 / 16;
  k_gather_rows<<<cdiv((i64)c.N * units, 256), 256, 0, stream()>>>((const u32x4*)x_src.p, x_src.size(0), units,
                                                                   row_map.ptr<int32_t>(), shift, c.N, (u32x4*)xg.p);
  CK(hipGetLastError());
  conv_impl(xg, nullptr, 0, w, b, residual, act, c, out);
}

// Conv of pre-activated rows: x = act_pre(LayerNorm(x_src[row_map >> shift]) * gamma + beta), then the conv with
// bias and act, plus the upsample block's skip residual when x_skip / skip_src are given (as subm_conv_skip).
// By default gather_ln_act writes x and the conv (and skip) run on it. With SPCONV_PRELN_FUSED set, and when the
// halo kernel serves the cache with no spill tiles, the pre-activation runs instead on each tile's halo rows in LDS
// before the K loop (one kernel for gather + LayerNorm + SiLU + conv + skip). Both give the same bits. The one
// kernel is the slower form (C5 children, 64 -> 64 with the skip: 0.694 ms against 0.620 for the two passes): the
// LayerNorm and SiLU of ~1.4 halo rows per output row sit on every tile's path between its halo DMA and its K loop.
bool preln_fused_enabled() {
  const char* e = getenv("SPCONV_PRELN_FUSED");
  return e && e[0] && e[0] != '0';
}

void subm_conv_preln(const Tensor& x_src, const Tensor* row_map, int shift, const Tensor* gamma, const Tensor* beta,
                     float eps, int pre_act, const Tensor& w, const Tensor* b, int act, const Tensor* x_skip,
                     const Tensor* skip_src, SpConvCache& c, Tensor& out) {
  REQ(x_src.dim() == 2 && (x_src.dt == BF16 || x_src.dt == F16) && w.dim() == 3, "x_src bf16/fp16 [M,Ci], w [Co,27,Ci]");
  REQ(pre_act == ACT_NONE || pre_act == ACT_SILU, "pre_act=%d", pre_act);
  REQ(!(act & EPI_F16_COMPAT), "no fp16-compatible epilogue with the fused pre-activation");
  REQ((x_skip == nullptr) == (skip_src == nullptr), "x_skip and skip_src go together");
  const int Ci = (int)x_src.size(1), Co = (int)w.size(0);
  if (row_map) {
    REQ(row_map->dt == I32 && row_map->numel() == c.N, "row_map must be int32 [%d]", c.N);
    REQ(shift >= 0 && shift < 31, "shift=%d", shift);
  } else {
    REQ(x_src.size(0) == c.N, "without a row map x_src must have the cache's %d rows", c.N);
  }
  if (gamma) REQ(gamma->dt == F32 && gamma->numel() == Ci, "gamma must be f32 [%d]", Ci);
  if (beta) REQ(beta->dt == F32 && beta->numel() == Ci, "beta must be f32 [%d]", Ci);
  if (x_skip) {
    REQ(skip_src->dt == I32 && skip_src->numel() == c.N, "skip_src must be int32 [%d]", c.N);
    REQ(x_skip->dim() == 2 && x_skip->dt == out.dt && out.dt == x_src.dt, "x_skip, x_src and out: one 16-bit dtype");
  }
  if (c.N == 0) return;
  bool fused = preln_fused_enabled() && Co == 64 && ((Ci == 64 && halo_enabled()) || (Ci == 128 && halo128_enabled()));
  if (fused) {
    const SpConvCache::HaloTable& ht =
        Ci == 64 ? c.halo_table(HaloShape<2>::B, HaloShape<2>::UM) : c.halo_table(HaloShape<4>::B, HaloShape<4>::UM);
    fused = ht.host_spills() == 0;  // the gathering kernel of spill tiles has no pre-activation prologue
  }
  if (fused) {
    const PreLN pl{gamma, beta, eps, pre_act};
    if (x_skip) {
      const SkipRes sk{x_skip, skip_src};
      const int Cin = (int)x_skip->size(1);
      REQ(Cin % 64 == 0 && Co % (Cin / 8) == 0 && ((Co / (Cin / 8)) & (Co / (Cin / 8) - 1)) == 0,
          "Cin=%d Co=%d: need Cin %% 64 == 0 and Co / (Cin/8) a power of two", Cin, Co);
      REQ((uint64_t)x_skip->bytes() <= kMaxBufferBytes && ((uintptr_t)x_skip->p % 16) == 0,
          "x_skip too large / unaligned");
      conv_impl(x_src, row_map, shift, w, b, nullptr, act, c, out, &sk, &pl);
    } else {
      conv_impl(x_src, row_map, shift, w, b, nullptr, act, c, out, nullptr, &pl);
    }
    return;
  }
  Tensor h = empty({(i64)c.N, Ci}, x_src.dt);
  gather_ln_act(x_src, row_map, shift, gamma, beta, eps, pre_act, h);
  if (x_skip) subm_conv_skip(h, w, b, act, *x_skip, *skip_src, c, out);
  else subm_conv_fused(h, w, b, nullptr, act, c, out);
}

Tensor subm_conv(const Tensor& x, const Tensor& w, const Tensor* b, SpConvCache& c) {
  REQ(x.dim() == 2 && w.dim() == 3, "x must be [N,Ci], w [Co,27,Ci]");
  Tensor y = empty({x.size(0), w.size(0)}, x.dt);
  subm_conv_fused(x, w, b, nullptr, ACT_NONE, c, y);
  return y;
}

void kernel_timing(bool on) {
  KernelTimer& t = ktimer();
  t.on = on;
  if (on) t.used = 0;
}

std::vector<float> kernel_times() {
  KernelTimer& t = ktimer();
  std::vector<float> ms;
  for (size_t i = 0; i + 1 < t.used; i += 2) {
    CK(hipEventSynchronize(t.ev[i + 1]));
    float v = 0.f;
    CK(hipEventElapsedTime(&v, t.ev[i], t.ev[i + 1]));
    ms.push_back(v);
  }
  return ms;
}
