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
#include "spconv.h"

namespace {
constexpr uint32_t EMPTY = 0xffffffffu;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

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
__device__ __forceinline__ f32x16 mfma32(uint4 a, uint4 b, f32x16 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

struct ConvArgs {
  const uint16_t* x;
  const uint16_t* w;
  const float* bias;
  const void* res;
  void* out;
  const uint32_t* nbr;
  const int32_t* order;
  const uint32_t* code;
  int N, Ci, Co, res_dt, out_dt, act;
  int tiles_m, tiles_n, grid;
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

  uint4 ra[AL], rb[BL];
  auto gload = [&]() {
    const int k0 = kc * KC;
#pragma unroll
    for (int j = 0; j < AL; j++) {
      int pc = (tid + j * NT) % PC;
      ra[j] = srcA[j] == EMPTY ? make_uint4(0, 0, 0, 0)
                               : *(const uint4*)(a.x + (i64)srcA[j] * Ci + k0 + pc * 8);
    }
#pragma unroll
    for (int j = 0; j < BL; j++) {
      int q = tid + j * NT, r = q / PC, pc = q % PC;
      rb[j] = *(const uint4*)(a.w + ((i64)(co0 + r) * 27 + cv) * Ci + k0 + pc * 8);
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
      *(uint4*)&As[buf][(q / PC) * LD + (q % PC) * 8] = ra[j];
    }
#pragma unroll
    for (int j = 0; j < BL; j++) {
      int q = tid + j * NT;
      *(uint4*)&Bs[buf][(q / PC) * LD + (q % PC) * 8] = rb[j];
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
      uint4 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; i++)
        fa[i] = *(const uint4*)&As[buf][(wm * WTM + i * 32 + (lane & 31)) * LD + ks * 16 + (lane >> 5) * 8];
#pragma unroll
      for (int j = 0; j < TN; j++)
        fb[j] = *(const uint4*)&Bs[buf][(wn * WTN + j * 32 + (lane & 31)) * LD + ks * 16 + (lane >> 5) * 8];
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
        float v = acc[i][j][e] + bv;
        if (a.act == ACT_SILU) v = v / (1.0f + expf(-v));
        if (a.res) v += load_elem(a.res, o, a.res_dt);
        store_elem(a.out, o, a.out_dt, v);
      }
    }
  }
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
  // Fixed tiles per channel width (no autotune): BM = 128 sorted rows per tile.
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

void subm_conv_fused(const Tensor& x, const Tensor& w, const Tensor* b, const Tensor* residual, int act,
                     SpConvCache& c, Tensor& out) {
  REQ(x.dim() == 2 && w.dim() == 3, "x must be [N,Ci], w [Co,27,Ci]");
  const int N = (int)x.size(0), Ci = (int)x.size(1), Co = (int)w.size(0);
  REQ((x.dt == BF16 || x.dt == F16) && w.dt == x.dt, "x and w must both be bf16 or both fp16 (x %s, w %s)",
      dname(x.dt), dname(w.dt));
  REQ(w.size(1) == 27 && w.size(2) == Ci, "w must be [Co,27,%d]", Ci);
  REQ(Ci > 0 && Ci % 32 == 0, "Ci=%d must be a multiple of 32", Ci);
  REQ(Co > 0 && Co % 64 == 0, "Co=%d must be a multiple of 64", Co);
  REQ(N == c.N, "x has %d rows, neighbour cache %d", N, c.N);
  REQ(act == ACT_NONE || act == ACT_SILU, "act=%d", act);
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
  const Tensor& code = c.block_masks(cfg.B1);
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
  a.code = code.ptr<uint32_t>();
  a.N = N;
  a.Ci = Ci;
  a.Co = Co;
  a.act = act;
  if (x.dt == F16) dispatch<true>(cfg, a);
  else dispatch<false>(cfg, a);
  CK(hipGetLastError());
}

Tensor subm_conv(const Tensor& x, const Tensor& w, const Tensor* b, SpConvCache& c) {
  REQ(x.dim() == 2 && w.dim() == 3, "x must be [N,Ci], w [Co,27,Ci]");
  Tensor y = empty({x.size(0), w.size(0)}, x.dt);
  subm_conv_fused(x, w, b, nullptr, ACT_NONE, c, y);
  return y;
}
