// (Gather +) LayerNorm + SiLU in one pass: the pre-activation of a decoder upsample block's second conv (reference
// src/sdec.cu:78-83: k_gather_rows, then layer_norm (src/ops.cu:30-75, fp32 statistics), then act_ SILU), which
// the reference runs as separate passes with a rounding after each.
//   y[i] = act(LN(x_src[row_map[i] >> shift]) * gamma + beta), statistics in fp32, one rounding to the output dtype.
// Without a row map it is the block's first pre-activation, LN(x) with the norm1 affine then SiLU (src/sdec.cu:72-73).
// Lanes per row: C/8 (8 channels per lane, one 16-byte load) up to 64, so a 64-channel row is 8 lanes and a
// wavefront handles 8 rows; the row sums reduce with lane shuffles inside the row's lane group.
#include "lnact.h"
#include "spconv.h"

namespace {
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kOOR = 0xffff0000u;

__device__ __forceinline__ float h2f(uint16_t h, bool bf) { return lnact_h2f(h, bf); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi, bool bf) { return lnact_pack2(lo, hi, bf); }

// LPR lanes per row, CH = C / (8 * LPR) 16-byte chunks per lane
template <int LPR, int CH>
__global__ void __launch_bounds__(256) k_gather_ln_act(const uint16_t* __restrict__ x, uint32_t x_bytes, int C,
                                                       const int32_t* __restrict__ row_map, int shift, i64 m,
                                                       const float* __restrict__ gamma, const float* __restrict__ beta,
                                                       float eps, int silu, bool bf, i64 n, uint16_t* __restrict__ y) {
  const i64 gid = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  const i64 i = gid / LPR;
  const int sub = (int)(gid % LPR);
  const bool live = i < n;
  const uint32_t r = !live ? 0xffffffffu : row_map ? (uint32_t)row_map[i] >> shift : (uint32_t)i;
  const bool ok = live && r < (uint64_t)m;  // rows outside the source read as zeros (LN of zeros is beta)
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), 0, (int)x_bytes,
                                                                      0x00020000);
  float v[CH][8];
#pragma unroll
  for (int k = 0; k < CH; k++) {
    const int c8 = (k * LPR + sub) * 8;
    const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? (r * (uint32_t)C + c8) * 2u : kOOR, 0, 0);
#pragma unroll
    for (int j = 0; j < 8; j++) v[k][j] = h2f((uint16_t)(q[j >> 1] >> ((j & 1) * 16)), bf);
  }
  float mean, rstd;
  ln_stats<LPR, CH>(v, C, eps, mean, rstd);
  if (!live) return;
#pragma unroll
  for (int k = 0; k < CH; k++) {
    const int c8 = (k * LPR + sub) * 8;
    float o[8];
    ln_out8(v[k], mean, rstd, gamma ? gamma + c8 : nullptr, beta ? beta + c8 : nullptr, silu, o);
    *(u32x4*)&y[i * C + c8] = u32x4{pack2(o[0], o[1], bf), pack2(o[2], o[3], bf), pack2(o[4], o[5], bf),
                                    pack2(o[6], o[7], bf)};
  }
}
}  // namespace

void gather_ln_act(const Tensor& x_src, const Tensor* row_map, int shift, const Tensor* gamma, const Tensor* beta,
                   float eps, int act, Tensor& out) {
  REQ(x_src.dim() == 2 && (x_src.dt == BF16 || x_src.dt == F16), "x_src must be bf16/fp16 [M,C]");
  const int C = (int)x_src.size(1);
  const i64 M = x_src.size(0), n = row_map ? row_map->numel() : M;
  REQ(C >= 8 && C <= 4096 && C % 8 == 0 && ((C / 8) & (C / 8 - 1)) == 0, "C=%d: 8 times a power of two, at most 4096",
      C);
  if (row_map) REQ(row_map->dt == I32 && row_map->dim() == 1, "row_map must be int32 [N]");
  REQ(shift >= 0 && shift < 31, "shift=%d", shift);
  REQ(act == ACT_NONE || act == ACT_SILU, "act=%d", act);
  REQ(out.dim() == 2 && out.size(0) == n && out.size(1) == C && out.dt == x_src.dt, "out must be [%lld,%d] like x",
      (long long)n, C);
  if (gamma) REQ(gamma->dt == F32 && gamma->numel() == C, "gamma must be f32 [C]");
  if (beta) REQ(beta->dt == F32 && beta->numel() == C, "beta must be f32 [C]");
  REQ((uint64_t)M * C * 2 <= 0xfffe0000ull, "x_src larger than 4 GiB");
  if (n == 0) return;
  const bool bf = x_src.dt == BF16;
  const float* g = gamma ? gamma->ptr<float>() : nullptr;
  const float* b = beta ? beta->ptr<float>() : nullptr;
  const uint32_t xb = (uint32_t)(M * C * 2);
  auto go = [&](auto L, auto K) {
    constexpr int LPR = decltype(L)::value, CH = decltype(K)::value;
    const i64 threads = n * LPR;
    k_gather_ln_act<LPR, CH><<<cdiv(threads, 256), 256, 0, stream()>>>(
        x_src.ptr<uint16_t>(), xb, C, row_map ? row_map->ptr<int32_t>() : nullptr, shift, M, g, b, eps, act, bf, n, out.ptr<uint16_t>());
  };
  using std::integral_constant;
  switch (C / 8) {
    case 1: go(integral_constant<int, 1>{}, integral_constant<int, 1>{}); break;
    case 2: go(integral_constant<int, 2>{}, integral_constant<int, 1>{}); break;
    case 4: go(integral_constant<int, 4>{}, integral_constant<int, 1>{}); break;
    case 8: go(integral_constant<int, 8>{}, integral_constant<int, 1>{}); break;
    case 16: go(integral_constant<int, 16>{}, integral_constant<int, 1>{}); break;
    case 32: go(integral_constant<int, 32>{}, integral_constant<int, 1>{}); break;
    case 64: go(integral_constant<int, 64>{}, integral_constant<int, 1>{}); break;
    case 128: go(integral_constant<int, 64>{}, integral_constant<int, 2>{}); break;
    case 256: go(integral_constant<int, 64>{}, integral_constant<int, 4>{}); break;
    case 512: go(integral_constant<int, 64>{}, integral_constant<int, 8>{}); break;
    default: REQ(false, "C=%d not supported", C);
  }
  CK(hipGetLastError());
}

// Skip connection of the upsample block (reference k_add_skip, src/sdec.cu:38-43, launched at :84), in place:
//   h[i, c] = round(h[i, c] + x[src[i] >> 3, (src[i] & 7) * Cs + c / rep]),  Cs = Cin / 8, rep = Co / Cs,
// i.e. h += repeat_interleave(C2S(x), rep, dim=1), the sum taken in fp32 and rounded once -- the reference's
// arithmetic, so the result is bit-identical. One thread per 8 channels of a child row (one 16-byte load and store of
// h); the x elements come from one 16-byte load when rep = 1, else 8 / rep (or one) 2-byte loads.
namespace {
template <int REP>
__global__ void __launch_bounds__(256) k_add_skip8(uint16_t* __restrict__ h, const uint16_t* __restrict__ x,
                                                   const int32_t* __restrict__ src, i64 m, i64 n, int Co, int Cin,
                                                   int rep, bool bf) {
  const i64 t = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  const int per = Co / 8;
  const i64 i = t / per;
  if (i >= m) return;
  const int c0 = (int)(t % per) * 8;
  const int s = src[i], p = s >> 3, Cs = Cin / 8;
  if ((uint32_t)s >= (uint64_t)n * 8) return;  // a map entry outside x leaves the row unchanged
  const uint16_t* xr = x + (i64)p * Cin + (s & 7) * Cs;
  u32x4* hp = (u32x4*)&h[i * Co + c0];
  u32x4 hv = *hp;
  float xv[8];
  if (REP == 1) {
    const u32x4 q = *(const u32x4*)&xr[c0];
#pragma unroll
    for (int j = 0; j < 8; j++) xv[j] = h2f((uint16_t)(q[j >> 1] >> ((j & 1) * 16)), bf);
  } else {
#pragma unroll
    for (int j = 0; j < 8; j++) xv[j] = h2f(xr[(c0 + j) / rep], bf);
  }
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; k++)
    o[k] = pack2(h2f((uint16_t)hv[k], bf) + xv[2 * k], h2f((uint16_t)(hv[k] >> 16), bf) + xv[2 * k + 1], bf);
  *hp = o;
}
}  // namespace

void add_skip(Tensor& h, const Tensor& x, const Tensor& src) {
  REQ(h.dim() == 2 && x.dim() == 2 && h.dt == x.dt && (h.dt == BF16 || h.dt == F16), "h, x: bf16/fp16 [m,Co], [n,Cin]");
  REQ(src.dt == I32 && src.numel() == h.size(0), "src must be int32 [m]");
  const i64 m = h.size(0), n = x.size(0);
  const int Co = (int)h.size(1), Cin = (int)x.size(1);
  REQ(Cin % 8 == 0 && Co % (Cin / 8) == 0 && Co % 8 == 0, "Co=%d Cin=%d: need Cin %% 8 == 0, Co a multiple of "
      "Cin/8 and of 8", Co, Cin);
  if (m == 0) return;
  REQ(n > 0, "x has no rows");
  REQ(((uintptr_t)h.p | (uintptr_t)x.p) % 16 == 0, "h and x must be 16-byte aligned");
  const int rep = Co / (Cin / 8);
  const i64 threads = m * (Co / 8);
  const bool bf = h.dt == BF16;
  if (rep == 1)
    k_add_skip8<1><<<cdiv(threads, 256), 256, 0, stream()>>>(h.ptr<uint16_t>(), x.ptr<uint16_t>(),
                                                             src.ptr<int32_t>(), m, n, Co, Cin, rep, bf);
  else
    k_add_skip8<0><<<cdiv(threads, 256), 256, 0, stream()>>>(h.ptr<uint16_t>(), x.ptr<uint16_t>(),
                                                             src.ptr<int32_t>(), m, n, Co, Cin, rep, bf);
  CK(hipGetLastError());
}
