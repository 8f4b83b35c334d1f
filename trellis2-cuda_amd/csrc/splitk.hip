// The reference's fp16 conv with a replayed FlexGEMM tile choice (B1, BK, S), rounding included: the operator of
// reference src/spconv.cu:90-175 when S > 1, where FlexGEMM's split-K kernel writes fp32 partials and ATen sums them.
//
//   split s of a B1-row block (sorted order) covers the K chunks [k0, k1) of the block's K sequence -- the block's
//   valid offsets (valid(B1), ascending) x Ci in 32-channel chunks, offset-major --
//       k0 = ceil(nk * vl * s / S) * (BK / 32),  k1 = ceil(nk * vl * (s + 1) / S) * (BK / 32),  nk = Ci / BK,
//   vl = the block's number of offsets (src/spconv.cu:98-99);
//   p[s, row, co] = sum over its chunks (fp32), plus the fp32 bias in split 0 (src/spconv.cu:144-147);
//   y = f16(((a0 + a1) + a2) + a3), a_j = sum over s = j (mod 4) of p[s] in ascending s (k_splitk_sum,
//   src/spconv.cu:152-157); then, for the fused forms, f16(silu(y)) and f16(y + residual) as the separate act_ and
//   add_ passes round (src/ops.cu:79-82, 105-113).
// With S == 1 the conv is the ordinary one with the fp16-compatible epilogue (f16(acc), then the fp16 bias add).
// Only the accumulation order inside a split's chunks differs from the reference (MFMA here, mma.sync there).
#include "spconv.h"

namespace {
constexpr uint32_t EMPTY = 0xffffffffu;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float f16r(float v) { return (float)(_Float16)v; }
__device__ __forceinline__ float silu_ieee(float v) { return v / (1.0f + expf(-v)); }

// One wavefront per (32 sorted positions, 32 output channels, split). Lane l: A row l%32 and B column l%32, 8 K
// values from (l/32)*8 of each 16-wide K step (v_mfma_f32_32x32x16_f16); result rows (i/4)*8 + (l/32)*4 + i%4.
__global__ void __launch_bounds__(64) k_split_partial(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                      const uint16_t* __restrict__ bias, const uint32_t* __restrict__ nbr,
                                                      const int32_t* __restrict__ sorted, const int32_t* __restrict__ list,
                                                      const int32_t* __restrict__ seg, int N, int Ci, int Co, int B1,
                                                      int BK, int S, float* __restrict__ part) {
  const int pos0 = blockIdx.x * 32, co0 = blockIdx.y * 32, s = blockIdx.z;
  const int lane = threadIdx.x, l32 = lane & 31, h = lane >> 5;
  const int blk = pos0 / B1;
  const int vs = seg[blk], vl = seg[blk + 1] - vs, nk = Ci / BK, cpv = Ci / 32;
  const i64 tot = (i64)nk * vl;
  const int k0 = (int)((tot * s + S - 1) / S) * (BK / 32), k1 = (int)((tot * (s + 1) + S - 1) / S) * (BK / 32);
  const int pa = pos0 + l32;
  const int row = pa < N ? sorted[pa] : -1;
  const int co = co0 + l32;
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.f;
  for (int kc = k0; kc < k1; kc++) {
    const int v = list[vs + kc / cpv], ci = (kc % cpv) * 32;
    const uint32_t src = row >= 0 ? nbr[(i64)row * 27 + v] : EMPTY;
#pragma unroll
    for (int st = 0; st < 2; st++) {
      const int k = ci + st * 16 + h * 8;
      u32x4 a = src == EMPTY ? u32x4{0, 0, 0, 0} : *(const u32x4*)(x + (i64)src * Ci + k);
      u32x4 b = *(const u32x4*)(w + ((i64)co * 27 + v) * Ci + k);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), acc,
                                                   0, 0, 0);
    }
  }
  const float bv = (bias && s == 0) ? (float)__builtin_bit_cast(_Float16, bias[co]) : 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int p = pos0 + (i / 4) * 8 + h * 4 + i % 4;
    if (p >= N) continue;
    part[((i64)s * N + sorted[p]) * Co + co] = acc[i] + bv;
  }
}

__global__ void k_split_sum(const float* __restrict__ part, int S, i64 M, const uint16_t* __restrict__ res, bool silu,
                            uint16_t* __restrict__ y) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < S; s++) a[s & 3] = a[s & 3] + part[(i64)s * M + i];
  float v = f16r(((a[0] + a[1]) + a[2]) + a[3]);
  if (silu) v = f16r(silu_ieee(v));
  if (res) v = f16r(v + (float)__builtin_bit_cast(_Float16, res[i]));
  y[i] = __builtin_bit_cast(uint16_t, (_Float16)v);
}
}  // namespace

void subm_conv_replay(const Tensor& x, const Tensor& w, const Tensor* b, const Tensor* residual, int act,
                      const SpConvCfg& cfg, SpConvCache& c, Tensor& out) {
  REQ(x.dim() == 2 && w.dim() == 3, "x must be [N,Ci], w [Co,27,Ci]");
  const int N = (int)x.size(0), Ci = (int)x.size(1), Co = (int)w.size(0);
  REQ(x.dt == F16 && w.dt == F16 && out.dt == F16 && (!b || b->dt == F16) && (!residual || residual->dt == F16),
      "the replayed fp16 conv takes fp16 x, w, out, bias and residual");
  REQ(w.size(1) == 27 && w.size(2) == Ci && N == c.N, "shapes: x [%d,%d], w [%lld,%lld,%lld], cache %d", N, Ci,
      (long long)w.size(0), (long long)w.size(1), (long long)w.size(2), c.N);
  REQ(act == ACT_NONE || act == ACT_SILU, "act=%d", act);
  REQ(cfg.B1 > 0 && cfg.B1 % 32 == 0 && cfg.BK > 0 && cfg.BK % 32 == 0 && Ci % cfg.BK == 0 && cfg.S >= 1 &&
          cfg.S <= 64,
      "cfg B1=%d BK=%d S=%d with Ci=%d (B1, BK multiples of 32, Ci %% BK == 0, 1 <= S <= 64)", cfg.B1, cfg.BK, cfg.S,
      Ci);
  REQ(Co % 32 == 0, "Co=%d must be a multiple of 32", Co);
  REQ(((uintptr_t)x.p | (uintptr_t)w.p) % 16 == 0, "x and w must be 16-byte aligned");
  REQ(out.dim() == 2 && out.size(0) == N && out.size(1) == Co, "out must be [N,Co]");
  if (residual) REQ(residual->numel() == (i64)N * Co, "residual must be [N,Co]");
  if (cfg.S == 1) {  // FlexGEMM's unsplit kernel: f16(acc), then the fp16 bias add
    subm_conv_fused(x, w, b, residual, act | EPI_F16_COMPAT, c, out);
    return;
  }
  if (N == 0) return;
  const auto& vl = c.valid(cfg.B1);
  Tensor part = empty({(i64)cfg.S, N, Co}, F32);
  hipStream_t s = stream();
  k_split_partial<<<dim3(cdiv(N, 32), Co / 32, cfg.S), 64, 0, s>>>(
      x.ptr<uint16_t>(), w.ptr<uint16_t>(), b ? b->ptr<uint16_t>() : nullptr, c.nbr.ptr<uint32_t>(),
      c.sorted.ptr<int32_t>(), vl.first.ptr<int32_t>(), vl.second.ptr<int32_t>(), N, Ci, Co, cfg.B1, cfg.BK, cfg.S,
      part.ptr<float>());
  const i64 M = (i64)N * Co;
  k_split_sum<<<cdiv(M, 256), 256, 0, s>>>(part.ptr<float>(), cfg.S, M, residual ? residual->ptr<uint16_t>() : nullptr,
                                           act == ACT_SILU, out.ptr<uint16_t>());
  CK(hipGetLastError());
}
