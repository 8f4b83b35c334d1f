// LayerNorm + activation of one feature row held by a group of LPR consecutive lanes, 8 channels per lane per
// 16-byte chunk (CH chunks per lane): the reference's layer_norm (src/ops.cu:30-75: fp32 statistics, mean then the
// centred variance, affine) followed by act_ SILU (src/ops.cu:79-82), with one rounding to the output type.
// gather_ln_act and the halo conv's pre-activation prologue both use these, so the two give the same bits.
#pragma once
#include <hip/hip_runtime.h>

// mean and 1/sqrt(var + eps) of the row whose values this lane holds in v; every lane of the group must call it
// (the sums reduce across the group with xor shuffles)
template <int LPR, int CH>
__device__ __forceinline__ void ln_stats(const float (&v)[CH][8], int C, float eps, float& mean, float& rstd) {
#pragma clang fp contract(off)
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < CH; k++)
#pragma unroll
    for (int j = 0; j < 8; j++) s += v[k][j];
#pragma unroll
  for (int d = 1; d < LPR; d <<= 1) s += __shfl_xor(s, d, 64);
  mean = s / (float)C;
  float q2 = 0.f;
#pragma unroll
  for (int k = 0; k < CH; k++)
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float d = v[k][j] - mean;
      q2 += d * d;
    }
#pragma unroll
  for (int d = 1; d < LPR; d <<= 1) q2 += __shfl_xor(q2, d, 64);
  rstd = rsqrtf(q2 / (float)C + eps);
}

// o = act((v - mean) * rstd * gamma + beta) for 8 channels; g8 / b8 point at those channels' affine terms (or null)
__device__ __forceinline__ void ln_out8(const float (&v)[8], float mean, float rstd, const float* g8, const float* b8,
                                        int silu, float (&o)[8]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int j = 0; j < 8; j++) {
    float t = (v[j] - mean) * rstd;
    if (g8) t *= g8[j];
    if (b8) t += b8[j];
    if (silu) t = t * __builtin_amdgcn_rcpf(1.0f + __expf(-t));
    o[j] = t;
  }
}

// 16-bit storage <-> fp32 (bf16 or fp16 by flag), 2 values per 32-bit word, round to nearest even
typedef __bf16 lnact_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 lnact_f16x2 __attribute__((ext_vector_type(2)));
typedef float lnact_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float lnact_h2f(uint16_t h, bool bf) {
  return bf ? __uint_as_float((uint32_t)h << 16) : (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint32_t lnact_pack2(float lo, float hi, bool bf) {
  return bf ? __builtin_bit_cast(uint32_t, __builtin_convertvector(lnact_f32x2{lo, hi}, lnact_bf16x2))
            : __builtin_bit_cast(uint32_t, __builtin_convertvector(lnact_f32x2{lo, hi}, lnact_f16x2));
}
