// A decoder-shaped C++ caller of the sparse-conv API, compiled against trellis2-cuda_amd/csrc/spconv.h with the
// reference's signatures and run on the GPU by tests/test_cxx_caller.py. The calls mirror the reference's callers:
//   SDecoder::conv  -> subm_conv(x, w.view({Co, 27, Ci}), &b, c)                       (src/sdec.cu:15-18)
//   level caches    -> std::make_shared<SpConvCache>(build_neighbors(coords, 4096, ...)) (src/sdec.cu:55, 92)
//   schedule        -> spconv_cfg(N, Ci, Co) and c.valid(B1)                           (src/spconv.cu:160-175)
// The conv output is checked against a double-precision gather-accumulate on the host over the same fp16 inputs;
// the valid lists against the block ORs of the cache's own masks. Prints "ok" and exits 0 on success.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <random>
#include <tuple>
#include <vector>

#include "spconv.h"

static uint16_t to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
static float from_f16(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

static int run(int Ci, int Co) {
  // sphere shell of radius 6 in a 16^3 grid, rows in x-major order
  std::vector<int32_t> cc;
  for (int x = 0; x < 16; x++)
    for (int y = 0; y < 16; y++)
      for (int z = 0; z < 16; z++) {
        const double d = std::sqrt((x - 7.5) * (x - 7.5) + (y - 7.5) * (y - 7.5) + (z - 7.5) * (z - 7.5));
        if (std::fabs(d - 6.0) <= 1.0) cc.insert(cc.end(), {0, x, y, z});
      }
  const int N = (int)cc.size() / 4;
  Tensor coords = from_host(cc.data(), {N, 4}, I32);
  auto nb = std::make_shared<SpConvCache>(build_neighbors(coords, 1 << 12, 1 << 12, 1 << 12));
  SpConvCache& c = *nb;
  if (c.N != N) return fprintf(stderr, "cache N %d != %d\n", c.N, N), 1;

  std::mt19937 rng(Ci * 131 + Co);
  std::normal_distribution<float> nd(0.f, 1.f);
  std::vector<uint16_t> hx((size_t)N * Ci), hw((size_t)Co * 27 * Ci), hb(Co);
  for (auto& v : hx) v = to_f16(nd(rng));
  for (auto& v : hw) v = to_f16(nd(rng) / std::sqrt(27.f * Ci));
  for (auto& v : hb) v = to_f16(0.1f * nd(rng));
  Tensor x = from_host(hx.data(), {N, Ci}, F16);
  Tensor w5 = from_host(hw.data(), {Co, 3, 3, 3, Ci}, F16);  // the checkpoint layout
  Tensor b = from_host(hb.data(), {Co}, F16);
  Tensor y = subm_conv(x, w5.view({w5.size(0), 27, w5.size(4)}), &b, c);
  if (y.dt != F16 || y.size(0) != N || y.size(1) != Co) return fprintf(stderr, "output shape/dtype\n"), 1;

  const SpConvCfg cfg = spconv_cfg(N, Ci, Co);
  const auto& lv = c.valid(cfg.B1);
  const auto nbr = to_host_vec<uint32_t>(c.nbr);
  const auto gray = to_host_vec<int32_t>(c.gray);
  const auto srt = to_host_vec<int32_t>(c.sorted);
  const auto seg = to_host_vec<int32_t>(lv.second);
  const auto lst = to_host_vec<int32_t>(lv.first);
  const auto hy = to_host_vec<uint16_t>(y);
  const int nblk = (N + cfg.B1 - 1) / cfg.B1;
  if ((int)seg.size() != nblk + 1 || seg[0] != 0) return fprintf(stderr, "seg size\n"), 1;
  for (int k = 0; k < nblk; k++) {
    uint32_t m = 0;
    for (int r = k * cfg.B1; r < std::min(N, (k + 1) * cfg.B1); r++) m |= (uint32_t)gray[srt[r]];
    int p = seg[k];
    for (int v = 0; v < 27; v++)
      if ((m >> v) & 1u) {
        if (p >= seg[k + 1] || lst[p] != v) return fprintf(stderr, "valid list of block %d\n", k), 1;
        p++;
      }
    if (p != seg[k + 1]) return fprintf(stderr, "valid list length of block %d\n", k), 1;
  }
  double num = 0, den = 0, mx = 0;
  for (int i = 0; i < N; i++)
    for (int o = 0; o < Co; o++) {
      double s = from_f16(hb[o]);
      for (int v = 0; v < 27; v++) {
        const uint32_t j = nbr[(size_t)i * 27 + v];
        if (j == 0xffffffffu) continue;
        for (int k = 0; k < Ci; k++)
          s += (double)from_f16(hx[(size_t)j * Ci + k]) * from_f16(hw[((size_t)o * 27 + v) * Ci + k]);
      }
      const double e = from_f16(hy[(size_t)i * Co + o]) - s;
      num += e * e;
      den += s * s;
      mx = std::max(mx, std::fabs(e));
    }
  const double rel = std::sqrt(num / den);
  printf("Ci=%d Co=%d N=%d B1=%d rel-L2 %.2e max-abs %.2e\n", Ci, Co, N, cfg.B1, rel, mx);
  return rel <= 1e-3 && mx <= 2e-2 ? 0 : 1;
}

int main() {
  try {
    for (auto [ci, co] : {std::make_tuple(64, 64), std::make_tuple(128, 64), std::make_tuple(256, 256)})
      if (run(ci, co)) return 1;
  } catch (const std::exception& e) {
    fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
  printf("ok\n");
  return 0;
}
