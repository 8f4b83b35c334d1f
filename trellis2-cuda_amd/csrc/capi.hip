// extern "C" boundary over the C++ API, with the reference's embedding convention (apps/t2lib.cu:1-23):
// 0 / -1 + last error string, all calls serialized by one mutex, exceptions never cross the ABI.
#include <algorithm>
#include <exception>
#include <mutex>

#include "../../include/spconv_amd.h"
#include "spconv.h"

#define SPC_API extern "C" __attribute__((visibility("default")))

struct spc_cache {
  SpConvCache c;
};

namespace {
std::mutex mu;
std::string last_error;

template <class F>
int guarded(F&& f) {
  std::lock_guard<std::mutex> lk(mu);
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    last_error = e.what();
  } catch (...) {
    last_error = "unknown error";
  }
  return -1;
}
DT float_dt(int d, const char* what) {
  REQ(d == SPC_F32 || d == SPC_F16 || d == SPC_BF16, "%s dtype code %d", what, d);
  return (DT)d;
}
}  // namespace

SPC_API const char* spc_last_error(void) { return last_error.c_str(); }

SPC_API int spc_set_stream(void* s) {
  return guarded([&] { set_stream((hipStream_t)s); });
}

SPC_API int spc_build_neighbors(const int32_t* coords, int64_t n, int W, int H, int D, spc_cache** out) {
  return guarded([&] {
    REQ(out, "out is null");
    REQ(n >= 0 && (n == 0 || coords), "coords null or n < 0");
    auto h = std::make_unique<spc_cache>();
    h->c = build_neighbors(borrow(coords, {n, 4}, I32), W, H, D);
    *out = h.release();
  });
}

SPC_API int spc_build_neighbors_ex(const int32_t* coords, int64_t n, int W, int H, int D, int flags,
                                   spc_cache** out) {
  return guarded([&] {
    REQ(out, "out is null");
    REQ(n >= 0 && (n == 0 || coords), "coords null or n < 0");
    REQ((flags & ~SPC_KEEP_HASH) == 0, "unknown flags %d", flags);
    auto h = std::make_unique<spc_cache>();
    h->c = build_neighbors(borrow(coords, {n, 4}, I32), W, H, D, (flags & SPC_KEEP_HASH) != 0);
    *out = h.release();
  });
}

SPC_API int spc_cache_lookup(const spc_cache* c, const int32_t* query, int64_t m, int32_t* rows) {
  return guarded([&] {
    REQ(c, "cache is null");
    REQ(m >= 0 && (m == 0 || (query && rows)), "null query/rows or m < 0");
    Tensor tr = borrow(rows, {m}, I32);
    lookup(c->c, borrow(query, {m, 4}, I32), tr);
  });
}

SPC_API int spc_fdg_quads(const spc_cache* c, const float* h, int32_t* quad, int32_t* ok) {
  return guarded([&] {
    REQ(c, "cache is null");
    const i64 n = c->c.N;
    REQ(n == 0 || (h && quad && ok), "null h/quad/ok");
    Tensor tq = borrow(quad, {3 * n, 4}, I32), to = borrow(ok, {3 * n}, I32);
    fdg_quads(c->c, borrow(h, {n, 7}, F32), tq, to);
  });
}

SPC_API int spc_cache_free(spc_cache* c) {
  return guarded([&] { delete c; });
}

SPC_API int spc_cache_info(const spc_cache* c, int64_t* n, const uint32_t** nbr, const int32_t** gray,
                           const int32_t** sorted) {
  return guarded([&] {
    REQ(c, "cache is null");
    if (n) *n = c->c.N;
    if (nbr) *nbr = c->c.nbr.ptr<uint32_t>();
    if (gray) *gray = c->c.gray.ptr<int32_t>();
    if (sorted) *sorted = c->c.sorted.ptr<int32_t>();
  });
}

SPC_API int spc_cache_valid(spc_cache* c, int B1, const int32_t** list, const int32_t** seg, int64_t* L) {
  return guarded([&] {
    REQ(c, "cache is null");
    auto& v = c->c.valid(B1);
    if (list) *list = v.first.ptr<int32_t>();
    if (seg) *seg = v.second.ptr<int32_t>();
    if (L) {
      i64 nb = cdiv(c->c.N, B1);
      *L = (int64_t)to_host_vec<int32_t>(v.second.slice0(nb, nb + 1))[0];
    }
  });
}

SPC_API int spc_conv_cfg(int64_t N, int Ci, int Co, int* B1, int* BK, int* S) {
  return guarded([&] {
    SpConvCfg k = spconv_cfg((int)N, Ci, Co);
    if (B1) *B1 = k.B1;
    if (BK) *BK = k.BK;
    if (S) *S = k.S;
  });
}

SPC_API int spc_subm_conv_fused(const void* x, const void* w, const void* b, const void* residual, int dtype,
                                int b_dtype, int res_dtype, int out_dtype, int act, int64_t N, int Ci, int Co,
                                spc_cache* c, void* out) {
  return guarded([&] {
    REQ(c, "cache is null");
    REQ(N >= 0 && Ci > 0 && Co > 0, "N=%lld Ci=%d Co=%d", (long long)N, Ci, Co);
    REQ(N == 0 || (x && w && out), "null x/w/out");
    DT dt = float_dt(dtype, "x/w");
    REQ(dt != F32, "x/w must be fp16 or bf16");
    Tensor tx = borrow(x, {N, Ci}, dt), tw = borrow(w, {Co, 27, Ci}, dt);
    Tensor tb, tr, to = borrow(out, {N, Co}, float_dt(out_dtype, "out"));
    if (b) tb = borrow(b, {Co}, float_dt(b_dtype, "bias"));
    if (residual) tr = borrow(residual, {N, Co}, float_dt(res_dtype, "residual"));
    if (N == 0) to.sh = {0, Co};
    subm_conv_fused(tx, tw, b ? &tb : nullptr, residual ? &tr : nullptr, act, c->c, to);
  });
}

SPC_API int spc_subm_conv_gathered(const void* x_src, int64_t M, const int32_t* row_map, int shift, const void* w,
                                   const void* b, const void* residual, int dtype, int b_dtype, int res_dtype,
                                   int out_dtype, int act, int64_t N, int Ci, int Co, spc_cache* c, void* out) {
  return guarded([&] {
    REQ(c, "cache is null");
    REQ(N == c->c.N, "N=%lld but the cache has %d rows", (long long)N, c->c.N);
    REQ(M >= 0 && Ci > 0 && Co > 0, "M=%lld Ci=%d Co=%d", (long long)M, Ci, Co);
    REQ(N == 0 || (x_src && row_map && w && out && M > 0), "null x_src/row_map/w/out or M = 0");
    DT dt = float_dt(dtype, "x/w");
    REQ(dt != F32, "x/w must be fp16 or bf16");
    Tensor tx = borrow(x_src, {M, Ci}, dt), tw = borrow(w, {Co, 27, Ci}, dt), tm = borrow(row_map, {N}, I32);
    Tensor tb, tr, to = borrow(out, {N, Co}, float_dt(out_dtype, "out"));
    if (b) tb = borrow(b, {Co}, float_dt(b_dtype, "bias"));
    if (residual) tr = borrow(residual, {N, Co}, float_dt(res_dtype, "residual"));
    if (N == 0) return;
    subm_conv_gathered(tx, tm, shift, tw, b ? &tb : nullptr, residual ? &tr : nullptr, act, c->c, to);
  });
}

SPC_API int spc_gather_ln_act(const void* x_src, int64_t M, int C, const int32_t* row_map, int shift,
                              const float* gamma, const float* beta, float eps, int act, int dtype, int64_t N,
                              void* out) {
  return guarded([&] {
    REQ(M >= 0 && N >= 0 && C > 0, "M=%lld N=%lld C=%d", (long long)M, (long long)N, C);
    DT dt = float_dt(dtype, "x");
    REQ(dt != F32, "x must be fp16 or bf16");
    if (N == 0) return;
    REQ(row_map || N == M, "without a row map N (%lld) must equal M (%lld)", (long long)N, (long long)M);
    REQ(x_src && out && M > 0, "null x_src/out or M = 0");
    Tensor tx = borrow(x_src, {M, C}, dt), to = borrow(out, {N, C}, dt), tm, tg, tb;
    if (row_map) tm = borrow(row_map, {N}, I32);
    if (gamma) tg = borrow(gamma, {C}, F32);
    if (beta) tb = borrow(beta, {C}, F32);
    gather_ln_act(tx, row_map ? &tm : nullptr, shift, gamma ? &tg : nullptr, beta ? &tb : nullptr, eps, act, to);
  });
}

SPC_API int spc_convnext_mlp(const void* h, const void* x, const void* gamma, const void* beta, float eps,
                             const void* w1, const void* b1, const void* w2, const void* b2, int dtype,
                             int param_dtype, int64_t N, int C, void* y) {
  return guarded([&] {
    REQ(N >= 0 && C > 0, "N=%lld C=%d", (long long)N, C);
    DT dt = float_dt(dtype, "h/x/w"), pdt = float_dt(param_dtype, "gamma/beta/b1/b2");
    REQ(dt != F32, "h/x/w must be fp16 or bf16");
    if (N == 0) return;
    REQ(h && x && w1 && w2 && y, "null h/x/w1/w2/y");
    Tensor th = borrow(h, {N, C}, dt), tx = borrow(x, {N, C}, dt), ty = borrow(y, {N, C}, dt);
    Tensor tw1 = borrow(w1, {4 * (i64)C, C}, dt), tw2 = borrow(w2, {C, 4 * (i64)C}, dt), tg, tb, tb1, tb2;
    if (gamma) tg = borrow(gamma, {C}, pdt);
    if (beta) tb = borrow(beta, {C}, pdt);
    if (b1) tb1 = borrow(b1, {4 * (i64)C}, pdt);
    if (b2) tb2 = borrow(b2, {C}, pdt);
    convnext_mlp(th, tx, gamma ? &tg : nullptr, beta ? &tb : nullptr, eps, tw1, b1 ? &tb1 : nullptr, tw2,
                 b2 ? &tb2 : nullptr, ty);
  });
}

SPC_API int spc_subm_conv_skip(const void* x, const void* w, const void* b, int dtype, int b_dtype, int act,
                               const void* x_skip, int64_t n_skip, int Cin, const int32_t* src, int64_t N, int Ci,
                               int Co, spc_cache* c, void* out) {
  return guarded([&] {
    REQ(c, "cache is null");
    REQ(N == c->c.N, "N=%lld but the cache has %d rows", (long long)N, c->c.N);
    REQ(n_skip >= 0 && Cin > 0 && Ci > 0 && Co > 0, "n_skip=%lld Cin=%d Ci=%d Co=%d", (long long)n_skip, Cin, Ci, Co);
    DT dt = float_dt(dtype, "x/w/x_skip/out");
    REQ(dt != F32, "x/w/x_skip/out must be fp16 or bf16");
    if (N == 0) return;
    REQ(x && w && x_skip && src && out && n_skip > 0, "null x/w/x_skip/src/out or n_skip = 0");
    Tensor tx = borrow(x, {N, Ci}, dt), tw = borrow(w, {Co, 27, Ci}, dt), ts = borrow(x_skip, {n_skip, Cin}, dt);
    Tensor tsrc = borrow(src, {N}, I32), to = borrow(out, {N, Co}, dt), tb;
    if (b) tb = borrow(b, {Co}, float_dt(b_dtype, "bias"));
    subm_conv_skip(tx, tw, b ? &tb : nullptr, act, ts, tsrc, c->c, to);
  });
}

SPC_API int spc_subm_conv_preln(const void* x_src, int64_t M, const int32_t* row_map, int shift, const float* gamma,
                                const float* beta, float eps, int pre_act, const void* w, const void* b, int dtype,
                                int b_dtype, int act, const void* x_skip, int64_t n_skip, int Cin,
                                const int32_t* skip_src, int64_t N, int Ci, int Co, spc_cache* c, void* out) {
  return guarded([&] {
    REQ(c, "cache is null");
    REQ(N == c->c.N, "N=%lld but the cache has %d rows", (long long)N, c->c.N);
    REQ(M >= 0 && Ci > 0 && Co > 0 && n_skip >= 0, "M=%lld Ci=%d Co=%d n_skip=%lld", (long long)M, Ci, Co,
        (long long)n_skip);
    REQ((x_skip == nullptr) == (skip_src == nullptr), "x_skip and skip_src go together");
    DT dt = float_dt(dtype, "x_src/w/x_skip/out");
    REQ(dt != F32, "x_src/w/x_skip/out must be fp16 or bf16");
    if (N == 0) return;
    REQ(row_map || M == N, "without a row map M (%lld) must equal N (%lld)", (long long)M, (long long)N);
    REQ(x_src && w && out && M > 0, "null x_src/w/out or M = 0");
    REQ(!x_skip || (Cin > 0 && n_skip > 0), "x_skip needs Cin > 0 and n_skip > 0");
    Tensor tx = borrow(x_src, {M, Ci}, dt), tw = borrow(w, {Co, 27, Ci}, dt), to = borrow(out, {N, Co}, dt);
    Tensor tm, tg, tbt, tb, ts, tsrc;
    if (row_map) tm = borrow(row_map, {N}, I32);
    if (gamma) tg = borrow(gamma, {Ci}, F32);
    if (beta) tbt = borrow(beta, {Ci}, F32);
    if (b) tb = borrow(b, {Co}, float_dt(b_dtype, "bias"));
    if (x_skip) {
      ts = borrow(x_skip, {n_skip, Cin}, dt);
      tsrc = borrow(skip_src, {N}, I32);
    }
    subm_conv_preln(tx, row_map ? &tm : nullptr, shift, gamma ? &tg : nullptr, beta ? &tbt : nullptr, eps, pre_act,
                    tw, b ? &tb : nullptr, act, x_skip ? &ts : nullptr, x_skip ? &tsrc : nullptr, c->c, to);
  });
}

SPC_API int spc_add_skip(void* h, const void* x, const int32_t* src, int64_t m, int Co, int64_t n, int Cin,
                         int dtype) {
  return guarded([&] {
    REQ(m >= 0 && n >= 0 && Co > 0 && Cin > 0, "m=%lld n=%lld Co=%d Cin=%d", (long long)m, (long long)n, Co, Cin);
    DT dt = float_dt(dtype, "h/x");
    REQ(dt != F32, "h/x must be fp16 or bf16");
    if (m == 0) return;
    REQ(h && x && src, "null h/x/src");
    Tensor th = borrow(h, {m, Co}, dt);
    add_skip(th, borrow(x, {n, Cin}, dt), borrow(src, {m}, I32));
  });
}

SPC_API int spc_conv_cfg_autotune_strict(const char* path, const char* device, int64_t N, int Ci, int Co, int strict,
                                         int* B1, int* BK, int* S) {
  return guarded([&] {
    REQ(path && device && B1 && BK && S, "null argument");
    REQ(N >= 0 && Ci > 0 && Co > 0, "N=%lld Ci=%d Co=%d", (long long)N, Ci, Co);
    const SpConvCfg c = spconv_cfg_autotune(path, device, N, Ci, Co, strict != 0);
    *B1 = c.B1;
    *BK = c.BK;
    *S = c.S;
  });
}

SPC_API int spc_conv_cfg_autotune(const char* path, const char* device, int64_t N, int Ci, int Co, int* B1, int* BK,
                                  int* S) {
  return spc_conv_cfg_autotune_strict(path, device, N, Ci, Co, 0, B1, BK, S);
}

SPC_API int spc_subm_conv(const void* x, const void* w, const void* b, int dtype, int b_dtype, int64_t N, int Ci,
                          int Co, spc_cache* c, void* out) {
  return spc_subm_conv_fused(x, w, b, nullptr, dtype, b_dtype, SPC_F32, dtype, SPC_ACT_NONE, N, Ci, Co, c, out);
}

SPC_API int spc_kernel_timing(int on) {
  return guarded([&] { kernel_timing(on != 0); });
}

SPC_API int spc_kernel_times(float* ms, int max, int* n) {
  return guarded([&] {
    REQ(n && (max <= 0 || ms), "null argument");
    const std::vector<float> t = kernel_times();
    const int k = (int)std::min<size_t>(t.size(), (size_t)std::max(max, 0));
    for (int i = 0; i < k; i++) ms[i] = t[i];
    *n = (int)t.size();
  });
}

SPC_API int spc_release_cached_memory(int64_t* bytes) {
  return guarded([&] {
    const i64 b = release_cached_memory();
    if (bytes) *bytes = b;
  });
}

SPC_API int spc_alloc_counts(int64_t* requests, int64_t* driver_allocs) {
  return guarded([&] {
    REQ(requests && driver_allocs, "null argument");
    i64 r = 0, d = 0;
    alloc_counts(&r, &d);
    *requests = r;
    *driver_allocs = d;
  });
}

SPC_API int spc_subm_conv_replay(const void* x, const void* w, const void* b, const void* residual, int act, int64_t N,
                                 int Ci, int Co, int B1, int BK, int S, spc_cache* c, void* out) {
  return guarded([&] {
    REQ(c, "cache is null");
    REQ(N == 0 || (x && w && out), "null argument");  // empty input: argument checks only, null buffers allowed
    Tensor tx = borrow(x, {N, Ci}, F16), tw = borrow(w, {Co, 27, Ci}, F16), to = borrow(out, {N, Co}, F16);
    Tensor tb, tr;
    if (b) tb = borrow(b, {Co}, F16);
    if (residual) tr = borrow(residual, {N, Co}, F16);
    subm_conv_replay(tx, tw, b ? &tb : nullptr, residual ? &tr : nullptr, act, SpConvCfg{B1, BK, S}, c->c, to);
  });
}

SPC_API int spc_grid_sample_map(const spc_cache* c, const float* grid, int64_t L, int batch, int flags, uint32_t* nb,
                                float* wt) {
  return guarded([&] {
    REQ(c, "cache is null");
    REQ(L >= 0 && (L == 0 || (grid && nb && wt)), "null argument or L < 0");
    REQ((flags & ~SPC_GS_NORMALIZE) == 0, "unknown flags %d", flags);
    Tensor tn = borrow(nb, {L, 8}, I32), tw = borrow(wt, {L, 8}, F32);
    grid_sample_map(c->c, borrow(grid, {L, 3}, F32), batch, (flags & SPC_GS_NORMALIZE) != 0, tn, tw);
  });
}

SPC_API int spc_grid_sample_sum(const float* x, int64_t M, int C, const uint32_t* nb, const float* wt, int64_t L,
                                float* y) {
  return guarded([&] {
    REQ(M >= 0 && L >= 0 && C >= 0, "sizes");
    REQ(L == 0 || C == 0 || (x && nb && wt && y), "null argument");
    Tensor ty = borrow(y, {L, C}, F32);
    grid_sample_sum(borrow(x, {M, C}, F32), borrow(nb, {L, 8}, I32), borrow(wt, {L, 8}, F32), ty);
  });
}

SPC_API int spc_subdivide_build(const int32_t* coords, const uint16_t* logits_f16, int64_t n, int W, int H, int D,
                                int32_t* child_coords, int32_t* src, int64_t* m, spc_cache** out) {
  return guarded([&] {
    REQ(m && out, "m or out is null");
    REQ(n >= 0 && (n == 0 || (coords && logits_f16 && child_coords && src)), "null argument");
    auto h = std::make_unique<spc_cache>();
    UpsampleLevel lv = subdivide_build(borrow(coords, {n, 4}, I32), borrow(logits_f16, {n, 8}, F16), W, H, D,
                                       child_coords, src);
    h->c = std::move(lv.cache);
    *m = lv.coords.size(0);
    *out = h.release();
  });
}

SPC_API int spc_subdivide(const int32_t* coords, const uint16_t* logits_f16, int64_t n, int32_t* child_coords,
                          int32_t* src, int64_t* m) {
  return guarded([&] {
    REQ(m, "m is null");
    REQ(n >= 0 && (n == 0 || (coords && logits_f16 && child_coords && src)), "null argument");
    Subdivision s = subdivide(borrow(coords, {n, 4}, I32), borrow(logits_f16, {n, 8}, F16));
    i64 k = s.coords.size(0);
    if (k) {
      CK(hipMemcpyAsync(child_coords, s.coords.p, (size_t)k * 16, hipMemcpyDeviceToDevice, stream()));
      CK(hipMemcpyAsync(src, s.src.p, (size_t)k * 4, hipMemcpyDeviceToDevice, stream()));
    }
    *m = k;
  });
}

SPC_API int spc_subdivide_noalloc(const int32_t* coords, const uint16_t* logits_f16, int64_t n, int32_t* child_coords,
                                  int32_t* src, int64_t* m_dev) {
  return guarded([&] { subdivide_noalloc(coords, logits_f16, n, child_coords, src, m_dev); });
}
