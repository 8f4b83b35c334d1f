#include "core.h"

#include <cstdarg>
#include <stdexcept>

void spc_fail(const char* fmt, ...) {
  char m[1024];
  va_list a;
  va_start(a, fmt);
  vsnprintf(m, sizeof(m), fmt, a);
  va_end(a);
  throw std::runtime_error(m);
}

size_t dsize(DT d) {
  static const size_t s[] = {4, 2, 2, 4, 8, 1, 8, 1};
  return s[d];
}
const char* dname(DT d) {
  static const char* s[] = {"F32", "F16", "BF16", "I32", "I64", "U8", "F64", "I8"};
  return s[d];
}

static hipStream_t g_stream = nullptr;
hipStream_t stream() { return g_stream; }
void set_stream(hipStream_t s) { g_stream = s; }
void dsync() { CK(hipStreamSynchronize(stream())); }

Tensor borrow(const void* p, std::vector<i64> sh, DT dt) {
  Tensor t;
  t.p = const_cast<void*>(p);
  t.sh = std::move(sh);
  t.dt = dt;
  return t;
}

Tensor empty(std::vector<i64> sh, DT dt) {
  Tensor t;
  t.sh = std::move(sh);
  t.dt = dt;
  size_t n = (t.bytes() + 16 + 511) & ~size_t(511);
  if (t.bytes()) {
    void* p = nullptr;
    hipStream_t s = stream();
    CK(hipMallocAsync(&p, n, s));
    t.p = p;
    // frees are ordered on the stream the tensor was allocated on
    t.own = std::shared_ptr<void>(p, [s](void* q) { (void)hipFreeAsync(q, s); });
  }
  return t;
}
Tensor zeros(std::vector<i64> sh, DT dt) {
  auto t = empty(std::move(sh), dt);
  if (t.bytes()) CK(hipMemsetAsync(t.p, 0, t.bytes(), stream()));
  return t;
}
Tensor from_host(const void* src, std::vector<i64> sh, DT dt) {
  auto t = empty(std::move(sh), dt);
  if (t.bytes()) CK(hipMemcpyAsync(t.p, src, t.bytes(), hipMemcpyHostToDevice, stream()));
  dsync();
  return t;
}
std::vector<char> to_host(const Tensor& t) {
  std::vector<char> v(t.bytes());
  if (t.bytes()) CK(hipMemcpyAsync(v.data(), t.p, t.bytes(), hipMemcpyDeviceToHost, stream()));
  dsync();
  return v;
}
Tensor Tensor::view(std::vector<i64> s) const {
  i64 n = 1, neg = -1;
  for (size_t i = 0; i < s.size(); i++) {
    if (s[i] < 0) neg = (i64)i;
    else n *= s[i];
  }
  if (neg >= 0) s[neg] = numel() / n;
  Tensor t = *this;
  t.sh = s;
  REQ(t.numel() == numel(), "bad view");
  return t;
}
Tensor Tensor::slice0(i64 a, i64 b) const {
  Tensor t = *this;
  i64 row = sh[0] ? numel() / sh[0] : 0;
  t.sh[0] = b - a;
  t.p = (char*)p + a * row * dsize(dt);
  return t;
}
