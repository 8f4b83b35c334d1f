// Minimal device-tensor runtime for the sparse-conv path: the subset of the reference's L0 core that
// spconv.h depends on (reference src/core.h:14-64), written for HIP on MI355X.
//
//  * Tensor: device pointer + dtype + shape + shared ownership, contiguous row-major (src/core.h:29-42).
//  * Allocation is stream-ordered (hipMallocAsync on the library stream), 512 B aligned with slack so 16 B vector
//    loads at the end of a row stay in bounds (src/core.cu:31-40).
//  * Errors: CK / REQ -> spc_fail -> std::runtime_error (src/core.h:14-17, src/core.cu:10-15).
//  * One library stream, default = the null stream so work orders with the caller's; spc_set_stream() lets a
//    host framework hand in its own stream (the reference owns one global non-blocking stream, src/core.cu:20-28).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#pragma GCC visibility push(default)  // exported for C++ callers (see spconv.h)

[[noreturn]] void spc_fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
#define CK(x)                                                                                             \
  do {                                                                                                    \
    hipError_t e_ = (x);                                                                                  \
    if (e_ != hipSuccess) spc_fail("HIP %s @ %s:%d: %s", #x, __FILE__, __LINE__, hipGetErrorString(e_)); \
  } while (0)
#define REQ(c, ...)                                                       \
  do {                                                                    \
    if (!(c)) {                                                           \
      char m_[512];                                                       \
      snprintf(m_, sizeof(m_), __VA_ARGS__);                              \
      spc_fail("check failed %s @ %s:%d: %s", #c, __FILE__, __LINE__, m_); \
    }                                                                     \
  } while (0)

using i64 = int64_t;
// Same enum order as the reference's DT (src/core.h:22), so dtype codes cross the C ABI unchanged.
enum DT : uint8_t { F32, F16, BF16, I32, I64, U8, F64, I8 };
size_t dsize(DT d);
const char* dname(DT d);

hipStream_t stream();
void set_stream(hipStream_t s);

struct Tensor {
  void* p = nullptr;
  DT dt = F32;
  std::vector<i64> sh;
  std::shared_ptr<void> own;
  i64 numel() const {
    i64 n = 1;
    for (auto s : sh) n *= s;
    return n;
  }
  size_t bytes() const { return (size_t)numel() * dsize(dt); }
  i64 size(int i) const { return sh[i < 0 ? i + (int)sh.size() : i]; }
  int dim() const { return (int)sh.size(); }
  bool defined() const { return p != nullptr || (numel() == 0 && !sh.empty()); }
  template <class T>
  T* ptr() const {
    return (T*)p;
  }
  Tensor view(std::vector<i64> s) const;
  Tensor slice0(i64 a, i64 b) const;
};

// Wraps caller-owned device memory (no ownership): how the C ABI hands pointers to the C++ API.
Tensor borrow(const void* p, std::vector<i64> sh, DT dt);
Tensor empty(std::vector<i64> sh, DT dt);
Tensor zeros(std::vector<i64> sh, DT dt);
// Device allocations the library has made since the process started: every request to empty() with a nonzero size
// (served from the free lists or not), and the hipMallocAsync calls among them.
void alloc_counts(i64* requests, i64* driver_allocs);
// Frees every cached (currently unused) device block back to the driver and trims the devices' memory pools: waits
// for the devices the blocks belong to. Blocks still owned by live tensors are untouched. Returns the bytes freed.
i64 release_cached_memory();
Tensor from_host(const void* src, std::vector<i64> sh, DT dt);
std::vector<char> to_host(const Tensor& t);
template <class T>
std::vector<T> to_host_vec(const Tensor& t) {
  auto b = to_host(t);
  std::vector<T> v(b.size() / sizeof(T));
  if (!b.empty()) memcpy(v.data(), b.data(), b.size());
  return v;
}
void dsync();

__host__ __device__ inline int cdiv(i64 a, i64 b) { return (int)((a + b - 1) / b); }

#pragma GCC visibility pop
