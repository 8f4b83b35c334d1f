#include "core.h"

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <mutex>
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

// Device memory: a caching allocator over hipMallocAsync. hipFreeAsync costs tens of microseconds of host time per
// call on this platform, and a kernel-map build allocates a dozen temporaries, so freed blocks are kept in per
// (device, stream, size class) free lists and handed out again. Reuse is stream-ordered: a block freed while
// kernels on its stream may still use it is only ever reissued to later work on that same stream. Size classes:
// powers of two up to 1 MiB, then multiples of 2 MiB. Cached blocks are kept until the process ends (like a
// framework's caching allocator); the pool's release threshold is raised too, so blocks that do go back to the
// driver stay mapped.
namespace {
struct BlockKey {
  int dev;
  hipStream_t stream;
  size_t size;
  bool operator<(const BlockKey& o) const {
    if (dev != o.dev) return dev < o.dev;
    if (stream != o.stream) return stream < o.stream;
    return size < o.size;
  }
};
std::mutex g_alloc_mu;
std::map<BlockKey, std::vector<void*>>& free_blocks() {
  static auto* m = new std::map<BlockKey, std::vector<void*>>();  // never destroyed: frees can run at exit
  return *m;
}
size_t size_class(size_t n) {
  if (n <= (1u << 20)) {
    size_t c = 512;
    while (c < n) c <<= 1;
    return c;
  }
  const size_t g = 2u << 20;
  return (n + g - 1) / g * g;
}
std::atomic<i64> g_alloc_requests{0}, g_driver_allocs{0};
void keep_pool_memory(int dev) {
  static bool done[64] = {};
  if (dev < 0 || dev >= 64 || done[dev]) return;
  hipMemPool_t pool;
  CK(hipDeviceGetDefaultMemPool(&pool, dev));
  uint64_t keep = UINT64_MAX;
  CK(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep));
  done[dev] = true;
}
}  // namespace

Tensor empty(std::vector<i64> sh, DT dt) {
  Tensor t;
  t.sh = std::move(sh);
  t.dt = dt;
  if (t.bytes()) {
    int dev = 0;
    CK(hipGetDevice(&dev));
    const BlockKey key{dev, stream(), size_class(t.bytes() + 16)};
    void* p = nullptr;
    {
      std::lock_guard<std::mutex> g(g_alloc_mu);
      keep_pool_memory(dev);
      auto& fl = free_blocks()[key];
      if (!fl.empty()) {
        p = fl.back();
        fl.pop_back();
      }
    }
    g_alloc_requests++;
    if (!p) {
      CK(hipMallocAsync(&p, key.size, key.stream));
      g_driver_allocs++;
    }
    t.p = p;
    t.own = std::shared_ptr<void>(p, [key](void* q) {
      std::lock_guard<std::mutex> g(g_alloc_mu);
      free_blocks()[key].push_back(q);
    });
  }
  return t;
}
i64 release_cached_memory() {
  std::map<BlockKey, std::vector<void*>> lists;
  {
    std::lock_guard<std::mutex> g(g_alloc_mu);
    lists.swap(free_blocks());
  }
  i64 bytes = 0;
  std::vector<int> devs;
  bool any = false;
  for (auto& kv : lists) any |= !kv.second.empty();
  if (!any) return 0;
  int cur = 0;
  CK(hipGetDevice(&cur));
  for (auto& kv : lists) {
    if (kv.second.empty()) continue;
    CK(hipSetDevice(kv.first.dev));
    for (void* p : kv.second) CK(hipFreeAsync(p, kv.first.stream));  // stream-ordered after the block's last use
    bytes += (i64)kv.first.size * (i64)kv.second.size();
    if (std::find(devs.begin(), devs.end(), kv.first.dev) == devs.end()) devs.push_back(kv.first.dev);
  }
  for (int d : devs) {  // hand the freed memory back to the device (the pool keeps it otherwise)
    CK(hipSetDevice(d));
    CK(hipDeviceSynchronize());
    hipMemPool_t pool;
    CK(hipDeviceGetDefaultMemPool(&pool, d));
    CK(hipMemPoolTrimTo(pool, 0));
  }
  CK(hipSetDevice(cur));
  return bytes;
}

void alloc_counts(i64* requests, i64* driver_allocs) {
  *requests = g_alloc_requests.load();
  *driver_allocs = g_driver_allocs.load();
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
