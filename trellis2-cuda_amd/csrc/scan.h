#pragma once
#include "core.h"

// out[i] = sum_{j<i} in[j] for i in [0,n); in and out may alias. If total_dev is non-null it receives the sum of
// all n inputs (device memory). Runs on the library stream; the tile-sum scratch is stream-ordered.
void excl_scan_u32(const uint32_t* in, uint32_t* out, i64 n, uint32_t* total_dev);
// The same scan with a caller-provided tile-sum workspace of excl_scan_parts(n) u32 (allocates nothing).
i64 excl_scan_parts(i64 n);
void excl_scan_u32_ws(const uint32_t* in, uint32_t* out, i64 n, uint32_t* total_dev, uint32_t* part);

// Workspace of the radix sort (9-bit digits, tiles of 256 * rch keys). A producer of the keys may count the first
// pass itself: it zeroes the first `zwords` u32 of `buf` beforehand (digit-sum slots, then the first pass's counts)
// and adds, for each key i of the first n, one to counts[(key_i & 511) * ntiles + i / (256 * rch)], the counts
// starting at u32 word `passes * 1024` of `buf`. Passing the workspace to the sort then skips the first count kernel.
struct SortWork {
  int passes = 0, rch = 0, ntiles = 0;
  i64 zwords = 0;
  Tensor buf;
  uint32_t* counts() const { return buf.ptr<uint32_t>() + (i64)passes * 1024; }
};
SortWork sort_work(i64 n, int bits);

// Stable ascending argsort of 27-bit keys: order[k] = row index of the k-th smallest key, ties in row order.
// ndev (device u32, optional): the number of keys, when n is only a capacity bound known to the host.
// pre (optional): a workspace from sort_work(n, 27) whose first pass was counted by the caller.
void stable_argsort27(const uint32_t* keys, i64 n, int32_t* order, const uint32_t* ndev = nullptr,
                      SortWork* pre = nullptr);

// Stable ascending sort of (key, value) pairs by the low `bits` bits of key; vals_out receives the values in key
// order (vals == nullptr means values 0..n-1). keys and vals are not modified; vals_out must not alias vals.
void stable_sort_pairs(const uint32_t* keys, const int32_t* vals, i64 n, int bits, int32_t* vals_out,
                       const uint32_t* ndev = nullptr, SortWork* pre = nullptr);
