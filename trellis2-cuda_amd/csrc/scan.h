#pragma once
#include "core.h"

// out[i] = sum_{j<i} in[j] for i in [0,n); in and out may alias. If total_dev is non-null it receives the sum of
// all n inputs (device memory). Runs on the library stream; the tile-sum scratch is stream-ordered.
void excl_scan_u32(const uint32_t* in, uint32_t* out, i64 n, uint32_t* total_dev);
// The same scan with a caller-provided tile-sum workspace of excl_scan_parts(n) u32 (allocates nothing).
i64 excl_scan_parts(i64 n);
void excl_scan_u32_ws(const uint32_t* in, uint32_t* out, i64 n, uint32_t* total_dev, uint32_t* part);

// Stable ascending argsort of 27-bit keys: order[k] = row index of the k-th smallest key, ties in row order.
// ndev (device u32, optional): the number of keys, when n is only a capacity bound known to the host.
void stable_argsort27(const uint32_t* keys, i64 n, int32_t* order, const uint32_t* ndev = nullptr);

// Stable ascending sort of (key, value) pairs by the low `bits` bits of key; vals_out receives the values in key
// order (vals == nullptr means values 0..n-1). keys and vals are not modified; vals_out must not alias vals.
void stable_sort_pairs(const uint32_t* keys, const int32_t* vals, i64 n, int bits, int32_t* vals_out,
                       const uint32_t* ndev = nullptr);
