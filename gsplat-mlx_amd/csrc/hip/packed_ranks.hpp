// The packed layout's rank structure, written by the packed projection's
// count pass (projection.hip): one bit per (b, c, n) pair, at flat pair index
// (b * C + c) * N + n, in 64-bit words, and each word's first packed row (the
// exclusive scan of the words' popcounts). It sits at the start of the
// packed count workspace: the words, then the prefixes, each section
// 256-byte aligned. A pair's packed row is its word's prefix plus the set
// bits below it, so kernels that take the workspace read and write packed
// rows without a dense index map.
#pragma once

#include "common.hpp"

namespace gsplat_hip {

struct PackedRanks {
  const uint64_t* mask;
  const int32_t* prefix;
};

inline size_t packed_ranks_align(size_t b) { return (b + 255) / 256 * 256; }

// Bytes of the words and prefixes for `total` pairs (the start of the count
// workspace).
inline size_t packed_ranks_bytes(int64_t total) {
  const size_t nw = static_cast<size_t>((total + 63) / 64);
  return packed_ranks_align(nw * 8) + packed_ranks_align(nw * 4);
}

inline PackedRanks packed_ranks_at(const void* base, int64_t total) {
  const size_t nw = static_cast<size_t>((total + 63) / 64);
  const char* p = static_cast<const char*>(base);
  return {reinterpret_cast<const uint64_t*>(p), reinterpret_cast<const int32_t*>(p + packed_ranks_align(nw * 8))};
}

// Packed row of pair idx, whose bit is set.
__device__ __forceinline__ int64_t packed_rank(const uint64_t* __restrict__ mask, const int32_t* __restrict__ prefix,
                                               int64_t idx) {
  const uint64_t w = mask[idx >> 6];
  const int bit = static_cast<int>(idx & 63);
  return static_cast<int64_t>(prefix[idx >> 6]) + __popcll(w & ((1ull << bit) - 1ull));
}

// Packed row of pair idx, or -1 when the pair has none (its bit is clear, or
// its rank is not below nnz).
__device__ __forceinline__ int64_t packed_row(const uint64_t* __restrict__ mask, const int32_t* __restrict__ prefix,
                                              int64_t idx, int64_t nnz) {
  const uint64_t w = mask[idx >> 6];
  const int bit = static_cast<int>(idx & 63);
  if (!((w >> bit) & 1ull)) return -1;
  const int64_t r = static_cast<int64_t>(prefix[idx >> 6]) + __popcll(w & ((1ull << bit) - 1ull));
  return r < nnz ? r : -1;
}

}  // namespace gsplat_hip
