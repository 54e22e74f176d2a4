// Stable LSD radix sort of 32- or 64-bit unsigned keys carrying int32 values
// (device-wide, for gfx950). Shared by the standalone intersection sort and
// the depth-presorted intersection pipeline.
#pragma once

#include "common.hpp"

namespace gsplat_hip {

// Workspace bytes for sorting n pairs with K-sized keys.
template <typename K>
size_t radix_sort_workspace_bytes(int64_t n);

// Sorts bits [bit_lo, bit_hi) of the keys, 8 bits per pass (stable: equal
// digits keep their input order). Key bits at and above bit_hi must be zero
// or equal for all keys, bits below bit_lo are ignored. The result always
// lands in keys_out / vals_out; the inputs are not modified.
//
// With asm_ids set (32-bit keys only), the sorted keys are not stored;
// instead asm_ids[i] = sorted key << 32 | bits of asm_depths[sorted value]
// (keys_out is then only scratch between passes). With asm_bits and
// asm_bits_alt also set (n entries each; asm_bits[i] holds the depth bits
// of input pair i, and both buffers are overwritten), the one-sweep passes
// carry the bits beside the values instead of gathering asm_depths at the
// end. With gather_dst set (not with asm_ids), gather_dst[i] =
// gather_src[sorted value] as well.
template <typename K>
int radix_sort_pairs(const K* keys_in, const int32_t* vals_in, int64_t n, int bit_lo, int bit_hi, K* keys_out,
                     int32_t* vals_out, void* workspace, size_t workspace_bytes, hipStream_t stream,
                     const char* what, const float* asm_depths = nullptr, int64_t* asm_ids = nullptr,
                     const int32_t* gather_src = nullptr, int32_t* gather_dst = nullptr, uint32_t* asm_bits = nullptr,
                     uint32_t* asm_bits_alt = nullptr);

// Whether radix_sort_tiles_generated takes n entries on a tw x th tile grid
// with keys of bit_hi bits.
bool tiles_generated_supported(int64_t n, int tw, int th, int bit_hi);

// The depth-presorted tile lists sorted by (image, tile) with the encode
// folded into the first pass: the same output as encoding the lists of the
// Gaussians in depth order (entry j of rank r: Gaussian perm[r], tile k =
// j - offsets[r] of its AABB rect in row-major order, key image << tile_bits
// | tile, carried depth bits) and sorting bits [0, bit_hi) of the keys with
// radix_sort_pairs into ids (key << 32 | depth bits) and vals_out (Gaussian),
// without the encoded keys ever being stored. n entries in all (offsets:
// exclusive scan of the rect sizes in rank order); numel Gaussians,
// n_per_image per image. Scratch: recs [2 numel] (16 bytes each), part_rank
// [n / 3072 + 2], keys_out, bits and bits_alt [n] each, and the
// radix_sort_workspace_bytes<uint32_t>(n) workspace. Requires
// tiles_generated_supported(n, tw, th).
int radix_sort_tiles_generated(const float* means2d, const int32_t* radii, const float* depths, const int32_t* perm,
                               const int32_t* offsets, int64_t numel, int64_t n_per_image, int ts, int tw, int th,
                               int tile_bits, int64_t n, int bit_hi, uint4* recs, int32_t* part_rank,
                               uint32_t* keys_out, int32_t* vals_out, int64_t* ids, uint32_t* bits,
                               uint32_t* bits_alt, void* workspace, size_t workspace_bytes, hipStream_t stream,
                               const char* what);

}  // namespace gsplat_hip
