// Tile intersection operator layer: validation, staging and the single
// device-to-host read of the intersection count follow
// gsplat_core/gsplat_intersect.cpp:60-307, 586-603 of the reference; compute
// is the HIP C-ABI (fused count+scan, encode, radix sort, offsets).
#include "gsplat_intersect.h"

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <limits>
#include <cstdlib>
#include <map>
#include <memory>
#include <mutex>

#include "core_util.h"

namespace gsplat_core {
namespace {
using namespace detail;

int floor_log2_plus_one(int64_t value) {
  if (value <= 0) throw std::runtime_error("intersect expects positive image/tile counts.");
  return static_cast<int>(std::floor(std::log2(static_cast<float>(value)))) + 1;
}

int bit_length(uint64_t v) {
  int b = 0;
  while (v) {
    ++b;
    v >>= 1;
  }
  return b;
}

// gsplat_intersect.cpp:114-148
// Packed layout (params.packed, rejected by the reference at :115-118):
// means2d / radii [nnz, 2], depths [nnz], image_ids [nnz] (the image of each
// row); gaussian_ids are accepted and not needed (flatten ids are rows).
void validate_packed_input(const IntersectTileInput& input) {
  if (input.means2d.dim() != 2 || input.means2d.size(-1) != 2)
    throw std::runtime_error("intersect_tile packed path expects means2d [nnz, 2].");
  const int64_t nnz = input.means2d.size(0);
  if (input.radii.dim() != 2 || input.radii.size(0) != nnz || input.radii.size(1) != 2)
    throw std::runtime_error("intersect_tile packed path expects radii [nnz, 2].");
  if (input.depths.dim() != 1 || input.depths.size(0) != nnz)
    throw std::runtime_error("intersect_tile packed path expects depths [nnz].");
  if (input.image_ids.numel() != nnz)
    throw std::runtime_error("intersect_tile packed path expects image_ids [nnz].");
  if (input.image_ids.scalar_type() != at::kInt && input.image_ids.scalar_type() != at::kLong)
    throw std::runtime_error("intersect_tile packed path expects int32 or int64 image_ids.");
  if (input.params.I <= 0) throw std::runtime_error("intersect_tile packed path expects I > 0.");
  require_device(input.image_ids, "image_ids");
}

void validate_intersect_tile_input(const IntersectTileInput& input) {
  if (input.params.segmented) throw std::runtime_error("intersect_tile segmented sort is not implemented yet.");
  if (input.params.use_conics != input.params.use_opacities)
    throw std::runtime_error("intersect_tile AccuTile path needs both conics and opacities.");
  if (input.params.packed) validate_packed_input(input);
  if (input.means2d.dim() < (input.params.packed ? 2 : 3) || input.means2d.size(-1) != 2)
    throw std::runtime_error("means2d must have shape [..., N, 2].");
  if (input.radii.dim() != input.means2d.dim() || input.radii.size(-1) != 2)
    throw std::runtime_error("radii must have shape [..., N, 2].");
  if (input.depths.dim() + 1 != input.means2d.dim()) throw std::runtime_error("depths must have shape [..., N].");
  if (input.means2d.scalar_type() != at::kFloat || input.radii.scalar_type() != at::kInt ||
      input.depths.scalar_type() != at::kFloat)
    throw std::runtime_error("intersect_tile dense path expects float32 means2d/depths and int32 radii.");
  require_device(input.means2d, "means2d");
  require_device(input.radii, "radii");
  require_device(input.depths, "depths");
  if (input.params.use_conics) {
    if (input.conics.scalar_type() != at::kFloat || input.opacities.scalar_type() != at::kFloat)
      throw std::runtime_error("intersect_tile AccuTile path expects float32 conics and opacities.");
    if (input.conics.numel() != input.depths.numel() * 3 || input.opacities.numel() != input.depths.numel())
      throw std::runtime_error("intersect_tile AccuTile path expects conics [..., N, 3] and opacities [..., N].");
    require_device(input.conics, "conics");
    require_device(input.opacities, "opacities");
  }
}

// Ellipse tiles (conics and opacities given), else the AABB rect.
bool accutile(const IntersectTileInput& input) { return input.params.use_conics && input.params.use_opacities; }

void check_dense_size(const IntersectTileInput& input, const char* op) {
  if (input.params.packed) return;  // validate_packed_input checked the nnz rows
  const int64_t n = input.means2d.size(-2);
  const int64_t numel = input.depths.numel();
  const int64_t I = input.params.I;
  if (I <= 0 || numel % I != 0 || numel != I * n)
    throw std::runtime_error(std::string(op) + " dense path expects depths size to equal I * N.");
  if (input.means2d.numel() != numel * 2 || input.radii.numel() != numel * 2)
    throw std::runtime_error(std::string(op) + " expects means2d and radii with two values per depth.");
}

// Workspace bytes from torch's caching allocator (no synchronisation).
array workspace(size_t bytes, const array& ref) {
  return at::empty({static_cast<int64_t>(bytes > 0 ? bytes : 1)}, u8_like(ref));
}

struct Counted {
  array tiles_per_gauss;
  array offsets;
  array total;  // int64 [1] on device
};

// with_offsets false: counts and total only (the depth-presorted path scans
// the counts in depth order itself).
Counted count_and_scan(const IntersectTileInput& input, void* stream, bool with_offsets = true) {
  const array means2d = contig(input.means2d);
  const array radii = contig(input.radii);
  const int64_t numel = input.depths.numel();
  Counted c;
  c.tiles_per_gauss = at::empty(input.depths.sizes(), i32_like(means2d));
  if (with_offsets) c.offsets = at::empty(input.depths.sizes(), i32_like(means2d));
  c.total = at::empty({1}, i64_like(means2d));
  const size_t ws_bytes = gsplat_hip_isect_count_scan_workspace_size(numel);
  array ws = workspace(ws_bytes, means2d);
  int32_t* offs = with_offsets ? c.offsets.data_ptr<int32_t>() : nullptr;
  if (accutile(input)) {
    const array conics = contig(input.conics);
    const array opac = contig(input.opacities);
    check(gsplat_hip_isect_count_scan_accutile(means2d.data_ptr<float>(), radii.data_ptr<int32_t>(),
                                               conics.data_ptr<float>(), opac.data_ptr<float>(), numel,
                                               input.params.tile_size, input.params.tile_width,
                                               input.params.tile_height, c.tiles_per_gauss.data_ptr<int32_t>(), offs,
                                               c.total.data_ptr<int64_t>(), ws.data_ptr<uint8_t>(), ws_bytes, stream));
    return c;
  }
  check(gsplat_hip_isect_count_scan(means2d.data_ptr<float>(), radii.data_ptr<int32_t>(), numel,
                                    input.params.tile_size, input.params.tile_width, input.params.tile_height,
                                    c.tiles_per_gauss.data_ptr<int32_t>(), offs, c.total.data_ptr<int64_t>(),
                                    ws.data_ptr<uint8_t>(), ws_bytes, stream));
  return c;
}

// Frames with more entries than this that hold a list longer than the LDS
// tile sort take the depth-presorted path (see intersect_bucketed_finish).
constexpr int64_t kPresortAboveIsects = int64_t{1} << 26;

// The bucketed intersection path (bucket.hip) is the default for sorted
// dense intersections, AABB or ellipse tiles, whose tile grid it supports;
// GSPLAT_ISECT_BUCKETED=0 selects the depth-presorted path instead (read
// once per process).
bool bucketed_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("GSPLAT_ISECT_BUCKETED");
    return !(v && v[0] == '0');
  }();
  return on;
}

// Packed inputs take it too when their rows are grouped by image (the packed
// projection's order), which the count step checks on the device; otherwise
// they fall back to the depth-presorted path after the read-back.
bool use_bucketed(const IntersectTileInput& input) {
  const auto& p = input.params;
  if (!p.sort || !bucketed_enabled()) return false;
  return accutile(input) ? gsplat_hip_isect_bucket_accutile_supported(p.I, p.tile_width, p.tile_height)
                         : gsplat_hip_isect_bucket_supported(p.I, p.tile_width, p.tile_height);
}

// The one device->host read of the chain (gsplat_intersect.cpp:155-170),
// ordered after the count/scan kernels on their stream. It is split in two so
// that work which does not need the count can be queued between the copy and
// the wait: the copy lands in a pinned host word and an event marks it, so
// the wait ends when the copy is done rather than when the stream drains.
struct CountReadback {
  // [3]: the count and, for the bucketed path, the longest tile list and
  // (packed rows) the ungrouped flag
  int64_t* host = nullptr;
  hipEvent_t done = nullptr;
};

CountReadback& readback_slot() {
  // one slot per host thread and device; the call that starts a read-back
  // also finishes it before returning
  thread_local std::map<int, CountReadback> slots;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) throw std::runtime_error("intersect_tile: no current HIP device.");
  CountReadback& r = slots[dev];
  if (!r.host) {
    void* p = nullptr;
    if (hipHostMalloc(&p, 4 * sizeof(int64_t), hipHostMallocDefault) != hipSuccess)
      throw std::runtime_error("intersect_tile: pinned host allocation for the count failed.");
    r.host = static_cast<int64_t*>(p);
  }
  if (!r.done && hipEventCreateWithFlags(&r.done, hipEventDisableTiming) != hipSuccess)
    throw std::runtime_error("intersect_tile: event creation failed.");
  return r;
}

void start_read_total(const array& total_dev, void* stream, CountReadback& r, int words = 1) {
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t err = hipMemcpyAsync(r.host, total_dev.data_ptr<int64_t>(), words * sizeof(int64_t),
                                  hipMemcpyDeviceToHost, s);
  if (err == hipSuccess) err = hipEventRecord(r.done, s);
  if (err != hipSuccess)
    throw std::runtime_error(std::string("intersect_tile: reading the intersection count failed: ") +
                             hipGetErrorString(err));
}

int finish_read_total(CountReadback& r) {
  const hipError_t err = hipEventSynchronize(r.done);
  if (err != hipSuccess)
    throw std::runtime_error(std::string("intersect_tile: reading the intersection count failed: ") +
                             hipGetErrorString(err));
  const int64_t total = *r.host;
  if (total > static_cast<int64_t>(INT32_MAX))
    throw std::runtime_error("intersect_tile: more than 2^31-1 intersections (int32 offsets overflow).");
  return static_cast<int>(total);
}

int read_total(const array& total_dev, void* stream) {
  CountReadback& r = readback_slot();
  start_read_total(total_dev, stream, r);
  return finish_read_total(r);
}

// Largest key the encoder can produce for I images of n_tiles tiles: the sort
// only needs that many low bits (higher bits are zero for every key).
int encoded_key_bits(int64_t I, int64_t n_tiles) {
  const int tile_bits = floor_log2_plus_one(n_tiles);
  const uint64_t max_key = (static_cast<uint64_t>(I - 1) << (32 + tile_bits)) |
                           (static_cast<uint64_t>(n_tiles - 1) << 32) | 0xFFFFFFFFull;
  return bit_length(max_key);
}

// Encode in pair-major order (no sort): {isect_ids, flatten_ids}.
std::vector<array> encode_unsorted(const IntersectTileInput& input, const array& means2d, const array& radii,
                                   const array& depths, const array& offsets, int total, void* stream) {
  array ids = at::empty({total}, i64_like(means2d));
  array flat = at::empty({total}, i32_like(means2d));
  if (input.params.packed) {
    const array conics = accutile(input) ? contig(input.conics) : array();
    const array opac = accutile(input) ? contig(input.opacities) : array();
    const array image_ids = contig(input.image_ids.to(at::kInt));
    check(gsplat_hip_isect_encode_packed(
        means2d.data_ptr<float>(), radii.data_ptr<int32_t>(), accutile(input) ? conics.data_ptr<float>() : nullptr,
        accutile(input) ? opac.data_ptr<float>() : nullptr, image_ids.data_ptr<int32_t>(), depths.data_ptr<float>(),
        offsets.data_ptr<int32_t>(), input.params.I, depths.numel(), input.params.tile_size, input.params.tile_width,
        input.params.tile_height, total, ids.data_ptr<int64_t>(), flat.data_ptr<int32_t>(), stream));
    return {ids, flat};
  }
  if (accutile(input)) {
    const array conics = contig(input.conics);
    const array opac = contig(input.opacities);
    check(gsplat_hip_isect_encode_accutile(means2d.data_ptr<float>(), radii.data_ptr<int32_t>(),
                                           conics.data_ptr<float>(), opac.data_ptr<float>(), depths.data_ptr<float>(),
                                           offsets.data_ptr<int32_t>(), input.params.I, depths.numel(),
                                           input.params.tile_size, input.params.tile_width, input.params.tile_height,
                                           total, ids.data_ptr<int64_t>(), flat.data_ptr<int32_t>(), stream));
  } else {
    check(gsplat_hip_isect_encode(means2d.data_ptr<float>(), radii.data_ptr<int32_t>(), depths.data_ptr<float>(),
                                  offsets.data_ptr<int32_t>(), input.params.I, depths.numel(), input.params.tile_size,
                                  input.params.tile_width, input.params.tile_height, total, ids.data_ptr<int64_t>(),
                                  flat.data_ptr<int32_t>(), stream));
  }
  return {ids, flat};
}

}  // namespace

array gsplat_intersect_tile_count(const IntersectTileInput& input) {
  validate_intersect_tile_input(input);
  check_dense_size(input, "intersect_tile_count");
  const c10::DeviceGuard guard(input.means2d.device());
  return count_and_scan(input, stream_for(input.s, input.means2d)).tiles_per_gauss;
}

array gsplat_intersect_tile_offsets(const array& tiles_per_gauss, StreamOrDevice s) {
  if (tiles_per_gauss.scalar_type() != at::kInt)
    throw std::runtime_error("intersect_tile_offsets expects int32 tiles_per_gauss.");
  require_device(tiles_per_gauss, "tiles_per_gauss");
  const c10::DeviceGuard guard(tiles_per_gauss.device());
  const array counts = contig(tiles_per_gauss);
  array out = at::empty(counts.sizes(), counts.options());
  const int64_t n = counts.numel();
  const size_t ws_bytes = gsplat_hip_exclusive_scan_i32_workspace_size(n);
  array ws = workspace(ws_bytes, counts);
  check(gsplat_hip_exclusive_scan_i32(counts.data_ptr<int32_t>(), out.data_ptr<int32_t>(), n, nullptr,
                                      ws.data_ptr<uint8_t>(), ws_bytes, stream_for(s, counts)));
  return out;
}

std::vector<array> gsplat_intersect_tile_encode(const IntersectTileInput& input, const array& tile_offsets,
                                                int total_isects) {
  validate_intersect_tile_input(input);
  check_dense_size(input, "intersect_tile_encode");
  if (total_isects < 0) throw std::runtime_error("intersect_tile_encode expects non-negative total_isects.");
  if (tile_offsets.scalar_type() != at::kInt || tile_offsets.numel() != input.depths.numel())
    throw std::runtime_error("intersect_tile_encode expects int32 tile_offsets with depths shape.");
  require_device(tile_offsets, "tile_offsets");
  const int64_t n_tiles = static_cast<int64_t>(input.params.tile_width) * input.params.tile_height;
  if (floor_log2_plus_one(input.params.I) + floor_log2_plus_one(n_tiles) > 32)
    throw std::runtime_error("intersect_tile_encode image id and tile id require more than 32 bits.");
  const c10::DeviceGuard guard(input.means2d.device());
  const array means2d = contig(input.means2d);
  const array radii = contig(input.radii);
  const array depths = contig(input.depths);
  const array offsets = contig(tile_offsets);
  return encode_unsorted(input, means2d, radii, depths, offsets, total_isects, stream_for(input.s, means2d));
}

std::vector<array> gsplat_intersect_tile_sort(const array& isect_ids, const array& flatten_ids, StreamOrDevice s) {
  if (isect_ids.scalar_type() != at::kLong) throw std::runtime_error("intersect_tile_sort expects int64 isect_ids.");
  if (flatten_ids.scalar_type() != at::kInt)
    throw std::runtime_error("intersect_tile_sort expects int32 flatten_ids.");
  if (isect_ids.dim() != 1 || flatten_ids.dim() != 1 || isect_ids.numel() != flatten_ids.numel())
    throw std::runtime_error("intersect_tile_sort expects matching 1D isect_ids and flatten_ids.");
  require_device(isect_ids, "isect_ids");
  require_device(flatten_ids, "flatten_ids");
  const c10::DeviceGuard guard(isect_ids.device());
  const array keys = contig(isect_ids);
  const array vals = contig(flatten_ids);
  if (keys.numel() == 0) return {keys.clone(), vals.clone()};
  // Arbitrary int64 keys, in signed order; the passes over digits that every
  // key shares are skipped on the device, so nothing is read back.
  const int64_t n = keys.numel();
  array ko = at::empty({n}, keys.options());
  array vo = at::empty({n}, vals.options());
  const size_t ws_bytes = gsplat_hip_isect_sort_workspace_size(n);
  array ws = workspace(ws_bytes, keys);
  check(gsplat_hip_isect_sort_i64(keys.data_ptr<int64_t>(), vals.data_ptr<int32_t>(), n, ko.data_ptr<int64_t>(),
                                  vo.data_ptr<int32_t>(), ws.data_ptr<uint8_t>(), ws_bytes, stream_for(s, keys)));
  return {ko, vo};
}

// Sorted dense intersections (AABB or ellipse tiles) by tile buckets
// (bucket.hip): counts, then M and the longest list read back together (the
// longest list selects the tile sort launches), then the bucketed scatter and
// per-tile sorts.
// The bucketed intersection in two halves around the read-back of M and the
// longest tile list: the count kernels (queued), then, once the two words are
// on the host, the M-long outputs and the scatter + tile sort.
struct BucketState {
  array means2d, radii, depths, conics, opacities, image_ids, tiles_per_gauss, totals, ws1;
  size_t ws1_bytes = 0;
  bool ell = false;     // ellipse tiles (conics and opacities held)
  bool packed = false;  // packed rows (image_ids held)
  void* stream = nullptr;
  int readback_words() const { return packed ? 3 : 2; }
};

BucketState intersect_bucketed_count(const IntersectTileInput& input, void* stream) {
  BucketState b;
  b.stream = stream;
  b.means2d = contig(input.means2d);
  b.radii = contig(input.radii);
  b.depths = contig(input.depths);
  const auto& p = input.params;
  const int64_t numel = b.depths.numel();
  b.tiles_per_gauss = at::empty(input.depths.sizes(), i32_like(b.means2d));
  b.totals = at::empty({3}, i64_like(b.means2d));
  b.ell = accutile(input);
  b.packed = p.packed;
  if (b.packed) {
    b.image_ids = contig(input.image_ids.to(at::kInt));
    if (b.ell) {
      b.conics = contig(input.conics);
      b.opacities = contig(input.opacities);
    }
    b.ws1_bytes =
        gsplat_hip_isect_bucket_count_packed_workspace_size(p.I, numel, p.tile_size, p.tile_width, p.tile_height);
    b.ws1 = workspace(b.ws1_bytes, b.means2d);
    check(gsplat_hip_isect_bucket_count_packed(
        b.means2d.data_ptr<float>(), b.radii.data_ptr<int32_t>(), b.ell ? b.conics.data_ptr<float>() : nullptr,
        b.ell ? b.opacities.data_ptr<float>() : nullptr, b.image_ids.data_ptr<int32_t>(), p.I, numel, p.tile_size,
        p.tile_width, p.tile_height, b.tiles_per_gauss.data_ptr<int32_t>(), b.totals.data_ptr<int64_t>(),
        b.ws1.data_ptr<uint8_t>(), b.ws1_bytes, stream));
    return b;
  }
  b.ws1_bytes = gsplat_hip_isect_bucket_count_workspace_size(p.I, numel, p.tile_size, p.tile_width, p.tile_height);
  b.ws1 = workspace(b.ws1_bytes, b.means2d);
  if (b.ell) {
    b.conics = contig(input.conics);
    b.opacities = contig(input.opacities);
    check(gsplat_hip_isect_bucket_count_accutile(
        b.means2d.data_ptr<float>(), b.radii.data_ptr<int32_t>(), b.conics.data_ptr<float>(),
        b.opacities.data_ptr<float>(), p.I, numel, p.tile_size, p.tile_width, p.tile_height,
        b.tiles_per_gauss.data_ptr<int32_t>(), b.totals.data_ptr<int64_t>(), b.ws1.data_ptr<uint8_t>(), b.ws1_bytes,
        stream));
    return b;
  }
  check(gsplat_hip_isect_bucket_count(b.means2d.data_ptr<float>(), b.radii.data_ptr<int32_t>(), p.I, numel,
                                      p.tile_size, p.tile_width, p.tile_height, b.tiles_per_gauss.data_ptr<int32_t>(),
                                      b.totals.data_ptr<int64_t>(), b.ws1.data_ptr<uint8_t>(), b.ws1_bytes, stream));
  return b;
}

std::vector<array> intersect_presorted(const IntersectTileInput& input, void* stream);

// Speculative scatter + tile sort: with the count kernels queued, the second
// step is launched at once into outputs sized by the M of the previous call
// on the same inputs' shape (plus an eighth), reading the new M on the
// device; the host then waits for M while the GPU sorts. The result is kept
// when M fits and the tile sort classes launched cover the longest list
// (otherwise the exact step runs after the read-back). Hints are per host
// thread and shape key.
struct SpecHint {
  int64_t capacity = 0, longest = 0, total = 0;
  int presorted_calls = 0;  // consecutive calls sent straight to the presorted path
};

SpecHint& spec_hint(const IntersectTileInput& input, int64_t numel) {
  thread_local std::map<std::vector<int64_t>, SpecHint> hints;
  int dev = 0;
  (void)hipGetDevice(&dev);
  const auto& p = input.params;
  return hints[{dev, p.I, p.tile_size, p.tile_width, p.tile_height, accutile(input), p.packed, numel}];
}

struct Speculation {
  bool active = false;
  int64_t capacity = 0, max_list = 0;
  array ids, flat, offsets, ws2;
};

// Frames whose long lists take the depth-presorted path (see
// intersect_bucketed_finish) are not speculated.
bool presorted_policy(int64_t longest, int64_t total) {
  return longest > gsplat_hip_isect_bucket_max_list() && total >= kPresortAboveIsects;
}

Speculation speculate(const IntersectTileInput& input, const BucketState& b, bool with_offsets) {
  Speculation sp;
  const auto& p = input.params;
  const SpecHint& h = spec_hint(input, b.depths.numel());
  if (h.capacity <= 0 || presorted_policy(h.longest, h.capacity)) return sp;
  sp.active = true;
  sp.capacity = h.capacity;
  sp.max_list = h.longest;
  sp.ids = at::empty({sp.capacity}, i64_like(b.means2d));
  sp.flat = at::empty({sp.capacity}, i32_like(b.means2d));
  if (with_offsets) sp.offsets = at::empty({p.I, p.tile_height, p.tile_width}, i32_like(b.means2d));
  const size_t ws2_bytes = gsplat_hip_isect_bucket_sort_workspace_size(sp.capacity);
  sp.ws2 = workspace(ws2_bytes, b.means2d);
  check(gsplat_hip_isect_bucket_sort_speculative(
      b.means2d.data_ptr<float>(), b.radii.data_ptr<int32_t>(), b.ell ? b.conics.data_ptr<float>() : nullptr,
      b.ell ? b.opacities.data_ptr<float>() : nullptr, b.depths.data_ptr<float>(), b.packed ? 1 : 0,
      b.packed ? b.image_ids.data_ptr<int32_t>() : nullptr, p.I, b.depths.numel(), p.tile_size, p.tile_width,
      p.tile_height, sp.capacity, sp.max_list, b.totals.data_ptr<int64_t>(), sp.ids.data_ptr<int64_t>(),
      sp.flat.data_ptr<int32_t>(), with_offsets ? sp.offsets.data_ptr<int32_t>() : nullptr,
      b.ws1.data_ptr<uint8_t>(), b.ws1_bytes, sp.ws2.data_ptr<uint8_t>(), ws2_bytes, b.stream));
  return sp;
}

// Shapes whose last bucket count chose the presorted path go there directly
// (the bucket count would be thrown away); every 32nd such call takes the
// bucket path again, so a frame that no longer needs the presorted path
// returns to the tile buckets.
bool presorted_by_hint(const IntersectTileInput& input) {
  SpecHint& h = spec_hint(input, input.depths.numel());
  if (h.capacity <= 0 || !presorted_policy(h.longest, h.total)) return false;
  if (++h.presorted_calls >= 32) {
    h.presorted_calls = 0;
    return false;
  }
  return true;
}

// After the read-back: the speculative result when it holds, else the exact
// step; the hint follows this call's M and longest list.
std::vector<array> intersect_bucketed_finish(const IntersectTileInput& input, const BucketState& b, int total,
                                             int64_t longest, bool ungrouped, array* tile_offsets);

std::vector<array> intersect_bucketed_settle(const IntersectTileInput& input, const BucketState& b,
                                             const Speculation& sp, int total, int64_t longest, bool ungrouped,
                                             array* tile_offsets) {
  if (!ungrouped) {
    SpecHint& h = spec_hint(input, b.depths.numel());
    h.capacity = total + std::max<int64_t>(total / 8, 4096);
    h.longest = longest;
    h.total = total;
    h.presorted_calls = 0;
  }
  if (sp.active && !ungrouped && total <= sp.capacity && gsplat_hip_isect_bucket_sort_covers(sp.max_list, longest) &&
      !presorted_policy(longest, total)) {
    if (tile_offsets) *tile_offsets = sp.offsets;
    return {b.tiles_per_gauss, sp.ids.narrow(0, 0, total), sp.flat.narrow(0, 0, total)};
  }
  return intersect_bucketed_finish(input, b, total, longest, ungrouped, tile_offsets);
}

std::vector<array> intersect_bucketed_finish(const IntersectTileInput& input, const BucketState& b, int total,
                                             int64_t longest, bool ungrouped, array* tile_offsets) {
  const auto& p = input.params;
  const int64_t numel = b.depths.numel();
  void* stream = b.stream;
  if (ungrouped) {
    // packed rows not grouped by image: the counts are not valid; the
    // depth-presorted path recounts
    auto out = intersect_presorted(input, stream);
    if (tile_offsets)
      *tile_offsets = gsplat_intersect_offset(out[kIsectIds], p.I, p.tile_width, p.tile_height, input.s);
    return out;
  }
  array ids = at::empty({total}, i64_like(b.means2d));
  array flat = at::empty({total}, i32_like(b.means2d));
  if (tile_offsets) *tile_offsets = at::empty({p.I, p.tile_height, p.tile_width}, i32_like(b.means2d));
  // Lists longer than the LDS tile sort holds are sorted inside the bucket
  // path (split by their leading depth bits); in frames of many entries that
  // hold such lists the depth-presorted path is faster (heavy_6m, 247M
  // entries: 6.97 against 9.98 ms for the intersection, the bucket scatter's
  // partial-line writes dominating), so those take it.
  if (longest <= gsplat_hip_isect_bucket_max_list() || total < kPresortAboveIsects) {
    const size_t ws2_bytes = gsplat_hip_isect_bucket_sort_workspace_size(total);
    array ws2 = workspace(ws2_bytes, b.means2d);
    int32_t* offsets_out = tile_offsets ? tile_offsets->data_ptr<int32_t>() : nullptr;
    if (b.packed)
      check(gsplat_hip_isect_bucket_sort_packed(
          b.means2d.data_ptr<float>(), b.radii.data_ptr<int32_t>(), b.ell ? b.conics.data_ptr<float>() : nullptr,
          b.ell ? b.opacities.data_ptr<float>() : nullptr, b.depths.data_ptr<float>(),
          b.image_ids.data_ptr<int32_t>(), p.I, numel, p.tile_size, p.tile_width, p.tile_height, total, longest,
          ids.data_ptr<int64_t>(), flat.data_ptr<int32_t>(), offsets_out, b.ws1.data_ptr<uint8_t>(), b.ws1_bytes,
          ws2.data_ptr<uint8_t>(), ws2_bytes, stream));
    else if (b.ell)
      check(gsplat_hip_isect_bucket_sort_accutile(
          b.means2d.data_ptr<float>(), b.radii.data_ptr<int32_t>(), b.conics.data_ptr<float>(),
          b.opacities.data_ptr<float>(), b.depths.data_ptr<float>(), p.I, numel, p.tile_size, p.tile_width,
          p.tile_height, total, longest, ids.data_ptr<int64_t>(), flat.data_ptr<int32_t>(), offsets_out,
          b.ws1.data_ptr<uint8_t>(), b.ws1_bytes, ws2.data_ptr<uint8_t>(), ws2_bytes, stream));
    else
      check(gsplat_hip_isect_bucket_sort(b.means2d.data_ptr<float>(), b.radii.data_ptr<int32_t>(),
                                         b.depths.data_ptr<float>(), p.I, numel, p.tile_size, p.tile_width,
                                         p.tile_height, total, longest, ids.data_ptr<int64_t>(),
                                         flat.data_ptr<int32_t>(), offsets_out, b.ws1.data_ptr<uint8_t>(), b.ws1_bytes,
                                         ws2.data_ptr<uint8_t>(), ws2_bytes, stream));
    return {b.tiles_per_gauss, ids, flat};
  }
  // a large frame with a list longer than the LDS tile sort: depth order, then encode + 32-bit sort
  array perm = at::empty({numel}, i32_like(b.means2d));
  array offs = at::empty({numel}, i32_like(b.means2d));
  const size_t ws3_bytes = gsplat_hip_isect_depth_order_workspace_size(numel);
  array ws3 = workspace(ws3_bytes, b.means2d);
  check(gsplat_hip_isect_depth_order(b.depths.data_ptr<float>(), b.tiles_per_gauss.data_ptr<int32_t>(), numel,
                                     perm.data_ptr<int32_t>(), offs.data_ptr<int32_t>(), ws3.data_ptr<uint8_t>(),
                                     ws3_bytes, stream));
  const size_t ws4_bytes = gsplat_hip_isect_encode_sorted_workspace_size(total);
  array ws4 = workspace(ws4_bytes, b.means2d);
  if (b.packed)
    check(gsplat_hip_isect_encode_sorted_packed(
        b.means2d.data_ptr<float>(), b.radii.data_ptr<int32_t>(), b.ell ? b.conics.data_ptr<float>() : nullptr,
        b.ell ? b.opacities.data_ptr<float>() : nullptr, b.image_ids.data_ptr<int32_t>(), b.depths.data_ptr<float>(),
        perm.data_ptr<int32_t>(), offs.data_ptr<int32_t>(), p.I, numel, p.tile_size, p.tile_width, p.tile_height,
        total, ids.data_ptr<int64_t>(), flat.data_ptr<int32_t>(), ws4.data_ptr<uint8_t>(), ws4_bytes, stream));
  else if (b.ell)
    check(gsplat_hip_isect_encode_sorted_accutile(
        b.means2d.data_ptr<float>(), b.radii.data_ptr<int32_t>(), b.conics.data_ptr<float>(),
        b.opacities.data_ptr<float>(), b.depths.data_ptr<float>(), perm.data_ptr<int32_t>(), offs.data_ptr<int32_t>(),
        p.I, numel, p.tile_size, p.tile_width, p.tile_height, total, ids.data_ptr<int64_t>(), flat.data_ptr<int32_t>(),
        ws4.data_ptr<uint8_t>(), ws4_bytes, stream));
  else
    check(gsplat_hip_isect_encode_sorted(b.means2d.data_ptr<float>(), b.radii.data_ptr<int32_t>(),
                                         b.depths.data_ptr<float>(), perm.data_ptr<int32_t>(),
                                         offs.data_ptr<int32_t>(), p.I, numel, p.tile_size, p.tile_width,
                                         p.tile_height, total, ids.data_ptr<int64_t>(), flat.data_ptr<int32_t>(),
                                         ws4.data_ptr<uint8_t>(), ws4_bytes, stream));
  if (tile_offsets)
    check(gsplat_hip_isect_offset(ids.data_ptr<int64_t>(), total, p.I, p.tile_width, p.tile_height,
                                  tile_offsets->data_ptr<int32_t>(), stream));
  return {b.tiles_per_gauss, ids, flat};
}

std::vector<array> intersect_bucketed(const IntersectTileInput& input, void* stream, array* tile_offsets = nullptr) {
  const BucketState b = intersect_bucketed_count(input, stream);
  CountReadback& r = readback_slot();
  start_read_total(b.totals, stream, r, b.readback_words());
  const Speculation sp = speculate(input, b, tile_offsets != nullptr);
  const int total = finish_read_total(r);
  return intersect_bucketed_settle(input, b, sp, total, r.host[1], b.packed && r.host[2] != 0, tile_offsets);
}

// Read-back slots of split intersections, one per pending call: pinned words
// and an event per device, reused once their call has finished (work queued
// between the halves may itself read a count back through readback_slot()).
struct ReadbackPool {
  std::mutex m;
  std::map<int, std::vector<CountReadback>> free;
};
ReadbackPool& readback_pool() {
  static ReadbackPool pool;
  return pool;
}

CountReadback acquire_readback(int dev) {
  {
    std::lock_guard<std::mutex> lock(readback_pool().m);
    auto& v = readback_pool().free[dev];
    if (!v.empty()) {
      CountReadback r = v.back();
      v.pop_back();
      return r;
    }
  }
  CountReadback r;
  void* p = nullptr;
  if (hipHostMalloc(&p, 4 * sizeof(int64_t), hipHostMallocDefault) != hipSuccess)
    throw std::runtime_error("intersect_tile: pinned host allocation for the count failed.");
  r.host = static_cast<int64_t*>(p);
  if (hipEventCreateWithFlags(&r.done, hipEventDisableTiming) != hipSuccess)
    throw std::runtime_error("intersect_tile: event creation failed.");
  return r;
}

void release_readback(int dev, const CountReadback& r) {
  std::lock_guard<std::mutex> lock(readback_pool().m);
  readback_pool().free[dev].push_back(r);
}

std::vector<array> gsplat_intersect_tile_gpu_staged(const IntersectTileInput& input) {
  validate_intersect_tile_input(input);
  check_dense_size(input, "intersect_tile");
  const int64_t n_tiles = static_cast<int64_t>(input.params.tile_width) * input.params.tile_height;
  if (floor_log2_plus_one(input.params.I) + floor_log2_plus_one(n_tiles) > 32)
    throw std::runtime_error("intersect_tile_encode image id and tile id require more than 32 bits.");
  const c10::DeviceGuard guard(input.means2d.device());
  void* stream = stream_for(input.s, input.means2d);
  if (use_bucketed(input) && !presorted_by_hint(input)) return intersect_bucketed(input, stream);
  return intersect_presorted(input, stream);
}

// Counts, then (sort) the depth-presorted encode and 32-bit tile-key sort, or
// (no sort) the pair-major encode.
std::vector<array> intersect_presorted(const IntersectTileInput& input, void* stream) {
  Counted c = count_and_scan(input, stream, !input.params.sort);
  const array means2d = contig(input.means2d);
  const array radii = contig(input.radii);
  const array depths = contig(input.depths);
  if (input.params.sort) {
    // depth-presorted encode + 32-bit key sort; same result as encode
    // followed by the stable 64-bit key sort. The depth order needs only the
    // counts, so it is queued before waiting for their total.
    CountReadback& r = readback_slot();
    start_read_total(c.total, stream, r);
    const int64_t numel = depths.numel();
    array perm = at::empty({numel}, i32_like(means2d));
    array offs = at::empty({numel}, i32_like(means2d));
    const size_t ws1_bytes = gsplat_hip_isect_depth_order_workspace_size(numel);
    array ws1 = workspace(ws1_bytes, means2d);
    check(gsplat_hip_isect_depth_order(depths.data_ptr<float>(), c.tiles_per_gauss.data_ptr<int32_t>(), numel,
                                       perm.data_ptr<int32_t>(), offs.data_ptr<int32_t>(), ws1.data_ptr<uint8_t>(),
                                       ws1_bytes, stream));
    const int total = finish_read_total(r);
    array ids = at::empty({total}, i64_like(means2d));
    array flat = at::empty({total}, i32_like(means2d));
    const size_t ws2_bytes = gsplat_hip_isect_encode_sorted_workspace_size(total);
    array ws2 = workspace(ws2_bytes, means2d);
    if (input.params.packed) {
      const array conics = accutile(input) ? contig(input.conics) : array();
      const array opac = accutile(input) ? contig(input.opacities) : array();
      const array image_ids = contig(input.image_ids.to(at::kInt));
      check(gsplat_hip_isect_encode_sorted_packed(
          means2d.data_ptr<float>(), radii.data_ptr<int32_t>(),
          accutile(input) ? conics.data_ptr<float>() : nullptr, accutile(input) ? opac.data_ptr<float>() : nullptr,
          image_ids.data_ptr<int32_t>(), depths.data_ptr<float>(), perm.data_ptr<int32_t>(), offs.data_ptr<int32_t>(),
          input.params.I, numel, input.params.tile_size, input.params.tile_width, input.params.tile_height, total,
          ids.data_ptr<int64_t>(), flat.data_ptr<int32_t>(), ws2.data_ptr<uint8_t>(), ws2_bytes, stream));
    } else if (accutile(input)) {
      const array conics = contig(input.conics);
      const array opac = contig(input.opacities);
      check(gsplat_hip_isect_encode_sorted_accutile(
          means2d.data_ptr<float>(), radii.data_ptr<int32_t>(), conics.data_ptr<float>(), opac.data_ptr<float>(),
          depths.data_ptr<float>(), perm.data_ptr<int32_t>(), offs.data_ptr<int32_t>(), input.params.I, numel,
          input.params.tile_size, input.params.tile_width, input.params.tile_height, total, ids.data_ptr<int64_t>(),
          flat.data_ptr<int32_t>(), ws2.data_ptr<uint8_t>(), ws2_bytes, stream));
    } else {
      check(gsplat_hip_isect_encode_sorted(means2d.data_ptr<float>(), radii.data_ptr<int32_t>(),
                                           depths.data_ptr<float>(), perm.data_ptr<int32_t>(),
                                           offs.data_ptr<int32_t>(), input.params.I, numel, input.params.tile_size,
                                           input.params.tile_width, input.params.tile_height, total,
                                           ids.data_ptr<int64_t>(), flat.data_ptr<int32_t>(),
                                           ws2.data_ptr<uint8_t>(), ws2_bytes, stream));
    }
    return {c.tiles_per_gauss, ids, flat};
  }
  const int total = read_total(c.total, stream);
  auto enc = encode_unsorted(input, means2d, radii, depths, c.offsets, total, stream);
  return {c.tiles_per_gauss, enc[0], enc[1]};
}

std::vector<array> gsplat_intersect_tile(const IntersectTileInput& input) {
  validate_intersect_tile_input(input);
  return gsplat_intersect_tile_gpu_staged(input);
}

// The sorted lists and their offsets by the depth-presorted path.
std::vector<array> gsplat_intersect_tile_with_offsets_unbucketed(const IntersectTileInput& input) {
  const auto& p = input.params;
  check_dense_size(input, "intersect_tile");
  const int64_t n_tiles = static_cast<int64_t>(p.tile_width) * p.tile_height;
  if (floor_log2_plus_one(p.I) + floor_log2_plus_one(n_tiles) > 32)
    throw std::runtime_error("intersect_tile_encode image id and tile id require more than 32 bits.");
  const c10::DeviceGuard guard(input.means2d.device());
  auto out = intersect_presorted(input, stream_for(input.s, input.means2d));
  out.push_back(gsplat_intersect_offset(out[kIsectIds], p.I, p.tile_width, p.tile_height, input.s));
  return out;
}

std::vector<array> gsplat_intersect_tile_with_offsets(const IntersectTileInput& input) {
  validate_intersect_tile_input(input);
  if (!input.params.sort) throw std::runtime_error("intersect_tile_with_offsets needs sort = true.");
  const auto& p = input.params;
  if (use_bucketed(input) && !presorted_by_hint(input)) {
    check_dense_size(input, "intersect_tile");
    const int64_t n_tiles = static_cast<int64_t>(p.tile_width) * p.tile_height;
    if (floor_log2_plus_one(p.I) + floor_log2_plus_one(n_tiles) > 32)
      throw std::runtime_error("intersect_tile_encode image id and tile id require more than 32 bits.");
    const c10::DeviceGuard guard(input.means2d.device());
    array offsets;
    auto out = intersect_bucketed(input, stream_for(input.s, input.means2d), &offsets);
    out.push_back(offsets);
    return out;
  }
  return gsplat_intersect_tile_with_offsets_unbucketed(input);
}

struct PendingIntersect {
  IntersectTileInput input;
  bool bucketed = false, finished = false;
  int dev = 0;
  BucketState state;
  Speculation spec;
  CountReadback rb;
  std::vector<array> result;
  ~PendingIntersect() {
    if (bucketed && !finished) {
      // the read-back may still be in flight: wait for it before the slot is reused
      (void)hipEventSynchronize(rb.done);
      release_readback(dev, rb);
    }
  }
};

std::shared_ptr<PendingIntersect> gsplat_intersect_tile_offsets_begin(const IntersectTileInput& input) {
  validate_intersect_tile_input(input);
  if (!input.params.sort) throw std::runtime_error("intersect_tile_with_offsets needs sort = true.");
  const auto& p = input.params;
  auto pending = std::make_shared<PendingIntersect>();
  pending->input = input;
  if (!use_bucketed(input) || presorted_by_hint(input)) {
    pending->result = gsplat_intersect_tile_with_offsets_unbucketed(input);
    pending->finished = true;
    return pending;
  }
  check_dense_size(input, "intersect_tile");
  const int64_t n_tiles = static_cast<int64_t>(p.tile_width) * p.tile_height;
  if (floor_log2_plus_one(p.I) + floor_log2_plus_one(n_tiles) > 32)
    throw std::runtime_error("intersect_tile_encode image id and tile id require more than 32 bits.");
  const c10::DeviceGuard guard(input.means2d.device());
  void* stream = stream_for(input.s, input.means2d);
  pending->state = intersect_bucketed_count(input, stream);
  if (hipGetDevice(&pending->dev) != hipSuccess) throw std::runtime_error("intersect_tile: no current HIP device.");
  pending->rb = acquire_readback(pending->dev);
  pending->bucketed = true;
  start_read_total(pending->state.totals, stream, pending->rb, pending->state.readback_words());
  pending->spec = speculate(input, pending->state, true);
  return pending;
}

std::vector<array> gsplat_intersect_tile_offsets_end(const std::shared_ptr<PendingIntersect>& pending) {
  if (!pending) throw std::runtime_error("intersect_tile_offsets_end: no pending intersection.");
  if (pending->finished) return pending->result;
  const c10::DeviceGuard guard(pending->input.means2d.device());
  const int total = finish_read_total(pending->rb);
  const int64_t longest = pending->rb.host[1];
  const bool ungrouped = pending->state.packed && pending->rb.host[2] != 0;
  pending->finished = true;
  release_readback(pending->dev, pending->rb);
  array offsets;
  auto out = intersect_bucketed_settle(pending->input, pending->state, pending->spec, total, longest, ungrouped,
                                       &offsets);
  out.push_back(offsets);
  pending->result = out;
  pending->state = BucketState();  // the count workspace goes back to the allocator
  pending->spec = Speculation();
  return out;
}

array gsplat_intersect_offset(const array& isect_ids, int I, int tile_width, int tile_height, StreamOrDevice s) {
  if (I <= 0 || tile_width <= 0 || tile_height <= 0)
    throw std::runtime_error("intersect_offset expects positive image and tile dimensions.");
  if (isect_ids.scalar_type() != at::kLong) throw std::runtime_error("intersect_offset expects int64 isect_ids.");
  require_device(isect_ids, "isect_ids");
  const c10::DeviceGuard guard(isect_ids.device());
  const array ids = contig(isect_ids);
  array out = at::empty({I, tile_height, tile_width}, i32_like(ids));
  check(gsplat_hip_isect_offset(ids.data_ptr<int64_t>(), ids.numel(), I, tile_width, tile_height,
                                out.data_ptr<int32_t>(), stream_for(s, ids)));
  return out;
}

}  // namespace gsplat_core
