// Internal helpers shared by the HIP translation units of libriemann_hip.
// gfx950 only: wave64, 64-lane ballots, 16-byte global loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <stdexcept>
#include <string>

#include "riemann_hip.h"

namespace rhip {

constexpr int kWave = 64;
constexpr uint64_t kEmptyWord = ~0ull;

// One hash slot: the key word (packed coordinates, or hash<<32 | unique row
// in row-reference mode), the first input row that inserted it (atomicMin
// target during the build) and the unique row index lookups return.
struct alignas(16) Slot {
  uint64_t word;
  uint32_t first_row;
  uint32_t uid;
};
static_assert(sizeof(Slot) == 16, "slot must stay 16 bytes");

// Error plumbing: entry points catch rhip::Error and return its status with
// the message stored for rhip_last_error().
struct Error : std::runtime_error {
  int status;
  Error(int s, const std::string &m) : std::runtime_error(m), status(s) {}
};

void set_last_error(const std::string &msg);

// The calling thread's pinned host buffer of at least `bytes` for small
// device-to-host read-backs (valid until the thread's next request): ptr for
// the host, dev the address a kernel writes it through (null when the
// runtime gives none; then read back with a copy).
struct PinnedReadback {
  void *ptr;
  void *dev;
};
PinnedReadback pinned_readback(size_t bytes);

#define RHIP_CHECK_ARG(cond, msg)                                              \
  do {                                                                         \
    if (!(cond))                                                               \
      throw ::rhip::Error(RHIP_ERR_INVALID, std::string(__func__) + ": " + msg); \
  } while (0)

#define RHIP_HIP(call)                                                         \
  do {                                                                         \
    hipError_t e_ = (call);                                                    \
    if (e_ != hipSuccess)                                                      \
      throw ::rhip::Error(RHIP_ERR_HIP, std::string(#call) + " failed: " +     \
                                            hipGetErrorString(e_));            \
  } while (0)

#define RHIP_LAUNCH_CHECK() RHIP_HIP(hipGetLastError())

// Runs `body` and converts exceptions into a status code.
template <typename F> int guarded(F &&body) {
  try {
    body();
    return RHIP_OK;
  } catch (const Error &e) {
    set_last_error(e.what());
    return e.status;
  } catch (const std::exception &e) {
    set_last_error(e.what());
    return RHIP_ERR_HIP;
  }
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Bump allocator over a caller workspace (256-byte aligned pieces).
struct Carve {
  char *base;
  size_t used = 0, cap;
  Carve(void *p, size_t c) : base(static_cast<char *>(p)), cap(c) {}
  template <typename T> T *take(size_t count) {
    size_t off = align_up(used, 256);
    size_t need = off + count * sizeof(T);
    if (base != nullptr && need > cap)
      throw Error(RHIP_ERR_WORKSPACE, "workspace too small: need " +
                                          std::to_string(need) + " bytes, have " +
                                          std::to_string(cap));
    used = need;
    return base ? reinterpret_cast<T *>(base + off) : nullptr;
  }
};

// ---------------------------------------------------------------- device

// Stable (key, int32 value) radix sorts over bits [0, end_bit) of the key
// (sort.hip). *_bytes gives the scratch size for n items.
size_t sort_pairs_u32_bytes(int64_t n);
size_t sort_pairs_u64_bytes(int64_t n);
void sort_pairs_u32(void *tmp, size_t tmp_bytes, const uint32_t *kin, uint32_t *kout,
                    const int32_t *vin, int32_t *vout, int64_t n, int end_bit, hipStream_t s);
void sort_pairs_u64(void *tmp, size_t tmp_bytes, const uint64_t *kin, uint64_t *kout,
                    const int32_t *vin, int32_t *vout, int64_t n, int end_bit, hipStream_t s);

// MurmurHash3 64-bit finalizer (Appleby, public domain) as the slot mixer.
__device__ __forceinline__ uint64_t mix64(uint64_t k) {
  k ^= k >> 33;
  k *= 0xff51afd7ed558ccdull;
  k ^= k >> 33;
  k *= 0xc4ceb9fe1a85ec53ull;
  k ^= k >> 33;
  return k;
}

// Table parameters passed by value to kernels.
struct TableView {
  Slot *slots;
  uint64_t mask;
  const int32_t *rows; // unique coordinates (row-reference mode probes these)
  int32_t ncol;
  int32_t mode;
  int32_t lo[RHIP_MAX_COLS];
  uint32_t span[RHIP_MAX_COLS]; // hi - lo
  int32_t shift[RHIP_MAX_COLS];
  int32_t tz[RHIP_MAX_COLS];    // common trailing zeros of (c - lo)
  // brick index (bricks NULL when absent)
  const int32_t *order;
  const struct Brick *bricks;
  int32_t morton_bits, levels;
  int32_t dims[RHIP_MAX_COLS];
};

// One entry of a table's brick grid: occupancy of the brick's cells (bit =
// the cell's Morton index within the brick) and the locality-order position
// of the brick's first row; the brick's rows follow it in cell order.
struct alignas(16) Brick {
  uint64_t mask;
  int32_t base;
  int32_t pad;
};
static_assert(sizeof(Brick) == 16, "brick entry must stay 16 bytes");

inline TableView make_view(const rhip_table &t) {
  TableView v{};
  v.slots = static_cast<Slot *>(t.slots);
  v.mask = static_cast<uint64_t>(t.capacity) - 1;
  v.rows = t.rows;
  v.ncol = t.ncol;
  v.mode = t.mode;
  for (int c = 0; c < RHIP_MAX_COLS; ++c) {
    v.lo[c] = t.lo[c];
    v.span[c] = static_cast<uint32_t>(static_cast<int64_t>(t.hi[c]) - t.lo[c]);
    v.shift[c] = t.shift[c];
  }
  for (int c = 0; c < RHIP_MAX_COLS; ++c) {
    v.tz[c] = t.tz[c];
    v.dims[c] = t.brick_dims[c];
  }
  v.order = t.order;
  v.bricks = static_cast<const Brick *>(t.bricks);
  v.morton_bits = t.morton_bits;
  v.levels = t.brick_levels;
  return v;
}

// Pack a row into its 63-bit key; false when a column leaves [lo, hi]
// (such a row cannot be in the table).
__device__ __forceinline__ bool pack_row(const TableView &t, const int32_t *c,
                                         uint64_t &key) {
  uint64_t k = 0;
#pragma unroll
  for (int i = 0; i < RHIP_MAX_COLS; ++i) {
    if (i < t.ncol) {
      uint32_t d = static_cast<uint32_t>(c[i]) - static_cast<uint32_t>(t.lo[i]);
      if (d > t.span[i])
        return false;
      k |= static_cast<uint64_t>(d) << t.shift[i];
    }
  }
  key = k;
  return true;
}

// 32-bit row hash for row-reference mode.
__device__ __forceinline__ uint32_t hash_row(const int32_t *c, int ncol) {
  uint64_t h = 0x9e3779b97f4a7c15ull;
  for (int i = 0; i < ncol; ++i)
    h = mix64(h ^ static_cast<uint32_t>(c[i]));
  return static_cast<uint32_t>(h >> 32);
}

__device__ __forceinline__ bool rows_equal(const int32_t *a, const int32_t *b,
                                           int ncol) {
  for (int i = 0; i < ncol; ++i)
    if (a[i] != b[i])
      return false;
  return true;
}

// Probe for a row (coordinates in registers/array `c`); returns its unique
// index or -1.
__device__ __forceinline__ int32_t table_find(const TableView &t,
                                              const int32_t *c) {
  if (t.mode == RHIP_KEY_PACKED64) {
    uint64_t key;
    if (!pack_row(t, c, key))
      return -1;
    uint64_t h = mix64(key) & t.mask;
    while (true) {
      Slot s = t.slots[h];
      if (s.word == key)
        return static_cast<int32_t>(s.uid);
      if (s.word == kEmptyWord)
        return -1;
      h = (h + 1) & t.mask;
    }
  } else {
    uint32_t hr = hash_row(c, t.ncol);
    uint64_t h = mix64(hr) & t.mask;
    while (true) {
      Slot s = t.slots[h];
      if (s.word == kEmptyWord)
        return -1;
      if (static_cast<uint32_t>(s.word >> 32) == hr) {
        uint32_t u = static_cast<uint32_t>(s.word);
        if (rows_equal(t.rows + static_cast<int64_t>(u) * t.ncol, c, t.ncol))
          return static_cast<int32_t>(u);
      }
      h = (h + 1) & t.mask;
    }
  }
}

// floor(a / s) * s for s > 0, exact in integers. The reference computes it
// through float division (CPU: floor((float)a / s) * s, engine/grid/
// stencil.hpp:46-53; GPU: __float2int_rd(__fdiv_rd(a, s)) * s,
// lattice_gpu.cu:328-332); both equal this for |a| < 2^24.
__device__ __forceinline__ int32_t floor_align(int32_t a, int32_t s) {
  int32_t q = a / s;
  if ((a % s) != 0 && a < 0)
    --q;
  return q * s;
}

// Stride of each spatial column, by value.
struct StrideArg {
  int32_t s[RHIP_MAX_COLS];
};

// Workgroup id -> tile id. Workgroups are dealt to the 8 XCDs of an MI355X
// round-robin (id b runs on XCD b % 8); this mapping hands each XCD runs of
// kXcdRun consecutive tiles, so tiles that share neighbour rows share an L2,
// while the runs stay interleaved over the whole map to keep the XCDs
// balanced. The grid is padded to a multiple of 8 * kXcdRun (padding ids map
// past the last tile).
constexpr int kXcds = 8;
constexpr int kXcdRun = 16;
__device__ __forceinline__ int64_t xcd_tile(int64_t b) {
  const int64_t x = b % kXcds, m = b / kXcds;
  return ((m / kXcdRun) * kXcds + x) * kXcdRun + (m % kXcdRun);
}
inline int64_t xcd_grid(int64_t tiles) {
  return ceil_div(tiles, kXcds * kXcdRun) * kXcds * kXcdRun;
}

// Lane index within the wave and wave-level prefix of a predicate.
__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(
                                       static_cast<uint32_t>(mask), 0u));
}

// Runs of lanes: `heads` has a bit for every lane that starts a run (lane 0
// always does); the first lane of this lane's run.
__device__ __forceinline__ int run_head(uint64_t heads) {
  const int lane = lane_id();
  const uint64_t upto = lane == kWave - 1 ? ~0ull : (2ull << lane) - 1ull;
  return 63 - __clzll(heads & upto);
}

// Whether this lane's coordinate row equals the previous lane's (lane 0 and
// lanes with valid false never do); every lane of the wave must call it.
__device__ __forceinline__ bool repeats_prev_row(const int32_t (&c)[RHIP_MAX_COLS], bool valid) {
  bool same = valid && lane_id() > 0;
#pragma unroll
  for (int j = 0; j < RHIP_MAX_COLS; ++j)
    same = (__shfl_up(c[j], 1, kWave) == c[j]) && same;
  return same;
}

// Segmented exclusive scan, one 1024-lane workgroup per segment (blockIdx.x):
// base[s*m + i] = sum(counts[s*m .. s*m+i)), total[s] = sum of segment s.
// The segment goes in chunks of 4096 entries, four consecutive ones per lane
// (loads issued together), one workgroup scan per chunk and a carry.
// segment_scan is the workgroup's part; it returns the segment's total in
// every thread.
template <typename TIn>
__device__ int64_t segment_scan(const TIn *counts, int64_t m, int64_t *base) {
  constexpr int kWaves = 1024 / kWave;
  __shared__ int64_t wave_sum[kWaves];
  const int t = threadIdx.x, lane = t & (kWave - 1), w = t / kWave;
  const int64_t seg = static_cast<int64_t>(blockIdx.x) * m;
  int64_t carry = 0;
  for (int64_t c0 = 0; c0 < m; c0 += 4 * 1024) {
    const int64_t e0 = c0 + 4 * t;
    int64_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v[i] = e0 + i < m ? static_cast<int64_t>(counts[seg + e0 + i]) : 0;
    const int64_t sum = v[0] + v[1] + v[2] + v[3];
    int64_t incl = sum;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int64_t o = __shfl_up(incl, off, kWave);
      if (lane >= off)
        incl += o;
    }
    if (lane == kWave - 1)
      wave_sum[w] = incl;
    __syncthreads();
    int64_t before = carry, chunk = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      const int64_t ws = wave_sum[i];
      before += i < w ? ws : 0;
      chunk += ws;
    }
    int64_t run = before + incl - sum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (e0 + i < m)
        base[seg + e0 + i] = run;
      run += v[i];
    }
    carry += chunk;
    __syncthreads(); // wave_sum is rewritten by the next chunk
  }
  return carry;
}

template <typename TIn>
__global__ __launch_bounds__(1024) void scan_kernel(const TIn *counts, int64_t m,
                                                    int64_t *base, int64_t *total) {
  const int64_t carry = segment_scan(counts, m, base);
  if (threadIdx.x == 0)
    total[blockIdx.x] = carry;
}

} // namespace rhip
