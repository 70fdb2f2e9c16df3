// Coordinate hashing for gfx950: dedup of int32 coordinate rows into an
// open-addressing table with 16-byte slots and linear probing.
//
// Semantics follow CoordinateMapCPU::insert_and_map<true>
// (RiemannEngine/engine/grid/lattice_cpu.hpp:419-444): unique rows are
// numbered by first occurrence, mapping[u] is the first input row of unique
// row u and inverse[r] the unique row of input row r. The GPU design differs
// from the reference's cuDF map (which CASes a pointer to the row and keeps
// the race winner, engine/grid/lattice_gpu.cu:26-51): keys are packed into
// one integer from the set's own column ranges, the first occurrence wins by
// atomicMin on the row index, and the unique numbering is a prefix sum over
// "is first" flags in row order, so the result is deterministic.
#include <algorithm>
#include <climits>
#include <cstring>

#include "rhip_internal.hpp"

namespace rhip {

constexpr int kBlock = 256;

__global__ void minmax_init_kernel(int32_t *mm, int ncol) {
  int c = threadIdx.x;
  if (c < ncol) {
    mm[c] = INT_MAX;
    mm[ncol + c] = INT_MIN;
    mm[2 * ncol + c] = 0;
  }
}

// Column-wise min, max and OR of (value ^ row 0's value) of coords [n, ncol]
// (the last gives the lowest bit in which a column varies); block-reduced in
// LDS then merged with global atomics.
__global__ __launch_bounds__(kBlock) void minmax_kernel(const int32_t *coords,
                                                        int64_t n, int ncol,
                                                        int32_t *mm) {
  __shared__ int32_t smin[RHIP_MAX_COLS], smax[RHIP_MAX_COLS], sor[RHIP_MAX_COLS];
  if (threadIdx.x < RHIP_MAX_COLS) {
    smin[threadIdx.x] = INT_MAX;
    smax[threadIdx.x] = INT_MIN;
    sor[threadIdx.x] = 0;
  }
  __syncthreads();
  int32_t lmin[RHIP_MAX_COLS], lmax[RHIP_MAX_COLS], lor[RHIP_MAX_COLS], c0[RHIP_MAX_COLS];
#pragma unroll
  for (int c = 0; c < RHIP_MAX_COLS; ++c) {
    lmin[c] = INT_MAX;
    lmax[c] = INT_MIN;
    lor[c] = 0;
    c0[c] = c < ncol ? coords[c] : 0;
  }
#pragma unroll 4
  for (int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x; r < n;
       r += (int64_t)gridDim.x * kBlock) {
    const int32_t *row = coords + r * ncol;
#pragma unroll
    for (int c = 0; c < RHIP_MAX_COLS; ++c) {
      if (c < ncol) {
        int32_t v = row[c];
        lmin[c] = min(lmin[c], v);
        lmax[c] = max(lmax[c], v);
        lor[c] |= v ^ c0[c];
      }
    }
  }
#pragma unroll
  for (int c = 0; c < RHIP_MAX_COLS; ++c) {
    if (c < ncol) {
      int32_t a = lmin[c], b = lmax[c], o = lor[c];
      for (int off = 32; off > 0; off >>= 1) {
        a = min(a, __shfl_xor(a, off));
        b = max(b, __shfl_xor(b, off));
        o |= __shfl_xor(o, off);
      }
      if (lane_id() == 0) {
        atomicMin(&smin[c], a);
        atomicMax(&smax[c], b);
        atomicOr(&sor[c], o);
      }
    }
  }
  __syncthreads();
  if (threadIdx.x < ncol) {
    atomicMin(&mm[threadIdx.x], smin[threadIdx.x]);
    atomicMax(&mm[ncol + threadIdx.x], smax[threadIdx.x]);
    atomicOr(&mm[2 * ncol + threadIdx.x], sor[threadIdx.x]);
  }
}

__global__ __launch_bounds__(kBlock) void slots_init_kernel(Slot *slots,
                                                            int64_t cap) {
  int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (i < cap) {
    Slot s;
    s.word = kEmptyWord;
    s.first_row = 0xffffffffu;
    s.uid = 0xffffffffu;
    slots[i] = s;
  }
}

// One lane per input row: claim or find the row's slot, then lower the
// slot's first_row to this row if it is earlier.
__global__ __launch_bounds__(kBlock) void insert_kernel(const int32_t *coords,
                                                        int64_t n,
                                                        TableView t,
                                                        uint32_t *slot_of_row) {
  int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (r >= n)
    return;
  int32_t c[RHIP_MAX_COLS];
#pragma unroll
  for (int i = 0; i < RHIP_MAX_COLS; ++i)
    c[i] = i < t.ncol ? coords[r * t.ncol + i] : 0;

  uint64_t key, h;
  uint32_t hr = 0;
  if (t.mode == RHIP_KEY_PACKED64) {
    pack_row(t, c, key); // always in range: the bounds come from this set
    h = mix64(key) & t.mask;
  } else {
    hr = hash_row(c, t.ncol);
    key = (static_cast<uint64_t>(hr) << 32) | static_cast<uint32_t>(r);
    h = mix64(hr) & t.mask;
  }
  while (true) {
    uint64_t *wp = &t.slots[h].word;
    uint64_t w = __hip_atomic_load(wp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (w == kEmptyWord) {
      uint64_t prev = atomicCAS(reinterpret_cast<unsigned long long *>(wp),
                                kEmptyWord, key);
      if (prev == kEmptyWord)
        break; // claimed
      w = prev;
    }
    bool same;
    if (t.mode == RHIP_KEY_PACKED64) {
      same = (w == key);
    } else {
      same = static_cast<uint32_t>(w >> 32) == hr &&
             rows_equal(coords + static_cast<int64_t>(static_cast<uint32_t>(w)) *
                                     t.ncol,
                        c, t.ncol);
    }
    if (same)
      break;
    h = (h + 1) & t.mask;
  }
  atomicMin(&t.slots[h].first_row, static_cast<uint32_t>(r));
  slot_of_row[r] = static_cast<uint32_t>(h);
}

// Per-block count of rows that are the first occurrence of their key.
__global__ __launch_bounds__(kBlock) void count_first_kernel(
    int64_t n, const Slot *slots, const uint32_t *slot_of_row,
    int32_t *block_counts) {
  __shared__ int32_t wave_counts[kBlock / kWave];
  int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  bool first = r < n && slots[slot_of_row[r]].first_row == static_cast<uint32_t>(r);
  uint64_t b = __ballot(first);
  if (lane_id() == 0)
    wave_counts[threadIdx.x / kWave] = __popcll(b);
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t s = 0;
    for (int w = 0; w < kBlock / kWave; ++w)
      s += wave_counts[w];
    block_counts[blockIdx.x] = s;
  }
}

// First rows get uid = block base + rank within the block; they also write
// mapping[uid] and the unique coordinates.
__global__ __launch_bounds__(kBlock) void assign_uid_kernel(
    const int32_t *coords, int64_t n, int ncol, const Slot *slots,
    const uint32_t *slot_of_row, const int64_t *block_base, int32_t *uid_by_row,
    int64_t *mapping, int32_t *unique_coords) {
  __shared__ int32_t wave_counts[kBlock / kWave];
  int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  bool first = r < n && slots[slot_of_row[r]].first_row == static_cast<uint32_t>(r);
  uint64_t b = __ballot(first);
  const int w = threadIdx.x / kWave;
  if (lane_id() == 0)
    wave_counts[w] = __popcll(b);
  __syncthreads();
  int32_t before = 0;
  for (int i = 0; i < w; ++i)
    before += wave_counts[i];
  if (first) {
    int64_t uid = block_base[blockIdx.x] + before + lanes_below(b);
    uid_by_row[r] = static_cast<int32_t>(uid);
    mapping[uid] = r;
    for (int c = 0; c < ncol; ++c)
      unique_coords[uid * ncol + c] = coords[r * ncol + c];
  }
}

// inverse[r] = uid of r's first occurrence; first rows publish their uid in
// the slot (and, in row-reference mode, re-point the key at the unique row).
__global__ __launch_bounds__(kBlock) void resolve_kernel(
    const int32_t *coords, int64_t n, TableView t, const uint32_t *slot_of_row,
    const int32_t *uid_by_row, int64_t *inverse) {
  int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (r >= n)
    return;
  uint32_t h = slot_of_row[r];
  uint32_t fr = t.slots[h].first_row;
  int32_t uid = uid_by_row[fr];
  if (inverse)
    inverse[r] = uid;
  if (fr == static_cast<uint32_t>(r)) {
    t.slots[h].uid = static_cast<uint32_t>(uid);
    if (t.mode == RHIP_KEY_ROWREF) {
      uint32_t hr = static_cast<uint32_t>(t.slots[h].word >> 32);
      t.slots[h].word = (static_cast<uint64_t>(hr) << 32) | static_cast<uint32_t>(uid);
    }
  }
}

__global__ __launch_bounds__(kBlock) void lookup_kernel(TableView t,
                                                        const int32_t *queries,
                                                        int64_t n,
                                                        int32_t *result) {
  int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (i >= n)
    return;
  int32_t c[RHIP_MAX_COLS];
#pragma unroll
  for (int j = 0; j < RHIP_MAX_COLS; ++j)
    c[j] = j < t.ncol ? queries[i * t.ncol + j] : 0;
  result[i] = table_find(t, c);
}

// Sort keys of the locality order. morton_bits > 0: batch offset in the top
// bits, then the spatial offsets from the column minima, each shifted right
// by the column's common trailing zeros, bit-interleaved, morton_bits bits
// each (bit i of column c at i * D + (D - c)); else the packed key.
__global__ __launch_bounds__(kBlock) void pack_keys_kernel(TableView t, int64_t n,
                                                           int morton_bits,
                                                           uint64_t *keys,
                                                           int32_t *rows) {
  int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (i >= n)
    return;
  int32_t c[RHIP_MAX_COLS];
#pragma unroll
  for (int j = 0; j < RHIP_MAX_COLS; ++j)
    c[j] = j < t.ncol ? t.rows[i * t.ncol + j] : 0;
  uint64_t key = 0;
  if (morton_bits > 0) {
    const int D = t.ncol - 1;
    for (int j = 1; j <= D; ++j) {
      const uint32_t v =
          (static_cast<uint32_t>(c[j]) - static_cast<uint32_t>(t.lo[j])) >> t.tz[j];
      for (int b = 0; b < morton_bits; ++b)
        key |= static_cast<uint64_t>((v >> b) & 1u) << (b * D + (D - j));
    }
    key |= static_cast<uint64_t>(static_cast<uint32_t>(c[0]) - static_cast<uint32_t>(t.lo[0]))
           << (morton_bits * D);
  } else {
    pack_row(t, c, key);
  }
  keys[i] = key;
  rows[i] = static_cast<int32_t>(i);
}

__global__ __launch_bounds__(kBlock) void brick_clear_kernel(Brick *grid, int64_t n) {
  const int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (i < n) {
    Brick b;
    b.mask = 0;
    b.base = -1;
    b.pad = 0;
    grid[i] = b;
  }
}

// The first row of each brick in the locality order (skeys: the sorted
// Morton keys, whose low cbits bits are the cell within the brick) writes the
// brick's grid entry: the OR of its rows' cell bits and its own position.
// A brick has at most 64 cells, so the scan of its rows is short.
__global__ __launch_bounds__(kBlock) void brick_fill_kernel(TableView t,
                                                            const uint64_t *__restrict__ skeys,
                                                            const int32_t *__restrict__ order,
                                                            int64_t n, int cbits,
                                                            Brick *__restrict__ grid) {
  const int64_t j = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (j >= n)
    return;
  const uint64_t code = skeys[j] >> cbits;
  if (j > 0 && (skeys[j - 1] >> cbits) == code)
    return;
  const uint64_t cmask = (1ull << cbits) - 1;
  uint64_t mask = 0;
  for (int64_t i = j; i < n && i < j + 64; ++i) {
    const uint64_t k = skeys[i];
    if ((k >> cbits) != code)
      break;
    mask |= 1ull << (k & cmask);
  }
  const int64_t r = order[j];
  int64_t g = static_cast<uint32_t>(t.rows[r * t.ncol]) - static_cast<uint32_t>(t.lo[0]);
  for (int c = 1; c < t.ncol; ++c) {
    const uint32_t v =
        (static_cast<uint32_t>(t.rows[r * t.ncol + c]) - static_cast<uint32_t>(t.lo[c])) >>
        t.tz[c];
    g = g * t.dims[c] + (v >> t.levels);
  }
  Brick b;
  b.mask = mask;
  b.base = static_cast<int32_t>(j);
  b.pad = 0;
  grid[g] = b;
}

__global__ __launch_bounds__(kBlock) void iota_kernel(int64_t n, int32_t *order,
                                                      int32_t *pos) {
  int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (i < n) {
    order[i] = static_cast<int32_t>(i);
    if (pos)
      pos[i] = static_cast<int32_t>(i);
  }
}

__global__ __launch_bounds__(kBlock) void invert_perm_kernel(int64_t n,
                                                             const int32_t *order,
                                                             int32_t *pos) {
  int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (i < n)
    pos[order[i]] = static_cast<int32_t>(i);
}

__global__ __launch_bounds__(kBlock) void stride_kernel(const int32_t *in,
                                                        int64_t n, int ncol,
                                                        StrideArg st,
                                                        int32_t *out) {
  int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (i >= n * ncol)
    return;
  int c = static_cast<int>(i % ncol);
  int32_t v = in[i];
  out[i] = c == 0 ? v : floor_align(v, st.s[c - 1]);
}

// Generative expansion: out row i*K + k = in row i + offsets[k] (batch kept,
// wrap-around int32 arithmetic as the coordinate type has).
__global__ __launch_bounds__(kBlock) void expand_kernel(const int32_t *in, int64_t n, int ncol,
                                                        int K, const int32_t *offsets,
                                                        int32_t *out) {
  const int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (i >= n * K * ncol)
    return;
  const int64_t row = i / ncol;
  const int c = static_cast<int>(i % ncol);
  const int64_t src = row / K;
  const int k = static_cast<int>(row % K);
  const int32_t v = in[src * ncol + c];
  out[i] = c == 0 ? v
                  : static_cast<int32_t>(static_cast<uint32_t>(v) +
                                         static_cast<uint32_t>(offsets[k * (ncol - 1) + c - 1]));
}

// ------------------------------------------------------------------ host

static int64_t table_capacity(int64_t n) {
  int64_t cap = 64;
  while (cap < 2 * n)
    cap <<= 1;
  return cap;
}

struct HashWs {
  int32_t *minmax;
  uint32_t *slot_of_row;
  int32_t *uid_by_row;
  int32_t *block_counts;
  int64_t *block_base;
  int64_t *total;
};

static HashWs carve_hash(Carve &cv, int64_t n, int ncol) {
  HashWs w;
  const int64_t nb = std::max<int64_t>(1, ceil_div(n, kBlock));
  w.minmax = cv.take<int32_t>(3 * RHIP_MAX_COLS);
  w.slot_of_row = cv.take<uint32_t>(std::max<int64_t>(n, 1));
  w.uid_by_row = cv.take<int32_t>(std::max<int64_t>(n, 1));
  w.block_counts = cv.take<int32_t>(nb);
  w.block_base = cv.take<int64_t>(nb);
  w.total = cv.take<int64_t>(1);
  (void)ncol;
  return w;
}

static int bit_width_u32(uint32_t v) { return v == 0 ? 0 : 32 - __builtin_clz(v); }

} // namespace rhip

using namespace rhip;

extern "C" size_t rhip_table_bytes(int64_t n) {
  return static_cast<size_t>(table_capacity(n < 0 ? 0 : n)) * sizeof(Slot);
}

extern "C" int rhip_hash_workspace_bytes(int64_t n, int32_t ncol,
                                         size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(n >= 0, "n must be >= 0");
    Carve cv(nullptr, 0);
    carve_hash(cv, n, ncol);
    *bytes = cv.used + 256;
  });
}

extern "C" int rhip_hash_build(const int32_t *coords, int64_t n, int32_t ncol,
                               void *slots, size_t slots_bytes, void *workspace,
                               size_t workspace_bytes, int32_t *unique_coords,
                               int64_t *mapping, int64_t *inverse,
                               rhip_table *table, hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(table != nullptr, "table is null");
    RHIP_CHECK_ARG(n >= 0 && n < INT32_MAX, "row count must be in [0, 2^31)");
    RHIP_CHECK_ARG(ncol >= 2 && ncol <= RHIP_MAX_COLS,
                   "ncol must be in [2, " + std::to_string(RHIP_MAX_COLS) + "]");
    RHIP_CHECK_ARG(slots != nullptr, "slots is null");
    RHIP_CHECK_ARG(n == 0 || (coords && unique_coords && mapping),
                   "coords/unique_coords/mapping must be non-null");
    const int64_t cap = table_capacity(n);
    RHIP_CHECK_ARG(slots_bytes >= static_cast<size_t>(cap) * sizeof(Slot),
                   "slots buffer smaller than rhip_table_bytes(n)");
    Carve cv(workspace, workspace_bytes);
    RHIP_CHECK_ARG(workspace != nullptr, "workspace is null");
    HashWs w = carve_hash(cv, n, ncol);

    std::memset(table, 0, sizeof(*table));
    table->slots = slots;
    table->capacity = cap;
    table->rows = unique_coords;
    table->ncol = ncol;
    Slot *sl = static_cast<Slot *>(slots);
    hipLaunchKernelGGL(slots_init_kernel, dim3(ceil_div(cap, kBlock)),
                       dim3(kBlock), 0, stream, sl, cap);
    RHIP_LAUNCH_CHECK();
    if (n == 0) {
      table->mode = RHIP_KEY_PACKED64;
      table->n_unique = 0;
      for (int c = 0; c < ncol; ++c)
        table->hi[c] = -1; // empty range: every probe misses on span check
      return;
    }

    // Column bounds -> packing layout (batch column in the top bits so the
    // packed order is batch-major lexicographic).
    hipLaunchKernelGGL(minmax_init_kernel, dim3(1), dim3(RHIP_MAX_COLS), 0,
                       stream, w.minmax, ncol);
    const int64_t nb = ceil_div(n, kBlock);
    // few workgroups: each merges its result with 2 * ncol atomics on the
    // same 2 * ncol addresses, which serialise
    hipLaunchKernelGGL(minmax_kernel, dim3(std::min<int64_t>(nb, 256)),
                       dim3(kBlock), 0, stream, coords, n, ncol, w.minmax);
    RHIP_LAUNCH_CHECK();
    int32_t mm[3 * RHIP_MAX_COLS];
    RHIP_HIP(hipMemcpyAsync(mm, w.minmax, sizeof(int32_t) * 3 * ncol,
                            hipMemcpyDeviceToHost, stream));
    RHIP_HIP(hipStreamSynchronize(stream));
    int total_bits = 0;
    int bits[RHIP_MAX_COLS];
    for (int c = 0; c < ncol; ++c) {
      table->lo[c] = mm[c];
      table->hi[c] = mm[ncol + c];
      bits[c] = bit_width_u32(static_cast<uint32_t>(
          static_cast<int64_t>(mm[ncol + c]) - mm[c]));
      total_bits += bits[c];
    }
    int sh = 0;
    for (int c = ncol - 1; c >= 0; --c) {
      table->shift[c] = total_bits <= 63 ? sh : 0;
      sh += bits[c];
    }
    table->mode = total_bits <= 63 ? RHIP_KEY_PACKED64 : RHIP_KEY_ROWREF;
    table->key_bits = total_bits <= 63 ? total_bits : 0;
    // the lowest bit in which each column varies (coordinates at tensor
    // stride 2^s vary from bit s up)
    for (int c = 0; c < ncol; ++c) {
      const uint32_t orx = static_cast<uint32_t>(mm[2 * ncol + c]);
      table->tz[c] = orx != 0 ? __builtin_ctz(orx) : 0;
    }

    // The row-reference build probes the caller's coordinates; lookups after
    // the build probe unique_coords (resolve_kernel re-points the slots).
    TableView tv = make_view(*table);
    tv.rows = coords;
    hipLaunchKernelGGL(insert_kernel, dim3(nb), dim3(kBlock), 0, stream, coords,
                       n, tv, w.slot_of_row);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(count_first_kernel, dim3(nb), dim3(kBlock), 0, stream, n,
                       sl, w.slot_of_row, w.block_counts);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(scan_kernel<int32_t>, dim3(1), dim3(1024), 0, stream,
                       w.block_counts, nb, w.block_base, w.total);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(assign_uid_kernel, dim3(nb), dim3(kBlock), 0, stream,
                       coords, n, ncol, sl, w.slot_of_row, w.block_base,
                       w.uid_by_row, mapping, unique_coords);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(resolve_kernel, dim3(nb), dim3(kBlock), 0, stream,
                       coords, n, tv, w.slot_of_row, w.uid_by_row, inverse);
    RHIP_LAUNCH_CHECK();
    int64_t nu = 0;
    RHIP_HIP(hipMemcpyAsync(&nu, w.total, sizeof(int64_t),
                            hipMemcpyDeviceToHost, stream));
    RHIP_HIP(hipStreamSynchronize(stream));
    table->n_unique = nu;
  });
}

extern "C" int rhip_hash_lookup(const rhip_table *table, const int32_t *queries,
                                int64_t n, int32_t *result, hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(table != nullptr, "table is null");
    RHIP_CHECK_ARG(n >= 0, "n must be >= 0");
    if (n == 0)
      return;
    RHIP_CHECK_ARG(queries && result, "queries/result must be non-null");
    hipLaunchKernelGGL(lookup_kernel, dim3(ceil_div(n, kBlock)), dim3(kBlock), 0,
                       stream, make_view(*table), queries, n, result);
    RHIP_LAUNCH_CHECK();
  });
}

extern "C" int rhip_order_workspace_bytes(int64_t n, size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    Carve cv(nullptr, 0);
    const int64_t m = std::max<int64_t>(n, 1);
    cv.take<uint64_t>(m);
    cv.take<uint64_t>(m);
    cv.take<int32_t>(m);
    cv.take<char>(sort_pairs_u64_bytes(m));
    *bytes = cv.used + 256;
  });
}

namespace rhip {
namespace {

// Locality-key layout of a table: bits per spatial column of the Morton
// code (0: the packed key orders the rows instead) and its total width.
struct OrderLayout {
  int morton_bits = 0, total_bits = 0;
};

OrderLayout order_layout(const rhip_table &t) {
  OrderLayout o;
  if (t.mode != RHIP_KEY_PACKED64 || t.key_bits == 0)
    return o;
  const int D = t.ncol - 1;
  int wide = 0;
  for (int c = 1; c <= D; ++c)
    wide = std::max(wide, bit_width_u32(static_cast<uint32_t>(
                              (static_cast<int64_t>(t.hi[c]) - t.lo[c]) >> t.tz[c])));
  const int batch_bits =
      bit_width_u32(static_cast<uint32_t>(static_cast<int64_t>(t.hi[0]) - t.lo[0]));
  if (D >= 1 && wide > 0 && batch_bits + D * wide <= 63) {
    o.morton_bits = wide;
    o.total_bits = batch_bits + D * wide;
  } else {
    o.total_bits = t.key_bits;
  }
  return o;
}

// Brick grid of a table: Morton levels per brick (cells = 2^(levels * D) <=
// 64) and the grid extent per column; entries 0 when there is none.
struct BrickLayout {
  int levels = 0;
  int32_t dims[RHIP_MAX_COLS] = {};
  int64_t entries = 0;
};

BrickLayout brick_layout(const rhip_table &t) {
  BrickLayout b;
  const int D = t.ncol - 1;
  if (order_layout(t).morton_bits == 0 || D < 1 || D > 6 || t.n_unique < 1)
    return b;
  b.levels = 6 / D;
  int64_t entries = static_cast<int64_t>(t.hi[0]) - t.lo[0] + 1;
  b.dims[0] = static_cast<int32_t>(entries);
  const int64_t limit = std::min<int64_t>(int64_t(1) << 23,
                                          std::max<int64_t>(4096, 16 * t.n_unique));
  for (int c = 1; c <= D && entries <= limit; ++c) {
    const int64_t ext = (((static_cast<int64_t>(t.hi[c]) - t.lo[c]) >> t.tz[c]) >> b.levels) + 1;
    b.dims[c] = static_cast<int32_t>(std::min<int64_t>(ext, INT32_MAX));
    entries *= ext;
  }
  b.entries = entries <= limit ? entries : 0;
  return b;
}

} // namespace
} // namespace rhip

extern "C" int rhip_brick_bytes(const rhip_table *table, size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(table != nullptr && bytes != nullptr, "table and bytes are required");
    *bytes = static_cast<size_t>(brick_layout(*table).entries) * sizeof(Brick);
  });
}

extern "C" int rhip_spatial_order(rhip_table *table, int32_t *order, int32_t *pos,
                                  void *bricks, size_t brick_bytes, void *workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(table != nullptr, "table is null");
    table->order = nullptr;
    table->bricks = nullptr;
    table->morton_bits = 0;
    table->brick_levels = 0;
    const int64_t n = table->n_unique;
    if (n == 0)
      return;
    RHIP_CHECK_ARG(order != nullptr, "order is null");
    const int64_t nb = ceil_div(n, kBlock);
    const OrderLayout ol = order_layout(*table);
    if (ol.total_bits == 0) {
      hipLaunchKernelGGL(iota_kernel, dim3(nb), dim3(kBlock), 0, stream, n,
                         order, pos);
      RHIP_LAUNCH_CHECK();
      return;
    }
    RHIP_CHECK_ARG(workspace != nullptr, "workspace is null");
    Carve cv(workspace, workspace_bytes);
    uint64_t *keys_in = cv.take<uint64_t>(n);
    uint64_t *keys_out = cv.take<uint64_t>(n);
    int32_t *rows_in = cv.take<int32_t>(n);
    const size_t temp = sort_pairs_u64_bytes(n);
    void *tmp = cv.take<char>(temp);
    hipLaunchKernelGGL(pack_keys_kernel, dim3(nb), dim3(kBlock), 0, stream,
                       make_view(*table), n, ol.morton_bits, keys_in, rows_in);
    RHIP_LAUNCH_CHECK();
    sort_pairs_u64(tmp, temp, keys_in, keys_out, rows_in, order, n, ol.total_bits, stream);
    if (pos) {
      hipLaunchKernelGGL(invert_perm_kernel, dim3(nb), dim3(kBlock), 0, stream,
                         n, order, pos);
      RHIP_LAUNCH_CHECK();
    }
    const BrickLayout bl = brick_layout(*table);
    table->morton_bits = ol.morton_bits;
    if (bricks == nullptr || bl.entries == 0 ||
        brick_bytes < static_cast<size_t>(bl.entries) * sizeof(Brick))
      return;
    Brick *grid = static_cast<Brick *>(bricks);
    hipLaunchKernelGGL(brick_clear_kernel, dim3(ceil_div(bl.entries, kBlock)), dim3(kBlock), 0,
                       stream, grid, bl.entries);
    RHIP_LAUNCH_CHECK();
    table->order = order;
    table->brick_levels = bl.levels;
    for (int c = 0; c < RHIP_MAX_COLS; ++c)
      table->brick_dims[c] = bl.dims[c];
    const int D = table->ncol - 1;
    hipLaunchKernelGGL(brick_fill_kernel, dim3(nb), dim3(kBlock), 0, stream, make_view(*table),
                       keys_out, order, n, bl.levels * D, grid);
    RHIP_LAUNCH_CHECK();
    table->bricks = bricks;
  });
}

extern "C" int rhip_stride_coords(const int32_t *coords, int64_t n,
                                  int32_t ncol,
                                  const int32_t *out_tensor_stride,
                                  int32_t *out, hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(ncol >= 2 && ncol <= RHIP_MAX_COLS, "bad ncol");
    RHIP_CHECK_ARG(out_tensor_stride != nullptr, "stride is null");
    StrideArg st{};
    for (int c = 0; c < ncol - 1; ++c) {
      RHIP_CHECK_ARG(out_tensor_stride[c] > 0, "stride must be positive");
      st.s[c] = out_tensor_stride[c];
    }
    if (n == 0)
      return;
    RHIP_CHECK_ARG(coords && out, "coords/out must be non-null");
    const int64_t total = n * ncol;
    hipLaunchKernelGGL(stride_kernel, dim3(ceil_div(total, kBlock)),
                       dim3(kBlock), 0, stream, coords, n, ncol, st, out);
    RHIP_LAUNCH_CHECK();
  });
}

extern "C" int rhip_expand_coords(const int32_t *coords, int64_t n, int32_t ncol,
                                  const int32_t *offsets, int32_t K, int32_t *out,
                                  hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(ncol >= 2 && ncol <= RHIP_MAX_COLS, "bad ncol");
    RHIP_CHECK_ARG(K >= 1, "K must be >= 1");
    RHIP_CHECK_ARG(n >= 0 && n <= INT64_MAX / (static_cast<int64_t>(K) * ncol),
                   "n * K * ncol overflows");
    if (n == 0)
      return;
    RHIP_CHECK_ARG(coords && offsets && out, "coords, offsets and out must be non-null");
    const int64_t total = n * K * ncol;
    hipLaunchKernelGGL(expand_kernel, dim3(ceil_div(total, kBlock)), dim3(kBlock), 0, stream,
                       coords, n, ncol, K, offsets, out);
    RHIP_LAUNCH_CHECK();
  });
}
