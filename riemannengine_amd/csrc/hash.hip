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
#include <type_traits>

#include "rhip_internal.hpp"

namespace rhip {

constexpr int kBlock = 256;

// Packing layout of a set, computed on the device so that the build needs
// no host round trip before the inserts: per column the minimum, maximum and
// common trailing zero bits, the packed key's shifts and width, and the key
// mode; dups is set when some row repeats an earlier one; n_unique is written
// by the numbering scan. row_bits > 0 when a packed key and a row index fit
// one 64-bit word together: the insert then claims a slot with the word
// (key << row_bits | row) in one compare-and-swap, a repeat lowers it with
// atomicMin (same key bits, so the smaller row wins), and the numbering puts
// the plain key back. Read back to the host once, at the end of the build.
struct HashLayout {
  int64_t n_unique;
  int32_t lo[RHIP_MAX_COLS], hi[RHIP_MAX_COLS], shift[RHIP_MAX_COLS], tz[RHIP_MAX_COLS];
  int32_t mode, key_bits, dups, row_bits;
};

constexpr int kMinmaxBlocks = 256;

// Blocks [0, mm_blocks): per-block column minimum, maximum and OR of
// (value ^ row 0's value) (its lowest set bit is the lowest bit in which the
// column varies), over the coordinates read as one flat array so that loads
// are coalesced (a lane keeps one column: the stride is a multiple of ncol);
// field f of block b at partials[f * kMinmaxBlocks + b], fields [0..ncol) =
// min, [8..) = max, [16..) = or (field-major: the layout's lanes read one
// field of consecutive blocks together). Blocks past
// mm_blocks clear the hash slots. Block 0 clears the layout's repeat flag
// and unique count, which the insert and numbering kernels then write.
__global__ __launch_bounds__(kBlock) void hash_prep_kernel(const int32_t *__restrict__ coords,
                                                           int64_t n, int ncol, int mm_blocks,
                                                           int32_t *__restrict__ partials,
                                                           Slot *__restrict__ slots,
                                                           int64_t cap, HashLayout *L) {
  if (blockIdx.x == 0 && threadIdx.x == 0 && L) {
    L->dups = 0;
    L->n_unique = 0;
  }
  if (static_cast<int>(blockIdx.x) >= mm_blocks) {
    const int64_t i = (blockIdx.x - mm_blocks) * (int64_t)kBlock + threadIdx.x;
    if (i < cap) {
      Slot s;
      s.word = kEmptyWord;
      s.first_row = 0xffffffffu;
      s.uid = 0xffffffffu;
      slots[i] = s;
    }
    return;
  }
  __shared__ int32_t smin[RHIP_MAX_COLS], smax[RHIP_MAX_COLS], sor[RHIP_MAX_COLS];
  if (threadIdx.x < RHIP_MAX_COLS) {
    smin[threadIdx.x] = INT_MAX;
    smax[threadIdx.x] = INT_MIN;
    sor[threadIdx.x] = 0;
  }
  __syncthreads();
  const int64_t threads = static_cast<int64_t>(mm_blocks) * kBlock;
  const int64_t stride = threads - threads % ncol;
  const int64_t i0 = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (i0 < stride) {
    const int c = static_cast<int>(i0 % ncol);
    const int32_t c0 = coords[c];
    int32_t lmin = INT_MAX, lmax = INT_MIN, lor = 0;
    // eight loads issued back to back per round (one load per round left
    // every round waiting on memory: config 2 prep 10.8 us)
    constexpr int kU = 8;
    const int64_t total = n * ncol;
    for (int64_t f0 = i0; f0 < total; f0 += kU * stride) {
      int32_t v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t f = f0 + u * stride;
        v[u] = f < total ? coords[f] : c0;
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        lmin = min(lmin, v[u]);
        lmax = max(lmax, v[u]);
        lor |= v[u] ^ c0;
      }
    }
    atomicMin(&smin[c], lmin);
    atomicMax(&smax[c], lmax);
    atomicOr(&sor[c], lor);
  }
  __syncthreads();
  if (threadIdx.x < ncol) {
    int32_t *p = partials + blockIdx.x;
    p[threadIdx.x * kMinmaxBlocks] = smin[threadIdx.x];
    p[(RHIP_MAX_COLS + threadIdx.x) * kMinmaxBlocks] = smax[threadIdx.x];
    p[(2 * RHIP_MAX_COLS + threadIdx.x) * kMinmaxBlocks] = sor[threadIdx.x];
  }
}

__device__ __forceinline__ int bit_width_dev(uint32_t v) { return v == 0 ? 0 : 32 - __clz(v); }

// One workgroup merges the prep partials into the layout (lane k reads
// block k's partials, field-major; wave shuffles, then LDS, combine them)
// and thread 0 writes it to *L (every field but dups and n_unique, which
// prep cleared). Columns are packed with the batch column in the top bits,
// so the packed order is batch-major lexicographic; more than 63 bits
// selects the row-reference mode. (The same merge at the start of every
// insert workgroup, to save this launch, ran the insert 29 -> 37 us on
// config 2: the serial tail and two barriers in each of 1,600 workgroups.)
__global__ __launch_bounds__(kBlock) void hash_layout_kernel(const int32_t *__restrict__ partials,
                                                             int mm_blocks, int ncol, int64_t n,
                                                             HashLayout *__restrict__ L) {
  constexpr int kWaves = kBlock / kWave;
  __shared__ int32_t red[kWaves][3 * RHIP_MAX_COLS];
  const int k = threadIdx.x, w = k / kWave, lane = lane_id();
  for (int c = 0; c < ncol; ++c) {
    int32_t a = INT_MAX, b = INT_MIN, o = 0;
    for (int j = k; j < mm_blocks; j += kBlock) {
      const int32_t *p = partials + j;
      a = min(a, p[c * kMinmaxBlocks]);
      b = max(b, p[(RHIP_MAX_COLS + c) * kMinmaxBlocks]);
      o |= p[(2 * RHIP_MAX_COLS + c) * kMinmaxBlocks];
    }
    for (int off = 32; off > 0; off >>= 1) {
      a = min(a, __shfl_xor(a, off));
      b = max(b, __shfl_xor(b, off));
      o |= __shfl_xor(o, off);
    }
    if (lane == 0) {
      red[w][c] = a;
      red[w][RHIP_MAX_COLS + c] = b;
      red[w][2 * RHIP_MAX_COLS + c] = o;
    }
  }
  __syncthreads();
  if (k != 0)
    return;
  int32_t mn[RHIP_MAX_COLS], mx[RHIP_MAX_COLS], ox[RHIP_MAX_COLS];
  int bits[RHIP_MAX_COLS] = {};
  int total = 0;
  for (int i = 0; i < ncol; ++i) {
    mn[i] = red[0][i];
    mx[i] = red[0][RHIP_MAX_COLS + i];
    ox[i] = red[0][2 * RHIP_MAX_COLS + i];
    for (int v = 1; v < kWaves; ++v) {
      mn[i] = min(mn[i], red[v][i]);
      mx[i] = max(mx[i], red[v][RHIP_MAX_COLS + i]);
      ox[i] |= red[v][2 * RHIP_MAX_COLS + i];
    }
    bits[i] = bit_width_dev(static_cast<uint32_t>(static_cast<int64_t>(mx[i]) - mn[i]));
    total += bits[i];
  }
  int sh = 0;
  for (int i = ncol - 1; i >= 0; --i) {
    L->shift[i] = total <= 63 ? sh : 0;
    sh += bits[i];
  }
  for (int i = 0; i < RHIP_MAX_COLS; ++i) {
    L->lo[i] = i < ncol ? mn[i] : 0;
    L->hi[i] = i < ncol ? mx[i] : 0;
    L->tz[i] = i < ncol && ox[i] != 0 ? __ffs(ox[i]) - 1 : 0;
    if (i >= ncol)
      L->shift[i] = 0;
  }
  L->mode = total <= 63 ? RHIP_KEY_PACKED64 : RHIP_KEY_ROWREF;
  L->key_bits = total <= 63 ? total : 0;
  const int rb = max(1, bit_width_dev(static_cast<uint32_t>(n - 1)));
  L->row_bits = total + rb <= 63 ? rb : 0;
}

// The device layout's ranges and mode in a table view.
__device__ __forceinline__ void apply_layout(TableView &t, const HashLayout *L) {
  t.mode = L->mode;
#pragma unroll
  for (int c = 0; c < RHIP_MAX_COLS; ++c) {
    t.lo[c] = L->lo[c];
    t.span[c] = static_cast<uint32_t>(static_cast<int64_t>(L->hi[c]) - L->lo[c]);
    t.shift[c] = L->shift[c];
  }
}

// One lane per input row: claim or find the row's slot; the slot keeps the
// earliest row that inserted the key (in the key word when row_bits > 0,
// else in first_row through atomicMin). A row that finds its key already
// there flags the set as having repeats.
// The wave cooperates on repeats: with packed keys, a lane whose key equals
// the previous lane's follows that run's first lane, which probes once for
// the whole run, and takes its slot by a shuffle. Points quantised in scan
// order repeat their voxel in runs (config 3's raw LiDAR sweeps: 107k of
// 250k rows repeat the previous row), and those runs would otherwise hammer
// one slot with compare-and-swaps that the L2 serialises. The run's first
// lane has its smallest row, so the first occurrence still wins.
__global__ __launch_bounds__(kBlock) void insert_kernel(const int32_t *coords,
                                                        int64_t n,
                                                        TableView t,
                                                        HashLayout *L,
                                                        uint32_t *slot_of_row) {
  const int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  const bool valid = r < n; // every lane stays for the wave's shuffles
  apply_layout(t, L);
  const int rb = L->row_bits;
  int32_t c[RHIP_MAX_COLS];
#pragma unroll
  for (int i = 0; i < RHIP_MAX_COLS; ++i)
    c[i] = valid && i < t.ncol ? coords[r * t.ncol + i] : 0;

  uint64_t key = 0, h = 0;
  uint32_t hr = 0;
  const bool packed = t.mode == RHIP_KEY_PACKED64; // uniform
  if (packed) {
    pack_row(t, c, key); // in range for valid rows: the bounds come from this set
    h = mix64(key) & t.mask;
  } else {
    hr = hash_row(c, t.ncol);
    key = (static_cast<uint64_t>(hr) << 32) | static_cast<uint32_t>(r);
    h = mix64(hr) & t.mask;
  }
  const int lane = lane_id();
  const uint64_t kprev = __shfl_up(key, 1, kWave);
  // lane - 1 holds row r - 1, valid whenever r is
  const bool follow = packed && valid && lane > 0 && kprev == key;
  const uint64_t heads = __ballot(!follow);
  if (valid && !follow) {
    const uint64_t mine = rb > 0 ? (key << rb) | static_cast<uint64_t>(r) : key;
    while (true) {
      // one round trip per probe: the CAS either claims the empty slot or
      // returns the word already there (a load before it, to spare the
      // atomic on occupied slots, adds a round trip: config 2's insert 31.6
      // -> 39.5 us)
      uint64_t *wp = &t.slots[h].word;
      const uint64_t w = atomicCAS(reinterpret_cast<unsigned long long *>(wp), kEmptyWord, mine);
      if (w == kEmptyWord) {
        if (rb == 0)
          atomicMin(&t.slots[h].first_row, static_cast<uint32_t>(r));
        break; // claimed
      }
      bool same;
      if (rb > 0) {
        same = (w >> rb) == key;
      } else if (packed) {
        same = (w == key);
      } else {
        same = static_cast<uint32_t>(w >> 32) == hr &&
               rows_equal(coords + static_cast<int64_t>(static_cast<uint32_t>(w)) * t.ncol, c,
                          t.ncol);
      }
      if (same) {
        L->dups = 1;
        if (rb > 0) {
          if (mine < w)
            atomicMin(reinterpret_cast<unsigned long long *>(wp), mine);
        } else {
          atomicMin(&t.slots[h].first_row, static_cast<uint32_t>(r));
        }
        break;
      }
      h = (h + 1) & t.mask;
    }
  }
  // the slot of this lane's run: its first lane's
  const uint32_t slot =
      static_cast<uint32_t>(__shfl(static_cast<uint32_t>(h), run_head(heads), kWave));
  if (__ballot(follow) != 0 && lane == 0)
    L->dups = 1;
  if (valid)
    slot_of_row[r] = slot;
}

// Per-block count of rows that are the first occurrence of their key (every
// row is when the set has no repeats). With repeats and row_bits > 0, the
// first row also copies itself into its slot's first_row, where the later
// kernels read it while the key word is rewritten.
__global__ __launch_bounds__(kBlock) void count_first_kernel(
    int64_t n, const HashLayout *L, Slot *slots, const uint32_t *slot_of_row,
    int32_t *block_counts) {
  __shared__ int32_t wave_counts[kBlock / kWave];
  int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  bool first = r < n;
  if (first && L->dups) {
    Slot &s = slots[slot_of_row[r]];
    const int rb = L->row_bits;
    if (rb > 0) {
      first = (s.word & ((1ull << rb) - 1)) == static_cast<uint64_t>(r);
      if (first)
        s.first_row = static_cast<uint32_t>(r);
    } else {
      first = s.first_row == static_cast<uint32_t>(r);
    }
  }
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

// First rows get uid = block base + rank within the block; they write
// mapping[uid], the unique coordinates, their own inverse entry and their
// slot's uid, and put the plain key back in the slot word (in row-reference
// mode the key is re-pointed at the unique row). With repeats, uid_by_row
// keeps the uid for the other rows' inverse.
// Without block_base (grids of at most kSelfScanBlocks workgroups) each
// workgroup sums the counts of the workgroups before it itself (none to sum
// for a set without repeats: every earlier block holds kBlock first rows),
// and the last workgroup writes n_unique: no scan launch in between. The
// last workgroup then copies the finished layout to host_L (pinned host
// memory mapped for the device, or null), which the host reads after its
// synchronisation without a copy launch.
constexpr int64_t kSelfScanBlocks = 4096;
__global__ __launch_bounds__(kBlock) void assign_uid_kernel(
    const int32_t *coords, int64_t n, int ncol, HashLayout *L, Slot *slots,
    const uint32_t *slot_of_row, const int32_t *block_counts, const int64_t *block_base,
    int32_t *uid_by_row, int64_t *mapping, int32_t *unique_coords, int64_t *inverse,
    HashLayout *host_L) {
  constexpr int kWaves = kBlock / kWave;
  __shared__ int32_t wave_counts[kWaves];
  __shared__ int64_t wave_prefix[kWaves];
  int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  const int dups = L->dups;
  const bool first =
      r < n && (dups == 0 || slots[slot_of_row[r]].first_row == static_cast<uint32_t>(r));
  uint64_t b = __ballot(first);
  const int w = threadIdx.x / kWave;
  int64_t prefix = 0;
  if (!block_base && dups) { // uniform: the earlier workgroups' first rows
    for (int64_t i = threadIdx.x; i < blockIdx.x; i += kBlock)
      prefix += block_counts[i];
    for (int off = 32; off > 0; off >>= 1)
      prefix += __shfl_xor(prefix, off);
  }
  if (lane_id() == 0) {
    wave_counts[w] = __popcll(b);
    wave_prefix[w] = prefix;
  }
  __syncthreads();
  int32_t before = 0, mine = 0;
  int64_t base = 0;
  for (int i = 0; i < kWaves; ++i) {
    before += i < w ? wave_counts[i] : 0;
    mine += wave_counts[i];
    base += wave_prefix[i];
  }
  if (block_base)
    base = block_base[blockIdx.x];
  else if (!dups)
    base = static_cast<int64_t>(blockIdx.x) * kBlock;
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) {
    if (!block_base)
      L->n_unique = base + mine;
    if (host_L) {
      HashLayout h;
      h.n_unique = block_base ? L->n_unique : base + mine;
      for (int i = 0; i < RHIP_MAX_COLS; ++i) {
        h.lo[i] = L->lo[i];
        h.hi[i] = L->hi[i];
        h.shift[i] = L->shift[i];
        h.tz[i] = L->tz[i];
      }
      h.mode = L->mode;
      h.key_bits = L->key_bits;
      h.dups = dups;
      h.row_bits = L->row_bits;
      *host_L = h;
    }
  }
  if (first) {
    const int64_t uid = base + before + lanes_below(b);
    if (L->dups)
      uid_by_row[r] = static_cast<int32_t>(uid);
    mapping[uid] = r;
    if (inverse)
      inverse[r] = uid;
    // the slot's final contents, from the row itself: one store, no read
    int32_t c[RHIP_MAX_COLS];
#pragma unroll
    for (int i = 0; i < RHIP_MAX_COLS; ++i)
      c[i] = i < ncol ? coords[r * ncol + i] : 0;
#pragma unroll
    for (int i = 0; i < RHIP_MAX_COLS; ++i)
      if (i < ncol)
        unique_coords[uid * ncol + i] = c[i];
    Slot out;
    out.first_row = static_cast<uint32_t>(r);
    out.uid = static_cast<uint32_t>(uid);
    if (L->mode == RHIP_KEY_PACKED64) {
      uint64_t key = 0;
#pragma unroll
      for (int i = 0; i < RHIP_MAX_COLS; ++i)
        if (i < ncol)
          key |= static_cast<uint64_t>(static_cast<uint32_t>(c[i]) -
                                       static_cast<uint32_t>(L->lo[i]))
                 << L->shift[i];
      out.word = key;
    } else {
      out.word = (static_cast<uint64_t>(hash_row(c, ncol)) << 32) | static_cast<uint32_t>(uid);
    }
    slots[slot_of_row[r]] = out;
  }
}

// Sets with repeats: inverse[r] = uid of the first occurrence of r's key.
__global__ __launch_bounds__(kBlock) void resolve_kernel(
    int64_t n, const HashLayout *L, const Slot *slots, const uint32_t *slot_of_row,
    const int32_t *uid_by_row, int64_t *inverse) {
  int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (r >= n || L->dups == 0)
    return;
  const uint32_t fr = slots[slot_of_row[r]].first_row;
  if (fr != static_cast<uint32_t>(r))
    inverse[r] = uid_by_row[fr];
}

__global__ __launch_bounds__(kBlock) void lookup_kernel(TableView t,
                                                        const int32_t *queries,
                                                        int64_t n,
                                                        int32_t *result) {
  const int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  const bool valid = i < n; // every lane stays for the wave's shuffles
  int32_t c[RHIP_MAX_COLS];
#pragma unroll
  for (int j = 0; j < RHIP_MAX_COLS; ++j)
    c[j] = valid && j < t.ncol ? queries[i * t.ncol + j] : 0;
  // a query that repeats the previous lane's takes that run's answer
  const bool follow = repeats_prev_row(c, valid);
  const uint64_t heads = __ballot(!follow);
  int32_t res = -1;
  if (valid && !follow)
    res = table_find(t, c);
  res = __shfl(res, run_head(heads), kWave);
  if (valid)
    result[i] = res;
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

// The brick grid in Morton space. A row's locality key is its batch above
// the bit-interleave of its spatial columns; with bricks of 2^levels cells
// per column, the key's low levels*D bits are the row's cell within its
// brick and the bits above are the Morton code of the brick's coordinates
// (with the batch). Keys order rows by brick, in brick Morton order, then by
// cell. The brick Morton index drops the bit positions that are zero for
// every brick of the grid (column c needs pbits[c] bits, its extent rounded
// up to a power of two), which keeps that order: bit l of brick coordinate c
// sits above bit l of the columns after c and below bit l + 1 of every
// column. Index m = (batch << mbits) | spatial index, total = batches << mbits.
struct BrickSpace {
  int32_t pbits[RHIP_MAX_COLS];
  int32_t top;   // largest pbits
  int32_t mbits; // sum of pbits
  int64_t total;
};

// Brick (batch, brick coordinates) of index m as a grid entry, or -1 when
// the coordinates leave the grid (the padding of the power-of-two extents).
template <int D>
__device__ __forceinline__ int64_t brick_at(const BrickSpace &s, const int32_t *dims,
                                            int64_t m) {
  uint64_t bits = static_cast<uint64_t>(m) & ((1ull << s.mbits) - 1);
  uint32_t b[D + 1];
#pragma unroll
  for (int j = 0; j <= D; ++j)
    b[j] = 0;
  for (int l = 0; l < s.top; ++l) {
#pragma unroll
    for (int j = D; j >= 1; --j) {
      if (l < s.pbits[j]) {
        b[j] |= static_cast<uint32_t>(bits & 1u) << l;
        bits >>= 1;
      }
    }
  }
  int64_t g = m >> s.mbits;
#pragma unroll
  for (int j = 1; j <= D; ++j) {
    if (b[j] >= static_cast<uint32_t>(dims[j]))
      return -1;
    g = g * dims[j] + b[j];
  }
  return g;
}

// Grid entry, cell and brick coordinates (b[0] = batch offset) of unique
// row r, as the neighbour probes compute them.
template <int D>
__device__ __forceinline__ int64_t brick_of_row(const TableView &t, int64_t r, uint32_t (&b)[D + 1],
                                                uint32_t &cell) {
  const int32_t *c = t.rows + r * (D + 1);
  b[0] = static_cast<uint32_t>(c[0]) - static_cast<uint32_t>(t.lo[0]);
  int64_t g = b[0];
  uint32_t cl = 0;
#pragma unroll
  for (int i = 1; i <= D; ++i) {
    const uint32_t w = (static_cast<uint32_t>(c[i]) - static_cast<uint32_t>(t.lo[i])) >> t.tz[i];
    b[i] = w >> t.levels;
    g = g * t.dims[i] + b[i];
    for (int l = 0; l < t.levels; ++l)
      cl |= ((w >> l) & 1u) << (l * D + (D - i));
  }
  cell = cl;
  return g;
}

// Rows per Morton chunk: a workgroup takes kSpanPer consecutive indices per
// lane, kSpan per workgroup.
// 4 indices per lane: config 2's grid (1.05M indices) walks in 1024
// workgroups (with 16 per lane, 256 workgroups: count 10.2 -> 4.8 us, base
// 9.3 -> 4.5 us)
constexpr int kSpanPer = 4;
constexpr int64_t kSpan = static_cast<int64_t>(kBlock) * kSpanPer;
// Most chunks a brick walk takes (2^26 indices).
constexpr int64_t kMaxSpaceChunks = (int64_t(1) << 26) / kSpan;

// One lane per unique row: sets the row's cell bit in its brick's mask (the
// grid is cleared first). Rows that arrive in coordinate order share bricks
// in runs: a run of lanes with the same brick combines its bits (segmented
// OR scan over the wave) and only its last lane issues the atomic. Rows in
// random order (config 2's scenes: 1.0002 rows per run) cost one atomic
// each.
template <int D>
__global__ __launch_bounds__(kBlock) void brick_mark_kernel(TableView t, int64_t n,
                                                            Brick *__restrict__ grid) {
  const int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  const int lane = lane_id();
  int64_t g = -1 - lane; // lanes past n: distinct, negative, in no run
  uint64_t bits = 0;
  if (r < n) {
    uint32_t b[D + 1], cell;
    g = brick_of_row<D>(t, r, b, cell);
    bits = 1ull << cell;
  }
  // a run starts where the brick differs from the previous lane's; a lane
  // takes bits only from lanes at or after the start of its own run
  const int64_t gprev = __shfl_up(g, 1, kWave);
  const uint64_t heads = __ballot(lane == 0 || gprev != g);
  const int start = run_head(heads);
  for (int off = 1; off < kWave; off <<= 1) {
    const uint64_t bp = __shfl_up(bits, off, kWave);
    if (lane - off >= start)
      bits |= bp;
  }
  const bool tail = lane == kWave - 1 || ((heads >> (lane + 1)) & 1ull);
  if (r < n && tail)
    atomicOr(reinterpret_cast<unsigned long long *>(&grid[g].mask), bits);
}

// The same marks without atomics, where the scratch holds a byte per cell:
// each unique row stores 1 in its cell's byte (cells[g * cpb + cell], cpb =
// cells per brick, 16, 32 or 64), and the counting walk folds each brick's
// bytes into its mask. Random plain stores retire at about 2.5 times the
// rate of random atomics on this device (config 2: the atomicOr marks took
// 24 us).
template <int D>
__global__ __launch_bounds__(kBlock) void brick_mark_bytes_kernel(TableView t, int64_t n,
                                                                  uint8_t *__restrict__ cells,
                                                                  int cpb) {
  const int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (r >= n)
    return;
  uint32_t b[D + 1], cell;
  const int64_t g = brick_of_row<D>(t, r, b, cell);
  cells[g * cpb + cell] = 1;
}

// Zeroes n16 16-byte words (the cell bytes before the marks).
__global__ __launch_bounds__(kBlock) void zero_u128_kernel(uint4 *__restrict__ p, int64_t n16) {
  const int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (i < n16)
    p[i] = uint4{0u, 0u, 0u, 0u};
}

// The occupancy mask of a brick from its cpb cell bytes (each 0 or 1; cpb
// a multiple of 16, the bytes 16-byte aligned): byte i becomes bit i. In a
// word of four such bytes b0..b3 the product with 0x204081 puts b_j at bit
// 21 + j with no carries (the sixteen partial products land on distinct
// bits).
__device__ __forceinline__ uint64_t mask_of_cells(const uint8_t *__restrict__ c, int cpb) {
  uint4 v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) // the loads issue back to back
    v[q] = 16 * q < cpb ? *reinterpret_cast<const uint4 *>(c + 16 * q) : uint4{0u, 0u, 0u, 0u};
  uint64_t m = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t w[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      m |= static_cast<uint64_t>(((w[e] * 0x204081u) >> 21) & 0xfu) << (16 * q + 4 * e);
  }
  return m;
}

// Grid entries of the kSpanPer indices m0 .. m0 + kSpanPer - 1 (m0 a
// multiple of kSpanPer; -1 for indices past the space or the grid). The
// decode is linear in the index bits, so the aligned base is decoded once and
// each index adds the (wave-uniform) decode of its low bits; brick_at per
// index spent most of the walk kernels' time in the bit loop.
template <int D>
__device__ __forceinline__ void brick_span(const BrickSpace &s, const int32_t *dims, int64_t m0,
                                           int64_t (&g)[kSpanPer]) {
  static_assert((kSpanPer & (kSpanPer - 1)) == 0, "kSpanPer must be a power of two");
  constexpr int LB = __builtin_ctz(kSpanPer);
  if (s.mbits < LB) {
#pragma unroll
    for (int i = 0; i < kSpanPer; ++i)
      g[i] = m0 + i < s.total ? brick_at<D>(s, dims, m0 + i) : -1;
    return;
  }
  // base coordinates of m0 (its low LB bits are zero)
  uint32_t bh[D + 1] = {};
  {
    uint64_t bits = static_cast<uint64_t>(m0) & ((1ull << s.mbits) - 1);
    for (int l = 0; l < s.top; ++l) {
#pragma unroll
      for (int j = D; j >= 1; --j) {
        if (l < s.pbits[j]) {
          bh[j] |= static_cast<uint32_t>(bits & 1u) << l;
          bits >>= 1;
        }
      }
    }
  }
  const int64_t batch = m0 >> s.mbits;
#pragma unroll
  for (int i = 0; i < kSpanPer; ++i) {
    // decode of the low bits i (the same for every lane)
    uint32_t bl[D + 1] = {};
    uint32_t bits = static_cast<uint32_t>(i);
    int used = 0;
    for (int l = 0; l < s.top && used < LB; ++l) {
#pragma unroll
      for (int j = D; j >= 1; --j) {
        if (l < s.pbits[j] && used < LB) {
          bl[j] |= (bits & 1u) << l;
          bits >>= 1;
          ++used;
        }
      }
    }
    int64_t gi = batch;
    bool ok = m0 + i < s.total;
#pragma unroll
    for (int j = 1; j <= D; ++j) {
      const uint32_t b = bh[j] | bl[j];
      ok = ok && b < static_cast<uint32_t>(dims[j]);
      gi = gi * dims[j] + b;
    }
    g[i] = ok ? gi : -1;
  }
}

// Occupied cells of each kSpan-index chunk of the brick Morton space. With
// cells (the byte marks) it first folds each entry's bytes into its mask and
// writes the whole entry (every entry of the grid has one index in the
// walk, so the grid itself needs no clearing; bases follow in
// brick_base_kernel).
template <int D>
__global__ __launch_bounds__(kBlock) void brick_count_kernel(BrickSpace s, TableView t,
                                                             Brick *__restrict__ grid,
                                                             const uint8_t *__restrict__ cells,
                                                             int cpb,
                                                             int32_t *__restrict__ chunk_rows) {
  __shared__ int32_t wave_sum[kBlock / kWave];
  const int64_t m0 = blockIdx.x * kSpan + static_cast<int64_t>(threadIdx.x) * kSpanPer;
  int64_t g[kSpanPer];
  brick_span<D>(s, t.dims, m0, g);
  uint64_t mk[kSpanPer];
  if (cells) { // uniform
#pragma unroll
    for (int i = 0; i < kSpanPer; ++i)
      mk[i] = g[i] >= 0 ? mask_of_cells(cells + g[i] * cpb, cpb) : 0;
#pragma unroll
    for (int i = 0; i < kSpanPer; ++i) {
      if (g[i] >= 0) {
        Brick b;
        b.mask = mk[i];
        b.base = -1;
        b.pad = 0;
        grid[g[i]] = b;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kSpanPer; ++i) // the loads issue back to back
      mk[i] = g[i] >= 0 ? grid[g[i]].mask : 0;
  }
  int32_t cnt = 0;
#pragma unroll
  for (int i = 0; i < kSpanPer; ++i)
    cnt += __popcll(mk[i]);
  for (int off = kWave / 2; off > 0; off >>= 1)
    cnt += __shfl_xor(cnt, off);
  if (lane_id() == 0)
    wave_sum[threadIdx.x / kWave] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t tot = 0;
    for (int w = 0; w < kBlock / kWave; ++w)
      tot += wave_sum[w];
    chunk_rows[blockIdx.x] = tot;
  }
}

// Each occupied brick's base: the locality-order position of its first row,
// the rows of every brick before it in Morton order (chunk base from the
// scan of brick_count_kernel's totals, then an in-workgroup scan). Without
// chunk_base (walks of at most kSelfScanBlocks chunks) each workgroup sums
// the earlier chunks' totals itself, which saves the scan launch.
template <int D>
__global__ __launch_bounds__(kBlock) void brick_base_kernel(BrickSpace s, TableView t,
                                                            const int32_t *__restrict__ chunk_rows,
                                                            const int64_t *__restrict__ chunk_base,
                                                            Brick *__restrict__ grid) {
  constexpr int kWaves = kBlock / kWave;
  __shared__ int32_t wave_sum[kWaves];
  __shared__ int64_t wave_prefix[kWaves];
  const int64_t m0 = blockIdx.x * kSpan + static_cast<int64_t>(threadIdx.x) * kSpanPer;
  int64_t g[kSpanPer];
  uint64_t mk[kSpanPer];
  brick_span<D>(s, t.dims, m0, g);
  int32_t cnt = 0;
#pragma unroll
  for (int i = 0; i < kSpanPer; ++i) {
    mk[i] = g[i] >= 0 ? grid[g[i]].mask : 0;
    cnt += __popcll(mk[i]);
  }
  const int lane = lane_id(), w = threadIdx.x / kWave;
  int64_t prefix = 0;
  if (!chunk_base) {
    for (int64_t i = threadIdx.x; i < blockIdx.x; i += kBlock)
      prefix += chunk_rows[i];
    for (int off = 32; off > 0; off >>= 1)
      prefix += __shfl_xor(prefix, off);
  }
  int32_t incl = cnt;
  for (int off = 1; off < kWave; off <<= 1) {
    const int32_t o = __shfl_up(incl, off, kWave);
    if (lane >= off)
      incl += o;
  }
  if (lane == kWave - 1)
    wave_sum[w] = incl;
  if (lane == 0)
    wave_prefix[w] = prefix;
  __syncthreads();
  int64_t run = incl - cnt;
  if (chunk_base) {
    run += chunk_base[blockIdx.x];
  } else {
    for (int i = 0; i < kWaves; ++i)
      run += wave_prefix[i];
  }
  for (int i = 0; i < w; ++i)
    run += wave_sum[i];
#pragma unroll
  for (int i = 0; i < kSpanPer; ++i) {
    if (mk[i] != 0)
      grid[g[i]].base = static_cast<int32_t>(run);
    run += __popcll(mk[i]);
  }
}

// One lane per unique row: its locality-order position is its brick's base
// plus the occupied cells below its own; order and pos are written there.
template <int D>
__global__ __launch_bounds__(kBlock) void brick_place_kernel(TableView t, int64_t n,
                                                             const Brick *__restrict__ grid,
                                                             int32_t *__restrict__ order,
                                                             int32_t *__restrict__ pos) {
  const int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (r >= n)
    return;
  uint32_t b3[D + 1], cell;
  const Brick b = grid[brick_of_row<D>(t, r, b3, cell)];
  const int32_t p = b.base + __popcll(b.mask & ((1ull << cell) - 1ull));
  if (p < 0 || p >= n)
    return; // unreachable for a consistent grid; never writes past order
  order[p] = static_cast<int32_t>(r);
  if (pos)
    pos[r] = p;
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
  HashLayout *layout;
  int32_t *partials;
  uint32_t *slot_of_row;
  int32_t *uid_by_row;
  int32_t *block_counts;
  int64_t *block_base;
};

static HashWs carve_hash(Carve &cv, int64_t n, int ncol) {
  HashWs w;
  const int64_t nb = std::max<int64_t>(1, ceil_div(n, kBlock));
  w.layout = cv.take<HashLayout>(1);
  w.partials = cv.take<int32_t>(static_cast<size_t>(kMinmaxBlocks) * 3 * RHIP_MAX_COLS);
  w.slot_of_row = cv.take<uint32_t>(std::max<int64_t>(n, 1));
  w.uid_by_row = cv.take<int32_t>(std::max<int64_t>(n, 1));
  w.block_counts = cv.take<int32_t>(nb);
  w.block_base = cv.take<int64_t>(nb);
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
    if (n == 0) {
      hipLaunchKernelGGL(hash_prep_kernel, dim3(ceil_div(cap, kBlock)), dim3(kBlock), 0, stream,
                         coords, n, ncol, 0, w.partials, sl, cap, nullptr);
      RHIP_LAUNCH_CHECK();
      table->mode = RHIP_KEY_PACKED64;
      table->n_unique = 0;
      for (int c = 0; c < ncol; ++c)
        table->hi[c] = -1; // empty range: every probe misses on span check
      return;
    }
    // column ranges and slot clearing in one launch, then the layout on the
    // device: the inserts start without a host round trip
    const int mm = static_cast<int>(std::min<int64_t>(
        kMinmaxBlocks, std::max<int64_t>(1, ceil_div(n * ncol, int64_t(kBlock) * 8))));
    hipLaunchKernelGGL(hash_prep_kernel, dim3(mm + ceil_div(cap, kBlock)), dim3(kBlock), 0,
                       stream, coords, n, ncol, mm, w.partials, sl, cap, w.layout);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(hash_layout_kernel, dim3(1), dim3(kBlock), 0, stream, w.partials, mm, ncol,
                       n, w.layout);
    RHIP_LAUNCH_CHECK();
    // The row-reference build probes the caller's coordinates; lookups after
    // the build probe unique_coords (assign_uid_kernel re-points the slots).
    TableView tv = make_view(*table);
    tv.rows = coords;
    const int64_t nb = ceil_div(n, kBlock);
    hipLaunchKernelGGL(insert_kernel, dim3(nb), dim3(kBlock), 0, stream, coords, n, tv, w.layout,
                       w.slot_of_row);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(count_first_kernel, dim3(nb), dim3(kBlock), 0, stream, n, w.layout, sl,
                       w.slot_of_row, w.block_counts);
    RHIP_LAUNCH_CHECK();
    // up to kSelfScanBlocks workgroups the numbering sums the earlier
    // workgroups' counts itself
    const bool self_scan = nb <= kSelfScanBlocks;
    if (!self_scan) {
      hipLaunchKernelGGL(scan_kernel<int32_t>, dim3(1), dim3(1024), 0, stream, w.block_counts, nb,
                         w.block_base, &w.layout->n_unique);
      RHIP_LAUNCH_CHECK();
    }
    HashLayout hl;
    {
      // the numbering's last workgroup writes the layout into the pinned
      // buffer when the device can address it, else one copy reads it back
      PinnedReadback rb = pinned_readback(sizeof(hl));
      hipLaunchKernelGGL(assign_uid_kernel, dim3(nb), dim3(kBlock), 0, stream, coords, n, ncol,
                         w.layout, sl, w.slot_of_row, w.block_counts,
                         self_scan ? nullptr : w.block_base, w.uid_by_row, mapping,
                         unique_coords, inverse, static_cast<HashLayout *>(rb.dev));
      RHIP_LAUNCH_CHECK();
      if (!rb.dev)
        RHIP_HIP(hipMemcpyAsync(rb.ptr, w.layout, sizeof(hl), hipMemcpyDeviceToHost, stream));
      RHIP_HIP(hipStreamSynchronize(stream));
      std::memcpy(&hl, rb.ptr, sizeof(hl));
    }
    // the repeats' inverse entries, launched after the read-back and only for
    // a set that has repeats (assign_uid_kernel wrote every first row's)
    if (inverse && hl.dups) {
      hipLaunchKernelGGL(resolve_kernel, dim3(nb), dim3(kBlock), 0, stream, n, w.layout, sl,
                         w.slot_of_row, w.uid_by_row, inverse);
      RHIP_LAUNCH_CHECK();
    }
    table->n_unique = hl.n_unique;
    table->mode = hl.mode;
    table->key_bits = hl.key_bits;
    for (int c = 0; c < RHIP_MAX_COLS; ++c) {
      table->lo[c] = hl.lo[c];
      table->hi[c] = hl.hi[c];
      table->shift[c] = hl.shift[c];
      table->tz[c] = hl.tz[c];
    }
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
    // the brick path's chunk totals and bases (carved on their own)
    cv.take<int32_t>(rhip::kMaxSpaceChunks);
    cv.take<int64_t>(rhip::kMaxSpaceChunks + 1);
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

// Morton space of a brick grid (see BrickSpace); total is 0 when walking
// it would cost more than sorting the rows: more than 8 indices per grid
// entry (power-of-two padding, up to 2^D per entry) beyond 2^22 indices, or
// more than kMaxSpaceChunks chunks.
BrickSpace brick_space(const BrickLayout &bl, int D) {
  BrickSpace s{};
  int mbits = 0, top = 0;
  for (int c = 1; c <= D; ++c) {
    const int pb = bit_width_u32(static_cast<uint32_t>(bl.dims[c] - 1));
    s.pbits[c] = pb;
    mbits += pb;
    top = std::max(top, pb);
  }
  s.top = top;
  s.mbits = mbits;
  if (bl.entries == 0 || mbits > 40)
    return s;
  const int64_t total = static_cast<int64_t>(bl.dims[0]) << mbits;
  if (total > std::max<int64_t>(8 * bl.entries, int64_t(1) << 22) ||
      ceil_div(total, kSpan) > kMaxSpaceChunks)
    return s;
  s.total = total;
  return s;
}

// Locality order through the brick grid, a counting sort: the rows mark
// their cells (a byte per cell in scratch, or atomic ORs into the cleared
// grid where the scratch cannot hold the bytes), a walk of the grid in brick
// Morton order
// counts the occupied cells per chunk, a scan of the chunk totals (inside
// the second walk for up to kSelfScanBlocks chunks) and a second walk give
// every occupied brick its base, and each row lands at its
// brick's base plus the occupied cells below its own. The order equals the
// sorted locality keys'. (Counting rows per chunk with atomics in the mark
// pass instead serialises on the few chunk counters: 1.2 ms against 12 us
// for the walk on 410k rows.)
template <int D>
void order_by_bricks(const rhip_table &table, const BrickLayout &bl, const BrickSpace &bs,
                     Brick *grid, int32_t *order, int32_t *pos, void *workspace,
                     size_t workspace_bytes, hipStream_t stream) {
  const int64_t n = table.n_unique, nb = ceil_div(n, kBlock);
  const int64_t chunks = ceil_div(bs.total, kSpan);
  Carve cv(workspace, workspace_bytes);
  int32_t *chunk_rows = cv.take<int32_t>(chunks);
  int64_t *chunk_base = cv.take<int64_t>(chunks);
  int64_t *total = cv.take<int64_t>(1);
  const TableView t = make_view(table);
  // a byte per cell where the rest of the workspace holds them (the key
  // sort's buffers, unused on this path: 32 bytes per row), else atomic ORs
  // into the cleared grid
  const int cpb = 1 << (bl.levels * D);
  const size_t cell_bytes = static_cast<size_t>(bl.entries) * cpb;
  uint8_t *cells = nullptr;
  if (align_up(cv.used, 256) + cell_bytes <= workspace_bytes)
    cells = cv.take<uint8_t>(cell_bytes);
  if (cells) {
    const int64_t n16 = static_cast<int64_t>(cell_bytes / 16);
    hipLaunchKernelGGL(zero_u128_kernel, dim3(ceil_div(n16, kBlock)), dim3(kBlock), 0, stream,
                       reinterpret_cast<uint4 *>(cells), n16);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(brick_mark_bytes_kernel<D>, dim3(nb), dim3(kBlock), 0, stream, t, n, cells,
                       cpb);
    RHIP_LAUNCH_CHECK();
  } else {
    hipLaunchKernelGGL(brick_clear_kernel, dim3(ceil_div(bl.entries, kBlock)), dim3(kBlock), 0,
                       stream, grid, bl.entries);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(brick_mark_kernel<D>, dim3(nb), dim3(kBlock), 0, stream, t, n, grid);
    RHIP_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL(brick_count_kernel<D>, dim3(chunks), dim3(kBlock), 0, stream, bs, t, grid,
                     cells, cpb, chunk_rows);
  RHIP_LAUNCH_CHECK();
  const bool self_scan = chunks <= kSelfScanBlocks;
  if (!self_scan) {
    hipLaunchKernelGGL(scan_kernel<int32_t>, dim3(1), dim3(1024), 0, stream, chunk_rows, chunks,
                       chunk_base, total);
    RHIP_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL(brick_base_kernel<D>, dim3(chunks), dim3(kBlock), 0, stream, bs, t,
                     chunk_rows, self_scan ? nullptr : chunk_base, grid);
  RHIP_LAUNCH_CHECK();
  hipLaunchKernelGGL(brick_place_kernel<D>, dim3(nb), dim3(kBlock), 0, stream, t, n, grid, order,
                     pos);
  RHIP_LAUNCH_CHECK();
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
    const BrickLayout bl = brick_layout(*table);
    const bool with_grid = bricks != nullptr && bl.entries > 0 &&
                           brick_bytes >= static_cast<size_t>(bl.entries) * sizeof(Brick);
    const int D = table->ncol - 1;
    if (with_grid) {
      table->brick_levels = bl.levels;
      for (int c = 0; c < RHIP_MAX_COLS; ++c)
        table->brick_dims[c] = bl.dims[c];
    }
    const BrickSpace bs = with_grid ? brick_space(bl, D) : BrickSpace{};
    if (bs.total > 0) {
      auto walk = [&](auto d) {
        order_by_bricks<decltype(d)::value>(*table, bl, bs, static_cast<Brick *>(bricks), order,
                                            pos, workspace, workspace_bytes, stream);
      };
      switch (D) {
      case 1: walk(std::integral_constant<int, 1>{}); break;
      case 2: walk(std::integral_constant<int, 2>{}); break;
      case 3: walk(std::integral_constant<int, 3>{}); break;
      case 4: walk(std::integral_constant<int, 4>{}); break;
      case 5: walk(std::integral_constant<int, 5>{}); break;
      default: walk(std::integral_constant<int, 6>{}); break;
      }
      table->morton_bits = ol.morton_bits;
      table->order = order;
      table->bricks = bricks;
      return;
    }
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
    table->morton_bits = ol.morton_bits;
    if (!with_grid)
      return;
    Brick *grid = static_cast<Brick *>(bricks);
    hipLaunchKernelGGL(brick_clear_kernel, dim3(ceil_div(bl.entries, kBlock)), dim3(kBlock), 0,
                       stream, grid, bl.entries);
    RHIP_LAUNCH_CHECK();
    table->order = order;
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
