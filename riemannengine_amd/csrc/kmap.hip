// Kernel-map generation for gfx950.
//
// Semantics: CoordinateMapCPU::kernel_map (RiemannEngine/engine/grid/
// lattice_cpu.hpp:606-673): for every output coordinate o and stencil offset
// k, the input row holding o + offset_k (batch column unchanged) is paired
// with o under k. The reference CPU map fills per-offset buckets from many
// threads through fetch_add, so only the *set* of pairs is defined there. The
// dormant reference GPU map sorts triplets by offset with a radix sort
// (engine/grid/lattice_gpu.cuh:438-488).
//
// The map built here serves the output-stationary convolution, so besides
// the pairs it fixes a *processing order* of the output rows (and of the
// input rows for the input gradient): rows are sorted by their neighbour
// mask (the set of offsets with a neighbour), ties kept in locality order.
// Consecutive rows then share their offset sets, so the convolution's
// 16-row MFMA groups rarely multiply a missing neighbour.
//
// Phase 1 (rhip_kmap_count):
//   probes   an output row's neighbour under offset k is found through the
//            input table's brick index when it has one (a dense grid of
//            brick entries over the locality order: one 16-byte load, a
//            popcount and a look-up in the order), else by probing the hash
//            table; probes are resolved 8 offsets at a time, their loads
//            issued together; a symmetric 3^3 map in 3-D reads the (at most
//            8) bricks of a row's neighbourhood once and derives all 27
//            probes from them (probe27_bricks);
//   masks    one lane per output row (in the output map's locality order)
//            folds the existence of its K neighbours into a sort key (the
//            mask for K <= 16, else the neighbour count above a 15-bit hash
//            of the mask);
//   sort     stable radix sort of the rows by key;
//   query    one lane per processing position p resolves its row's K
//            neighbours and writes nbr[k][p] (coalesced over p), out_order[p]
//            and per wave and offset the count of hits (ballots);
//   scan     per-offset exclusive scans of the wave counts, then the CSR
//            offsets of the pairs.
// Phase 2 (rhip_kmap_fill):
//   emit     ballot + mbcnt compaction of nbr into per-offset pair lists
//            (ordered by offset, then processing position);
//   symmetric maps (a set onto itself with a stencil closed under negation):
//            the input order is the output order and the transposed table is
//            the forward table with partner offsets, stored by the emit from
//            the entries it reads: i pairs with o under k iff o pairs with i
//            under the partner of k;
//   otherwise: the input rows' transposed masks (atomicOr during the emit),
//            a sort of the input rows by them -> in_order / in_pos, and
//            nbr_t[k][in_pos[i]] = output row paired with i under k.
#include <algorithm>
#include <cstring>
#include <type_traits>
#include <vector>

#include "rhip_internal.hpp"

namespace rhip {

constexpr int kMapBlock = 256;

// Up to kSmallUpload int32 from the host, passed by value in a kernel's
// arguments (the stencil and its partners of a 3^3 map: 108 values).
constexpr int kSmallUpload = 128;
struct SmallUpload {
  int32_t v[kSmallUpload];
};
constexpr int kMaskedK = 128; // neighbour masks (and mask order) for K <= 128
constexpr int kKeyBits = 16;  // sort-key width of a neighbour mask
static int64_t map_waves(int64_t n) { return std::max<int64_t>(1, ceil_div(n, kWave)); }

// Sort key of a neighbour mask: the mask itself for K <= 16; else the
// neighbour count (largest first) above a hash of the mask: 5 + 11 bits for
// K <= 31 (two 8-bit sort passes), 7 + 15 bits up to K = 128 (three). Equal
// masks get equal keys; unequal ones with the same count rarely collide,
// which only costs MFMA fill, never correctness. Largest first puts the
// tiles with the most stages at the front of the convolution grid, so the
// grid does not end on a few long workgroups.
__device__ __forceinline__ uint32_t mask_key(uint64_t m0, uint64_t m1, int K) {
  if (K <= kKeyBits)
    return static_cast<uint32_t>(m0);
  const uint32_t count = static_cast<uint32_t>(__popcll(m0) + __popcll(m1));
  const uint64_t h = mix64(m0 ^ mix64(m1 ^ 0x9e3779b97f4a7c15ull));
  if (K <= 31)
    return ((31u - count) << 11) | static_cast<uint32_t>(h >> 53);
  return ((127u - min(127u, count)) << 15) | static_cast<uint32_t>(h >> 49);
}
// Bits of mask_key for K offsets.
static int mask_key_bits(int K) { return K <= kKeyBits ? K : (K <= 31 ? 16 : 22); }

// Resolves probes k0 .. k0+7 of an output row with coordinates c (batch
// offset d0 = c[0] - lo[0], row_ok = the batch is in range): r[u] = the
// input row at c + offsets[k0 + u] (batch kept, wrap-around int32 arithmetic
// as the coordinate type has), or -1. With kRows false only r[u] >= 0
// matters, and brick tables skip the locality-order lookup.
//   brick index: the neighbour's brick entry, then the rank of its cell among
//     the brick's occupied cells gives its locality-order position;
//   packed keys: each neighbour's key is packed column by column (a column
//     leaving [lo, hi] is a miss, as in pack_row), the home slots of all 8
//     probes are loaded before any chain is followed;
//   row-reference tables: table_find.
template <int D, bool kRows>
__device__ __forceinline__ void probe8(const TableView &t, const int32_t *c, uint32_t d0,
                                       bool row_ok, const int32_t *__restrict__ offsets, int k0,
                                       int K, int32_t (&r)[8]) {
  if constexpr (D <= 6) {
    if (t.bricks != nullptr) {
      constexpr int L = 6 / D;
      uint64_t g[8];
      uint32_t cell[8];
      bool ok[8];
      Brick br[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + u;
        ok[u] = row_ok && k < K;
        g[u] = d0;
        cell[u] = 0;
        const int kk = k < K ? k : 0;
#pragma unroll
        for (int i = 1; i <= D; ++i) {
          const uint32_t v = static_cast<uint32_t>(c[i]) +
                             static_cast<uint32_t>(offsets[kk * D + (i - 1)]) -
                             static_cast<uint32_t>(t.lo[i]);
          ok[u] = ok[u] && v <= t.span[i] && (v & ((1u << t.tz[i]) - 1u)) == 0;
          const uint32_t w = v >> t.tz[i];
          g[u] = g[u] * static_cast<uint32_t>(t.dims[i]) + (w >> L);
#pragma unroll
          for (int l = 0; l < L; ++l)
            cell[u] |= ((w >> l) & 1u) << (l * D + (D - i));
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (ok[u])
          br[u] = t.bricks[g[u]];
      int32_t jj[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        jj[u] = -1;
        if (ok[u] && ((br[u].mask >> cell[u]) & 1ull))
          jj[u] = br[u].base + __popcll(br[u].mask & ((1ull << cell[u]) - 1ull));
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        r[u] = kRows ? (jj[u] >= 0 ? t.order[jj[u]] : -1) : jj[u];
      return;
    }
  }
  if (t.mode == RHIP_KEY_PACKED64) {
    const uint64_t base = static_cast<uint64_t>(d0) << t.shift[0];
    uint64_t key[8], h[8];
    bool ok[8];
    Slot sl[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u;
      ok[u] = row_ok && k < K;
      key[u] = base;
      const int kk = k < K ? k : 0;
#pragma unroll
      for (int i = 1; i <= D; ++i) {
        const uint32_t v = static_cast<uint32_t>(c[i]) +
                           static_cast<uint32_t>(offsets[kk * D + (i - 1)]);
        const uint32_t d = v - static_cast<uint32_t>(t.lo[i]);
        ok[u] = ok[u] && d <= t.span[i];
        key[u] |= static_cast<uint64_t>(d) << t.shift[i];
      }
      h[u] = mix64(key[u]) & t.mask;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (ok[u])
        sl[u] = t.slots[h[u]];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      r[u] = -1;
      if (ok[u]) {
        while (sl[u].word != key[u] && sl[u].word != kEmptyWord) {
          h[u] = (h[u] + 1) & t.mask;
          sl[u] = t.slots[h[u]];
        }
        if (sl[u].word == key[u])
          r[u] = static_cast<int32_t>(sl[u].uid);
      }
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int k = k0 + u;
    r[u] = -1;
    if (k < K) {
      int32_t q[RHIP_MAX_COLS] = {};
      q[0] = c[0];
#pragma unroll
      for (int i = 1; i <= D; ++i)
        q[i] = static_cast<int32_t>(static_cast<uint32_t>(c[i]) +
                                    static_cast<uint32_t>(offsets[k * D + (i - 1)]));
      r[u] = table_find(t, q);
    }
  }
}

// The 3^3 neighbourhood of a row of a symmetric map through the brick grid:
// D = 3, bricks of 4 x 4 x 4 cells (brick levels 2), and the stencil in cell
// units (offsets divided by the column's 2^tz) the canonical 3^3 region,
// offset k = (k % 3 - 1, k / 3 % 3 - 1, k / 9 - 1) along columns 1..3. The
// row is one of the table's own rows, so its cell w = (c - lo) >> tz is
// exact. Its 27 neighbours lie in at most 8 bricks: along each column the
// row's brick and, where the cell sits on the brick's low (high) face, the
// brick below (above). The row loads those bricks once, corner cc holding
// the brick shifted along column i when bit i - 1 of cc is set (probe8 loads
// one brick per offset: 27 loads, most of them the row's own brick again),
// and reads every neighbour's occupancy bit and rank from the brick its
// offset reaches. kRows: r[k] = the neighbour's row (through the locality
// order) or -1, else r[k] >= 0 marks a neighbour.
template <bool kRows>
__device__ __forceinline__ void probe27_bricks(const TableView &t, const int32_t *c, uint32_t d0,
                                               bool row_ok, int32_t (&r)[27]) {
  uint32_t q[4], b[4];
  bool lo_face[4], hi_face[4];
#pragma unroll
  for (int i = 1; i <= 3; ++i) {
    const uint32_t w = (static_cast<uint32_t>(c[i]) - static_cast<uint32_t>(t.lo[i])) >> t.tz[i];
    q[i] = w & 3u;
    b[i] = w >> 2;
    lo_face[i] = q[i] == 0u;
    hi_face[i] = q[i] == 3u;
  }
  uint64_t mk[8];
  int32_t base[8];
#pragma unroll
  for (int cc = 0; cc < 8; ++cc) {
    bool need = row_ok;
    int64_t g = d0;
#pragma unroll
    for (int i = 1; i <= 3; ++i) {
      const bool sh = (cc >> (i - 1)) & 1;
      // a shifted column is needed only on a face; the brick below a cell
      // in brick 0 wraps to 2^32 - 1 and fails the extent check
      if (sh)
        need = need && (lo_face[i] || hi_face[i]);
      const uint32_t bc = b[i] + (sh ? (lo_face[i] ? 0xffffffffu : 1u) : 0u);
      need = need && bc < static_cast<uint32_t>(t.dims[i]);
      g = g * t.dims[i] + bc;
    }
    mk[cc] = 0;
    base[cc] = 0;
    if (need) {
      const Brick br = t.bricks[g];
      mk[cc] = br.mask;
      base[cc] = br.base;
    }
  }
  // cell bit of in-brick coordinate v along column i: bit l of v at l*3 + 3 - i
  auto spread = [](uint32_t v, int i) {
    return ((v & 1u) << (3 - i)) | (((v >> 1) & 1u) << (6 - i));
  };
#pragma unroll
  for (int k = 0; k < 27; ++k) {
    const int dl[4] = {0, k % 3 - 1, (k / 3) % 3 - 1, k / 9 - 1};
    bool x[4];
    uint32_t cell = 0;
#pragma unroll
    for (int i = 1; i <= 3; ++i) {
      x[i] = dl[i] < 0 ? lo_face[i] : (dl[i] > 0 ? hi_face[i] : false);
      cell |= spread((q[i] + static_cast<uint32_t>(dl[i])) & 3u, i);
    }
    // mk[x1 + 2 x2 + 4 x3] as a select tree over the columns the offset moves
    uint64_t m4[4];
    int32_t b4[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      m4[a] = x[3] ? mk[a + 4] : mk[a];
      b4[a] = x[3] ? base[a + 4] : base[a];
    }
    const uint64_t m2_0 = x[2] ? m4[2] : m4[0], m2_1 = x[2] ? m4[3] : m4[1];
    const int32_t b2_0 = x[2] ? b4[2] : b4[0], b2_1 = x[2] ? b4[3] : b4[1];
    const uint64_t m = x[1] ? m2_1 : m2_0;
    const int32_t bs = x[1] ? b2_1 : b2_0;
    const bool hit = (m >> cell) & 1ull;
    if constexpr (kRows) {
      const int32_t jj = bs + __popcll(m & ((1ull << cell) - 1ull));
      r[k] = hit ? t.order[jj] : -1;
    } else {
      r[k] = hit ? 0 : -1;
    }
  }
}

// The 3^4 neighbourhood of a row of a symmetric 4-D map through the brick
// grid: D = 4, bricks of 2 x 2 x 2 x 2 cells (brick level 1), and the stencil
// in cell units the canonical 3^4 region in its order, offset k =
// (k % 3 - 1, k / 3 % 3 - 1, k / 9 % 3 - 1, k / 27 - 1) along columns 1..4.
// A cell sits on a face of its brick along every column (cell coordinate 0:
// the low face, 1: the high one), so its 81 neighbours lie in 16 bricks: the
// row's own and, along each column, the one below (cell 0) or above (cell
// 1). The row loads those 16 once, corner cc holding the brick shifted along
// column i when bit i - 1 of cc is set (probe8 loads one brick per offset:
// 81 loads), and each offset reads its neighbour's occupancy bit and rank
// from the brick it reaches, selected by a 16-way tree. f(k, v) receives
// each offset's result: the neighbour's row (through the locality order) or
// -1 with kRows, else v >= 0 marks a neighbour.
template <bool kRows, typename F>
__device__ __forceinline__ void probe81_bricks(const TableView &t, const int32_t *c, uint32_t d0,
                                               bool row_ok, F &&f) {
  uint32_t q[5], b[5];
#pragma unroll
  for (int i = 1; i <= 4; ++i) {
    const uint32_t w = (static_cast<uint32_t>(c[i]) - static_cast<uint32_t>(t.lo[i])) >> t.tz[i];
    q[i] = w & 1u;
    b[i] = w >> 1;
  }
  uint32_t mk[16]; // 16 cells: the low half of the brick's mask
  int32_t base[16];
#pragma unroll
  for (int cc = 0; cc < 16; ++cc) {
    bool need = row_ok;
    int64_t g = d0;
#pragma unroll
    for (int i = 1; i <= 4; ++i) {
      const bool sh = (cc >> (i - 1)) & 1;
      // the brick below a cell in brick 0 wraps to 2^32 - 1 and fails the
      // extent check
      const uint32_t bc = b[i] + (sh ? (q[i] == 0u ? 0xffffffffu : 1u) : 0u);
      need = need && bc < static_cast<uint32_t>(t.dims[i]);
      g = g * t.dims[i] + bc;
    }
    mk[cc] = 0;
    base[cc] = 0;
    if (need) {
      const Brick br = t.bricks[g];
      mk[cc] = static_cast<uint32_t>(br.mask);
      base[cc] = br.base;
    }
  }
#pragma unroll
  for (int k = 0; k < 81; ++k) {
    const int dl[5] = {0, k % 3 - 1, (k / 3) % 3 - 1, (k / 9) % 3 - 1, k / 27 - 1};
    bool x[5];
    uint32_t cell = 0;
#pragma unroll
    for (int i = 1; i <= 4; ++i) {
      // the offset leaves the brick along column i: down from cell 0, up
      // from cell 1
      x[i] = dl[i] < 0 ? q[i] == 0u : (dl[i] > 0 ? q[i] == 1u : false);
      cell |= ((q[i] + static_cast<uint32_t>(dl[i])) & 1u) << (4 - i);
    }
    // mk[x1 + 2 x2 + 4 x3 + 8 x4] as a select tree over the columns
    uint32_t m8[8];
    int32_t b8[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      m8[a] = x[4] ? mk[a + 8] : mk[a];
      b8[a] = x[4] ? base[a + 8] : base[a];
    }
    uint32_t m4[4];
    int32_t b4[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      m4[a] = x[3] ? m8[a + 4] : m8[a];
      b4[a] = x[3] ? b8[a + 4] : b8[a];
    }
    const uint32_t m2_0 = x[2] ? m4[2] : m4[0], m2_1 = x[2] ? m4[3] : m4[1];
    const int32_t b2_0 = x[2] ? b4[2] : b4[0], b2_1 = x[2] ? b4[3] : b4[1];
    const uint32_t m = x[1] ? m2_1 : m2_0;
    const int32_t bs = x[1] ? b2_1 : b2_0;
    const bool hit = (m >> cell) & 1u;
    if constexpr (kRows) {
      const int32_t jj = bs + __popc(m & ((1u << cell) - 1u));
      f(k, hit ? t.order[jj] : -1);
    } else {
      f(k, hit ? 0 : -1);
    }
  }
}

// Mask pass: one lane per output row j in spatial order (row spatial[j]):
// keys[j] = the sort key of the row's neighbour mask, vals[j] = its output
// row spatial[j].
// KC > 0: K == KC at compile time (the probe rounds unroll and the stencil
// loads hoist out of them). NBHD: the symmetric 3^3 map through
// probe27_bricks (KC == 27, D == 3) or 3^4 map through probe81_bricks
// (KC == 81, D == 4).
template <int D, int KC = 0, bool NBHD = false>
__global__ __launch_bounds__(kMapBlock) void kmap_mask_kernel(
    TableView t, const int32_t *__restrict__ out_coords, const int32_t *__restrict__ spatial,
    int64_t n_out, const int32_t *__restrict__ offsets, int K, uint32_t *__restrict__ keys,
    int32_t *__restrict__ vals) {
  if constexpr (KC > 0)
    K = KC;
  const int64_t j = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (j >= n_out)
    return;
  const int64_t o = spatial ? spatial[j] : j;
  int32_t c[D + 1];
#pragma unroll
  for (int i = 0; i <= D; ++i)
    c[i] = out_coords[o * (D + 1) + i];
  const uint32_t d0 = static_cast<uint32_t>(c[0]) - static_cast<uint32_t>(t.lo[0]);
  const bool row_ok = d0 <= t.span[0];
  uint64_t m0 = 0, m1 = 0;
  if constexpr (NBHD) {
    static_assert((D == 3 && KC == 27) || (D == 4 && KC == 81),
                  "the neighbourhood probes are the 3^3 stencil in 3-D and 3^4 in 4-D");
    if constexpr (D == 3) {
      int32_t r[27];
      probe27_bricks<false>(t, c, d0, row_ok, r);
#pragma unroll
      for (int k = 0; k < 27; ++k)
        if (r[k] >= 0)
          m0 |= 1ull << k;
    } else {
      probe81_bricks<false>(t, c, d0, row_ok, [&](int k, int32_t v) {
        if (v >= 0) {
          if (k < 64)
            m0 |= 1ull << k;
          else
            m1 |= 1ull << (k - 64);
        }
      });
    }
    keys[j] = mask_key(m0, m1, K);
    vals[j] = static_cast<int32_t>(o);
    return;
  }
#pragma unroll
  for (int k0 = 0; k0 < (KC > 0 ? KC : K); k0 += 8) {
    int32_t r[8];
    probe8<D, false>(t, c, d0, row_ok, offsets, k0, K, r);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u;
      if (r[u] >= 0) {
        if (k < 64)
          m0 |= 1ull << k;
        else
          m1 |= 1ull << (k - 64);
      }
    }
  }
  keys[j] = mask_key(m0, m1, K);
  vals[j] = static_cast<int32_t>(o);
}

// Query pass: one lane per processing position p (output row jpos[p] from
// the mask sort, else spatial[p], else p): nbr[k][p] = the input row paired
// with it under k
// (coalesced over p; streaming stores for it ran the kernel 22.8 -> 28.9 us
// on config 2), out_order[p] = its row, and per offset k the number of
// hits of each wave w, wave_counts[k][w]. Workgroup 0 also clears the
// ticket of kmap_totals_kernel, which runs next.
template <int D, int KC = 0, bool NBHD = false>
__global__ __launch_bounds__(kMapBlock) void kmap_query_kernel(
    TableView t, const int32_t *__restrict__ out_coords, const int32_t *__restrict__ spatial,
    const int32_t *__restrict__ jpos, int64_t n_out, const int32_t *__restrict__ offsets, int K,
    int64_t nw, int32_t *__restrict__ nbr, int32_t *__restrict__ out_order,
    int32_t *__restrict__ wave_counts, SmallUpload up, int32_t *__restrict__ up_dst0, int up_n0,
    int32_t *__restrict__ up_dst1, int up_n1, uint32_t *__restrict__ ticket) {
  if constexpr (KC > 0)
    K = KC;
  // a few host values for later launches, carried in the arguments: the
  // first up_n0 go to up_dst0, the next up_n1 to up_dst1
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i < up_n0; i += kMapBlock)
      up_dst0[i] = up.v[i];
    for (int i = threadIdx.x; i < up_n1; i += kMapBlock)
      up_dst1[i] = up.v[up_n0 + i];
    if (threadIdx.x == 0)
      *ticket = 0;
  }
  const int64_t p = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  const int64_t w = p / kWave;
  if (w >= nw) // whole waves past the last row
    return;
  const bool in = p < n_out;
  int32_t c[D + 1] = {};
  if (in) {
    // the mask sort carries the output row itself: one dependent load less
    const int64_t o = jpos ? jpos[p] : (spatial ? spatial[p] : p);
    out_order[p] = static_cast<int32_t>(o);
#pragma unroll
    for (int i = 0; i <= D; ++i)
      c[i] = out_coords[o * (D + 1) + i];
  }
  const uint32_t d0 = static_cast<uint32_t>(c[0]) - static_cast<uint32_t>(t.lo[0]);
  const bool row_ok = in && d0 <= t.span[0];
  if constexpr (NBHD) {
    static_assert((D == 3 && KC == 27) || (D == 4 && KC == 81),
                  "the neighbourhood probes are the 3^3 stencil in 3-D and 3^4 in 4-D");
    auto put = [&](int k, int32_t v) {
      if (in)
        nbr[k * n_out + p] = v;
      const uint64_t hits = __ballot(v >= 0);
      if (lane_id() == 0)
        wave_counts[k * nw + w] = __popcll(hits);
    };
    if constexpr (D == 3) {
      int32_t r[27];
      probe27_bricks<true>(t, c, d0, row_ok, r);
#pragma unroll
      for (int k = 0; k < 27; ++k)
        put(k, r[k]);
    } else {
      probe81_bricks<true>(t, c, d0, row_ok, put);
    }
    return;
  }
#pragma unroll
  for (int k0 = 0; k0 < (KC > 0 ? KC : K); k0 += 8) {
    int32_t r[8];
    probe8<D, true>(t, c, d0, row_ok, offsets, k0, K, r);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u;
      if (k < K) {
        if (in)
          nbr[k * n_out + p] = r[u];
        const uint64_t hits = __ballot(r[u] >= 0);
        if (lane_id() == 0)
          wave_counts[k * nw + w] = __popcll(hits);
      }
    }
  }
}

// The CSR offsets of K pair totals, by one 1024-thread workgroup: total(i)
// reads total i; the offsets go to kmap_offsets and, when given, to host
// memory mapped for the device.
template <typename Total>
__device__ void offsets_from_totals(Total total, int K, int64_t *kmap_offsets,
                                    int64_t *host_offsets) {
  __shared__ int64_t partial[1024];
  const int t = threadIdx.x;
  const int per = (K + 1023) / 1024;
  const int b = t * per, e = min(K, b + per);
  int64_t s = 0;
  for (int i = b; i < e; ++i)
    s += total(i);
  partial[t] = s;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    int64_t v = t >= off ? partial[t - off] : 0;
    __syncthreads();
    partial[t] += v;
    __syncthreads();
  }
  int64_t run = partial[t] - s;
  for (int i = b; i < e; ++i) {
    kmap_offsets[i] = run;
    if (host_offsets)
      host_offsets[i] = run;
    run += total(i);
  }
  if (t == 1023) {
    kmap_offsets[K] = partial[1023];
    if (host_offsets)
      host_offsets[K] = partial[1023];
  }
}

__global__ __launch_bounds__(1024) void kmap_offsets_kernel(const int64_t *ktotal, int K,
                                                            int64_t *kmap_offsets,
                                                            int64_t *host_offsets) {
  offsets_from_totals([&](int i) { return ktotal[i]; }, K, kmap_offsets, host_offsets);
}

// Workgroup k: the exclusive scan of offset k's wave counts (wave_base, for
// phase 2's emit) and its pair total. The workgroup that finishes last (by
// a ticket the query kernel cleared) turns the K totals into the CSR
// offsets: one launch where a scan and an offsets launch were. The totals
// are stored and read as agent-scope atomics, after a release (the ticket's
// increment) and an acquire, so the last workgroup sees every other
// workgroup's total whichever XCD wrote it.
__global__ __launch_bounds__(1024) void kmap_totals_kernel(const int32_t *wave_counts, int64_t nw,
                                                           int K, int64_t *wave_base,
                                                           int64_t *ktotal, uint32_t *ticket,
                                                           int64_t *kmap_offsets,
                                                           int64_t *host_offsets) {
  __shared__ int last;
  const int64_t total = segment_scan(wave_counts, nw, wave_base);
  if (threadIdx.x == 0) {
    __hip_atomic_store(&ktotal[blockIdx.x], total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __threadfence();
    last = atomicAdd(ticket, 1u) == static_cast<uint32_t>(K - 1);
    __threadfence();
  }
  __syncthreads();
  if (!last)
    return; // uniform
  offsets_from_totals(
      [&](int i) {
        return __hip_atomic_load(&ktotal[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      },
      K, kmap_offsets, host_offsets);
}

__global__ __launch_bounds__(kMapBlock) void fill_i32_kernel(int32_t *p,
                                                             int64_t n,
                                                             int32_t v) {
  int64_t i = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (i < n)
    p[i] = v;
}

__global__ __launch_bounds__(kMapBlock) void zero_u64_kernel(unsigned long long *p,
                                                             int64_t n) {
  int64_t i = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (i < n)
    p[i] = 0ull;
}

// Lane per processing position p and offset k = blockIdx.y: a hit is written
// at its offset's start + its wave's run (wave_base) + its rank in the wave.
// Symmetric maps (partner given): the transposed table is the forward table
// with partner rows, nbr_t[partner[k]][p] = nbr[k][p] (partner is its own
// inverse), and the input order is the output order; the emit stores both
// from the values it already holds instead of a second pass over nbr.
__global__ __launch_bounds__(kMapBlock) void kmap_emit_kernel(
    const int32_t *__restrict__ nbr, const int32_t *__restrict__ out_order,
    int64_t n_out, int64_t nw, const int64_t *__restrict__ kofs,
    const int64_t *__restrict__ wave_base, int32_t *__restrict__ in_rows,
    int32_t *__restrict__ out_rows, unsigned long long *__restrict__ mask_t,
    const int32_t *__restrict__ partner, int K, int32_t *__restrict__ nbr_t,
    int32_t *__restrict__ in_order) {
  const int k = blockIdx.y;
  const int64_t p = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  const int64_t w = p / kWave;
  if (w >= nw)
    return;
  const int32_t v = p < n_out ? nbr[k * n_out + p] : -1;
  if (partner != nullptr && p < n_out) {
    const int32_t pk = partner[k];
    if (pk >= 0 && pk < K) // a workspace not prepared by phase 1 writes nothing
      nbr_t[static_cast<int64_t>(pk) * n_out + p] = v;
    if (k == 0)
      in_order[p] = out_order[p];
  }
  const uint64_t b = __ballot(v >= 0);
  if (v >= 0) {
    if (in_rows != nullptr) { // pair lists requested
      const int64_t q = kofs[k] + wave_base[k * nw + w] + lanes_below(b);
      in_rows[q] = v;
      out_rows[q] = out_order[p];
    }
    if (mask_t)
      atomicOr(&mask_t[2 * static_cast<int64_t>(v) + (k >> 6)], 1ull << (k & 63));
  }
}

// Hits of each wave and offset in a finished table (lane per processing
// position p, offset k = blockIdx.y): wave_counts[k][w], as the query pass
// counts them, for pair lists emitted after the build.
__global__ __launch_bounds__(kMapBlock) void kmap_wave_count_kernel(
    const int32_t *__restrict__ nbr, int64_t n_out, int64_t nw,
    int32_t *__restrict__ wave_counts) {
  const int k = blockIdx.y;
  const int64_t p = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  const int64_t w = p / kWave;
  if (w >= nw)
    return;
  const int32_t v = p < n_out ? nbr[k * n_out + p] : -1;
  const uint64_t b = __ballot(v >= 0);
  if (lane_id() == 0)
    wave_counts[k * nw + w] = __popcll(b);
}

__global__ __launch_bounds__(kMapBlock) void in_key_kernel(
    const unsigned long long *__restrict__ mask_t, const int32_t *__restrict__ spatial,
    int64_t n, int K, uint32_t *__restrict__ keys, int32_t *__restrict__ vals) {
  const int64_t q = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (q >= n)
    return;
  const int64_t i = spatial ? spatial[q] : q;
  keys[q] = mask_key(mask_t[2 * i], mask_t[2 * i + 1], K);
  vals[q] = static_cast<int32_t>(q);
}

__global__ __launch_bounds__(kMapBlock) void in_order_kernel(
    const int32_t *__restrict__ qpos, const int32_t *__restrict__ spatial, int64_t n,
    int32_t *__restrict__ in_order, int32_t *__restrict__ in_pos) {
  const int64_t q = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (q >= n)
    return;
  const int64_t qs = qpos ? qpos[q] : q;
  const int32_t i = spatial ? spatial[qs] : static_cast<int32_t>(qs);
  in_order[q] = i;
  in_pos[i] = static_cast<int32_t>(q);
}

__global__ __launch_bounds__(kMapBlock) void kmap_transpose_kernel(
    const int32_t *__restrict__ nbr, const int32_t *__restrict__ out_order,
    int64_t n_out, const int32_t *__restrict__ in_pos, int64_t n_in,
    int32_t *__restrict__ nbr_t) {
  const int k = blockIdx.y;
  const int64_t p = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (p >= n_out)
    return;
  const int32_t v = nbr[k * n_out + p];
  if (v >= 0)
    nbr_t[k * n_in + in_pos[v]] = out_order[p];
}

// Workspace: the per-block counts, their scans and the per-offset totals
// persist from phase 1 to phase 2; each phase's scratch reuses the same
// region after them.
// Host-to-device upload of a few int32 through kernel arguments: launched
// asynchronously like any kernel, no staging copy. 960 values per launch
// keep the arguments under 4 KB.
constexpr int kUploadInts = 960;
struct UploadArg {
  int32_t v[kUploadInts];
};
static __global__ void upload_i32_kernel(UploadArg a, int32_t *__restrict__ dst, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x)
    dst[i] = a.v[i];
}

static void upload_i32(int32_t *dst, const int32_t *src, size_t n, hipStream_t stream) {
  for (size_t o = 0; o < n; o += kUploadInts) {
    UploadArg a{};
    const int m = static_cast<int>(std::min<size_t>(kUploadInts, n - o));
    std::memcpy(a.v, src + o, sizeof(int32_t) * m);
    hipLaunchKernelGGL(upload_i32_kernel, dim3(1), dim3(256), 0, stream, a, dst + o, m);
    RHIP_LAUNCH_CHECK();
  }
}

struct KmapWs {
  int32_t *wave_counts; // [K][waves] hits per wave and offset (phase 1)
  int64_t *wave_base;   // their per-offset exclusive scans (phase 1 -> 2)
  int64_t *ktotal;
  uint32_t *ticket;     // kmap_totals_kernel's finished workgroups
  int32_t *offsets;     // [K][D] stencil (D = the table's ncol - 1)
  int32_t *partner;     // [K] partner offsets of a symmetric map (phase 1 -> 2)
  // phase 1
  uint32_t *keys_a, *keys_b;
  int32_t *vals_a, *vals_b;
  void *sort_tmp;
  size_t sort_bytes;
  // phase 2
  unsigned long long *mask_t;
  uint32_t *tkeys_a, *tkeys_b;
  int32_t *tvals_a, *tvals_b, *in_pos;
  void *tsort_tmp;
  size_t tsort_bytes;
};

static KmapWs carve_kmap(Carve &cv, int64_t n_in, int64_t n_out, int32_t K, int32_t D) {
  const int64_t nw = map_waves(n_out);
  const int64_t mo = std::max<int64_t>(n_out, 1), mi = std::max<int64_t>(n_in, 1);
  KmapWs w{};
  w.wave_counts = cv.take<int32_t>(nw * K);
  w.wave_base = cv.take<int64_t>(nw * K);
  w.ktotal = cv.take<int64_t>(K);
  w.ticket = cv.take<uint32_t>(1);
  w.offsets = cv.take<int32_t>(static_cast<size_t>(K) * std::max(D, 1));
  w.partner = cv.take<int32_t>(K);
  const size_t base = cv.used;
  w.keys_a = cv.take<uint32_t>(mo);
  w.keys_b = cv.take<uint32_t>(mo);
  w.vals_a = cv.take<int32_t>(mo);
  w.vals_b = cv.take<int32_t>(mo);
  w.sort_bytes = sort_pairs_u32_bytes(mo);
  w.sort_tmp = cv.take<char>(w.sort_bytes);
  const size_t end1 = cv.used;
  cv.used = base;
  w.mask_t = cv.take<unsigned long long>(2 * mi);
  w.tkeys_a = cv.take<uint32_t>(mi);
  w.tkeys_b = cv.take<uint32_t>(mi);
  w.tvals_a = cv.take<int32_t>(mi);
  w.tvals_b = cv.take<int32_t>(mi);
  w.in_pos = cv.take<int32_t>(mi);
  w.tsort_bytes = sort_pairs_u32_bytes(mi);
  w.tsort_tmp = cv.take<char>(w.tsort_bytes);
  cv.used = std::max(cv.used, end1);
  return w;
}

// Calls f(std::integral_constant<int, D>) for the table's spatial dimension.
template <typename F> void with_dim(int D, F &&f) {
  switch (D) {
  case 1: f(std::integral_constant<int, 1>{}); break;
  case 2: f(std::integral_constant<int, 2>{}); break;
  case 3: f(std::integral_constant<int, 3>{}); break;
  case 4: f(std::integral_constant<int, 4>{}); break;
  case 5: f(std::integral_constant<int, 5>{}); break;
  case 6: f(std::integral_constant<int, 6>{}); break;
  case 7: f(std::integral_constant<int, 7>{}); break;
  default: throw Error(RHIP_ERR_INVALID, "coordinate rows need 1 to 7 spatial columns");
  }
}

// Partner offsets of a symmetric map: a map of a set onto itself (same rows,
// same order) whose offsets are distinct and closed under negation. Empty
// when the map is not symmetric.
static std::vector<int32_t> symmetric_partners(const rhip_table *in_table,
                                               const int32_t *out_coords, int64_t n_out,
                                               int32_t K, const int32_t *offsets_host) {
  const int D = in_table->ncol - 1;
  std::vector<int32_t> partner(static_cast<size_t>(K), -1);
  if (out_coords != in_table->rows || n_out != in_table->n_unique || n_out < 2 ||
      K > kMaskedK)
    return {};
  auto row = [&](int k) { return offsets_host + static_cast<size_t>(k) * D; };
  for (int a = 0; a < K; ++a) {
    for (int b = 0; b < K; ++b) {
      bool same = b != a, neg = true;
      for (int d = 0; d < D; ++d) {
        same = same && row(b)[d] == row(a)[d];
        neg = neg && static_cast<uint32_t>(row(b)[d]) ==
                         0u - static_cast<uint32_t>(row(a)[d]); // wrap-around negation
      }
      if (same)
        return {}; // repeated offsets: the general path
      if (neg)
        partner[a] = b;
    }
    if (partner[a] < 0)
      return {};
  }
  return partner;
}

// Whether a symmetric 3-D map takes probe27_bricks: a brick grid of
// 4 x 4 x 4 cells and the stencil, in cell units of the table (offset
// column i divided by 2^tz[i]), the canonical 3^3 region in its order.
static bool nbhd27(const rhip_table *t, int32_t K, const int32_t *offsets_host) {
  if (K != 27 || t->ncol != 4 || t->bricks == nullptr || t->order == nullptr ||
      t->brick_levels != 2)
    return false;
  for (int k = 0; k < 27; ++k) {
    const int dl[3] = {k % 3 - 1, (k / 3) % 3 - 1, k / 9 - 1};
    for (int i = 0; i < 3; ++i) {
      const int tz = t->tz[i + 1];
      if (tz < 0 || tz > 30 ||
          static_cast<int64_t>(offsets_host[k * 3 + i]) != int64_t(dl[i]) * (int64_t(1) << tz))
        return false;
    }
  }
  return true;
}

// Whether a symmetric 4-D map takes probe81_bricks: a brick grid of
// 2 x 2 x 2 x 2 cells and the stencil, in cell units of the table, the
// canonical 3^4 region in its order.
static bool nbhd81(const rhip_table *t, int32_t K, const int32_t *offsets_host) {
  if (K != 81 || t->ncol != 5 || t->bricks == nullptr || t->order == nullptr ||
      t->brick_levels != 1)
    return false;
  for (int k = 0; k < 81; ++k) {
    const int dl[4] = {k % 3 - 1, (k / 3) % 3 - 1, (k / 9) % 3 - 1, k / 27 - 1};
    for (int i = 0; i < 4; ++i) {
      const int tz = t->tz[i + 1];
      if (tz < 0 || tz > 30 ||
          static_cast<int64_t>(offsets_host[k * 4 + i]) != int64_t(dl[i]) * (int64_t(1) << tz))
        return false;
    }
  }
  return true;
}

} // namespace rhip

using namespace rhip;

extern "C" int rhip_kmap_workspace_bytes(int64_t n_in, int64_t n_out, int32_t K,
                                         size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0 && K >= 1, "need n_in, n_out >= 0 and K >= 1");
    Carve cv(nullptr, 0);
    carve_kmap(cv, n_in, n_out, K, RHIP_MAX_COLS - 1);
    *bytes = cv.used + 256;
  });
}

extern "C" int rhip_kmap_count(const rhip_table *in_table, const int32_t *out_coords,
                               const int32_t *out_spatial_order, int64_t n_out,
                               int32_t K, const int32_t *offsets_host, void *workspace,
                               size_t workspace_bytes, int32_t *nbr, int32_t *out_order,
                               int64_t *kmap_offsets, int64_t *kmap_offsets_host,
                               int32_t *flags, hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(in_table != nullptr, "in_table is null");
    RHIP_CHECK_ARG(K >= 1 && K <= 65535, "K must be in [1, 65535]");
    RHIP_CHECK_ARG(n_out >= 0 && n_out < INT32_MAX, "bad n_out");
    RHIP_CHECK_ARG(kmap_offsets && workspace && offsets_host,
                   "offsets_host, kmap_offsets and workspace are required");
    const int D = in_table->ncol - 1;
    Carve cv(workspace, workspace_bytes);
    KmapWs w = carve_kmap(cv, in_table->n_unique, n_out, K, RHIP_MAX_COLS - 1);
    const int64_t nb = std::max<int64_t>(1, ceil_div(n_out, kMapBlock));
    const int64_t nw = map_waves(n_out);
    const std::vector<int32_t> partner =
        symmetric_partners(in_table, out_coords, n_out, K, offsets_host);
    const bool sym = !partner.empty();
    if (flags)
      *flags = sym ? RHIP_KMAP_SYMMETRIC : 0;
    if (n_out == 0) {
      hipLaunchKernelGGL(fill_i32_kernel, dim3(ceil_div(nw * K, kMapBlock)),
                         dim3(kMapBlock), 0, stream, w.wave_counts, nw * K, 0);
      RHIP_LAUNCH_CHECK();
    } else {
      RHIP_CHECK_ARG(out_coords && nbr && out_order, "out_coords, nbr and out_order are required");
      // small host arrays go in kernel arguments (a copy from pageable
      // memory would wait for the device)
      // the stencil and the partners are consecutive in the workspace: one
      // upload for both
      std::vector<int32_t> up(offsets_host, offsets_host + static_cast<size_t>(K) * D);
      if (sym) {
        up.resize(static_cast<size_t>(w.partner - w.offsets));
        up.insert(up.end(), partner.begin(), partner.end());
      }
      const bool masks = K <= kMaskedK && n_out > 1 && in_table->n_unique > 0;
      const TableView tv = make_view(*in_table);
      const int32_t *jpos = nullptr;
      // the symmetric 3^3 map reads each row's neighbourhood bricks once; its
      // probes need no stencil on the device, so the stencil and the partners
      // ride in the query's arguments (two spans: the partners sit after the
      // stencil's padded slot in the workspace)
      const int n_sten = K * D, n_part = sym ? K : 0;
      const bool nbhd = sym && nbhd27(in_table, K, offsets_host) &&
                        n_sten + n_part <= kSmallUpload;
      // the symmetric 3^4 map reads its 16 neighbourhood bricks once per row
      // (its stencil and partners are too many for the arguments: uploaded)
      const bool nbhd4 = sym && nbhd81(in_table, K, offsets_host);
      SmallUpload small{};
      if ((nbhd || nbhd4) && flags)
        *flags |= RHIP_KMAP_BRICK_NBHD;
      if (nbhd) {
        std::memcpy(small.v, offsets_host, sizeof(int32_t) * n_sten);
        std::memcpy(small.v + n_sten, partner.data(), sizeof(int32_t) * n_part);
      } else {
        upload_i32(w.offsets, up.data(), up.size(), stream);
      }
      with_dim(D, [&](auto dc) {
        constexpr int DD = decltype(dc)::value;
        // the 3^3 stencil unrolled (config 2: mask 30 -> 25 us, query 36 -> 33 us)
        const bool k27 = K == 27 && DD == 3;
        if constexpr (DD == 3) {
          if (nbhd) {
            if (masks) {
              hipLaunchKernelGGL((kmap_mask_kernel<3, 27, true>), dim3(nb), dim3(kMapBlock), 0,
                                 stream, tv, out_coords, out_spatial_order, n_out, w.offsets, K,
                                 w.keys_a, w.vals_a);
              RHIP_LAUNCH_CHECK();
              sort_pairs_u32(w.sort_tmp, w.sort_bytes, w.keys_a, w.keys_b, w.vals_a, w.vals_b,
                             n_out, mask_key_bits(K), stream);
              jpos = w.vals_b;
            }
            hipLaunchKernelGGL((kmap_query_kernel<3, 27, true>), dim3(nb), dim3(kMapBlock), 0,
                               stream, tv, out_coords, out_spatial_order, jpos, n_out, w.offsets,
                               K, nw, nbr, out_order, w.wave_counts, small, w.offsets,
                               n_sten, w.partner, n_part, w.ticket);
            RHIP_LAUNCH_CHECK();
            return;
          }
        }
        if constexpr (DD == 4) {
          if (nbhd4) {
            if (masks) {
              hipLaunchKernelGGL((kmap_mask_kernel<4, 81, true>), dim3(nb), dim3(kMapBlock), 0,
                                 stream, tv, out_coords, out_spatial_order, n_out, w.offsets, K,
                                 w.keys_a, w.vals_a);
              RHIP_LAUNCH_CHECK();
              sort_pairs_u32(w.sort_tmp, w.sort_bytes, w.keys_a, w.keys_b, w.vals_a, w.vals_b,
                             n_out, mask_key_bits(K), stream);
              jpos = w.vals_b;
            }
            hipLaunchKernelGGL((kmap_query_kernel<4, 81, true>), dim3(nb), dim3(kMapBlock), 0,
                               stream, tv, out_coords, out_spatial_order, jpos, n_out, w.offsets,
                               K, nw, nbr, out_order, w.wave_counts, small, w.offsets, 0,
                               w.partner, 0, w.ticket);
            RHIP_LAUNCH_CHECK();
            return;
          }
        }
        if (masks) {
          if (k27)
            hipLaunchKernelGGL((kmap_mask_kernel<DD, 27>), dim3(nb), dim3(kMapBlock), 0, stream,
                               tv, out_coords, out_spatial_order, n_out, w.offsets, K, w.keys_a,
                               w.vals_a);
          else
            hipLaunchKernelGGL((kmap_mask_kernel<DD>), dim3(nb), dim3(kMapBlock), 0, stream, tv,
                               out_coords, out_spatial_order, n_out, w.offsets, K, w.keys_a,
                               w.vals_a);
          RHIP_LAUNCH_CHECK();
          sort_pairs_u32(w.sort_tmp, w.sort_bytes, w.keys_a, w.keys_b, w.vals_a, w.vals_b,
                         n_out, mask_key_bits(K), stream);
          jpos = w.vals_b;
        }
        if (k27)
          hipLaunchKernelGGL((kmap_query_kernel<DD, 27>), dim3(nb), dim3(kMapBlock), 0, stream,
                             tv, out_coords, out_spatial_order, jpos, n_out, w.offsets, K, nw,
                             nbr, out_order, w.wave_counts, small, w.offsets, 0, w.partner, 0,
                             w.ticket);
        else
          hipLaunchKernelGGL((kmap_query_kernel<DD>), dim3(nb), dim3(kMapBlock), 0, stream, tv,
                             out_coords, out_spatial_order, jpos, n_out, w.offsets, K, nw, nbr,
                             out_order, w.wave_counts, small, w.offsets, 0, w.partner, 0,
                             w.ticket);
        RHIP_LAUNCH_CHECK();
      });
    }
    // with kmap_offsets_host, the offsets also go to the thread's pinned
    // read-back buffer: written by the kernel where the device can address
    // it, else copied
    const size_t hb = sizeof(int64_t) * (K + 1);
    PinnedReadback rb{nullptr, nullptr};
    if (kmap_offsets_host)
      rb = pinned_readback(hb);
    int64_t *host_dev = static_cast<int64_t *>(rb.dev);
    if (n_out > 0) { // the query kernel cleared the ticket
      hipLaunchKernelGGL(kmap_totals_kernel, dim3(K), dim3(1024), 0, stream, w.wave_counts, nw, K,
                         w.wave_base, w.ktotal, w.ticket, kmap_offsets, host_dev);
      RHIP_LAUNCH_CHECK();
    } else {
      hipLaunchKernelGGL(scan_kernel<int32_t>, dim3(K), dim3(1024), 0, stream, w.wave_counts,
                         nw, w.wave_base, w.ktotal);
      RHIP_LAUNCH_CHECK();
      hipLaunchKernelGGL(kmap_offsets_kernel, dim3(1), dim3(1024), 0, stream, w.ktotal, K,
                         kmap_offsets, host_dev);
      RHIP_LAUNCH_CHECK();
    }
    if (kmap_offsets_host) { // else asynchronous: the caller reads kmap_offsets later
      if (!host_dev)
        RHIP_HIP(hipMemcpyAsync(rb.ptr, kmap_offsets, hb, hipMemcpyDeviceToHost, stream));
      RHIP_HIP(hipStreamSynchronize(stream));
      std::memcpy(kmap_offsets_host, rb.ptr, hb);
    }
  });
}

extern "C" int rhip_kmap_fill(const int32_t *nbr, const int32_t *out_order, int64_t n_out,
                              int32_t K, const int32_t *in_spatial_order, int64_t n_in,
                              int32_t flags, void *workspace, size_t workspace_bytes,
                              const int64_t *kmap_offsets, int32_t *in_rows,
                              int32_t *out_rows, int32_t *nbr_t, int32_t *in_order,
                              hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(K >= 1 && K <= 65535, "K must be in [1, 65535]");
    RHIP_CHECK_ARG(workspace != nullptr && kmap_offsets != nullptr,
                   "workspace and kmap_offsets are required");
    RHIP_CHECK_ARG(n_in >= 0 && n_in < INT32_MAX && n_out >= 0 && n_out < INT32_MAX,
                   "bad sizes");
    const bool sym = (flags & RHIP_KMAP_SYMMETRIC) != 0;
    RHIP_CHECK_ARG(!sym || n_in == n_out, "a symmetric map has n_in == n_out");
    Carve cv(workspace, workspace_bytes);
    KmapWs w = carve_kmap(cv, n_in, n_out, K, RHIP_MAX_COLS - 1);
    const int64_t nb = std::max<int64_t>(1, ceil_div(n_out, kMapBlock));
    const int64_t nw = map_waves(n_out);
    const bool want_t = nbr_t != nullptr && n_in > 0;
    RHIP_CHECK_ARG(!want_t || in_order != nullptr, "in_order is required with nbr_t");
    const bool masks = want_t && !sym && K <= kMaskedK && n_in > 1;
    if (masks) {
      hipLaunchKernelGGL(zero_u64_kernel, dim3(ceil_div(2 * n_in, kMapBlock)),
                         dim3(kMapBlock), 0, stream, w.mask_t, 2 * n_in);
      RHIP_LAUNCH_CHECK();
    }
    const bool fuse_t = want_t && sym; // the emit writes nbr_t and in_order
    RHIP_CHECK_ARG((in_rows == nullptr) == (out_rows == nullptr),
                   "in_rows and out_rows go together");
    // nothing to emit: no pair lists, no transposed masks, no symmetric copy
    if (n_out > 0 && (in_rows != nullptr || masks || fuse_t)) {
      RHIP_CHECK_ARG(nbr && out_order, "nbr and out_order are required");
      hipLaunchKernelGGL(kmap_emit_kernel, dim3(nb, K), dim3(kMapBlock), 0, stream, nbr,
                         out_order, n_out, nw, kmap_offsets, w.wave_base, in_rows, out_rows,
                         masks ? w.mask_t : nullptr, fuse_t ? w.partner : nullptr, K,
                         fuse_t ? nbr_t : nullptr, fuse_t ? in_order : nullptr);
      RHIP_LAUNCH_CHECK();
    }
    if (!want_t || sym)
      return;
    const int64_t nbi = ceil_div(n_in, kMapBlock);
    const int32_t *qpos = nullptr;
    if (masks) {
      hipLaunchKernelGGL(in_key_kernel, dim3(nbi), dim3(kMapBlock), 0, stream, w.mask_t,
                         in_spatial_order, n_in, K, w.tkeys_a, w.tvals_a);
      RHIP_LAUNCH_CHECK();
      sort_pairs_u32(w.tsort_tmp, w.tsort_bytes, w.tkeys_a, w.tkeys_b, w.tvals_a, w.tvals_b,
                     n_in, mask_key_bits(K), stream);
      qpos = w.tvals_b;
    }
    hipLaunchKernelGGL(in_order_kernel, dim3(nbi), dim3(kMapBlock), 0, stream, qpos,
                       in_spatial_order, n_in, in_order, w.in_pos);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(fill_i32_kernel, dim3(ceil_div(n_in * K, kMapBlock)),
                       dim3(kMapBlock), 0, stream, nbr_t, n_in * K, -1);
    RHIP_LAUNCH_CHECK();
    if (n_out > 0) {
      hipLaunchKernelGGL(kmap_transpose_kernel, dim3(nb, K), dim3(kMapBlock), 0, stream,
                         nbr, out_order, n_out, w.in_pos, n_in, nbr_t);
      RHIP_LAUNCH_CHECK();
    }
  });
}

extern "C" int rhip_kmap_pairs_workspace_bytes(int64_t n_out, int32_t K, size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(n_out >= 0 && K >= 1, "need n_out >= 0 and K >= 1");
    const int64_t nw = map_waves(n_out);
    Carve cv(nullptr, 0); // the layout rhip_kmap_pairs carves
    cv.take<int32_t>(nw * K);
    cv.take<int64_t>(nw * K);
    cv.take<int64_t>(K);
    *bytes = cv.used + 256;
  });
}

extern "C" int rhip_kmap_pairs(const int32_t *nbr, const int32_t *out_order, int64_t n_out,
                               int32_t K, const int64_t *kmap_offsets, void *workspace,
                               size_t workspace_bytes, int32_t *in_rows, int32_t *out_rows,
                               hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(K >= 1 && K <= 65535, "K must be in [1, 65535]");
    RHIP_CHECK_ARG(n_out >= 0 && n_out < INT32_MAX, "bad n_out");
    RHIP_CHECK_ARG(workspace != nullptr && kmap_offsets != nullptr,
                   "workspace and kmap_offsets are required");
    if (n_out == 0)
      return;
    RHIP_CHECK_ARG(nbr && out_order && in_rows && out_rows,
                   "nbr, out_order, in_rows and out_rows are required");
    const int64_t nw = map_waves(n_out);
    const int64_t nb = std::max<int64_t>(1, ceil_div(n_out, kMapBlock));
    Carve cv(workspace, workspace_bytes);
    int32_t *counts = cv.take<int32_t>(nw * K);
    int64_t *base = cv.take<int64_t>(nw * K);
    int64_t *total = cv.take<int64_t>(K);
    hipLaunchKernelGGL(kmap_wave_count_kernel, dim3(nb, K), dim3(kMapBlock), 0, stream, nbr,
                       n_out, nw, counts);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(scan_kernel<int32_t>, dim3(K), dim3(1024), 0, stream, counts, nw, base,
                       total);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(kmap_emit_kernel, dim3(nb, K), dim3(kMapBlock), 0, stream, nbr, out_order,
                       n_out, nw, kmap_offsets, base, in_rows, out_rows, nullptr, nullptr, K,
                       nullptr, nullptr);
    RHIP_LAUNCH_CHECK();
  });
}

extern "C" int rhip_stencil_partners(const int32_t *offsets_host, int32_t K, int32_t D,
                                     int32_t *partner_host) {
  return guarded([&] {
    RHIP_CHECK_ARG(offsets_host && partner_host, "offsets_host and partner_host are required");
    RHIP_CHECK_ARG(K >= 1 && D >= 1 && D < RHIP_MAX_COLS, "bad K or D");
    for (int a = 0; a < K; ++a) {
      int32_t found = -1;
      for (int b = 0; b < K; ++b) {
        bool same = b != a, neg = true;
        for (int d = 0; d < D; ++d) {
          const int32_t oa = offsets_host[static_cast<size_t>(a) * D + d];
          const int32_t ob = offsets_host[static_cast<size_t>(b) * D + d];
          same = same && oa == ob;
          neg = neg && static_cast<uint32_t>(ob) == 0u - static_cast<uint32_t>(oa);
        }
        if (same)
          throw Error(RHIP_ERR_UNSUPPORTED, "the stencil repeats an offset");
        if (neg)
          found = b;
      }
      if (found < 0)
        throw Error(RHIP_ERR_UNSUPPORTED, "the stencil is not closed under negation");
      partner_host[a] = found;
    }
  });
}
