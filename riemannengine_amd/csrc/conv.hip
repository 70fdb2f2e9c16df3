// Sparse convolution on gfx950 MFMA (fp32 and bf16 inputs, fp32 accumulate).
//
// Reference semantics (RiemannEngine/engine/nn/conv.cpp:47-64):
//   Y = 0; for k: Y.index_add_(0, out_k, X[in_k] @ W[k]);  Y += bias
// with the backward produced by LibTorch autograd:
//   dX = sum_k scatter_add(in_k, dY[out_k] @ W[k]^T),
//   dW[k] = X[in_k]^T @ dY[out_k].
//
// MI355X design:
//  * Forward and dX are one output-stationary implicit GEMM over the dense
//    neighbour table of the kernel map, whose rows come grouped by neighbour
//    mask (so a 16-row group rarely multiplies a missing neighbour). Each
//    stage stages one active offset's weight slice in LDS and gathers the
//    rows straight into MFMA operands. conv_os_lds_kernel (stencils of up to
//    96 offsets) keeps its row groups' neighbour indices in LDS and walks the
//    workgroup's offsets as a bit mask; conv_os_kernel is the general form
//    (larger stencils, fp32 offset splits, padded 16-channel bf16 layers);
//    conv_fr_kernel keeps every offset's weights for its columns resident in
//    LDS (bf16 maps the first does not take whose weights fit). Without an
//    offset split each output row is written once: no atomics, no zero
//    fill; with one, fp32 partial sums are added in split order.
//  * Gathered rows are loaded in quad order (four consecutive lanes read 64
//    contiguous bytes of one row, one L1 access) and moved to the MFMA layout
//    with ds_bpermute.
//  * dW has three kernels, all writing per-workgroup partial tiles that a
//    second kernel adds in a fixed order (deterministic, no atomics):
//    conv_dw_kernel over the per-offset pair lists (split-pair reduction),
//    conv_dw_rows_kernel over the neighbour table for narrow bf16 layers, and
//    the position-stationary conv_dw_pos_kernel / conv_dw_pos_bf16_kernel,
//    which keep the tiles of up to 28 offsets in registers while they stream
//    the output positions.
//  * The reduction order inside an MFMA is a permutation of the reduced axis
//    chosen so that each lane reads 16 contiguous bytes; A and B use the same
//    permutation, so the sum is unchanged.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "rhip_internal.hpp"

namespace rhip {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// LDS transpose read: within a 16-lane group, lane i receives the (i % 4)-th
// 16-bit element at the address of lane 4e + i/4 as element e.
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

__device__ __forceinline__ v4s ds_read_tr16(const void *p) {
  // generic LDS pointer -> LDS address space (the low 32 bits are the offset)
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<lds_v4s *>(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p))));
}

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaskWords = 4; // the MFMA paths handle K <= 128 offsets
constexpr int kWideRG = 2;    // row groups per wave of conv_os_lds_kernel's bf16 128-column tiles

template <typename T> struct Mfma;

// v_mfma_f32_16x16x4_f32: lane l supplies A[l%16][l/16], B[l/16][l%16];
// D[4*(l/16)+e][l%16] lands in element e. A 16-byte lane load covers four
// consecutive channels, consumed by four MFMAs.
template <> struct Mfma<float> {
  static constexpr int kCh = 16; // channels per wave-wide 16-byte load
  using Frag = v4f;
  __device__ static __forceinline__ Frag load(const float *p) {
    return *reinterpret_cast<const v4f *>(p);
  }
  __device__ static __forceinline__ Frag zero() { return v4f{0.f, 0.f, 0.f, 0.f}; }
  // v where keep, else zeros (bitwise, so the load it masks stays unconditional)
  __device__ static __forceinline__ Frag mask(const Frag &v, bool keep) {
    const uint32_t m = keep ? ~0u : 0u;
    uint4 u = __builtin_bit_cast(uint4, v);
    u.x &= m, u.y &= m, u.z &= m, u.w &= m;
    return __builtin_bit_cast(Frag, u);
  }
  __device__ static __forceinline__ void mma(const Frag &a, const Frag &b, v4f &c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], c, 0, 0, 0);
  }
};

// v_mfma_f32_16x16x32_bf16 (gfx950): lane l supplies eight consecutive
// reduction elements of row l%16 (A) / column l%16 (B), group l/16.
template <> struct Mfma<__bf16> {
  static constexpr int kCh = 32;
  using Frag = v8bf;
  __device__ static __forceinline__ Frag load(const __bf16 *p) {
    return *reinterpret_cast<const v8bf *>(p);
  }
  __device__ static __forceinline__ Frag zero() {
    return __builtin_bit_cast(v8bf, uint4{0u, 0u, 0u, 0u});
  }
  __device__ static __forceinline__ void mma(const Frag &a, const Frag &b, v4f &c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // v where keep, else zeros (bitwise, so the load it masks stays unconditional)
  __device__ static __forceinline__ Frag mask(const Frag &v, bool keep) {
    const uint32_t m = keep ? ~0u : 0u;
    uint4 u = __builtin_bit_cast(uint4, v);
    u.x &= m, u.y &= m, u.z &= m, u.w &= m;
    return __builtin_bit_cast(Frag, u);
  }
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(__bf16 v) { return static_cast<float>(v); }
template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float v) {
  return static_cast<__bf16>(v);
}

// Raw buffer loads (stride 0): a load at a byte offset at or past the
// buffer's size returns zero without a memory access, so an absent row needs
// no predicate. Kernels put such offsets at kBufOob, past every buffer they
// make (host code keeps buffers below kBufMaxBytes).
constexpr uint32_t kBufOob = 0x80000000u;
constexpr int64_t kBufMaxBytes = (int64_t(1) << 31) - 256; // offsets stay below kBufOob

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, static_cast<int>(bytes),
                                           0x00020000);
}

// A value the optimiser cannot see through: keeps `load | mask` a bitwise
// OR instead of a select that would become a branch around the load.
__device__ __forceinline__ int32_t opaque(int32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// off where keep is all ones, else kBufOob (keep is 0 or -1)
__device__ __forceinline__ uint32_t pick_off(uint32_t off, int32_t keep) {
  return (off & static_cast<uint32_t>(keep)) | (kBufOob & ~static_cast<uint32_t>(keep));
}

// Gathered rows in quad order. The L1 serves a vector load four lanes at a
// time and looks up one cache line per distinct line among them; in the MFMA
// operand layout (lane (i16, g): row i16, bytes 16g..16g+15 of a 64-byte
// slice) the four lanes of a quad hold four rows, so every lane costs an
// access. Loading lane 4m + c with row m's bytes 16c..16c+15 instead makes
// each quad one 64-byte access (a quarter of the accesses); quad_to_mfma
// then moves lane 4m + c's 16 bytes to lane 16c + m with four ds_bpermute.
__device__ __forceinline__ int quad_src(int lane) { return (4 * (lane & 15) + (lane >> 4)) * 4; }

__device__ __forceinline__ v4u quad_to_mfma(const v4u &v, int src) {
  v4u o;
#pragma unroll
  for (int d = 0; d < 4; ++d)
    o[d] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int32_t>(v[d])));
  return o;
}


// ------------------------------------------------ output-stationary GEMM
//
// y[order[j]][col] = sum_k sum_c x[nbr[k][j]][c] * wt[k][col][c] (+ bias[col])
// wt is [K][ncols][credw] (reduction axis contiguous; credw >= cred, the
// rows past cred zero: a bf16 reduction of 16 channels is padded to the
// 32 of one MFMA, PADC, and lanes whose channels lie past cred read
// nothing and contribute zeros). A workgroup owns
// 4 * RG * 16 output rows and NT columns; RG: 16-row groups per wave; CSUB:
// 16-byte lane loads per staged channel chunk (chunk = CSUB * kCh channels).
// A stage is one (active offset, channel chunk); G stages go at once: their
// neighbour indices, then their weight chunks (to G LDS slots) and gathered
// rows (to registers) are all in flight together, so a group costs about
// two memory latencies and two barriers however many stages it holds.
template <typename T, int NT, int RG, int CSUB, int G, int WAVES = 1, bool COAL = true,
          bool PADC = false, int CW = 0>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(WAVES))) void conv_os_kernel(
    const T *__restrict__ x, int cred, const T *__restrict__ wt, int credw, int ncols,
    const float *__restrict__ bias, const int32_t *__restrict__ nbr,
    int64_t n_rows, int K, const int32_t *__restrict__ order,
    T *__restrict__ y, float *__restrict__ partial) {
  if constexpr (CW > 0) { // the host guarantees cred == credw == CW
    cred = CW;
    credw = CW;
  }
  using M = Mfma<T>;
  using Frag = typename M::Frag;
  constexpr int CH = M::kCh;
  constexpr int EPL = CH / 4;            // elements per lane per load
  constexpr int VE = 16 / sizeof(T);     // elements per 16 bytes
  constexpr int CCH = CSUB * CH;         // channels per staged chunk
  constexpr int LDW = CCH + VE;          // LDS row stride (elements)
  constexpr int ROWS = kWaves * RG * 16; // output rows per workgroup
  constexpr int NB = NT / 16;
  constexpr int NV = NT * (CCH / VE);    // 16-byte pieces per staged chunk
  constexpr int NPT = (NV + kThreads - 1) / kThreads;

  __shared__ __align__(16) T sB[G][NT * LDW];
  __shared__ uint32_t smask[kWaves * RG][kMaskWords];
  __shared__ int32_t slist[32 * kMaskWords];
  __shared__ int32_t scount;

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const int64_t tile = xcd_tile(blockIdx.x);
  const int64_t tile0 = tile * ROWS;
  if (tile0 >= n_rows)
    return; // padding workgroup (uniform)
  const int col0 = blockIdx.y * NT;

  // Offsets with any neighbour in each 16-row group: lanes of group g test
  // offset k0+g for the 16 rows; one ballot covers four offsets. For
  // K <= 4*kRegQ the bf16 kernels keep the indices in registers (lane
  // (i16, g) holds row i16's under offsets g, g+4, ...): their loads issue
  // back to back, and a stage later takes its rows' indices from them with
  // ds_bpermute instead of a second global load. Measured on MI355X, config
  // 2 forward: bf16 115-123 us against 122-131; the fp32 kernel, whose
  // 8-wave budget has no room for the 8 registers, spills and loses (446
  // against 351 us), so it keeps the global loads.
  constexpr int kRegQ = 8;
  constexpr bool kRegIdx = !std::is_same<T, float>::value;
  const bool kreg = kRegIdx && K <= 4 * kRegQ;
  int32_t kidx[RG][kRegQ];
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int64_t pos = tile0 + (wv * RG + r) * 16 + i16;
    uint32_t words[kMaskWords] = {0u, 0u, 0u, 0u};
    auto note = [&](int k0, int32_t v) {
      const uint64_t bal = __ballot(v >= 0);
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        if ((bal >> (16 * gg)) & 0xffffull) {
          const int kk = k0 + gg;
          words[kk >> 5] |= 1u << (kk & 31);
        }
      }
    };
    if (kreg) {
      const bool in = pos < n_rows;
      const int64_t pc = in ? pos : n_rows - 1;
#pragma unroll
      for (int q = 0; q < kRegQ; ++q) {
        const int k = 4 * q + g;
        const bool ok = in && k < K;
        // a mask, not a select of the load: the loads issue back to back
        kidx[r][q] = nbr[(k < K ? k : K - 1) * n_rows + pc] | (ok ? 0 : -1);
      }
#pragma unroll
      for (int q = 0; q < kRegQ; ++q)
        if (4 * q < K)
          note(4 * q, kidx[r][q]);
    } else {
      for (int k0 = 0; k0 < K; k0 += 4) {
        const int k = k0 + g;
        note(k0, (k < K && pos < n_rows) ? nbr[k * n_rows + pos] : -1);
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int q = 0; q < kMaskWords; ++q)
        smask[wv * RG + r][q] = words[q];
    }
  }
  __syncthreads();
  // The workgroup's active offsets, in ascending order.
  if (threadIdx.x == 0) {
    int c = 0;
    for (int q = 0; q < kMaskWords; ++q) {
      uint32_t m = 0;
      for (int i = 0; i < kWaves * RG; ++i)
        m |= smask[i][q];
      while (m) {
        slist[c++] = q * 32 + __builtin_ctz(m);
        m &= m - 1;
      }
    }
    scount = c;
  }
  __syncthreads();
  const int nch = credw / CCH;
  // stages: (active offset, channel chunk); split z of gridDim.z takes an
  // equal share of them and writes fp32 partial sums
  const int S = scount * nch;
  const int s_begin = static_cast<int>(static_cast<int64_t>(S) * blockIdx.z / gridDim.z);
  const int s_end = static_cast<int>(static_cast<int64_t>(S) * (blockIdx.z + 1) / gridDim.z);

  v4f acc[RG][NB];
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      acc[r][nb] = v4f{0.f, 0.f, 0.f, 0.f};

  // the row this lane loads: row i16 in the MFMA layout, row lane / 4 when
  // the rows are gathered in quad order (then moved with quad_to_mfma)
  const int rsel = COAL ? (lane >> 2) : i16;
  const int tsrc = quad_src(lane);
  const int64_t pos0 = tile0 + wv * RG * 16 + rsel;
  for (int s0 = s_begin; s0 < s_end; s0 += G) {
    // The loads of a group are branch-free so that they issue back to back:
    // a stage past the end repeats the last one (its results are unused),
    // indices are read at clamped positions and masked, and a missing
    // neighbour reads row 0 (an active stage has at least one input row)
    // and is replaced by zeros.
    int kj[G], ccj[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int sj = min(s0 + j, s_end - 1);
      kj[j] = slist[sj / nch];
      ccj[j] = (sj % nch) * CCH;
    }
    int32_t idx[G][RG];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        const int64_t pos = pos0 + r * 16;
        int32_t v;
        if (kreg) { // row i16's index under kj from lane (kj % 4, i16)
          const int q = kj[j] >> 2;
          int32_t held = kidx[r][0];
#pragma unroll
          for (int qq = 1; qq < kRegQ; ++qq)
            held = qq == q ? kidx[r][qq] : held;
          v = __builtin_amdgcn_ds_bpermute(((kj[j] & 3) * 16 + rsel) * 4, held);
        } else {
          v = nbr[kj[j] * n_rows + (pos < n_rows ? pos : n_rows - 1)];
        }
        const bool act = s0 + j < s_end && pos < n_rows &&
                         ((smask[wv * RG + r][kj[j] >> 5] >> (kj[j] & 31)) & 1u);
        idx[j][r] = v | (act ? 0 : -1); // a mask, not a select of the load
      }
    uint4 wreg[G][NPT];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        const int li = min(static_cast<int>(threadIdx.x) + i * kThreads, NV - 1);
        wreg[j][i] = *reinterpret_cast<const uint4 *>(
            wt + (static_cast<int64_t>(kj[j]) * ncols + col0 + li / (CCH / VE)) * credw +
            ccj[j] + (li % (CCH / VE)) * VE);
      }
    Frag a[G][RG][CSUB];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int r = 0; r < RG; ++r)
#pragma unroll
        for (int sub = 0; sub < CSUB; ++sub) {
          const int ch = ccj[j] + sub * CH + (COAL ? (lane & 3) : g) * EPL;
          const bool cok = !PADC || ch < cred; // a padded lane reads channel 0, zeroed
          const Frag v = M::load(x + static_cast<int64_t>(idx[j][r] < 0 ? 0 : idx[j][r]) * cred +
                                 (cok ? ch : 0));
          a[j][r][sub] = M::mask(v, idx[j][r] >= 0 && cok);
        }
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        const int li = threadIdx.x + i * kThreads;
        if (NV % kThreads == 0 || li < NV)
          *reinterpret_cast<uint4 *>(&sB[j][(li / (CCH / VE)) * LDW + (li % (CCH / VE)) * VE]) =
              wreg[j][i];
      }
    __syncthreads(); // the group's weights are staged
#pragma unroll
    for (int j = 0; j < G; ++j) {
      bool wave_act = false;
#pragma unroll
      for (int r = 0; r < RG; ++r)
        wave_act |= __ballot(idx[j][r] >= 0) != 0;
      if (wave_act) { // uniform; false for j >= ns
#pragma unroll
        for (int sub = 0; sub < CSUB; ++sub) {
          Frag at[RG];
#pragma unroll
          for (int r = 0; r < RG; ++r)
            at[r] = COAL ? __builtin_bit_cast(
                               Frag, quad_to_mfma(__builtin_bit_cast(v4u, a[j][r][sub]), tsrc))
                         : a[j][r][sub];
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const Frag b = *reinterpret_cast<const Frag *>(
                &sB[j][(nb * 16 + i16) * LDW + sub * CH + g * EPL]);
#pragma unroll
            for (int r = 0; r < RG; ++r)
              M::mma(at[r], b, acc[r][nb]);
          }
        }
      }
    }
    __syncthreads(); // every wave is done reading the group's weights
  }

  if (partial) { // [split][position][column], reduced by conv_os_reduce_kernel
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t pos = tile0 + (wv * RG + r) * 16 + 4 * g + e;
        if (pos < n_rows) {
          float *dst = partial + (blockIdx.z * n_rows + pos) * ncols + col0 + i16;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            dst[nb * 16] = acc[r][nb][e];
        }
      }
    return;
  }
#pragma unroll
  for (int r = 0; r < RG; ++r) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t pos = tile0 + (wv * RG + r) * 16 + 4 * g + e;
      if (pos < n_rows) {
        const int64_t o = order ? order[pos] : pos;
        T *dst = y + o * ncols + col0 + i16;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          float v = acc[r][nb][e];
          if (bias)
            v += bias[col0 + nb * 16 + i16];
          dst[nb * 16] = from_f32<T>(v);
        }
      }
    }
  }
}

// conv_os_kernel's fast form for stencils of at most 4 * KQ offsets (KQ = 8:
// 32 offsets, one mask word; KQ = 24: 96, three words), reduction widths of
// 1, 2 or 4 channel chunks (CW = cred = credw, a compile-time
// constant), no split of the offset axis and inputs addressable by 32-bit
// buffer offsets. It computes the same sums in the same order; what differs
// is the control around them:
//  * each wave stores its row groups' neighbour indices (offsets 4q + g in
//    lane (i16, g) of slot q) in LDS once, and a stage reads its row's index
//    with one ds_read instead of a register select chain and a ds_bpermute;
//  * the workgroup's offsets are a wave-uniform bit mask (OR of the row
//    groups' masks, one barrier) walked with ctz: no serial offset list
//    (config 4's 81 offsets in three words: forward 308 -> 300 us against
//    conv_os_kernel);
//  * a missing neighbour is an out-of-range buffer offset, which loads
//    zeros, so nothing is masked after the loads.
// Measured on MI355X, config 2 bf16 forward (quad-order gathers both): 76 us
// against 108 for conv_os_kernel with runtime widths. SPLIT: gridDim.z
// workgroups share a tile's (offset, chunk) stages and write fp32 partial
// sums (config 5 step 5.87 -> 5.73 ms against conv_os_kernel's split).
// REGK: the indices stay in registers instead, one vector of slots per row
// group; a stage takes its slot with one uniform indexed register move and
// moves the row's index to the lane with a ds_bpermute. LDS then holds only
// the staged weights, which is what limits occupancy where a stencil has
// many slots (config 4's 81 offsets: 48 KB of indices per workgroup).
// WTR (bf16): the weights are W itself, [K][CW][ncols] (the forward needs no
// transposed copy): a stage's chunk goes to LDS as CCH rows of NT columns
// and each B operand is two transposed reads (ds_read_b64_tr_b16) that give
// lane (n, g) reduction rows 8g..8g+7 of column n, the order of the A
// operand's channels.
template <typename T, int NT, int RG, int CSUB, int G, int WAVES, int CW, int KQ, bool SPLIT,
          bool REGK = false, bool WTR = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(WAVES))) void
conv_os_lds_kernel(const T *__restrict__ x, int64_t n_x, const T *__restrict__ wt,
                   const int32_t *__restrict__ wperm, int ncols,
                   const float *__restrict__ bias, const int32_t *__restrict__ nbr,
                   int64_t n_rows, int K, const int32_t *__restrict__ order, T *__restrict__ y,
                   float *__restrict__ partial) {
  using M = Mfma<T>;
  using Frag = typename M::Frag;
  constexpr int CH = M::kCh;
  constexpr int EPL = CH / 4;            // elements per lane per load
  constexpr int VE = 16 / sizeof(T);     // elements per 16 bytes
  constexpr int CCH = CSUB * CH;         // channels per staged chunk
  constexpr int NCH = CW / CCH;          // chunks per offset
  static_assert(CW % CCH == 0, "reduction width must be whole chunks");
  // LDS row stride (elements): 16 bytes of padding, 32 for bf16 64-column
  // tiles of 64-channel chunks (config 2 bf16 forward 79.7 -> 77.7 us, the
  // same occupancy; 48 or 80 bytes leave room for fewer workgroups)
  constexpr int LDW = CCH + ((!std::is_same<T, float>::value && NT == 64 && CCH == 64) ? 2 * VE : VE);
  constexpr int ROWS = kWaves * RG * 16; // output rows per workgroup
  constexpr int NB = NT / 16;
  constexpr int NV = NT * (CCH / VE);    // 16-byte pieces per staged chunk
  constexpr int NPT = (NV + kThreads - 1) / kThreads;
  // KQ: index slots of four offsets (K <= 4 KQ); MW: 32-bit mask words
  static_assert(KQ % 8 == 0, "index slots come in groups of eight");
  constexpr int MW = KQ / 8;

  static_assert(!WTR || !std::is_same<T, float>::value, "untransposed weights: bf16 only");
  constexpr int LDT = NT + 8; // WTR: LDS row stride (elements) of a chunk's CCH rows
  __shared__ __align__(16) T sB[G][WTR ? CCH * LDT : NT * LDW];
  __shared__ int32_t sK[REGK ? 1 : kWaves][REGK ? 1 : RG][REGK ? 1 : KQ][kWave];
  static_assert(!REGK || KQ <= 32, "register-held slots fit one vector");
  constexpr int KV = KQ <= 8 ? 8 : (KQ <= 16 ? 16 : 32);
  typedef int32_t vki __attribute__((ext_vector_type(KV)));
  vki kreg[RG]; // REGK: lane (i16, g) of slot q holds offset 4q + g of row i16
  __shared__ uint32_t smask[kWaves * RG][MW];

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const int64_t tile0 = xcd_tile(blockIdx.x) * ROWS;
  if (tile0 >= n_rows)
    return; // padding workgroup (uniform)
  const int col0 = blockIdx.y * NT;

  // Neighbour indices of the wave's row groups to LDS or registers (absent
  // or past the end: -1) and the offsets with any neighbour in each group.
  uint32_t wmask[MW] = {};
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int64_t pos = tile0 + (wv * RG + r) * 16 + i16;
    const bool in = pos < n_rows;
    const int64_t pc = in ? pos : n_rows - 1;
#pragma unroll
    for (int mw = 0; mw < MW; ++mw) { // eight slots (32 offsets) at a time
      int32_t v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int k = 32 * mw + 4 * q + g;
        // a mask, not a select of the load: the loads issue back to back
        v[q] = nbr[(k < K ? k : K - 1) * n_rows + pc] | ((in && k < K) ? 0 : -1);
      }
      uint32_t w = 0;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        if constexpr (REGK)
          kreg[r][8 * mw + q] = v[q];
        else
          sK[wv][r][8 * mw + q][lane] = v[q];
        const uint64_t bal = __ballot(v[q] >= 0);
#pragma unroll
        for (int gg = 0; gg < 4; ++gg)
          w |= (((bal >> (16 * gg)) & 0xffffull) != 0 ? 1u : 0u) << (4 * q + gg);
      }
      w = __builtin_amdgcn_readfirstlane(w);
      wmask[mw] |= w;
      if (lane == 0)
        smask[wv * RG + r][mw] = w;
    }
  }
  __syncthreads();
  uint32_t m[MW] = {}; // the workgroup's offsets, walked in ascending order
#pragma unroll
  for (int mw = 0; mw < MW; ++mw) {
#pragma unroll
    for (int i = 0; i < kWaves * RG; ++i)
      m[mw] |= smask[i][mw];
    m[mw] = __builtin_amdgcn_readfirstlane(m[mw]);
  }
  auto lowest = [&]() { // the smallest offset left (some word is non-zero)
    int k = 0;
#pragma unroll
    for (int mw = MW - 1; mw >= 0; --mw)
      if (m[mw])
        k = 32 * mw + __builtin_ctz(m[mw]);
    return k;
  };

  v4f acc[RG][NB];
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      acc[r][nb] = v4f{0.f, 0.f, 0.f, 0.f};

  // the row this lane loads: row lane / 4 in quad order (moved to the MFMA
  // layout with quad_to_mfma)
  const int rsel = lane >> 2;
  const int tsrc = quad_src(lane);
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, n_x * CW * static_cast<int64_t>(sizeof(T)));
  const uint32_t lane_byte = static_cast<uint32_t>((lane & 3) * EPL * sizeof(T));
  int cc = 0; // channel chunk of the next stage
  auto advance = [&](int k) {
    if (++cc == NCH) {
      cc = 0;
      m[k >> 5] &= m[k >> 5] - 1; // k is that word's lowest bit
    }
  };
  // split z of gridDim.z takes an equal share of the (offset, chunk) stages
  // and writes fp32 partial sums (reduced by conv_os_reduce_kernel)
  int left = 0;
  if constexpr (SPLIT) {
#pragma unroll
    for (int mw = 0; mw < MW; ++mw)
      left += __builtin_popcount(m[mw]) * NCH;
    const int s_begin = static_cast<int>(static_cast<int64_t>(left) * blockIdx.z / gridDim.z);
    const int s_end = static_cast<int>(static_cast<int64_t>(left) * (blockIdx.z + 1) / gridDim.z);
    for (int i = 0; i < s_begin; ++i)
      advance(lowest());
    left = s_end - s_begin;
  }
  auto more = [&]() {
    if constexpr (SPLIT)
      return left > 0;
    uint32_t o = 0;
#pragma unroll
    for (int mw = 0; mw < MW; ++mw)
      o |= m[mw];
    return o != 0;
  };
  while (more()) {
    // G stages: (offset, chunk) in order; past the last one a stage repeats
    // the previous one with every load out of range and no multiply
    int kj[G], ccj[G];
    bool live[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      live[j] = more();
      kj[j] = live[j] ? lowest() : kj[j > 0 ? j - 1 : 0];
      ccj[j] = cc;
      if (live[j]) {
        advance(kj[j]);
        if constexpr (SPLIT)
          --left;
      }
    }
    uint32_t off[G][RG];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        int32_t id;
        if constexpr (REGK) // kj is uniform: one indexed move, then the row's lane
          id = __builtin_amdgcn_ds_bpermute(((kj[j] & 3) * 16 + rsel) * 4, kreg[r][kj[j] >> 2]);
        else
          id = sK[wv][r][kj[j] >> 2][(kj[j] & 3) * 16 + rsel];
        const int32_t keep = live[j] ? ~(id >> 31) : 0;
        off[j][r] = pick_off(static_cast<uint32_t>(id) * static_cast<uint32_t>(CW * sizeof(T)) +
                                 static_cast<uint32_t>(ccj[j] * CCH * sizeof(T)) + lane_byte,
                             keep);
      }
    uint4 wreg[G][NPT];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      // table row kj multiplies weight slice wperm[kj] (uniform) when given
      const int kw = wperm ? wperm[kj[j]] : kj[j];
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        const int li = min(static_cast<int>(threadIdx.x) + i * kThreads, NV - 1);
        if constexpr (WTR) // row li / (NT / VE) of the chunk, 16-byte piece li % (NT / VE)
          wreg[j][i] = *reinterpret_cast<const uint4 *>(
              wt + (static_cast<int64_t>(kw) * CW + ccj[j] * CCH + li / (NT / VE)) * ncols +
              col0 + (li % (NT / VE)) * VE);
        else
          wreg[j][i] = *reinterpret_cast<const uint4 *>(
              wt + (static_cast<int64_t>(kw) * ncols + col0 + li / (CCH / VE)) * CW +
              ccj[j] * CCH + (li % (CCH / VE)) * VE);
      }
    }
    v4u a[G][RG][CSUB];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int r = 0; r < RG; ++r)
#pragma unroll
        for (int sub = 0; sub < CSUB; ++sub)
          a[j][r][sub] = __builtin_bit_cast(
              v4u, __builtin_amdgcn_raw_buffer_load_b128(
                       rx, off[j][r] + static_cast<uint32_t>(sub * CH * sizeof(T)), 0, 0));
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        const int li = threadIdx.x + i * kThreads;
        if (NV % kThreads == 0 || li < NV) {
          if constexpr (WTR)
            *reinterpret_cast<uint4 *>(&sB[j][(li / (NT / VE)) * LDT + (li % (NT / VE)) * VE]) =
                wreg[j][i];
          else
            *reinterpret_cast<uint4 *>(&sB[j][(li / (CCH / VE)) * LDW + (li % (CCH / VE)) * VE]) =
                wreg[j][i];
        }
      }
    __syncthreads(); // the group's weights are staged
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (live[j] && ((wmask[kj[j] >> 5] >> (kj[j] & 31)) & 1u)) { // uniform
#pragma unroll
        for (int sub = 0; sub < CSUB; ++sub) {
          Frag at[RG];
#pragma unroll
          for (int r = 0; r < RG; ++r)
            at[r] = __builtin_bit_cast(Frag, quad_to_mfma(a[j][r][sub], tsrc));
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            Frag b;
            if constexpr (WTR) {
              const T *base = &sB[j][(sub * CH + 8 * g + i16 / 4) * LDT + nb * 16 + 4 * (i16 % 4)];
              const v4s lo = ds_read_tr16(base), hi = ds_read_tr16(base + 4 * LDT);
              b = __builtin_bit_cast(Frag, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            } else {
              b = *reinterpret_cast<const Frag *>(&sB[j][(nb * 16 + i16) * LDW + sub * CH + g * EPL]);
            }
#pragma unroll
            for (int r = 0; r < RG; ++r)
              M::mma(at[r], b, acc[r][nb]);
          }
        }
      }
    }
    __syncthreads(); // every wave is done reading the group's weights
  }

  if constexpr (SPLIT) { // [split][position][column]
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t pos = tile0 + (wv * RG + r) * 16 + 4 * g + e;
        if (pos < n_rows) {
          float *dst = partial + (blockIdx.z * n_rows + pos) * ncols + col0 + i16;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            dst[nb * 16] = acc[r][nb][e];
        }
      }
    return;
  }
#pragma unroll
  for (int r = 0; r < RG; ++r) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t pos = tile0 + (wv * RG + r) * 16 + 4 * g + e;
      if (pos < n_rows) {
        const int64_t o = order ? order[pos] : pos;
        T *dst = y + o * ncols + col0 + i16;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          float v = acc[r][nb][e];
          if (bias)
            v += bias[col0 + nb * 16 + i16];
          // streaming stores: the output is read by a later pass, and keeping
          // it out of the L2 and the MALL leaves room for the rows the next
          // passes gather (config 2 step: bf16 dX 81.5 -> 74.6 us, dW 140 ->
          // 131, fp32 forward 339 -> 334, dX 324 -> 319)
          __builtin_nontemporal_store(from_f32<T>(v), &dst[nb * 16]);
        }
      }
    }
  }
}

// Any-shape fallback of conv_os_kernel: one lane per output element.
template <typename T>
__global__ __launch_bounds__(kThreads) void conv_os_generic_kernel(
    const T *__restrict__ x, int cred, const T *__restrict__ wt, int credw, int ncols,
    const float *__restrict__ bias, const int32_t *__restrict__ nbr,
    int64_t n_rows, int K, const int32_t *__restrict__ order,
    T *__restrict__ y) {
  const int64_t t = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  if (t >= n_rows * ncols)
    return;
  const int64_t pos = t / ncols;
  const int col = static_cast<int>(t % ncols);
  float acc = 0.f;
  for (int k = 0; k < K; ++k) {
    const int32_t s = nbr[k * n_rows + pos];
    if (s < 0)
      continue;
    const T *xr = x + static_cast<int64_t>(s) * cred;
    const T *wr = wt + (static_cast<int64_t>(k) * ncols + col) * credw;
    for (int c = 0; c < cred; ++c)
      acc += to_f32(xr[c]) * to_f32(wr[c]);
  }
  if (bias)
    acc += bias[col];
  const int64_t o = order ? order[pos] : pos;
  y[o * ncols + col] = from_f32<T>(acc);
}

// ------------------------------------ resident-weight gather GEMM (bf16)
//
// The product of conv_os_kernel for bf16 maps whose weights for NT output
// columns of every offset fit in LDS (4*KQ offset slots of NT rows of
// cred + 8 elements): a workgroup copies them in once, and after that one
// barrier its waves never wait for each other. A wave takes units of 32
// output rows (two 16-row MFMA groups, which share every B-fragment read)
// and walks the offsets with a neighbour among them, with the gathered rows
// of D offsets in flight:
//  * a unit's neighbour indices arrive one unit ahead, lane (i16, g) holding
//    row i16 of group r under offsets g, g + 4, ...; a stage takes its rows'
//    indices from the owning lanes with ds_bpermute;
//  * rows are raw buffer loads: a missing neighbour, or a stage past the
//    unit's last offset, reads past the buffer and gets zeros without a
//    memory access, so the D slots always hold D stages' loads and the waits
//    for them are static;
//  * a group without a neighbour under an offset skips its MFMAs.
// The grid is one workgroup per CU. XCD x takes chunks x, x + 8, ... of
// consecutive units and runs every column slice of a chunk at the same time,
// so the slices after the first find the chunk's rows in its L2.
template <int NT, int KS, int KQ, int D, int WAVES, bool COAL = true>
__global__ __launch_bounds__(WAVES *kWave) void conv_fr_kernel(
    const __bf16 *__restrict__ x, int64_t n_x, const __bf16 *__restrict__ wt, int ncols,
    const float *__restrict__ bias, const int32_t *__restrict__ nbr, int64_t n_rows, int K,
    const int32_t *__restrict__ order, __bf16 *__restrict__ y) {
  constexpr int C = 32 * KS; // reduction width
  constexpr int LDW = C + 8; // LDS row stride (elements)
  constexpr int NB = NT / 16;
  constexpr int RG = 2; // 16-row groups per unit
  constexpr int KL = KQ == 2 ? 8 : 28; // offset slots in LDS
  __shared__ __align__(16) __bf16 sW[KL * NT * LDW];

  const int slices = ncols / NT;
  const int xcd = static_cast<int>(blockIdx.x % kXcds);
  const int m = static_cast<int>(blockIdx.x / kXcds);
  const int slots = static_cast<int>(gridDim.x / kXcds) / slices;
  const int slice = m % slices, slot = m / slices;
  if (slot >= slots)
    return; // a workgroup the slices do not divide (uniform)
  const int col0 = slice * NT;

  { // this slice's weights, [k][n][c] with padded rows
    constexpr int VPR = C / 8;
    const int total = K * NT * VPR;
    for (int i = threadIdx.x; i < total; i += WAVES * kWave) {
      const int row = i / VPR, v = i - row * VPR;
      const int k = row / NT, n = row - k * NT;
      *reinterpret_cast<v4u *>(&sW[row * LDW + 8 * v]) = *reinterpret_cast<const v4u *>(
          wt + (static_cast<int64_t>(k) * ncols + col0 + n) * C + 8 * v);
    }
  }
  __syncthreads();

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int i16 = lane & 15, g = lane >> 4;
  const int64_t units = (n_rows + 31) / 32;
  const int64_t chunk = static_cast<int64_t>(slots) * WAVES;
  const int64_t ustep = kXcds * chunk;
  int64_t u = xcd * chunk + slot * WAVES + wv;

  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, n_x * C * 2);
  const __amdgpu_buffer_rsrc_t rn = buf_rsrc(nbr, static_cast<int64_t>(K) * n_rows * 4);
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(order, order ? n_rows * 4 : 0);
  const int tsrc = quad_src(lane);
  float bv[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
    bv[nb] = bias ? bias[col0 + nb * 16 + i16] : 0.f;

  // an index vector, read with a wave-uniform subscript (v_movrels, no
  // memory): an array would be demoted to scratch by the dynamic subscript
  typedef int32_t IdxVec __attribute__((ext_vector_type(KQ)));
  struct Idx {
    IdxVec k[RG]; // row 16r + i16 under offset 4q + g (-1 = none)
    int32_t orow; // output row of position 32u + lane % 32 (-1 past the end)
  };
  auto load_idx = [&](int64_t uu, Idx &I) {
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const int64_t pos = uu * 32 + r * 16 + i16;
      const int32_t in = opaque(static_cast<int32_t>((pos - n_rows) >> 63));
#pragma unroll
      for (int q = 0; q < KQ; ++q) {
        const int k = 4 * q + g;
        const int32_t keep = in & opaque(k < K ? -1 : 0);
        I.k[r][q] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
                        rn, pick_off(static_cast<uint32_t>((k * n_rows + pos) * 4), keep), 0,
                        0)) |
                    ~keep;
      }
    }
    const int64_t pos = uu * 32 + (lane & 31);
    const int32_t in = opaque(static_cast<int32_t>((pos - n_rows) >> 63));
    if (order)
      I.orow = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
                   ro, pick_off(static_cast<uint32_t>(pos * 4), in), 0, 0)) |
               ~in;
    else
      I.orow = static_cast<int32_t>(pos) | ~in;
  };

  v4f acc[RG][NB];
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      acc[r][nb] = v4f{0.f, 0.f, 0.f, 0.f};

  struct Rows {
    v4u a[RG][KS];
  };
  auto run_unit = [&](const Idx &I) {
    // offsets with a neighbour in each group (wave-uniform)
    uint32_t mr[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      uint32_t w = 0;
#pragma unroll
      for (int q = 0; q < KQ; ++q) {
        const uint64_t bal = __ballot(I.k[r][q] >= 0);
#pragma unroll
        for (int gg = 0; gg < 4; ++gg)
          w |= (((bal >> (16 * gg)) & 0xffffull) != 0 ? 1u : 0u) << (4 * q + gg);
      }
      mr[r] = __builtin_amdgcn_readfirstlane(w);
    }
    uint32_t mi = 0;
#pragma unroll
    for (int r = 0; r < RG; ++r)
      mi |= mr[r];
    uint32_t mc = mi;
    const int na = __builtin_popcount(mi);

    // stage = the next offset of mi (none left: zeros without memory access)
    auto issue = [&](Rows &R) {
      const bool real = mi != 0;
      const int k = real ? __builtin_ctz(mi) : 0;
      mi &= mi - 1;
      const int q = k >> 2;
      const int src = ((k & 3) * 16 + (COAL ? (lane >> 2) : i16)) * 4;
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        const int32_t idx = __builtin_amdgcn_ds_bpermute(src, I.k[r][q]);
        const int32_t keep = opaque(real ? ~(idx >> 31) : 0);
        const uint32_t base = pick_off(
            static_cast<uint32_t>(idx * (2 * C) + 16 * (COAL ? (lane & 3) : g)), keep);
#pragma unroll
        for (int s = 0; s < KS; ++s)
          R.a[r][s] = __builtin_amdgcn_raw_buffer_load_b128(rx, base + 64 * s, 0, 0);
      }
    };
    auto consume = [&](const Rows &R) {
      const int k = __builtin_ctz(mc);
      mc &= mc - 1;
      v8bf b[KS][NB];
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          b[s][nb] = *reinterpret_cast<const v8bf *>(
              &sW[(k * NT + nb * 16 + i16) * LDW + 32 * s + 8 * g]);
#pragma unroll
      for (int r = 0; r < RG; ++r)
        if ((mr[r] >> k) & 1u) { // wave-uniform
#pragma unroll
          for (int s = 0; s < KS; ++s) {
            const v8bf a = __builtin_bit_cast(v8bf, COAL ? quad_to_mfma(R.a[r][s], tsrc) : R.a[r][s]);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              acc[r][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[s][nb], acc[r][nb], 0, 0, 0);
          }
        }
    };

    Rows R[D];
#pragma unroll
    for (int j = 0; j < D; ++j)
      issue(R[j]);
    for (int t = 0; t < na; t += D) {
#pragma unroll
      for (int j = 0; j < D; ++j) {
        if (t + j < na)
          consume(R[j]);
        issue(R[j]);
      }
    }

    // lane (i16, g) holds row 16r + 4g + e, column 16nb + i16
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int32_t o = __builtin_amdgcn_ds_bpermute((r * 16 + 4 * g + e) * 4, I.orow);
        if (o >= 0) {
          __bf16 *dst = y + static_cast<int64_t>(o) * ncols + col0 + i16;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            dst[nb * 16] = static_cast<__bf16>(acc[r][nb][e] + bv[nb]);
        }
      }
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        acc[r][nb] = v4f{0.f, 0.f, 0.f, 0.f};
  };

  // two index slots in alternation: no in-flight load is ever copied
  Idx IA, IB;
  load_idx(u, IA);
  while (u < units) {
    load_idx(u + ustep, IB);
    run_unit(IA);
    u += ustep;
    if (u >= units)
      break;
    load_idx(u + ustep, IA);
    run_unit(IB);
    u += ustep;
  }
}

// y[order[pos]][c] = sum over splits z (in order) of partial[z][pos][c]
// (+ bias[c]); four columns per lane.
template <typename T>
__global__ __launch_bounds__(kThreads) void conv_os_reduce_kernel(
    const float *__restrict__ partial, int splits, int64_t n_rows, int ncols,
    const float *__restrict__ bias, const int32_t *__restrict__ order, T *__restrict__ y) {
  const int64_t t = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  const int q = ncols / 4;
  const int64_t pos = t / q;
  if (pos >= n_rows)
    return;
  const int c = static_cast<int>(t - pos * q) * 4;
  float4 a = *reinterpret_cast<const float4 *>(partial + pos * ncols + c);
  for (int z = 1; z < splits; ++z) {
    const float4 b =
        *reinterpret_cast<const float4 *>(partial + (z * n_rows + pos) * ncols + c);
    a.x += b.x, a.y += b.y, a.z += b.z, a.w += b.w;
  }
  if (bias)
    a.x += bias[c], a.y += bias[c + 1], a.z += bias[c + 2], a.w += bias[c + 3];
  T *dst = y + (order ? order[pos] : pos) * ncols + c;
  dst[0] = from_f32<T>(a.x);
  dst[1] = from_f32<T>(a.y);
  dst[2] = from_f32<T>(a.z);
  dst[3] = from_f32<T>(a.w);
}

// wt[k][n][c] = w[k][c][n] (weights [K, cin, cout] -> [K, cout, credw]),
// zero for cin <= c < credw.
template <typename T>
__global__ __launch_bounds__(kThreads) void transpose_w_kernel(const T *__restrict__ w, int K,
                                                               int cin, int cout, int credw,
                                                               T *__restrict__ wt) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  const int64_t per = static_cast<int64_t>(cout) * credw;
  if (i >= K * per)
    return;
  const int64_t k = i / per, rem = i % per;
  const int n = static_cast<int>(rem / credw), c = static_cast<int>(rem % credw);
  wt[i] = c < cin ? w[(k * cin + c) * cout + n] : from_f32<T>(0.f);
}

// dst[r][c] = src[r'][c] for c < cols, zero up to credw (rows of cols ->
// credw), where r' = r, or with perm the row of slice perm[r / rpk] that r
// is of slice r / rpk (slices of rpk rows reordered).
template <typename T>
__global__ __launch_bounds__(kThreads) void pad_rows_kernel(const T *__restrict__ src,
                                                            int64_t rows, int cols, int credw,
                                                            const int32_t *__restrict__ perm,
                                                            int64_t rpk, T *__restrict__ dst) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  if (i >= rows * credw)
    return;
  int64_t r = i / credw;
  if (perm)
    r = static_cast<int64_t>(perm[r / rpk]) * rpk + r % rpk;
  const int c = static_cast<int>(i % credw);
  dst[i] = c < cols ? src[r * cols + c] : from_f32<T>(0.f);
}

// Reduction width the MFMA forward / input-gradient kernels read the weights
// at: a bf16 reduction of an odd multiple of 16 channels is padded to the
// next multiple of 32 (one 16x16x32 MFMA); everything else as it is.
static int red_width(int32_t dtype, int c) {
  return dtype == RHIP_BF16 && c % 32 == 16 ? c + 16 : c;
}

// ------------------------------------------------------------------- dW

// ------------------------------------------------------------------- dW
//
// dw[k][ci][co] += sum over the pairs p of offset k in this workgroup's range
// of x[in_rows[p]][ci] * gy[out_rows[p]][co], for a (16*VA) x (16*VB)
// channel tile (ci0, co0). The pair axis is the MFMA reduction axis.
//
// Pairs stream through LDS in chunks of 4 * PW pairs: every thread loads
// 16-byte pieces of the chunk's X and dY rows (coalesced row reads) and
// stores them row-major, double-buffered so that the next chunk's rows are in
// flight while the current one is multiplied. Each wave owns one 16-channel
// block of dY (waves sharing a block split the chunk's steps) against all
// 16*VA channels of X:
//  * fp32 (PW = 16, v_mfma_f32_16x16x4_f32): lane (i16, g) reads VA
//    consecutive channels of pair row 4s+g (one vector read) and one dY
//    channel; channel ci0 + VA*m + ea belongs to MFMA block ea, row m, so one
//    vector read feeds VA blocks and no transpose is needed;
//  * bf16 (PW = 32, v_mfma_f32_16x16x32_bf16): the K-major operands come
//    from ds_read_b64_tr_b16. Within a 16-lane group, lane i receives the
//    (i % 4)-th 16-bit element at the address of lane 4e + i/4 as element e;
//    lane j points at row (pair) 4h + j/4, channels 4*(j%4) of a 16-channel
//    block, so lane i gets channel i of four consecutive pairs, two reads
//    give the eight pairs 8g..8g+7 of group g.
// The four waves' tiles are summed in LDS; each workgroup stores its tile in
// its own slot of a partial buffer and a second kernel sums the slots of each
// offset in a fixed order (deterministic, no atomics).
template <typename T> struct DwShape;
template <> struct DwShape<float> { static constexpr int kPairsPerWave = 16; };
template <> struct DwShape<__bf16> { static constexpr int kPairsPerWave = 32; };


template <typename T, int VA, int VB, bool DB, int WAVES = 1>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(WAVES))) void conv_dw_kernel(
    const T *__restrict__ x, int cin, const T *__restrict__ gy, int cout,
    const int64_t *__restrict__ kofs, const int32_t *__restrict__ in_rows,
    const int32_t *__restrict__ out_rows, int64_t ppb, float *__restrict__ partial) {
  constexpr bool F32 = std::is_same<T, float>::value;
  constexpr int TM = 16 * VA, TN = 16 * VB;
  constexpr int PW = DwShape<T>::kPairsPerWave;
  constexpr int CP = kWaves * PW;      // pairs per chunk
  constexpr int VE = 16 / sizeof(T);   // elements per 16-byte piece
  constexpr int LDX = TM + VE, LDG = TN + VE;
  constexpr int XV = CP * (TM / VE), GV = CP * (TN / VE);  // pieces per chunk
  constexpr int XPT = (XV + kThreads - 1) / kThreads, GPT = (GV + kThreads - 1) / kThreads;
  static_assert(CP * LDX * sizeof(T) >= TM * TN * sizeof(float), "reduction reuses sX");

  constexpr int NBUF = DB ? 2 : 1;
  __shared__ __align__(16) T sX[NBUF][CP * LDX];
  __shared__ __align__(16) T sG[NBUF][CP * LDG];

  const int k = blockIdx.y;
  const int tiles_n = cout / TN;
  const int ci0 = (blockIdx.z / tiles_n) * TM;
  const int co0 = (blockIdx.z % tiles_n) * TN;
  const int64_t kb = kofs[k], ke = kofs[k + 1];
  const int64_t b0 = kb + static_cast<int64_t>(blockIdx.x) * ppb;
  if (b0 >= ke)
    return; // uniform across the workgroup
  const int64_t b1 = min(ke, b0 + ppb);
  const int nch = static_cast<int>((b1 - b0 + CP - 1) / CP);

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int i16 = lane & 15;
  const int g = lane >> 4;

  // row indices of this thread's pieces of chunk c (-1 past the range)
  int32_t xi[2][XPT], gi[2][GPT];
  auto load_idx = [&](int c, int slot) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int li = threadIdx.x + i * kThreads;
      const int64_t pp = b0 + static_cast<int64_t>(c) * CP + li / (TM / VE);
      xi[slot][i] = (li < XV && c < nch && pp < b1) ? in_rows[pp] : -1;
    }
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int li = threadIdx.x + i * kThreads;
      const int64_t pp = b0 + static_cast<int64_t>(c) * CP + li / (TN / VE);
      gi[slot][i] = (li < GV && c < nch && pp < b1) ? out_rows[pp] : -1;
    }
  };
  uint4 xr[XPT], gr[GPT];
  auto load_rows = [&](int slot) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int li = threadIdx.x + i * kThreads;
      const int cv = li % (TM / VE);
      xr[i] = xi[slot][i] >= 0
                  ? *reinterpret_cast<const uint4 *>(
                        x + static_cast<int64_t>(xi[slot][i]) * cin + ci0 + cv * VE)
                  : uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int li = threadIdx.x + i * kThreads;
      const int cv = li % (TN / VE);
      gr[i] = gi[slot][i] >= 0
                  ? *reinterpret_cast<const uint4 *>(
                        gy + static_cast<int64_t>(gi[slot][i]) * cout + co0 + cv * VE)
                  : uint4{0u, 0u, 0u, 0u};
    }
  };
  auto store_rows = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int li = threadIdx.x + i * kThreads;
      if (li < XV)
        *reinterpret_cast<uint4 *>(&sX[buf][(li / (TM / VE)) * LDX + (li % (TM / VE)) * VE]) =
            xr[i];
    }
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int li = threadIdx.x + i * kThreads;
      if (li < GV)
        *reinterpret_cast<uint4 *>(&sG[buf][(li / (TN / VE)) * LDG + (li % (TN / VE)) * VE]) =
            gr[i];
    }
  };

  // wave -> one 16-channel block nb of dY and every PG-th step of the chunk
  constexpr int PG = kWaves / VB; // waves sharing a dY block split the steps
  const int nb = wv % VB;
  const int ps = PG == 1 ? 0 : wv / VB; // 0 at compile time when a wave owns its block
  v4f acc[VA];
#pragma unroll
  for (int ea = 0; ea < VA; ++ea)
    acc[ea] = v4f{0.f, 0.f, 0.f, 0.f};

  load_idx(0, 0);
  load_idx(1, 1);
  load_rows(0);
  store_rows(0);
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const int buf = DB ? (c & 1) : 0;
    const int slot = (c + 1) & 1;
    if (c + 1 < nch)
      load_rows(slot); // rows of chunk c+1 (indices loaded one chunk ago)
    load_idx(c + 2, c & 1);
    const T *bx = sX[buf];
    const T *bg = sG[buf];
    if constexpr (F32) {
      // step s covers pairs 4s..4s+3, one per 16-lane group
#pragma unroll
      for (int s = ps; s < CP / 4; s += PG) {
        const float *ra = reinterpret_cast<const float *>(bx) + (4 * s + g) * LDX + VA * i16;
        const float b = reinterpret_cast<const float *>(bg)[(4 * s + g) * LDG + 16 * nb + i16];
        float a[VA];
        if constexpr (VA == 4) {
          const v4f t = *reinterpret_cast<const v4f *>(ra);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            a[e] = t[e];
        } else {
#pragma unroll
          for (int e = 0; e < VA; ++e)
            a[e] = ra[e];
        }
#pragma unroll
        for (int ea = 0; ea < VA; ++ea)
          acc[ea] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[ea], b, acc[ea], 0, 0, 0);
      }
    } else {
      // step s covers pairs 32s..32s+31; group g takes 8g..8g+7 of them and
      // lane i16 points at pair 8g + 4h + i16/4, channels 16*blk + 4*(i16%4)
#pragma unroll
      for (int s = ps; s < CP / 32; s += PG) {
        const int prow = 32 * s + 8 * g + i16 / 4;
        const int pcol = 4 * (i16 % 4);
        const v4s blo = ds_read_tr16(bg + prow * LDG + 16 * nb + pcol);
        const v4s bhi = ds_read_tr16(bg + (prow + 4) * LDG + 16 * nb + pcol);
        const v8bf bf = __builtin_bit_cast(v8bf, __builtin_shufflevector(blo, bhi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int ea = 0; ea < VA; ++ea) {
          const v4s lo = ds_read_tr16(bx + prow * LDX + 16 * ea + pcol);
          const v4s hi = ds_read_tr16(bx + (prow + 4) * LDX + 16 * ea + pcol);
          const v8bf af = __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
          acc[ea] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf, acc[ea], 0, 0, 0);
        }
      }
    }
    if (DB) {
      if (c + 1 < nch)
        store_rows(buf ^ 1);
      __syncthreads();
    } else {
      __syncthreads(); // every wave is done with the chunk
      if (c + 1 < nch)
        store_rows(0);
      __syncthreads();
    }
  }

  // sum the four waves' tiles in LDS (reusing sX) and store the workgroup's
  // tile in its partial slot
  float *red = reinterpret_cast<float *>(sX[0]);
  for (int i = threadIdx.x; i < TM * TN; i += kThreads)
    red[i] = 0.f;
  __syncthreads();
#pragma unroll
  for (int ea = 0; ea < VA; ++ea)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // lane holds D[4g+e][i16] of block (ea, nb)
      const int m = 4 * g + e;
      const int ci = F32 ? VA * m + ea : 16 * ea + m;
      atomicAdd(&red[ci * TN + 16 * nb + i16], acc[ea][e]);
    }
  __syncthreads();
  float *slot = partial + ((static_cast<int64_t>(k) * gridDim.z + blockIdx.z) * gridDim.x +
                           blockIdx.x) * (TM * TN);
  for (int i = threadIdx.x; i < TM * TN; i += kThreads)
    slot[i] = red[i];
}

// dw[k][ci0 + i / TN][co0 + i % TN] (colmajor: dw[k][ci0 + i % TM][co0 + i /
// TM]) = sum over the chunks c of offset k of partial[k][tile][c][i]: a
// deterministic second stage. The chunks are those holding pairs of offset k
// (ppb pairs each), or all of them when ppb is 0. A workgroup owns 256
// consecutive elements (64 lanes x 4 floats); its 4 waves sum the chunks
// c = wave (mod 4) with 16-byte loads, then the 4 phase sums are added in a
// fixed order.
template <typename OutT>
__global__ __launch_bounds__(kThreads) void conv_dw_reduce_kernel(
    const float *__restrict__ partial, const int64_t *__restrict__ kofs, int64_t ppb,
    int chunks, int tiles, int tiles_n, int TM, int TN, int cin, int cout, int colmajor,
    OutT *__restrict__ dw) {
  __shared__ v4f phase_sum[kWaves][kWave];
  const int k = blockIdx.y, t = blockIdx.z;
  const int lane = threadIdx.x & (kWave - 1), ph = threadIdx.x / kWave;
  const int n4 = TM * TN / 4; // a multiple of 64
  const int i4 = blockIdx.x * kWave + lane;
  const int64_t pk = kofs[k + 1] - kofs[k];
  const int nck = ppb > 0 ? static_cast<int>(min<int64_t>(chunks, (pk + ppb - 1) / ppb)) : chunks;
  const v4f *src = reinterpret_cast<const v4f *>(partial) +
                   (static_cast<int64_t>(k) * tiles + t) * chunks * n4 + i4;
  v4f sum = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int c = ph; c < nck; c += kWaves)
    sum += src[static_cast<int64_t>(c) * n4];
  phase_sum[ph][lane] = sum;
  __syncthreads();
  if (ph != 0)
    return;
  v4f v = phase_sum[0][lane];
#pragma unroll
  for (int q = 1; q < kWaves; ++q)
    v += phase_sum[q][lane];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = 4 * i4 + e;
    const int ci = (t / tiles_n) * TM + (colmajor ? i % TM : i / TN);
    const int co = (t % tiles_n) * TN + (colmajor ? i / TM : i % TN);
    dw[(static_cast<int64_t>(k) * cin + ci) * cout + co] = from_f32<OutT>(v[e]);
  }
}

// Pair-list dW for bf16 layers whose channel counts are multiples of 64, in
// tiles of TM x TN channels (64 or 128 each). Workgroup (r, k, tile) takes
// the r-th of `ranges` equal parts of offset k's pairs (split on the device
// from the CSR offsets, so the grid has no idle workgroups) and stores its
// TM x TN tile, column-major, in partial slot [k][tile][r]; the second stage
// (conv_dw_reduce_kernel) adds the slots of each offset in order. Inside a
// workgroup the waves share no rows: the part's pair indices go to LDS in
// batches of up to kDwPairsMaxPpb (two barriers per batch), and wave w takes
// the w-th quarter of a batch in steps of 32 pairs on its own. It loads a
// step's X and dY rows (lane l: row l / P of a load instruction's 64 / P
// rows, 16-byte piece l % P of the tile's P pieces per row), D steps ahead in
// registers, stores them to its own LDS rows and reads them back transposed
// (ds_read_b64_tr_b16, as in conv_dw_kernel) as the operands of its whole
// TM x TN tile. DS instructions of one wave execute in order, so a step's
// stores follow the previous step's reads without a wait. The four waves'
// tiles are added in LDS in wave order.
constexpr int kDwPairsMaxPpb = 2048; // pairs per index batch (the LDS index rows)
template <int TM, int TN>
constexpr int dw_pairs_lds_bytes() {
  constexpr int stage = kWaves * 32 * ((TM + 8) + (TN + 8)) * 2 + 2 * kDwPairsMaxPpb * 4;
  constexpr int red = kWaves * (TM + 4) * TN * 4 / (TM * TN > 4096 ? 2 : 1);
  return stage > red ? stage : red;
}
template <int TM, int TN, int D, int WAVES>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(WAVES))) void
conv_dw_pairs_bf16_kernel(const __bf16 *__restrict__ x, int64_t n_in, int cin,
                          const __bf16 *__restrict__ gy, int64_t n_out, int cout,
                          const int64_t *__restrict__ kofs, const int32_t *__restrict__ in_rows,
                          const int32_t *__restrict__ out_rows, int ranges,
                          float *__restrict__ partial) {
  static_assert((TM == 64 || TM == 128) && (TN == 64 || TN == 128), "64- or 128-channel tiles");
  constexpr int PX = TM / 8, PY = TN / 8;   // 16-byte pieces per row
  constexpr int NX = TM / 16, NY = TN / 16; // load instructions per 32-pair step
  constexpr int LDX = TM + 8, LDY = TN + 8; // LDS row strides (elements)
  constexpr int MB = TM / 16, NB = TN / 16;
  constexpr int RR = TM * TN > 4096 ? 2 : 1; // rounds of the final sum
  constexpr int NBR = NB / RR;               // column blocks per round
  constexpr int LDR = TM + 4;                // column stride of the sum (floats)
  __shared__ __align__(16) char smem[dw_pairs_lds_bytes<TM, TN>()];

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const int k = blockIdx.y;
  const int tiles_n = cout / TN;
  const int ci0 = (blockIdx.z / tiles_n) * TM;
  const int co0 = (blockIdx.z % tiles_n) * TN;
  const int64_t kb = kofs[k], pk = kofs[k + 1] - kb;
  const int64_t b0 = kb + pk * blockIdx.x / ranges;
  const int64_t len = kb + pk * (blockIdx.x + 1) / ranges - b0; // may be 0: the slot is zeros

  __bf16 *sX = reinterpret_cast<__bf16 *>(smem) + wv * 32 * (LDX + LDY);
  __bf16 *sY = sX + 32 * LDX;
  int32_t *sIn = reinterpret_cast<int32_t *>(smem + kWaves * 32 * (LDX + LDY) * 2);
  int32_t *sOut = sIn + kDwPairsMaxPpb;
  int wb = 0, wlen = 0; // this wave's pairs of the current batch (LDS rows)
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, n_in * cin * 2);
  const __amdgpu_buffer_rsrc_t ry = buf_rsrc(gy, n_out * cout * 2);
  const uint32_t xcol = static_cast<uint32_t>((ci0 + (lane % PX) * 8) * 2);
  const uint32_t ycol = static_cast<uint32_t>((co0 + (lane % PY) * 8) * 2);

  // step s's rows (all out of range, so no memory access, past the wave's pairs)
  auto load_step = [&](int s, v4u (&r)[NX + NY]) {
#pragma unroll
    for (int j = 0; j < NX; ++j) {
      const int li = 32 * s + j * (64 / PX) + lane / PX;
      const bool ok = li < wlen;
      const int32_t id = sIn[ok ? wb + li : 0];
      r[j] = __builtin_amdgcn_raw_buffer_load_b128(
          rx, pick_off(static_cast<uint32_t>(id) * static_cast<uint32_t>(cin * 2) + xcol,
                       ok ? -1 : 0),
          0, 0);
    }
#pragma unroll
    for (int j = 0; j < NY; ++j) {
      const int li = 32 * s + j * (64 / PY) + lane / PY;
      const bool ok = li < wlen;
      const int32_t id = sOut[ok ? wb + li : 0];
      r[NX + j] = __builtin_amdgcn_raw_buffer_load_b128(
          ry, pick_off(static_cast<uint32_t>(id) * static_cast<uint32_t>(cout * 2) + ycol,
                       ok ? -1 : 0),
          0, 0);
    }
  };
  auto store_step = [&](const v4u (&r)[NX + NY]) {
#pragma unroll
    for (int j = 0; j < NX; ++j)
      *reinterpret_cast<v4u *>(sX + (j * (64 / PX) + lane / PX) * LDX + (lane % PX) * 8) = r[j];
#pragma unroll
    for (int j = 0; j < NY; ++j)
      *reinterpret_cast<v4u *>(sY + (j * (64 / PY) + lane / PY) * LDY + (lane % PY) * 8) =
          r[NX + j];
  };
  const int prow = 8 * g + i16 / 4, pcol = 4 * (i16 % 4);
  auto operand = [&](const __bf16 *base, int ld, int col) {
    const v4s lo = ds_read_tr16(base + prow * ld + col + pcol);
    const v4s hi = ds_read_tr16(base + (prow + 4) * ld + col + pcol);
    return __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  v4f acc[MB][NB];
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int n = 0; n < NB; ++n)
      acc[m][n] = v4f{0.f, 0.f, 0.f, 0.f};
  v4u R[D][NX + NY];
  for (int64_t bs = 0; bs < len; bs += kDwPairsMaxPpb) {
    const int blen = static_cast<int>(min<int64_t>(kDwPairsMaxPpb, len - bs));
    if (bs > 0)
      __syncthreads(); // every wave is done with the previous batch's indices
    { // every load issued before the first store: one round trip
      constexpr int kPer = kDwPairsMaxPpb / kThreads;
      int32_t vi[kPer], vo[kPer];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int i = threadIdx.x + j * kThreads;
        const int64_t p = b0 + bs + (i < blen ? i : 0);
        vi[j] = in_rows[p];
        vo[j] = out_rows[p];
      }
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int i = threadIdx.x + j * kThreads;
        if (i < blen) {
          sIn[i] = vi[j];
          sOut[i] = vo[j];
        }
      }
    }
    __syncthreads();
    const int q = (blen + 4 * 32 - 1) / (4 * 32) * 32; // pairs per wave, a multiple of 32
    wb = wv * q;
    wlen = max(0, min(blen - wb, q));
    const int nst = (wlen + 31) / 32;
#pragma unroll
    for (int d = 0; d < D; ++d)
      load_step(d, R[d]);
    for (int s0 = 0; s0 < nst; s0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        if (s0 + d < nst) { // uniform
          store_step(R[d]);
          load_step(s0 + d + D, R[d]);
          v8bf b[NB];
#pragma unroll
          for (int n = 0; n < NB; ++n)
            b[n] = operand(sY, LDY, 16 * n);
#pragma unroll
          for (int m = 0; m < MB; ++m) {
            const v8bf a = operand(sX, LDX, 16 * m);
#pragma unroll
            for (int n = 0; n < NB; ++n)
              acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[n], acc[m][n], 0, 0, 0);
          }
        }
      }
    }
  }

  // the four tiles, added in wave order, into the slot [TN][TM] (column-
  // major); RR rounds of NBR column blocks. Lane (i16, g) holds rows
  // 4g..4g+3 of column i16 of block (m, n): one 16-byte LDS store each
  // (columns LDR floats apart: the 16 lanes of a row group hit distinct banks)
  float *red = reinterpret_cast<float *>(smem);
  float *slot = partial + ((static_cast<int64_t>(k) * gridDim.z + blockIdx.z) * ranges +
                           blockIdx.x) * (TM * TN);
#pragma unroll
  for (int rr = 0; rr < RR; ++rr) {
    __syncthreads(); // the staging rows (or the previous round) are free
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
      for (int n = 0; n < NBR; ++n)
        *reinterpret_cast<v4f *>(red + (wv * 16 * NBR + 16 * n + i16) * LDR + 16 * m + 4 * g) =
            acc[m][rr * NBR + n];
    __syncthreads();
    for (int i = threadIdx.x; i < TM * 16 * NBR / 4; i += kThreads) {
      const int c = i / (TM / 4), r4 = 4 * (i % (TM / 4)); // column of the round, first row
      v4f v = *reinterpret_cast<const v4f *>(red + c * LDR + r4);
#pragma unroll
      for (int w = 1; w < kWaves; ++w)
        v += *reinterpret_cast<const v4f *>(red + (w * 16 * NBR + c) * LDR + r4);
      *reinterpret_cast<v4f *>(slot + (rr * 16 * NBR + c) * TM + r4) = v;
    }
  }
}

// ------------------------------------------------------------ dW by rows
//
// For narrow bf16 layers (cin, cout in {16, 32}) dW is computed from the
// dense neighbour table instead of the pair list: each dY row is read once
// per group of offsets rather than once per pair, which halves the gathered
// bytes of a 3^3 map (about 10 neighbours per row).
//
// A workgroup owns a range of output positions and KW offsets (grid.y picks
// the offset group); its four waves take alternate 32-position sub-tiles and
// work independently, each with its own LDS rows: the sub-tile's dY rows
// (32 x cout) and, one offset at a time, the gathered X rows (32 x cin),
// read back K-major with ds_read_tr16 (as in conv_dw_kernel) and multiplied
// on v_mfma_f32_16x16x32_bf16 with the positions as the reduction axis. The
// next offset's rows are in flight while the current one multiplies. LDS
// traffic of a wave is ordered within the wave, so no workgroup barrier is
// needed until the end, where the four waves' tiles are added in wave order
// and the workgroup writes one partial slot per offset.
constexpr int kDwRowsSP = 32; // positions per sub-tile (one MFMA reduction step)

template <int VA, int VB, int KW>
__global__ __launch_bounds__(kThreads) void conv_dw_rows_kernel(
    const __bf16 *__restrict__ x, const __bf16 *__restrict__ gy,
    const int32_t *__restrict__ nbr, const int32_t *__restrict__ out_order, int64_t n_out,
    int K, int64_t rows_per_block, int row_blocks, int xcd_map, float *__restrict__ partial) {
  constexpr int TM = 16 * VA, TN = 16 * VB, SP = kDwRowsSP;
  constexpr int LDX = TM + 8, LDG = TN + 8; // 16-byte row padding
  __shared__ __align__(16) __bf16 sG[kWaves][SP * LDG];
  __shared__ __align__(16) __bf16 sX[kWaves][SP * LDX];
  __shared__ __align__(16) float red[KW * TM * TN];

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int i16 = lane & 15;
  const int g = lane >> 4;
  // row block and offset group: with xcd_map the grid is 1-D and each XCD
  // runs every offset group of its row blocks back to back (shared L2)
  int rb = blockIdx.x, grp = blockIdx.y;
  if (xcd_map) {
    const int groups = (K + KW - 1) / KW;
    const int xcd = static_cast<int>(blockIdx.x % kXcds), m = static_cast<int>(blockIdx.x / kXcds);
    grp = m % groups;
    rb = (m / groups) * kXcds + xcd;
  }
  if (rb >= row_blocks)
    return; // padding workgroup (uniform)
  const int64_t p0 = rb * rows_per_block;
  const int64_t p1 = min(n_out, p0 + rows_per_block);
  const int k0 = grp * KW;

  v4f acc[KW][VA][VB];
#pragma unroll
  for (int j = 0; j < KW; ++j)
#pragma unroll
    for (int ea = 0; ea < VA; ++ea)
#pragma unroll
      for (int eb = 0; eb < VB; ++eb)
        acc[j][ea][eb] = v4f{0.f, 0.f, 0.f, 0.f};

  // lane pieces (16 bytes) of a 32-row sub-tile: X piece i of offset j is
  // row (lane + 64 i) / (TM / 8), 8 channels at (lane + 64 i) % (TM / 8)
  const int prow = 8 * g + i16 / 4, pcol = 4 * (i16 % 4);
  // indices of sub-tile q: the dY rows' output rows and every offset's
  // neighbours (-1: none or past the range; clamped reads, masked)
  int64_t orow[VB];
  int32_t id[KW][VA];
  auto load_ids = [&](int64_t q, int64_t (&orow_)[VB], int32_t (&id_)[KW][VA]) {
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      const int64_t pos = q + (lane + kWave * i) / (TN / 8);
      const int64_t pc_ = pos < p1 ? pos : p1 - 1;
      orow_[i] = (out_order ? out_order[pc_] : pc_) | (pos < p1 ? 0 : -1);
    }
#pragma unroll
    for (int j = 0; j < KW; ++j)
#pragma unroll
      for (int i = 0; i < VA; ++i) {
        const int64_t pos = q + (lane + kWave * i) / (TM / 8);
        const int kk = k0 + j < K ? k0 + j : K - 1;
        const int32_t v = nbr[kk * n_out + (pos < p1 ? pos : p1 - 1)];
        id_[j][i] = v | ((k0 + j < K && pos < p1) ? 0 : -1);
      }
  };
  const int64_t q_first = p0 + wv * SP;
  if (q_first < p1)
    load_ids(q_first, orow, id);
  for (int64_t q = q_first; q < p1; q += kWaves * SP) {
    // this sub-tile's dY rows and first offset's rows, then the next
    // sub-tile's indices, all in flight together
    uint4 gv[VB];
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      const int pc = lane + kWave * i;
      gv[i] = *reinterpret_cast<const uint4 *>(gy + (orow[i] < 0 ? 0 : orow[i]) * TN +
                                               (pc % (TN / 8)) * 8);
    }
    uint4 xv[VA], xn[VA];
#pragma unroll
    for (int i = 0; i < VA; ++i) {
      const int pc = lane + kWave * i;
      xv[i] = *reinterpret_cast<const uint4 *>(
          x + static_cast<int64_t>(id[0][i] < 0 ? 0 : id[0][i]) * TM + (pc % (TM / 8)) * 8);
    }
    int64_t orow_n[VB];
    int32_t id_n[KW][VA];
    const bool more = q + kWaves * SP < p1; // uniform
    if (more)
      load_ids(q + kWaves * SP, orow_n, id_n);
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      const int pc = lane + kWave * i;
      uint4 v = gv[i];
      const uint32_t m = orow[i] >= 0 ? ~0u : 0u;
      v.x &= m, v.y &= m, v.z &= m, v.w &= m;
      *reinterpret_cast<uint4 *>(&sG[wv][(pc / (TN / 8)) * LDG + (pc % (TN / 8)) * 8]) = v;
    }
    __builtin_amdgcn_wave_barrier();
    v8bf bfr[VB];
#pragma unroll
    for (int eb = 0; eb < VB; ++eb) {
      const v4s lo = ds_read_tr16(&sG[wv][prow * LDG + 16 * eb + pcol]);
      const v4s hi = ds_read_tr16(&sG[wv][(prow + 4) * LDG + 16 * eb + pcol]);
      bfr[eb] = __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
#pragma unroll
    for (int j = 0; j < KW; ++j) {
      if (j + 1 < KW) { // the next offset's rows
#pragma unroll
        for (int i = 0; i < VA; ++i) {
          const int pc = lane + kWave * i;
          xn[i] = *reinterpret_cast<const uint4 *>(
              x + static_cast<int64_t>(id[j + 1][i] < 0 ? 0 : id[j + 1][i]) * TM +
              (pc % (TM / 8)) * 8);
        }
      }
      bool any = false;
#pragma unroll
      for (int i = 0; i < VA; ++i) {
        const int pc = lane + kWave * i;
        uint4 v = xv[i];
        const uint32_t m = id[j][i] >= 0 ? ~0u : 0u;
        v.x &= m, v.y &= m, v.z &= m, v.w &= m;
        *reinterpret_cast<uint4 *>(&sX[wv][(pc / (TM / 8)) * LDX + (pc % (TM / 8)) * 8]) = v;
        any |= id[j][i] >= 0;
      }
      __builtin_amdgcn_wave_barrier();
      if (__ballot(any) != 0) { // uniform
#pragma unroll
        for (int ea = 0; ea < VA; ++ea) {
          const v4s lo = ds_read_tr16(&sX[wv][prow * LDX + 16 * ea + pcol]);
          const v4s hi = ds_read_tr16(&sX[wv][(prow + 4) * LDX + 16 * ea + pcol]);
          const v8bf af =
              __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
          for (int eb = 0; eb < VB; ++eb)
            acc[j][ea][eb] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[eb], acc[j][ea][eb], 0, 0, 0);
        }
      }
      __builtin_amdgcn_wave_barrier();
      if (j + 1 < KW) {
#pragma unroll
        for (int i = 0; i < VA; ++i)
          xv[i] = xn[i];
      }
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < VB; ++i)
        orow[i] = orow_n[i];
#pragma unroll
      for (int j = 0; j < KW; ++j)
#pragma unroll
        for (int i = 0; i < VA; ++i)
          id[j][i] = id_n[j][i];
    }
  }

  // add the four waves' tiles in wave order, then one partial slot per
  // offset: partial[blockIdx.x][k][ci][co]; lane holds D[4g+e][i16] of
  // block (ea, eb), i.e. ci = 16 ea + 4 g + e, co = 16 eb + i16
  for (int w = 0; w < kWaves; ++w) {
    if (wv == w) {
#pragma unroll
      for (int j = 0; j < KW; ++j)
#pragma unroll
        for (int ea = 0; ea < VA; ++ea)
#pragma unroll
          for (int eb = 0; eb < VB; ++eb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float &r = red[(j * TM + 16 * ea + 4 * g + e) * TN + 16 * eb + i16];
              r = w == 0 ? acc[j][ea][eb][e] : r + acc[j][ea][eb][e];
            }
    }
    __syncthreads();
  }
  const int kn = min(KW, K - k0);
  float *slot = partial + (static_cast<int64_t>(rb) * K + k0) * (TM * TN);
  for (int i = threadIdx.x; i < kn * TM * TN; i += kThreads)
    slot[i] = red[i];
}

// dw[k][ci][co] = sum over the slots s (in order) of partial[s][k][ci][co].
// A workgroup of 16 waves owns 256 consecutive elements (a float4 per lane);
// wave w sums the slots s = w (mod 16), the 16 sums are then added in order.
template <typename OutT>
__global__ __launch_bounds__(1024) void conv_dw_rows_reduce_kernel(
    const float *__restrict__ partial, int slots, int64_t n_elem, OutT *__restrict__ dw) {
  __shared__ v4f part[16][kWave];
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int64_t i4 = static_cast<int64_t>(blockIdx.x) * kWave + lane;
  const int64_t n4 = n_elem / 4;
  v4f sum = v4f{0.f, 0.f, 0.f, 0.f};
  if (i4 < n4) {
    const v4f *src = reinterpret_cast<const v4f *>(partial) + i4;
#pragma unroll 4
    for (int s = w; s < slots; s += 16)
      sum += src[static_cast<int64_t>(s) * n4];
  }
  part[w][lane] = sum;
  __syncthreads();
  if (w != 0 || i4 >= n4)
    return;
  v4f v = part[0][lane];
#pragma unroll
  for (int q = 1; q < 16; ++q)
    v += part[q][lane];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    dw[4 * i4 + e] = from_f32<OutT>(v[e]);
}

// ---------------------------------------------------- fp32 dW by positions
//
// fp32 dW from the neighbour table, position-stationary: a workgroup owns a
// range of processing positions, a 16-channel input slice ci0 and 16*VB
// output channels co0, and up to 4*KPW offsets (one offset group); wave w
// keeps the 16 x 16*VB tiles of offsets k0 + w + 4j (j < KPW) in registers
// for the whole range. A step covers 4 consecutive positions (the reduction
// axis of v_mfma_f32_16x16x4f32):
//  * lane (i16, g) reads dY[out_order[p0 + 4s + g]][co0 + VB*i16 .. +VB-1]
//    (one vector load; channel co0 + VB*n + eb belongs to MFMA block eb,
//    column n) and, per offset, X[nbr[k][p0 + 4s + g]][ci0 + i16];
//  * a step whose four positions have no neighbour under k skips that
//    offset's MFMAs (wave-uniform); in the mask-grouped processing order
//    nearly every step is full or empty;
//  * absent neighbours and positions past the range are buffer loads with
//    an offset past the buffer's size, which the hardware returns as zero
//    without a memory access, so no load is predicated.
// Indices are loaded two steps ahead, rows one step ahead. Every X row a
// range touches is read from memory about once and then hits the caches
// (neighbouring positions share rows under different offsets); the pair
// list kernel reads one X row and one dY row per pair.
// Each wave writes its offsets' tiles to the range's partial slot
// [range][k][cin][cout]; conv_dw_rows_reduce_kernel sums the slots.

template <int VB> struct DyVec;
template <> struct DyVec<1> {
  using T = float;
  __device__ static __forceinline__ T load(__amdgpu_buffer_rsrc_t r, uint32_t o) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0));
  }
  __device__ static __forceinline__ float at(T v, int) { return v; }
};
template <> struct DyVec<2> {
  using T = v2u;
  __device__ static __forceinline__ T load(__amdgpu_buffer_rsrc_t r, uint32_t o) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, o, 0, 0);
  }
  __device__ static __forceinline__ float at(T v, int e) {
    const uint32_t t = v[e]; // bit_cast of the subscript itself reads element 0
    return __builtin_bit_cast(float, t);
  }
};
template <> struct DyVec<4> {
  using T = v4u;
  __device__ static __forceinline__ T load(__amdgpu_buffer_rsrc_t r, uint32_t o) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0);
  }
  __device__ static __forceinline__ float at(T v, int e) {
    const uint32_t t = v[e]; // bit_cast of the subscript itself reads element 0
    return __builtin_bit_cast(float, t);
  }
};

template <int VB, int KPW, int NSLOT, int WAVES>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(WAVES))) void
conv_dw_pos_kernel(const float *__restrict__ x, int64_t n_in, int cin,
                   const float *__restrict__ gy, int cout, const int32_t *__restrict__ nbr,
                   const int32_t *__restrict__ out_order, int64_t n_out, int K, int ranges,
                   int ci_tiles, int co_tiles, float *__restrict__ partial) {
  using DV = DyVec<VB>;
  constexpr int GK = kWaves * KPW; // offsets per group
  const int groups = (K + GK - 1) / GK;
  const int units = ci_tiles * co_tiles * groups;
  // XCD x runs ranges [x*R8, (x+1)*R8) with every unit (slice, group) of a
  // range back to back; ranges is a multiple of 8
  const int r8 = ranges / kXcds;
  const int xcd = static_cast<int>(blockIdx.x % kXcds), m = static_cast<int>(blockIdx.x / kXcds);
  const int rg = xcd * r8 + m / units;
  int u = m % units;
  const int grp = u % groups;
  u /= groups;
  const int ci0 = (u % ci_tiles) * 16, co0 = (u / ci_tiles) * (16 * VB);

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int i16 = lane & 15;
  const int g = lane >> 4;
  // segments of 64 positions (16 steps) are dealt to the ranges in turn
  // (range rg takes segments rg, rg + ranges, ...), which spreads the dense
  // and the sparse neighbour masks of the processing order evenly; an even
  // count per range: segments past the end load nothing and multiply nothing
  const int64_t total = (n_out + 63) / 64;
  const int segs = static_cast<int>((total + 2LL * ranges - 1) / (2LL * ranges)) * 2;
  int kk[KPW], kval[KPW];
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    kk[j] = grp * GK + wv + kWaves * j;
    kval[j] = opaque(kk[j] < K ? -1 : 0);
  }

  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, n_in * cin * 4);
  const __amdgpu_buffer_rsrc_t ry = buf_rsrc(gy, n_out * cout * 4);
  const __amdgpu_buffer_rsrc_t rn = buf_rsrc(nbr, static_cast<int64_t>(K) * n_out * 4);
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(out_order, out_order ? n_out * 4 : 0);
  const int32_t has_order = opaque(out_order ? -1 : 0);
  // offsets are chosen with opaque all-ones / zero masks rather than
  // selects, so that no load ends up behind a divergent branch
  auto pick = [](uint32_t off, int32_t keep) {
    return (off & static_cast<uint32_t>(keep)) | (kBufOob & ~static_cast<uint32_t>(keep));
  };

  // a segment's indices, lane l holding position 64*sg + l: the neighbour
  // row under each offset (-1 = none) and the dY row (-1 past the range)
  // raw loads: the masks for absent entries (-1) are applied in prep, a
  // segment later, so that nothing waits for these loads when they are issued
  // (an in-order wait would also wait for the rows prefetched before them)
  struct Seg {
    int32_t id[KPW];
    int32_t orow;
    int32_t pos;
    int32_t in; // -1 for a position of the map, 0 past its end
  };
  struct Dat {
    float a[KPW];
    typename DV::T d;
  };
  auto load_seg = [&](int sg, Seg &S) {
    const int64_t p = 64 * (rg + static_cast<int64_t>(sg) * ranges) + lane;
    const int32_t in = opaque(static_cast<int32_t>((p - n_out) >> 63)); // -1 for a position
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int32_t keep = in & kval[j];
      S.id[j] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
          rn, pick(static_cast<uint32_t>((kk[j] * n_out + p) * 4), keep), 0, 0));
    }
    // loaded also without an order (from an empty buffer, as zero): a load
    // behind a branch leaves the in-order waits for the rows prefetched
    // before it uncounted, and the loop head then waits for every load
    S.orow = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
        ro, pick(static_cast<uint32_t>(p * 4), in & has_order), 0, 0));
    S.pos = static_cast<int32_t>(p);
    S.in = in;
  };
  // Once a segment's indices have arrived: the live masks (bit l: position
  // l has a neighbour under offset j), then the indices become byte offsets
  // of the rows' first channel (out of range for an absent row).
  auto prep = [&](Seg &S, uint64_t (&live)[KPW]) {
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int32_t r = S.id[j] | ~(S.in & kval[j]);
      live[j] = __ballot(r >= 0);
      S.id[j] = static_cast<int32_t>(pick(static_cast<uint32_t>((r * cin + ci0) * 4), opaque(~(r >> 31))));
    }
    const int32_t r = (S.orow & has_order) | (S.pos & ~has_order) | ~S.in;
    S.orow = static_cast<int32_t>(pick(static_cast<uint32_t>((r * cout + co0) * 4), opaque(~(r >> 31))));
  };
  // rows of step s of a segment: lane (i16, g) takes position 4s + g's
  // offsets from lane 4s + g (ds_bpermute); an absent row's offset stays
  // out of range after the lane's channel is added
  auto load_dat = [&](const Seg &S, int s, Dat &D) {
    const int src = (4 * s + g) * 4;
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const uint32_t o = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, S.id[j])) + 4 * i16;
      D.a[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, o, 0, 0));
    }
    const uint32_t o = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, S.orow)) + 4 * VB * i16;
    D.d = DV::load(ry, o);
    // a compiler-only barrier: the loads stay here instead of sinking into
    // the live branch of their step, where they would be waited for at once
    asm volatile("" ::: "memory");
  };

  v4f acc[KPW][VB];
#pragma unroll
  for (int j = 0; j < KPW; ++j)
#pragma unroll
    for (int eb = 0; eb < VB; ++eb)
      acc[j][eb] = v4f{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Dat &D, const uint64_t (&live)[KPW], int s) {
#pragma unroll
    for (int j = 0; j < KPW; ++j)
      if ((live[j] >> (4 * s)) & 0xfu) { // wave-uniform
#pragma unroll
        for (int eb = 0; eb < VB; ++eb)
          acc[j][eb] = __builtin_amdgcn_mfma_f32_16x16x4f32(D.a[j], DV::at(D.d, eb), acc[j][eb], 0,
                                                             0, 0);
      }
  };

  // Two segment slots used in alternation and NSLOT row slots (NSLOT
  // divides 16, so step s of every segment uses slot s % NSLOT): no
  // in-flight load is ever copied. Indices are loaded one segment ahead,
  // rows NSLOT - 1 steps ahead.
  static_assert(16 % NSLOT == 0, "row slots must divide a segment");
  Seg SA, SB;
  uint64_t LA[KPW], LB[KPW];
  Dat D[NSLOT];
  auto run_seg = [&](Seg &S, const uint64_t (&LS)[KPW], Seg &N, uint64_t (&LN)[KPW],
                     int next_load) {
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int ahead = s + NSLOT - 1;
      if (ahead < 16) {
        load_dat(S, ahead, D[ahead % NSLOT]);
      } else {
        if (ahead == 16)
          prep(N, LN);
        load_dat(N, ahead - 16, D[ahead % NSLOT]);
      }
      compute(D[s % NSLOT], LS, s);
    }
    load_seg(next_load, S);
  };
  load_seg(0, SA);
  load_seg(1, SB);
  prep(SA, LA);
#pragma unroll
  for (int s = 0; s + 1 < NSLOT; ++s)
    load_dat(SA, s, D[s]);
  for (int sg = 0; sg < segs; sg += 2) {
    run_seg(SA, LA, SB, LB, sg + 2);
    run_seg(SB, LB, SA, LA, sg + 3);
  }

  // lane holds D[4g+e][i16] of block eb: dW[k][ci0 + 4g + e][co0 + VB*i16 + eb]
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    if (kk[j] >= K)
      continue;
    float *dst = partial + ((static_cast<int64_t>(rg) * K + kk[j]) * cin + ci0 + 4 * g) * cout +
                 co0 + VB * i16;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (VB == 4) {
        *reinterpret_cast<v4f *>(dst + static_cast<int64_t>(e) * cout) =
            v4f{acc[j][0][e], acc[j][1][e], acc[j][2][e], acc[j][3][e]};
      } else {
#pragma unroll
        for (int eb = 0; eb < VB; ++eb)
          dst[static_cast<int64_t>(e) * cout + eb] = acc[j][eb][e];
      }
    }
  }
}

// Lane n of each 16-lane row of v, broadcast to the whole row (DPP
// row_newbcast; n must fold to a constant).
__device__ __forceinline__ int32_t row_bcast(int32_t v, int n) {
  switch (n) {
  case 0: return __builtin_amdgcn_mov_dpp(v, 0x150, 0xf, 0xf, false);
  case 1: return __builtin_amdgcn_mov_dpp(v, 0x151, 0xf, 0xf, false);
  case 2: return __builtin_amdgcn_mov_dpp(v, 0x152, 0xf, 0xf, false);
  case 3: return __builtin_amdgcn_mov_dpp(v, 0x153, 0xf, 0xf, false);
  case 4: return __builtin_amdgcn_mov_dpp(v, 0x154, 0xf, 0xf, false);
  case 5: return __builtin_amdgcn_mov_dpp(v, 0x155, 0xf, 0xf, false);
  case 6: return __builtin_amdgcn_mov_dpp(v, 0x156, 0xf, 0xf, false);
  case 7: return __builtin_amdgcn_mov_dpp(v, 0x157, 0xf, 0xf, false);
  case 8: return __builtin_amdgcn_mov_dpp(v, 0x158, 0xf, 0xf, false);
  case 9: return __builtin_amdgcn_mov_dpp(v, 0x159, 0xf, 0xf, false);
  case 10: return __builtin_amdgcn_mov_dpp(v, 0x15a, 0xf, 0xf, false);
  case 11: return __builtin_amdgcn_mov_dpp(v, 0x15b, 0xf, 0xf, false);
  case 12: return __builtin_amdgcn_mov_dpp(v, 0x15c, 0xf, 0xf, false);
  case 13: return __builtin_amdgcn_mov_dpp(v, 0x15d, 0xf, 0xf, false);
  case 14: return __builtin_amdgcn_mov_dpp(v, 0x15e, 0xf, 0xf, false);
  default: return __builtin_amdgcn_mov_dpp(v, 0x15f, 0xf, 0xf, false);
  }
}

// fp32 dW from the neighbour table for 64-channel input and output tiles
// (C_in and C_out multiples of 64), the same position-stationary design as
// conv_dw_pos_kernel with each lane's X load widened to 16 bytes:
//  * lane (i16, g) reads X[nbr[k][p0 + 4s + g]][ci0 + 4*i16 .. +3] and
//    dY[out_order[p0 + 4s + g]][co0 + 4*i16 .. +3]; element m of the X vector
//    is the A operand of MFMA row block m (row i16 = channel ci0 + 4*i16 + m)
//    and element e of the dY vector the B operand of column block e, so one
//    X load and one index move feed 16 MFMAs (4 with 16-channel slices);
//  * wave w of a WPB-wave workgroup of offset group q keeps the 64 x 64
//    tiles of offsets q + G*(w + WPB*j) (j < KPW, G groups) in registers (64
//    floats per lane and offset). Dealing the offsets with stride G mixes the
//    dense and the sparse ones in every group: on config 2's scenes the
//    heaviest group holds 1.05x the mean pair count, against 1.86x for
//    groups of consecutive offsets (every plane of a 3^3 stencil has its
//    own density);
//  * a segment's indices are loaded transposed, lane (i16, g) holding
//    position 4*i16 + g, so that step s's four positions are column s of the
//    four 16-lane rows and one DPP row broadcast hands each lane its
//    position's index (no LDS round trip before the row loads, which a
//    ds_bpermute puts between every step's multiplies and its next loads);
//  * segment dealing, row slots, skipped steps and the partial slots
//    [range][k][cin][cout] are as in conv_dw_pos_kernel.
// Lane (i16, g) ends with D[4g+r][i16] of block (m, e), which is
// dW[k][ci0 + 16g + 4r + m][co0 + 4*i16 + e].
template <int KPW, int NSLOT, int WAVES, int WPB>
__global__ __launch_bounds__(WPB * kWave) __attribute__((amdgpu_waves_per_eu(WAVES))) void
conv_dw_pos64_kernel(const float *__restrict__ x, int64_t n_in, int cin,
                     const float *__restrict__ gy, int cout, const int32_t *__restrict__ nbr,
                     const int32_t *__restrict__ out_order, int64_t n_out, int K, int ranges,
                     int ci_tiles, int co_tiles, float *__restrict__ partial) {
  constexpr int GK = WPB * KPW; // offsets per group
  const int groups = (K + GK - 1) / GK;
  const int units = ci_tiles * co_tiles * groups;
  const int r8 = ranges / kXcds;
  const int xcd = static_cast<int>(blockIdx.x % kXcds), m = static_cast<int>(blockIdx.x / kXcds);
  const int rg = xcd * r8 + m / units;
  int u = m % units;
  const int grp = u % groups;
  u /= groups;
  const int ci0 = (u % ci_tiles) * 64, co0 = (u / ci_tiles) * 64;

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int i16 = lane & 15;
  const int g = lane >> 4;
  if (grp + groups * wv >= K) // a wave without offsets (no barrier follows)
    return;
  const int64_t total = (n_out + 63) / 64;
  const int segs = static_cast<int>((total + 2LL * ranges - 1) / (2LL * ranges)) * 2;
  int kk[KPW], kval[KPW];
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    kk[j] = grp + groups * (wv + WPB * j);
    kval[j] = opaque(kk[j] < K ? -1 : 0);
  }

  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, n_in * cin * 4);
  const __amdgpu_buffer_rsrc_t ry = buf_rsrc(gy, n_out * cout * 4);
  const __amdgpu_buffer_rsrc_t rn = buf_rsrc(nbr, static_cast<int64_t>(K) * n_out * 4);
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(out_order, out_order ? n_out * 4 : 0);
  const int32_t has_order = opaque(out_order ? -1 : 0);

  struct Seg {
    int32_t id[KPW];
    int32_t orow;
    int32_t pos;
    int32_t in;
  };
  struct Dat {
    v4u a[KPW];
    v4u d;
  };
  auto load_seg = [&](int sg, Seg &S) {
    const int64_t p = 64 * (rg + static_cast<int64_t>(sg) * ranges) + 4 * i16 + g;
    const int32_t in = opaque(static_cast<int32_t>((p - n_out) >> 63)); // -1 for a position
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int32_t keep = in & kval[j];
      S.id[j] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
          rn, pick_off(static_cast<uint32_t>((kk[j] * n_out + p) * 4), keep), 0, 0));
    }
    // loaded also without an order (from an empty buffer, as zero): a load
    // behind a branch leaves the in-order waits for the rows prefetched
    // before it uncounted, and the loop head then waits for every load
    S.orow = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
        ro, pick_off(static_cast<uint32_t>(p * 4), in & has_order), 0, 0));
    S.pos = static_cast<int32_t>(p);
    S.in = in;
  };
  auto prep = [&](Seg &S, uint64_t (&live)[KPW]) {
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int32_t r = S.id[j] | ~(S.in & kval[j]);
      live[j] = __ballot(r >= 0);
      S.id[j] = static_cast<int32_t>(
          pick_off(static_cast<uint32_t>((r * cin + ci0) * 4), opaque(~(r >> 31))));
    }
    const int32_t r = (S.orow & has_order) | (S.pos & ~has_order) | ~S.in;
    S.orow = static_cast<int32_t>(
        pick_off(static_cast<uint32_t>((r * cout + co0) * 4), opaque(~(r >> 31))));
  };
  auto load_dat = [&](const Seg &S, int s, Dat &D) {
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const uint32_t o = static_cast<uint32_t>(row_bcast(S.id[j], s)) + 16 * i16;
      D.a[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0);
    }
    const uint32_t o = static_cast<uint32_t>(row_bcast(S.orow, s)) + 16 * i16;
    D.d = __builtin_amdgcn_raw_buffer_load_b128(ry, o, 0, 0);
    // a compiler-only barrier: the loads stay here instead of sinking into
    // the live branch of their step, where they would be waited for at once
    asm volatile("" ::: "memory");
  };

  v4f acc[KPW][4][4];
#pragma unroll
  for (int j = 0; j < KPW; ++j)
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int eb = 0; eb < 4; ++eb)
        acc[j][mb][eb] = v4f{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Dat &D, const uint64_t (&live)[KPW], int s) {
#pragma unroll
    for (int j = 0; j < KPW; ++j)
      if ((live[j] >> s) & 0x0001000100010001ull) { // wave-uniform: column s of the rows
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          const uint32_t av = D.a[j][mb];
#pragma unroll
          for (int eb = 0; eb < 4; ++eb) {
            const uint32_t dv = D.d[eb];
            acc[j][mb][eb] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                __builtin_bit_cast(float, av), __builtin_bit_cast(float, dv), acc[j][mb][eb], 0, 0,
                0);
          }
        }
      }
  };

  static_assert(16 % NSLOT == 0, "row slots must divide a segment");
  Seg SA, SB;
  uint64_t LA[KPW], LB[KPW];
  Dat D[NSLOT];
  auto run_seg = [&](Seg &S, const uint64_t (&LS)[KPW], Seg &N, uint64_t (&LN)[KPW],
                     int next_load) {
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int ahead = s + NSLOT - 1;
      if (ahead < 16) {
        load_dat(S, ahead, D[ahead % NSLOT]);
      } else {
        if (ahead == 16)
          prep(N, LN);
        load_dat(N, ahead - 16, D[ahead % NSLOT]);
      }
      compute(D[s % NSLOT], LS, s);
    }
    load_seg(next_load, S);
  };
  load_seg(0, SA);
  load_seg(1, SB);
  prep(SA, LA);
#pragma unroll
  for (int s = 0; s + 1 < NSLOT; ++s)
    load_dat(SA, s, D[s]);
  for (int sg = 0; sg < segs; sg += 2) {
    run_seg(SA, LA, SB, LB, sg + 2);
    run_seg(SB, LB, SA, LA, sg + 3);
  }

#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    if (kk[j] >= K)
      continue;
    float *dst = partial + ((static_cast<int64_t>(rg) * K + kk[j]) * cin + ci0 + 16 * g) * cout +
                 co0 + 4 * i16;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        *reinterpret_cast<v4f *>(dst + static_cast<int64_t>(4 * r + mb) * cout) =
            v4f{acc[j][mb][0][r], acc[j][mb][1][r], acc[j][mb][2][r], acc[j][mb][3][r]};
  }
}

// bf16 dW from the neighbour table, position-stationary like
// conv_dw_pos_kernel: a workgroup owns a 16-channel input slice ci0, 16*NB
// output channels co0 and up to 4*KPW offsets; wave w keeps the 16 x 16*NB
// tiles of offsets k0 + w + 4j in registers. A step covers 32 positions
// (the reduction axis of v_mfma_f32_16x16x32_bf16), and its rows go through
// the wave's own LDS rows so that ds_read_b64_tr_b16 can hand each lane the
// eight positions of one channel:
//  * lane l loads half of position l/2's dY row (8*NB channels, NB x 16
//    bytes) and, per offset, half of its X slice (8 channels, 16 bytes);
//  * at the step, the wave writes them row-major to its LDS rows and reads
//    the K-major operands back (two transposed reads per 16 x 32 operand);
//    LDS traffic of one wave completes in order, so no barrier is needed;
//  * an offset without a neighbour among the step's 32 positions skips its
//    LDS traffic and MFMAs (wave-uniform).
// Indices, out-of-range buffer loads, segments dealt to ranges and the
// partial slots are as in conv_dw_pos_kernel; rows are loaded one step
// (32 positions) ahead. With SHY the workgroup shares one dY tile per step:
// wave w loads and stores positions 8w .. 8w+7 into one of two LDS buffers
// and a barrier publishes it (a wave at step t writes the buffer of step
// t-2, which every wave finished before the barrier of step t-1).
template <int NB, int KPW, int WAVES, bool SHY = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(WAVES))) void
conv_dw_pos_bf16_kernel(const __bf16 *__restrict__ x, int64_t n_in, int cin,
                        const __bf16 *__restrict__ gy, int cout, const int32_t *__restrict__ nbr,
                        const int32_t *__restrict__ out_order, int64_t n_out, int K, int ranges,
                        int ci_tiles, int co_tiles, float *__restrict__ partial) {
  constexpr int GK = kWaves * KPW;
  constexpr int LDY = 16 * NB + 8, LDX = 16 + 8; // LDS row strides (elements), 16-byte multiples
  // SHY: one dY tile per step for the whole workgroup (wave w loads and
  // writes positions 8w .. 8w+7), two buffers, one barrier per step
  __shared__ __align__(16) __bf16 sY[SHY ? 2 : kWaves][32 * LDY];
  __shared__ __align__(16) __bf16 sX[kWaves][32 * LDX];
  const int groups = (K + GK - 1) / GK;
  const int units = ci_tiles * co_tiles * groups;
  const int r8 = ranges / kXcds;
  const int xcd = static_cast<int>(blockIdx.x % kXcds), m = static_cast<int>(blockIdx.x / kXcds);
  const int rg = xcd * r8 + m / units;
  int u = m % units;
  const int grp = u % groups;
  u /= groups;
  const int ci0 = (u % ci_tiles) * 16, co0 = (u / ci_tiles) * (16 * NB);

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const int half = lane & 1;
  const int64_t total = (n_out + 63) / 64;
  const int segs = static_cast<int>((total + 2LL * ranges - 1) / (2LL * ranges)) * 2;
  int kk[KPW], kval[KPW];
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    kk[j] = grp * GK + wv + kWaves * j;
    kval[j] = opaque(kk[j] < K ? -1 : 0);
  }

  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, n_in * cin * 2);
  const __amdgpu_buffer_rsrc_t ry = buf_rsrc(gy, n_out * cout * 2);
  const __amdgpu_buffer_rsrc_t rn = buf_rsrc(nbr, static_cast<int64_t>(K) * n_out * 4);
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(out_order, out_order ? n_out * 4 : 0);
  const int32_t has_order = opaque(out_order ? -1 : 0);
  auto pick = [](uint32_t off, int32_t keep) {
    return (off & static_cast<uint32_t>(keep)) | (kBufOob & ~static_cast<uint32_t>(keep));
  };

  // raw loads: the masks for absent entries (-1) are applied in prep, a
  // segment later, so that nothing waits for these loads when they are issued
  // (an in-order wait would also wait for the rows prefetched before them)
  struct Seg {
    int32_t id[KPW];
    int32_t orow;
    int32_t pos;
    int32_t in; // -1 for a position of the map, 0 past its end
  };
  constexpr int kYv = SHY ? 1 : NB;
  struct Dat {
    v4u xv[KPW];
    v4u yv[kYv];
  };
  auto load_seg = [&](int sg, Seg &S) {
    const int64_t p = 64 * (rg + static_cast<int64_t>(sg) * ranges) + lane;
    const int32_t in = opaque(static_cast<int32_t>((p - n_out) >> 63));
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int32_t keep = in & kval[j];
      S.id[j] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
          rn, pick(static_cast<uint32_t>((kk[j] * n_out + p) * 4), keep), 0, 0));
    }
    // loaded also without an order (from an empty buffer, as zero): a load
    // behind a branch leaves the in-order waits for the rows prefetched
    // before it uncounted, and the loop head then waits for every load
    S.orow = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
        ro, pick(static_cast<uint32_t>(p * 4), in & has_order), 0, 0));
    S.pos = static_cast<int32_t>(p);
    S.in = in;
  };
  auto prep = [&](Seg &S, uint64_t (&live)[KPW]) {
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int32_t r = S.id[j] | ~(S.in & kval[j]);
      live[j] = __ballot(r >= 0);
      S.id[j] = static_cast<int32_t>(pick(static_cast<uint32_t>((r * cin + ci0) * 2), opaque(~(r >> 31))));
    }
    const int32_t r = (S.orow & has_order) | (S.pos & ~has_order) | ~S.in;
    S.orow = static_cast<int32_t>(pick(static_cast<uint32_t>((r * cout + co0) * 2), opaque(~(r >> 31))));
  };
  // step s (0 or 1) of a segment: lane l takes position 32s + l/2's offsets
  auto load_dat = [&](const Seg &S, int s, Dat &D) {
    const int src = (32 * s + (lane >> 1)) * 4;
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const uint32_t o = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, S.id[j])) + 16 * half;
      D.xv[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0);
    }
    if constexpr (SHY) {
      // lane L: position 8w + L/(2NB) of the step, 16-byte chunk L%(2NB) of
      // its row; lanes past 16*NB load nothing
      const int q = 8 * wv + lane / (2 * NB);
      const uint32_t o =
          static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute((32 * s + (q & 31)) * 4, S.orow)) +
          16 * (lane % (2 * NB));
      D.yv[0] = __builtin_amdgcn_raw_buffer_load_b128(
          ry, pick(o, opaque(lane < 16 * NB ? -1 : 0)), 0, 0);
    } else {
      const uint32_t o =
          static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, S.orow)) + 16 * NB * half;
#pragma unroll
      for (int q = 0; q < NB; ++q)
        D.yv[q] = __builtin_amdgcn_raw_buffer_load_b128(ry, o + 16 * q, 0, 0);
    }
  };

  v4f acc[KPW][NB];
#pragma unroll
  for (int j = 0; j < KPW; ++j)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      acc[j][nb] = v4f{0.f, 0.f, 0.f, 0.f};
  __bf16 *const wy = sY[SHY ? 0 : wv];
  __bf16 *const wx = sX[wv];
  // SHY: publish step data D's dY chunk into buffer buf for every wave
  auto share_dy = [&](const Dat &D, int buf) {
    if (lane < 16 * NB)
      *reinterpret_cast<v4u *>(sY[buf] + (8 * wv + lane / (2 * NB)) * LDY +
                               8 * (lane % (2 * NB))) = D.yv[0];
    __syncthreads();
  };
  const int prow = 8 * g + i16 / 4, pcol = 4 * (i16 % 4);
  auto operand = [&](const __bf16 *base, int ld, int col) {
    const v4s lo = ds_read_tr16(base + prow * ld + col + pcol);
    const v4s hi = ds_read_tr16(base + (prow + 4) * ld + col + pcol);
    return __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };
  auto compute = [&](const Dat &D, const uint64_t (&live)[KPW], int s, int buf) {
    bool any = false;
#pragma unroll
    for (int j = 0; j < KPW; ++j)
      any |= ((live[j] >> (32 * s)) & 0xffffffffull) != 0;
    if (!any)
      return; // wave-uniform
    const __bf16 *ty = wy;
    if constexpr (SHY) {
      ty = sY[buf];
    } else {
#pragma unroll
      for (int q = 0; q < NB; ++q)
        *reinterpret_cast<v4u *>(wy + (lane >> 1) * LDY + 8 * NB * half + 8 * q) = D.yv[q];
    }
    v8bf b[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      b[nb] = operand(ty, LDY, 16 * nb);
#pragma unroll
    for (int j = 0; j < KPW; ++j)
      if ((live[j] >> (32 * s)) & 0xffffffffull) { // wave-uniform
        *reinterpret_cast<v4u *>(wx + (lane >> 1) * LDX + 8 * half) = D.xv[j];
        const v8bf a = operand(wx, LDX, 0);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[j][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[nb], acc[j][nb], 0, 0, 0);
      }
  };

  // segments in two slots, steps in two row slots (two steps a segment)
  Seg SA, SB;
  uint64_t LA[KPW], LB[KPW];
  Dat DA, DB;
  // SHY: step 0 of a segment uses buffer 0, step 1 buffer 1; each step's dY
  // is published before the next step's loads are issued
  auto run_seg = [&](Seg &S, const uint64_t (&LS)[KPW], Seg &N, uint64_t (&LN)[KPW],
                     int next_load) {
    if constexpr (SHY)
      share_dy(DA, 0);
    load_dat(S, 1, DB);
    compute(DA, LS, 0, 0);
    if constexpr (SHY)
      share_dy(DB, 1);
    prep(N, LN);
    load_dat(N, 0, DA);
    compute(DB, LS, 1, 1);
    load_seg(next_load, S);
  };
  load_seg(0, SA);
  load_seg(1, SB);
  prep(SA, LA);
  load_dat(SA, 0, DA);
  for (int sg = 0; sg < segs; sg += 2) {
    run_seg(SA, LA, SB, LB, sg + 2);
    run_seg(SB, LB, SA, LA, sg + 3);
  }

  // lane holds D[4g+e][i16] of block nb: dW[k][ci0 + 4g + e][co0 + 16nb + i16]
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    if (kk[j] >= K)
      continue;
    float *dst = partial + ((static_cast<int64_t>(rg) * K + kk[j]) * cin + ci0 + 4 * g) * cout +
                 co0 + i16;
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        dst[static_cast<int64_t>(e) * cout + 16 * nb] = acc[j][nb][e];
  }
}

// bf16 dW from the neighbour table with the X rows shared by the workgroup:
// position-stationary like conv_dw_pos_bf16_kernel, but a workgroup owns a
// 64-channel input chunk c0 (wave w takes channels c0 + 16w .. c0 + 16w + 15),
// 16*NB output channels co0 and KPW consecutive offsets that all four waves
// multiply. At each step (32 positions) wave w loads the whole 128-byte rows
// (the chunk) of positions 8w .. 8w+7 under every offset of the group (lane
// l: position 8w + l/8, 16-byte piece l%8), so a load instruction touches 8
// cache lines where the per-wave 16-channel slices of conv_dw_pos_bf16_kernel
// touch 32, and the dY rows of the same positions; both go to one of two LDS
// buffers that one barrier per step publishes (a wave at step t writes the
// buffer of step t-2, which every wave finished before the barrier of step
// t-1). Each wave then reads its 16-channel column of the rows transposed
// (ds_read_b64_tr_b16) as the MFMA's A operand. The offsets' live masks are
// the same in every wave (the same positions), so a step without a
// neighbour under an offset skips that offset's LDS stores and MFMAs in the
// whole workgroup. Indices, out-of-range buffer loads, segments dealt to
// ranges and the partial slots [range][k][cin][cout] are as in
// conv_dw_pos_bf16_kernel.
template <int NB, int KPW, int WAVES>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(WAVES))) void
conv_dw_shx_bf16_kernel(const __bf16 *__restrict__ x, int64_t n_in, int cin,
                        const __bf16 *__restrict__ gy, int cout, const int32_t *__restrict__ nbr,
                        const int32_t *__restrict__ out_order, int64_t n_out, int K, int ranges,
                        int c_chunks, int co_tiles, float *__restrict__ partial) {
  static_assert(NB * 16 <= 64, "a dY row piece per lane: at most 64 output channels");
  constexpr int LDX = 64 + 8, LDY = 16 * NB + 8; // LDS row strides (elements)
  __shared__ __align__(16) __bf16 sX[2][KPW][32 * LDX];
  __shared__ __align__(16) __bf16 sY[2][32 * LDY];
  const int groups = (K + KPW - 1) / KPW;
  const int units = c_chunks * co_tiles * groups;
  const int r8 = ranges / kXcds;
  const int xcd = static_cast<int>(blockIdx.x % kXcds), m = static_cast<int>(blockIdx.x / kXcds);
  const int rg = xcd * r8 + m / units;
  int u = m % units;
  const int grp = u % groups;
  u /= groups;
  const int c0 = (u % c_chunks) * 64, co0 = (u / c_chunks) * (16 * NB);

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const int ci0 = c0 + 16 * wv; // this wave's input channels
  const int64_t total = (n_out + 63) / 64;
  const int segs = static_cast<int>((total + 2LL * ranges - 1) / (2LL * ranges)) * 2;
  int kk[KPW], kval[KPW];
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    kk[j] = grp * KPW + j;
    kval[j] = opaque(kk[j] < K ? -1 : 0);
  }

  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, n_in * cin * 2);
  const __amdgpu_buffer_rsrc_t ry = buf_rsrc(gy, n_out * cout * 2);
  const __amdgpu_buffer_rsrc_t rn = buf_rsrc(nbr, static_cast<int64_t>(K) * n_out * 4);
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(out_order, out_order ? n_out * 4 : 0);
  const int32_t has_order = opaque(out_order ? -1 : 0);
  auto pick = [](uint32_t off, int32_t keep) {
    return (off & static_cast<uint32_t>(keep)) | (kBufOob & ~static_cast<uint32_t>(keep));
  };

  // raw loads: the masks for absent entries (-1) are applied in prep, a
  // segment later, so that nothing waits for these loads when they are issued
  // (an in-order wait would also wait for the rows prefetched before them)
  struct Seg {
    int32_t id[KPW];
    int32_t orow;
    int32_t pos;
    int32_t in; // -1 for a position of the map, 0 past its end
  };
  struct Dat {
    v4u xv[KPW];
    v4u yv;
  };
  // a segment's indices, lane l holding position 64*sg + l
  auto load_seg = [&](int sg, Seg &S) {
    const int64_t p = 64 * (rg + static_cast<int64_t>(sg) * ranges) + lane;
    const int32_t in = opaque(static_cast<int32_t>((p - n_out) >> 63));
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int32_t keep = in & kval[j];
      S.id[j] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
          rn, pick(static_cast<uint32_t>((kk[j] * n_out + p) * 4), keep), 0, 0));
    }
    // loaded also without an order (from an empty buffer, as zero): a load
    // behind a branch leaves the in-order waits for the rows prefetched
    // before it uncounted, and the loop head then waits for every load
    S.orow = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(
        ro, pick(static_cast<uint32_t>(p * 4), in & has_order), 0, 0));
    S.pos = static_cast<int32_t>(p);
    S.in = in;
  };
  // live masks, then byte offsets of the rows' chunk (out of range if absent)
  auto prep = [&](Seg &S, uint64_t (&live)[KPW]) {
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int32_t r = S.id[j] | ~(S.in & kval[j]);
      live[j] = __ballot(r >= 0);
      S.id[j] = static_cast<int32_t>(pick(static_cast<uint32_t>((r * cin + c0) * 2), opaque(~(r >> 31))));
    }
    const int32_t r = (S.orow & has_order) | (S.pos & ~has_order) | ~S.in;
    S.orow = static_cast<int32_t>(pick(static_cast<uint32_t>((r * cout + co0) * 2), opaque(~(r >> 31))));
  };
  // step s (0 or 1) of a segment: lane l loads position 32s + 8*wv + l/8,
  // 16-byte piece l%8 of its X rows (64 channels) and of its dY row (16*NB
  // channels: lanes past 16*NB load nothing)
  const int prow8 = 8 * wv + (lane >> 3);
  auto load_dat = [&](const Seg &S, int s, Dat &D) {
    const int src = (32 * s + prow8) * 4;
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const uint32_t o = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, S.id[j])) + 16 * (lane & 7);
      D.xv[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0);
    }
    const int q = 8 * wv + lane / (2 * NB);
    const uint32_t o =
        static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute((32 * s + (q & 31)) * 4, S.orow)) +
        16 * (lane % (2 * NB));
    D.yv = __builtin_amdgcn_raw_buffer_load_b128(ry, pick(o, opaque(lane < 16 * NB ? -1 : 0)), 0,
                                                 0);
  };
  auto step_live = [](const uint64_t (&live)[KPW], int j, int s) {
    return ((live[j] >> (32 * s)) & 0xffffffffull) != 0;
  };
  // publish step data D into buffer buf (offsets without a neighbour in the
  // step are not stored: nobody reads them)
  auto share = [&](const Dat &D, const uint64_t (&live)[KPW], int s, int buf) {
#pragma unroll
    for (int j = 0; j < KPW; ++j)
      if (step_live(live, j, s)) // uniform
        *reinterpret_cast<v4u *>(sX[buf][j] + prow8 * LDX + 8 * (lane & 7)) = D.xv[j];
    if (lane < 16 * NB)
      *reinterpret_cast<v4u *>(sY[buf] + (8 * wv + lane / (2 * NB)) * LDY +
                               8 * (lane % (2 * NB))) = D.yv;
    __syncthreads();
  };

  v4f acc[KPW][NB];
#pragma unroll
  for (int j = 0; j < KPW; ++j)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      acc[j][nb] = v4f{0.f, 0.f, 0.f, 0.f};
  const int prow = 8 * g + i16 / 4, pcol = 4 * (i16 % 4);
  auto operand = [&](const __bf16 *base, int ld, int col) {
    const v4s lo = ds_read_tr16(base + prow * ld + col + pcol);
    const v4s hi = ds_read_tr16(base + (prow + 4) * ld + col + pcol);
    return __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };
  auto compute = [&](const uint64_t (&live)[KPW], int s, int buf) {
    bool any = false;
#pragma unroll
    for (int j = 0; j < KPW; ++j)
      any |= step_live(live, j, s);
    if (!any)
      return; // uniform
    v8bf b[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      b[nb] = operand(sY[buf], LDY, 16 * nb);
#pragma unroll
    for (int j = 0; j < KPW; ++j)
      if (step_live(live, j, s)) { // uniform
        const v8bf a = operand(sX[buf][j], LDX, 16 * wv);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[j][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[nb], acc[j][nb], 0, 0, 0);
      }
  };

  // segments in two slots; step 0 of a segment uses buffer 0, step 1
  // buffer 1; each step's rows are published before the next step's loads
  // are issued
  Seg SA, SB;
  uint64_t LA[KPW], LB[KPW];
  Dat DA, DB;
  auto run_seg = [&](Seg &S, const uint64_t (&LS)[KPW], Seg &N, uint64_t (&LN)[KPW],
                     int next_load) {
    share(DA, LS, 0, 0);
    load_dat(S, 1, DB);
    compute(LS, 0, 0);
    share(DB, LS, 1, 1);
    prep(N, LN);
    load_dat(N, 0, DA);
    compute(LS, 1, 1);
    load_seg(next_load, S);
  };
  load_seg(0, SA);
  load_seg(1, SB);
  prep(SA, LA);
  load_dat(SA, 0, DA);
  for (int sg = 0; sg < segs; sg += 2) {
    run_seg(SA, LA, SB, LB, sg + 2);
    run_seg(SB, LB, SA, LA, sg + 3);
  }

  // lane holds D[4g+e][i16] of block nb: dW[k][ci0 + 4g + e][co0 + 16nb + i16]
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    if (kk[j] >= K)
      continue;
    float *dst = partial + ((static_cast<int64_t>(rg) * K + kk[j]) * cin + ci0 + 4 * g) * cout +
                 co0 + i16;
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        dst[static_cast<int64_t>(e) * cout + 16 * nb] = acc[j][nb][e];
  }
}

// Any-shape fallback: one lane per dW element, looping over its pairs.
template <typename T>
__global__ __launch_bounds__(kThreads) void conv_dw_generic_kernel(
    const T *__restrict__ x, int cin, const T *__restrict__ gy, int cout,
    const int64_t *__restrict__ kofs, int K, const int32_t *__restrict__ in_rows,
    const int32_t *__restrict__ out_rows, float *__restrict__ dw) {
  const int64_t t = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  if (t >= static_cast<int64_t>(K) * cin * cout)
    return;
  const int k = static_cast<int>(t / (static_cast<int64_t>(cin) * cout));
  const int ci = static_cast<int>((t / cout) % cin);
  const int co = static_cast<int>(t % cout);
  float acc = 0.f;
  for (int64_t p = kofs[k]; p < kofs[k + 1]; ++p)
    acc += to_f32(x[static_cast<int64_t>(in_rows[p]) * cin + ci]) *
           to_f32(gy[static_cast<int64_t>(out_rows[p]) * cout + co]);
  dw[t] += acc;
}

__global__ __launch_bounds__(kThreads) void zero_f32_kernel(float *p, int64_t n) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  if (i < n)
    p[i] = 0.f;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void cast_from_f32_kernel(const float *src,
                                                                 T *dst, int64_t n) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  if (i < n)
    dst[i] = from_f32<T>(src[i]);
}

// ------------------------------------------------------------------ host

// Bias gradient: dbias[c] = sum over rows of grad_y[r][c] in fp32. Each of
// kBiasChunks workgroups sums a contiguous run of rows (thread t: column
// t % C, row lane t / C, rows in order, row lanes combined in LDS in lane
// order) into partial[chunk][c]; the final kernel adds the chunks in order:
// deterministic.
constexpr int kBiasChunks = 256;
template <typename T>
__global__ __launch_bounds__(kThreads) void colsum_partial_kernel(const T *__restrict__ gy,
                                                                  int64_t n, int C, int64_t rpc,
                                                                  float *__restrict__ partial) {
  __shared__ float red[kThreads];
  const int64_t r0 = blockIdx.x * rpc, r1 = min(n, r0 + rpc);
  const int lanes = C <= kThreads ? kThreads / C : 1;
  for (int c0 = 0; c0 < C; c0 += kThreads) {
    const int t = threadIdx.x;
    const int c = c0 + (C <= kThreads ? t % C : t);
    const int rl = C <= kThreads ? t / C : 0;
    float acc = 0.f;
    if (rl < lanes && c < C)
      for (int64_t r = r0 + rl; r < r1; r += lanes)
        acc += to_f32(gy[r * C + c]);
    red[t] = acc;
    __syncthreads();
    if (rl == 0 && c < C) {
      float v = red[t];
      for (int l = 1; l < lanes; ++l)
        v += red[l * C + t];
      partial[static_cast<int64_t>(blockIdx.x) * C + c] = v;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(kThreads) void colsum_final_kernel(const float *__restrict__ partial,
                                                                int chunks, int C,
                                                                float *__restrict__ out) {
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= C)
    return;
  float v = 0.f;
  for (int b = 0; b < chunks; ++b)
    v += partial[static_cast<int64_t>(b) * C + c];
  out[c] = v;
}

static bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

template <typename T> constexpr int kChOf = Mfma<T>::kCh;
template <typename T> constexpr bool kIsF32 = std::is_same<T, float>::value;

template <typename T, int NT, int RG, int CSUB, int WAVES, int G>
static void launch_os(const T *x, int cred, const T *wt, int credw, int ncols,
                      const float *bias, const int32_t *nbr, int64_t n_rows,
                      int K, const int32_t *order, T *y, int splits, float *partial,
                      hipStream_t s) {
  constexpr int ROWS = kWaves * RG * 16;
  dim3 grid(static_cast<unsigned>(xcd_grid(ceil_div(n_rows, ROWS))), ncols / NT, splits);
  float *part = splits > 1 ? partial : nullptr;
  bool padded = false;
  if constexpr (!kIsF32<T> && CSUB == 1) {
    if (credw != cred) { // bf16 reduction padded to the MFMA width
      hipLaunchKernelGGL((conv_os_kernel<T, NT, RG, CSUB, G, WAVES, true, true>), grid,
                         dim3(kThreads), 0, s, x, cred, wt, credw, ncols, bias, nbr, n_rows, K,
                         order, y, part);
      padded = true;
    }
  }
  // Reduction widths of one, two or four channel chunks are compile-time
  // constants in the kernel: the stage's offset and chunk then come from
  // shifts instead of integer divisions, and the row addressing folds
  // (config 2 bf16 forward 108 -> 96 us).
  constexpr int CCH = CSUB * kChOf<T>;
  if (!padded) {
    if (cred == credw && credw == CCH)
      hipLaunchKernelGGL((conv_os_kernel<T, NT, RG, CSUB, G, WAVES, true, false, CCH>), grid,
                         dim3(kThreads), 0, s, x, cred, wt, credw, ncols, bias, nbr, n_rows, K,
                         order, y, part);
    else if (cred == credw && credw == 2 * CCH)
      hipLaunchKernelGGL((conv_os_kernel<T, NT, RG, CSUB, G, WAVES, true, false, 2 * CCH>), grid,
                         dim3(kThreads), 0, s, x, cred, wt, credw, ncols, bias, nbr, n_rows, K,
                         order, y, part);
    else if (cred == credw && credw == 4 * CCH)
      hipLaunchKernelGGL((conv_os_kernel<T, NT, RG, CSUB, G, WAVES, true, false, 4 * CCH>), grid,
                         dim3(kThreads), 0, s, x, cred, wt, credw, ncols, bias, nbr, n_rows, K,
                         order, y, part);
    else
      hipLaunchKernelGGL((conv_os_kernel<T, NT, RG, CSUB, G, WAVES>), grid, dim3(kThreads), 0, s,
                         x, cred, wt, credw, ncols, bias, nbr, n_rows, K, order, y, part);
  }
  if (splits > 1) {
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL((conv_os_reduce_kernel<T>),
                       dim3(static_cast<unsigned>(ceil_div(n_rows * (ncols / 4), kThreads))),
                       dim3(kThreads), 0, s, partial, splits, n_rows, ncols, bias, order, y);
  }
}

// Launch shape, measured on MI355X. One 16-row group per wave (64 rows per
// workgroup: more workgroups in flight hide the gather latency better than
// more rows per wave) and the widest channel chunk the reduction width
// allows. fp32 (config 2, C64): a register budget for 6 waves per SIMD at
// 64 columns with quad-order gathers (dX 393-396 us against 404-406 at the
// 8-wave budget, which fits in 60 registers; the 8-wave budget led before the
// quad-order gathers), one stage per barrier. bf16 (config-5 stages): 8 waves per SIMD and one stage
// per barrier at 64 columns; 128-column tiles (4 waves per SIMD, 2 stages
// per barrier) for 128 and 256 channels; 4 stages per barrier for 32-channel
// chunks (6 waves per SIMD at 64 columns, where 8 do not fit the registers).
template <typename T> static int os_nt(int ncols) {
  if (!kIsF32<T> && ncols % 128 == 0)
    return 128;
  return ncols % 64 == 0 ? 64 : (ncols % 32 == 0 ? 32 : 16);
}

template <typename T, int NT, int CSUB>
static void launch_shape(const T *x, int cred, const T *wt, int credw, int ncols, const float *bias,
                         const int32_t *nbr, int64_t n_rows, int K, const int32_t *order, T *y,
                         int splits, float *partial, hipStream_t s) {
  // bf16 at 64 columns and 64 reduction channels: two row groups per wave
  // share each weight fragment read (config 2, quad-order gathers: 104 us
  // against 117 with one group per wave)
  constexpr int RG = !kIsF32<T> && NT == 64 && CSUB == 2 ? 2 : 1;
  constexpr int W = kIsF32<T> ? (NT == 64 ? 6 : 8)
                              : (NT >= 128 || RG == 2 ? 4 : (CSUB == 1 && NT >= 64 ? 6 : 8));
  constexpr int G = kIsF32<T> ? 1 : (NT >= 128 || RG == 2 ? 2 : (CSUB == 1 ? 4 : 1));
  launch_os<T, NT, RG, CSUB, W, G>(x, cred, wt, credw, ncols, bias, nbr, n_rows, K, order, y,
                                   splits, partial, s);
}

template <typename T, int NT>
static void pick_csub(const T *x, int cred, const T *wt, int credw, int ncols,
                      const float *bias, const int32_t *nbr, int64_t n_rows,
                      int K, const int32_t *order, T *y, int splits, float *partial,
                      hipStream_t s) {
  constexpr int CH = kChOf<T>;
  if constexpr (kIsF32<T>) {
    if (cred % (4 * CH) == 0) {
      launch_shape<T, NT, 4>(x, cred, wt, credw, ncols, bias, nbr, n_rows, K, order, y, splits,
                             partial, s);
      return;
    }
  }
  if (cred == credw && cred % (2 * CH) == 0)
    launch_shape<T, NT, 2>(x, cred, wt, credw, ncols, bias, nbr, n_rows, K, order, y, splits,
                           partial, s);
  else
    launch_shape<T, NT, 1>(x, cred, wt, credw, ncols, bias, nbr, n_rows, K, order, y, splits,
                           partial, s);
}

// Whether run_os takes the MFMA kernel for these operands (a padded bf16
// reduction needs 16-byte aligned rows of 16 channels at least).
template <typename T>
static bool os_fast(const T *x, int cred, const T *wt, int credw, int ncols, int K) {
  const bool red = cred == credw ? cred % kChOf<T> == 0
                                 : (!kIsF32<T> && credw == cred + 16 && credw % kChOf<T> == 0);
  return red && ncols % 16 == 0 && K <= 32 * kMaskWords && aligned16(x) && aligned16(wt);
}

// Splits of the offset axis for the MFMA kernel: a map with few rows and
// wide channels gives too few workgroups to hide the gathers (one per CU
// for 9k rows at 256 channels), so the (offset, channel chunk) stages are
// shared among up to 8 workgroups per tile, aiming at ~640 workgroups
// (measured on the config-5 stages), each keeping at least 4 stages on
// average. 1 = no split. The tiles counted are the fast kernel's (bf16
// 128-column tiles hold kWideRG row groups per wave).
template <typename T> static int os_splits(int64_t n_rows, int cred, int ncols, int K) {
  if (n_rows <= 0 || ncols % 16 != 0)
    return 1;
  const int nt = os_nt<T>(ncols);
  const int rows = kWaves * 16 * (!kIsF32<T> && nt >= 128 ? kWideRG : 1);
  const int64_t blocks = ceil_div(n_rows, rows) * (ncols / nt);
  const int64_t stages = static_cast<int64_t>(K) * std::max(1, cred / 64);
  const int64_t want = (640 + blocks / 2) / blocks; // nearest
  return static_cast<int>(
      std::max<int64_t>(1, std::min<int64_t>({8, want, std::max<int64_t>(1, stages / 4)})));
}

// Floats of split partial sums run_os needs (0 without a split).
template <typename T>
static size_t os_partial_floats(int64_t n_rows, int cred, int ncols, int K) {
  const int sp = os_splits<T>(n_rows, cred, ncols, K);
  return sp > 1 ? static_cast<size_t>(sp) * n_rows * ncols : 0;
}

// One conv_os_lds_kernel launch; the split form is built for bf16 only (fp32
// splits stay on conv_os_kernel).
template <typename T, int NT, int RG, int CSUB, int G, int WAVES, int CW, int KQ, bool REGK>
static void launch_os_lds_cw(dim3 grid, bool split, const T *x, int64_t n_x, const T *wt,
                             const int32_t *wperm, int ncols, const float *bias,
                             const int32_t *nbr, int64_t n_rows, int K, const int32_t *order,
                             T *y, float *partial, hipStream_t s, bool wtr = false) {
  if constexpr (!kIsF32<T>) {
    if constexpr (NT >= 128) {
      if (wtr && !split) { // weights as [K][CW][ncols] (not transposed)
        hipLaunchKernelGGL(
            (conv_os_lds_kernel<T, NT, RG, CSUB, G, WAVES, CW, KQ, false, REGK, true>), grid,
            dim3(kThreads), 0, s, x, n_x, wt, wperm, ncols, bias, nbr, n_rows, K, order, y,
            nullptr);
        return;
      }
    }
    if (split) {
      hipLaunchKernelGGL((conv_os_lds_kernel<T, NT, RG, CSUB, G, WAVES, CW, KQ, true, REGK>), grid,
                         dim3(kThreads), 0, s, x, n_x, wt, wperm, ncols, bias, nbr, n_rows, K,
                         order, y, partial);
      return;
    }
  }
  hipLaunchKernelGGL((conv_os_lds_kernel<T, NT, RG, CSUB, G, WAVES, CW, KQ, false, REGK>), grid,
                     dim3(kThreads), 0, s, x, n_x, wt, wperm, ncols, bias, nbr, n_rows, K, order,
                     y, nullptr);
}

// conv_os_lds_kernel launches: the reduction width as one, two or four
// chunks; false where it is none of these (or an fp32 split).
template <typename T, int NT, int RG, int CSUB, int G, int WAVES, int KQ, bool REGK = false>
static bool launch_os_lds(const T *x, int64_t n_x, int cred, const T *wt, const int32_t *wperm,
                          int ncols, const float *bias, const int32_t *nbr, int64_t n_rows,
                          int K, const int32_t *order, T *y, int splits, float *partial,
                          hipStream_t s, bool wtr = false) {
  constexpr int CCH = CSUB * kChOf<T>;
  constexpr int ROWS = kWaves * RG * 16;
  const bool sp = splits > 1;
  if ((kIsF32<T> && sp) || (wtr && (kIsF32<T> || sp || NT < 128)))
    return false; // untransposed weights: bf16 128-column tiles without a split only
  const dim3 grid(static_cast<unsigned>(xcd_grid(ceil_div(n_rows, ROWS))), ncols / NT, splits);
  if (cred == CCH)
    launch_os_lds_cw<T, NT, RG, CSUB, G, WAVES, CCH, KQ, REGK>(grid, sp, x, n_x, wt, wperm, ncols, bias,
                                                         nbr, n_rows, K, order, y, partial, s, wtr);
  else if (cred == 2 * CCH)
    launch_os_lds_cw<T, NT, RG, CSUB, G, WAVES, 2 * CCH, KQ, REGK>(grid, sp, x, n_x, wt, wperm, ncols,
                                                             bias, nbr, n_rows, K, order, y,
                                                             partial, s, wtr);
  else if (cred == 4 * CCH)
    launch_os_lds_cw<T, NT, RG, CSUB, G, WAVES, 4 * CCH, KQ, REGK>(grid, sp, x, n_x, wt, wperm, ncols,
                                                             bias, nbr, n_rows, K, order, y,
                                                             partial, s, wtr);
  else
    return false;
  if (splits > 1) {
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL((conv_os_reduce_kernel<T>),
                       dim3(static_cast<unsigned>(ceil_div(n_rows * (ncols / 4), kThreads))),
                       dim3(kThreads), 0, s, partial, splits, n_rows, ncols, bias, order, y);
  }
  return true;
}

// Launch shape of conv_os_lds_kernel, measured on MI355X: bf16 at 64 columns
// and 64-channel chunks takes two row groups per wave and one stage per
// barrier (6 waves per SIMD; config 2 forward 76 us against 78 with two
// stages per barrier and 80 with three row groups); bf16 128-column tiles
// (layers of 128 or 256 channels) take two row groups and one stage per
// barrier too, which halves the weight slices each row re-stages (config 5
// stage 4, 9,342 rows at C256: forward 118.8 -> 102.8 us, dX 106.5 -> 91.9
// us with the splits os_splits then picks; stage 3, 43,444 rows at C128:
// 81.0 -> 78.9 and 75.1 -> 74.5 us), or one row group where the offset axis
// is not split (config 3's 87,195 coarse rows at C64->128, forward and the
// transposed layer's dX: 32.9 -> 31.1 and 29.3 -> 27.8 us per call); fp32 at 32 columns with
// 24 index slots (stencils of 33 to 96 offsets) holds the indices in
// registers and takes two stages per barrier at 5 waves per SIMD (config 4
// forward 305 -> 256 us; the LDS indices with two stages: 309 us; register
// indices in config 2's shapes: fp32 314 against 312 us, bf16 80 against
// 75); the other shapes keep conv_os_kernel's.
template <typename T, int NT, int CSUB, int KQ>
static bool os_lds_shape(const T *x, int64_t n_x, int cred, const T *wt, const int32_t *wperm,
                         int ncols, const float *bias, const int32_t *nbr, int64_t n_rows, int K,
                         const int32_t *order, T *y, int splits, float *partial, hipStream_t s,
                         bool wtr = false) {
  if (kIsF32<T> && wtr)
    return false; // untransposed weights: bf16 only
  if constexpr (kIsF32<T> && NT == 32 && KQ == 24) {
    return launch_os_lds<T, NT, 1, CSUB, 2, 5, KQ, true>(
        x, n_x, cred, wt, wperm, ncols, bias, nbr, n_rows, K, order, y, splits, partial, s);
  } else if constexpr (kIsF32<T>) {
    // tiles of at most 32 columns: four 16-channel chunks per barrier group
    // (config 1, 51,554 rows: a workgroup's stages are a chain of memory
    // round trips; forward C16->32 39.2 -> 35.2 us at G = 4, dX C32->16 39.6
    // -> 36.0 us at G = 2, per call)
    constexpr int G = NT <= 32 ? 4 / CSUB : 1;
    return launch_os_lds<T, NT, 1, CSUB, G, NT == 64 ? 6 : 8, KQ>(
        x, n_x, cred, wt, wperm, ncols, bias, nbr, n_rows, K, order, y, splits, partial, s);
  } else if constexpr (NT < 128) {
    // untransposed weights only in 128-column tiles: the narrower shapes run
    // at 6-8 waves per SIMD, where the transposed reads' registers spill
    // (config 2 bf16 forward 92-99 -> 103 us)
    if (wtr)
      return false;
    if constexpr (NT == 64 && CSUB == 2)
      return launch_os_lds<T, NT, 2, CSUB, 1, 6, KQ>(x, n_x, cred, wt, wperm, ncols, bias, nbr,
                                                     n_rows, K, order, y, splits, partial, s);
    constexpr int W = CSUB == 1 && NT >= 64 ? 6 : 8;
    constexpr int G = CSUB == 1 ? 4 : 1;
    return launch_os_lds<T, NT, 1, CSUB, G, W, KQ>(x, n_x, cred, wt, wperm, ncols, bias, nbr,
                                                   n_rows, K, order, y, splits, partial, s);
  } else { // bf16 128-column tiles: 4 waves per SIMD, one stage per barrier group
    if (splits <= 1) // without a split: one row group, twice the workgroups
      return launch_os_lds<T, NT, 1, CSUB, 1, 4, KQ>(x, n_x, cred, wt, wperm, ncols, bias, nbr,
                                                     n_rows, K, order, y, splits, partial, s, wtr);
    // untransposed weights only without a split (config 3's C64->128 forward
    // 33.4 -> 29.0 us per call; config 5's split stages gained nothing)
    if (wtr)
      return false;
    return launch_os_lds<T, NT, kWideRG, CSUB, 1, 4, KQ>(x, n_x, cred, wt, wperm, ncols, bias,
                                                         nbr, n_rows, K, order, y, splits, partial,
                                                         s);
  }
}

template <typename T, int NT, int KQ>
static bool os_lds_csub(const T *x, int64_t n_x, int cred, const T *wt, const int32_t *wperm,
                        int ncols, const float *bias, const int32_t *nbr, int64_t n_rows, int K,
                        const int32_t *order, T *y, int splits, float *partial,
                        hipStream_t s, bool wtr = false) {
  constexpr int CH = kChOf<T>;
  if constexpr (kIsF32<T>) {
    if (cred % (4 * CH) == 0)
      return os_lds_shape<T, NT, 4, KQ>(x, n_x, cred, wt, wperm, ncols, bias, nbr, n_rows, K,
                                        order, y, splits, partial, s, wtr);
  }
  if (cred % (2 * CH) == 0)
    return os_lds_shape<T, NT, 2, KQ>(x, n_x, cred, wt, wperm, ncols, bias, nbr, n_rows, K, order,
                                      y, splits, partial, s, wtr);
  return os_lds_shape<T, NT, 1, KQ>(x, n_x, cred, wt, wperm, ncols, bias, nbr, n_rows, K, order,
                                    y, splits, partial, s, wtr);
}

template <typename T, int KQ>
static bool run_os_lds_nt(const T *x, int64_t n_x, int cred, const T *wt, const int32_t *wperm,
                          int ncols, const float *bias, const int32_t *nbr, int64_t n_rows,
                          int K, const int32_t *order, T *y, int splits, float *partial,
                          hipStream_t s, bool wtr = false) {
  const int nt = os_nt<T>(ncols);
  if constexpr (!kIsF32<T>) {
    if (nt == 128)
      return os_lds_csub<T, 128, KQ>(x, n_x, cred, wt, wperm, ncols, bias, nbr, n_rows, K, order,
                                     y, splits, partial, s, wtr);
  }
  if (nt == 64)
    return os_lds_csub<T, 64, KQ>(x, n_x, cred, wt, wperm, ncols, bias, nbr, n_rows, K, order, y,
                                  splits, partial, s, wtr);
  if (nt == 32)
    return os_lds_csub<T, 32, KQ>(x, n_x, cred, wt, wperm, ncols, bias, nbr, n_rows, K, order, y,
                                  splits, partial, s, wtr);
  return os_lds_csub<T, 16, KQ>(x, n_x, cred, wt, wperm, ncols, bias, nbr, n_rows, K, order, y,
                                splits, partial, s, wtr);
}

// The fast forward/dX kernel where it applies: at most 96 offsets, no split,
// unpadded reductions of one, two or four chunks and inputs that 32-bit
// buffer offsets reach. Returns whether it launched.
template <typename T>
static bool run_os_lds(const T *x, int64_t n_x, int cred, const T *wt, const int32_t *wperm,
                       int credw, int ncols, const float *bias, const int32_t *nbr,
                       int64_t n_rows, int K, const int32_t *order, T *y, int splits,
                       float *partial, hipStream_t s, bool wtr = false) {
  if (K > 96 || cred != credw || n_x < 1 || !os_fast(x, cred, wt, credw, ncols, K) ||
      n_x * cred * static_cast<int64_t>(sizeof(T)) > kBufMaxBytes)
    return false;
  if (K > 32)
    return run_os_lds_nt<T, 24>(x, n_x, cred, wt, wperm, ncols, bias, nbr, n_rows, K, order, y,
                                splits, partial, s, wtr);
  return run_os_lds_nt<T, 8>(x, n_x, cred, wt, wperm, ncols, bias, nbr, n_rows, K, order, y,
                             splits, partial, s, wtr);
}

// Shape of the resident-weight kernel (conv_fr_kernel) for a bf16 map: the
// widest column slice whose weights fit in LDS, taken only when one slice
// covers every column of a large map. Each further slice would gather every
// row again, which costs more than the per-stage weight reloads of
// conv_os_kernel save; measured on MI355X (quad-order gathers both):
// config-5 stage 1 (808k rows, C32->32, 27 offsets) 105 us against 133, its
// 2^3 downsample (C32->64) 28 against 33; config 2 (C64, two slices) 117
// against 104; config 3's maps (40k-85k rows) 19-20 against 16-19. Where the
// LDS-indexed kernel applies it is faster still, so run_os tries that first
// and this kernel serves the maps it does not take.
constexpr int kCus = 256;
constexpr int kFrLdsBytes = 160 * 1024;
constexpr int kFrMaxSlices = 1;
constexpr int64_t kFrMinRows = 131072;
// waves per workgroup and stages in flight, within the register budget
template <int NT, int KS> constexpr int kFrWaves = NT <= 32 && KS == 1 ? 12 : 8;
template <int KS> constexpr int kFrDepth = KS == 4 ? 2 : 4;
static int fr_kq(int K) { return K <= 8 ? 2 : (K <= 28 ? 8 : 0); }
static int64_t fr_lds(int kq, int nt, int cred) {
  return static_cast<int64_t>(kq == 2 ? 8 : 28) * nt * (cred + 8) * 2;
}
static int fr_nt(int cred, int ncols, int K, int64_t n_x, int64_t n_rows) {
  const int kq = fr_kq(K);
  if (kq == 0 || (cred != 32 && cred != 64 && cred != 128) || ncols % 16 != 0)
    return 0;
  if (n_rows < kFrMinRows || n_x * cred * 2 > kBufMaxBytes ||
      static_cast<int64_t>(K) * n_rows * 4 > kBufMaxBytes)
    return 0;
  for (int nt : {128, 64, 32, 16}) {
    if (ncols % nt != 0 || fr_lds(kq, nt, cred) > kFrLdsBytes)
      continue;
    return ncols / nt <= kFrMaxSlices ? nt : 0;
  }
  return 0;
}

// Grid of the resident-weight kernel: at most one workgroup per CU (its LDS
// allows no more), fewer for a small map (each wave at least one unit),
// always a multiple of 8 (one share per XCD) whose per-XCD count the slices
// divide.
static int fr_grid(int64_t n_rows, int slices, int waves) {
  const int64_t per_xcd = ceil_div(ceil_div(n_rows, 32) * slices, int64_t(kXcds) * waves);
  const int64_t q = std::min<int64_t>(kCus / kXcds, ceil_div(per_xcd, slices) * slices);
  return static_cast<int>(kXcds * std::max<int64_t>(q, slices));
}

template <int NT, int KS, int KQ>
static void launch_fr(const __bf16 *x, int64_t n_x, const __bf16 *wt, int ncols,
                      const float *bias, const int32_t *nbr, int64_t n_rows, int K,
                      const int32_t *order, __bf16 *y, hipStream_t s) {
  constexpr int W = kFrWaves<NT, KS>;
  hipLaunchKernelGGL((conv_fr_kernel<NT, KS, KQ, kFrDepth<KS>, W>),
                     dim3(fr_grid(n_rows, ncols / NT, W)), dim3(W * kWave), 0, s, x, n_x, wt,
                     ncols, bias, nbr, n_rows, K, order, y);
}

// Runs the resident-weight kernel where fr_nt takes the map; false if not.
static bool run_fr(const __bf16 *x, int64_t n_x, int cred, const __bf16 *wt, int ncols,
                   const float *bias, const int32_t *nbr, int64_t n_rows, int K,
                   const int32_t *order, __bf16 *y, hipStream_t s) {
  if (!aligned16(x) || !aligned16(wt))
    return false;
  const int nt = fr_nt(cred, ncols, K, n_x, n_rows);
  if (nt == 0)
    return false;
  auto go = [&](auto ntc, auto ksc, auto kqc) {
    launch_fr<decltype(ntc)::value, decltype(ksc)::value, decltype(kqc)::value>(
        x, n_x, wt, ncols, bias, nbr, n_rows, K, order, y, s);
  };
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  using I8 = std::integral_constant<int, 8>;
  using N16 = std::integral_constant<int, 16>;
  using N32 = std::integral_constant<int, 32>;
  using N64 = std::integral_constant<int, 64>;
  using N128 = std::integral_constant<int, 128>;
  if (fr_kq(K) == 8) {
    if (cred == 32)
      nt == 64 ? go(N64{}, I1{}, I8{}) : nt == 32 ? go(N32{}, I1{}, I8{}) : go(N16{}, I1{}, I8{});
    else if (cred == 64)
      nt == 32 ? go(N32{}, I2{}, I8{}) : go(N16{}, I2{}, I8{});
    else
      go(N16{}, I4{}, I8{});
  } else {
    if (cred == 32)
      nt == 128  ? go(N128{}, I1{}, I2{})
      : nt == 64 ? go(N64{}, I1{}, I2{})
      : nt == 32 ? go(N32{}, I1{}, I2{})
                 : go(N16{}, I1{}, I2{});
    else if (cred == 64)
      nt == 128  ? go(N128{}, I2{}, I2{})
      : nt == 64 ? go(N64{}, I2{}, I2{})
      : nt == 32 ? go(N32{}, I2{}, I2{})
                 : go(N16{}, I2{}, I2{});
    else
      nt == 64 ? go(N64{}, I4{}, I2{}) : nt == 32 ? go(N32{}, I4{}, I2{}) : go(N16{}, I4{}, I2{});
  }
  RHIP_LAUNCH_CHECK();
  return true;
}

// Weight slices reordered for a table whose row k multiplies slice
// perm[k]: dst[k][r][c] = src[perm[k]][r][c] ([K][rows][cols], same layout).
template <typename T>
__global__ __launch_bounds__(kThreads) void permute_w_kernel(const T *__restrict__ src,
                                                             const int32_t *__restrict__ perm,
                                                             int K, int64_t per,
                                                             T *__restrict__ dst) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  if (i >= K * per)
    return;
  const int64_t k = i / per;
  dst[i] = src[static_cast<int64_t>(perm[k]) * per + i % per];
}

// y[order[j]] = sum_k x[nbr[k][j]] @ W'[wperm[k]] with W'[k][c][n] = wt[k][n][c]
// (wperm NULL: the identity); x has n_x rows. partial: os_partial_floats(...)
// floats, or null to run without a split. credw: row stride of wt (cred, or
// the padded reduction of red_width). The LDS-indexed kernel reads slice
// wperm[k] itself; for the other kernels the slices are first copied in
// table order to wperm_buf (K * ncols * credw elements; required with wperm).
template <typename T>
static void run_os(const T *x, int64_t n_x, int cred, const T *wt, int credw, int ncols,
                   const float *bias, const int32_t *nbr, int64_t n_rows, int K,
                   const int32_t *order, T *y, float *partial, hipStream_t s,
                   bool resident = true, const int32_t *wperm = nullptr,
                   T *wperm_buf = nullptr) {
  if (n_rows == 0)
    return;
  // the LDS-indexed kernel first: it beats the resident-weight kernel on the
  // maps that took that one (config 5 step 6.01 -> 5.86 ms), and with an
  // offset-axis split it takes the small coarse maps as well
  const int splits = partial ? os_splits<T>(n_rows, credw, ncols, K) : 1;
  if (run_os_lds(x, n_x, cred, wt, wperm, credw, ncols, bias, nbr, n_rows, K, order, y, splits,
                 partial, s)) {
    RHIP_LAUNCH_CHECK();
    return;
  }
  if (wperm != nullptr) {
    if (wperm_buf == nullptr)
      throw Error(RHIP_ERR_INVALID, "a weight permutation needs the workspace for this shape");
    const int64_t per = static_cast<int64_t>(ncols) * credw;
    hipLaunchKernelGGL((permute_w_kernel<T>), dim3(static_cast<unsigned>(ceil_div(K * per,
                                                                                   kThreads))),
                       dim3(kThreads), 0, s, wt, wperm, K, per, wperm_buf);
    RHIP_LAUNCH_CHECK();
    wt = wperm_buf;
  }
  if constexpr (!kIsF32<T>) {
    if (resident && cred == credw &&
        run_fr(x, n_x, cred, wt, ncols, bias, nbr, n_rows, K, order, y, s))
      return;
  }
  if (!os_fast(x, cred, wt, credw, ncols, K)) {
    hipLaunchKernelGGL((conv_os_generic_kernel<T>), dim3(ceil_div(n_rows * ncols, kThreads)),
                       dim3(kThreads), 0, s, x, cred, wt, credw, ncols, bias, nbr, n_rows, K,
                       order, y);
  } else if (os_nt<T>(ncols) == 128) {
    if constexpr (!kIsF32<T>)
      pick_csub<T, 128>(x, cred, wt, credw, ncols, bias, nbr, n_rows, K, order, y, splits,
                        partial, s);
  } else if (ncols % 64 == 0) {
    pick_csub<T, 64>(x, cred, wt, credw, ncols, bias, nbr, n_rows, K, order, y, splits, partial,
                     s);
  } else if (ncols % 32 == 0) {
    pick_csub<T, 32>(x, cred, wt, credw, ncols, bias, nbr, n_rows, K, order, y, splits, partial,
                     s);
  } else {
    pick_csub<T, 16>(x, cred, wt, credw, ncols, bias, nbr, n_rows, K, order, y, splits, partial,
                     s);
  }
  RHIP_LAUNCH_CHECK();
}

// Launch plan of the dW kernel: pairs per workgroup, chunks per offset and
// channel tiles, shared by the workspace query and the launch.
struct DwPlan {
  int va = 1, vb = 1, tiles = 1;
  int64_t ppb = 1, chunks = 1;
  bool fast = false;
  // bf16 tiles of tm x tn channels on conv_dw_pairs_bf16_kernel (else
  // conv_dw_kernel's 16va x 16vb tiles)
  bool pw = false;
  int tm = 0, tn = 0;
  size_t partial_floats() const {
    const size_t tile = pw ? static_cast<size_t>(tm) * tn : static_cast<size_t>(16 * va) * (16 * vb);
    return fast ? static_cast<size_t>(chunks) * tiles * tile : 0;
  }
};

static int dw_width(int c) { return c % 64 == 0 ? 4 : (c % 32 == 0 ? 2 : 1); }

// wgs: busy workgroups to aim for over the whole map (0 = the measured best
// on MI355X: 2048 for fp32, where the MFMA work dominates, 512 for bf16).
// conv_dw_pairs_bf16_kernel's shape: 64 x 64 tiles, rows kDwPairsD steps
// ahead per wave, kDwPairsWaves waves per SIMD, so 256 * kDwPairsWaves
// workgroups fill the chip once. Measured on MI355X, config 3's two dW passes
// (kernel alone, 2^3 stride-2 down C64->128 and up C128->64): 13.9 us each,
// against 16.4-17.5 for 64 x 128 / 128 x 64 tiles (each row staged once, but
// 256 registers), 14.9 with 2048-pair ranges on a grid sized by the row
// counts (most workgroups idle), 15.5 at 3 waves per SIMD, 15.9-18.7 with
// rows 2 to 4 steps ahead, and 36.3 for conv_dw_kernel.
constexpr int kDwPairsD = 1, kDwPairsWaves = 2;
static DwPlan dw_plan(int32_t dtype, int cin, int cout, int K, int64_t n_pairs, int64_t n_in,
                      int64_t n_out, int wgs = 0) {
  DwPlan p;
  const int64_t max_pk = std::min(n_in, n_out); // an offset pairs each row at most once
  if (dtype == RHIP_BF16 && n_pairs > 0 && cin % 64 == 0 && cout % 64 == 0 &&
      n_in * cin * 2 <= kBufMaxBytes && n_out * cout * 2 <= kBufMaxBytes) {
    p.fast = p.pw = true;
    p.tm = p.tn = 64;
    p.tiles = (cin / p.tm) * (cout / p.tn);
    // ranges per (offset, tile): about `target` workgroups over the map, at
    // least 128 pairs (one step per wave) per range on average
    const int64_t target = wgs > 0 ? wgs : 256 * kDwPairsWaves;
    const int64_t per_k = ceil_div(n_pairs, static_cast<int64_t>(K));
    p.chunks = std::max<int64_t>(1, std::min(target / (static_cast<int64_t>(K) * p.tiles),
                                             ceil_div(per_k, kWaves * 32)));
    p.ppb = 0; // the kernel splits each offset's pairs itself
    return p;
  }
  if (wgs <= 0)
    wgs = dtype == RHIP_F32 ? 2048 : 512;
  const int VE = dtype == RHIP_F32 ? 4 : 8;
  p.fast = n_pairs > 0 && cin % 16 == 0 && cout % 16 == 0 && cin % VE == 0 && cout % VE == 0;
  if (!p.fast)
    return p;
  p.va = dw_width(cin);
  p.vb = dw_width(cout);
  p.tiles = (cin / (16 * p.va)) * (cout / (16 * p.vb));
  const int64_t CP = kWaves * (dtype == RHIP_F32 ? DwShape<float>::kPairsPerWave
                                                 : DwShape<__bf16>::kPairsPerWave);
  // ~wgs busy workgroups over the whole map, at least 4 chunks each
  const int64_t target = std::max<int64_t>(1, wgs / p.tiles);
  p.ppb = std::max<int64_t>(4 * CP, ceil_div(n_pairs, target));
  p.ppb = ceil_div(p.ppb, CP) * CP;
  p.chunks = std::max<int64_t>(1, ceil_div(max_pk, p.ppb));
  return p;
}

// Register budget of the dW kernel (measured on MI355X, config 2): 4 waves
// per SIMD for fp32; bf16 gains nothing from a tighter budget.
template <typename T> constexpr int kDwWaves = std::is_same<T, float>::value ? 3 : 1;

template <typename T, int VA, int VB, bool DB = false>
static void launch_dw(const T *x, int cin, const T *gy, int cout, const int64_t *kofs, int K,
                      const int32_t *in_rows, const int32_t *out_rows, const DwPlan &p,
                      float *partial, hipStream_t s) {
  dim3 grid(static_cast<unsigned>(p.chunks), K, p.tiles);
  hipLaunchKernelGGL((conv_dw_kernel<T, VA, VB, DB, kDwWaves<T>>), grid, dim3(kThreads), 0, s, x,
                     cin, gy,
                     cout, kofs, in_rows, out_rows, p.ppb, partial);
}

template <typename T, int VA>
static void pick_dw_b(const T *x, int cin, const T *gy, int cout, const int64_t *kofs, int K,
                      const int32_t *in_rows, const int32_t *out_rows, const DwPlan &p,
                      float *partial, hipStream_t s) {
  if (p.vb == 4)
    launch_dw<T, VA, 4>(x, cin, gy, cout, kofs, K, in_rows, out_rows, p, partial, s);
  else if (p.vb == 2)
    launch_dw<T, VA, 2>(x, cin, gy, cout, kofs, K, in_rows, out_rows, p, partial, s);
  else
    launch_dw<T, VA, 1>(x, cin, gy, cout, kofs, K, in_rows, out_rows, p, partial, s);
}

// dw [K, cin, cout] in T (fully overwritten). `partial` holds
// plan.partial_floats() * K floats; `acc` (generic path) K*cin*cout floats.
template <typename T>
static void run_dw(const T *x, int64_t n_in, int cin, const T *gy, int64_t n_out, int cout,
                   const int64_t *kofs, int K, const int32_t *in_rows, const int32_t *out_rows,
                   int64_t n_pairs, const DwPlan &p, float *partial, float *acc, T *dw,
                   hipStream_t s) {
  const int64_t nw = static_cast<int64_t>(K) * cin * cout;
  if constexpr (!std::is_same<T, float>::value) {
    // the plan checked the shape and the buffer sizes; rows that are not
    // 16-byte aligned take the any-shape path below
    if (p.pw && aligned16(x) && aligned16(gy)) {
      const dim3 grid(static_cast<unsigned>(p.chunks), K, p.tiles);
      hipLaunchKernelGGL((conv_dw_pairs_bf16_kernel<64, 64, kDwPairsD, kDwPairsWaves>), grid,
                         dim3(kThreads), 0, s, x, n_in, cin, gy, n_out, cout, kofs, in_rows,
                         out_rows, static_cast<int>(p.chunks), partial);
      RHIP_LAUNCH_CHECK();
      const dim3 rgrid(static_cast<unsigned>(p.tm * p.tn / (4 * kWave)), K, p.tiles);
      hipLaunchKernelGGL((conv_dw_reduce_kernel<T>), rgrid, dim3(kThreads), 0, s, partial, kofs,
                         int64_t(0), static_cast<int>(p.chunks), p.tiles, cout / p.tn, p.tm, p.tn,
                         cin, cout, 1, dw);
      RHIP_LAUNCH_CHECK();
      return;
    }
  }
  if (p.fast && !p.pw && aligned16(x) && aligned16(gy)) {
    if (p.va == 4)
      pick_dw_b<T, 4>(x, cin, gy, cout, kofs, K, in_rows, out_rows, p, partial, s);
    else if (p.va == 2)
      pick_dw_b<T, 2>(x, cin, gy, cout, kofs, K, in_rows, out_rows, p, partial, s);
    else
      pick_dw_b<T, 1>(x, cin, gy, cout, kofs, K, in_rows, out_rows, p, partial, s);
    RHIP_LAUNCH_CHECK();
    const int TM = 16 * p.va, TN = 16 * p.vb;
    dim3 grid(static_cast<unsigned>(TM * TN / (4 * kWave)), K, p.tiles);
    hipLaunchKernelGGL((conv_dw_reduce_kernel<T>), grid, dim3(kThreads), 0, s, partial, kofs,
                       p.ppb, static_cast<int>(p.chunks), p.tiles, cout / TN, TM, TN, cin, cout, 0,
                       dw);
    RHIP_LAUNCH_CHECK();
    return;
  }
  // any shape: one lane per dW element into an fp32 accumulator
  hipLaunchKernelGGL(zero_f32_kernel, dim3(ceil_div(nw, kThreads)), dim3(kThreads), 0, s, acc,
                     nw);
  RHIP_LAUNCH_CHECK();
  if (n_pairs > 0) {
    hipLaunchKernelGGL((conv_dw_generic_kernel<T>), dim3(ceil_div(nw, kThreads)),
                       dim3(kThreads), 0, s, x, cin, gy, cout, kofs, K, in_rows, out_rows, acc);
    RHIP_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL((cast_from_f32_kernel<T>), dim3(ceil_div(nw, kThreads)), dim3(kThreads), 0,
                     s, acc, dw, nw);
  RHIP_LAUNCH_CHECK();
}

static void check_dtype(int32_t dtype) {
  if (dtype != RHIP_F32 && dtype != RHIP_BF16)
    throw Error(RHIP_ERR_UNSUPPORTED, "dtype must be RHIP_F32 or RHIP_BF16");
}

// dW from the neighbour table (conv_dw_rows_kernel): bf16 with 16 or 32
// input and output channels. Measured on MI355X (config-5 stage 1, 808k
// rows, C32): 3 offsets per wave, 256 row blocks, each XCD running all
// offset groups of its row blocks back to back (183 us against the
// pair-list kernel's 397; 225 us with the groups spread over the XCDs).
constexpr int kDwRowsKW = 3;
constexpr int kDwRowsBlocks = 256;

// fp32 dW from the neighbour table (conv_dw_pos_kernel): 16-channel input
// slices, 64 output channels per tile (32 where C_out is not a multiple of
// 64), 7 offsets per wave (all 27 of a 3^3 stencil in one workgroup), rows
// loaded 3 steps ahead; 2 waves per SIMD for 64-channel tiles, 3 for
// 32-channel ones. The grid is one round of resident workgroups.
// Measured on MI355X, kernel + reduce: config 2 (410k rows, C64, 128
// ranges) 419 us against the pair-list kernel's 578 (contiguous ranges
// instead of dealt segments 481, 4 offsets per wave 434-444); config 4
// (233k rows, 81 offsets, C32->32, 128 ranges) 217 against 242; config 1
// (52k rows, C16->32, 256 ranges) 35 against 46. Stencils of fewer than 20
// offsets would leave most of 7 offset slots per wave empty (config 3's 2^3
// transposed map, C128->64: 118 us against the pair list's 71); stencils of
// at most 8 offsets take 2 offsets per wave instead (config 3, kernel +
// reduce against the pair list: fp32 down 45 us against 70, up 58 against
// 71; bf16 down 32 against 48, up 45 against 52), and 9 to 19 offsets stay
// on the pair list.
constexpr int kDwPosKPW = 7;
constexpr int kDwPosKPWSmall = 2;
constexpr int kDwPosSlots = 4;
constexpr int kDwPosMinK = 20;
constexpr int kDwPosMaxKSmall = 4 * kDwPosKPWSmall;
static int dw_pos_kpw(int K) { return K <= kDwPosMaxKSmall ? kDwPosKPWSmall : kDwPosKPW; }

template <int VB> constexpr int kDwPosWaves = VB == 4 ? 2 : 3;

// bf16 (conv_dw_pos_bf16_kernel): 64-channel output tiles (32 where C_out
// is not a multiple of 64), 7 offsets per wave, 2 waves per SIMD, the same
// one-round grid. Measured on MI355X, kernel + reduce against the pair-list
// kernel: config 2 (C64, 410k rows, 128 ranges) 157 us against 230; config
// 5's stages C64 (191k rows) 91 against 141, C128 (43k rows, 32 ranges) 89
// against 142, C256 (9k rows, 8 ranges) 93 against 146; its 808k-row stage
// against the narrow-channel conv_dw_rows_kernel: C32->32 139 us against
// 189, C16->32 94 against 161 (3 waves per SIMD spills: 200 and 153).
// 64-channel tiles with 7 offsets per wave share each step's dY tile through
// LDS (a quarter loaded by each wave, one barrier per step): config 2
// 145-147 us against 162-168 alternating on one box, config 5 6.22 ms a step
// against 6.37; with 32-channel tiles (half of each wave's fill lanes idle)
// or 2 offsets per wave the barrier costs more than it saves (config 1
// 42 us against 37, config 3's 2^3 down map 32 against 27), so those load
// their own dY.
static bool dw_pos_supported(int32_t dtype, int cin, int cout, int K, int64_t n_in,
                             int64_t n_out) {
  const int64_t s = dtype == RHIP_F32 ? 4 : 2;
  return (K >= kDwPosMinK || K <= kDwPosMaxKSmall) && cin % 16 == 0 && cout % 32 == 0 &&
         n_in * cin * s <= kBufMaxBytes && n_out * cout * s <= kBufMaxBytes &&
         static_cast<int64_t>(K) * n_out * 4 <= kBufMaxBytes;
}

static bool dw_narrow_bf16(int32_t dtype, int cin, int cout) {
  return dtype == RHIP_BF16 && (cin == 16 || cin == 32) && (cout == 16 || cout == 32);
}

static bool dw_rows_supported(int32_t dtype, int cin, int cout, int K, int64_t n_in,
                              int64_t n_out) {
  return dw_narrow_bf16(dtype, cin, cout) || dw_pos_supported(dtype, cin, cout, K, n_in, n_out);
}

// Ranges of the neighbour-table kernels: a multiple of 8 (one share per
// XCD), one round of resident workgroups (256 CUs x the waves per SIMD:
// each workgroup puts one wave on every SIMD of its CU), at most
// kDwRowsBlocks (the partial slots of the workspace), at least min_segs
// segments of 64 positions each (2 for fp32: config 1's dW 44.7 -> 39.0 us
// per call against 4; 16 for bf16, whose small maps lose more to partial
// slots than they gain from a full round: config 3's down map 32 us at 32
// ranges, 38 at 128).
static int dw_ranges_for(int units, int waves, int64_t n_out, int min_segs) {
  int64_t r = std::max<int64_t>(kXcds, (256 * waves / units) / kXcds * kXcds);
  const int64_t segs = ceil_div(std::max<int64_t>(n_out, 1), 64);
  r = std::min<int64_t>(r, std::max<int64_t>(kXcds, segs / min_segs / kXcds * kXcds));
  return static_cast<int>(std::min<int64_t>(r, kDwRowsBlocks));
}
static int dw_pos_ranges(int K, int cin, int cout, int vb, int waves, int64_t n_out,
                         int min_segs) {
  const int groups = static_cast<int>(ceil_div(K, kWaves * dw_pos_kpw(K)));
  return dw_ranges_for((cin / 16) * (cout / (16 * vb)) * groups, waves, n_out, min_segs);
}

// The shared-X bf16 kernel (conv_dw_shx_bf16_kernel): 64-channel input
// chunks, 64 output channels and 7 offsets per workgroup, 2 waves per SIMD.
// Measured on MI355X, config 2 dW (kernel + reduce): 133-138 us against
// conv_dw_pos_bf16_kernel's 136-142, alternating in one process. Stencils of
// at most 8 offsets and channel counts that are not multiples of 64 keep
// conv_dw_pos_bf16_kernel.
constexpr int kDwShxKPW = 7;
static bool dw_shx_bf16(int K, int cin, int cout) {
  return K > kDwPosMaxKSmall && cin % 64 == 0 && cout % 64 == 0;
}

// Ranges of conv_dw_pos_bf16_kernel (or conv_dw_shx_bf16_kernel) and
// conv_dw_pos_kernel for a shape (the workspace query and the launches share
// them).
static int dw_pos_bf16_ranges(int K, int cin, int cout, int64_t n_out) {
  if (dw_shx_bf16(K, cin, cout))
    return dw_ranges_for((cin / 64) * (cout / 64) * static_cast<int>(ceil_div(K, kDwShxKPW)), 2,
                         n_out, 16);
  const int waves = K <= kDwPosMaxKSmall ? 4 : 2;
  return dw_pos_ranges(K, cin, cout, cout % 64 == 0 ? 4 : 2, waves, n_out, 16);
}
// fp32 dW on 64-channel input and output tiles (conv_dw_pos64_kernel):
// 2 offsets per wave, 2-wave workgroups (groups of 4 offsets: 28 offset
// slots for a 3^3 stencil), 2 waves per SIMD, the one-round grid. Measured
// on MI355X, config 2 (C64, 410k rows, 144 ranges), kernel + reduce per
// call: 381-385 us against 437-440 for conv_dw_pos_kernel's 16-channel
// slices in the same run; with ds_bpermute index moves instead of the DPP
// row broadcasts 390-399; with groups of consecutive offsets 473; 4-wave
// workgroups 432; one offset per wave at 3 or 4 waves per SIMD 489-576
// (each offset re-reads the dY rows). Without the multiplies the kernel
// takes 216 us, without the row loads 357: the MFMA issue, not the
// gathers, sets its time.
constexpr int kDwPos64KPW = 2, kDwPos64WPB = 2, kDwPos64Waves = 2;
static bool dw_pos64(int K, int cin, int cout) {
  return K > kDwPosMaxKSmall && cin % 64 == 0 && cout % 64 == 0;
}
static int dw_pos64_ranges(int K, int cin, int cout, int64_t n_out) {
  const int groups = static_cast<int>(ceil_div(K, kDwPos64WPB * kDwPos64KPW));
  // workgroups of WPB waves: 4 / WPB of them put one wave on each SIMD
  return dw_ranges_for((cin / 64) * (cout / 64) * groups, kDwPos64Waves * (kWaves / kDwPos64WPB),
                       n_out, 2);
}

static int dw_pos_f32_ranges(int K, int cin, int cout, int64_t n_out) {
  if (dw_pos64(K, cin, cout))
    return dw_pos64_ranges(K, cin, cout, n_out);
  const int vb = cout % 64 == 0 ? 4 : 2;
  const int waves = K <= kDwPosMaxKSmall ? 3 : (vb == 4 ? kDwPosWaves<4> : kDwPosWaves<2>);
  return dw_pos_ranges(K, cin, cout, vb, waves, n_out, 2);
}

// grad_w [K, cin, cout] (bf16, overwritten) from the neighbour table.
static void run_dw_pos_bf16(const __bf16 *x, int64_t n_in, int cin, const __bf16 *gy,
                            int64_t n_out, int cout, int K, const int32_t *nbr,
                            const int32_t *out_order, float *partial, __bf16 *dw,
                            hipStream_t s) {
  const bool small = K <= kDwPosMaxKSmall;
  const int vb = cout % 64 == 0 ? 4 : 2;
  const int ranges = dw_pos_bf16_ranges(K, cin, cout, n_out);
  const int groups = static_cast<int>(ceil_div(K, kWaves * dw_pos_kpw(K)));
  const int ct = cin / 16, ot = cout / (16 * vb);
  if (n_in > 0 && n_out > 0 && dw_shx_bf16(K, cin, cout)) {
    const int cc = cin / 64, sgroups = static_cast<int>(ceil_div(K, kDwShxKPW));
    hipLaunchKernelGGL((conv_dw_shx_bf16_kernel<4, kDwShxKPW, 2>),
                       dim3(static_cast<unsigned>(ranges * cc * ot * sgroups)), dim3(kThreads), 0,
                       s, x, n_in, cin, gy, cout, nbr, out_order, n_out, K, ranges, cc, ot,
                       partial);
    RHIP_LAUNCH_CHECK();
  } else if (n_in > 0 && n_out > 0) {
    const dim3 grid(static_cast<unsigned>(ranges * ct * ot * groups));
    auto go = [&](auto nb, auto kpw, auto w) {
      hipLaunchKernelGGL((conv_dw_pos_bf16_kernel<decltype(nb)::value, decltype(kpw)::value,
                                                  decltype(w)::value,
                                                  decltype(nb)::value == 4 &&
                                                      decltype(kpw)::value == kDwPosKPW>),
                         grid, dim3(kThreads), 0, s, x, n_in, cin, gy, cout, nbr, out_order, n_out,
                         K, ranges, ct, ot, partial);
    };
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    using IK = std::integral_constant<int, kDwPosKPW>;
    using IKS = std::integral_constant<int, kDwPosKPWSmall>;
    if (small)
      vb == 4 ? go(I4{}, IKS{}, I4{}) : go(I2{}, IKS{}, I4{});
    else
      vb == 4 ? go(I4{}, IK{}, I2{}) : go(I2{}, IK{}, I2{});
    RHIP_LAUNCH_CHECK();
  }
  const int64_t ne = static_cast<int64_t>(K) * cin * cout;
  hipLaunchKernelGGL((conv_dw_rows_reduce_kernel<__bf16>), dim3(static_cast<unsigned>(
                         ceil_div(ne / 4, kWave))), dim3(1024), 0, s, partial,
                     n_in > 0 && n_out > 0 ? ranges : 0, ne, dw);
  RHIP_LAUNCH_CHECK();
}

// grad_w [K, cin, cout] (fp32, overwritten) from the neighbour table.
static void run_dw_pos(const float *x, int64_t n_in, int cin, const float *gy, int64_t n_out,
                       int cout, int K, const int32_t *nbr, const int32_t *out_order,
                       float *partial, float *dw, hipStream_t s) {
  const bool small = K <= kDwPosMaxKSmall;
  const int vb = cout % 64 == 0 ? 4 : 2;
  const int ranges = dw_pos_f32_ranges(K, cin, cout, n_out);
  const int groups = static_cast<int>(ceil_div(K, kWaves * dw_pos_kpw(K)));
  const int ct = cin / 16, ot = cout / (16 * vb);
  if (n_in > 0 && n_out > 0 && dw_pos64(K, cin, cout)) {
    const int g64 = static_cast<int>(ceil_div(K, kDwPos64WPB * kDwPos64KPW));
    const dim3 grid(static_cast<unsigned>(ranges * (cin / 64) * (cout / 64) * g64));
    hipLaunchKernelGGL((conv_dw_pos64_kernel<kDwPos64KPW, kDwPosSlots, kDwPos64Waves, kDwPos64WPB>),
                       grid, dim3(kDwPos64WPB * kWave), 0, s, x, n_in, cin, gy, cout, nbr,
                       out_order, n_out, K, ranges, cin / 64, cout / 64, partial);
    RHIP_LAUNCH_CHECK();
  } else if (n_in > 0 && n_out > 0) {
    const dim3 grid(static_cast<unsigned>(ranges * ct * ot * groups));
    auto go = [&](auto v, auto kpw, auto w) {
      hipLaunchKernelGGL((conv_dw_pos_kernel<decltype(v)::value, decltype(kpw)::value, kDwPosSlots,
                                             decltype(w)::value>),
                         grid, dim3(kThreads), 0, s, x, n_in, cin, gy, cout, nbr, out_order, n_out,
                         K, ranges, ct, ot, partial);
    };
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using I4 = std::integral_constant<int, 4>;
    using IK = std::integral_constant<int, kDwPosKPW>;
    using IKS = std::integral_constant<int, kDwPosKPWSmall>;
    using W4 = std::integral_constant<int, kDwPosWaves<4>>;
    using W2 = std::integral_constant<int, kDwPosWaves<2>>;
    if (small)
      vb == 4 ? go(I4{}, IKS{}, I3{}) : go(I2{}, IKS{}, I3{});
    else
      vb == 4 ? go(I4{}, IK{}, W4{}) : go(I2{}, IK{}, W2{});
    RHIP_LAUNCH_CHECK();
  }
  const int64_t ne = static_cast<int64_t>(K) * cin * cout;
  // without rows every slot sum is empty: zeros
  hipLaunchKernelGGL((conv_dw_rows_reduce_kernel<float>), dim3(static_cast<unsigned>(
                         ceil_div(ne / 4, kWave))), dim3(1024), 0, s, partial,
                     n_in > 0 && n_out > 0 ? ranges : 0, ne, dw);
  RHIP_LAUNCH_CHECK();
}

// Row blocks of conv_dw_rows_kernel for n_out output rows.
static int dw_rows_blocks(int64_t n_out) {
  return static_cast<int>(std::min<int64_t>(kDwRowsBlocks, ceil_div(n_out, kDwRowsSP)));
}

// Partial-slot floats the neighbour-table dW kernels use for this shape
// (0 where rhip_conv_backward_weight_rows does not take it): one fp32 tile
// per range or row block and offset.
static size_t dw_table_floats(int32_t dtype, int cin, int cout, int K, int64_t n_in,
                              int64_t n_out) {
  if (!dw_rows_supported(dtype, cin, cout, K, n_in, n_out) || n_in == 0 || n_out == 0)
    return 0;
  int slots;
  if (dtype == RHIP_F32)
    slots = dw_pos_f32_ranges(K, cin, cout, n_out);
  else if (dw_pos_supported(dtype, cin, cout, K, n_in, n_out))
    slots = dw_pos_bf16_ranges(K, cin, cout, n_out);
  else
    slots = dw_rows_blocks(n_out);
  return static_cast<size_t>(slots) * K * cin * cout;
}

template <int VA, int VB, int KW = kDwRowsKW>
static void launch_dw_rows(const __bf16 *x, const __bf16 *gy, const int32_t *nbr,
                           const int32_t *out_order, int64_t n_out, int K, int64_t rpb,
                           int blocks, float *partial, hipStream_t s, bool xcd_map = false) {
  const int groups = static_cast<int>(ceil_div(K, KW));
  dim3 grid = xcd_map ? dim3(static_cast<unsigned>(ceil_div(blocks, kXcds) * kXcds * groups))
                      : dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(groups));
  hipLaunchKernelGGL((conv_dw_rows_kernel<VA, VB, KW>), grid, dim3(kThreads), 0, s, x, gy, nbr,
                     out_order, n_out, K, rpb, blocks, xcd_map ? 1 : 0, partial);
}

// grad_w [K, cin, cout] (bf16, overwritten) from the neighbour table.
static void run_dw_rows(const __bf16 *x, int64_t n_in, int cin, const __bf16 *gy, int64_t n_out,
                        int cout, int K, const int32_t *nbr, const int32_t *out_order,
                        float *partial, __bf16 *dw, hipStream_t s) {
  int blocks = 0;
  if (n_in > 0 && n_out > 0) { // without rows every slot sum is empty: zeros
    const int64_t rb = dw_rows_blocks(n_out);
    const int64_t rpb = ceil_div(ceil_div(n_out, rb), kDwRowsSP) * kDwRowsSP;
    blocks = static_cast<int>(ceil_div(n_out, rpb));
    auto go = [&](auto va, auto vb) {
      launch_dw_rows<decltype(va)::value, decltype(vb)::value>(x, gy, nbr, out_order, n_out, K,
                                                               rpb, blocks, partial, s, true);
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    if (cin == 32 && cout == 32)
      go(I2{}, I2{});
    else if (cin == 32)
      go(I2{}, I1{});
    else if (cout == 32)
      go(I1{}, I2{});
    else
      go(I1{}, I1{});
    RHIP_LAUNCH_CHECK();
  }
  const int64_t ne = static_cast<int64_t>(K) * cin * cout;
  hipLaunchKernelGGL((conv_dw_rows_reduce_kernel<__bf16>), dim3(static_cast<unsigned>(
                         ceil_div(ne / 4, kWave))), dim3(1024), 0, s, partial, blocks, ne, dw);
  RHIP_LAUNCH_CHECK();
}

// One workspace serves the calls of a layer. Its front holds what the
// forward, the input gradient and the bias gradient use: the transposed
// weights, the split partial sums of the output-stationary kernel and the
// bias gradient's chunk sums. Behind them, used by dW
// only: the per-workgroup partial tiles (sized from the dW plans of this map)
// and the fp32 accumulator of the any-shape kernel. A workspace of
// rhip_conv_forward_workspace_bytes serves the forward and input gradient.
struct ConvWs {
  void *wt = nullptr;
  float *os_partial = nullptr;
  float *bias_partial = nullptr;
  float *partial = nullptr;
  float *acc = nullptr;
};

static ConvWs carve_conv_front(Carve &cv, int32_t K, int32_t cin, int32_t cout, int32_t dtype,
                               int64_t n_in, int64_t n_out) {
  ConvWs w;
  // transposed forward weights, or the padded copy of dX's
  const size_t nw = static_cast<size_t>(K) *
                    std::max(static_cast<size_t>(cout) * red_width(dtype, cin),
                             static_cast<size_t>(cin) * red_width(dtype, cout));
  w.wt = cv.take<char>(nw * (dtype == RHIP_F32 ? 4 : 2));
  const bool f32 = dtype == RHIP_F32;
  auto osp = [&](int64_t n, int cred, int ncols) {
    return f32 ? os_partial_floats<float>(n, cred, ncols, K)
               : os_partial_floats<__bf16>(n, cred, ncols, K);
  };
  w.os_partial = cv.take<float>(std::max<size_t>({1, osp(n_out, cin, cout), osp(n_in, cout, cin)}));
  w.bias_partial = cv.take<float>(static_cast<size_t>(kBiasChunks) * cout);
  return w;
}

static ConvWs carve_conv(Carve &cv, int32_t K, int32_t cin, int32_t cout, int32_t dtype,
                         int64_t n_in, int64_t n_out, const DwPlan &p) {
  ConvWs w = carve_conv_front(cv, K, cin, cout, dtype, n_in, n_out);
  w.partial = cv.take<float>(std::max<size_t>(
      {1, p.partial_floats() * K, dw_table_floats(dtype, cin, cout, K, n_in, n_out)}));
  w.acc = cv.take<float>(static_cast<size_t>(K) * cin * cout);
  return w;
}

// The forward with the transposed weights at wt (K * cin * cout elements) and
// the split partial sums at os_partial (null: no split).
static void conv_forward_into(const void *x, int64_t n_in, int32_t cin, const void *weight,
                              int32_t K, int32_t cout, const float *bias, const int32_t *nbr,
                              const int32_t *out_order, int64_t n_out, void *y, int32_t dtype,
                              void *wt, float *os_partial, hipStream_t stream) {
  // the MFMA path reads W[k] column-wise: stage the [K, cout, credw] copy
  const int credw = red_width(dtype, cin);
  const int64_t nw = static_cast<int64_t>(K) * cout * credw;
  if (dtype == RHIP_F32) {
    float *w = static_cast<float *>(wt);
    hipLaunchKernelGGL((transpose_w_kernel<float>), dim3(ceil_div(nw, kThreads)),
                       dim3(kThreads), 0, stream, static_cast<const float *>(weight), K, cin,
                       cout, credw, w);
    RHIP_LAUNCH_CHECK();
    run_os<float>(static_cast<const float *>(x), n_in, cin, w, credw, cout, bias, nbr, n_out, K,
                  out_order, static_cast<float *>(y), os_partial, stream);
  } else {
    // the LDS-indexed kernel reads W itself where it takes the shape
    // (unpadded reductions, unsplit 128-column tiles): no transposed copy
    if (n_out > 0 && credw == cin) {
      const int splits = os_partial ? os_splits<__bf16>(n_out, cin, cout, K) : 1;
      if (run_os_lds(static_cast<const __bf16 *>(x), n_in, cin,
                     static_cast<const __bf16 *>(weight), nullptr, cin, cout, bias, nbr, n_out, K,
                     out_order, static_cast<__bf16 *>(y), splits, os_partial, stream, true)) {
        RHIP_LAUNCH_CHECK();
        return;
      }
    }
    __bf16 *w = static_cast<__bf16 *>(wt);
    hipLaunchKernelGGL((transpose_w_kernel<__bf16>), dim3(ceil_div(nw, kThreads)),
                       dim3(kThreads), 0, stream, static_cast<const __bf16 *>(weight), K, cin,
                       cout, credw, w);
    RHIP_LAUNCH_CHECK();
    run_os<__bf16>(static_cast<const __bf16 *>(x), n_in, cin, w, credw, cout, bias, nbr, n_out,
                   K, out_order, static_cast<__bf16 *>(y), os_partial, stream);
  }
}

// Device scratch of rhip_conv_forward_noalloc: the transposed weights go
// here instead of into a caller workspace. Every GPU the library runs on
// holds its own copy until the process ends; calls that overlap on one GPU
// share it and race.
constexpr size_t kConvScratchBytes = size_t(8) << 20;
static __device__ __align__(256) char scratch[kConvScratchBytes];

// Per device: the address of `scratch` (the host-side name is only a
// stand-in for it), looked up once with that device current, and the
// stream and completion event of the last call that used it. A call on
// another stream waits for that event on the device (hipStreamWaitEvent),
// so eager calls from several streams take their turns; a call under graph
// capture cannot wait on an event recorded outside the capture, so it is
// refused while another stream's call may still be using the array. Replays
// of a captured graph are not tracked (the caller orders them). The event
// is created once per device at set-up.
struct ScratchSlot {
  void *addr = nullptr;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
  bool used = false;
};
constexpr int kMaxDevices = 64;
static std::mutex scratch_mu;
static ScratchSlot scratch_slots[kMaxDevices];

// Runs f(scratch address) in this device's turn on `stream` (see above).
template <typename F> static void with_device_scratch(hipStream_t stream, F &&f) {
  int dev = 0;
  RHIP_HIP(hipGetDevice(&dev));
  RHIP_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device index out of range");
  std::lock_guard<std::mutex> lock(scratch_mu);
  ScratchSlot &sl = scratch_slots[dev];
  if (sl.addr == nullptr) {
    void *p = nullptr;
    RHIP_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    RHIP_HIP(hipEventCreateWithFlags(&sl.done, hipEventDisableTiming));
    sl.addr = p;
  }
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  RHIP_HIP(hipStreamIsCapturing(stream, &cap));
  const bool capturing = cap != hipStreamCaptureStatusNone;
  if (sl.used && sl.last != stream) {
    if (capturing) {
      const hipError_t q = hipEventQuery(sl.done);
      if (q == hipErrorNotReady)
        throw Error(RHIP_ERR_INVALID,
                    "rhip_conv_forward_noalloc: a call on another stream may still be using "
                    "the device scratch; synchronise it before capturing");
      RHIP_HIP(q);
    } else {
      RHIP_HIP(hipStreamWaitEvent(stream, sl.done, 0));
    }
  }
  f(sl.addr);
  if (!capturing)
    RHIP_HIP(hipEventRecord(sl.done, stream));
  sl.last = stream;
  sl.used = !capturing || sl.used;
}

} // namespace rhip

using namespace rhip;

extern "C" int rhip_conv_workspace_bytes(int32_t K, int32_t cin, int32_t cout,
                                         int32_t dtype, int64_t n_in, int64_t n_out,
                                         int64_t n_pairs, size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(K >= 1 && cin >= 1 && cout >= 1, "sizes must be positive");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0 && n_pairs >= 0, "counts must be >= 0");
    check_dtype(dtype);
    Carve cv(nullptr, 0);
    carve_conv(cv, K, cin, cout, dtype, n_in, n_out,
               dw_plan(dtype, cin, cout, K, n_pairs, n_in, n_out));
    *bytes = cv.used + 256;
  });
}

extern "C" int rhip_conv_forward_workspace_bytes(int32_t K, int32_t cin, int32_t cout,
                                                 int32_t dtype, int64_t n_in, int64_t n_out,
                                                 size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(K >= 1 && cin >= 1 && cout >= 1, "sizes must be positive");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0, "counts must be >= 0");
    check_dtype(dtype);
    Carve cv(nullptr, 0);
    carve_conv_front(cv, K, cin, cout, dtype, n_in, n_out);
    *bytes = cv.used + 256;
  });
}

extern "C" int rhip_conv_forward(const void *x, int64_t n_in, int32_t cin,
                                 const void *weight, int32_t K, int32_t cout,
                                 const float *bias, const int32_t *nbr,
                                 const int32_t *out_order, int64_t n_out, void *y,
                                 int32_t dtype, void *workspace,
                                 size_t workspace_bytes, hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    RHIP_CHECK_ARG(K >= 1 && cin >= 1 && cout >= 1, "sizes must be positive");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0, "row counts must be >= 0");
    if (n_out == 0)
      return;
    RHIP_CHECK_ARG(y && weight && nbr, "y, weight and nbr are required");
    RHIP_CHECK_ARG(n_in == 0 || x != nullptr, "x is null");
    RHIP_CHECK_ARG(workspace != nullptr, "workspace is null");
    // the workspace was sized for this layer's map (n_in, n_out); the dW
    // plan does not change the forward's pieces
    Carve cv(workspace, workspace_bytes);
    const ConvWs w = carve_conv_front(cv, K, cin, cout, dtype, n_in, n_out);
    conv_forward_into(x, n_in, cin, weight, K, cout, bias, nbr, out_order, n_out, y, dtype, w.wt,
                      w.os_partial, stream);
  });
}

extern "C" int rhip_conv_forward_noalloc(const void *x, int64_t n_in, int32_t cin,
                                         const void *weight, int32_t K, int32_t cout,
                                         const float *bias, const int32_t *nbr,
                                         const int32_t *out_order, int64_t n_out, void *y,
                                         int32_t dtype, hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    RHIP_CHECK_ARG(K >= 1 && cin >= 1 && cout >= 1, "sizes must be positive");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0, "row counts must be >= 0");
    const size_t wt_bytes = static_cast<size_t>(K) * cout * red_width(dtype, cin) *
                            (dtype == RHIP_F32 ? 4 : 2);
    if (wt_bytes > kConvScratchBytes)
      throw Error(RHIP_ERR_UNSUPPORTED,
                  "rhip_conv_forward_noalloc: the weights need " + std::to_string(wt_bytes) +
                      " bytes of device scratch, more than its " +
                      std::to_string(kConvScratchBytes) +
                      " (use rhip_conv_forward with a workspace)");
    if (n_out == 0)
      return;
    RHIP_CHECK_ARG(y && weight && nbr, "y, weight and nbr are required");
    RHIP_CHECK_ARG(n_in == 0 || x != nullptr, "x is null");
    // no split of the offset axis: it would need partial sums beyond the scratch
    with_device_scratch(stream, [&](void *scratch_ptr) {
      conv_forward_into(x, n_in, cin, weight, K, cout, bias, nbr, out_order, n_out, y, dtype,
                        scratch_ptr, nullptr, stream);
    });
  });
}

extern "C" int rhip_conv_bias_grad(const void *grad_y, int64_t n_out, int32_t cout,
                                   int32_t dtype, float *grad_bias, void *workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    RHIP_CHECK_ARG(cout >= 1 && n_out >= 0, "bad sizes");
    RHIP_CHECK_ARG(grad_bias != nullptr, "grad_bias is null");
    RHIP_CHECK_ARG(n_out == 0 || grad_y != nullptr, "grad_y is null");
    RHIP_CHECK_ARG(workspace != nullptr, "workspace is null");
    // the chunk sums go to the front of the layer workspace, whose forward
    // part reserves room for them
    Carve cv(workspace, workspace_bytes);
    float *partial = cv.take<float>(static_cast<size_t>(kBiasChunks) * cout);
    const int64_t rpc = ceil_div(std::max<int64_t>(n_out, 1), kBiasChunks);
    const int chunks = static_cast<int>(ceil_div(std::max<int64_t>(n_out, 1), rpc));
    if (dtype == RHIP_F32)
      hipLaunchKernelGGL((colsum_partial_kernel<float>), dim3(chunks), dim3(kThreads), 0, stream,
                         static_cast<const float *>(grad_y), n_out, cout, rpc, partial);
    else
      hipLaunchKernelGGL((colsum_partial_kernel<__bf16>), dim3(chunks), dim3(kThreads), 0, stream,
                         static_cast<const __bf16 *>(grad_y), n_out, cout, rpc, partial);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(colsum_final_kernel, dim3(static_cast<unsigned>(ceil_div(cout, kThreads))),
                       dim3(kThreads), 0, stream, partial, chunks, cout, grad_bias);
    RHIP_LAUNCH_CHECK();
  });
}

extern "C" int rhip_conv_backward_input(const void *grad_y, int64_t n_out,
                                        int32_t cout, const void *weight,
                                        int32_t K, int32_t cin,
                                        const int32_t *nbr_t,
                                        const int32_t *weight_perm,
                                        const int32_t *in_order, int64_t n_in,
                                        void *grad_x, int32_t dtype,
                                        void *workspace, size_t workspace_bytes,
                                        hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    RHIP_CHECK_ARG(K >= 1 && cin >= 1 && cout >= 1, "sizes must be positive");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0, "row counts must be >= 0");
    if (n_in == 0)
      return;
    RHIP_CHECK_ARG(grad_x && weight && nbr_t, "grad_x, weight and nbr_t are required");
    RHIP_CHECK_ARG(n_out == 0 || grad_y != nullptr, "grad_y is null");
    // without a workspace the offset axis is not split, and a reduction the
    // MFMA kernels would pad goes to the one-lane-per-output kernel
    float *os_partial = nullptr;
    const void *wk = weight;
    const int32_t *wperm = weight_perm;
    void *wperm_buf = nullptr;
    int credw = cout;
    if (workspace != nullptr) {
      Carve cv(workspace, workspace_bytes);
      const ConvWs w = carve_conv_front(cv, K, cin, cout, dtype, n_in, n_out);
      os_partial = w.os_partial;
      wperm_buf = w.wt;
      if (red_width(dtype, cout) != cout) { // [K][cin][cout] rows padded to credw
        credw = red_width(dtype, cout);
        const int64_t ne = static_cast<int64_t>(K) * cin * credw;
        hipLaunchKernelGGL((pad_rows_kernel<__bf16>), dim3(ceil_div(ne, kThreads)),
                           dim3(kThreads), 0, stream, static_cast<const __bf16 *>(weight),
                           static_cast<int64_t>(K) * cin, cout, credw, wperm,
                           static_cast<int64_t>(cin), static_cast<__bf16 *>(w.wt));
        RHIP_LAUNCH_CHECK();
        wk = w.wt;
        wperm = nullptr; // applied by the padding copy
      }
    }
    // dX rows gather dY rows; W[k] [cin][cout] is already [n = cin][c = cout].
    if (dtype == RHIP_F32)
      run_os<float>(static_cast<const float *>(grad_y), n_out, cout,
                    static_cast<const float *>(wk), credw, cin, nullptr, nbr_t, n_in, K,
                    in_order, static_cast<float *>(grad_x), os_partial, stream, true, wperm,
                    static_cast<float *>(wperm_buf));
    else
      run_os<__bf16>(static_cast<const __bf16 *>(grad_y), n_out, cout,
                     static_cast<const __bf16 *>(wk), credw, cin, nullptr, nbr_t, n_in, K,
                     in_order, static_cast<__bf16 *>(grad_x), os_partial, stream, true, wperm,
                     static_cast<__bf16 *>(wperm_buf));
  });
}

extern "C" int rhip_conv_backward_weight(
    const void *x, int64_t n_in, int32_t cin, const void *grad_y, int64_t n_out,
    int32_t cout, int32_t K, const int64_t *kmap_offsets, int64_t n_pairs,
    const int32_t *in_rows, const int32_t *out_rows, void *grad_w, int32_t dtype,
    void *workspace, size_t workspace_bytes, hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    RHIP_CHECK_ARG(K >= 1 && cin >= 1 && cout >= 1, "sizes must be positive");
    RHIP_CHECK_ARG(n_pairs >= 0 && n_in >= 0 && n_out >= 0, "bad sizes");
    RHIP_CHECK_ARG(grad_w != nullptr, "grad_w is null");
    RHIP_CHECK_ARG(n_pairs == 0 || (x && grad_y && kmap_offsets && in_rows && out_rows),
                   "x, grad_y, kmap_offsets, in_rows and out_rows are required");
    RHIP_CHECK_ARG(workspace != nullptr, "workspace is null");
    // an offset pairs each input and each output row at most once
    const DwPlan plan = dw_plan(dtype, cin, cout, K, n_pairs, n_in, n_out);
    Carve cv(workspace, workspace_bytes);
    const ConvWs w = carve_conv(cv, K, cin, cout, dtype, n_in, n_out, plan);
    if (dtype == RHIP_F32)
      run_dw<float>(static_cast<const float *>(x), n_in, cin,
                    static_cast<const float *>(grad_y), n_out, cout, kmap_offsets, K, in_rows,
                    out_rows, n_pairs, plan, w.partial, w.acc, static_cast<float *>(grad_w),
                    stream);
    else
      run_dw<__bf16>(static_cast<const __bf16 *>(x), n_in, cin,
                     static_cast<const __bf16 *>(grad_y), n_out, cout, kmap_offsets, K, in_rows,
                     out_rows, n_pairs, plan, w.partial, w.acc, static_cast<__bf16 *>(grad_w),
                     stream);
  });
}

extern "C" int rhip_conv_backward_weight_rows(
    const void *x, int64_t n_in, int32_t cin, const void *grad_y, int64_t n_out,
    int32_t cout, int32_t K, const int32_t *nbr, const int32_t *out_order, void *grad_w,
    int32_t dtype, void *workspace, size_t workspace_bytes, hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    RHIP_CHECK_ARG(K >= 1 && cin >= 1 && cout >= 1, "sizes must be positive");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0, "bad sizes");
    if (!dw_rows_supported(dtype, cin, cout, K, n_in, n_out))
      throw Error(RHIP_ERR_UNSUPPORTED,
                  "rhip_conv_backward_weight_rows: bf16 with 16 or 32 input and output "
                  "channels, or at most 8 or at least 20 offsets with input channels a "
                  "multiple of 16 and output channels a multiple of 32 (use "
                  "rhip_conv_backward_weight)");
    RHIP_CHECK_ARG(grad_w != nullptr, "grad_w is null");
    RHIP_CHECK_ARG(n_in == 0 || n_out == 0 || (x && grad_y && nbr),
                   "x, grad_y and nbr are required");
    RHIP_CHECK_ARG(workspace != nullptr, "workspace is null");
    RHIP_CHECK_ARG(aligned16(x) && aligned16(grad_y), "x and grad_y must be 16-byte aligned");
    Carve cv(workspace, workspace_bytes);
    const ConvWs w = carve_conv(cv, K, cin, cout, dtype, n_in, n_out, DwPlan{});
    if (dtype == RHIP_F32)
      run_dw_pos(static_cast<const float *>(x), n_in, cin, static_cast<const float *>(grad_y),
                 n_out, cout, K, nbr, out_order, w.partial, static_cast<float *>(grad_w), stream);
    else if (dw_pos_supported(dtype, cin, cout, K, n_in, n_out))
      run_dw_pos_bf16(static_cast<const __bf16 *>(x), n_in, cin,
                      static_cast<const __bf16 *>(grad_y), n_out, cout, K, nbr, out_order,
                      w.partial, static_cast<__bf16 *>(grad_w), stream);
    else
      run_dw_rows(static_cast<const __bf16 *>(x), n_in, cin,
                  static_cast<const __bf16 *>(grad_y), n_out, cout, K, nbr, out_order, w.partial,
                  static_cast<__bf16 *>(grad_w), stream);
  });
}

extern "C" int rhip_conv_backward_weight_rows_supported(int32_t dtype, int32_t cin, int32_t cout,
                                                        int32_t K, int64_t n_in,
                                                        int64_t n_out) {
  if ((dtype != RHIP_F32 && dtype != RHIP_BF16) || K < 1 || cin < 1 || cout < 1 || n_in < 0 ||
      n_out < 0)
    return 0;
  return dw_rows_supported(dtype, cin, cout, K, n_in, n_out) ? 1 : 0;
}
