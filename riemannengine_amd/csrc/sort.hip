// Stable device radix sorts used by the hash table (locality order) and the
// kernel map (neighbour-mask order). rocPRIM's default dispatch switches to a
// merge sort below 2^20 items, which ignores the key-bit range; the config
// below keeps the onesweep radix path so that sorts over narrow keys (26-bit
// packed coordinates, 27-bit masks) take only as many passes as the bits need.
#include <rocprim/device/device_radix_sort.hpp>

#include "rhip_internal.hpp"

namespace rhip {

using OnesweepOnly = rocprim::radix_sort_config<rocprim::default_config, rocprim::default_config,
                                                rocprim::default_config, 0>;

template <typename K>
static size_t sort_bytes(int64_t n) {
  size_t bytes = 0;
  const int64_t m = n < 1 ? 1 : n;
  RHIP_HIP(rocprim::radix_sort_pairs<OnesweepOnly>(
      nullptr, bytes, static_cast<const K *>(nullptr), static_cast<K *>(nullptr),
      static_cast<const int32_t *>(nullptr), static_cast<int32_t *>(nullptr),
      static_cast<unsigned int>(m), 0u, static_cast<unsigned>(8 * sizeof(K)), hipStream_t(0)));
  return bytes;
}

template <typename K>
static void sort_run(void *tmp, size_t tmp_bytes, const K *kin, K *kout, const int32_t *vin,
                     int32_t *vout, int64_t n, int end_bit, hipStream_t s) {
  if (n <= 0)
    return;
  size_t need = sort_bytes<K>(n);
  if (tmp_bytes < need)
    throw Error(RHIP_ERR_WORKSPACE, "sort scratch too small");
  end_bit = end_bit < 1 ? 1 : (end_bit > 8 * (int)sizeof(K) ? 8 * (int)sizeof(K) : end_bit);
  RHIP_HIP(rocprim::radix_sort_pairs<OnesweepOnly>(tmp, tmp_bytes, kin, kout, vin, vout,
                                                   static_cast<unsigned int>(n), 0u,
                                                   static_cast<unsigned>(end_bit), s));
}

size_t sort_pairs_u32_bytes(int64_t n) { return sort_bytes<uint32_t>(n); }
size_t sort_pairs_u64_bytes(int64_t n) { return sort_bytes<uint64_t>(n); }

void sort_pairs_u32(void *tmp, size_t tmp_bytes, const uint32_t *kin, uint32_t *kout,
                    const int32_t *vin, int32_t *vout, int64_t n, int end_bit, hipStream_t s) {
  sort_run<uint32_t>(tmp, tmp_bytes, kin, kout, vin, vout, n, end_bit, s);
}

void sort_pairs_u64(void *tmp, size_t tmp_bytes, const uint64_t *kin, uint64_t *kout,
                    const int32_t *vin, int32_t *vout, int64_t n, int end_bit, hipStream_t s) {
  sort_run<uint64_t>(tmp, tmp_bytes, kin, kout, vin, vout, n, end_bit, s);
}

} // namespace rhip
