// Device-wide descending sort of 64-bit keys for the wide top-k path (rocPRIM's LSD radix sort).
#include <rocprim/device/device_radix_sort.hpp>

#include "kls_internal.h"

namespace kls {

hipError_t sort_keys_desc(void* tmp, size_t* bytes, const uint64_t* in, uint64_t* out, size_t n, int end_bit,
                          hipStream_t s) {
    return rocprim::radix_sort_keys_desc(tmp, *bytes, in, out, n, 0u, (unsigned) end_bit, s);
}

}  // namespace kls
