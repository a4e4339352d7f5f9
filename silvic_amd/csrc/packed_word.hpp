// packed_word.hpp - the packed histogram word and its unpacking, shared by the kernels and a host test.
//
// A row's quantized gradient pair is packed as h * 65536 + g (quantize.rs:100-107). Sums of such words, as the LDS
// atomics form them with 32-bit wrap-around, keep g in the low 16 bits as a signed value and h in the high 16 bits
// as an unsigned one, exactly, while the sum of g stays within +-32767 and the sum of h within 0..65535. Unpacking
// subtracts in unsigned arithmetic: a word with h >= 32768 and g < 0 would overflow a signed subtraction.
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#define SROCM_PACKED_HD __host__ __device__ __forceinline__
#else
#define SROCM_PACKED_HD inline
#endif

namespace srocm {

// the signed low half
SROCM_PACKED_HD int32_t packed_g(int32_t word) {
    return static_cast<int16_t>(static_cast<uint16_t>(static_cast<uint32_t>(word)));
}

// the unsigned high half, given the low half g = packed_g(word)
SROCM_PACKED_HD int32_t packed_h(int32_t word, int32_t g) {
    return static_cast<int32_t>((static_cast<uint32_t>(word) - static_cast<uint32_t>(g)) >> 16);
}

}  // namespace srocm
