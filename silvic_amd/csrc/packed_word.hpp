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

// A row's packed word in one byte, for units of at most 7 gradient and 15 hessian units (num_grad_quant_bins of at
// most 14): g + 8 in the low four bits, h in the high four. The split steps carry it beside each row id, so that
// the histogram of a built child reads it with the row instead of gathering the packed word.
constexpr int32_t CODE_MAX_G = 7, CODE_MAX_H = 15;
SROCM_PACKED_HD uint8_t packed_code(int32_t word) {
    const int32_t g = packed_g(word);
    return static_cast<uint8_t>((g + 8) | (packed_h(word, g) << 4));
}
SROCM_PACKED_HD int32_t code_word(uint32_t code) {
    return static_cast<int32_t>((code >> 4) << 16) + static_cast<int32_t>(code & 15u) - 8;
}

}  // namespace srocm
