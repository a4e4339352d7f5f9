// Unpacks every (g, h) with g in -32767..32767 and h in a sweep of 0..65535 that includes the upper half
// (h >= 32768) from the word the 32-bit wrapping sums form, with silvic_amd/csrc/packed_word.hpp built for the host,
// and round-trips every small-unit word through its one-byte code.
// Built with -fsanitize=undefined, so a signed overflow in the unpacking aborts. Prints the mismatches.
#include <cstdio>
#include <cstdint>

#include "../silvic_amd/csrc/packed_word.hpp"

int main() {
    const int32_t hs[] = {0, 1, 2, 4, 255, 256, 32766, 32767, 32768, 32769, 40000, 49151, 65534, 65535};
    long bad = 0, n = 0;
    for (int32_t h : hs) {
        for (int32_t g = -32767; g <= 32767; ++g) {
            // the word a wrapping sum of packed rows leaves: h * 65536 + g modulo 2^32
            const int32_t word = static_cast<int32_t>(static_cast<uint32_t>(h) * 65536u + static_cast<uint32_t>(g));
            const int32_t gq = srocm::packed_g(word);
            const int32_t hq = srocm::packed_h(word, gq);
            bad += (gq != g || hq != h);
            ++n;
        }
    }
    // the one-byte code of a row's word for small units (g in -7..7, h in 0..15) gives the word back
    long code_bad = 0, codes = 0;
    for (int32_t h = 0; h <= srocm::CODE_MAX_H; ++h) {
        for (int32_t g = -srocm::CODE_MAX_G; g <= srocm::CODE_MAX_G; ++g) {
            const int32_t word = h * 65536 + g;
            code_bad += srocm::code_word(srocm::packed_code(word)) != word;
            ++codes;
        }
    }
    std::printf("%ld %ld %ld %ld\n", bad, n, code_bad, codes);
    return 0;
}
