// 64-bit addresses assembled from 32-bit words (plain C++: host and device).
//
// Kernels that keep an address wave-uniform read its two words from the first
// active lane (v_readfirstlane_b32, whose builtin returns int).  Joined as
// signed values, a low word with bit 31 set is sign-extended into the high
// word (s_bfe_i64 in the ISA) and the address becomes 0xffffffff'xxxxxxxx.
// join_words takes both words as unsigned, so no bit of the low word reaches
// the high one.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MMUON_HD __host__ __device__
#else
#define MMUON_HD
#endif

namespace mmuon {

MMUON_HD inline uint64_t join_words(uint32_t lo, uint32_t hi) { return (uint64_t(hi) << 32) | uint64_t(lo); }

MMUON_HD inline uint32_t low_word(uint64_t a) { return uint32_t(a); }
MMUON_HD inline uint32_t high_word(uint64_t a) { return uint32_t(a >> 32); }

}  // namespace mmuon
