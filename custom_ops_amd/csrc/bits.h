// bits.h — integer helpers shared by device and host code of fa_fwd.hip.
//
// Host-compilable on purpose (plain C++, no HIP types): tests/test_bits.py
// builds a host program from this header with g++ and checks it.
#ifndef MI355_FA_BITS_H
#define MI355_FA_BITS_H

#include <stdint.h>

#if defined(__HIPCC__)
#define MI355_HD __host__ __device__
#else
#define MI355_HD
#endif

namespace mi355fa {

// The 64-bit value whose low and high 32-bit halves are lo and hi. Every
// pointer or address this library rebuilds from two halves (for instance two
// __builtin_amdgcn_readfirstlane results, which are typed int) must go through
// here: the parameters are uint32_t, so a half held as a signed int converts
// without sign extension. Widening an int half directly, ((uint64_t)hi << 32)
// | lo with lo an int >= 2^31, sign-extends lo and sets every upper bit, which
// turns a valid address into a wild one.
MI355_HD inline uint64_t compose_u64(uint32_t lo, uint32_t hi) {
  return ((uint64_t)hi << 32) | (uint64_t)lo;
}

MI355_HD inline uint32_t low_u32(uint64_t x) { return (uint32_t)x; }
MI355_HD inline uint32_t high_u32(uint64_t x) { return (uint32_t)(x >> 32); }

}  // namespace mi355fa

#endif  // MI355_FA_BITS_H
