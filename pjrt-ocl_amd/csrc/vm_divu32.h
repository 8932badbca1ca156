// Division by an invariant 32-bit integer d >= 1 (Granlund and Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994, fig. 4.1):
// for every 32-bit x, x / d = (t + ((x - t) >> s1)) >> s2 with t = umulhi(m, x),
// l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1 = floor(2^(32+l) / d) - 2^32 + 1,
// s1 = min(l, 1), s2 = max(l - 1, 0).  A quotient costs a multiply-high, a
// subtract, an add and two shifts instead of the ~25 instructions of a division
// by a variable; the view index maps of the elementwise tiles divide by the
// same dims for every element of a tile.
//
// Host and device: the kernel includes it with VM_HD = __device__ inline, the
// CPU test of the quotients compiles the same text with g++.
#pragma once
#include <stdint.h>

#ifndef VM_HD
#define VM_HD __device__ __forceinline__
#endif

namespace vm {

struct DivU32 {
  uint32_t d, m, s1, s2;
  VM_HD uint32_t quo(uint32_t x) const {
    const uint32_t t = uint32_t((uint64_t(m) * x) >> 32);
    return (t + ((x - t) >> s1)) >> s2;
  }
};

// The quotient floor(2^(32+l) / d) (<= 2^33) comes from a double division,
// within one of the exact one, and is corrected with the exact remainder: a
// 64-bit integer division is a sequence of a few hundred instructions on the
// GPU, this about thirty.
VM_HD DivU32 div_u32(uint32_t d) {
  const uint32_t l = d > 1 ? 32u - uint32_t(__builtin_clz(d - 1)) : 0u;
  const uint64_t num = uint64_t(1) << (32 + l);
  uint64_t q = uint64_t(double(num) / double(d));
  const int64_t r = int64_t(num - q * d);
  if (r < 0) --q;
  else if (uint64_t(r) >= d) ++q;
  return DivU32{d, uint32_t(q - (uint64_t(1) << 32) + 1), l > 0 ? 1u : 0u, l > 0 ? l - 1 : 0u};
}

}  // namespace vm
