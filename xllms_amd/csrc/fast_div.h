// Division of 32-bit indices by run-time constants, for the element-wise
// kernels (activation.hip, paged_kv_append.hip).
#pragma once

#include <stdint.h>

namespace xhip {

// Unsigned 32-bit division by a run-time constant through a multiply-high
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, the round-up variant): for every n < 2^32,
//   n / d == (umulhi(n, mul) + n) >> shift, the sum taken in 64 bits,
// with shift = ceil(log2 d) and mul = floor(2^32 (2^shift - d) / d) + 1.
struct DivMagic {
    uint32_t mul;
    uint32_t shift;
    uint32_t d;
};

constexpr DivMagic div_magic(uint32_t d) {
    uint32_t shift = 0;
    while (shift < 32 && (1ull << shift) < d) shift++;
    const uint64_t mul = (((1ull << 32) * ((1ull << shift) - d)) / d) + 1;
    return DivMagic{(uint32_t)mul, shift, d};
}

constexpr uint32_t div_by(uint32_t n, const DivMagic &m) {
    const uint32_t hi = (uint32_t)(((uint64_t)n * m.mul) >> 32);
    return (uint32_t)(((uint64_t)hi + n) >> m.shift);
}

}  // namespace xhip
