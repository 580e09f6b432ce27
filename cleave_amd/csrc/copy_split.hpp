// copy_split.hpp -- how host.cpp splits one memcpy of n bytes over several
// threads.  Plain C++ with no HIP dependency, so a CPU test can check the
// split on its own (every byte copied exactly once, for every length).
#pragma once

#include <algorithm>
#include <cstddef>

namespace ch {

struct CopySplit {
    size_t parts;  // number of ranges (1: one plain memcpy)
    size_t step;   // bytes per range, a multiple of 64; the last range may be shorter
};

// Splits n bytes over at most `threads` ranges of at least `min_slice` bytes
// each.  The step is ceil(n / parts) rounded up to a multiple of 64, so the
// ranges start on 64-byte boundaries and parts * step >= n: the ranges cover
// all n bytes (the last one clamped to n, and empty when the rounding leaves
// nothing for it).
inline CopySplit copy_split(size_t n, size_t threads, size_t min_slice) {
    const size_t parts = std::min<size_t>(std::max<size_t>(1, threads), std::max<size_t>(1, n / min_slice));
    if (parts <= 1) return CopySplit{1, n};
    const size_t step = ((n + parts - 1) / parts + 63) & ~size_t(63);
    return CopySplit{parts, step};
}

// Byte range [*off, *off + *len) of range p (0 <= p < s.parts) of n bytes.
inline void copy_range(const CopySplit& s, size_t n, size_t p, size_t* off, size_t* len) {
    const size_t o = std::min(n, p * s.step);
    *off = o;
    *len = std::min(n, o + s.step) - o;
}

}  // namespace ch
