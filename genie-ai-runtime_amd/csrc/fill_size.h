// fill_size.h -- size of the zero fill of the namespace jllm layer's error
// path.  Host-only, header-only, so a CPU test compiles it with g++.
#pragma once
#include <cstddef>
#include <initializer_list>

namespace jllm_fill {

// No valid call of this library addresses more than this many bytes of one
// output (a GPU holds 288 GB); larger products are treated as invalid.
constexpr unsigned long long kMaxFillBytes = 1ull << 40;

// Bytes of an output of `elem`-byte elements shaped by `dims`: 0 when any
// dimension is negative or the product exceeds kMaxFillBytes (an invalid
// call then writes nothing instead of a huge range past the output).
inline size_t fill_bytes(std::initializer_list<long long> dims, size_t elem) {
    unsigned long long n = elem;
    for (long long d : dims) {
        if (d < 0) return 0;
        if (d == 0) return 0;
        if (n > kMaxFillBytes / (unsigned long long)d) return 0;
        n *= (unsigned long long)d;
    }
    return n > kMaxFillBytes ? 0 : (size_t)n;
}

}  // namespace jllm_fill
