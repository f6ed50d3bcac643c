// CPU check of the zero-fill size of the namespace jllm layer's error path
// (genie-ai-runtime_amd/csrc/fill_size.h): prints one value per case, the
// Python test compares them.  Test infrastructure, not part of the library.
#include <cstdio>
#include "fill_size.h"

using jllm_fill::fill_bytes;

int main() {
    const long long big = 1ll << 31;
    std::printf("%zu\n", fill_bytes({9728}, 2));               // 19456
    std::printf("%zu\n", fill_bytes({-1}, 2));                 // negative M
    std::printf("%zu\n", fill_bytes({9728, -4}, 2));           // negative N
    std::printf("%zu\n", fill_bytes({-2560 / 32}, 36));        // negative K
    std::printf("%zu\n", fill_bytes({-32, 128}, 2));           // negative n_heads
    std::printf("%zu\n", fill_bytes({big - 1, big - 1}, 2));   // M*N*2 overflows the cap
    std::printf("%zu\n", fill_bytes({1ll << 20, 1ll << 19}, 2)); // exactly 2^40: allowed
    std::printf("%zu\n", fill_bytes({1ll << 20, 1ll << 19}, 4)); // 2^41: refused
    std::printf("%zu\n", fill_bytes({0, 5}, 2));               // empty
    std::printf("%zu\n", fill_bytes({512, 32, 128}, 2));       // 4194304
    std::printf("%zu\n", fill_bytes({8, 127}, 1));             // odd byte count is exact: 1016
    return 0;
}
