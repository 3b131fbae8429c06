// Host check of bmo::FastDiv (kernels.hpp) against integer division: every
// divisor below 3000 with every numerator below 2^16 and a spread of larger
// ones, and random divisors up to 2^31 - 1 with numerators at the range edges
// and at multiples of the divisor.  Prints "ok <count>" or the first failure.
#include <cstdio>
#include <cstdint>
#include <random>

#include "kernels.hpp"

int main() {
    std::mt19937_64 rng(12345);
    uint64_t count = 0;
    auto check = [&](uint32_t d, uint32_t n) {
        static bmo::FastDiv f{};
        static uint32_t fd = 0;
        if (fd != d) {
            f = bmo::make_fastdiv(d);
            fd = d;
        }
        ++count;
        if (f.div(n) != n / d) {
            std::printf("FAIL d=%u n=%u got %u\n", d, n, f.div(n));
            return false;
        }
        return true;
    };
    for (uint32_t d = 1; d < 3000; ++d) {
        for (uint32_t n = 0; n < 65536; ++n)
            if (!check(d, n)) return 1;
        for (int i = 0; i < 64; ++i)
            if (!check(d, (uint32_t) (rng() & 0x7FFFFFFFu))) return 1;
        if (!check(d, 0x7FFFFFFFu) || !check(d, 0x7FFFFFFEu)) return 1;
    }
    for (int i = 0; i < 20000; ++i) {
        uint32_t d = (uint32_t) (rng() % 0x7FFFFFFFu) + 1;
        if (i < 8) d = 0x7FFFFFFFu - (uint32_t) i;
        const uint32_t edges[] = {0u, 1u, d - 1, d, 0x7FFFFFFFu, 0x7FFFFFFEu};
        for (uint32_t n : edges)
            if (n <= 0x7FFFFFFFu && !check(d, n)) return 1;
        for (uint64_t k = 1; k * d < 0x80000000ull && k < 64; ++k)
            for (int r = -1; r <= 1; ++r) {
                const int64_t n = (int64_t) (k * d) + r;
                if (n >= 0 && n < 0x80000000ll && !check(d, (uint32_t) n)) return 1;
            }
        for (int j = 0; j < 16; ++j)
            if (!check(d, (uint32_t) (rng() & 0x7FFFFFFFu))) return 1;
    }
    std::printf("ok %llu\n", (unsigned long long) count);
    return 0;
}
