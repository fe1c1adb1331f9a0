// Host-side check of the decode kernel's division by launch constants
// (leap::make_fastdiv / leap::fast_div): every quotient the prologue takes
// equals the integer quotient, for divisors 1..5000 against numerators
// 0..19999, both sides of multiples, the top of the range (2^31 - 1) and
// random numerators, and random divisors up to 2^31 - 1.  Built and run on
// the host by tests/test_fastdiv.py.
#include "decode_attention.hpp"
#include <cstdio>
#include <random>
int main() {
    std::mt19937_64 rng(1);
    long long bad = 0, n_checked = 0;
    auto check = [&](uint32_t n, uint32_t d, leap::FastDiv f) {
        n_checked++;
        if (leap::fast_div(n, f) != n / d) { if (bad++ < 5) printf("mismatch n=%u d=%u\n", n, d); }
    };
    for (uint32_t d = 1; d <= 5000; d++) {
        const leap::FastDiv f = leap::make_fastdiv(d);
        for (uint32_t n = 0; n < 20000; n++) check(n, d, f);
        for (uint32_t k = 1; k < 40; k++) { uint32_t n = 0x7fffffffu - k; check(n, d, f); check(k * d - 1, d, f); check(k * d, d, f); }
        for (int i = 0; i < 200; i++) check((uint32_t)(rng() & 0x7fffffffu), d, f);
    }
    for (int i = 0; i < 200000; i++) {
        uint32_t d = (uint32_t)(rng() % 0x7fffffffu) + 1, n = (uint32_t)(rng() & 0x7fffffffu);
        check(n, d, leap::make_fastdiv(d));
    }
    printf("checked %lld, mismatches %lld\n", n_checked, bad);
    return bad != 0;
}
