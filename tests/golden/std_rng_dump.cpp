// Writes the libstdc++ streams the oracle restates, for tests/test_oracle_rng.py:
//   std_rng_dump mt <seed> <n>      -> n std::mt19937 outputs (uint32, binary)
//   std_rng_dump normal <seed> <n>  -> n std::normal_distribution<float> draws
// Built and run by the CPU test in this container (g++ 11.4 / libstdc++).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <cstdint>
#include <random>
#include <vector>

int main(int argc, char** argv) {
    if (argc != 4) { std::fprintf(stderr, "usage: %s mt|normal seed n\n", argv[0]); return 2; }
    const uint32_t seed = (uint32_t)std::strtoul(argv[2], nullptr, 0);
    const size_t n = (size_t)std::strtoull(argv[3], nullptr, 0);
    std::mt19937 rng(seed);
    if (std::strcmp(argv[1], "mt") == 0) {
        std::vector<uint32_t> v(n);
        for (auto& x : v) x = (uint32_t)rng();
        std::fwrite(v.data(), 4, n, stdout);
    } else {
        std::normal_distribution<float> nd(0.f, 1.f);
        std::vector<float> v(n);
        for (auto& x : v) x = nd(rng);
        std::fwrite(v.data(), 4, n, stdout);
    }
    return 0;
}
