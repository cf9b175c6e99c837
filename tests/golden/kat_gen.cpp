// Regenerates the input of the reference's only GroupNorm+SiLU known-answer
// test (tests/test_operators.cpp:200-238 in pomagrenate/soar.cpp): C=16,
// G=4, H=W=32, eps=1e-5, gamma=1.2, beta=-0.3, x from std::mt19937(999)
// through std::uniform_real_distribution<float>(-2, 2), as libstdc++
// implements them.  Writes the 16384 floats little-endian to argv[1].
//
// Also prints the 10000th output of a default-seeded std::mt19937, which
// the C++ standard fixes at 4123659995 ([rand.predef]), so the fixture
// script can check that this library's engine is the standard one.
#include <cstdio>
#include <random>
#include <vector>

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s OUT.bin\n", argv[0]);
        return 2;
    }
    std::mt19937 probe;
    probe.discard(9999);
    unsigned long v10000 = probe();

    constexpr int C = 16, H = 32, W = 32;
    std::vector<float> x(C * H * W);
    std::mt19937 rng(999);
    std::uniform_real_distribution<float> dist(-2.0f, 2.0f);
    for (auto& v : x) v = dist(rng);

    std::FILE* f = std::fopen(argv[1], "wb");
    if (!f) return 1;
    std::fwrite(x.data(), sizeof(float), x.size(), f);
    std::fclose(f);
    std::printf("%lu\n", v10000);
    return 0;
}
