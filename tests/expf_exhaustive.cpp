// Host build of the device header's uq_expf (the same source the kernels
// compile), compared bit for bit with the oracle's uqo_expf on every one of
// the 2^32 f32 inputs; NaN results compare equal when both are NaN. Exit
// status 0 when no input differs.
#include "../uefi-gpu_amd/csrc/uq_device.h"
#include <atomic>
#include <cmath>
#include <cstdio>
#include <thread>
#include <vector>

extern "C" float uqo_expf(float x);

int main(int argc, char** argv) {
    const unsigned nt = argc > 1 ? (unsigned)atoi(argv[1]) : 8;
    std::atomic<long long> bad{0};
    std::vector<std::thread> pool;
    for (unsigned w = 0; w < nt; w++)
        pool.emplace_back([&, w]() {
            long long local = 0;
            for (uint64_t i = w; i < (1ull << 32); i += nt) {
                const float x = __builtin_bit_cast(float, (uint32_t)i);
                const float a = uqo_expf(x), b = uq_expf(x);
                if (__builtin_bit_cast(uint32_t, a) != __builtin_bit_cast(uint32_t, b) && !(std::isnan(a) && std::isnan(b))) {
                    if (local < 4) printf("x=0x%08x oracle=0x%08x device-source=0x%08x\n", (uint32_t)i,
                                          __builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
                    local++;
                }
            }
            bad += local;
        });
    for (auto& t : pool) t.join();
    printf("inputs differing: %lld of 2^32\n", (long long)bad);
    return bad != 0;
}
