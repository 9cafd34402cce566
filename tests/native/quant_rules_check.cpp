// Host checks of the device quantizer rules (objeta_amd/csrc/quant_rules.hpp),
// compiled by tests/test_fp8_rules_cpu.py with g++ -fopenmp and linked against the
// oracle. Prints one line per check: "<name> <mismatches> <first mismatching input
// bits in hex>"; every mismatch count must be 0.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "quant_rules.hpp"

extern "C" uint8_t orc_f32_to_f8e4m3_exact(float v);
extern "C" float orc_f8e4m3_to_f32(uint8_t raw);

namespace {
float bits_f32(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
uint32_t f32_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

template <class F>
void run(const char* name, uint64_t lo, uint64_t hi, F&& bad) {
    uint64_t n = 0, first = UINT64_MAX;
#pragma omp parallel for reduction(+ : n) reduction(min : first) schedule(static)
    for (int64_t u = static_cast<int64_t>(lo); u <= static_cast<int64_t>(hi); ++u) {
        if (bad(static_cast<uint32_t>(u))) {
            ++n;
            if (static_cast<uint64_t>(u) < first) first = static_cast<uint64_t>(u);
        }
    }
    std::printf("%s %llu %llx\n", name, static_cast<unsigned long long>(n), static_cast<unsigned long long>(first));
}
}  // namespace

int main() {
    using namespace objeta::rules;
    // Every positive finite float y: the integer rule for ceil(log2f(y)) (glibc's
    // log2f), and, with y taken as a block maximum, cpu_act_quant's block exponent,
    // scale byte and exact reciprocal factor.
    run("ceil_log2_and_act_scale", 0, 0x7F7FFFFFu, [](uint32_t u) {
        const float y = bits_f32(u);
        if (u != 0 && ceil_log2_cr(y) != static_cast<int32_t>(std::ceil(std::log2(y)))) return true;
        const float raw = std::fmax(y, 1e-4f) * (1.0f / 448.0f);
        const int32_t l = raw == y ? ceil_log2_cr(y) : static_cast<int32_t>(std::ceil(std::log2(raw)));
        if (fp8_act_log2_scale(y) != l) return true;
        const Fp8ActScale s = fp8_act_scale(y);
        const int32_t e = l + 127;
        const uint8_t byte = static_cast<uint8_t>(e < 0 ? 0 : (e > 255 ? 255 : e));
        return s.raw != byte || s.inv != std::ldexp(1.0f, -l);
    });
    // Every float bit pattern: the device encoder against the oracle's restatement,
    // and one act_quant element (x * 2^-l against clamp(x / 2^l)) at a scale
    // exponent l in [-22, 120] that cycles with the pattern.
    run("f8e4m3_encode_and_act_code", 0, 0xFFFFFFFFu, [](uint32_t u) {
        const float x = bits_f32(u);
        const uint8_t ref = orc_f32_to_f8e4m3_exact(x);
        if (f32_to_f8e4m3_exact(x) != ref) return true;
        const int32_t l = static_cast<int32_t>(u % 143u) - 22;
        float v = x / bits_f32(static_cast<uint32_t>(l + 127) << 23);  // 2^l, a normal float
        if (v < -448.0f) v = -448.0f;
        else if (v > 448.0f) v = 448.0f;
        return fp8_act_code(x, bits_f32(static_cast<uint32_t>(127 - l) << 23)) != orc_f32_to_f8e4m3_exact(v);
    });
    // the decoder against the oracle's, all codes
    run("f8e4m3_decode", 0, 255, [](uint32_t u) {
        return f32_bits(f8e4m3_to_f32(u)) != f32_bits(orc_f8e4m3_to_f32(static_cast<uint8_t>(u)));
    });
    return 0;
}
