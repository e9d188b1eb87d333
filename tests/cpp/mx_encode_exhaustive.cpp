// Every magnitude an MX block can hold after division by its E8M0 scale,
// through the kernels' element encoders (jalapenos-at-home_amd/csrc/
// mx_encode.h, the same source the gfx950 quantizers compile) and through the
// oracle's quantizers:
//  * E2M1 (python/quantize_mxfp4.py:18-39 restated): every float in [0, 8),
//    each in a block whose maximum is 4, so the block's scale byte is 127;
//  * E4M3 (the MX-FP8 activation rule): every float in [0, 512), each in a
//    block whose maximum is 256, so again the scale byte is 127.
// With scale 2^0 the value's code is exactly the encoder's input. Exit status
// 0 when every code agrees.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "mx_encode.h"
#include "mx4_oracle.h"

template <bool FP8>
static bool check(uint32_t end, float block_max, const char* what) {
    const uint32_t per_chunk = 31u * (1u << 16);  // 31 test values per 32-element block
    uint64_t bad = 0, checked = 0;
#pragma omp parallel for schedule(dynamic) reduction(+ : bad, checked)
    for (int64_t c0 = 0; c0 < (int64_t)end; c0 += per_chunk) {
        const uint32_t lo = (uint32_t)c0, hi = (uint32_t)(c0 + per_chunk < end ? c0 + per_chunk : end);
        const uint32_t nvals = hi - lo, nblk = (nvals + 30) / 31;
        std::vector<float> x((size_t)nblk * 32, 0.0f);
        for (uint32_t i = 0; i < nvals; ++i) {
            const uint32_t bits = lo + i;
            std::memcpy(&x[(size_t)(i / 31) * 32 + 1 + i % 31], &bits, 4);
        }
        for (uint32_t b = 0; b < nblk; ++b) x[(size_t)b * 32] = block_max;
        std::vector<uint8_t> codes((size_t)nblk * (FP8 ? 32 : 16)), scales(nblk);
        const int st = FP8 ? oracle_quantize_fp8(x.data(), nblk, 32, codes.data(), scales.data())
                           : oracle_quantize(x.data(), nblk, 32, codes.data(), scales.data());
        if (st != 0) {
            ++bad;
            continue;
        }
        for (uint32_t i = 0; i < nvals; ++i) {
            const uint32_t b = i / 31, e = 1 + i % 31;
            const uint32_t want = FP8 ? codes[(size_t)b * 32 + e] : (codes[(size_t)b * 16 + e / 2] >> (4 * (e & 1))) & 15u;
            const uint32_t bits = lo + i;
            float v;
            std::memcpy(&v, &bits, 4);
            const uint32_t got = FP8 ? mx4::e4m3_magnitude_code(v) : mx4::e2m1_magnitude_code(v);
            if (scales[b] != 127 || got != want) {
                if (bad < 5) std::printf("%s mismatch: %08x want %u got %u (scale %u)\n", what, bits, want, got, scales[b]);
                ++bad;
            }
            ++checked;
        }
    }
    std::printf("%s: checked %llu values, %llu mismatches\n", what, (unsigned long long)checked,
                (unsigned long long)bad);
    return bad == 0 && checked == end;
}

int main() {
    const bool e2m1 = check<false>(0x41000000u, 4.0f, "E2M1 [0, 8)");
    const bool e4m3 = check<true>(0x44000000u, 256.0f, "E4M3 [0, 512)");
    return e2m1 && e4m3 ? 0 : 1;
}
