// Recorded-pass lifecycle check, built against a host-AddressSanitizer copy of
// the library (`make pass_cycle_asan`; device code unchanged) and run on a GPU:
// for each Qwen3-8B projection shape (q, k, gate, down, lm_head over a few
// distinct copies) and M in {1, 2, 4, 8, 16, 32}: fresh x and y, one pass
// recording every copy's mx4_matmul, 4 launches, a wait, mx4_pass_release, then
// the same calls eagerly, whose y must equal the replays' bit for bit; x and y
// are freed before the next block. The sequence is the record -> launch ->
// release cycle per (projection, M) block of a speculative-verify sweep.
#include <cstdio>
#include <cstring>
#include <cstdint>
#include <vector>
#include "mx4.h"

#define CK(x) do { mx4_status s_ = (x); if (s_ != MX4_OK) { std::printf("FAIL %s line %d: %s\n", #x, __LINE__, mx4_last_error()); return 1; } } while (0)

int main() {
    mx4_context* ctx = nullptr;
    CK(mx4_create(0, &ctx));
    struct Shape { const char* name; uint32_t n, k; int copies; } shapes[] = {
        {"q", 4096, 4096, 6}, {"k", 1024, 4096, 8}, {"gate", 12288, 4096, 3}, {"down", 4096, 12288, 3},
        {"lm_head", 151936, 4096, 2}};
    const uint32_t ms[] = {1, 2, 4, 8, 16, 32};
    uint64_t seed = 40000;
    int blocks = 0;
    for (const Shape& sh : shapes) {
        std::vector<void*> mem;
        std::vector<mx4_weight*> ws;
        for (int c = 0; c < sh.copies; ++c) {
            const uint64_t pb = (uint64_t)sh.n * sh.k / 2, sb = (uint64_t)sh.n * sh.k / 32;
            void* p = nullptr;
            CK(mx4_malloc(ctx, pb + 256 + sb, &p));
            uint8_t* base = (uint8_t*)p;
            CK(mx4_synth_weight(ctx, seed++, 0.02, sh.n, sh.k, base, base + pb + 256 - (pb % 256)));
            mx4_weight* w = nullptr;
            CK(mx4_weight_wrap(ctx, base, base + pb + 256 - (pb % 256), sh.n, sh.k, &w));
            mem.push_back(p);
            ws.push_back(w);
        }
        for (uint32_t m : ms) {
            void *x = nullptr, *y = nullptr, *y2 = nullptr;
            CK(mx4_malloc(ctx, (uint64_t)m * sh.k * 2, &x));
            CK(mx4_malloc(ctx, (uint64_t)m * sh.n * 4, &y));
            CK(mx4_malloc(ctx, (uint64_t)m * sh.n * 4, &y2));
            CK(mx4_synth_bf16(ctx, 2, 1.0, 0, (uint64_t)m * sh.k, (uint16_t*)x));
            CK(mx4_pass_begin(ctx));
            for (mx4_weight* w : ws) CK(mx4_matmul(ctx, x, MX4_BF16, m, w, (float*)y));
            mx4_pass* p = nullptr;
            CK(mx4_pass_end(ctx, &p));
            for (int r = 0; r < 4; ++r) CK(mx4_pass_launch(ctx, p));
            CK(mx4_synchronize(ctx));
            mx4_pass_release(p);
            for (mx4_weight* w : ws) CK(mx4_matmul(ctx, x, MX4_BF16, m, w, (float*)y2));
            CK(mx4_synchronize(ctx));
            std::vector<uint32_t> a((size_t)m * sh.n), b((size_t)m * sh.n);
            CK(mx4_download(ctx, a.data(), y, a.size() * 4));
            CK(mx4_download(ctx, b.data(), y2, b.size() * 4));
            if (std::memcmp(a.data(), b.data(), a.size() * 4) != 0) {
                std::printf("FAIL %s M=%u: replay differs from eager\n", sh.name, m);
                return 1;
            }
            CK(mx4_free(ctx, x));
            CK(mx4_free(ctx, y));
            CK(mx4_free(ctx, y2));
            ++blocks;
            std::printf("block %s M=%u ok\n", sh.name, m);
            std::fflush(stdout);
        }
        CK(mx4_synchronize(ctx));
        for (mx4_weight* w : ws) mx4_weight_release(w);
        for (void* p : mem) CK(mx4_free(ctx, p));
    }
    mx4_destroy(ctx);
    std::printf("pass cycle under host ASan: %d blocks, no error\n", blocks);
    std::fflush(stdout);
    return 0;
}
