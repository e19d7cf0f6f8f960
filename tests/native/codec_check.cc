// Host build of the shipped device codec (infer_amd/csrc/codec.h) compared against the parity
// oracle (oracle/feather_oracle.c) on every 32-bit float pattern (FP8, BF16) and every 16-bit
// pattern (FP16 decode), plus every FP16-relevant float via the same sweep.
// Built and run by tests/test_codec_exhaustive.py; prints "OK" or the first mismatches.
#include <cstdio>
#include <cstring>
#include "../../infer_amd/csrc/codec.h"
extern "C" {
#include "../../oracle/feather_oracle.h"
}

static float f(uint32_t u) { float x; std::memcpy(&x, &u, 4); return x; }
static uint32_t b(float x) { uint32_t u; std::memcpy(&u, &x, 4); return u; }

int main() {
    long bad = 0;
    #pragma omp parallel for reduction(+:bad) schedule(static, 1 << 16)
    for (long long i = 0; i < (1ll << 32); ++i) {
        const float x = f((uint32_t)i);
        if (fhip::fp8_encode(x, false) != fo_fp8_encode(12, x)) { if (bad < 4) std::printf("e4m3 %08llx\n", i); ++bad; }
        if (fhip::fp8_encode(x, true) != fo_fp8_encode(13, x)) { if (bad < 4) std::printf("e5m2 %08llx\n", i); ++bad; }
        if (fhip::bf16_encode(x) != fo_bf16_encode(x)) { if (bad < 4) std::printf("bf16 %08llx\n", i); ++bad; }
        if (fhip::bf16_encode_plain(x) != fo_bf16_encode_plain(x)) { if (bad < 4) std::printf("bf16p %08llx\n", i); ++bad; }
        if (fhip::fp16_encode(x) != fo_fp16_encode(x)) { if (bad < 4) std::printf("fp16 %08llx\n", i); ++bad; }
        if (fhip::fp16_encode_cast(x) != fo_fp16_encode_cast(x)) { if (bad < 4) std::printf("fp16c %08llx\n", i); ++bad; }
    }
    for (int c = 0; c < 256; ++c)
        for (int d = 12; d <= 13; ++d)
            if (b(fhip::fp8_decode((uint8_t)c, d == 13)) != b(fo_fp8_decode(d, (uint8_t)c))) { std::printf("dec %d %02x\n", d, c); ++bad; }
    for (int h = 0; h < 65536; ++h)
        if (b(fhip::fp16_decode((uint16_t)h)) != b(fo_fp16_decode((uint16_t)h))) { if (bad < 4) std::printf("f16dec %04x\n", h); ++bad; }
    if (bad) { std::printf("MISMATCHES %ld\n", bad); return 1; }
    std::printf("OK\n");
    return 0;
}
