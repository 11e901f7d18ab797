// Host check of the gfx950 weight-tile layout: GGML blocks of random codes
// are packed into 16-row tiles (jfh::build_tile) and every value decoded with
// the device tile decoder evaluated on the host (gfx950 kernels' tile_value)
// must equal the oracle's GGML dequantization bit for bit.
#include "jfh_engine.hpp"

extern "C" {
#include "jfo.h"
}

#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

namespace {

int failures = 0;

uint16_t f16_bits(float x) { return jfo_f32_to_f16(x); }

// A random GGML block of `type` (256 values) with finite, modest scales.
std::vector<uint8_t> random_block(uint32_t type, std::mt19937& rng) {
    uint32_t be = 0, bb = 0;
    jfo_type_block(static_cast<int>(type), &be, &bb);
    const uint32_t bytes = 256 / be * bb;
    std::vector<uint8_t> b(bytes);
    for (auto& v : b) v = static_cast<uint8_t>(rng());
    std::uniform_real_distribution<float> u(1e-4F, 0.05F);
    auto put16 = [&](uint32_t off, float x) {
        const uint16_t h = f16_bits(x);
        std::memcpy(b.data() + off, &h, 2);
    };
    switch (type) {
    case 11: put16(0, u(rng)); put16(2, u(rng)); break;
    case 13: put16(208, u(rng)); break;
    case 9: put16(80, u(rng)); put16(82, u(rng)); break;
    case 7:
        for (uint32_t j = 0; j < 8; ++j) put16(34 * j, u(rng));
        break;
    }
    return b;
}

void check_type(uint32_t type, int missing_row) {
    std::mt19937 rng(1234 + type);
    std::vector<std::vector<uint8_t>> blocks(16);
    const uint8_t* ptrs[16];
    for (int i = 0; i < 16; ++i) {
        blocks[i] = random_block(type, rng);
        ptrs[i] = i == missing_row ? nullptr : blocks[i].data();
    }
    std::vector<uint8_t> tile(jfh::gpu::tile_bytes(type));
    jfh::build_tile(type, ptrs, tile.data());
    int bad = 0;
    for (int i = 0; i < 16; ++i) {
        float ref[256];
        if (i == missing_row) {
            std::memset(ref, 0, sizeof(ref));
        } else if (jfo_dequantize_row(static_cast<int>(type), blocks[i].data(), ref, 256) != 0) {
            std::printf("FAIL: oracle rejected type %u\n", type);
            ++failures;
            return;
        }
        for (uint32_t k = 0; k < 256; ++k) {
            const float got = jfh::gpu::dequant_tile_value(type, tile.data(), static_cast<uint32_t>(i), k);
            if (std::memcmp(&got, &ref[k], 4) != 0 && !(got == 0.0F && ref[k] == 0.0F)) {
                if (bad < 4) std::printf("FAIL: type %u row %d value %u: tile %g oracle %g\n", type, i, k, got, ref[k]);
                ++bad;
            }
        }
    }
    if (bad) ++failures;
    else std::printf("tile layout of type %u matches the GGML dequantization\n", type);
}

}  // namespace

int main() {
    for (uint32_t type : {11u, 13u, 7u, 9u}) {
        check_type(type, -1);
        check_type(type, 5);  // a padding row decodes to zero
    }
    if (failures) {
        std::printf("%d tile check(s) failed\n", failures);
        return 1;
    }
    std::printf("tile tests passed\n");
    return 0;
}
