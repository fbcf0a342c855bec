// Host-side encoder: fp32 weights to WPC v4 / v3 blocks, as the reference's
// artifact compiler writes them (wpc-core/src/quant_encoder.rs:7-96). Per
// 128-value block: min and max (NaN skipped by the comparisons), scale =
// (max - min) / levels or 1 for a flat block, code = round half away from
// zero of (w - min) / scale clamped to [0, levels] (NaN -> 0), then
// zero_point = f16(min), scale = f16(scale), both rounded to nearest even.
// Codes are computed from the fp32 min and scale, not the f16 ones.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "wpcg_internal.hpp"

namespace {

inline uint16_t f16_bits(float v)
{
    const _Float16 h = (_Float16)v;  // IEEE binary16, round to nearest even
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

void fit_block(const float* w, float levels, uint8_t codes[128], uint16_t* zp, uint16_t* sc)
{
    float lo = 3.40282347e+38f, hi = -3.40282347e+38f;
    for (int i = 0; i < 128; i++) {
        if (w[i] < lo) lo = w[i];
        if (w[i] > hi) hi = w[i];
    }
    const float scale = hi > lo ? (hi - lo) / levels : 1.0f;
    for (int i = 0; i < 128; i++) {
        float c = std::round((w[i] - lo) / scale);  // half away from zero, as f32::round
        if (!(c >= 0.0f)) c = 0.0f;                 // NaN and negatives
        if (c > levels) c = levels;
        codes[i] = (uint8_t)c;
    }
    *zp = f16_bits(lo);
    *sc = f16_bits(scale);
}

void put16(uint8_t* p, uint16_t v)
{
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}

// v4: byte j = code j | code j+64 << 4 (wpc-format/src/lib.rs:324-339)
void block_v4(const float* w, uint8_t* out)
{
    uint8_t c[128];
    uint16_t zp, sc;
    fit_block(w, 15.0f, c, &zp, &sc);
    put16(out, zp);
    put16(out + 2, sc);
    for (int j = 0; j < 64; j++) out[4 + j] = (uint8_t)(c[j] | c[j + 64] << 4);
}

// v3: four 6-bit codes per three bytes, little-endian 24-bit groups
// (wpc-format/src/lib.rs:206-240)
void block_v3(const float* w, uint8_t* out)
{
    uint8_t c[128];
    uint16_t zp, sc;
    fit_block(w, 63.0f, c, &zp, &sc);
    put16(out, zp);
    put16(out + 2, sc);
    for (int g = 0; g < 32; g++) {
        const uint32_t v = c[4 * g] | c[4 * g + 1] << 6 | c[4 * g + 2] << 12 | (uint32_t)c[4 * g + 3] << 18;
        out[4 + 3 * g] = (uint8_t)v;
        out[5 + 3 * g] = (uint8_t)(v >> 8);
        out[6 + 3 * g] = (uint8_t)(v >> 16);
    }
}

}  // namespace

extern "C" int wpcg_encode(int scheme, const float* w, uint64_t n, void* out_blocks)
{
    using namespace wpcg;
    if (scheme != WPCG_SCHEME_V3 && scheme != WPCG_SCHEME_V4) return fail(WPCG_E_ARG, "scheme must be 3 or 4");
    if ((!w || !out_blocks) && n) return fail(WPCG_E_ARG, "null argument");
    if (n % 128) return fail(WPCG_E_SHAPE, "the value count must be a multiple of 128");
    const uint64_t nb = n / 128, bpb = scheme == 4 ? 68 : 100;
    uint8_t* out = static_cast<uint8_t*>(out_blocks);
    const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    const uint64_t per = std::max<uint64_t>(4096, (nb + hw - 1) / hw);
    std::vector<std::thread> ts;
    for (uint64_t b0 = 0; b0 < nb; b0 += per) {
        const uint64_t b1 = std::min(nb, b0 + per);
        ts.emplace_back([=] {
            for (uint64_t b = b0; b < b1; b++) {
                if (scheme == 4) block_v4(w + 128 * b, out + bpb * b);
                else block_v3(w + 128 * b, out + bpb * b);
            }
        });
    }
    for (auto& t : ts) t.join();
    return WPCG_OK;
}
