// Host transcodes from the reference's on-disk blocks to the device planes
// (layout described in wpcg_internal.hpp). Pure byte permutation: the device
// holds exactly the reference's codes, zero points and scales.
#include <algorithm>
#include <thread>

#include "wpcg_internal.hpp"

namespace wpcg {
namespace {

template <typename Fn>
void parallel_blocks(uint64_t n, Fn fn)
{
    unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (n < (1u << 14) || hw == 1) { fn(0, n); return; }
    std::vector<std::thread> ts;
    uint64_t per = (n + hw - 1) / hw;
    for (unsigned t = 0; t < hw; t++) {
        uint64_t a = t * per, b = std::min(n, a + per);
        if (a >= b) break;
        ts.emplace_back([=] { fn(a, b); });
    }
    for (auto& t : ts) t.join();
}

inline uint32_t rd_params(const uint8_t* blk)
{
    // [zero_point f16 LE][scale f16 LE] -> zp | scale << 16
    return (uint32_t)blk[0] | (uint32_t)blk[1] << 8 | (uint32_t)blk[2] << 16 | (uint32_t)blk[3] << 24;
}

}  // namespace

// v4: QuantBlockV4 (wpc-format/src/lib.rs:324-339) -> params + lane-major codes
void transcode_v4(const uint8_t* blocks, uint64_t n_blocks, uint8_t* codes, uint32_t* params)
{
    parallel_blocks(n_blocks, [&](uint64_t a, uint64_t b) {
        for (uint64_t i = a; i < b; i++) {
            const uint8_t* blk = blocks + 68 * i;
            params[i] = rd_params(blk);
            uint8_t* dst = codes + 64 * i;
            for (int l = 0; l < 8; l++)
                for (int g = 0; g < 8; g++) dst[l * 8 + g] = blk[4 + g * 8 + l];
        }
    });
}

// v3: QuantBlockV3 (wpc-format/src/lib.rs:206-220), four 6-bit codes per three
// bytes -> unpack exactly as QuantBlockV3::unpack_codes (:245-257) -> two
// planes:  lp[j] = (c[j]&15) | (c[j+64]&15) << 4            (j < 64)
//          hp[j] = sum_q ((c[j+32q] >> 4) & 3) << 2q          (j < 32)
// then both planes lane-major.
void transcode_v3(const uint8_t* blocks, uint64_t n_blocks, uint8_t* lp_out, uint8_t* hp_out,
                  uint32_t* params)
{
    parallel_blocks(n_blocks, [&](uint64_t a, uint64_t b) {
        for (uint64_t i = a; i < b; i++) {
            const uint8_t* blk = blocks + 100 * i;
            params[i] = rd_params(blk);
            uint8_t c[128];
            for (int g = 0; g < 32; g++) {
                uint32_t w = (uint32_t)blk[4 + 3 * g] | (uint32_t)blk[5 + 3 * g] << 8 |
                             (uint32_t)blk[6 + 3 * g] << 16;
                c[4 * g + 0] = w & 63;
                c[4 * g + 1] = (w >> 6) & 63;
                c[4 * g + 2] = (w >> 12) & 63;
                c[4 * g + 3] = (w >> 18) & 63;
            }
            uint8_t lp[64], hp[32];
            for (int j = 0; j < 64; j++) lp[j] = (uint8_t)((c[j] & 15) | (c[j + 64] & 15) << 4);
            for (int j = 0; j < 32; j++)
                hp[j] = (uint8_t)(((c[j] >> 4) & 3) | ((c[j + 32] >> 4) & 3) << 2 |
                                  ((c[j + 64] >> 4) & 3) << 4 | ((c[j + 96] >> 4) & 3) << 6);
            uint8_t* dl = lp_out + 64 * i;
            uint8_t* dh = hp_out + 32 * i;
            for (int l = 0; l < 8; l++) {
                for (int g = 0; g < 8; g++) dl[l * 8 + g] = lp[g * 8 + l];
                for (int m = 0; m < 4; m++) dh[l * 4 + m] = hp[m * 8 + l];
            }
        }
    });
}

}  // namespace wpcg
