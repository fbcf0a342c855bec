// Host transcodes from the reference's on-disk blocks to the device planes
// (layout described in wpcg_internal.hpp). Pure byte permutation: the device
// holds exactly the reference's codes, zero points and scales.
#include <algorithm>
#include <thread>

#include "wpcg_internal.hpp"

namespace wpcg {
namespace {

template <typename Fn>
void parallel_rows(uint64_t n, Fn fn)
{
    unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (n < 256 || hw == 1) { fn(0, n); return; }
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

// QuantBlockV3::unpack_codes (wpc-format/src/lib.rs:245-257) written as the
// 24-bit little-endian group it is.
inline void v3_unpack(const uint8_t* p, uint8_t c[128])
{
    for (int g = 0; g < 32; g++) {
        uint32_t w = (uint32_t)p[3 * g] | (uint32_t)p[3 * g + 1] << 8 | (uint32_t)p[3 * g + 2] << 16;
        c[4 * g + 0] = w & 63;
        c[4 * g + 1] = (w >> 6) & 63;
        c[4 * g + 2] = (w >> 12) & 63;
        c[4 * g + 3] = (w >> 18) & 63;
    }
}

}  // namespace

// v4: QuantBlockV4 (wpc-format/src/lib.rs:324-339): the 64 code bytes are
// permuted into paired-lane order. v3: QuantBlockV3 (lib.rs:206-220) is
// unpacked to 128 codes and re-packed as two planes,
//   lp[j] = (c[j]&15) | (c[j+64]&15) << 4              (j < 64)
//   hp[j] = sum_q ((c[j+32q] >> 4) & 3) << 2q            (j < 32)
// whose low plane has v4's byte shape, then both planes are permuted.
void transcode_rows(int scheme, const uint8_t* blocks, uint64_t r0, uint64_t nrows, uint64_t nb,
                    uint8_t* codes, uint8_t* hp, uint32_t* params)
{
    const uint64_t bpb = scheme == 4 ? 68 : 100;
    parallel_rows(nrows, [&](uint64_t a, uint64_t b) {
        for (uint64_t r = a; r < b; r++) {
            const uint64_t row = r0 + r;
            const int tr = (int)(r % TILE_ROWS);
            const uint64_t t = r / TILE_ROWS;  // tile relative to `codes`/`hp`
            for (uint64_t k = 0; k < nb; k++) {
                const uint8_t* blk = blocks + (r * nb + k) * bpb;
                params[((row / TILE_ROWS) * nb + k) * TILE_ROWS + row % TILE_ROWS] = rd_params(blk);
                uint8_t* dc = codes + (t * nb + k) * CODE_REC;
                if (scheme == 4) {
                    for (int L = 0; L < 8; L++)
                        for (int g = 0; g < 8; g++) dc[code_pos(tr, L) + g] = blk[4 + g * 8 + L];
                } else {
                    uint8_t c[128], lp[64], h[32];
                    v3_unpack(blk + 4, c);
                    for (int j = 0; j < 64; j++) lp[j] = (uint8_t)((c[j] & 15) | (c[j + 64] & 15) << 4);
                    for (int j = 0; j < 32; j++)
                        h[j] = (uint8_t)(((c[j] >> 4) & 3) | ((c[j + 32] >> 4) & 3) << 2 |
                                         ((c[j + 64] >> 4) & 3) << 4 | ((c[j + 96] >> 4) & 3) << 6);
                    uint8_t* dh = hp + (t * nb + k) * HP_REC;
                    for (int L = 0; L < 8; L++) {
                        for (int g = 0; g < 8; g++) dc[code_pos(tr, L) + g] = lp[g * 8 + L];
                        for (int m = 0; m < 4; m++) dh[hp_pos(tr, L) + m] = h[m * 8 + L];
                    }
                }
            }
        }
    });
}

}  // namespace wpcg
