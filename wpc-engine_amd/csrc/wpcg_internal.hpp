// Internal declarations shared by the host-side C++ of the wpcg library and
// its HIP kernel launchers. Nothing here crosses the C ABI.
#pragma once

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstdint>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/wpcg.h"

namespace wpcg {

// ---- errors -------------------------------------------------------------
// Sets the calling thread's last-error text and returns `code`.
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);
#define WPCG_HIP(call)                                              \
    do {                                                            \
        hipError_t e_ = (call);                                     \
        if (e_ != hipSuccess) return ::wpcg::hip_fail(e_, #call);   \
    } while (0)

// ---- device layout ------------------------------------------------------
// Both schemes keep the reference's bytes per block (68 for v4, 100 for v3)
// but split each block into planes that vector loads can reach. Rows are
// padded to a multiple of 16 (one matrix-core tile); padding is zero.
// Every plane is tile-major: the data of block `blk` of the 16 rows of tile
// t is one contiguous record, so one wave's 16-byte-per-lane load of a
// block is a single fully used 1 KiB span.
//
//   codes[t][blk][1024]  the 64 nibble-pair bytes of each of the 16 rows'
//                        reference blocks. AVX2 lane L of the reference
//                        kernel reads ref bytes g*8+L (g < 8) of row r; they
//                        sit at code_pos(r, L) + g, so lane L alone is one
//                        8-byte word and lanes L, L+4 together are one
//                        16-byte word, at ((L&3)*16 + r)*16.
//   hp[t][blk][512]      (v3) the two-plane high bits, same pairing:
//                        hp[m*8 + L] of row r at hp_pos(r, L) + m  (m < 4)
//   params[t][blk][16]   u32 zero_point f16 | scale f16 << 16 of row t*16+i
//                        at i, so one 16-byte load returns four rows.
constexpr int TILE_ROWS = 16;
constexpr uint64_t CODE_REC = 1024;  // code bytes per (tile, block)
constexpr uint64_t HP_REC = 512;     // high-plane bytes per (tile, block)

inline uint64_t pad_rows(uint64_t rows) { return (rows + TILE_ROWS - 1) / TILE_ROWS * TILE_ROWS; }

inline uint64_t code_pos(int r, int L) { return (uint64_t)(((L & 3) * 16 + r) * 16 + (L >> 2) * 8); }
inline uint64_t hp_pos(int r, int L) { return (uint64_t)(((L & 3) * 16 + r) * 8 + (L >> 2) * 4); }

struct DeviceMatrix {
    int scheme = 0;
    uint64_t rows = 0, cols = 0, nb = 0;  // nb = cols / 128 blocks per row
    uint64_t rows_pad = 0;
    uint8_t* codes = nullptr;
    uint8_t* hp = nullptr;
    uint32_t* params = nullptr;
};

// Split of a FAST-mode GEMV over workgroups, fixed at creation so captured
// graphs keep valid workspace pointers.
struct FastPlan {
    int kg = 1;               // K-slices across workgroups
    float* part = nullptr;    // [kg][rows_pad] partial sums (kg > 1)
    uint32_t* counters = nullptr;  // one per workgroup tile group, self-resetting
};

// Host transcodes from the reference's on-disk blocks (AoS) to the planes
// above, for rows [r0, r0 + nrows) of a matrix with nb blocks per row.
// r0 is a multiple of 16 and `codes`/`hp` point at tile r0/16's records;
// `params` at the matrix's parameter base. Bytes of padding rows in the
// last tile are left as they are (the caller zeroes them).
void transcode_rows(int scheme, const uint8_t* blocks, uint64_t r0, uint64_t nrows, uint64_t nb,
                    uint8_t* codes, uint8_t* hp, uint32_t* params_tile_major);

// ---- kernel launchers (gemv.hip) ----------------------------------------
struct GemvJob {
    const DeviceMatrix* m;
    const FastPlan* plan;
    const float* x;
    const float* bias;
    float* y;
};
// FAST mode: a workgroup computes fast_tiles_per_wg 16-row tiles over a
// K-slice of at most fast_max_slice blocks (the slice's x digits live in LDS).
constexpr int FAST_MAXBK = 64;
inline int fast_tiles_per_wg(uint64_t rows) { return pad_rows(rows) / TILE_ROWS >= 512 ? 2 : 1; }
inline uint64_t fast_max_slice(uint64_t rows) { return FAST_MAXBK / fast_tiles_per_wg(rows); }
hipError_t launch_gemv_exact(const DeviceMatrix& m, const float* x, const float* bias, float* y,
                             hipStream_t s);
// All jobs must share the scheme. At most MAX_JOBS per launch.
constexpr int MAX_JOBS = 8;
hipError_t launch_gemv_fast(const GemvJob* jobs, int n, hipStream_t s);
hipError_t launch_embed(const DeviceMatrix& m, uint32_t row, float* out, hipStream_t s);
hipError_t launch_dequant(const DeviceMatrix& m, int rounding, float* w, hipStream_t s);
int fast_kslices(uint64_t rows, uint64_t nb);
// Slices of nbk = ceil(nb/kg) blocks; returns the number of non-empty
// slices, ceil(nb/nbk), so that every slice starts inside the row.
inline int fast_normalize_kslices(uint64_t nb, int kg)
{
    if (nb == 0 || kg <= 1) return 1;
    const uint64_t nbk = (nb + kg - 1) / kg;
    return (int)((nb + nbk - 1) / nbk);
}

// ---- minimal JSON (for model_v{3,4}.meta) ---------------------------------
struct MetaEntry {
    std::vector<uint64_t> shape;
    uint64_t offset = 0, size = 0;
};
// Parses {"layers":[{"name","shape","offset_bytes","size_bytes"},...],
// "block_size":N}. Returns WPCG_OK or WPCG_E_FORMAT (with the error set).
int parse_meta(const std::string& text, std::unordered_map<std::string, MetaEntry>& out,
               uint64_t& block_size);

}  // namespace wpcg

// ---- handle definitions ----------------------------------------------------
// A context lives until wpcg_ctx_destroy has been called AND every handle
// created on it (linears, events, graphs) has been destroyed: each holds a
// reference, so handles may be released in any order.
struct wpcg_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::atomic<int> refs{1};
};

namespace wpcg {
void ctx_retain(wpcg_ctx* c);
void ctx_release(wpcg_ctx* c);
}  // namespace wpcg

struct wpcg_artifact {
    int scheme = 0;
    const uint8_t* map = nullptr;
    uint64_t map_size = 0;
    std::unordered_map<std::string, wpcg::MetaEntry> tensors;
};

struct wpcg_linear {
    wpcg_ctx* ctx = nullptr;
    wpcg::DeviceMatrix m;
    wpcg::FastPlan plan;
    float* bias = nullptr;  // device, out_f floats, or null
    int mode = WPCG_MODE_EXACT;
    // staging for the synchronous *_host twins
    std::mutex host_mu;
    float* x_stage = nullptr;
    float* y_stage = nullptr;
};

struct wpcg_event {
    wpcg_ctx* ctx = nullptr;
    hipEvent_t ev = nullptr;
};

struct wpcg_graph {
    wpcg_ctx* ctx = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};
