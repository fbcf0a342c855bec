// Internal declarations shared by the host-side C++ of the wpcg library and
// its HIP kernel launchers. Nothing here crosses the C ABI.
#pragma once

#include <hip/hip_runtime_api.h>

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

// ---- device layouts -----------------------------------------------------
// Both schemes keep the reference's bytes per block (68 for v4, 100 for v3)
// but split each block into planes that vector loads can reach:
//   params[row][blk]   u32 = zero_point f16 | scale f16 << 16
//   codes[row][blk][64]  the 64 nibble-pair bytes, stored "lane-major":
//                      dev[l*8 + g] = ref[g*8 + l]   (l, g < 8)
//                      so the eight bytes that AVX2 lane l of the reference
//                      kernel consumes are one contiguous 8-byte word.
//   hp[row][blk][32]   (v3 only) the two-plane high bits, also lane-major:
//                      dev[l*4 + m] = hp[m*8 + l]    (l < 8, m < 4)
struct DeviceMatrix {
    int scheme = 0;
    uint64_t rows = 0, cols = 0, nb = 0;  // nb = cols / 128 blocks per row
    uint8_t* codes = nullptr;
    uint8_t* hp = nullptr;
    uint32_t* params = nullptr;
};

// Host transcodes from the reference's on-disk blocks (AoS) to the planes
// above. `threads` splits rows across std::threads.
void transcode_v4(const uint8_t* blocks, uint64_t n_blocks, uint8_t* codes, uint32_t* params);
void transcode_v3(const uint8_t* blocks, uint64_t n_blocks, uint8_t* lp, uint8_t* hp,
                  uint32_t* params);

// ---- kernel launchers (gemv.hip) ----------------------------------------
hipError_t launch_gemv(const DeviceMatrix& m, int mode, const float* x, const float* bias,
                       float* y, hipStream_t s);
hipError_t launch_embed(const DeviceMatrix& m, uint32_t row, float* out, hipStream_t s);
hipError_t launch_dequant(const DeviceMatrix& m, int rounding, float* w, hipStream_t s);

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
struct wpcg_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
};

struct wpcg_artifact {
    int scheme = 0;
    const uint8_t* map = nullptr;
    uint64_t map_size = 0;
    std::unordered_map<std::string, wpcg::MetaEntry> tensors;
};

struct wpcg_linear {
    wpcg_ctx* ctx = nullptr;
    wpcg::DeviceMatrix m;
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
