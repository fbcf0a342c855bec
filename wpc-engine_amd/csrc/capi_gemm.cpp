// C ABI of the batched dequant-GEMM (include/wpcg.h). No reference
// counterpart: the reference decodes one token at a time (README.md:174-180).
#include <algorithm>
#include <cstring>
#include <memory>

#include "wpcg_internal.hpp"

namespace wpcg {

void free_gemm(GemmWork& w)
{
    if (w.xf) (void)hipFree(w.xf);
    if (w.xsum) (void)hipFree(w.xsum);
    if (w.part) (void)hipFree(w.part);
    if (w.counters) (void)hipFree(w.counters);
    const int req = w.kg_req;
    w = GemmWork{};
    w.kg_req = req;
}

namespace {

int make_gemm(wpcg_linear* L, hipStream_t s)
{
    const DeviceMatrix& m = L->m;
    GemmWork& w = L->gemm;
    w.kg = gemm_kslices(m.rows, m.nb, w.kg_req);
    w.kg_small = gemm_small_kslices(m.rows, m.nb, w.kg_req);
    const uint64_t part = std::max<uint64_t>((uint64_t)w.kg * GEMM_MAX_M, (uint64_t)w.kg_small * 16) * m.rows_pad;
    // partial sums are addressed with 32-bit byte offsets
    if (part * 4 >= (1ull << 31))
        return fail(WPCG_E_SHAPE, "batched GEMM: too many rows for the split-K workspace");
    const uint64_t rgs = (uint64_t)std::max(gemm_row_groups(m.rows), gemm_small_row_groups(m.rows));
    hipError_t e = hipMalloc(&w.xf, m.nb * 4 * 4096);
    if (e == hipSuccess) e = hipMalloc(&w.xsum, m.nb * GEMM_MAX_M * sizeof(float));
    if (e == hipSuccess && (w.kg > 1 || w.kg_small > 1)) e = hipMalloc(&w.part, part * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&w.counters, std::max<uint64_t>(1, rgs) * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemsetAsync(w.counters, 0, std::max<uint64_t>(1, rgs) * sizeof(uint32_t), s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        free_gemm(w);
        return hip_fail(e, "batched GEMM workspace");
    }
    return WPCG_OK;
}

int run_gemm(wpcg_linear* L, const void* x, int x_dtype, uint32_t M, float* y, hipStream_t s)
{
    const DeviceMatrix& m = L->m;
    if (M == 0 || m.rows == 0) return WPCG_OK;
    if (m.nb == 0) {  // no inputs: every row of Y is the bias (or 0)
        for (uint32_t r = 0; r < M; r++)
            if (int rc = wpcg_linear_matvec(L, nullptr, y + (uint64_t)r * m.rows, s)) return rc;
        return WPCG_OK;
    }
    if (x_dtype == WPCG_DTYPE_F32 && M == 1)
        return wpcg_linear_matvec(L, static_cast<const float*>(x), y, s);
    if (!L->gemm.xf) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        WPCG_HIP(hipStreamIsCapturing(s, &st));
        if (st != hipStreamCaptureStatusNone)
            return fail(WPCG_E_ARG, "the first batched call on a linear allocates its workspace: "
                                    "make it before capturing a graph");
        if (int rc = make_gemm(L, s)) return rc;
    }
    const uint64_t es = x_dtype == WPCG_DTYPE_BF16 ? 2 : 4;
    const uint32_t step = x_dtype == WPCG_DTYPE_F32_SPLIT ? GEMM_MAX_M_SPLIT : GEMM_MAX_M;
    for (uint32_t c = 0; c < M; c += step) {
        const int mc = (int)std::min<uint32_t>(step, M - c);
        WPCG_HIP(launch_gemm(m, L->gemm, static_cast<const uint8_t*>(x) + (uint64_t)c * m.cols * es, x_dtype, mc,
                             L->bias, nullptr, y + (uint64_t)c * m.rows, s));
    }
    return WPCG_OK;
}

}  // namespace

int linear_gemm(wpcg_linear* L, const float* x, int x_mode, uint32_t M, const float* res, float* y, hipStream_t s)
{
    const DeviceMatrix& m = L->m;
    if (M == 0 || m.rows == 0) return WPCG_OK;
    if (m.nb == 0) return fail(WPCG_E_SHAPE, "batched GEMM of a matrix without inputs");
    if (!L->gemm.xf) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        WPCG_HIP(hipStreamIsCapturing(s, &st));
        if (st != hipStreamCaptureStatusNone)
            return fail(WPCG_E_ARG, "the first batched call on a linear allocates its workspace: "
                                    "make it before capturing a graph");
        if (int rc = make_gemm(L, s)) return rc;
    }
    const uint32_t step = x_mode == GX_SPLIT ? GEMM_MAX_M_SPLIT : GEMM_MAX_M;
    for (uint32_t c = 0; c < M; c += step) {
        const int mc = (int)std::min<uint32_t>(step, M - c);
        WPCG_HIP(launch_gemm(m, L->gemm, x + (uint64_t)c * m.cols, x_mode, mc, L->bias,
                             res ? res + (uint64_t)c * m.rows : nullptr, y + (uint64_t)c * m.rows, s));
    }
    return WPCG_OK;
}

namespace {

int check_gemm_args(wpcg_linear* L, const void* x, int x_dtype, uint32_t M, const float* y)
{
    if (!L) return fail(WPCG_E_ARG, "null linear");
    if (x_dtype != WPCG_DTYPE_F32 && x_dtype != WPCG_DTYPE_BF16 && x_dtype != WPCG_DTYPE_F32_SPLIT)
        return fail(WPCG_E_ARG, "unknown x dtype");
    if (M && L->m.rows && (!y || (!x && L->m.cols))) return fail(WPCG_E_ARG, "null x or y");
    if ((uint64_t)M * L->m.cols > (1ull << 40)) return fail(WPCG_E_SHAPE, "batch too large");
    return check_ctx(L->ctx);
}

}  // namespace
}  // namespace wpcg

using namespace wpcg;

extern "C" {

int wpcg_linear_gemm(wpcg_linear* L, const void* x, int x_dtype, uint32_t M, float* y, wpcg_stream stream)
{
    if (int rc = check_gemm_args(L, x, x_dtype, M, y)) return rc;
    return run_gemm(L, x, x_dtype, M, y, pick(L->ctx, stream));
}

int wpcg_linear_gemm_noalloc(wpcg_linear* L, const void* x, int x_dtype, uint32_t M, float* y,
                             wpcg_stream stream)
{
    if (int rc = check_gemm_args(L, x, x_dtype, M, y)) return rc;
    const DeviceMatrix& m = L->m;
    hipStream_t s = pick(L->ctx, stream);
    if (M == 0 || m.rows == 0) return WPCG_OK;
    // the cases the matvec serves use no batched workspace
    if (m.nb == 0 || (x_dtype == WPCG_DTYPE_F32 && M == 1)) return run_gemm(L, x, x_dtype, M, y, s);
    // the workspace make_gemm would allocate, at 256-byte aligned offsets
    GemmWork w{};
    w.kg_req = L->gemm.kg_req;
    w.kg = gemm_kslices(m.rows, m.nb, w.kg_req);
    w.kg_small = gemm_small_kslices(m.rows, m.nb, w.kg_req);
    const uint64_t ncnt = std::max<uint64_t>(
        1, (uint64_t)std::max(gemm_row_groups(m.rows), gemm_small_row_groups(m.rows)));
    const uint64_t part = (w.kg > 1 || w.kg_small > 1)
                              ? std::max<uint64_t>((uint64_t)w.kg * GEMM_MAX_M, (uint64_t)w.kg_small * 16) *
                                    m.rows_pad * sizeof(float)
                              : 0;
    auto up = [](uint64_t b) { return (b + 255) / 256 * 256; };
    const uint64_t o_xsum = up(ncnt * sizeof(uint32_t));
    const uint64_t o_xf = o_xsum + up(m.nb * GEMM_MAX_M * sizeof(float));
    const uint64_t o_part = o_xf + up(m.nb * 4 * 4096);
    const uint64_t need = o_part + up(part);
    if (need > WPCG_NOALLOC_SCRATCH_BYTES)
        return fail(WPCG_E_UNSUPPORTED, "batched GEMM without allocation: this matrix needs " + std::to_string(need) +
                                            " bytes of workspace, the fixed array holds " +
                                            std::to_string(WPCG_NOALLOC_SCRATCH_BYTES));
    uint8_t* base = static_cast<uint8_t*>(scratch_ptr(L->ctx->device));
    if (!base) return fail(WPCG_E_DEVICE, "the no-allocation workspace is not set up on this device");
    w.counters = reinterpret_cast<uint32_t*>(base);
    w.xsum = reinterpret_cast<float*>(base + o_xsum);
    w.xf = base + o_xf;
    w.part = part ? reinterpret_cast<float*>(base + o_part) : nullptr;
    // the array keeps the last call's contents: the counters must start at 0
    WPCG_HIP(launch_fill_u32(w.counters, (int)ncnt, 0u, s));
    const uint64_t es = x_dtype == WPCG_DTYPE_BF16 ? 2 : 4;
    const uint32_t step = x_dtype == WPCG_DTYPE_F32_SPLIT ? GEMM_MAX_M_SPLIT : GEMM_MAX_M;
    for (uint32_t c = 0; c < M; c += step) {
        const int mc = (int)std::min<uint32_t>(step, M - c);
        WPCG_HIP(launch_gemm(m, w, static_cast<const uint8_t*>(x) + (uint64_t)c * m.cols * es, x_dtype, mc,
                             L->bias, nullptr, y + (uint64_t)c * m.rows, s));
    }
    return WPCG_OK;
}

int wpcg_linear_gemm_host(wpcg_linear* L, const void* x, int x_dtype, uint32_t M, float* y)
{
    if (int rc = check_gemm_args(L, x, x_dtype, M, y)) return rc;
    if (M == 0 || L->m.rows == 0) return WPCG_OK;
    const uint64_t xb = (uint64_t)M * L->m.cols * (x_dtype == WPCG_DTYPE_BF16 ? 2 : 4);
    const uint64_t yb = (uint64_t)M * L->m.rows * sizeof(float);
    std::lock_guard<std::mutex> g(L->host_mu);
    hipStream_t s = L->ctx->stream;
    void *dx = nullptr, *dy = nullptr;
    hipError_t e = hipMalloc(&dx, std::max<uint64_t>(xb, 4));
    if (e == hipSuccess) e = hipMalloc(&dy, yb);
    if (e == hipSuccess && xb) e = hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, s);
    int rc = e == hipSuccess ? run_gemm(L, dx, x_dtype, M, static_cast<float*>(dy), s) : hip_fail(e, "staging");
    if (rc == WPCG_OK) {
        e = hipMemcpyAsync(y, dy, yb, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "batched GEMM copy-back");
    } else {
        (void)hipStreamSynchronize(s);
    }
    if (dx) (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
    return rc;
}

int wpcg_linear_set_gemm_kslices(wpcg_linear* L, int kslices)
{
    if (!L) return fail(WPCG_E_ARG, "null linear");
    if (kslices < 0) return fail(WPCG_E_ARG, "kslices must be >= 0");
    if (int rc = check_ctx(L->ctx)) return rc;
    WPCG_HIP(hipStreamSynchronize(L->ctx->stream));
    free_gemm(L->gemm);
    L->gemm.kg_req = kslices;
    return WPCG_OK;
}

int wpcg_linear_gemm_kslices(wpcg_linear* L, int* kslices_small, int* kslices)
{
    if (!L || !kslices_small || !kslices) return fail(WPCG_E_ARG, "null argument");
    *kslices_small = L->gemm.xf ? L->gemm.kg_small : gemm_small_kslices(L->m.rows, L->m.nb, L->gemm.kg_req);
    *kslices = L->gemm.xf ? L->gemm.kg : gemm_kslices(L->m.rows, L->m.nb, L->gemm.kg_req);
    return WPCG_OK;
}

}  // extern "C"
