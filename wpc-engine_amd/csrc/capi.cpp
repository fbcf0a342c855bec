// The extern "C" boundary (include/wpcg.h): handles, status codes, the
// artifact reader and Linear/Embedding upload + dispatch.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <fstream>
#include <memory>
#include <new>
#include <sstream>

#include "wpcg_internal.hpp"

namespace wpcg {

namespace {
thread_local std::string g_last_error;
}

int fail(int code, const std::string& msg)
{
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what)
{
    return fail(WPCG_E_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

void ctx_retain(wpcg_ctx* c) { c->refs.fetch_add(1, std::memory_order_relaxed); }

void ctx_release(wpcg_ctx* c)
{
    if (c->refs.fetch_sub(1, std::memory_order_acq_rel) != 1) return;
    (void)hipSetDevice(c->device);
    if (c->stream) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipStreamDestroy(c->stream);
    }
    delete c;
}

hipStream_t pick(wpcg_ctx* ctx, wpcg_stream s)
{
    return s ? reinterpret_cast<hipStream_t>(s) : ctx->stream;
}

int check_ctx(wpcg_ctx* ctx)
{
    if (!ctx) return fail(WPCG_E_ARG, "null context");
    WPCG_HIP(hipSetDevice(ctx->device));
    return WPCG_OK;
}

uint64_t block_bytes(int scheme) { return scheme == 4 ? 68 : 100; }

void free_matrix(DeviceMatrix& m)
{
    if (m.codes) (void)hipFree(m.codes);
    if (m.hp) (void)hipFree(m.hp);
    if (m.params) (void)hipFree(m.params);
    m.codes = m.hp = nullptr;
    m.params = nullptr;
}

void free_plan(FastPlan& p)
{
    if (p.part) (void)hipFree(p.part);
    if (p.counters) (void)hipFree(p.counters);
    p.part = nullptr;
    p.counters = nullptr;
}

uint64_t plane_blocks(const DeviceMatrix& m) { return std::max<uint64_t>(1, m.rows_pad * m.nb); }

int alloc_planes(DeviceMatrix& m, uint64_t count, hipStream_t s)
{
    const uint64_t nb = std::max<uint64_t>(1, count * plane_blocks(m));
    WPCG_HIP(hipMalloc(&m.codes, nb * 64));
    WPCG_HIP(hipMalloc(&m.params, nb * 4));
    if (m.scheme == 3) WPCG_HIP(hipMalloc(&m.hp, nb * 32));
    WPCG_HIP(hipMemsetAsync(m.codes, 0, nb * 64, s));
    WPCG_HIP(hipMemsetAsync(m.params, 0, nb * 4, s));
    if (m.hp) WPCG_HIP(hipMemsetAsync(m.hp, 0, nb * 32, s));
    WPCG_HIP(hipStreamSynchronize(s));
    return WPCG_OK;
}

int upload_rows(wpcg_ctx* ctx, const uint8_t* blocks, const DeviceMatrix& m, uint64_t tile0)
{
    const uint64_t nb = m.nb;
    if (nb == 0 || m.rows == 0) return WPCG_OK;
    hipStream_t s = ctx->stream;
    const uint64_t bpb = block_bytes(m.scheme);
    const uint64_t base = tile0 * TILE_ROWS * nb;  // first block record of the range
    // ~4 MiB of codes per chunk, a whole number of tiles
    uint64_t chunk_rows = std::max<uint64_t>(TILE_ROWS, ((1u << 16) / nb) / TILE_ROWS * TILE_ROWS);
    std::vector<uint8_t> c(chunk_rows * nb * 64), h(m.scheme == 3 ? chunk_rows * nb * 32 : 0);
    std::vector<uint32_t> p(chunk_rows * nb);
    for (uint64_t r0 = 0; r0 < m.rows; r0 += chunk_rows) {
        const uint64_t n = std::min(chunk_rows, m.rows - r0);
        const uint64_t ntile_rows = (n + TILE_ROWS - 1) / TILE_ROWS * TILE_ROWS;
        std::fill(p.begin(), p.begin() + ntile_rows * nb, 0u);
        if (n != ntile_rows) {  // padding rows of a ragged last tile
            std::fill(c.begin(), c.begin() + ntile_rows * nb * 64, 0);
            std::fill(h.begin(), h.end(), 0);
        }
        // planes are tile-major, so whole tiles of rows are contiguous
        transcode_rows(m.scheme, blocks + r0 * nb * bpb, 0, n, nb, c.data(), h.data(), p.data());
        const uint64_t off = base + r0 * nb;
        WPCG_HIP(hipMemcpyAsync(m.codes + off * 64, c.data(), ntile_rows * nb * 64, hipMemcpyHostToDevice, s));
        WPCG_HIP(hipMemcpyAsync(m.params + off, p.data(), ntile_rows * nb * 4, hipMemcpyHostToDevice, s));
        if (m.hp)
            WPCG_HIP(hipMemcpyAsync(m.hp + off * 32, h.data(), ntile_rows * nb * 32, hipMemcpyHostToDevice, s));
        WPCG_HIP(hipStreamSynchronize(s));
    }
    return WPCG_OK;
}

int plan_kslices(uint64_t rows, uint64_t nb, int kg)
{
    const uint64_t mb = fast_max_slice(rows, nb);
    const int kmin = (int)std::max<uint64_t>(1, (nb + mb - 1) / mb);
    const int k = kg > 0 ? std::max(kmin, std::min(kg, (int)std::max<uint64_t>(1, nb)))
                         : fast_kslices(rows, nb);
    return fast_normalize_kslices(nb, k);
}

int make_plan(const DeviceMatrix& m, FastPlan& plan, hipStream_t s, int kg)
{
    plan.kg = plan_kslices(m.rows, m.nb, kg);
    if (plan.kg <= 1) return WPCG_OK;
    const uint64_t tiles = std::max<uint64_t>(1, m.rows_pad / TILE_ROWS);
    WPCG_HIP(hipMalloc(&plan.part, (uint64_t)plan.kg * m.rows_pad * sizeof(float)));
    WPCG_HIP(hipMalloc(&plan.counters, tiles * sizeof(uint32_t)));
    WPCG_HIP(hipMemsetAsync(plan.counters, 0, tiles * sizeof(uint32_t), s));
    WPCG_HIP(hipStreamSynchronize(s));
    return WPCG_OK;
}

namespace {

const char* meta_name(int scheme) { return scheme == 4 ? "model_v4.meta" : "model_v3.meta"; }
const char* wpc_name(int scheme) { return scheme == 4 ? "model_v4.wpc" : "model_v3.wpc"; }

// Transcodes reference blocks to the device planes and uploads them.
int upload_matrix(wpcg_ctx* ctx, const uint8_t* blocks, DeviceMatrix& m)
{
    if (int rc = alloc_planes(m, 1, ctx->stream)) return rc;
    return upload_rows(ctx, blocks, m, 0);
}

hipError_t run_gemv(wpcg_linear* L, const float* x, float* y, hipStream_t s)
{
    // K = 0 has no blocks to stream: the EXACT kernel writes 0 (+ bias)
    if (L->mode == WPCG_MODE_EXACT || L->m.nb == 0) return launch_gemv_exact(L->m, x, L->bias, y, s);
    GemvJob job{&L->m, &L->plan, x, L->bias, y};
    return launch_gemv_fast(&job, 1, s);
}

}  // namespace
}  // namespace wpcg

using namespace wpcg;

extern "C" {

const char* wpcg_last_error_string(void) { return g_last_error.c_str(); }

const char* wpcg_version(void) { return "wpcg 0.1 (gfx950)"; }

int wpcg_device_count(int* n)
{
    if (!n) return fail(WPCG_E_ARG, "null output");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    if (e != hipSuccess) {
        *n = 0;
        return hip_fail(e, "hipGetDeviceCount");
    }
    *n = c;
    return WPCG_OK;
}

// ---------------------------------------------------------------- context
int wpcg_ctx_create(int device, wpcg_ctx** out)
{
    if (!out) return fail(WPCG_E_ARG, "null output");
    *out = nullptr;
    int n = 0;
    if (int rc = wpcg_device_count(&n)) return rc;
    if (device < 0 || device >= n)
        return fail(WPCG_E_DEVICE, "device " + std::to_string(device) + " not present (" +
                                       std::to_string(n) + " visible)");
    WPCG_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    WPCG_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(WPCG_E_DEVICE, std::string("device is ") + prop.gcnArchName +
                                       "; this library is built for gfx950 only");
    std::unique_ptr<wpcg_ctx> c(new (std::nothrow) wpcg_ctx);
    if (!c) return fail(WPCG_E_NOMEM, "context allocation");
    c->device = device;
    if (int rc = scratch_setup(device)) return rc;  // the no-allocation workspace's address
    WPCG_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    *out = c.release();
    return WPCG_OK;
}

int wpcg_ctx_destroy(wpcg_ctx* ctx)
{
    if (!ctx) return WPCG_OK;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    ctx_release(ctx);
    return WPCG_OK;
}

int wpcg_ctx_stream(wpcg_ctx* ctx, wpcg_stream* out)
{
    if (!ctx || !out) return fail(WPCG_E_ARG, "null argument");
    *out = reinterpret_cast<wpcg_stream>(ctx->stream);
    return WPCG_OK;
}

int wpcg_ctx_sync(wpcg_ctx* ctx)
{
    if (int rc = check_ctx(ctx)) return rc;
    WPCG_HIP(hipStreamSynchronize(ctx->stream));
    return WPCG_OK;
}

int wpcg_dev_alloc(wpcg_ctx* ctx, size_t bytes, void** out_dev)
{
    if (!out_dev) return fail(WPCG_E_ARG, "null output");
    *out_dev = nullptr;
    if (int rc = check_ctx(ctx)) return rc;
    hipError_t e = hipMalloc(out_dev, bytes ? bytes : 1);
    if (e != hipSuccess) return fail(WPCG_E_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    return WPCG_OK;
}

int wpcg_dev_free(wpcg_ctx* ctx, void* dev)
{
    if (int rc = check_ctx(ctx)) return rc;
    if (dev) WPCG_HIP(hipFree(dev));
    return WPCG_OK;
}

static int copy(wpcg_ctx* ctx, void* dst, const void* src, size_t bytes, hipMemcpyKind k)
{
    if (int rc = check_ctx(ctx)) return rc;
    if (!bytes) return WPCG_OK;
    if (!dst || !src) return fail(WPCG_E_ARG, "null copy pointer");
    WPCG_HIP(hipMemcpyAsync(dst, src, bytes, k, ctx->stream));
    WPCG_HIP(hipStreamSynchronize(ctx->stream));
    return WPCG_OK;
}

int wpcg_memcpy_h2d(wpcg_ctx* ctx, void* d, const void* s, size_t n) { return copy(ctx, d, s, n, hipMemcpyHostToDevice); }
int wpcg_memcpy_d2h(wpcg_ctx* ctx, void* d, const void* s, size_t n) { return copy(ctx, d, s, n, hipMemcpyDeviceToHost); }
int wpcg_memcpy_d2d(wpcg_ctx* ctx, void* d, const void* s, size_t n) { return copy(ctx, d, s, n, hipMemcpyDeviceToDevice); }

int wpcg_event_create(wpcg_ctx* ctx, wpcg_event** out)
{
    if (!out) return fail(WPCG_E_ARG, "null output");
    *out = nullptr;
    if (int rc = check_ctx(ctx)) return rc;
    std::unique_ptr<wpcg_event> ev(new (std::nothrow) wpcg_event);
    if (!ev) return fail(WPCG_E_NOMEM, "event allocation");
    ev->ctx = ctx;
    WPCG_HIP(hipEventCreate(&ev->ev));
    ctx_retain(ctx);
    *out = ev.release();
    return WPCG_OK;
}

int wpcg_event_destroy(wpcg_event* ev)
{
    if (!ev) return WPCG_OK;
    (void)hipSetDevice(ev->ctx->device);
    (void)hipEventDestroy(ev->ev);
    ctx_release(ev->ctx);
    delete ev;
    return WPCG_OK;
}

int wpcg_event_record(wpcg_event* ev, wpcg_stream stream)
{
    if (!ev) return fail(WPCG_E_ARG, "null event");
    if (int rc = check_ctx(ev->ctx)) return rc;
    WPCG_HIP(hipEventRecord(ev->ev, pick(ev->ctx, stream)));
    return WPCG_OK;
}

int wpcg_event_elapsed_ms(wpcg_event* a, wpcg_event* b, float* ms)
{
    if (!a || !b || !ms) return fail(WPCG_E_ARG, "null argument");
    WPCG_HIP(hipEventSynchronize(b->ev));
    WPCG_HIP(hipEventElapsedTime(ms, a->ev, b->ev));
    return WPCG_OK;
}

// ---------------------------------------------------------------- artifact
int wpcg_artifact_open(const char* dir, int scheme, wpcg_artifact** out)
{
    if (!out) return fail(WPCG_E_ARG, "null output");
    *out = nullptr;
    if (!dir) return fail(WPCG_E_ARG, "null directory");
    if (scheme != 3 && scheme != 4) return fail(WPCG_E_ARG, "scheme must be 3 or 4");
    const std::string base(dir);
    const std::string meta_path = base + "/" + meta_name(scheme);
    std::ifstream f(meta_path, std::ios::binary);
    if (!f) return fail(WPCG_E_IO, "cannot read " + meta_path);
    std::stringstream ss;
    ss << f.rdbuf();
    std::unique_ptr<wpcg_artifact> a(new (std::nothrow) wpcg_artifact);
    if (!a) return fail(WPCG_E_NOMEM, "artifact allocation");
    a->scheme = scheme;
    uint64_t bs = 0;
    if (int rc = parse_meta(ss.str(), a->tensors, bs)) return rc;
    // WpcModelDataV4::open (wpc_weights_v4.rs:51-56)
    if (bs != 128)
        return fail(WPCG_E_FORMAT, std::string(meta_name(scheme)) + " block_size " +
                                       std::to_string(bs) + " doesn't match 128");
    const std::string wpc_path = base + "/" + wpc_name(scheme);
    int fd = ::open(wpc_path.c_str(), O_RDONLY);
    if (fd < 0) return fail(WPCG_E_IO, "cannot open " + wpc_path);
    struct stat st;
    if (fstat(fd, &st) != 0) { ::close(fd); return fail(WPCG_E_IO, "cannot stat " + wpc_path); }
    a->map_size = (uint64_t)st.st_size;
    if (a->map_size) {
        void* p = mmap(nullptr, a->map_size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) { ::close(fd); return fail(WPCG_E_IO, "cannot mmap " + wpc_path); }
        a->map = static_cast<const uint8_t*>(p);
    }
    ::close(fd);
    *out = a.release();
    return WPCG_OK;
}

int wpcg_artifact_close(wpcg_artifact* a)
{
    if (!a) return WPCG_OK;
    if (a->map) munmap(const_cast<uint8_t*>(a->map), a->map_size);
    delete a;
    return WPCG_OK;
}

int wpcg_artifact_tensor(wpcg_artifact* a, const char* name, const void** bytes, uint64_t* size)
{
    if (!a || !name || !bytes || !size) return fail(WPCG_E_ARG, "null argument");
    auto it = a->tensors.find(name);
    if (it == a->tensors.end())
        return fail(WPCG_E_NOTFOUND, std::string("tensor ") + name + " not found in " + meta_name(a->scheme));
    const MetaEntry& e = it->second;
    if (e.offset > a->map_size || e.size > a->map_size - e.offset)
        return fail(WPCG_E_FORMAT, std::string("tensor ") + name + " range [" +
                                       std::to_string(e.offset) + ", +" + std::to_string(e.size) +
                                       ") exceeds the " + std::to_string(a->map_size) + "-byte file");
    // blocks_for (wpc_weights_v4.rs:92-98)
    if (e.size % block_bytes(a->scheme) != 0)
        return fail(WPCG_E_FORMAT, std::string("misaligned v") + std::to_string(a->scheme) +
                                       " block range for tensor " + name);
    *bytes = a->map + e.offset;
    *size = e.size;
    return WPCG_OK;
}

int wpcg_artifact_tensor_count(wpcg_artifact* a, uint64_t* n)
{
    if (!a || !n) return fail(WPCG_E_ARG, "null argument");
    *n = a->tensors.size();
    return WPCG_OK;
}

// ---------------------------------------------------------------- linear
int wpcg_linear_from_blocks(wpcg_ctx* ctx, int scheme, const void* blocks, uint64_t nbytes,
                            uint64_t out_f, uint64_t in_f, const float* bias, wpcg_linear** out)
{
    if (!out) return fail(WPCG_E_ARG, "null output");
    *out = nullptr;
    if (scheme != 3 && scheme != 4) return fail(WPCG_E_ARG, "scheme must be 3 or 4");
    if (!blocks && nbytes) return fail(WPCG_E_ARG, "null blocks");
    // WpcLinearV4::new (wpc_weights_v4.rs:134-147)
    if (in_f % 128 != 0)
        return fail(WPCG_E_SHAPE, "in_features must be a multiple of 128 for WPC v" +
                                      std::to_string(scheme) + " blocks");
    const uint64_t bpb = block_bytes(scheme);
    if (nbytes % bpb != 0)
        return fail(WPCG_E_FORMAT, "misaligned v" + std::to_string(scheme) + " block range");
    const uint64_t expected = out_f * (in_f / 128);
    if (nbytes / bpb != expected)
        return fail(WPCG_E_SHAPE, "v" + std::to_string(scheme) + " block count mismatch (data holds " +
                                      std::to_string(nbytes / bpb) + ", shape implies " +
                                      std::to_string(expected) + ")");
    if (in_f / 128 > (uint64_t)INT32_MAX || out_f > (uint64_t)INT32_MAX)
        return fail(WPCG_E_SHAPE, "matrix too large");
    if (int rc = check_ctx(ctx)) return rc;
    std::unique_ptr<wpcg_linear> L(new (std::nothrow) wpcg_linear);
    if (!L) return fail(WPCG_E_NOMEM, "linear allocation");
    L->ctx = ctx;
    L->m.scheme = scheme;
    L->m.rows = out_f;
    L->m.cols = in_f;
    L->m.nb = in_f / 128;
    L->m.rows_pad = pad_rows(out_f);
    int rc = upload_matrix(ctx, static_cast<const uint8_t*>(blocks), L->m);
    if (rc == WPCG_OK) rc = make_plan(L->m, L->plan, ctx->stream);
    if (rc == WPCG_OK && bias) {
        hipError_t e = hipMalloc(&L->bias, (out_f ? out_f : 1) * sizeof(float));
        if (e == hipSuccess)
            e = hipMemcpy(L->bias, bias, out_f * sizeof(float), hipMemcpyHostToDevice);
        if (e != hipSuccess) rc = hip_fail(e, "bias upload");
    }
    if (rc != WPCG_OK) {
        free_matrix(L->m);
        free_plan(L->plan);
        if (L->bias) (void)hipFree(L->bias);
        return rc;
    }
    ctx_retain(ctx);
    *out = L.release();
    return WPCG_OK;
}

int wpcg_linear_create(wpcg_ctx* ctx, wpcg_artifact* a, const char* name, uint64_t out_f,
                       uint64_t in_f, const float* bias, wpcg_linear** out)
{
    if (!out) return fail(WPCG_E_ARG, "null output");
    *out = nullptr;
    if (!a || !name) return fail(WPCG_E_ARG, "null argument");
    if (in_f % 128 != 0)
        return fail(WPCG_E_SHAPE, "in_features must be a multiple of 128 for WPC v" +
                                      std::to_string(a->scheme) + " blocks");
    const void* bytes;
    uint64_t size;
    if (int rc = wpcg_artifact_tensor(a, name, &bytes, &size)) return rc;
    const uint64_t bpb = block_bytes(a->scheme), expected = out_f * (in_f / 128);
    if (size / bpb != expected)
        return fail(WPCG_E_SHAPE, std::string("tensor ") + name + ": v" + std::to_string(a->scheme) +
                                      " block count mismatch (meta says " + std::to_string(size / bpb) +
                                      ", shape implies " + std::to_string(expected) + ")");
    return wpcg_linear_from_blocks(ctx, a->scheme, bytes, size, out_f, in_f, bias, out);
}

int wpcg_linear_destroy(wpcg_linear* L)
{
    if (!L) return WPCG_OK;
    (void)hipSetDevice(L->ctx->device);
    (void)hipStreamSynchronize(L->ctx->stream);
    free_matrix(L->m);
    free_plan(L->plan);
    free_gemm(L->gemm);
    if (L->bias) (void)hipFree(L->bias);
    if (L->x_stage) (void)hipFree(L->x_stage);
    if (L->y_stage) (void)hipFree(L->y_stage);
    ctx_release(L->ctx);
    delete L;
    return WPCG_OK;
}

int wpcg_linear_shape(wpcg_linear* L, uint64_t* out_f, uint64_t* in_f)
{
    if (!L || !out_f || !in_f) return fail(WPCG_E_ARG, "null argument");
    *out_f = L->m.rows;
    *in_f = L->m.cols;
    return WPCG_OK;
}

int wpcg_linear_set_mode(wpcg_linear* L, int mode)
{
    if (!L) return fail(WPCG_E_ARG, "null linear");
    if (mode != WPCG_MODE_EXACT && mode != WPCG_MODE_FAST) return fail(WPCG_E_ARG, "unknown mode");
    L->mode = mode;
    return WPCG_OK;
}

int wpcg_linear_set_kslices(wpcg_linear* L, int kslices)
{
    if (!L) return fail(WPCG_E_ARG, "null linear");
    if (kslices < 0) return fail(WPCG_E_ARG, "kslices must be >= 0");
    if (int rc = check_ctx(L->ctx)) return rc;
    WPCG_HIP(hipStreamSynchronize(L->ctx->stream));
    free_plan(L->plan);
    if (int rc = make_plan(L->m, L->plan, L->ctx->stream, kslices)) {
        free_plan(L->plan);
        L->plan.kg = 1;
        return rc;
    }
    return WPCG_OK;
}

int wpcg_linear_set_fast_kernel(wpcg_linear* L, int kernel)
{
    if (!L) return fail(WPCG_E_ARG, "null linear");
    if (kernel != WPCG_FAST_KERNEL_MFMA && kernel != WPCG_FAST_KERNEL_VALU)
        return fail(WPCG_E_ARG, "kernel must be WPCG_FAST_KERNEL_MFMA or WPCG_FAST_KERNEL_VALU");
    L->plan.valu = kernel == WPCG_FAST_KERNEL_VALU;
    return WPCG_OK;
}

int wpcg_linear_kslices(wpcg_linear* L, int* kslices)
{
    if (!L || !kslices) return fail(WPCG_E_ARG, "null argument");
    *kslices = L->plan.kg;
    return WPCG_OK;
}

int wpcg_plan_kslices(uint64_t out_f, uint64_t in_f, int requested, int* kslices)
{
    if (!kslices) return fail(WPCG_E_ARG, "null output");
    if (in_f % 128 != 0) return fail(WPCG_E_SHAPE, "in_features must be a multiple of 128");
    if (requested < 0) return fail(WPCG_E_ARG, "requested must be >= 0");
    *kslices = plan_kslices(out_f, in_f / 128, requested);
    return WPCG_OK;
}

int wpcg_linear_device_bytes(wpcg_linear* L, uint64_t* bytes)
{
    if (!L || !bytes) return fail(WPCG_E_ARG, "null argument");
    const uint64_t nb = L->m.rows * L->m.nb;
    *bytes = nb * (L->m.scheme == 4 ? 68 : 100);
    return WPCG_OK;
}

int wpcg_linear_matvec(wpcg_linear* L, const float* x, float* y, wpcg_stream stream)
{
    if (!L) return fail(WPCG_E_ARG, "null linear");
    if (int rc = check_ctx(L->ctx)) return rc;
    if (L->m.rows == 0) return WPCG_OK;
    if (!y || (!x && L->m.cols)) return fail(WPCG_E_ARG, "null x or y");
    WPCG_HIP(run_gemv(L, x, y, pick(L->ctx, stream)));
    return WPCG_OK;
}

int wpcg_linear_matvec_multi(int n, wpcg_linear* const* lins, const float* const* xs,
                             float* const* ys, wpcg_stream stream)
{
    if (n < 0 || (n > 0 && (!lins || !xs || !ys))) return fail(WPCG_E_ARG, "null argument");
    if (n == 0) return WPCG_OK;
    wpcg_ctx* ctx = nullptr;
    for (int i = 0; i < n; i++) {
        if (!lins[i]) return fail(WPCG_E_ARG, "null linear in group");
        if (!ctx) ctx = lins[i]->ctx;
        if (lins[i]->ctx->device != ctx->device)
            return fail(WPCG_E_ARG, "linears of one group must share a device");
        if (lins[i]->m.rows && (!ys[i] || (!xs[i] && lins[i]->m.cols)))
            return fail(WPCG_E_ARG, "null x or y in group");
    }
    if (int rc = check_ctx(ctx)) return rc;
    hipStream_t s = pick(ctx, stream);
    // members of one scheme and mode share launches of up to MAX_JOBS
    for (int scheme : {3, 4}) {
        GemvJob jobs[MAX_JOBS], ejobs[MAX_JOBS];
        int nj = 0, ne = 0;
        for (int i = 0; i < n; i++) {
            wpcg_linear* L = lins[i];
            if (L->m.scheme != scheme || L->m.rows == 0) continue;
            if (L->m.nb == 0) {
                WPCG_HIP(launch_gemv_exact(L->m, xs[i], L->bias, ys[i], s));
                continue;
            }
            if (L->mode == WPCG_MODE_EXACT) {
                ejobs[ne++] = GemvJob{&L->m, &L->plan, xs[i], L->bias, ys[i]};
                if (ne == MAX_JOBS) {
                    WPCG_HIP(launch_gemv_exact_multi(ejobs, ne, s));
                    ne = 0;
                }
                continue;
            }
            jobs[nj++] = GemvJob{&L->m, &L->plan, xs[i], L->bias, ys[i]};
            if (nj == MAX_JOBS) {
                WPCG_HIP(launch_gemv_fast(jobs, nj, s));
                nj = 0;
            }
        }
        if (nj) WPCG_HIP(launch_gemv_fast(jobs, nj, s));
        if (ne) WPCG_HIP(launch_gemv_exact_multi(ejobs, ne, s));
    }
    return WPCG_OK;
}

int wpcg_linear_matvec_host(wpcg_linear* L, const float* x, float* y)
{
    if (!L) return fail(WPCG_E_ARG, "null linear");
    if (int rc = check_ctx(L->ctx)) return rc;
    if (L->m.rows == 0) return WPCG_OK;
    if (!y || (!x && L->m.cols)) return fail(WPCG_E_ARG, "null x or y");
    std::lock_guard<std::mutex> g(L->host_mu);
    if (!L->x_stage) WPCG_HIP(hipMalloc(&L->x_stage, (L->m.cols ? L->m.cols : 1) * sizeof(float)));
    if (!L->y_stage) WPCG_HIP(hipMalloc(&L->y_stage, L->m.rows * sizeof(float)));
    hipStream_t s = L->ctx->stream;
    if (L->m.cols)
        WPCG_HIP(hipMemcpyAsync(L->x_stage, x, L->m.cols * sizeof(float), hipMemcpyHostToDevice, s));
    WPCG_HIP(run_gemv(L, L->x_stage, L->y_stage, s));
    WPCG_HIP(hipMemcpyAsync(y, L->y_stage, L->m.rows * sizeof(float), hipMemcpyDeviceToHost, s));
    WPCG_HIP(hipStreamSynchronize(s));
    return WPCG_OK;
}

int wpcg_linear_embed(wpcg_linear* L, uint32_t token, float* out, wpcg_stream stream)
{
    if (!L) return fail(WPCG_E_ARG, "null linear");
    if (int rc = check_ctx(L->ctx)) return rc;
    if (token >= L->m.rows)
        return fail(WPCG_E_ARG, "token " + std::to_string(token) + " >= vocab " + std::to_string(L->m.rows));
    if (L->m.cols == 0) return WPCG_OK;
    if (!out) return fail(WPCG_E_ARG, "null output");
    WPCG_HIP(launch_embed(L->m, token, out, pick(L->ctx, stream)));
    return WPCG_OK;
}

int wpcg_linear_embed_host(wpcg_linear* L, uint32_t token, float* out)
{
    if (!L) return fail(WPCG_E_ARG, "null linear");
    if (int rc = check_ctx(L->ctx)) return rc;
    if (token >= L->m.rows)
        return fail(WPCG_E_ARG, "token " + std::to_string(token) + " >= vocab " + std::to_string(L->m.rows));
    if (L->m.cols == 0) return WPCG_OK;
    if (!out) return fail(WPCG_E_ARG, "null output");
    std::lock_guard<std::mutex> g(L->host_mu);
    if (!L->x_stage) WPCG_HIP(hipMalloc(&L->x_stage, L->m.cols * sizeof(float)));
    hipStream_t s = L->ctx->stream;
    WPCG_HIP(launch_embed(L->m, token, L->x_stage, s));
    WPCG_HIP(hipMemcpyAsync(out, L->x_stage, L->m.cols * sizeof(float), hipMemcpyDeviceToHost, s));
    WPCG_HIP(hipStreamSynchronize(s));
    return WPCG_OK;
}

int wpcg_linear_clone(wpcg_linear* L, wpcg_linear** out)
{
    if (!L || !out) return fail(WPCG_E_ARG, "null argument");
    *out = nullptr;
    if (int rc = check_ctx(L->ctx)) return rc;
    std::unique_ptr<wpcg_linear> c(new (std::nothrow) wpcg_linear);
    if (!c) return fail(WPCG_E_NOMEM, "linear allocation");
    c->ctx = L->ctx;
    c->m = L->m;
    c->m.codes = c->m.hp = nullptr;
    c->m.params = nullptr;
    c->mode = L->mode;
    c->gemm.kg_req = L->gemm.kg_req;  // the same batched split, made on first use
    const uint64_t nb = plane_blocks(L->m);
    hipStream_t s = L->ctx->stream;
    if (int rc = make_plan(c->m, c->plan, s, L->plan.kg)) {  // same split: same results
        free_plan(c->plan);
        return rc;
    }
    c->plan.valu = L->plan.valu;
    auto dup = [&](void** dst, const void* src, size_t n) -> hipError_t {
        hipError_t e = hipMalloc(dst, n);
        if (e == hipSuccess) e = hipMemcpyAsync(*dst, src, n, hipMemcpyDeviceToDevice, s);
        return e;
    };
    hipError_t e = dup((void**)&c->m.codes, L->m.codes, nb * 64);
    if (e == hipSuccess) e = dup((void**)&c->m.params, L->m.params, nb * 4);
    if (e == hipSuccess && L->m.hp) e = dup((void**)&c->m.hp, L->m.hp, nb * 32);
    if (e == hipSuccess && L->bias) e = dup((void**)&c->bias, L->bias, std::max<uint64_t>(1, L->m.rows) * 4);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        free_matrix(c->m);
        free_plan(c->plan);
        if (c->bias) (void)hipFree(c->bias);
        return hip_fail(e, "clone");
    }
    ctx_retain(c->ctx);
    *out = c.release();
    return WPCG_OK;
}

int wpcg_graph_begin(wpcg_ctx* ctx)
{
    if (int rc = check_ctx(ctx)) return rc;
    WPCG_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return WPCG_OK;
}

int wpcg_graph_end(wpcg_ctx* ctx, wpcg_graph** out)
{
    if (!out) return fail(WPCG_E_ARG, "null output");
    *out = nullptr;
    if (int rc = check_ctx(ctx)) return rc;
    std::unique_ptr<wpcg_graph> g(new (std::nothrow) wpcg_graph);
    if (!g) return fail(WPCG_E_NOMEM, "graph allocation");
    g->ctx = ctx;
    WPCG_HIP(hipStreamEndCapture(ctx->stream, &g->graph));
    hipError_t e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g->graph);
        return hip_fail(e, "hipGraphInstantiate");
    }
    ctx_retain(ctx);
    *out = g.release();
    return WPCG_OK;
}

int wpcg_graph_launch(wpcg_graph* g, wpcg_stream stream)
{
    if (!g) return fail(WPCG_E_ARG, "null graph");
    if (int rc = check_ctx(g->ctx)) return rc;
    WPCG_HIP(hipGraphLaunch(g->exec, pick(g->ctx, stream)));
    return WPCG_OK;
}

int wpcg_graph_destroy(wpcg_graph* g)
{
    if (!g) return WPCG_OK;
    (void)hipSetDevice(g->ctx->device);
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    ctx_release(g->ctx);
    delete g;
    return WPCG_OK;
}

int wpcg_linear_dequant(wpcg_linear* L, int rounding, float* w, wpcg_stream stream)
{
    if (!L) return fail(WPCG_E_ARG, "null linear");
    if (rounding != WPCG_ROUND_FMA && rounding != WPCG_ROUND_TWO) return fail(WPCG_E_ARG, "unknown rounding");
    if (int rc = check_ctx(L->ctx)) return rc;
    if (L->m.rows * L->m.cols == 0) return WPCG_OK;
    if (!w) return fail(WPCG_E_ARG, "null output");
    WPCG_HIP(launch_dequant(L->m, rounding, w, pick(L->ctx, stream)));
    return WPCG_OK;
}

}  // extern "C"
