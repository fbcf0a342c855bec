// The extern "C" boundary for the Qwen3-MoE sparse MLP (include/wpcg.h):
// fp32 dense linear (router), softmax, routing, SiLU*up and the routed
// expert FFN of one layer.
#include <algorithm>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "wpcg_internal.hpp"

using namespace wpcg;

namespace {

int valid_mode(int mode) { return mode == WPCG_MODE_EXACT || mode == WPCG_MODE_FAST; }

void free_dense(wpcg_dense* d)
{
    if (d->w) (void)hipFree(d->w);
    if (d->bias) (void)hipFree(d->bias);
}

void free_moe(wpcg_moe* m)
{
    free_matrix(m->gate);
    free_matrix(m->up);
    free_matrix(m->down);
    free_plan(m->plan);
    for (void* p : {(void*)m->scores, (void*)m->w, (void*)m->g, (void*)m->u, (void*)m->h,
                    (void*)m->ys, (void*)m->ids, (void*)m->xn})
        if (p) (void)hipFree(p);
    if (m->router) {
        free_dense(m->router);
        ctx_release(m->router->ctx);
        delete m->router;
    }
}

// One expert's matrix of the stack: `rows` x `cols` in `scheme` blocks.
DeviceMatrix expert_view(int scheme, uint64_t rows, uint64_t cols)
{
    DeviceMatrix v;
    v.scheme = scheme;
    v.rows = rows;
    v.cols = cols;
    v.nb = cols / 128;
    v.rows_pad = pad_rows(rows);
    return v;
}

}  // namespace

// x_add (FAST, routed, with nw): the layer input is x + x_add, a deferred
// K-slice of the GEMV that wrote x; the router and gate/up add it as they
// read x, and the down projection adds it to `add`.
int wpcg::moe_run(wpcg_moe* m, const float* x_dev, float* out_dev, const float* add, hipStream_t s,
                  const float* nw, float eps, const float* x_add, bool defer_combine)
{
    const int K = (int)m->top_k, H = (int)m->hidden, I = (int)m->inter;
    if (x_add && !(m->mode == WPCG_MODE_FAST && m->routed && nw && add))
        return fail(WPCG_E_UNSUPPORTED, "a deferred input slice needs the FAST routed path");
    if (m->mode == WPCG_MODE_FAST && m->routed) {
        WPCG_HIP(launch_dense(m->router->w, (int)m->n_exp, H, m->mode, x_dev, nullptr, m->scores, s, nw, eps,
                              x_add));
        GemvJob jobs[MAX_JOBS];
        for (int k = 0; k < 2 * K; k++) {
            GemvJob& J = jobs[k];
            J = GemvJob{k % 2 ? &m->up : &m->gate, &m->plan, x_dev, nullptr,
                        (k % 2 ? m->u : m->g) + (size_t)(k / 2) * I};
            J.sel_k = k / 2;
            J.xform = nw ? XF_NORM : XF_NONE;
            J.nw = nw;
            J.eps = eps;
            J.scores = m->scores;
            J.n_exp = (int)m->n_exp;
            J.top_k = K;
            J.norm_topk = m->norm_topk;
            J.ids_out = m->ids;
            J.w_out = m->w;
            J.x_add = x_add;
        }
        WPCG_HIP(launch_gemv_fast(jobs, 2 * K, s));
        GemvJob down{&m->down, &m->plan, m->g, add, out_dev, m->ids};
        down.xform = XF_SILU;
        down.x2 = m->u;
        down.routed = 1;
        down.rw = m->w;
        down.top_k = K;
        down.bias2 = x_add;
        WPCG_HIP(launch_gemv_fast(&down, 1, s));
        return WPCG_OK;
    }
    if (nw) {  // the norm in a launch of its own
        WPCG_HIP(launch_rms_norm(m->mode, x_dev, nw, H, eps, m->xn, s));
        x_dev = m->xn;
    }
    WPCG_HIP(launch_dense(m->router->w, (int)m->n_exp, H, m->mode, x_dev, nullptr, m->scores, s));
    // EXACT: the gate/up launch routes itself when it holds every chosen
    // expert's two GEMVs (one launch); otherwise a routing launch first
    const bool self_route = m->mode == WPCG_MODE_EXACT && 2 * K <= MAX_JOBS;
    if (!self_route)
        WPCG_HIP(launch_softmax_route(m->scores, (int)m->n_exp, K, m->norm_topk, m->ids, m->w, s));
    // gate and up of the chosen experts, then SiLU(gate) * up
    if (m->mode == WPCG_MODE_FAST) {
        GemvJob jobs[MAX_JOBS];
        for (int k = 0; k < K; k++) {
            jobs[2 * k] = GemvJob{&m->gate, &m->plan, x_dev, nullptr, m->g + (size_t)k * I, m->ids, k};
            jobs[2 * k + 1] = GemvJob{&m->up, &m->plan, x_dev, nullptr, m->u + (size_t)k * I, m->ids, k};
        }
        WPCG_HIP(launch_gemv_fast(jobs, 2 * K, s));
    } else {  // the chosen experts' gate and up, MAX_JOBS GEMVs per launch
        GemvJob jobs[2 * MAX_JOBS];
        for (int k = 0; k < K; k++) {
            jobs[2 * k] = GemvJob{&m->gate, &m->plan, x_dev, nullptr, m->g + (size_t)k * I, m->ids, k};
            jobs[2 * k + 1] = GemvJob{&m->up, &m->plan, x_dev, nullptr, m->u + (size_t)k * I, m->ids, k};
        }
        if (self_route)
            for (int j = 0; j < 2 * K; j++) {
                GemvJob& J = jobs[j];
                J.sel = nullptr;
                J.scores = m->scores;
                J.n_exp = (int)m->n_exp;
                J.top_k = K;
                J.norm_topk = m->norm_topk;
                J.ids_out = m->ids;
                J.w_out = m->w;
            }
        for (int j0 = 0; j0 < 2 * K; j0 += MAX_JOBS)
            WPCG_HIP(launch_gemv_exact_multi(jobs + j0, std::min(MAX_JOBS, 2 * K - j0), s));
    }
    WPCG_HIP(launch_silu_mul(m->g, m->u, m->h, (size_t)K * I, s));
    // down of the chosen experts, then the weighted sum in chosen order
    if (m->mode == WPCG_MODE_FAST) {
        GemvJob jobs[MAX_JOBS];
        for (int k = 0; k < K; k++)
            jobs[k] = GemvJob{&m->down, &m->plan, m->h + (size_t)k * I, nullptr, m->ys + (size_t)k * H,
                              m->ids, k};
        WPCG_HIP(launch_gemv_fast(jobs, K, s));
    } else {
        GemvJob jobs[MAX_JOBS];
        for (int k = 0; k < K; k++)
            jobs[k] = GemvJob{&m->down, &m->plan, m->h + (size_t)k * I, nullptr, m->ys + (size_t)k * H, m->ids, k};
        WPCG_HIP(launch_gemv_exact_multi(jobs, K, s));
    }
    if (defer_combine && m->mode == WPCG_MODE_EXACT) return WPCG_OK;  // folded into the caller's next norm
    WPCG_HIP(launch_combine(m->ys, m->ids, m->w, K, out_dev, H, add, s));
    return WPCG_OK;
}

extern "C" {

// ------------------------------------------------------------ dense linear
int wpcg_dense_create(wpcg_ctx* ctx, const float* w, uint64_t out_f, uint64_t in_f,
                      const float* bias, wpcg_dense** out)
{
    if (!out) return fail(WPCG_E_ARG, "null output");
    *out = nullptr;
    if (!w || out_f == 0 || in_f == 0) return fail(WPCG_E_ARG, "empty or null weight");
    if (out_f > (1u << 30) || in_f > (1u << 30)) return fail(WPCG_E_SHAPE, "dense shape too large");
    if (int rc = check_ctx(ctx)) return rc;
    std::unique_ptr<wpcg_dense> d(new (std::nothrow) wpcg_dense);
    if (!d) return fail(WPCG_E_NOMEM, "dense allocation");
    d->ctx = ctx;
    d->out_f = out_f;
    d->in_f = in_f;
    hipError_t e = hipMalloc(&d->w, out_f * in_f * sizeof(float));
    if (e == hipSuccess) e = hipMemcpy(d->w, w, out_f * in_f * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess && bias) {
        e = hipMalloc(&d->bias, out_f * sizeof(float));
        if (e == hipSuccess) e = hipMemcpy(d->bias, bias, out_f * sizeof(float), hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        free_dense(d.get());
        return hip_fail(e, "dense upload");
    }
    ctx_retain(ctx);
    *out = d.release();
    return WPCG_OK;
}

int wpcg_dense_destroy(wpcg_dense* d)
{
    if (!d) return WPCG_OK;
    (void)hipSetDevice(d->ctx->device);
    (void)hipStreamSynchronize(d->ctx->stream);
    free_dense(d);
    ctx_release(d->ctx);
    delete d;
    return WPCG_OK;
}

int wpcg_dense_set_mode(wpcg_dense* d, int mode)
{
    if (!d || !valid_mode(mode)) return fail(WPCG_E_ARG, "null dense or bad mode");
    d->mode = mode;
    return WPCG_OK;
}

int wpcg_dense_matvec(wpcg_dense* d, const float* x_dev, float* y_dev, wpcg_stream stream)
{
    if (!d || !x_dev || !y_dev) return fail(WPCG_E_ARG, "null argument");
    if (int rc = check_ctx(d->ctx)) return rc;
    WPCG_HIP(launch_dense(d->w, (int)d->out_f, (int)d->in_f, d->mode, x_dev, d->bias, y_dev,
                          pick(d->ctx, stream)));
    return WPCG_OK;
}

// ------------------------------------------------------------ elementwise
int wpcg_softmax(wpcg_ctx* ctx, float* x_dev, uint32_t n, wpcg_stream stream)
{
    if (!x_dev && n) return fail(WPCG_E_ARG, "null input");
    if (int rc = check_ctx(ctx)) return rc;
    if (n == 0) return WPCG_OK;
    WPCG_HIP(launch_softmax(x_dev, (int)n, pick(ctx, stream)));
    return WPCG_OK;
}

int wpcg_route(wpcg_ctx* ctx, const float* probs_dev, uint32_t n, uint32_t top_k, int norm_topk,
               int32_t* ids_dev, float* weights_dev, wpcg_stream stream)
{
    if (!probs_dev || !ids_dev || !weights_dev) return fail(WPCG_E_ARG, "null argument");
    if (n == 0 || n > (uint32_t)route_max_n() || top_k == 0 || top_k > n)
        return fail(WPCG_E_ARG, "route needs 0 < top_k <= n <= " + std::to_string(route_max_n()));
    if (int rc = check_ctx(ctx)) return rc;
    WPCG_HIP(launch_route(probs_dev, (int)n, (int)top_k, norm_topk ? 1 : 0, ids_dev, weights_dev,
                          pick(ctx, stream)));
    return WPCG_OK;
}

int wpcg_silu_mul(wpcg_ctx* ctx, const float* g_dev, const float* u_dev, float* out_dev,
                  uint64_t n, wpcg_stream stream)
{
    if ((!g_dev || !u_dev || !out_dev) && n) return fail(WPCG_E_ARG, "null argument");
    if (int rc = check_ctx(ctx)) return rc;
    WPCG_HIP(launch_silu_mul(g_dev, u_dev, out_dev, n, pick(ctx, stream)));
    return WPCG_OK;
}

// ------------------------------------------------------------ MoE layer
int wpcg_moe_create(wpcg_ctx* ctx, int scheme, uint32_t n_exp, uint32_t hidden, uint32_t inter,
                    uint32_t top_k, int norm_topk, wpcg_moe** out)
{
    if (!out) return fail(WPCG_E_ARG, "null output");
    *out = nullptr;
    if (scheme != WPCG_SCHEME_V3 && scheme != WPCG_SCHEME_V4) return fail(WPCG_E_ARG, "scheme must be 3 or 4");
    if (n_exp == 0 || hidden == 0 || inter == 0 || top_k == 0 || top_k > n_exp)
        return fail(WPCG_E_ARG, "need n_exp, hidden, inter > 0 and 0 < top_k <= n_exp");
    if (n_exp > (uint32_t)route_max_n() || top_k > MAX_JOBS / 2)
        return fail(WPCG_E_UNSUPPORTED, "this build routes at most " + std::to_string(route_max_n()) +
                                            " experts and top_k <= " + std::to_string(MAX_JOBS / 2));
    if (hidden % 128 || inter % 128)
        return fail(WPCG_E_SHAPE, "hidden and moe_intermediate must be multiples of 128");
    if (int rc = check_ctx(ctx)) return rc;
    std::unique_ptr<wpcg_moe> m(new (std::nothrow) wpcg_moe);
    if (!m) return fail(WPCG_E_NOMEM, "moe allocation");
    m->ctx = ctx;
    m->scheme = scheme;
    m->n_exp = n_exp;
    m->hidden = hidden;
    m->inter = inter;
    m->top_k = top_k;
    m->norm_topk = norm_topk ? 1 : 0;
    m->gate = expert_view(scheme, inter, hidden);
    m->up = expert_view(scheme, inter, hidden);
    m->down = expert_view(scheme, hidden, inter);
    // routed GEMVs run unsplit: one partial-sum workspace could not serve
    // the top_k experts of one launch
    if (plan_kslices(inter, hidden / 128, 0) != 1 || plan_kslices(hidden, inter / 128, 0) != 1) {
        return fail(WPCG_E_UNSUPPORTED, "expert shape needs a split-K GEMV");
    }
    hipStream_t s = ctx->stream;
    int rc = alloc_planes(m->gate, n_exp, s);
    if (rc == WPCG_OK) rc = alloc_planes(m->up, n_exp, s);
    if (rc == WPCG_OK) rc = alloc_planes(m->down, n_exp, s);
    hipError_t e = hipSuccess;
    auto dev = [&](void** p, size_t bytes) {
        if (e == hipSuccess) e = hipMalloc(p, std::max<size_t>(bytes, 4));
    };
    dev((void**)&m->scores, n_exp * 4u);
    dev((void**)&m->w, top_k * 4u);
    dev((void**)&m->ids, top_k * 4u);
    dev((void**)&m->g, (size_t)top_k * inter * 4);
    dev((void**)&m->u, (size_t)top_k * inter * 4);
    dev((void**)&m->h, (size_t)top_k * inter * 4);
    dev((void**)&m->ys, (size_t)top_k * hidden * 4);
    dev((void**)&m->xn, (size_t)hidden * 4);
    // the FAST path's routed down projection: the chosen experts' rows side
    // by side must fit one K-slice, and the stack's parameters are addressed
    // with 32-bit offsets below 2^31 bytes
    const uint64_t down_params = (uint64_t)n_exp * (m->down.rows_pad / TILE_ROWS) * m->down.nb * TILE_ROWS * 4;
    m->routed = (uint64_t)top_k * (inter / 128) <= fast_max_slice(hidden, (uint64_t)top_k * (inter / 128)) &&
                down_params < 0x7FFFFFF0ull;
    if (rc == WPCG_OK && e != hipSuccess) rc = hip_fail(e, "moe workspace");
    if (rc != WPCG_OK) {
        free_moe(m.get());
        return rc;
    }
    ctx_retain(ctx);
    *out = m.release();
    return WPCG_OK;
}

int wpcg_moe_destroy(wpcg_moe* m)
{
    if (!m) return WPCG_OK;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    free_moe(m);
    ctx_release(m->ctx);
    delete m;
    return WPCG_OK;
}

int wpcg_moe_set_router(wpcg_moe* m, const float* w)
{
    if (!m || !w) return fail(WPCG_E_ARG, "null argument");
    wpcg_dense* d = nullptr;
    if (int rc = wpcg_dense_create(m->ctx, w, m->n_exp, m->hidden, nullptr, &d)) return rc;
    d->mode = m->mode;
    if (m->router) wpcg_dense_destroy(m->router);
    m->router = d;
    return WPCG_OK;
}

int wpcg_moe_set_expert(wpcg_moe* m, uint32_t e, const void* gate, const void* up, const void* down)
{
    if (!m || !gate || !up || !down) return fail(WPCG_E_ARG, "null argument");
    if (e >= m->n_exp) return fail(WPCG_E_ARG, "expert index out of range");
    if (int rc = check_ctx(m->ctx)) return rc;
    const uint64_t tg = m->gate.rows_pad / TILE_ROWS, td = m->down.rows_pad / TILE_ROWS;
    if (int rc = upload_rows(m->ctx, static_cast<const uint8_t*>(gate), m->gate, e * tg)) return rc;
    if (int rc = upload_rows(m->ctx, static_cast<const uint8_t*>(up), m->up, e * tg)) return rc;
    return upload_rows(m->ctx, static_cast<const uint8_t*>(down), m->down, e * td);
}

int wpcg_moe_load_experts(wpcg_moe* m, wpcg_artifact* a, uint32_t layer)
{
    if (!m || !a) return fail(WPCG_E_ARG, "null argument");
    if (a->scheme != m->scheme) return fail(WPCG_E_ARG, "artifact scheme differs from the layer's");
    const uint64_t bpb = block_bytes(m->scheme);
    const uint64_t n_gu = (uint64_t)m->inter * (m->hidden / 128), n_d = (uint64_t)m->hidden * (m->inter / 128);
    for (uint32_t e = 0; e < m->n_exp; e++) {
        const std::string p = "model.layers." + std::to_string(layer) + ".mlp.experts." + std::to_string(e);
        const void* t[3];
        const uint64_t want[3] = {n_gu, n_gu, n_d};
        const char* proj[3] = {".gate_proj.weight", ".up_proj.weight", ".down_proj.weight"};
        for (int k = 0; k < 3; k++) {
            uint64_t size = 0;
            if (int rc = wpcg_artifact_tensor(a, (p + proj[k]).c_str(), &t[k], &size)) return rc;
            if (size != want[k] * bpb)  // WpcLinearV4::new's block-count assert
                return fail(WPCG_E_SHAPE, p + proj[k] + ": block count does not match the expert shape");
        }
        if (int rc = wpcg_moe_set_expert(m, e, t[0], t[1], t[2])) return rc;
    }
    return WPCG_OK;
}

int wpcg_moe_set_mode(wpcg_moe* m, int mode)
{
    if (!m || !valid_mode(mode)) return fail(WPCG_E_ARG, "null moe or bad mode");
    m->mode = mode;
    if (m->router) m->router->mode = mode;
    return WPCG_OK;
}

int wpcg_moe_forward(wpcg_moe* m, const float* x_dev, float* out_dev, int32_t* ids_dev,
                     float* weights_dev, wpcg_stream stream)
{
    if (!m || !x_dev || !out_dev) return fail(WPCG_E_ARG, "null argument");
    if (!m->router) return fail(WPCG_E_ARG, "router not set");
    if (int rc = check_ctx(m->ctx)) return rc;
    hipStream_t s = pick(m->ctx, stream);
    if (int rc = moe_run(m, x_dev, out_dev, nullptr, s)) return rc;
    const size_t K = m->top_k;
    if (ids_dev) WPCG_HIP(hipMemcpyAsync(ids_dev, m->ids, K * 4, hipMemcpyDeviceToDevice, s));
    if (weights_dev) WPCG_HIP(hipMemcpyAsync(weights_dev, m->w, K * 4, hipMemcpyDeviceToDevice, s));
    return WPCG_OK;
}

}  // extern "C"
