// The extern "C" boundary for the device-resident decode step: a dense
// Qwen3 or Qwen3-MoE decoder whose weights, KV cache, activations, position
// and tokens all stay on the GPU. One step (Model::forward_token,
// model.rs:419-547; Qwen3MoeModel::forward_token, qwen3_moe_model.rs:406-542)
// plus the greedy argmax (sampling.rs:3-14) is a fixed sequence of launches
// that is captured once as a HIP graph and replayed per token.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "wpcg_internal.hpp"

using namespace wpcg;

namespace {

struct Layer {
    float *in_ln = nullptr, *post_ln = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    wpcg_linear *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
    wpcg_linear *gate = nullptr, *up = nullptr, *down = nullptr;  // dense MLP
    wpcg_moe* moe = nullptr;                                       // sparse MLP
    std::vector<uint8_t> experts_set;                              // 3 bits per expert
};

// Batch buffers of the FAST prefill, made by the first prefill call: rows
// are the chunk's tokens (at most cap of them).
struct Prefill {
    uint32_t cap = 0;
    float *x = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
    float *g = nullptr, *u = nullptr;           // dense MLP [cap][inter]
    float *r = nullptr, *w = nullptr;           // router logits [cap][E], weights [cap][top_k]
    int32_t* ids = nullptr;                     // [cap][top_k]
    int *pair_tok = nullptr, *pair_pos = nullptr, *items = nullptr, *nitems = nullptr;
    float *ge = nullptr, *ue = nullptr, *de = nullptr;  // per sorted pair: [P][moe_inter] x2, [P][hidden]
    void* xf = nullptr;       // packed X of the batched GEMMs (launch_gemm_pack_rows)
    float* xsum = nullptr;
    float* part = nullptr;    // K-slice partials of o_proj / the dense down
    int cus = 0;              // the device's CUs: the expert-grouped GEMMs' workgroups
    void* dg = nullptr;       // the expert-grouped GEMMs' X digits (launch_pf_digits)
    float* dxs = nullptr;
    float* vlogits = nullptr;  // verification: [WPCG_VERIFY_MAX][vocab], made on first use
    uint32_t* vids = nullptr;  // [WPCG_VERIFY_MAX]
};

}  // namespace

struct wpcg_model {
    wpcg_ctx* ctx = nullptr;
    int scheme = 4, mode = WPCG_MODE_EXACT;
    wpcg_model_config cfg{};
    std::vector<Layer> layers;
    wpcg_linear *embed = nullptr, *lm_head = nullptr;
    float* final_norm = nullptr;
    float *cos_t = nullptr, *sin_t = nullptr;  // [max_pos][head_dim/2]
    float *kc = nullptr, *vc = nullptr;        // [layer][kv_head][max_pos][head_dim]
    DecodeState* st = nullptr;
    uint32_t* tokens = nullptr;                // [max_pos + 1]
    float *residual = nullptr, *normed = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
    float *attn = nullptr, *g = nullptr, *u = nullptr,
          *h = nullptr, *logits = nullptr;
    // FAST attention's chunk states, merged by the o_proj GEMV (null: the
    // head shape needs the one-workgroup-per-head kernel)
    float *part_o = nullptr, *part_ml = nullptr;
    // the step's RoPE row (cos, sin at the position), which the step's
    // embedding launch copies for the FAST attention launches
    float* rope = nullptr;
    // o_proj's second K-slice when its two slices are left to the readers
    // of the residual (the router, gate/up and down add it as they read)
    float* o2 = nullptr;
    // the dense down projection's K-slices 1 and 2, left the same way to the
    // next layer's q/k/v and o_proj, or to the head
    float* d2 = nullptr;
    // the FAST head's per-workgroup argmax keys (one per 16-row tile at most)
    uint64_t* amax = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int graph_mode = -1;
    bool use_graph = true;  // false: steps are enqueued launch by launch
    bool use_prefill = true;  // FAST: prompts go through the batched prefill
    Prefill pf;
    std::vector<void*> allocs;
};

namespace {

int set_dev_f32(wpcg_model* m, float** dst, const void* data, uint64_t nbytes, uint64_t n,
                const std::string& name)
{
    if (nbytes != n * 4) return fail(WPCG_E_SHAPE, name + ": expected " + std::to_string(n) + " fp32 values");
    if (!*dst) {
        WPCG_HIP(hipMalloc(dst, n * 4));
        m->allocs.push_back(*dst);
    }
    WPCG_HIP(hipMemcpy(*dst, data, nbytes, hipMemcpyHostToDevice));
    return WPCG_OK;
}

int set_linear(wpcg_model* m, wpcg_linear** dst, const void* data, uint64_t nbytes, uint64_t out_f,
               uint64_t in_f, const std::string& name)
{
    wpcg_linear* l = nullptr;
    if (int rc = wpcg_linear_from_blocks(m->ctx, m->scheme, data, nbytes, out_f, in_f, nullptr, &l))
        return fail(rc, name + ": " + wpcg_last_error_string());
    l->mode = m->mode;
    if (*dst) wpcg_linear_destroy(*dst);
    *dst = l;
    return WPCG_OK;
}

void free_model(wpcg_model* m)
{
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    for (auto& L : m->layers) {
        for (wpcg_linear* l : {L.q, L.k, L.v, L.o, L.gate, L.up, L.down})
            if (l) wpcg_linear_destroy(l);
        if (L.moe) wpcg_moe_destroy(L.moe);
    }
    if (m->embed) wpcg_linear_destroy(m->embed);
    if (m->lm_head) wpcg_linear_destroy(m->lm_head);
    for (void* p : m->allocs) (void)hipFree(p);
}

void drop_graph(wpcg_model* m)
{
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
    m->graph_mode = -1;
}

// The logits head as the reference's loaders choose it: the dense decoder
// always the embedding table (model.rs:545, embed.logits), Qwen3-MoE always
// its own lm_head (qwen3_moe_model.rs:337-343, 540). wpcg_model_create
// refuses a config whose `tied` disagrees.
wpcg_linear* logits_head(const wpcg_model* m) { return m->cfg.n_experts ? m->lm_head : m->embed; }

// First missing tensor, or "" when the model is complete.
std::string missing(const wpcg_model* m)
{
    const wpcg_model_config& c = m->cfg;
    if (!m->embed) return "model.embed_tokens.weight";
    if (c.n_experts && !m->lm_head) return "lm_head.weight";
    if (!m->final_norm) return "model.norm.weight";
    for (uint32_t l = 0; l < c.n_layers; l++) {
        const Layer& L = m->layers[l];
        const std::string p = "model.layers." + std::to_string(l) + ".";
        if (!L.in_ln) return p + "input_layernorm.weight";
        if (!L.post_ln) return p + "post_attention_layernorm.weight";
        if (!L.q_norm) return p + "self_attn.q_norm.weight";
        if (!L.k_norm) return p + "self_attn.k_norm.weight";
        if (!L.q) return p + "self_attn.q_proj.weight";
        if (!L.k) return p + "self_attn.k_proj.weight";
        if (!L.v) return p + "self_attn.v_proj.weight";
        if (!L.o) return p + "self_attn.o_proj.weight";
        if (c.n_experts == 0) {
            if (!L.gate) return p + "mlp.gate_proj.weight";
            if (!L.up) return p + "mlp.up_proj.weight";
            if (!L.down) return p + "mlp.down_proj.weight";
        } else {
            if (!L.moe->router) return p + "mlp.gate.weight";
            for (uint32_t e = 0; e < c.n_experts; e++)
                if (L.experts_set[e] != 7) return p + "mlp.experts." + std::to_string(e) + ".*";
        }
    }
    return "";
}

// A FAST job y = lin(RMSNorm(x; nw)) with the norm folded into the GEMV, or
// without nw a plain FAST job; `ok` turns false when the linear cannot fold
// the norm in (its row needs more than one K-slice).
GemvJob fast_job(wpcg_linear* lin, const float* x, float* y, const float* nw, float eps, bool& ok)
{
    GemvJob J{&lin->m, &lin->plan, x, lin->bias, y};
    if (nw) {
        J.xform = XF_NORM;
        J.nw = nw;
        J.eps = eps;
        ok = ok && lin->plan.kg == 1 && lin->m.nb > 0;
    }
    return J;
}

// Whether FAST mode leaves the dense down projection's K-slices to their
// readers: every reader folds the RMSNorm into its GEMV (one K-slice each)
// or is the merging o_proj, and the down has 2 or 3 slices.
bool defer_down(const wpcg_model* m)
{
    const wpcg_model_config& c = m->cfg;
    if (m->mode != WPCG_MODE_FAST || c.n_experts || !m->part_o || !m->d2) return false;
    const wpcg_linear* head = logits_head(m);
    if (head->plan.kg != 1 || head->m.nb == 0) return false;
    for (uint32_t l = 0; l < c.n_layers; l++) {
        const Layer& L = m->layers[l];
        for (const wpcg_linear* r : {L.q, L.k, L.v})
            if (r->plan.kg != 1 || r->m.nb == 0) return false;
        if (L.down->plan.kg < 2 || L.down->plan.kg > 3 || L.gate->plan.kg != 1 || L.up->plan.kg != 1)
            return false;
    }
    return true;
}

// One decode step on stream s: the token at tokens[pos] through every layer,
// logits, argmax, position + 1. FAST mode folds the RMSNorms into the
// GEMVs that read them and runs the MoE layer as three launches (moe_run);
// EXACT mode keeps every operation of the reference as its own launch.
int enqueue_step(wpcg_model* m, hipStream_t s)
{
    const wpcg_model_config& c = m->cfg;
    const int H = (int)c.hidden, hd = (int)c.head_dim, nh = (int)c.n_heads, nkv = (int)c.n_kv_heads;
    const int mode = m->mode;
    const bool fast = mode == WPCG_MODE_FAST;
    const float scale = 1.0f / std::sqrt((float)hd);  // model.rs: 1/sqrt(head_dim) in f32
    if (fast && m->part_o)
        WPCG_HIP(launch_embed_tok(m->embed->m, m->tokens, m->st, m->residual, s, m->cos_t, m->sin_t, hd / 2,
                                  m->rope));
    else
        WPCG_HIP(launch_embed_tok(m->embed->m, m->tokens, m->st, m->residual, s));
    const bool defer_d = defer_down(m);
    const float* d2 = nullptr;  // the previous down's deferred slices, if any
    int n_d2 = 1;
    // EXACT MoE: the last layer's expert combine, left to the next RMSNorm of
    // the residual (one launch fewer per layer)
    const wpcg_moe* pend = nullptr;
    auto norm_residual = [&](const float* nw) -> hipError_t {
        if (const wpcg_moe* p = pend) {
            pend = nullptr;
            return launch_rms_norm_combine(m->residual, nw, H, c.eps, m->normed, p->ys, p->ids, p->w,
                                           (int)p->top_k, s);
        }
        return launch_rms_norm(mode, m->residual, nw, H, c.eps, m->normed, s);
    };
    for (uint32_t l = 0; l < c.n_layers; l++) {
        Layer& L = m->layers[l];
        bool fused = fast;
        const float* o2 = nullptr;  // o_proj's deferred second slice, if any
        GemvJob qkv_jobs[3] = {fast_job(L.q, m->residual, m->q, L.in_ln, c.eps, fused),
                               fast_job(L.k, m->residual, m->k, L.in_ln, c.eps, fused),
                               fast_job(L.v, m->residual, m->v, L.in_ln, c.eps, fused)};
        for (GemvJob& J : qkv_jobs) {
            J.x_add = d2;
            J.n_xa = n_d2;
        }
        if (fused) {
            WPCG_HIP(launch_gemv_fast(qkv_jobs, 3, s));
        } else {
            if (d2) return fail(WPCG_E_UNSUPPORTED, "deferred down slices without a FAST reader");
            WPCG_HIP(norm_residual(L.in_ln));
            wpcg_linear* qkv[3] = {L.q, L.k, L.v};
            const float* xs[3] = {m->normed, m->normed, m->normed};
            float* ys[3] = {m->q, m->k, m->v};
            if (int rc = wpcg_linear_matvec_multi(3, qkv, xs, ys, s)) return rc;
        }
        float* kc = m->kc + (size_t)l * nkv * c.max_pos * hd;
        float* vc = m->vc + (size_t)l * nkv * c.max_pos * hd;
        if (fast && m->part_o) {
            // chunked attention; o_proj merges the chunks, residual += o_proj(attn)
            WPCG_HIP(launch_attention_chunks(m->q, m->k, m->v, L.q_norm, L.k_norm, nh, nkv, hd, c.eps, scale,
                                             m->rope, (int)c.max_pos, m->st, kc, vc, m->part_o, m->part_ml, s));
            // The dense model merges the chunks once, in a launch of its own,
            // and runs o_proj as a plain GEMV: its o_proj is unsplit (32
            // blocks per workgroup), so each of its 160 workgroups merged
            // the chunk states of every head, 43 MB of reads per launch
            // (o_proj 9.3 us; merge 2.x us + plain GEMV). The MoE model's
            // two-slice o_proj merges half the heads per workgroup and keeps
            // the merge in its prep.
            const bool merge_apart = !c.n_experts;
            if (merge_apart) WPCG_HIP(launch_attention_merge(m->part_o, m->part_ml, nh, hd, m->attn, s));
            GemvJob o{&L.o->m, &L.o->plan, merge_apart ? m->attn : m->part_o, m->residual, m->residual};
            if (!merge_apart) {
                o.xform = XF_MERGE;
                o.x2 = m->part_ml;
                o.st = m->st;
                o.head_dim = hd;
                o.n_heads = nh;
            }
            // Two K-slices: no handoff between them. Slice 0 adds its sum to
            // the residual in place, slice 1 writes o2, and the next ops read
            // residual + o2 (a handoff of three device-scope round trips
            // cost ~1-2 us at the end of the launch).
            if (L.o->plan.kg == 2) o.y2 = m->o2;
            o.bias2 = d2;  // the residual's deferred down slices join it here
            o.n_b2 = n_d2;
            WPCG_HIP(launch_gemv_fast(&o, 1, s));
            o2 = o.y2;
            d2 = nullptr;
        } else {
            WPCG_HIP(launch_attention(mode, m->q, m->k, m->v, L.q_norm, L.k_norm, nh, nkv, hd, c.eps, scale,
                                      m->cos_t, m->sin_t, m->st, kc, vc, m->attn, s));
            // residual += o_proj(attn): the residual is the GEMV's bias and output
            float* saved = L.o->bias;
            L.o->bias = m->residual;
            const int rc = wpcg_linear_matvec(L.o, m->attn, m->residual, s);
            L.o->bias = saved;
            if (rc) return rc;
        }
        if (c.n_experts && fast) {
            if (int rc = moe_run(L.moe, m->residual, m->residual, m->residual, s, L.post_ln, c.eps, o2)) return rc;
            continue;
        }
        if (!c.n_experts && fast) {  // dense SwiGLU: norm into gate/up, SiLU*up into down
            fused = true;
            GemvJob gu_jobs[2] = {fast_job(L.gate, m->residual, m->g, L.post_ln, c.eps, fused),
                                  fast_job(L.up, m->residual, m->u, L.post_ln, c.eps, fused)};
            if (fused) {
                gu_jobs[0].x_add = gu_jobs[1].x_add = o2;
                WPCG_HIP(launch_gemv_fast(gu_jobs, 2, s));
                GemvJob down{&L.down->m, &L.down->plan, m->g, m->residual, m->residual};
                down.xform = XF_SILU;
                down.x2 = m->u;
                down.bias2 = o2;
                // its K-slices 1.. go to the next layer's q/k/v and o_proj (or
                // the head) instead of a handoff at the end of the launch
                if (defer_d) {
                    down.y2 = m->d2;
                    d2 = m->d2;
                    n_d2 = L.down->plan.kg - 1;
                }
                WPCG_HIP(launch_gemv_fast(&down, 1, s));
                continue;
            }
        }
        if (o2) return fail(WPCG_E_UNSUPPORTED, "deferred o_proj slice without a FAST reader");
        WPCG_HIP(norm_residual(L.post_ln));
        if (c.n_experts) {
            const bool defer = mode == WPCG_MODE_EXACT && rms_norm_combine_ok(H, (int)L.moe->top_k);
            if (int rc = moe_run(L.moe, m->normed, m->residual, m->residual, s, nullptr, 0.0f, nullptr, defer))
                return rc;
            if (defer) pend = L.moe;
        } else {
            wpcg_linear* gu[2] = {L.gate, L.up};
            const float* x2[2] = {m->normed, m->normed};
            float* y2[2] = {m->g, m->u};
            if (int rc = wpcg_linear_matvec_multi(2, gu, x2, y2, s)) return rc;
            WPCG_HIP(launch_silu_mul(m->g, m->u, m->h, c.inter, s));
            float* saved = L.down->bias;
            L.down->bias = m->residual;
            const int rc = wpcg_linear_matvec(L.down, m->h, m->residual, s);
            L.down->bias = saved;
            if (rc) return rc;
        }
    }
    wpcg_linear* head = logits_head(m);
    bool fused = fast;
    GemvJob head_job = fast_job(head, m->residual, m->logits, m->final_norm, c.eps, fused);
    head_job.x_add = d2;
    head_job.n_xa = n_d2;
    if (d2 && !fused) return fail(WPCG_E_UNSUPPORTED, "deferred down slices without a FAST reader");
    if (fused) {
        // each workgroup of the head also leaves the argmax key of its rows,
        // so the argmax reads one key per workgroup instead of every logit
        // (one workgroup over 151936 logits: 8.9 us)
        const bool keys = m->amax && head->plan.kg == 1;
        if (keys) head_job.amax = m->amax;
        WPCG_HIP(launch_gemv_fast(&head_job, 1, s));
        if (keys) {
            const uint64_t tiles = head->m.rows_pad / TILE_ROWS;
            const int tw = fast_tiles_per_wg(head->m.rows, head->m.nb);
            WPCG_HIP(launch_argmax_keys_next(m->amax, (int)((tiles + tw - 1) / tw), m->st, m->tokens, s));
            return WPCG_OK;
        }
    } else {
        WPCG_HIP(norm_residual(m->final_norm));
        if (int rc = wpcg_linear_matvec(head, m->normed, m->logits, s)) return rc;
    }
    WPCG_HIP(launch_argmax_next(m->logits, (int)c.vocab, m->st, m->tokens, s));
    return WPCG_OK;
}

// ---- batched prefill (FAST) --------------------------------------------------
// Rows of tokens per prefill pass; longer prompts run pass after pass.
constexpr uint32_t PF_CAP = 256;
constexpr int PF_MAX_KG = 4;  // K-slices of the prefill's hidden-size GEMMs
static_assert(PF_CAP <= (uint32_t)PF_GROUP_MAXT, "the expert grouping holds PF_GROUP_MAXT tokens");

// Whether the batched path covers this model: FAST attention's head shapes,
// and for MoE the router width, the pair count and one-slice expert GEMMs.
bool prefill_ok(const wpcg_model* m)
{
    const wpcg_model_config& c = m->cfg;
    if (!attention_fast_ok((int)c.n_heads, (int)c.n_kv_heads, (int)c.head_dim)) return false;
    if (!c.n_experts) return true;
    const uint32_t cap = std::min(PF_CAP, c.max_pos);
    return c.n_experts <= (uint32_t)ROUTE_MAXN && cap * c.top_k <= (uint32_t)PF_MAX_PAIRS &&
           c.hidden / 128 <= (uint32_t)GEMM_GROUP_MAXBK && c.moe_inter / 128 <= (uint32_t)GEMM_GROUP_MAXBK &&
           pad_rows(c.hidden) <= (uint64_t)GEMM_GROUP_MAXROWS && pad_rows(c.moe_inter) <= (uint64_t)GEMM_GROUP_MAXROWS &&
           c.moe_inter % 128 == 0;
}

int make_prefill(wpcg_model* m)
{
    Prefill& P = m->pf;
    if (P.cap) return WPCG_OK;
    const wpcg_model_config& c = m->cfg;
    WPCG_HIP(hipDeviceGetAttribute(&P.cus, hipDeviceAttributeMultiprocessorCount, m->ctx->device));
    const size_t cap = std::min(PF_CAP, c.max_pos), H = c.hidden, qd = (size_t)c.n_heads * c.head_dim,
                 kvd = (size_t)c.n_kv_heads * c.head_dim;
    int rc = WPCG_OK;
    auto dev = [&](void** p, size_t bytes) {
        if (rc != WPCG_OK) return;
        const hipError_t e = hipMalloc(p, std::max<size_t>(bytes, 4));
        if (e != hipSuccess) {
            rc = hip_fail(e, "prefill buffers");
            return;
        }
        m->allocs.push_back(*p);
    };
    dev((void**)&P.x, cap * H * 4);
    dev((void**)&P.xn, cap * H * 4);
    dev((void**)&P.q, cap * qd * 4);
    dev((void**)&P.k, cap * kvd * 4);
    dev((void**)&P.v, cap * kvd * 4);
    dev((void**)&P.attn, cap * qd * 4);
    const size_t kmax = std::max<size_t>({H, qd, c.n_experts ? 0 : (size_t)c.inter});
    dev((void**)&P.xf, kmax / 128 * gemm_rows_tiles((int)cap) * 4096);
    dev((void**)&P.xsum, kmax / 128 * gemm_rows_tiles((int)cap) * 16 * 4);
    dev((void**)&P.part, (size_t)PF_MAX_KG * (gemm_rows_tiles((int)cap) / 4 * 32) * pad_rows(H) * 4);
    if (c.n_experts) {
        const size_t pairs = cap * c.top_k, E = c.n_experts, I = c.moe_inter;
        dev((void**)&P.r, cap * E * 4);
        dev((void**)&P.w, pairs * 4);
        dev((void**)&P.ids, pairs * 4);
        dev((void**)&P.pair_tok, pairs * 4);
        dev((void**)&P.pair_pos, pairs * 4);
        dev((void**)&P.items, 3 * (pairs / GEMM_GROUP_COLS + E + 1) * 4);
        dev((void**)&P.nitems, 4);
        dev((void**)&P.ge, pairs * I * 4);
        dev((void**)&P.ue, pairs * I * 4);
        dev((void**)&P.de, pairs * H * 4);
        const size_t dvals = std::max(cap * H, pairs * I);  // gate/up's token rows, then down's pair rows
        dev(&P.dg, dvals * 4);
        dev((void**)&P.dxs, dvals / 128 * 8);
    } else {
        dev((void**)&P.g, cap * c.inter * 4);
        dev((void**)&P.u, cap * c.inter * 4);
    }
    if (rc == WPCG_OK) P.cap = (uint32_t)cap;
    return rc;
}

// K-slices of a packed-rows GEMM of the prefill whose rows are the hidden
// size (o_proj, the dense down): enough for about 256 workgroups, slices of
// at least 8 blocks (o_proj of the Qwen3-30B-A3B shape at 256 rows: 128
// workgroups of 32 blocks took 26.3 us, 256 of 16 plus the slice sum ~18).
int pf_kslices(const DeviceMatrix& m, int n)
{
    const int live = gemm_row_groups(m.rows) * (gemm_rows_tiles(n) / 4);
    return std::max(1, std::min({256 / std::max(live, 1), (int)m.nb / 8, PF_MAX_KG}));
}

// Tokens tokens[pos0 .. pos0+n-1] (already on the device) through every
// layer as one batch, n <= cap: keys and values of those positions land in
// the caches; the last row's final hidden state is left in pf.x[n-1].
int prefill_pass(wpcg_model* m, uint32_t pos0, uint32_t n, hipStream_t s)
{
    const wpcg_model_config& c = m->cfg;
    Prefill& P = m->pf;
    const int H = (int)c.hidden, hd = (int)c.head_dim, nh = (int)c.n_heads, nkv = (int)c.n_kv_heads;
    const float scale = 1.0f / std::sqrt((float)hd);
    const int F = WPCG_MODE_FAST;
    WPCG_HIP(launch_embed_rows(m->embed->m, m->tokens + pos0, (int)n, P.x, s));
    for (uint32_t l = 0; l < c.n_layers; l++) {
        Layer& L = m->layers[l];
        WPCG_HIP(launch_rms_pack_rows(P.x, L.in_ln, (int)n, H, c.eps, P.xf, P.xsum, s));
        float* kc = m->kc + (size_t)l * nkv * c.max_pos * hd;
        float* vc = m->vc + (size_t)l * nkv * c.max_pos * hd;
        // 128-wide heads: the q/k/v GEMM's epilogue applies the head norms
        // and the rotation and appends the keys and values to the caches
        const bool qk_fused = hd == 128;
        {
            const DeviceMatrix* ms[3] = {&L.q->m, &L.k->m, &L.v->m};
            const float* bs[3] = {L.q->bias, L.k->bias, L.v->bias};
            float* ys[3] = {P.q, P.k, P.v};
            GemmRope rope{{GEMM_ROPE_Q, GEMM_ROPE_K, GEMM_ROPE_V}, {nullptr, kc, vc}, {L.q_norm, L.k_norm, nullptr},
                          m->cos_t, m->sin_t, (int)pos0, (int)c.max_pos, c.eps};
            WPCG_HIP(launch_gemm_packed_rows_multi(ms, bs, ys, 3, P.xf, P.xsum, (int)n, s, qk_fused ? &rope : nullptr));
        }
        WPCG_HIP(launch_prefill_attention(P.q, P.k, P.v, L.q_norm, L.k_norm, nh, nkv, hd, c.eps, scale, m->cos_t,
                                          m->sin_t, (int)pos0, (int)n, (int)c.max_pos, kc, vc, P.attn, P.xf, P.xsum,
                                          s, qk_fused));
        // residual += o_proj(attn); 128-wide heads leave the attention packed
        if (hd != 128) WPCG_HIP(launch_gemm_pack_rows(P.attn, (int)n, nh * hd, P.xf, P.xsum, s));
        // o_proj in K-slices; for the MoE model the slice sum joins the
        // post-attention RMSNorm (the router and the experts read fp32 rows)
        const int okg = pf_kslices(L.o->m, (int)n);
        const bool fuse_norm = c.n_experts && okg > 1 && H <= PF_NORM_MAXH;
        WPCG_HIP(launch_gemm_packed_rows(L.o->m, P.xf, P.xsum, (int)n, L.o->bias, P.x, P.x, s, okg, P.part,
                                         !fuse_norm));
        if (!c.n_experts) {
            WPCG_HIP(launch_rms_pack_rows(P.x, L.post_ln, (int)n, H, c.eps, P.xf, P.xsum, s));
            const DeviceMatrix* ms[2] = {&L.gate->m, &L.up->m};
            const float* bs[2] = {L.gate->bias, L.up->bias};
            float* ys[2] = {P.g, P.u};
            WPCG_HIP(launch_gemm_packed_rows_multi(ms, bs, ys, 2, P.xf, P.xsum, (int)n, s));
            WPCG_HIP(launch_silu_mul(P.g, P.u, P.g, (size_t)n * c.inter, s));
            WPCG_HIP(launch_gemm_pack_rows(P.g, (int)n, (int)c.inter, P.xf, P.xsum, s));
            WPCG_HIP(launch_gemm_packed_rows(L.down->m, P.xf, P.xsum, (int)n, L.down->bias, P.x, P.x, s,
                                             pf_kslices(L.down->m, (int)n), P.part));
            continue;
        }
        // experts: route every row, sort the (row, slot) pairs by expert, one
        // grouped launch for gate and up and one for down, then the ordered
        // combine
        // (the fused slice sum + norm also writes the experts' X digits)
        const bool digits_done = fuse_norm && H % 128 == 0;
        if (fuse_norm)
            WPCG_HIP(launch_pf_reduce_norm(P.part, okg, (int)n, H, (int)L.o->m.rows_pad, L.o->bias, P.x, L.post_ln,
                                           c.eps, P.xn, digits_done ? P.dg : nullptr,
                                           digits_done ? P.dxs : nullptr, s));
        else
            WPCG_HIP(launch_rms_norm_rows(F, P.x, L.post_ln, H, (int)n, c.eps, P.xn, s));
        wpcg_moe* E = L.moe;
        const int ne = (int)c.n_experts, K = (int)c.top_k, pairs = (int)n * K;
        WPCG_HIP(launch_pf_router(P.xn, E->router->w, (int)n, ne, H, P.r, s));
        WPCG_HIP(launch_route_rows(P.r, ne, (int)n, K, (int)c.norm_topk, P.ids, P.w, s));
        WPCG_HIP(launch_pf_group(P.ids, pairs, ne, K, P.pair_tok, P.pair_pos, P.items, P.nitems, s));
        if (!digits_done) WPCG_HIP(launch_pf_digits(P.xn, nullptr, (int)n, H, P.dg, P.dxs, s));
        WPCG_HIP(launch_gemm_grouped(E->gate, &E->up, P.dg, P.dxs, (int)n, P.pair_tok, P.items, P.nitems, P.cus,
                                     P.ge, P.ue, s));
        WPCG_HIP(launch_pf_digits(P.ge, P.ue, pairs, (int)c.moe_inter, P.dg, P.dxs, s));
        WPCG_HIP(launch_gemm_grouped(E->down, nullptr, P.dg, P.dxs, pairs, nullptr, P.items, P.nitems, P.cus, P.de,
                                     nullptr, s));
        WPCG_HIP(launch_pf_combine(P.x, P.de, P.w, P.pair_pos, (int)n, K, H, s));
    }
    return WPCG_OK;
}

// FAST prefill of tokens[pos0 .. pos0+n-1] in passes of at most cap rows,
// then the last row's logits and the argmax step (st holds pos0 + n - 1 and
// the caller's n_prompt, so the argmax lands in tokens[] as a step's would).
int prefill_run(wpcg_model* m, uint32_t pos0, uint32_t n, uint32_t n_prompt)
{
    if (int rc = make_prefill(m)) return rc;
    hipStream_t s = m->ctx->stream;
    const wpcg_model_config& c = m->cfg;
    uint32_t last = 0;
    for (uint32_t done = 0; done < n;) {
        const uint32_t len = std::min(m->pf.cap, n - done);
        if (int rc = prefill_pass(m, pos0 + done, len, s)) return rc;
        last = len - 1;
        done += len;
    }
    const float* xl = m->pf.x + (size_t)last * c.hidden;
    wpcg_linear* head = logits_head(m);
    bool fused = true;
    GemvJob head_job = fast_job(head, xl, m->logits, m->final_norm, c.eps, fused);
    if (fused) {
        WPCG_HIP(launch_gemv_fast(&head_job, 1, s));
    } else {
        WPCG_HIP(launch_rms_norm(WPCG_MODE_FAST, xl, m->final_norm, (int)c.hidden, c.eps, m->normed, s));
        if (int rc = wpcg_linear_matvec(head, m->normed, m->logits, s)) return rc;
    }
    WPCG_HIP(hipStreamSynchronize(s));
    DecodeState st{pos0 + n - 1, n_prompt, c.max_pos, 0};
    WPCG_HIP(hipMemcpy(m->st, &st, sizeof st, hipMemcpyHostToDevice));
    WPCG_HIP(launch_argmax_next(m->logits, (int)c.vocab, m->st, m->tokens, s));
    return WPCG_OK;
}

// FAST verification of tokens[pos0 .. pos0+n-1] (n <= WPCG_VERIFY_MAX <= cap,
// one pass): every row's logits (final norm, head as one batched GEMM) and
// argmax; the position ends at pos0 + n with the last argmax as st.last.
int verify_run(wpcg_model* m, uint32_t pos0, uint32_t n)
{
    if (int rc = make_prefill(m)) return rc;
    const wpcg_model_config& c = m->cfg;
    Prefill& P = m->pf;
    hipStream_t s = m->ctx->stream;
    if (!P.vlogits) {
        WPCG_HIP(hipMalloc(&P.vlogits, (size_t)WPCG_VERIFY_MAX * c.vocab * 4));
        m->allocs.push_back(P.vlogits);
        WPCG_HIP(hipMalloc(&P.vids, WPCG_VERIFY_MAX * 4));
        m->allocs.push_back(P.vids);
    }
    if (int rc = prefill_pass(m, pos0, n, s)) return rc;
    wpcg_linear* head = logits_head(m);
    WPCG_HIP(launch_rms_pack_rows(P.x, m->final_norm, (int)n, (int)c.hidden, c.eps, P.xf, P.xsum, s));
    WPCG_HIP(launch_gemm_packed_rows(head->m, P.xf, P.xsum, (int)n, head->bias, nullptr, P.vlogits, s));
    WPCG_HIP(launch_argmax_rows(P.vlogits, (int)c.vocab, (int)n, P.vids, s));
    WPCG_HIP(hipStreamSynchronize(s));
    uint32_t last = 0;
    WPCG_HIP(hipMemcpy(&last, P.vids + (n - 1), 4, hipMemcpyDeviceToHost));
    DecodeState st{pos0 + n, 0xffffffffu, c.max_pos, last};
    WPCG_HIP(hipMemcpy(m->st, &st, sizeof st, hipMemcpyHostToDevice));
    return WPCG_OK;
}

int ensure_graph(wpcg_model* m)
{
    if (!m->use_graph) return WPCG_OK;
    if (m->exec && m->graph_mode == m->mode) return WPCG_OK;
    drop_graph(m);
    hipStream_t s = m->ctx->stream;
    WPCG_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    const int rc = enqueue_step(m, s);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(s, &g);
    if (rc != WPCG_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "capture of the decode step");
    m->graph = g;
    WPCG_HIP(hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0));
    m->graph_mode = m->mode;
    return WPCG_OK;
}

// One step on the context stream: the captured graph, or the launches.
int run_step(wpcg_model* m)
{
    hipStream_t s = m->ctx->stream;
    if (!m->use_graph) return enqueue_step(m, s);
    WPCG_HIP(hipGraphLaunch(m->exec, s));
    return WPCG_OK;
}

int ready(wpcg_model* m)
{
    const std::string miss = missing(m);
    if (!miss.empty()) return fail(WPCG_E_ARG, "tensor not set: " + miss);
    if (int rc = check_ctx(m->ctx)) return rc;
    return ensure_graph(m);
}

}  // namespace

extern "C" {

int wpcg_rms_norm(wpcg_ctx* ctx, const float* x_dev, const float* w_dev, uint32_t n, float eps,
                  float* out_dev, int mode, wpcg_stream stream)
{
    if (!x_dev || !w_dev || !out_dev) return fail(WPCG_E_ARG, "null argument");
    if (n == 0) return fail(WPCG_E_ARG, "empty vector");
    if (mode != WPCG_MODE_EXACT && mode != WPCG_MODE_FAST) return fail(WPCG_E_ARG, "bad mode");
    if (int rc = check_ctx(ctx)) return rc;
    WPCG_HIP(launch_rms_norm(mode, x_dev, w_dev, (int)n, eps, out_dev, pick(ctx, stream)));
    return WPCG_OK;
}

int wpcg_model_create(wpcg_ctx* ctx, int scheme, const wpcg_model_config* cfg, wpcg_model** out)
{
    if (!out) return fail(WPCG_E_ARG, "null output");
    *out = nullptr;
    if (!cfg) return fail(WPCG_E_ARG, "null config");
    if (scheme != WPCG_SCHEME_V3 && scheme != WPCG_SCHEME_V4) return fail(WPCG_E_ARG, "scheme must be 3 or 4");
    const wpcg_model_config& c = *cfg;
    if (!c.n_layers || !c.hidden || !c.n_heads || !c.n_kv_heads || !c.head_dim || !c.vocab || !c.max_pos)
        return fail(WPCG_E_ARG, "every size in the config must be positive");
    if (c.n_heads % c.n_kv_heads || c.head_dim % 32 || c.head_dim > 256)
        return fail(WPCG_E_SHAPE, "n_heads must be a multiple of n_kv_heads; head_dim a multiple of 32, <= 256");
    if (c.max_pos > (uint32_t)attention_max_pos())
        return fail(WPCG_E_UNSUPPORTED, "max_pos above " + std::to_string(attention_max_pos()));
    if (c.hidden % 128 || (c.n_heads * c.head_dim) % 128 || (c.n_experts == 0 && c.inter % 128))
        return fail(WPCG_E_SHAPE, "matrix input sizes must be multiples of 128");
    if (c.n_experts == 0 && !c.inter) return fail(WPCG_E_ARG, "dense model needs intermediate_size");
    if (c.tied != (c.n_experts == 0 ? 1 : 0))
        return fail(WPCG_E_UNSUPPORTED, c.n_experts ? "tied = 1 with experts: Qwen3-MoE takes its logits from "
                                                      "lm_head.weight (qwen3_moe_model.rs:337-343)"
                                                    : "tied = 0 without experts: the dense decoder takes its "
                                                      "logits from the embedding table (model.rs:545)");
    if (int rc = check_ctx(ctx)) return rc;
    std::unique_ptr<wpcg_model> m(new (std::nothrow) wpcg_model);
    if (!m) return fail(WPCG_E_NOMEM, "model allocation");
    m->ctx = ctx;
    m->scheme = scheme;
    m->cfg = c;
    m->layers.resize(c.n_layers);
    int rc = WPCG_OK;
    for (uint32_t l = 0; l < c.n_layers && rc == WPCG_OK && c.n_experts; l++) {
        rc = wpcg_moe_create(ctx, scheme, c.n_experts, c.hidden, c.moe_inter, c.top_k, c.norm_topk,
                             &m->layers[l].moe);
        m->layers[l].experts_set.assign(c.n_experts, 0);
    }
    const size_t hd = c.head_dim, half = hd / 2, qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
    const size_t inter = c.n_experts ? c.moe_inter : c.inter;
    auto dev = [&](void** p, size_t bytes) {
        if (rc != WPCG_OK) return;
        hipError_t e = hipMalloc(p, std::max<size_t>(bytes, 4));
        if (e != hipSuccess) {
            rc = hip_fail(e, "model workspace");
            return;
        }
        m->allocs.push_back(*p);
    };
    dev((void**)&m->cos_t, (size_t)c.max_pos * half * 4);
    dev((void**)&m->sin_t, (size_t)c.max_pos * half * 4);
    const size_t cache = (size_t)c.n_layers * kvd * c.max_pos * 4;
    dev((void**)&m->kc, cache);
    dev((void**)&m->vc, cache);
    dev((void**)&m->st, sizeof(DecodeState));
    dev((void**)&m->tokens, ((size_t)c.max_pos + 1) * 4);
    dev((void**)&m->residual, c.hidden * 4u);
    dev((void**)&m->normed, c.hidden * 4u);
    dev((void**)&m->q, qd * 4);
    dev((void**)&m->k, kvd * 4);
    dev((void**)&m->v, kvd * 4);
    dev((void**)&m->attn, qd * 4);
    dev((void**)&m->g, inter * 4);
    dev((void**)&m->u, inter * 4);
    dev((void**)&m->h, inter * 4);
    dev((void**)&m->logits, (size_t)c.vocab * 4);
    if (attention_fast_ok((int)c.n_heads, (int)c.n_kv_heads, (int)hd)) {
        dev((void**)&m->part_o, (size_t)ATTN_CHUNKS * qd * 4);
        dev((void**)&m->part_ml, (size_t)ATTN_CHUNKS * c.n_heads * 2 * 4);
        dev((void**)&m->rope, (size_t)hd * 4);
        dev((void**)&m->amax, (size_t)(c.vocab + TILE_ROWS - 1) / TILE_ROWS * 8);
        dev((void**)&m->o2, (size_t)c.hidden * 4);
        dev((void**)&m->d2, (size_t)2 * c.hidden * 4);
    }
    if (rc == WPCG_OK) {
        // RoPE angles as rope.rs:29-33 computes them: f64 pow, sin, cos, cast to f32
        std::vector<float> cs((size_t)c.max_pos * half), sn((size_t)c.max_pos * half);
        for (size_t p = 0; p < c.max_pos; p++)
            for (size_t i = 0; i < half; i++) {
                const double inv_freq = std::pow(c.rope_theta, -(2.0 * (double)i) / (double)hd);
                const double angle = (double)p * inv_freq;
                cs[p * half + i] = (float)std::cos(angle);
                sn[p * half + i] = (float)std::sin(angle);
            }
        hipError_t e = hipMemcpy(m->cos_t, cs.data(), cs.size() * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(m->sin_t, sn.data(), sn.size() * 4, hipMemcpyHostToDevice);
        DecodeState st{0, 0, c.max_pos, 0};
        if (e == hipSuccess) e = hipMemcpy(m->st, &st, sizeof st, hipMemcpyHostToDevice);
        if (e != hipSuccess) rc = hip_fail(e, "model tables");
    }
    if (rc != WPCG_OK) {
        free_model(m.get());
        return rc;
    }
    ctx_retain(ctx);
    *out = m.release();
    return WPCG_OK;
}

int wpcg_model_destroy(wpcg_model* m)
{
    if (!m) return WPCG_OK;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    free_model(m);
    ctx_release(m->ctx);
    delete m;
    return WPCG_OK;
}

int wpcg_model_set_tensor(wpcg_model* m, const char* name_c, const void* data, uint64_t nbytes)
{
    if (!m || !name_c || !data) return fail(WPCG_E_ARG, "null argument");
    if (int rc = check_ctx(m->ctx)) return rc;
    drop_graph(m);
    const wpcg_model_config& c = m->cfg;
    const std::string name(name_c);
    const uint64_t qd = (uint64_t)c.n_heads * c.head_dim, kvd = (uint64_t)c.n_kv_heads * c.head_dim;
    if (name == "model.embed_tokens.weight") return set_linear(m, &m->embed, data, nbytes, c.vocab, c.hidden, name);
    if (name == "lm_head.weight") {
        // the reference's dense loader never reads lm_head.weight (qwen3_model.rs:187-206)
        if (!c.n_experts) return fail(WPCG_E_NOTFOUND, "lm_head.weight: the dense decoder takes its logits "
                                                       "from model.embed_tokens.weight (model.rs:545)");
        return set_linear(m, &m->lm_head, data, nbytes, c.vocab, c.hidden, name);
    }
    if (name == "model.norm.weight") return set_dev_f32(m, &m->final_norm, data, nbytes, c.hidden, name);
    const std::string pre = "model.layers.";
    if (name.compare(0, pre.size(), pre) != 0) return fail(WPCG_E_NOTFOUND, "unknown tensor " + name);
    size_t dot = name.find('.', pre.size());
    if (dot == std::string::npos) return fail(WPCG_E_NOTFOUND, "unknown tensor " + name);
    uint32_t l = 0;
    try {
        l = (uint32_t)std::stoul(name.substr(pre.size(), dot - pre.size()));
    } catch (...) {
        return fail(WPCG_E_NOTFOUND, "unknown tensor " + name);
    }
    if (l >= c.n_layers) return fail(WPCG_E_NOTFOUND, "layer out of range: " + name);
    Layer& L = m->layers[l];
    const std::string t = name.substr(dot + 1);
    if (t == "input_layernorm.weight") return set_dev_f32(m, &L.in_ln, data, nbytes, c.hidden, name);
    if (t == "post_attention_layernorm.weight") return set_dev_f32(m, &L.post_ln, data, nbytes, c.hidden, name);
    if (t == "self_attn.q_norm.weight") return set_dev_f32(m, &L.q_norm, data, nbytes, c.head_dim, name);
    if (t == "self_attn.k_norm.weight") return set_dev_f32(m, &L.k_norm, data, nbytes, c.head_dim, name);
    if (t == "self_attn.q_proj.weight") return set_linear(m, &L.q, data, nbytes, qd, c.hidden, name);
    if (t == "self_attn.k_proj.weight") return set_linear(m, &L.k, data, nbytes, kvd, c.hidden, name);
    if (t == "self_attn.v_proj.weight") return set_linear(m, &L.v, data, nbytes, kvd, c.hidden, name);
    if (t == "self_attn.o_proj.weight") {
        // FAST mode merges the attention's chunk states while o_proj reads its
        // input. When one workgroup per 16-row tile leaves CUs idle even at
        // two K-slices, split K in two: each workgroup then merges only half
        // the heads (Qwen3-30B-A3B, 128 tiles: 2 slices 443 tok/s, 1 slice
        // 430, 4 slices 397; Qwen3-4B, 160 tiles: 1 slice 645, 2 slices 582).
        int cus = 0;
        WPCG_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, m->ctx->device));
        if (int rc = set_linear(m, &L.o, data, nbytes, c.hidden, qd, name)) return rc;
        const uint64_t tiles = pad_rows(c.hidden) / TILE_ROWS;
        // The split is a speed choice: when it cannot be planned the linear
        // keeps its one-slice plan (a valid state) and the tensor counts as set.
        if (2 * tiles <= (uint64_t)cus) (void)wpcg_linear_set_kslices(L.o, 2);
        return WPCG_OK;
    }
    if (c.n_experts == 0) {
        if (t == "mlp.gate_proj.weight") return set_linear(m, &L.gate, data, nbytes, c.inter, c.hidden, name);
        if (t == "mlp.up_proj.weight") return set_linear(m, &L.up, data, nbytes, c.inter, c.hidden, name);
        if (t == "mlp.down_proj.weight") return set_linear(m, &L.down, data, nbytes, c.hidden, c.inter, name);
        return fail(WPCG_E_NOTFOUND, "unknown tensor " + name);
    }
    if (t == "mlp.gate.weight") {
        if (nbytes != (uint64_t)c.n_experts * c.hidden * 4)
            return fail(WPCG_E_SHAPE, name + ": expected [n_experts, hidden] fp32");
        return wpcg_moe_set_router(L.moe, static_cast<const float*>(data));
    }
    const std::string ep = "mlp.experts.";
    if (t.compare(0, ep.size(), ep) == 0) {
        const size_t d2 = t.find('.', ep.size());
        if (d2 == std::string::npos) return fail(WPCG_E_NOTFOUND, "unknown tensor " + name);
        uint32_t e = 0;
        try {
            e = (uint32_t)std::stoul(t.substr(ep.size(), d2 - ep.size()));
        } catch (...) {
            return fail(WPCG_E_NOTFOUND, "unknown tensor " + name);
        }
        if (e >= c.n_experts) return fail(WPCG_E_NOTFOUND, "expert out of range: " + name);
        const std::string proj = t.substr(d2 + 1);
        wpcg_moe* moe = L.moe;
        const uint64_t bpb = block_bytes(m->scheme);
        DeviceMatrix* dm = nullptr;
        int bit = 0;
        if (proj == "gate_proj.weight") { dm = &moe->gate; bit = 1; }
        else if (proj == "up_proj.weight") { dm = &moe->up; bit = 2; }
        else if (proj == "down_proj.weight") { dm = &moe->down; bit = 4; }
        else return fail(WPCG_E_NOTFOUND, "unknown tensor " + name);
        if (nbytes != dm->rows * dm->nb * bpb)  // WpcLinearV4::new's block-count assert
            return fail(WPCG_E_SHAPE, name + ": block count does not match the expert shape");
        if (int rc = upload_rows(m->ctx, static_cast<const uint8_t*>(data), *dm, e * (dm->rows_pad / TILE_ROWS)))
            return rc;
        L.experts_set[e] |= (uint8_t)bit;
        return WPCG_OK;
    }
    return fail(WPCG_E_NOTFOUND, "unknown tensor " + name);
}

int wpcg_model_load_artifact(wpcg_model* m, wpcg_artifact* a)
{
    if (!m || !a) return fail(WPCG_E_ARG, "null argument");
    if (a->scheme != m->scheme) return fail(WPCG_E_ARG, "artifact scheme differs from the model's");
    std::vector<std::string> names = {"model.embed_tokens.weight"};
    if (m->cfg.n_experts) names.push_back("lm_head.weight");
    for (uint32_t l = 0; l < m->cfg.n_layers; l++) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        for (const char* t : {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                              "self_attn.o_proj.weight"})
            names.push_back(p + t);
        if (m->cfg.n_experts == 0) {
            for (const char* t : {"mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"})
                names.push_back(p + t);
        } else {
            for (uint32_t e = 0; e < m->cfg.n_experts; e++)
                for (const char* t : {"gate_proj.weight", "up_proj.weight", "down_proj.weight"})
                    names.push_back(p + "mlp.experts." + std::to_string(e) + "." + t);
        }
    }
    for (const std::string& n : names) {
        const void* bytes = nullptr;
        uint64_t size = 0;
        if (int rc = wpcg_artifact_tensor(a, n.c_str(), &bytes, &size)) return rc;
        if (int rc = wpcg_model_set_tensor(m, n.c_str(), bytes, size)) return rc;
    }
    return WPCG_OK;
}

int wpcg_model_load_safetensors(wpcg_model* m, wpcg_safetensors* st)
{
    if (!m || !st) return fail(WPCG_E_ARG, "null argument");
    const wpcg_model_config& c = m->cfg;
    std::vector<std::pair<std::string, uint64_t>> names = {{"model.norm.weight", c.hidden}};
    for (uint32_t l = 0; l < c.n_layers; l++) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        names.push_back({p + "input_layernorm.weight", c.hidden});
        names.push_back({p + "post_attention_layernorm.weight", c.hidden});
        names.push_back({p + "self_attn.q_norm.weight", c.head_dim});
        names.push_back({p + "self_attn.k_norm.weight", c.head_dim});
        if (c.n_experts) names.push_back({p + "mlp.gate.weight", (uint64_t)c.n_experts * c.hidden});
    }
    std::vector<float> buf;
    for (const auto& [n, count] : names) {
        buf.resize(count);
        if (int rc = wpcg_safetensors_read_f32(st, n.c_str(), buf.data(), count)) return rc;
        if (int rc = wpcg_model_set_tensor(m, n.c_str(), buf.data(), count * sizeof(float))) return rc;
    }
    return WPCG_OK;
}

int wpcg_model_set_mode(wpcg_model* m, int mode)
{
    if (!m || (mode != WPCG_MODE_EXACT && mode != WPCG_MODE_FAST)) return fail(WPCG_E_ARG, "null model or bad mode");
    m->mode = mode;
    auto lin = [mode](wpcg_linear* l) { if (l) l->mode = mode; };
    lin(m->embed);
    lin(m->lm_head);
    for (auto& L : m->layers) {
        for (wpcg_linear* l : {L.q, L.k, L.v, L.o, L.gate, L.up, L.down}) lin(l);
        if (L.moe) wpcg_moe_set_mode(L.moe, mode);
    }
    return WPCG_OK;
}

int wpcg_model_set_graphs(wpcg_model* m, int enabled)
{
    if (!m) return fail(WPCG_E_ARG, "null model");
    m->use_graph = enabled != 0;
    drop_graph(m);
    return WPCG_OK;
}

int wpcg_model_reset(wpcg_model* m)
{
    if (!m) return fail(WPCG_E_ARG, "null model");
    if (int rc = check_ctx(m->ctx)) return rc;
    DecodeState st{0, 0, m->cfg.max_pos, 0};
    WPCG_HIP(hipMemcpy(m->st, &st, sizeof st, hipMemcpyHostToDevice));
    return WPCG_OK;
}

int wpcg_model_position(wpcg_model* m, uint32_t* pos)
{
    if (!m || !pos) return fail(WPCG_E_ARG, "null argument");
    if (int rc = check_ctx(m->ctx)) return rc;
    DecodeState st;
    WPCG_HIP(hipStreamSynchronize(m->ctx->stream));
    WPCG_HIP(hipMemcpy(&st, m->st, sizeof st, hipMemcpyDeviceToHost));
    *pos = st.pos;
    return WPCG_OK;
}

int wpcg_model_forward_token(wpcg_model* m, uint32_t token, float* logits, uint32_t* argmax)
{
    if (!m) return fail(WPCG_E_ARG, "null model");
    if (token >= m->cfg.vocab) return fail(WPCG_E_ARG, "token id out of range");
    if (int rc = ready(m)) return rc;
    hipStream_t s = m->ctx->stream;
    DecodeState st;
    WPCG_HIP(hipStreamSynchronize(s));
    WPCG_HIP(hipMemcpy(&st, m->st, sizeof st, hipMemcpyDeviceToHost));
    if (st.pos >= m->cfg.max_pos) return fail(WPCG_E_ARG, "KV cache full (max_pos reached)");
    // every token comes from the host: keep the argmax out of tokens[]
    st.n_prompt = 0xffffffffu;
    WPCG_HIP(hipMemcpy(m->st, &st, sizeof st, hipMemcpyHostToDevice));
    WPCG_HIP(hipMemcpy(m->tokens + st.pos, &token, 4, hipMemcpyHostToDevice));
    if (int rc = run_step(m)) return rc;
    WPCG_HIP(hipStreamSynchronize(s));
    if (logits) WPCG_HIP(hipMemcpy(logits, m->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost));
    if (argmax) {
        WPCG_HIP(hipMemcpy(&st, m->st, sizeof st, hipMemcpyDeviceToHost));
        *argmax = st.last;
    }
    return WPCG_OK;
}

int wpcg_model_debug_read(wpcg_model* m, int which, float* out, uint64_t n)
{
    if (!m || !out) return fail(WPCG_E_ARG, "null argument");
    const wpcg_model_config& c = m->cfg;
    const uint64_t qd = (uint64_t)c.n_heads * c.head_dim, kvd = (uint64_t)c.n_kv_heads * c.head_dim;
    const float* src = nullptr;
    uint64_t len = 0;
    switch (which) {
        case 0: src = m->residual; len = c.hidden; break;
        case 1: src = m->normed; len = c.hidden; break;
        case 2: src = m->q; len = qd; break;
        case 3: src = m->k; len = kvd; break;
        case 4: src = m->v; len = kvd; break;
        case 5: src = m->attn; len = qd; break;
        case 7: src = m->logits; len = c.vocab; break;
        case 9: src = m->kc; len = (uint64_t)c.n_layers * kvd * c.max_pos; break;
        case 10: src = m->vc; len = (uint64_t)c.n_layers * kvd * c.max_pos; break;
        default: return fail(WPCG_E_ARG, "unknown buffer");
    }
    if (n > len) return fail(WPCG_E_ARG, "buffer holds " + std::to_string(len) + " floats");
    if (int rc = check_ctx(m->ctx)) return rc;
    WPCG_HIP(hipStreamSynchronize(m->ctx->stream));
    WPCG_HIP(hipMemcpy(out, src, n * 4, hipMemcpyDeviceToHost));
    return WPCG_OK;
}

int wpcg_model_generate(wpcg_model* m, const uint32_t* prompt, uint32_t n_prompt, uint32_t n_new,
                        uint32_t* out, float* decode_ms)
{
    if (!m || !prompt || !out) return fail(WPCG_E_ARG, "null argument");
    if (n_prompt == 0 || n_new == 0) return fail(WPCG_E_ARG, "need a prompt and at least one new token");
    if ((uint64_t)n_prompt + n_new - 1 > m->cfg.max_pos) return fail(WPCG_E_ARG, "prompt + new tokens exceed max_pos");
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= m->cfg.vocab) return fail(WPCG_E_ARG, "prompt token id out of range");
    if (int rc = ready(m)) return rc;
    hipStream_t s = m->ctx->stream;
    WPCG_HIP(hipStreamSynchronize(s));
    DecodeState st{0, n_prompt, m->cfg.max_pos, 0};
    WPCG_HIP(hipMemcpy(m->st, &st, sizeof st, hipMemcpyHostToDevice));
    WPCG_HIP(hipMemcpy(m->tokens, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice));
    hipEvent_t e0 = nullptr, e1 = nullptr;
    WPCG_HIP(hipEventCreate(&e0));
    WPCG_HIP(hipEventCreate(&e1));
    int rc = WPCG_OK;
    if (m->mode == WPCG_MODE_FAST && m->use_prefill && prefill_ok(m)) {
        // the prompt as batches (yielding the first new token), then n_new-1
        // decode steps
        rc = prefill_run(m, 0, n_prompt, n_prompt);
        (void)hipEventRecord(e0, s);
        for (uint32_t i = 1; i < n_new && rc == WPCG_OK; i++) rc = run_step(m);
    } else {
        // steps at positions 0..n_prompt-1 consume the prompt (the last one
        // yields the first new token); the n_new-1 after it are pure decode
        for (uint32_t i = 0; i < n_prompt + n_new - 1 && rc == WPCG_OK; i++) {
            if (i == n_prompt) (void)hipEventRecord(e0, s);
            rc = run_step(m);
        }
    }
    (void)hipEventRecord(e1, s);
    if (rc == WPCG_OK) {
        const hipError_t e = hipEventSynchronize(e1);
        if (e != hipSuccess) rc = hip_fail(e, "decode");
    }
    if (rc == WPCG_OK && decode_ms) {
        float ms = 0.0f;
        if (n_new > 1 && hipEventElapsedTime(&ms, e0, e1) != hipSuccess) ms = 0.0f;
        *decode_ms = ms;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc != WPCG_OK) return rc;
    WPCG_HIP(hipMemcpy(out, m->tokens + n_prompt, (size_t)n_new * 4, hipMemcpyDeviceToHost));
    return WPCG_OK;
}

int wpcg_model_set_prefill(wpcg_model* m, int enabled)
{
    if (!m) return fail(WPCG_E_ARG, "null model");
    m->use_prefill = enabled != 0;
    return WPCG_OK;
}

int wpcg_model_prefill(wpcg_model* m, const uint32_t* tokens, uint32_t n, float* logits, uint32_t* argmax)
{
    if (!m || !tokens) return fail(WPCG_E_ARG, "null argument");
    if (n == 0) return fail(WPCG_E_ARG, "no tokens");
    for (uint32_t i = 0; i < n; i++)
        if (tokens[i] >= m->cfg.vocab) return fail(WPCG_E_ARG, "token id out of range");
    if (int rc = ready(m)) return rc;
    hipStream_t s = m->ctx->stream;
    DecodeState st;
    WPCG_HIP(hipStreamSynchronize(s));
    WPCG_HIP(hipMemcpy(&st, m->st, sizeof st, hipMemcpyDeviceToHost));
    if ((uint64_t)st.pos + n > m->cfg.max_pos) return fail(WPCG_E_ARG, "KV cache full (max_pos reached)");
    WPCG_HIP(hipMemcpy(m->tokens + st.pos, tokens, (size_t)n * 4, hipMemcpyHostToDevice));
    // every token comes from the host: keep the argmax out of tokens[]
    const uint32_t pos0 = st.pos;
    st.n_prompt = 0xffffffffu;
    if (m->mode == WPCG_MODE_FAST && m->use_prefill && prefill_ok(m)) {
        if (int rc = prefill_run(m, pos0, n, st.n_prompt)) return rc;
    } else {
        WPCG_HIP(hipMemcpy(m->st, &st, sizeof st, hipMemcpyHostToDevice));
        for (uint32_t i = 0; i < n; i++)
            if (int rc = run_step(m)) return rc;
    }
    WPCG_HIP(hipStreamSynchronize(s));
    if (logits) WPCG_HIP(hipMemcpy(logits, m->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost));
    if (argmax) {
        WPCG_HIP(hipMemcpy(&st, m->st, sizeof st, hipMemcpyDeviceToHost));
        *argmax = st.last;
    }
    return WPCG_OK;
}

int wpcg_model_verify(wpcg_model* m, const uint32_t* tokens, uint32_t n, uint32_t* argmax, float* logits)
{
    if (!m || !tokens || !argmax) return fail(WPCG_E_ARG, "null argument");
    if (n == 0 || n > WPCG_VERIFY_MAX) return fail(WPCG_E_ARG, "verify takes 1.." + std::to_string(WPCG_VERIFY_MAX) + " tokens");
    for (uint32_t i = 0; i < n; i++)
        if (tokens[i] >= m->cfg.vocab) return fail(WPCG_E_ARG, "token id out of range");
    if (int rc = ready(m)) return rc;
    hipStream_t s = m->ctx->stream;
    const size_t V = m->cfg.vocab;
    DecodeState st;
    WPCG_HIP(hipStreamSynchronize(s));
    WPCG_HIP(hipMemcpy(&st, m->st, sizeof st, hipMemcpyDeviceToHost));
    if ((uint64_t)st.pos + n > m->cfg.max_pos) return fail(WPCG_E_ARG, "KV cache full (max_pos reached)");
    WPCG_HIP(hipMemcpy(m->tokens + st.pos, tokens, (size_t)n * 4, hipMemcpyHostToDevice));
    const uint32_t pos0 = st.pos;
    if (m->mode == WPCG_MODE_FAST && m->use_prefill && prefill_ok(m)) {
        if (int rc = verify_run(m, pos0, n)) return rc;
        WPCG_HIP(hipMemcpy(argmax, m->pf.vids, (size_t)n * 4, hipMemcpyDeviceToHost));
        if (logits) WPCG_HIP(hipMemcpy(logits, m->pf.vlogits, (size_t)n * V * 4, hipMemcpyDeviceToHost));
        return WPCG_OK;
    }
    // step by step (EXACT: the reference's steps exactly)
    st.n_prompt = 0xffffffffu;
    WPCG_HIP(hipMemcpy(m->st, &st, sizeof st, hipMemcpyHostToDevice));
    for (uint32_t i = 0; i < n; i++) {
        if (int rc = run_step(m)) return rc;
        WPCG_HIP(hipStreamSynchronize(s));
        if (logits) WPCG_HIP(hipMemcpy(logits + i * V, m->logits, V * 4, hipMemcpyDeviceToHost));
        WPCG_HIP(hipMemcpy(&st, m->st, sizeof st, hipMemcpyDeviceToHost));
        argmax[i] = st.last;
    }
    return WPCG_OK;
}

int wpcg_model_set_position(wpcg_model* m, uint32_t pos)
{
    if (!m) return fail(WPCG_E_ARG, "null model");
    if (int rc = check_ctx(m->ctx)) return rc;
    DecodeState st;
    WPCG_HIP(hipStreamSynchronize(m->ctx->stream));
    WPCG_HIP(hipMemcpy(&st, m->st, sizeof st, hipMemcpyDeviceToHost));
    if (pos > st.pos) return fail(WPCG_E_ARG, "set_position only moves back (to drop rejected tokens)");
    st.pos = pos;
    WPCG_HIP(hipMemcpy(m->st, &st, sizeof st, hipMemcpyHostToDevice));
    return WPCG_OK;
}

}  // extern "C"
