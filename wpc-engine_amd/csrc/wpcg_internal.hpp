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
    int valu = 0;             // plain GEMVs on the vector-ALU kernel (WPCG_FAST_KERNEL_VALU)
};

// Host transcodes from the reference's on-disk blocks (AoS) to the planes
// above, for rows [r0, r0 + nrows) of a matrix with nb blocks per row.
// r0 is a multiple of 16 and `codes`/`hp` point at tile r0/16's records;
// `params` at the matrix's parameter base. Bytes of padding rows in the
// last tile are left as they are (the caller zeroes them).
void transcode_rows(int scheme, const uint8_t* blocks, uint64_t r0, uint64_t nrows, uint64_t nb,
                    uint8_t* codes, uint8_t* hp, uint32_t* params_tile_major);

// ---- decode state (decode.hip, gemv.hip) ------------------------------------
// Device-resident position and token bookkeeping of a decode: the step at
// position `pos` reads tokens[pos]; its argmax is `last`, and is written to
// tokens[pos+1] when pos+1 >= n_prompt (a generated token).
struct DecodeState {
    uint32_t pos, n_prompt, max_pos, last;
};
// ---- kernel launchers (gemv.hip) ----------------------------------------
// One GEMV y = W x (+ bias). With `sel` set, `m` describes one expert
// (rows, rows_pad, nb) and its planes are the first of a stack of experts;
// the job is expert sel[sel_k] of the stack (device-resident routing).
// FAST-mode input transforms (the GEMV applies them to x as it reads it):
//   XF_NORM  RMSNorm of x with weights nw and epsilon eps (norm.rs:4-13):
//            y = W (x * nw) / sqrt(mean(x^2) + eps); needs kg = 1;
//   XF_SILU  x = silu(x) * x2 (qwen3_moe_model.rs:518-522);
//   XF_MERGE x = the attention output merged from the chunk states of
//            launch_attention_chunks: x = part_o, x2 = part_ml, with st,
//            head_dim and the query head count in the job.
constexpr int XF_NONE = 0, XF_NORM = 1, XF_SILU = 2, XF_MERGE = 3;
// Router scores routed inside a FAST launch: at most this many experts.
constexpr int ROUTE_MAXN = 256;
struct GemvJob {
    const DeviceMatrix* m;
    const FastPlan* plan;
    const float* x;
    const float* bias;
    float* y;
    const int32_t* sel = nullptr;
    int sel_k = 0;
    // FAST mode only
    int xform = XF_NONE;
    const float* x2 = nullptr;
    const float* nw = nullptr;
    float eps = 0.0f;
    const DecodeState* st = nullptr;  // XF_MERGE: checked present (the merge reads every chunk)
    int head_dim = 0, n_heads = 0;    // XF_MERGE
    // Deferred K-split (plan->kg >= 2, not routed): slice 0 writes its sum
    // (+ bias) to y and slice k >= 1 its sum to y2 + (k-1)*rows, with no
    // handoff between the slices; the readers add them (x_add, bias2 below).
    float* y2 = nullptr;
    // XF_NORM: x + x_add[0] + ... + x_add[n_xa-1] (vectors of cols floats,
    // added in that order) is the vector normalised; n_xa <= 2
    const float* x_add = nullptr;
    int n_xa = 1;
    // with bias: y = sum + (bias + bias2[0] + ... + bias2[n_b2-1]) (vectors
    // of rows floats); n_b2 <= 2
    const float* bias2 = nullptr;
    int n_b2 = 1;
    // routed: the rows of experts sel[0..top_k) side by side as one K of
    // top_k * cols (one K-slice: plan->kg = 1), x of slot k at x + k*cols
    // (g) and x2 + k*cols (u), scaled by rw[k]; y = bias + the row sum
    int routed = 0;
    const float* rw = nullptr;
    // route from router scores: softmax + top_k over n_exp scores in the
    // kernel; the job is slot sel_k; ids and weights also go to ids_out / w_out
    const float* scores = nullptr;
    int n_exp = 0, top_k = 0, norm_topk = 0;
    int32_t* ids_out = nullptr;
    float* w_out = nullptr;
    // one K-slice, not routed: workgroup w also stores at amax[w] the key of
    // the first largest of its output rows (see launch_argmax_keys_next)
    uint64_t* amax = nullptr;
};
// The deferred K-split's shape: its readers add at most two deferred
// vectors (n_xa, n_b2 <= 2) and a model's deferral buffer holds two, so a
// deferred job has 2 or 3 K-slices, and a routed job (one slice per slot)
// cannot defer.
inline bool deferred_split_ok(int kg, bool routed) { return kg >= 2 && kg <= 3 && !routed; }

// FAST mode: a workgroup computes fast_tiles_per_wg 16-row tiles over a
// K-slice of at most fast_max_slice blocks (the slice's x digits live in LDS).
constexpr int FAST_MAXBK = 64;
// Tiles per workgroup: as many as keep a whole row in one slice, so that
// each wave streams more blocks and a launch needs fewer workgroups: 4 tiles
// for rows of at most 16 blocks once the matrix has 32 tiles (measured: 11%
// faster Qwen3-30B-A3B-shaped decode than one tile per workgroup), 2 for
// rows of at most 32 blocks once it has 192 (a 160-tile matrix of 32-block
// rows ran 10% faster on 160 workgroups than on 80). Rows longer than one
// slice take 2 tiles from 128 tiles on (2560x9728: 240 workgroups beat
// 480), and matrices of 512 tiles or more take 2 in any case. Short rows
// (at most 8 blocks) of a matrix of 256 tiles or more take 2, not 4: the
// config-0 GEMV (4864x896, 304 tiles of 7 blocks) ran 3.69 us on 152
// workgroups against 3.87 on 76 and 4.53 on 304.
inline int fast_tiles_per_wg(uint64_t rows, uint64_t nb)
{
    const uint64_t tiles = pad_rows(rows) / TILE_ROWS;
    if (tiles >= 256 && nb <= 8) return 2;
    if (tiles >= 32 && nb <= FAST_MAXBK / 4) return 4;
    if (tiles >= 192 && nb <= FAST_MAXBK / 2) return 2;
    if (tiles >= 128 && nb > FAST_MAXBK) return 2;
    return tiles >= 512 ? 2 : 1;
}
inline uint64_t fast_max_slice(uint64_t rows, uint64_t nb) { return FAST_MAXBK / fast_tiles_per_wg(rows, nb); }
hipError_t launch_gemv_exact(const DeviceMatrix& m, const float* x, const float* bias, float* y,
                             hipStream_t s, const int32_t* sel = nullptr, int sel_k = 0);
// All jobs must share the scheme. At most MAX_JOBS per launch.
constexpr int MAX_JOBS = 16;
hipError_t launch_gemv_fast(const GemvJob* jobs, int n, hipStream_t s);
// Up to MAX_JOBS EXACT GEMVs of one scheme in one launch (m, x, bias, y,
// sel, sel_k of each job), each bit-identical to launch_gemv_exact's.
hipError_t launch_gemv_exact_multi(const GemvJob* jobs, int n, hipStream_t s);
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

// ---- batched GEMM (gemm.hip) -------------------------------------------------
// Y = X W^T for up to GEMM_MAX_M activations per launch. Up to 16 columns one
// kernel packs X into LDS itself (a wave per row tile, K-slices of at most
// GEMM_SMALL_MAXBK blocks); above that X is packed by a first kernel and a
// workgroup of GEMM_WG_THREADS / 64 waves covers a row group of 8 row tiles,
// GEMM_TILES_PER_WAVE per wave.
constexpr int GEMM_WG_THREADS = 512;
constexpr int GEMM_TILES_PER_WAVE = 1;
constexpr int GEMM_MAX_M = 64;
constexpr int GEMM_SMALL_MAXBK = 30;
// Workspace of one matrix, sized for GEMM_MAX_M columns; fixed once made so
// captured graphs keep valid pointers.
struct GemmWork {
    int kg_req = 0;                 // requested K-slices (0 = the library's choice)
    int kg = 1;                     // K-slices, more than 16 columns
    int kg_small = 1;               // K-slices, up to 16 columns
    void* xf = nullptr;             // packed X: nb * 4 column tiles * 4 KiB
    float* xsum = nullptr;          // per-block column sums: nb * 64
    float* part = nullptr;          // partial Y: [kg][64][rows_pad] or [kg_small][16][rows_pad]
    uint32_t* counters = nullptr;   // one per row group, self-resetting
};
void free_gemm(GemmWork& w);  // keeps kg_req
int gemm_row_groups(uint64_t rows);        // more than 16 columns
int gemm_small_row_groups(uint64_t rows);  // up to 16 columns
// Splits (requested kg, 0 = the library's choice), normalised to non-empty
// slices (and, for the small kernel, slices of at most GEMM_SMALL_MAXBK).
int gemm_kslices(uint64_t rows, uint64_t nb, int req);
int gemm_small_kslices(uint64_t rows, uint64_t nb, int req);
// x_mode: GX_F32 (x rounded to bf16), GX_BF16, GX_SPLIT (fp32 x as hi + lo
// bf16 terms, relative 2^-18; at most GEMM_MAX_M_SPLIT columns). res: [M][rows]
// added to Y (may alias y) or null.
constexpr int GX_F32 = 0, GX_BF16 = 1, GX_SPLIT = 2;
constexpr int GEMM_MAX_M_SPLIT = 32;
hipError_t launch_gemm(const DeviceMatrix& m, const GemmWork& w, const void* x, int x_mode, int M,
                       const float* bias, const float* res, float* y, hipStream_t s);
// Expert-grouped GEMM, one launch for every expert of a stack (or of two
// stacks of one shape over the same X: m2 and y2, else null): m is one
// expert's shape, its planes the first of the stack (expert e at e * its
// plane sizes). X comes as launch_pf_digits' records of its xrows rows.
// Work item i = items[3i..3i+2] = {expert, first pair p0, count <=
// GEMM_GROUP_COLS}; its column c reads X row rowidx[p0 + c] (null: row
// p0 + c) and writes Y row p0 + c. *nitems (device) items are live; their
// (item, matrix, row tile) units are split evenly over wgs workgroups (one
// per CU).
// Needs m.nb <= GEMM_GROUP_MAXBK (the item's X digits sit in LDS whole) and
// m.rows_pad <= GEMM_GROUP_MAXROWS (keeps every buffer offset of an expert's
// planes well inside 32 bits).
constexpr int GEMM_GROUP_COLS = 16;
constexpr int GEMM_GROUP_MAXBK = 16;
constexpr int GEMM_GROUP_MAXROWS = 2048;
// Many rows of fp32 X in the SPLIT mode as one launch per matrix: X packed
// once (launch_gemm_pack_rows; the pack serves every matrix with K inputs),
// then workgroups over (row group, group of 32 rows of X); xf holds
// K/128 * gemm_rows_tiles(M) * 4 KiB, xsum K/128 * gemm_rows_tiles(M) * 16
// floats.
inline int gemm_rows_tiles(int M) { return (M + 31) / 32 * 4; }
hipError_t launch_gemm_pack_rows(const float* x, int M, int K, void* xf, float* xsum, hipStream_t s);
// kg > 1: K in kg slices whose partials go to part (kg * (gemm_rows_tiles(M) /
// 4 * 32) * m.rows_pad floats), added in slice order by a second launch
// (reduce), or left there for launch_pf_reduce_norm (bias, res, y unused).
hipError_t launch_gemm_packed_rows(const DeviceMatrix& m, const void* xf, const float* xsum, int M, const float* bias,
                                   const float* res, float* y, hipStream_t s, int kg = 1, float* part = nullptr,
                                   bool reduce = true);
// Up to three matrices of the same K and scheme over one packed X in one
// launch (the projections that share an input: q, k, v; gate, up); no
// residual. With rope, matrix e's epilogue per mode[e] (128-wide heads,
// rows % 128 == 0; M rows of X are the tokens at positions pos0 ..):
// GEMM_ROPE_Q the head RMSNorm (weights nw[e]) and the rotation (cos_t /
// sin_t [max_pos][64]) into Y, GEMM_ROPE_K the same into cache[e]
// ([head][max_pos][128]), GEMM_ROPE_V the rows as computed into cache[e];
// 0 the plain output.
constexpr int GEMM_ROPE_Q = 1, GEMM_ROPE_K = 2, GEMM_ROPE_V = 3;
struct GemmRope {
    int mode[3];
    float* cache[3];
    const float* nw[3];
    const float* cos_t;
    const float* sin_t;
    int pos0, max_pos;
    float eps;
};
hipError_t launch_gemm_packed_rows_multi(const DeviceMatrix* const* ms, const float* const* biases, float* const* ys,
                                         int count, const void* xf, const float* xsum, int M, hipStream_t s,
                                         const GemmRope* rope = nullptr);
// The grouped GEMM's X: rows x rows of K fp32 (xu non-null: silu(x) * xu,
// the FAST steps' arithmetic, xu of x's shape) to int8 digits, dg
// rows * K * 4 bytes, and per 128-value block {s_b 2^-7, sum}, dxs
// rows * K / 128 * 2 floats.
hipError_t launch_pf_digits(const float* x, const float* xu, int rows, int K, void* dg, float* dxs, hipStream_t s);
hipError_t launch_gemm_grouped(const DeviceMatrix& m, const DeviceMatrix* m2, const void* dg, const float* dxs,
                               int xrows, const int* rowidx, const int* items, const int* nitems, int wgs, float* y,
                               float* y2, hipStream_t s);

// ---- the no-allocation workspace (scratch.hip) --------------------------------
// scratch_setup(device) looks up the device address of the library's fixed
// workspace array on `device` (which must be current) and keeps it;
// wpcg_ctx_create runs it. scratch_ptr(device) returns that address (null
// before set-up). launch_fill_u32 writes v to p[0..n) with a kernel (no
// memset node, so a captured graph replays it correctly).
int scratch_setup(int device);
void* scratch_ptr(int device);
hipError_t launch_fill_u32(uint32_t* p, int n, uint32_t v, hipStream_t s);

// ---- host helpers shared by the C ABI files (capi*.cpp) -----------------
hipStream_t pick(wpcg_ctx* ctx, wpcg_stream s);  // NULL = the context stream
int check_ctx(wpcg_ctx* ctx);                     // non-null, device current
uint64_t block_bytes(int scheme);                 // 68 (v4) / 100 (v3)
void free_matrix(DeviceMatrix& m);
void free_plan(FastPlan& p);
uint64_t plane_blocks(const DeviceMatrix& m);     // rows_pad * nb (at least 1)
// Zeroed planes for `count` matrices of m's shape, stacked tile after tile.
int alloc_planes(DeviceMatrix& m, uint64_t count, hipStream_t s);
// Transcodes m.rows rows of reference blocks into m's planes from tile
// `tile0` on (synchronous; bounded host staging). Padding rows stay 0.
int upload_rows(wpcg_ctx* ctx, const uint8_t* blocks, const DeviceMatrix& m, uint64_t tile0);
// FAST split-K: slices for a rows x nb matrix (kg 0 = the library's choice)
// and the workspace for it, fixed for the matrix's lifetime (captured
// graphs keep using it).
int plan_kslices(uint64_t rows, uint64_t nb, int kg);
int make_plan(const DeviceMatrix& m, FastPlan& plan, hipStream_t s, int kg = 0);

// ---- MoE pieces (moe.hip) -------------------------------------------------
// nw (FAST only): RMSNorm of x with weights nw and epsilon eps folded in.
// FAST: x_add, if set, is added to x as it is read (a deferred K-slice).
hipError_t launch_dense(const float* w, int out_f, int in_f, int mode, const float* x,
                        const float* bias, float* y, hipStream_t s, const float* nw = nullptr,
                        float eps = 0.0f, const float* x_add = nullptr);
hipError_t launch_softmax(float* x, int n, hipStream_t s);
int route_max_n();
hipError_t launch_route(const float* p, int n, int top_k, int norm_topk, int32_t* ids, float* w,
                        hipStream_t s);
hipError_t launch_silu_mul(const float* g, const float* u, float* out, size_t n, hipStream_t s);
hipError_t launch_combine(const float* ys, const int32_t* ids, const float* w, int top_k,
                          float* out, int h, const float* add, hipStream_t s);
hipError_t launch_softmax_route(const float* scores, int n, int top_k, int norm_topk, int32_t* ids,
                                float* w, hipStream_t s);
// The routed MLP of one layer: out = (add ? add + : ) sum_k w_k expert_k(xn),
// xn = x, or with nw set RMSNorm(x) with weights nw and epsilon eps. FAST
// mode runs it as three launches: the router (norm folded in), the chosen
// experts' gate and up (each workgroup routes from the scores itself and
// folds the norm in), and one routed down projection whose K-slices are
// the chosen experts (SiLU*up and the routing weight folded into its x,
// the combine and the residual into its ordered split-K sum).
// defer_combine (EXACT): the combine is left out; the caller folds it into
// the next RMSNorm of `out` (launch_rms_norm_combine with ys, ids and w).
int moe_run(wpcg_moe* m, const float* x, float* out, const float* add, hipStream_t s,
            const float* nw = nullptr, float eps = 0.0f, const float* x_add = nullptr,
            bool defer_combine = false);

// ---- decode step (decode.hip) ----------------------------------------------
// With rope set, workgroup 0 also copies the RoPE row at the position
// (cos_t / sin_t rows of `half` floats) to rope: cos then sin.
hipError_t launch_embed_tok(const DeviceMatrix& m, const uint32_t* tokens, const DecodeState* st,
                            float* out, hipStream_t s, const float* cos_t = nullptr,
                            const float* sin_t = nullptr, int half = 0, float* rope = nullptr);
hipError_t launch_rms_norm(int mode, const float* x, const float* w, int n, float eps, float* out,
                           hipStream_t s);
// EXACT: x += the MoE combine sum_k cw[k] * ys[k] (chosen order, slots with
// ids[k] >= 0; as the combine launch), then out = RMSNorm(x) as
// launch_rms_norm in EXACT mode, in one launch.
bool rms_norm_combine_ok(int n, int top_k);
hipError_t launch_rms_norm_combine(float* x, const float* w, int n, float eps, float* out, const float* ys,
                                   const int32_t* ids, const float* cw, int top_k, hipStream_t s);
// q/k RMSNorm + RoPE, KV append, scores, softmax and output of one layer's
// attention at the state's position; max_pos <= attention_max_pos().
int attention_max_pos();
hipError_t launch_attention(int mode, const float* q, const float* k, const float* v, const float* qn,
                            const float* kn, int nh, int nkv, int hd, float eps, float scale,
                            const float* cos_t, const float* sin_t, const DecodeState* st, float* kc,
                            float* vc, float* out, hipStream_t s);
// FAST attention over ATTN_CHUNKS chunks of the positions: each chunk's
// softmax state goes to part_o [ATTN_CHUNKS][nh][hd] (unnormalised output)
// and part_ml [ATTN_CHUNKS][nh][2] (max, sum of exps); the o_proj GEMV
// merges them (XF_MERGE). Needs attention_fast_ok (head_dim 64 or 128).
// rope: the step's RoPE row, cos then sin at the position (hd floats, as
// launch_embed_tok leaves it); cache_pos: positions per head in kc / vc.
constexpr int ATTN_CHUNKS = 16;
bool attention_fast_ok(int nh, int nkv, int hd);
hipError_t launch_attention_chunks(const float* q, const float* k, const float* v, const float* qn,
                                   const float* kn, int nh, int nkv, int hd, float eps, float scale,
                                   const float* rope, int cache_pos, const DecodeState* st, float* kc,
                                   float* vc, float* part_o, float* part_ml, hipStream_t s);
// The chunk states of launch_attention_chunks merged into out [nh][hd], as
// the XF_MERGE transform merges them (hd <= 128).
hipError_t launch_attention_merge(const float* part_o, const float* part_ml, int nh, int hd, float* out,
                                  hipStream_t s);
hipError_t launch_add(float* x, const float* y, int n, hipStream_t s);
// ---- batched prefill (decode.hip, gemv.hip, moe.hip, prefill.hip) ---------
// n tokens at positions pos0 .. pos0+n-1, row t of every batch buffer being
// position pos0 + t.
hipError_t launch_embed_rows(const DeviceMatrix& m, const uint32_t* tokens, int n, float* out, hipStream_t s);
hipError_t launch_rms_norm_rows(int mode, const float* x, const float* w, int n, int rows, float eps, float* out,
                                hipStream_t s);
// q_norm/k_norm + RoPE (Q in place, keys into kc), values into vc (unless
// qk_done: the q/k/v GEMM's epilogue did that, head_dim 128 only), then
// causal attention of every row over positions 0..pos0+t: with head_dim 128
// written as o_proj's packed X (xf, xsum: launch_gemm_pack_rows's layout for
// n rows of nh*128), with 64 into out [n][nh*hd]. Needs attention_fast_ok.
hipError_t launch_prefill_attention(float* Q, const float* Kx, const float* Vx, const float* qn, const float* kn,
                                    int nh, int nkv, int hd, float eps, float scale, const float* cos_t,
                                    const float* sin_t, int pos0, int n, int max_pos, float* kc, float* vc,
                                    float* out, void* xf, float* xsum, hipStream_t s, bool qk_done = false);
// FAST routing of score rows [rows][n]: the FAST one-token projection's own
// routing per row (n <= ROUTE_MAXN, top_k <= MAX_JOBS).
hipError_t launch_route_rows(const float* scores, int n, int rows, int top_k, int norm_topk, int32_t* ids, float* w,
                             hipStream_t s);
// RMSNorm (FAST) of n rows of H into the GEMM's packed X (xf, xsum in
// launch_gemm_pack_rows's layout), H % 128 == 0.
hipError_t launch_rms_pack_rows(const float* X, const float* w, int n, int H, float eps, void* xf, float* xsum,
                                hipStream_t s);
// A K-sliced packed-rows GEMM's partials (launch_gemm_packed_rows with
// reduce = false) summed with bias and the residual into X [M][H], then each
// row's FAST RMSNorm with weights w into XN; H <= PF_NORM_MAXH. dg non-null:
// XN's rows also as launch_pf_digits writes them (dg, dxs), H % 128 == 0.
constexpr int PF_NORM_MAXH = 4096;
hipError_t launch_pf_reduce_norm(const float* part, int kg, int M, int H, int rows_pad, const float* bias, float* X,
                                 const float* w, float eps, float* XN, void* dg, float* dxs, hipStream_t s);
// R[t][e] = X[t] . W[e] (fp32 router rows), R is [T][E].
hipError_t launch_pf_router(const float* X, const float* W, int T, int E, int K, float* R, hipStream_t s);
// (token, slot) pairs sorted by expert for launch_gemm_grouped: pair_tok
// [P], pair_pos [P], items [3 * (P / GEMM_GROUP_COLS + E)], nitems [1].
constexpr int PF_MAX_PAIRS = 8192;
constexpr int PF_GROUP_MAXT = 256;  // tokens per grouping (the prefill pass holds at most 256 rows)
hipError_t launch_pf_group(const int32_t* ids, int P, int E, int top_k, int* pair_tok, int* pair_pos, int* items,
                           int* nitems, hipStream_t s);
hipError_t launch_pf_combine(float* X, const float* D, const float* w, const int* pair_pos, int T, int top_k, int H,
                             hipStream_t s);
// Y = X W^T (+ res) for M rows of fp32 X with the linear's batched kernels
// (x_mode GX_*), its workspace made on first use (not under capture).
int linear_gemm(wpcg_linear* L, const float* x, int x_mode, uint32_t M, const float* res, float* y, hipStream_t s);
// The same from the keys a FAST GEMV's workgroups left (GemvJob::amax), one
// per workgroup in row order: a row's key is (its value's order-preserving
// bits, -0 read as +0) << 32 | ~row, 0 for a value that does not beat -inf
// (NaN included), so the largest key is the first largest value.
hipError_t launch_argmax_keys_next(const uint64_t* keys, int n, DecodeState* st, uint32_t* tokens,
                                   hipStream_t s);
hipError_t launch_argmax_next(const float* logits, int n, DecodeState* st, uint32_t* tokens,
                              hipStream_t s);
// out[r] = the first index of the largest logit of row r (logits [rows][n]).
hipError_t launch_argmax_rows(const float* logits, int n, int rows, uint32_t* out, hipStream_t s);

// ---- JSON DOM (json.cpp): safetensors headers, their index, config.json ----
struct JsonValue {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0.0;
    bool is_uint = false;  // an integer literal that fits uint64 (u holds it)
    uint64_t u = 0;
    std::string str;
    std::vector<JsonValue> arr;
    std::vector<std::pair<std::string, JsonValue>> obj;
    const JsonValue* get(const std::string& key) const;  // null if absent or not an object
};
bool json_parse(const char* text, size_t n, JsonValue& out, std::string& err);

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
    wpcg::GemmWork gemm;    // made by the first batched call
    float* bias = nullptr;  // device, out_f floats, or null
    int mode = WPCG_MODE_EXACT;
    // staging for the synchronous *_host twins
    std::mutex host_mu;
    float* x_stage = nullptr;
    float* y_stage = nullptr;
};

struct wpcg_dense {
    wpcg_ctx* ctx = nullptr;
    uint64_t out_f = 0, in_f = 0;
    float* w = nullptr;     // device, row-major [out_f][in_f]
    float* bias = nullptr;  // device or null
    int mode = WPCG_MODE_EXACT;
};

// One layer's routed experts. The three projections are stored as stacks:
// expert e's gate rows are tiles [e*T, (e+1)*T) of `gate` (T = the
// expert's tile count), likewise up and down, so a routed GEMV finds its
// expert from the id alone. The DeviceMatrix fields describe one expert.
struct wpcg_moe {
    wpcg_ctx* ctx = nullptr;
    int scheme = 4, mode = WPCG_MODE_EXACT, norm_topk = 1;
    uint32_t n_exp = 0, hidden = 0, inter = 0, top_k = 0;
    wpcg_dense* router = nullptr;
    wpcg::DeviceMatrix gate, up, down;
    wpcg::FastPlan plan;  // kg = 1 for every expert shape (checked at creation)
    // FAST: the chosen experts' down rows side by side fit one K-slice
    // (false: the unfused path)
    bool routed = false;
    float *scores = nullptr, *w = nullptr, *g = nullptr, *u = nullptr, *h = nullptr, *ys = nullptr;
    float* xn = nullptr;  // the normed input when the norm is not folded in
    int32_t* ids = nullptr;
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
