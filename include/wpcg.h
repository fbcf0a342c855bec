/*
 * wpcg.h -- C ABI of the MI355X (gfx950) decode backend for WPC-quantized
 * weights: the drop-in boundary for the reference's quantized GEMV path.
 *
 * Plain C types only: opaque handles, pointers, sizes, int status codes. No
 * exceptions or panics cross this boundary. Every call returns WPCG_OK or an
 * error code; wpcg_last_error_string() describes the last failure on the
 * calling thread.
 *
 * Reference interfaces replaced (paths relative to the reference repository,
 * jpytka666-jpg/wpc-engine):
 *   trait Linear            wpc-runtime/src/weights.rs:17-22
 *   trait EmbeddingTable    wpc-runtime/src/weights.rs:25-31
 *   WpcModelDataV4          wpc-runtime/src/wpc_weights_v4.rs:39-99
 *   WpcLinearV4             wpc-runtime/src/wpc_weights_v4.rs:117-194
 *   WpcEmbeddingV4          wpc-runtime/src/wpc_weights_v4.rs:196-273
 *   WpcModelDataV3/LinearV3/EmbeddingV3  wpc-runtime/src/wpc_weights_v3.rs
 *
 * Device pointers, streams and threading:
 *   - `*_dev` arguments are device pointers on the handle's device;
 *     `wpcg_stream` is a hipStream_t passed as void*, NULL meaning the
 *     context's own stream. Device calls are stream-ordered and return
 *     before the work completes; `*_host` twins are synchronous.
 *   - Handles may be used from several threads; calls on one handle that
 *     use its internal staging buffers (`*_host`) are serialized internally.
 */
#ifndef WPCG_H
#define WPCG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define WPCG_OK             0
#define WPCG_E_IO           1 /* file missing or unreadable                   */
#define WPCG_E_FORMAT       2 /* malformed meta / block range / block_size    */
#define WPCG_E_SHAPE        3 /* in_features % 128, block-count mismatch      */
#define WPCG_E_NOTFOUND     4 /* tensor name absent from the meta             */
#define WPCG_E_DEVICE       5 /* no usable GPU, or a HIP runtime failure      */
#define WPCG_E_ARG          6 /* NULL handle / pointer, bad enum, bad size    */
#define WPCG_E_NOMEM        7 /* host or device allocation failed             */
#define WPCG_E_UNSUPPORTED  8 /* valid request this build does not provide    */

/* ---- enums ---- */
#define WPCG_SCHEME_V3 3 /* 6-bit codes, 100-byte blocks (wpc-format/src/lib.rs:202-292) */
#define WPCG_SCHEME_V4 4 /* 4-bit codes, 68-byte blocks  (wpc-format/src/lib.rs:318-391) */

/* GEMV arithmetic. EXACT reproduces matvec_v4_fused / matvec_v3_fused
 * (wpc-eval/src/fused_kernel.rs:163-189, 237-271) bit for bit: eight fp32
 * accumulators with dequant fma(code, scale, zp), then hsum_avx2's order.
 * FAST regroups each block as scale*sum(code*x) + zp*sum(x) with fp32
 * accumulation; it is within the reference's 1e-4 relative tolerance but
 * not bit-identical. */
#define WPCG_MODE_EXACT 0
#define WPCG_MODE_FAST  1

/* Dequantization rounding. FMA: fma(code, scale, zp), one rounding, as the
 * AVX2 GEMV does. TWO: zp + code*scale, two roundings, as row_decode_into_v4
 * and the scalar fallbacks do (wpc_weights_v4.rs:111, fused_kernel.rs:289). */
#define WPCG_ROUND_FMA 0
#define WPCG_ROUND_TWO 1

typedef struct wpcg_ctx wpcg_ctx;
typedef struct wpcg_artifact wpcg_artifact;
typedef struct wpcg_linear wpcg_linear;
typedef struct wpcg_event wpcg_event;
typedef struct wpcg_model_config_s wpcg_model_config; /* defined with the decode step below */
typedef void* wpcg_stream;

/* ---- library ---- */
const char* wpcg_last_error_string(void);
const char* wpcg_version(void);
int wpcg_device_count(int* n);

/* ---- context: one GPU plus a default stream (no reference counterpart:
 * the reference is CPU-only; this is the device the handles live on) ----
 * Handles created on a context (linears, events, graphs) keep it alive:
 * after wpcg_ctx_destroy the caller must not use `ctx` again, but existing
 * handles keep working, and the stream is released with the last of them. */
int wpcg_ctx_create(int device, wpcg_ctx** out);
int wpcg_ctx_destroy(wpcg_ctx* ctx);
int wpcg_ctx_stream(wpcg_ctx* ctx, wpcg_stream* out);
int wpcg_ctx_sync(wpcg_ctx* ctx);

/* Device memory and copies on the context's stream (synchronous copies). */
int wpcg_dev_alloc(wpcg_ctx* ctx, size_t bytes, void** out_dev);
int wpcg_dev_free(wpcg_ctx* ctx, void* dev);
int wpcg_memcpy_h2d(wpcg_ctx* ctx, void* dst_dev, const void* src, size_t bytes);
int wpcg_memcpy_d2h(wpcg_ctx* ctx, void* dst, const void* src_dev, size_t bytes);
int wpcg_memcpy_d2d(wpcg_ctx* ctx, void* dst_dev, const void* src_dev, size_t bytes);

/* Timing events recorded on a stream (NULL = context stream). */
int wpcg_event_create(wpcg_ctx* ctx, wpcg_event** out);
int wpcg_event_destroy(wpcg_event* ev);
int wpcg_event_record(wpcg_event* ev, wpcg_stream stream);
int wpcg_event_elapsed_ms(wpcg_event* start, wpcg_event* stop, float* ms);

/* ---- artifact: model_v{3,4}.meta + model_v{3,4}.wpc ----
 * Replaces WpcModelDataV4::open (wpc_weights_v4.rs:46-77) and its v3 twin:
 * reads the JSON meta ({"layers":[{"name","shape","offset_bytes",
 * "size_bytes"}],"block_size"}), requires block_size == 128, memory-maps the
 * .wpc file. Errors: E_IO (missing/unreadable), E_FORMAT (bad JSON,
 * block_size != 128). */
int wpcg_artifact_open(const char* dir, int scheme, wpcg_artifact** out);
int wpcg_artifact_close(wpcg_artifact* a);
/* tensor_range + blocks_for (wpc_weights_v4.rs:80-98): the tensor's bytes in
 * the mapping. E_NOTFOUND for an unknown name; E_FORMAT when size is not a
 * whole number of blocks or the range exceeds the file. */
int wpcg_artifact_tensor(wpcg_artifact* a, const char* name, const void** bytes,
                         uint64_t* size);
int wpcg_artifact_tensor_count(wpcg_artifact* a, uint64_t* n);

/* ---- Linear ----
 * Replaces WpcLinearV4::new (wpc_weights_v4.rs:127-155) / WpcLinearV3::new:
 * E_SHAPE unless in_f % 128 == 0 and the tensor holds out_f*(in_f/128)
 * blocks. The blocks are transcoded on the host into the device layout and
 * uploaded; `bias` (host, out_f floats) may be NULL. */
int wpcg_linear_create(wpcg_ctx* ctx, wpcg_artifact* a, const char* name, uint64_t out_f,
                       uint64_t in_f, const float* bias, wpcg_linear** out);
/* The same from blocks in memory (reference on-disk byte layout). */
int wpcg_linear_from_blocks(wpcg_ctx* ctx, int scheme, const void* blocks, uint64_t nbytes,
                            uint64_t out_f, uint64_t in_f, const float* bias,
                            wpcg_linear** out);
int wpcg_linear_destroy(wpcg_linear* lin);
/* Linear::in_features / out_features (weights.rs:18-19) */
int wpcg_linear_shape(wpcg_linear* lin, uint64_t* out_f, uint64_t* in_f);
int wpcg_linear_set_mode(wpcg_linear* lin, int mode);
/* FAST mode splits K over `kslices` workgroups per group of output rows
 * (0 = the library's choice for the shape). A workgroup covers 16, 32 or
 * 64 rows (one, two or four 16-row tiles, chosen from the matrix's shape)
 * and a slice at most 64, 32 or 16 blocks respectively; requests are
 * raised to that minimum and capped at one block per slice. When the
 * library must split, it uses slices of at most 32 blocks. Replaces the
 * matrix's split-K workspace: graphs captured
 * earlier with this linear must be destroyed first. No reference
 * counterpart (a tuning knob). */
int wpcg_linear_set_kslices(wpcg_linear* lin, int kslices);
int wpcg_linear_kslices(wpcg_linear* lin, int* kslices);
/* Which FAST kernel a plain GEMV of this linear runs (no reference
 * counterpart; the reference's AVX2 row kernel is the one restated):
 * WPCG_FAST_KERNEL_MFMA (the default) puts the block dot products on the
 * matrix cores with x as four int8 digits; WPCG_FAST_KERNEL_VALU computes
 * them on the vector ALU in fp32 with x read as fp32 (codes unpacked by
 * shift/mask in registers). Both are held to the same bounds against the
 * reference kernel. Launches with an input transform (the decode step's
 * folded RMSNorm, SiLU, attention merge, routing) always use the MFMA
 * kernel. */
#define WPCG_FAST_KERNEL_MFMA 0
#define WPCG_FAST_KERNEL_VALU 1
int wpcg_linear_set_fast_kernel(wpcg_linear* lin, int kernel);
/* The split wpcg_linear_set_kslices would use for an out_f x in_f matrix
 * (host-only query; every slice is non-empty and within the limits above). */
int wpcg_plan_kslices(uint64_t out_f, uint64_t in_f, int requested, int* kslices);
/* Device bytes the weights occupy (codes + block parameters). */
int wpcg_linear_device_bytes(wpcg_linear* lin, uint64_t* bytes);

/* Linear::matvec (weights.rs:20-21, wpc_weights_v4.rs:165-193):
 * y = W x (+ bias); y is fully overwritten. x_dev: in_f floats, y_dev:
 * out_f floats; x and y must not overlap. */
int wpcg_linear_matvec(wpcg_linear* lin, const float* x_dev, float* y_dev, wpcg_stream stream);
/* Host-pointer twin with exactly Linear::matvec's synchronous semantics. */
int wpcg_linear_matvec_host(wpcg_linear* lin, const float* x, float* y);

/* n independent matvecs, ys[i] = W_i xs[i] (+ bias_i), issued together: FAST
 * members of one scheme share one launch (up to 16 per launch), EXACT members
 * launch one by one. Matrices that read the same input (q/k/v, gate/up, the
 * experts of a token) fill the GPU together. The linears' outputs must not
 * overlap each other or any input. No reference counterpart: the reference
 * calls Linear::matvec once per matrix (qwen3_moe_model.rs:430-432, 516-517). */
int wpcg_linear_matvec_multi(int n, wpcg_linear* const* lins, const float* const* xs,
                             float* const* ys, wpcg_stream stream);

/* Batched GEMM Y = X W^T (+ bias on every row of Y) for M activations.
 * No reference counterpart: the reference runs one token at a time, and
 * names batched prefill its principal missing piece (README.md:174-180).
 * X: M rows of in_f values, contiguous, fp32 (x_dtype WPCG_DTYPE_F32) or
 * bf16 bit patterns (WPCG_DTYPE_BF16); Y: M rows of out_f floats. With
 * M == 1 and fp32 X this is wpcg_linear_matvec in the linear's mode. Else
 * the matrix-core kernel runs (64 rows of X per launch pair): the codes
 * are exact, X is rounded to bf16 (exact when given as bf16), each block's
 * dots accumulate in fp32 and its scale and zero point are applied in fp32
 * (the weights are never rounded). The first batched call on a linear
 * allocates its workspace (about 16 KiB per 128 inputs plus the split-K
 * partials); make it before capturing a graph that contains the call.
 * WPCG_DTYPE_F32_SPLIT: fp32 X fed to the matrix cores as two bf16 terms
 * hi = bf16(x), lo = bf16(x - hi), so X is carried to a relative 2^-18
 * (32 rows of X per launch; twice the matrix-core work). */
#define WPCG_DTYPE_F32  0
#define WPCG_DTYPE_BF16 1
#define WPCG_DTYPE_F32_SPLIT 2
int wpcg_linear_gemm(wpcg_linear* lin, const void* x_dev, int x_dtype, uint32_t M, float* y_dev,
                     wpcg_stream stream);
/* Host-pointer twin (synchronous). */
int wpcg_linear_gemm_host(wpcg_linear* lin, const void* x, int x_dtype, uint32_t M, float* y);
/* wpcg_linear_gemm that allocates nothing: the same kernels, splits and
 * results (bit for bit), with the workspace (packed X, per-block column
 * sums, split-K partials, counters) carved from a fixed device array of
 * WPCG_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on
 * until the process ends, instead of the linear's own workspace. No
 * reference counterpart: for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc); the first batched call on a linear may be this one even
 * while a graph is being captured. Every call on one GPU uses that GPU's
 * one array: calls that overlap on a GPU (other streams, other threads)
 * race and must be serialized by the caller. E_UNSUPPORTED (naming the
 * bytes needed) when the call's workspace exceeds the array; with M == 1
 * and fp32 X it runs wpcg_linear_matvec, whose workspace the linear made
 * when it was created. */
#define WPCG_NOALLOC_SCRATCH_BYTES (16u << 20)
int wpcg_linear_gemm_noalloc(wpcg_linear* lin, const void* x_dev, int x_dtype, uint32_t M, float* y_dev,
                             wpcg_stream stream);
/* K-slices of the batched kernels (0 = the library's choice; a tuning knob,
 * no reference counterpart), applied to both (M <= 16 and M > 16) within
 * their limits. Frees the workspace; the next batched call makes it. The
 * query returns the splits in use (or planned) for M <= 16 and M > 16. */
int wpcg_linear_set_gemm_kslices(wpcg_linear* lin, int kslices);
int wpcg_linear_gemm_kslices(wpcg_linear* lin, int* kslices_small, int* kslices);

/* EmbeddingTable::embed (weights.rs:28; wpc_weights_v4.rs:241-249): decode
 * row `token` into out (in_f floats) as zp + code*scale with two roundings.
 * EmbeddingTable::logits (weights.rs:30) is wpcg_linear_matvec on the same
 * table. E_ARG when token >= out_f. */
int wpcg_linear_embed(wpcg_linear* lin, uint32_t token, float* out_dev, wpcg_stream stream);
int wpcg_linear_embed_host(wpcg_linear* lin, uint32_t token, float* out);

/* Whole-matrix dequantization to fp32, row-major [out_f][in_f], natural
 * weight order, in the given rounding (WPCG_ROUND_*). For parity checks. */
int wpcg_linear_dequant(wpcg_linear* lin, int rounding, float* w_dev, wpcg_stream stream);

/* A second device copy of the same weights (device-to-device; no reference
 * counterpart). Used to rotate a working set larger than the 256 MB
 * Infinity Cache when measuring HBM-bound throughput. */
int wpcg_linear_clone(wpcg_linear* lin, wpcg_linear** out);

/* ---- encoder (host only) ----
 * encode_tensor_v4 / encode_tensor_v3 (wpc-core/src/quant_encoder.rs:49-57,
 * 88-96): n fp32 values (n % 128 == 0) to n/128 blocks of 68 / 100 bytes in
 * the reference layout, as the artifact compiler writes them. Multithreaded;
 * needs no GPU. */
int wpcg_encode(int scheme, const float* w, uint64_t n, void* out_blocks);

/* ---- fp32 dense linear: the MoE router ----
 * Replaces DenseLinear (wpc-runtime/src/weights.rs:35-79), which the
 * Qwen3-MoE model builds for `mlp.gate.weight` (qwen3_moe_model.rs:182-187).
 * `w` is host [out_f][in_f] row-major fp32, `bias` host out_f floats or NULL.
 * EXACT matches DenseLinear::matvec bit for bit (index-order sums, product
 * and sum rounded separately); FAST sums in parallel. */
typedef struct wpcg_dense wpcg_dense;
int wpcg_dense_create(wpcg_ctx* ctx, const float* w, uint64_t out_f, uint64_t in_f,
                      const float* bias, wpcg_dense** out);
int wpcg_dense_destroy(wpcg_dense* d);
int wpcg_dense_set_mode(wpcg_dense* d, int mode);
int wpcg_dense_matvec(wpcg_dense* d, const float* x_dev, float* y_dev, wpcg_stream stream);

/* softmax_inplace (wpc-runtime/src/norm.rs:28-43) over n floats in place,
 * bit for bit: exp is the reference host libm's expf. */
int wpcg_softmax(wpcg_ctx* ctx, float* x_dev, uint32_t n, wpcg_stream stream);

/* Qwen3MoeModel::route (qwen3_moe_model.rs:376-402): the top_k largest of n
 * probabilities (ties to the lowest index, NaN never chosen), written in
 * descending order to ids/weights (top_k each); with norm_topk the weights
 * are divided by their sum. Slots left unfilled get id -1, weight 0.
 * n <= 512, top_k <= n. */
int wpcg_route(wpcg_ctx* ctx, const float* probs_dev, uint32_t n, uint32_t top_k, int norm_topk,
               int32_t* ids_dev, float* weights_dev, wpcg_stream stream);

/* out[i] = silu(g[i]) * u[i], silu(g) = g / (1 + exp(-g)), as the expert
 * and dense MLPs compute it (qwen3_moe_model.rs:518-522, model.rs:527-531). */
int wpcg_silu_mul(wpcg_ctx* ctx, const float* g_dev, const float* u_dev, float* out_dev,
                  uint64_t n, wpcg_stream stream);

/* ---- Qwen3-MoE sparse MLP of one layer ----
 * Replaces the router + route + expert loop of Qwen3MoeModel::forward_token
 * (qwen3_moe_model.rs:500-530) with the experts' weights resident on the
 * device. n_exp experts, each gate/up [inter x hidden] and down
 * [hidden x inter] in `scheme` blocks; the router [n_exp x hidden] fp32.
 * The routing stays on the device: the chosen experts' GEMVs read their ids
 * from device memory. EXACT mode is bit-identical to the reference; FAST
 * uses the FAST GEMV and router. */
typedef struct wpcg_moe wpcg_moe;
int wpcg_moe_create(wpcg_ctx* ctx, int scheme, uint32_t n_exp, uint32_t hidden, uint32_t inter,
                    uint32_t top_k, int norm_topk, wpcg_moe** out);
int wpcg_moe_destroy(wpcg_moe* m);
int wpcg_moe_set_router(wpcg_moe* m, const float* w);
/* Expert e's three matrices, blocks in the reference layout (as
 * WpcLinearV4::new takes them for experts.{e}.{gate,up,down}_proj.weight). */
int wpcg_moe_set_expert(wpcg_moe* m, uint32_t e, const void* gate, const void* up,
                        const void* down);
/* All experts of layer `layer` from an artifact: tensors
 * model.layers.{layer}.mlp.experts.{e}.{gate,up,down}_proj.weight. */
int wpcg_moe_load_experts(wpcg_moe* m, wpcg_artifact* a, uint32_t layer);
int wpcg_moe_set_mode(wpcg_moe* m, int mode);
/* out = sum over the router's top_k experts of weight * down(silu(gate x) *
 * up x), in chosen order. ids/weights (top_k each, device) receive the
 * routing when non-NULL. x and out must not overlap. */
int wpcg_moe_forward(wpcg_moe* m, const float* x_dev, float* out_dev, int32_t* ids_dev,
                     float* weights_dev, wpcg_stream stream);

/* rms_norm (wpc-runtime/src/norm.rs:4-13): out = x * (1 / sqrt(mean(x^2) +
 * eps)) * w over n floats. EXACT sums the squares in index order (bit for
 * bit the reference); FAST sums them as a tree. */
int wpcg_rms_norm(wpcg_ctx* ctx, const float* x_dev, const float* w_dev, uint32_t n, float eps,
                  float* out_dev, int mode, wpcg_stream stream);

/* ---- checkpoint I/O: safetensors and config.json ----
 * The dense checkpoint the reference reads the fp32 tensors from (norms and
 * routers; WPC only compresses 2-D matrices), as one model.safetensors or
 * as shards named by model.safetensors.index.json. Every file is mapped and
 * validated as the `safetensors` crate 0.4.5 validates it (header length,
 * '{' start, offsets tiling the data in order, sizes matching shape and
 * dtype); where the reference panics (invalid file, missing tensor,
 * unsupported dtype) these return E_FORMAT, E_NOTFOUND, E_UNSUPPORTED. */
typedef struct wpcg_safetensors wpcg_safetensors;
/* ShardedSafetensors::open (wpc-runtime/src/weights.rs:197-244): the
 * directory's model.safetensors when present, else the shards of its
 * model.safetensors.index.json `weight_map` (E_IO when neither exists). */
int wpcg_safetensors_open(const char* model_dir, wpcg_safetensors** out);
/* SafetensorsFile::open (weights.rs:130-138), one file. */
int wpcg_safetensors_open_file(const char* path, wpcg_safetensors** out);
int wpcg_safetensors_close(wpcg_safetensors* st);
/* SafetensorsFile::names (weights.rs:140-142): every tensor, header order,
 * shard after shard. The name stays valid until close. */
int wpcg_safetensors_tensor_count(wpcg_safetensors* st, uint64_t* n);
int wpcg_safetensors_name(wpcg_safetensors* st, uint64_t i, const char** name);
/* ShardedSafetensors::shape (weights.rs:256-263): *ndim always set; E_ARG
 * when it exceeds max_dims. */
int wpcg_safetensors_shape(wpcg_safetensors* st, const char* name, uint32_t* ndim, uint64_t* dims,
                           uint32_t max_dims);
/* The header's dtype string ("F32", "BF16", ...). No reference counterpart. */
int wpcg_safetensors_dtype(wpcg_safetensors* st, const char* name, const char** dtype);
/* ShardedSafetensors::read_f32 / SafetensorsFile::read_f32
 * (weights.rs:149-178, 246-254): F32 as stored, F16 exactly (a NaN gains
 * the quiet bit, as half 2.x converts it), BF16 as its bits << 16; n must
 * equal the element count (E_SHAPE). */
int wpcg_safetensors_read_f32(wpcg_safetensors* st, const char* name, float* out, uint64_t n);
/* Config::load / Config::from_json_str (wpc-runtime/src/config.rs:85-95)
 * into a model config: required vocab_size, hidden_size,
 * num_hidden_layers, num_attention_heads, num_key_value_heads,
 * intermediate_size, rope_theta, rms_norm_eps; tie_word_embeddings is
 * type-checked but does not choose the head: `tied` is 1 for a dense
 * decoder (qwen3_model.rs:187-206 builds no lm_head, model.rs:545 calls
 * embed.logits) and 0 for Qwen3-MoE (qwen3_moe_model.rs:337-343 always
 * loads lm_head.weight); head_dim falls back to hidden_size /
 * num_attention_heads (Config::head_dim, config.rs:59-62). model_type
 * "qwen3_moe" selects the MoE decoder, as wpc-runtime/src/main.rs:73-77
 * does, with the fields of moe_dims (qwen3_moe_model.rs:121-135: each
 * required, top_k in 1..=num_experts, norm_topk_prob defaulting to true);
 * any other config is a dense decoder (n_experts = 0). max_pos, the
 * KV-cache length, is the caller's. E_FORMAT names the offending field. */
int wpcg_config_parse(const char* json_text, uint32_t max_pos, wpcg_model_config* out);
int wpcg_config_load(const char* path, uint32_t max_pos, wpcg_model_config* out);

/* ---- device-resident decode step ----
 * A dense Qwen3 (n_experts == 0, SwiGLU MLP) or Qwen3-MoE decoder whose
 * weights, fp32 KV cache, activations, position and tokens stay on the GPU.
 * One step is Model::forward_token (wpc-runtime/src/model.rs:419-547) or
 * Qwen3MoeModel::forward_token (qwen3_moe_model.rs:406-542) followed by
 * argmax (sampling.rs:3-14); it runs as one replayed HIP graph. EXACT mode
 * reproduces the reference's logits bit for bit, one launch per operation.
 * FAST mode computes the same step within a tolerance (FAST GEMVs and
 * router, tree sums) in six launches per MoE layer (five dense): the
 * RMSNorms are folded into the GEMVs that read them, attention is split
 * over chunks of positions whose softmax states o_proj merges, routing runs
 * inside the expert gate/up launch, and one routed down projection covers
 * the chosen experts with SiLU*up, the routing weights and the residual. */
struct wpcg_model_config_s {
    uint32_t n_layers, hidden, n_heads, n_kv_heads, head_dim;
    uint32_t inter;                          /* dense MLP width (n_experts == 0)   */
    uint32_t vocab;
    uint32_t n_experts, top_k, moe_inter;    /* Qwen3-MoE (n_experts > 0)          */
    int32_t norm_topk;                       /* renormalise the top-k weights      */
    int32_t tied;                            /* logits from the embedding table: 1 */
                                             /* exactly when n_experts == 0 (the   */
                                             /* reference's loaders; see below)    */
    uint32_t max_pos;                        /* KV-cache length                    */
    float eps;                               /* RMSNorm epsilon                    */
    double rope_theta;
};
typedef struct wpcg_model wpcg_model;
/* E_UNSUPPORTED when cfg->tied is not (n_experts == 0): the head is the
 * embedding table for a dense decoder and lm_head for Qwen3-MoE, as the
 * reference's loaders build them. */
int wpcg_model_create(wpcg_ctx* ctx, int scheme, const wpcg_model_config* cfg, wpcg_model** out);
int wpcg_model_destroy(wpcg_model* m);
/* A tensor by the reference's name: quantized matrices (model.embed_tokens,
 * lm_head, model.layers.{l}.self_attn.{q,k,v,o}_proj, mlp.{gate,up,down}_proj,
 * mlp.experts.{e}.{gate,up,down}_proj; all `.weight`) take blocks in the
 * model's scheme; model.norm, {input,post_attention}_layernorm,
 * self_attn.{q,k}_norm and the router mlp.gate take fp32. E_NOTFOUND for a
 * name the config has no place for, E_SHAPE for a size that disagrees. */
int wpcg_model_set_tensor(wpcg_model* m, const char* name, const void* data, uint64_t nbytes);
/* Every quantized matrix of the config from an artifact (the fp32 tensors,
 * which the reference reads from safetensors, go through set_tensor). */
int wpcg_model_load_artifact(wpcg_model* m, wpcg_artifact* a);
/* The fp32 tensors from a checkpoint by the reference's names, as
 * build_layers and the loaders read them (qwen3_moe_model.rs:140-196,
 * 327-365; qwen3_model.rs:40-90, 187-206): model.norm.weight and per
 * layer {input,post_attention}_layernorm, self_attn.{q,k}_norm and, for
 * MoE, the router mlp.gate.weight (F32/F16/BF16 widened to fp32). */
int wpcg_model_load_safetensors(wpcg_model* m, wpcg_safetensors* st);
int wpcg_model_set_mode(wpcg_model* m, int mode);
/* Steps as one replayed HIP graph (enabled, the default) or enqueued launch
 * by launch (for tools that cannot trace graph replays). No reference
 * counterpart. */
int wpcg_model_set_graphs(wpcg_model* m, int enabled);
/* Empty the KV cache (position 0). */
int wpcg_model_reset(wpcg_model* m);
int wpcg_model_position(wpcg_model* m, uint32_t* pos);
/* One step at the next position with input `token`: logits (host, vocab
 * floats) and/or their argmax, either may be NULL. E_ARG when the cache is
 * full. */
int wpcg_model_forward_token(wpcg_model* m, uint32_t token, float* logits, uint32_t* argmax);
/* The prompt loop of wpc-runtime/src/main.rs:259-262 (forward_token per
 * prompt token, keeping the last logits) for n tokens at the next n
 * positions: the same result as n forward_token calls, logits and argmax of
 * the last. EXACT mode runs exactly those steps (bit-identical). FAST mode
 * runs the tokens as batches of up to 256 rows (the reference's missing
 * batched prefill, README.md:174-180): every layer reads each weight once
 * per batch; the dense projections run on the matrix cores with X carried
 * as two bf16 terms (WPCG_DTYPE_F32_SPLIT), attention is causal over the
 * cache, and the experts run grouped: the (token, slot) pairs are sorted by
 * expert and one launch per projection covers every expert's tokens. Its
 * results match the step-by-step FAST ones within FAST's tolerance. E_ARG
 * when the cache cannot hold n more positions. */
int wpcg_model_prefill(wpcg_model* m, const uint32_t* tokens, uint32_t n, float* logits, uint32_t* argmax);
/* FAST mode: prompts of wpcg_model_prefill and wpcg_model_generate go
 * through the batched prefill (enabled, the default) or step by step. No
 * reference counterpart. */
int wpcg_model_set_prefill(wpcg_model* m, int enabled);
/* Speculative verification, the hook the reference names as blocked on a
 * batched pass (WHITEPAPER.md:576-586, 662-693): the n tokens (the last
 * accepted token, then the drafts) at the next n positions in one batch,
 * and argmax[i] = the greedy next token after tokens[0..i], which is what
 * forward_token(tokens[i]) would return at that point. A draft d_{i+1} is
 * accepted while it equals argmax[i]; wpcg_model_set_position then drops
 * the rejected positions. logits (may be NULL) receives n rows of vocab
 * floats. FAST mode: one prefill pass plus the final norm and head as one
 * batched GEMM over the n rows (within FAST's tolerance of the steps);
 * EXACT mode: the n steps (bit-identical). 1 <= n <= WPCG_VERIFY_MAX. No
 * reference counterpart. */
#define WPCG_VERIFY_MAX 64
int wpcg_model_verify(wpcg_model* m, const uint32_t* tokens, uint32_t n, uint32_t* argmax, float* logits);
/* Move the position back to pos (<= the current one): later cache entries
 * are ignored and overwritten by the next steps. No reference counterpart. */
int wpcg_model_set_position(wpcg_model* m, uint32_t pos);
/* Greedy generation from position 0: the prompt, then n_new tokens, each
 * the argmax of the previous step's logits, written to out (n_new ids).
 * Steps run back to back on the device with no host round trip; in FAST
 * mode the prompt goes through the batched prefill (wpcg_model_prefill).
 * decode_ms (may be NULL) receives the time of the n_new-1 steps after the
 * prompt. */
int wpcg_model_generate(wpcg_model* m, const uint32_t* prompt, uint32_t n_prompt, uint32_t n_new,
                        uint32_t* out, float* decode_ms);

/* Diagnostics, no reference counterpart: copies n floats of one of the
 * decode step's device buffers as the last step left them. which: 0
 * residual, 1 normed (after the final norm; EXACT mode), 2 q (the
 * projection), 3 k and 4 v (the last layer's projections), 5 attention
 * output (EXACT mode, and FAST dense models, which merge the attention
 * chunks in a launch of their own; FAST Qwen3-MoE merges them inside
 * o_proj and leaves this buffer unwritten), 7 logits, 9 K cache, 10 V
 * cache ([layer][kv_head][max_pos][head_dim]). In FAST dense models whose
 * down projection defers its K-slices to its readers, the residual (0)
 * excludes the last layer's deferred slices: the head adds them as it
 * reads the residual. */
int wpcg_model_debug_read(wpcg_model* m, int which, float* out, uint64_t n);

/* ---- HIP graphs over the context stream (no reference counterpart) ----
 * wpcg_graph_begin starts capturing the context's stream; device calls with
 * stream NULL are then recorded instead of run, until wpcg_graph_end
 * instantiates them. Synchronous *_host calls must not be made while
 * capturing. */
typedef struct wpcg_graph wpcg_graph;
int wpcg_graph_begin(wpcg_ctx* ctx);
int wpcg_graph_end(wpcg_ctx* ctx, wpcg_graph** out);
int wpcg_graph_launch(wpcg_graph* g, wpcg_stream stream);
int wpcg_graph_destroy(wpcg_graph* g);

#ifdef __cplusplus
}
#endif
#endif /* WPCG_H */
