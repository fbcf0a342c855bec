/*
 * wpc_oracle.h -- CPU restatement of the reference's quantized GEMV / MoE
 * routing path, used ONLY as the checker.
 *
 * TEST INFRASTRUCTURE. Nothing in the product (the HIP library, its C-ABI,
 * the host mirror) links, loads or calls this code. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
 *
 * Block byte layouts are the reference's on-disk ones (little-endian):
 *   v4 block, 68 B : [zero_point f16][scale f16][64 B codes], byte j holds
 *                    code j in its low nibble and code j+64 in its high nibble
 *                    (wpc-format/src/lib.rs:324-339).
 *   v3 block, 100 B: [zero_point f16][scale f16][96 B codes, four 6-bit codes
 *                    per three bytes] (wpc-format/src/lib.rs:206-220).
 *   v2 block, 132 B: [zero_point f16][scale f16][128 B codes, one per byte]
 *                    (wpc-format/src/lib.rs:128-145).
 *
 * Floating-point contract: this file is compiled with -ffp-contract=off, so
 * an expression `a + b * c` rounds twice exactly as the Rust reference does
 * (Rust never contracts); single-rounding steps are written as fmaf(), which
 * is what `_mm256_fmadd_ps` computes per lane.
 */
#ifndef WPC_ORACLE_H
#define WPC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    OR_BLOCK = 128,
    OR_V4_BYTES = 68,
    OR_V4_PACKED = 64,
    OR_V3_BYTES = 100,
    OR_V3_PACKED = 96,
    OR_V2_BYTES = 132,
};

/* ---- binary16 (half 2.7.1 `f16::to_f32` / `f16::from_f32`) ---- */
float    or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
void     or_f16_to_f32_array(const uint16_t* h, float* out, size_t n);
void     or_f32_to_f16_array(const float* f, uint16_t* out, size_t n);

/* ---- block codecs ---- */
void or_v4_pack_codes(const uint8_t codes[128], uint8_t packed[64]);
void or_v4_unpack_codes(const uint8_t packed[64], uint8_t codes[128]);
void or_v3_pack_codes(const uint8_t codes[128], uint8_t packed[96]);
void or_v3_unpack_codes(const uint8_t packed[96], uint8_t codes[128]);
/* v3 two-plane layout (defined by this build; absent from the reference):
 *   lp[j] = (c[j] & 15) | (c[j+64] & 15) << 4            j < 64
 *   hp[j] = sum_q ((c[j+32q] >> 4) & 3) << 2q             j < 32, q < 4   */
void or_v3tp_pack(const uint8_t codes[128], uint8_t lp[64], uint8_t hp[32]);
void or_v3tp_unpack(const uint8_t lp[64], const uint8_t hp[32], uint8_t codes[128]);

/* ---- encoder (wpc-core/src/quant_encoder.rs) ---- */
void or_affine_quant_block_v2(const float w[128], uint8_t out[132]);
void or_affine_quant_block_v3(const float w[128], uint8_t out[100]);
void or_affine_quant_block_v4(const float w[128], uint8_t out[68]);
/* n must be a multiple of 128; out receives n/128 blocks. */
void or_encode_tensor_v4(const float* data, size_t n, uint8_t* out);
void or_encode_tensor_v3(const float* data, size_t n, uint8_t* out);

/* ---- row kernels (wpc-eval/src/fused_kernel.rs) ---- */
float or_matvec_v4_scalar(const uint8_t* blocks, const float* x, size_t n_blocks);
float or_matvec_v4_fused(const uint8_t* blocks, const float* x, size_t n_blocks);
float or_matvec_v3_scalar(const uint8_t* blocks, const float* x, size_t n_blocks);
float or_matvec_v3_fused(const uint8_t* blocks, const float* x, size_t n_blocks);
float or_matvec_v2_scalar(const uint8_t* blocks, const float* x, size_t n_blocks);
/* The same two fused kernels written with the reference's AVX2 intrinsics.
 * Return 0 and leave *out untouched when the CPU lacks AVX2+FMA. */
int   or_have_avx2_fma(void);
int   or_matvec_v4_fused_avx2(const uint8_t* blocks, const float* x, size_t n_blocks, float* out);
int   or_matvec_v3_fused_avx2(const uint8_t* blocks, const float* x, size_t n_blocks, float* out);

/* ---- Linear / EmbeddingTable (wpc-runtime/src/wpc_weights_v{3,4}.rs) ----
 * kernel: 0 = scalar fallback, 1 = fused restatement, 2 = AVX2 intrinsics.
 * Rows are split over `threads` POSIX threads (rayon in the reference);
 * each row is independent, so the result does not depend on `threads`. */
void or_linear_v4_matvec(const uint8_t* blocks, size_t out_f, size_t in_f,
                         const float* x, const float* bias, float* y,
                         int kernel, int threads);
void or_linear_v3_matvec(const uint8_t* blocks, size_t out_f, size_t in_f,
                         const float* x, const float* bias, float* y,
                         int kernel, int threads);
void or_embed_v4(const uint8_t* blocks, size_t hidden, uint32_t token, float* out);
void or_embed_v3(const uint8_t* blocks, size_t hidden, uint32_t token, float* out);
/* Batched: Y[m] = W X[m] for m < M (M independent matvec calls). */
void or_linear_v4_matmul(const uint8_t* blocks, size_t out_f, size_t in_f,
                         const float* X, size_t M, float* Y, int kernel, int threads);

/* ---- dense ops (wpc-runtime/src/{weights,norm,rope,sampling}.rs) ---- */
void     or_dense_matvec(const float* W, size_t out_f, size_t in_f, const float* x,
                         const float* bias, float* y);
void     or_softmax_inplace(float* x, size_t n);
void     or_rms_norm(const float* x, const float* w, size_t n, float eps, float* out);
void     or_apply_rope(float* x, size_t d, size_t pos, double theta);
uint32_t or_argmax(const float* logits, size_t n);
float    or_silu_mul(float g, float u);
/* out[i] = or_silu_mul(g[i], u[i]) for i < n */
void     or_silu_mul_array(const float* g, const float* u, float* out, size_t n);

/* Qwen3MoeModel::route (qwen3_moe_model.rs:376-402). Returns the number of
 * experts chosen (top_k unless fewer are selectable). */
size_t or_route(const float* scores, size_t n, size_t top_k, int norm_topk,
                int32_t* ids, float* weights);

/* Sparse MLP block of Qwen3MoeModel::forward_token (qwen3_moe_model.rs:500-530)
 * for one token: router -> softmax -> route -> expert loop; writes mlp_out
 * (NOT added to the residual). Experts are v4 matrices; expert e's gate/up
 * are [inter, hidden], down is [hidden, inter], all in reference blocks. */
typedef struct {
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
} or_expert_v4;
void or_moe_ffn_v4(const float* router_w, size_t n_exp, size_t hidden, size_t inter,
                   size_t top_k, int norm_topk, const or_expert_v4* experts,
                   const float* x, float* mlp_out, int32_t* chosen_ids,
                   float* chosen_w, int kernel, int threads);

/* ---- decode step (model.rs:419-547, qwen3_moe_model.rs:406-542) ---- */
typedef struct {
    size_t n_layers, hidden, n_heads, n_kv_heads, head_dim, inter, vocab;
    size_t n_exp, top_k, moe_inter; /* n_exp == 0 -> dense SwiGLU */
    int norm_topk;
    double rope_theta;
    float eps;
} or_model_cfg;

typedef struct {
    const float* input_ln;   /* [hidden] */
    const float* post_ln;    /* [hidden] */
    const float* q_norm;     /* [head_dim] */
    const float* k_norm;     /* [head_dim] */
    const uint8_t *q, *k, *v, *o;          /* v4 blocks */
    const uint8_t *gate, *up, *down;       /* dense MLP (n_exp == 0) */
    const float* router;                   /* [n_exp, hidden] fp32 */
    const or_expert_v4* experts;           /* [n_exp] */
} or_layer_v4;

typedef struct {
    or_model_cfg cfg;
    const uint8_t* embed;   /* [vocab, hidden] v4 */
    const uint8_t* lm_head; /* [vocab, hidden] v4: the MoE head; a dense model ignores it */
    const float* final_norm;
    const or_layer_v4* layers;
} or_model_v4;

typedef struct or_kv_cache or_kv_cache;
or_kv_cache* or_kv_cache_new(const or_model_cfg* cfg, size_t max_pos);
void         or_kv_cache_free(or_kv_cache* c);
size_t       or_kv_cache_len(const or_kv_cache* c);
/* One token through the stack; logits [vocab]. Returns 0 on success. */
int or_forward_token_v4(const or_model_v4* m, uint32_t token, or_kv_cache* cache,
                        float* logits, int kernel, int threads);

#ifdef __cplusplus
}
#endif
#endif
