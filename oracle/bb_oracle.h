/*
 * bb_oracle.h — TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the reference (maximecb/bebelm 0.3.6, pure Rust) MoE FFN path, used
 * as the parity checker for the HIP library and as the timed CPU baseline in bench.py.
 * Nothing in the product (bebelm_amd/) links, loads or calls this code: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg do.
 *
 * Every function names the reference file:line it restates. Dtype codes are ggml's
 * (src/tensor.rs:41-63): F32=0, F16=1, Q4_K=12, Q6_K=14.
 *
 * Pinning status (what fixes each function's bits; tests/test_oracle_*.py):
 *   f16_to_f32, get_scale_min_k4, dequantize_*     known answers dequant.rs:189-276 + exhaustive f16
 *   quantize_q8, dot_q4k/q6k_block_q8              known answer matmul.rs:1192-1204, LCG precision
 *                                                  values 0.0041545 / 0.0057328 (matmul.rs:1343-1421),
 *                                                  brute force vs dequantised f64 dot
 *   row / batch / fused-batch / matmul             exact-equality invariants matmul.rs:1273-1548
 *   sigmoid / silu                                 call the platform expf, which is what the
 *                                                  reference's f32::exp resolves to (glibc 2.35)
 *   dot (router, f32)                              PARITY UNPINNED for its last bits: the lane
 *                                                  reduce order lives in the `wide` 0.7.33 crate,
 *                                                  absent from /root/reference. Restated as
 *                                                  fmaf chains + the AVX reduce_add tree.
 *   sort tie order                                 PARITY UNPINNED for exactly equal keys
 *                                                  (sort_unstable_by); ties are counted.
 *   conv_step / conv_prefill                       known answers conv.rs:77-144 (432, 400, 15,
 *                                                  [12, 64]) and prefill == rolled steps
 *   softmax                                        known answers softmax.rs:34-108, the f64-sum
 *                                                  discrimination test, closed forms
 *   attention_decode                               known answers attention.rs:64-92, brute force
 *                                                  in f64, invariants (one position -> v)
 *   rope_neox                                      rope.rs:37-78 (identity at 0, angle = pos for
 *                                                  the first pair, split-half pairing, norm);
 *                                                  sin/cos/pow are the platform libm's, as the
 *                                                  reference's f32 sin_cos / powf
 *   conv / attention operators                     batch == token by token (model.rs:668-705)
 */
#ifndef BB_ORACLE_H
#define BB_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { BBO_F32 = 0, BBO_F16 = 1, BBO_Q4_K = 12, BBO_Q6_K = 14 };

/* One activation vector quantised to the reference's Q8 (matmul.rs:130-137). */
typedef struct {
  int8_t* q;       /* [n]      */
  float* scales;   /* [n/256]  */
  int32_t* sums;   /* [n/32]   */
} bbo_q8;

/* FusedJob (matmul.rs:995-1005). has_qx selects the Q8 integer arm. */
typedef struct {
  uint32_t dtype;
  const uint8_t* w;
  size_t n_in, n_out;
  const float* x;
  int has_qx;
  bbo_q8 qx;
} bbo_job;

/* One MoE layer's weights, as Model::moe_ffn reads them (model.rs:473-481). */
typedef struct {
  uint32_t router_dtype;        /* F32 in the real model          */
  const uint8_t* router;        /* [n_experts rows x hidden]      */
  const float* exp_probs_b;     /* [n_experts]                    */
  uint32_t gate_dtype, up_dtype, down_dtype;
  const uint8_t* gate_exps;     /* stacked [hidden, moe_ff, E]    */
  const uint8_t* up_exps;
  const uint8_t* down_exps;     /* stacked [moe_ff, hidden, E]    */
  int hidden, moe_ff, n_experts, n_used;
} bbo_moe;

/* Optional routing trace; any pointer may be NULL. */
typedef struct {
  float* logits;      /* [T*E] raw router logits                        */
  int32_t* sel;       /* [T*k] selected experts, selection order        */
  float* w;           /* [T*k] renormalised weights                     */
  int32_t* counts;    /* [E]                                             */
  int32_t* offsets;   /* [E+1]                                           */
  int32_t* perm;      /* [T*k] entry t*k+slot listed in group order      */
  int32_t* ties;      /* [1]   equal keys among the first k+1 sorted     */
  float* margin;      /* [T]   key[k-1] - key[k] (selection margin)      */
} bbo_trace;

/* Dense SwiGLU layer (model.rs:459-469). */
typedef struct {
  uint32_t gate_dtype, up_dtype, down_dtype;
  const uint8_t* gate; const uint8_t* up; const uint8_t* down;
  int hidden, ff;
} bbo_dense;

/* Gated short-conv operator weights (model.rs:399-427): in_proj [hidden, 3·hidden], conv filter
 * f32[hidden·l_cache] (tap-contiguous), out_proj [hidden, hidden]. */
typedef struct {
  int hidden, l_cache;
  uint32_t in_dtype, out_dtype;
  const uint8_t* in_proj;
  const uint8_t* out_proj;
  const float* conv_w;
} bbo_conv_op;

/* GQA attention operator weights (model.rs:430-456): q [hidden, n_heads·head_dim], k/v [hidden,
 * n_kv·head_dim], o [n_heads·head_dim, hidden]; q/k norm gains f32[head_dim]. */
typedef struct {
  int hidden, n_heads, n_kv_heads, head_dim;
  uint32_t q_dtype, k_dtype, v_dtype, o_dtype;
  const uint8_t *q, *k, *v, *o;
  const float *q_norm, *k_norm;
  float eps, freq_base;
} bbo_attn_op;

/* One FFN-path layer of the config-5 stack: rmsnorm gain + dense or MoE FFN. */
typedef struct {
  const float* ffn_norm;   /* [hidden] */
  int is_moe;
  bbo_dense dense;
  bbo_moe moe;
} bbo_layer;

void bbo_set_threads(int n);
int bbo_get_threads(void);

float bbo_f16_to_f32(uint16_t h);
void bbo_get_scale_min_k4(int j, const uint8_t* scales, uint8_t* sc, uint8_t* m);
int bbo_dequantize(uint32_t dtype, const uint8_t* data, size_t n_elements, float* out);

void bbo_quantize_q8(const float* x, size_t n, bbo_q8 out);
float bbo_dot(const float* a, const float* b, size_t n);
float bbo_dot_q4k_block_q8(const uint8_t* block, const int8_t* qx, float sx, const int32_t* sums);
float bbo_dot_q6k_block_q8(const uint8_t* block, const int8_t* qx, float sx);
int32_t bbo_q4k_block_sd(const uint8_t* block, const int8_t* qx);
int32_t bbo_q6k_block_idot(const uint8_t* block, const int8_t* qx);
int32_t bbo_q6k_block_idot_buffered(const uint8_t* block, const int8_t* qx);
float bbo_fused_row_dot(uint32_t dtype, const uint8_t* row, const float* x, size_t n_in);

int bbo_matvec(uint32_t dtype, const uint8_t* w, size_t n_in, size_t n_out, const float* x, float* y);
int bbo_matmul(uint32_t dtype, const uint8_t* w, size_t n_in, size_t n_out, const float* x,
               size_t n_tokens, float* y);
int bbo_matvec_fused_batch(const bbo_job* jobs, size_t n_jobs, float* out);

float bbo_sigmoid(float x);
float bbo_silu(float x);
void bbo_swiglu(const float* gate, const float* up, float* out, size_t n);
void bbo_add_scaled(float* out, const float* b, float s, size_t n);
void bbo_add_assign(float* a, const float* b, size_t n);
void bbo_rmsnorm(const float* x, const float* gain, float eps, size_t n, float* out);

/* Routing robustness (test infrastructure): the router dot under other plausible evaluation
 * orders of matmul.rs:36-66 (variant 0 = bbo_dot; see dot_variant), and model.rs:485-495's
 * gating of T tokens from given logits. */
float bbo_dot_variant(const float* a, const float* b, size_t n, int variant);
void bbo_router_logits_variant(const float* W, const float* x, size_t T, int H, int E, int variant, float* logits);
void bbo_gate(const float* logits, const float* bias, size_t T, int E, int k, int32_t* sel, float* w, int32_t* ties,
              float* margin);
int bbo_moe_ffn(const bbo_moe* m, const float* x, float* out, bbo_trace* trace);
int bbo_moe_ffn_batch(const bbo_moe* m, const float* x, size_t t, float* out, bbo_trace* trace);
int bbo_dense_ffn(const bbo_dense* d, const float* x, size_t t, float* out);
int bbo_ffn_stack(const bbo_layer* layers, size_t n_layers, const float* x, size_t t, float eps,
                  float* h_out);

/* Operators of the decoder layer: conv.rs:18-39 / :48-68, softmax.rs:9-22, attention.rs:17-55,
 * rope.rs:17-30, model.rs:692-701 (per-head norm + RoPE), model.rs:399-427 / :190-216 (gated
 * short conv, one token / a batch), model.rs:430-456 / :222-259 (GQA attention). */
void bbo_conv_step(const float* state, const float* bx, const float* w, size_t C, size_t L, float* out);
void bbo_conv_prefill(float* state, const float* bx, const float* w, size_t C, size_t L, size_t n, float* out);
void bbo_softmax(float* x, size_t n);
void bbo_attention_decode(const float* q, const float* k, const float* v, size_t n_ctx, size_t n_heads, size_t n_kv,
                          size_t hd, float* out);
void bbo_rope_neox(float* x, size_t d, size_t pos, float freq_base);
void bbo_norm_rope_heads(float* buf, size_t n_heads, size_t hd, const float* gain, float eps, size_t pos,
                         float freq_base);
int bbo_conv_forward(const bbo_conv_op* op, float* state, const float* x, size_t t, float* out);
int bbo_attn_forward(const bbo_attn_op* op, float* k_cache, float* v_cache, size_t cap, size_t* n_cached, size_t pos0,
                const float* x, size_t t, float* out);

#ifdef __cplusplus
}
#endif
#endif
