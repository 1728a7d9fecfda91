/*
 * bebelm_moe.h — C ABI of the MI355X (gfx950) MoE FFN library, libbebelm_moe.so.
 *
 * This is the drop-in boundary for the reference's (maximecb/bebelm 0.3.6, Rust) sparse-MoE
 * FFN path. The reference has no FFI of its own; each entry point below names the Rust
 * function or signature it replaces (paths relative to the reference's src/). A Rust caller
 * binds these with `extern "C"` declarations in an `unsafe` FFI module.
 *
 * Conventions
 *   - Every entry point returns int: 0 (BB_OK) on success, a BB_ERR_* code otherwise, with a
 *     message in bb_last_error() (thread-local). No C++ exception or abort crosses the ABI;
 *     where the reference panics on a shape/dtype violation (matmul.rs:851-857, :909-918,
 *     :1023-1033) this library returns BB_ERR_ARG / BB_ERR_SHAPE / BB_ERR_DTYPE instead.
 *   - Dtype codes are ggml's (tensor.rs:41-63): F32=0, F16=1, Q4_K=12, Q6_K=14.
 *   - Weights are uploaded once (bb_tensor_upload) in their native GGUF block layout (Q4_K:
 *     144-byte blocks, Q6_K: 210-byte blocks) and are immutable afterwards; a tensor may be
 *     shared by any number of layers.
 *   - Activation pointers are host memory when `loc` is BB_LOC_HOST (the call copies in,
 *     computes and copies out before returning) or device memory of the context's GPU when
 *     `loc` is BB_LOC_DEVICE (the call only enqueues work on the context's stream; device
 *     pointers must be 16-byte aligned).
 *   - A context owns one HIP stream (default priority) and one workspace; calls on one context
 *     must not overlap. Use one context per calling thread.
 *   - Results are bit-identical to the reference CPU path on the same inputs (integer dots
 *     exact, f32 epilogues in the reference's order), except rmsnorm's f64 sum order (see
 *     bb_rmsnorm).
 */
#ifndef BEBELM_MOE_H
#define BEBELM_MOE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum bb_status {
  BB_OK = 0,
  BB_ERR_ARG = 1,    /* null pointer, bad flag, misaligned device pointer            */
  BB_ERR_DTYPE = 2,  /* dtype not supported on this path                             */
  BB_ERR_SHAPE = 3,  /* sizes inconsistent (byte_size mismatch, n_in % block != 0)   */
  BB_ERR_HIP = 4,    /* a HIP runtime call failed                                     */
  BB_ERR_OOM = 5,    /* device allocation failed                                      */
  BB_ERR_RANGE = 6,  /* size beyond what this build supports                          */
  BB_ERR_FORMAT = 7, /* malformed GGUF, or metadata / tensor table not what is expected */
  BB_ERR_IO = 8,     /* a file could not be opened or mapped                           */
  BB_ERR_MISSING = 9 /* metadata key or tensor absent, or of another value type        */
};

enum bb_dtype { BB_F32 = 0, BB_F16 = 1, BB_Q4_K = 12, BB_Q6_K = 14 };
enum bb_loc { BB_LOC_HOST = 0, BB_LOC_DEVICE = 1 };

typedef struct bb_ctx bb_ctx;
typedef struct bb_tensor bb_tensor;
typedef struct bb_moe bb_moe;
typedef struct bb_dense bb_dense;
typedef struct bb_stack bb_stack;
typedef struct bb_conv_op bb_conv_op;
typedef struct bb_attn_op bb_attn_op;
typedef struct bb_kv_cache bb_kv_cache;
typedef struct bb_model bb_model;
typedef struct bb_cache bb_cache;
typedef struct bb_gguf bb_gguf;

/* Message for the last failed call on this thread ("" if none). */
const char* bb_last_error(void);
/* Library version string. */
const char* bb_version(void);

/* ---- context ---------------------------------------------------------------------------- */
/* New: there is no device context in the reference (one process, rayon pool, main.rs:155-165). */
int bb_ctx_create(int device, bb_ctx** out);
int bb_ctx_destroy(bb_ctx* ctx);
/* Run subsequent work on a caller-owned hipStream_t (NULL restores the context's own stream). */
int bb_ctx_set_stream(bb_ctx* ctx, void* hip_stream);
int bb_ctx_get_stream(bb_ctx* ctx, void** hip_stream);
int bb_ctx_synchronize(bb_ctx* ctx);
/* Per-kernel timing with HIP events around every launch (off by default). */
int bb_ctx_profile(bb_ctx* ctx, int enable);
/* Accumulated device time of kernel `idx` (0 <= idx < bb_kernel_count()) since the last reset. */
int bb_kernel_count(void);
int bb_ctx_kernel_stats(bb_ctx* ctx, int idx, const char** name, double* total_ms, int64_t* launches);
int bb_ctx_reset_stats(bb_ctx* ctx);
/* New (no counterpart in the reference, which has one CPU path): MoE calls with T*k >=
 * min_entries route all tokens, group the entries by expert and run the grouped-GEMM kernels;
 * smaller calls take the per-expert GEMV kernels. Both give the reference's bits. Default 64. */
int bb_ctx_set_batched_min_entries(bb_ctx* ctx, size_t min_entries);

/* ---- weights ------------------------------------------------------------------------------ */
/* Replaces the zero-copy `GgufFile::tensor_data` view (gguf.rs:191-193) with a one-time copy
 * into HBM, native block layout kept. `dims` are GGUF dims ([in, out] or [in, out, n_expert]);
 * nbytes must equal GgmlType::byte_size(prod(dims)) (tensor.rs:99-105). */
int bb_tensor_upload(bb_ctx* ctx, uint32_t dtype, const void* bytes, size_t nbytes, const uint64_t* dims,
                     int ndims, bb_tensor** out);
int bb_tensor_free(bb_tensor* t);
int bb_tensor_device_ptr(const bb_tensor* t, void** dev);

/* ---- kernel-level mirrors of src/kernels ----------------------------------------------- */
/* quantize_q8(x: &[f32]) -> Q8Vec (kernels/matmul.rs:141). q[n], scales[n/256], sums[n/32]
 * live where `loc` says; n % 256 == 0. */
int bb_quantize_q8(bb_ctx* ctx, const float* x, size_t n, int8_t* q, float* scales, int32_t* sums, int loc);

/* matvec(dtype, w, n_in, n_out, x, y) (kernels/matmul.rs:850). The weight matrix is the
 * n_out rows starting `byte_off` bytes into tensor `w` (an expert slice is e*expert_bytes,
 * model.rs:612-615). */
int bb_matvec(bb_ctx* ctx, uint32_t dtype, const bb_tensor* w, size_t byte_off, size_t n_in, size_t n_out,
              const float* x, float* y, int loc);

/* matmul(dtype, w, n_in, n_out, x, n_tokens, y) with token-major x and y (kernels/matmul.rs:908). */
int bb_matmul(bb_ctx* ctx, uint32_t dtype, const bb_tensor* w, size_t byte_off, size_t n_in, size_t n_out,
              const float* x, size_t n_tokens, float* y, int loc);

/* FusedJob (kernels/matmul.rs:995-1005). With qx_q set (`qx: Some`, the arm every MoE job
 * takes, model.rs:507, :512, :544) the rows take the Q8-activation integer dot; with qx_q NULL
 * (`qx: None`) they take the f32 fused dot over x (fused_row_dot, matmul.rs:777-785, :1045). */
typedef struct {
  uint32_t dtype;           /* Q4_K or Q6_K                         */
  const bb_tensor* w;
  size_t byte_off;          /* first row of this job inside w       */
  size_t n_in, n_out;
  const int8_t* qx_q;       /* Q8 of this job's x (bb_quantize_q8), or NULL */
  const float* qx_scales;
  const int32_t* qx_sums;
  const float* x;           /* f32[n_in], read when qx_q is NULL    */
} bb_fused_job;
/* matvec_fused_batch(jobs, out) (kernels/matmul.rs:1015): out = Σ n_out values, jobs in order. */
int bb_matvec_fused_batch(bb_ctx* ctx, const bb_fused_job* jobs, size_t n_jobs, float* out, int loc);

/* swiglu(gate, up, out) (kernels/activation.rs:16) and sigmoid_slice(x) (:25). */
int bb_swiglu(bb_ctx* ctx, const float* gate, const float* up, float* out, size_t n, int loc);
int bb_sigmoid_slice(bb_ctx* ctx, float* x, size_t n, int loc);
/* add_scaled(out, b, s) (kernels/elementwise.rs:12) and add_assign(a, b) (:4). */
int bb_add_scaled(bb_ctx* ctx, float* out, const float* b, float s, size_t n, int loc);
int bb_add_assign(bb_ctx* ctx, float* a, const float* b, size_t n, int loc);
/* rmsnorm(x, gain, eps, out) (kernels/rmsnorm.rs:10) over n_vec rows of n. The f64 sum of
 * squares is a tree, not the reference's left-to-right sum; the f32 result agrees unless the
 * two f64 sums fall on opposite sides of an f32 rounding boundary. */
int bb_rmsnorm(bb_ctx* ctx, const float* x, const float* gain, float eps, size_t n, size_t n_vec, float* out,
               int loc);

/* Model::logits_from_hidden(h) (model.rs:380-388): rmsnorm(h, gain, eps) (as bb_rmsnorm), then
 * matvec(token_embd dtype, token_embd, hidden, vocab, normed, logits). token_embd is [hidden,
 * vocab] (any dtype bb_matvec takes); h and gain f32[hidden], logits f32[vocab]. */
int bb_logits_from_hidden(bb_ctx* ctx, const bb_tensor* tok_embd, const float* gain, float eps, const float* h,
                          float* logits, int loc);

/* ---- MoE layer (model.rs:473-555 decode, model.rs:286-371 batched) ----------------------- */
/* Tensors as Model::moe_ffn resolves them (model.rs:474-478): router `ffn_gate_inp` F32
 * [hidden, E]; `exp_probs_b` f32[E] (host); stacked experts gate/up [hidden, ff, E] and
 * down [ff, hidden, E] in Q4_K or Q6_K. Requires E <= 32, k <= 8, hidden and ff multiples
 * of 256. The layer keeps its own device copies of the router and experts, regrouped for
 * coalesced loads (same bytes, other order); the tensors may be freed after this call. */
int bb_moe_create(bb_ctx* ctx, const bb_tensor* router, const float* exp_probs_b, const bb_tensor* gate_exps,
                  const bb_tensor* up_exps, const bb_tensor* down_exps, int n_used, bb_moe** out);
int bb_moe_destroy(bb_moe* moe);

/* Routing trace (host arrays; any may be NULL), for bit-exact checks of the route. */
typedef struct {
  float* logits;     /* [T*E] router logits                                  */
  int32_t* sel;      /* [T*k] experts in selection order                     */
  float* w;          /* [T*k] renormalised weights                           */
  int32_t* counts;   /* [E]                                                  */
  int32_t* offsets;  /* [E+1] exclusive prefix sum of counts                 */
  int32_t* perm;     /* [T*k] entry t*k+slot, grouped by expert, stable      */
  int32_t* ties;     /* [1] exactly equal keys among the first k+1 sorted   */
  float* margin;     /* [T] key[k-1] - key[k]                                */
} bb_route_trace;

/* T == 1: Model::moe_ffn(layer, x) -> Vec<f32>. T > 1: Model::moe_ffn_batch(layer, x, t)
 * (token-major x[T*hidden], out[T*hidden]); both bit-identical to the reference. */
int bb_moe_forward(bb_ctx* ctx, bb_moe* moe, const float* x, size_t T, float* out, int loc,
                   bb_route_trace* trace);

/* No counterpart in the reference (its CPU path allocates per call). For callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. bb_moe_forward on device pointers (x, out: f32[T*hidden], 16-byte aligned,
 * on the context's device) with the same kernels and bits, whose workspace is a fixed scratch
 * area of BB_NOALLOC_SCRATCH_BYTES in the library's static device memory (one per GPU, set up
 * by bb_ctx_create and held until the process ends) instead of the context's workspace. It
 * calls no hipMalloc, hipFree or other allocating routine. A call whose workspace exceeds the
 * area returns BB_ERR_RANGE (at hidden = ff = 2048, k = 4: up to 440 tokens). Every call
 * on one GPU shares that GPU's area: calls that overlap on one GPU (other contexts, other
 * streams) race and must be ordered by the caller. No route trace; calls made while per-kernel
 * profiling is on are not timed. */
#define BB_NOALLOC_SCRATCH_BYTES (32u << 20)
int bb_moe_forward_noalloc(bb_ctx* ctx, bb_moe* moe, const float* x, size_t T, float* out);

/* ---- dense FFN and the FFN-path layer stack ---------------------------------------------- */
/* dense_ffn (model.rs:459-469) / dense_ffn_batch (:262-278): gate/up [hidden, ff], down [ff, hidden].
 * Unlike bb_moe_create, the layer reads the three tensors in place: they must outlive it. */
int bb_dense_create(bb_ctx* ctx, const bb_tensor* gate, const bb_tensor* up, const bb_tensor* down, bb_dense** out);
int bb_dense_destroy(bb_dense* d);
int bb_dense_forward(bb_ctx* ctx, bb_dense* d, const float* x, size_t T, float* out, int loc);

/* run_layers (model.rs:105-130) with the operator sub-layer contributing nothing:
 * per layer h += FFN(rmsnorm(h, ffn_norm)). Exactly one of moe / dense is set per layer, created
 * on the same context; the stack keeps copies of the gains but uses the layers in place, so
 * they must outlive it. Hidden sizes up to 2048. */
typedef struct {
  const float* ffn_norm; /* host f32[hidden] */
  bb_moe* moe;
  bb_dense* dense;
} bb_layer_desc;
int bb_stack_create(bb_ctx* ctx, const bb_layer_desc* layers, size_t n_layers, float eps, bb_stack** out);
int bb_stack_destroy(bb_stack* s);
int bb_stack_forward(bb_ctx* ctx, bb_stack* s, const float* x, size_t T, float* h_out, int loc);

/* ---- the decoder layer's operators (model.rs:105-130) --------------------------------------- */
/* Kernel-level mirrors. conv_step(state, bx, weight, channels, l_cache, out) (kernels/conv.rs:18):
 * state f32[(l_cache-1)*channels] (oldest column first), bx and out f32[channels], weight
 * f32[channels*l_cache] tap-contiguous; the last tap multiplies bx. */
int bb_conv_step(bb_ctx* ctx, const float* state, const float* bx, const float* weight, size_t channels, size_t l_cache,
                 float* out, int loc);
/* conv_prefill(state, bx, weight, channels, l_cache, n_tokens, out) (kernels/conv.rs:48): token-major
 * bx and out f32[n_tokens*channels]; state is updated in place to the batch's last l_cache-1
 * columns. l_cache >= 2 (the reference's slice ranges panic below that). */
int bb_conv_prefill(bb_ctx* ctx, float* state, const float* bx, const float* weight, size_t channels, size_t l_cache,
                    size_t n_tokens, float* out, int loc);
/* softmax(x) (kernels/softmax.rs:9) on each of n_vec rows of n, in place. */
int bb_softmax(bb_ctx* ctx, float* x, size_t n, size_t n_vec, int loc);
/* attention_decode(q, k, v, n_ctx, n_heads, n_kv_heads, head_dim, out) (kernels/attention.rs:17):
 * q and out f32[n_heads*head_dim], k and v f32[n_ctx*n_kv_heads*head_dim]; head_dim <= 256. */
int bb_attention_decode(bb_ctx* ctx, const float* q, const float* k, const float* v, size_t n_ctx, size_t n_heads,
                        size_t n_kv_heads, size_t head_dim, float* out, int loc);
/* rope_neox(x, pos, freq_base) (kernels/rope.rs:17) on each of n_vec head vectors of head_dim. */
int bb_rope_neox(bb_ctx* ctx, float* x, size_t head_dim, size_t n_vec, size_t pos, float freq_base, int loc);

/* Gated short-conv operator: Model::conv_step_op (model.rs:399-427) for T == 1 and conv_batch
 * (model.rs:190-216) for T > 1, with the tensors Model resolves: in_proj [hidden, 3*hidden],
 * the conv filter `shortconv.conv.weight` (host f32[hidden*l_cache], copied), out_proj
 * [hidden, hidden] (projection tensors F32, F16, Q4_K or Q6_K; used in place, they must outlive
 * the operator). state is the layer's conv cache f32[(l_cache-1)*hidden] (cache.rs:16-17),
 * updated in place; x and out token-major f32[T*hidden]. */
int bb_conv_op_create(bb_ctx* ctx, const bb_tensor* in_proj, const float* conv_w, size_t l_cache,
                      const bb_tensor* out_proj, bb_conv_op** out);
int bb_conv_op_destroy(bb_conv_op* op);
int bb_conv_op_forward(bb_ctx* ctx, bb_conv_op* op, float* state, const float* x, size_t T, float* out, int loc);

/* One attention layer's key/value history (cache.rs:10-17), resident in device memory:
 * `capacity` positions of kv_dim floats each for k and v. bb_kv_cache_read copies the n cached
 * positions out (k and v f32[n*kv_dim]); bb_kv_cache_evict_front drops the oldest n positions
 * (Cache::evict_front, cache.rs:40-50). */
int bb_kv_cache_create(bb_ctx* ctx, size_t kv_dim, size_t capacity, bb_kv_cache** out);
int bb_kv_cache_destroy(bb_kv_cache* kv);
int bb_kv_cache_length(const bb_kv_cache* kv, size_t* n);
int bb_kv_cache_read(bb_ctx* ctx, const bb_kv_cache* kv, float* k, float* v, int loc);
int bb_kv_cache_evict_front(bb_ctx* ctx, bb_kv_cache* kv, size_t n);

/* GQA attention operator: Model::attn_step (model.rs:430-456) for T == 1 and attn_batch
 * (model.rs:222-259) for T > 1: q [hidden, n_heads*head_dim], k and v [hidden, n_kv_heads*head_dim],
 * o [n_heads*head_dim, hidden] (used in place), q/k norm gains host f32[head_dim] (copied),
 * rmsnorm eps and RoPE base. Token t of the batch sits at position pos0 + t; its key and value
 * are appended to `kv` and it attends over every cached position up to its own. */
int bb_attn_op_create(bb_ctx* ctx, const bb_tensor* q, const bb_tensor* k, const bb_tensor* v, const bb_tensor* o,
                      const float* q_norm, const float* k_norm, size_t n_heads, size_t n_kv_heads, float eps,
                      float freq_base, bb_attn_op** out);
int bb_attn_op_destroy(bb_attn_op* op);
int bb_attn_op_forward(bb_ctx* ctx, bb_attn_op* op, bb_kv_cache* kv, size_t pos0, const float* x, size_t T, float* out,
                       int loc);

/* ---- the decoder (Model, model.rs:25-31; Cache, cache.rs:10-19) ------------------------------- */
/* One decoder layer (run_layers, model.rs:114-127): attn_norm and ffn_norm gains (host
 * f32[hidden], copied), exactly one operator (conv or attn) and exactly one FFN (moe or dense),
 * all created on the model's context and used in place (they must outlive the model). */
typedef struct {
  const float* attn_norm;
  const float* ffn_norm;
  bb_conv_op* conv;
  bb_attn_op* attn;
  bb_moe* moe;
  bb_dense* dense;
} bb_decoder_layer;
/* token_embd [hidden, vocab] (embedding rows and the tied logits head), final norm gain host
 * f32[hidden] (`token_embd_norm`), rmsnorm eps. The model holds weights only (Model,
 * model.rs:25-31): the decode-time state is a bb_cache, so one loaded model serves any number
 * of caches (agent.rs:85-86: several agents on one model). Calls on one model are ordered on its
 * context's stream (the model keeps per-call scratch buffers). */
int bb_model_create(bb_ctx* ctx, const bb_tensor* token_embd, const float* final_norm, const bb_decoder_layer* layers,
                    size_t n_layers, float eps, bb_model** out);
/* Destroy the model's caches first. */
int bb_model_destroy(bb_model* m);

/* Cache::new (cache.rs:21-28) for the layers of `m`: a zeroed conv state per conv layer, an
 * empty device KV history per attention layer with room for kv_capacity positions (grown on
 * demand, as the reference's Vec histories grow), position 0. The cache is used with `m` only
 * and must be destroyed before it. */
int bb_cache_create(bb_ctx* ctx, const bb_model* m, size_t kv_capacity, bb_cache** out);
/* Cache: Clone (cache.rs:9; Agent: Clone, agent.rs:87-91): an independent copy of the conv
 * states, KV histories and position, e.g. to fork a prefilled prompt into several continuations. */
int bb_cache_clone(bb_ctx* ctx, const bb_cache* src, bb_cache** out);
int bb_cache_destroy(bb_cache* cache);
/* Cache::new again (Agent::clear, agent.rs): zero conv states, empty KV histories, position 0. */
int bb_cache_reset(bb_ctx* ctx, bb_cache* cache);
/* cache.pos (the next token's position) and Cache::kv_len (cache.rs:32-35). */
int bb_cache_position(const bb_cache* cache, size_t* pos);
int bb_cache_kv_length(const bb_cache* cache, size_t* n);
/* Cache::evict_front (cache.rs:40-50) on every attention layer: a layer holding fewer than n
 * positions is left as it is; pos is unchanged. */
int bb_cache_evict_front(bb_ctx* ctx, bb_cache* cache, size_t n);
/* Copies layer `layer`'s state out: its conv state (conv layers, f32[(l_cache-1)*hidden]) or its
 * n cached keys and values (attention layers, f32[n*kv_dim] each); NULL outputs are skipped. */
int bb_cache_layer_state(bb_ctx* ctx, const bb_cache* cache, size_t layer, float* conv_state, float* k, float* v,
                         int loc);

/* Model::run_layers(&self, token, &mut Cache) (model.rs:105-130) for T == 1 and
 * run_layers_batch(&self, tokens, &mut Cache) (model.rs:146-181) for T > 1: host token ids[T]
 * at positions cache.pos.., the cache updated, final hidden states into h_out f32[T*hidden]
 * (may be NULL). */
int bb_model_run_layers(bb_ctx* ctx, bb_model* m, const uint32_t* tokens, size_t T, bb_cache* cache, float* h_out,
                        int loc);
/* Model::forward_step(&self, token, &mut Cache) (model.rs:97-103): run_layers for one token,
 * then logits_from_hidden into logits f32[vocab]. */
int bb_model_forward_step(bb_ctx* ctx, bb_model* m, uint32_t token, bb_cache* cache, float* logits, int loc);
/* Agent::absorb(model, cache, tokens, max_context) (agent.rs:454-465): when the whole batch fits
 * max_context, run_layers_batch over chunks of 512 tokens (agent.rs:31); otherwise token by
 * token, sliding the KV window down to max_context after each (Agent::trim_context,
 * agent.rs:471-476). Token ids are checked before anything runs. */
int bb_model_absorb(bb_ctx* ctx, bb_model* m, bb_cache* cache, const uint32_t* tokens, size_t n, size_t max_context);

/* ---- GGUF files (gguf.rs, config.rs:51-89, model.rs:36-50, :572-584, :619-660) ---------------- */
/* GgufFile::open (gguf.rs:171-177): maps the file read-only and parses the header, the metadata
 * and the tensor table. Errors as gguf.rs:22-55 (bad magic, version other than 2 or 3, a read
 * past the end, an unknown value type, a string that is not UTF-8, a tensor of an unmodelled
 * ggml type or whose data falls outside the file): BB_ERR_FORMAT with the reference's message;
 * an open or map failure: BB_ERR_IO. */
int bb_gguf_open(const char* path, bb_gguf** out);
/* GgufFile::from_bytes (gguf.rs:181-184): the same parse over a copy of n in-memory bytes. */
int bb_gguf_open_bytes(const void* bytes, size_t n, bb_gguf** out);
int bb_gguf_close(bb_gguf* g);
/* version, alignment, data_offset (gguf.rs:152-160) and the table sizes. Any pointer may be NULL. */
int bb_gguf_header(const bb_gguf* g, uint32_t* version, uint64_t* alignment, uint64_t* data_offset,
                   size_t* n_tensors, size_t* n_metadata);

/* TensorInfo (gguf.rs:123-140); name and dims point into the bb_gguf and live as long as it. */
typedef struct {
  const char* name;
  uint32_t n_dims;
  const uint64_t* dims;       /* GGUF order, fastest-varying first */
  uint32_t ggml_type;
  uint64_t offset;            /* relative to the tensor-data section */
  uint64_t data_start;        /* absolute file offset */
  uint64_t data_len;          /* GgmlType::byte_size of the element count (tensor.rs:99-105) */
} bb_gguf_tensor_info;
int bb_gguf_tensor(const bb_gguf* g, size_t index, bb_gguf_tensor_info* info);
/* Model::tensor's name lookup (model.rs:80-82): BB_ERR_MISSING when absent. */
int bb_gguf_find_tensor(const bb_gguf* g, const char* name, size_t* index);
/* tensor_data (gguf.rs:191-193): zero-copy view of the tensor's bytes in the mapping. */
int bb_gguf_tensor_data(const bb_gguf* g, size_t index, const void** data, size_t* nbytes);

/* Metadata (gguf.rs:195-266). Every accessor returns BB_ERR_MISSING when the key is absent or
 * its value has another type, as the reference's Option-returning getters give None.
 * bb_gguf_meta_key enumerates the keys in file order (a key repeated in the file keeps the
 * last value, as the reference's HashMap insert does). bb_gguf_meta_type gives the value type
 * (gguf.rs:61-75 codes), and for arrays the element type and length (else 0 and 0). */
int bb_gguf_meta_key(const bb_gguf* g, size_t index, const char** key);
int bb_gguf_meta_type(const bb_gguf* g, const char* key, uint32_t* value_type, uint32_t* elem_type, size_t* n_items);
/* get_u32 (gguf.rs:200-212): any integer type, converted as Rust's `as u32`. */
int bb_gguf_get_u32(const bb_gguf* g, const char* key, uint32_t* value);
/* get_f32 (gguf.rs:250-256): F32, or F64 rounded to f32. */
int bb_gguf_get_f32(const bb_gguf* g, const char* key, float* value);
/* get_str (gguf.rs:258-263): a pointer into the bb_gguf (not NUL-terminated) and its length. */
int bb_gguf_get_str(const bb_gguf* g, const char* key, const char** str, size_t* len);
/* get_u32_array (gguf.rs:215-233): *n_items = the array length; up to `cap` values written.
 * BB_ERR_MISSING when an item is not an integer. */
int bb_gguf_get_u32_array(const bb_gguf* g, const char* key, uint32_t* out, size_t cap, size_t* n_items);
/* get_str_array (gguf.rs:236-248), one item at a time: item `index` of a string array. */
int bb_gguf_get_str_item(const bb_gguf* g, const char* key, size_t index, const char** str, size_t* len);

/* config::validate (config.rs:51-89): the file is LFM2.5-8B-A1B (architecture "lfm2moe", its
 * sizes, RoPE base, rmsnorm eps and conv/attention schedule). BB_ERR_FORMAT with the
 * reference's message on the first mismatch, BB_ERR_MISSING for an absent key. */
int bb_gguf_validate(const bb_gguf* g);
/* Model::check_tensors (model.rs:572-584) against expected_tensors (model.rs:619-660), the list
 * derived from the file's own lfm2moe.* sizes and schedule (equal to the reference's hardcoded
 * list for a file that passes bb_gguf_validate). *n_expected (may be NULL) = the list's length. */
int bb_gguf_check_tensors(const bb_gguf* g, size_t* n_expected);
/* One tensor into HBM (what bb_tensor_upload does with tensor_data's bytes and the table's
 * dims and dtype). */
int bb_gguf_upload(bb_ctx* ctx, const bb_gguf* g, size_t index, bb_tensor** out);
/* Model::load (model.rs:36-50) after the open: check_tensors, then every tensor the forward
 * pass reads uploaded to HBM, the operators, FFNs and the decoder built from them with the
 * file's sizes (hidden, heads and kv heads per layer, expert counts, conv length, RoPE base,
 * eps; the small F32 tensors read as precompute_f32 reads them, :54-67). Caches for it come
 * from bb_cache_create. The returned model owns all of it: bb_model_destroy frees it. The
 * bb_gguf may be closed once this returns. Call bb_gguf_validate first to also pin the
 * LFM2.5-8B-A1B constants, as Model::load does. */
int bb_model_load(bb_ctx* ctx, const bb_gguf* g, bb_model** out);

#ifdef __cplusplus
}
#endif
#endif
