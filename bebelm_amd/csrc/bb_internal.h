// bb_internal.h — launcher declarations shared by the kernels TU and the C-ABI TU.
#ifndef BB_INTERNAL_H
#define BB_INTERNAL_H
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/bebelm_moe.h"

namespace bb {

// Sets the calling thread's bb_last_error message (for entry points outside bb_api.hip).
void set_last_error(const std::string& msg);

// What bb_model_load created for a model: bb_model_destroy frees these after the model itself,
// operators and FFNs before the tensors they read.
struct ModelOwned {
  std::vector<bb_conv_op*> conv;
  std::vector<bb_attn_op*> attn;
  std::vector<bb_moe*> moe;
  std::vector<bb_dense*> dense;
  std::vector<bb_tensor*> tensors;
};
void free_owned(ModelOwned& o);
void model_adopt(bb_model* m, ModelOwned&& o);

// Profiling: when set, kernels are launched with hipExtLaunchKernelGGL, which has the kernel's
// own dispatch stamp the events (exact start and end, no queue gaps in between). A launcher
// that runs several kernels has the first stamp the start and each one the stop, so the pair
// spans all of them.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
LaunchEvents& launch_events();  // per host thread

#define BB_LAUNCH(kernel, grid, block, shmem, stream, ...)                                                  \
  do {                                                                                                     \
    ::bb::LaunchEvents& bb_ev_ = ::bb::launch_events();                                                    \
    if (bb_ev_.stop) {                                                                                     \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, bb_ev_.start, bb_ev_.stop, 0, __VA_ARGS__); \
      bb_ev_.start = nullptr;                                                                              \
    } else {                                                                                               \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                                 \
    }                                                                                                      \
  } while (0)

// Device-side routing state for one forward call. All arrays live in the context workspace.
struct RouteBufs {
  float* logits;      // [T*E]
  int32_t* sel;       // [T*K]
  float* wts;         // [T*K]
  int32_t* counts;    // [E]
  int32_t* offsets;   // [E+1]
  int32_t* perm;      // [T*K]  group position -> entry t*K+k
  int32_t* hit;       // [E+1]  hit[0] = number of experts with members, hit[1..] ascending ids
  int32_t* ties;      // [T]  exactly equal keys among the first k+1 of each token
  float* margin;      // [T]
};

struct Q8Bufs {
  int8_t* q;
  float* scales;
  int32_t* sums;
};

// One launch = one kernel; names are used for the per-kernel profile table.
enum KernelId : int {
  K_ROUTE = 0,
  K_GATEUP,
  K_DOWN,
  K_QUANT,
  K_ROWS_Q8,
  K_ROWS_F32,
  K_ELEMWISE,
  K_RMSNORM,
  K_ROUTE_LARGE,
  K_DISPATCH,
  K_GEMM_GATEUP,
  K_GEMM_DOWN,
  K_COMBINE,
  K_RESIDUAL_NORM,
  K_RESIDUAL_ROUTE,
  K_CONV,
  K_CONV_STATE,
  K_NORM_ROPE,
  K_ATTN_SCORES,
  K_ATTN_PV,
  K_SOFTMAX,
  K_EMBED,
  K_COUNT
};
const char* kernel_name(int id);

// Q8 activation record used by the decode GEMV kernels: quants, per-256 scales and the int16
// sum pairs consumed by v_dot2 (12 dwords per 256-block; see bb_rowlane.h).
struct XQBufs {
  int8_t* q;
  float* sx;
  uint32_t* pairs;
  uint16_t* ms = nullptr;  // per 256-block: the split per-32 sums (min_split_record), when set
};

// Decode / small-batch path limits: T*k (token, slot) entries per call; members of one expert
// staged in LDS at a time (MCH); largest hidden / ff (8 super-blocks, one per wave).
constexpr int MAX_ENTRIES = 1024;
constexpr int MCH = 8;
constexpr int GU_H_MAX = 2048;
constexpr int DN_F_MAX = 2048;
// Target number of blocks of one decode GEMV launch (one 8-wave block per CU at the VGPR
// budget of the double-buffered rows); each block walks enough row tiles to cover the work.
constexpr int GEMV_BLOCKS = 256;

// Tile-packed expert rows (built once per layer by launch_pack_rows): the 64 rows of a tile and
// one 256-weight super-block form a tile-block of NC chunks of 64 x 16 bytes, chunk c holding
// bytes 16c..16c+15 of the block of each row (row r of the tile at lane r), followed for Q6_K
// by the 64 rows' trailing 2 bytes (the f16 d). One 16-byte load per lane of a wave then reads
// 1 KB of contiguous memory. Layout: [expert][tile][block][chunk][lane][16 B] (+ tail).
// Gate/up tiles interleave the two tensors: lanes 0-31 gate rows 32t.., lanes 32-63 up rows.
constexpr int TILE_ROWS = 64;
__host__ __device__ constexpr int pack_chunks(int dt) { return dt == 12 ? 9 : 13; }
__host__ __device__ constexpr int pack_tail(int dt) { return dt == 12 ? 0 : 2; }
__host__ __device__ constexpr size_t pack_tile_block_bytes(int dt) {
  return (size_t)pack_chunks(dt) * 1024 + (size_t)pack_tail(dt) * TILE_ROWS;
}

// Packs n_exp experts of raw GGUF rows (a, and b for the interleaved gate/up form; b null for
// plain tiles of 64 rows of a) into dst. stride_a/b: raw bytes per expert; rows_a: rows per
// expert of a; nb: super-blocks per row.
hipError_t launch_pack_rows(hipStream_t s, int dtype, const uint8_t* a, const uint8_t* b, size_t stride_a,
                            size_t stride_b, int rows_a, int nb, int n_exp, uint8_t* dst);

// tpb tokens per block (the router is read once per block); xq.pairs may be null.
hipError_t launch_route(hipStream_t s, const float* router, const float* bias, const float* x, int T, int H, int E,
                        int K, int tpb, XQBufs xq, RouteBufs rb);

hipError_t launch_router_chain_major(hipStream_t s, const float* W, int H, int E, float* Wc);

// Gate/up GEMV of at most ROUTE_IN_GATEUP_MAX_T tokens that routes the tokens itself (route
// of launch_route, rb written by the first block): no launch_route before it.
constexpr int ROUTE_IN_GATEUP_MAX_T = 4;
hipError_t launch_route_gateup(hipStream_t s, int dtype, const uint8_t* gu, size_t stride_gu, int T, int H, int F,
                               int E, int K, int max_hit, int batch_mode, int publish, const RouteBufs& rb,
                               const float* router, const float* bias, const float* x, float* act);
// The same gate/up GEMV with the tokens gated in every block from router logits computed before
// (launch_residual_norm_route) and their XQ records in xq: no launch_route before it.
hipError_t launch_gate_gateup(hipStream_t s, int dtype, const uint8_t* gu, size_t stride_gu, int T, int H, int F,
                              int E, int K, int max_hit, int batch_mode, int publish, const RouteBufs& rb,
                              const float* logits, const float* bias, XQBufs xq, float* act);
// The layer boundary of a stack of at most ROUTE_IN_GATEUP_MAX_T tokens before an MoE layer:
// h_out = h_in + the combine of slots (or + ffn when slots is null), normed = its rmsnorm with
// gain, and the next layer's router logits (router in k_route's chain-major layout, E experts)
// and the XQ records (with pairs) of normed. h_out must not alias h_in.
hipError_t launch_residual_norm_route(hipStream_t s, const float* h_in, float* h_out, const float* slots,
                                      const float* wts, int K, const float* ffn, const float* gain, float eps, int n,
                                      int T, float* normed, const float* router, int E, float* logits, XQBufs xq);

// gu / dn: tile-packed gate+up and down tensors; stride_*: packed bytes per expert.
hipError_t launch_gateup(hipStream_t s, int dtype, const uint8_t* gu, size_t stride_gu, int T, int H, int F, int E,
                         int K, int max_hit, int batch_mode, int publish, const RouteBufs& rb, XQBufs xq, float* act);

hipError_t launch_down(hipStream_t s, int dtype, const uint8_t* dn, size_t stride_dn, int T, int H, int F, int K,
                       int max_hit, int batch_mode, const RouteBufs& rb, const float* act, float* slots);
// Down GEMV and combine of one token (K <= 4, F/256 <= 8): out[H] = Σ_k wts[k] · (down row of the
// expert of slot k · Q8(act row k)), no slot rows written.
hipError_t launch_down_combine1(hipStream_t s, int dtype, const uint8_t* dn, size_t stride_dn, int H, int F, int K,
                                const RouteBufs& rb, const float* act, float* out);

// ---- batched (prefill) path ----------------------------------------------------------------------
// Largest T*k of one call on this path (the dispatch keeps per-64-entry counts in LDS).
constexpr int PF_MAX_ENTRIES = 32768;

// counts/offsets/perm/hit of rb from sel (stable grouping, model.rs:316-322).
hipError_t launch_dispatch(hipStream_t s, int n_ent, int E, const RouteBufs& rb);
// Member tile of the grouped GEMMs in units of 16 members; 1 means the GEMMs derive the
// grouping from rb.sel themselves and need no dispatch kernel before them.
int gemm_member_tiles(int n_ent, int E);
// Whether launch_gemm_gateup runs the gate/up GEMM of this call as k_gateup16 (decode batches of
// Q4_K experts, the act Q8 written by the kernel: act_q8).
bool gateup16_applies(int dtype, int T, int H, int F, int E, int K, bool act_q8);

// Grouped expert GEMM over the members of each expert (int8 MFMA with exact integer
// sub-dots and the reference's f32 per-block epilogue).
//   gate/up: x = XQ records of the members' tokens, out = act in group order [pos][F].
//   down:    x = Q8 of act in group order, out = slots[entry][H].
struct GemmX {
  const int8_t* q;  // Q8 rows
  const float* sx;  // per-256 scales of the rows
  // per-256 split per-32 sums of the rows (16 halves, min_split_record), or null: then the Q4_K
  // GEMMs form the min term with a third int8 pass instead of one f16 MFMA
  const uint16_t* ms = nullptr;
};
// Q4_K GEMMs whose groups hold 128+ members on average read the min-term records (tiles of 64
// members with the f16 min pass); smaller launches never do, so their callers carve none
constexpr int GEMM_MS_MIN_AVG = 128;
inline bool gemm_reads_ms(int dtype, size_t n_ent, size_t E) {
  return dtype == BB_Q4_K && n_ent >= (size_t)GEMM_MS_MIN_AVG * E;
}
// With aq set, a launch that can also writes the Q8 of the act rows (aq, aq_sx: the
// k_quant_rows output) and sets *quantized; otherwise the caller quantises them.
// act_pad (decode batches whose gate/up runs as k_gateup16 and whose down runs as k_down16:
// gateup16_applies and down16_applies): the Q8 act rows of expert e's member m are row 16e + m of
// aq (E·16 rows) instead of its group position, so the down GEMM copies them without reading the
// selections first.
hipError_t launch_gemm_gateup(hipStream_t s, int dtype, const uint8_t* gu, size_t stride_gu, int T, int H, int F,
                              int E, int K, const RouteBufs& rb, GemmX x, float* act, int8_t* aq = nullptr,
                              float* aq_sx = nullptr, bool* quantized = nullptr, bool act_pad = false);
hipError_t launch_gemm_down(hipStream_t s, int dtype, const uint8_t* dn, size_t stride_dn, int T, int H, int F, int E,
                            int K, const RouteBufs& rb, GemmX x, float* slots, bool act_pad = false);
// Whether launch_gemm_down runs the down GEMM of this call as k_down16 (decode batches of Q4_K
// experts, at most 16 members per expert).
bool down16_applies(int dtype, int T, int H, int F, int E, int K);

// A Q4_K / Q6_K weight matrix in the grouped GEMM's packed tile layout as a single expert: plain
// 64-row tiles (GEMM_DOWN form, n_out % 128 == 0) or gate and up interleaved (GEMM_GATEUP form,
// n_out % 64 == 0). w null: the matrix has no packed form and stays on the row kernels.
struct PackedW {
  uint8_t* w = nullptr;
  size_t stride = 0;  // bytes of the packed matrix
  int dt = 0;
};
// Batches of at least this many tokens run a packed projection on the grouped GEMM (every token
// a member of the one group); smaller ones take the row kernels.
constexpr size_t PROJ_GEMM_MIN_T = 32;
// The route of "every one of T tokens in group 0": counts[0] = T, offsets = {0, T}, perm = 0..T-1.
hipError_t launch_one_group(hipStream_t s, int T, RouteBufs rb);

// Q8 rows (quants and per-256 scales only) of n_rows vectors of n floats.
hipError_t launch_quant_rows(hipStream_t s, const float* x, size_t n_rows, int n, int8_t* q, float* sx,
                             uint16_t* ms = nullptr);

hipError_t launch_combine(hipStream_t s, const float* slots, const float* wts, int T, int H, int K, float* out);

hipError_t launch_quantize(hipStream_t s, const float* x, size_t n_vec, size_t n, Q8Bufs q);

hipError_t launch_rows_q8(hipStream_t s, int dtype, const uint8_t* w, size_t row_bytes, int nb, size_t n_rows,
                          Q8Bufs q, size_t q_stride, size_t n_tok, float* y, size_t y_tok_stride, int neg_zero_start);
// Dense FFN gate/up/swiglu in one pass: y[t][o] = silu(gate row o · x_t) * (up row o · x_t), both
// sums as launch_rows_q8's (gate and up of one dtype and row length, nb <= 64).
hipError_t launch_rows_q8_swiglu(hipStream_t s, int dtype, const uint8_t* gate, const uint8_t* up, size_t row_bytes,
                                 int nb, size_t n_rows, Q8Bufs q, size_t q_stride, size_t n_tok, float* y,
                                 size_t y_tok_stride, int neg_zero_start);

hipError_t launch_rows_f32(hipStream_t s, int dtype, const uint8_t* w, size_t n_in, size_t n_rows, const float* x,
                           size_t n_tok, float* y);
// The f32 fused dot (fused_row_dot) of n_rows Q4_K / Q6_K rows with one f32 vector x.
hipError_t launch_fused_rows_f32(hipStream_t s, int dtype, const uint8_t* w, size_t row_bytes, int nb, size_t n_rows,
                                 const float* x, float* y);

enum ElemOp : int { EW_SWIGLU = 0, EW_SIGMOID, EW_ADD_SCALED, EW_ADD_ASSIGN };
hipError_t launch_elementwise(hipStream_t s, int op, float* out, const float* a, const float* b, float scalar,
                              size_t n);

hipError_t launch_rmsnorm(hipStream_t s, const float* x, const float* gain, float eps, size_t n, size_t n_vec,
                          float* out);
// The same, and the Q8 of each normed row into q (n <= GU_H_MAX, n % 256 == 0; out may be null).
hipError_t launch_rmsnorm_q8(hipStream_t s, const float* x, const float* gain, float eps, size_t n, size_t n_vec,
                             float* out, Q8Bufs q);
// h += (slots, wts, K) combine or ffn row; then normed = rmsnorm(h, gain) unless gain is null.
hipError_t launch_residual_norm(hipStream_t s, float* h, const float* slots, const float* wts, int K, const float* ffn,
                                const float* gain, float eps, size_t n, size_t n_vec, float* normed, Q8Bufs q = Q8Bufs{});

// ---- decoder-layer operators (bb_ops.hip) ----
constexpr int OPS_HD_MAX = 256;     // head_dim bound of the attention kernels
// score rows up to this length are worked on in LDS: 40000 floats (156 KB of the CU's 160 KB, one
// such wave per CU), past the reference agent's 32,768-position window (agent.rs:25-26)
constexpr int OPS_ROW_LDS = 40000;
// out[t][c] = causal conv of token t over [state; bx] (op: bx = B·x_gate from the in_proj output
// src [T][3C], and out = C·conv); the state is read, not written.
hipError_t launch_conv(hipStream_t s, bool op, const float* src, const float* state, const float* w, int C, int L,
                       int T, float* out);
// state <- the last L-1 columns of [state; bx] (run after launch_conv on the same batch).
hipError_t launch_conv_state(hipStream_t s, bool op, const float* src, float* state, int C, int L, int T);
// One token: conv, state update and the Q8 of y in one launch (C % 256 == 0; y f32[C] too).
hipError_t launch_conv1_q8(hipStream_t s, const float* src, float* state, const float* w, int C, int L, float* y,
                           Q8Bufs q);
// per-head rmsnorm (gain null: none) and RoPE from (cos, sin) rows [T][hd/2], in place on buf [T][n_heads][hd].
hipError_t launch_norm_rope(hipStream_t s, float* buf, int T, int n_heads, int hd, const float* gain, float eps,
                            const float2* rope, float* buf2 = nullptr, int n2 = 0,
                            const float* gain2 = nullptr);
// scores [T][n_heads][n0+T]: token t's query against cached positions j < n0 + t + 1.
hipError_t launch_attn_scores(hipStream_t s, const float* q, const float* kc, int n0, int T, int n_heads, int n_kv,
                              int hd, float scale, float* scores);
// softmax of each score row (in place), then out [T][n_heads][hd] = Σ_j w_j·v_j. scores needs one
// float of slack after its last row (the long-row P·V reads a row's last position 8 bytes at a time).
hipError_t launch_attn_pv(hipStream_t s, float* scores, const float* vc, int n0, int T, int n_heads, int n_kv, int hd,
                          float* out);
hipError_t launch_softmax(hipStream_t s, float* x, size_t n, size_t n_vec);
hipError_t launch_zero(hipStream_t s, float* x, size_t n);
// out [T][H] = rows tokens[t] (device) of an embedding table in F32 / F16 / Q4_K / Q6_K rows.
hipError_t launch_embed(hipStream_t s, const uint8_t* te, int dtype, size_t row_bytes, const uint32_t* tokens, int T,
                        int H, float* out);

}  // namespace bb
#endif
