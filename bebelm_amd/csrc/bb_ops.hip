// bb_ops.hip — the decoder layer's operators around the MoE block (model.rs:105-130): the gated
// short conv (model.rs:399-427 one token, :190-216 a batch) and GQA attention (model.rs:430-456,
// :222-259), with their kernel-level pieces conv_step / conv_prefill (kernels/conv.rs:18-68),
// softmax (kernels/softmax.rs:9-22), attention_decode (kernels/attention.rs:17-55) and the
// per-head q/k norm + NEOX RoPE (model.rs:692-701, kernels/rope.rs:17-30). Projections run on
// the Q4_K/Q6_K row kernels of bb_kernels.hip.
//
// Exactness. Every value is computed with the reference's operations in its order:
//   conv      sum = w[L-1]·bx, then += w[k]·col_k for k = 0..L-2 (columns oldest first; the
//             columns before the batch come from the state). One thread per (token, channel):
//             every output depends only on its own L columns, so the batch is the rolled loop.
//   scores    matmul.rs's dot (32 fmaf chains, the `wide` lane reduce) on a half-wave, times
//             1/sqrt(head_dim).
//   softmax   max, f32 exps (bb_expf: glibc's expf restated), their f64 sum left to right in one
//             lane, each value times (float)(1.0 / sum).
//   P·V       out[d] = Σ_j w_j·v[j][d] in position order from 0.0, one lane per d.
//   q/k norm  rmsnorm over head_dim with its f64 sum left to right in one lane (the reference's
//             order; the hidden-size rmsnorm kernel sums as a tree), then RoPE with (cos, sin)
//             of each (position, pair) taken from a table the host fills with libm's sinf and
//             cosf of the reference's angle sequence (theta from (float)pos, times
//             powf(base, -2/d) per pair): the same functions the reference's f32 sin_cos calls.
#include "bb_device.h"
#include "bb_internal.h"

namespace bb {

// ---- gated short conv ------------------------------------------------------------------------
// Column j of [state; bx] for channel c (j < L-1: the state; else token j-(L-1) of the batch).
// OP: the batch is the in_proj output (B, C, x_gate chunks of 3C per token) and bx = B·x_gate.
template <bool OP>
__device__ __forceinline__ float conv_col(const float* __restrict__ src, const float* __restrict__ state, int C, int L,
                                          int j, int c) {
  if (j < L - 1) return state[(size_t)j * C + c];
  const size_t r = (size_t)(j - (L - 1));
  if constexpr (OP) return src[r * 3 * C + c] * src[r * 3 * C + 2 * C + c];
  else return src[r * C + c];
}

// out[t][c] = conv of token t (OP: times the C chunk, y = C·conv_out).
template <bool OP>
__global__ void __launch_bounds__(256) k_conv(const float* __restrict__ src, const float* __restrict__ state,
                                              const float* __restrict__ w, int C, int L, int T, float* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)T * C) return;
  const int t = (int)(i / C), c = (int)(i % C);
  const float* wc = w + (size_t)c * L;
  float sum = wc[L - 1] * conv_col<OP>(src, state, C, L, t + L - 1, c);
  for (int k = 0; k + 1 < L; ++k) sum += wc[k] * conv_col<OP>(src, state, C, L, t + k, c);
  if constexpr (OP) out[(size_t)t * C + c] = src[(size_t)t * 3 * C + C + c] * sum;
  else out[(size_t)t * C + c] = sum;
}

// The state after the batch: its last L-1 columns. Column k takes column T+k of [state; bx],
// read before it is overwritten (k ascending, T+k > k).
template <bool OP>
__global__ void __launch_bounds__(256) k_conv_state(const float* __restrict__ src, float* state, int C, int L, int T) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  for (int k = 0; k + 1 < L; ++k) state[(size_t)k * C + c] = conv_col<OP>(src, state, C, L, T + k, c);
}

hipError_t launch_conv(hipStream_t s, bool op, const float* src, const float* state, const float* w, int C, int L,
                       int T, float* out) {
  const unsigned blocks = (unsigned)(((size_t)T * C + 255) / 256);
  if (op) BB_LAUNCH(k_conv<true>, dim3(blocks), dim3(256), 0, s, src, state, w, C, L, T, out);
  else BB_LAUNCH(k_conv<false>, dim3(blocks), dim3(256), 0, s, src, state, w, C, L, T, out);
  return hipGetLastError();
}

hipError_t launch_conv_state(hipStream_t s, bool op, const float* src, float* state, int C, int L, int T) {
  if (L < 2) return hipSuccess;
  const unsigned sb = (unsigned)((C + 255) / 256);
  if (op) BB_LAUNCH(k_conv_state<true>, dim3(sb), dim3(256), 0, s, src, state, C, L, T);
  else BB_LAUNCH(k_conv_state<false>, dim3(sb), dim3(256), 0, s, src, state, C, L, T);
  return hipGetLastError();
}

// ---- per-head rmsnorm + RoPE -----------------------------------------------------------------
// One 64-thread block per (token, head) of buf [T][n_heads][hd] (hd <= OPS_HD_MAX, even).
// rope: (cos, sin) pairs [position][hd/2]; token t uses position row t of the table slice.
__global__ void __launch_bounds__(64) k_norm_rope(float* buf, int n_heads, int hd, const float* __restrict__ gain,
                                                  float eps, const float2* __restrict__ rope, int norm) {
  __shared__ float sx[OPS_HD_MAX];
  __shared__ float s_scale;
  const int head = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  float* x = buf + ((size_t)t * n_heads + head) * hd;
  for (int d = lane; d < hd; d += 64) sx[d] = x[d];
  __syncthreads();
  if (norm) {
    if (lane == 0) {
      double ss = -0.0;
      for (int d = 0; d < hd; ++d) ss += (double)(sx[d] * sx[d]);
      const float mean = (float)(ss / (double)hd);
      s_scale = 1.0f / sqrtf(mean + eps);
    }
    __syncthreads();
    const float sc = s_scale;
    for (int d = lane; d < hd; d += 64) sx[d] = sx[d] * sc * gain[d];
    __syncthreads();
  }
  const int half = hd / 2;
  const float2* cs = rope + (size_t)t * half;
  for (int i = lane; i < half; i += 64) {
    const float a = sx[i], b = sx[i + half], cv = cs[i].x, sv = cs[i].y;
    x[i] = a * cv - b * sv;
    x[i + half] = a * sv + b * cv;
  }
}

hipError_t launch_norm_rope(hipStream_t s, float* buf, int T, int n_heads, int hd, const float* gain, float eps,
                            const float2* rope) {
  BB_LAUNCH(k_norm_rope, dim3(n_heads, T), dim3(64), 0, s, buf, n_heads, hd, gain, eps, rope, gain != nullptr);
  return hipGetLastError();
}

// ---- attention -------------------------------------------------------------------------------
// matmul.rs:36-66's dot of q (LDS) and a key row on a 32-lane half-wave: lane c runs chain c,
// then the lane combine and the `wide` reduce tree through shuffles; valid on lane c == 0.
__device__ __forceinline__ float dot_half(const float* q, const float* __restrict__ k, int n, int c) {
  float acc = 0.0f;
  const int n32 = n & ~31;
  int i = 0;
  for (; i < n32; i += 32) acc = fmaf(q[i + c], k[i + c], acc);
  for (; i + 8 <= n; i += 8)
    if (c < 8) acc = fmaf(q[i + c], k[i + c], acc);
  const float A = acc + __shfl_down(acc, 8, 32);
  const float v = A + __shfl_down(A, 16, 32);
  const float u = v + __shfl_down(v, 4, 32);
  const float y = u + __shfl_down(u, 2, 32);
  float r = y + __shfl_down(y, 1, 32);
  for (; i < n; ++i) r = r + q[i] * k[i];
  return r;
}

// scores[t][h][j] = dot(q[t][h], k[j][h / group]) · scale for j < n0 + t + 1 (the positions
// token t sees once its own key is in the cache). Block = 8 half-waves = 8 positions.
__global__ void __launch_bounds__(256) k_attn_scores(const float* __restrict__ q, const float* __restrict__ kc, int n0,
                                                     int n_heads, int n_kv, int hd, float scale, float* __restrict__ sc,
                                                     int ld) {
  __shared__ float sq[OPS_HD_MAX];
  const int h = blockIdx.y, t = blockIdx.z;
  for (int d = threadIdx.x; d < hd; d += 256) sq[d] = q[((size_t)t * n_heads + h) * hd + d];
  __syncthreads();
  const int j = blockIdx.x * 8 + (threadIdx.x >> 5), c = threadIdx.x & 31;
  if (j >= n0 + t + 1) return;  // whole half-waves leave together
  const int kv = h / (n_heads / n_kv);
  const float r = dot_half(sq, kc + ((size_t)j * n_kv + kv) * hd, hd, c);
  if (c == 0) sc[((size_t)t * n_heads + h) * ld + j] = r * scale;
}

// A score row as one wave reads and rewrites it: in LDS (rows up to OPS_ROW_LDS values), else in
// global memory through agent-scope accesses. The row is re-read after other lanes of the wave
// rewrote it, so it must not be read through the non-coherent vector L1 cache.
template <bool LDS>
struct Row {
  float* p;
  __device__ __forceinline__ float ld(int j) const {
    if constexpr (LDS) return p[j];
    else return __hip_atomic_load(p + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __device__ __forceinline__ void st(int j, float v) const {
    if constexpr (LDS) p[j] = v;
    else __hip_atomic_store(p + j, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
};

// softmax.rs:9-22 on row r[0..n) by one wave (exps written back, then scaled).
template <bool LDS>
__device__ void wave_softmax(const Row<LDS> r, int n, const uint64_t* exptab, float* s_inv) {
  const int lane = threadIdx.x;
  float m = -__builtin_inff();
  for (int j = lane; j < n; j += 64) m = fmaxf(m, r.ld(j));
  m = wave_max(m);
  for (int j = lane; j < n; j += 64) r.st(j, bb_expf_tab(r.ld(j) - m, exptab));
  __syncthreads();
  if (lane == 0) {
    double sum = 0.0;
    for (int j = 0; j < n; ++j) sum += (double)r.ld(j);
    *s_inv = (float)(1.0 / sum);
  }
  __syncthreads();
  const float inv = *s_inv;
  for (int j = lane; j < n; j += 64) r.st(j, r.ld(j) * inv);
  __syncthreads();
}

// One wave per (token, head): softmax of the score row, then out[d] = Σ_j w_j·v[j][kv][d]. The
// LDS form copies the row (written by k_attn_scores) into dynamic LDS first.
template <bool LDS>
__global__ void __launch_bounds__(64) k_attn_softmax_pv(float* sc, const float* __restrict__ vc, int n0, int n_heads,
                                                        int n_kv, int hd, int ld, float* __restrict__ out) {
  extern __shared__ float lrow[];
  __shared__ uint64_t exptab[32];
  __shared__ float s_inv;
  const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  if (lane < 32) exptab[lane] = exp_table_entry();
  const int n = n0 + t + 1;
  float* s = sc + ((size_t)t * n_heads + h) * ld;
  if constexpr (LDS)
    for (int j = lane; j < n; j += 64) lrow[j] = s[j];
  __syncthreads();
  const Row<LDS> r{LDS ? lrow : s};
  wave_softmax<LDS>(r, n, exptab, &s_inv);
  const int kv = h / (n_heads / n_kv);
  for (int d = lane; d < hd; d += 64) {
    float o = 0.0f;
    for (int j = 0; j < n; ++j) o += r.ld(j) * vc[((size_t)j * n_kv + kv) * hd + d];
    out[((size_t)t * n_heads + h) * hd + d] = o;
  }
}

hipError_t launch_attn_scores(hipStream_t s, const float* q, const float* kc, int n0, int T, int n_heads, int n_kv,
                              int hd, float scale, float* scores) {
  const int ld = n0 + T;
  BB_LAUNCH(k_attn_scores, dim3((unsigned)((ld + 7) / 8), n_heads, T), dim3(256), 0, s, q, kc, n0, n_heads, n_kv, hd,
            scale, scores, ld);
  return hipGetLastError();
}

hipError_t launch_attn_pv(hipStream_t s, float* scores, const float* vc, int n0, int T, int n_heads, int n_kv, int hd,
                          float* out) {
  const int ld = n0 + T;
  if (ld <= OPS_ROW_LDS)
    BB_LAUNCH(k_attn_softmax_pv<true>, dim3(n_heads, T), dim3(64), (size_t)ld * 4, s, scores, vc, n0, n_heads, n_kv, hd,
              ld, out);
  else
    BB_LAUNCH(k_attn_softmax_pv<false>, dim3(n_heads, T), dim3(64), 0, s, scores, vc, n0, n_heads, n_kv, hd, ld, out);
  return hipGetLastError();
}

// softmax of n_vec rows of n (kernels/softmax.rs:9-22), one wave per row (through LDS when the
// row fits).
template <bool LDS>
__global__ void __launch_bounds__(64) k_softmax(float* x, int n) {
  extern __shared__ float lrow[];
  __shared__ uint64_t exptab[32];
  __shared__ float s_inv;
  if (threadIdx.x < 32) exptab[threadIdx.x] = exp_table_entry();
  float* g = x + (size_t)blockIdx.x * n;
  if constexpr (LDS)
    for (int j = threadIdx.x; j < n; j += 64) lrow[j] = g[j];
  __syncthreads();
  wave_softmax<LDS>(Row<LDS>{LDS ? lrow : g}, n, exptab, &s_inv);
  if constexpr (LDS)
    for (int j = threadIdx.x; j < n; j += 64) g[j] = lrow[j];
}

hipError_t launch_softmax(hipStream_t s, float* x, size_t n, size_t n_vec) {
  if (n == 0 || n_vec == 0) return hipSuccess;
  if (n <= (size_t)OPS_ROW_LDS) BB_LAUNCH(k_softmax<true>, dim3((unsigned)n_vec), dim3(64), n * 4, s, x, (int)n);
  else BB_LAUNCH(k_softmax<false>, dim3((unsigned)n_vec), dim3(64), 0, s, x, (int)n);
  return hipGetLastError();
}

// ---- embedding lookup -------------------------------------------------------------------------
// Element i of a row in the GGUF block layouts, as dequantize_into produces it (dequant.rs:75-175):
// Q4_K (d·sc)·q - dmin·m, Q6_K (d·sc)·(q - 32), F16 widened, F32 as is.
__device__ __forceinline__ float dequant_elem(int dtype, const uint8_t* __restrict__ row, int i) {
  if (dtype == DT_F32) return reinterpret_cast<const float*>(row)[i];
  if (dtype == DT_F16) return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(row)[i]);
  const int e = i & 255;
  if (dtype == DT_Q4_K) {
    const uint8_t* b = row + (size_t)(i >> 8) * 144;
    const float d = f16_bits_to_f32(b[0] | (b[1] << 8)), dmin = f16_bits_to_f32(b[2] | (b[3] << 8));
    const uint8_t* sc = b + 4;
    const int chunk = e >> 6, hi = (e >> 5) & 1, l = e & 31, j = 2 * chunk + hi;
    int s, m;
    if (j < 4) {
      s = sc[j] & 63;
      m = sc[j + 4] & 63;
    } else {
      s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
      m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
    const uint8_t qb = b[16 + chunk * 32 + l];
    const int q = hi ? (qb >> 4) : (qb & 15);
    return (d * (float)s) * (float)q - dmin * (float)m;
  }
  // Q6_K
  const uint8_t* b = row + (size_t)(i >> 8) * 210;
  const int n = e >> 7, r = e & 127, qtr = r >> 5, l = r & 31, is = l >> 4;
  const uint8_t* ql = b + 64 * n;
  const uint8_t* qh = b + 128 + 32 * n;
  const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192 + 8 * n);
  const float d = f16_bits_to_f32(b[208] | (b[209] << 8));
  const int lo = (qtr & 1) ? ql[l + 32] : ql[l];
  const int q = ((qtr & 2) ? (lo >> 4) : (lo & 15)) | (((qh[l] >> (2 * qtr)) & 3) << 4);
  return d * (float)sc[is + 2 * qtr] * (float)(q - 32);
}

// out[t] = row tokens[t] of the embedding table (Model::embed_token, model.rs:390-397).
__global__ void __launch_bounds__(256) k_embed(const uint8_t* __restrict__ te, int dtype, size_t row_bytes,
                                               const uint32_t* __restrict__ tokens, int H, float* __restrict__ out) {
  const int t = blockIdx.y;
  const uint8_t* row = te + (size_t)tokens[t] * row_bytes;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < H; i += gridDim.x * 256) out[(size_t)t * H + i] = dequant_elem(dtype, row, i);
}

hipError_t launch_embed(hipStream_t s, const uint8_t* te, int dtype, size_t row_bytes, const uint32_t* tokens, int T,
                        int H, float* out) {
  BB_LAUNCH(k_embed, dim3((unsigned)((H + 255) / 256), T), dim3(256), 0, s, te, dtype, row_bytes, tokens, H, out);
  return hipGetLastError();
}

// x[0..n) = 0 (a kernel rather than a memset, so that the clear can sit in a captured graph).
__global__ void __launch_bounds__(256) k_zero(float* x, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) x[i] = 0.0f;
}

hipError_t launch_zero(hipStream_t s, float* x, size_t n) {
  if (n == 0) return hipSuccess;
  BB_LAUNCH(k_zero, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n);
  return hipGetLastError();
}

}  // namespace bb
