// bb_kernels.hip — the MoE FFN hot path on gfx950 (decode / small-batch path and the
// kernel-level mirrors of the reference's src/kernels API).
//
// Work decomposition shared by the GEMV kernels: an 8-lane group owns one weight row and
// walks its 256-weight super-blocks left to right; each lane handles 16 bytes of a Q4_K
// block's quants (or 24 bytes of a Q6_K block's), does the exact int8 sub-dots with
// v_dot4_i32_i8, and the group sums the integer partials with DPP. The f32 epilogue then
// runs once per block in the reference's operation order, so every row value is bit-identical
// to the CPU path's.
#include "bb_device.h"
#include "bb_internal.h"

namespace bb {

const char* kernel_name(int id) {
  static const char* names[K_COUNT] = {"route_small",  "gateup_swiglu", "down_combine", "quantize_q8",
                                       "rows_q8",      "rows_f32",      "elementwise",  "rmsnorm",
                                       "route_large",  "dispatch",      "gemm_gateup",  "gemm_down",
                                       "combine"};
  return (id >= 0 && id < K_COUNT) ? names[id] : "?";
}

// ---------------------------------------------------------------------------------------------
// f32 dot (matmul.rs:36-66) on one 32-lane half-wave: lane c runs fmaf chain c over elements
// i = c (mod 32), the `i + 8 <= n` loop extends chains 0..7, then the lane combine
// (acc0+acc1)+(acc2+acc3) and the reduce_add tree ((v0+v4)+(v2+v6))+((v1+v5)+(v3+v7)); the
// scalar tail is added last. The value is valid on lane c == 0.
template <int DT>
__device__ __forceinline__ float ld_w(const uint8_t* w, size_t i) {
  if constexpr (DT == DT_F32) return reinterpret_cast<const float*>(w)[i];
  else return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(w)[i]);
}

template <int DT>
__device__ __forceinline__ float dot32_half(const uint8_t* __restrict__ a, const float* __restrict__ b, int n, int c) {
  float acc = 0.0f;
  const int n32 = n & ~31;
  int i = 0;
  for (; i < n32; i += 32) acc = fmaf(ld_w<DT>(a, i + c), b[i + c], acc);
  for (; i + 8 <= n; i += 8)
    if (c < 8) acc = fmaf(ld_w<DT>(a, i + c), b[i + c], acc);
  const float A = acc + __shfl_down(acc, 8, 32);
  const float v = A + __shfl_down(A, 16, 32);
  const float u = v + __shfl_down(v, 4, 32);
  const float y = u + __shfl_down(u, 2, 32);
  float r = y + __shfl_down(y, 1, 32);
  for (; i < n; ++i) r = r + ld_w<DT>(a, i) * b[i];
  return r;
}

// ---------------------------------------------------------------------------------------------
// Router + gating + dispatch for a small token batch (model.rs:483-495 per token, :316-322).
// Blocks [0, E): router row e for every token. Blocks [E, ...): Q8 quantisation of x, one
// 256-block per wave (model.rs:501). The last block to finish (grid-completion counter) runs
// sigmoid / top-k / renormalisation per token on 32-lane half-waves and the stable counting
// sort by expert.
__global__ void __launch_bounds__(256) k_route_small(const float* __restrict__ W, const float* __restrict__ bias,
                                                     const float* __restrict__ x, int T, int H, int E, int K,
                                                     Q8Bufs xq, RouteBufs rb) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, c = lane & 31;
  const int nbx = H / QK;
  if ((int)blockIdx.x < E) {
    const int e = blockIdx.x;
    const uint8_t* wr = reinterpret_cast<const uint8_t*>(W + (size_t)e * H);
    for (int base = wave * 2; base < T; base += 8) {
      const int t = base + half;
      const int tc = t < T ? t : T - 1;
      const float r = dot32_half<DT_F32>(wr, x + (size_t)tc * H, H, c);
      if (c == 0 && t < T) rb.logits[(size_t)t * E + e] = r;
    }
  } else {
    const int qi = ((int)blockIdx.x - E) * 4 + wave;
    if (qi < T * nbx) {
      const int t = qi / nbx, b = qi % nbx;
      const float4 v = *reinterpret_cast<const float4*>(x + (size_t)t * H + b * QK + 4 * lane);
      wave_quantize_block(v, xq.q + (size_t)t * H + b * QK, xq.scales + (size_t)t * nbx + b,
                          xq.sums + (size_t)t * (H / 32) + b * 8);
    }
  }

  __shared__ int s_last;
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(rb.counter, 1u) == gridDim.x - 1;
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  __shared__ int32_t s_sel[1024];
  __shared__ int32_t s_cnt[64];
  __shared__ int32_t s_off[65];
  __shared__ int32_t s_ties;
  if (tid == 0) s_ties = 0;
  if (tid < 64) s_cnt[tid] = 0;
  __syncthreads();

  for (int base = wave * 2; base < T; base += 8) {
    const int t = base + half;
    const int tc = t < T ? t : T - 1;
    const bool live = c < E;
    const float s = live ? sigmoid(rb.logits[(size_t)tc * E + c]) : 0.0f;
    const float key = live ? s + bias[c] : 0.0f;
    const int32_t kk = total_key(key);
    // (key, -index) packed so a plain max picks the highest key, lowest index first.
    long long cand = live ? (((long long)kk << 8) | (long long)(255 - c)) : (long long)(-0x7fffffffffffffffLL - 1);
    int32_t prev_kk = 0;
    float prev_key = 0.0f, denom = -0.0f;
    int sel_r[8];
    float s_r[8];
    int ties = 0;
    float margin = __builtin_inff();
    const int rounds = K < E ? K + 1 : K;
    for (int r = 0; r < rounds; ++r) {
      long long m = cand;
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) {
        const int lo = __shfl_xor((int)(m & 0xffffffffLL), o, 32);
        const int hi = __shfl_xor((int)(m >> 32), o, 32);
        const long long other = ((long long)hi << 32) | (unsigned)lo;
        m = other > m ? other : m;
      }
      const int ew = 255 - (int)(m & 0xff);
      const int32_t kw = (int32_t)(m >> 8);
      const float kwf = __shfl(key, ew, 32);
      if (c == ew) cand = (long long)(-0x7fffffffffffffffLL - 1);
      if (r > 0 && kw == prev_kk) ++ties;
      if (r == K) margin = prev_key - kwf;
      if (r < K) {
        sel_r[r] = ew;
        s_r[r] = __shfl(s, ew, 32);
      }
      prev_kk = kw;
      prev_key = kwf;
    }
    for (int r = 0; r < K; ++r) denom += s_r[r];
    denom = denom + 1e-6f;
    if (c == 0 && t < T) {
      for (int r = 0; r < K; ++r) {
        rb.sel[(size_t)t * K + r] = sel_r[r];
        rb.wts[(size_t)t * K + r] = s_r[r] / denom;
        s_sel[t * K + r] = sel_r[r];
      }
      rb.margin[t] = margin;
      if (ties) atomicAdd(&s_ties, ties);
    }
  }
  __syncthreads();
  const int n_ent = T * K;
  for (int i = tid; i < n_ent; i += 256) atomicAdd(&s_cnt[s_sel[i]], 1);
  __syncthreads();
  if (tid == 0) {
    int acc = 0, nh = 0;
    s_off[0] = 0;
    for (int e = 0; e < E; ++e) {
      rb.counts[e] = s_cnt[e];
      if (s_cnt[e] > 0) rb.hit[1 + nh++] = e;
      acc += s_cnt[e];
      s_off[e + 1] = acc;
      rb.offsets[e + 1] = acc;
    }
    rb.offsets[0] = 0;
    rb.hit[0] = nh;
    rb.ties[0] = s_ties;
    *rb.counter = 0u;
  }
  __syncthreads();
  // model.rs:317-322: within an expert, entries keep (token, slot) order.
  for (int i = tid; i < n_ent; i += 256) {
    const int e = s_sel[i];
    int rank = 0;
    for (int j = 0; j < i; ++j) rank += s_sel[j] == e;
    rb.perm[s_off[e] + rank] = i;
  }
}

hipError_t launch_route_small(hipStream_t s, const float* router, const float* bias, const float* x, int T, int H,
                              int E, int K, Q8Bufs xq, RouteBufs rb) {
  const int nq = (T * (H / QK) + 3) / 4;
  hipLaunchKernelGGL(k_route_small, dim3(E + nq), dim3(256), 0, s, router, bias, x, T, H, E, K, xq, rb);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Gate/up GEMV + SwiGLU for every (hit expert, member token) (model.rs:497-524, :340-351).
// Block (rt, u): 4 waves x 8 groups; groups 0-3 take gate rows o, groups 4-7 the matching up
// rows, so silu(gate)*up is formed in registers. The last block of each 256-row slice of an
// expert quantises that slice of act for all its members (model.rs:530-534, matmul.rs:933).
constexpr int GU_ROWS = 16;

template <int DT>
__global__ void __launch_bounds__(256) k_gateup(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
                                                size_t stride_g, size_t stride_u, int H, int F, int K, int batch_mode,
                                                RouteBufs rb, Q8Bufs xq, float* __restrict__ act, Q8Bufs actq,
                                                uint32_t* __restrict__ counters) {
  const int u = blockIdx.y;
  if (u >= rb.hit[0]) return;
  const int e = rb.hit[1 + u];
  const int p0 = rb.offsets[e], p1 = rb.offsets[e + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 3, p = lane & 7;
  const int o = blockIdx.x * GU_ROWS + wave * 4 + (g & 3);
  const int nb = H / QK;
  const size_t row_bytes = (size_t)nb * RowDot<DT>::BLOCK_BYTES;
  const uint8_t* row = (g < 4 ? gate + (size_t)e * stride_g : up + (size_t)e * stride_u) + (size_t)o * row_bytes;
  const float start = (batch_mode && p1 - p0 > 1) ? 0.0f : -0.0f;
  for (int j = p0; j < p1; ++j) {
    const int t = rb.perm[j] / K;
    const float acc = row_dot_q8<DT>(row, nb, p, xq.q + (size_t)t * H, xq.scales + (size_t)t * nb,
                                     xq.sums + (size_t)t * (H / 32), start);
    const float upv = __shfl(acc, (lane + 32) & 63);
    if (g < 4 && p == 0) act[(size_t)j * F + o] = silu(acc) * upv;
  }

  __shared__ int s_last;
  const int nbf = F / QK;
  const int blk = (blockIdx.x * GU_ROWS) / QK;
  uint32_t* ctr = counters + (size_t)u * nbf + blk;
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(ctr, 1u) == (uint32_t)(QK / GU_ROWS - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int j = p0 + wave; j < p1; j += 4) {
    const float4 v = *reinterpret_cast<const float4*>(act + (size_t)j * F + blk * QK + 4 * lane);
    wave_quantize_block(v, actq.q + (size_t)j * F + blk * QK, actq.scales + (size_t)j * nbf + blk,
                        actq.sums + (size_t)j * (F / 32) + blk * 8);
  }
  if (tid == 0) *ctr = 0u;
}

hipError_t launch_gateup(hipStream_t s, int dtype, const uint8_t* gate, const uint8_t* up, size_t stride_g,
                         size_t stride_u, int H, int F, int K, int max_hit, int batch_mode, const RouteBufs& rb,
                         Q8Bufs xq, float* act, Q8Bufs actq, uint32_t* counters) {
  dim3 grid(F / GU_ROWS, max_hit);
  if (dtype == DT_Q4_K)
    hipLaunchKernelGGL(k_gateup<DT_Q4_K>, grid, dim3(256), 0, s, gate, up, stride_g, stride_u, H, F, K, batch_mode,
                       rb, xq, act, actq, counters);
  else
    hipLaunchKernelGGL(k_gateup<DT_Q6_K>, grid, dim3(256), 0, s, gate, up, stride_g, stride_u, H, F, K, batch_mode,
                       rb, xq, act, actq, counters);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Down GEMV per (hit expert, member) into its (token, slot) row, then the ordered combine
// out[t] = Σ_k w[t,k]·down[t,k] in selection order (model.rs:547-553, :361-369), run by the
// last expert block to finish each 32-row tile.
constexpr int DN_ROWS = 32;

template <int DT>
__global__ void __launch_bounds__(256) k_down(const uint8_t* __restrict__ down, size_t stride_d, int H, int F, int K,
                                              int T, int batch_mode, RouteBufs rb, Q8Bufs actq,
                                              float* __restrict__ slots, float* __restrict__ out,
                                              uint32_t* __restrict__ counters) {
  const int u = blockIdx.y;
  const int n_hit = rb.hit[0];
  if (u >= n_hit) return;
  const int e = rb.hit[1 + u];
  const int p0 = rb.offsets[e], p1 = rb.offsets[e + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 3, p = lane & 7;
  const int o = blockIdx.x * DN_ROWS + wave * 8 + g;
  const int nb = F / QK;
  const size_t row_bytes = (size_t)nb * RowDot<DT>::BLOCK_BYTES;
  const uint8_t* row = down + (size_t)e * stride_d + (size_t)o * row_bytes;
  const float start = (batch_mode && p1 - p0 > 1) ? 0.0f : -0.0f;
  for (int j = p0; j < p1; ++j) {
    const int i = rb.perm[j];
    const float acc = row_dot_q8<DT>(row, nb, p, actq.q + (size_t)j * F, actq.scales + (size_t)j * nb,
                                     actq.sums + (size_t)j * (F / 32), start);
    if (p == 0) slots[(size_t)i * H + o] = acc;
  }

  __shared__ int s_last;
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&counters[blockIdx.x], 1u) == (uint32_t)(n_hit - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int idx = tid; idx < T * DN_ROWS; idx += 256) {
    const int t = idx / DN_ROWS, oo = blockIdx.x * DN_ROWS + idx % DN_ROWS;
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) acc = acc + rb.wts[(size_t)t * K + k] * slots[((size_t)t * K + k) * H + oo];
    out[(size_t)t * H + oo] = acc;
  }
  if (tid == 0) counters[blockIdx.x] = 0u;
}

hipError_t launch_down(hipStream_t s, int dtype, const uint8_t* down, size_t stride_d, int H, int F, int K, int T,
                       int max_hit, int batch_mode, const RouteBufs& rb, Q8Bufs actq, float* slots, float* out,
                       uint32_t* counters) {
  dim3 grid(H / DN_ROWS, max_hit);
  if (dtype == DT_Q4_K)
    hipLaunchKernelGGL(k_down<DT_Q4_K>, grid, dim3(256), 0, s, down, stride_d, H, F, K, T, batch_mode, rb, actq,
                       slots, out, counters);
  else
    hipLaunchKernelGGL(k_down<DT_Q6_K>, grid, dim3(256), 0, s, down, stride_d, H, F, K, T, batch_mode, rb, actq,
                       slots, out, counters);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Kernel-level mirrors of src/kernels: quantize_q8, matvec/matmul row kernels, elementwise.
__global__ void __launch_bounds__(256) k_quantize(const float* __restrict__ x, size_t n_vec, size_t n, Q8Bufs q) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const size_t nbk = n / QK;
  const size_t wi = (size_t)blockIdx.x * 4 + wave;
  if (wi >= n_vec * nbk) return;
  const size_t v = wi / nbk, b = wi % nbk;
  const float4 val = *reinterpret_cast<const float4*>(x + v * n + b * QK + 4 * lane);
  wave_quantize_block(val, q.q + v * n + b * QK, q.scales + v * nbk + b, q.sums + v * (n / 32) + b * 8);
}

hipError_t launch_quantize(hipStream_t s, const float* x, size_t n_vec, size_t n, Q8Bufs q) {
  const size_t waves = n_vec * (n / QK);
  if (waves == 0) return hipSuccess;
  hipLaunchKernelGGL(k_quantize, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, x, n_vec, n, q);
  return hipGetLastError();
}

// y[t*y_tok_stride + o] = row o · Q8 vector t, for all rows and tokens (matvec when n_tok == 1
// with the -0.0-started sum; the batched matmul path starts from +0.0).
template <int DT>
__global__ void __launch_bounds__(256) k_rows_q8(const uint8_t* __restrict__ w, size_t row_bytes, int nb,
                                                 size_t n_rows, Q8Bufs q, size_t q_stride, size_t n_tok,
                                                 float* __restrict__ y, size_t y_tok_stride, int neg_zero_start) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 3, p = lane & 7;
  const size_t o = (size_t)blockIdx.x * 32 + wave * 8 + g;
  if (o >= n_rows) return;
  const uint8_t* row = w + o * row_bytes;
  const float start = neg_zero_start ? -0.0f : 0.0f;
  for (size_t t = 0; t < n_tok; ++t) {
    const float acc = row_dot_q8<DT>(row, nb, p, q.q + t * q_stride, q.scales + t * nb, q.sums + t * (q_stride / 32),
                                     start);
    if (p == 0) y[t * y_tok_stride + o] = acc;
  }
}

hipError_t launch_rows_q8(hipStream_t s, int dtype, const uint8_t* w, size_t row_bytes, int nb, size_t n_rows,
                          Q8Bufs q, size_t q_stride, size_t n_tok, float* y, size_t y_tok_stride, int neg_zero_start) {
  if (n_rows == 0) return hipSuccess;
  dim3 grid((unsigned)((n_rows + 31) / 32));
  if (dtype == DT_Q4_K)
    hipLaunchKernelGGL(k_rows_q8<DT_Q4_K>, grid, dim3(256), 0, s, w, row_bytes, nb, n_rows, q, q_stride, n_tok, y,
                       y_tok_stride, neg_zero_start);
  else
    hipLaunchKernelGGL(k_rows_q8<DT_Q6_K>, grid, dim3(256), 0, s, w, row_bytes, nb, n_rows, q, q_stride, n_tok, y,
                       y_tok_stride, neg_zero_start);
  return hipGetLastError();
}

// F32 / F16 rows (dequantised exactly) dotted with f32 tokens; y token-major [t][n_rows].
template <int DT>
__global__ void __launch_bounds__(256) k_rows_f32(const uint8_t* __restrict__ w, size_t n_in, size_t n_rows,
                                                  const float* __restrict__ x, size_t n_tok, float* __restrict__ y) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, c = lane & 31;
  const size_t elem = DT == DT_F32 ? 4 : 2;
  const size_t total = n_rows * n_tok;
  const size_t base = ((size_t)blockIdx.x * 4 + wave) * 2;
  if (base >= total) return;
  const size_t item = base + half;
  const size_t ic = item < total ? item : total - 1;
  const size_t o = ic / n_tok, t = ic % n_tok;
  const float r = dot32_half<DT>(w + o * n_in * elem, x + t * n_in, (int)n_in, c);
  if (c == 0 && item < total) y[t * n_rows + o] = r;
}

hipError_t launch_rows_f32(hipStream_t s, int dtype, const uint8_t* w, size_t n_in, size_t n_rows, const float* x,
                           size_t n_tok, float* y) {
  const size_t items = n_rows * n_tok;
  if (items == 0) return hipSuccess;
  dim3 grid((unsigned)((items + 7) / 8));
  if (dtype == DT_F32)
    hipLaunchKernelGGL(k_rows_f32<DT_F32>, grid, dim3(256), 0, s, w, n_in, n_rows, x, n_tok, y);
  else
    hipLaunchKernelGGL(k_rows_f32<DT_F16>, grid, dim3(256), 0, s, w, n_in, n_rows, x, n_tok, y);
  return hipGetLastError();
}

// activation.rs:16-29, elementwise.rs:4-17.
__global__ void __launch_bounds__(256) k_elementwise(int op, float* __restrict__ out, const float* __restrict__ a,
                                                     const float* __restrict__ b, float scalar, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  switch (op) {
    case EW_SWIGLU: out[i] = silu(a[i]) * b[i]; break;
    case EW_SIGMOID: out[i] = sigmoid(a[i]); break;
    case EW_ADD_SCALED: out[i] = out[i] + scalar * a[i]; break;
    default: out[i] = out[i] + a[i]; break;
  }
}

hipError_t launch_elementwise(hipStream_t s, int op, float* out, const float* a, const float* b, float scalar,
                              size_t n) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_elementwise, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, op, out, a, b, scalar, n);
  return hipGetLastError();
}

// rmsnorm.rs:10-21. The sum of the f32 squares is taken in f64 as a tree instead of the
// reference's left-to-right f64 sum; after narrowing `mean` to f32 the two agree unless the
// two f64 sums straddle an f32 rounding boundary. One block per vector.
__global__ void __launch_bounds__(256) k_rmsnorm(const float* __restrict__ x, const float* __restrict__ gain,
                                                 float eps, size_t n, float* __restrict__ out) {
  const float* xv = x + (size_t)blockIdx.x * n;
  float* ov = out + (size_t)blockIdx.x * n;
  double ss = 0.0;
  for (size_t i = threadIdx.x; i < n; i += 256) {
    const float v = xv[i];
    ss += (double)(v * v);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  __shared__ double s_part[4];
  __shared__ float s_scale;
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0) {
    const double tot = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    const float mean = (float)(tot / (double)n);
    s_scale = 1.0f / sqrtf(mean + eps);
  }
  __syncthreads();
  const float scale = s_scale;
  for (size_t i = threadIdx.x; i < n; i += 256) ov[i] = xv[i] * scale * gain[i];
}

hipError_t launch_rmsnorm(hipStream_t s, const float* x, const float* gain, float eps, size_t n, size_t n_vec,
                          float* out) {
  if (n_vec == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)n_vec), dim3(256), 0, s, x, gain, eps, n, out);
  return hipGetLastError();
}

}  // namespace bb
