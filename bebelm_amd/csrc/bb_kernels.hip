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

LaunchEvents& launch_events() {
  static thread_local LaunchEvents ev;
  return ev;
}

const char* kernel_name(int id) {
  static const char* names[K_COUNT] = {"route_gating",  "gateup_swiglu", "down_combine", "quantize_q8",
                                       "rows_q8",      "rows_f32",      "elementwise",  "rmsnorm",
                                       "route_large",  "dispatch",      "gemm_gateup",  "gemm_down",
                                       "combine",      "residual_norm", "residual_route", "conv",
                                       "conv_state",   "norm_rope",     "attn_scores",  "attn_pv",
                                       "softmax",      "embed"};
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
  BB_LAUNCH(k_quantize, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, x, n_vec, n, q);
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

// The same with one wave per row: lane group g (8 lanes) takes blocks g, g+8, ... of the row, J
// of them per pass, and every load of a pass (the weights and the Q8 activations they meet) is
// issued before the first is used, so a row costs a memory round trip per pass instead of one
// per block. The groups' block values meet in LDS and lane 0 adds them left to right from the
// start value (the reference's order). With at most 8J blocks the row's weights stay in
// registers from token to token. With SWIGLU the wave also takes row o of w2 (same shape) against
// the same activations and stores silu(row o of w · x) * (row o of w2 · x), the dense FFN's
// gate, up and swiglu (model.rs:464-466) in one pass. With RPW > 1 a wave takes RPW consecutive
// rows and issues all their loads together (the activations once for all of them): more bytes in
// flight per wave for the long matrices, where one row per wave leaves HBM under-fed.
constexpr int RW_MAX_NB = 64;
template <int DT, int J, bool SWIGLU, int RPW>
__global__ void __launch_bounds__(256) k_rows_q8w(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
                                                  size_t row_bytes, int nb, size_t n_rows, Q8Bufs q, size_t q_stride,
                                                  size_t n_tok, float* __restrict__ y, size_t y_tok_stride,
                                                  int neg_zero_start) {
  static_assert(!SWIGLU || RPW == 1, "SwiGLU pairs: one row per wave");
  using R = RowDot<DT>;
  __shared__ float vals[4][RPW][RW_MAX_NB];
  __shared__ float vals2[SWIGLU ? 4 : 1][SWIGLU ? RW_MAX_NB : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 3, p = lane & 7;
  const size_t o0 = ((size_t)blockIdx.x * 4 + wave) * RPW;
  if (o0 >= n_rows) return;  // (a whole wave: the block has no barrier)
  const uint8_t* row2 = SWIGLU ? w2 + o0 * row_bytes : nullptr;
  const bool resident = nb <= 8 * J;
  typename R::Lane wl[RPW][J], wl2[SWIGLU ? J : 1];
  for (size_t t = 0; t < n_tok; ++t) {
    const int8_t* qx = q.q + t * q_stride;
    const float* sx = q.scales + t * nb;
    const int32_t* sums = q.sums + t * (q_stride / 32);
    for (int c0 = 0; c0 < nb; c0 += 8 * J) {
      typename R::X xv[J];
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int b = min(c0 + g + 8 * j, nb - 1);  // (past the row: a block of it again, value unused)
        if (t == 0 || !resident) {
#pragma unroll
          for (int r = 0; r < RPW; ++r) {
            // (rows past the matrix: its last row again, value unused)
            const size_t o = min(o0 + r, n_rows - 1);
            wl[r][j] = R::load(w + o * row_bytes + (size_t)b * R::BLOCK_BYTES, p);
          }
          if constexpr (SWIGLU) wl2[j] = R::load(row2 + (size_t)b * R::BLOCK_BYTES, p);
        }
        xv[j] = R::xload(qx + b * QK, sums + b * 8, sx + b, p);
      }
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int b = c0 + g + 8 * j;
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          const float v = R::block_value_x(wl[r][j], p, xv[j]);
          if (p == 0 && b < nb) vals[wave][r][b] = v;
        }
        if constexpr (SWIGLU) {
          const float v2 = R::block_value_x(wl2[j], p, xv[j]);
          if (p == 0 && b < nb) vals2[wave][b] = v2;
        }
      }
    }
    // (one wave writes and reads its rows of vals: its LDS accesses are performed in order)
    if (lane < RPW && o0 + lane < n_rows) {
      float acc = neg_zero_start ? -0.0f : 0.0f;
      for (int b = 0; b < nb; ++b) acc += vals[wave][lane][b];
      if constexpr (SWIGLU) {
        float acc2 = neg_zero_start ? -0.0f : 0.0f;
        for (int b = 0; b < nb; ++b) acc2 += vals2[wave][b];
        acc = silu(acc) * acc2;
      }
      y[t * y_tok_stride + o0 + lane] = acc;
    }
  }
}

// Rows of at most 8 blocks in matrices of at least RW_MULTI_ROWS rows take several rows per wave:
// 4 of Q4_K, 2 of Q6_K (whose lanes hold 27 bytes a row; 4 rows cost occupancy). On the logits
// head's 2048 -> 128000 rows this is 34.7 -> 24.3 µs (Q4_K) and 43.4 -> 36.7 µs (Q6_K).
constexpr size_t RW_MULTI_ROWS = 16384;
template <int DT>
constexpr int rw_rows_per_wave() { return DT == DT_Q6_K ? 2 : 4; }
template <int DT, bool SWIGLU>
static hipError_t launch_rows_q8w(hipStream_t s, const uint8_t* w, const uint8_t* w2, size_t row_bytes, int nb,
                                  size_t n_rows, Q8Bufs q, size_t q_stride, size_t n_tok, float* y,
                                  size_t y_tok_stride, int nz) {
  dim3 grid((unsigned)((n_rows + 3) / 4));
  if (!SWIGLU && nb <= 8 && n_rows >= RW_MULTI_ROWS) {
    constexpr int RPW = rw_rows_per_wave<DT>();
    BB_LAUNCH((k_rows_q8w<DT, 1, false, RPW>), dim3((unsigned)((n_rows + 4 * RPW - 1) / (4 * RPW))), dim3(256), 0, s, w,
              w2, row_bytes, nb, n_rows, q, q_stride, n_tok, y, y_tok_stride, nz);
  } else if (nb <= 8)
    BB_LAUNCH((k_rows_q8w<DT, 1, SWIGLU, 1>), grid, dim3(256), 0, s, w, w2, row_bytes, nb, n_rows, q, q_stride, n_tok,
              y, y_tok_stride, nz);
  else if (nb <= 16)
    BB_LAUNCH((k_rows_q8w<DT, 2, SWIGLU, 1>), grid, dim3(256), 0, s, w, w2, row_bytes, nb, n_rows, q, q_stride, n_tok,
              y, y_tok_stride, nz);
  else
    BB_LAUNCH((k_rows_q8w<DT, 4, SWIGLU, 1>), grid, dim3(256), 0, s, w, w2, row_bytes, nb, n_rows, q, q_stride, n_tok,
              y, y_tok_stride, nz);
  return hipGetLastError();
}

hipError_t launch_rows_q8_swiglu(hipStream_t s, int dtype, const uint8_t* gate, const uint8_t* up, size_t row_bytes,
                                 int nb, size_t n_rows, Q8Bufs q, size_t q_stride, size_t n_tok, float* y,
                                 size_t y_tok_stride, int neg_zero_start) {
  if (n_rows == 0) return hipSuccess;
  if (nb < 1 || nb > RW_MAX_NB) return hipErrorInvalidValue;
  if (dtype == DT_Q4_K)
    return launch_rows_q8w<DT_Q4_K, true>(s, gate, up, row_bytes, nb, n_rows, q, q_stride, n_tok, y, y_tok_stride,
                                          neg_zero_start);
  return launch_rows_q8w<DT_Q6_K, true>(s, gate, up, row_bytes, nb, n_rows, q, q_stride, n_tok, y, y_tok_stride,
                                        neg_zero_start);
}

hipError_t launch_rows_q8(hipStream_t s, int dtype, const uint8_t* w, size_t row_bytes, int nb, size_t n_rows,
                          Q8Bufs q, size_t q_stride, size_t n_tok, float* y, size_t y_tok_stride, int neg_zero_start) {
  if (n_rows == 0) return hipSuccess;
  if (nb >= 1 && nb <= RW_MAX_NB) {
    if (dtype == DT_Q4_K)
      return launch_rows_q8w<DT_Q4_K, false>(s, w, nullptr, row_bytes, nb, n_rows, q, q_stride, n_tok, y, y_tok_stride,
                                             neg_zero_start);
    return launch_rows_q8w<DT_Q6_K, false>(s, w, nullptr, row_bytes, nb, n_rows, q, q_stride, n_tok, y, y_tok_stride,
                                           neg_zero_start);
  }
  dim3 grid((unsigned)((n_rows + 31) / 32));
  if (dtype == DT_Q4_K)
    BB_LAUNCH(k_rows_q8<DT_Q4_K>, grid, dim3(256), 0, s, w, row_bytes, nb, n_rows, q, q_stride, n_tok, y,
                       y_tok_stride, neg_zero_start);
  else
    BB_LAUNCH(k_rows_q8<DT_Q6_K>, grid, dim3(256), 0, s, w, row_bytes, nb, n_rows, q, q_stride, n_tok, y,
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
    BB_LAUNCH(k_rows_f32<DT_F32>, grid, dim3(256), 0, s, w, n_in, n_rows, x, n_tok, y);
  else
    BB_LAUNCH(k_rows_f32<DT_F16>, grid, dim3(256), 0, s, w, n_in, n_rows, x, n_tok, y);
  return hipGetLastError();
}

// ---- the f32 arm of matvec_fused_batch (FusedJob with qx: None) ------------------------------
// fused_row_dot (matmul.rs:777-785): per 256-block the f32 fused dot of the row with x, summed
// over blocks from -0.0. One lane per row; x (shared by every row) is read through the cache.
__device__ __forceinline__ float reduce8(const float (&v)[8]) {
  return ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
}

// dot_q4k_block (matmul.rs:104-122): per 64-element chunk, nibble_dot32 (:73-94) of the low
// then the high nibbles (8 lanes of fmaf chains for Σq·x and of adds for Σx, each reduced by the
// reduce tree), then sum += (d·sc)·Σqx − (dmin·m)·Σx per sub-block.
__device__ float q4k_block_f32(const uint8_t* __restrict__ blk, const float* __restrict__ x) {
  const float d = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
  const float dmin = f16_bits_to_f32((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
  uint32_t sw[3];
  for (int i = 0; i < 3; ++i)
    sw[i] = (uint32_t)blk[4 + 4 * i] | ((uint32_t)blk[5 + 4 * i] << 8) | ((uint32_t)blk[6 + 4 * i] << 16) |
            ((uint32_t)blk[7 + 4 * i] << 24);
  float sum = 0.0f;
  for (int chunk = 0; chunk < 4; ++chunk) {
    const uint8_t* q = blk + 16 + 32 * chunk;
    float part[2];
    for (int hi = 0; hi < 2; ++hi) {
      const float* xs = x + 64 * chunk + 32 * hi;
      float qx[8], xa[8];
#pragma unroll
      for (int l = 0; l < 8; ++l) qx[l] = xa[l] = 0.0f;
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int l = 0; l < 8; ++l) {
          const uint8_t b = q[8 * k + l];
          const float xv = xs[8 * k + l];
          qx[l] = fmaf((float)(hi ? (b >> 4) : (b & 0xF)), xv, qx[l]);
          xa[l] = xa[l] + xv;
        }
      int sc, m;
      q4k_scale_min(sw[0], sw[1], sw[2], 2 * chunk + hi, sc, m);
      part[hi] = (d * (float)sc) * reduce8(qx) - (dmin * (float)m) * reduce8(xa);
    }
    sum += part[0];
    sum += part[1];
  }
  return sum;
}

// dot_q6k_block (matmul.rs:455-479): acc += sc·q6_dot16 over the 16 sub-blocks (q6_dot16,
// :430-444: 8 lanes of fmaf chains over two 8-element steps, reduced), then d·acc.
__device__ float q6k_block_f32(const uint8_t* __restrict__ blk, const float* __restrict__ x) {
  const float d = f16_bits_to_f32((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
  float acc = 0.0f;
  for (int n = 0; n < 2; ++n) {
    const uint8_t* ql = blk + 64 * n;
    const uint8_t* qh = blk + 128 + 32 * n;
    const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * n);
    for (int g = 0; g < 4; ++g) {
      const int ql_off = (g & 1) ? 32 : 0, high = g >> 1, shift = 2 * g;
      for (int sub = 0; sub < 2; ++sub) {
        const float* xg = x + 128 * n + 32 * g + 16 * sub;
        float qx[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) qx[j] = 0.0f;
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int li = 16 * sub + 8 * c + j;
            const int lo = high ? (ql[ql_off + li] >> 4) : (ql[ql_off + li] & 0x0F);
            const int h2 = (qh[li] >> shift) & 3;
            qx[j] = fmaf((float)((lo | (h2 << 4)) - 32), xg[8 * c + j], qx[j]);
          }
        acc += (float)sc[2 * g + sub] * reduce8(qx);
      }
    }
  }
  return d * acc;
}

template <int DT>
__global__ void __launch_bounds__(256) k_fused_rows_f32(const uint8_t* __restrict__ w, size_t row_bytes, int nb,
                                                        size_t n_rows, const float* __restrict__ x,
                                                        float* __restrict__ y) {
  const size_t o = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= n_rows) return;
  const uint8_t* row = w + o * row_bytes;
  float sum = -0.0f;
  for (int b = 0; b < nb; ++b) {
    if constexpr (DT == DT_Q4_K) sum += q4k_block_f32(row + (size_t)b * 144, x + (size_t)b * QK);
    else sum += q6k_block_f32(row + (size_t)b * 210, x + (size_t)b * QK);
  }
  y[o] = sum;
}

hipError_t launch_fused_rows_f32(hipStream_t s, int dtype, const uint8_t* w, size_t row_bytes, int nb, size_t n_rows,
                                 const float* x, float* y) {
  if (n_rows == 0) return hipSuccess;
  const dim3 grid((unsigned)((n_rows + 255) / 256));
  if (dtype == DT_Q4_K) BB_LAUNCH(k_fused_rows_f32<DT_Q4_K>, grid, dim3(256), 0, s, w, row_bytes, nb, n_rows, x, y);
  else BB_LAUNCH(k_fused_rows_f32<DT_Q6_K>, grid, dim3(256), 0, s, w, row_bytes, nb, n_rows, x, y);
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
  BB_LAUNCH(k_elementwise, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, op, out, a, b, scalar, n);
  return hipGetLastError();
}

// rmsnorm.rs:10-21. The sum of the f32 squares is taken in f64 as a tree instead of the
// reference's left-to-right f64 sum; after narrowing `mean` to f32 the two agree unless the
// two f64 sums straddle an f32 rounding boundary. One block per vector.
// With q.q set (rows of at most GU_H_MAX, n % 256 == 0) the normed row is also quantised to Q8
// (k_quantize's arithmetic, one wave per 256-block, from a copy in LDS), and out may be null.
__global__ void __launch_bounds__(256) k_rmsnorm(const float* __restrict__ x, const float* __restrict__ gain,
                                                 float eps, size_t n, float* __restrict__ out, Q8Bufs q) {
  const float* xv = x + (size_t)blockIdx.x * n;
  float* ov = out + (size_t)blockIdx.x * n;
  constexpr int NI = GU_H_MAX / 256;
  const bool regs = n <= (size_t)GU_H_MAX;  // rows up to GU_H_MAX stay in registers, read once
  float xr[NI], gr[NI];
  double ss = 0.0;
  if (regs) {
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const size_t i = min((size_t)(threadIdx.x + 256 * it), n - 1);  // in bounds; elements past n unused
      xr[it] = xv[i];
      gr[it] = gain[i];
    }
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      if (threadIdx.x + 256 * it >= n) break;
      ss += (double)(xr[it] * xr[it]);
    }
  } else {
    for (size_t i = threadIdx.x; i < n; i += 256) {
      const float v = xv[i];
      ss += (double)(v * v);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  __shared__ double s_part[4];
  __shared__ float s_scale;
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  lds_barrier();
  if (threadIdx.x == 0) {
    const double tot = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    const float mean = (float)(tot / (double)n);
    s_scale = 1.0f / sqrtf(mean + eps);
  }
  lds_barrier();
  const float scale = s_scale;
  if (q.q) {
    __shared__ __align__(16) float s_norm[GU_H_MAX];
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const size_t i = threadIdx.x + 256 * it;
      if (i >= n) break;
      const float v = xr[it] * scale * gr[it];
      s_norm[i] = v;
      if (out) ov[i] = v;
    }
    lds_barrier();
    const size_t nbk = n / QK, v = blockIdx.x;
    const int lane = threadIdx.x & 63;
    for (size_t b = threadIdx.x >> 6; b < nbk; b += 4) {
      const float4 val = *reinterpret_cast<const float4*>(s_norm + b * QK + 4 * lane);
      wave_quantize_block(val, q.q + v * n + b * QK, q.scales + v * nbk + b, q.sums + v * (n / 32) + b * 8);
    }
  } else if (regs) {
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const size_t i = threadIdx.x + 256 * it;
      if (i >= n) break;
      ov[i] = xr[it] * scale * gr[it];
    }
  } else {
    for (size_t i = threadIdx.x; i < n; i += 256) ov[i] = xv[i] * scale * gain[i];
  }
}

// The FFN path's layer boundary for one token per block (model.rs:105-130 with the operator
// sub-layer as identity): h += y, where y is the MoE combine of the token's k slot rows in
// selection order from +0.0 (model.rs:550-553 / :362-369) or a dense FFN output row; then the
// next layer's rmsnorm of h (as k_rmsnorm: the same f64 partial sums and tree) unless gain is
// null. One launch instead of combine, add_assign and rmsnorm.
__global__ void __launch_bounds__(256) k_residual_norm(float* __restrict__ h, const float* __restrict__ slots,
                                                       const float* __restrict__ wts, int K,
                                                       const float* __restrict__ ffn, const float* __restrict__ gain,
                                                       float eps, size_t n, float* __restrict__ normed, Q8Bufs q) {
  const size_t t = blockIdx.x;
  float* hv = h + t * n;
  // thread j takes elements j, j+256, ... (k_rmsnorm's order); every load is issued before the
  // first use, so the block waits for memory once
  constexpr int NI = GU_H_MAX / 256;
  float hr[NI], yr[NI], gr[NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) gr[it] = gain ? gain[min((size_t)(threadIdx.x + 256 * it), n - 1)] : 0.0f;
  if (slots) {
    // the K slot rows (slot indices clamped to K-1, so every load is unconditional and in
    // bounds; slots past K are not used)
    float wk[8], sv[8][NI];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const size_t row = t * K + min(k, K - 1);
      wk[k] = wts[row];
#pragma unroll
      for (int it = 0; it < NI; ++it) {
        const size_t i = min((size_t)(threadIdx.x + 256 * it), n - 1);
        sv[k][it] = slots[row * n + i];
      }
    }
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const size_t i = min((size_t)(threadIdx.x + 256 * it), n - 1);
      hr[it] = hv[i];
      yr[it] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < K) {
#pragma unroll
        for (int it = 0; it < NI; ++it) yr[it] = yr[it] + wk[k] * sv[k][it];
      }
  } else {
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const size_t i = min((size_t)(threadIdx.x + 256 * it), n - 1);
      hr[it] = hv[i];
      yr[it] = ffn[t * n + i];
    }
  }
  double ss = 0.0;
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const size_t i = threadIdx.x + 256 * it;
    if (i >= n) break;
    const float v = hr[it] + yr[it];
    hv[i] = v;
    hr[it] = v;
    ss += (double)(v * v);
  }
  if (!gain) return;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  __shared__ double s_part[4];
  __shared__ float s_scale;
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  lds_barrier();  // (LDS only: the h stores stay in flight)
  if (threadIdx.x == 0) {
    const double tot = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    const float mean = (float)(tot / (double)n);
    s_scale = 1.0f / sqrtf(mean + eps);
  }
  lds_barrier();
  const float scale = s_scale;
  float* ov = normed + t * n;
  if (q.q) {
    // the normed row's Q8 as well (k_rmsnorm's q form: a copy in LDS, one wave per 256-block)
    __shared__ __align__(16) float s_norm[GU_H_MAX];
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const size_t i = threadIdx.x + 256 * it;
      if (i >= n) break;
      const float v = hr[it] * scale * gr[it];
      s_norm[i] = v;
      ov[i] = v;
    }
    lds_barrier();
    const size_t nbk = n / QK;
    const int lane = threadIdx.x & 63;
    for (size_t b = threadIdx.x >> 6; b < nbk; b += 4) {
      const float4 val = *reinterpret_cast<const float4*>(s_norm + b * QK + 4 * lane);
      wave_quantize_block(val, q.q + t * n + b * QK, q.scales + t * nbk + b, q.sums + t * (n / 32) + b * 8);
    }
    return;
  }
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const size_t i = threadIdx.x + 256 * it;
    if (i >= n) break;
    ov[i] = hr[it] * scale * gr[it];
  }
}

hipError_t launch_residual_norm(hipStream_t s, float* h, const float* slots, const float* wts, int K, const float* ffn,
                                const float* gain, float eps, size_t n, size_t n_vec, float* normed, Q8Bufs q) {
  if (n_vec == 0) return hipSuccess;
  if (n > (size_t)GU_H_MAX || K > 8) return hipErrorInvalidValue;  // the kernel's register tiles
  if (q.q && (!gain || n % QK != 0)) return hipErrorInvalidValue;
  BB_LAUNCH(k_residual_norm, dim3((unsigned)n_vec), dim3(256), 0, s, h, slots, wts, K, ffn, gain, eps, n, normed, q);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(hipStream_t s, const float* x, const float* gain, float eps, size_t n, size_t n_vec,
                          float* out) {
  if (n_vec == 0) return hipSuccess;
  BB_LAUNCH(k_rmsnorm, dim3((unsigned)n_vec), dim3(256), 0, s, x, gain, eps, n, out, Q8Bufs{});
  return hipGetLastError();
}

hipError_t launch_rmsnorm_q8(hipStream_t s, const float* x, const float* gain, float eps, size_t n, size_t n_vec,
                             float* out, Q8Bufs q) {
  if (n_vec == 0) return hipSuccess;
  if (!q.q || n > (size_t)GU_H_MAX || n % QK != 0) return hipErrorInvalidValue;
  BB_LAUNCH(k_rmsnorm, dim3((unsigned)n_vec), dim3(256), 0, s, x, gain, eps, n, out, q);
  return hipGetLastError();
}

}  // namespace bb
