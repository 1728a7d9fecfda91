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
//   scores    matmul.rs's dot (32 fmaf chains, the `wide` lane reduce) in one lane per position,
//             times 1/sqrt(head_dim).
//   softmax   max, f32 exps (bb_expf: glibc's expf restated), their f64 sum left to right in one
//             lane, each value times (float)(1.0 / sum).
//   P·V       out[d] = Σ_j w_j·v[j][d] in position order from 0.0, one lane per d.
//   q/k norm  rmsnorm over head_dim with its f64 sum left to right in one lane (the reference's
//             order; the hidden-size rmsnorm kernel sums as a tree), then RoPE with (cos, sin)
//             of each (position, pair) taken from a table the host fills with libm's sinf and
//             cosf of the reference's angle sequence (theta from (float)pos, times
//             powf(base, -2/d) per pair): the same functions the reference's f32 sin_cos calls.
#include "bb_device.h"
#include <utility>
#include "bb_internal.h"

namespace bb {

constexpr int PV_CHUNK = 32;    // value-column loads in flight per lane in P·V of one row
constexpr int PVL_MIN_LD = 0;   // rows from this length take the softmax + k_attn_pv_long pair
constexpr int AT_PV_MIN_T = 8;  // batches of this many tokens take the tiled softmax + P·V

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

// One token, the whole conv step in one launch: wave w takes channels 256w..256w+255 (four per
// lane, lane l holding 4l..4l+3): y = C·conv over [state; bx] as k_conv computes it, the state
// shifted by one column as k_conv_state does (each channel's reads before its writes, in the
// same thread), and the 256-block of y quantised to Q8 (quantize_q8's arithmetic) for out_proj.
__global__ void __launch_bounds__(64) k_conv1_q8(const float* __restrict__ src, float* state,
                                                 const float* __restrict__ w, int C, int L, float* __restrict__ y,
                                                 Q8Bufs q) {
  const int c0 = blockIdx.x * QK + 4 * threadIdx.x;
  float out[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = c0 + u;
    const float* wc = w + (size_t)c * L;
    float sum = wc[L - 1] * conv_col<true>(src, state, C, L, L - 1, c);
    for (int k = 0; k + 1 < L; ++k) sum += wc[k] * conv_col<true>(src, state, C, L, k, c);
    out[u] = src[C + c] * sum;
    for (int k = 0; k + 1 < L; ++k) state[(size_t)k * C + c] = conv_col<true>(src, state, C, L, 1 + k, c);
  }
  *reinterpret_cast<float4*>(y + c0) = make_float4(out[0], out[1], out[2], out[3]);
  wave_quantize_block(make_float4(out[0], out[1], out[2], out[3]), q.q + blockIdx.x * QK, q.scales + blockIdx.x,
                      q.sums + blockIdx.x * 8);
}

hipError_t launch_conv1_q8(hipStream_t s, const float* src, float* state, const float* w, int C, int L, float* y,
                           Q8Bufs q) {
  if (C % QK != 0 || L < 2 || !q.q) return hipErrorInvalidValue;
  BB_LAUNCH(k_conv1_q8, dim3((unsigned)(C / QK)), dim3(64), 0, s, src, state, w, C, L, y, q);
  return hipGetLastError();
}

// ---- per-head rmsnorm + RoPE -----------------------------------------------------------------
// One 64-thread block per (token, head) of buf [T][n_heads][hd] (hd <= OPS_HD_MAX, even).
// rope: (cos, sin) pairs [position][hd/2]; token t uses position row t of the table slice.
// Blocks past n_heads take the heads of a second buffer (buf2: n2 heads per token, gain2), so q
// and k are normed and rotated in one launch.
__global__ void __launch_bounds__(64) k_norm_rope(float* buf, int n_heads, int hd, const float* __restrict__ gain,
                                                  float eps, const float2* __restrict__ rope, int norm, float* buf2,
                                                  int n2, const float* __restrict__ gain2) {
  __shared__ float sx[OPS_HD_MAX];
  __shared__ float s_scale;
  const int t = blockIdx.y, lane = threadIdx.x;
  const bool second = (int)blockIdx.x >= n_heads;
  const int head = second ? (int)blockIdx.x - n_heads : (int)blockIdx.x;
  if (second) gain = gain2;
  float* x = second ? buf2 + ((size_t)t * n2 + head) * hd : buf + ((size_t)t * n_heads + head) * hd;
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
                            const float2* rope, float* buf2, int n2, const float* gain2) {
  if (buf2 && (gain == nullptr) != (gain2 == nullptr)) return hipErrorInvalidValue;
  BB_LAUNCH(k_norm_rope, dim3(n_heads + (buf2 ? n2 : 0), T), dim3(64), 0, s, buf, n_heads, hd, gain, eps, rope,
            gain != nullptr, buf2, n2, gain2);
  return hipGetLastError();
}

// ---- attention -------------------------------------------------------------------------------
// matmul.rs:36-66's dot of q (LDS) and a key row in one lane: 32 fmaf chains (chain c over the
// elements i = c mod 32, then for a tail of whole groups of 8 the chains c < 8 over it), the lane
// combine v_c = (a_c + a_{c+8}) + (a_{c+16} + a_{c+24}), the `wide` reduce tree
// ((v0+v4)+(v2+v6))+((v1+v5)+(v3+v7)), then the last n % 8 products added left to right.
// V4: n % 4 == 0 and 16-byte aligned rows (float4 loads).
template <bool V4>
__device__ __forceinline__ float dot_lane(const float* q, const float* __restrict__ k, int n) {
  float a[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) a[c] = 0.0f;
  int i = 0;
  for (; i + 32 <= n; i += 32) {
    if constexpr (V4) {
#pragma unroll
      for (int c4 = 0; c4 < 8; ++c4) {
        const float4 kv = *reinterpret_cast<const float4*>(k + i + 4 * c4);
        const float4 qv = *reinterpret_cast<const float4*>(q + i + 4 * c4);
        a[4 * c4] = fmaf(qv.x, kv.x, a[4 * c4]);
        a[4 * c4 + 1] = fmaf(qv.y, kv.y, a[4 * c4 + 1]);
        a[4 * c4 + 2] = fmaf(qv.z, kv.z, a[4 * c4 + 2]);
        a[4 * c4 + 3] = fmaf(qv.w, kv.w, a[4 * c4 + 3]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 32; ++c) a[c] = fmaf(q[i + c], k[i + c], a[c]);
    }
  }
  for (; i + 8 <= n; i += 8) {
#pragma unroll
    for (int c = 0; c < 8; ++c) a[c] = fmaf(q[i + c], k[i + c], a[c]);
  }
  float v[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) v[c] = (a[c] + a[c + 8]) + (a[c + 16] + a[c + 24]);
  float r = ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
  for (; i < n; ++i) r = r + q[i] * k[i];
  return r;
}

// scores[t][h][j] = dot(q[t][h], k[j][h / group]) · scale for j < n0 + t + 1 (the positions
// token t sees once its own key is in the cache). Block = one wave = 64 positions of one token
// and one kv head: lane j's key row is read once for the G heads that share it, q of those
// heads from LDS (dynamic, G·hd floats; the same address in every lane).
template <bool V4>
__global__ void __launch_bounds__(64) k_attn_scores_gqa(const float* __restrict__ q, const float* __restrict__ kc,
                                                        int n0, int n_heads, int n_kv, int hd, float scale,
                                                        float* __restrict__ sc, int ld) {
  extern __shared__ __align__(16) float sq[];
  const int g = blockIdx.y, t = blockIdx.z, G = n_heads / n_kv;
  const int n = n0 + t + 1, j0 = blockIdx.x * 64;
  if (j0 >= n) return;  // the whole block
  const float* qt = q + ((size_t)t * n_heads + (size_t)g * G) * hd;  // heads gG .. gG+G-1, contiguous
  for (int i = threadIdx.x; i < G * hd; i += 64) sq[i] = qt[i];
  __syncthreads();
  const int j = j0 + threadIdx.x;
  if (j >= n) return;  // (no barrier follows)
  const float* kr = kc + ((size_t)j * n_kv + g) * hd;
  for (int hh = 0; hh < G; ++hh)
    sc[((size_t)t * n_heads + (size_t)g * G + hh) * ld + j] = dot_lane<V4>(sq + hh * hd, kr, hd) * scale;
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

// A score row of n floats into LDS by the block's NW waves: whole chunks of 64 by LDS DMA (wave w
// takes chunks w, w + NW, ...), all issued before the one wait (a plain load-then-store loop
// waited for every load in turn: at 16K positions, 256 round trips a row), the partial last
// chunk by plain loads. The caller's barrier publishes the row.
template <int NW = 1>
__device__ __forceinline__ void row_to_lds(const float* src, float* lrow, int n) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nfull = n / 64;
  for (int c = w; c < nfull; c += NW) __builtin_amdgcn_global_load_lds(src + 64 * c + lane, lrow + 64 * c, 4, 0, 0);
  if (w == 0 && 64 * nfull + lane < n) lrow[64 * nfull + lane] = src[64 * nfull + lane];
  __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): the copies landed
}

// softmax.rs:9-22 on row r[0..n) by the block's NW waves (exps written back, then scaled).
template <bool LDS, int NW = 1>
__device__ void row_softmax(const Row<LDS> r, int n, const uint64_t* exptab, float* s_inv) {
  constexpr int NT = 64 * NW;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float m = -__builtin_inff();
#pragma unroll 8
  for (int j = tid; j < n; j += NT) m = fmaxf(m, r.ld(j));
  m = wave_max(m);
  if constexpr (NW > 1) {
    __shared__ float wmax[NW];
    if (lane == 0) wmax[w] = m;
    __syncthreads();
    m = wmax[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) m = fmaxf(m, wmax[i]);
  }
#pragma unroll 4
  for (int j = tid; j < n; j += NT) r.st(j, bb_expf_tab(r.ld(j) - m, exptab));
  __syncthreads();
  // The reference's sum is one left-to-right chain of f64 adds (softmax.rs:14-17), but only
  // inv = (float)(1 / sum) leaves it. Every summand is >= 0, so the chain's sum S_c and this
  // block's tree sum S_t (each thread's elements in order, a butterfly over the wave, then the
  // waves' sums in order) are both within (n + n/64 + 6 + NW)·u·S of the exact sum S (u = 2^-53,
  // recursive summation bounds), and so within B = (n + 64)·2^-51·S_t of each other with room to
  // spare for the rounding of B and of the interval's ends. (float)(1 / x) never increases as x
  // grows: when the ends S_t − B and S_t + B give the same float, S_c gives it too. Otherwise
  // (about one row in 10^4 at 16K positions, and rows holding NaN or infinities) thread 0 runs
  // the chain itself.
  // (IEEE addition commutes, so both lanes of every butterfly pair form the same sum, all 64
  // lanes end with the same value, and every thread adds the waves' sums in the same order.)
  double st = 0.0;
  for (int j = tid; j < n; j += NT) st += (double)r.ld(j);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) st += __shfl_xor(st, o);
  if constexpr (NW > 1) {
    __shared__ double wsum[NW];
    if (lane == 0) wsum[w] = st;
    __syncthreads();
    st = wsum[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) st += wsum[i];
  }
  const double bnd = (double)(n + 64) * 0x1p-51 * st;
  const float f_lo = (float)(1.0 / (st - bnd)), f_hi = (float)(1.0 / (st + bnd));
  if (f_lo == f_hi) {
    if (tid == 0) *s_inv = f_lo;
  } else if (tid == 0) {
    // left to right; the next 16 values are read while the adds of the current 16 run (the adds
    // are one dependent chain, the reads are not)
    constexpr int U = 16;
    double sum = 0.0;
    const int nfull = n / U;
    float ea[U], eb[U];
    auto rd = [&](float(&e)[U], int c) {
#pragma unroll
      for (int u = 0; u < U; ++u) e[u] = r.ld(c * U + u);
    };
    auto add = [&](const float(&e)[U]) {
#pragma unroll
      for (int u = 0; u < U; ++u) sum += (double)e[u];
    };
    if (nfull > 0) rd(ea, 0);
    int c = 0;
    for (; c + 2 <= nfull; c += 2) {
      rd(eb, c + 1);
      add(ea);
      if (c + 2 < nfull) rd(ea, c + 2);
      add(eb);
    }
    if (c < nfull) add(ea);
    for (int j = nfull * U; j < n; ++j) sum += (double)r.ld(j);
    *s_inv = (float)(1.0 / sum);
  }
  __syncthreads();
  const float inv = *s_inv;
#pragma unroll 8
  for (int j = tid; j < n; j += NT) r.st(j, r.ld(j) * inv);
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
    row_to_lds(s, lrow, n);
  __syncthreads();
  const Row<LDS> r{LDS ? lrow : s};
  row_softmax<LDS>(r, n, exptab, &s_inv);
  const int kv = h / (n_heads / n_kv);
  const size_t vs = (size_t)n_kv * hd;  // between consecutive positions of one value column
  for (int d = lane; d < hd; d += 64) {
    // position order from 0.0; the values of the next 32 positions are loaded while the adds of
    // the current 32 run (the adds are a dependent chain, the loads are not)
    const float* vp = vc + (size_t)kv * hd + d;
    float o = 0.0f;
    float xa[PV_CHUNK], xb[PV_CHUNK];
    const int nfull = n / PV_CHUNK;
    auto load = [&](float(&x)[PV_CHUNK], int c) {
#pragma unroll
      for (int u = 0; u < PV_CHUNK; ++u) x[u] = vp[(size_t)(c * PV_CHUNK + u) * vs];
    };
    auto accum = [&](const float(&x)[PV_CHUNK], int c) {
#pragma unroll
      for (int u = 0; u < PV_CHUNK; ++u) o += r.ld(c * PV_CHUNK + u) * x[u];
    };
    if (nfull > 0) load(xa, 0);
    int c = 0;
    for (; c + 2 <= nfull; c += 2) {
      load(xb, c + 1);
      accum(xa, c);
      if (c + 2 < nfull) load(xa, c + 2);
      accum(xb, c + 1);
    }
    if (c < nfull) accum(xa, c);
    for (int j = nfull * PV_CHUNK; j < n; ++j) o += r.ld(j) * vp[(size_t)j * vs];
    out[((size_t)t * n_heads + h) * hd + d] = o;
  }
}

// ---- attention tiles (head_dim 64) ------------------------------------------------------------
// Items are (token, head) pairs of one kv head g: a block takes AT_ITEMS / G tokens, so that its
// items (token-major, then the G heads) number at most AT_ITEMS, and 4 waves take items w, w+4, ...
constexpr int AT_HD = 64;
constexpr int AT_KS = AT_HD + 4;  // padded LDS row of a key (conflict-free float4 reads)
constexpr int AT_ITEMS = 64;     // items of a scores block
constexpr int AT_PV_ITEMS = 16;  // items of a P·V block (more blocks: its waves run long chains)
constexpr int AT_IPW = AT_PV_ITEMS / 4;  // P·V items per wave

__host__ __device__ constexpr int at_tokens(int G, int items = AT_ITEMS) { return G >= items ? 1 : items / G; }

// matmul.rs:36-66's dot (dot_lane's order) of a key row held in registers and q in LDS.
__device__ __forceinline__ float dot64_reg(const float (&k)[AT_HD], const float* q) {
  float a[32];
#pragma unroll
  for (int c4 = 0; c4 < 8; ++c4) {
    const float4 qv = *reinterpret_cast<const float4*>(q + 4 * c4);
    a[4 * c4] = fmaf(qv.x, k[4 * c4], 0.0f);
    a[4 * c4 + 1] = fmaf(qv.y, k[4 * c4 + 1], 0.0f);
    a[4 * c4 + 2] = fmaf(qv.z, k[4 * c4 + 2], 0.0f);
    a[4 * c4 + 3] = fmaf(qv.w, k[4 * c4 + 3], 0.0f);
  }
#pragma unroll
  for (int c4 = 0; c4 < 8; ++c4) {
    const float4 qv = *reinterpret_cast<const float4*>(q + 32 + 4 * c4);
    a[4 * c4] = fmaf(qv.x, k[32 + 4 * c4], a[4 * c4]);
    a[4 * c4 + 1] = fmaf(qv.y, k[32 + 4 * c4 + 1], a[4 * c4 + 1]);
    a[4 * c4 + 2] = fmaf(qv.z, k[32 + 4 * c4 + 2], a[4 * c4 + 2]);
    a[4 * c4 + 3] = fmaf(qv.w, k[32 + 4 * c4 + 3], a[4 * c4 + 3]);
  }
  float v[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) v[c] = (a[c] + a[c + 8]) + (a[c + 16] + a[c + 24]);
  return ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
}

// Scores of the block's tokens x the G heads of kv head g against positions j0..j0+63: the 64
// key rows are copied into LDS (coalesced) and lane j keeps row j in registers; q of every item
// is read from LDS (the same address in every lane). Causal: item (t, .) covers j <= n0 + t.
__global__ void __launch_bounds__(256) k_attn_scores_tile(const float* __restrict__ q, const float* __restrict__ kc,
                                                          int n0, int T, int n_heads, int n_kv, float scale,
                                                          float* __restrict__ sc, int ld) {
  __shared__ __align__(16) float sq[AT_ITEMS * AT_HD];
  __shared__ __align__(16) float sk[64 * AT_KS];
  const int G = n_heads / n_kv, TT = at_tokens(G);
  const int g = blockIdx.y, t0 = blockIdx.z * TT, j0 = blockIdx.x * 64;
  const int nt = min(TT, T - t0), n_items = nt * G;
  if (j0 > n0 + t0 + nt - 1) return;  // no token of the block sees these positions
  const int tid = threadIdx.x;
  for (int i = tid; i < n_items * (AT_HD / 4); i += 256) {
    const int it = i / (AT_HD / 4), c4 = i % (AT_HD / 4), tt = it / G, hh = it % G;
    reinterpret_cast<float4*>(sq)[i] =
        reinterpret_cast<const float4*>(q + ((size_t)(t0 + tt) * n_heads + (size_t)g * G + hh) * AT_HD)[c4];
  }
  const int jlast = n0 + T - 1;  // last cached position (rows past it are clamped, never used)
  for (int i = tid; i < 64 * (AT_HD / 4); i += 256) {
    const int r = i / (AT_HD / 4), c4 = i % (AT_HD / 4);
    const int jj = min(j0 + r, jlast);
    *reinterpret_cast<float4*>(sk + r * AT_KS + 4 * c4) =
        reinterpret_cast<const float4*>(kc + ((size_t)jj * n_kv + g) * AT_HD)[c4];
  }
  __syncthreads();
  const int lane = tid & 63, w = tid >> 6, j = j0 + lane;
  float kr[AT_HD];
#pragma unroll
  for (int c4 = 0; c4 < AT_HD / 4; ++c4) {
    const float4 v = *reinterpret_cast<const float4*>(sk + lane * AT_KS + 4 * c4);
    kr[4 * c4] = v.x;
    kr[4 * c4 + 1] = v.y;
    kr[4 * c4 + 2] = v.z;
    kr[4 * c4 + 3] = v.w;
  }
  for (int it = w; it < n_items; it += 4) {
    const int tt = it / G, hh = it % G, t = t0 + tt;
    if (j > n0 + t) continue;  // (no barrier follows)
    sc[((size_t)t * n_heads + (size_t)g * G + hh) * ld + j] = dot64_reg(kr, sq + it * AT_HD) * scale;
  }
}

// softmax.rs:9-22 of every score row (t, h), each of its own length n0 + t + 1, in place, by
// SM_WAVES waves per row.
constexpr int SM_WAVES = 8;
template <bool LDS>
__global__ void __launch_bounds__(64 * SM_WAVES) k_attn_softmax(float* sc, int n0, int n_heads, int ld) {
  extern __shared__ float lrow[];
  __shared__ uint64_t exptab[32];
  __shared__ float s_inv;
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  if (tid < 32) exptab[tid] = exp_table_entry();
  const int n = n0 + t + 1;
  float* s = sc + ((size_t)t * n_heads + h) * ld;
  if constexpr (LDS)
    row_to_lds<SM_WAVES>(s, lrow, n);
  __syncthreads();
  row_softmax<LDS, SM_WAVES>(Row<LDS>{LDS ? lrow : s}, n, exptab, &s_inv);
  if constexpr (LDS)
    for (int j = tid; j < n; j += 64 * SM_WAVES) s[j] = lrow[j];
}

// out[t][h][d] = Σ_j p[t][h][j]·v[j][g][d] for the block's items, position order from 0.0. Per
// chunk of 64 positions the value rows and the items' probabilities are copied into LDS; lane d
// of wave w keeps the running sums of items w, w+4, ... (independent chains side by side).
__global__ void __launch_bounds__(256) k_attn_pv_tile(const float* __restrict__ p, const float* __restrict__ vc,
                                                      int n0, int T, int n_heads, int n_kv, int ld,
                                                      float* __restrict__ out) {
  __shared__ __align__(16) float sv[64 * AT_HD];
  __shared__ __align__(16) float sp[AT_PV_ITEMS * 64];
  const int G = n_heads / n_kv, TT = at_tokens(G, AT_PV_ITEMS);
  const int g = blockIdx.x, t0 = blockIdx.y * TT;
  const int nt = min(TT, T - t0), n_items = nt * G;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int jlast = n0 + t0 + nt - 1;  // the last position any item uses
  float o[AT_IPW];
  int lim[AT_IPW];  // item w + 4k uses positions j <= lim[k] (-1: no such item)
#pragma unroll
  for (int k = 0; k < AT_IPW; ++k) {
    const int it = w + 4 * k;
    o[k] = 0.0f;
    lim[k] = it < n_items ? n0 + t0 + it / G : -1;
  }
  for (int c0 = 0; c0 <= jlast; c0 += 64) {
    __syncthreads();  // the previous chunk has been used
    for (int i = tid; i < 64 * (AT_HD / 4); i += 256) {
      const int r = i / (AT_HD / 4), c4 = i % (AT_HD / 4);
      const int jj = min(c0 + r, jlast);
      reinterpret_cast<float4*>(sv)[i] = reinterpret_cast<const float4*>(vc + ((size_t)jj * n_kv + g) * AT_HD)[c4];
    }
    for (int i = tid; i < n_items * 64; i += 256) {
      const int it = i >> 6, jj = c0 + (i & 63), t = t0 + it / G, hh = it % G;
      sp[i] = jj <= n0 + t ? p[((size_t)t * n_heads + (size_t)g * G + hh) * ld + jj] : 0.0f;
    }
    __syncthreads();
    const int jn = min(64, jlast - c0 + 1);
    for (int jj = 0; jj < jn; ++jj) {
      const float v = sv[jj * AT_HD + lane];
      const int j = c0 + jj;
      // branch-free: every item adds its product, with the bits cleared (+0.0) where the item
      // does not see position j. Adding +0.0 leaves a sum unchanged: the sums start at +0.0 and
      // never become -0.0 (x + y rounds an exact zero to +0.0), so they are the ones of adding
      // only the positions seen.
#pragma unroll
      for (int k = 0; k < AT_IPW; ++k) {
        const uint32_t keep = j <= lim[k] ? 0xffffffffu : 0u;
        const float pv = sp[(w + 4 * k) * 64 + jj] * v;
        o[k] += __uint_as_float(__float_as_uint(pv) & keep);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < AT_IPW; ++k) {
    const int it = w + 4 * k;
    if (it < n_items)
      out[((size_t)(t0 + it / G) * n_heads + (size_t)g * G + it % G) * AT_HD + lane] = o[k];
  }
}

// P·V of a few tokens over long rows (after k_attn_softmax): out[t][h][d] = Σ_j p[t][h][j]·v[j][g][d]
// in position order from 0.0 (attention.rs:46-54), the sums of k_attn_softmax_pv. Each
// (head, dim) is one serial chain of adds, and a decode step has few of them (64 per head), so
// what bounds a long row is how fast one wave can issue its chain: a wave issues one instruction
// every four cycles, and a wave that also multiplied and read its operands spent about three of
// them a position. Block (kv head g, dim slice q, token t) is 1 + NP waves: wave 0 holds the 64
// chains (lane L = head hh of the group x dim d of the slice, G heads x 64/G dims) and only adds;
// the NP producer waves (four for slices of 16 or more dims, else two) read the slice's values
// and the group's probabilities straight into registers through buffer resources (positions
// past the row read zero), D chunks ahead, and write the
// products of each chunk of 64 positions to a ring of PVL_NB chunks in LDS, one row of products per
// chain. The chain wave reads a row 16 bytes (four positions) at a time, so a position costs it
// one add and a quarter of a read. A block barrier a chunk hands the chunks over: in step k the
// producers write chunk k and the chain wave sums chunk k-2 (reading ahead into chunk k-1). A
// product past the row is p·v with p set to 0 and v read as 0, +0.0, and adding +0.0 leaves a
// chain that starts at +0.0 unchanged, so every chunk is summed whole.
constexpr int PVL_CH = 64;              // positions a chunk
constexpr int PVL_ROW = PVL_CH + 4;     // floats a chain's row of products (the pad spreads rows over the banks)
constexpr int PVL_NB = 3;               // chunks of products in the LDS ring
constexpr int PVL_BUF = 64 * PVL_ROW;   // floats a chunk of products
template <int G>
struct PvlCfg {
  static constexpr int DS = 64 / G;                  // dims of a slice
  static constexpr int PC = DS / 4;                  // 16-byte pieces of a position's slice
  static constexpr int PCL = PC < 4 ? PC : 4;        // pieces side by side in a load ...
  static constexpr int PPL = 64 / PCL;               // ... over this many positions (lane = position x piece)
  static constexpr bool SPLIT_HEADS = PCL == 1;      // a load covers the chunk: the producers split the heads
  static constexpr int NP = PCL == 4 ? 4 : 2;        // producer waves
  static constexpr int HP = SPLIT_HEADS ? G / 2 : G; // heads of a producer
  static constexpr int NK = SPLIT_HEADS ? 1 : PCL / NP;  // adjacent positions of a lane (a producer: NK·PPL)
  static constexpr int NQG = PC / PCL;               // piece groups (of PCL)
  static constexpr int NL = NK * NQG;                // 16-byte value loads of a lane a chunk
  static constexpr int HPL = (HP + PCL - 1) / PCL;   // probabilities a lane loads a position (the PCL
                                                     // lanes of a position share theirs)
  static constexpr int NV = NL * 4 + NK * HPL;       // registers of a chunk's loads
  static constexpr int NLD = NL + HPL;               // loads a chunk (a lane's NK probabilities in one)
  static constexpr int D0 = 176 / NV < 63 / NLD ? 176 / NV : 63 / NLD;
  static constexpr int D = D0 < 12 ? D0 : 12;        // chunks of loads in flight (NLD·D fits vmcnt)
  static_assert(NL * 4 * HP * NP == 64, "the producers' lanes make the chunk's 64 x 64 products");
};

template <class F, int... I>
__device__ __forceinline__ void unroll_seq(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}

template <int G>
__global__ void __launch_bounds__(320) k_attn_pv_long(const float* __restrict__ p, const float* __restrict__ vc,
                                                     int n0, int n_heads, int n_kv, int ld, float* __restrict__ out) {
  using C = PvlCfg<G>;
  constexpr int DS = C::DS, PCL = C::PCL, PPL = C::PPL, HP = C::HP, NK = C::NK, NQG = C::NQG, NL = C::NL, D = C::D;
  __shared__ __align__(16) float prod[PVL_NB * PVL_BUF];
  const int g = blockIdx.x, q = blockIdx.y, t = blockIdx.z;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  const int n = n0 + t + 1;
  const int nch = (n + PVL_CH - 1) / PVL_CH;
  const int nsteps = nch + 2;  // step k: chunk k made, chunk k-2 summed; a barrier after all but the last

  if (w == 0) {
    // the chains: lane L reads row L of each chunk, four positions a read
    float o = 0.0f;
    struct Half {
      float4 v[8];
    };
    auto read_half = [&](const float* r, int h, Half& x) {
#pragma unroll
      for (int m = 0; m < 8; ++m) x.v[m] = *reinterpret_cast<const float4*>(r + 32 * h + 4 * m);
    };
    auto add_half = [&](const Half& x) {
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        o += x.v[m].x;
        o += x.v[m].y;
        o += x.v[m].z;
        o += x.v[m].w;
      }
    };
    // (the chain wave loads nothing from memory; the wait tells the compiler so, which otherwise
    // waits in the loop for the producers' loads on a path it cannot rule out)
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    asm volatile("" ::"s"(out));          // (the argument's load done before the loop, not in flight in it)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const float* const row = prod + lane * PVL_ROW;
    int b = 0;  // ring slot of chunk s
    Half x0, x1;
    // each half's reads go out before the adds of the half before (the scheduling barriers keep
    // the compiler from moving the next half's reads above the adds, which cost copies of x0)
    read_half(row, 0, x0);
    // one wait a half for its eight reads, issued a half of adds earlier, with the next half's
    // eight still in flight
    constexpr int LGKM8 = 0xc87f;  // lgkmcnt(8)
    for (int s = 0; s < nch - 1; ++s) {
      const int bn = b == PVL_NB - 1 ? 0 : b + 1;
      read_half(row + b * PVL_BUF, 1, x1);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(LGKM8);
      __builtin_amdgcn_sched_barrier(0);
      add_half(x0);
      __builtin_amdgcn_sched_barrier(0);
      read_half(row + bn * PVL_BUF, 0, x0);  // chunk s+1
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(LGKM8);
      __builtin_amdgcn_sched_barrier(0);
      add_half(x1);
      // no wait for the reads in flight: they are of a chunk the producers overwrite only after the
      // barrier after next
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      b = bn;
    }
    read_half(row + b * PVL_BUF, 1, x1);
    add_half(x0);
    add_half(x1);
    const int hh = lane / DS, dl = lane % DS;
    out[((size_t)t * n_heads + (size_t)g * G + hh) * 64 + q * DS + dl] = o;
    return;
  }

  // producers: lane = (position lp of PPL, piece lc of PCL); producer pw takes positions
  // [pw·NK·PPL, (pw+1)·NK·PPL) of a chunk (heads split instead when a load covers the chunk), a
  // lane the NK adjacent positions pos0 + NK·lp + k
  const int pw = w - 1;
  const int lp = lane / PCL, lc = lane % PCL;
  const int h0 = C::SPLIT_HEADS ? pw * HP : 0;
  const int pos0 = (C::SPLIT_HEADS ? 0 : pw * NK * PPL) + NK * lp;
  const __amdgpu_buffer_rsrc_t rv = buf_rsrc(vc, (uint32_t)n * (uint32_t)n_kv * 256u);
  // (one float past the group's rows in range: a lane's two positions load as one 8-byte read, which
  // at a row's last position takes the float after it; the caller leaves that float in its buffer)
  const __amdgpu_buffer_rsrc_t rp =
      buf_rsrc(p + ((size_t)t * n_heads + (size_t)g * G) * ld, (uint32_t)(G * ld + 1) * 4u);
  const uint32_t row_b = (uint32_t)n_kv * 256u;  // bytes of a cache row
  const uint32_t v_lane = (uint32_t)pos0 * row_b + (uint32_t)g * 256u + (uint32_t)(q * DS + lc * 4) * 4u;
  const uint32_t p_lane = (uint32_t)(h0 * ld + pos0) * 4u;
  const uint32_t chunk_v = (uint32_t)PVL_CH * row_b;
  constexpr int HPL = C::HPL;
  struct Set {
    float4 v[NL];
    float p[HPL][NK];  // head (j·PCL + lc) mod HP of the lane's positions
  };
  auto load = [&](Set& x, int c) {
    const uint32_t cv = (uint32_t)c * chunk_v, cp = (uint32_t)c * (PVL_CH * 4u);
#pragma unroll
    for (int k = 0; k < NK; ++k)
#pragma unroll
      for (int m = 0; m < NQG; ++m)
        x.v[k * NQG + m] =
            __builtin_bit_cast(float4, buf_load16(rv, v_lane + cv + (uint32_t)k * row_b + (uint32_t)(m * PCL * 16), 0));
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
      const uint32_t off = p_lane + cp + (uint32_t)(((j * PCL + lc) % HP) * ld) * 4u;
      if constexpr (NK == 2) {
        const float2 v2 = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rp, (int)off, 0, 0));
        x.p[j][0] = v2.x;
        x.p[j][1] = v2.y;
      } else {
        x.p[j][0] = buf_load4f(rp, off, 0);
      }
    }
  };
  // probability of head H at the lane's position k: from the lane of its position that loaded it
  auto prob = [&](const Set& x, auto H, int k) -> float {
    constexpr int h = decltype(H)::value;
    const float v = x.p[h / PCL][k];
    if constexpr (PCL == 1) {
      return v;
    } else {
      constexpr int s = h % PCL;  // quad lanes [s,s,s,s] (PCL 4) or [s,s,2+s,2+s] (PCL 2)
      constexpr int ctrl = PCL == 4 ? s * 0x55 : (s | s << 2 | (2 + s) << 4 | (2 + s) << 6);
      return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xf, 0xf, false));
    }
  };
  // product (k, m, i, h) goes to row (h0+h)·DS + (m·PCL + lc)·4 + i, column pos0 + k
  float* const wbase = prod + (h0 * DS + lc * 4) * PVL_ROW + pos0;
  auto make = [&](Set& x, int c) {
    float* const dst = wbase + (c % PVL_NB) * PVL_BUF;
    bool in[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) in[k] = c * PVL_CH + pos0 + k < n;
    unroll_seq(
        [&](auto H) {
          constexpr int h = decltype(H)::value;
          float ph[NK];
#pragma unroll
          for (int k = 0; k < NK; ++k) {
            const float pk = prob(x, H, k);  // (outside the select: the broadcast needs every lane)
            ph[k] = in[k] ? pk : 0.0f;
          }
#pragma unroll
          for (int m = 0; m < NQG; ++m) {
            float* d = dst + (h * DS + m * PCL * 4) * PVL_ROW;
            if constexpr (NK == 2) {
              const float4 v0 = x.v[m], v1 = x.v[NQG + m];
              *reinterpret_cast<float2*>(d + 0 * PVL_ROW) = make_float2(ph[0] * v0.x, ph[1] * v1.x);
              *reinterpret_cast<float2*>(d + 1 * PVL_ROW) = make_float2(ph[0] * v0.y, ph[1] * v1.y);
              *reinterpret_cast<float2*>(d + 2 * PVL_ROW) = make_float2(ph[0] * v0.z, ph[1] * v1.z);
              *reinterpret_cast<float2*>(d + 3 * PVL_ROW) = make_float2(ph[0] * v0.w, ph[1] * v1.w);
            } else {
              const float4 v0 = x.v[m];
              d[0 * PVL_ROW] = ph[0] * v0.x;
              d[1 * PVL_ROW] = ph[0] * v0.y;
              d[2 * PVL_ROW] = ph[0] * v0.z;
              d[3 * PVL_ROW] = ph[0] * v0.w;
            }
          }
        },
        std::make_integer_sequence<int, HP>{});
  };
  // every step loads, also chunks past the row (through the buffers' range checks; never made):
  // with a load skipped on some path the compiler could only wait for every load in flight
  Set ring[D];
  // (in ring order: the steady state's waits count on set u's loads being older than set u+1's)
  // (the scheduling barriers keep each set's loads in ring order: empty asm statements do not
  // order buffer loads)
  unroll_seq(
      [&](auto U) {
        load(ring[decltype(U)::value], decltype(U)::value);
        __builtin_amdgcn_sched_barrier(0);
      },
      std::make_integer_sequence<int, D>{});
  for (int k0 = 0; k0 < nsteps - 1; k0 += D) {
    unroll_seq(
        [&](auto U) {
          constexpr int u = decltype(U)::value;
          const int k = k0 + u;
          if (k < nch) make(ring[u], k);
          __builtin_amdgcn_sched_barrier(0);
          load(ring[u], k + D);
          __builtin_amdgcn_sched_barrier(0);
          if (k < nsteps - 1) lds_barrier();
        },
        std::make_integer_sequence<int, D>{});
  }
}

hipError_t launch_attn_scores(hipStream_t s, const float* q, const float* kc, int n0, int T, int n_heads, int n_kv,
                              int hd, float scale, float* scores) {
  const int ld = n0 + T;
  if (hd == AT_HD && n_heads / n_kv <= AT_ITEMS) {
    const int TT = at_tokens(n_heads / n_kv);
    BB_LAUNCH(k_attn_scores_tile, dim3((unsigned)((ld + 63) / 64), n_kv, (unsigned)((T + TT - 1) / TT)), dim3(256), 0,
              s, q, kc, n0, T, n_heads, n_kv, scale, scores, ld);
    return hipGetLastError();
  }
  const size_t lds = (size_t)(n_heads / n_kv) * hd * sizeof(float);
  const dim3 grid((unsigned)((ld + 63) / 64), n_kv, T);
  if (hd % 4 == 0)
    BB_LAUNCH(k_attn_scores_gqa<true>, grid, dim3(64), lds, s, q, kc, n0, n_heads, n_kv, hd, scale, scores, ld);
  else
    BB_LAUNCH(k_attn_scores_gqa<false>, grid, dim3(64), lds, s, q, kc, n0, n_heads, n_kv, hd, scale, scores, ld);
  return hipGetLastError();
}

hipError_t launch_attn_pv(hipStream_t s, float* scores, const float* vc, int n0, int T, int n_heads, int n_kv, int hd,
                          float* out) {
  const int ld = n0 + T;
  if (T >= AT_PV_MIN_T && hd == AT_HD && n_heads / n_kv <= AT_PV_ITEMS) {
    // a batch: every row's softmax, then P·V in tiles of (tokens x heads of one kv head)
    if (ld <= OPS_ROW_LDS)
      BB_LAUNCH(k_attn_softmax<true>, dim3(n_heads, T), dim3(64 * SM_WAVES), (size_t)ld * 4, s, scores, n0, n_heads, ld);
    else
      BB_LAUNCH(k_attn_softmax<false>, dim3(n_heads, T), dim3(64 * SM_WAVES), 0, s, scores, n0, n_heads, ld);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int TT = at_tokens(n_heads / n_kv, AT_PV_ITEMS);
    BB_LAUNCH(k_attn_pv_tile, dim3(n_kv, (unsigned)((T + TT - 1) / TT)), dim3(256), 0, s, scores, vc, n0, T, n_heads,
              n_kv, ld, out);
    return hipGetLastError();
  }
  const int G = n_heads / n_kv;
  if (hd == AT_HD && ld >= PVL_MIN_LD && (G == 1 || G == 2 || G == 4 || G == 8 || G == 16)) {
    // long rows: the softmax, then P·V with the values streamed through LDS (k_attn_pv_long)
    if (ld <= OPS_ROW_LDS)
      BB_LAUNCH(k_attn_softmax<true>, dim3(n_heads, T), dim3(64 * SM_WAVES), (size_t)ld * 4, s, scores, n0, n_heads, ld);
    else
      BB_LAUNCH(k_attn_softmax<false>, dim3(n_heads, T), dim3(64 * SM_WAVES), 0, s, scores, n0, n_heads, ld);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 grid(n_kv, G, T);
    auto blk = [](int np) { return dim3(64 * (1 + np)); };  // the chain wave and the producers
    switch (G) {
      case 1: BB_LAUNCH(k_attn_pv_long<1>, grid, blk(PvlCfg<1>::NP), 0, s, scores, vc, n0, n_heads, n_kv, ld, out); break;
      case 2: BB_LAUNCH(k_attn_pv_long<2>, grid, blk(PvlCfg<2>::NP), 0, s, scores, vc, n0, n_heads, n_kv, ld, out); break;
      case 4: BB_LAUNCH(k_attn_pv_long<4>, grid, blk(PvlCfg<4>::NP), 0, s, scores, vc, n0, n_heads, n_kv, ld, out); break;
      case 8: BB_LAUNCH(k_attn_pv_long<8>, grid, blk(PvlCfg<8>::NP), 0, s, scores, vc, n0, n_heads, n_kv, ld, out); break;
      default:
        BB_LAUNCH(k_attn_pv_long<16>, grid, blk(PvlCfg<16>::NP), 0, s, scores, vc, n0, n_heads, n_kv, ld, out);
        break;
    }
    return hipGetLastError();
  }
  if (ld <= OPS_ROW_LDS)
    BB_LAUNCH(k_attn_softmax_pv<true>, dim3(n_heads, T), dim3(64), (size_t)ld * 4, s, scores, vc, n0, n_heads, n_kv, hd,
              ld, out);
  else
    BB_LAUNCH(k_attn_softmax_pv<false>, dim3(n_heads, T), dim3(64), 0, s, scores, vc, n0, n_heads, n_kv, hd, ld, out);
  return hipGetLastError();
}

// softmax of n_vec rows of n (kernels/softmax.rs:9-22), SM_WAVES waves per row (through LDS when
// the row fits).
template <bool LDS>
__global__ void __launch_bounds__(64 * SM_WAVES) k_softmax(float* x, int n) {
  extern __shared__ float lrow[];
  __shared__ uint64_t exptab[32];
  __shared__ float s_inv;
  if (threadIdx.x < 32) exptab[threadIdx.x] = exp_table_entry();
  float* g = x + (size_t)blockIdx.x * n;
  if constexpr (LDS)
    row_to_lds<SM_WAVES>(g, lrow, n);
  __syncthreads();
  row_softmax<LDS, SM_WAVES>(Row<LDS>{LDS ? lrow : g}, n, exptab, &s_inv);
  if constexpr (LDS)
    for (int j = threadIdx.x; j < n; j += 64 * SM_WAVES) g[j] = lrow[j];
}

hipError_t launch_softmax(hipStream_t s, float* x, size_t n, size_t n_vec) {
  if (n == 0 || n_vec == 0) return hipSuccess;
  const dim3 block(64 * SM_WAVES);
  if (n <= (size_t)OPS_ROW_LDS) BB_LAUNCH(k_softmax<true>, dim3((unsigned)n_vec), block, n * 4, s, x, (int)n);
  else BB_LAUNCH(k_softmax<false>, dim3((unsigned)n_vec), block, 0, s, x, (int)n);
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
