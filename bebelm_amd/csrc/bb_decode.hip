// bb_decode.hip — the MoE block for decode / small batches (T·k <= 1024 entries).
//
// Four kernels; no block ever waits on another inside a kernel (on gfx950 an agent-scope
// fence writes back and invalidates the whole L2), so kernel boundaries are the only hand-offs:
//   k_route         router logits, gating (sigmoid, top-k, renormalisation) and the XQ record
//                   of x, one block per token                                     (model.rs:484-501)
//   k_gateup        gate and up rows of one expert, SwiGLU, for the entries that selected
//                   the expert                                                     (model.rs:504-524)
//   k_down          Q8 of the expert's act rows, then its down rows               (model.rs:529-548)
//   k_combine       out[t] = Σ_k w[t,k]·down[t,k] in selection order              (model.rs:550-553)
// The GEMV kernels run one weight row per lane: each of the 8 waves of a block owns one
// 256-weight super-block of the tile's 64 rows, computes its exact value for every member,
// and lanes sum the per-block values left to right through LDS. Blocks walk several tiles of
// one expert with the next tile's weights in flight, so HBM streams while the SIMDs compute.
#include "bb_internal.h"
#include "bb_rowlane.h"

namespace bb {

// ---- router + gating + XQ of x, one block per token -------------------------------------------
// Block t (1024 threads): lane (e = tid/32, c = tid%32) runs fmaf chain c of router row e
// (matmul.rs:36-66: chains i = c mod 32, lane combine (acc0+acc1)+(acc2+acc3), reduce_add
// ((v0+v4)+(v2+v6))+((v1+v5)+(v3+v7))). The router is held chain-major (Wc[e][c][m] =
// W[e][32m+c], built once per layer) so each lane reads its chain as contiguous float4s; x is
// staged in LDS. Then one half-wave does the gating of model.rs:485-495 (sigmoid, rank of
// score+bias by total_cmp with lower index first on exact ties, renormalisation), and waves
// quantise x into its XQ record (model.rs:501).
__global__ void __launch_bounds__(1024) k_route(const float* __restrict__ Wc, const float* __restrict__ bias,
                                                const float* __restrict__ x, int H, int E, int K, XQBufs xq,
                                                RouteBufs rb) {
  __shared__ __align__(16) float xs[GU_H_MAX];
  __shared__ float lg[32];
  __shared__ int32_t s_key[32];
  __shared__ float s_rank_s[8];
  __shared__ int32_t s_rank_e[8];
  __shared__ float s_rank_key[9];
  const int t = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e = tid >> 5, c = tid & 31;
  const int nm = H / 32;
  // issue this lane's chain operands first; they are independent of everything below
  float4 wv[GU_H_MAX / 32 / 4];
  const float4* wr = reinterpret_cast<const float4*>(Wc + ((size_t)(e < E ? e : 0) * 32 + c) * nm);
#pragma unroll
  for (int k = 0; k < GU_H_MAX / 32 / 4; ++k)
    if (k < nm / 4) wv[k] = wr[k];
  const float* xr = x + (size_t)t * H;
  for (int i = tid; i < H / 4; i += 1024) reinterpret_cast<float4*>(xs)[i] = reinterpret_cast<const float4*>(xr)[i];
  __syncthreads();
  const int nbx = H / QK;
  if (wave < nbx) {
    const float4 v = reinterpret_cast<const float4*>(xs + wave * QK)[lane];
    wave_quantize_xq(v, xq.q + (size_t)t * H + wave * QK, xq.sx + (size_t)t * nbx + wave,
                     xq.pairs + ((size_t)t * nbx + wave) * 12);
  }
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < GU_H_MAX / 32 / 4; ++k) {
    if (k < nm / 4) {
      acc = fmaf(wv[k].x, xs[32 * (4 * k + 0) + c], acc);
      acc = fmaf(wv[k].y, xs[32 * (4 * k + 1) + c], acc);
      acc = fmaf(wv[k].z, xs[32 * (4 * k + 2) + c], acc);
      acc = fmaf(wv[k].w, xs[32 * (4 * k + 3) + c], acc);
    }
  }
  const float A = acc + __shfl_down(acc, 8, 32);
  const float v = A + __shfl_down(A, 16, 32);
  const float u = v + __shfl_down(v, 4, 32);
  const float y = u + __shfl_down(u, 2, 32);
  const float r = y + __shfl_down(y, 1, 32);
  if (c == 0 && e < E) {
    lg[e] = r;
    rb.logits[(size_t)t * E + e] = r;
  }
  __syncthreads();
  if (tid < 32) {
    const bool live = c < E;
    const float s = live ? sigmoid(lg[c]) : 0.0f;
    const float key = live ? s + bias[c] : 0.0f;
    const int32_t kk = total_key(key);
    if (live) s_key[c] = kk;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    int rank = 0, eq_after = 0;
    if (live) {
      for (int j = 0; j < E; ++j) {
        const int32_t kj = s_key[j];
        rank += (kj > kk) || (kj == kk && j < c);
        eq_after += (kj == kk && j > c);
      }
    }
    if (live && rank < K) {
      s_rank_s[rank] = s;
      s_rank_e[rank] = c;
    }
    if (live && rank <= K) s_rank_key[rank] = key;
    const int tie = (live && rank < K && eq_after > 0) ? 1 : 0;
    const unsigned long long tm = __ballot(tie);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if (c == 0) {
      float denom = -0.0f;
      for (int k = 0; k < K; ++k) denom += s_rank_s[k];
      denom = denom + 1e-6f;
      for (int k = 0; k < K; ++k) {
        rb.sel[(size_t)t * K + k] = s_rank_e[k];
        rb.wts[(size_t)t * K + k] = s_rank_s[k] / denom;
      }
      rb.margin[t] = K < E ? s_rank_key[K - 1] - s_rank_key[K] : __builtin_inff();
      rb.ties[t] = __popcll(tm);
    }
  }
}

// Wc[e][c][m] = W[e][32m + c]: the router rows regrouped by dot chain (layout only).
__global__ void k_router_chain_major(const float* __restrict__ W, int H, int E, float* __restrict__ Wc) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)E * H) return;
  const size_t e = i / H, r = i % H, c = r % 32, m = r / 32;
  Wc[(e * 32 + c) * (H / 32) + m] = W[i];
}

hipError_t launch_router_chain_major(hipStream_t s, const float* W, int H, int E, float* Wc) {
  hipLaunchKernelGGL(k_router_chain_major, dim3((unsigned)(((size_t)E * H + 255) / 256)), dim3(256), 0, s, W, H, E, Wc);
  return hipGetLastError();
}

hipError_t launch_route(hipStream_t s, const float* router, const float* bias, const float* x, int T, int H, int E,
                        int K, XQBufs xq, RouteBufs rb) {
  hipLaunchKernelGGL(k_route, dim3(T), dim3(1024), 0, s, router, bias, x, H, E, K, xq, rb);
  return hipGetLastError();
}

// The u-th expert (ascending id) that some entry selected, and its members: the entries
// i (= token*K + slot) with sel[i] == e, ascending — the order model.rs:317-322 groups them in.
// One ballot per 64 entries and a prefix over the per-chunk counts. Returns the member count
// (0 when fewer than u+1 experts were selected); uniform across the block.
struct SmemMembers {
  int32_t list[MAX_ENTRIES];
  int32_t chunk[MAX_ENTRIES / 64 + 1];
  uint32_t mask;
  int32_t e;
};

__device__ int members_of(const int32_t* __restrict__ sel, int n_ent, int u, SmemMembers& sm) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int n_chunks = (n_ent + 63) >> 6;
  constexpr int KMAX = MAX_ENTRIES / 64 / 8 + 1;
  int sv[KMAX];
  uint32_t present = 0;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int i = (wave + k * nw) * 64 + lane;
    sv[k] = i < n_ent ? sel[i] : -1;
    if (sv[k] >= 0) present |= 1u << sv[k];
  }
  if (tid == 0) sm.mask = 0;
  __syncthreads();
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) present |= (uint32_t)__shfl_xor((int)present, o);
  if (lane == 0) atomicOr(&sm.mask, present);
  __syncthreads();
  uint32_t mask = sm.mask;
  for (int k = 0; k < u && mask; ++k) mask &= mask - 1;  // drop the u lowest experts
  const int e = mask ? __builtin_ctz(mask) : -1;
  if (e < 0) return 0;
  unsigned long long masks[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int ch = wave + k * nw;
    masks[k] = __ballot(sv[k] == e);
    if (ch < n_chunks && lane == 0) sm.chunk[ch] = __popcll(masks[k]);
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int ch = 0; ch < n_chunks; ++ch) {
      const int v = sm.chunk[ch];
      sm.chunk[ch] = acc;
      acc += v;
    }
    sm.chunk[n_chunks] = acc;
    sm.e = e;
  }
  __syncthreads();
  const unsigned long long lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int ch = wave + k * nw;
    if (ch < n_chunks && ((masks[k] >> lane) & 1ull)) sm.list[sm.chunk[ch] + __popcll(masks[k] & lt)] = ch * 64 + lane;
  }
  const int cnt = sm.chunk[n_chunks];
  __syncthreads();
  return cnt;
}

// The dispatch of model.rs:316-322 for the route trace (counts, offsets, grouped entries).
__device__ void publish_dispatch(const int32_t* __restrict__ sel, int n_ent, int E, RouteBufs rb) {
  __shared__ int32_t cnt[32];
  const int tid = threadIdx.x;
  if (tid < 32) cnt[tid] = 0;
  __syncthreads();
  for (int i = tid; i < n_ent; i += blockDim.x) atomicAdd(&cnt[sel[i]], 1);
  __syncthreads();
  if (tid == 0) {
    int acc = 0, nh = 0;
    rb.offsets[0] = 0;
    for (int e = 0; e < E; ++e) {
      rb.counts[e] = cnt[e];
      if (cnt[e]) rb.hit[1 + nh++] = e;
      acc += cnt[e];
      rb.offsets[e + 1] = acc;
    }
    rb.hit[0] = nh;
  }
  __syncthreads();
  for (int i = tid; i < n_ent; i += blockDim.x) {
    const int e = sel[i];
    int off = 0, rank = 0;
    for (int x = 0; x < e; ++x) off += cnt[x];
    for (int j = 0; j < i; ++j) rank += sel[j] == e;
    rb.perm[off + rank] = i;
  }
}

// XQ records of up to MCH members in LDS.
struct SmemXQ {
  int8_t q[MCH][GU_H_MAX];
  uint32_t pairs[MCH][GU_H_MAX / QK][12];
  float sx[MCH][GU_H_MAX / QK];
};

// Per-(member, block, row) values waiting for the left-to-right block sum.
struct SmemT {
  float v[MCH][GU_H_MAX / QK][64];
};

// Stages the XQ records of members [c0, c0+cnt) into LDS; row_of(m) is the record index.
template <class RowOf>
__device__ __forceinline__ void stage_xq(SmemXQ& xs, XQBufs src, int n, int cnt, RowOf row_of) {
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int nq16 = n / 16, nb = n / QK;
  for (int idx = tid; idx < cnt * nq16; idx += nthr) {
    const int m = idx / nq16, k = idx % nq16;
    reinterpret_cast<uint4*>(xs.q[m])[k] = reinterpret_cast<const uint4*>(src.q + row_of(m) * n)[k];
  }
  for (int idx = tid; idx < cnt * nb * 12; idx += nthr) {
    const int m = idx / (nb * 12), k = idx % (nb * 12);
    xs.pairs[m][k / 12][k % 12] = src.pairs[row_of(m) * nb * 12 + k];
  }
  for (int idx = tid; idx < cnt * nb; idx += nthr) {
    const int m = idx / nb, k = idx % nb;
    xs.sx[m][k] = src.sx[row_of(m) * nb + k];
  }
}

// ---- gate/up + SwiGLU --------------------------------------------------------------------------
// Block (g, u): tiles g*ntile .. of hit expert u; a tile is 32 outputs, lanes 0-31 holding the
// gate rows and lanes 32-63 the up rows of the same outputs; wave w owns super-block w of all
// 64 rows. The next tile's weights are in flight while the current one is computed; the
// members' x records are staged once per block.
template <int DT>
__global__ void __launch_bounds__(512) k_gateup(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
                                                size_t stride_g, size_t stride_u, int T, int H, int F, int K,
                                                int batch_mode, int ntile, int publish, int E, RouteBufs rb, XQBufs xq,
                                                float* __restrict__ act) {
  using R = LaneRow<DT>;
  __shared__ SmemMembers mem;
  __shared__ __align__(16) SmemXQ xs;
  __shared__ SmemT tv;
  const int n_ent = T * K;
  if (publish && blockIdx.x == 0 && blockIdx.y == 0) publish_dispatch(rb.sel, n_ent, E, rb);
  const int n_mem = members_of(rb.sel, n_ent, blockIdx.y, mem);
  if (n_mem == 0) return;
  const int e = mem.e;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nb = H / QK;
  const int tile0 = blockIdx.x * ntile, tile1 = min(tile0 + ntile, F / 32);
  const size_t row_bytes = (size_t)nb * R::BLOCK_BYTES;
  const uint8_t* base = lane < 32 ? gate + (size_t)e * stride_g + (size_t)lane * row_bytes
                                  : up + (size_t)e * stride_u + (size_t)(lane - 32) * row_bytes;
  base += (size_t)w * R::BLOCK_BYTES;
  const bool has_blk = w < nb;
  const float start = (batch_mode && n_mem > 1) ? 0.0f : -0.0f;
  typename R::Loaded cur, nxt;
  if (has_blk) R::load(cur, base + (size_t)tile0 * 32 * row_bytes);
  const int n_chunks = (n_mem + MCH - 1) / MCH;
  for (int tile = tile0; tile < tile1; ++tile) {
    if (has_blk && tile + 1 < tile1) R::load(nxt, base + (size_t)(tile + 1) * 32 * row_bytes);
    typename R::Blk B;
    if (has_blk) R::prep(B, cur);
    for (int ch = 0; ch < n_chunks; ++ch) {
      const int c0 = ch * MCH, cnt = min(n_mem - c0, MCH);
      if (tile == tile0 || n_chunks > 1) {
        stage_xq(xs, xq, H, cnt, [&](int m) { return (size_t)(mem.list[c0 + m] / K); });
        __syncthreads();
      }
      if (has_blk)
        for (int m = 0; m < cnt; ++m) tv.v[m][w][lane] = R::value(B, xs.q[m] + w * QK, xs.pairs[m][w], xs.sx[m][w]);
      __syncthreads();
      for (int m = w; m < cnt; m += 8) {
        float acc = start;
        for (int b = 0; b < nb; ++b) acc += tv.v[m][b][lane];
        const float upv = __shfl(acc, (lane + 32) & 63);
        if (lane < 32) act[(size_t)mem.list[c0 + m] * F + tile * 32 + lane] = silu(acc) * upv;
      }
      __syncthreads();
    }
    if (has_blk) cur = nxt;
  }
}

hipError_t launch_gateup(hipStream_t s, int dtype, const uint8_t* gate, const uint8_t* up, size_t stride_g,
                         size_t stride_u, int T, int H, int F, int E, int K, int max_hit, int batch_mode, int publish,
                         const RouteBufs& rb, XQBufs xq, float* act) {
  const int tiles = F / 32;
  const int ntile = max(1, (tiles * max_hit + GEMV_BLOCKS - 1) / GEMV_BLOCKS);
  dim3 grid((tiles + ntile - 1) / ntile, max_hit);
  if (dtype == DT_Q4_K)
    hipLaunchKernelGGL(k_gateup<DT_Q4_K>, grid, dim3(512), 0, s, gate, up, stride_g, stride_u, T, H, F, K, batch_mode,
                       ntile, publish, E, rb, xq, act);
  else
    hipLaunchKernelGGL(k_gateup<DT_Q6_K>, grid, dim3(512), 0, s, gate, up, stride_g, stride_u, T, H, F, K, batch_mode,
                       ntile, publish, E, rb, xq, act);
  return hipGetLastError();
}

// ---- down --------------------------------------------------------------------------------------
// Block (g, u): 64-row tiles g*ntile .. of hit expert u. The prologue quantises the members'
// act rows (quantize_q8 per member, model.rs:530-534) straight into LDS.
template <int DT>
__global__ void __launch_bounds__(512) k_down(const uint8_t* __restrict__ down, size_t stride_d, int T, int H, int F,
                                              int K, int batch_mode, int ntile, RouteBufs rb,
                                              const float* __restrict__ act, float* __restrict__ slots) {
  using R = LaneRow<DT>;
  __shared__ SmemMembers mem;
  __shared__ __align__(16) SmemXQ xs;
  __shared__ SmemT tv;
  const int n_mem = members_of(rb.sel, T * K, blockIdx.y, mem);
  if (n_mem == 0) return;
  const int e = mem.e;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nb = F / QK;
  const int tile0 = blockIdx.x * ntile, tile1 = min(tile0 + ntile, H / 64);
  const size_t row_bytes = (size_t)nb * R::BLOCK_BYTES;
  const uint8_t* base = down + (size_t)e * stride_d + (size_t)lane * row_bytes + (size_t)w * R::BLOCK_BYTES;
  const bool has_blk = w < nb;
  const float start = (batch_mode && n_mem > 1) ? 0.0f : -0.0f;
  typename R::Loaded cur, nxt;
  if (has_blk) R::load(cur, base + (size_t)tile0 * 64 * row_bytes);
  const int n_chunks = (n_mem + MCH - 1) / MCH;
  for (int tile = tile0; tile < tile1; ++tile) {
    if (has_blk && tile + 1 < tile1) R::load(nxt, base + (size_t)(tile + 1) * 64 * row_bytes);
    typename R::Blk B;
    if (has_blk) R::prep(B, cur);
    for (int ch = 0; ch < n_chunks; ++ch) {
      const int c0 = ch * MCH, cnt = min(n_mem - c0, MCH);
      if (tile == tile0 || n_chunks > 1) {
        for (int task = w; task < cnt * nb; task += 8) {
          const int m = task / nb, b = task % nb;
          const float4 v = *reinterpret_cast<const float4*>(act + (size_t)mem.list[c0 + m] * F + b * QK + 4 * lane);
          wave_quantize_xq(v, xs.q[m] + b * QK, &xs.sx[m][b], xs.pairs[m][b]);
        }
        __syncthreads();
      }
      if (has_blk)
        for (int m = 0; m < cnt; ++m) tv.v[m][w][lane] = R::value(B, xs.q[m] + w * QK, xs.pairs[m][w], xs.sx[m][w]);
      __syncthreads();
      for (int m = w; m < cnt; m += 8) {
        float acc = start;
        for (int b = 0; b < nb; ++b) acc += tv.v[m][b][lane];
        slots[(size_t)mem.list[c0 + m] * H + tile * 64 + lane] = acc;
      }
      __syncthreads();
    }
    if (has_blk) cur = nxt;
  }
}

hipError_t launch_down(hipStream_t s, int dtype, const uint8_t* down, size_t stride_d, int T, int H, int F, int K,
                       int max_hit, int batch_mode, const RouteBufs& rb, const float* act, float* slots) {
  const int tiles = H / 64;
  const int ntile = max(1, (tiles * max_hit + GEMV_BLOCKS - 1) / GEMV_BLOCKS);
  dim3 grid((tiles + ntile - 1) / ntile, max_hit);
  if (dtype == DT_Q4_K)
    hipLaunchKernelGGL(k_down<DT_Q4_K>, grid, dim3(512), 0, s, down, stride_d, T, H, F, K, batch_mode, ntile, rb, act,
                       slots);
  else
    hipLaunchKernelGGL(k_down<DT_Q6_K>, grid, dim3(512), 0, s, down, stride_d, T, H, F, K, batch_mode, ntile, rb, act,
                       slots);
  return hipGetLastError();
}

// ---- combine -----------------------------------------------------------------------------------
// out[t][o] = Σ_k w[t,k]·slots[t*K+k][o], k ascending from +0.0 (add_scaled, elementwise.rs:12).
__global__ void __launch_bounds__(256) k_combine(const float* __restrict__ slots, const float* __restrict__ wts, int T,
                                                 int H, int K, float* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)T * H) return;
  const size_t t = i / H, o = i % H;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) acc = acc + wts[t * K + k] * slots[(t * K + k) * H + o];
  out[i] = acc;
}

hipError_t launch_combine(hipStream_t s, const float* slots, const float* wts, int T, int H, int K, float* out) {
  hipLaunchKernelGGL(k_combine, dim3((unsigned)(((size_t)T * H + 255) / 256)), dim3(256), 0, s, slots, wts, T, H, K,
                     out);
  return hipGetLastError();
}

}  // namespace bb
