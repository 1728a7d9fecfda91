// bb_prefill.hip — the batched MoE path for many tokens (Model::moe_ffn_batch, model.rs:286-371).
//
//   k_dispatch      counts, offsets and the stable grouping of (token, slot) entries by
//                   expert — token-ascending, slot-ascending within an expert (model.rs:316-322)
//   k_gemm_q4/q6    grouped expert GEMM on int8 MFMA: gate/up + SwiGLU (model.rs:325-334),
//                   down (model.rs:335-341)
//   k_quant_rows    Q8 of the act rows (quantize_q8, kernels/matmul.rs:141-160)
//
// Exactness. Each output is matmul's row dot (kernels/matmul.rs:211-300 Q4_K, :648-760 Q6_K):
// per 256-block an exact int32 integer part, then the f32 epilogue
//   Q4_K  v = sx·(d·(float)sd − dmin·(float)sm)      Q6_K  v = sx·(d·(float)s)
// summed over blocks left to right from +0.0 (−0.0 when the expert has one member, where
// matmul delegates to matvec). The MFMA produces the integer parts exactly:
//   Q4_K  sd = Σ_j sc_j·Σ_{k∈j} q_k·x_k. With sc_j = 8·h_j + l_j (h_j, l_j ≤ 7) the weights
//         h_j·q_k and l_j·q_k (≤ 105) fit int8, so two MFMA passes over the whole block give
//         Dh and Dl with sd = 8·Dh + Dl. The min term sm = Σ_j m_j·S_j is a third pass whose
//         weight for element k is m_j (the 6-bit min of its sub-block).
//   Q6_K  s = Σ_j sc_j·Σ_{k∈j} (q_k − 32)·x_k with i8 scales: one MFMA per 16-element
//         sub-block (q − 32 fits int8) and an exact integer multiply-add by sc_j.
// The MFMA runs with the activations as the A operand and the weight rows as the B operand, so
// every output a lane holds belongs to one weight row and the row's scales stay in the lane.
#include "bb_device.h"
#include "bb_internal.h"

namespace bb {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

enum : int { GEMM_GATEUP = 0, GEMM_DOWN = 1 };

constexpr int BN = 64;                 // members per tile
constexpr int PSTRIDE = BN * 8 + 128;  // bytes per row of 8-byte activation pieces in LDS
constexpr size_t TB4 = pack_tile_block_bytes(DT_Q4_K);
constexpr size_t TB6 = pack_tile_block_bytes(DT_Q6_K);

// ---- dispatch ------------------------------------------------------------------------------------
// One block of 1024 threads (16 waves). Per 64-entry chunk and expert a ballot count; an
// exclusive scan over chunks per expert gives each chunk's first group position; an entry's
// position is that plus its rank among the chunk's entries of the same expert.
__global__ void __launch_bounds__(1024) k_dispatch(const int32_t* __restrict__ sel, int n_ent, int E, RouteBufs rb) {
  __shared__ int32_t cc[PF_MAX_ENTRIES / 64][32];
  __shared__ int32_t part[32][33];
  __shared__ int32_t off[33];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_chunks = (n_ent + 63) >> 6;
  for (int ch = wave; ch < n_chunks; ch += 16) {
    const int i = ch * 64 + lane;
    const int v = i < n_ent ? sel[i] : -1;
    int mine = 0;
    for (int x = 0; x < E; ++x) {
      const int c = __popcll(__ballot(v == x));
      if (lane == x) mine = c;
    }
    if (lane < 32) cc[ch][lane] = mine;
  }
  if (tid < 33) off[tid] = 0;
  __syncthreads();
  const int e = tid & 31, p = tid >> 5;  // 32 parts of the chunk range per expert
  const int cpp = (n_chunks + 31) >> 5;
  const int c0 = min(p * cpp, n_chunks), c1 = min(c0 + cpp, n_chunks);
  int s = 0;
  for (int ch = c0; ch < c1; ++ch) s += cc[ch][e];
  part[e][p] = s;
  __syncthreads();
  if (tid < 32) {
    int acc = 0;
    for (int q = 0; q < 32; ++q) {
      const int v = part[tid][q];
      part[tid][q] = acc;
      acc += v;
    }
    part[tid][32] = acc;
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0, nh = 0;
    for (int x = 0; x < E; ++x) {
      const int c = part[x][32];
      rb.counts[x] = c;
      rb.offsets[x] = acc;
      off[x] = acc;
      if (c) rb.hit[1 + nh++] = x;
      acc += c;
    }
    rb.offsets[E] = acc;
    rb.hit[0] = nh;
  }
  __syncthreads();
  {
    int acc = part[e][p] + off[e];
    for (int ch = c0; ch < c1; ++ch) {
      const int v = cc[ch][e];
      cc[ch][e] = acc;
      acc += v;
    }
  }
  __syncthreads();
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int ch = wave; ch < n_chunks; ch += 16) {
    const int i = ch * 64 + lane;
    const int v = i < n_ent ? sel[i] : -1;
    unsigned long long mb = 0;
    for (int x = 0; x < E; ++x) {
      const unsigned long long b = __ballot(v == x);
      if (v == x) mb = b;
    }
    if (v >= 0) rb.perm[cc[ch][v] + __popcll(mb & lt)] = i;
  }
}

hipError_t launch_dispatch(hipStream_t s, int n_ent, int E, const RouteBufs& rb) {
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, s, rb.sel, n_ent, E, rb);
  return hipGetLastError();
}

// ---- member tiles --------------------------------------------------------------------------------
// Tiles are enumerated expert by expert, BN members each (an expert's last tile partial).
struct TileInfo {
  int e, m0, cnt, base, g;
};

__device__ bool find_tile(const RouteBufs& rb, int E, int tile, TileInfo& ti, int32_t* sh) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int c = lane < E ? rb.counts[lane] : 0;
    const int nt = (c + BN - 1) / BN;
    int incl = nt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    const int excl = incl - nt;
    if (lane < E && tile >= excl && tile < incl) {
      sh[0] = lane;
      sh[1] = (tile - excl) * BN;
      sh[2] = c;
      sh[3] = rb.offsets[lane];
    }
    if (lane == 63) sh[4] = incl;
  }
  __syncthreads();
  if (tile >= sh[4]) return false;
  ti.e = sh[0];
  ti.m0 = sh[1];
  ti.g = sh[2];
  ti.base = sh[3];
  ti.cnt = min(BN, ti.g - ti.m0);
  return true;
}

// Member rows of the tile: x row (the token for gate/up, the group position for down) and
// output row (group position for gate/up, entry for down). Padding members repeat the last
// real one so every load stays inside the inputs; their outputs are not stored.
template <int KIND>
__device__ void member_rows(const RouteBufs& rb, const TileInfo& ti, int K, int32_t* rowidx, int32_t* outrow) {
  const int tid = threadIdx.x;
  if (tid < BN) {
    const int pos = ti.base + ti.m0 + min(tid, ti.cnt - 1);
    const int ent = rb.perm[pos];
    rowidx[tid] = KIND == GEMM_GATEUP ? ent / K : pos;
    outrow[tid] = KIND == GEMM_GATEUP ? pos : ent;
  }
}

// Bytes of q (each <= 15) times s (<= 7), per byte; the products stay below 256.
__device__ __forceinline__ uint32_t mul_bytes(uint32_t q, uint32_t s) {
  const v2u16 a = __builtin_bit_cast(v2u16, q);
  const v2u16 m = {(unsigned short)s, (unsigned short)s};
  return __builtin_bit_cast(uint32_t, a * m);
}

__device__ __forceinline__ long as_long(uint32_t lo, uint32_t hi) {
  return (long)(((unsigned long)hi << 32) | lo);
}

// ---- Q4_K grouped GEMM -----------------------------------------------------------------------------
// Block (member tile of 64, row tile = two 64-row packed tiles), 4 waves. Each wave owns two
// 16-row weight tiles of one packed tile: for gate/up the gate rows and the up rows of the
// same 16 outputs (so the SwiGLU pairs meet in one lane), for down two consecutive 16-row
// tiles. MFMA v_mfma_i32_16x16x32_i8 per 32-element sub-block: A = 16 members x 32
// activations (lane: member l%16, elements 8(l/16)..+7), B = 32 weights x 16 rows (lane: row
// l%16, same elements), D lane l = members 4(l/16)..+3 of row l%16.
//
// Block b's operands are copied from HBM straight into LDS (global_load_lds_dwordx4: lane l's
// 16 bytes land at base + 16l), double-buffered, so block b+1 streams in while block b is
// computed and no registers hold data in flight:
//   weights      the two packed tile-blocks verbatim (2 x 9216 B)
//   activations  member m's 256 quants as 16-byte chunks, chunk c at position c ^ (m%16) of
//                the member's 256-byte row (conflict-free 8-byte reads of a sub-block piece)
//   scales       sx of the 64 members
constexpr int Q4_WBUF = 2 * (int)TB4;
constexpr int XBUF = BN * QK;

template <int KIND>
struct Q4Gemm {
  const uint8_t* w0;  // tile-block 0 of the block's first packed tile
  size_t tile_bytes;  // bytes of one packed tile (all super-blocks)
  GemmX x;
  int n_in;
  const int32_t* rowidx;

  // Issue the copies of super-block b into one buffer set (every wave issues its share).
  __device__ __forceinline__ void issue(int b, uint8_t* wb, uint8_t* xb, float* sb) const {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nb = n_in / QK;
    // weights: 1152 16-byte units, 18 per lane-instruction group
    for (int i = w; i < Q4_WBUF / 1024; i += 4) {
      const int u = i * 64 + lane;
      const int k = u / (int)(TB4 / 16), o = u % (int)(TB4 / 16);
      const uint8_t* src = w0 + (size_t)k * tile_bytes + (size_t)b * TB4 + 16 * o;
      __builtin_amdgcn_global_load_lds(src, wb + i * 1024, 16, 0, 0);
    }
    // activations: 1024 units
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int i = w + 4 * s;
      const int u = i * 64 + lane, m = u >> 4, c = (u & 15) ^ (m & 15);
      const int8_t* src = x.q + (size_t)rowidx[m] * n_in + b * QK + 16 * c;
      __builtin_amdgcn_global_load_lds(src, xb + i * 1024, 16, 0, 0);
    }
    if (w == 0) __builtin_amdgcn_global_load_lds(x.sx + (size_t)rowidx[lane] * nb + b, sb, 4, 0, 0);
  }
};

__device__ __forceinline__ long q4_read_x(const uint8_t* xb, int j, int g, int m) {
  const int c = 2 * j + (g >> 1);
  return *reinterpret_cast<const long*>(xb + m * QK + 16 * (c ^ (m & 15)) + 8 * (g & 1));
}

// One super-block of the wave's 2 x 16 rows against the 64 members, added to acc.
__device__ __forceinline__ void q4_block(const uint8_t* wb, const uint8_t* xb, const float* sb, int t16a, int t16b,
                                         float (&acc)[2][4][4]) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  uint2 qs[2][4];
  uint4 hd[2];
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int row = 16 * (a ? t16b : t16a) + r;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      qs[a][c] = *reinterpret_cast<const uint2*>(wb + 1024 * (1 + 2 * c + (g >> 1)) + 16 * row + 8 * (g & 1));
    hd[a] = *reinterpret_cast<const uint4*>(wb + 16 * row);
  }
  // get_scale_min_k4 (dequant.rs:64-72) four bytes at a time
  uint32_t scw[2][2], mw[2][2];
  float dd[2], dm[2];
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    dd[a] = f16_bits_to_f32(hd[a].x & 0xffff);
    dm[a] = f16_bits_to_f32(hd[a].x >> 16);
    const uint32_t s0 = hd[a].y, s1 = hd[a].z, s2 = hd[a].w;
    scw[a][0] = s0 & 0x3F3F3F3Fu;
    scw[a][1] = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    mw[a][0] = s1 & 0x3F3F3F3Fu;
    mw[a][1] = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
  }
  // sd = 8*Dh + Dl: the high-scale pass accumulates first, is multiplied by 8 in place, and
  // the low-scale pass continues into the same accumulator
  v4i Dsd[2][4], Dm[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) Dsd[a][mt] = Dm[a][mt] = v4i{0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    long Bh[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const uint2 qq = qs[a][j >> 1];
      const uint32_t q0 = (j & 1) ? (qq.x >> 4) & 0x0F0F0F0Fu : qq.x & 0x0F0F0F0Fu;
      const uint32_t q1 = (j & 1) ? (qq.y >> 4) & 0x0F0F0F0Fu : qq.y & 0x0F0F0F0Fu;
      const uint32_t hs = (scw[a][j >> 2] >> (8 * (j & 3) + 3)) & 7u;
      Bh[a] = as_long(mul_bytes(q0, hs), mul_bytes(q1, hs));
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const long ax = q4_read_x(xb, j, g, mt * 16 + r);
#pragma unroll
      for (int a = 0; a < 2; ++a) Dsd[a][mt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, Bh[a], Dsd[a][mt], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep each sub-block's operands short-lived
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) Dsd[a][mt] = Dsd[a][mt] << 3;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    long Bl[2], Bm[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const uint2 qq = qs[a][j >> 1];
      const uint32_t q0 = (j & 1) ? (qq.x >> 4) & 0x0F0F0F0Fu : qq.x & 0x0F0F0F0Fu;
      const uint32_t q1 = (j & 1) ? (qq.y >> 4) & 0x0F0F0F0Fu : qq.y & 0x0F0F0F0Fu;
      const uint32_t ls = (scw[a][j >> 2] >> (8 * (j & 3))) & 7u;
      Bl[a] = as_long(mul_bytes(q0, ls), mul_bytes(q1, ls));
      const uint32_t ms = ((mw[a][j >> 2] >> (8 * (j & 3))) & 0xffu) * 0x01010101u;
      Bm[a] = as_long(ms, ms);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const long ax = q4_read_x(xb, j, g, mt * 16 + r);
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        Dsd[a][mt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, Bl[a], Dsd[a][mt], 0, 0, 0);
        Dm[a][mt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, Bm[a], Dm[a][mt], 0, 0, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // matmul.rs:242 epilogue, in the reference's order of f32 operations
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const float4 sx4 = *reinterpret_cast<const float4*>(sb + mt * 16 + 4 * g);
    const float sxv[4] = {sx4.x, sx4.y, sx4.z, sx4.w};
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = sxv[i] * ((dd[a] * (float)Dsd[a][mt][i]) - (dm[a] * (float)Dm[a][mt][i]));
        acc[a][mt][i] += v;
      }
  }
}

template <int KIND>
__global__ void __launch_bounds__(256, 2) k_gemm_q4(const uint8_t* __restrict__ wpk, size_t stride_e, int n_in,
                                                    int n_t64, int K, int n_out, int E, RouteBufs rb, GemmX x,
                                                    float* __restrict__ out) {
  __shared__ __align__(16) uint8_t wb0[Q4_WBUF], wb1[Q4_WBUF];
  __shared__ __align__(16) uint8_t xb0[XBUF], xb1[XBUF];
  __shared__ __align__(16) float sb0[BN], sb1[BN];
  __shared__ int32_t rowidx[BN], outrow[BN];
  __shared__ int32_t sh[8];
  TileInfo ti;
  if (!find_tile(rb, E, blockIdx.x, ti, sh)) return;
  member_rows<KIND>(rb, ti, K, rowidx, outrow);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, g = lane >> 4;
  const int nb = n_in / QK;
  const int t64 = 2 * blockIdx.y + (w >> 1);  // n_t64 is even: both packed tiles exist
  const int t16a = KIND == GEMM_GATEUP ? (w & 1) : 2 * (w & 1);
  const int t16b = KIND == GEMM_GATEUP ? (w & 1) + 2 : 2 * (w & 1) + 1;
  const size_t tile_bytes = (size_t)nb * TB4;
  Q4Gemm<KIND> G{wpk + (size_t)ti.e * stride_e + (size_t)(2 * blockIdx.y) * tile_bytes, tile_bytes, x, n_in, rowidx};
  const float start = ti.g > 1 ? 0.0f : -0.0f;
  float acc[2][4][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[a][mt][i] = start;
  __syncthreads();  // rowidx
  G.issue(0, wb0, xb0, sb0);
  const int wo = (w >> 1) * (int)TB4;  // this wave's packed tile inside a weight buffer
  for (int b = 0; b < nb; b += 2) {
    __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): this wave's copies into buffer 0 landed
    __syncthreads();
    if (b + 1 < nb) G.issue(b + 1, wb1, xb1, sb1);
    q4_block(wb0 + wo, xb0, sb0, t16a, t16b, acc);
    if (b + 1 >= nb) break;
    __builtin_amdgcn_s_waitcnt(0x3f70);
    __syncthreads();
    if (b + 2 < nb) G.issue(b + 2, wb0, xb0, sb0);
    q4_block(wb1 + wo, xb1, sb1, t16a, t16b, acc);
  }
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = mt * 16 + 4 * g + i;
      if (n >= ti.cnt) continue;
      if constexpr (KIND == GEMM_GATEUP) {
        const int o = 32 * t64 + 16 * (w & 1) + r;
        out[(size_t)outrow[n] * n_out + o] = silu(acc[0][mt][i]) * acc[1][mt][i];
      } else {
        out[(size_t)outrow[n] * n_out + 64 * t64 + 16 * t16a + r] = acc[0][mt][i];
        out[(size_t)outrow[n] * n_out + 64 * t64 + 16 * t16b + r] = acc[1][mt][i];
      }
    }
  (void)n_t64;
}

// ---- Q6_K grouped GEMM -----------------------------------------------------------------------------
// Block (member tile of 64, row tile = two 64-row packed tiles), 4 waves; operands copied
// into LDS as for Q4_K (weights verbatim, 2 x 13440 B). v_mfma_i32_32x32x16_i8 per 16-element
// sub-block: A = 32 members x 16 activations (lane: member l%32, elements 8(l/32)..+7),
// B = 16 weights x 32 rows (lane: row l%32), D lane l = members 8(i/4) + 4(l/32) + i%4
// (i = 0..15) of row l%32, so the row's i8 scale multiplies all 16 values in the lane.
//   down:    wave w owns the 32-row half (w&1) of packed tile (w>>1), all 64 members
//   gate/up: wave w owns packed tile (w>>1) — its gate half and its up half, the 32 outputs'
//            SwiGLU pairs — for the 32 members of half (w&1)
constexpr int Q6_WBUF = 2 * (int)TB6;

__device__ __forceinline__ void q6_issue(const uint8_t* w0, size_t tile_bytes, GemmX x, int n_in, int b,
                                         const int32_t* rowidx, uint8_t* wb, uint8_t* xb, float* sb) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nb = n_in / QK;
  constexpr int units = Q6_WBUF / 16, per_tile = (int)(TB6 / 16);
  for (int i = w; i < (units + 63) / 64; i += 4) {
    const int u = i * 64 + lane;
    if (u < units) {
      const int k = u / per_tile, o = u % per_tile;
      __builtin_amdgcn_global_load_lds(w0 + (size_t)k * tile_bytes + (size_t)b * TB6 + 16 * o, wb + i * 1024, 16, 0, 0);
    }
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int i = w + 4 * s;
    const int u = i * 64 + lane, m = u >> 4, c = (u & 15) ^ (m & 15);
    __builtin_amdgcn_global_load_lds(x.q + (size_t)rowidx[m] * n_in + b * QK + 16 * c, xb + i * 1024, 16, 0, 0);
  }
  if (w == 0) __builtin_amdgcn_global_load_lds(x.sx + (size_t)rowidx[lane] * nb + b, sb, 4, 0, 0);
}

// One super-block: NT 32-row weight tiles (rows 32*half[a] + l%32 of packed tile wt) against
// MT groups of 32 members starting at member m0.
template <int NT, int MT>
__device__ __forceinline__ void q6_block(const uint8_t* wt, const uint8_t* xb, const float* sb, const int (&half)[NT],
                                         int m0, float (&acc)[NT][MT][16]) {
  const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
  uint2 ql[NT][8], qh[NT][4];
  uint4 sc[NT];
  float dd[NT];
#pragma unroll
  for (int a = 0; a < NT; ++a) {
    const int row = 32 * half[a] + r;
#pragma unroll
    for (int k = 0; k < 8; ++k) ql[a][k] = *reinterpret_cast<const uint2*>(wt + 1024 * k + 16 * row + 8 * h);
#pragma unroll
    for (int k = 0; k < 4; ++k) qh[a][k] = *reinterpret_cast<const uint2*>(wt + 1024 * (8 + k) + 16 * row + 8 * h);
    sc[a] = *reinterpret_cast<const uint4*>(wt + 1024 * 12 + 16 * row);
    dd[a] = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(wt + 1024 * 13 + 2 * row));
  }
  int S[NT][MT][16];
#pragma unroll
  for (int a = 0; a < NT; ++a)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) S[a][mt][i] = 0;
  // sub-block j = elements 16j..16j+15 = 128n + 32gq + 16m + (0..15), n = j/8, gq = (j/2)%4,
  // m = j%2: low nibbles of ql[64n + 32(gq&1) + 16m + ..] (high nibbles for gq >= 2) and bits
  // 2gq of qh[32n + 16m + ..] (dequant.rs:122-138); the weight is q − 32 (per byte, no borrows)
  auto weights = [&](int j, int a) -> long {
    const int n = j >> 3, gq = (j >> 1) & 3, m = j & 1;
    const uint2 l4 = ql[a][4 * n + 2 * (gq & 1) + m];
    const uint2 h2 = qh[a][2 * n + m];
    const uint32_t lo0 = (gq >> 1) ? (l4.x >> 4) & 0x0F0F0F0Fu : l4.x & 0x0F0F0F0Fu;
    const uint32_t lo1 = (gq >> 1) ? (l4.y >> 4) & 0x0F0F0F0Fu : l4.y & 0x0F0F0F0Fu;
    const uint32_t q0 = lo0 | (((h2.x >> (2 * gq)) & 0x03030303u) << 4);
    const uint32_t q1 = lo1 | (((h2.y >> (2 * gq)) & 0x03030303u) << 4);
    return as_long(((q0 | 0x80808080u) - 0x20202020u) ^ 0x80808080u, ((q1 | 0x80808080u) - 0x20202020u) ^ 0x80808080u);
  };
  auto scale = [&](int j, int a) -> int {
    const uint32_t scd = j < 4 ? sc[a].x : j < 8 ? sc[a].y : j < 12 ? sc[a].z : sc[a].w;
    return (int)(int8_t)((scd >> (8 * (j & 3))) & 0xffu);
  };
  auto mfmas = [&](int j, v16i (&D)[NT][MT]) {
    long cw[NT];
#pragma unroll
    for (int a = 0; a < NT; ++a) cw[a] = weights(j, a);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int mm = m0 + mt * 32 + r;
      const long ax = *reinterpret_cast<const long*>(xb + mm * QK + 16 * (j ^ (mm & 15)) + 8 * h);
#pragma unroll
      for (int a = 0; a < NT; ++a) {
        const v16i z = {};
        D[a][mt] = __builtin_amdgcn_mfma_i32_32x32x16_i8(ax, cw[a], z, 0, 0, 0);
      }
    }
  };
  // two result sets: the MFMAs of sub-block j+1 run while the VALU scales sub-block j
  v16i D0[NT][MT], D1[NT][MT];
  mfmas(0, D0);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    v16i(&Dc)[NT][MT] = (j & 1) ? D1 : D0;
    v16i(&Dn)[NT][MT] = (j & 1) ? D0 : D1;
    if (j + 1 < 16) mfmas(j + 1, Dn);
#pragma unroll
    for (int a = 0; a < NT; ++a) {
      const int sj = scale(j, a);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) S[a][mt][i] += __mul24(sj, Dc[a][mt][i]);  // |D| < 2^17: exact in 24 bits
    }
    // one multiply-add per value and sub-block, in order: keep the sums from being regrouped
#pragma unroll
    for (int a = 0; a < NT; ++a)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(S[a][mt][i]));
    __builtin_amdgcn_sched_barrier(0);
  }
  // matmul.rs:641 epilogue: sx·(d·(float)s)
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const float4 sx4 = *reinterpret_cast<const float4*>(sb + m0 + mt * 32 + 8 * q4 + 4 * h);
      const float sxv[4] = {sx4.x, sx4.y, sx4.z, sx4.w};
#pragma unroll
      for (int a = 0; a < NT; ++a)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float v = sxv[k] * (dd[a] * (float)S[a][mt][4 * q4 + k]);
          acc[a][mt][4 * q4 + k] += v;
        }
    }
}

template <int KIND>
__global__ void __launch_bounds__(256, 2) k_gemm_q6(const uint8_t* __restrict__ wpk, size_t stride_e, int n_in,
                                                 int n_t64, int K, int n_out, int E, RouteBufs rb, GemmX x,
                                                 float* __restrict__ out) {
  constexpr int NT = KIND == GEMM_GATEUP ? 2 : 1;
  constexpr int MT = KIND == GEMM_GATEUP ? 1 : 2;
  __shared__ __align__(16) uint8_t wb0[Q6_WBUF], wb1[Q6_WBUF];
  __shared__ __align__(16) uint8_t xb0[XBUF], xb1[XBUF];
  __shared__ __align__(16) float sb0[BN], sb1[BN];
  __shared__ int32_t rowidx[BN], outrow[BN];
  __shared__ int32_t sh[8];
  TileInfo ti;
  if (!find_tile(rb, E, blockIdx.x, ti, sh)) return;
  member_rows<KIND>(rb, ti, K, rowidx, outrow);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 31, h = lane >> 5;
  const int nb = n_in / QK;
  const int t64 = 2 * blockIdx.y + (w >> 1);
  int half[NT];
  if constexpr (KIND == GEMM_GATEUP) {
    half[0] = 0;
    half[NT - 1] = 1;
  } else {
    half[0] = w & 1;
  }
  const int m0 = KIND == GEMM_GATEUP ? 32 * (w & 1) : 0;
  const size_t tile_bytes = (size_t)nb * TB6;
  const uint8_t* w0 = wpk + (size_t)ti.e * stride_e + (size_t)(2 * blockIdx.y) * tile_bytes;
  const int wo = (w >> 1) * (int)TB6;
  const float start = ti.g > 1 ? 0.0f : -0.0f;
  float acc[NT][MT][16];
#pragma unroll
  for (int a = 0; a < NT; ++a)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][mt][i] = start;
  __syncthreads();  // rowidx
  q6_issue(w0, tile_bytes, x, n_in, 0, rowidx, wb0, xb0, sb0);
  for (int b = 0; b < nb; b += 2) {
    __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): this wave's copies into buffer 0 landed
    __syncthreads();
    if (b + 1 < nb) q6_issue(w0, tile_bytes, x, n_in, b + 1, rowidx, wb1, xb1, sb1);
    q6_block<NT, MT>(wb0 + wo, xb0, sb0, half, m0, acc);
    if (b + 1 >= nb) break;
    __builtin_amdgcn_s_waitcnt(0x3f70);
    __syncthreads();
    if (b + 2 < nb) q6_issue(w0, tile_bytes, x, n_in, b + 2, rowidx, wb0, xb0, sb0);
    q6_block<NT, MT>(wb1 + wo, xb1, sb1, half, m0, acc);
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int n = m0 + mt * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
      if (n >= ti.cnt) continue;
      if constexpr (KIND == GEMM_GATEUP) {
        out[(size_t)outrow[n] * n_out + 32 * t64 + r] = silu(acc[0][mt][i]) * acc[NT - 1][mt][i];
      } else {
        out[(size_t)outrow[n] * n_out + 64 * t64 + 32 * half[0] + r] = acc[0][mt][i];
      }
    }
  (void)n_t64;
}

static int max_tiles(int T, int K, int E) { return (T * K + BN - 1) / BN + E; }

hipError_t launch_gemm_gateup(hipStream_t s, int dtype, const uint8_t* gu, size_t stride_gu, int T, int H, int F,
                              int E, int K, const RouteBufs& rb, GemmX x, float* act) {
  const int n_t64 = F / 32;
  if (dtype == DT_Q4_K)
    hipLaunchKernelGGL(k_gemm_q4<GEMM_GATEUP>, dim3(max_tiles(T, K, E), n_t64 / 2), dim3(256), 0, s, gu,
                       stride_gu, H, n_t64, K, F, E, rb, x, act);
  else
    hipLaunchKernelGGL(k_gemm_q6<GEMM_GATEUP>, dim3(max_tiles(T, K, E), n_t64 / 2), dim3(256), 0, s, gu,
                       stride_gu, H, n_t64, K, F, E, rb, x, act);
  return hipGetLastError();
}

hipError_t launch_gemm_down(hipStream_t s, int dtype, const uint8_t* dn, size_t stride_dn, int T, int H, int F, int E,
                            int K, const RouteBufs& rb, GemmX x, float* slots) {
  const int n_t64 = H / 64;
  dim3 grid(max_tiles(T, K, E), n_t64 / 2);
  if (dtype == DT_Q4_K)
    hipLaunchKernelGGL(k_gemm_q4<GEMM_DOWN>, grid, dim3(256), 0, s, dn, stride_dn, F, n_t64, K, H, E, rb, x, slots);
  else
    hipLaunchKernelGGL(k_gemm_q6<GEMM_DOWN>, grid, dim3(256), 0, s, dn, stride_dn, F, n_t64, K, H, E, rb, x, slots);
  return hipGetLastError();
}

// ---- Q8 rows ---------------------------------------------------------------------------------------
// One wave per 256-block: amax, scale amax/127, quants round(v·127/amax) (kernels/matmul.rs:141-160).
__global__ void __launch_bounds__(256) k_quant_rows(const float* __restrict__ x, size_t n_rows, int n,
                                                    int8_t* __restrict__ q, float* __restrict__ sx) {
  const int lane = threadIdx.x & 63;
  const size_t nbk = n / QK;
  const size_t wi = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wi >= n_rows * nbk) return;
  const float4 v = *reinterpret_cast<const float4*>(x + wi * QK + 4 * lane);
  const float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  const float amax = wave_max(a);
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  const int q0 = q8_round(v.x * inv), q1 = q8_round(v.y * inv), q2 = q8_round(v.z * inv), q3 = q8_round(v.w * inv);
  reinterpret_cast<uint32_t*>(q + wi * QK)[lane] = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                                                   ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
  if (lane == 0) sx[wi] = amax / 127.0f;
}

hipError_t launch_quant_rows(hipStream_t s, const float* x, size_t n_rows, int n, int8_t* q, float* sx) {
  const size_t waves = n_rows * (size_t)(n / QK);
  if (waves == 0) return hipSuccess;
  hipLaunchKernelGGL(k_quant_rows, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, x, n_rows, n, q, sx);
  return hipGetLastError();
}

}  // namespace bb
