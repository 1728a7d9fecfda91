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
//   Q6_K  s = Σ_j sc_j·Σ_{k∈j} (q_k − 32)·x_k with i8 scales. The per-element weight
//         a_k = sc_j·(q_k − 32) (|a_k| <= 4096) is split as a_k = 64·h_k + l_k, h_k in
//         [−64, 64], l_k in [0, 63], both int8: two MFMA passes give s = 64·Dh + Dl.
// The MFMA runs with the activations as the A operand and the weight rows as the B operand, so
// every output a lane holds belongs to one weight row and the row's scales stay in the lane.
#include "bb_device.h"
#include "bb_internal.h"
#include "bb_members.h"
#include "bb_mfma.h"

namespace bb {

// ---- dispatch ------------------------------------------------------------------------------------
// One block of 1024 threads (16 waves); wave w takes the 64-entry chunks w, w+16, ... An entry's
// rank among the chunk's entries of its expert comes from five ballots (one per bit of the
// expert id, E <= 32): the lanes whose ids agree in every bit. The first entry of each expert
// in a chunk records the chunk's count; an exclusive scan over chunks per expert (shuffles in
// half-waves) and over experts gives each chunk's first group position, and an entry's position
// is that plus its rank: the stable grouping of model.rs:316-322.
__global__ void __launch_bounds__(1024) k_dispatch(const int32_t* __restrict__ sel, int n_ent, int E, RouteBufs rb) {
  constexpr int NCH = PF_MAX_ENTRIES / 64;
  constexpr int CPW = NCH / 16;  // chunks per wave
  __shared__ int32_t cc[NCH][32];
  __shared__ int32_t part[32][33];
  __shared__ int32_t off[33];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_chunks = (n_ent + 63) >> 6;
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int i = tid; i < n_chunks * 32; i += 1024) cc[i >> 5][i & 31] = 0;
  int v[CPW];
#pragma unroll
  for (int k = 0; k < CPW; ++k) {
    const int i = (wave + 16 * k) * 64 + lane;
    v[k] = i < n_ent ? sel[i] : -1;
  }
  __syncthreads();
  int rank[CPW];
#pragma unroll
  for (int k = 0; k < CPW; ++k) {
    const int ch = wave + 16 * k;
    rank[k] = 0;
    if (ch >= n_chunks) continue;
    unsigned long long same = __ballot(v[k] >= 0);
#pragma unroll
    for (int bit = 0; bit < 5; ++bit) {
      const unsigned long long b = __ballot((v[k] >> bit) & 1);
      same &= ((v[k] >> bit) & 1) ? b : ~b;
    }
    rank[k] = __popcll(same & lt);
    if (v[k] >= 0 && rank[k] == 0) cc[ch][v[k]] = __popcll(same);
  }
  __syncthreads();
  // thread (e = tid % 32, p = tid / 32) sums chunks [p*cpp, (p+1)*cpp) of expert e
  const int e = tid & 31, p = tid >> 5;
  const int cpp = (n_chunks + 31) >> 5;
  const int c0 = min(p * cpp, n_chunks), c1 = min(c0 + cpp, n_chunks);
  int s = 0;
  for (int ch = c0; ch < c1; ++ch) s += cc[ch][e];
  part[e][p] = s;
  __syncthreads();
  if (wave < 16) {
    // half-wave h of wave w scans the 32 parts of expert 2w + h
    const int ex = 2 * wave + (lane >> 5), q = lane & 31;
    const int val = part[ex][q];
    int incl = val;
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
      const int y = __shfl_up(incl, o, 32);
      if (q >= o) incl += y;
    }
    part[ex][q] = incl - val;
    if (q == 31) part[ex][32] = incl;
  }
  __syncthreads();
  if (tid < 64) {
    const int c = tid < E ? part[tid & 31][32] : 0;
    int incl = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o);
      if (tid >= o) incl += y;
    }
    const unsigned long long hitm = __ballot(c > 0);
    if (tid < E) {
      off[tid] = incl - c;
      rb.counts[tid] = c;
      rb.offsets[tid] = incl - c;
      if (c > 0) rb.hit[1 + __popcll(hitm & ((1ull << tid) - 1ull))] = tid;
    }
    if (tid == E - 1) rb.offsets[E] = incl;
    if (tid == 0) rb.hit[0] = __popcll(hitm);
  }
  __syncthreads();
  {
    int acc = part[e][p] + off[e];
    for (int ch = c0; ch < c1; ++ch) {
      const int x = cc[ch][e];
      cc[ch][e] = acc;
      acc += x;
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < CPW; ++k) {
    const int ch = wave + 16 * k;
    if (ch >= n_chunks) break;
    if (v[k] >= 0) rb.perm[cc[ch][v[k]] + rank[k]] = ch * 64 + lane;
  }
}

hipError_t launch_dispatch(hipStream_t s, int n_ent, int E, const RouteBufs& rb) {
  BB_LAUNCH(k_dispatch, dim3(1), dim3(1024), 0, s, rb.sel, n_ent, E, rb);
  return hipGetLastError();
}

// ---- member tiles --------------------------------------------------------------------------------
// Tiles are enumerated expert by expert, bn members each (an expert's last tile partial).
struct TileInfo {
  int e, m0, cnt, base, g;
};

__device__ bool find_tile(const RouteBufs& rb, int E, int bn, int tile, TileInfo& ti, int32_t* sh) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int c = lane < E ? rb.counts[lane] : 0;
    const int nt = (c + bn - 1) / bn;
    int incl = nt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    const int excl = incl - nt;
    if (lane < E && tile >= excl && tile < incl) {
      sh[0] = lane;
      sh[1] = (tile - excl) * bn;
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
  ti.cnt = min(bn, ti.g - ti.m0);
  return true;
}

// Member rows of the tile: x row (the token for gate/up, the group position for down) and
// output row (group position for gate/up, entry for down; -1: not stored). Padding members
// repeat the last real one so every load stays inside the inputs.
template <int KIND>
__device__ void member_rows(const RouteBufs& rb, const TileInfo& ti, int K, int bn, int32_t* rowidx, int32_t* outrow) {
  for (int n = threadIdx.x; n < bn; n += blockDim.x) {
    const int pos = ti.base + ti.m0 + min(n, ti.cnt - 1);
    const int ent = rb.perm[pos];
    rowidx[n] = KIND == GEMM_GATEUP ? ent / K : pos;
    outrow[n] = n < ti.cnt ? (KIND == GEMM_GATEUP ? pos : ent) : -1;
  }
}

// Small batches (member tiles of 16, at most MAX_ENTRIES entries): the block's unit is member
// tile mt_e of expert e, and the block derives the tile from the selections instead of a
// dispatch kernel's output (the grouping k_dispatch would publish): counts by LDS atomics,
// base = the expert's first group position. The selections must have been loaded into sr.
// Its barriers order LDS only. Needs blockDim.x == 512.
__device__ bool expert_tile(int E, int bn, int e, int mt_e, TileInfo& ti, const SelRegs& sr, int32_t* cnt) {
  const int tid = threadIdx.x;
  if (tid < 32) cnt[tid] = 0;
  lds_barrier();
#pragma unroll
  for (int k = 0; k < SEL_REGS; ++k)
    if (sr.v[k] >= 0) atomicAdd(&cnt[sr.v[k]], 1);
  lds_barrier();
  const int c = cnt[e];
  if (mt_e * bn >= c) return false;
  int base = 0;
  for (int x = 0; x < e; ++x) base += cnt[x];
  ti.e = e;
  ti.m0 = mt_e * bn;
  ti.g = c;
  ti.base = base;
  ti.cnt = min(bn, c - ti.m0);
  return true;
}

// As expert_tile for the h-th expert that has members (ascending ids) instead of expert h;
// false when fewer than h + 1 experts have members.
__device__ bool hit_expert_tile(int E, int bn, int h, int mt_e, TileInfo& ti, const SelRegs& sr, int32_t* cnt) {
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid < 32) cnt[tid] = 0;
  lds_barrier();
#pragma unroll
  for (int k = 0; k < SEL_REGS; ++k)
    if (sr.v[k] >= 0) atomicAdd(&cnt[sr.v[k]], 1);
  lds_barrier();
  const uint32_t mask = (uint32_t)__ballot(lane < E && cnt[lane & 31] > 0);  // the same in every wave
  if (h >= __popc(mask)) return false;
  const int e = nth_expert(mask, h);
  const int c = cnt[e];
  if (mt_e * bn >= c) return false;
  int base = 0;
  for (int x = 0; x < e; ++x) base += cnt[x];
  ti.e = e;
  ti.m0 = mt_e * bn;
  ti.g = c;
  ti.base = base;
  ti.cnt = min(bn, c - ti.m0);
  return true;
}

// member_rows from the expert's member list (entries in ascending order).
template <int KIND>
__device__ void member_rows_list(const int32_t* list, const TileInfo& ti, int K, int bn, int32_t* rowidx,
                                 int32_t* outrow) {
  for (int n = threadIdx.x; n < bn; n += blockDim.x) {
    const int j = ti.m0 + min(n, ti.cnt - 1);
    const int ent = list[j];
    rowidx[n] = KIND == GEMM_GATEUP ? ent / K : ti.base + j;
    outrow[n] = n < ti.cnt ? (KIND == GEMM_GATEUP ? ti.base + j : ent) : -1;
  }
}

// ---- grouped GEMM ------------------------------------------------------------------------------
// Block (member tile of 16*MT members, row tile = two 64-row packed tiles), 8 waves; wave w owns
// the 16-row tile (w&3) of packed tile (w>>2) against all members of the tile. For gate/up,
// 16-row tiles 0-1 of a packed tile are gate rows and 2-3 the up rows of the same 32 outputs;
// the up waves hand their values to the gate waves through LDS at the end (SwiGLU).
//
// MFMA v_mfma_i32_16x16x64_i8 with the activations as A (16 members x 64 elements; lane l:
// member l%16) and the weights as B (64 elements x 16 rows; lane l: row l%16); lane group
// g = l/16 supplies elements 16g..16g+15 of each 64-element step for both, so a lane's weights
// lie in one sub-block (Q4_K: 32 elements, Q6_K: 16) and its activations are one 16-byte chunk
// of the member's row. D lane l = members 4(l/16)..+3 of row l%16.
//
// Super-block b's operands are copied from HBM straight into LDS (global_load_lds_dwordx4: lane
// l's 16 bytes land at base + 16l), double-buffered, so block b+1 streams in while block b is
// computed and no registers hold data in flight:
//   weights      the two packed tile-blocks verbatim
//   activations  member m's 256 quants as 16-byte chunks, chunk c at position c ^ (m%16) of
//                the member's 256-byte row (conflict-free 16-byte reads)
//   scales       sx of the members
// Copies of super-block b: the two packed tile-blocks' weights, the members' activation chunks
// and their scales, as a list of 64-lane copies. Wave w issues copies w, w+8, ... of the list,
// OPS of them per super-block (the list is padded with repeats of the first scale copy into
// spare bytes), so the copies a wave has in flight after a super-block are a known count.
// PARTS selects the weight copies, the activation copies or both (the weights of the first
// super-block are requested before the member rows are known).
template <int DT, int MT>
struct GemmCfg {
  static constexpr int TB = GemmTraits<DT>::TB;
  static constexpr int NBM = 16 * MT;
  static constexpr int W_UNITS = 2 * TB / 16;
  static constexpr int WCH = (W_UNITS + 63) / 64;
  static constexpr int XCH = NBM * QK / 1024;
  static constexpr int SCH = (NBM + 63) / 64;
  static constexpr int OPS = (WCH + XCH + SCH + 7) / 8;
  static constexpr int SB_FLOATS = (SCH + 1) * 64;  // scales, then the spare copies' bytes
};

enum : int { ISSUE_W = 1, ISSUE_X = 2, ISSUE_ALL = 3 };

template <int DT, int MT, int PARTS>
__device__ __forceinline__ void gemm_issue(const uint8_t* w0, size_t tile_bytes, GemmX x, int n_in, int b,
                                           const int32_t* rowidx, uint8_t* wb, uint8_t* xb, float* sb) {
  using C = GemmCfg<DT, MT>;
  constexpr int TB = C::TB;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = n_in / QK;
#pragma unroll
  for (int t = 0; t < C::OPS; ++t) {
    const int j = w + 8 * t;
    if (j < C::WCH) {
      if (PARTS & ISSUE_W) {
        const int u = j * 64 + lane;
        if (u < C::W_UNITS) {
          const int k = u / (TB / 16), o = u % (TB / 16);
          __builtin_amdgcn_global_load_lds(w0 + (size_t)k * tile_bytes + (size_t)b * TB + 16 * o, wb + j * 1024, 16,
                                           0, 0);
        }
      }
    } else if (PARTS & ISSUE_X) {
      if (j < C::WCH + C::XCH) {
        const int i = j - C::WCH;
        const int u = i * 64 + lane, m = u >> 4, c = (u & 15) ^ (m & 15);
        __builtin_amdgcn_global_load_lds(x.q + (size_t)rowidx[m] * n_in + b * QK + 16 * c, xb + i * 1024, 16, 0, 0);
      } else {
        const int i = min(j - C::WCH - C::XCH, C::SCH);  // SCH: the spare bytes
        const int m = min((i < C::SCH ? i : 0) * 64 + lane, C::NBM - 1);
        __builtin_amdgcn_global_load_lds(x.sx + (size_t)rowidx[m] * nb + b, sb + i * 64, 4, 0, 0);
      }
    }
  }
}

// The same copies with each lane's source addresses of super-block 0 computed once (per
// super-block only b times the op's stride is added): for the member tiles of 64 and more,
// whose per-block address arithmetic would otherwise be a tenth of the VALU work.
// One lane's copy of 16 (or 4) bytes from global memory into LDS (lane l at dst + 16l, or 4l).
__device__ __forceinline__ void lds_dma16(const uint8_t* src, uint8_t* dst) {
  __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}
__device__ __forceinline__ void lds_dma4(const uint8_t* src, uint8_t* dst) {
  __builtin_amdgcn_global_load_lds(src, dst, 4, 0, 0);
}

template <int DT, int MT>
struct IssuePlan {
  uint8_t* src[8];  // GemmCfg<DT, MT>::OPS <= 8 used

  __device__ __forceinline__ void issue(int b, uint8_t* wb, uint8_t* xb, float* sb) {
    using C = GemmCfg<DT, MT>;
    constexpr int TB = C::TB;
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int t = 0; t < C::OPS; ++t) {
      const int j = w + 8 * t;
      if (j < C::WCH) {
        if (j * 64 + lane < C::W_UNITS)
          lds_dma16(src[t] + (size_t)b * TB, wb + j * 1024);
      } else if (j < C::WCH + C::XCH) {
        lds_dma16(src[t] + (size_t)b * QK, xb + (j - C::WCH) * 1024);
      } else {
        lds_dma4(src[t] + 4 * b, reinterpret_cast<uint8_t*>(sb + min(j - C::WCH - C::XCH, C::SCH) * 64));
      }
    }
  }
};

template <int DT, int MT>
__device__ __forceinline__ void plan_build(IssuePlan<DT, MT>& p, const uint8_t* w0, size_t tile_bytes, GemmX x,
                                           int n_in, const int32_t* rowidx) {
  using C = GemmCfg<DT, MT>;
  static_assert(C::OPS <= 8, "copy plan size");
  constexpr int TB = C::TB;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = n_in / QK;
#pragma unroll
  for (int t = 0; t < C::OPS; ++t) {
    const int j = w + 8 * t;
    if (j < C::WCH) {
      const int u = min(j * 64 + lane, C::W_UNITS - 1);
      const int k = u / (TB / 16), o = u % (TB / 16);
      p.src[t] = const_cast<uint8_t*>(w0 + (size_t)k * tile_bytes + 16 * o);
    } else if (j < C::WCH + C::XCH) {
      const int u = (j - C::WCH) * 64 + lane, m = u >> 4, c = (u & 15) ^ (m & 15);
      p.src[t] = (uint8_t*)(x.q + (size_t)rowidx[m] * n_in + 16 * c);
    } else {
      const int i = min(j - C::WCH - C::XCH, C::SCH);
      const int m = min((i < C::SCH ? i : 0) * 64 + lane, C::NBM - 1);
      p.src[t] = (uint8_t*)(x.sx + (size_t)rowidx[m] * nb);
    }
    asm volatile("" : "+v"(p.src[t]));  // kept in registers, not recomputed in the loop
  }
}

template <int DT, int KIND, int MT>
__global__ void __launch_bounds__(512) k_gemm(const uint8_t* __restrict__ wpk, size_t stride_e, int n_in, int K,
                                              int n_out, int E, int n_ent, RouteBufs rb, GemmX x,
                                              float* __restrict__ out) {
  using C = GemmCfg<DT, MT>;
  constexpr int TB = C::TB;
  constexpr int NBM = C::NBM;  // members per tile
  // double-buffered stages: the weights, then the activations followed by their scales
  constexpr int XS = NBM * QK + 4 * C::SB_FLOATS;
  __shared__ __align__(16) uint8_t wb0[2 * TB], wb1[2 * TB];
  __shared__ __align__(16) uint8_t xb0[XS], xb1[XS];
  float* const sb0 = reinterpret_cast<float*>(xb0 + NBM * QK);
  float* const sb1 = reinterpret_cast<float*>(xb1 + NBM * QK);
  __shared__ int32_t rowidx[NBM], outrow[NBM];
  __shared__ int32_t sh[8];
  __shared__ uint64_t exptab[32];
  const uint64_t exp_e = KIND == GEMM_GATEUP ? exp_table_entry() : 0;
  // Workgroups are handed to the 8 XCDs round-robin by id. With member tiles of 16 (small
  // batches: the weights dominate and each expert has about one member tile) consecutive ids
  // take consecutive row tiles of one member tile, so every XCD streams an equal share of the
  // weights; member tile m is tile m / E of expert m % E. With larger member tiles XCD k takes
  // member tiles k, k+8, ... and sweeps all row tiles of one member tile before the next, so
  // the member tile's activations are fetched once into that XCD's L2; the sweep direction
  // alternates so the weights used last are used first again.
  const int n_rt = gridDim.y, n_mt = gridDim.x;  // n_mt: an upper bound (a multiple of 8 when MT > 1)
  const int lin = blockIdx.y * n_mt + blockIdx.x;
  int mtile, rtile;
  if constexpr (MT == 1) {
    mtile = lin / n_rt;
    rtile = lin % n_rt;
  } else {
    const int xcd = lin & 7, slot = lin >> 3;
    const int mt_local = slot / n_rt, rt_step = slot % n_rt;
    mtile = mt_local * 8 + xcd;
    rtile = (mt_local & 1) ? n_rt - 1 - rt_step : rt_step;
  }
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, g = lane >> 4;
  const int nb = n_in / QK;
  const int k64 = w >> 2, t16 = w & 3, row = 16 * t16 + r;
  const int t64 = 2 * rtile + k64;
  const size_t tile_bytes = (size_t)nb * TB;
  const int wo = k64 * TB;
  TileInfo ti;
  const uint8_t* w0;
  // the first block's weights are requested as soon as the expert is known
  if constexpr (MT == 1) {
    // unit = (expert, its member tile mt_e, row tile). Down: the expert is e = mtile % E, known
    // from the block id, so the first block's weights of an expert's first member tile are
    // requested before the selections are even read (wasted only when the expert has no
    // member). Gate/up: the (mtile % E)-th expert that has members, so the blocks of the experts
    // nobody chose are the last of the grid and leave at once instead of holding a slot while
    // their weights arrive (the gate/up grid is larger than the resident blocks).
    __shared__ SmemMembers mem;
    __shared__ int32_t cnt[32];
    constexpr bool BY_HIT = KIND == GEMM_GATEUP;
    const int e = mtile % E, mt_e = mtile / E;
    w0 = wpk + (size_t)e * stride_e + (size_t)(2 * rtile) * tile_bytes;
    // gate/up of at most 16 tokens: the member tile is every token of the batch (outputs of the
    // tokens that did not choose the expert are computed and dropped), so the activations of
    // the first block are requested with its weights, before the selections are read
    const int n_tok = n_ent / K;
    const bool all_tokens = KIND == GEMM_GATEUP && n_tok <= 16;
    SelRegs sr;
#pragma unroll
    for (int k = 0; k < SEL_REGS; ++k) {
      const int i = k * 512 + tid;
      sr.v[k] = i < n_ent ? rb.sel[i] : -1;
    }
    if (!BY_HIT && mt_e == 0) gemm_issue<DT, MT, ISSUE_W>(w0, tile_bytes, x, n_in, 0, rowidx, wb0, xb0, sb0);
    if (all_tokens) {
      if (tid < NBM) rowidx[tid] = min(tid, n_tok - 1);
      lds_barrier();
      gemm_issue<DT, MT, ISSUE_X>(w0, tile_bytes, x, n_in, 0, rowidx, wb0, xb0, sb0);
    }
    const bool live = BY_HIT ? hit_expert_tile(E, NBM, e, mt_e, ti, sr, cnt) : expert_tile(E, NBM, e, mt_e, ti, sr, cnt);
    if (!live) {
      __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): no copy may land after the block's LDS is released
      return;
    }
    if (BY_HIT) w0 = wpk + (size_t)ti.e * stride_e + (size_t)(2 * rtile) * tile_bytes;
    if (BY_HIT || mt_e > 0) gemm_issue<DT, MT, ISSUE_W>(w0, tile_bytes, x, n_in, 0, rowidx, wb0, xb0, sb0);
    member_list(sr, n_ent, ti.e, mem);
    if (all_tokens) {
      // output row of token n: its group position, or -1 when it did not choose the expert
      if (tid < NBM) outrow[tid] = -1;
      lds_barrier();
      if (tid < ti.cnt) outrow[mem.list[tid] / K] = ti.base + tid;
    } else {
      member_rows_list<KIND>(mem.list, ti, K, NBM, rowidx, outrow);
    }
  } else {
    if (!find_tile(rb, E, NBM, mtile, ti, sh)) return;
    w0 = wpk + (size_t)ti.e * stride_e + (size_t)(2 * rtile) * tile_bytes;
    gemm_issue<DT, MT, ISSUE_W>(w0, tile_bytes, x, n_in, 0, rowidx, wb0, xb0, sb0);
    member_rows<KIND>(rb, ti, K, NBM, rowidx, outrow);
  }
  const float start = ti.g > 1 ? 0.0f : -0.0f;
  float acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[mt][i] = start;
  auto block = [&](const uint8_t* wb, const uint8_t* xb, const float* sb) {
    if constexpr (DT == DT_Q4_K) q4_block<MT>(wb + wo, xb, sb, row, acc);
    else q6_block<MT>(wb + wo, xb, sb, row, acc);
  };
  lds_barrier();  // rowidx, outrow; the first block's copies stay in flight
  if (MT > 1 || !(KIND == GEMM_GATEUP && n_ent / K <= 16))
    gemm_issue<DT, MT, ISSUE_X>(w0, tile_bytes, x, n_in, 0, rowidx, wb0, xb0, sb0);
  IssuePlan<DT, MT> plan;
  if constexpr (MT > 1) plan_build<DT, MT>(plan, w0, tile_bytes, x, n_in, rowidx);
  for (int b = 0; b < nb; b += 2) {
    __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): this wave's copies into buffer 0 landed
    if (KIND == GEMM_GATEUP && b == 0 && tid < 32) exptab[tid] = exp_e;
    __syncthreads();
    if (b + 1 < nb) {
      if constexpr (MT > 1) plan.issue(b + 1, wb1, xb1, sb1);
      else gemm_issue<DT, MT, ISSUE_ALL>(w0, tile_bytes, x, n_in, b + 1, rowidx, wb1, xb1, sb1);
    }
    block(wb0, xb0, sb0);
    if (b + 1 >= nb) break;
    __builtin_amdgcn_s_waitcnt(0x3f70);
    __syncthreads();
    if (b + 2 < nb) {
      if constexpr (MT > 1) plan.issue(b + 2, wb0, xb0, sb0);
      else gemm_issue<DT, MT, ISSUE_ALL>(w0, tile_bytes, x, n_in, b + 2, rowidx, wb0, xb0, sb0);
    }
    block(wb1, xb1, sb1);
  }
  if constexpr (KIND == GEMM_GATEUP) {
    // the up waves hand their values to the gate waves of the same outputs
    __syncthreads();
    float* upv = reinterpret_cast<float*>(xb0);  // 4 up waves x MT*4 values x 64 lanes = sizeof xb0
    if (t16 >= 2) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) upv[((k64 * 2 + (t16 - 2)) * (4 * MT) + mt * 4 + i) * 64 + lane] = acc[mt][i];
    }
    __syncthreads();
    if (t16 < 2) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = mt * 16 + 4 * g + i;
          if (outrow[n] < 0) continue;
          const float up = upv[((k64 * 2 + t16) * (4 * MT) + mt * 4 + i) * 64 + lane];
          out[(size_t)outrow[n] * n_out + 32 * t64 + 16 * t16 + r] = silu_tab(acc[mt][i], exptab) * up;
        }
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = mt * 16 + 4 * g + i;
        if (outrow[n] < 0) continue;
        out[(size_t)outrow[n] * n_out + 64 * t64 + 16 * t16 + r] = acc[mt][i];
      }
  }
}

// Member tile (in units of 16 members): 16 for decode-sized batches (these tiles take their
// grouping from the selections), else 64; Q6_K rows take 128 when the groups fill such tiles
// on average. (A Q4_K block of 64 members leaves room for two blocks per CU, which beat one
// block of 128 members: 483 vs 554 µs for config 4's gate/up. A Q6_K block of 64 members
// still fills a CU's LDS alone.)
int gemm_member_tiles(int n_ent, int E) { return n_ent >= 16 * E ? 4 : 1; }

template <int DT, int KIND>
static hipError_t launch_gemm(hipStream_t s, const uint8_t* w, size_t stride_e, int T, int n_in, int n_out,
                              int n_t64, int E, int K, const RouteBufs& rb, GemmX x, float* out) {
  const int n_ent = T * K;
  const int mt = DT == DT_Q6_K && n_ent >= 128 * E ? 8 : gemm_member_tiles(n_ent, E);
  const int bn = 16 * mt;
  // enough member tiles: with tiles of 16, ceil(T/16) per expert (an expert has at most T
  // members); else every hit expert adds at most one partial tile
  const int n_mt = mt == 1 ? E * ((T + bn - 1) / bn) : ((n_ent + bn - 1) / bn + E + 7) / 8 * 8;
  dim3 grid(n_mt, n_t64 / 2);
  if (DT == DT_Q6_K && mt == 8)
    BB_LAUNCH((k_gemm<DT_Q6_K, KIND, 8>), grid, dim3(512), 0, s, w, stride_e, n_in, K, n_out, E, n_ent, rb, x, out);
  else if (mt == 4)
    BB_LAUNCH((k_gemm<DT, KIND, 4>), grid, dim3(512), 0, s, w, stride_e, n_in, K, n_out, E, n_ent, rb, x, out);
  else
    BB_LAUNCH((k_gemm<DT, KIND, 1>), grid, dim3(512), 0, s, w, stride_e, n_in, K, n_out, E, n_ent, rb, x, out);
  return hipGetLastError();
}

hipError_t launch_gemm_gateup(hipStream_t s, int dtype, const uint8_t* gu, size_t stride_gu, int T, int H, int F,
                              int E, int K, const RouteBufs& rb, GemmX x, float* act) {
  if (dtype == DT_Q4_K) return launch_gemm<DT_Q4_K, GEMM_GATEUP>(s, gu, stride_gu, T, H, F, F / 32, E, K, rb, x, act);
  return launch_gemm<DT_Q6_K, GEMM_GATEUP>(s, gu, stride_gu, T, H, F, F / 32, E, K, rb, x, act);
}

hipError_t launch_gemm_down(hipStream_t s, int dtype, const uint8_t* dn, size_t stride_dn, int T, int H, int F, int E,
                            int K, const RouteBufs& rb, GemmX x, float* slots) {
  if (dtype == DT_Q4_K) return launch_gemm<DT_Q4_K, GEMM_DOWN>(s, dn, stride_dn, T, F, H, H / 64, E, K, rb, x, slots);
  return launch_gemm<DT_Q6_K, GEMM_DOWN>(s, dn, stride_dn, T, F, H, H / 64, E, K, rb, x, slots);
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
  BB_LAUNCH(k_quant_rows, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, x, n_rows, n, q, sx);
  return hipGetLastError();
}

}  // namespace bb
