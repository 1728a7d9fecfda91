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
#include <type_traits>

#include "bb_internal.h"
#include "bb_members.h"
#include "bb_mfma.h"
#include "bb_rowlane.h"

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
// g = l/16 supplies 16 consecutive elements of each 64-element step for both (the order of
// steps and groups is bb_mfma.h's), so a lane's weights of a step lie in one sub-block and its
// activations are one 16-byte chunk of the member's row. D lane l = members 4(l/16)..+3 of
// row l%16.
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
// MF: the Q4_K min term from the activations' split per-32 sums (one f16 MFMA per member tile,
// min_split_record) instead of a third int8 pass; the stage then also holds the members' sum
// records (32 bytes each), copied after the activations.
template <int DT, int MT, bool MF = false>
struct GemmCfg {
  static constexpr int TB = GemmTraits<DT>::TB;
  static constexpr int NBM = 16 * MT;
  static constexpr int W_UNITS = 2 * TB / 16;
  static constexpr int WCH = (W_UNITS + 63) / 64;
  static constexpr int XCH = NBM * QK / 1024;
  static constexpr int MSCH = MF ? (NBM * 32 + 1023) / 1024 : 0;  // 1 KB = 32 members' records
  static constexpr int SCH = (NBM + 63) / 64;
  static constexpr int OPS = (WCH + XCH + MSCH + SCH + 7) / 8;
  static constexpr int SB_FLOATS = (SCH + 1) * 64;  // scales, then the spare copies' bytes
  static constexpr int MS_BYTES = MSCH * 1024;      // the records (the last copy's tail is spare)
};

// Waves per SIMD the registers of k_gemm are budgeted for: two blocks of 8 waves share a CU
// where the LDS stages leave room (Q4_K tiles of 16 and 64 members), else one.
constexpr int gemm_waves_per_simd(int dt) { return dt == DT_Q4_K ? 4 : 2; }

enum : int { ISSUE_W = 1, ISSUE_X = 2, ISSUE_ALL = 3 };

template <int DT, int MT, int PARTS, bool MF = false>
__device__ __forceinline__ void gemm_issue(const uint8_t* w0, size_t tile_bytes, GemmX x, int n_in, int b,
                                           const int32_t* rowidx, uint8_t* wb, uint8_t* xb, float* sb) {
  using C = GemmCfg<DT, MT, MF>;
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
          // a decode batch's weight tiles are read once (one member tile per expert): streamed
          __builtin_amdgcn_global_load_lds(w0 + (size_t)k * tile_bytes + (size_t)b * TB + 16 * o, wb + j * 1024, 16,
                                           0, MT == 1 ? CPOL_NT : 0);
        }
      }
    } else if (PARTS & ISSUE_X) {
      if (j < C::WCH + C::XCH) {
        const int i = j - C::WCH;
        const int u = i * 64 + lane, m = u >> 4, c = (u & 15) ^ (m & 15);
        __builtin_amdgcn_global_load_lds(x.q + (size_t)rowidx[m] * n_in + b * QK + 16 * c, xb + i * 1024, 16, 0, 0);
      } else if (j < C::WCH + C::XCH + C::MSCH) {
        // sum records: lane l copies half l & 1 of member 32i + l/2's record (members past the
        // tile repeat its last one into the spare tail)
        const int i = j - C::WCH - C::XCH;
        const int m = min(32 * i + (lane >> 1), C::NBM - 1);
        const uint8_t* src = reinterpret_cast<const uint8_t*>(x.ms) + ((size_t)rowidx[m] * nb + b) * 32 + 16 * (lane & 1);
        uint8_t* dst = reinterpret_cast<uint8_t*>(sb + C::SB_FLOATS) + i * 1024;
        __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
      } else {
        const int i = min(j - C::WCH - C::XCH - C::MSCH, C::SCH);  // SCH: the spare bytes
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

template <int DT, int MT, bool MF = false>
struct IssuePlan {
  uint8_t* src[8];  // GemmCfg<DT, MT, MF>::OPS <= 8 used

  __device__ __forceinline__ void issue(int b, uint8_t* wb, uint8_t* xb, float* sb) {
    using C = GemmCfg<DT, MT, MF>;
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
      } else if (j < C::WCH + C::XCH + C::MSCH) {
        lds_dma16(src[t] + (size_t)b * 32, reinterpret_cast<uint8_t*>(sb) + 4 * C::SB_FLOATS +
                                               (j - C::WCH - C::XCH) * 1024);
      } else {
        lds_dma4(src[t] + 4 * b, reinterpret_cast<uint8_t*>(sb + min(j - C::WCH - C::XCH - C::MSCH, C::SCH) * 64));
      }
    }
  }
};

template <int DT, int MT, bool MF>
__device__ __forceinline__ void plan_build(IssuePlan<DT, MT, MF>& p, const uint8_t* w0, size_t tile_bytes, GemmX x,
                                           int n_in, const int32_t* rowidx) {
  using C = GemmCfg<DT, MT, MF>;
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
    } else if (j < C::WCH + C::XCH + C::MSCH) {
      const int m = min(32 * (j - C::WCH - C::XCH) + (lane >> 1), C::NBM - 1);
      p.src[t] = (uint8_t*)(x.ms + (size_t)rowidx[m] * nb * 16 + 8 * (lane & 1));
    } else {
      const int i = min(j - C::WCH - C::XCH - C::MSCH, C::SCH);
      const int m = min((i < C::SCH ? i : 0) * 64 + lane, C::NBM - 1);
      p.src[t] = (uint8_t*)(x.sx + (size_t)rowidx[m] * nb);
    }
    asm volatile("" : "+v"(p.src[t]));  // kept in registers, not recomputed in the loop
  }
}

// IssuePlan's copies through buffer resources: a lane's 32-bit source offset of each copy is fixed
// and super-block b adds a wave-uniform offset (b times the stream's stride), so a copy costs no
// vector address arithmetic. For inputs whose offsets fit 31 bits.
template <int DT, int MT, bool MF = false>
struct BufPlan {
  __amdgpu_buffer_rsrc_t rw, rx, rs, rm;
  uint32_t off[8];  // GemmCfg<DT, MT, MF>::OPS <= 8 used

  __device__ __forceinline__ void issue(int b, uint8_t* wb, uint8_t* xb, float* sb) {
    using C = GemmCfg<DT, MT, MF>;
    constexpr int TB = C::TB;
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int t = 0; t < C::OPS; ++t) {
      const int j = w + 8 * t;
      if (j < C::WCH) {
        if (j * 64 + lane < C::W_UNITS) buf_dma16(rw, off[t], (uint32_t)(b * TB), wb + j * 1024);
      } else if (j < C::WCH + C::XCH) {
        buf_dma16(rx, off[t], (uint32_t)(b * QK), xb + (j - C::WCH) * 1024);
      } else if (j < C::WCH + C::XCH + C::MSCH) {
        buf_dma16(rm, off[t], (uint32_t)(b * 32), reinterpret_cast<uint8_t*>(sb) + 4 * C::SB_FLOATS +
                                                      (j - C::WCH - C::XCH) * 1024);
      } else {
        buf_dma4(rs, off[t], (uint32_t)(4 * b),
                 reinterpret_cast<uint8_t*>(sb + min(j - C::WCH - C::XCH - C::MSCH, C::SCH) * 64));
      }
    }
  }
};

// w0: the block's two packed tiles (wave-uniform); x_rows: rows of x.q / x.sx.
template <int DT, int MT, bool MF>
__device__ __forceinline__ void bufplan_build(BufPlan<DT, MT, MF>& p, const uint8_t* w0, size_t tile_bytes, GemmX x,
                                              int n_in, int x_rows, const int32_t* rowidx) {
  using C = GemmCfg<DT, MT, MF>;
  static_assert(C::OPS <= 8, "copy plan size");
  constexpr int TB = C::TB;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = n_in / QK;
  p.rw = buf_rsrc(w0, (uint32_t)(2 * tile_bytes));
  p.rx = buf_rsrc(x.q, (uint32_t)x_rows * (uint32_t)n_in);
  p.rs = buf_rsrc(x.sx, (uint32_t)x_rows * (uint32_t)nb * 4u);
  p.rm = MF ? buf_rsrc(x.ms, (uint32_t)x_rows * (uint32_t)nb * 32u) : p.rs;
#pragma unroll
  for (int t = 0; t < C::OPS; ++t) {
    const int j = w + 8 * t;
    if (j < C::WCH) {
      const int u = min(j * 64 + lane, C::W_UNITS - 1);
      const int k = u / (TB / 16), o = u % (TB / 16);
      p.off[t] = (uint32_t)(k * tile_bytes) + 16u * (uint32_t)o;
    } else if (j < C::WCH + C::XCH) {
      const int u = (j - C::WCH) * 64 + lane, m = u >> 4, c = (u & 15) ^ (m & 15);
      p.off[t] = (uint32_t)rowidx[m] * (uint32_t)n_in + 16u * (uint32_t)c;
    } else if (j < C::WCH + C::XCH + C::MSCH) {
      const int m = min(32 * (j - C::WCH - C::XCH) + (lane >> 1), C::NBM - 1);
      p.off[t] = (uint32_t)rowidx[m] * (uint32_t)nb * 32u + 16u * (uint32_t)(lane & 1);
    } else {
      const int i = min(j - C::WCH - C::XCH - C::MSCH, C::SCH);
      const int m = min((i < C::SCH ? i : 0) * 64 + lane, C::NBM - 1);
      p.off[t] = (uint32_t)rowidx[m] * (uint32_t)nb * 4u;
    }
  }
}

template <int DT, int KIND, int MT, bool BUF = false, bool MF = false>
__global__ void __launch_bounds__(512, gemm_waves_per_simd(DT)) k_gemm(const uint8_t* __restrict__ wpk, size_t stride_e, int n_in, int K,
                                              int n_out, int E, int n_ent, RouteBufs rb, GemmX x,
                                              float* __restrict__ out) {
  static_assert(!MF || (DT == DT_Q4_K && MT > 1), "the f16 min term serves the Q4_K member tiles of 64 and 80");
  using C = GemmCfg<DT, MT, MF>;
  constexpr int TB = C::TB;
  constexpr int NBM = C::NBM;  // members per tile
  // double-buffered stages: the weights, then the activations followed by their scales (and, MF,
  // the members' sum records)
  constexpr int XS = NBM * QK + 4 * C::SB_FLOATS + (MF ? C::MS_BYTES : 0);
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
    if (!BY_HIT && mt_e == 0) gemm_issue<DT, MT, ISSUE_W, MF>(w0, tile_bytes, x, n_in, 0, rowidx, wb0, xb0, sb0);
    if (all_tokens) {
      if (tid < NBM) rowidx[tid] = min(tid, n_tok - 1);
      lds_barrier();
      gemm_issue<DT, MT, ISSUE_X, MF>(w0, tile_bytes, x, n_in, 0, rowidx, wb0, xb0, sb0);
    }
    const bool live = BY_HIT ? hit_expert_tile(E, NBM, e, mt_e, ti, sr, cnt) : expert_tile(E, NBM, e, mt_e, ti, sr, cnt);
    if (!live) {
      __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): no copy may land after the block's LDS is released
      return;
    }
    if (BY_HIT) w0 = wpk + (size_t)ti.e * stride_e + (size_t)(2 * rtile) * tile_bytes;
    if (BY_HIT || mt_e > 0) gemm_issue<DT, MT, ISSUE_W, MF>(w0, tile_bytes, x, n_in, 0, rowidx, wb0, xb0, sb0);
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
    w0 = wpk + (size_t)__builtin_amdgcn_readfirstlane(ti.e) * stride_e + (size_t)(2 * rtile) * tile_bytes;
    gemm_issue<DT, MT, ISSUE_W, MF>(w0, tile_bytes, x, n_in, 0, rowidx, wb0, xb0, sb0);
    member_rows<KIND>(rb, ti, K, NBM, rowidx, outrow);
  }
  const float start = ti.g > 1 ? 0.0f : -0.0f;
  float acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[mt][i] = start;
  lds_barrier();  // rowidx, outrow; the first block's copies stay in flight
  if (MT > 1 || !(KIND == GEMM_GATEUP && n_ent / K <= 16))
    gemm_issue<DT, MT, ISSUE_X, MF>(w0, tile_bytes, x, n_in, 0, rowidx, wb0, xb0, sb0);
  using Plan = std::conditional_t<BUF, BufPlan<DT, MT, MF>, IssuePlan<DT, MT, MF>>;
  Plan plan;
  if constexpr (MT > 1) {
    if constexpr (BUF) bufplan_build<DT, MT, MF>(plan, w0, tile_bytes, x, n_in, KIND == GEMM_GATEUP ? n_ent / K : n_ent,
                                             rowidx);
    else plan_build<DT, MT, MF>(plan, w0, tile_bytes, x, n_in, rowidx);
  }
  // The super-block loop over the first M member tiles (the copies still bring all MT).
  auto sweep = [&](auto m) {
    constexpr int M = decltype(m)::value;
    float(&am)[M][4] = reinterpret_cast<float(&)[M][4]>(acc);
    auto block = [&](const uint8_t* wb, const uint8_t* xb, const float* sb) {
      if constexpr (DT == DT_Q4_K)
        q4_block<M, MF>(wb + wo, xb, sb, reinterpret_cast<const uint8_t*>(sb) + 4 * C::SB_FLOATS, row, am);
      else q6_block<M>(wb + wo, xb, sb, row, am);
    };
    for (int b = 0; b < nb; b += 2) {
      __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): this wave's copies into buffer 0 landed
      if (KIND == GEMM_GATEUP && b == 0 && tid < 32) exptab[tid] = exp_e;
      __syncthreads();
      if (b + 1 < nb) {
        if constexpr (MT > 1) plan.issue(b + 1, wb1, xb1, sb1);
        else gemm_issue<DT, MT, ISSUE_ALL, MF>(w0, tile_bytes, x, n_in, b + 1, rowidx, wb1, xb1, sb1);
      }
      block(wb0, xb0, sb0);
      if (b + 1 >= nb) break;
      __builtin_amdgcn_s_waitcnt(0x3f70);
      __syncthreads();
      if (b + 2 < nb) {
        if constexpr (MT > 1) plan.issue(b + 2, wb0, xb0, sb0);
        else gemm_issue<DT, MT, ISSUE_ALL, MF>(w0, tile_bytes, x, n_in, b + 2, rowidx, wb0, xb0, sb0);
      }
      block(wb1, xb1, sb1);
    }
  };
  // A tile of MT = 5 that holds at most 64 members computes only its first 4 member tiles (the
  // others' outputs are not stored), so it costs what a tile of 64 does.
  if constexpr (MT == 5) {
    if (__builtin_amdgcn_readfirstlane(ti.cnt) <= 64) sweep(std::integral_constant<int, 4>{});
    else sweep(std::integral_constant<int, 5>{});
  } else {
    sweep(std::integral_constant<int, MT>{});
  }
  if constexpr (KIND == GEMM_GATEUP) {
    // SwiGLU of the wave pair (gate rows t16, up rows t16 + 2 of the same outputs): the gate wave
    // takes member tiles mt < MG, the up wave the rest; each hands the other its values of the
    // other's tiles through LDS
    constexpr int MG = MT - MT / 2;
    __syncthreads();
    float* upv = reinterpret_cast<float*>(xb0);  // 4 up waves x MG*4 values x 64 lanes <= sizeof xb0
    float* gtv = reinterpret_cast<float*>(xb1);  // 4 gate waves x (MT-MG)*4 values x 64 lanes
    const int pair = k64 * 2 + (t16 & 1);
    if (t16 >= 2) {
#pragma unroll
      for (int mt = 0; mt < MG; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) upv[(pair * (4 * MG) + mt * 4 + i) * 64 + lane] = acc[mt][i];
    } else {
#pragma unroll
      for (int mt = MG; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) gtv[(pair * (4 * (MT - MG)) + (mt - MG) * 4 + i) * 64 + lane] = acc[mt][i];
    }
    __syncthreads();
    const int col = 32 * t64 + 16 * (t16 & 1) + r;
    if (t16 < 2) {
#pragma unroll
      for (int mt = 0; mt < MG; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = mt * 16 + 4 * g + i;
          if (outrow[n] < 0) continue;
          const float up = upv[(pair * (4 * MG) + mt * 4 + i) * 64 + lane];
          out[(size_t)outrow[n] * n_out + col] = silu_tab(acc[mt][i], exptab) * up;
        }
    } else {
#pragma unroll
      for (int mt = MG; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = mt * 16 + 4 * g + i;
          if (outrow[n] < 0) continue;
          const float gate = gtv[(pair * (4 * (MT - MG)) + (mt - MG) * 4 + i) * 64 + lane];
          out[(size_t)outrow[n] * n_out + col] = silu_tab(gate, exptab) * acc[mt][i];
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

// ---- grouped GEMM for large groups ------------------------------------------------------------
// Block = up to 256 members (NT <= 16 member tiles of 16) x 128 weight rows (two 64-row packed
// tiles), 8 waves, one block per CU (two waves per SIMD with up to 256 VGPRs each). Wave w owns
// the 16 rows (w&3) of packed tile (w>>2) against all the block's members.
// The GEMM is bound by VALU issue: per output and super-block the exact f32 epilogue takes 8
// (Q4_K) or 5 (Q6_K) VALU instructions against 3 or 2 MFMA passes, and the nibble / scale
// operand build (~100 VALU per lane and super-block) is shared by the wave's member tiles, so a
// wave takes as many member tiles as its registers hold. Within a wave the work is
// software-pipelined so that the MFMA unit and the VALU work side by side:
//   * the epilogue of member tile t-1 is issued between the MFMAs of tile t;
//   * the operands of super-block b+1 are built during the second half of b's member tiles,
//     into a second operand set, from weight bytes loaded into registers at the start of b
//     (no other wave reads a wave's weight rows, so they skip LDS).
// Activations (the members' 256 quants per super-block, chunks XOR-swizzled as in k_gemm, and
// their scales) are copied HBM -> LDS with buffer loads to LDS, double-buffered per super-block.
// Nothing is in flight when a wave ends: the last super-block issues no copies or loads.
// An expert's members are cut into chunks of 256 and the rest into chunks of 8, 4, 2 and 1
// member tiles (a partial last tile wastes at most 15 members per expert); the tile loop of a
// chunk is straight-line code. Epilogues and sums are those of k_gemm.
constexpr int WIDE_LOG = 4;                // chunks of at most 2^WIDE_LOG member tiles
constexpr int WIDE_NB = 16 << WIDE_LOG;    // members per block at most (256)
constexpr int WIDE_WAVES = 8;
constexpr int WIDE_PT = WIDE_WAVES / 4;    // 64-row packed tiles per block
constexpr int WIDE_XS = WIDE_NB * QK;      // activation bytes per stage

// A lane's weight bytes of one super-block: Q4_K the header and the 4 qs chunks its MFMA
// operands come from, Q6_K its 2 ql, 2 qh and sc chunks and d.
template <int DT>
struct WideW;
template <>
struct WideW<DT_Q4_K> {
  uint4 hd, q[4];
};
template <>
struct WideW<DT_Q6_K> {
  uint4 sc, ql[2], qh[2];
  uint32_t d;
};

// A lane's offsets in its packed tile (row = its weight row, g = its K group): the row's 16
// bytes of a 1 KB chunk, shifted by chunk g or g & 1; Q6_K's d field of the row.
struct WideOff {
  uint32_t row, g, g1, d;
};

// Loads super-block b's bytes (sb = b·TB, wave-uniform) from the wave's packed tile.
template <int DT>
__device__ __forceinline__ void wide_load(WideW<DT>& w, __amdgpu_buffer_rsrc_t r, const WideOff& o, uint32_t sb) {
  if constexpr (DT == DT_Q4_K) {
    w.hd = buf_load16(r, o.row, sb);
#pragma unroll
    for (int c = 0; c < 4; ++c) w.q[c] = buf_load16(r, o.g1, sb + 1024 * (1 + 2 * c));
  } else {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      w.ql[n] = buf_load16(r, o.g, sb + 4096 * n);
      w.qh[n] = buf_load16(r, o.g1, sb + 1024 * (8 + 2 * n));
    }
    w.sc = buf_load16(r, o.row, sb + 1024 * 12);
    w.d = __builtin_amdgcn_raw_buffer_load_b16(r, (int)o.d, (int)sb, 0);
  }
}

// The lane's MFMA weight operands of one super-block (as q4_block / q6_block build them):
// B[0..3] the high, B[4..7] the low parts; Q4_K's min pass takes for chunk c the byte ms[c]
// in every position (splat when used).
template <int DT>
struct WideB {
  v4i B[8];
  uint32_t ms[4];
  float d, dm;
};

__device__ __forceinline__ void wide_build(const WideW<DT_Q4_K>& w, int g, WideB<DT_Q4_K>& o) {
  o.d = f16_bits_to_f32(w.hd.x & 0xffff);
  o.dm = f16_bits_to_f32(w.hd.x >> 16);
  const uint32_t s0 = w.hd.y, s1 = w.hd.z, s2 = w.hd.w;
  const uint32_t scw[2] = {s0 & 0x3F3F3F3Fu, (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u)};
  const uint32_t mw[2] = {s1 & 0x3F3F3F3Fu, ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u)};
  const int hi = g >> 1;
  const uint32_t nsh = 4 * hi;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int sh = 8 * (2 * (c & 1) + hi);
    const uint4 qv = w.q[c];
    const uint32_t q[4] = {(qv.x >> nsh) & 0x0F0F0F0Fu, (qv.y >> nsh) & 0x0F0F0F0Fu, (qv.z >> nsh) & 0x0F0F0F0Fu,
                           (qv.w >> nsh) & 0x0F0F0F0Fu};
    const uint32_t scv = (scw[c >> 1] >> sh) & 0xffu;
    const uint32_t hs = scv >> 3, ls = scv & 7u;
    o.ms[c] = splat_byte(mw[c >> 1] >> sh);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o.B[c][k] = (int)mul_bytes(q[k], hs);
      o.B[4 + c][k] = (int)mul_bytes(q[k], ls);
    }
  }
}

__device__ __forceinline__ void wide_build(const WideW<DT_Q6_K>& w, int g, WideB<DT_Q6_K>& o) {
  o.d = f16_bits_to_f32(w.d & 0xffff);
  o.dm = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    // elements 64c + 16g + t: ql chunk 4(c/2) + g (high nibbles when c is odd), qh chunk
    // 8 + 2(c/2) + (g&1) bits 2·gq with gq = 2(c&1) + g/2; sub-block 4c + g (dequant.rs:122-138)
    const int gq = 2 * (c & 1) + (g >> 1);
    const uint4 qlv = w.ql[c >> 1], qhv = w.qh[c >> 1];
    const uint32_t lsh = 4 * (c & 1), hsh = 2 * gq;
    const uint32_t scd = c == 0 ? w.sc.x : c == 1 ? w.sc.y : c == 2 ? w.sc.z : w.sc.w;
    const int scj = (int)(int8_t)((scd >> (8 * g)) & 0xffu);
    const uint32_t scp = ((uint32_t)scj & 0xffffu) * 0x00010001u;
    const uint32_t bias = ((uint32_t)(-32 * scj) & 0xffffu) * 0x00010001u;
    const uint32_t qlw[4] = {qlv.x, qlv.y, qlv.z, qlv.w}, qhw[4] = {qhv.x, qhv.y, qhv.z, qhv.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t q = ((qlw[k] >> lsh) & 0x0F0F0F0Fu) | (((qhw[k] >> hsh) & 0x03030303u) << 4);
      uint32_t hh, ll;
      q6_split(q, scp, bias, hh, ll);
      o.B[c][k] = (int)hh;
      o.B[4 + c][k] = (int)ll;
    }
    o.ms[c] = 0;
  }
}

// One member tile's integer sums of one super-block (16 members x 16 rows, 4 a lane): ax holds
// the tile's four activation chunks; each is replaced by the next tile's (nx) once its MFMAs
// are issued, so the LDS reads of tile t+1 are in flight during tile t.
template <int DT, bool NEXT>
__device__ __forceinline__ void wide_mfma(v4i (&ax)[4], const uint8_t* nx, const uint32_t (&xo)[4], const WideB<DT>& B,
                                          v4i (&D)[3]) {
  D[0] = D[1] = D[2] = (v4i){0, 0, 0, 0};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    D[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[c], B.B[c], D[0], 0, 0, 0);
    D[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[c], B.B[4 + c], D[1], 0, 0, 0);
    if constexpr (DT == DT_Q4_K) {
      const int m = (int)B.ms[c];
      D[2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[c], ((v4i){m, m, m, m}), D[2], 0, 0, 0);
    }
    if constexpr (NEXT) ax[c] = *reinterpret_cast<const v4i*>(nx + xo[c]);
  }
}

// The f32 epilogue of one member tile and super-block (matmul.rs:242 Q4_K, :641 Q6_K).
template <int DT>
__device__ __forceinline__ void wide_epi(float (&acc)[4], const v4i (&D)[3], const float4 sx4, float d, float dm) {
  const float sxv[4] = {sx4.x, sx4.y, sx4.z, sx4.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (DT == DT_Q4_K) {
      const int sd = 8 * D[0][i] + D[1][i];
      acc[i] += sxv[i] * ((d * (float)sd) - (dm * (float)D[2][i]));
    } else {
      const int sv = 64 * D[0][i] + D[1][i];
      acc[i] += sxv[i] * (d * (float)sv);
    }
  }
}

// Chunk `tile` of the member chunks, enumerated class by class (every expert's chunks of 16
// member tiles, then those of 8, 4, 2 and 1), so the largest blocks come first in the grid.
struct WideTile {
  int e, m0, cnt, base, g, nt;
};

__device__ bool find_wide_tile(const RouteBufs& rb, int E, int tile, WideTile& wt, int32_t* sh) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int c = lane < E ? rb.counts[lane] : 0;
    const int st = (c + 15) >> 4;  // member tiles of the expert
    int n[WIDE_LOG + 1];
    n[0] = st >> WIDE_LOG;
#pragma unroll
    for (int k = 1; k <= WIDE_LOG; ++k) n[k] = (st >> (WIDE_LOG - k)) & 1;
    int before = 0;  // chunks of the classes enumerated before class k
    int m0 = 0;      // members of the expert's chunks of classes before k
#pragma unroll
    for (int k = 0; k <= WIDE_LOG; ++k) {
      int incl = n[k];
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
      }
      const int total = __shfl(incl, 63);
      const int excl = incl - n[k];
      if (lane < E && tile >= before + excl && tile < before + incl) {
        sh[0] = lane;
        sh[1] = m0 + (tile - before - excl) * (WIDE_NB >> k);
        sh[2] = c;
        sh[3] = rb.offsets[lane];
        sh[5] = (1 << WIDE_LOG) >> k;
      }
      before += total;
      m0 += n[k] * (WIDE_NB >> k);
    }
    if (lane == 63) sh[4] = before;
  }
  __syncthreads();
  if (tile >= sh[4]) return false;
  wt.e = __builtin_amdgcn_readfirstlane(sh[0]);
  wt.m0 = __builtin_amdgcn_readfirstlane(sh[1]);
  wt.g = __builtin_amdgcn_readfirstlane(sh[2]);
  wt.base = __builtin_amdgcn_readfirstlane(sh[3]);
  wt.nt = __builtin_amdgcn_readfirstlane(sh[5]);
  wt.cnt = min(16 * wt.nt, wt.g - wt.m0);
  return true;
}

struct WideSmem {
  uint8_t *xa0, *xa1;  // activation stages
  float *sxa0, *sxa1;
  uint8_t* trash;      // destination of the padding copies
  int32_t *rowidx, *outrow;
  uint64_t* exptab;
};

template <int DT, int KIND, int NT>
__device__ __forceinline__ void wide_body(const WideTile wt, const uint8_t* __restrict__ wpk, size_t stride_e,
                                          int n_rows, int n_in, int K, int n_out, int t64, const RouteBufs& rb, GemmX x,
                                          float* __restrict__ out, const WideSmem& sm) {
  constexpr int TB = GemmTraits<DT>::TB;
  constexpr int NM = 16 * NT;                    // members of the chunk (the last tile may be partial)
  constexpr int NW = WIDE_WAVES;
  constexpr int XOPS = (NT * 4 + NW - 1) / NW;   // activation copies of 1 KB per wave and super-block
  constexpr int SOPS = (NM + 63) / 64;           // scale copies (64 members each)
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, g = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(w);
  const int nb = n_in / QK;
  const int t16 = w & 3, row = 16 * t16 + r;
  const size_t tile_bytes = (size_t)nb * TB;
  // this lane's weight stream: its row in packed tile t64 of the expert
  const uint8_t* wtile = wpk + (size_t)wt.e * stride_e + (size_t)t64 * tile_bytes;
  const __amdgpu_buffer_rsrc_t rw = buf_rsrc(wtile, (uint32_t)tile_bytes);
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x.q, (uint32_t)n_rows * (uint32_t)n_in);
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(x.sx, (uint32_t)n_rows * (uint32_t)nb * 4u);
  const WideOff wo{(uint32_t)(16 * row), (uint32_t)(16 * row + 1024 * g), (uint32_t)(16 * row + 1024 * (g & 1)),
                   (uint32_t)(1024 * 13 + 2 * row)};
  WideW<DT> wq;
  wide_load<DT>(wq, rw, wo, 0);
  for (int n = tid; n < NM; n += blockDim.x) {
    const int pos = wt.base + wt.m0 + min(n, wt.cnt - 1);  // padding repeats the last member
    const int ent = rb.perm[pos];
    sm.rowidx[n] = KIND == GEMM_GATEUP ? ent / K : pos;
    sm.outrow[n] = n < wt.cnt ? (KIND == GEMM_GATEUP ? pos : ent) : -1;
  }
  lds_barrier();  // rowidx, outrow (and the exp table)
  // per-lane source offsets of the wave's activation copies (copy j = wv + NW·t: members 4j..4j+3)
  uint32_t xoff[XOPS];
#pragma unroll
  for (int t = 0; t < XOPS; ++t) {
    const int j = min(wv + NW * t, NT * 4 - 1), m = 4 * j + (lane >> 4), c = (lane & 15) ^ (m & 15);
    xoff[t] = (uint32_t)sm.rowidx[m] * (uint32_t)n_in + 16u * (uint32_t)c;
  }
  const uint32_t soff = (uint32_t)sm.rowidx[min(64 * min(wv, SOPS - 1) + lane, NM - 1)] * (uint32_t)nb * 4u;
  // every wave issues XOPS + 1 copies per super-block (short lists are padded with copies into
  // a scratch area)
  auto issue_x = [&](int b, uint8_t* xd, float* sd) {
#pragma unroll
    for (int t = 0; t < XOPS; ++t) {
      const int j = wv + NW * t;
      buf_dma16(rx, xoff[t], (uint32_t)(b * QK), j < NT * 4 ? xd + j * 1024 : sm.trash);
    }
    buf_dma4(rs, soff, (uint32_t)(4 * b), wv < SOPS ? reinterpret_cast<uint8_t*>(sd + 64 * wv) : sm.trash);
  };
  issue_x(0, sm.xa0, sm.sxa0);
  // per-lane LDS byte offsets of the activation chunk a lane reads at step c of a member tile
  uint32_t xo[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) xo[c] = (uint32_t)(r * QK + 16 * ((4 * c + g) ^ r));
  const float start = wt.g > 1 ? 0.0f : -0.0f;
  float acc[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[t][i] = start;
  WideB<DT> B0, B1;
  wide_build(wq, g, B0);
  // super-block b: activations in (xb, sb), operands in Bc; the copies of b+1 go to (xn, sn) and
  // its operands are built into Bn
  auto step = [&](int b, const uint8_t* xb, const float* sb, uint8_t* xn, float* sn, const WideB<DT>& Bc,
                  WideB<DT>& Bn) {
    // this wave's copies of super-block b landed, then every wave's; the barrier orders LDS only
    // (__syncthreads' release fence would also wait for the weight loads issued below)
    __builtin_amdgcn_s_waitcnt(0x3f70);
    lds_barrier();  // and the stages written next are no longer read
    if (b + 1 < nb) {
      wide_load<DT>(wq, rw, wo, (uint32_t)((b + 1) * TB));  // first: waiting for them leaves the copies in flight
      issue_x(b + 1, xn, sn);
    }
    v4i ax[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) ax[c] = *reinterpret_cast<const v4i*>(xb + xo[c]);
    v4i Dp[3];
    float4 sxp;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t == (NT + 1) / 2) {
        // the second half of the tiles hides the build of b+1's operands
        __builtin_amdgcn_sched_barrier(0);
        wide_build(wq, g, Bn);
      }
      v4i D[3];
      if (t + 1 < NT) wide_mfma<DT, true>(ax, xb + (t + 1) * 16 * QK, xo, Bc, D);
      else wide_mfma<DT, false>(ax, xb, xo, Bc, D);
      if (t > 0) wide_epi<DT>(acc[t - 1], Dp, sxp, Bc.d, Bc.dm);
#pragma unroll
      for (int k = 0; k < 3; ++k) Dp[k] = D[k];
      sxp = *reinterpret_cast<const float4*>(sb + t * 16 + 4 * g);
    }
    if constexpr (NT == 1) wide_build(wq, g, Bn);
    wide_epi<DT>(acc[NT - 1], Dp, sxp, Bc.d, Bc.dm);
  };
  for (int b = 0; b < nb; b += 2) {
    step(b, sm.xa0, sm.sxa0, sm.xa1, sm.sxa1, B0, B1);
    if (b + 1 >= nb) break;
    step(b + 1, sm.xa1, sm.sxa1, sm.xa0, sm.sxa0, B1, B0);
  }
  if constexpr (KIND == GEMM_GATEUP) {
    // the up waves hand their values to the gate waves of the same outputs (through the first
    // activation stage, no longer read after this barrier)
    __builtin_amdgcn_s_waitcnt(0x3f70);
    __syncthreads();
    const int k64 = w >> 2;
    float* upv = reinterpret_cast<float*>(sm.xa0);  // 2PT up waves x 4NT values x 64 lanes <= 64 KB
    if (t16 >= 2) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) upv[((k64 * 2 + (t16 - 2)) * (4 * NT) + t * 4 + i) * 64 + lane] = acc[t][i];
    }
    __syncthreads();
    if (t16 < 2) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = t * 16 + 4 * g + i;
          if (sm.outrow[n] < 0) continue;
          const float up = upv[((k64 * 2 + t16) * (4 * NT) + t * 4 + i) * 64 + lane];
          out[(size_t)sm.outrow[n] * n_out + 32 * t64 + 16 * t16 + r] = silu_tab(acc[t][i], sm.exptab) * up;
        }
    }
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = t * 16 + 4 * g + i;
        if (sm.outrow[n] < 0) continue;
        out[(size_t)sm.outrow[n] * n_out + 64 * t64 + 16 * t16 + r] = acc[t][i];
      }
  }
}

template <int DT, int KIND>
__global__ void __launch_bounds__(64 * WIDE_WAVES, 2) k_gemm_wide(const uint8_t* __restrict__ wpk, size_t stride_e, int n_rows, int n_in, int K,
                                                   int n_out, int E, RouteBufs rb, GemmX x, float* __restrict__ out) {
  // every stage a separate array: the compiler then knows a copy into one stage does not write
  // what is read from another, and waits for no copy in flight when it reads the current stage
  __shared__ __align__(16) uint8_t xa0[WIDE_XS], xa1[WIDE_XS];
  __shared__ __align__(16) float sxa0[WIDE_NB], sxa1[WIDE_NB];
  __shared__ __align__(16) uint8_t trash[1024];
  __shared__ int32_t rowidx[WIDE_NB], outrow[WIDE_NB];
  __shared__ int32_t sh[8];
  __shared__ uint64_t exptab[32];
  const uint64_t exp_e = KIND == GEMM_GATEUP ? exp_table_entry() : 0;
  // XCD k takes chunks k, k+8, ... and sweeps every row tile of one chunk before the next
  // (snake order), so a chunk's activations are fetched into that XCD's L2 once
  const int n_rt = gridDim.y, n_mt = gridDim.x;
  const int lin = blockIdx.y * n_mt + blockIdx.x;
  const int xcd = lin & 7, slot = lin >> 3;
  const int mt_local = slot / n_rt, rt_step = slot % n_rt;
  const int mtile = mt_local * 8 + xcd;
  const int rtile = (mt_local & 1) ? n_rt - 1 - rt_step : rt_step;
  WideTile wt;
  if (!find_wide_tile(rb, E, mtile, wt, sh)) return;
  if (KIND == GEMM_GATEUP && threadIdx.x < 32) exptab[threadIdx.x] = exp_e;  // published by wide_body's barrier
  const int t64 = WIDE_PT * rtile + (__builtin_amdgcn_readfirstlane(threadIdx.x) >> 8);
  const WideSmem sm{xa0, xa1, sxa0, sxa1, trash, rowidx, outrow, exptab};
  static_assert(WIDE_LOG == 4, "chunk sizes of the switch below");
  switch (wt.nt) {
    case 16: wide_body<DT, KIND, 16>(wt, wpk, stride_e, n_rows, n_in, K, n_out, t64, rb, x, out, sm); break;
    case 8: wide_body<DT, KIND, 8>(wt, wpk, stride_e, n_rows, n_in, K, n_out, t64, rb, x, out, sm); break;
    case 4: wide_body<DT, KIND, 4>(wt, wpk, stride_e, n_rows, n_in, K, n_out, t64, rb, x, out, sm); break;
    case 2: wide_body<DT, KIND, 2>(wt, wpk, stride_e, n_rows, n_in, K, n_out, t64, rb, x, out, sm); break;
    default: wide_body<DT, KIND, 1>(wt, wpk, stride_e, n_rows, n_in, K, n_out, t64, rb, x, out, sm); break;
  }
}

// Member tile (in units of 16 members): 16 for decode-sized batches (these tiles take their
// grouping from the selections), else 64; Q6_K rows take 128 when the groups fill such tiles
// on average. (A Q4_K block of 64 members leaves room for two blocks per CU, which beat one
// block of 128 members: 483 vs 554 µs for config 4's gate/up. A Q6_K block of 64 members
// still fills a CU's LDS alone.)
int gemm_member_tiles(int n_ent, int E) { return n_ent >= 16 * E ? 4 : 1; }

bool gateup16_applies(int dtype, int T, int H, int F, int E, int K, bool act_q8) {
  const int n_ent = T * K;
  return dtype == DT_Q4_K && act_q8 && gemm_member_tiles(n_ent, E) == 1 && T <= 16 && n_ent <= 64 && E <= 32 &&
         F % QK == 0 && (H == 2048 || H == 512);
}

bool down16_applies(int dtype, int T, int H, int F, int E, int K) {
  const int n_ent = T * K;
  return dtype == DT_Q4_K && gemm_member_tiles(n_ent, E) == 1 && T <= 16 && n_ent <= 64 && H % 256 == 0 &&
         F % QK == 0 && F / QK >= 1 && F / QK <= 8;
}

// ---- Q4_K gate/up of decode batches (at most 16 tokens): weight rows straight into registers -------
// Work unit = one expert x 16 outputs: the gate rows 16t.. and the up rows 32 + 16t.. of a 64-row
// packed tile (t = 0, 1), so one wave holds both values of its outputs and applies SwiGLU itself.
// Block = GU16_WAVES = 16 waves on 16 consecutive units of one expert, i.e. the expert's outputs
// 256j..256j+255 (unit = block·16 + wave, expert-major): E·F/256 blocks (224 for config 2's 32
// experts and F = 1792), one per CU, each CU the same work. The member tile is every token of
// the batch (outputs of tokens that did not choose the expert are computed and dropped), so its
// activations do not depend on the selections: all NB super-blocks of the tokens' Q8 rows
// (XOR-swizzled 16-byte chunks, as k_gemm stages them) and their scales are copied into LDS
// once, at the block's start, and shared by its waves. No wave reads another wave's weight rows,
// so a lane loads its 48 bytes per row and super-block (header and two qs words, the g-major
// order of q4_block) straight into registers, a super-block ahead, through a buffer resource
// on its packed tile (fixed per-lane offsets, the super-block's offset wave-uniform).
// The block's expert is known from its id, so its first weights are requested before the
// selections are read (a block of an expert nobody chose wastes them and leaves). The integer
// sums and the f32 epilogue are q4_block's, in the same order; the sum over super-blocks starts
// at +0.0 (-0.0 for an expert with one member).
// The block then also writes the Q8 of its members' act rows at super-block j (quantize_q8,
// model.rs:530-534, the k_quant_rows arithmetic) from its SwiGLU values gathered in LDS, so the
// down GEMM's input needs no launch of its own.
// Register slots of one row tile and super-block per lane: gate/up 3 (a super-block in flight
// while one half is computed), down 2 (k_down16: one half ahead). Deeper rings measured slower
// (config 2, same box, gate/up and down slots 5/5: 49.2 µs a step, 3/4: 48.2, 5/2: 48.3, 2/2:
// 47.4, 3/2: 46.85): the 224-256 blocks' first requests all go out at once, and the deeper the
// ring the longer the burst that delays the selection and activation reads behind it.
constexpr int GU16_SLOTS = 3;
constexpr int DN16_SLOTS = 2;
constexpr int GU16_WAVES = 16;

// A lane's bytes of one row tile and super-block (header and its two qs words). The wave streams
// its 2·NB (super-block, tile) halves through GU16_SLOTS register slots: half h is computed while
// halves h+1 .. h+GU16_SLOTS-1 are in flight.
struct Gu16H {
  uint4 h, q0, q1;
};

__device__ __forceinline__ void gu16_load(Gu16H& v, __amdgpu_buffer_rsrc_t r, uint32_t orow, uint32_t oq, uint32_t sb) {
  v.h = buf_load16nt(r, orow, sb);
  v.q0 = buf_load16nt(r, orow + oq, sb);
  v.q1 = buf_load16nt(r, orow + oq + 1024u, sb);
}

// One super-block of one of the wave's row tiles (header h, qs words q0 and q1) against the 16
// tokens: q4_block's three passes and epilogue.
__device__ __forceinline__ void gu16_tile(uint4 h, uint4 q0, uint4 q1, const uint8_t* xb, const float* sb,
                                          float (&acc)[4]) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const Q4Lane L = q4_lane(h, g);
  v4i Dh = {0, 0, 0, 0}, Dl = {0, 0, 0, 0}, Dm = {0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int hh = s >> 1;
    const v4i ax = read_x16(xb, r, 4 * g + s);
    v4i Bh, Bl;
    q4_step_ops((s & 1) ? q1 : q0, hh, L, Bh, Bl);
    const v4i Bm = {L.ms[hh], L.ms[hh], L.ms[hh], L.ms[hh]};
    Dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, Bh, Dh, 0, 0, 0);
    Dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, Bl, Dl, 0, 0, 0);
    Dm = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, Bm, Dm, 0, 0, 0);
  }
  const float4 sx4 = *reinterpret_cast<const float4*>(sb + 4 * g);
  const float sxv[4] = {sx4.x, sx4.y, sx4.z, sx4.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int sd = 8 * Dh[i] + Dl[i];
    acc[i] += sxv[i] * ((L.dd * (float)sd) - (L.dm * (float)Dm[i]));
  }
}

template <int NB>
__global__ void __launch_bounds__(64 * GU16_WAVES, 4) k_gateup16(const uint8_t* __restrict__ wpk, size_t stride_e,
                                                                int E, int K, int n_out, int n_tok,
                                                                const int32_t* __restrict__ sel, GemmX x,
                                                                float* __restrict__ out, int8_t* __restrict__ aq,
                                                                float* __restrict__ aq_sx, int act_pad) {
  constexpr int TB = (int)TB4;
  constexpr int XB = 16 * QK;  // one super-block of the 16 tokens' quants
  constexpr int NW = GU16_WAVES;
  constexpr int NC = (4 * NB + NW - 1) / NW;  // activation copies per wave
  __shared__ __align__(16) uint8_t xs[NB * XB];
  __shared__ __align__(16) float sxs[NW * 64];  // scales [b][16] (waves 0-1); the rest absorbs copies
  __shared__ uint64_t exptab[NW * 32];
  __shared__ int32_t selw[NW * 64];
  __shared__ __align__(16) float actv[16 * QK];  // the block's 256 outputs of each token
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_ot = n_out / 16;                 // units per expert
  const int unit = blockIdx.x * NW + w;
  const bool real = unit < E * n_ot;
  const int e = real ? unit / n_ot : 0, o = real ? unit % n_ot : 0;
  const int n_ent = n_tok * K;
  {
    // the exp table of the SwiGLU (32 x 8 bytes) and the selections (T*K <= 64 entries; their
    // workspace slot holds 64) into the wave's own LDS slots
    lds_dma4(reinterpret_cast<const uint8_t*>(bb_exp2f_tab_dev) + 4 * lane,
             reinterpret_cast<uint8_t*>(exptab + 32 * w));
    lds_dma4(reinterpret_cast<const uint8_t*>(sel + lane), reinterpret_cast<uint8_t*>(selw + 64 * w));
    // activation copies: NB super-blocks x 4 KB as 4·NB wave copies of 1 KB, copy j = super-block
    // j/4, tokens 4(j%4)..+3; wave w issues copies w, w+NW, ... (NC per wave; repeats of the last
    // copy rewrite the same bytes)
    const int m = lane >> 4, p = lane & 15;
#pragma unroll
    for (int t = 0; t < NC; ++t) {
      const int j = min(w + NW * t, 4 * NB - 1);
      const int b = j >> 2, mm = 4 * (j & 3) + m;
      const int row = min(mm, n_tok - 1);
      lds_dma16(reinterpret_cast<const uint8_t*>(x.q) + (size_t)row * (NB * QK) + b * QK + 16 * (p ^ mm),
                xs + j * 1024);
    }
    // scales: wave w < 2 copies entries 64w.. of [b][16]; the others copy into spare space
    const int u = min(64 * w + lane, 16 * NB - 1);
    const int row = min(u & 15, n_tok - 1);
    lds_dma4(reinterpret_cast<const uint8_t*>(x.sx + (size_t)row * NB + (u >> 4)),
             reinterpret_cast<uint8_t*>(sxs + 64 * w));
  }
  __builtin_amdgcn_sched_barrier(0);  // the copies stay ahead of the weight loads (vmcnt below)
  const int t64 = o >> 1, t16 = o & 1;
  const size_t tile_bytes = (size_t)NB * TB;
  const __amdgpu_buffer_rsrc_t rsrc =
      buf_rsrc(wpk + (size_t)e * stride_e + (size_t)t64 * tile_bytes, real ? (uint32_t)tile_bytes : 0u);
  // half h = (super-block h/2, row tile h%2: gate rows 16·t16.., up rows 32 + 16·t16..)
  const uint32_t og = 16u * (uint32_t)(16 * t16 + r), oq = 1024u * (uint32_t)(1 + 2 * g);
  constexpr int NH = 2 * NB, AHEAD = GU16_SLOTS - 1;
  auto half_load = [&](Gu16H& v, int h) { gu16_load(v, rsrc, og + 512u * (uint32_t)(h & 1), oq, (uint32_t)((h >> 1) * TB)); };
  Gu16H wr[GU16_SLOTS];
  // the first half goes out before the selections are known, the rest of the halves in flight
  // only once the expert is known to have members (an expert nobody chose then wastes one half
  // a wave instead of AHEAD)
  half_load(wr[0], 0);
  __builtin_amdgcn_sched_barrier(0);
  // this wave's copies landed (the weight loads issued after them may still be in flight)
  constexpr int WL = 3;
  __builtin_amdgcn_s_waitcnt(0x3f70 | (WL & 15) | ((WL >> 4) << 14));
  lds_barrier();
  // the expert's entries (entry i = token·K + slot on lane i), the entries of smaller expert ids
  // (the first group position of its members) and each token's group position
  const int sv = lane < n_ent ? selw[64 * w + lane] : -1;
  const unsigned long long me = __ballot(sv == e);
  const int cnt = __popcll(me);
  if (!real || cnt == 0) {
    __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
    return;
  }
#pragma unroll
  for (int h = 1; h < AHEAD; ++h)
    if (h < NH) half_load(wr[h], h);
  __builtin_amdgcn_sched_barrier(0);
  const int base = __popcll(__ballot(sv >= 0 && sv < e));
  const unsigned long long kmask = K >= 64 ? ~0ull : (1ull << K) - 1ull;
  int orow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = 4 * g + i;
    orow[i] = -1;
    if (n < n_tok) {
      const unsigned long long bits = (me >> (n * K)) & kmask;
      if (bits) {
        const int ii = n * K + __builtin_ctzll(bits);
        orow[i] = base + __popcll(me & ((1ull << ii) - 1ull));
      }
    }
  }
  const float start = cnt > 1 ? 0.0f : -0.0f;
  float acc[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[t][i] = start;
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    // the slot half h-1 used takes half h+AHEAD
    if (h + AHEAD < NH) half_load(wr[(h + AHEAD) % GU16_SLOTS], h + AHEAD);
    __builtin_amdgcn_sched_barrier(0);
    const Gu16H& cur = wr[h % GU16_SLOTS];
    gu16_tile(cur.h, cur.q0, cur.q1, xs + (h >> 1) * XB, sxs + 16 * (h >> 1), acc[h & 1]);
    // the sums are formed here (the compiler would otherwise sink every super-block's epilogue
    // into the conditional stores below and keep all their integer sums live)
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[h & 1][i]));
    __builtin_amdgcn_sched_barrier(0);
  }
  const int col = 32 * t64 + 16 * t16 + r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (orow[i] < 0) continue;
    const float a = silu_tab(acc[0][i], exptab + 32 * w) * acc[1][i];
    out[(size_t)orow[i] * n_out + col] = a;
    actv[(4 * g + i) * QK + (col & (QK - 1))] = a;
  }
  // wave n quantises token n's 256 values when the token chose the expert (the block's outputs
  // are super-block col / 256 of the expert's act rows)
  lds_barrier();
  const int n = w;
  if (n < n_tok) {
    const unsigned long long bits = (me >> (n * K)) & kmask;
    if (bits) {
      const int ii = n * K + __builtin_ctzll(bits);
      const int mi = __popcll(me & ((1ull << ii) - 1ull));  // the entry's rank among the expert's
      const int row = act_pad ? 16 * e + mi : base + mi;
      const int jb = col / QK;
      const float4 v = *reinterpret_cast<const float4*>(actv + n * QK + 4 * lane);
      wave_quantize_xq(v, aq + (size_t)row * n_out + jb * QK, aq_sx + (size_t)row * (n_out / QK) + jb, nullptr);
    }
  }
}

// ---- Q4_K down of decode batches (at most 16 members per expert): weight rows into registers ------
// k_gateup16's form for the down GEMM. Work unit = one expert x 16 output rows (a quarter of a
// 64-row packed tile); block = GU16_WAVES waves on the expert's rows 256j..256j+255, H/256 blocks
// per expert, expert-major. A token chooses an expert at most once, so an expert of a batch of at
// most 16 tokens has at most 16 members: its entries in ascending order, whose Q8 act rows are the
// group positions base..base+cnt-1 (the order k_gateup16 and k_quant_rows write them in). The
// block requests its first weights from its id, reads the selections, copies its members' act
// rows (all NB super-blocks, XOR-swizzled chunks as k_gemm stages them) and their scales into LDS,
// and streams the rest of its weights through the register ring while it computes. The integer
// sums and the f32 epilogue are q4_block's (gu16_tile), from +0.0 (-0.0 for an expert with one
// member, as k_gemm); member m's outputs go to the slot row of its entry.
template <int NB>
__global__ void __launch_bounds__(64 * GU16_WAVES, 4) k_down16(const uint8_t* __restrict__ wpk, size_t stride_e,
                                                              int n_out, int n_ent,
                                                              const int32_t* __restrict__ sel, GemmX x,
                                                              float* __restrict__ out, int act_pad) {
  constexpr int TB = (int)TB4;
  constexpr int XB = 16 * QK;  // one super-block of 16 members' quants
  constexpr int NW = GU16_WAVES;
  constexpr int NC = (4 * NB + NW - 1) / NW;  // activation copies per wave
  __shared__ __align__(16) uint8_t xs[NB * XB];
  __shared__ __align__(16) float sxs[NW * 64];  // scales [b][16] (waves 0-1); the rest absorbs copies
  __shared__ int32_t selw[NW * 64];
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bpe = n_out / (16 * NW);          // blocks per expert
  const int e = blockIdx.x / bpe;
  const int o = (blockIdx.x % bpe) * NW + w;  // the wave's 16-row group of the expert
  const int t64 = o >> 2, t16 = o & 3;
  // the selections (T*K <= 64 entries; their workspace slot holds 64) into the wave's own slots
  lds_dma4(reinterpret_cast<const uint8_t*>(sel + lane), reinterpret_cast<uint8_t*>(selw + 64 * w));
  // act copies: NB super-blocks x 4 KB as 4·NB wave copies of 1 KB, copy j = super-block j/4,
  // members 4(j%4)..+3; wave w issues copies w, w+NW, ... (repeats of the last copy rewrite the
  // same bytes). Member m's row: 16e + m with act_pad (rows past the expert's members hold
  // whatever was there; their outputs are not stored), else group position first + m (members
  // past the last repeat its row).
  auto act_copies = [&](int first, int cnt) {
    const int m = lane >> 4, p = lane & 15;
#pragma unroll
    for (int t = 0; t < NC; ++t) {
      const int j = min(w + NW * t, 4 * NB - 1);
      const int b = j >> 2, mm = 4 * (j & 3) + m;
      const int row = first + min(mm, cnt - 1);
      lds_dma16(reinterpret_cast<const uint8_t*>(x.q) + (size_t)row * (NB * QK) + b * QK + 16 * (p ^ mm),
                xs + j * 1024);
    }
    // scales: wave w < 2 copies entries 64w.. of [b][16]; the others copy into spare space
    const int u = min(64 * w + lane, 16 * NB - 1);
    const int row = first + min(u & 15, cnt - 1);
    lds_dma4(reinterpret_cast<const uint8_t*>(x.sx + (size_t)row * NB + (u >> 4)),
             reinterpret_cast<uint8_t*>(sxs + 64 * w));
  };
  if (act_pad) act_copies(16 * e, 16);
  const size_t tile_bytes = (size_t)NB * TB;
  const __amdgpu_buffer_rsrc_t rsrc = buf_rsrc(wpk + (size_t)e * stride_e + (size_t)t64 * tile_bytes,
                                               (uint32_t)tile_bytes);
  // half h = super-block h of the wave's 16 rows
  const uint32_t og = 16u * (uint32_t)(16 * t16 + r), oq = 1024u * (uint32_t)(1 + 2 * g);
  constexpr int AHEAD = DN16_SLOTS - 1;
  auto half_load = [&](Gu16H& v, int h) { gu16_load(v, rsrc, og, oq, (uint32_t)(h * TB)); };
  Gu16H wr[DN16_SLOTS];
  half_load(wr[0], 0);
  __builtin_amdgcn_sched_barrier(0);
  // this wave's selection copy (and act copies) landed (the weight loads issued after them may
  // still be in flight)
  constexpr int WS = 3;
  __builtin_amdgcn_s_waitcnt(0x3f70 | (WS & 15) | ((WS >> 4) << 14));
  // the expert's entries (entry i on lane i) and the entries of smaller expert ids (the first
  // group position of its members)
  const int sv = lane < n_ent ? selw[64 * w + lane] : -1;
  const unsigned long long me = __ballot(sv == e);
  const int cnt = __popcll(me);  // the same in every wave of the block
  if (cnt == 0) {
    __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
    return;
  }
  if (!act_pad) act_copies(__popcll(__ballot(sv >= 0 && sv < e)), cnt);
  constexpr int NL = AHEAD - 1 < NB - 1 ? AHEAD - 1 : NB - 1;  // halves requested after the copies
#pragma unroll
  for (int h = 1; h <= NL; ++h) half_load(wr[h], h);
  __builtin_amdgcn_sched_barrier(0);
  // this wave's copies landed (the weight loads issued after them may still be in flight)
  constexpr int WL = 3 * NL;
  __builtin_amdgcn_s_waitcnt(0x3f70 | (WL & 15) | ((WL >> 4) << 14));
  lds_barrier();
  const float start = cnt > 1 ? 0.0f : -0.0f;
  float acc[4] = {start, start, start, start};
#pragma unroll
  for (int h = 0; h < NB; ++h) {
    // the slot half h-1 used takes half h+AHEAD
    if (h + AHEAD < NB) half_load(wr[(h + AHEAD) % DN16_SLOTS], h + AHEAD);
    __builtin_amdgcn_sched_barrier(0);
    const Gu16H& cur = wr[h % DN16_SLOTS];
    gu16_tile(cur.h, cur.q0, cur.q1, xs + h * XB, sxs + 16 * h, acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[i]));
    __builtin_amdgcn_sched_barrier(0);
  }
  const int col = 64 * t64 + 16 * t16 + r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = 4 * g + i;  // member n: the n-th entry of the expert
    if (n >= cnt) continue;
    unsigned long long rest = me;
    for (int k = 0; k < n; ++k) rest &= rest - 1ull;
    out[(size_t)__builtin_ctzll(rest) * n_out + col] = acc[i];
  }
}

// Q6_K down GEMMs whose groups hold this many members on average take k_gemm_wide (blocks of up
// to 256 members). For config 4 (4096 tokens, Zipf-skewed groups) it runs the Q6_K down GEMM in
// 228 µs against k_gemm's 274; the Q4_K gate/up GEMM, whose 3-pass epilogue and operand build
// are heavier, runs in 578 µs against k_gemm's 442 at its two waves per SIMD, so gate/up and Q4_K
// rows stay on k_gemm.
constexpr int WIDE_MIN_AVG = 192;

template <int DT, int KIND>
static hipError_t launch_gemm(hipStream_t s, const uint8_t* w, size_t stride_e, int T, int n_in, int n_out,
                              int n_t64, int E, int K, const RouteBufs& rb, GemmX x, float* out,
                              int8_t* aq = nullptr, float* aq_sx = nullptr, bool* quantized = nullptr,
                              bool act_pad = false) {
  if (quantized) *quantized = false;
  const int n_ent = T * K;
  if constexpr (DT == DT_Q6_K && KIND == GEMM_DOWN) {
    // (the kernel addresses x with 32-bit byte offsets)
    if (n_ent >= WIDE_MIN_AVG * E && (uint64_t)n_ent * (uint64_t)n_in < (1ull << 31)) {
      // chunks: the expert's c members give at most c/256 chunks of 16 member tiles (summed
      // over experts: n_ent/256 + E) and one chunk of each smaller size
      const int n_mt = (n_ent / WIDE_NB + (WIDE_LOG + 1) * E + 7) / 8 * 8;
      BB_LAUNCH((k_gemm_wide<DT, KIND>), dim3(n_mt, n_t64 / WIDE_PT), dim3(64 * WIDE_WAVES), 0, s, w, stride_e, n_ent,
                n_in, K, n_out, E, rb, x, out);
      return hipGetLastError();
    }
  }
  int mt = DT == DT_Q6_K && n_ent >= 128 * E ? 8 : gemm_member_tiles(n_ent, E);
  // Q4_K groups of 48+ members on average: member tiles of 80 (groups of 64 +- 8 then take one
  // tile where tiles of 64 often took a second one nearly empty); one group of known size takes
  // the tile that pads it less
  // (launches that read the min-term records keep tiles of 64: with the records' LDS and the f16
  // pass's registers, tiles of 80 fit one block per SIMD pair less)
  const bool ms = x.ms && gemm_reads_ms(DT, n_ent, E);
  if (DT == DT_Q4_K && mt == 4 && n_ent >= 48 * E && !ms)
    mt = E > 1 || (n_ent + 79) / 80 * 5 < (n_ent + 63) / 64 * 4 ? 5 : 4;
  if constexpr (DT == DT_Q4_K && KIND == GEMM_GATEUP) {
    // decode batches of at most 16 tokens: k_gateup16 (input rows of 512 or 2048), which also
    // quantises the act rows into the caller's buffers
    if (rb.sel && gateup16_applies(DT, T, n_in, n_out, E, K, aq != nullptr)) {
      const dim3 grid(E * (n_out / QK)), block(64 * GU16_WAVES);
      if (n_in == 2048)
        BB_LAUNCH(k_gateup16<8>, grid, block, 0, s, w, stride_e, E, K, n_out, T, rb.sel, x, out, aq, aq_sx,
                  (int)act_pad);
      else
        BB_LAUNCH(k_gateup16<2>, grid, block, 0, s, w, stride_e, E, K, n_out, T, rb.sel, x, out, aq, aq_sx,
                  (int)act_pad);
      if (quantized) *quantized = true;
      return hipGetLastError();
    }
  }
  if constexpr (DT == DT_Q4_K && KIND == GEMM_DOWN) {
    // decode batches of at most 16 tokens (an expert then has at most 16 members): k_down16
    if (rb.sel && down16_applies(DT, T, n_out, n_in, E, K)) {
      const dim3 grid(E * (n_out / 256)), block(64 * GU16_WAVES);
      switch (n_in / QK) {
#define BB_DOWN16(nb) \
  case nb: BB_LAUNCH(k_down16<nb>, grid, block, 0, s, w, stride_e, n_out, n_ent, rb.sel, x, out, (int)act_pad); break;
        BB_DOWN16(1) BB_DOWN16(2) BB_DOWN16(3) BB_DOWN16(4) BB_DOWN16(5) BB_DOWN16(6) BB_DOWN16(7) BB_DOWN16(8)
#undef BB_DOWN16
      }
      return hipGetLastError();
    }
  }
  const int bn = 16 * mt;
  // enough member tiles: with tiles of 16, ceil(T/16) per expert (an expert has at most T
  // members); else every hit expert adds at most one partial tile
  const int n_mt = mt == 1 ? E * ((T + bn - 1) / bn) : ((n_ent + bn - 1) / bn + E + 7) / 8 * 8;
  dim3 grid(n_mt, n_t64 / 2);
  // copies through buffer resources when every source offset fits 31 bits
  const uint64_t x_rows = KIND == GEMM_GATEUP ? (uint64_t)T : (uint64_t)n_ent;
  const uint64_t tile2 = 2ull * (uint64_t)(n_in / QK) * (uint64_t)GemmTraits<DT>::TB;
  const bool buf = x_rows * (uint64_t)n_in < (1ull << 31) && tile2 < (1ull << 31);
  if (DT == DT_Q6_K && mt == 8 && buf)
    BB_LAUNCH((k_gemm<DT_Q6_K, KIND, 8, true>), grid, dim3(512), 0, s, w, stride_e, n_in, K, n_out, E, n_ent, rb, x,
              out);
  else if (DT == DT_Q6_K && mt == 8)
    BB_LAUNCH((k_gemm<DT_Q6_K, KIND, 8>), grid, dim3(512), 0, s, w, stride_e, n_in, K, n_out, E, n_ent, rb, x, out);
  else if (DT == DT_Q4_K && mt == 5 && buf)
    BB_LAUNCH((k_gemm<DT_Q4_K, KIND, 5, true>), grid, dim3(512), 0, s, w, stride_e, n_in, K, n_out, E, n_ent, rb, x,
              out);
  else if (DT == DT_Q4_K && mt == 5)
    BB_LAUNCH((k_gemm<DT_Q4_K, KIND, 5>), grid, dim3(512), 0, s, w, stride_e, n_in, K, n_out, E, n_ent, rb, x, out);
  else if (DT == DT_Q4_K && mt == 4 && buf && ms)
    BB_LAUNCH((k_gemm<DT_Q4_K, KIND, 4, true, true>), grid, dim3(512), 0, s, w, stride_e, n_in, K, n_out, E, n_ent,
              rb, x, out);
  else if (mt == 4 && buf)
    BB_LAUNCH((k_gemm<DT, KIND, 4, true>), grid, dim3(512), 0, s, w, stride_e, n_in, K, n_out, E, n_ent, rb, x, out);
  else if (mt == 4)
    BB_LAUNCH((k_gemm<DT, KIND, 4>), grid, dim3(512), 0, s, w, stride_e, n_in, K, n_out, E, n_ent, rb, x, out);
  else
    BB_LAUNCH((k_gemm<DT, KIND, 1>), grid, dim3(512), 0, s, w, stride_e, n_in, K, n_out, E, n_ent, rb, x, out);
  return hipGetLastError();
}

hipError_t launch_gemm_gateup(hipStream_t s, int dtype, const uint8_t* gu, size_t stride_gu, int T, int H, int F,
                              int E, int K, const RouteBufs& rb, GemmX x, float* act, int8_t* aq, float* aq_sx,
                              bool* quantized, bool act_pad) {
  // act_pad: only where k_gateup16 and k_down16 both run (the act rows' layout is theirs)
  if (act_pad && !(gateup16_applies(dtype, T, H, F, E, K, aq != nullptr) && rb.sel)) return hipErrorInvalidValue;
  if (dtype == DT_Q4_K)
    return launch_gemm<DT_Q4_K, GEMM_GATEUP>(s, gu, stride_gu, T, H, F, F / 32, E, K, rb, x, act, aq, aq_sx, quantized,
                                             act_pad);
  return launch_gemm<DT_Q6_K, GEMM_GATEUP>(s, gu, stride_gu, T, H, F, F / 32, E, K, rb, x, act, aq, aq_sx, quantized);
}

hipError_t launch_gemm_down(hipStream_t s, int dtype, const uint8_t* dn, size_t stride_dn, int T, int H, int F, int E,
                            int K, const RouteBufs& rb, GemmX x, float* slots, bool act_pad) {
  if (act_pad && !(down16_applies(dtype, T, H, F, E, K) && rb.sel)) return hipErrorInvalidValue;
  if (dtype == DT_Q4_K)
    return launch_gemm<DT_Q4_K, GEMM_DOWN>(s, dn, stride_dn, T, F, H, H / 64, E, K, rb, x, slots, nullptr, nullptr,
                                           nullptr, act_pad);
  return launch_gemm<DT_Q6_K, GEMM_DOWN>(s, dn, stride_dn, T, F, H, H / 64, E, K, rb, x, slots);
}

// ---- one group of T tokens (dense projections on the grouped GEMM) ----------------------------------
__global__ void __launch_bounds__(256) k_one_group(int T, RouteBufs rb) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < T) rb.perm[i] = i;
  if (i == 0) {
    rb.counts[0] = T;
    rb.offsets[0] = 0;
    rb.offsets[1] = T;
  }
}

hipError_t launch_one_group(hipStream_t s, int T, RouteBufs rb) {
  if (T < 1) return hipErrorInvalidValue;
  BB_LAUNCH(k_one_group, dim3((unsigned)((T + 255) / 256)), dim3(256), 0, s, T, rb);
  return hipGetLastError();
}

// ---- Q8 rows ---------------------------------------------------------------------------------------
// One wave per 256-block: amax, scale amax/127, quants round(v·127/amax) (kernels/matmul.rs:141-160).
__global__ void __launch_bounds__(256) k_quant_rows(const float* __restrict__ x, size_t n_rows, int n,
                                                    int8_t* __restrict__ q, float* __restrict__ sx,
                                                    uint16_t* __restrict__ ms) {
  const int lane = threadIdx.x & 63;
  const size_t nbk = n / QK;
  const size_t wi = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wi >= n_rows * nbk) return;
  const float4 v = *reinterpret_cast<const float4*>(x + wi * QK + 4 * lane);
  wave_quantize_xq(v, q + wi * QK, sx + wi, nullptr, ms ? ms + wi * 16 : nullptr);
}

hipError_t launch_quant_rows(hipStream_t s, const float* x, size_t n_rows, int n, int8_t* q, float* sx,
                             uint16_t* ms) {
  const size_t waves = n_rows * (size_t)(n / QK);
  if (waves == 0) return hipSuccess;
  BB_LAUNCH(k_quant_rows, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, x, n_rows, n, q, sx, ms);
  return hipGetLastError();
}

}  // namespace bb
