// bb_decode.hip — the MoE block for decode / small batches (T·k <= 1024 entries).
//
// Four kernels; no block ever waits on another inside a kernel (on gfx950 an agent-scope
// fence writes back and invalidates the whole L2), so kernel boundaries are the only hand-offs:
//   k_route         router logits, gating (sigmoid, top-k, renormalisation) and the XQ record
//                   of x, one block per token                                     (model.rs:484-501)
//   k_experts       gate and up rows of the hit experts, SwiGLU, for the entries that
//     <GATEUP>      selected each expert                                           (model.rs:504-524)
//   k_experts       Q8 of the experts' act rows, then their down rows             (model.rs:529-548)
//     <DOWN>
//   k_combine       out[t] = Σ_k w[t,k]·down[t,k] in selection order              (model.rs:550-553)
// The GEMV kernels run one weight row per lane: each of the 8 waves of a block owns one
// 256-weight super-block of the tile's 64 rows, computes its exact value for every member,
// and lanes sum the per-block values left to right through LDS. Blocks walk an equal share of
// (expert, tile) units with the next unit's weights in flight, so HBM streams while the SIMDs
// compute.
#include "bb_internal.h"
#include "bb_members.h"
#include "bb_rowlane.h"
#include "bb_gating.h"

namespace bb {

// ---- router + gating + XQ of x ------------------------------------------------------------------
// Block of 1024 threads for tpb consecutive tokens. The router dot (matmul.rs:36-66) runs as 32
// fmaf chains per (token, expert), chain c over the elements i = c mod 32, then the lane combine
// (acc0+acc1)+(acc2+acc3) and reduce_add ((v0+v4)+(v2+v6))+((v1+v5)+(v3+v7)). Lane (e, h) of
// wave w runs chain c = 2w + h of expert e for every token, its 64 router values in registers
// (the router is held regrouped so these loads are contiguous per chain); the token's x is
// staged in LDS transposed, chain-major, so the 32 lanes of a half-wave read the same 16 bytes
// (a broadcast) for four steps of their chains. Each token's 32 x 32 chain values meet in LDS and
// one lane per expert adds them in the reference's tree order.
//
// Then half-wave i gates token i (gate_halfwave). The XQ records (model.rs:501; the pair dwords
// only when xq.pairs is set) are written from the staged rows while the gating runs.
constexpr int ROUTE_TPB_MAX = 16;
constexpr int XT_STRIDE = GU_H_MAX / 32 + 4;  // a chain's row in LDS, padded: chains c, c+1 on other banks

__global__ void __launch_bounds__(1024) k_route(const float* __restrict__ Wr, const float* __restrict__ bias,
                                                const float* __restrict__ x, int T, int H, int E, int K, int tpb,
                                                XQBufs xq, RouteBufs rb) {
  __shared__ __align__(16) float xT[ROUTE_TPB_MAX][32][XT_STRIDE];
  __shared__ float part[2][32][33];  // a token's chain values [expert][chain], two tokens in turn
  __shared__ float lg[ROUTE_TPB_MAX][32];
  __shared__ uint64_t exptab[32];
  const uint64_t exp_e = exp_table_entry();
  const int t0 = blockIdx.x * tpb, nt = min(tpb, T - t0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e = lane & 31, c = 2 * wave + (lane >> 5);  // this lane's expert and chain
  const int nm4 = H / 128;                             // float4 steps of a chain
  const int nbx = H / QK;
  const float bias_c = bias[min(e, E - 1)];
  // the block's x rows, 4 elements per thread and step, written transposed: xT[tk][i % 32][i / 32]
  constexpr int XSTEPS = ROUTE_TPB_MAX * GU_H_MAX / 4 / 1024;
  float4 xr[XSTEPS];
  const int nq = H / 4, n_x = nt * nq;
  // every load is unconditional, its index clamped into bounds (values of steps past H/128 and
  // of experts past E are not used), so the loads go out together
#pragma unroll
  for (int k = 0; k < XSTEPS; ++k)
    xr[k] = reinterpret_cast<const float4*>(x)[(size_t)t0 * nq + min(k * 1024 + tid, n_x - 1)];
  float4 wv[GU_H_MAX / 128];
  const float4* wr = reinterpret_cast<const float4*>(Wr) + (size_t)c * nm4 * E + min(e, E - 1);
#pragma unroll
  for (int k = 0; k < GU_H_MAX / 128; ++k) wv[k] = wr[(size_t)min(k, nm4 - 1) * E];
#pragma unroll
  for (int k = 0; k < XSTEPS; ++k) {
    const int idx = k * 1024 + tid;
    if (idx < n_x) {
      const int tk = idx / nq, i = 4 * (idx % nq), cc = i & 31, m = i >> 5;
      xT[tk][cc][m] = xr[k].x;
      xT[tk][cc + 1][m] = xr[k].y;
      xT[tk][cc + 2][m] = xr[k].z;
      xT[tk][cc + 3][m] = xr[k].w;
    }
  }
  if (tid < 32) exptab[tid] = exp_e;
  __syncthreads();
  for (int tk = 0; tk < nt; ++tk) {
    const float* xc = xT[tk][c];
    // the steps' x is read eight float4 at a time, unconditionally (the row is GU_H_MAX long;
    // steps past H/128 are not used), so the reads are issued together
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < GU_H_MAX / 1024; ++h) {
      float4 xv[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) xv[k] = *reinterpret_cast<const float4*>(xc + 32 * h + 4 * k);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (8 * h + k < nm4) {
          const float4 w = wv[8 * h + k];
          acc = fmaf(w.x, xv[k].x, acc);
          acc = fmaf(w.y, xv[k].y, acc);
          acc = fmaf(w.z, xv[k].z, acc);
          acc = fmaf(w.w, xv[k].w, acc);
        }
      }
    }
    part[tk & 1][e][c] = acc;
    lds_barrier();  // (not __syncthreads: it would wait for the logits stores in flight)
    if (wave == (tk & 15) && lane < E) {
      const float* p = part[tk & 1][lane];
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (p[j] + p[j + 8]) + (p[j + 16] + p[j + 24]);
      const float r = ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
      lg[tk][lane] = r;
      rb.logits[(size_t)(t0 + tk) * E + lane] = r;
    }
  }
  lds_barrier();
  // half-wave i gates token t0 + i
  if (2 * wave < nt) {
    const int i = tid >> 5;
    const bool tok = i < nt, live = tok && e < E;
    gate_halfwave(live ? lg[i][e] : 0.0f, live, tok, bias_c, t0 + i, E, K, exptab, rb);
  }
  // XQ records of the staged rows, one wave per 256-block: the waves that gate nothing first
  const int first = (nt + 1) / 2;  // waves 0 .. first-1 gate
  for (int task = (wave + 16 - first) % 16; task < nt * nbx; task += 16) {
    const int tk = task / nbx, bk = task % nbx, t = t0 + tk;
    const int i0 = bk * QK + 4 * lane;  // elements i0 .. i0+3: chains (i0 % 32) + j, step i0 / 32
    const float* col = &xT[tk][i0 & 31][i0 >> 5];
    const float4 v = make_float4(col[0], col[XT_STRIDE], col[2 * XT_STRIDE], col[3 * XT_STRIDE]);
    wave_quantize_xq(v, xq.q + (size_t)t * H + bk * QK, xq.sx + (size_t)t * nbx + bk,
                     xq.pairs ? xq.pairs + ((size_t)t * nbx + bk) * 12 : nullptr,
                     xq.ms ? xq.ms + ((size_t)t * nbx + bk) * 16 : nullptr);
  }
}

// ---- route inside the gate/up GEMV block (a few tokens) ------------------------------------------
// For a few tokens the route is recomputed by every block of the gate/up GEMV instead of in a
// kernel of its own: the router (256 KB) is read from L2 once per block, and the blocks learn
// their experts without a launch and a round trip through memory in between. The arithmetic is
// k_route's (the same fmaf chains over the same elements, x staged transposed in LDS, one lane
// per expert adding the 32 chain values in the tree order, gate_halfwave) on 512 threads. The
// XQ records of the tokens are built in LDS. Block 0 writes the route's
// outputs (logits, selections, weights, margins, ties) for the kernels after it.
constexpr int RT_MAX = ROUTE_IN_GATEUP_MAX_T;
struct SmemRoute {
  float xT[RT_MAX][32][XT_STRIDE];
  float xdummy[64 + 3 * XT_STRIDE];  // where lanes past the rows store (keeps the stores unconditional)
  float part[2][32][33];
  float lg[RT_MAX][32];
  int32_t sel[RT_MAX * 8];
  int8_t q[RT_MAX][GU_H_MAX];
  uint32_t pairs[RT_MAX][GU_H_MAX / QK][12];
  float sx[RT_MAX][GU_H_MAX / QK];
};

// One token gated in the block (RM_GATE, T = 1): the token's XQ record, copied into LDS at the
// block's start so the dots do not wait for its reads after the weights (the spare tails take
// the copies' clamped lanes).
struct SmemXrec {
  int8_t q[GU_H_MAX];
  uint32_t pairs[128];  // [GU_H_MAX / QK][12]
  float sx[64];         // [GU_H_MAX / QK]
};

__device__ void route_block(const float* __restrict__ Wr, const float* __restrict__ bias, const float* __restrict__ x,
                            int T, int H, int E, int K, bool global_out, RouteBufs rb, SmemRoute& sm,
                            uint64_t* exptab, uint64_t exp_e) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // lane group g (16 lanes) of wave w runs chain c = 4w + g of experts e0 = lane % 16 and
  // e0 + 16: one read of x from LDS serves two experts
  const int c = 4 * wave + (lane >> 4), e0 = lane & 15, e1 = e0 + 16;
  const int nm4 = H / 128, nq = H / 4, n_x = T * nq, nbx = H / QK;
  // every load is unconditional, its index clamped into bounds (values of steps past H/128 and
  // of experts past E are not used), so the loads go out together, x first
  const float bias_i = bias[min(tid & 31, E - 1)];
  constexpr int XSTEPS = RT_MAX * GU_H_MAX / 4 / 512;
  float4 xr[XSTEPS];
#pragma unroll
  for (int k = 0; k < XSTEPS; ++k) xr[k] = reinterpret_cast<const float4*>(x)[min(k * 512 + tid, n_x - 1)];
  float4 wa[GU_H_MAX / 128], wb[GU_H_MAX / 128];
  const float4* wr = reinterpret_cast<const float4*>(Wr) + (size_t)c * nm4 * E;
  const int ea = min(e0, E - 1), eb = min(e1, E - 1);
#pragma unroll
  for (int k = 0; k < GU_H_MAX / 128; ++k) {
    const int kc = min(k, nm4 - 1);
    wa[k] = wr[(size_t)kc * E + ea];
    wb[k] = wr[(size_t)kc * E + eb];
  }
#pragma unroll
  for (int k = 0; k < XSTEPS; ++k) {
    const int idx = k * 512 + tid;
    const int tk = idx / nq, i = 4 * (idx % nq), cc = i & 31, m = i >> 5;
    float* dst = idx < n_x ? &sm.xT[tk][cc][m] : sm.xdummy + lane;
    dst[0] = xr[k].x;
    dst[XT_STRIDE] = xr[k].y;
    dst[2 * XT_STRIDE] = xr[k].z;
    dst[3 * XT_STRIDE] = xr[k].w;
  }
  if (tid < 32) exptab[tid] = exp_e;
  lds_barrier();  // (LDS only: the router loads stay in flight)
  // the XQ records of the tokens in LDS, one wave per 256-block, while the router arrives
  for (int task = wave; task < T * nbx; task += 8) {
    const int tk = task / nbx, bk = task % nbx;
    const int i0 = bk * QK + 4 * lane;
    const float* col = &sm.xT[tk][i0 & 31][i0 >> 5];
    const float4 v = make_float4(col[0], col[XT_STRIDE], col[2 * XT_STRIDE], col[3 * XT_STRIDE]);
    wave_quantize_xq(v, sm.q[tk] + bk * QK, &sm.sx[tk][bk], sm.pairs[tk][bk]);
  }
  for (int tk = 0; tk < T; ++tk) {
    const float* xc = sm.xT[tk][c];
    float acc_a = 0.0f, acc_b = 0.0f;
#pragma unroll
    for (int h = 0; h < GU_H_MAX / 1024; ++h) {
      float4 xv[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) xv[k] = *reinterpret_cast<const float4*>(xc + 32 * h + 4 * k);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (8 * h + k < nm4) {
          const float4 wa4 = wa[8 * h + k], wb4 = wb[8 * h + k];
          acc_a = fmaf(wa4.x, xv[k].x, acc_a);
          acc_a = fmaf(wa4.y, xv[k].y, acc_a);
          acc_a = fmaf(wa4.z, xv[k].z, acc_a);
          acc_a = fmaf(wa4.w, xv[k].w, acc_a);
          acc_b = fmaf(wb4.x, xv[k].x, acc_b);
          acc_b = fmaf(wb4.y, xv[k].y, acc_b);
          acc_b = fmaf(wb4.z, xv[k].z, acc_b);
          acc_b = fmaf(wb4.w, xv[k].w, acc_b);
        }
      }
    }
    sm.part[tk & 1][e0][c] = acc_a;
    sm.part[tk & 1][e1][c] = acc_b;
    lds_barrier();
    if (wave == (tk & 7) && lane < E) {
      const float* p = sm.part[tk & 1][lane];
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (p[j] + p[j + 8]) + (p[j + 16] + p[j + 24]);
      const float r = ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
      sm.lg[tk][lane] = r;
      if (global_out) rb.logits[(size_t)tk * E + lane] = r;
    }
  }
  lds_barrier();
  if (2 * wave < T) {  // half-wave i gates token i
    const int i = tid >> 5, e = lane & 31;
    const bool tok = i < T, live = tok && e < E;
    gate_halfwave(live ? sm.lg[i][e] : 0.0f, live, tok, bias_i, i, E, K, exptab, rb, global_out, sm.sel);
  }
  lds_barrier();
}

// Wr[c][k][e][j] = W[e][32(4k + j) + c]: float4 k of dot chain c of expert e (elements
// 128k + c, +32, +64, +96), the 32 experts of a chain step contiguous (layout only).
__global__ void k_router_chain_major(const float* __restrict__ W, int H, int E, float* __restrict__ Wr) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)E * H) return;
  const size_t e = i / H, r = i % H, c = r % 32, m = r / 32;
  Wr[((c * (H / 128) + m / 4) * E + e) * 4 + m % 4] = W[i];
}

hipError_t launch_router_chain_major(hipStream_t s, const float* W, int H, int E, float* Wc) {
  BB_LAUNCH(k_router_chain_major, dim3((unsigned)(((size_t)E * H + 255) / 256)), dim3(256), 0, s, W, H, E, Wc);
  return hipGetLastError();
}

hipError_t launch_route(hipStream_t s, const float* router, const float* bias, const float* x, int T, int H, int E,
                        int K, int tpb, XQBufs xq, RouteBufs rb) {
  tpb = max(1, min(tpb, ROUTE_TPB_MAX));
  BB_LAUNCH(k_route, dim3((T + tpb - 1) / tpb), dim3(1024), 0, s, router, bias, x, T, H, E, K, tpb, xq, rb);
  return hipGetLastError();
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

// Members' XQ records in LDS (up to MST at a time) and the per-(member, block, row) values
// waiting for the left-to-right block sum (MCH members at a time).
constexpr int MST = 16;
struct SmemXQ {
  int8_t q[MST][GU_H_MAX];
  uint32_t pairs[MST][GU_H_MAX / QK][12];
  float sx[MST][GU_H_MAX / QK];
};

struct SmemT {
  float v[MCH][GU_H_MAX / QK][64];
};

// ---- expert GEMV (gate/up + SwiGLU, or down) ---------------------------------------------------
// Work units are (hit expert u, row tile) pairs in u-major order; block b of G takes units
// [b*U/G, (b+1)*U/G), so every block streams the same number of tiles whatever the expert
// load. A tile is 64 rows in the tile-packed layout: for gate/up, lanes 0-31 the gate rows and
// lanes 32-63 the up rows of 32 outputs (model.rs:504-524); for down, 64 outputs of the down
// rows (model.rs:529-548). Wave w owns super-block w of the tile. A tile's weights are
// unpacked into registers, the next unit's loads are issued, and only then are the current
// tile's values computed, so one tile per block is always in flight (the barriers below order
// LDS only and do not wait for it).
//
// Members' activations: for gate/up the route kernel's XQ record of the member's token; for
// down the member's act row, quantised here (quantize_q8 per member, model.rs:530-534).
enum : int { GEMV_GATEUP = 0, GEMV_DOWN = 1 };

// Route modes of the gate/up GEMV (at most RT_MAX tokens): RM_ROUTE, the block routes the tokens
// itself (route_block) from the router, bias and f32 rows x_in, and reads the XQ records from
// LDS; RM_GATE, the block gates the tokens (gate_block) from logits already computed (passed as
// router) and reads the XQ records from memory; RM_NONE, the selections come from rb.
enum : int { RM_NONE = 0, RM_ROUTE = 1, RM_GATE = 2 };
template <int DT, int KIND, int RM>
__global__ void __launch_bounds__(512) k_experts(const uint8_t* __restrict__ wpk, size_t stride_e, int T, int H,
                                                 int F, int K, int batch_mode, int publish, int E, RouteBufs rb,
                                                 const int8_t* __restrict__ xq_q, const float* __restrict__ xq_sx,
                                                 const uint32_t* __restrict__ xq_pairs,
                                                 const float* __restrict__ act_in, float* __restrict__ out,
                                                 const float* __restrict__ router, const float* __restrict__ bias,
                                                 const float* __restrict__ x_in) {
  using R = LaneRow<DT>;
  __shared__ SmemMembers mem;
  __shared__ __align__(16) SmemXQ xs;  // down: the members' Q8 of act
  __shared__ SmemT tv;
  __shared__ uint64_t exptab[32];
  const uint64_t exp_e = KIND == GEMV_GATEUP ? exp_table_entry() : 0;
  const int n_ent = T * K;
  const int n_in = KIND == GEMV_GATEUP ? H : F;  // row length
  const int nb = n_in / QK;
  const int tiles = KIND == GEMV_GATEUP ? F / 32 : H / 64;
  const int out_w = KIND == GEMV_GATEUP ? F : H;  // output row stride
  const int32_t* sel = rb.sel;
  constexpr bool ROUTE = RM == RM_ROUTE;
  __shared__ __align__(16) typename std::conditional<ROUTE, SmemRoute, char>::type rt;
  __shared__ int32_t gsel[RM == RM_GATE ? RT_MAX * 8 : 1];
  constexpr bool XREC = KIND == GEMV_GATEUP && RM == RM_GATE;
  __shared__ __align__(16) typename std::conditional<XREC, SmemXrec, char>::type xr;
  // (XREC, one token: waves 1-4, which gate nothing, read the token's XQ record while wave 0
  // gates, and store it to LDS after; the barrier before the dots publishes it)
  uint4 xr_q = {0, 0, 0, 0};
  uint32_t xr_p0 = 0, xr_p1 = 0;
  float xr_s = 0.0f;
  const int xr_w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), xr_l = threadIdx.x & 63;
  if constexpr (XREC) {
    if (T == 1) {
      const int nbq = H / QK;
      if (xr_w == 1 || xr_w == 2) {
        xr_q = reinterpret_cast<const uint4*>(xq_q)[min(64 * (xr_w - 1) + xr_l, H / 16 - 1)];
      } else if (xr_w == 3) {
        xr_p0 = xq_pairs[min(xr_l, 12 * nbq - 1)];
        xr_p1 = xq_pairs[min(64 + xr_l, 12 * nbq - 1)];
      } else if (xr_w == 4) {
        xr_s = xq_sx[min(xr_l, nbq - 1)];
      }
    }
  }
  if constexpr (ROUTE) {
    route_block(router, bias, x_in, T, H, E, K, blockIdx.x == 0, rb, rt, exptab, exp_e);
    sel = rt.sel;
  } else if constexpr (RM == RM_GATE) {
    gate_block(router, bias, T, E, K, blockIdx.x == 0, rb, gsel, exptab, exp_e);
    sel = gsel;
  }
  if (publish && blockIdx.x == 0) publish_dispatch(sel, n_ent, E, rb);
  // One token routed or gated in the block: its K entries are the members, one per selected
  // expert, and its selections are in LDS, so every thread finds the block's experts and their
  // entries from them directly (no member lists and none of their barriers).
  const bool one = KIND == GEMV_GATEUP && RM != RM_NONE && T == 1;
  if constexpr (XREC) {
    if (one) {
      if (xr_w == 1 || xr_w == 2) reinterpret_cast<uint4*>(xr.q)[64 * (xr_w - 1) + xr_l] = xr_q;
      else if (xr_w == 3) {
        xr.pairs[xr_l] = xr_p0;
        xr.pairs[64 + xr_l] = xr_p1;
      } else if (xr_w == 4) {
        xr.sx[xr_l] = xr_s;
      }
    }
  }
  auto entry_of = [&](int ex) {
    int k0 = 0;
    for (int k = 0; k < K; ++k) k0 = sel[k] == ex ? k : k0;
    return k0;
  };
  SelRegs sr;
  uint32_t mask = 0;
  if (one) {
    for (int k = 0; k < K; ++k) mask |= 1u << sel[k];
  } else {
    mask = read_selection(sel, n_ent, sr, mem);
  }
  const int n_units = __popc(mask) * tiles;
  const int lo = (int)((long long)blockIdx.x * n_units / gridDim.x);
  const int hi = (int)((long long)(blockIdx.x + 1) * n_units / gridDim.x);
  if (lo >= hi) return;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool has_blk = w < nb;
  const size_t tile_bytes = (size_t)nb * R::TB_BYTES;
  auto tile_addr = [&](int e, int tile) {
    return wpk + (size_t)e * stride_e + (size_t)tile * tile_bytes + (size_t)w * R::TB_BYTES;
  };
  // down: stage the Q8 of the act rows of members [c0, c0 + cnt) of the current list in LDS.
  // gate/up reads the route kernel's XQ records straight from memory with uniform (scalar)
  // loads: every lane of a wave needs the same activations, and scalar operands of v_dot4 cost
  // no LDS bandwidth.
  auto stage = [&](int c0, int cnt) {
    if constexpr (KIND == GEMV_DOWN) {
      for (int task = w; task < cnt * nb; task += 8) {
        const int m = task / nb, b = task % nb;
        const float4 v = *reinterpret_cast<const float4*>(act_in + (size_t)mem.list[c0 + m] * F + b * QK + 4 * lane);
        wave_quantize_xq(v, xs.q[m] + b * QK, &xs.sx[m][b], xs.pairs[m][b]);
      }
    }
  };

  int u = lo / tiles, tile = lo % tiles;
  int e = nth_expert(mask, u);
  int one_ent = 0;  // (one) the entry of expert e
  int n_mem = 1;
  if (one) {
    one_ent = entry_of(e);
  } else {
    n_mem = member_list(sr, n_ent, e, mem);
  }
  typename R::Loaded L;
  if (has_blk) R::load(L, tile_addr(e, tile));
  if (XREC && one) lds_barrier();  // the XQ record in LDS
  if (!one) {
    if (n_mem <= MST) stage(0, n_mem);
    lds_barrier();
  }
  for (int unit = lo; unit < hi; ++unit) {
    typename R::Blk B;
    if (has_blk) R::prep(B, L);
    if (KIND == GEMV_GATEUP && RM == RM_NONE && unit == lo && tid < 32) exptab[tid] = exp_e;  // loaded before the weights
    // the next unit's weights go in flight before this tile is computed
    const bool more = unit + 1 < hi;
    const int tile_n = tile + 1 == tiles ? 0 : tile + 1;
    const int u_n = tile + 1 == tiles ? u + 1 : u;
    const int e_n = u_n == u ? e : nth_expert(mask, u_n);
    if (has_blk && more) R::load(L, tile_addr(e_n, tile_n));
    const float start = (batch_mode && n_mem > 1) ? 0.0f : -0.0f;
    for (int c0 = 0; c0 < n_mem; c0 += MCH) {
      const int cnt = min(n_mem - c0, MCH);
      int sb = c0;  // index of member c0 in xs
      if (KIND == GEMV_DOWN && n_mem > MST) {
        stage(c0, cnt);
        lds_barrier();
        sb = 0;
      }
      if (has_blk) {
        if constexpr (KIND == GEMV_GATEUP) {
          for (int m = 0; m < cnt; ++m) {
            const int tok = one ? 0 : __builtin_amdgcn_readfirstlane(mem.list[c0 + m] / K);
            if constexpr (ROUTE) {
              tv.v[m][w][lane] = R::value(B, rt.q[tok] + w * QK, rt.pairs[tok][w], rt.sx[tok][w]);
            } else if constexpr (XREC) {
              if (one) {
                tv.v[m][w][lane] = R::value(B, xr.q + w * QK, xr.pairs + 12 * w, xr.sx[w]);
              } else {
                const size_t xb = (size_t)tok * nb + w;
                tv.v[m][w][lane] = R::value(B, xq_q + xb * QK, xq_pairs + xb * 12, xq_sx[xb]);
              }
            } else {
              const size_t xb = (size_t)tok * nb + w;
              tv.v[m][w][lane] = R::value(B, xq_q + xb * QK, xq_pairs + xb * 12, xq_sx[xb]);
            }
          }
        } else {
          for (int m = 0; m < cnt; ++m)
            tv.v[m][w][lane] = R::value(B, xs.q[sb + m] + w * QK, xs.pairs[sb + m][w], xs.sx[sb + m][w]);
        }
      }
      lds_barrier();
      for (int m = w; m < cnt; m += 8) {
        float acc = start;
        for (int b = 0; b < nb; ++b) acc += tv.v[m][b][lane];
        const int ent = one ? one_ent : mem.list[c0 + m];
        if constexpr (KIND == GEMV_GATEUP) {
          const float upv = __shfl(acc, (lane + 32) & 63);
          if (lane < 32) out[(size_t)ent * out_w + tile * 32 + lane] = silu_tab(acc, exptab) * upv;
        } else {
          out[(size_t)ent * out_w + tile * 64 + lane] = acc;
        }
      }
      lds_barrier();
    }
    if (more && u_n != u) {
      e = e_n;
      if (one) {
        one_ent = entry_of(e);
      } else {
        n_mem = member_list(sr, n_ent, e, mem);
        if (n_mem <= MST) stage(0, n_mem);
        lds_barrier();
      }
    }
    u = u_n;
    tile = tile_n;
  }
}

template <int KIND>
static hipError_t launch_experts(hipStream_t s, int dtype, const uint8_t* wpk, size_t stride_e, int T, int H, int F,
                                 int E, int K, int max_hit, int batch_mode, int publish, const RouteBufs& rb,
                                 XQBufs xq, const float* act_in, float* out, int rm = RM_NONE,
                                 const float* router = nullptr, const float* bias = nullptr,
                                 const float* x_in = nullptr) {
  const int tiles = KIND == GEMV_GATEUP ? F / 32 : H / 64;
  const int grid = min(GEMV_BLOCKS, max_hit * tiles);
  if constexpr (KIND == GEMV_GATEUP) {
    if (rm != RM_NONE) {
      if (T > RT_MAX || E > 32 || K > 8 || H > GU_H_MAX) return hipErrorInvalidValue;
      if (rm == RM_ROUTE && dtype == DT_Q4_K)
        BB_LAUNCH((k_experts<DT_Q4_K, KIND, RM_ROUTE>), dim3(grid), dim3(512), 0, s, wpk, stride_e, T, H, F, K,
                  batch_mode, publish, E, rb, xq.q, xq.sx, xq.pairs, act_in, out, router, bias, x_in);
      else if (rm == RM_ROUTE)
        BB_LAUNCH((k_experts<DT_Q6_K, KIND, RM_ROUTE>), dim3(grid), dim3(512), 0, s, wpk, stride_e, T, H, F, K,
                  batch_mode, publish, E, rb, xq.q, xq.sx, xq.pairs, act_in, out, router, bias, x_in);
      else if (dtype == DT_Q4_K)
        BB_LAUNCH((k_experts<DT_Q4_K, KIND, RM_GATE>), dim3(grid), dim3(512), 0, s, wpk, stride_e, T, H, F, K,
                  batch_mode, publish, E, rb, xq.q, xq.sx, xq.pairs, act_in, out, router, bias, x_in);
      else
        BB_LAUNCH((k_experts<DT_Q6_K, KIND, RM_GATE>), dim3(grid), dim3(512), 0, s, wpk, stride_e, T, H, F, K,
                  batch_mode, publish, E, rb, xq.q, xq.sx, xq.pairs, act_in, out, router, bias, x_in);
      return hipGetLastError();
    }
  }
  if (dtype == DT_Q4_K)
    BB_LAUNCH((k_experts<DT_Q4_K, KIND, RM_NONE>), dim3(grid), dim3(512), 0, s, wpk, stride_e, T, H, F, K, batch_mode,
              publish, E, rb, xq.q, xq.sx, xq.pairs, act_in, out, nullptr, nullptr, nullptr);
  else
    BB_LAUNCH((k_experts<DT_Q6_K, KIND, RM_NONE>), dim3(grid), dim3(512), 0, s, wpk, stride_e, T, H, F, K, batch_mode,
              publish, E, rb, xq.q, xq.sx, xq.pairs, act_in, out, nullptr, nullptr, nullptr);
  return hipGetLastError();
}

hipError_t launch_gateup(hipStream_t s, int dtype, const uint8_t* gu, size_t stride_gu, int T, int H, int F, int E,
                         int K, int max_hit, int batch_mode, int publish, const RouteBufs& rb, XQBufs xq, float* act) {
  return launch_experts<GEMV_GATEUP>(s, dtype, gu, stride_gu, T, H, F, E, K, max_hit, batch_mode, publish, rb, xq,
                                     nullptr, act);
}

hipError_t launch_route_gateup(hipStream_t s, int dtype, const uint8_t* gu, size_t stride_gu, int T, int H, int F,
                               int E, int K, int max_hit, int batch_mode, int publish, const RouteBufs& rb,
                               const float* router, const float* bias, const float* x, float* act) {
  return launch_experts<GEMV_GATEUP>(s, dtype, gu, stride_gu, T, H, F, E, K, max_hit, batch_mode, publish, rb,
                                     XQBufs{}, nullptr, act, RM_ROUTE, router, bias, x);
}

hipError_t launch_gate_gateup(hipStream_t s, int dtype, const uint8_t* gu, size_t stride_gu, int T, int H, int F,
                              int E, int K, int max_hit, int batch_mode, int publish, const RouteBufs& rb,
                              const float* logits, const float* bias, XQBufs xq, float* act) {
  return launch_experts<GEMV_GATEUP>(s, dtype, gu, stride_gu, T, H, F, E, K, max_hit, batch_mode, publish, rb, xq,
                                     nullptr, act, RM_GATE, logits, bias, nullptr);
}

hipError_t launch_down(hipStream_t s, int dtype, const uint8_t* dn, size_t stride_dn, int T, int H, int F, int K,
                       int max_hit, int batch_mode, const RouteBufs& rb, const float* act, float* slots) {
  return launch_experts<GEMV_DOWN>(s, dtype, dn, stride_dn, T, H, F, 0, K, max_hit, batch_mode, 0, rb, XQBufs{}, act,
                                   slots);
}

// ---- down GEMV and combine of one token ---------------------------------------------------------
// Block b takes output rows 16b..16b+15 for all K (<= 4) selected experts: lane l = (slot
// k = l/16, row r = l%16) holds super-block w of row r of the expert of slot k, wave w owning
// super-block w as in k_experts. The block first quantises the token's K act rows into LDS
// (quantize_q8 per row, model.rs:530-534), sums each (slot, row)'s block values left to right
// from -0.0 (the decode path's Iterator::sum, model.rs:529-548), and combines the slots in
// selection order from +0.0 (k_combine, model.rs:550-553): every term of its outputs is in the
// block, so the expert outputs make no round trip through memory and need no combine launch.
template <int DT>
__global__ void __launch_bounds__(512) k_down_combine1(const uint8_t* __restrict__ wpk, size_t stride_e, int H,
                                                       int F, int K, RouteBufs rb, const float* __restrict__ act,
                                                       float* __restrict__ out) {
  using R = LaneRow<DT>;
  __shared__ __align__(16) int8_t xq[4][DN_F_MAX];
  __shared__ uint32_t pairs[4][DN_F_MAX / QK][12];
  __shared__ float sxs[4][DN_F_MAX / QK];
  __shared__ float tv[8][64];  // [super-block][lane]
  __shared__ float slot[4][16];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int k = min(lane >> 4, K - 1), r = lane & 15;
  const int nb = F / QK;
  const int orow = 16 * blockIdx.x + r;
  // the act rows of the K entries, one wave per 256-block (at most 4 a wave), read first: they
  // do not wait for the selections, which the weight reads do
  constexpr int NTASK = 4 * 8 / 8;
  float4 av[NTASK];
#pragma unroll
  for (int i = 0; i < NTASK; ++i) {
    const int task = min(w + 8 * i, K * nb - 1), m = task / nb, b = task % nb;
    av[i] = *reinterpret_cast<const float4*>(act + (size_t)m * F + b * QK + 4 * lane);
  }
  const int e = rb.sel[k];  // T = 1: entry k is slot k
  // the combine weights as well, here rather than after the barriers (another kernel wrote them)
  float wk[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) wk[j] = rb.wts[min(j, K - 1)];
  const size_t tile_bytes = (size_t)nb * R::TB_BYTES;
  const bool has_blk = w < nb;
  typename R::Loaded L;
  if (has_blk) R::load(L, wpk + (size_t)e * stride_e + (size_t)(orow / 64) * tile_bytes + (size_t)w * R::TB_BYTES,
                       orow % 64);
#pragma unroll
  for (int i = 0; i < NTASK; ++i) {
    const int task = w + 8 * i;
    if (task < K * nb)
      wave_quantize_xq(av[i], xq[task / nb] + (task % nb) * QK, &sxs[task / nb][task % nb], pairs[task / nb][task % nb]);
  }
  lds_barrier();
  float v = 0.0f;
  if (has_blk) {
    typename R::Blk B;
    R::prep(B, L);
    v = R::value(B, xq[k] + w * QK, pairs[k][w], sxs[k][w]);
  }
  tv[w][lane] = v;
  lds_barrier();
  if (w == 0) {
    float acc = -0.0f;
    for (int b = 0; b < nb; ++b) acc += tv[b][lane];
    if ((lane >> 4) < K) slot[lane >> 4][r] = acc;
  }
  lds_barrier();
  if (tid < 16) {
    float y = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < K) y = y + wk[j] * slot[j][tid];
    out[16 * blockIdx.x + tid] = y;
  }
}

hipError_t launch_down_combine1(hipStream_t s, int dtype, const uint8_t* dn, size_t stride_dn, int H, int F, int K,
                                const RouteBufs& rb, const float* act, float* out) {
  if (K < 1 || K > 4 || H % 16 != 0 || F % QK != 0 || F / QK > 8 || F > DN_F_MAX) return hipErrorInvalidValue;
  if (dtype == DT_Q4_K)
    BB_LAUNCH(k_down_combine1<DT_Q4_K>, dim3(H / 16), dim3(512), 0, s, dn, stride_dn, H, F, K, rb, act, out);
  else
    BB_LAUNCH(k_down_combine1<DT_Q6_K>, dim3(H / 16), dim3(512), 0, s, dn, stride_dn, H, F, K, rb, act, out);
  return hipGetLastError();
}

// ---- tile packing ------------------------------------------------------------------------------
// One thread per 16-byte chunk (and per tail u16) of the packed output; raw blocks are only
// 2-byte aligned (Q6_K), so the chunk is read as eight u16.
__global__ void k_pack_rows(int dtype, const uint8_t* __restrict__ a, const uint8_t* __restrict__ b, size_t stride_a,
                            size_t stride_b, int rows_a, int nb, int n_exp, uint8_t* __restrict__ dst) {
  const int NC = pack_chunks(dtype), TAIL = pack_tail(dtype);
  const size_t TB = pack_tile_block_bytes(dtype);
  const int blk_bytes = dtype == DT_Q4_K ? Q4K_BYTES : Q6K_BYTES;
  const int tile_rows = b ? 32 : 64;
  const int n_tiles = rows_a / tile_rows;
  const size_t units_per_tb = (size_t)(NC + 1) * 64;  // chunk slots plus tail slots
  const size_t total = (size_t)n_exp * n_tiles * nb * units_per_tb;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const size_t tbi = i / units_per_tb;
  const int u = (int)(i % units_per_tb), c = u / 64, lane = u % 64;
  const int blk = (int)(tbi % nb);
  const size_t et = tbi / nb;
  const int t = (int)(et % n_tiles), e = (int)(et / n_tiles);
  const uint8_t* src;
  if (b) src = lane < 32 ? a + (size_t)e * stride_a + (size_t)(32 * t + lane) * nb * blk_bytes
                         : b + (size_t)e * stride_b + (size_t)(32 * t + lane - 32) * nb * blk_bytes;
  else src = a + (size_t)e * stride_a + (size_t)(64 * t + lane) * nb * blk_bytes;
  src += (size_t)blk * blk_bytes;
  uint8_t* o = dst + tbi * TB;
  const uint16_t* s16 = reinterpret_cast<const uint16_t*>(src);
  if (c < NC) {
    uint16_t v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = s16[8 * c + k];
    uint4 q;
    q.x = v[0] | ((uint32_t)v[1] << 16);
    q.y = v[2] | ((uint32_t)v[3] << 16);
    q.z = v[4] | ((uint32_t)v[5] << 16);
    q.w = v[6] | ((uint32_t)v[7] << 16);
    *reinterpret_cast<uint4*>(o + 1024 * c + 16 * lane) = q;
  } else if (TAIL) {
    reinterpret_cast<uint16_t*>(o + 1024 * NC)[lane] = s16[8 * NC];
  }
}

hipError_t launch_pack_rows(hipStream_t s, int dtype, const uint8_t* a, const uint8_t* b, size_t stride_a,
                            size_t stride_b, int rows_a, int nb, int n_exp, uint8_t* dst) {
  const int n_tiles = rows_a / (b ? 32 : 64);
  const size_t total = (size_t)n_exp * n_tiles * nb * (pack_chunks(dtype) + 1) * 64;
  if (total == 0) return hipSuccess;
  BB_LAUNCH(k_pack_rows, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, dtype, a, b, stride_a,
                     stride_b, rows_a, nb, n_exp, dst);
  return hipGetLastError();
}

// ---- layer boundary with the next layer's router logits (a stack of at most RT_MAX tokens) ------
// k_residual_norm's work for token t (h_out = h_in + the combine of the K slot rows from +0.0 in
// selection order, or + the dense output; then the next layer's rmsnorm with an f64 tree sum) on
// ceil(E/4) blocks per token, block eb also taking the router logits of experts 4eb..4eb+3 of
// the next (MoE) layer from the normed row, with k_route's arithmetic (matmul.rs:36-66: 32 fmaf
// chains per expert, chain c over the elements i = c mod 32, then the lane combine and
// reduce_add tree). The router is read as 32 KB per block instead of 256 KB in every gate/up
// block. Every block recomputes the residual, so h_out must not alias h_in; block 0 of a token
// writes h_out and normed, and the blocks share out the XQ records of normed (model.rs:501,
// with the pair dwords).
constexpr int RN_EXPERTS = 4;

// The router values of the chain a thread of a 256-thread block runs: chain c = tid % 32 of
// expert 4eb + (tid / 32) % 4 (threads 128.. load the same values again and drop them).
struct RouterChain {
  float4 v[GU_H_MAX / 128];
};
__device__ __forceinline__ void rl_load(const float* __restrict__ Wr, int n, int E, int eb, RouterChain& rc) {
  const int tid = threadIdx.x, el = (tid >> 5) & (RN_EXPERTS - 1), c = tid & 31, nm4 = n / 128;
  const int e = min(RN_EXPERTS * eb + el, E - 1);
  const float4* wr = reinterpret_cast<const float4*>(Wr) + (size_t)c * nm4 * E + e;
#pragma unroll
  for (int k = 0; k < GU_H_MAX / 128; ++k) rc.v[k] = wr[(size_t)min(k, nm4 - 1) * E];
}

// From token t's row xs (LDS, after a barrier): the XQ records of 256-blocks eb, eb + nblk, ...
// by the last wave (the pair dwords when xq.pairs is set), the logits of experts 4eb..4eb+3
// (k_route's chains and tree) by the rest.
__device__ __forceinline__ void rl_finish(const float* xs, const RouterChain& rc, int n, int E, int t, int eb,
                                          int nblk, float* __restrict__ logits, XQBufs xq,
                                          float (&part)[RN_EXPERTS][33]) {
  const int tid = threadIdx.x, lane = tid & 63, el = (tid >> 5) & (RN_EXPERTS - 1), c = tid & 31;
  const int nm4 = n / 128, nbx = n / QK;
  if ((tid >> 6) == 3)
    for (int bk = eb; bk < nbx; bk += nblk) {
      const float4 v = *reinterpret_cast<const float4*>(xs + bk * QK + 4 * lane);
      wave_quantize_xq(v, xq.q + (size_t)t * n + bk * QK, xq.sx + (size_t)t * nbx + bk,
                       xq.pairs ? xq.pairs + ((size_t)t * nbx + bk) * 12 : nullptr);
    }
  if (tid < 32 * RN_EXPERTS) {
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < GU_H_MAX / 128; ++k) {
      if (k < nm4) {
        const float* xk = xs + 128 * k + c;
        acc = fmaf(rc.v[k].x, xk[0], acc);
        acc = fmaf(rc.v[k].y, xk[32], acc);
        acc = fmaf(rc.v[k].z, xk[64], acc);
        acc = fmaf(rc.v[k].w, xk[96], acc);
      }
    }
    part[el][c] = acc;
  }
  lds_barrier();
  if (tid < RN_EXPERTS && RN_EXPERTS * eb + tid < E) {
    const float* p = part[tid];
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (p[j] + p[j + 8]) + (p[j + 16] + p[j + 24]);
    logits[(size_t)t * E + RN_EXPERTS * eb + tid] = ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
  }
}

__global__ void __launch_bounds__(256) k_residual_norm_route(const float* __restrict__ h_in, float* __restrict__ h_out,
                                                             const float* __restrict__ slots,
                                                             const float* __restrict__ wts, int K,
                                                             const float* __restrict__ ffn,
                                                             const float* __restrict__ gain, float eps, int n,
                                                             float* __restrict__ normed, const float* __restrict__ Wr,
                                                             int E, float* __restrict__ logits, XQBufs xq) {
  __shared__ __align__(16) float xs[GU_H_MAX];
  __shared__ float part[RN_EXPERTS][33];
  __shared__ double s_part[4];
  __shared__ float s_scale;
  const int t = blockIdx.y, eb = blockIdx.x, tid = threadIdx.x;
  // the residual (thread j: elements j, j+256, ...), every load before the first use; the
  // router's after them, so the residual waits for its own loads only
  constexpr int NI = GU_H_MAX / 256;
  float hr[NI], yr[NI], gr[NI];
  const size_t row = (size_t)t * n;
#pragma unroll
  for (int it = 0; it < NI; ++it) gr[it] = gain[min(tid + 256 * it, n - 1)];
  if (slots) {
    float wk[8], sv[8][NI];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const size_t srow = (size_t)t * K + min(k, K - 1);
      wk[k] = wts[srow];
#pragma unroll
      for (int it = 0; it < NI; ++it) sv[k][it] = slots[srow * n + min(tid + 256 * it, n - 1)];
    }
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      hr[it] = h_in[row + min(tid + 256 * it, n - 1)];
      yr[it] = 0.0f;
    }
    // the weights' loads complete here, behind the rows' (the compiler would otherwise issue
    // each just before its use below, one round trip after another)
#pragma unroll
    for (int k = 0; k < 8; ++k) asm volatile("" ::"s"(wk[k]));
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < K) {
#pragma unroll
        for (int it = 0; it < NI; ++it) yr[it] = yr[it] + wk[k] * sv[k][it];
      }
  } else {
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      hr[it] = h_in[row + min(tid + 256 * it, n - 1)];
      yr[it] = ffn[row + min(tid + 256 * it, n - 1)];
    }
  }
  RouterChain rc;
  rl_load(Wr, n, E, eb, rc);
  double ss = 0.0;
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int i = tid + 256 * it;
    if (i >= n) break;
    const float v = hr[it] + yr[it];
    hr[it] = v;
    ss += (double)(v * v);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  lds_barrier();
  if (tid == 0) {
    const double tot = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    const float mean = (float)(tot / (double)n);
    s_scale = 1.0f / sqrtf(mean + eps);
  }
  lds_barrier();
  const float scale = s_scale;
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int i = tid + 256 * it;
    if (i >= n) break;
    const float nv = hr[it] * scale * gr[it];
    xs[i] = nv;
    if (eb == 0) {
      h_out[row + i] = hr[it];
      normed[row + i] = nv;
    }
  }
  lds_barrier();
  rl_finish(xs, rc, n, E, t, eb, gridDim.x, logits, xq, part);
}

hipError_t launch_residual_norm_route(hipStream_t s, const float* h_in, float* h_out, const float* slots,
                                      const float* wts, int K, const float* ffn, const float* gain, float eps, int n,
                                      int T, float* normed, const float* router, int E, float* logits, XQBufs xq) {
  if (n > GU_H_MAX || n % 128 != 0 || E > 32 || K > 8 || T < 1 || !gain || !xq.pairs) return hipErrorInvalidValue;
  BB_LAUNCH(k_residual_norm_route, dim3((unsigned)((E + RN_EXPERTS - 1) / RN_EXPERTS), (unsigned)T), dim3(256), 0, s,
            h_in, h_out, slots, wts, K, ffn, gain, eps, n, normed, router, E, logits, xq);
  return hipGetLastError();
}

// ---- combine -----------------------------------------------------------------------------------
// out[t][o] = Σ_k w[t,k]·slots[t*K+k][o], k ascending from +0.0 (add_scaled, elementwise.rs:12).
// KT > 0: K = KT known at compile time, every slot's loads issued before the first add (one
// memory round trip instead of one per slot); KT = 0: any K, one slot after the other.
template <int KT>
__global__ void __launch_bounds__(256) k_combine(const float* __restrict__ slots, const float* __restrict__ wts, int T,
                                                 int H, int K, float* __restrict__ out) {
  // block (x, t): outputs 4·(256x + thread) .. +3 of token t
  const int t = blockIdx.y, o4 = blockIdx.x * 256 + threadIdx.x;
  if (o4 * 4 >= H) return;
  if constexpr (KT > 0) K = KT;
  const float4* s4 = reinterpret_cast<const float4*>(slots);
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  constexpr int NR = KT > 0 ? KT : 1;
  float wk[NR];
  float4 v[NR];
  for (int k0 = 0; k0 < K; k0 += NR) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      wk[i] = wts[(size_t)t * K + k0 + i];
      v[i] = s4[((size_t)t * K + k0 + i) * (H / 4) + o4];
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      acc.x = acc.x + wk[i] * v[i].x;
      acc.y = acc.y + wk[i] * v[i].y;
      acc.z = acc.z + wk[i] * v[i].z;
      acc.w = acc.w + wk[i] * v[i].w;
    }
  }
  reinterpret_cast<float4*>(out)[(size_t)t * (H / 4) + o4] = acc;
}

hipError_t launch_combine(hipStream_t s, const float* slots, const float* wts, int T, int H, int K, float* out) {
  const dim3 grid((unsigned)((H / 4 + 255) / 256), (unsigned)T);
  switch (K) {
#define BB_COMBINE_K(k) \
  case k: BB_LAUNCH(k_combine<k>, grid, dim3(256), 0, s, slots, wts, T, H, K, out); break;
    BB_COMBINE_K(1) BB_COMBINE_K(2) BB_COMBINE_K(3) BB_COMBINE_K(4)
    BB_COMBINE_K(5) BB_COMBINE_K(6) BB_COMBINE_K(7) BB_COMBINE_K(8)
#undef BB_COMBINE_K
    default: BB_LAUNCH(k_combine<0>, grid, dim3(256), 0, s, slots, wts, T, H, K, out);
  }
  return hipGetLastError();
}

}  // namespace bb
