// bb_device.h — gfx950 device building blocks shared by every kernel in the library.
//
// Arithmetic contract: integer sub-dots are exact; every f32 operation is issued in the
// reference's evaluation order (the library is compiled with -ffp-contract=off and with
// correctly rounded f32 divide/sqrt), so results are bit-identical to the reference's CPU path.
#ifndef BB_DEVICE_H
#define BB_DEVICE_H
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "bb_expf.h"

namespace bb {

constexpr int QK = 256;
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BYTES = 210;
enum : int { DT_F32 = 0, DT_F16 = 1, DT_Q4_K = 12, DT_Q6_K = 14 };

// ---- scalar helpers ----------------------------------------------------------------------

// f16 -> f32 (dequant.rs:22-54). The hardware conversion is exact for every finite f16 and
// infinity; it differs from the reference's bit shuffle only in quieting a signalling NaN.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// activation.rs:5-13: 1/(1+e^-x) and x/(1+e^-x) with the glibc-identical expf.
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + bb_expf(-x)); }
__device__ __forceinline__ float silu(float x) { return x / (1.0f + bb_expf(-x)); }

// The same with the exp table in LDS: kernels whose epilogue would otherwise wait for the
// table's first read from memory load it at their start (exp_table_entry, threads 0-31) and
// store it where they wait for their first loads anyway; a barrier then publishes it.
__device__ __forceinline__ float sigmoid_tab(float x, const uint64_t* tab) { return 1.0f / (1.0f + bb_expf_tab(-x, tab)); }
__device__ __forceinline__ float silu_tab(float x, const uint64_t* tab) { return x / (1.0f + bb_expf_tab(-x, tab)); }
__device__ __forceinline__ uint64_t exp_table_entry() {
  return bb_exp2f_tab_dev[threadIdx.x & 31];  // unconditional: other loads are not held behind it
}

// Rust f32::total_cmp key: signed compare of the sign-magnitude-flipped bits (-0 < +0).
__device__ __forceinline__ int32_t total_key(float f) {
  int32_t b = (int32_t)bb_f32_bits(f);
  return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
}

// matmul.rs:153: round half away from zero, clamp to ±127, NaN -> 0 (Rust's saturating cast).
__device__ __forceinline__ int q8_round(float y) {
  if (y != y) return 0;
  float r = truncf(y);
  if (fabsf(y - r) >= 0.5f) r += copysignf(1.0f, y);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int)r;
}

// ---- buffer resources ------------------------------------------------------------------------
// gfx9 raw buffers (base, byte size, word 3 = 0x00020000): loads through them take a 32-bit
// per-lane offset and a wave-uniform one, so a lane keeps one register per stream instead of a
// 64-bit address per load. An access at or past the size reads zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
// Cache policy of the loads that stream expert weights read once per call (the decode paths):
// non-temporal ("nt"), so a layer's weights pass through L2 without displacing the data that
// the next kernels read again (the router, the tokens' rows and Q8 records, the selections).
constexpr int CPOL_NT = 2;
__device__ __forceinline__ uint4 buf_load16nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, CPOL_NT));
}
// A 16-byte global load with the same policy.
__device__ __forceinline__ uint4 ld16_nt(const uint8_t* p) {
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p)));
}
__device__ __forceinline__ float buf_load4f(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}
// global_load_lds through a buffer: 16 (or 4) bytes a lane into dst + 16·lane (4·lane)
__device__ __forceinline__ void buf_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint8_t* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, (int)voff, (int)soff, 0,
                                           0);
}
__device__ __forceinline__ void buf_dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint8_t* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4, (int)voff, (int)soff, 0,
                                           0);
}

// ---- block barrier for LDS traffic only ----------------------------------------------------
// __syncthreads() also waits for every global load the wave has in flight (its release fence
// waits on vmcnt, which counts loads and LDS-DMA copies alike). Where a barrier only orders LDS
// accesses, this one waits for the wave's LDS operations alone, so prefetches stay in flight
// across it. The empty asm statements keep the compiler from moving memory accesses across.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---- cross-lane reductions -----------------------------------------------------------------

// Sum over each aligned group of 8 lanes, result in all 8 lanes (DPP: half-row mirror, then
// quad permutes [1,0,3,2] and [2,3,0,1]). Integer only: the order is irrelevant.
__device__ __forceinline__ int sum8(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false);
  return v;
}

// Max over the wave, in every lane: DPP within each 16-lane row (quad swaps, then the half-row
// and row mirrors, which pair each group with the other half of its row), then the four rows'
// results read as scalars. For non-negative, non-NaN inputs (|x| values) the order is free.
__device__ __forceinline__ float wave_max(float v) {
  auto dpp = [](float x, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(ctrl)::value,
                                                                 0xf, 0xf, false));
  };
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad [1,0,3,2]
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad [2,3,0,1]
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x141>{}));  // half-row mirror
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x140>{}));  // row mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// ---- Q8 activation quantisation (matmul.rs:141-160), one 256-block per wave -----------------
// Lane L holds elements 4L..4L+3 of the block. amax is an order-free max; the eight 32-wide
// sums are exact integer sums over 8 lanes.
__device__ __forceinline__ void wave_quantize_block(float4 v, int8_t* __restrict__ q, float* __restrict__ scale,
                                                    int32_t* __restrict__ sums) {
  const int lane = threadIdx.x & 63;
  float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  float amax = wave_max(a);
  float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  int q0 = q8_round(v.x * inv), q1 = q8_round(v.y * inv), q2 = q8_round(v.z * inv), q3 = q8_round(v.w * inv);
  uint32_t packed = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
                    ((uint32_t)(q3 & 0xff) << 24);
  reinterpret_cast<uint32_t*>(q)[lane] = packed;
  int s = sum8(q0 + q1 + q2 + q3);
  if ((lane & 7) == 0) sums[lane >> 3] = s;
  if (lane == 0) *scale = amax / 127.0f;
}

// ---- Q4_K (144 B: d, dmin f16 | scales[12] | qs[128]; dequant.rs:6-9) ---------------------
// get_scale_min_k4 (dequant.rs:64-72) for sub-block j, with the 12 scale bytes held as three
// little-endian dwords s0 = scales[0..3], s1 = scales[4..7], s2 = scales[8..11].
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int& sc, int& m) {
  if (j < 4) {
    sc = (s0 >> (8 * j)) & 63;
    m = (s1 >> (8 * j)) & 63;
  } else {
    const int k = 8 * (j - 4);
    sc = ((s2 >> k) & 0xF) | (((s0 >> (k + 6)) & 3) << 4);
    m = ((s2 >> (k + 4)) & 0xF) | (((s1 >> (k + 6)) & 3) << 4);
  }
}

// One lane of an 8-lane row group owns 16 bytes of qs: lane p covers bytes 16p..16p+15, i.e.
// chunk c = p>>1, half h = p&1; their low nibbles are elements 64c+16h+[0,16) (sub-block 2c)
// and their high nibbles elements 64c+32+16h+[0,16) (sub-block 2c+1) (dequant.rs:87-105).
struct Q4kLane {
  uint4 hd;  // d|dmin, scales[0..3], scales[4..7], scales[8..11]
  uint4 qs;  // 16 bytes of qs
};

__device__ __forceinline__ Q4kLane q4k_load(const uint8_t* __restrict__ block, int p) {
  Q4kLane r;
  r.hd = *reinterpret_cast<const uint4*>(block);
  r.qs = *reinterpret_cast<const uint4*>(block + 16 + 16 * p);
  return r;
}

// The activations lane p of a group needs for one block: quants of its two 16-element pieces,
// the Q8 sum of its sub-block 2(p>>1) + (p&1), and the block's scale.
struct Q4kX {
  uint4 xl, xh;
  int32_t sum;
  float sx;
};
__device__ __forceinline__ Q4kX q4k_xload(const int8_t* __restrict__ qxb, const int32_t* __restrict__ sumsb,
                                          const float* __restrict__ sxp, int p) {
  const int c = p >> 1, h = p & 1;
  return Q4kX{*reinterpret_cast<const uint4*>(qxb + 64 * c + 16 * h),
              *reinterpret_cast<const uint4*>(qxb + 64 * c + 32 + 16 * h), sumsb[2 * c + h], *sxp};
}

// Partial (sd, sm) of one block for this lane: sd_part = sc_2c·<lo, qx> + sc_2c+1·<hi, qx>,
// sm_part = m_j·sums_j for the one sub-block this lane accounts for (j = 2c + h).
__device__ __forceinline__ void q4k_lane_partial_x(const Q4kLane& w, int p, uint4 xl, uint4 xh, int32_t sum, int& sd,
                                                   int& sm) {
  const int c = p >> 1, h = p & 1;
  int sc0, m0, sc1, m1;
  q4k_scale_min(w.hd.y, w.hd.z, w.hd.w, 2 * c, sc0, m0);
  q4k_scale_min(w.hd.y, w.hd.z, w.hd.w, 2 * c + 1, sc1, m1);
  const uint32_t M = 0x0F0F0F0Fu;
  int dl = __builtin_amdgcn_sdot4((int)(w.qs.x & M), (int)xl.x, 0, false);
  dl = __builtin_amdgcn_sdot4((int)(w.qs.y & M), (int)xl.y, dl, false);
  dl = __builtin_amdgcn_sdot4((int)(w.qs.z & M), (int)xl.z, dl, false);
  dl = __builtin_amdgcn_sdot4((int)(w.qs.w & M), (int)xl.w, dl, false);
  int dh = __builtin_amdgcn_sdot4((int)((w.qs.x >> 4) & M), (int)xh.x, 0, false);
  dh = __builtin_amdgcn_sdot4((int)((w.qs.y >> 4) & M), (int)xh.y, dh, false);
  dh = __builtin_amdgcn_sdot4((int)((w.qs.z >> 4) & M), (int)xh.z, dh, false);
  dh = __builtin_amdgcn_sdot4((int)((w.qs.w >> 4) & M), (int)xh.w, dh, false);
  sd = sc0 * dl + sc1 * dh;
  sm = (h == 0 ? m0 : m1) * sum;
}

__device__ __forceinline__ void q4k_lane_partial(const Q4kLane& w, int p, const int8_t* __restrict__ qxb,
                                                 const int32_t* __restrict__ sumsb, int& sd, int& sm) {
  const int c = p >> 1, h = p & 1;
  q4k_lane_partial_x(w, p, *reinterpret_cast<const uint4*>(qxb + 64 * c + 16 * h),
                     *reinterpret_cast<const uint4*>(qxb + 64 * c + 32 + 16 * h), sumsb[2 * c + h], sd, sm);
}

// matmul.rs:242: sx·(d·sd − dmin·sm), operation by operation.
__device__ __forceinline__ float q4k_block_value(uint32_t dd, int sd, int sm, float sx) {
  const float d = f16_bits_to_f32(dd & 0xffff), dmin = f16_bits_to_f32(dd >> 16);
  const float a = d * (float)sd;
  const float b = dmin * (float)sm;
  return sx * (a - b);
}

// ---- Q6_K (210 B: ql[128] | qh[64] | sc i8[16] | d f16; dequant.rs:6-9) -------------------
// Q6_K rows are 1470 B, so blocks are only 2-byte aligned: fields are read as aligned dwords
// and funnel-shifted. Every uploaded tensor carries tail padding that covers the one dword
// read past a block's last byte.
__device__ __forceinline__ uint2 ld8_a2(const uint8_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t* base = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
  const uint32_t sh = (uint32_t)(a & 3);
  const uint32_t w0 = base[0], w1 = base[1], w2 = base[2];
  return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
}

// Lane p of an 8-lane group: half n = p>>2, l0 = 8(p&3); it covers elements 128n+32g+l0+[0,8)
// for g = 0..3 (dequant.rs:127-137), whose sub-blocks are 8n+2g+(l0>=16) (matmul.rs:656-678).
struct Q6kLane {
  uint2 a, b, h;  // ql[64n+l0..], ql[64n+32+l0..], qh[32n+l0..]
  uint2 sc;       // sc[8n..8n+7]
  uint32_t d;     // f16 bits
};

__device__ __forceinline__ Q6kLane q6k_load(const uint8_t* __restrict__ block, int p) {
  const int n = p >> 2, l0 = 8 * (p & 3);
  Q6kLane r;
  r.a = ld8_a2(block + 64 * n + l0);
  r.b = ld8_a2(block + 64 * n + 32 + l0);
  r.h = ld8_a2(block + 128 + 32 * n + l0);
  r.sc = ld8_a2(block + 192 + 8 * n);
  r.d = *reinterpret_cast<const uint16_t*>(block + 208);
  return r;
}

// Bytes q in 0..63 -> bytes (q-32) as i8: q+0x60 never carries across bytes, and flipping
// bit 7 maps q+96 to q-32 mod 256.
__device__ __forceinline__ int q6_center(uint32_t q) { return (int)((q + 0x60606060u) ^ 0x80808080u); }

// The activations lane p needs for one block: four 8-element pieces, 32 apart, and the scale.
struct Q6kX {
  uint2 x0, x1, x2, x3;
  float sx;
};
__device__ __forceinline__ Q6kX q6k_xload(const int8_t* __restrict__ qxb, const float* __restrict__ sxp, int p) {
  const int8_t* xg = qxb + 128 * (p >> 2) + 8 * (p & 3);
  return Q6kX{*reinterpret_cast<const uint2*>(xg), *reinterpret_cast<const uint2*>(xg + 32),
              *reinterpret_cast<const uint2*>(xg + 64), *reinterpret_cast<const uint2*>(xg + 96), *sxp};
}

__device__ __forceinline__ int q6k_lane_partial_x(const Q6kLane& w, int p, uint2 x0, uint2 x1, uint2 x2, uint2 x3) {
  const int s = (p & 3) >> 1;
  const uint32_t scw = s ? ((w.sc.x >> 8) | (w.sc.y << 24)) : w.sc.x;  // bytes s, s+2 in scw.x
  const uint32_t scv = s ? (w.sc.y >> 8) : w.sc.y;                      // bytes s+4, s+6
  const int sc0 = (int)(int8_t)(scw & 0xff), sc1 = (int)(int8_t)((scw >> 16) & 0xff);
  const int sc2 = (int)(int8_t)(scv & 0xff), sc3 = (int)(int8_t)((scv >> 16) & 0xff);
  const uint32_t M4 = 0x0F0F0F0Fu, M2 = 0x30303030u;
  int d0 = 0, d1 = 0, d2 = 0, d3 = 0;
#define BB_Q6_STEP(A, B, H, X0, X1, X2, X3)                                                           \
  d0 = __builtin_amdgcn_sdot4(q6_center(((A) & M4) | (((H) << 4) & M2)), (int)(X0), d0, false);     \
  d1 = __builtin_amdgcn_sdot4(q6_center(((B) & M4) | (((H) << 2) & M2)), (int)(X1), d1, false);     \
  d2 = __builtin_amdgcn_sdot4(q6_center((((A) >> 4) & M4) | ((H) & M2)), (int)(X2), d2, false);    \
  d3 = __builtin_amdgcn_sdot4(q6_center((((B) >> 4) & M4) | (((H) >> 2) & M2)), (int)(X3), d3, false);
  BB_Q6_STEP(w.a.x, w.b.x, w.h.x, x0.x, x1.x, x2.x, x3.x)
  BB_Q6_STEP(w.a.y, w.b.y, w.h.y, x0.y, x1.y, x2.y, x3.y)
#undef BB_Q6_STEP
  return sc0 * d0 + sc1 * d1 + sc2 * d2 + sc3 * d3;
}

__device__ __forceinline__ int q6k_lane_partial(const Q6kLane& w, int p, const int8_t* __restrict__ qxb) {
  const int8_t* xg = qxb + 128 * (p >> 2) + 8 * (p & 3);
  return q6k_lane_partial_x(w, p, *reinterpret_cast<const uint2*>(xg), *reinterpret_cast<const uint2*>(xg + 32),
                            *reinterpret_cast<const uint2*>(xg + 64), *reinterpret_cast<const uint2*>(xg + 96));
}

// matmul.rs:641: sx·(d·s).
__device__ __forceinline__ float q6k_block_value(uint32_t dbits, int s, float sx) {
  const float d = f16_bits_to_f32(dbits);
  return sx * (d * (float)s);
}

// ---- One row dot for an 8-lane group (dot_q4k_row_q8 / dot_q6k_row_q8) ------------------------
// Blocks are summed left to right into `acc` (start value chosen by the caller: the decode
// path's Iterator::sum starts at -0.0, the batched path accumulates into a +0.0 buffer).
// All 8 lanes of the group return the same value.
template <int DT>
struct RowDot;

template <>
struct RowDot<DT_Q4_K> {
  static constexpr int BLOCK_BYTES = Q4K_BYTES;
  using Lane = Q4kLane;
  using X = Q4kX;
  static __device__ __forceinline__ Lane load(const uint8_t* block, int p) { return q4k_load(block, p); }
  static __device__ __forceinline__ X xload(const int8_t* qxb, const int32_t* sumsb, const float* sxp, int p) {
    return q4k_xload(qxb, sumsb, sxp, p);
  }
  // The block's value from registers only (all 8 lanes of the group return it).
  static __device__ __forceinline__ float block_value_x(const Lane& w, int p, const X& x) {
    int sd, sm;
    q4k_lane_partial_x(w, p, x.xl, x.xh, x.sum, sd, sm);
    sd = sum8(sd);
    sm = sum8(sm);
    return q4k_block_value(w.hd.x, sd, sm, x.sx);
  }
  static __device__ __forceinline__ float block_value(const Lane& w, int p, const int8_t* qxb, const int32_t* sumsb,
                                                      float sx) {
    int sd, sm;
    q4k_lane_partial(w, p, qxb, sumsb, sd, sm);
    sd = sum8(sd);
    sm = sum8(sm);
    return q4k_block_value(w.hd.x, sd, sm, sx);
  }
};

template <>
struct RowDot<DT_Q6_K> {
  static constexpr int BLOCK_BYTES = Q6K_BYTES;
  using Lane = Q6kLane;
  using X = Q6kX;
  static __device__ __forceinline__ Lane load(const uint8_t* block, int p) { return q6k_load(block, p); }
  static __device__ __forceinline__ X xload(const int8_t* qxb, const int32_t*, const float* sxp, int p) {
    return q6k_xload(qxb, sxp, p);
  }
  static __device__ __forceinline__ float block_value_x(const Lane& w, int p, const X& x) {
    const int s = sum8(q6k_lane_partial_x(w, p, x.x0, x.x1, x.x2, x.x3));
    return q6k_block_value(w.d, s, x.sx);
  }
  static __device__ __forceinline__ float block_value(const Lane& w, int p, const int8_t* qxb, const int32_t*,
                                                      float sx) {
    int s = sum8(q6k_lane_partial(w, p, qxb));
    return q6k_block_value(w.d, s, sx);
  }
};

// Row dot against one Q8 vector, weights loaded per block (runtime block count).
template <int DT>
__device__ __forceinline__ float row_dot_q8(const uint8_t* __restrict__ row, int nb, int p,
                                            const int8_t* __restrict__ qx, const float* __restrict__ sx,
                                            const int32_t* __restrict__ sums, float acc) {
  using R = RowDot<DT>;
  for (int b = 0; b < nb; ++b) {
    typename R::Lane w = R::load(row + (size_t)b * R::BLOCK_BYTES, p);
    acc += R::block_value(w, p, qx + b * QK, sums + b * 8, sx[b]);
  }
  return acc;
}

}  // namespace bb
#endif
