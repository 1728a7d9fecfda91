// bb_rowlane.h — "one lane, one weight row" building blocks for the decode GEMV kernels.
//
// A lane holds one 256-weight super-block of its row in registers, unpacks it once, and
// computes that block's exact value against each member's Q8 activations:
//   Q4_K: sx·(d·sd − dmin·sm)   (matmul.rs:242)      Q6_K: sx·(d·s)   (matmul.rs:641)
// with sd, sm, s exact int32. No cross-lane reduction is needed; per-block values are summed
// left to right by the caller (matmul.rs:293-298, :748-753), so results are bit-identical to
// the reference.
//
// Activation record ("XQ"), per vector of n elements (n % 256 == 0):
//   q      int8[n]               the Q8 quants (matmul.rs:153)
//   sx     f32[n/256]            per-block scale amax/127 (matmul.rs:149)
//   pairs  u32[n/256][12]        int16 pairs of quant sums, the operands of v_dot2_i32_i16:
//            [0..3]  32-wide sums (S0,S2) (S1,S3) (S4,S6) (S5,S7)  -> Q4_K min term Σ m_j·S_j
//            [4..11] 16-wide sums (T0,T2) (T1,T3) (T4,T6) (T5,T7) ... (T13,T15)
//                                                                  -> Q6_K −32·Σ sc_k·T_k
// |S| <= 32·127 and |T| <= 16·127 fit int16 exactly.
#ifndef BB_ROWLANE_H
#define BB_ROWLANE_H
#include "bb_device.h"
#include "bb_internal.h"

namespace bb {

typedef short v2s __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int dot2(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, a), __builtin_bit_cast(v2s, b), c, false);
}
__device__ __forceinline__ uint32_t pack16(int lo, int hi) { return ((uint32_t)lo & 0xffffu) | ((uint32_t)hi << 16); }

// Q8 quantisation of one 256-block by one wave into the XQ record (lane L holds elements
// 4L..4L+3). The quants, scale and sums are those of quantize_q8 (matmul.rs:141-160).
// The min term of a Q4_K block, sm = Σ_j m_j·S_j over the eight per-32 sums S_j of the Q8
// activations (|S_j| <= 4064), as one f16 MFMA (16x16x16): each S_j is split S = 64·Sh + Sl with
// Sl = S & 63 in [0, 63] and Sh = S >> 6 in [-64, 63], both exact in f16, and the weights take
// 64·m_j (<= 4032) and m_j (<= 63), exact too. Every product (<= 258048) and every partial sum of
// the 16 (<= 2.1e6 < 2^24) is an exact integer in f32, so the MFMA returns sm exactly, in any
// order of its sums. The record of a 256-block: 16 halves, lane group g's four
// [Sh_{2g}, Sh_{2g+1}, Sl_{2g}, Sl_{2g+1}] (the sub-blocks of its qs bytes in the GEMM's order).
// s32: S_j in lanes 8j..8j+7 of the wave.
__device__ __forceinline__ void min_split_record(int s32, uint16_t* __restrict__ ms) {
  const int lane = threadIdx.x & 63;
  if ((lane & 7) == 0) {
    const int j = lane >> 3, g = j >> 1, o = j & 1;
    const _Float16 hs = (_Float16)(s32 >> 6), ls = (_Float16)(s32 & 63);
    ms[4 * g + o] = __builtin_bit_cast(uint16_t, hs);
    ms[4 * g + 2 + o] = __builtin_bit_cast(uint16_t, ls);
  }
}

__device__ __forceinline__ void wave_quantize_xq(float4 v, int8_t* __restrict__ q, float* __restrict__ sx,
                                                 uint32_t* __restrict__ pairs, uint16_t* __restrict__ ms = nullptr) {
  const int lane = threadIdx.x & 63;
  const float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  const float amax = wave_max(a);
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  const int q0 = q8_round(v.x * inv), q1 = q8_round(v.y * inv), q2 = q8_round(v.z * inv), q3 = q8_round(v.w * inv);
  reinterpret_cast<uint32_t*>(q)[lane] = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                                         ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
  int s4 = q0 + q1 + q2 + q3;
  int t16 = s4 + __builtin_amdgcn_update_dpp(0, s4, 0xB1, 0xf, 0xf, false);  // quad [1,0,3,2]
  t16 += __builtin_amdgcn_update_dpp(0, t16, 0x4E, 0xf, 0xf, false);         // quad [2,3,0,1]
  const int s32 = t16 + __builtin_amdgcn_update_dpp(0, t16, 0x141, 0xf, 0xf, false);  // lanes 8j..8j+7: S_j
  // (half-row mirror: the other quad of the 8-lane group, whose lanes all hold its sum)
  if (lane == 0) *sx = amax / 127.0f;
  if (ms) min_split_record(s32, ms);
  if (!pairs) return;
  // pair dword j is built by lane j: sources are lanes holding the two sums
  int srcA, srcB;
  bool wide;
  if (lane < 4) {
    wide = true;
    srcA = 8 * ((lane & 1) + 4 * (lane >> 1));  // S0, S1, S4, S5
    srcB = srcA + 16;                            // S2, S3, S6, S7
  } else {
    const int i2 = (lane - 4) & 7, i = i2 >> 1, odd = i2 & 1;
    wide = false;
    srcA = 4 * (4 * i + odd);
    srcB = srcA + 8;
  }
  const int a32 = __shfl(s32, srcA), b32 = __shfl(s32, srcB);
  const int a16 = __shfl(t16, srcA), b16 = __shfl(t16, srcB);
  if (lane < 12) pairs[lane] = wide ? pack16(a32, b32) : pack16(a16, b16);
}

// ---- Q4_K row block ----------------------------------------------------------------------------
struct Q4Blk {
  uint32_t lo[32], hi[32];  // nibbles: lo[8c+k] = sub-block 2c elements 4k..4k+3, hi = sub-block 2c+1
  int sc[8];
  uint32_t mp[4];           // 6-bit mins as int16 pairs (m0,m2) (m1,m3) (m4,m6) (m5,m7)
  float d, dmin;
};

// tb: the tile-block (tile-packed layout); chunk k of row j's block is at tb + 1024k + 16j.
// Row = lane: each load of the wave reads 1 KB of contiguous memory. The GEMVs read each weight
// once per call, so the loads stream (non-temporal).
__device__ __forceinline__ void q4_load(uint4 (&w)[9], const uint8_t* __restrict__ tb, int row) {
#pragma unroll
  for (int k = 0; k < 9; ++k) w[k] = ld16_nt(tb + 1024 * k + 16 * row);
}

// get_scale_min_k4 (dequant.rs:64-72) on four bytes at a time, then the nibble unpack
// (dequant.rs:87-105).
__device__ __forceinline__ void q4_prep(Q4Blk& B, const uint4 (&w)[9]) {
  B.d = f16_bits_to_f32(w[0].x & 0xffff);
  B.dmin = f16_bits_to_f32(w[0].x >> 16);
  const uint32_t s0 = w[0].y, s1 = w[0].z, s2 = w[0].w;
  const uint32_t scA = s0 & 0x3F3F3F3Fu;
  const uint32_t scB = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
  const uint32_t mA = s1 & 0x3F3F3F3Fu;
  const uint32_t mB = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    B.sc[j] = (scA >> (8 * j)) & 0xff;
    B.sc[j + 4] = (scB >> (8 * j)) & 0xff;
  }
  B.mp[0] = mA & 0x00FF00FFu;
  B.mp[1] = (mA >> 8) & 0x00FF00FFu;
  B.mp[2] = mB & 0x00FF00FFu;
  B.mp[3] = (mB >> 8) & 0x00FF00FFu;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const uint4 a = w[1 + 2 * c], b = w[2 + 2 * c];
    const uint32_t qd[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      B.lo[8 * c + k] = qd[k] & 0x0F0F0F0Fu;
      B.hi[8 * c + k] = (qd[k] >> 4) & 0x0F0F0F0Fu;
    }
  }
}

// Exact value of the block against one member: xq = the member's 256 quants of this block,
// pairs = its 12 pair dwords, sx its block scale.
__device__ __forceinline__ float q4_value(const Q4Blk& B, const int8_t* __restrict__ xq,
                                          const uint32_t* __restrict__ pairs, float sx) {
  int sd = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const uint4 xl0 = reinterpret_cast<const uint4*>(xq + 64 * c)[0];
    const uint4 xl1 = reinterpret_cast<const uint4*>(xq + 64 * c)[1];
    const uint4 xh0 = reinterpret_cast<const uint4*>(xq + 64 * c + 32)[0];
    const uint4 xh1 = reinterpret_cast<const uint4*>(xq + 64 * c + 32)[1];
    const uint32_t xl[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
    const uint32_t xh[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};
    int dl = 0, dh = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      dl = __builtin_amdgcn_sdot4((int)B.lo[8 * c + k], (int)xl[k], dl, false);
      dh = __builtin_amdgcn_sdot4((int)B.hi[8 * c + k], (int)xh[k], dh, false);
    }
    sd += B.sc[2 * c] * dl + B.sc[2 * c + 1] * dh;
  }
  int sm = dot2(B.mp[0], pairs[0], 0);
  sm = dot2(B.mp[1], pairs[1], sm);
  sm = dot2(B.mp[2], pairs[2], sm);
  sm = dot2(B.mp[3], pairs[3], sm);
  const float a = B.d * (float)sd;
  const float b = B.dmin * (float)sm;
  return sx * (a - b);
}

// ---- Q6_K row block ----------------------------------------------------------------------------
struct Q6Blk {
  uint32_t q[64];   // 6-bit quants 0..63 in element order (dword i = elements 4i..4i+3)
  uint32_t sc4[4];  // the 16 i8 scales, four per dword
  uint32_t scp[8];  // i8 scales as int16 pairs (sc4i, sc4i+2), (sc4i+1, sc4i+3)
  float d;
};

// Bytes 0..207 of the block (ql, qh, scales) in 13 chunks, then the f16 d from the tail.
__device__ __forceinline__ void q6_load(uint4 (&w)[13], uint32_t& dbits, const uint8_t* __restrict__ tb, int row) {
#pragma unroll
  for (int k = 0; k < 13; ++k) w[k] = ld16_nt(tb + 1024 * k + 16 * row);
  dbits = *reinterpret_cast<const uint16_t*>(tb + 13 * 1024 + 2 * row);
}

// dequant.rs:122-138 / matmul.rs:496-525: element 128n + 32g + l takes the low (g<2) or high
// nibble of ql[64n + 32(g&1) + l] and bits 2g..2g+1 of qh[32n + l].
__device__ __forceinline__ void q6_prep(Q6Blk& B, const uint4 (&w)[13], uint32_t dbits) {
  uint32_t bd[52];  // block dwords
#pragma unroll
  for (int k = 0; k < 13; ++k) {
    bd[4 * k] = w[k].x;
    bd[4 * k + 1] = w[k].y;
    bd[4 * k + 2] = w[k].z;
    bd[4 * k + 3] = w[k].w;
  }
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    const int n = i >> 5, g = (i & 31) >> 3, k = i & 7;
    const uint32_t ql = bd[16 * n + 8 * (g & 1) + k];
    const uint32_t qh = bd[32 + 8 * n + k];
    const uint32_t lo = (g >> 1) ? ((ql >> 4) & 0x0F0F0F0Fu) : (ql & 0x0F0F0F0Fu);
    B.q[i] = lo | (((qh >> (2 * g)) & 0x03030303u) << 4);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t s = bd[48 + i];
    B.sc4[i] = s;
    const int s0 = (int)(int8_t)(s & 0xff), s1 = (int)(int8_t)((s >> 8) & 0xff);
    const int s2 = (int)(int8_t)((s >> 16) & 0xff), s3 = (int)(int8_t)(s >> 24);
    B.scp[2 * i] = pack16(s0, s2);
    B.scp[2 * i + 1] = pack16(s1, s3);
  }
  B.d = f16_bits_to_f32(dbits);
}

// s = Σ_k sc_k·Σ_{i∈k}(q_i − 32)·x_i = Σ_k sc_k·D_k − 32·Σ_k sc_k·T_k (exact; matmul.rs:692-742).
__device__ __forceinline__ float q6_value(const Q6Blk& B, const int8_t* __restrict__ xq,
                                          const uint32_t* __restrict__ pairs, float sx) {
  int s = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint4 x = reinterpret_cast<const uint4*>(xq + 16 * k)[0];
    int dk = __builtin_amdgcn_sdot4((int)B.q[4 * k], (int)x.x, 0, false);
    dk = __builtin_amdgcn_sdot4((int)B.q[4 * k + 1], (int)x.y, dk, false);
    dk = __builtin_amdgcn_sdot4((int)B.q[4 * k + 2], (int)x.z, dk, false);
    dk = __builtin_amdgcn_sdot4((int)B.q[4 * k + 3], (int)x.w, dk, false);
    s += (int)(int8_t)(B.sc4[k >> 2] >> (8 * (k & 3))) * dk;
  }
  int corr = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) corr = dot2(B.scp[j], pairs[4 + j], corr);
  s -= 32 * corr;
  return sx * (B.d * (float)s);
}

// Policy wrappers used by the kernels; load() takes the tile-block address.
template <int DT>
struct LaneRow;

template <>
struct LaneRow<DT_Q4_K> {
  static constexpr size_t TB_BYTES = pack_tile_block_bytes(DT_Q4_K);
  using Blk = Q4Blk;
  struct Loaded {
    uint4 w[9];
  };
  // row j of the tile-block at blk (j = the lane when omitted)
  static __device__ __forceinline__ void load(Loaded& L, const uint8_t* blk, int j = threadIdx.x & 63) {
    q4_load(L.w, blk, j);
  }
  static __device__ __forceinline__ void prep(Blk& B, const Loaded& L) { q4_prep(B, L.w); }
  static __device__ __forceinline__ float value(const Blk& B, const int8_t* xq, const uint32_t* pairs, float sx) {
    return q4_value(B, xq, pairs, sx);
  }
};

template <>
struct LaneRow<DT_Q6_K> {
  static constexpr size_t TB_BYTES = pack_tile_block_bytes(DT_Q6_K);
  using Blk = Q6Blk;
  struct Loaded {
    uint4 w[13];
    uint32_t dbits;
  };
  static __device__ __forceinline__ void load(Loaded& L, const uint8_t* tb, int j = threadIdx.x & 63) {
    q6_load(L.w, L.dbits, tb, j);
  }
  static __device__ __forceinline__ void prep(Blk& B, const Loaded& L) { q6_prep(B, L.w, L.dbits); }
  static __device__ __forceinline__ float value(const Blk& B, const int8_t* xq, const uint32_t* pairs, float sx) {
    return q6_value(B, xq, pairs, sx);
  }
};

}  // namespace bb
#endif
