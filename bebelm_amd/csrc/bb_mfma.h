// bb_mfma.h — int8 MFMA building blocks of the grouped expert GEMMs (Q4_K / Q6_K rows against
// Q8 activation rows).
//
// MFMA v_mfma_i32_16x16x64_i8 with the activations as A (16 members x 64 elements; lane l:
// member l%16) and the weights as B (64 elements x 16 rows; lane l: row l%16); lane group
// g = l/16 supplies 16 consecutive elements of each 64-element step for both (Q6_K: elements
// 64c + 16g.. of step c; Q4_K: 64g + 16s.. of step s, see q4_block), so a lane's weights of a
// step lie in one sub-block and its activations are one 16-byte chunk of the member's row.
// D lane l = members 4(l/16)..+3 of row l%16.
//
// Operands in LDS, per 256-element super-block b:
//   weights      the packed tile-block of the 64-row tile verbatim (chunk k of lane/row j at
//                1024k + 16j, Q6_K's d values after the 13 chunks)
//   activations  member m's 256 quants as 16-byte chunks, chunk c at position c ^ (m%16) of
//                the member's 256-byte row (conflict-free 16-byte reads)
//   scales       sx of the members
#ifndef BB_MFMA_H
#define BB_MFMA_H
#include "bb_device.h"
#include "bb_internal.h"

namespace bb {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

enum : int { GEMM_GATEUP = 0, GEMM_DOWN = 1 };

constexpr size_t TB4 = pack_tile_block_bytes(DT_Q4_K);
constexpr size_t TB6 = pack_tile_block_bytes(DT_Q6_K);

// Bytes of q (each <= 15) times s (<= 7), per byte; the products stay below 256.
__device__ __forceinline__ uint32_t mul_bytes(uint32_t q, uint32_t s) {
  const v2u16 a = __builtin_bit_cast(v2u16, q);
  const v2u16 m = {(unsigned short)s, (unsigned short)s};
  return __builtin_bit_cast(uint32_t, a * m);
}

__device__ __forceinline__ long as_long(uint32_t lo, uint32_t hi) {
  return (long)(((unsigned long)hi << 32) | lo);
}

template <int DT>
struct GemmTraits;
template <>
struct GemmTraits<DT_Q4_K> {
  static constexpr int TB = (int)TB4;
};
template <>
struct GemmTraits<DT_Q6_K> {
  static constexpr int TB = (int)TB6;
};

__device__ __forceinline__ v4i read_x16(const uint8_t* xb, int m, int chunk) {
  return *reinterpret_cast<const v4i*>(xb + m * QK + 16 * (chunk ^ (m & 15)));
}

__device__ __forceinline__ uint32_t splat_byte(uint32_t v) { return __builtin_amdgcn_perm(0u, v, 0u); }

// Q4_K: sd = Σ_j sc_j·Σ q·x with sc = 8·(sc>>3) + (sc&7): both weight products stay <= 105, so
// the high- and low-scale passes give sd = 8·Dh + Dl; a third pass with weight m_j for every
// element of sub-block j gives sm = Σ_j m_j·S_j. Epilogue matmul.rs:242 in the reference's order.
//
// The elements of a super-block are dealt to steps and lane groups g-major: step s, lane group
// g takes elements 64g + 16s .. +15 (activation chunk 4g + s). A lane group then covers the
// two sub-blocks of qs bytes 32g..32g+31 (dequant.rs:87-104): their low nibbles in steps 0-1
// (sub-block 2g) and their high nibbles in steps 2-3 (sub-block 2g+1), so a lane loads two
// 16-byte qs words per super-block instead of four and each sub-block's scale and min serve
// two steps. The sums over the 256 elements are the same integers in any order.
struct Q4Lane {
  float dd, dm;
  uint32_t hs[2], ls[2];  // sub-block 2g + h: sc >> 3, sc & 7
  int ms[2];              // its min in every byte
  int m[2];               // its min
};

__device__ __forceinline__ Q4Lane q4_lane(uint4 hd, int g) {
  Q4Lane o;
  o.dd = f16_bits_to_f32(hd.x & 0xffff);
  o.dm = f16_bits_to_f32(hd.x >> 16);
  // get_scale_min_k4 (dequant.rs:64-72) four bytes at a time; sub-blocks 2g, 2g+1 lie in the
  // dword of sub-blocks 0-3 (g < 2) or 4-7, bytes 2(g&1) and 2(g&1) + 1
  // (bitwise selects: the lane groups differ, and a branch would run both arms one after the other)
  const uint32_t s0 = hd.y, s1 = hd.z, s2 = hd.w;
  const uint32_t upper = 0u - (uint32_t)(g >> 1);  // all ones for g >= 2
  const uint32_t sw = (((s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u)) & upper) | (s0 & 0x3F3F3F3Fu & ~upper);
  const uint32_t mw = ((((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u)) & upper) | (s1 & 0x3F3F3F3Fu & ~upper);
  const uint32_t sh = 16 * (g & 1);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t scv = (sw >> (sh + 8 * h)) & 0xffu;
    o.hs[h] = scv >> 3;
    o.ls[h] = scv & 7u;
    o.ms[h] = (int)splat_byte(mw >> (sh + 8 * h));
    o.m[h] = (int)((mw >> (sh + 8 * h)) & 0xffu);
  }
  return o;
}

// the weight operands of step s (h = s >> 1, a compile-time constant) from the lane's qs half
// s & 1: its low (h = 0) or high (h = 1) nibbles times the scale of sub-block 2g + h
__device__ __forceinline__ void q4_step_ops(const uint4 qv, int h, const Q4Lane& L, v4i& Bh, v4i& Bl) {
  const uint32_t nsh = 4 * h;
  const uint32_t q[4] = {(qv.x >> nsh) & 0x0F0F0F0Fu, (qv.y >> nsh) & 0x0F0F0F0Fu, (qv.z >> nsh) & 0x0F0F0F0Fu,
                         (qv.w >> nsh) & 0x0F0F0F0Fu};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    Bh[k] = (int)mul_bytes(q[k], L.hs[h]);
    Bl[k] = (int)mul_bytes(q[k], L.ls[h]);
  }
}

// MF: the min term sm from the members' sum records in msb (min_split_record: member m's 16
// halves at msb + 32m, lane group g's four at + 8g) by one f16 MFMA per member tile, against
// weights [64·m_{2g}, 64·m_{2g+1}, m_{2g}, m_{2g+1}]: sm arrives as an exact f32, instead of a
// third int8 pass over the block (four MFMAs) and a conversion.
template <int MT, bool MF = false>
__device__ __forceinline__ void q4_block(const uint8_t* wt, const uint8_t* xb, const float* sb, const uint8_t* msb,
                                         int row, float (&acc)[MT][4]) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const Q4Lane L = q4_lane(*reinterpret_cast<const uint4*>(wt + 16 * row), g);
  uint4 qv[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) qv[k] = *reinterpret_cast<const uint4*>(wt + 1024 * (1 + 2 * g + k) + 16 * row);
  v4i Bm[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) Bm[h] = (v4i){L.ms[h], L.ms[h], L.ms[h], L.ms[h]};
  if constexpr (MT == 1) {
    // one member tile: the operands of step s feed its three MFMAs right away (fewer live
    // registers, so more blocks fit on a CU)
    v4i Dh = {0, 0, 0, 0}, Dl = {0, 0, 0, 0}, Dm = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      v4i Bh, Bl;
      q4_step_ops(qv[s & 1], s >> 1, L, Bh, Bl);
      const v4i ax = read_x16(xb, r, 4 * g + s);
      Dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, Bh, Dh, 0, 0, 0);
      Dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, Bl, Dl, 0, 0, 0);
      Dm = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, Bm[s >> 1], Dm, 0, 0, 0);
    }
    const float4 sx4 = *reinterpret_cast<const float4*>(sb + 4 * g);
    const float sxv[4] = {sx4.x, sx4.y, sx4.z, sx4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int sd = 8 * Dh[i] + Dl[i];
      const float v = sxv[i] * ((L.dd * (float)sd) - (L.dm * (float)Dm[i]));
      acc[0][i] += v;
    }
    return;
  }
  // the lane's weight operands for the whole block first, then member tile by member tile:
  // twelve MFMAs, during which the next tile's activation chunks are read (each chunk once its
  // three MFMAs are issued), and the tile's f32 epilogue
  v4i Bh[4], Bl[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) q4_step_ops(qv[s & 1], s >> 1, L, Bh[s], Bl[s]);
  v4h bmin;
  if constexpr (MF)
    bmin = (v4h){(_Float16)(64 * L.m[0]), (_Float16)(64 * L.m[1]), (_Float16)L.m[0], (_Float16)L.m[1]};
  v4i ax[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) ax[s] = read_x16(xb, r, 4 * g + s);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    v4i D[3] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
    v4f Dmf = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (MF) {
      const v4h am = *reinterpret_cast<const v4h*>(msb + (mt * 16 + r) * 32 + 8 * g);
      Dmf = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bmin, Dmf, 0, 0, 0);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      D[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[s], Bh[s], D[0], 0, 0, 0);
      D[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[s], Bl[s], D[1], 0, 0, 0);
      if constexpr (!MF) D[2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[s], Bm[s >> 1], D[2], 0, 0, 0);
      if (mt + 1 < MT) ax[s] = read_x16(xb, (mt + 1) * 16 + r, 4 * g + s);
    }
    const float4 sx4 = *reinterpret_cast<const float4*>(sb + mt * 16 + 4 * g);
    const float sxv[4] = {sx4.x, sx4.y, sx4.z, sx4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int sd = 8 * D[0][i] + D[1][i];
      const float smf = MF ? Dmf[i] : (float)D[2][i];
      const float v = sxv[i] * ((L.dd * (float)sd) - (L.dm * smf));
      acc[mt][i] += v;
    }
  }
}

// (hi, lo) int8 parts of sc*(q - 32) for four quant bytes q (<= 63): the products are formed
// in 16-bit lanes (even and odd bytes) and the bytes put back in order.
__device__ __forceinline__ void q6_split(uint32_t q, uint32_t scp, uint32_t bias, uint32_t& h, uint32_t& l) {
  typedef short v2i16 __attribute__((ext_vector_type(2)));
  const v2i16 ev = __builtin_bit_cast(v2i16, q & 0x00FF00FFu);
  const v2i16 od = __builtin_bit_cast(v2i16, (q >> 8) & 0x00FF00FFu);
  const v2i16 sc2 = __builtin_bit_cast(v2i16, scp), b2 = __builtin_bit_cast(v2i16, bias);
  const v2i16 ae = ev * sc2 + b2, ao = od * sc2 + b2;  // sc*q - 32*sc, exact in 16 bits
  const uint32_t ue = __builtin_bit_cast(uint32_t, ae), uo = __builtin_bit_cast(uint32_t, ao);
  const uint32_t he = __builtin_bit_cast(uint32_t, ae >> (v2i16){6, 6});
  const uint32_t ho = __builtin_bit_cast(uint32_t, ao >> (v2i16){6, 6});
  // bytes {e0, o0, e1, o1} from the low bytes of the 16-bit lanes (v_perm: bytes 0-3 of the
  // second operand, 4-7 of the first)
  l = __builtin_amdgcn_perm(uo & 0x003F003Fu, ue & 0x003F003Fu, 0x06020400u);
  h = __builtin_amdgcn_perm(ho, he, 0x06020400u);
}

// Q6_K: s = Σ_j sc_j·Σ (q − 32)·x. With a = sc_j·(q − 32) (|a| <= 4096) split as a = 64·h + l,
// h in [−64, 64] and l in [0, 63] both fit int8: two passes give s = 64·Dh + Dl. Epilogue
// matmul.rs:641: sx·(d·(float)s).
template <int MT>
__device__ __forceinline__ void q6_block(const uint8_t* wt, const uint8_t* xb, const float* sb, int row,
                                         float (&acc)[MT][4]) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const uint4 sc = *reinterpret_cast<const uint4*>(wt + 1024 * 12 + 16 * row);
  const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(wt + 1024 * 13 + 2 * row));
  v4i Bh[4], Bl[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    // elements 64c + 16g + t = 128n + 32gq + 16(g&1) + t with n = c/2, gq = 2(c&1) + g/2
    // (dequant.rs:122-138): ql[64n + 32(g/2) + 16(g&1) + t] (high nibble when c is odd) and
    // bits 2gq of qh[32n + 16(g&1) + t]; sub-block j = 4c + g
    const int n2 = c >> 1, gq = 2 * (c & 1) + (g >> 1);
    const uint4 qlv = *reinterpret_cast<const uint4*>(wt + 1024 * (4 * n2 + 2 * (g >> 1) + (g & 1)) + 16 * row);
    const uint4 qhv = *reinterpret_cast<const uint4*>(wt + 1024 * (8 + 2 * n2 + (g & 1)) + 16 * row);
    const uint32_t lsh = 4 * (c & 1), hsh = 2 * gq;
    const uint32_t scd = c == 0 ? sc.x : c == 1 ? sc.y : c == 2 ? sc.z : sc.w;
    const int scj = (int)(int8_t)((scd >> (8 * g)) & 0xffu);
    const uint32_t scp = ((uint32_t)scj & 0xffffu) * 0x00010001u;
    const uint32_t bias = ((uint32_t)(-32 * scj) & 0xffffu) * 0x00010001u;
    const uint32_t qlw[4] = {qlv.x, qlv.y, qlv.z, qlv.w}, qhw[4] = {qhv.x, qhv.y, qhv.z, qhv.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t q = ((qlw[k] >> lsh) & 0x0F0F0F0Fu) | (((qhw[k] >> hsh) & 0x03030303u) << 4);
      uint32_t hh, ll;
      q6_split(q, scp, bias, hh, ll);
      Bh[c][k] = (int)hh;
      Bl[c][k] = (int)ll;
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    v4i Dh = {0, 0, 0, 0}, Dl = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const v4i ax = read_x16(xb, mt * 16 + r, 4 * c + g);
      Dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, Bh[c], Dh, 0, 0, 0);
      Dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, Bl[c], Dl, 0, 0, 0);
    }
    const float4 sx4 = *reinterpret_cast<const float4*>(sb + mt * 16 + 4 * g);
    const float sxv[4] = {sx4.x, sx4.y, sx4.z, sx4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int sv = 64 * Dh[i] + Dl[i];
      const float v = sxv[i] * (d * (float)sv);
      acc[mt][i] += v;
    }
  }
}

}  // namespace bb
#endif
