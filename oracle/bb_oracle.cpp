// bb_oracle.cpp — TEST INFRASTRUCTURE ONLY (see bb_oracle.h for scope and pinning status).
//
// A C++ restatement of the reference's CPU MoE FFN path. All f32 arithmetic follows the
// Rust source's evaluation order with no FMA contraction (built with -ffp-contract=off);
// fmaf appears only where the reference's `wide::f32x8::mul_add` fuses. Integer dots are
// exact, so the reference's several SIMD variants (portable / NEON sdot / AVX-512 VNNI) all
// reduce to one integer here. OpenMP parallelism is over output rows only, mirroring rayon's
// partition (matmul.rs:888-891, :946-984, :1048-1052); results are thread-count independent.
#include "bb_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__AVX2__)
#include <immintrin.h>
#endif

namespace {

constexpr int QK = 256;
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BYTES = 210;
constexpr int PAR_MIN_ROWS = 64;  // matmul.rs:20

inline float f32_from_bits(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t bits_of(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

// dequant.rs:22-54 — exact f16 -> f32 widening, subnormals normalised by a shift loop.
float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t(h) & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t mant = h & 0x03ff;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      int e = -1;
      uint32_t m = mant;
      do { e += 1; m <<= 1; } while ((m & 0x0400) == 0);
      bits = sign | (uint32_t(127 - 15 - e) << 23) | ((m & 0x03ff) << 13);
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else {
    bits = sign | (uint32_t(int(exp) - 15 + 127) << 23) | (mant << 13);
  }
  return f32_from_bits(bits);
}

inline float rd_f16(const uint8_t* p) { return f16_to_f32(uint16_t(p[0] | (p[1] << 8))); }

// dequant.rs:64-72 (ggml get_scale_min_k4).
inline void scale_min_k4(int j, const uint8_t* s, uint8_t& sc, uint8_t& m) {
  if (j < 4) {
    sc = s[j] & 63;
    m = s[j + 4] & 63;
  } else {
    sc = uint8_t((s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4));
    m = uint8_t((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}

// dequant.rs:75-106.
void dequant_q4k_block(const uint8_t* block, float* out) {
  float d = rd_f16(block), dmin = rd_f16(block + 2);
  const uint8_t* scales = block + 4;
  const uint8_t* qs = block + 16;
  int oi = 0;
  for (int chunk = 0; chunk < 4; ++chunk) {
    uint8_t sc1, m1, sc2, m2;
    scale_min_k4(2 * chunk, scales, sc1, m1);
    scale_min_k4(2 * chunk + 1, scales, sc2, m2);
    float d1 = d * float(sc1), min1 = dmin * float(m1);
    float d2 = d * float(sc2), min2 = dmin * float(m2);
    const uint8_t* q = qs + chunk * 32;
    for (int i = 0; i < 32; ++i) out[oi++] = d1 * float(q[i] & 0x0f) - min1;
    for (int i = 0; i < 32; ++i) out[oi++] = d2 * float(q[i] >> 4) - min2;
  }
}

// dequant.rs:112-139. `d * sc as f32 * q as f32` evaluates left to right.
void dequant_q6k_block(const uint8_t* block, float* out) {
  float d = rd_f16(block + 208);
  for (int n = 0; n < 2; ++n) {
    const uint8_t* ql = block + n * 64;
    const uint8_t* qh = block + 128 + n * 32;
    const int8_t* sc = reinterpret_cast<const int8_t*>(block + 192 + n * 8);
    float* o = out + n * 128;
    for (int l = 0; l < 32; ++l) {
      int is = l / 16;
      int q1 = int((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
      int q2 = int((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
      int q3 = int((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
      int q4 = int((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
      o[l] = d * float(sc[is]) * float(q1);
      o[l + 32] = d * float(sc[is + 2]) * float(q2);
      o[l + 64] = d * float(sc[is + 4]) * float(q3);
      o[l + 96] = d * float(sc[is + 6]) * float(q4);
    }
  }
}

bool dtype_block(uint32_t dt, int& elems, int& bytes) {
  switch (dt) {  // tensor.rs:68-93
    case BBO_F32: elems = 1; bytes = 4; return true;
    case BBO_F16: elems = 1; bytes = 2; return true;
    case BBO_Q4_K: elems = QK; bytes = Q4K_BYTES; return true;
    case BBO_Q6_K: elems = QK; bytes = Q6K_BYTES; return true;
    default: return false;
  }
}

// dequant.rs:151-175.
bool dequantize_into(uint32_t dt, const uint8_t* data, size_t n, float* out) {
  switch (dt) {
    case BBO_F32: std::memcpy(out, data, n * 4); return true;
    case BBO_F16: for (size_t i = 0; i < n; ++i) out[i] = rd_f16(data + 2 * i); return true;
    case BBO_Q4_K: for (size_t b = 0; b < n / QK; ++b) dequant_q4k_block(data + b * Q4K_BYTES, out + b * QK); return true;
    case BBO_Q6_K: for (size_t b = 0; b < n / QK; ++b) dequant_q6k_block(data + b * Q6K_BYTES, out + b * QK); return true;
    default: return false;
  }
}

// --- Q8 activations (matmul.rs:130-160) ---
struct Q8 {
  std::vector<int8_t> q;
  std::vector<float> scales;
  std::vector<int32_t> sums;
};

// Rust f32::round: half away from zero (== C roundf). `as i8` saturates, NaN -> 0.
inline int8_t q8_round(float v) {
  float r = std::round(v);
  r = std::min(std::max(r, -127.0f), 127.0f);
  if (std::isnan(r)) return 0;
  return int8_t(r);
}

void quantize_q8_into(const float* x, size_t n, int8_t* q, float* scales, int32_t* sums) {
  size_t nb = n / QK;
  for (size_t b = 0; b < nb; ++b) {
    const float* xb = x + b * QK;
    float amax = 0.0f;
    for (int i = 0; i < QK; ++i) amax = std::fmax(amax, std::fabs(xb[i]));  // f32::max ignores NaN
    scales[b] = amax / 127.0f;
    float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    int8_t* qb = q + b * QK;
    for (int i = 0; i < QK; ++i) qb[i] = q8_round(xb[i] * inv);
    for (int s = 0; s < 8; ++s) {
      int32_t acc = 0;
      for (int i = 0; i < 32; ++i) acc += qb[s * 32 + i];
      sums[b * 8 + s] = acc;
    }
  }
}

Q8 quantize_q8(const float* x, size_t n) {
  Q8 r;
  r.q.resize(n);
  r.scales.resize(n / QK);
  r.sums.resize(n / 32);
  quantize_q8_into(x, n, r.q.data(), r.scales.data(), r.sums.data());
  return r;
}

struct Q8View {
  const int8_t* q;
  const float* scales;
  const int32_t* sums;
};
inline Q8View view(const Q8& a) { return {a.q.data(), a.scales.data(), a.sums.data()}; }

// --- f32 dot (matmul.rs:36-66) ---
// Four f32x8 accumulators = 32 independent fmaf chains over i = c (mod 32); the lane-wise
// combine `(acc0+acc1)+(acc2+acc3)` then `reduce_add` in the `wide` 0.7.33 AVX order
// ((v0+v4)+(v2+v6))+((v1+v5)+(v3+v7)). The crate is not vendored: this order is an assumption.
inline float reduce_add8(const float v[8]) {
  return ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
}

float dot_f32(const float* a, const float* b, size_t n) {
  float acc[4][8] = {};
  size_t i = 0;
  while (i + 32 <= n) {
    for (int k = 0; k < 4; ++k)
      for (int l = 0; l < 8; ++l) acc[k][l] = std::fmaf(a[i + 8 * k + l], b[i + 8 * k + l], acc[k][l]);
    i += 32;
  }
  while (i + 8 <= n) {
    for (int l = 0; l < 8; ++l) acc[0][l] = std::fmaf(a[i + l], b[i + l], acc[0][l]);
    i += 8;
  }
  float v[8];
  for (int l = 0; l < 8; ++l) v[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
  float sum = reduce_add8(v);
  while (i < n) { sum += a[i] * b[i]; ++i; }
  return sum;
}

// Other plausible evaluation orders of the same dot (matmul.rs:36-66), for the routing
// robustness check (tests/test_router_orders.py): the `wide` crate's lane reduce and its
// mul_add fallback differ by target, and the reference's CI also builds x86-64-v2 (no FMA,
// .github/workflows/ci.yml:28-35), where mul_add is a rounded multiply, then an add.
//   0  dot_f32: FMA chains, AVX reduce tree (the order the restatement assumes)
//   1  multiply-then-add chains, AVX reduce tree
//   2  FMA chains; lanes folded v_i + v_{i+4}, then (s0+s1)+(s2+s3) (a pairwise horizontal add)
//   3  multiply-then-add chains; the 8 lanes summed left to right
//   4  left-to-right f32 sum of rounded products (scalar loop)
//   5  f64 sum of the exact products, rounded once to f32
//   6  multiply-then-add chains; lanes folded v_i + v_{i+4}, then (s0+s1)+(s2+s3) (what a
//      non-AVX x86-64-v2 build computes when its reduce is the pairwise fold)
float dot_variant(const float* a, const float* b, size_t n, int variant) {
  if (variant == 0) return dot_f32(a, b, n);
  if (variant == 4) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += a[i] * b[i];
    return s;
  }
  if (variant == 5) {
    double s = 0.0;
    for (size_t i = 0; i < n; ++i) s += double(a[i]) * double(b[i]);
    return float(s);
  }
  const bool fma = variant == 2;
  const bool pairwise = variant == 2 || variant == 6;
  float acc[4][8] = {};
  size_t i = 0;
  while (i + 32 <= n) {
    for (int k = 0; k < 4; ++k)
      for (int l = 0; l < 8; ++l) {
        const float p = a[i + 8 * k + l], q = b[i + 8 * k + l];
        acc[k][l] = fma ? std::fmaf(p, q, acc[k][l]) : acc[k][l] + p * q;
      }
    i += 32;
  }
  while (i + 8 <= n) {
    for (int l = 0; l < 8; ++l) acc[0][l] = fma ? std::fmaf(a[i + l], b[i + l], acc[0][l]) : acc[0][l] + a[i + l] * b[i + l];
    i += 8;
  }
  float v[8];
  for (int l = 0; l < 8; ++l) v[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
  float sum;
  if (variant == 1) {
    sum = reduce_add8(v);
  } else if (pairwise) {
    float f[4];
    for (int l = 0; l < 4; ++l) f[l] = v[l] + v[l + 4];
    sum = (f[0] + f[1]) + (f[2] + f[3]);
  } else {
    sum = v[0];
    for (int l = 1; l < 8; ++l) sum += v[l];
  }
  while (i < n) { sum += a[i] * b[i]; ++i; }
  return sum;
}

// --- integer dots of unsigned weight bytes against Q8 activations -------------------------------
// The reference computes its Q4_K / Q6_K block dots with AVX-512 VNNI byte dots on x86 builds
// that have them (matmul.rs:262-289, :699-744) and with widening multiply-adds elsewhere. The
// sums are exact integers (no overflow: |sd| < 2^25), so any grouping gives the same value;
// the vector forms below only make the restatement run at a speed comparable to the
// reference's, for the CPU baseline. Each has the scalar loop it must equal beside it
// (tests/test_oracle_pins.py checks them against brute-force dequantised dots).
#if defined(__AVX2__)
// 32 bytes: u8 a[i]·s8 b[i] summed in groups of four, 8 i32 lanes (lane k: bytes 4k..4k+3).
inline __m256i dot_u8s8(__m256i a, __m256i b) {
#if defined(__AVX512VNNI__) && defined(__AVX512VL__)
  return _mm256_dpbusd_epi32(_mm256_setzero_si256(), a, b);
#else
  // pairs of products in i16: a <= 63 and |b| <= 127, so a pair stays below 2^14 (no saturation)
  return _mm256_madd_epi16(_mm256_maddubs_epi16(a, b), _mm256_set1_epi16(1));
#endif
}
inline int32_t hsum8(__m256i v) {
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
  return _mm_cvtsi128_si32(s);
}
inline __m256i load32(const void* p) { return _mm256_loadu_si256(static_cast<const __m256i*>(p)); }
// lanes 0-3 = a, lanes 4-7 = b (the scales of a 32-byte run's two 16-element sub-blocks)
inline __m256i two_scales(int32_t a, int32_t b) { return _mm256_setr_epi32(a, a, a, a, b, b, b, b); }
#endif

// --- Q4_K x Q8 (matmul.rs:210-298) ---
// Σ_j sc_j·<nib_j, qx_j>, exact i32 (q4k_block_sd_portable, :251-260; equal to the VNNI
// and sdot variants by the reference's own tests :1456-1485): sub-block 2c is the low nibbles
// of qs bytes 32c.., 2c+1 their high nibbles.
int32_t q4k_sd(const uint8_t* qs, const int32_t sc[8], const int8_t* qx) {
#if defined(__AVX2__)
  const __m256i m4 = _mm256_set1_epi8(0x0f);
  __m256i acc = _mm256_setzero_si256();
  for (int c = 0; c < 4; ++c) {
    const __m256i q = load32(qs + 32 * c);
    const __m256i lo = _mm256_and_si256(q, m4), hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
    acc = _mm256_add_epi32(acc, _mm256_mullo_epi32(dot_u8s8(lo, load32(qx + 64 * c)), _mm256_set1_epi32(sc[2 * c])));
    acc = _mm256_add_epi32(acc,
                           _mm256_mullo_epi32(dot_u8s8(hi, load32(qx + 64 * c + 32)), _mm256_set1_epi32(sc[2 * c + 1])));
  }
  return hsum8(acc);
#else
  int32_t sd = 0;
  for (int c = 0; c < 4; ++c) {
    int32_t lo = 0, hi = 0;
    for (int i = 0; i < 32; ++i) {
      lo += int32_t(qs[c * 32 + i] & 0x0f) * qx[(2 * c) * 32 + i];
      hi += int32_t(qs[c * 32 + i] >> 4) * qx[(2 * c + 1) * 32 + i];
    }
    sd += sc[2 * c] * lo + sc[2 * c + 1] * hi;
  }
  return sd;
#endif
}

// matmul.rs:220-243.
float dot_q4k_block_q8(const uint8_t* block, const int8_t* qx, float sx, const int32_t* sums) {
  float d = rd_f16(block), dmin = rd_f16(block + 2);
  int32_t sc[8];
  int32_t sm = 0;
  for (int j = 0; j < 8; ++j) {
    uint8_t s, m;
    scale_min_k4(j, block + 4, s, m);
    sc[j] = s;
    sm += int32_t(m) * sums[j];
  }
  int32_t sd = q4k_sd(block + 16, sc, qx);
  return sx * (d * float(sd) - dmin * float(sm));
}

// matmul.rs:293-298. `Iterator::sum` for f32 starts from -0.0 on the Rust toolchains this
// crate needs (it calls u64::is_multiple_of, stable since 1.87); it only decides the sign
// of an all-(-0.0) row.
float dot_q4k_row_q8(const uint8_t* row, size_t n_blocks, Q8View a) {
  float sum = -0.0f;
  for (size_t b = 0; b < n_blocks; ++b)
    sum += dot_q4k_block_q8(row + b * Q4K_BYTES, a.q + b * QK, a.scales[b], a.sums + b * 8);
  return sum;
}

// --- Q6_K x Q8 (matmul.rs:496-771) ---
// unpack_q6k_block (:496-525): 256 recentred int8 weights in sub-block order + 16 scales.
void unpack_q6k(const uint8_t* block, int8_t wq[256], int32_t sc[16]) {
  static const int GROUPS[4][3] = {{0, 0, 0}, {32, 0, 2}, {0, 1, 4}, {32, 1, 6}};
  int k = 0;
  for (int n = 0; n < 2; ++n) {
    const uint8_t* ql = block + n * 64;
    const uint8_t* qh = block + 128 + n * 32;
    const uint8_t* scn = block + 192 + n * 8;
    for (int g = 0; g < 4; ++g) {
      int ql_off = GROUPS[g][0], high = GROUPS[g][1], shift = GROUPS[g][2];
      for (int sub = 0; sub < 2; ++sub) {
        sc[k] = int32_t(int8_t(scn[2 * g + sub]));
        for (int i = 0; i < 16; ++i) {
          int li = sub * 16 + i;
          int low = high ? (ql[ql_off + li] >> 4) : (ql[ql_off + li] & 0x0f);
          int hi = (qh[li] >> shift) & 3;
          wq[k * 16 + i] = int8_t((low | (hi << 4)) - 32);
        }
        ++k;
      }
    }
  }
}

// wsd_q6k (:559-572): Σ_s sc[s]·<wq_s, qx_s>, exact i32. Vector form: wq + 32 is the unsigned
// quant q, and Σ sc·Σ wq·x = Σ sc·Σ q·x − 32·Σ sc·Σ x.
int32_t wsd_q6k(const int8_t* wq, const int8_t* qx, const int32_t sc[16]) {
#if defined(__AVX2__)
  const __m256i off = _mm256_set1_epi8(32), ones = _mm256_set1_epi8(1);
  __m256i aq = _mm256_setzero_si256(), ax = _mm256_setzero_si256();
  for (int j = 0; j < 8; ++j) {
    const __m256i q = _mm256_add_epi8(load32(wq + 32 * j), off), x = load32(qx + 32 * j);
    const __m256i scv = two_scales(sc[2 * j], sc[2 * j + 1]);
    aq = _mm256_add_epi32(aq, _mm256_mullo_epi32(dot_u8s8(q, x), scv));
    ax = _mm256_add_epi32(ax, _mm256_mullo_epi32(dot_u8s8(ones, x), scv));
  }
  return hsum8(aq) - 32 * hsum8(ax);
#else
  int32_t acc = 0;
  for (int s = 0; s < 16; ++s) {
    int32_t d = 0;
    for (int i = 0; i < 16; ++i) d += int32_t(wq[s * 16 + i]) * qx[s * 16 + i];
    acc += d * sc[s];
  }
  return acc;
#endif
}

// q6k_block_idot_portable (:650-682): the fused unpack, same exact integer. Vector form: group g
// of half n is 32 unsigned quants q = (ql nibble) | (2 qh bits << 4) of sub-blocks 2g, 2g+1,
// and Σ sc·Σ (q − 32)·x = Σ sc·Σ q·x − 32·Σ sc·Σ x.
int32_t q6k_idot_fused(const uint8_t* block, const int8_t* qx) {
#if defined(__AVX2__)
  const __m256i m4 = _mm256_set1_epi8(0x0f), m2 = _mm256_set1_epi8(0x03), ones = _mm256_set1_epi8(1);
  __m256i aq = _mm256_setzero_si256(), ax = _mm256_setzero_si256();
  for (int n = 0; n < 2; ++n) {
    const __m256i qh = load32(block + 128 + 32 * n);
    const int8_t* scn = reinterpret_cast<const int8_t*>(block + 192 + 8 * n);
    for (int g = 0; g < 4; ++g) {
      const __m256i ql = load32(block + 64 * n + 32 * (g & 1));
      const __m256i nib = (g >> 1) ? _mm256_and_si256(_mm256_srli_epi16(ql, 4), m4) : _mm256_and_si256(ql, m4);
      const __m256i h2 = _mm256_and_si256(_mm256_srl_epi16(qh, _mm_cvtsi32_si128(2 * g)), m2);
      const __m256i q = _mm256_or_si256(nib, _mm256_slli_epi16(h2, 4));
      const __m256i x = load32(qx + 128 * n + 32 * g);
      const __m256i scv = two_scales(scn[2 * g], scn[2 * g + 1]);
      aq = _mm256_add_epi32(aq, _mm256_mullo_epi32(dot_u8s8(q, x), scv));
      ax = _mm256_add_epi32(ax, _mm256_mullo_epi32(dot_u8s8(ones, x), scv));
    }
  }
  return hsum8(aq) - 32 * hsum8(ax);
#else
  static const int GROUPS[4][3] = {{0, 0, 0}, {32, 0, 2}, {0, 1, 4}, {32, 1, 6}};
  int32_t acc = 0;
  for (int n = 0; n < 2; ++n) {
    const uint8_t* ql = block + n * 64;
    const uint8_t* qh = block + 128 + n * 32;
    const uint8_t* scn = block + 192 + n * 8;
    for (int g = 0; g < 4; ++g) {
      for (int sub = 0; sub < 2; ++sub) {
        int k = n * 8 + 2 * g + sub;
        int32_t d = 0;
        for (int i = 0; i < 16; ++i) {
          int li = sub * 16 + i;
          int b = ql[GROUPS[g][0] + li];
          int low = GROUPS[g][1] ? (b >> 4) : (b & 0x0f);
          int hi = (qh[li] >> GROUPS[g][2]) & 3;
          d += ((low | (hi << 4)) - 32) * int32_t(qx[k * 16 + i]);
        }
        acc += d * int32_t(int8_t(scn[2 * g + sub]));
      }
    }
  }
  return acc;
#endif
}

// dot_q6k_block_q8 (:633-642).
float dot_q6k_block_q8(const uint8_t* block, const int8_t* qx, float sx) {
  float d = rd_f16(block + 208);
  int32_t s = q6k_idot_fused(block, qx);
  return sx * (d * float(s));
}

// dot_q6k_row_q8 (:748-753), -0.0-started sum as above.
float dot_q6k_row_q8(const uint8_t* row, size_t n_blocks, Q8View a) {
  float sum = -0.0f;
  for (size_t b = 0; b < n_blocks; ++b) sum += dot_q6k_block_q8(row + b * Q6K_BYTES, a.q + b * QK, a.scales[b]);
  return sum;
}

// --- f32 fused K-quant dots (the `qx == None` arm of matvec_fused_batch) ---
// nibble_dot32 (:73-94): per-lane fmaf into qx, plain add into xs, two reduce_adds.
void nibble_dot32(const uint8_t* q, const float* x, bool high, float& qxs, float& xss) {
  float qx[8] = {}, xs[8] = {};
  for (int k = 0; k < 4; ++k)
    for (int l = 0; l < 8; ++l) {
      uint8_t b = q[k * 8 + l];
      float nib = float(high ? (b >> 4) : (b & 0xf));
      float xv = x[k * 8 + l];
      qx[l] = std::fmaf(nib, xv, qx[l]);
      xs[l] = xs[l] + xv;
    }
  qxs = reduce_add8(qx);
  xss = reduce_add8(xs);
}

// dot_q4k_block (:104-122).
float dot_q4k_block_f32(const uint8_t* block, const float* x) {
  float d = rd_f16(block), dmin = rd_f16(block + 2);
  float sum = 0.0f;
  for (int chunk = 0; chunk < 4; ++chunk) {
    uint8_t sc1, m1, sc2, m2;
    scale_min_k4(2 * chunk, block + 4, sc1, m1);
    scale_min_k4(2 * chunk + 1, block + 4, sc2, m2);
    const uint8_t* q = block + 16 + chunk * 32;
    float qx_lo, xs_lo, qx_hi, xs_hi;
    nibble_dot32(q, x + chunk * 64, false, qx_lo, xs_lo);
    nibble_dot32(q, x + chunk * 64 + 32, true, qx_hi, xs_hi);
    sum += (d * float(sc1)) * qx_lo - (dmin * float(m1)) * xs_lo;
    sum += (d * float(sc2)) * qx_hi - (dmin * float(m2)) * xs_hi;
  }
  return sum;
}

// q6_dot16 (:430-444) and dot_q6k_block (:455-479).
float q6_dot16(const uint8_t* ql, const uint8_t* qh, int ql_off, bool high, int shift, int l_start,
               const float* x) {
  float qx[8] = {};
  for (int c = 0; c < 2; ++c) {
    int l = l_start + c * 8;
    for (int j = 0; j < 8; ++j) {
      int li = l + j;
      int low = high ? (ql[ql_off + li] >> 4) : (ql[ql_off + li] & 0x0f);
      int hi = (qh[li] >> shift) & 3;
      float q = float((low | (hi << 4)) - 32);
      qx[j] = std::fmaf(q, x[c * 8 + j], qx[j]);
    }
  }
  return reduce_add8(qx);
}

float dot_q6k_block_f32(const uint8_t* block, const float* x) {
  static const int GROUPS[4][3] = {{0, 0, 0}, {32, 0, 2}, {0, 1, 4}, {32, 1, 6}};
  float d = rd_f16(block + 208);
  float acc = 0.0f;
  for (int n = 0; n < 2; ++n) {
    const uint8_t* ql = block + n * 64;
    const uint8_t* qh = block + 128 + n * 32;
    const uint8_t* sc = block + 192 + n * 8;
    const float* xh = x + n * 128;
    for (int g = 0; g < 4; ++g) {
      const float* xg = xh + g * 32;
      for (int sub = 0; sub < 2; ++sub) {
        float sc_s = float(int8_t(sc[2 * g + sub]));
        acc += sc_s * q6_dot16(ql, qh, GROUPS[g][0], GROUPS[g][1] != 0, GROUPS[g][2], sub * 16, xg + sub * 16);
      }
    }
  }
  return d * acc;
}

// fused_row_dot (:777-785), -0.0-started sum.
float fused_row_dot(uint32_t dt, const uint8_t* row, const float* x, size_t n_in) {
  float sum = -0.0f;
  size_t nb = n_in / QK;
  if (dt == BBO_Q4_K)
    for (size_t b = 0; b < nb; ++b) sum += dot_q4k_block_f32(row + b * Q4K_BYTES, x + b * QK);
  else
    for (size_t b = 0; b < nb; ++b) sum += dot_q6k_block_f32(row + b * Q6K_BYTES, x + b * QK);
  return sum;
}

// --- matvec / matmul / fused batch ---
template <class F>
void for_rows(size_t n, bool parallel, F&& f) {
  if (parallel) {
#pragma omp parallel for schedule(static)
    for (long o = 0; o < long(n); ++o) f(size_t(o));
  } else {
    for (size_t o = 0; o < n; ++o) f(o);
  }
}

// matmul.rs:850-893.
int matvec(uint32_t dt, const uint8_t* w, size_t n_in, size_t n_out, const float* x, float* y) {
  int be, bb;
  if (!dtype_block(dt, be, bb) || n_in % size_t(be) != 0) return -1;
  size_t row_bytes = (n_in / be) * bb;
  bool par = n_out >= size_t(PAR_MIN_ROWS);
  if (dt == BBO_Q4_K || dt == BBO_Q6_K) {
    Q8 q8 = quantize_q8(x, n_in);
    Q8View v = view(q8);
    size_t nb = n_in / QK;
    for_rows(n_out, par, [&](size_t o) {
      const uint8_t* row = w + o * row_bytes;
      y[o] = dt == BBO_Q4_K ? dot_q4k_row_q8(row, nb, v) : dot_q6k_row_q8(row, nb, v);
    });
  } else {
    for_rows(n_out, par, [&](size_t o) {
      std::vector<float> scratch(n_in);
      dequantize_into(dt, w + o * row_bytes, n_in, scratch.data());
      y[o] = dot_f32(scratch.data(), x, n_in);
    });
  }
  return 0;
}

// matmul.rs:908-991. Q4_K row tiles (dot_q4k_rowtile_q8_batch :800-844) and the single-row
// batch kernels (:390-423, :761-771) both accumulate `out += scale*(…)` into a +0.0-filled
// feature-major scratch, block by block; per (row, token) that is one sequential sum.
int matmul(uint32_t dt, const uint8_t* w, size_t n_in, size_t n_out, const float* x, size_t nt, float* y) {
  if (nt == 1) return matvec(dt, w, n_in, n_out, x, y);
  int be, bb;
  if (!dtype_block(dt, be, bb) || n_in % size_t(be) != 0) return -1;
  size_t row_bytes = (n_in / be) * bb;
  bool par = n_out >= size_t(PAR_MIN_ROWS);
  std::vector<float> out_fm(n_out * nt, 0.0f);
  if (dt == BBO_Q4_K || dt == BBO_Q6_K) {
    std::vector<Q8> q8(nt);
    for (size_t t = 0; t < nt; ++t) q8[t] = quantize_q8(x + t * n_in, n_in);
    size_t nb = n_in / QK;
    for_rows(n_out, par, [&](size_t o) {
      const uint8_t* row = w + o * row_bytes;
      float* dst = out_fm.data() + o * nt;
      if (dt == BBO_Q4_K) {
        for (size_t b = 0; b < nb; ++b) {
          const uint8_t* block = row + b * Q4K_BYTES;
          float d = rd_f16(block), dmin = rd_f16(block + 2);
          int32_t sc[8], m[8];
          for (int s = 0; s < 8; ++s) {
            uint8_t a, c;
            scale_min_k4(s, block + 4, a, c);
            sc[s] = a;
            m[s] = c;
          }
          for (size_t t = 0; t < nt; ++t) {
            const int8_t* qx = q8[t].q.data() + b * QK;
            const int32_t* sums = q8[t].sums.data() + b * 8;
            int32_t sd = q4k_sd(block + 16, sc, qx);
            int32_t sm = 0;
            for (int s = 0; s < 8; ++s) sm += m[s] * sums[s];
            dst[t] += q8[t].scales[b] * (d * float(sd) - dmin * float(sm));
          }
        }
      } else {
        for (size_t b = 0; b < nb; ++b) {
          const uint8_t* block = row + b * Q6K_BYTES;
          float d = rd_f16(block + 208);
          int8_t wq[256];
          int32_t sc[16];
          unpack_q6k(block, wq, sc);
          for (size_t t = 0; t < nt; ++t) {
            int32_t s = wsd_q6k(wq, q8[t].q.data() + b * QK, sc);
            dst[t] += q8[t].scales[b] * (d * float(s));
          }
        }
      }
    });
  } else {
    for_rows(n_out, par, [&](size_t o) {
      std::vector<float> scratch(n_in);
      dequantize_into(dt, w + o * row_bytes, n_in, scratch.data());
      for (size_t t = 0; t < nt; ++t) out_fm[o * nt + t] = dot_f32(scratch.data(), x + t * n_in, n_in);
    });
  }
  for (size_t o = 0; o < n_out; ++o)
    for (size_t t = 0; t < nt; ++t) y[t * n_out + o] = out_fm[o * nt + t];
  return 0;
}

// matmul.rs:1015-1053.
int matvec_fused_batch(const bbo_job* jobs, size_t n_jobs, float* out) {
  std::vector<size_t> starts, row_bytes;
  size_t total = 0;
  for (size_t j = 0; j < n_jobs; ++j) {
    int be, bb;
    if (!dtype_block(jobs[j].dtype, be, bb) || jobs[j].n_in % size_t(be) != 0) return -1;
    if (jobs[j].has_qx && jobs[j].dtype != BBO_Q4_K && jobs[j].dtype != BBO_Q6_K) return -1;
    if (!jobs[j].has_qx && jobs[j].dtype != BBO_Q4_K && jobs[j].dtype != BBO_Q6_K) return -1;
    starts.push_back(total);
    row_bytes.push_back((jobs[j].n_in / be) * bb);
    total += jobs[j].n_out;
  }
  for_rows(total, total >= size_t(PAR_MIN_ROWS), [&](size_t gr) {
    size_t j = size_t(std::upper_bound(starts.begin(), starts.end(), gr) - starts.begin()) - 1;
    size_t local = gr - starts[j];
    const bbo_job& job = jobs[j];
    const uint8_t* rb = job.w + local * row_bytes[j];
    size_t nb = job.n_in / QK;
    Q8View v{job.qx.q, job.qx.scales, job.qx.sums};
    if (job.has_qx && job.dtype == BBO_Q4_K) out[gr] = dot_q4k_row_q8(rb, nb, v);
    else if (job.has_qx && job.dtype == BBO_Q6_K) out[gr] = dot_q6k_row_q8(rb, nb, v);
    else out[gr] = fused_row_dot(job.dtype, rb, job.x, job.n_in);
  });
  return 0;
}

// --- activations / elementwise (activation.rs:5-29, elementwise.rs:4-17) ---
// f32::exp is libm expf on linux-gnu; that is the function called here.
inline float sigmoid(float x) { return 1.0f / (1.0f + std::exp(-x)); }
inline float silu(float x) { return x / (1.0f + std::exp(-x)); }

// Rust f32::total_cmp: order by the sign-magnitude-flipped bit pattern (-0 < +0).
inline int32_t total_key(float f) {
  int32_t b = int32_t(bits_of(f));
  b ^= int32_t(uint32_t(b >> 31) >> 1);
  return b;
}

// model.rs:485-495 / :303-314 for one token. Sort is descending by total_cmp of
// (score+bias); equal keys keep ascending expert index (sort_unstable_by leaves that
// unspecified, so ties are counted for the caller to assert on).
void gate_one(const float* logits, const float* bias, int E, int k, int32_t* sel, float* w,
              int32_t* ties, float* margin) {
  std::vector<float> s(E), key(E);
  std::vector<int> order(E);
  for (int e = 0; e < E; ++e) {
    s[e] = sigmoid(logits[e]);
    key[e] = s[e] + bias[e];
    order[e] = e;
  }
  std::stable_sort(order.begin(), order.end(),
                   [&](int a, int b) { return total_key(key[b]) < total_key(key[a]); });
  float denom = -0.0f;
  for (int i = 0; i < k; ++i) denom += s[order[i]];
  denom = denom + 1e-6f;
  for (int i = 0; i < k; ++i) {
    sel[i] = order[i];
    w[i] = s[order[i]] / denom;
  }
  if (ties) {
    for (int i = 0; i < k && i + 1 < E; ++i)
      if (total_key(key[order[i]]) == total_key(key[order[i + 1]])) ++*ties;
  }
  if (margin) *margin = (k < E) ? key[order[k - 1]] - key[order[k]] : INFINITY;
}

size_t expert_bytes(uint32_t dt, size_t n_in, size_t n_out) {  // model.rs:612-615
  int be = 1, bb = 0;
  dtype_block(dt, be, bb);
  return n_out * (n_in / be) * bb;
}

void swiglu(const float* g, const float* u, float* o, size_t n) {
  for (size_t i = 0; i < n; ++i) o[i] = silu(g[i]) * u[i];
}
void add_scaled(float* o, const float* b, float s, size_t n) {
  for (size_t i = 0; i < n; ++i) o[i] += s * b[i];
}

// model.rs:473-555 (one token).
int moe_ffn(const bbo_moe* m, const float* x, float* out, bbo_trace* tr) {
  const int H = m->hidden, F = m->moe_ff, E = m->n_experts, K = m->n_used;
  size_t gate_stride = expert_bytes(m->gate_dtype, H, F);
  size_t up_stride = expert_bytes(m->up_dtype, H, F);
  size_t down_stride = expert_bytes(m->down_dtype, F, H);

  std::vector<float> scores(E);
  if (matvec(m->router_dtype, m->router, H, E, x, scores.data())) return -1;
  if (tr && tr->logits) std::memcpy(tr->logits, scores.data(), E * 4);
  std::vector<int32_t> sel(K);
  std::vector<float> w(K);
  gate_one(scores.data(), m->exp_probs_b, E, K, sel.data(), w.data(), tr ? tr->ties : nullptr,
           tr ? tr->margin : nullptr);

  Q8 x_q8 = quantize_q8(x, H);
  bool gate_q8 = m->gate_dtype == BBO_Q4_K || m->gate_dtype == BBO_Q6_K;
  bool up_q8 = m->up_dtype == BBO_Q4_K || m->up_dtype == BBO_Q6_K;
  std::vector<bbo_job> jobs;
  bbo_q8 xq{x_q8.q.data(), x_q8.scales.data(), x_q8.sums.data()};
  for (int i = 0; i < K; ++i)
    jobs.push_back({m->gate_dtype, m->gate_exps + sel[i] * gate_stride, size_t(H), size_t(F), x, gate_q8, xq});
  for (int i = 0; i < K; ++i)
    jobs.push_back({m->up_dtype, m->up_exps + sel[i] * up_stride, size_t(H), size_t(F), x, up_q8, xq});
  std::vector<float> gate_up(2 * K * F);
  if (matvec_fused_batch(jobs.data(), jobs.size(), gate_up.data())) return -1;
  std::vector<float> act(K * F);
  for (int i = 0; i < K; ++i) swiglu(gate_up.data() + i * F, gate_up.data() + (K + i) * F, act.data() + i * F, F);

  bool down_q8 = m->down_dtype == BBO_Q4_K || m->down_dtype == BBO_Q6_K;
  std::vector<Q8> dq(K);
  std::vector<bbo_job> djobs;
  for (int i = 0; i < K; ++i) {
    bbo_q8 v{nullptr, nullptr, nullptr};
    if (down_q8) {
      dq[i] = quantize_q8(act.data() + i * F, F);
      v = {dq[i].q.data(), dq[i].scales.data(), dq[i].sums.data()};
    }
    djobs.push_back({m->down_dtype, m->down_exps + sel[i] * down_stride, size_t(F), size_t(H),
                     act.data() + i * F, down_q8, v});
  }
  std::vector<float> down_all(K * H);
  if (matvec_fused_batch(djobs.data(), djobs.size(), down_all.data())) return -1;
  for (int i = 0; i < H; ++i) out[i] = 0.0f;
  for (int i = 0; i < K; ++i) add_scaled(out, down_all.data() + i * H, w[i], H);

  if (tr) {
    if (tr->sel) std::memcpy(tr->sel, sel.data(), K * 4);
    if (tr->w) std::memcpy(tr->w, w.data(), K * 4);
    if (tr->counts || tr->offsets || tr->perm) {
      std::vector<int32_t> counts(E, 0);
      for (int i = 0; i < K; ++i) counts[sel[i]]++;
      if (tr->counts) std::memcpy(tr->counts, counts.data(), E * 4);
      std::vector<int32_t> off(E + 1, 0);
      for (int e = 0; e < E; ++e) off[e + 1] = off[e] + counts[e];
      if (tr->offsets) std::memcpy(tr->offsets, off.data(), (E + 1) * 4);
      if (tr->perm) {
        std::vector<int32_t> fill(off.begin(), off.end() - 1);
        for (int i = 0; i < K; ++i) tr->perm[fill[sel[i]]++] = i;
      }
    }
  }
  return 0;
}

// model.rs:286-371 (T tokens, token-grouped).
int moe_ffn_batch(const bbo_moe* m, const float* x, size_t t, float* out, bbo_trace* tr) {
  const int H = m->hidden, F = m->moe_ff, E = m->n_experts, K = m->n_used;
  size_t gate_stride = expert_bytes(m->gate_dtype, H, F);
  size_t up_stride = expert_bytes(m->up_dtype, H, F);
  size_t down_stride = expert_bytes(m->down_dtype, F, H);

  std::vector<float> scores(t * E);
  if (matmul(m->router_dtype, m->router, H, E, x, t, scores.data())) return -1;
  if (tr && tr->logits) std::memcpy(tr->logits, scores.data(), t * E * 4);
  std::vector<int32_t> sel(t * K);
  std::vector<float> wts(t * K);
  for (size_t i = 0; i < t; ++i)
    gate_one(scores.data() + i * E, m->exp_probs_b, E, K, sel.data() + i * K, wts.data() + i * K,
             tr ? tr->ties : nullptr, (tr && tr->margin) ? tr->margin + i : nullptr);

  // model.rs:317-322: groups[e] in token-ascending, slot-ascending order.
  std::vector<std::vector<int32_t>> groups(E);
  for (size_t i = 0; i < t; ++i)
    for (int k = 0; k < K; ++k) groups[sel[i * K + k]].push_back(int32_t(i * K + k));

  std::vector<float> slots(t * K * H, 0.0f);
  for (int e = 0; e < E; ++e) {
    const auto& mem = groups[e];
    if (mem.empty()) continue;
    size_t g = mem.size();
    std::vector<float> xe(g * H);
    for (size_t j = 0; j < g; ++j) std::memcpy(xe.data() + j * H, x + (mem[j] / K) * H, H * 4);
    std::vector<float> gate(g * F), up(g * F), act(g * F), down(g * H);
    if (matmul(m->gate_dtype, m->gate_exps + e * gate_stride, H, F, xe.data(), g, gate.data())) return -1;
    if (matmul(m->up_dtype, m->up_exps + e * up_stride, H, F, xe.data(), g, up.data())) return -1;
    for (size_t j = 0; j < g; ++j) swiglu(gate.data() + j * F, up.data() + j * F, act.data() + j * F, F);
    if (matmul(m->down_dtype, m->down_exps + e * down_stride, F, H, act.data(), g, down.data())) return -1;
    for (size_t j = 0; j < g; ++j) std::memcpy(slots.data() + size_t(mem[j]) * H, down.data() + j * H, H * 4);
  }
  for (size_t i = 0; i < t; ++i) {
    float* oi = out + i * H;
    for (int c = 0; c < H; ++c) oi[c] = 0.0f;
    for (int k = 0; k < K; ++k) add_scaled(oi, slots.data() + (i * K + k) * H, wts[i * K + k], H);
  }

  if (tr) {
    if (tr->sel) std::memcpy(tr->sel, sel.data(), t * K * 4);
    if (tr->w) std::memcpy(tr->w, wts.data(), t * K * 4);
    size_t pos = 0;
    if (tr->offsets) tr->offsets[0] = 0;
    for (int e = 0; e < E; ++e) {
      if (tr->counts) tr->counts[e] = int32_t(groups[e].size());
      for (int32_t v : groups[e]) {
        if (tr->perm) tr->perm[pos] = v;
        ++pos;
      }
      if (tr->offsets) tr->offsets[e + 1] = int32_t(pos);
    }
  }
  return 0;
}

// model.rs:459-469 (decode) and :262-278 (batched).
int dense_ffn(const bbo_dense* d, const float* x, size_t t, float* out) {
  const int H = d->hidden, F = d->ff;
  std::vector<float> gate(t * F), up(t * F), act(t * F);
  if (matmul(d->gate_dtype, d->gate, H, F, x, t, gate.data())) return -1;
  if (matmul(d->up_dtype, d->up, H, F, x, t, up.data())) return -1;
  for (size_t i = 0; i < t; ++i) swiglu(gate.data() + i * F, up.data() + i * F, act.data() + i * F, F);
  return matmul(d->down_dtype, d->down, F, H, act.data(), t, out);
}

// rmsnorm.rs:10-21: f32 squares summed in f64 (Sum from -0.0), mean narrowed to f32.
void rmsnorm(const float* x, const float* g, float eps, size_t n, float* out) {
  double ss = -0.0;
  for (size_t i = 0; i < n; ++i) ss += double(x[i] * x[i]);
  float mean = float(ss / double(n));
  float scale = 1.0f / std::sqrt(mean + eps);
  for (size_t i = 0; i < n; ++i) out[i] = x[i] * scale * g[i];
}

// ---- operators of the decoder layer (full decode layer and batched prefill) ----

// conv.rs:18-39: causal depthwise conv, one token. The filter's last tap multiplies the current
// column, earlier taps the cached columns (oldest first); sum = w[L-1]·bx, then += w[k]·state[k].
void conv_step(const float* state, const float* bx, const float* w, size_t C, size_t L, float* out) {
  for (size_t c = 0; c < C; ++c) {
    const float* wc = w + c * L;
    float sum = wc[L - 1] * bx[c];
    for (size_t k = 0; k + 1 < L; ++k) sum += wc[k] * state[k * C + c];
    out[c] = sum;
  }
}

// conv.rs:48-68: conv_step per position, then the state slides one column and takes bx_t.
// (The reference's slice ranges require L >= 2 here.)
void conv_prefill(float* state, const float* bx, const float* w, size_t C, size_t L, size_t n, float* out) {
  for (size_t t = 0; t < n; ++t) {
    const float* bxt = bx + t * C;
    conv_step(state, bxt, w, C, L, out + t * C);
    std::memmove(state, state + C, (L - 2) * C * sizeof(float));
    std::memcpy(state + (L - 2) * C, bxt, C * sizeof(float));
  }
}

// softmax.rs:9-22: max by `if a >= b { a } else { b }` from the first element, exps of
// (v - max) with f32 exp (libm expf), their sum in f64 left to right from 0.0, then each
// value times (float)(1.0 / sum).
void softmax(float* x, size_t n) {
  if (n == 0) return;
  float mx = x[0];
  for (size_t i = 1; i < n; ++i) mx = mx >= x[i] ? mx : x[i];
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) {
    x[i] = std::exp(x[i] - mx);
    sum += double(x[i]);
  }
  const float inv = float(1.0 / sum);
  for (size_t i = 0; i < n; ++i) x[i] *= inv;
}

// attention.rs:17-55: one query per head against n_ctx cached positions; kv head = h / group;
// score = dot(q, k) * (1 / sqrt(head_dim)) with matmul.rs's dot; softmax; out = Σ_j w_j·v_j
// accumulated in position order from 0.0 (a rounded multiply, then an add).
void attention_decode(const float* q, const float* k, const float* v, size_t n_ctx, size_t n_heads, size_t n_kv,
                      size_t hd, float* out) {
  const float scale = 1.0f / std::sqrt(float(hd));
  const size_t group = n_heads / n_kv;
  std::vector<float> sc(n_ctx);
  for (size_t h = 0; h < n_heads; ++h) {
    const size_t kv = h / group;
    const float* qh = q + h * hd;
    for (size_t j = 0; j < n_ctx; ++j) sc[j] = dot_f32(qh, k + (j * n_kv + kv) * hd, hd) * scale;
    softmax(sc.data(), n_ctx);
    float* o = out + h * hd;
    for (size_t d = 0; d < hd; ++d) o[d] = 0.0f;
    for (size_t j = 0; j < n_ctx; ++j) {
      const float* vj = v + (j * n_kv + kv) * hd;
      for (size_t d = 0; d < hd; ++d) o[d] += sc[j] * vj[d];
    }
  }
}

// rope.rs:17-30: NEOX split-half rotation; theta_scale = powf(freq_base, -2/d), the angle
// starts at (float)pos and is multiplied by theta_scale per pair (f32), sin/cos are libm's.
void rope_neox(float* x, size_t d, size_t pos, float freq_base) {
  const size_t half = d / 2;
  const float theta_scale = std::pow(freq_base, -2.0f / float(d));
  float theta = float(pos);
  for (size_t i = 0; i < half; ++i) {
    const float sn = std::sin(theta), cs = std::cos(theta);
    const float a = x[i], b = x[i + half];
    x[i] = a * cs - b * sn;
    x[i + half] = a * sn + b * cs;
    theta *= theta_scale;
  }
}

// model.rs:692-701: per head rmsnorm over head_dim (into a temporary, copied back), then RoPE.
void norm_rope_heads(float* buf, size_t n_heads, size_t hd, const float* gain, float eps, size_t pos,
                     float freq_base) {
  std::vector<float> tmp(hd);
  for (size_t h = 0; h < n_heads; ++h) {
    float* head = buf + h * hd;
    rmsnorm(head, gain, eps, hd, tmp.data());
    std::memcpy(head, tmp.data(), hd * sizeof(float));
    rope_neox(head, hd, pos, freq_base);
  }
}

// y = W·x for t token-major rows as the reference's operators call it: matvec1 for one token
// (model.rs:557-560), matmul1 for a batch (model.rs:372-375).
int project(uint32_t dt, const uint8_t* w, size_t n_in, size_t n_out, const float* x, size_t t, float* y) {
  return t == 1 ? matvec(dt, w, n_in, n_out, x, y) : matmul(dt, w, n_in, n_out, x, t, y);
}

// model.rs:399-427 (one token, conv_step + the state shift) and :190-216 (a batch,
// conv_prefill): in_proj -> (B, C, x_gate) chunks; Bx = B·x_gate; conv; y = C·conv; out_proj.
int conv_op(const bbo_conv_op* op, float* state, const float* x, size_t t, float* out) {
  const size_t H = size_t(op->hidden), L = size_t(op->l_cache);
  std::vector<float> bcx(t * 3 * H), bx(t * H), conv(t * H), y(t * H);
  if (project(op->in_dtype, op->in_proj, H, 3 * H, x, t, bcx.data())) return -1;
  for (size_t i = 0; i < t; ++i)
    for (size_t c = 0; c < H; ++c) bx[i * H + c] = bcx[i * 3 * H + c] * bcx[i * 3 * H + 2 * H + c];
  if (t == 1) {
    conv_step(state, bx.data(), op->conv_w, H, L, conv.data());
    std::memmove(state, state + H, (L - 2) * H * sizeof(float));
    std::memcpy(state + (L - 2) * H, bx.data(), H * sizeof(float));
  } else {
    conv_prefill(state, bx.data(), op->conv_w, H, L, t, conv.data());
  }
  for (size_t i = 0; i < t; ++i)
    for (size_t c = 0; c < H; ++c) y[i * H + c] = bcx[i * 3 * H + H + c] * conv[i * H + c];
  return project(op->out_dtype, op->out_proj, H, H, y.data(), t, out);
}

// model.rs:430-456 (one token) and :222-259 (a batch): q/k/v projections, per-head q/k norm
// and RoPE at each token's position, k/v appended to the cache, each token attending over the
// cache as it stands after its own append, o projection. The caches hold `cap` positions of
// n_kv·head_dim floats; *n_cached grows by t.
int attn_op(const bbo_attn_op* op, float* k_cache, float* v_cache, size_t cap, size_t* n_cached, size_t pos0,
            const float* x, size_t t, float* out) {
  const size_t H = size_t(op->hidden), NH = size_t(op->n_heads), NKV = size_t(op->n_kv_heads),
               HD = size_t(op->head_dim), KV = NKV * HD;
  if (*n_cached + t > cap) return -2;
  std::vector<float> q(t * NH * HD), k(t * KV), v(t * KV), attn(t * NH * HD);
  if (project(op->q_dtype, op->q, H, NH * HD, x, t, q.data())) return -1;
  if (project(op->k_dtype, op->k, H, KV, x, t, k.data())) return -1;
  if (project(op->v_dtype, op->v, H, KV, x, t, v.data())) return -1;
  for (size_t i = 0; i < t; ++i) {
    norm_rope_heads(q.data() + i * NH * HD, NH, HD, op->q_norm, op->eps, pos0 + i, op->freq_base);
    norm_rope_heads(k.data() + i * KV, NKV, HD, op->k_norm, op->eps, pos0 + i, op->freq_base);
  }
  for (size_t i = 0; i < t; ++i) {
    std::memcpy(k_cache + *n_cached * KV, k.data() + i * KV, KV * sizeof(float));
    std::memcpy(v_cache + *n_cached * KV, v.data() + i * KV, KV * sizeof(float));
    *n_cached += 1;
    attention_decode(q.data() + i * NH * HD, k_cache, v_cache, *n_cached, NH, NKV, HD, attn.data() + i * NH * HD);
  }
  return project(op->o_dtype, op->o, NH * HD, H, attn.data(), t, out);
}

}  // namespace

extern "C" {

void bbo_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n > 0 ? n : 1);
#else
  (void)n;
#endif
}
int bbo_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

float bbo_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
void bbo_get_scale_min_k4(int j, const uint8_t* scales, uint8_t* sc, uint8_t* m) { scale_min_k4(j, scales, *sc, *m); }
int bbo_dequantize(uint32_t dt, const uint8_t* data, size_t n, float* out) { return dequantize_into(dt, data, n, out) ? 0 : -1; }
void bbo_quantize_q8(const float* x, size_t n, bbo_q8 o) { quantize_q8_into(x, n, o.q, o.scales, o.sums); }
float bbo_dot(const float* a, const float* b, size_t n) { return dot_f32(a, b, n); }
float bbo_dot_q4k_block_q8(const uint8_t* b, const int8_t* qx, float sx, const int32_t* sums) { return dot_q4k_block_q8(b, qx, sx, sums); }
float bbo_dot_q6k_block_q8(const uint8_t* b, const int8_t* qx, float sx) { return dot_q6k_block_q8(b, qx, sx); }
int32_t bbo_q4k_block_sd(const uint8_t* block, const int8_t* qx) {
  int32_t sc[8];
  for (int j = 0; j < 8; ++j) { uint8_t s, m; scale_min_k4(j, block + 4, s, m); sc[j] = s; }
  return q4k_sd(block + 16, sc, qx);
}
int32_t bbo_q6k_block_idot(const uint8_t* block, const int8_t* qx) { return q6k_idot_fused(block, qx); }
int32_t bbo_q6k_block_idot_buffered(const uint8_t* block, const int8_t* qx) {
  int8_t wq[256];
  int32_t sc[16];
  unpack_q6k(block, wq, sc);
  return wsd_q6k(wq, qx, sc);
}
float bbo_fused_row_dot(uint32_t dt, const uint8_t* row, const float* x, size_t n_in) { return fused_row_dot(dt, row, x, n_in); }
int bbo_matvec(uint32_t dt, const uint8_t* w, size_t n_in, size_t n_out, const float* x, float* y) { return matvec(dt, w, n_in, n_out, x, y); }
int bbo_matmul(uint32_t dt, const uint8_t* w, size_t n_in, size_t n_out, const float* x, size_t nt, float* y) { return matmul(dt, w, n_in, n_out, x, nt, y); }
int bbo_matvec_fused_batch(const bbo_job* jobs, size_t n, float* out) { return matvec_fused_batch(jobs, n, out); }
float bbo_sigmoid(float x) { return sigmoid(x); }
float bbo_silu(float x) { return silu(x); }
void bbo_swiglu(const float* g, const float* u, float* o, size_t n) { swiglu(g, u, o, n); }
void bbo_add_scaled(float* o, const float* b, float s, size_t n) { add_scaled(o, b, s, n); }
void bbo_add_assign(float* a, const float* b, size_t n) { for (size_t i = 0; i < n; ++i) a[i] += b[i]; }
void bbo_rmsnorm(const float* x, const float* g, float eps, size_t n, float* out) { rmsnorm(x, g, eps, n, out); }
float bbo_dot_variant(const float* a, const float* b, size_t n, int variant) { return dot_variant(a, b, n, variant); }
// logits[t][e] = dot_variant(W row e, x row t) for T tokens (W: E rows of H f32, as the router).
void bbo_router_logits_variant(const float* W, const float* x, size_t T, int H, int E, int variant, float* logits) {
  for_rows(T * size_t(E), true, [&](size_t i) {
    const size_t t = i / E, e = i % E;
    logits[i] = dot_variant(W + e * size_t(H), x + t * size_t(H), size_t(H), variant);
  });
}
// model.rs:485-495 for T tokens from given logits: sel/w [T*k], ties [1] (accumulated), margin [T].
void bbo_gate(const float* logits, const float* bias, size_t T, int E, int k, int32_t* sel, float* w, int32_t* ties,
              float* margin) {
  for (size_t t = 0; t < T; ++t)
    gate_one(logits + t * E, bias, E, k, sel + t * k, w + t * k, ties, margin ? margin + t : nullptr);
}
int bbo_moe_ffn(const bbo_moe* m, const float* x, float* out, bbo_trace* tr) { return moe_ffn(m, x, out, tr); }
int bbo_moe_ffn_batch(const bbo_moe* m, const float* x, size_t t, float* out, bbo_trace* tr) { return moe_ffn_batch(m, x, t, out, tr); }
int bbo_dense_ffn(const bbo_dense* d, const float* x, size_t t, float* out) { return dense_ffn(d, x, t, out); }

// model.rs:105-130 with the operator sub-layer contributing nothing: h += FFN(rmsnorm(h)).
int bbo_ffn_stack(const bbo_layer* layers, size_t n_layers, const float* x, size_t t, float eps, float* h) {
  if (n_layers == 0) return -1;
  const int H = layers[0].is_moe ? layers[0].moe.hidden : layers[0].dense.hidden;
  std::memcpy(h, x, t * H * 4);
  std::vector<float> normed(t * H), ffn(t * H);
  for (size_t l = 0; l < n_layers; ++l) {
    for (size_t i = 0; i < t; ++i) rmsnorm(h + i * H, layers[l].ffn_norm, eps, H, normed.data() + i * H);
    int rc;
    if (layers[l].is_moe)
      rc = t == 1 ? moe_ffn(&layers[l].moe, normed.data(), ffn.data(), nullptr)
                  : moe_ffn_batch(&layers[l].moe, normed.data(), t, ffn.data(), nullptr);
    else
      rc = dense_ffn(&layers[l].dense, normed.data(), t, ffn.data());
    if (rc) return rc;
    for (size_t i = 0; i < t * H; ++i) h[i] += ffn[i];
  }
  return 0;
}

void bbo_conv_step(const float* state, const float* bx, const float* w, size_t C, size_t L, float* out) {
  conv_step(state, bx, w, C, L, out);
}
void bbo_conv_prefill(float* state, const float* bx, const float* w, size_t C, size_t L, size_t n, float* out) {
  conv_prefill(state, bx, w, C, L, n, out);
}
void bbo_softmax(float* x, size_t n) { softmax(x, n); }
void bbo_attention_decode(const float* q, const float* k, const float* v, size_t n_ctx, size_t n_heads, size_t n_kv,
                          size_t hd, float* out) {
  attention_decode(q, k, v, n_ctx, n_heads, n_kv, hd, out);
}
void bbo_rope_neox(float* x, size_t d, size_t pos, float freq_base) { rope_neox(x, d, pos, freq_base); }
void bbo_norm_rope_heads(float* buf, size_t n_heads, size_t hd, const float* gain, float eps, size_t pos,
                         float freq_base) {
  norm_rope_heads(buf, n_heads, hd, gain, eps, pos, freq_base);
}
int bbo_conv_forward(const bbo_conv_op* op, float* state, const float* x, size_t t, float* out) {
  return conv_op(op, state, x, t, out);
}
int bbo_attn_forward(const bbo_attn_op* op, float* k_cache, float* v_cache, size_t cap, size_t* n_cached, size_t pos0,
                const float* x, size_t t, float* out) {
  return attn_op(op, k_cache, v_cache, cap, n_cached, pos0, x, t, out);
}

}  // extern "C"
