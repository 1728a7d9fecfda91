// bb_gating.h — the router gating (model.rs:485-495) on one half-wave per token, shared by the
// kernels that gate: the route kernels and the gate/up GEMV.
#ifndef BB_GATING_H
#define BB_GATING_H
#include "bb_device.h"
#include "bb_internal.h"

namespace bb {

// ---- gating ----------------------------------------------------------------------------------------
// max over each 32-lane half of the wave (all 64 lanes active); lanes < 32 get the low half's
__device__ __forceinline__ int half_max(int v) {
  auto dpp = [](int x, auto ctrl) {
    return __builtin_amdgcn_update_dpp(0, x, decltype(ctrl)::value, 0xf, 0xf, false);
  };
  v = max(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad [1,0,3,2]
  v = max(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad [2,3,0,1]
  v = max(v, dpp(v, std::integral_constant<int, 0x141>{}));  // half-row mirror
  v = max(v, dpp(v, std::integral_constant<int, 0x140>{}));  // row mirror
  const int lo = max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16));
  const int hi = max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48));
  return (threadIdx.x & 32) ? hi : lo;
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Gating of one token per half-wave (model.rs:485-495): lane e of the half-wave holds expert e's
// logit. sigmoid, key = score + bias, the top k by total_cmp in k rounds of a half-wave maximum
// (the lowest expert index first among equal keys), weights = score / (scores summed in rank
// order from -0.0, + 1e-6). Also the margin between the k-th and (k+1)-th keys and the number
// of selected experts whose key another expert after them shares. Every lane of the wave
// calls it; live is false for lanes of absent tokens or experts. The results go to rb when
// global_out is set, and the selections also to lds_sel[t*K + rank] when it is not null.
__device__ __forceinline__ void gate_halfwave(float logit, bool live, bool tok, float bias_e, int t, int E, int K,
                                              const uint64_t* exptab, RouteBufs rb, bool global_out = true,
                                              int32_t* lds_sel = nullptr) {
  const int lane = threadIdx.x & 63, e = lane & 31;
  const float s = live ? sigmoid_tab(logit, exptab) : 0.0f;
  const float key = live ? s + bias_e : 0.0f;
  const int32_t kk = total_key(key);
  bool avail = live;
  int rank = 64, ties = 0;
  float denom = -0.0f, key_k1 = 0.0f, key_k = 0.0f;
  const bool hi = (lane & 32) != 0;
  const int nr = min(K + 1, E);
  for (int rd = 0; rd < nr; ++rd) {
    const int m = half_max(avail ? kk : -2147483647 - 1);
    const uint64_t eq = __ballot(avail && kk == m);
    const uint32_t e0 = (uint32_t)eq, e1 = (uint32_t)(eq >> 32);
    const int f0 = e0 ? __builtin_ctz(e0) : 0, f1 = e1 ? __builtin_ctz(e1) : 0;
    const float s0 = readlane_f(s, f0), s1 = readlane_f(s, 32 + f1);
    const float k0 = readlane_f(key, f0), k1 = readlane_f(key, 32 + f1);
    const uint32_t eh = hi ? e1 : e0;
    if (eh != 0 && e == (hi ? f1 : f0)) {
      rank = rd;
      avail = false;
    }
    if (rd < K) {
      if (eh != 0) denom += hi ? s1 : s0;
      ties += __popc(eh) > 1 ? 1 : 0;
    }
    if (rd == K - 1) key_k1 = hi ? k1 : k0;
    if (rd == K) key_k = hi ? k1 : k0;
  }
  denom = denom + 1e-6f;
  if (live && rank < K) {
    if (lds_sel) lds_sel[t * K + rank] = e;
    if (global_out) {
      rb.sel[(size_t)t * K + rank] = e;
      rb.wts[(size_t)t * K + rank] = s / denom;
    }
  }
  if (global_out && tok && e == 0) {
    rb.margin[t] = K < E ? key_k1 - key_k : __builtin_inff();
    rb.ties[t] = ties;
  }
}

// The gating alone (gate_halfwave per token, T <= 2 * blockDim.x / 64), from logits computed
// before the launch (k_residual_norm_route): selections into sel_lds, and the
// route's outputs to rb when global_out (the logits too, when they come from elsewhere).
__device__ inline void gate_block(const float* __restrict__ logits, const float* __restrict__ bias, int T, int E, int K,
                           bool global_out, RouteBufs rb, int32_t* sel_lds, uint64_t* exptab, uint64_t exp_e) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = tid >> 5, e = lane & 31;  // half-wave i gates token i
  const bool tok = i < T, live = tok && e < E;
  const float lg = logits[min(i, T - 1) * E + min(e, E - 1)];
  const float be = bias[min(e, E - 1)];
  if (tid < 32) exptab[tid] = exp_e;
  lds_barrier();
  if (2 * wave < T) gate_halfwave(live ? lg : 0.0f, live, tok, be, i, E, K, exptab, rb, global_out, sel_lds);
  if (global_out && live && logits != rb.logits) rb.logits[(size_t)i * E + e] = lg;
  lds_barrier();
}

}  // namespace bb
#endif
