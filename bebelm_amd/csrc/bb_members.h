// bb_members.h — the members of an expert from the selections, inside one block.
//
// Every block of a kernel that needs the grouping of (token, slot) entries by expert derives it
// from the T*k selections itself instead of reading a separate dispatch kernel's output: the
// selections are few (at most MAX_ENTRIES) and one block sorts them out in a few LDS passes.
#ifndef BB_MEMBERS_H
#define BB_MEMBERS_H
#include "bb_device.h"
#include "bb_internal.h"

namespace bb {

// Each block reads the T*K selections once into registers (entry i = token*K + slot lives on
// lane i%64 of wave (i/64)%8, slot k = i/512), forms the mask of selected experts, and builds
// member lists on demand: the entries with sel == e in ascending order, the order
// model.rs:316-322 groups them in (one ballot per 64 entries and a prefix over chunk counts).
constexpr int SEL_REGS = MAX_ENTRIES / 512;

struct SelRegs {
  int32_t v[SEL_REGS];
};

struct SmemMembers {
  int32_t list[MAX_ENTRIES];
  int32_t chunk[MAX_ENTRIES / 64 + 1];
  uint32_t mask;
};

// Uniform across the block; needs blockDim.x == 512.
__device__ inline uint32_t read_selection(const int32_t* __restrict__ sel, int n_ent, SelRegs& sr, SmemMembers& sm) {
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t present = 0;
#pragma unroll
  for (int k = 0; k < SEL_REGS; ++k) {
    const int i = k * 512 + tid;
    sr.v[k] = i < n_ent ? sel[i] : -1;
    if (sr.v[k] >= 0) present |= 1u << sr.v[k];
  }
  if (tid == 0) sm.mask = 0;
  __syncthreads();
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) present |= (uint32_t)__shfl_xor((int)present, o);
  if (lane == 0) atomicOr(&sm.mask, present);
  __syncthreads();
  return sm.mask;
}

// Fills sm.list with the members of expert e; returns their count (uniform). Its barriers order
// LDS only, so loads in flight stay in flight.
__device__ inline int member_list(const SelRegs& sr, int n_ent, int e, SmemMembers& sm) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_chunks = (n_ent + 63) >> 6;
  unsigned long long masks[SEL_REGS];
#pragma unroll
  for (int k = 0; k < SEL_REGS; ++k) {
    const int ch = k * 8 + wave;
    masks[k] = __ballot(sr.v[k] == e);
    if (ch < n_chunks && lane == 0) sm.chunk[ch] = __popcll(masks[k]);
  }
  lds_barrier();
  if (tid == 0) {
    int acc = 0;
    for (int ch = 0; ch < n_chunks; ++ch) {
      const int v = sm.chunk[ch];
      sm.chunk[ch] = acc;
      acc += v;
    }
    sm.chunk[n_chunks] = acc;
  }
  lds_barrier();
  const unsigned long long lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int k = 0; k < SEL_REGS; ++k) {
    const int ch = k * 8 + wave;
    if (ch < n_chunks && ((masks[k] >> lane) & 1ull)) sm.list[sm.chunk[ch] + __popcll(masks[k] & lt)] = ch * 64 + lane;
  }
  const int cnt = sm.chunk[n_chunks];
  lds_barrier();
  return cnt;
}

// Id of the u-th set bit of mask (ascending).
__device__ __forceinline__ int nth_expert(uint32_t mask, int u) {
  for (int k = 0; k < u; ++k) mask &= mask - 1;
  return __builtin_ctz(mask);
}

}  // namespace bb
#endif
