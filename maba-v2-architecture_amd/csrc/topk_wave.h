// Wave-level (64-lane) top-K selection on 64-bit ordering keys.
//
// A key packs an fp32 score and an index so that "greater key" means "better":
// the high word is the order-preserving bit pattern of the score, the low word
// is ~index, so equal scores rank the lower index first.  This gives the
// deterministic order "score descending, then index ascending".
//
// A wave keeps its running top-64 as a descending sorted list, one key per lane.
// A batch of 64 new candidates (one per lane) is merged by a bitonic sort of
// the batch followed by a bitonic merge with the list; a batch that cannot
// beat the current K-th key is rejected with one ballot.
#pragma once
#include "maba_common.h"

namespace maba {

typedef unsigned long long key64;

__device__ __forceinline__ uint32_t order_f32(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float unorder_f32(uint32_t o) {
  const uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(u);
}

__device__ __forceinline__ key64 make_key(float score, uint32_t idx) {
  return ((key64)order_f32(score) << 32) | (key64)(~idx);
}

__device__ __forceinline__ uint32_t key_index(key64 k) { return ~(uint32_t)(k & 0xffffffffull); }
__device__ __forceinline__ float key_score(key64 k) { return unorder_f32((uint32_t)(k >> 32)); }

// Key that loses against every real key (real keys have a non-zero high word).
constexpr key64 KEY_NONE = 0ull;

__device__ __forceinline__ key64 kmax(key64 a, key64 b) { return a > b ? a : b; }
__device__ __forceinline__ key64 kmin(key64 a, key64 b) { return a < b ? a : b; }

// Sort the 64 keys of a wave in descending lane order.
__device__ __forceinline__ key64 wave_sort_desc(key64 key) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const key64 other = __shfl_xor(key, j);
      const bool desc = (lane & k) == 0;
      const bool lower = (lane & j) == 0;
      key = (lower == desc) ? kmax(key, other) : kmin(key, other);
    }
  }
  return key;
}

// list: descending top-64 so far; cand: one new key per lane (any order).
// Returns the descending top-64 of both.
__device__ __forceinline__ key64 wave_merge_topk(key64 list, key64 cand, int K) {
  const int lane = threadIdx.x & 63;
  const key64 kth = __shfl(list, K - 1);
  if (__ballot(cand > kth) == 0ull) return list;
  cand = wave_sort_desc(cand);
  const key64 rev = __shfl(cand, 63 - lane);
  key64 m = kmax(list, rev);  // bitonic, holds the top 64 of the union
#pragma unroll
  for (int j = 32; j > 0; j >>= 1) {
    const key64 other = __shfl_xor(m, j);
    m = ((lane & j) == 0) ? kmax(m, other) : kmin(m, other);
  }
  return m;
}

}  // namespace maba
