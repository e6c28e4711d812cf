// Per-token router step shared by the routing kernels: softmax over E
// logits (+ bias), top-k with ties to the lower expert index, weights
// renormalised over the k, one wave per token.
#pragma once

#include "moe_common.h"

#include <math.h>

namespace moe {

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Order-preserving uint32 key of a float: larger float -> larger key; -0.0
// keys as +0.0 (they compare equal) and NaN as 1, below every number.  Key 0
// marks an expert past E.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7fffffffu) == 0) b = 0;
  if ((b & 0x7fffffffu) > 0x7f800000u) return 1u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key ^ 0x80000000u) : ~key);
}

// Routes token t from its logits v[j] = logit of expert l + 64 j (bias already
// added; -inf where the expert is past E, `valid` bit j set otherwise).  Lane
// j < k writes choice j to ids / wout at t * kout + j; with e_shared >= 0, lane
// k appends the always-on shared expert (id e_shared, weight 1) as choice k
// (kout = k + 1).
//
// Selection works on ballots and lane reads only, no cross-lane shuffles:
//   1. tau = the k-th largest key, bit by bit from the top (a key prefix is
//      kept when at least k keys reach it);
//   2. the chosen set is every key > tau plus the lowest-numbered experts
//      whose key equals tau, k in all;
//   3. lanes 0..k-1 receive the chosen experts in ascending expert order, and
//      each lane's choice index is the number of chosen keys above its own
//      plus the equal keys of lower experts -- descending logit, ties to the
//      lower expert;
//   4. the softmax maximum is the key of choice 0; the probabilities of the k
//      are renormalised over their sum taken in choice order.
template <int VPL>
__device__ __forceinline__ void route_token_values(const float (&v)[VPL], uint32_t valid, int t, int k,
                                                   int32_t* __restrict__ ids, float* __restrict__ wout,
                                                   int kout, int e_shared) {
  const int l = lane_id();
  uint32_t key[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) key[j] = (valid & (1u << j)) ? order_key(v[j]) : 0u;

  uint32_t tau = 0;
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = tau | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j) cnt += __popcll(__ballot(key[j] >= cand));
    if (cnt >= k) tau = cand;
  }

  uint64_t sel[VPL];
  int need = k;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    sel[j] = __ballot(key[j] > tau);
    need -= __popcll(sel[j]);
  }
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    uint64_t eq = __ballot(key[j] == tau);
    while (need > 0 && eq) {
      sel[j] |= eq & (~eq + 1);
      eq &= eq - 1;
      --need;
    }
  }

  uint32_t mykey = 0;
  int mye = 0, pos = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    uint64_t msk = sel[j];
    while (msk) {
      const int src = __ffsll((unsigned long long)msk) - 1;
      msk &= msk - 1;
      const uint32_t kk = (uint32_t)__builtin_amdgcn_readlane((int)key[j], src);
      if (l == pos) {
        mykey = kk;
        mye = src + 64 * j;
      }
      ++pos;
    }
  }
  int rank = 0;
  for (int q = 0; q < k; ++q) {
    const uint32_t kq = (uint32_t)__builtin_amdgcn_readlane((int)mykey, q);
    rank += (kq > mykey || (kq == mykey && q < l)) ? 1 : 0;
  }
  const bool chosen = l < k;

  const int top = __ffsll((unsigned long long)__ballot(chosen && rank == 0)) - 1;
  const float m = key_value((uint32_t)__builtin_amdgcn_readlane((int)mykey, top));
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
    if (valid & (1u << j)) s += expf(v[j] - m);
  s = wave_sum(s);

  const float pr = expf(key_value(mykey) - m) / s;
  float denom = 0.0f;
  for (int r = 0; r < k; ++r) {  // choice order, identical in every lane
    const int src = __ffsll((unsigned long long)__ballot(chosen && rank == r)) - 1;
    denom = denom + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr), src));
  }
  if (chosen) {
    ids[(int64_t)t * kout + rank] = mye;
    wout[(int64_t)t * kout + rank] = pr / denom;
  } else if (l == k && e_shared >= 0) {
    ids[(int64_t)t * kout + k] = e_shared;
    wout[(int64_t)t * kout + k] = 1.0f;
  }
}

// Routes token t from its logits row (lane l takes experts l, l + 64, ...)
// and the optional bias; kout as route_token_values (0: k).  Every value is
// loaded unconditionally, at expert min(e, E - 1) (E >= 1), with the logits
// row standing in for a missing bias, and selected afterwards: a load guarded
// by e < E or by the bias compiles to a branch that waits for every earlier
// load, one memory round trip per value instead of one for all.  The sum is
// logit + bias only when a bias is given, as before (no + 0 that would turn a
// -0 logit into +0).
template <int VPL>
__device__ __forceinline__ void route_token_row(const float* __restrict__ row, const float* __restrict__ bias,
                                                int t, int E, int k, int32_t* __restrict__ ids,
                                                float* __restrict__ wout, int kout = 0, int e_shared = -1) {
  const int l = lane_id();
  const float* bsrc = bias ? bias : row;
  float lv[VPL], bv[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = l + 64 * j;
    const int ec = e < E ? e : E - 1;
    lv[j] = row[ec];
    bv[j] = bsrc[ec];
  }
  float v[VPL];
  uint32_t valid = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const bool in = l + 64 * j < E;
    v[j] = in ? (bias ? lv[j] + bv[j] : lv[j]) : -INFINITY;
    valid |= in ? 1u << j : 0u;
  }
  route_token_values<VPL>(v, valid, t, k, ids, wout, kout == 0 ? k : kout, e_shared);
}

}  // namespace moe
