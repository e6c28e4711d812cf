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

// Routes token t from its logits v[j] = logit of expert l + 64 j (bias already
// added; -inf where the expert is past E, `valid` bit j set otherwise).  Lane
// j < k writes choice j to ids / wout at t * kout + j; with e_shared >= 0, lane
// k appends the always-on shared expert (id e_shared, weight 1) as choice k
// (kout = k + 1).
template <int VPL>
__device__ __forceinline__ void route_token_values(const float (&v)[VPL], uint32_t valid, int t, int k,
                                                   int32_t* __restrict__ ids, float* __restrict__ wout,
                                                   int kout, int e_shared) {
  const int l = lane_id();
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
    if (valid & (1u << j)) m = fmaxf(m, v[j]);
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
    if (valid & (1u << j)) s += expf(v[j] - m);
  s = wave_sum(s);

  uint32_t taken = 0;
  float my_p = 0.0f;
  int my_id = 0;
  float denom = 0.0f;
  constexpr int kNone = 0x7fffffff;
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int be = kNone;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const uint32_t bit = 1u << j;
      if ((valid & bit) && !(taken & bit) && (be == kNone || v[j] > bv)) {
        bv = v[j];
        be = l + 64 * j;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oe = __shfl_xor(be, o);
      const bool take = oe != kNone && (be == kNone || ov > bv || (ov == bv && oe < be));
      if (take) {
        bv = ov;
        be = oe;
      }
    }
    if ((be & 63) == l) taken |= 1u << (be >> 6);
    const float pr = expf(bv - m) / s;
    denom = denom + pr;  // selection order, identical in every lane
    if (l == r) {
      my_p = pr;
      my_id = be;
    }
  }
  if (l < k) {
    ids[(int64_t)t * kout + l] = my_id;
    wout[(int64_t)t * kout + l] = my_p / denom;
  } else if (l == k && e_shared >= 0) {
    ids[(int64_t)t * kout + k] = e_shared;
    wout[(int64_t)t * kout + k] = 1.0f;
  }
}

// Routes token t; logit(e) returns its logit for expert e (lane l asks for
// experts l, l + 64, ...); kout as route_token_values (0: k).
template <int VPL, typename Logit>
__device__ __forceinline__ void route_token_with(Logit&& logit, const float* __restrict__ bias, int t, int E,
                                                 int k, int32_t* __restrict__ ids, float* __restrict__ wout,
                                                 int kout = 0, int e_shared = -1) {
  const int l = lane_id();
  float v[VPL];
  uint32_t valid = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = l + 64 * j;
    v[j] = -INFINITY;
    if (e < E) {
      float x = logit(e);
      if (bias) x = x + bias[e];
      v[j] = x;
      valid |= 1u << j;
    }
  }
  route_token_values<VPL>(v, valid, t, k, ids, wout, kout == 0 ? k : kout, e_shared);
}

}  // namespace moe
