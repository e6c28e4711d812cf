// Router GEMM upstream of the top-k: logits = x . w_router^T (fp16 inputs,
// fp32 accumulation) for x [T, H] and w_router [E, H], split over K so that a
// long hidden dimension still gives enough work items, followed by routing
// (softmax -> top-k -> renormalise, as route_topk) of the K-split partial
// sums, summed in split order so the result is deterministic.
//
// There is no router in the reference (problem_detail.json:18, :30: the
// operator receives routed tokens); this is the step before it in a MoE layer.
#include "launch.h"
#include "moe_common.h"
#include "route_token.h"

namespace moe {

// BM tokens x BN experts per item, NW waves in a 2 x (NW/2) grid, K in
// 128-byte steps through an S-stage ring (token rows, then expert rows).  Rows
// past T or E are loaded from the last valid row and never stored.
template <int BM, int BN, int NW, int S>
__global__ __launch_bounds__(64 * NW) void router_gemm_kernel(const _Float16* __restrict__ x,
                                                               const _Float16* __restrict__ wr, int T, int E,
                                                               int64_t H, int ks_count, float* __restrict__ part) {
  constexpr int WN = NW / 2;             // waves along the experts
  constexpr int WTM = BM / 2, WTN = BN / WN;
  constexpr int NBM = WTM / 32, NBN = WTN / 32;
  static_assert(NBM >= 1 && NBN >= 1, "32 x 32 blocks per wave");
  constexpr int ROWS = BM + BN;
  using LD = DmaTile<ROWS, NW>;
  constexpr int STAGE = ROWS * kRowBytes;
  static_assert(S >= 2 && S * STAGE <= 160 * 1024, "LDS ring exceeds the 160 KiB of a CU");
  __shared__ __attribute__((aligned(16))) char smem[S * STAGE];

  const int mt = (T + BM - 1) / BM, nt = (E + BN - 1) / BN;
  const int g = blockIdx.x;
  const int m_tile = g % mt;
  const int n_tile = (g / mt) % nt;
  const int ks = g / (mt * nt);
  if (ks >= ks_count) return;
  const int64_t kbytes = H * 2;
  const int nk_all = (int)(kbytes / kRowBytes);
  const int k0 = (int)((int64_t)nk_all * ks / ks_count), k1 = (int)((int64_t)nk_all * (ks + 1) / ks_count);
  const int nk = k1 - k0;
  const int t0 = m_tile * BM, e0 = n_tile * BN;

  LD ld;
#pragma unroll
  for (int i = 0; i < LD::NI; ++i) {
    const int r = LD::row_of(i);
    const char* src;
    if (r < BM) {
      const int t = t0 + r < T ? t0 + r : T - 1;
      src = reinterpret_cast<const char*>(x) + (int64_t)t * kbytes;
    } else {
      const int e = e0 + r - BM < E ? e0 + r - BM : E - 1;
      src = reinterpret_cast<const char*>(wr) + (int64_t)e * kbytes;
    }
    ld.set(i, src + (int64_t)k0 * kRowBytes);
  }

  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  f32x16 acc[NBN][NBM];
#pragma unroll
  for (int a = 0; a < NBN; ++a)
#pragma unroll
    for (int b = 0; b < NBM; ++b) acc[a][b] = f32x16{};
  constexpr int Q = LD::NI;
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) ld.issue(smem + s * STAGE, s);
  int cur = 0;
  for (int k = 0; k < nk; ++k) {
    wait_stages<Q, S - 2>(nk - 1 - k);
    barrier_no_fence();
    if (k + S - 1 < nk) ld.issue(smem + (cur == 0 ? S - 1 : cur - 1) * STAGE, k + S - 1);
    const char* st = smem + cur * STAGE;
    cur = cur + 1 == S ? 0 : cur + 1;
    u32x4 xf[2][NBM], wf[2][NBN];
    auto load_frags = [&](int buf, int s) {
#pragma unroll
      for (int b = 0; b < NBM; ++b) xf[buf][b] = frag(st, WTM * wm + 32 * b, s);
#pragma unroll
      for (int a = 0; a < NBN; ++a) wf[buf][a] = frag(st, BM + WTN * wn + 32 * a, s);
    };
    load_frags(0, 0);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int fb = s & 1;
      if (s < 3) load_frags(fb ^ 1, s + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int a = 0; a < NBN; ++a)
#pragma unroll
        for (int b = 0; b < NBM; ++b) acc[a][b] = mma(wf[fb][a], xf[fb][b], acc[a][b]);  // D[expert][token]
    }
  }

  // lane l: token l%32 of block b, experts 8*(r/4) + 4*(l/32) + r%4 of block a
  const int l = lane_id();
#pragma unroll
  for (int b = 0; b < NBM; ++b) {
    const int t = t0 + WTM * wm + 32 * b + (l & 31);
    if (t >= T) continue;
    float* row = part + ((int64_t)ks * T + t) * E;
#pragma unroll
    for (int a = 0; a < NBN; ++a)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int e = e0 + WTN * wn + 32 * a + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
        if (e < E) row[e] = acc[a][b][r];
      }
  }
}

// Routing of the summed partials: one wave per token.  A lane sums the
// ks_count splits of each of its VPL logits in split order; the loads of a
// batch of 8 splits are issued for all VPL logits before any is summed, so a
// lane has VPL * 8 loads in flight.  The summed logits are also written to
// `logits` when it is not null.
template <int VPL>
__global__ __launch_bounds__(256) void route_partials_kernel(const float* __restrict__ part, int ks_count,
                                                             const float* __restrict__ bias, int T, int E,
                                                             int k, int32_t* __restrict__ ids,
                                                             float* __restrict__ wout,
                                                             float* __restrict__ logits, int e_shared) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // uniform per wave
  constexpr int kBatch = 8;
  const int l = lane_id();
  const float* src = part + (int64_t)t * E + l;
  const int64_t stride = (int64_t)T * E;
  float v[VPL];
  uint32_t valid = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    v[j] = 0.0f;
    if (l + 64 * j < E) valid |= 1u << j;
  }
  for (int s0 = 0; s0 < ks_count; s0 += kBatch) {
    float pv[VPL][kBatch];
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        pv[j][u] = (valid & (1u << j)) && s0 + u < ks_count ? src[(s0 + u) * stride + 64 * j] : 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (s0 + u < ks_count) v[j] += pv[j][u];
  }
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    if (!(valid & (1u << j))) {
      v[j] = -INFINITY;
      continue;
    }
    if (logits) logits[(int64_t)t * E + l + 64 * j] = v[j];
    if (bias) v[j] = v[j] + bias[l + 64 * j];
  }
  route_token_values<VPL>(v, valid, t, k, ids, wout, e_shared >= 0 ? k + 1 : k, e_shared);
}

// Tile of the router GEMM: 128 tokens x MOE_ROUTER_BN experts (8 waves) when
// E is wide, 128 x 64 (4 waves) otherwise.  At dsv3 (T 4096, H 7168, E 256)
// 128 x 128 measured 32 us + 14 us routing, against 39 + 16 for 128 x 256
// (fewer, longer K splits) and 41 + 14 for 64 x 64 tiles.
#ifndef MOE_ROUTER_BN
#define MOE_ROUTER_BN 128
#endif
static bool router_wide(int64_t E) { return E >= 192; }
static int64_t router_items(int64_t T, int64_t E) {
  const int bn = router_wide(E) ? MOE_ROUTER_BN : 64;
  return ((T + 127) / 128) * ((E + bn - 1) / bn);
}

// Splits of K: about one item per CU (>= 256), at least 4 K steps each.
int router_splits(int64_t T, int64_t H, int64_t E) {
  const int64_t items = router_items(T, E);
  const int64_t nk = H / kRowBytes * 2;  // 128-byte steps of an fp16 row
  int64_t ks = (256 + items - 1) / items;
  const int64_t max_ks = nk / 4 > 1 ? nk / 4 : 1;
  ks = ks < 1 ? 1 : (ks > max_ks ? max_ks : ks);
  return (int)ks;
}

int64_t router_partial_floats(int64_t T, int64_t H, int64_t E) { return router_splits(T, H, E) * T * E; }

hipError_t launch_router(const void* x, const void* w_router, const float* bias, int T, int64_t H, int E,
                         int k, int32_t* ids, float* w, float* logits, float* part, hipStream_t s,
                         int e_shared) {
  if (T == 0) return hipSuccess;
  const int ks = router_splits(T, H, E);
  const int64_t grid = router_items(T, E) * ks;
  const _Float16* xp = reinterpret_cast<const _Float16*>(x);
  const _Float16* wp = reinterpret_cast<const _Float16*>(w_router);
  if (router_wide(E))
    hipLaunchKernelGGL((router_gemm_kernel<128, MOE_ROUTER_BN, 8, MOE_ROUTER_BN == 256 ? 3 : 4>), dim3((unsigned)grid),
                       dim3(512), 0, s, xp, wp, T, E, H, ks, part);
  else
    hipLaunchKernelGGL((router_gemm_kernel<128, 64, 4, 4>), dim3((unsigned)grid), dim3(256), 0, s, xp, wp, T, E, H,
                       ks, part);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const dim3 rgrid((T + 3) / 4), block(256);
  const int vpl = (E + 63) / 64;
#define MOE_RP(V) hipLaunchKernelGGL((route_partials_kernel<V>), rgrid, block, 0, s, part, ks, bias, T, E, k, ids, w, logits, \
                                     e_shared)
  if (vpl <= 1) MOE_RP(1);
  else if (vpl <= 2) MOE_RP(2);
  else if (vpl <= 4) MOE_RP(4);
  else if (vpl <= 8) MOE_RP(8);
  else MOE_RP(16);
#undef MOE_RP
  return hipGetLastError();
}

}  // namespace moe
