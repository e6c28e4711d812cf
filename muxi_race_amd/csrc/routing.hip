// Router (softmax -> top-k -> renormalise), moe_align (expert-sorted,
// block-padded permutation + group metadata), k-way combine, and per-row
// int8 quantisation.  All integer outputs are deterministic: no result depends
// on the order in which atomics land.
#include "launch.h"
#include "moe_common.h"
#include "route_token.h"

namespace moe {

// ---------------------------------------------------------------------------
// Router: one wave per token, VPL = ceil(E/64) logits per lane.
// ---------------------------------------------------------------------------
template <int VPL>
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ logits,
                                                         const float* __restrict__ bias, int T,
                                                         int E, int k, int32_t* __restrict__ ids,
                                                         float* __restrict__ wout, int e_shared) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // uniform per wave
  route_token_row<VPL>(logits + (int64_t)t * E, bias, t, E, k, ids, wout, e_shared >= 0 ? k + 1 : k, e_shared);
}

hipError_t launch_route_topk(const float* logits, const float* bias, int T, int E, int k,
                             int32_t* ids, float* w, hipStream_t s, int e_shared) {
  if (T == 0) return hipSuccess;
  const dim3 grid((T + 3) / 4), block(256);
  const int vpl = (E + 63) / 64;
#define MOE_RT(V) hipLaunchKernelGGL(route_topk_kernel<V>, grid, block, 0, s, logits, bias, T, E, k, ids, w, e_shared)
  if (vpl <= 1) MOE_RT(1);
  else if (vpl <= 2) MOE_RT(2);
  else if (vpl <= 4) MOE_RT(4);
  else if (vpl <= 8) MOE_RT(8);
  else MOE_RT(16);
#undef MOE_RT
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// moe_align: one workgroup of NW waves; wave w owns the contiguous pair range
// [w*R, (w+1)*R).  Ranks come from ballots: the lanes of a wave that hold the
// same expert are found by ANDing ballots of the expert-id bits, and a lane's
// rank is the number of such lanes below it.  No barrier inside the walks and
// no atomics, so placement follows pair order exactly:
//   1. count:  each wave builds its private per-expert histogram hist[w][e];
//   2. scan:   hist[w][e] becomes the wave's first row for expert e
//              (padded expert offset + counts of the waves before it), and
//              wave 0 writes group_sizes / group_offsets / padded offsets;
//   3. place:  each wave re-walks its range in order and writes pair p at
//              hist[w][e] + rank, then advances the cursor;
//   4. fill:   sentinel P in every padding row, block -> expert map.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t same_expert_mask(int e, bool ok, int nbits) {
  uint64_t same = __ballot(ok);
  for (int b = 0; b < nbits; ++b) {
    const int bit = (e >> b) & 1;
    const uint64_t bal = __ballot(bit);
    same &= bit ? bal : ~bal;
  }
  return same;
}

// Walks of one wave over its contiguous pair range [p0, p1).  The walks load
// kU rounds of ids at once so one load latency is exposed per kU rounds, not
// per round.  Out-of-range ids are dropped.
constexpr int kAlignUnroll = 8;

// count: the wave's private histogram hw[E] (no other wave touches it)
__device__ __forceinline__ void align_count_range(const int32_t* __restrict__ ids, int p0, int p1, int E,
                                                  int e_off, int nbits, int* hw) {
  const int l = lane_id();
  for (int i = l; i < E; i += 64) hw[i] = 0;
  const uint64_t lt_mask = (l == 0) ? 0ull : (~0ull >> (64 - l));
  for (int base = p0; base < p1; base += 64 * kAlignUnroll) {
    int ev[kAlignUnroll];
#pragma unroll
    for (int u = 0; u < kAlignUnroll; ++u) {
      const int p = base + 64 * u + l;
      ev[u] = p < p1 ? ids[p] : -1;
    }
#pragma unroll
    for (int u = 0; u < kAlignUnroll; ++u) {
      const unsigned ue = (unsigned)ev[u] - (unsigned)e_off;  // expert relative to the first one kept
      const bool ok = ue < (unsigned)E;
      const int e = ok ? (int)ue : 0;
      const uint64_t same = same_expert_mask(e, ok, nbits);
      if (ok && __popcll(same & lt_mask) == 0) hw[e] += __popcll(same);
    }
  }
}

// place, in pair order: pair p goes to hw[e] + rank, then the cursor advances
__device__ __forceinline__ void align_place_range(const int32_t* __restrict__ ids, int p0, int p1, int E,
                                                  int e_off, int nbits, int* hw, int32_t* __restrict__ sorted_ids) {
  const int l = lane_id();
  const uint64_t lt_mask = (l == 0) ? 0ull : (~0ull >> (64 - l));
  for (int base = p0; base < p1; base += 64 * kAlignUnroll) {
    int ev[kAlignUnroll];
#pragma unroll
    for (int u = 0; u < kAlignUnroll; ++u) {
      const int p = base + 64 * u + l;
      ev[u] = p < p1 ? ids[p] : -1;
    }
#pragma unroll
    for (int u = 0; u < kAlignUnroll; ++u) {
      const int p = base + 64 * u + l;
      const unsigned ue = (unsigned)ev[u] - (unsigned)e_off;
      const bool ok = ue < (unsigned)E;
      const int e = ok ? (int)ue : 0;
      const uint64_t same = same_expert_mask(e, ok, nbits);
      const int rank = __popcll(same & lt_mask);
      if (ok) {
        const int dst = hw[e] + rank;
        sorted_ids[dst] = p;
        if (rank == 0) hw[e] = dst + __popcll(same);
      }
    }
  }
}

// Inclusive prefix sum over the wave's 64 lanes: Hillis-Steele inside each
// 16-lane row with DPP row shifts (lanes shifted in from outside the row read
// 0), then each row adds the totals of the rows before it (read from lanes 15,
// 31, 47).  Integer adds, so the order of the terms does not matter.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31),
            r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane_id() >> 4;
  return v + (row > 0 ? r0 : 0) + (row > 1 ? r1 : 0) + (row > 2 ? r2 : 0);
}

// Expert scan by one wave: tot[E] -> padded offsets pstart[E+1] in LDS, and
// (when `out`) group sizes / offsets / padded offsets in global memory.
__device__ __forceinline__ void align_expert_scan(const int* tot, int E, int BM, int* pstart, bool out,
                                                  int32_t* __restrict__ gs, int32_t* __restrict__ go,
                                                  int32_t* __restrict__ gpo) {
  const int l = lane_id();
  int carry = 0, carry_p = 0;
  for (int base = 0; base < E; base += 64) {
    const int e = base + l;
    const int c = e < E ? tot[e] : 0;
    const int pc = (c + BM - 1) / BM * BM;
    const int ic = wave_inclusive_scan(c), ip = wave_inclusive_scan(pc);
    if (e < E) {
      pstart[e] = carry_p + ip - pc;
      if (out) {
        gs[e] = c;
        go[e] = carry + ic - c;
        gpo[e] = carry_p + ip - pc;
      }
    }
    carry += __builtin_amdgcn_readlane(ic, 63);
    carry_p += __builtin_amdgcn_readlane(ip, 63);
  }
  if (l == 0) {
    pstart[E] = carry_p;
    if (out) {
      go[E] = carry;
      gpo[E] = carry_p;
    }
  }
}

// padding rows of experts e0, e0 + step, ... -> sentinel P; their blocks ->
// owning expert (rows disjoint from the placed ones); by one wave
__device__ __forceinline__ void align_fill(const int* pstart, const int* tot, int E, int BM, int P, int e0,
                                           int step, int32_t* __restrict__ sorted_ids,
                                           int32_t* __restrict__ block_expert) {
  const int l = lane_id();
  for (int e = e0; e < E; e += step) {
    const int lo = pstart[e] + tot[e], hi = pstart[e + 1];
    for (int r = lo + l; r < hi; r += 64) sorted_ids[r] = P;
    for (int b = pstart[e] / BM + l; b < hi / BM; b += 64) block_expert[b] = e;
  }
}

__device__ __forceinline__ int bits_for(int E) {
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  return nbits;
}

// Small batches (up to 64 * kAlignUnroll pairs per wave): the one-workgroup
// kernel below with each wave's ids, ranks and group counts loaded once and
// kept in registers from the count to the placement, rounds past the wave's
// range skipped, and the padding written by all threads at once -- every used
// row is first set to the sentinel P, then (after a barrier, which orders the
// two writes of a row) the pairs overwrite their rows.  Same output as
// align_kernel.
template <int NW>
__global__ __launch_bounds__(64 * NW) void align_small_kernel(
    const int32_t* __restrict__ ids, int P, int E, int e_off, int BM, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ block_expert, int32_t* __restrict__ gs, int32_t* __restrict__ go,
    int32_t* __restrict__ gpo) {
  extern __shared__ int sm[];
  int* hist = sm;                 // [NW][E]: wave w's count of expert e, then its first row among e's
  int* tot = sm + NW * E;         // [E]
  int* pstart = tot + E;          // [E+1] padded offsets
  const int tid = threadIdx.x, w = tid >> 6, l = lane_id();
  const int nbits = bits_for(E);
  const int R = ((P + NW - 1) / NW + 63) / 64 * 64;  // <= 64 * kAlignUnroll (launch_align checks)
  const int p0 = w * R, p1 = min(P, p0 + R);
  const int nwa = R > 0 ? min(NW, (P + R - 1) / R) : 0;  // waves that hold pairs
  int* hw = hist + w * E;
  for (int i = l; i < E; i += 64) hw[i] = 0;
  const uint64_t lt_mask = (l == 0) ? 0ull : (~0ull >> (64 - l));
  int ev[kAlignUnroll], rk[kAlignUnroll], cn[kAlignUnroll];
#pragma unroll
  for (int u = 0; u < kAlignUnroll; ++u) {
    const int p = p0 + 64 * u + l;
    ev[u] = p < p1 ? ids[p] : -1;
  }
#pragma unroll
  for (int u = 0; u < kAlignUnroll; ++u) {
    rk[u] = 0;
    cn[u] = 0;
    if (p0 + 64 * u >= p1) {  // uniform: past the wave's range
      ev[u] = -1;
      continue;
    }
    const unsigned ue = (unsigned)ev[u] - (unsigned)e_off;
    const bool ok = ue < (unsigned)E;
    const int e = ok ? (int)ue : 0;
    const uint64_t same = same_expert_mask(e, ok, nbits);
    rk[u] = __popcll(same & lt_mask);
    cn[u] = __popcll(same);
    ev[u] = ok ? e : -1;
    if (ok && rk[u] == 0) hw[e] += cn[u];
  }
  __syncthreads();
  for (int e = tid; e < E; e += 64 * NW) {
    int run = 0;
    for (int v = 0; v < nwa; ++v) {
      const int c = hist[v * E + e];
      hist[v * E + e] = run;
      run += c;
    }
    tot[e] = run;
  }
  __syncthreads();
  if (w == 0) align_expert_scan(tot, E, BM, pstart, true, gs, go, gpo);
  __syncthreads();
  const int rows = pstart[E];
  for (int r = tid; r < rows; r += 64 * NW) sorted_ids[r] = P;
  for (int e = tid; e < E; e += 64 * NW)
    for (int b = pstart[e] / BM; b < pstart[e + 1] / BM; ++b) block_expert[b] = e;
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kAlignUnroll; ++u) {
    const int e = ev[u];
    if (e >= 0) {
      sorted_ids[pstart[e] + hw[e] + rk[u]] = p0 + 64 * u + l;
      if (rk[u] == 0) hw[e] += cn[u];
    }
  }
}

// One workgroup of NW waves; wave w owns the contiguous pair range
// [w*R, (w+1)*R).  1. count into per-wave histograms; 2. per-wave exclusive
// prefix per expert and the expert scan; 3. place; 4. fill.
template <int NW>
__global__ __launch_bounds__(64 * NW) void align_kernel(
    const int32_t* __restrict__ ids, int P, int E, int e_off, int BM, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ block_expert, int32_t* __restrict__ gs, int32_t* __restrict__ go,
    int32_t* __restrict__ gpo) {
  extern __shared__ int sm[];
  int* hist = sm;                 // [NW][E]
  int* tot = sm + NW * E;         // [E]
  int* pstart = tot + E;          // [E+1] padded offsets
  const int tid = threadIdx.x, w = tid >> 6;
  const int nbits = bits_for(E);
  const int R = ((P + NW - 1) / NW + 63) / 64 * 64;
  const int p0 = w * R, p1 = min(P, p0 + R);
  int* hw = hist + w * E;
  align_count_range(ids, p0, p1, E, e_off, nbits, hw);
  __syncthreads();
  for (int e = tid; e < E; e += 64 * NW) {
    int run = 0;
    for (int v = 0; v < NW; ++v) {
      const int c = hist[v * E + e];
      hist[v * E + e] = run;
      run += c;
    }
    tot[e] = run;
  }
  __syncthreads();
  if (w == 0) align_expert_scan(tot, E, BM, pstart, true, gs, go, gpo);
  __syncthreads();
  for (int e = tid; e < E; e += 64 * NW)
    for (int v = 0; v < NW; ++v) hist[v * E + e] += pstart[e];
  __syncthreads();
  align_place_range(ids, p0, p1, E, e_off, nbits, hw, sorted_ids);
  align_fill(pstart, tot, E, BM, P, w, NW, sorted_ids, block_expert);
}

// Large P: G workgroups, workgroup g owning pairs [g*RW, (g+1)*RW) (wave w of
// it the sub-range [w*R, (w+1)*R)).  Kernel 1 writes each workgroup's expert
// histogram to whist[g][E]; kernel 2 derives from all of them the expert scan
// and the workgroup's first row per expert, recounts per wave, and places.
// Pair order within an expert, hence the output, is the one-workgroup kernel's.
template <int NW>
__global__ __launch_bounds__(64 * NW) void align_count_kernel(const int32_t* __restrict__ ids, int P, int E,
                                                              int e_off, int RW, int32_t* __restrict__ whist) {
  extern __shared__ int sm[];
  int* hist = sm;  // [NW][E]
  const int tid = threadIdx.x, w = tid >> 6;
  const int g0 = blockIdx.x * RW, g1 = min(P, g0 + RW);
  const int R = RW / NW;
  const int p0 = min(g1, g0 + w * R), p1 = min(g1, p0 + R);
  align_count_range(ids, p0, p1, E, e_off, bits_for(E), hist + w * E);
  __syncthreads();
  for (int e = tid; e < E; e += 64 * NW) {
    int run = 0;
    for (int v = 0; v < NW; ++v) run += hist[v * E + e];
    whist[(int64_t)blockIdx.x * E + e] = run;
  }
}

template <int NW>
__global__ __launch_bounds__(64 * NW) void align_place_kernel(
    const int32_t* __restrict__ ids, int P, int E, int e_off, int BM, int RW, const int32_t* __restrict__ whist,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ block_expert, int32_t* __restrict__ gs,
    int32_t* __restrict__ go, int32_t* __restrict__ gpo) {
  extern __shared__ int sm[];
  int* hist = sm;                 // [NW][E]
  int* tot = sm + NW * E;         // [E]
  int* pstart = tot + E;          // [E+1]
  int* before = pstart + E + 1;   // [E] pairs of expert e in the workgroups before this one
  const int tid = threadIdx.x, w = tid >> 6;
  const int G = gridDim.x, g = blockIdx.x;
  // Every workgroup's count of expert e, loaded kBatch at a time before any is
  // added, so one load latency is exposed per batch rather than per workgroup.
  constexpr int kBatch = 16;
  for (int e = tid; e < E; e += 64 * NW) {
    int run = 0, mine = 0;
    for (int v0 = 0; v0 < G; v0 += kBatch) {
      int c[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) c[u] = v0 + u < G ? whist[(int64_t)(v0 + u) * E + e] : 0;
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (v0 + u == g) mine = run;
        run += c[u];
      }
    }
    tot[e] = run;
    before[e] = mine;
  }
  const int g0 = g * RW, g1 = min(P, g0 + RW);
  const int R = RW / NW;
  const int p0 = min(g1, g0 + w * R), p1 = min(g1, p0 + R);
  const int nbits = bits_for(E);
  int* hw = hist + w * E;
  align_count_range(ids, p0, p1, E, e_off, nbits, hw);
  __syncthreads();
  if (w == 0) align_expert_scan(tot, E, BM, pstart, g == 0, gs, go, gpo);
  __syncthreads();
  for (int e = tid; e < E; e += 64 * NW) {
    int run = pstart[e] + before[e];
    for (int v = 0; v < NW; ++v) {
      const int c = hist[v * E + e];
      hist[v * E + e] = run;
      run += c;
    }
  }
  __syncthreads();
  align_place_range(ids, p0, p1, E, e_off, nbits, hw, sorted_ids);
  align_fill(pstart, tot, E, BM, P, g * NW + w, G * NW, sorted_ids, block_expert);
}

hipError_t launch_align(const int32_t* ids, int P, int E, int BM, int32_t* sorted_ids,
                        int32_t* block_expert, int32_t* gs, int32_t* go, int32_t* gpo,
                        int32_t* whist, hipStream_t s, int e_off) {
  // 16 waves while the histograms fit 48 KiB of LDS, else 8 (E <= 1024)
  const bool w16 = 16 * E <= 12288;
  const int nw = w16 ? 16 : 8;
  const int per_wave = (P + nw - 1) / nw;  // pairs per wave in one workgroup
  if (per_wave <= 64 * kAlignUnroll) {  // one workgroup, each wave's pairs held in registers
    const size_t lds = sizeof(int) * (nw * (size_t)E + 2 * (size_t)E + 1);
    if (w16)
      hipLaunchKernelGGL(align_small_kernel<16>, dim3(1), dim3(1024), lds, s, ids, P, E, e_off, BM, sorted_ids,
                         block_expert, gs, go, gpo);
    else
      hipLaunchKernelGGL(align_small_kernel<8>, dim3(1), dim3(512), lds, s, ids, P, E, e_off, BM, sorted_ids,
                         block_expert, gs, go, gpo);
    return hipGetLastError();
  }
  const int G = align_groups(P);
  if (whist && G > 1) {
    const int RW = align_pairs_per_group(P, G, nw);
    const size_t lds1 = sizeof(int) * ((size_t)nw * E);
    const size_t lds2 = sizeof(int) * ((size_t)nw * E + 3 * (size_t)E + 1);
    if (w16) {
      hipLaunchKernelGGL(align_count_kernel<16>, dim3(G), dim3(1024), lds1, s, ids, P, E, e_off, RW, whist);
      hipLaunchKernelGGL(align_place_kernel<16>, dim3(G), dim3(1024), lds2, s, ids, P, E, e_off, BM, RW, whist,
                         sorted_ids, block_expert, gs, go, gpo);
    } else {
      hipLaunchKernelGGL(align_count_kernel<8>, dim3(G), dim3(512), lds1, s, ids, P, E, e_off, RW, whist);
      hipLaunchKernelGGL(align_place_kernel<8>, dim3(G), dim3(512), lds2, s, ids, P, E, e_off, BM, RW, whist,
                         sorted_ids, block_expert, gs, go, gpo);
    }
    return hipGetLastError();
  }
  const size_t lds = sizeof(int) * (nw * (size_t)E + 2 * (size_t)E + 1);
  if (w16)
    hipLaunchKernelGGL(align_kernel<16>, dim3(1), dim3(1024), lds, s, ids, P, E, e_off, BM, sorted_ids,
                       block_expert, gs, go, gpo);
  else
    hipLaunchKernelGGL(align_kernel<8>, dim3(1), dim3(512), lds, s, ids, P, E, e_off, BM, sorted_ids,
                       block_expert, gs, go, gpo);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Combine: out[t, :] = sum_j y_pair[pos[t*k + j], :], fp32 in choice order ->
// fp16 (Stage 2 writes each pair's row at its expert-sorted position pos).
// One thread per 8 output columns.  The k rows are loaded in batches of 8
// before they are summed (in choice order), so each thread keeps several loads
// in flight; y_pair is read once, so the loads are non-temporal, and so are the
// stores of out (dsv3: 90-91 us against 96-97 with default stores).  With `ids`
// (an expert shard), only pairs routed to experts [e_lo, e_lo + e_n) are
// summed: the others' rows were never written.
// ---------------------------------------------------------------------------
template <int KC>
__global__ __launch_bounds__(256) void combine_kernel(const _Float16* __restrict__ y,
                                                      const int32_t* __restrict__ pos, int64_t T,
                                                      int64_t H, int k_rt, _Float16* __restrict__ out,
                                                      const int32_t* __restrict__ ids, int e_lo, int e_n) {
  const int k = KC > 0 ? KC : k_rt;  // KC > 0: k known at compile time (no masked batch slots)
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t cpr = H / 8;
  if (idx >= T * cpr) return;
  const int64_t t = idx / cpr, c = idx % cpr;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const _Float16* src = y + 8 * c;
  const int32_t* prow = pos + t * k;
  constexpr int kBatch = KC > 0 ? KC : 8;
  for (int j0 = 0; j0 < k; j0 += kBatch) {
    // Every load of the batch is issued unconditionally, positions first,
    // then the pair rows: a predicated load compiles to a branch that waits
    // for all earlier loads, which serialised a thread's k row loads.  A slot
    // past k or a pair outside the expert range (whose position was never
    // written) reads row 0 and is dropped by a select.
    int32_t pj[kBatch];
    bool in[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int j = j0 + u < k ? j0 + u : k - 1;  // an entry of token t (k >= 1)
      pj[u] = prow[j];
      in[u] = j0 + u < k && (!ids || (unsigned)ids[t * k + j] - (unsigned)e_lo < (unsigned)e_n);
    }
    f16x8 v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(src + (int64_t)(in[u] ? pj[u] : 0) * H));
    __builtin_amdgcn_sched_barrier(0);  // every row load issued before any use
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] = in[u] ? acc[q] + (float)v[u][q] : acc[q];
  }
  f16x8 r;
#pragma unroll
  for (int q = 0; q < 8; ++q) r[q] = (_Float16)acc[q];
  __builtin_nontemporal_store(r, reinterpret_cast<f16x8*>(out + t * H + 8 * c));
}

hipError_t launch_combine(const void* y_pair, const int32_t* pos, int64_t T, int64_t H, int k, void* out,
                          hipStream_t s, const int32_t* ids, int e_lo, int e_n) {
  const int64_t n = T * (H / 8);
  if (n == 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  const _Float16* yp = reinterpret_cast<const _Float16*>(y_pair);
  _Float16* o = reinterpret_cast<_Float16*>(out);
  switch (k) {
    case 2: hipLaunchKernelGGL(combine_kernel<2>, grid, block, 0, s, yp, pos, T, H, k, o, ids, e_lo, e_n); break;
    case 6: hipLaunchKernelGGL(combine_kernel<6>, grid, block, 0, s, yp, pos, T, H, k, o, ids, e_lo, e_n); break;
    case 8: hipLaunchKernelGGL(combine_kernel<8>, grid, block, 0, s, yp, pos, T, H, k, o, ids, e_lo, e_n); break;
    default: hipLaunchKernelGGL(combine_kernel<0>, grid, block, 0, s, yp, pos, T, H, k, o, ids, e_lo, e_n); break;
  }
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void zero_kernel(u32x4* __restrict__ p, int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n16) p[i] = u32x4{0, 0, 0, 0};
}

hipError_t launch_zero(void* p, int64_t n, hipStream_t s) {
  const int64_t n16 = n / 16;
  if (n16 == 0) return hipSuccess;
  hipLaunchKernelGGL(zero_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, s,
                     reinterpret_cast<u32x4*>(p), n16);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Per-row symmetric int8: one wave per row, 8 fp16 per lane per chunk.  Rows
// of up to 64 * 8 * NCH elements are held in registers (all NCH chunk loads
// in flight at once, one pass over memory); longer rows take two passes.
// ---------------------------------------------------------------------------
template <bool F8>
__device__ __forceinline__ u32x2 quant_pack8(f16x8 v, float inv) {
  return u32x2{quant_code4<F8>((float)v[0], (float)v[1], (float)v[2], (float)v[3], inv),
               quant_code4<F8>((float)v[4], (float)v[5], (float)v[6], (float)v[7], inv)};
}

// One wave quantises one row of K fp16 values: amax over the row, codes of
// x * (qmax / amax) into qrow, amax / qmax into *scale (written by lane 0).
// Rows of up to 512 * NCH values are held in registers: quant_row_load issues
// every load of the row at once, quant_row_store finishes the row, so a
// caller can run other work while the loads are in flight.
// Every load is unconditional (a chunk past the row reads the row's last
// chunk and is zeroed by a select): a predicated load compiles to a branch
// that waits for all earlier loads, which serialised the row's loads.
// K is a positive multiple of 8.
template <int NCH>
__device__ __forceinline__ void quant_row_load(const _Float16* __restrict__ row, int64_t K, f16x8 (&v)[NCH]) {
  const int l = lane_id();
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t c = 512 * j + 8 * l;
    v[j] = *reinterpret_cast<const f16x8*>(row + (c < K ? c : K - 8));
  }
  __builtin_amdgcn_sched_barrier(0);  // every load issued before any use of a result
#pragma unroll
  for (int j = 0; j < NCH; ++j)
    if (512 * j + 8 * l >= K) v[j] = f16x8{};
}
template <int NCH, bool F8>
__device__ __forceinline__ void quant_row_store(const f16x8 (&v)[NCH], int64_t K, uint8_t* __restrict__ qrow,
                                                float* __restrict__ scale) {
  const int l = lane_id();
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf((float)v[j][i]));
  amax = wave_max(amax);
  const float inv = amax > 0.0f ? qmax<F8>() / amax : 0.0f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t c = 512 * j + 8 * l;
    if (c < K) *reinterpret_cast<u32x2*>(qrow + c) = quant_pack8<F8>(v[j], inv);
  }
  if (l == 0) *scale = amax / qmax<F8>();
}
template <int NCH, bool F8>
__device__ __forceinline__ void quant_row_wave(const _Float16* __restrict__ row, int64_t K,
                                               uint8_t* __restrict__ qrow, float* __restrict__ scale) {
  if constexpr (NCH > 0) {
    f16x8 v[NCH];
    quant_row_load<NCH>(row, K, v);
    quant_row_store<NCH, F8>(v, K, qrow, scale);
  } else {
    const int l = lane_id();
    float amax = 0.0f;
    for (int64_t c = 8 * l; c < K; c += 512) {
      const f16x8 v = *reinterpret_cast<const f16x8*>(row + c);
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf((float)v[i]));
    }
    amax = wave_max(amax);
    const float inv = amax > 0.0f ? qmax<F8>() / amax : 0.0f;
    for (int64_t c = 8 * l; c < K; c += 512)
      *reinterpret_cast<u32x2*>(qrow + c) = quant_pack8<F8>(*reinterpret_cast<const f16x8*>(row + c), inv);
    if (l == 0) *scale = amax / qmax<F8>();
  }
}

//
// With `ids` set, row r is quantised only if r < *used_rows and ids[r] <
// sentinel: the intermediate's rows in the expert-sorted space, where rows
// past the experts' padded range and padding rows (sentinel id) are never
// written by Stage 1 and are left alone here.
template <int NCH, bool F8>
__global__ __launch_bounds__(256) void quant_rows_kernel(const _Float16* __restrict__ w, int64_t R,
                                                         int64_t K, uint8_t* __restrict__ q,
                                                         float* __restrict__ scale,
                                                         const int32_t* __restrict__ ids, int32_t sentinel,
                                                         const int32_t* __restrict__ used_rows) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  if (ids && (r >= *used_rows || ids[r] >= sentinel)) return;
  quant_row_wave<NCH, F8>(w + r * K, K, q + r * K, scale + r);
}

// Routing of token t (as route_topk_kernel) and, in the same wave, the 8-bit
// quantisation of its activation row x[t] (as quant_rows_kernel): both are
// per-token passes over independent inputs, so the 8-bit paths run them as
// one launch instead of two, with the row's loads issued before the routing
// so that their latency overlaps it.
template <int VPL, int NCH, bool F8>
__global__ __launch_bounds__(256) void route_quant_kernel(const float* __restrict__ logits,
                                                          const float* __restrict__ bias, int T, int E, int k,
                                                          int32_t* __restrict__ ids, float* __restrict__ wout,
                                                          const _Float16* __restrict__ x, int64_t H,
                                                          uint8_t* __restrict__ xq, float* __restrict__ sx) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // uniform per wave
  const float* row = logits + (int64_t)t * E;
  if constexpr (NCH > 0) {
    // logits (and bias) first, then the row: loads retire in order, so the
    // routing waits only for its own values while the row is in flight
    // (unconditional loads at clamped experts, then selected: see route_token_row)
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
    f16x8 v[NCH];
    quant_row_load<NCH>(x + (int64_t)t * H, H, v);
    uint32_t valid = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const bool in = l + 64 * j < E;
      lv[j] = in ? (bias ? lv[j] + bv[j] : lv[j]) : -INFINITY;
      valid |= in ? 1u << j : 0u;
    }
    route_token_values<VPL>(lv, valid, t, k, ids, wout, k, -1);
    quant_row_store<NCH, F8>(v, H, xq + (int64_t)t * H, sx + t);
  } else {
    route_token_row<VPL>(row, bias, t, E, k, ids, wout, k, -1);
    quant_row_wave<NCH, F8>(x + (int64_t)t * H, H, xq + (int64_t)t * H, sx + t);
  }
}

hipError_t launch_route_quant(const float* logits, const float* bias, int T, int E, int k, int32_t* ids,
                              float* w, const void* x, int64_t H, void* xq, float* sx, int qt, hipStream_t s) {
  if (T == 0) return hipSuccess;
  const dim3 grid((T + 3) / 4), block(256);
  const int vpl = (E + 63) / 64;
  const int64_t nch = (H + 511) / 512;
  const _Float16* xs = reinterpret_cast<const _Float16*>(x);
  uint8_t* q = reinterpret_cast<uint8_t*>(xq);
#define MOE_RQ2(V, N, F) \
  hipLaunchKernelGGL((route_quant_kernel<V, N, F>), grid, block, 0, s, logits, bias, T, E, k, ids, w, xs, H, q, sx)
#define MOE_RQ1(V, F)            \
  do {                           \
    if (nch <= 4) MOE_RQ2(V, 4, F);       \
    else if (nch <= 8) MOE_RQ2(V, 8, F);  \
    else if (nch <= 16) MOE_RQ2(V, 16, F); \
    else MOE_RQ2(V, 0, F);                \
  } while (0)
#define MOE_RQ(V)                          \
  do {                                     \
    if (qt == kQF8) MOE_RQ1(V, true);      \
    else MOE_RQ1(V, false);                \
  } while (0)
  if (vpl <= 1) MOE_RQ(1);
  else if (vpl <= 2) MOE_RQ(2);
  else if (vpl <= 4) MOE_RQ(4);
  else if (vpl <= 8) MOE_RQ(8);
  else MOE_RQ(16);
#undef MOE_RQ
#undef MOE_RQ1
#undef MOE_RQ2
  return hipGetLastError();
}

hipError_t launch_quant_rows(const void* w, int64_t R, int64_t K, void* q, float* scale, int qt,
                             hipStream_t s, const int32_t* ids, int32_t sentinel, const int32_t* used_rows) {
  if (R == 0) return hipSuccess;
  const dim3 grid((unsigned)((R + 3) / 4)), block(256);
  const _Float16* src = reinterpret_cast<const _Float16*>(w);
  uint8_t* dst = reinterpret_cast<uint8_t*>(q);
  const int64_t nch = (K + 511) / 512;
#define MOE_QR(N)                                                                               \
  do {                                                                                          \
    if (qt == kQF8)                                                                             \
      hipLaunchKernelGGL((quant_rows_kernel<N, true>), grid, block, 0, s, src, R, K, dst, scale, ids, sentinel, used_rows);  \
    else                                                                                        \
      hipLaunchKernelGGL((quant_rows_kernel<N, false>), grid, block, 0, s, src, R, K, dst, scale, ids, sentinel, used_rows); \
  } while (0)
  if (nch <= 4) MOE_QR(4);
  else if (nch <= 8) MOE_QR(8);
  else if (nch <= 16) MOE_QR(16);
  else MOE_QR(0);
#undef MOE_QR
  return hipGetLastError();
}

}  // namespace moe
