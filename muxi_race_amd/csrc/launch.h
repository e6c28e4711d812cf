// Internal launcher interface between the C ABI (capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Fused Stage 2 scatter-reduce (1): each weighted pair row is added straight
// into its token's fp16 output row with packed fp16 atomics (the output is
// zeroed first, and no combine runs), instead of (0, the default) a per-pair
// row that the deterministic combine sums in choice order.  Off by default:
// device-scope atomics on MI355X run far below plain stores.  A/B in one run
// (2 x 2 interleaved): dsv3's step 5.26 -> 5.61 ms (Stage 2 1.855 -> 2.321 ms
// against the combine's 0.090), mixtral 1.543 -> 1.583, w8a8 int8 0.890 ->
// 1.178, fp8 0.833 -> 1.124, decode level (0.501 -> 0.499).  And the order of
// the additions, so the fp16 rounding of the sum, varies from call to call.
#ifndef MOE_S2_SCATTER
#define MOE_S2_SCATTER 0
#endif

namespace moe {

// Operand formats of the expert GEMMs: fp16, or 8-bit codes with fp32 row
// scales -- int8 (i8 MFMA, int32 accumulation) or OCP fp8 e4m3 (f8 MFMA, fp32
// accumulation).
enum QuantType : int { kQF16 = 0, kQI8 = 1, kQF8 = 2 };

// Stage 1: h = silu(X Wg^T) * (X Wu^T) for the rows of every M block.
struct Stage1Params {
  const char* x;            // fp16 [rows, H] (direct) / fp16|int8 [T, H] (gather)
  const char* wg;           // [E, I, H]
  const char* wu;           // [E, I, H]
  char* h;                  // fp16 [padded rows, I] (fp16 and int8 operands) | fp8 [padded rows, I]
  float* h_scale;           // fp8 only: [I/128][hs_stride] (block-major)
  int64_t hs_stride;        // fp8 only: rows of each h_scale block (>= padded rows)
  const float* x_scale;     // 8-bit only: [T]
  const float* sg;          // 8-bit only: [E, I]
  const float* su;          // 8-bit only: [E, I]
  const int32_t* gs;        // [E]
  const int32_t* gpo;       // [E+1]
  const int32_t* sorted_ids;  // gather only: [padded rows], sentinel = T*topk
  const int32_t* gidx;      // direct only: block -> expert ([host_blocks] entries)
  const char* wg_shared;    // weights of expert e_shared ([I, H]) when e_shared >= 0
  const char* wu_shared;
  int e_shared = -1;        // always-on shared expert's index, or -1
  int64_t w_ld = 0;         // bytes between rows of wg / wu / the shared ones (0: H elements)
  int64_t w_es = 0;         // bytes between experts of wg / wu (0: I rows)
  int64_t h_ld = 0;         // elements between rows of h (0: I)
  int topk;
  int E;
  int64_t H;
  int64_t I;
  int host_blocks;          // BM-row blocks the row buffers hold (set by the launcher);
                            // direct: blocks of the launch (gidx entries, clamped)
  int absorb = 0;           // fp16, 256-row or 128-row paired items, E <= 256: absorbed
                            // rows; the blocks a pair must keep (moe_common.h), 0: off
};

// Stage 2: y = h Wd^T, scaled by the routing weight of each row.
struct Stage2Params {
  const char* a;            // fp16|int8|fp8 [padded rows, I]
  const float* a_scale;     // int8: [padded rows] (per row); fp8: [I/128][as_stride] (block-major)
  int64_t as_stride;        // fp8 only: rows of each a_scale block (>= padded rows)
  const char* wd;           // [E, H, I]
  const float* sd;          // 8-bit only: [E, H]
  char* out;                // pre-routed: fp16 [P, H]; fused: fp16 [T*topk, H], row = the pair's
                            // unpadded expert-sorted position go[e] + (row - gpo[e])
  int32_t* pos;             // fused only: pos[pair] = that row (written by the first N tile's items)
  const void* routed;       // pre-routed: [V] raw order (fp32|fp16); fused: fp32 [T*topk]
  int routed_f16;
  const int32_t* gs;
  const int32_t* go;
  const int32_t* gpo;
  const int32_t* sorted_ids;  // fused only
  const int32_t* gidx;      // pre-routed only: block -> expert ([host_blocks] entries)
  const char* wd_shared;    // down weights of expert e_shared ([H, I]) when e_shared >= 0
  int e_shared = -1;        // always-on shared expert's index, or -1
  int64_t a_ld = 0;         // bytes between rows of a (0: I elements)
  int64_t wd_ld = 0;        // bytes between rows of wd / wd_shared (0: I elements)
  int64_t wd_es = 0;        // bytes between experts of wd (0: H rows)
  int E;
  int64_t H;
  int64_t I;
  int64_t V;                // pre-routed: entries of `routed` (raw index is clamped to V-1)
  int host_blocks;          // BM-row blocks the row buffers hold (set by the launcher);
                            // pre-routed: blocks of the launch (gidx entries, clamped)
  int absorb = 0;           // fp16, 128-row paired items, E <= 256: absorbed rows; as in Stage 1
  int topk = 0;             // fused, built with MOE_S2_SCATTER: choices per token; `out` is then
                            // fp16 [T, H] (zeroed first) and each pair row is added to its token's
                            // row with packed fp16 atomics
};

// Zeroes n bytes (n a multiple of 16, p 16-byte aligned) with vector stores:
// a kernel, not hipMemsetAsync, so that it can be captured in a graph.
hipError_t launch_zero(void* p, int64_t n, hipStream_t stream);

// qt: a QuantType
hipError_t launch_stage1(const Stage1Params& p, int block_m, int qt, bool gather,
                         int64_t max_blocks, hipStream_t stream);
hipError_t launch_stage2(const Stage2Params& p, int block_m, int qt, bool fused,
                         int64_t max_blocks, hipStream_t stream);

// With e_shared >= 0 every token also gets the shared expert as choice k
// (id e_shared, weight 1): ids / w rows hold k + 1 entries.
hipError_t launch_route_topk(const float* logits, const float* bias, int T, int E, int k,
                             int32_t* ids, float* w, hipStream_t stream, int e_shared = -1);
// `whist` (int32 [align_groups(P) * E], may be null) lets a large P be aligned
// by align_groups(P) workgroups in two launches instead of one workgroup.
constexpr int kAlignPairsPerGroup = 2048;
constexpr int kAlignMaxGroups = 64;
// (below 4 groups' worth of pairs the second launch costs more than it saves)
inline int align_groups(int P) {
  const int g = (P + kAlignPairsPerGroup - 1) / kAlignPairsPerGroup;
  return g < 4 ? 1 : (g > kAlignMaxGroups ? kAlignMaxGroups : g);
}
// pairs per workgroup: a multiple of 64 * nw covering P in `groups` workgroups
inline int align_pairs_per_group(int P, int groups, int nw) {
  const int per = (P + groups - 1) / groups;
  return (per + 64 * nw - 1) / (64 * nw) * (64 * nw);
}
// e_off: pairs are bucketed by id - e_off; ids outside [e_off, e_off + E)
// are dropped (an expert shard of a wider routing).
hipError_t launch_align(const int32_t* ids, int P, int E, int BM, int32_t* sorted_ids,
                        int32_t* block_expert, int32_t* gs, int32_t* go, int32_t* gpo,
                        int32_t* whist, hipStream_t stream, int e_off = 0);
// Router GEMM (x . w_router^T, K split in router_splits parts) + routing of
// the summed partials; `part` holds router_partial_floats fp32, `logits`
// (fp32 [T, E]) may be null.
int router_splits(int64_t T, int64_t H, int64_t E);
int64_t router_partial_floats(int64_t T, int64_t H, int64_t E);
hipError_t launch_router(const void* x, const void* w_router, const float* bias, int T, int64_t H, int E,
                         int k, int32_t* ids, float* w, float* logits, float* part, hipStream_t stream,
                         int e_shared = -1);
// ids (may be null): sum only pairs whose expert is in [e_lo, e_lo + e_n).
// y_pair row of pair t*k + j: pos[t*k + j].
hipError_t launch_combine(const void* y_pair, const int32_t* pos, int64_t T, int64_t H, int k, void* out,
                          hipStream_t stream, const int32_t* ids = nullptr, int e_lo = 0, int e_n = 0);
// Routing (as launch_route_topk, no shared expert) and the per-token 8-bit
// quantisation of x [T, H] (as launch_quant_rows) in one launch.
hipError_t launch_route_quant(const float* logits, const float* bias, int T, int E, int k, int32_t* ids,
                              float* w, const void* x, int64_t H, void* xq, float* sx, int qt,
                              hipStream_t stream);
// Per-row 8-bit quantisation of an fp16 [R, K] matrix to the format qt
// (kQI8 or kQF8): codes into q, amax / qmax into scale.  With `ids` set only
// rows r < *used_rows (a device value) with ids[r] < sentinel are quantised
// (the int8 intermediate: rows in the expert-sorted space).
hipError_t launch_quant_rows(const void* w, int64_t R, int64_t K, void* q, float* scale, int qt,
                             hipStream_t stream, const int32_t* ids = nullptr, int32_t sentinel = 0,
                             const int32_t* used_rows = nullptr);

}  // namespace moe
