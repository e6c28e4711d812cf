// extern "C" entry points of libmoe_gfx950.so (declared in include/moe_gfx950.h).
// Host-side only: argument validation, workspace carving, launch order.  All
// work is enqueued on the caller's stream; nothing here allocates or waits.
#include "../../include/moe_gfx950.h"
#include "launch.h"
#include "moe_common.h"

#include <stdarg.h>
#include <stdio.h>

#include <mutex>

// fp16 Stage 2 over the 256-row padding: 256-row items (1) or 128-row paired
// items (0).
#ifndef MOE_S2_F16_256
#define MOE_S2_F16_256 1
#endif

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(MOE_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return MOE_OK;
}

constexpr int64_t kAlign = 256;
int64_t up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

int64_t cap_rows(int64_t T, int64_t k, int64_t E, int64_t bm) {
  const int64_t P = T * k;
  const int64_t owners = E < P ? E : P;
  return (P + owners * (bm - 1)) / bm * bm;
}

struct FusedLayout {
  int64_t ids, w, sorted, bexp, gs, go, gpo, whist, h, hq, hs, xq, sx, ypair, pos, total;
};

// qt: moe::kQF16, kQI8 or kQF8.  The intermediate h is fp16 for fp16 and int8
// operands (int8 quantises it per row afterwards, into hq + hs), fp8 codes
// for fp8 (with per-(row, 128-column) scales in hs).
FusedLayout fused_layout(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int64_t bm,
                         int qt) {
  FusedLayout L{};
  const bool w8 = qt != moe::kQF16, i8 = qt == moe::kQI8;
  const int64_t P = T * k, rows = cap_rows(T, k, E, bm);
  int64_t o = 0;
  L.ids = o; o += up(P * 4);
  L.w = o; o += up(P * 4);
  L.sorted = o; o += up(rows * 4);
  L.bexp = o; o += up((rows / bm) * 4);
  L.gs = o; o += up(E * 4);
  L.go = o; o += up((E + 1) * 4);
  L.gpo = o; o += up((E + 1) * 4);
  L.whist = o; o += up((int64_t)moe::align_groups((int)P) * E * 4);  // align workgroup histograms
  L.h = o; o += up(rows * I * (qt == moe::kQF8 ? 1 : 2));
  L.hq = o; o += i8 ? up(rows * I) : 0;                   // int8: per-row codes of h
  L.hs = o; o += w8 ? up(rows * (i8 ? 1 : I / moe::kBN) * 4) : 0;  // int8 [rows]; fp8 [I/128][rows], block-major
  L.xq = o; o += w8 ? up(T * H) : 0;
  L.sx = o; o += w8 ? up(T * 4) : 0;
  L.ypair = o; o += up(P * H * 2);                        // per-pair outputs, expert-sorted rows
  L.pos = o; o += up(P * 4);                              // pair -> its y_pair row
  L.total = o;
  return L;
}

int64_t pick_bm(int64_t T, int64_t E, int64_t k) {
  const int64_t avg = E > 0 ? (T * k + E - 1) / E : 0;
  if (avg <= 32) return 32;
  if (avg <= 64) return 64;
  return 128;
}

// Rows per block of the align padding.  block_m != 0 is the caller's choice,
// used by both stages.  0: pick_bm's size, except that 128 becomes 256 when
// experts hold >= 192 routed rows on average and H is a multiple of 256: then
// both stages run 256-row items for every format, measured faster on each.
// (Built with MOE_S2_F16_256=0, fp16 Stage 2 keeps 128-row paired items over
// the 256-row padding; those that fall in a block's empty second half end at
// once.)  At fewer rows per expert half-empty 256-row blocks cost more than
// they save.
int64_t align_bm(int64_t T, int64_t E, int64_t k, int64_t H, int64_t block_m) {
  if (block_m) return block_m;
  const int64_t bm = pick_bm(T, E, k);
  if (bm != 128 || H % 256) return bm;
  const int64_t avg = (T * k + E - 1) / E;
  return avg >= 192 ? 256 : 128;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int check_dims(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int64_t bm) {
  if (T < 0 || E <= 0 || k <= 0) return fail(MOE_ERR_INVALID_ARG, "bad sizes T=%lld E=%lld k=%lld", (long long)T, (long long)E, (long long)k);
  if (k > E || k > 32) return fail(MOE_ERR_UNSUPPORTED, "top_k=%lld must be <= min(E, 32)", (long long)k);
  if (E > 1024) return fail(MOE_ERR_UNSUPPORTED, "E=%lld > 1024", (long long)E);
  if (H <= 0 || I <= 0 || H % 128 || I % 128) return fail(MOE_ERR_UNSUPPORTED, "H=%lld and I=%lld must be positive multiples of 128", (long long)H, (long long)I);
  if (bm != 32 && bm != 64 && bm != 128 && bm != 256) return fail(MOE_ERR_UNSUPPORTED, "block_m=%lld not in {32,64,128}", (long long)bm);
  if (cap_rows(T, k, E, bm) * I >= ((int64_t)1 << 31) * 2 || T * k >= ((int64_t)1 << 31)) return fail(MOE_ERR_UNSUPPORTED, "problem too large for 32-bit row indices");
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_version(void) { return 1; }

const char* moe_last_error_string(void) { return g_err; }

int64_t moe_prerouted_workspace_bytes(int64_t P, int64_t I) { return P > 0 && I > 0 ? P * I * 2 : 0; }

int moe_run_prerouted_events(const void* x, const void* w_gate, const void* w_up, const void* w_down,
                             const void* routed, int routed_dtype, const int32_t* group_sizes,
                             const int32_t* group_offsets, const int32_t* group_padded_offsets,
                             const int32_t* group_idx_for_bx, void* out, int64_t P, int64_t H, int64_t I,
                             int64_t E, int64_t V, int64_t nblk, void* workspace, int64_t workspace_bytes,
                             void* stream, void* const* stage_events) {
  if (P < 0 || H <= 0 || I <= 0 || E <= 0 || V < 0 || nblk < 0)
    return fail(MOE_ERR_INVALID_ARG, "bad sizes P=%lld H=%lld I=%lld E=%lld V=%lld", (long long)P, (long long)H, (long long)I, (long long)E, (long long)V);
  if (P == 0) return MOE_OK;  // nothing to write (submission.py:2117-2120)
  if (H % 128 || I % 128 || P % 128)
    return fail(MOE_ERR_UNSUPPORTED, "H=%lld, I=%lld and P=%lld must be multiples of 128", (long long)H, (long long)I, (long long)P);
  if (E > 65536) return fail(MOE_ERR_UNSUPPORTED, "E=%lld too large", (long long)E);
  if (P * (H > I ? H : I) >= ((int64_t)1 << 40)) return fail(MOE_ERR_UNSUPPORTED, "problem too large");
  if (routed_dtype != MOE_ROUTED_F32 && routed_dtype != MOE_ROUTED_F16)
    return fail(MOE_ERR_INVALID_ARG, "routed_dtype=%d", routed_dtype);
  if (!x || !w_gate || !w_up || !w_down || !group_sizes || !group_offsets || !group_padded_offsets || !out || (V > 0 && !routed) ||
      (nblk > 0 && !group_idx_for_bx))
    return fail(MOE_ERR_INVALID_ARG, "null pointer argument");
  if (!aligned16(x) || !aligned16(w_gate) || !aligned16(w_up) || !aligned16(w_down) || !aligned16(out) || !aligned16(workspace))
    return fail(MOE_ERR_INVALID_ARG, "x, weights, out and workspace must be 16-byte aligned");
  if (workspace_bytes < moe_prerouted_workspace_bytes(P, I) || !workspace)
    return fail(MOE_ERR_WORKSPACE, "workspace %lld < %lld bytes", (long long)workspace_bytes, (long long)moe_prerouted_workspace_bytes(P, I));
  hipStream_t s = (hipStream_t)stream;
  // Block b (rows [128 b, 128 b + 128)) belongs to expert group_idx_for_bx[b];
  // the launch covers the gidx entries, as submission.py:2115 launches
  // group_idx_for_bx.numel() blocks (rows past them are left untouched), and
  // never more blocks than x, out and the workspace hold.
  const int64_t blocks = nblk < P / 128 ? nblk : P / 128;
  if (blocks == 0) return MOE_OK;

  moe::Stage1Params p1{};
  p1.x = (const char*)x;
  p1.wg = (const char*)w_gate;
  p1.wu = (const char*)w_up;
  p1.h = (char*)workspace;
  p1.gs = group_sizes;
  p1.gpo = group_padded_offsets;
  p1.gidx = group_idx_for_bx;
  p1.topk = 1;
  p1.E = (int)E;
  p1.H = H;
  p1.I = I;
  p1.absorb = 2;  // absorbed rows, pairs kept: few items here (moe_common.h kAbsorbRows)
  // optional stage markers: ev[0] start, [1] stage 1, [2] stage 2
  auto mark = [&](int i) { if (stage_events && stage_events[i]) (void)hipEventRecord((hipEvent_t)stage_events[i], s); };
  mark(0);
  int rc = check_launch(moe::launch_stage1(p1, 128, moe::kQF16, false, blocks, s), "stage1");
  if (rc) return rc;
  mark(1);

  moe::Stage2Params p2{};
  p2.a = (const char*)workspace;
  p2.wd = (const char*)w_down;
  p2.out = (char*)out;
  p2.routed = routed;
  p2.routed_f16 = routed_dtype == MOE_ROUTED_F16;
  p2.gs = group_sizes;
  p2.go = group_offsets;
  p2.gpo = group_padded_offsets;
  p2.gidx = group_idx_for_bx;
  p2.E = (int)E;
  p2.H = H;
  p2.I = I;
  p2.V = V;
  p2.absorb = 2;  // as in Stage 1
  rc = check_launch(moe::launch_stage2(p2, 128, moe::kQF16, false, blocks, s), "stage2");
  mark(2);
  return rc;
}

int moe_run_prerouted(const void* x, const void* w_gate, const void* w_up, const void* w_down,
                      const void* routed, int routed_dtype, const int32_t* group_sizes,
                      const int32_t* group_offsets, const int32_t* group_padded_offsets,
                      const int32_t* group_idx_for_bx, void* out, int64_t P, int64_t H, int64_t I,
                      int64_t E, int64_t V, int64_t nblk, void* workspace, int64_t workspace_bytes,
                      void* stream) {
  return moe_run_prerouted_events(x, w_gate, w_up, w_down, routed, routed_dtype, group_sizes, group_offsets,
                                  group_padded_offsets, group_idx_for_bx, out, P, H, I, E, V, nblk, workspace,
                                  workspace_bytes, stream, nullptr);
}

int moe_route_topk(const float* logits, const float* bias, int64_t T, int64_t E, int64_t k,
                   int32_t* topk_ids, float* topk_weights, void* stream) {
  if (T < 0 || E <= 0 || k <= 0) return fail(MOE_ERR_INVALID_ARG, "bad sizes T=%lld E=%lld k=%lld", (long long)T, (long long)E, (long long)k);
  if (E > 1024 || k > 32 || k > E) return fail(MOE_ERR_UNSUPPORTED, "need E <= 1024 and k <= min(E, 32)");
  if (T == 0) return MOE_OK;
  if (!logits || !topk_ids || !topk_weights) return fail(MOE_ERR_INVALID_ARG, "null pointer argument");
  return check_launch(moe::launch_route_topk(logits, bias, (int)T, (int)E, (int)k, topk_ids, topk_weights, (hipStream_t)stream), "route_topk");
}

int64_t moe_router_workspace_bytes(int64_t T, int64_t H, int64_t E) {
  if (T < 0 || H <= 0 || E <= 0 || H % 128) return 0;
  return up(moe::router_partial_floats(T, H, E) * 4);
}

static int check_router(const void* x, const void* w_router, int64_t T, int64_t H, int64_t E, int64_t k) {
  if (T < 0 || H <= 0 || E <= 0 || k <= 0) return fail(MOE_ERR_INVALID_ARG, "bad sizes T=%lld H=%lld E=%lld k=%lld", (long long)T, (long long)H, (long long)E, (long long)k);
  if (H % 128) return fail(MOE_ERR_UNSUPPORTED, "H=%lld must be a multiple of 128", (long long)H);
  if (E > 1024 || k > 32 || k > E) return fail(MOE_ERR_UNSUPPORTED, "need E <= 1024 and k <= min(E, 32)");
  if (T * E >= ((int64_t)1 << 31)) return fail(MOE_ERR_UNSUPPORTED, "T*E too large");
  if (T > 0 && (!x || !w_router)) return fail(MOE_ERR_INVALID_ARG, "null pointer argument");
  if (T > 0 && (!aligned16(x) || !aligned16(w_router))) return fail(MOE_ERR_INVALID_ARG, "x and w_router must be 16-byte aligned");
  return MOE_OK;
}

int moe_route_hidden(const void* x, const void* w_router, const float* bias, int64_t T, int64_t H, int64_t E,
                     int64_t k, int32_t* topk_ids, float* topk_weights, float* logits_out, void* workspace,
                     int64_t workspace_bytes, void* stream) {
  int rc = check_router(x, w_router, T, H, E, k);
  if (rc) return rc;
  if (T == 0) return MOE_OK;
  if (!topk_ids || !topk_weights || !workspace) return fail(MOE_ERR_INVALID_ARG, "null pointer argument");
  if (workspace_bytes < moe_router_workspace_bytes(T, H, E)) return fail(MOE_ERR_WORKSPACE, "workspace %lld < %lld bytes", (long long)workspace_bytes, (long long)moe_router_workspace_bytes(T, H, E));
  return check_launch(moe::launch_router(x, w_router, bias, (int)T, H, (int)E, (int)k, topk_ids, topk_weights, logits_out, (float*)workspace, (hipStream_t)stream), "router");
}

int64_t moe_align_capacity_rows(int64_t T, int64_t k, int64_t E, int64_t block_m) {
  if (T < 0 || k <= 0 || E <= 0 || block_m <= 0) return 0;
  return cap_rows(T, k, E, block_m);
}

int64_t moe_align_scratch_bytes(int64_t T, int64_t k, int64_t E) {
  if (T < 0 || k <= 0 || E <= 0 || T * k >= ((int64_t)1 << 30)) return 0;
  return (int64_t)moe::align_groups((int)(T * k)) * E * 4;
}

int moe_align(const int32_t* topk_ids, int64_t T, int64_t k, int64_t E, int64_t block_m,
              int32_t* sorted_pair_ids, int32_t* block_expert, int32_t* group_sizes,
              int32_t* group_offsets, int32_t* group_padded_offsets, void* scratch,
              int64_t scratch_bytes, void* stream) {
  if (T < 0 || k <= 0 || E <= 0 || block_m <= 0) return fail(MOE_ERR_INVALID_ARG, "bad sizes");
  if (E > 1024) return fail(MOE_ERR_UNSUPPORTED, "E=%lld > 1024", (long long)E);
  if (T * k >= ((int64_t)1 << 30)) return fail(MOE_ERR_UNSUPPORTED, "too many pairs");
  if ((T > 0 && (!topk_ids || !sorted_pair_ids || !block_expert)) || !group_sizes || !group_offsets || !group_padded_offsets)
    return fail(MOE_ERR_INVALID_ARG, "null pointer argument");
  int32_t* whist = nullptr;
  if (scratch && scratch_bytes > 0) {
    if (scratch_bytes < moe_align_scratch_bytes(T, k, E)) return fail(MOE_ERR_WORKSPACE, "align scratch %lld < %lld bytes", (long long)scratch_bytes, (long long)moe_align_scratch_bytes(T, k, E));
    if (!aligned16(scratch)) return fail(MOE_ERR_INVALID_ARG, "align scratch must be 16-byte aligned");
    whist = (int32_t*)scratch;
  }
  return check_launch(moe::launch_align(topk_ids, (int)(T * k), (int)E, (int)block_m, sorted_pair_ids, block_expert, group_sizes, group_offsets, group_padded_offsets, whist, (hipStream_t)stream), "align");
}

int64_t moe_pick_block_m(int64_t T, int64_t E, int64_t k) { return pick_bm(T, E, k); }

int64_t moe_fused_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                                  int64_t block_m, int w8a8) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  // w8a8: 0 fp16, 1 int8, 2 fp8 (one padding rule for all)
  if (w8a8 < 0 || w8a8 > 2) return 0;
  block_m = align_bm(T, E, k, H, block_m);
  return fused_layout(T, H, I, E, k, block_m, w8a8 == 2 ? moe::kQF8 : (w8a8 ? moe::kQI8 : moe::kQF16)).total;
}

// The always-on shared expert (wg_s / wu_s / wd_s non-null, fp16 only) runs as
// expert E: every token takes it as choice k with weight 1, so the pipeline
// works on E + 1 experts and k + 1 choices and the combine adds it last.
// ids_in / w_in (both non-null): the routing is given, int32 [T, k] ids and
// fp32 [T, k] weights, instead of computed from logits or the router weight;
// choices whose id lies outside [e_begin, e_begin + E) add nothing.
static int fused_common(int qt, const void* x, const float* logits, const void* w_router, const float* bias,
                        const void* wg, const float* sg, const void* wu, const float* su,
                        const void* wd, const float* sd, const void* wg_s, const void* wu_s,
                        const void* wd_s, const int64_t* wstr, int64_t e_begin, int64_t E_route,
                        void* out, int64_t T, int64_t H,
                        int64_t I, int64_t E, int64_t k, int64_t block_m, void* workspace,
                        int64_t workspace_bytes, int32_t* ids_out, float* w_out, void* stream,
                        void* const* ev, const int32_t* ids_in = nullptr, const float* w_in = nullptr) {
  const bool w8 = qt != moe::kQF16;  // 8-bit operands: int8 or fp8
  const bool given = ids_in || w_in;  // routing given by the caller
  // expert shard: routing over E_route experts, this call's weights hold
  // experts [e_begin, e_begin + E); only their pairs are computed and summed
  const bool shard = E_route > 0;
  if (!shard) E_route = E;
  if (shard && (e_begin < 0 || E <= 0 || e_begin + E > E_route || w_router || wg_s || wu_s || wd_s))
    return fail(MOE_ERR_INVALID_ARG, "expert shard [%lld, %lld) of %lld experts (logits only, no shared expert)",
                (long long)e_begin, (long long)(e_begin + E), (long long)E_route);
  if (given && (!shard || logits || !ids_in || !w_in))
    return fail(MOE_ERR_INVALID_ARG, "a given routing takes ids and weights, no logits, and an expert range");
  const bool shared = wg_s || wu_s || wd_s;
  if (shared && (w8 || !wg_s || !wu_s || !wd_s))
    return fail(w8 ? MOE_ERR_UNSUPPORTED : MOE_ERR_INVALID_ARG, w8 ? "the shared expert is supported on the fp16 path" : "null pointer argument");
  const int64_t Ee = E + (shared ? 1 : 0), ke = k + (shared ? 1 : 0);  // experts / choices incl. the shared one
  if (block_m != 0 && block_m != 32 && block_m != 64 && block_m != 128)
    return fail(MOE_ERR_UNSUPPORTED, "block_m=%lld not in {0,32,64,128}", (long long)block_m);
  block_m = align_bm(T, shard ? E_route : Ee, ke, H, block_m);
  int rc = check_dims(T, H, I, shard ? E_route : Ee, ke, block_m);
  if (rc) return rc;
  if (T == 0) return MOE_OK;
  if (!x || (!logits && !w_router && !given) || !wg || !wu || !wd || !out || !workspace || (w8 && (!sg || !su || !sd)))
    return fail(MOE_ERR_INVALID_ARG, "null pointer argument");
  if (w_router && (rc = check_router(x, w_router, T, H, E, k))) return rc;
  // weight strides in elements, {row, expert} of gate/up then of down (null
  // or 0: dense); rows must not overlap and stay 16-byte aligned
  const int64_t eb = w8 ? 1 : 2;
  int64_t ld_gu = wstr ? wstr[0] : 0, es_gu = wstr ? wstr[1] : 0, ld_d = wstr ? wstr[2] : 0, es_d = wstr ? wstr[3] : 0;
  ld_gu = ld_gu ? ld_gu : H;
  ld_d = ld_d ? ld_d : I;
  es_gu = es_gu ? es_gu : I * ld_gu;
  es_d = es_d ? es_d : H * ld_d;
  if (ld_gu < H || ld_d < I || es_gu < I * ld_gu || es_d < H * ld_d || (ld_gu | es_gu | ld_d | es_d) * eb % 16)
    return fail(MOE_ERR_INVALID_ARG, "weight strides (rows %lld / %lld, experts %lld / %lld) must not overlap rows and must keep 16-byte alignment",
                (long long)ld_gu, (long long)ld_d, (long long)es_gu, (long long)es_d);
  if (!aligned16(x) || !aligned16(wg) || !aligned16(wu) || !aligned16(wd) || !aligned16(out) || !aligned16(workspace) || (w8 && (!aligned16(sg) || !aligned16(su) || !aligned16(sd))) ||
      (shared && (!aligned16(wg_s) || !aligned16(wu_s) || !aligned16(wd_s))))
    return fail(MOE_ERR_INVALID_ARG, "x, weights, scales, out and workspace must be 16-byte aligned");
  const int64_t router_ws = w_router ? moe_router_workspace_bytes(T, H, E) : 0;
  // a workspace sized for the 128-row padding (block_m = 128) keeps it
  if (block_m == 256 && workspace_bytes < fused_layout(T, H, I, Ee, ke, 256, qt).total + router_ws) block_m = 128;
  const FusedLayout L = fused_layout(T, H, I, Ee, ke, block_m, qt);
  const int64_t need = L.total + router_ws;
  if (workspace_bytes < need) return fail(MOE_ERR_WORKSPACE, "workspace %lld < %lld bytes", (long long)workspace_bytes, (long long)need);
  // rows per item of each stage: block_m for both stages and every format
  // (over the 256-row padding, 256-row items), unless built with
  // MOE_S2_F16_256=0, where fp16 Stage 2 keeps 128-row paired items there
  const int64_t bm1 = block_m;
  const int64_t bm2 = block_m == 256 && qt == moe::kQF16 && MOE_S2_F16_256 == 0 ? 128 : block_m;
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  // routing written by route / router (ids, wts), read by align, Stage 2 and the combine (rids, rwts)
  int32_t* ids = ids_out ? ids_out : (int32_t*)(ws + L.ids);
  float* wts = w_out ? w_out : (float*)(ws + L.w);
  const int32_t* rids = given ? ids_in : ids;
  const float* rwts = given ? w_in : wts;
  int32_t* sorted = (int32_t*)(ws + L.sorted);
  int32_t* gs = (int32_t*)(ws + L.gs);
  int32_t* go = (int32_t*)(ws + L.go);
  int32_t* gpo = (int32_t*)(ws + L.gpo);
  const int64_t rows = cap_rows(T, ke, Ee, block_m);
  const int e_shared = shared ? (int)E : -1;

  // optional stage markers: ev[0] start, [1] routed, [2] aligned, [3] x quantised,
  // [4] stage 1, [5] stage 2, [6] combined
  auto mark = [&](int i) { if (ev && ev[i]) (void)hipEventRecord((hipEvent_t)ev[i], s); };
  mark(0);
  // 8-bit operands from logits: the routing and the per-token quantisation of
  // x run as one launch (route_quant_kernel)
  const bool route_quant = w8 && !given && !w_router;
  if (given) {
    // routed by the caller: nothing to launch (ids and weights are only read)
  } else if (route_quant) {
    if ((rc = check_launch(moe::launch_route_quant(logits, bias, (int)T, (int)E_route, (int)k, ids, wts, x, H,
                                                   ws + L.xq, (float*)(ws + L.sx), qt, s), "route_quantize_x")))
      return rc;
  } else if (w_router) {  // router GEMM + routing; its partial sums sit after the fused workspace
    if ((rc = check_launch(moe::launch_router(x, w_router, bias, (int)T, H, (int)E, (int)k, ids, wts, nullptr, (float*)(ws + L.total), s, e_shared), "router"))) return rc;
  } else if ((rc = check_launch(moe::launch_route_topk(logits, bias, (int)T, (int)E_route, (int)k, ids, wts, s, e_shared), "route_topk"))) {
    return rc;
  }
  mark(1);
  if ((rc = check_launch(moe::launch_align(rids, (int)(T * ke), (int)Ee, (int)block_m, sorted, (int32_t*)(ws + L.bexp), gs, go, gpo, (int32_t*)(ws + L.whist), s, (int)e_begin), "align"))) return rc;
  mark(2);
  if (w8 && !route_quant && (rc = check_launch(moe::launch_quant_rows(x, T, H, ws + L.xq, (float*)(ws + L.sx), qt, s), "quantize_x"))) return rc;
  mark(3);

  moe::Stage1Params p1{};
  p1.x = w8 ? (const char*)(ws + L.xq) : (const char*)x;
  p1.wg = (const char*)wg;
  p1.wu = (const char*)wu;
  p1.h = ws + L.h;
  p1.h_scale = qt == moe::kQF8 ? (float*)(ws + L.hs) : nullptr;
  p1.hs_stride = rows;
  p1.x_scale = w8 ? (const float*)(ws + L.sx) : nullptr;
  p1.sg = sg;
  p1.su = su;
  p1.gs = gs;
  p1.gpo = gpo;
  p1.sorted_ids = sorted;
  p1.wg_shared = (const char*)wg_s;
  p1.wu_shared = (const char*)wu_s;
  p1.e_shared = e_shared;
  p1.w_ld = ld_gu * eb;
  p1.w_es = es_gu * eb;
  p1.topk = (int)ke;
  p1.E = (int)Ee;
  p1.H = H;
  p1.I = I;
  p1.absorb = 1;  // absorbed rows, pairs may become single items (moe_common.h kAbsorbRows)
  if ((rc = check_launch(moe::launch_stage1(p1, (int)bm1, qt, true, rows / bm1, s), "stage1"))) return rc;
  // int8: h (fp16) -> per-row int8 codes + scales, for the routed rows only
  // (sorted id below the sentinel T * ke, row below gpo[E])
  if (qt == moe::kQI8 &&
      (rc = check_launch(moe::launch_quant_rows(ws + L.h, rows, I, ws + L.hq, (float*)(ws + L.hs), moe::kQI8, s,
                                                sorted, (int32_t)(T * ke), gpo + Ee), "quantize_h")))
    return rc;
  mark(4);

  moe::Stage2Params p2{};
  p2.a = qt == moe::kQI8 ? ws + L.hq : ws + L.h;
  p2.a_scale = w8 ? (const float*)(ws + L.hs) : nullptr;
  p2.as_stride = rows;
  p2.wd = (const char*)wd;
  p2.sd = sd;
  p2.out = MOE_S2_SCATTER ? (char*)out : ws + L.ypair;
  p2.topk = (int)ke;
  p2.pos = (int32_t*)(ws + L.pos);
  p2.absorb = 1;  // as in Stage 1
  p2.routed = rwts;
  p2.routed_f16 = 0;
  p2.gs = gs;
  p2.go = go;
  p2.gpo = gpo;
  p2.sorted_ids = sorted;
  p2.wd_shared = (const char*)wd_s;
  p2.e_shared = e_shared;
  p2.wd_ld = ld_d * eb;
  p2.wd_es = es_d * eb;
  p2.E = (int)Ee;
  p2.H = H;
  p2.I = I;
  if (MOE_S2_SCATTER && (rc = check_launch(moe::launch_zero(out, T * H * 2, s), "zero_out"))) return rc;
  if ((rc = check_launch(moe::launch_stage2(p2, (int)bm2, qt, true, rows / bm2, s), "stage2"))) return rc;
  mark(5);
  if (MOE_S2_SCATTER) {  // Stage 2 added every pair row into `out`
    mark(6);
    return MOE_OK;
  }
  rc = check_launch(moe::launch_combine(ws + L.ypair, (const int32_t*)(ws + L.pos), T, H, (int)ke, out, s,
                                        shard ? rids : nullptr, (int)e_begin, (int)E),
                    "combine");
  mark(6);
  return rc;
}

int moe_fused_forward(const void* x, const float* logits, const float* bias, const void* w_gate,
                      const void* w_up, const void* w_down, void* out, int64_t T, int64_t H,
                      int64_t I, int64_t E, int64_t k, int64_t block_m, void* workspace,
                      int64_t workspace_bytes, int32_t* topk_ids_out, float* topk_weights_out,
                      void* stream) {
  return fused_common(moe::kQF16, x, logits, nullptr, bias, w_gate, nullptr, w_up, nullptr, w_down, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, out,
                      T, H, I, E, k, block_m, workspace, workspace_bytes, topk_ids_out,
                      topk_weights_out, stream, nullptr);
}

int64_t moe_fused_hidden_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                                         int64_t block_m) {
  const int64_t f = moe_fused_workspace_bytes(T, H, I, E, k, block_m, 0);
  return f ? f + moe_router_workspace_bytes(T, H, E) : 0;
}

int moe_fused_forward_hidden(const void* x, const void* w_router, const float* bias, const void* w_gate,
                             const void* w_up, const void* w_down, void* out, int64_t T, int64_t H,
                             int64_t I, int64_t E, int64_t k, int64_t block_m, void* workspace,
                             int64_t workspace_bytes, int32_t* topk_ids_out, float* topk_weights_out,
                             void* stream) {
  if (!w_router && T > 0) return fail(MOE_ERR_INVALID_ARG, "null pointer argument");
  return fused_common(moe::kQF16, x, nullptr, w_router, bias, w_gate, nullptr, w_up, nullptr, w_down, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, out,
                      T, H, I, E, k, block_m, workspace, workspace_bytes, topk_ids_out,
                      topk_weights_out, stream, nullptr);
}

int64_t moe_fused_shared_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                                         int64_t block_m) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  block_m = align_bm(T, E + 1, k + 1, H, block_m);
  return fused_layout(T, H, I, E + 1, k + 1, block_m, moe::kQF16).total + moe_router_workspace_bytes(T, H, E);
}

int moe_fused_forward_shared(const void* x, const float* logits, const void* w_router, const float* bias,
                             const void* w_gate, const void* w_up, const void* w_down, const void* w_gate_shared,
                             const void* w_up_shared, const void* w_down_shared, void* out, int64_t T,
                             int64_t H, int64_t I, int64_t E, int64_t k, int64_t block_m, void* workspace,
                             int64_t workspace_bytes, int32_t* topk_ids_out, float* topk_weights_out,
                             void* stream) {
  if (T > 0 && (!logits) == (!w_router)) return fail(MOE_ERR_INVALID_ARG, "give exactly one of logits and w_router");
  if (T > 0 && (!w_gate_shared || !w_up_shared || !w_down_shared)) return fail(MOE_ERR_INVALID_ARG, "null pointer argument");
  return fused_common(moe::kQF16, x, logits, w_router, bias, w_gate, nullptr, w_up, nullptr, w_down, nullptr,
                      w_gate_shared, w_up_shared, w_down_shared, nullptr, 0, 0, out, T, H, I, E, k, block_m, workspace,
                      workspace_bytes, topk_ids_out, topk_weights_out, stream, nullptr);
}

int64_t moe_fused_ex_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int64_t block_m,
                                     int shared, int with_router) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  const int64_t s = shared ? 1 : 0;
  block_m = align_bm(T, E + s, k + s, H, block_m);
  return fused_layout(T, H, I, E + s, k + s, block_m, moe::kQF16).total + (with_router ? moe_router_workspace_bytes(T, H, E) : 0);
}

int moe_fused_forward_ex(const void* x, const float* logits, const void* w_router, const float* bias,
                         const void* w_gate, const void* w_up, const void* w_down, const void* w_gate_shared,
                         const void* w_up_shared, const void* w_down_shared, const int64_t* weight_strides,
                         void* out, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int64_t block_m,
                         void* workspace, int64_t workspace_bytes, int32_t* topk_ids_out,
                         float* topk_weights_out, void* stream, void* const* stage_events) {
  if (T > 0 && (!logits) == (!w_router)) return fail(MOE_ERR_INVALID_ARG, "give exactly one of logits and w_router");
  const bool any = w_gate_shared || w_up_shared || w_down_shared;
  if (T > 0 && any && !(w_gate_shared && w_up_shared && w_down_shared)) return fail(MOE_ERR_INVALID_ARG, "null pointer argument");
  return fused_common(moe::kQF16, x, logits, w_router, bias, w_gate, nullptr, w_up, nullptr, w_down, nullptr,
                      w_gate_shared, w_up_shared, w_down_shared, weight_strides, 0, 0, out, T, H, I, E, k, block_m,
                      workspace, workspace_bytes, topk_ids_out, topk_weights_out, stream, stage_events);
}

int64_t moe_fused_shard_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E_total, int64_t k,
                                        int64_t E_local, int64_t block_m) {
  if (T < 0 || H <= 0 || I <= 0 || E_total <= 0 || E_local <= 0 || k <= 0) return 0;
  block_m = align_bm(T, E_total, k, H, block_m);
  return fused_layout(T, H, I, E_local, k, block_m, moe::kQF16).total;
}

int moe_fused_forward_shard(const void* x, const float* logits, const float* bias, const void* w_gate,
                            const void* w_up, const void* w_down, void* out, int64_t T, int64_t H, int64_t I,
                            int64_t E_total, int64_t k, int64_t expert_begin, int64_t E_local, int64_t block_m,
                            void* workspace, int64_t workspace_bytes, int32_t* topk_ids_out,
                            float* topk_weights_out, void* stream, void* const* stage_events) {
  if (E_total <= 0) return fail(MOE_ERR_INVALID_ARG, "E_total=%lld", (long long)E_total);
  return fused_common(moe::kQF16, x, logits, nullptr, bias, w_gate, nullptr, w_up, nullptr, w_down, nullptr, nullptr,
                      nullptr, nullptr, nullptr, expert_begin, E_total, out, T, H, I, E_local, k, block_m, workspace,
                      workspace_bytes, topk_ids_out, topk_weights_out, stream, stage_events);
}

int64_t moe_fused_routed_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E_total, int64_t k,
                                         int64_t E_local, int64_t block_m) {
  return moe_fused_shard_workspace_bytes(T, H, I, E_total, k, E_local, block_m);
}

int moe_fused_forward_routed(const void* x, const int32_t* topk_ids, const float* topk_weights, const void* w_gate,
                             const void* w_up, const void* w_down, void* out, int64_t T, int64_t H, int64_t I,
                             int64_t E_total, int64_t k, int64_t expert_begin, int64_t E_local, int64_t block_m,
                             void* workspace, int64_t workspace_bytes, void* stream, void* const* stage_events) {
  if (E_total <= 0) return fail(MOE_ERR_INVALID_ARG, "E_total=%lld", (long long)E_total);
  if (T > 0 && (!topk_ids || !topk_weights)) return fail(MOE_ERR_INVALID_ARG, "null pointer argument");
  return fused_common(moe::kQF16, x, nullptr, nullptr, nullptr, w_gate, nullptr, w_up, nullptr, w_down, nullptr,
                      nullptr, nullptr, nullptr, nullptr, expert_begin, E_total, out, T, H, I, E_local, k, block_m,
                      workspace, workspace_bytes, nullptr, nullptr, stream, stage_events, topk_ids, topk_weights);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free fused forward.  Its workspace is `scratch`, a static device
// array that every GPU the library runs on holds (one copy per device, at its
// own address) until the process ends.  Host code never uses the array's name
// as an address: at a device's first call, with that device current,
// hipGetSymbolAddress gives that device's copy, kept in g_scratch_ptr.
// Nothing in the fused workspace has to start at zero (every piece is fully
// written before it is read), so the array is never cleared; it keeps the
// last call's contents.  Calls that overlap on one GPU share the array and
// race.
// ---------------------------------------------------------------------------
namespace {
constexpr int64_t kNoAllocScratchBytes = (int64_t)64 << 20;  // 64 MiB per GPU
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

// This device's copy of `scratch` (looked up once per device).
static int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MOE_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MOE_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(MOE_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOE_OK;
}

extern "C" {

int moe_fused_forward_noalloc(const void* x, const float* logits, const float* bias, const void* w_gate,
                              const void* w_up, const void* w_down, void* out, int64_t T, int64_t H,
                              int64_t I, int64_t E, int64_t k, int64_t block_m, int32_t* topk_ids_out,
                              float* topk_weights_out, void* stream) {
  if (block_m != 0 && block_m != 32 && block_m != 64 && block_m != 128)
    return fail(MOE_ERR_UNSUPPORTED, "block_m=%lld not in {0,32,64,128}", (long long)block_m);
  int64_t bm = align_bm(T, E, k, H, block_m);
  int rc = check_dims(T, H, I, E, k, bm);
  if (rc) return rc;
  if (T == 0) return MOE_OK;
  // the padding the call will use: 256-row blocks only where they fit (as
  // for any workspace sized for 128-row blocks)
  int64_t need = fused_layout(T, H, I, E, k, bm, moe::kQF16).total;
  if (bm == 256 && need > kNoAllocScratchBytes) need = fused_layout(T, H, I, E, k, 128, moe::kQF16).total;
  if (need > kNoAllocScratchBytes)
    return fail(MOE_ERR_WORKSPACE,
                "moe_fused_forward_noalloc: T=%lld H=%lld I=%lld E=%lld k=%lld needs %lld bytes of scratch, the "
                "static scratch holds %lld; pass a workspace to moe_fused_forward instead",
                (long long)T, (long long)H, (long long)I, (long long)E, (long long)k, (long long)need,
                (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_of_current_device(&ws))) return rc;
  return fused_common(moe::kQF16, x, logits, nullptr, bias, w_gate, nullptr, w_up, nullptr, w_down, nullptr, nullptr,
                      nullptr, nullptr, nullptr, 0, 0, out, T, H, I, E, k, block_m, ws, kNoAllocScratchBytes,
                      topk_ids_out, topk_weights_out, stream, nullptr);
}

int moe_fused_forward_events(const void* x, const float* logits, const float* bias,
                             const void* w_gate, const void* w_up, const void* w_down, void* out,
                             int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                             int64_t block_m, void* workspace, int64_t workspace_bytes,
                             int32_t* topk_ids_out, float* topk_weights_out, void* stream,
                             void* const* stage_events) {
  return fused_common(moe::kQF16, x, logits, nullptr, bias, w_gate, nullptr, w_up, nullptr, w_down, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, out,
                      T, H, I, E, k, block_m, workspace, workspace_bytes, topk_ids_out,
                      topk_weights_out, stream, stage_events);
}

static int quantize_rows(const void* w, int64_t R, int64_t K, void* q, float* scale, int qt, void* stream) {
  if (R < 0 || K <= 0 || K % 8) return fail(MOE_ERR_INVALID_ARG, "need R >= 0 and K a positive multiple of 8");
  if (R == 0) return MOE_OK;
  if (!w || !q || !scale) return fail(MOE_ERR_INVALID_ARG, "null pointer argument");
  if (!aligned16(w) || ((uintptr_t)q & 7)) return fail(MOE_ERR_INVALID_ARG, "w must be 16-byte and q 8-byte aligned");
  return check_launch(moe::launch_quant_rows(w, R, K, q, scale, qt, (hipStream_t)stream), "quantize_rows");
}

int moe_quantize_rows_w8(const void* w, int64_t R, int64_t K, int8_t* q, float* scale,
                         void* stream) {
  return quantize_rows(w, R, K, q, scale, moe::kQI8, stream);
}

int moe_quantize_rows_fp8(const void* w, int64_t R, int64_t K, uint8_t* q, float* scale,
                          void* stream) {
  return quantize_rows(w, R, K, q, scale, moe::kQF8, stream);
}

int moe_fused_forward_fp8(const void* x, const float* logits, const float* bias,
                          const uint8_t* wq_gate, const float* s_gate, const uint8_t* wq_up,
                          const float* s_up, const uint8_t* wq_down, const float* s_down,
                          void* out, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                          int64_t block_m, void* workspace, int64_t workspace_bytes,
                          int32_t* topk_ids_out, float* topk_weights_out, void* stream,
                          void* const* stage_events) {
  return fused_common(moe::kQF8, x, logits, nullptr, bias, wq_gate, s_gate, wq_up, s_up, wq_down, s_down, nullptr,
                      nullptr, nullptr, nullptr, 0, 0, out, T, H, I, E, k, block_m, workspace, workspace_bytes,
                      topk_ids_out, topk_weights_out, stream, stage_events);
}

int moe_fused_forward_w8a8(const void* x, const float* logits, const float* bias,
                           const int8_t* wq_gate, const float* s_gate, const int8_t* wq_up,
                           const float* s_up, const int8_t* wq_down, const float* s_down,
                           void* out, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                           int64_t block_m, void* workspace, int64_t workspace_bytes,
                           int32_t* topk_ids_out, float* topk_weights_out, void* stream) {
  return fused_common(moe::kQI8, x, logits, nullptr, bias, wq_gate, s_gate, wq_up, s_up, wq_down, s_down, nullptr, nullptr, nullptr, nullptr, 0, 0, out,
                      T, H, I, E, k, block_m, workspace, workspace_bytes, topk_ids_out,
                      topk_weights_out, stream, nullptr);
}

int moe_fused_forward_w8a8_events(const void* x, const float* logits, const float* bias,
                                  const int8_t* wq_gate, const float* s_gate, const int8_t* wq_up,
                                  const float* s_up, const int8_t* wq_down, const float* s_down,
                                  void* out, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                                  int64_t block_m, void* workspace, int64_t workspace_bytes,
                                  int32_t* topk_ids_out, float* topk_weights_out, void* stream,
                                  void* const* stage_events) {
  return fused_common(moe::kQI8, x, logits, nullptr, bias, wq_gate, s_gate, wq_up, s_up, wq_down, s_down, nullptr, nullptr, nullptr, nullptr, 0, 0, out,
                      T, H, I, E, k, block_m, workspace, workspace_bytes, topk_ids_out,
                      topk_weights_out, stream, stage_events);
}

}  // extern "C"
