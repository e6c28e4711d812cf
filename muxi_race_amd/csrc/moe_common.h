// Shared device-side building blocks for the gfx950 fused-MoE kernels.
//
// Tile geometry.  Every GEMM operand tile is a stack of rows that are
// contiguous along K in global memory (token rows of x / the intermediate,
// output-feature rows of the expert weights).  One K step moves 128 bytes of
// each row (64 fp16 or 128 int8 elements) = eight 16-byte chunks.  In LDS a
// row occupies 128 bytes and chunk c of row r sits at chunk slot
// c ^ swz(r), so the 32 rows read by one MFMA fragment load spread over the
// banks.  One MFMA K sub-step consumes two chunks per row (lanes 0-31 the
// first, lanes 32-63 the second), i.e. 16 fp16 or 32 int8 per row.
//
// MFMA roles.  D[n][m] = sum_k W[n][k] * X[m][k]: the weight tile is the A
// operand (32 output features per MFMA block) and the token tile the B
// operand (32 tokens).  In the 32x32 accumulator lane l holds token
// m = l % 32 and features n = 8*(r/4) + 4*(l/32) + r%4 for register r, so each
// lane owns runs of 4 consecutive output features of one token row: the
// epilogues store 8-byte (fp16) or 4-byte (int8) vectors.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kRowBytes = 128;     // bytes of one tile row per K step
constexpr int kBN = 128;           // output-feature tile (N) of every GEMM
constexpr int kNumXcd = 8;         // MI355X: 8 XCDs, workgroups dealt round-robin
constexpr float kLog2e = 1.44269504088896341f;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// LDS byte offset of 16-byte chunk c of tile row r.  gfx950 serves a
// ds_read_b128 16 lanes at a time across 64 four-byte banks: a fragment read
// (16 consecutive rows, one chunk) is conflict-free when the 16 (row parity,
// chunk slot) pairs are distinct, i.e. when the slot is c ^ f(r) with f taking
// 8 distinct values over the even rows and over the odd rows of any 16-row
// group.  f(r) = (r >> 1) & 7 does that (f(r) = r & 7 puts rows r and r + 8 on
// the same banks: a 2-way conflict on every read, measured).
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int lds_swz(int r, int c) {
  return (r << 7) | (((c ^ swz(r)) & 7) << 4);
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Pipelines issue Q loads per wave per stage, in stage order, and vector-memory
// loads retire in order: waiting until at most Q*min(ahead, N) loads are
// outstanding completes every stage but the last min(ahead, N) issued.
template <int Q, int N>
__device__ __forceinline__ void wait_stages(int ahead) {
  if constexpr (N <= 0) {
    wait_vmcnt<0>();
  } else {
    if (ahead >= N) wait_vmcnt<Q * N>();
    else wait_stages<Q, N - 1>(ahead);
  }
}

// s_waitcnt vmcnt(n) for a wave-uniform n known only at run time: the
// immediate is picked by scalar branches; n above MAX waits for MAX instead
// (a stricter wait).
template <int MAX>
__device__ __forceinline__ void wait_vmcnt_rt(int n) {
  if constexpr (MAX <= 0) {
    wait_vmcnt<0>();
  } else {
    if (n >= MAX) wait_vmcnt<MAX>();
    else wait_vmcnt_rt<MAX - 1>(n);
  }
}

// wait_stages for waves that issue q <= Q loads per stage (q wave-uniform,
// the same for every stage of the wave).
template <int Q, int N>
__device__ __forceinline__ void wait_stages_q(int q, int ahead) {
  if constexpr (N <= 0) {
    wait_vmcnt<0>();
  } else {
    if (ahead >= N) wait_vmcnt_rt<Q * N>(q * N);
    else wait_stages_q<Q, N - 1>(q, ahead);
  }
}

// Workgroup barrier without a memory fence.  __syncthreads() would first wait
// for every outstanding vector-memory operation (vmcnt(0)), which includes the
// direct-to-LDS loads of the stages still in flight; the pipelines below wait
// for exactly the stage they consume (wait_vmcnt) and then use this barrier.
// The empty asm statements keep the compiler from moving memory accesses
// across it.
__device__ __forceinline__ void barrier_no_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

#define MOE_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// Cache policy of weight loads that no other tile repeats, used by the
// decode-sized (32-row) kernels.  A weight tile read by exactly one item is
// loaded non-temporal (the gfx950 `nt` bit, cache-policy immediate 2):
// decode went from 0.575 to 0.533 ms with it (a load-only copy of the 96-row
// decode ring streamed 6.15 -> 7.12 TB/s at rows 14 KiB apart, 5.45 -> 6.14
// TB/s at 4 KiB).  Weight tiles that sibling items of a multi-block
// expert re-read from L2, and token / intermediate rows, keep the default
// policy (non-temporal there measured slower: fewer L2 hits).  Of the
// wide-tile kernels, only the 8-bit 256-row items stream their unshared
// weight tiles (MOE_W8_STREAM in grouped_gemm.hip, measured faster there);
// the fp16 ones load everything with the default policy (no gain measured,
// and the per-instruction choice cost 2-5%).  0 turns streaming off.
#ifndef MOE_W_POLICY
#define MOE_W_POLICY 2
#endif
constexpr int kPolicyDefault = 0;
constexpr int kPolicyWeights = MOE_W_POLICY;
constexpr int kNoStream = 1 << 30;  // `weights_from` that streams no row

// global_load_lds_dword[x4]: per-lane global address -> LDS at m0 + 4|16 * lane,
// cache policy POLICY.  The host compilation pass only needs kernel
// signatures (for the launch stubs); the builtin is kept out of that pass,
// where clang's deferred diagnostic for it otherwise stops the remaining
// kernel stubs from being emitted.
template <int BYTES, int POLICY = kPolicyDefault>
__device__ __forceinline__ void dma_to_lds(const void* g, void* lds) {
  static_assert(BYTES == 4 || BYTES == 16, "dword or dwordx4");
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (BYTES == 16)
    __builtin_amdgcn_global_load_lds(g, MOE_LDS_PTR(lds), 16, 0, POLICY);
  else
    __builtin_amdgcn_global_load_lds(g, MOE_LDS_PTR(lds), 4, 0, POLICY);
#else
  (void)g;
  (void)lds;
#endif
}

// Direct global -> LDS loader (global_load_lds_dwordx4) for a tile of ROWS rows
// x 128 bytes, issued by the NW waves of a workgroup.  One wave instruction
// writes 1 KiB of LDS = 8 consecutive tile rows, lane l landing at byte 16*l:
// row r = r0 + l/8, chunk slot l%8.  With the swizzle above that slot holds
// logical chunk (l%8) ^ swz(r), so lane l loads that chunk of its row; the 8
// lanes of a row still cover its 128 contiguous bytes.  Wave w issues the
// instructions for row groups NW*i + w.
template <int ROWS, int NW, bool WEIGHTS_FIRST = false>
struct DmaTile {
  static constexpr int NI = ROWS / (8 * NW);  // instructions per wave per K step
  static_assert(NI >= 1 && ROWS == 8 * NW * NI, "tile rows must be a multiple of 8 * waves");
  const char* src[NI];

  __device__ __forceinline__ static int row_of(int i) { return 8 * (NW * i + wave_id()) + (lane_id() >> 3); }
  // rowp: address of K-step 0 of tile row row_of(i).
  __device__ __forceinline__ void set(int i, const char* rowp) {
    const int l = lane_id();
    src[i] = rowp + (((l & 7) ^ swz(row_of(i))) << 4);
  }
  // WEIGHTS_FIRST: instructions go out last row group first.  A stage holds
  // token rows, then weight rows; the weight rows (HBM misses) are its long
  // pole and the token rows (L2 hits) its short one.  Measured per kernel:
  // the fp16 two-stage rings (mixtral's Stage 1 1.000 -> 0.982 ms, Stage 2
  // 0.495 -> 0.482 ms) take it; the 8-bit 256-row Stage 2 (+2.5%) and the
  // three-stage rings with their spread issue (dsv3 Stage 2 +1%) do not.
  __device__ __forceinline__ static constexpr int order(int j) { return WEIGHTS_FIRST ? NI - 1 - j : j; }
  __device__ __forceinline__ void issue(char* lds, int ks) const {
    const int w = wave_id();
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int i = order(j);
      dma_to_lds<16>(src[i] + (size_t)ks * kRowBytes, lds + 1024 * (NW * i + w));
    }
  }
  // The instructions i with i % PARTS == part of issue(lds, ks).
  template <int PARTS>
  __device__ __forceinline__ void issue_part(char* lds, int ks, int part) const {
    const int w = wave_id();
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int i = order(j);
      if (j % PARTS == part) dma_to_lds<16>(src[i] + (size_t)ks * kRowBytes, lds + 1024 * (NW * i + w));
    }
  }
  // As issue(), with tile rows from `weights_from` on loaded under the
  // streaming weight policy (kNoStream: none); an instruction's 8 rows never
  // straddle that boundary when it is a multiple of 8, so the choice is
  // wave-uniform.
  __device__ __forceinline__ void issue(char* lds, int ks, int weights_from) const {
    const int w = wave_id();
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const char* g = src[i] + (size_t)ks * kRowBytes;
      char* d = lds + 1024 * (NW * i + w);
      if (8 * (NW * i + w) >= weights_from) dma_to_lds<16, kPolicyWeights>(g, d);
      else dma_to_lds<16>(g, d);
    }
  }
};

// MFMA fragment of the 32 tile rows starting at `row0`, K sub-step s (0..3).
__device__ __forceinline__ u32x4 frag(const char* lds, int row0, int s) {
  const int l = lane_id();
  return *reinterpret_cast<const u32x4*>(lds + lds_swz(row0 + (l & 31), 2 * s + (l >> 5)));
}

// The same reads by 32-bit LDS address, for the K loops.  A fragment's first
// tile row is a multiple of 32 there, so its row swizzle depends on the lane
// alone (swz(r0 + (l & 31)) = swz(l & 31)) and its address splits into a
// wave-uniform row base, lds + 128 * r0, and a per-lane offset for each K
// sub-step.  With the base taken through readfirstlane (a scalar register,
// recomputed per ring stage) and the four lane offsets held once, the
// compiler keeps one VGPR per sub-step instead of hoisting one address per
// fragment and sub-step out of the K loop.
struct FragLane {
  uint32_t off[4];
  __device__ __forceinline__ FragLane() {
    const int l = lane_id();
#pragma unroll
    for (int s = 0; s < 4; ++s) off[s] = (uint32_t)lds_swz(l & 31, 2 * s + (l >> 5));
  }
};
__device__ __forceinline__ uint32_t row_base(const char* lds, int row0) {
  const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)lds;
  return __builtin_amdgcn_readfirstlane(a + ((uint32_t)row0 << 7));
}
__device__ __forceinline__ u32x4 frag_at(uint32_t base, uint32_t lane_off) {
  typedef __attribute__((address_space(3))) const u32x4 LdsVec;
  return *(LdsVec*)(uintptr_t)(base + lane_off);
}

__device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                               __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ i32x16 mma(u32x4 a, u32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a),
                                              __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

// fp8 (OCP e4m3) x fp8 over 64 K elements: the lane supplies 32 bytes, the
// fragments of two consecutive 32-byte K sub-steps (frag(.., s) and
// frag(.., s + 1)).  Which K index each byte takes does not matter as long as
// both operands come from the same LDS layout through the same fragment loads.
__device__ __forceinline__ f32x16 mma8(u32x4 a0, u32x4 a1, u32x4 b0, u32x4 b1, f32x16 c) {
  const i32x8 a = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
  const i32x8 b = {(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
  // format 0 (fp8 e4m3) for both operands, no block scaling
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// As mma8, with the B operand's rows scaled by 2^(sb - 127) (E8M0 byte sb):
// lane l gives the scale of B row l % 32 -- lanes l and l + 32 each cover one
// 32-element K block of that row, and the callers pass the same scale for
// both, since a row's scale is constant over the 64 K elements.
__device__ __forceinline__ f32x16 mma8_scale_b(u32x4 a0, u32x4 a1, u32x4 b0, u32x4 b1, f32x16 c, int sb) {
  const i32x8 a = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
  const i32x8 b = {(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, sb);
}

// Power-of-two scale for an fp8 block of maximum |value| amax > 0: 2^j with
// the smallest j such that amax <= 448 * 2^j (so amax / 2^j lies in (224,
// 448] and dividing by it is exact), j >= -127.  Returned as its E8M0 byte
// j + 127; scale_from_e8m0 gives the float (2^-127 as a denormal).
__device__ __forceinline__ int pow2_scale_e8m0(float amax) {
  const uint32_t u = __float_as_uint(amax);
  const int e = (int)((u >> 23) & 0xFF) - 127;                  // amax = m * 2^e, m in [1, 2)
  int j = e - 8 + ((u & 0x7FFFFFu) > 0x600000u ? 1 : 0);       // 448 = 1.75 * 2^8
  return j < -127 ? 0 : j + 127;
}
__device__ __forceinline__ float scale_from_e8m0(int b) {
  return b == 0 ? __uint_as_float(0x00400000u) : __uint_as_float((uint32_t)b << 23);
}

// silu(g) * u = u * g / (1 + 2^(-g*log2e)) in fp32 (v_exp_f32 + v_rcp_f32).
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * kLog2e));
  return u * (g * sig);
}

// q = clamp(trunc(x*inv +- 0.5), +-127): the product and the +-0.5 are two
// separately rounded fp32 operations (never one fused multiply-add), so the
// result is bit-identical to the same two IEEE operations on the CPU.
__device__ __forceinline__ int quant_i8(float x, float inv) {
#pragma clang fp contract(off)
  const float v = x * inv;
  float t = v + (v >= 0.0f ? 0.5f : -0.5f);
  int q = (int)t;  // truncates toward zero
  q = q > 127 ? 127 : q;
  q = q < -127 ? -127 : q;
  return q;
}

// OCP fp8 e4m3 code of v, round to nearest even, saturating at +-448 (the
// callers scale so that |v| <= 448): the gfx950 conversion instruction
// (v_cvt_pk_fp8_f32, two codes per instruction) on v clamped to [-448, 448].
// Its codes equal a bit-level restatement of the format -- the fp32 mantissa
// rounded to 3 bits with the carry running into the rebiased exponent, and
// below 2^-6 the round-to-even multiple of 2^-9 -- for every float of
// magnitude <= 448 (checked exhaustively by the fp8 GPU tests).
__device__ __forceinline__ float f8_clamp(float v) { return __builtin_amdgcn_fmed3f(v, -448.0f, 448.0f); }
__device__ __forceinline__ uint32_t f8_e4m3(float v) {
  const float c = f8_clamp(v);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, c, 0, false) & 0xffu;
}
// codes of a, b, c, d in bytes 0..3
__device__ __forceinline__ uint32_t f8_e4m3x4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(f8_clamp(a), f8_clamp(b), 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(f8_clamp(c), f8_clamp(d), lo, true);
}

// Largest code magnitude of the 8-bit formats: int8 (symmetric) and fp8 e4m3.
template <bool F8> constexpr float qmax() { return F8 ? 448.0f : 127.0f; }

// 8-bit codes (int8 round-half-away or fp8 e4m3) of x[0..3] * inv packed
// into bytes 0..3.
template <bool F8>
__device__ __forceinline__ uint32_t quant_code4(float x0, float x1, float x2, float x3, float inv) {
#pragma clang fp contract(off)
  if constexpr (F8) {
    return f8_e4m3x4(x0 * inv, x1 * inv, x2 * inv, x3 * inv);
  } else {
    return ((uint32_t)quant_i8(x0, inv) & 0xffu) | (((uint32_t)quant_i8(x1, inv) & 0xffu) << 8) |
           (((uint32_t)quant_i8(x2, inv) & 0xffu) << 16) | (((uint32_t)quant_i8(x3, inv) & 0xffu) << 24);
  }
}

// ---------------------------------------------------------------------------
// Work schedule.  A launch covers the BM-row blocks of all experts times the
// nt output-feature tiles of width BN.  M blocks of expert e are
// [gpo[e]/BM, gpo[e+1]/BM); `host_blocks` is the number of BM-row blocks the
// caller's buffers hold: expert blocks beyond it are never scheduled (so
// inconsistent metadata cannot move an access out of the buffers), and with
// `tail` set, blocks between the experts' last block and host_blocks are
// scheduled as tail items (e = -1) covering padded rows that no expert owns.
//
// Pairing.  With `pair` set, two consecutive blocks of one expert form one
// item of 2*BM rows x BN/2 features instead of two items of BM x BN: the same
// LDS stage (2*BM + 2*(BN/2) = BM + 2*BN rows when BN = BM) and the same MFMA
// work, but the expert's weight tile is streamed once for both blocks instead
// of once per block.  An expert of nb blocks then has P = nb/2 paired blocks
// and nb%2 single blocks; either way it yields nb * nt items.  Its items are
// ordered by N tile t: the 2P paired items of the two half tiles of t, then
// the single block's item of t, so all items reading one weight tile are
// adjacent.
//
// Items are numbered expert-major and the item range is cut into 8
// contiguous chunks, one per XCD (workgroup g runs on XCD g % 8 and is that
// XCD's (g / 8)-th workgroup), so the items sharing a weight tile or a token
// tile run close together on one XCD and re-read it from that XCD's L2.
// ---------------------------------------------------------------------------
struct Work {
  int e;        // expert, or -1 for a tail block owned by no expert
  int row0;     // first row of the tile (in the expert-sorted row space)
  int rows;     // BM, 2*BM for a paired item, 3*BM for a triple item
  int n0;       // first output feature of the tile
  int bn;       // BN, or BN/2 for a paired or triple item
  bool shared;  // other items of this launch read the same weight rows
  int ar0 = 0;  // absorbed rows (see below): first sorted row ...
  int nar = 0;  // ... and count (0: none)
};

// Absorbed rows.  An expert's rows rarely fill its last block: at mixtral's
// ~512 rows per expert, 256-row blocks leave 5 of 8 experts a third block of
// 2-30 rows, and its items (a quarter of Stage 1's) each stream a whole weight
// tile for those few rows.  With absorption on, an expert whose last block
// holding routed rows holds at most kAbsorbRows of them, after at least one
// other block, gets no items for that block (nor for an empty block after it,
// which the 256-row padding leaves to 128-row launches): its first item group
// -- block 0's item, or both halves of pair 0 when paired -- takes those rows
// as w.nar extra token rows from sorted row w.ar0, against the weight tile it
// streams anyway.  The item count drops by those blocks' items, and the
// launch's items are renumbered so that the 8 XCD chunks stay even.  The
// expert scan keeps 4 values per chunk of 64 experts in registers, so
// absorption needs E <= kAbsorbMaxE.  `absorb` is 0 (off) or the blocks of
// items a paired launch must keep: 1 lets a two-block expert's pair become
// one full-width item with the rows (fewer, longer items: measured faster in
// saturated launches, dsv3's Stage 2 1.88 -> 1.82 ms), 2 keeps such pairs
// (launches of few items, such as the reference's run_kernel cases 1-2,
// measured slower with fewer items: 0.41 -> 0.43 and 0.73 -> 0.80 ms).
constexpr int kAbsorbRows = 32;
constexpr int kAbsorbMaxE = 256;

// Triple items.  With pairing, an expert with an odd number nm >= 3 of blocks
// holding items runs, per N tile, its (nm - 1) / 2 pairs on each half tile
// and one single block over the whole tile; the single streams the tile
// again at its own pace, and a 4 MiB L2 does not keep it across the lag.
// With `triple` set (schedule_absorbed only), the expert's last three blocks
// instead form one item per half tile, 3*BM rows x BN/2 features, so every
// weight row of the expert's tile is streamed by exactly one item per pair
// group: (nm - 1) * nt items instead of nm * nt.  An expert whose absorbed
// rows would have to ride with the triple (nm == 3) keeps its pair and
// single.


__device__ __forceinline__ bool schedule_absorbed(int g, const int32_t* __restrict__ gpo,
                                                  const int32_t* __restrict__ gs, int E, int BM, int BN,
                                                  int nt, int host_blocks, bool pair, int absorb, bool triple,
                                                  Work& w);

__device__ __forceinline__ bool schedule(int g, const int32_t* __restrict__ gpo, int E, int BM, int BN,
                                         int nt, int host_blocks, bool tail, bool pair, Work& w,
                                         const int32_t* __restrict__ gs = nullptr, int absorb = 0,
                                         bool triple = false) {
  if (absorb > 0 && !tail && E <= kAbsorbMaxE)
    return schedule_absorbed(g, gpo, gs, E, BM, BN, nt, host_blocks, pair, absorb, triple, w);
  int expert_blocks = gpo[E] / BM;
  expert_blocks = expert_blocks < host_blocks ? expert_blocks : host_blocks;
  const int total_blocks = tail ? host_blocks : expert_blocks;
  const int total = total_blocks * nt;
  const int per = (total + kNumXcd - 1) / kNumXcd;
  const int slot = g / kNumXcd;
  const int v = (g % kNumXcd) * per + slot;
  if (slot >= per || v >= total) return false;
  const int expert_items = expert_blocks * nt;
  if (v >= expert_items) {
    const int t = v - expert_items;
    w.e = -1;
    w.row0 = (expert_blocks + t / nt) * BM;
    w.rows = BM;
    w.n0 = (t % nt) * BN;
    w.bn = BN;
    w.shared = false;
    return true;
  }
  // e = (number of experts whose first item is <= v) - 1, found with ballots.
  const int l = lane_id();
  int cnt = 0;
  for (int base = 0; base < E; base += 64) {
    const int e = base + l;
    int le = 0;
    if (e < E) le = (gpo[e] / BM) * nt <= v;
    cnt += __popcll(__ballot(le));
  }
  const int e = cnt - 1;
  if (e < 0) return false;  // only with inconsistent metadata (gpo[0] > 0)
  const int b0 = gpo[e] / BM;
  const int nb = gpo[e + 1] / BM - b0;
  if (nb <= 0) return false;
  const int local = v - b0 * nt;
  const int t = local / nb;  // N tile
  const int r = local % nb;  // item within tile t
  const int P = pair ? nb / 2 : 0;
  w.e = e;
  w.shared = pair ? nb > 2 : nb > 1;
  if (r < 2 * P) {
    w.rows = 2 * BM;
    w.row0 = (b0 + 2 * (r % P)) * BM;
    w.bn = BN / 2;
    w.n0 = (2 * t + r / P) * (BN / 2);
  } else {
    w.rows = BM;
    w.row0 = (b0 + r) * BM;
    w.bn = BN;
    w.n0 = t * BN;
  }
  return (w.row0 + w.rows) / BM <= host_blocks && t < nt;
}

// schedule() with absorbed rows (E <= kAbsorbMaxE, no ownerless tail items).
// Lane l scans expert 64c + l of chunk c: nb blocks, of which d (the last
// block with routed rows, if absorbed, and any empty block after it) get no
// items, and one more block's worth of items goes when the expert takes a
// triple item.  Expert e's items start at (gpo[e]/BM - sum of those below e)
// * nt, counted with three ballots per chunk; the selected expert is the last
// whose first item is <= the workgroup's item.
__device__ __forceinline__ bool schedule_absorbed(int g, const int32_t* __restrict__ gpo,
                                                  const int32_t* __restrict__ gs, int E, int BM, int BN,
                                                  int nt, int host_blocks, bool pair, int absorb, bool triple,
                                                  Work& w) {
  constexpr int C = kAbsorbMaxE / 64;
  const int l = lane_id();
  int cb0[C], cnb[C], cd[C];
  uint64_t cm1[C], cm2[C], cm3[C];
  int dtot = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int e = 64 * c + l;
    int b0 = 0, nb = 0, d = 0;
    bool tri = false;
    if (e < E) {
      b0 = gpo[e] / BM;
      nb = gpo[e + 1] / BM - b0;
      const int n = gs[e];
      const int v = (n + BM - 1) / BM;  // blocks holding routed rows
      if (v >= (pair ? absorb : 1) + 1 && n - (v - 1) * BM <= kAbsorbRows && nb >= v && nb - (v - 1) <= 3)
        d = nb - (v - 1);
      const int nm = nb - d;
      tri = triple && pair && nm >= 3 && (nm & 1) && (d == 0 || nm >= 5);
    }
    cb0[c] = b0;
    cnb[c] = nb;
    cd[c] = d + (tri ? 4 : 0);  // bit 2: the expert takes a triple item
    cm1[c] = __ballot(d & 1);
    cm2[c] = __ballot((d >> 1) & 1);
    cm3[c] = __ballot(tri);
    dtot += __popcll(cm1[c]) + 2 * __popcll(cm2[c]) + __popcll(cm3[c]);
  }
  int expert_blocks = gpo[E] / BM;
  expert_blocks = expert_blocks < host_blocks ? expert_blocks : host_blocks;
  const int total = (expert_blocks - dtot) * nt;
  const int per = (total + kNumXcd - 1) / kNumXcd;
  const int slot = g / kNumXcd;
  const int v = (g % kNumXcd) * per + slot;
  if (total <= 0 || slot >= per || v >= total) return false;
  const uint64_t below = (1ull << l) - 1;  // l <= 63
  int e = -1, eb0 = 0, enb = 0, ed = 0, estart = 0, carry = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int start = (cb0[c] - carry - __popcll(cm1[c] & below) - 2 * __popcll(cm2[c] & below) -
                       __popcll(cm3[c] & below)) * nt;
    const int k = __popcll(__ballot(64 * c + l < E && start <= v));
    if (k > 0) {  // wave-uniform
      e = 64 * c + k - 1;
      eb0 = __shfl(cb0[c], k - 1);
      enb = __shfl(cnb[c], k - 1);
      ed = __shfl(cd[c], k - 1);
      estart = __shfl(start, k - 1);
    }
    carry += __popcll(cm1[c]) + 2 * __popcll(cm2[c]) + __popcll(cm3[c]);
  }
  if (e < 0) return false;  // only with inconsistent metadata (gpo[0] > 0)
  const int etri = triple ? ed >> 2 : 0;  // the expert takes a triple item
  if (triple) ed &= 3;
  const int nm = enb - ed;  // blocks with items
  if (nm <= 0) return false;
  const int ni = nm - etri;  // items per N tile
  const int local = v - estart;
  const int t = local / ni;  // N tile
  const int r = local % ni;  // item within tile t
  const int P = pair ? (nm - 3 * etri) / 2 : 0;  // pairs per half tile (besides the triple)
  w.e = e;
  w.shared = pair ? ni > 2 : ni > 1;
  if (r < 2 * P) {
    w.rows = 2 * BM;
    w.row0 = (eb0 + 2 * (r % P)) * BM;
    w.bn = BN / 2;
    w.n0 = (2 * t + r / P) * (BN / 2);
  } else if (etri) {  // r = 2P, 2P + 1: the triple on half tile r - 2P
    w.rows = 3 * BM;
    w.row0 = (eb0 + 2 * P) * BM;
    w.bn = BN / 2;
    w.n0 = (2 * t + r - 2 * P) * (BN / 2);
  } else {
    w.rows = BM;
    w.row0 = (eb0 + r) * BM;
    w.bn = BN;
    w.n0 = t * BN;
  }
  w.ar0 = 0;
  w.nar = 0;
  if (ed > 0 && (P > 0 ? (r < 2 * P && r % P == 0) : r == 0)) {
    w.ar0 = (eb0 + nm) * BM;
    w.nar = gs[e] - nm * BM;  // 1 .. kAbsorbRows
  }
  return (w.row0 + w.rows) / BM <= host_blocks && (w.nar == 0 || w.ar0 / BM < host_blocks) && t < nt;
}

// Pre-routed launches (the reference operator): block b's expert is
// gidx[b] (problem_detail.json:50 note 5; submission.py:1444), and the launch
// covers blocks [0, nblk) with nblk = min(gidx entries, blocks of the row
// buffers), as submission.py:2115 launches group_idx_for_bx.numel() blocks.
// Item v belongs to block v / nt; the maximal run of consecutive blocks with
// that block's gidx value is treated as one expert's blocks above (paired
// items, N-tile-major order), so items [s * nt, (s + n) * nt) cover run
// [s, s + n) exactly once whatever the values are.  Two blocks of one run
// form a valid paired item for any group metadata: row m of the pair is
// valid iff m < gs[e] - (row0 - gpo[e]), which is the per-block rule of each
// half.  A gidx value outside [0, E) gives w.e = -1 (rows owned by no expert).
//
// Absorbed rows here keep the numbering: with `absorb` set, a run of two or
// more blocks whose last block holds 1..kAbsorbRows routed rows (by gs and
// gpo) gives that block's items nothing to do (they end at once), and the
// run's first item group takes its rows, as schedule_absorbed describes.
__device__ __forceinline__ bool schedule_bx(int g, const int32_t* __restrict__ gidx, int nblk, int E, int BM,
                                            int BN, int nt, bool pair, Work& w,
                                            const int32_t* __restrict__ gs = nullptr,
                                            const int32_t* __restrict__ gpo = nullptr, int absorb = 0) {
  const int total = nblk * nt;
  const int per = (total + kNumXcd - 1) / kNumXcd;
  const int slot = g / kNumXcd;
  const int v = (g % kNumXcd) * per + slot;
  if (slot >= per || v >= total) return false;
  const int bs = v / nt;
  const int val = gidx[bs];
  const int l = lane_id();
  // run start: the nearest block below bs with another value (or -1)
  int s = -1;
  for (int base = bs - 1; base >= 0 && s < 0; base -= 64) {
    const int b = base - l;
    const bool diff = b < 0 || gidx[b] != val;
    const uint64_t m = __ballot(diff);
    if (m) s = base - (__ffsll((unsigned long long)m) - 1) + 1;
  }
  if (s < 0) s = 0;
  // run end: the nearest block above bs with another value (or nblk)
  int end = -1;
  for (int base = bs + 1; end < 0; base += 64) {
    const int b = base + l;
    const bool diff = b >= nblk || gidx[b] != val;
    const uint64_t m = __ballot(diff);
    if (m) end = base + (__ffsll((unsigned long long)m) - 1);
  }
  const int nb = end - s;
  w.e = val >= 0 && val < E ? val : -1;
  int nm = nb, last = 0;  // blocks with items; routed rows of an absorbed last block
  if (absorb > 0 && w.e >= 0 && nb >= (pair ? absorb : 1) + 1) {
    last = gs[w.e] - ((s + nb - 1) * BM - gpo[w.e]);
    if (last >= 1 && last <= kAbsorbRows) nm = nb - 1;
  }
  const int local = v - s * nt;
  const int t = local / nb;
  const int r = local % nb;
  if (r >= nm) return false;  // the absorbed block's item: its rows ride with the run's first items
  const int P = pair ? nm / 2 : 0;
  w.shared = pair ? nm > 2 : nm > 1;
  if (r < 2 * P) {
    w.rows = 2 * BM;
    w.row0 = (s + 2 * (r % P)) * BM;
    w.bn = BN / 2;
    w.n0 = (2 * t + r / P) * (BN / 2);
  } else {
    w.rows = BM;
    w.row0 = (s + r) * BM;
    w.bn = BN;
    w.n0 = t * BN;
  }
  w.ar0 = 0;
  w.nar = 0;
  if (nm < nb && (P > 0 ? (r < 2 * P && r % P == 0) : r == 0)) {
    w.ar0 = (s + nm) * BM;
    w.nar = last;
  }
  return true;
}

// Upper bound on the workgroups `schedule` needs for `blocks` M blocks.
inline int64_t schedule_grid(int64_t blocks, int64_t ntiles) {
  const int64_t total = blocks * ntiles;
  const int64_t per = (total + kNumXcd - 1) / kNumXcd;
  return per * kNumXcd;
}

}  // namespace moe
