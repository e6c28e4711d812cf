// Grouped expert GEMMs for gfx950: Stage 1 (gate/up + SiLU*up) and Stage 2
// (down projection * routing weight) on fp16 MFMA (v_mfma_f32_32x32x16_f16),
// int8 MFMA (v_mfma_i32_32x32x32_i8) or fp8 MFMA (v_mfma_f32_32x32x64_f8f6f4,
// OCP e4m3).
//
// Reference algorithm: 初审材料/源代码/submission.py Stage1 family (:136-247,
// :1391-1635) and Stage2 family (:655-795, :1132-1378); base form
// xpuoj_data/submission.py:31-129 and :253-331.  The tiling here is this
// build's own.  One workgroup per item:
//   - 32- and 64-row tiles (4 waves) for decode-sized batches; fp16 Stage 1 of
//     32-row tiles runs the narrow kernel (32 gate + 32 up features per item);
//   - 128-row tiles (8 waves): BM rows x 256 weight rows (Stage 1: 128 gate +
//     128 up, sharing the token tile; Stage 2: 256 features), or a paired item
//     of 2*BM rows x 128 weight rows for two blocks of one expert, which
//     streams their weight tile once;
//   - 256-row tiles (8 waves) when experts average >= 192 rows: two 64 KiB
//     stages, or the split ring below for 8-bit Stage 1;
// and an expert's last block of at most 32 rows rides with its first item
// group (absorbed rows, moe_common.h schedule_absorbed).  K advances 128 bytes
// per step through an S-stage ring of XOR-swizzled LDS tiles filled by direct
// global->LDS loads (global_load_lds_dwordx4), so S-2 steps of loads stay in
// flight behind the MFMAs of the current step, with one barrier per step.
#include "launch.h"
#include "moe_common.h"

#include <type_traits>

// Whole-stage rings of three or more stages issue the next stage's loads
// spread over a step's sub-steps (1) or in one burst after the barrier (0).
// A/B: mixtral Stage 2 0.680 -> 0.648 ms, dsv3 and the pre-routed cases level.
// Two-stage rings (256-row items) keep the burst: spread there, a stage is
// issued later in the step and arrives late (mixtral Stage 1 +10%, int8
// Stage 2 +5%).
#ifndef MOE_SPREAD_ISSUE
#define MOE_SPREAD_ISSUE 1
#endif
// Stage 1 8-bit 256-row items on the split ring (1) or on two whole 64 KiB
// stages (0).
// Absorbed rows (see schedule_absorbed): fp16 256-row items and 128-row
// paired items of both stages take an expert's last few rows instead of
// giving them items of their own; 0 turns it off.
#ifndef MOE_ABSORB
#define MOE_ABSORB 1
#endif
#ifndef MOE_S1_SPLIT
#define MOE_S1_SPLIT 1
#endif
// 8-bit 256-row items: weight tiles that no other item of the launch reads
// are loaded non-temporal -- int8 Stage 1's weight slots of the split ring and
// both formats' Stage 2 weight rows (1, the default); 0: the default policy
// everywhere.  A/B at the w8a8 shape, 3 runs each, interleaved: int8 step
// 0.853 -> 0.822 ms (Stage 1 0.489 -> 0.479, Stage 2 0.284 -> 0.274); fp8
// Stage 2 0.275 -> 0.268 but fp8 Stage 1 0.440 -> 0.450, so fp8's Stage 1
// keeps the default policy.  (These items' weight tiles miss: the L1 waits on
// L2 for 66% of int8 Stage 1's cycles.)
#ifndef MOE_W8_STREAM
#define MOE_W8_STREAM 1
#endif
// Triple items (moe_common.h schedule_absorbed) for fp16 Stage 1 on paired
// 128-row items: an expert with an odd number (>= 3) of blocks streams each
// half weight tile once, for its last three blocks together, instead of once
// for a pair and again for a single block (1); 0, the default: pairs and a
// single.  Off because it measured slower: A/B at dsv3 in one run, 3 x 3
// interleaved, Stage 1 3.294 ms (pairs and singles) against 3.364-3.371
// (triples, loads issued in one burst after the barrier) and 3.415-3.428 (the
// token slot's loads spread over the first three sub-steps instead).
#ifndef MOE_S1_TRIPLE
#define MOE_S1_TRIPLE 0
#endif
// Stage 2 output through LDS as whole row segments (1) or direct 16-byte
// pieces of 32 rows per store (0).
#ifndef MOE_S2_STAGED_OUT
#define MOE_S2_STAGED_OUT 1
#endif

namespace moe {

// out[0..3] += v (two packed fp16 atomic adds; no return value)
__device__ __forceinline__ void atomic_add_f16x4(_Float16* out, f16x4 v) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(1))) h2 GlobalH2;
  GlobalH2* p = (GlobalH2*)(uintptr_t)out;
  __builtin_amdgcn_global_atomic_fadd_v2f16(p, h2{v[0], v[1]});
  __builtin_amdgcn_global_atomic_fadd_v2f16(p + 1, h2{v[2], v[3]});
#else
  (void)out;
  (void)v;
#endif
}

template <int BM, int WAVES_M, int BN, int NW>
struct Layout {
  static constexpr int WAVES_N = NW / WAVES_M;
  static constexpr int WTM = BM / WAVES_M;   // tokens per wave
  static constexpr int WTN = BN / WAVES_N;   // output features per wave
  static constexpr int NBM = WTM / 32;
  static constexpr int NBN = WTN / 32;
  static_assert(NBM >= 1 && NBN >= 1, "wave tile must hold at least one 32x32 block");
};

// Wave placement in a tile: the template layout for a BM-row item; a paired
// item (2*BM rows, half the features) stacks twice the waves along M and half
// along N, so every wave keeps the same WTM x WTN sub-tile.
template <typename L>
struct WavePos {
  int wm, wn;
  __device__ __forceinline__ WavePos(int wave, bool paired) {
    const int wn_count = paired ? L::WAVES_N / 2 : L::WAVES_N;
    wm = wave / wn_count;
    wn = wave % wn_count;
  }
};

// Runs f(std::integral_constant<int, NB>) with NB = min(live, MAX), live >= 0:
// the K loops are instantiated per count of live 32-row token blocks.
template <int MAX, typename F>
__device__ __forceinline__ void with_live(int live, F&& f) {
  if constexpr (MAX == 0) {
    f(std::integral_constant<int, 0>{});
  } else {
    if (live >= MAX) f(std::integral_constant<int, MAX>{});
    else with_live<MAX - 1>(live, f);
  }
}

// Stage 1 triple item (fp16, kBN-row blocks, 8 waves): 3 * kBN = 384 token
// rows x (64 gate + 64 up) weight rows of one half tile.  Waves are 4 (M) x 2
// (N), each owning 96 token rows x 32 features: three 32x32 blocks of gate
// and three of up.  A whole stage would be 64 KiB, and two of them would
// leave one in flight, so the ring is split as the 8-bit 256-row one: two
// 48 KiB token slots and three 16 KiB weight slots (144 KiB).  After step j's
// barrier T(j+1) and then W(j+2) are issued: the weight rows (HBM misses) run
// two steps ahead, the token rows (L2 hits) one, and the wait for step j
// leaves W(j+1) in flight.  `actual`: routed rows of the item (1..384).
template <int NW>
__device__ __forceinline__ void stage1_triple(const Stage1Params& p, const Work& w, int actual, char* smem) {
  static_assert(NW == 8, "triple items run 8 waves");
  constexpr int TR = 3 * kBN;        // token rows
  constexpr int WR = kBN;            // weight rows: kBN / 2 gate, then kBN / 2 up
  constexpr int TS = TR * kRowBytes;  // 48 KiB
  constexpr int WS = WR * kRowBytes;  // 16 KiB
  constexpr int NBM = 3;              // 32-row token blocks per wave
  using LT = DmaTile<TR, NW>;
  using LW = DmaTile<WR, NW>;
  const int e = w.e, row0 = w.row0, n0 = w.n0;
  const int64_t kbytes = p.H * 2;
  const int nk = (int)(kbytes / kRowBytes);
  const bool sh = p.e_shared >= 0 && e == p.e_shared;
  const char* gexp = sh ? p.wg_shared : p.wg + (int64_t)e * p.w_es;
  const char* uexp = sh ? p.wu_shared : p.wu + (int64_t)e * p.w_es;
  LT ldt;
  LW ldw;
#pragma unroll
  for (int i = 0; i < LT::NI; ++i) {
    const int r = LT::row_of(i);
    const int pid = r < actual ? p.sorted_ids[row0 + r] : 0;  // padding rows: token 0's row
    ldt.set(i, p.x + (int64_t)(pid / p.topk) * kbytes);
  }
#pragma unroll
  for (int i = 0; i < LW::NI; ++i) {
    const int r = LW::row_of(i);
    ldw.set(i, r < WR / 2 ? gexp + (int64_t)(n0 + r) * p.w_ld : uexp + (int64_t)(n0 + r - WR / 2) * p.w_ld);
  }
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int xr0 = 32 * NBM * wm;      // stage row of this wave's first token row
  const int gr0 = 32 * wn, ur0 = WR / 2 + 32 * wn;
  const int live = (actual - xr0 + 31) / 32;  // this wave's blocks holding routed rows
  const FragLane fl;
  f32x16 ag[NBM], au[NBM];
#pragma unroll
  for (int b = 0; b < NBM; ++b) {
    ag[b] = f32x16{};
    au[b] = f32x16{};
  }
  auto tslot = [&](int j) { return smem + (j & 1) * TS; };
  auto wslot = [&](int j) { return smem + 2 * TS + (j % 3) * WS; };
  auto main_loop = [&](auto nb_c) {
    constexpr int NB = decltype(nb_c)::value;
    ldt.issue(tslot(0), 0);
    ldw.issue(wslot(0), 0);
    if (nk > 1) ldw.issue(wslot(1), 1);
    for (int ks = 0; ks < nk; ++ks) {
      // T(ks) and W(ks) are done when at most W(ks + 1)'s loads are outstanding
      if (ks + 1 < nk) wait_vmcnt<LW::NI>();
      else wait_vmcnt<0>();
      barrier_no_fence();
      if (ks + 1 < nk) ldt.issue(tslot(ks + 1), ks + 1);
      if (ks + 2 < nk) ldw.issue(wslot(ks + 2), ks + 2);
      if constexpr (NB > 0) {
        u32x4 xf[2][NB], gf[2], uf[2];
        const uint32_t xb = row_base(tslot(ks), xr0);
        const uint32_t gb = row_base(wslot(ks), gr0), ub = row_base(wslot(ks), ur0);
        auto load_frags = [&](int buf, int s) {
#pragma unroll
          for (int b = 0; b < NB; ++b) xf[buf][b] = frag_at(xb + 4096 * b, fl.off[s]);
          gf[buf] = frag_at(gb, fl.off[s]);
          uf[buf] = frag_at(ub, fl.off[s]);
        };
        load_frags(0, 0);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int fb = s & 1;
          if (s < 3) load_frags(fb ^ 1, s + 1);
          __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            ag[b] = mma(gf[fb], xf[fb][b], ag[b]);
            au[b] = mma(uf[fb], xf[fb][b], au[b]);
          }
        }
      }
    }
  };
  with_live<NBM>(live < 0 ? 0 : live, main_loop);
  // h = silu(g) * u -> fp16, routed rows only (as the other items' epilogue)
  const int l = lane_id();
#pragma unroll
  for (int b = 0; b < NBM; ++b) {
    const int m = xr0 + 32 * b + (l & 31);
    if (m < actual) {
      _Float16* hrow = reinterpret_cast<_Float16*>(p.h) + (int64_t)(row0 + m) * p.h_ld;
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int n = n0 + 32 * wn + 8 * rg + 4 * (l >> 5);
        f16x4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = (_Float16)silu_mul(ag[b][4 * rg + q], au[b][4 * rg + q]);
        *reinterpret_cast<f16x4*>(hrow + n) = v;
      }
    }
  }
}

// One ring stage holds the tile's token rows, then its weight rows (Stage 1:
// gate rows, then up rows), ROWS x 128 bytes in all, filled by one DmaTile;
// fragment reads address it by stage row.
//
// Split ring (8-bit 256-row items, MOE_S1_SPLIT): instead of S whole stages the ring
// is 5 slots of 32 KiB, each holding either the 256 token rows or the 256
// weight rows of a K step, issued in the order T0 W0 W1 | T1 W2 | T2 W3 | ...
// (after step j's barrier: T(j+1), then W(j+2)).  Weight rows (HBM misses)
// are then issued two steps ahead and token rows (L2 hits) one, and while step
// j's wait runs, W(j+1) is still queued behind T(j), so the memory pipeline
// never drains at a step boundary (a two-stage ring of whole 64 KiB stages
// drains there).  A/B at the w8a8 shape: Stage 1 int8 0.505 -> 0.496 ms, fp8
// 0.474 -> 0.453 ms.  fp16 (mixtral) measured slower on it, 1.158 -> 1.197 ms:
// its token rows, 4 MiB per expert, often come from beyond L2, and one step of
// lead is not enough for them; it keeps the two-stage ring.
template <int BM, int WAVES_M, int S, int NW, int QT, bool GATHER, bool PAIR>
__global__ __launch_bounds__(64 * NW) void stage1_kernel(Stage1Params p) {
  constexpr bool I8 = QT != kQF16;  // 8-bit operands (int8 or fp8) with row scales
  constexpr bool F8 = QT == kQF8;
  using L = Layout<BM, WAVES_M, kBN, NW>;
  using Acc = typename std::conditional<I8 && !F8, i32x16, f32x16>::type;
  constexpr int ROWS = BM + 2 * kBN;
  using LD = DmaTile<ROWS, NW, !I8 && S == 2>;  // weight rows first on the fp16 two-stage ring
  // Absorbed rows (fp16; 256-row items on the two-stage ring and 128-row
  // paired items on the three-stage one): kAbsorbRows more token rows
  // at stage rows [ROWS, ROWS + 32), loaded by waves 0-3 with one 8-row
  // instruction each (those waves wait for one more load per stage).  A wave
  // multiplies them with one of its weight blocks: 1 MFMA per sub-step.
  constexpr bool ABS = MOE_ABSORB != 0 && !I8 && NW == 8 &&
                       ((!PAIR && BM == 2 * kBN && S == 2) || (PAIR && BM == kBN && S == 3));
  constexpr int STAGE = (ROWS + (ABS ? kAbsorbRows : 0)) * kRowBytes;
  static_assert(!PAIR || (BM == kBN && L::WAVES_N % 2 == 0), "a paired item must fill the same stage");
  static_assert(!(PAIR && F8), "fp8 quantises h per 128-column tile: items must span 128 columns");
  static_assert(S >= 2 && S * STAGE <= 160 * 1024, "LDS ring exceeds the 160 KiB of a CU");
  constexpr bool TRI = MOE_S1_TRIPLE != 0 && ABS && PAIR && GATHER;  // triple items (stage1_triple)
  static_assert(!TRI || (NW == 8 && 2 * 3 * kBN * kRowBytes + 3 * kBN * kRowBytes <= S * STAGE),
                "a triple item's split ring must fit the stage ring's LDS");
  constexpr bool SPLIT = MOE_S1_SPLIT != 0 && I8 && !PAIR && BM == 2 * kBN && NW == 8;
  constexpr int HALF = (SPLIT ? BM : 0) * kRowBytes;  // one slot of the split ring: 32 KiB
  using LDH = DmaTile<SPLIT ? BM : 8 * NW, NW>;       // split ring: 256 rows per slot
  __shared__ __attribute__((aligned(16))) char smem[SPLIT ? 5 * HALF : S * STAGE];

  const int nt = (int)(p.I / kBN);
  Work w;
  // gathered (fused) launches follow the align metadata; direct (pre-routed)
  // ones map block -> expert through gidx
  if (GATHER ? !schedule(blockIdx.x, p.gpo, p.E, BM, kBN, nt, p.host_blocks, false, PAIR, w, p.gs,
                         ABS ? p.absorb : 0, TRI)
             : !schedule_bx(blockIdx.x, p.gidx, p.host_blocks, p.E, BM, kBN, nt, PAIR, w, p.gs, p.gpo,
                            ABS ? p.absorb : 0)) return;
  const int e = w.e;
  if (e < 0) return;  // a block owned by no expert: Stage 2 writes its rows as 0
  const int gpo_e = p.gpo[e];
  const int row0 = w.row0;
  const int n0 = w.n0;
  const int rx = PAIR ? w.rows : BM;   // token rows of the tile (stage rows [0, rx))
  const int rw = PAIR ? w.bn : kBN;    // gate rows [rx, rx+rw), up rows [rx+rw, rx+2rw)
  int actual = p.gs[e] - (row0 - gpo_e);
  actual = actual < 0 ? 0 : (actual > rx ? rx : actual);
  if (actual == 0) return;  // empty block: intermediate rows left untouched
  if constexpr (TRI) {
    if (w.rows == 3 * BM) {
      stage1_triple<NW>(p, w, actual, smem);
      return;
    }
  }

  const int64_t kbytes = p.H * (I8 ? 1 : 2);
  const int nk = (int)(kbytes / kRowBytes);
  // this expert's [I, H] gate / up weights, experts w_es and rows w_ld bytes
  // apart (the shared expert's own tensors, same row stride)
  const bool sh = p.e_shared >= 0 && e == p.e_shared;
  const char* gexp = sh ? p.wg_shared : p.wg + (int64_t)e * p.w_es;
  const char* uexp = sh ? p.wu_shared : p.wu + (int64_t)e * p.w_es;

  // tile row r of the stage: token rows [0, rx), gate rows, then up rows
  auto row_src = [&](int r) -> const char* {
    if (r < rx) {
      int64_t src_row;
      if (GATHER) {
        const int pid = r < actual ? p.sorted_ids[row0 + r] : 0;
        src_row = pid / p.topk;
      } else {
        src_row = row0 + (r < actual ? r : 0);  // padding rows: the item's first row, a cache hit
      }
      return p.x + src_row * kbytes;
    }
    if (r < rx + rw) return gexp + (int64_t)(n0 + r - rx) * p.w_ld;
    return uexp + (int64_t)(n0 + r - rx - rw) * p.w_ld;
  };
  LD ld;
  LDH ldt, ldw;  // split ring: token rows, weight rows
  // split ring, MOE_W8_STREAM (int8): an unshared weight tile's slots load non-temporal
  const int wstream = MOE_W8_STREAM && !F8 && !w.shared ? 0 : kNoStream;
  if constexpr (SPLIT) {
#pragma unroll
    for (int i = 0; i < LDH::NI; ++i) {
      ldt.set(i, row_src(LDH::row_of(i)));
      ldw.set(i, row_src(rx + LDH::row_of(i)));
    }
  } else {
#pragma unroll
    for (int i = 0; i < LD::NI; ++i) ld.set(i, row_src(LD::row_of(i)));
  }
  // absorbed rows: waves 0-3 each load 8 of them (rows past nar: the first one)
  const int nar = ABS ? __builtin_amdgcn_readfirstlane(w.nar) : 0;
  const bool adma = ABS && nar > 0 && wave_id() < 4;
  const char* asrc = nullptr;
  if (adma) {
    const int r = 8 * wave_id() + (lane_id() >> 3);
    const int ra = w.ar0 + (r < nar ? r : 0);  // sorted row
    const int64_t src_row = GATHER ? p.sorted_ids[ra] / p.topk : ra;
    asrc = p.x + src_row * kbytes + ((((lane_id() & 7) ^ swz(ROWS + r)) & 7) << 4);
  }
  auto issue_abs = [&](char* stage, int k) {
    if (adma) dma_to_lds<16>(asrc + (size_t)k * kRowBytes, stage + ROWS * kRowBytes + 1024 * wave_id());
  };

  const int wave = threadIdx.x >> 6;
  const WavePos<L> wp(wave, rx != BM);
  const int wm = wp.wm, wn = wp.wn;
  // 32-row token blocks of this wave that hold at least one routed row
  // (wave-uniform); padding-only blocks skip their LDS reads and MFMAs.
  // (Skipping costs L2 sharing between the M blocks of one expert -- a block
  // with less MFMA work runs ahead of its siblings -- but measured faster
  // overall than keeping siblings in step.)
  const int live = (actual - wm * L::WTM + 31) / 32;
  const int xr0 = wm * L::WTM;           // stage row of this wave's first token row
  // ... of its first gate / up row (split ring: rows of the weight slot)
  const int gr0 = (SPLIT ? 0 : rx) + wn * L::WTN;
  const int ur0 = (SPLIT ? 0 : rx) + rw + wn * L::WTN;
  const FragLane fl;

  // 8-bit: the dequantisation scales of this lane's token rows and output
  // features, loaded before the K loop so that their latency hides behind it
  // (padding rows read token 0's scale and are never stored).  The feature
  // scales stay in registers only for wave tiles of up to two 32x32 blocks;
  // larger tiles load them in the epilogue (registers would spill).
  constexpr bool kHoistFeat = L::NBN * L::NBM <= 2;
  const float* sgrow = I8 ? p.sg + (int64_t)e * p.I : nullptr;
  const float* surow = I8 ? p.su + (int64_t)e * p.I : nullptr;
  float sxv[L::NBM];
  f32x4 sgv[L::NBN][4], suv[L::NBN][4];
  if constexpr (I8) {
    const int lq = lane_id();
    int pid[L::NBM];
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) pid[b] = p.sorted_ids[row0 + xr0 + 32 * b + (lq & 31)];
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) {
      const bool valid = xr0 + 32 * b + (lq & 31) < actual;
      sxv[b] = p.x_scale[valid ? pid[b] / p.topk : 0];
    }
    if constexpr (kHoistFeat) {
#pragma unroll
      for (int a = 0; a < L::NBN; ++a)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const int n = n0 + wn * L::WTN + 32 * a + 8 * rg + 4 * (lq >> 5);
          sgv[a][rg] = *reinterpret_cast<const f32x4*>(sgrow + n);
          suv[a][rg] = *reinterpret_cast<const f32x4*>(surow + n);
        }
    }
  }
  Acc ag[L::NBN][L::NBM], au[L::NBN][L::NBM];
#pragma unroll
  for (int a = 0; a < L::NBN; ++a)
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) {
      ag[a][b] = Acc{};
      au[a][b] = Acc{};
    }
  // absorbed rows x one weight block of this wave.  256-row items (two gate
  // and two up blocks per wave): every wave, gate blocks 0, 1 for wm = 0, 1,
  // up blocks 0, 1 for wm = 2, 3.  128-row items (one of each): the gate
  // block for even wm, the up block for odd wm, on every wave of a single
  // item and on wm < 2 (one wave per SIMD) of a paired one.
  f32x16 aa = {};
  const bool awave = ABS && nar > 0 && (L::NBN == 2 || rx == BM || wm < 2);
  const bool agate = L::NBN == 2 ? wm < 2 : (wm & 1) == 0;
  const int aj = L::NBN == 2 ? (wm & 1) : 0;   // block among the wave's gate / up blocks
  const int awr0 = (agate ? gr0 : ur0) + 32 * aj;
  const int q_wave = LD::NI + (adma ? 1 : 0);  // loads per stage of this wave

  // S-stage ring: stages ks+1 .. ks+S-2 stay in flight while stage ks is used.
  constexpr int Q = LD::NI;  // loads per wave per stage
  // The K loop is instantiated per count NB of this wave's token blocks that
  // hold routed rows (chosen once, outside the loop: a branch inside it would
  // move the accumulators out of AGPRs every step); padding-only blocks get no
  // LDS reads and no MFMAs.  Every variant issues the same loads and barriers.
  // split ring: slot of the i-th issued half stage is i % 5; T(j) is issued
  // i = j ? 2j + 1 : 0, W(j) i = j > 1 ? 2j : j + 1
  auto slot = [&](int i) { return smem + (i % 5) * HALF; };
  auto main_loop = [&](auto nb_c, auto abs_c) {
    constexpr int NB = decltype(nb_c)::value;
    constexpr bool A = decltype(abs_c)::value;  // absorbed rows in this item
    if constexpr (SPLIT) {
      ldt.issue(slot(0), 0);
      ldw.issue(slot(1), 0, wstream);
      if (nk > 1) ldw.issue(slot(2), 1, wstream);
    } else {
#pragma unroll
      for (int s = 0; s < S - 1; ++s)
        if (s < nk) {
          ld.issue(smem + s * STAGE, s);
          issue_abs(smem + s * STAGE, s);
        }
    }
    int cur = 0;
    for (int ks = 0; ks < nk; ++ks) {
      const char* st;   // token rows of step ks
      const char* stw;  // weight rows of step ks
      if constexpr (SPLIT) {
        // T(ks) and W(ks) are done when at most W(ks + 1)'s loads are outstanding
        if (ks + 1 < nk) wait_vmcnt<LDH::NI>();
        else wait_vmcnt<0>();
        barrier_no_fence();
        if (ks + 1 < nk) ldt.issue(slot(2 * ks + 3), ks + 1);
        if (ks + 2 < nk) ldw.issue(slot(2 * ks + 4), ks + 2, wstream);
        st = slot(ks ? 2 * ks + 1 : 0);
        stw = slot(ks > 1 ? 2 * ks : ks + 1);
      } else {
        if constexpr (ABS) wait_stages_q<Q + 1, S - 2>(q_wave, nk - 1 - ks);
        else wait_stages<Q, S - 2>(nk - 1 - ks);
        barrier_no_fence();
        st = stw = smem + cur * STAGE;
      }
      // The next stage's loads (whole-stage ring): issued in one burst, or
      // (rings of three or more stages, MOE_SPREAD_ISSUE) spread over the
      // step's sub-steps so that no wave waits behind a long run of its own
      // DMA issues before its MFMAs.
      const bool pend = !SPLIT && ks + S - 1 < nk;
      char* pbuf = smem + (cur == 0 ? S - 1 : cur - 1) * STAGE;
      const int pk = ks + S - 1;
      if constexpr (!SPLIT) cur = cur + 1 == S ? 0 : cur + 1;
      constexpr bool kSpread = MOE_SPREAD_ISSUE != 0 && NB > 0 && S >= 3;
      if (!kSpread && pend) {
        ld.issue(pbuf, pk);
        issue_abs(pbuf, pk);
      }
      if constexpr (NB > 0 || A) {
        // Fragments double-buffered across the 4 K sub-steps: the LDS reads of
        // sub-step s+1 are in flight while the MFMAs of sub-step s run.
        u32x4 xf[2][NB > 0 ? NB : 1], gf[2][L::NBN], uf[2][L::NBN], xa[2], wa[2];
        const uint32_t xb = row_base(st, xr0), gb = row_base(stw, gr0), ub = row_base(stw, ur0);
        const uint32_t ab = A ? row_base(st, ROWS) : 0, wab = A ? row_base(stw, awr0) : 0;
        auto load_frags = [&](int buf, int s) {
#pragma unroll
          for (int b = 0; b < NB; ++b) xf[buf][b] = frag_at(xb + 4096 * b, fl.off[s]);
          if constexpr (NB > 0) {
#pragma unroll
            for (int a = 0; a < L::NBN; ++a) {
              gf[buf][a] = frag_at(gb + 4096 * a, fl.off[s]);
              uf[buf][a] = frag_at(ub + 4096 * a, fl.off[s]);
            }
          }
          if constexpr (A) {
            xa[buf] = frag_at(ab, fl.off[s]);
            wa[buf] = frag_at(wab, fl.off[s]);
          }
        };
        if constexpr (F8) {
          // fp8: one MFMA per 64-byte half step, on the fragments of two sub-steps
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            load_frags(0, 2 * j);
            load_frags(1, 2 * j + 1);
            if (kSpread && pend) ld.template issue_part<2>(pbuf, pk, j);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int a = 0; a < L::NBN; ++a)
#pragma unroll
              for (int b = 0; b < NB; ++b) {
                ag[a][b] = mma8(gf[0][a], gf[1][a], xf[0][b], xf[1][b], ag[a][b]);
                au[a][b] = mma8(uf[0][a], uf[1][a], xf[0][b], xf[1][b], au[a][b]);
              }
          }
        } else {
          load_frags(0, 0);
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int fb = s & 1;
            if (s < 3) load_frags(fb ^ 1, s + 1);
            if (kSpread && pend) {
              ld.template issue_part<4>(pbuf, pk, s);
              if (s == 0) issue_abs(pbuf, pk);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
            for (int a = 0; a < L::NBN; ++a)
#pragma unroll
              for (int b = 0; b < NB; ++b) {
                ag[a][b] = mma(gf[fb][a], xf[fb][b], ag[a][b]);
                au[a][b] = mma(uf[fb][a], xf[fb][b], au[a][b]);
              }
            if constexpr (A) aa = mma(wa[fb], xa[fb], aa);
          }
        }
      }
    }
  };
  if (awave)
    with_live<L::NBM>(live < 0 ? 0 : live, [&](auto nb_c) { main_loop(nb_c, std::integral_constant<bool, ABS>{}); });
  else
    with_live<L::NBM>(live < 0 ? 0 : live, [&](auto nb_c) { main_loop(nb_c, std::false_type{}); });
  __syncthreads();  // every wave is done with the ring before LDS is reused

  const int l = lane_id();
  if constexpr (!F8) {
    // h = silu(g) * u -> fp16, valid rows only (submission.py:1532-1542).
    // int8: g and u dequantised first, (acc * s_x[token]) * s_w[e, n]; the
    // intermediate is quantised per row afterwards (quant_rows_kernel), so
    // Stage 2 accumulates in int32 over the whole of K.
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) {
      const int m = xr0 + 32 * b + (l & 31);
      if (m < actual) {
        _Float16* hrow = reinterpret_cast<_Float16*>(p.h) + (int64_t)(row0 + m) * p.h_ld;
#pragma unroll
        for (int a = 0; a < L::NBN; ++a)
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const int n = n0 + wn * L::WTN + 32 * a + 8 * rg + 4 * (l >> 5);
            f16x4 v;
            if constexpr (I8) {
              f32x4 gs, us;
              if constexpr (kHoistFeat) {
                gs = sgv[a][rg];
                us = suv[a][rg];
              } else {
                gs = *reinterpret_cast<const f32x4*>(sgrow + n);
                us = *reinterpret_cast<const f32x4*>(surow + n);
              }
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const float g = ((float)ag[a][b][4 * rg + q] * sxv[b]) * gs[q];
                const float u = ((float)au[a][b][4 * rg + q] * sxv[b]) * us[q];
                v[q] = (_Float16)silu_mul(g, u);
              }
            } else {
#pragma unroll
              for (int q = 0; q < 4; ++q)
                v[q] = (_Float16)silu_mul(ag[a][b][4 * rg + q], au[a][b][4 * rg + q]);
            }
            *reinterpret_cast<f16x4*>(hrow + n) = v;
          }
      }
    }
    if constexpr (ABS) {
      if (nar > 0) {
        // absorbed rows: each up wave hands its block through LDS to the gate
        // wave of the same features (same wn and block), which writes h
        float* red = reinterpret_cast<float*>(smem);  // [wn * NBN + j][16][64]; the ring is free
        const int aslot = wn * L::NBN + aj;
        if (awave && !agate) {
#pragma unroll
          for (int q = 0; q < 16; ++q) red[(aslot * 16 + q) * 64 + l] = aa[q];
        }
        __syncthreads();
        const int m = l & 31;
        if (awave && agate && m < nar) {
          _Float16* hrow = reinterpret_cast<_Float16*>(p.h) + (int64_t)(w.ar0 + m) * p.h_ld;
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const int n = n0 + wn * L::WTN + 32 * aj + 8 * rg + 4 * (l >> 5);
            f16x4 v;
#pragma unroll
            for (int q = 0; q < 4; ++q)
              v[q] = (_Float16)silu_mul(aa[4 * rg + q], red[(aslot * 16 + 4 * rg + q) * 64 + l]);
            *reinterpret_cast<f16x4*>(hrow + n) = v;
          }
        }
      }
    }
  } else {
    // fp8: dequantise (acc * s_x[token]) * s_w[e, n], h = silu(g) * u, then quantise
    // h per (row, this 128-column tile) to e4m3: amax over the tile's columns,
    // which are spread over the lane pair (l, l^32) and the WAVES_N waves.
    float* red = reinterpret_cast<float*>(smem);  // [WAVES_N][BM]; loop ended with a barrier
    float hv[L::NBM][L::NBN][16];
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) {
      const int m = xr0 + 32 * b + (l & 31);
      const float sx = m < actual ? sxv[b] : 0.0f;
      float amax = 0.0f;
#pragma unroll
      for (int a = 0; a < L::NBN; ++a)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          f32x4 gs, us;
          if constexpr (kHoistFeat) {
            gs = sgv[a][rg];
            us = suv[a][rg];
          } else {
            const int n = n0 + wn * L::WTN + 32 * a + 8 * rg + 4 * (l >> 5);
            gs = *reinterpret_cast<const f32x4*>(sgrow + n);
            us = *reinterpret_cast<const f32x4*>(surow + n);
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float g = ((float)ag[a][b][4 * rg + q] * sx) * gs[q];
            const float u = ((float)au[a][b][4 * rg + q] * sx) * us[q];
            const float h = silu_mul(g, u);
            hv[b][a][4 * rg + q] = h;
            amax = fmaxf(amax, fabsf(h));
          }
        }
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      if (l < 32) red[wn * BM + xr0 + 32 * b + l] = amax;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) {
      const int mrow = xr0 + 32 * b + (l & 31);
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < L::WAVES_N; ++j) amax = fmaxf(amax, red[j * BM + mrow]);
      // The power-of-two scale 2^j (amax <= 448 * 2^j), which Stage 2's f8
      // MFMA applies itself; dividing by it is exact.
      const int sb = pow2_scale_e8m0(amax);
      const float hscale = amax > 0.0f ? scale_from_e8m0(sb) : 0.0f;
      const float inv = amax > 0.0f ? scale_from_e8m0(254 - sb) : 0.0f;  // 2^-j (sb = 0: 2^127, the exact inverse of 2^-127)
      if (mrow < actual) {
        const int64_t grow = row0 + mrow;
        int8_t* hrow = reinterpret_cast<int8_t*>(p.h) + grow * p.h_ld;
#pragma unroll
        for (int a = 0; a < L::NBN; ++a)
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const int n = n0 + wn * L::WTN + 32 * a + 8 * rg + 4 * (l >> 5);
            *reinterpret_cast<uint32_t*>(hrow + n) =
                quant_code4<true>(hv[b][a][4 * rg], hv[b][a][4 * rg + 1], hv[b][a][4 * rg + 2], hv[b][a][4 * rg + 3], inv);
          }
        // scales are stored block-major: [I/128][hs_stride]
        if (wn == 0 && l < 32) p.h_scale[(int64_t)(n0 / kBN) * p.hs_stride + grow] = hscale;
      }
    }
  }
}

// Stage 1 (fp16) for 32-row tiles with narrow gate / up tiles (BN = 64 or
// 32 features each): two or four times the items of the 128-wide tiles, for
// shapes with few items per CU (decode), where the last round of workgroups
// would otherwise stream on a fraction of the CUs.  Each of the 4 waves owns
// one 32 x 32 accumulator: gate (waves 0, 1) or up (waves 2, 3), and
//   BN = 64: features 32 * (w & 1) of the tile, all 4 K sub-steps of a step;
//   BN = 32: all 32 features, K sub-steps 2 * (w & 1) and 2 * (w & 1) + 1,
//            the two halves summed in the epilogue.
// The other accumulators reach the wave writing h through LDS.
template <int BN, int S>
__global__ __launch_bounds__(256) void stage1_narrow_kernel(Stage1Params p) {
  constexpr int BM = 32, NW = 4;
  static_assert(BN == 64 || BN == 32, "narrow tiles are 64 or 32 features wide");
  constexpr bool KSPLIT = BN == 32;
  constexpr int ROWS = BM + 2 * BN;  // stage rows: tokens, gate rows, up rows
  using LD = DmaTile<ROWS, NW>;
  constexpr int STAGE = ROWS * kRowBytes;
  static_assert(S >= 2 && S * STAGE <= 160 * 1024, "LDS ring exceeds the 160 KiB of a CU");
  static_assert(S * STAGE >= 4 * 16 * 64 * 4, "the epilogue exchange reuses the ring");
  __shared__ __attribute__((aligned(16))) char smem[S * STAGE];

  const int nt = (int)(p.I / BN);
  Work w;
  if (!schedule(blockIdx.x, p.gpo, p.E, BM, BN, nt, p.host_blocks, false, false, w)) return;
  const int e = w.e;
  const int row0 = w.row0;
  const int n0 = w.n0;
  int actual = p.gs[e] - (row0 - p.gpo[e]);
  actual = actual < 0 ? 0 : (actual > BM ? BM : actual);
  if (actual == 0) return;

  const int64_t kbytes = p.H * 2;
  const int nk = (int)(kbytes / kRowBytes);
  const bool sh = p.e_shared >= 0 && e == p.e_shared;  // see stage1_kernel
  const char* gexp = sh ? p.wg_shared : p.wg + (int64_t)e * p.w_es;
  const char* uexp = sh ? p.wu_shared : p.wu + (int64_t)e * p.w_es;
  LD ld;
#pragma unroll
  for (int i = 0; i < LD::NI; ++i) {
    const int r = LD::row_of(i);
    const char* src;
    if (r < BM) {
      const int pid = r < actual ? p.sorted_ids[row0 + r] : 0;
      src = p.x + (int64_t)(pid / p.topk) * kbytes;
    } else if (r < BM + BN) {
      src = gexp + (int64_t)(n0 + r - BM) * p.w_ld;
    } else {
      src = uexp + (int64_t)(n0 + r - BM - BN) * p.w_ld;
    }
    ld.set(i, src);
  }

  const int wave = threadIdx.x >> 6;
  const int mat = wave >> 1;  // 0: gate, 1: up
  const int half = wave & 1;  // feature half (BN = 64) or K half (BN = 32)
  const int wr0 = BM + mat * BN + (KSPLIT ? 0 : 32 * half);
  constexpr int SUB = KSPLIT ? 2 : 4;    // K sub-steps per wave per step
  const int s0 = KSPLIT ? 2 * half : 0;  // first of them
  f32x16 acc = f32x16{};
  const int stream_from = w.shared ? kNoStream : BM;  // weight rows no other item reads: streamed
  constexpr int Q = LD::NI;
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) ld.issue(smem + s * STAGE, s, stream_from);
  int cur = 0;
  for (int ks = 0; ks < nk; ++ks) {
    wait_stages<Q, S - 2>(nk - 1 - ks);
    barrier_no_fence();
    if (ks + S - 1 < nk) ld.issue(smem + (cur == 0 ? S - 1 : cur - 1) * STAGE, ks + S - 1, stream_from);
    const char* st = smem + cur * STAGE;
    cur = cur + 1 == S ? 0 : cur + 1;
    u32x4 xf[2], wf[2];
    xf[0] = frag(st, 0, s0);
    wf[0] = frag(st, wr0, s0);
#pragma unroll
    for (int s = 0; s < SUB; ++s) {
      const int b = s & 1;
      if (s + 1 < SUB) {
        xf[b ^ 1] = frag(st, 0, s0 + s + 1);
        wf[b ^ 1] = frag(st, wr0, s0 + s + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      acc = mma(wf[b], xf[b], acc);
    }
  }
  __syncthreads();  // every wave is done with the ring before LDS is reused

  // Accumulator register r of lane l holds the same (token, feature) in every
  // wave that covers the same features, so the hand-over is by (r, l):
  // slot(w, r) for the waves other than the one writing h.
  float* xs = reinterpret_cast<float*>(smem);
  const int l = lane_id();
  auto slot = [&](int wv, int r) -> float& { return xs[(wv * 16 + r) * 64 + l]; };
  const bool writer = KSPLIT ? wave == 0 : mat == 0;
  if (!writer) {
#pragma unroll
    for (int r = 0; r < 16; ++r) slot(wave, r) = acc[r];
  }
  __syncthreads();
  if (writer) {
    const int m = l & 31;
    if (m < actual) {
      _Float16* hrow = reinterpret_cast<_Float16*>(p.h) + (int64_t)(row0 + m) * p.h_ld;
      const int fbase = KSPLIT ? 0 : 32 * half;
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int n = n0 + fbase + 8 * rg + 4 * (l >> 5);
        f16x4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = 4 * rg + q;
          float g, u;
          if constexpr (KSPLIT) {  // waves: 0 gate k0, 1 gate k1, 2 up k0, 3 up k1
            g = acc[r] + slot(1, r);
            u = slot(2, r) + slot(3, r);
          } else {                 // waves: 0/1 gate halves, 2/3 up halves
            g = acc[r];
            u = slot(2 + half, r);
          }
          v[q] = (_Float16)silu_mul(g, u);
        }
        *reinterpret_cast<f16x4*>(hrow + n) = v;
      }
    }
  }
}

// STREAM: weight tiles no other item reads are loaded non-temporal.
template <int BM, int WAVES_M, int BN, int S, int NW, int QT, bool FUSED, bool PAIR, bool STREAM>
__global__ __launch_bounds__(64 * NW) void stage2_kernel(Stage2Params p) {
  constexpr bool I8 = QT != kQF16;  // 8-bit operands (int8 or fp8) with row / block scales
  constexpr bool F8 = QT == kQF8;
  using L = Layout<BM, WAVES_M, BN, NW>;
  // int8: exact int32 accumulation over the whole of K (the intermediate has
  // one scale per row, applied in the epilogue); fp16 / fp8: fp32
  using Acc = typename std::conditional<I8 && !F8, i32x16, f32x16>::type;
  constexpr int ROWS = BM + BN;
  using LD = DmaTile<ROWS, NW, !I8 && S == 2>;  // weight rows first on the fp16 two-stage ring
  // Absorbed rows (fp16; 128-row paired items on the three-stage ring and
  // 256-row items on the two-stage one): kAbsorbRows more token rows at stage
  // rows [ROWS, ROWS + 32), loaded by waves 0-3 with one 8-row instruction
  // each (those waves wait for one more load per stage).  In a paired item
  // the waves with wm < 2 (one per SIMD) multiply them with one of their two
  // weight blocks; in a single or 256-row item every wave does.
  constexpr bool ABS = MOE_ABSORB != 0 && !I8 && NW == 8 &&
                       ((PAIR && BM == 128 && S == 3) || (!PAIR && BM == 256 && S == 2));
  constexpr int SCALES = (ROWS + (ABS ? kAbsorbRows : 0)) * kRowBytes;  // fp8: row scales of the step
  constexpr int STAGE = SCALES + (F8 ? 256 * NW : 0);
  static_assert(!PAIR || (BN == 2 * BM && L::WAVES_N % 2 == 0), "a paired item must fill the same stage");
  static_assert(S >= 2 && S * STAGE <= 160 * 1024, "LDS ring exceeds the 160 KiB of a CU");
  __shared__ __attribute__((aligned(16))) char smem[S * STAGE];

  const int nt = (int)(p.H / BN);
  Work w;
  // fused launches follow the align metadata; pre-routed ones map block ->
  // expert through gidx (every block of the launch is an item)
  if (FUSED ? !schedule(blockIdx.x, p.gpo, p.E, BM, BN, nt, p.host_blocks, false, PAIR, w, p.gs,
                        ABS ? p.absorb : 0)
            : !schedule_bx(blockIdx.x, p.gidx, p.host_blocks, p.E, BM, BN, nt, PAIR, w, p.gs, p.gpo,
                           ABS ? p.absorb : 0)) return;
  const int row0 = w.row0;
  const int n0 = w.n0;
  const int rx = PAIR ? w.rows : BM;  // token rows of the tile (stage rows [0, rx))
  const int rw = PAIR ? w.bn : BN;    // weight rows [rx, rx+rw)
  int actual = 0, gpo_e = 0, go_e = 0;
  const int e = w.e;
  if (e >= 0) {
    gpo_e = p.gpo[e];
    go_e = p.go[e];
    actual = p.gs[e] - (row0 - gpo_e);
    actual = actual < 0 ? 0 : (actual > rx ? rx : actual);
  }
  if (actual == 0) {
    if (!FUSED) {
      // Rows owned by no valid token are written as 0 (problem_detail.json:50 note 4).
      _Float16* o = reinterpret_cast<_Float16*>(p.out);
      for (int idx = threadIdx.x; idx < rx * (rw / 8); idx += 64 * NW) {
        const int r = idx / (rw / 8), c = idx % (rw / 8);
        *reinterpret_cast<u32x4*>(o + (int64_t)(row0 + r) * p.H + n0 + 8 * c) = u32x4{0, 0, 0, 0};
      }
    }
    return;
  }

  const int64_t kbytes = p.I * (I8 ? 1 : 2);
  const int nk = (int)(kbytes / kRowBytes);
  // this expert's [H, I] down weights, experts wd_es and rows wd_ld bytes
  // apart (the shared expert's own tensor, same row stride); intermediate rows
  // a_ld bytes apart
  const char* dexp = p.e_shared >= 0 && e == p.e_shared ? p.wd_shared : p.wd + (int64_t)e * p.wd_es;
  // Token rows past the expert's count (never written by Stage 1) read the
  // item's first row instead: a cache hit rather than an HBM fetch.  Their
  // results are never stored.
  LD ld;
#pragma unroll
  for (int i = 0; i < LD::NI; ++i) {
    const int r = LD::row_of(i);
    ld.set(i, r < rx ? p.a + (int64_t)(row0 + (r < actual ? r : 0)) * p.a_ld : dexp + (int64_t)(n0 + r - rx) * p.wd_ld);
  }

  const int nar = ABS ? __builtin_amdgcn_readfirstlane(w.nar) : 0;  // absorbed rows
  const bool adma = ABS && nar > 0 && wave_id() < 4;
  const char* asrc = nullptr;
  if (adma) {
    const int r = 8 * wave_id() + (lane_id() >> 3);
    asrc = p.a + (int64_t)(w.ar0 + (r < nar ? r : 0)) * p.a_ld + ((((lane_id() & 7) ^ swz(ROWS + r)) & 7) << 4);
  }

  const int wave = threadIdx.x >> 6;
  const WavePos<L> wp(wave, rx != BM);
  const int wm = wp.wm, wn = wp.wn;
  const int l = lane_id();
  const bool awave = nar > 0 && (rx == BM || wm < 2);  // this wave multiplies absorbed rows
  const int live = (actual - wm * L::WTM + 31) / 32;  // see Stage 1
  const int xr0 = wm * L::WTM;       // stage row of this wave's first token row
  const int wr0 = rx + wn * L::WTN;  // ... of its first weight row
  const FragLane fl;

  // Output row and routing weight of each of this lane's token rows, loaded
  // before the K loop so that their latency hides behind it.
  // (Loads are unconditional, all rows' ids first: row0 + m lies inside the
  // item's rows of the sorted buffer; padding rows take pair 0's weight and
  // are never stored.)
  int64_t orow[L::NBM];
  float wr[L::NBM];
  float shv[L::NBM];  // int8: the intermediate's row scale (0 for padding rows)
  if constexpr (FUSED) {
    int pid[L::NBM];
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) pid[b] = p.sorted_ids[row0 + xr0 + 32 * b + (l & 31)];
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) {
      const bool valid = xr0 + 32 * b + (l & 31) < actual;
      // the pair's output row: its unpadded position in the expert-sorted
      // order, so an item writes one contiguous run of rows; the combine
      // finds it through pos[pair], written here once per row
      orow[b] = MOE_S2_SCATTER ? (int64_t)(valid ? pid[b] / p.topk : 0)
                               : (int64_t)go_e + (row0 - gpo_e) + xr0 + 32 * b + (l & 31);
      wr[b] = reinterpret_cast<const float*>(p.routed)[valid ? pid[b] : 0];
      if (valid && n0 == 0 && wn == 0 && l < 32) p.pos[pid[b]] = (int32_t)orow[b];
      if constexpr (I8 && !F8) shv[b] = valid ? p.a_scale[row0 + xr0 + 32 * b + (l & 31)] : 0.0f;
    }
  } else {
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) {
      const int m = xr0 + 32 * b + (l & 31);
      orow[b] = row0 + m;
      // raw-order index (problem_detail.json:50 note 2), clamped to the
      // buffer as submission.py:1286-1288 does
      int64_t ridx = (int64_t)go_e + (row0 - gpo_e) + m;
      ridx = ridx >= p.V ? p.V - 1 : ridx;
      ridx = ridx < 0 ? 0 : ridx;
      wr[b] = 0.0f;
      if (m < actual && p.V > 0)
        wr[b] = p.routed_f16 ? (float)reinterpret_cast<const _Float16*>(p.routed)[ridx]
                             : reinterpret_cast<const float*>(p.routed)[ridx];
    }
  }
  Acc acc[L::NBN][L::NBM];
#pragma unroll
  for (int a = 0; a < L::NBN; ++a)
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) acc[a][b] = Acc{};
  // absorbed rows x weight block aj of this wave (256-row items: block wm of
  // its four; 128-row items: block wm & 1 of its two); their pair, output
  // row and routing weight (lane l: absorbed row l % 32)
  f32x16 aa = {};
  const int aj = L::NBN >= 4 ? wm : (wm & 1);
  const int awr0 = wr0 + 32 * aj;
  int64_t aorow = 0;
  float awr = 0.0f;
  if (ABS && awave) {
    const int m = l & 31;
    if constexpr (FUSED) {
      const int pid = p.sorted_ids[w.ar0 + (m < nar ? m : 0)];
      aorow = MOE_S2_SCATTER ? (int64_t)(pid / p.topk) : (int64_t)go_e + (w.ar0 - gpo_e) + m;
      awr = m < nar ? reinterpret_cast<const float*>(p.routed)[pid] : 0.0f;
      if (m < nar && n0 == 0 && wn == 0 && aj == 0 && l < 32) p.pos[pid] = (int32_t)aorow;
    } else {
      // padded order; raw-order routing weight as for the item's own rows
      aorow = w.ar0 + m;
      int64_t ridx = (int64_t)go_e + (w.ar0 - gpo_e) + m;
      ridx = ridx >= p.V ? p.V - 1 : ridx;
      ridx = ridx < 0 ? 0 : ridx;
      if (m < nar && p.V > 0)
        awr = p.routed_f16 ? (float)reinterpret_cast<const _Float16*>(p.routed)[ridx]
                           : reinterpret_cast<const float*>(p.routed)[ridx];
    }
  }

  // fp8: the row scales of K step ks (block-major layout, so contiguous) ride
  // in the same stage: wave w loads rows 64w..64w+63 (clamped inside the tile)
  // with one dword DMA, so every wave issues the same number of loads.
  const float* scale_src = nullptr;
  if constexpr (F8) {
    const int r = 64 * wave_id() + l;
    scale_src = p.a_scale + row0 + (r < actual ? r : 0);
  }
  constexpr int Q = LD::NI + (F8 ? 1 : 0);
  auto issue_abs = [&](char* st, int k) {
    if (adma) dma_to_lds<16>(asrc + (size_t)k * kRowBytes, st + ROWS * kRowBytes + 1024 * wave_id());
  };
  auto issue = [&](int buf, int k) {
    char* st = smem + buf * STAGE;
    if constexpr (STREAM) ld.issue(st, k, w.shared ? kNoStream : rx);
    else ld.issue(st, k);
    issue_abs(st, k);
    if constexpr (F8) dma_to_lds<4>(scale_src + (int64_t)k * p.as_stride, st + SCALES + 256 * wave_id());
  };
  // part `part` of PARTS of issue(buf, k) (the scale row and the absorbed rows ride with part 0)
  auto issue_part = [&](int buf, int k, auto parts_c, int part) {
    constexpr int PARTS = decltype(parts_c)::value;
    char* st = smem + buf * STAGE;
    ld.template issue_part<PARTS>(st, k, part);
    if (part == 0) issue_abs(st, k);
    if constexpr (F8)
      if (part == 0) dma_to_lds<4>(scale_src + (int64_t)k * p.as_stride, st + SCALES + 256 * wave_id());
  };
  const int q_wave = Q + (adma ? 1 : 0);  // loads per stage of this wave
  // K loop instantiated per count of live token blocks (see Stage 1) and
  // whether this wave multiplies absorbed rows.
  auto main_loop = [&](auto nb_c, auto abs_c) {
    constexpr int NB = decltype(nb_c)::value;
    constexpr bool A = decltype(abs_c)::value;
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
      if (s < nk) issue(s, s);
    int cur = 0;
    for (int ks = 0; ks < nk; ++ks) {
      if constexpr (ABS) wait_stages_q<Q + 1, S - 2>(q_wave, nk - 1 - ks);
      else wait_stages<Q, S - 2>(nk - 1 - ks);
      barrier_no_fence();
      // the next stage's loads: one burst, or spread over the sub-steps (see Stage 1)
      const bool pend = ks + S - 1 < nk;
      const int pbuf = cur == 0 ? S - 1 : cur - 1, pk = ks + S - 1;
      constexpr bool kSpread = MOE_SPREAD_ISSUE != 0 && NB > 0 && !STREAM && S >= 3;
      if (!kSpread && pend) issue(pbuf, pk);
      const char* st = smem + cur * STAGE;
      cur = cur + 1 == S ? 0 : cur + 1;
      if constexpr (NB > 0 || A) {
        u32x4 af[2][NB > 0 ? NB : 1], wf[2][L::NBN], xa[2], wa[2];
        const uint32_t xb = row_base(st, xr0), wb = row_base(st, wr0);
        const uint32_t ab = A ? row_base(st, ROWS) : 0, wab = A ? row_base(st, awr0) : 0;
        auto load_frags = [&](int buf, int s) {
#pragma unroll
          for (int b = 0; b < NB; ++b) af[buf][b] = frag_at(xb + 4096 * b, fl.off[s]);
          if constexpr (NB > 0) {
#pragma unroll
            for (int a = 0; a < L::NBN; ++a) wf[buf][a] = frag_at(wb + 4096 * a, fl.off[s]);
          }
          if constexpr (A) {
            xa[buf] = frag_at(ab, fl.off[s]);
            wa[buf] = frag_at(wab, fl.off[s]);
          }
        };
        if constexpr (!F8) {
          // fp16 (fp32 accumulation) or int8 (int32 accumulation)
          load_frags(0, 0);
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int fb = s & 1;
            if (s < 3) load_frags(fb ^ 1, s + 1);
            if (kSpread && pend) issue_part(pbuf, pk, std::integral_constant<int, 4>{}, s);
            __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
            for (int a = 0; a < L::NBN; ++a)
#pragma unroll
              for (int b = 0; b < NB; ++b) acc[a][b] = mma(wf[fb][a], af[fb][b], acc[a][b]);
            if constexpr (A) aa = mma(wa[fb], xa[fb], aa);
          }
        } else {
          // One K step of fp8 operands is one 128-column scale block of the
          // intermediate, with one scale per token row.
          const float* scl = reinterpret_cast<const float*>(st + SCALES);
          float sc[NB];
#pragma unroll
          for (int b = 0; b < NB; ++b) sc[b] = scl[xr0 + 32 * b + (l & 31)];
          // The row scales are powers of two, applied by the MFMA itself
          // (E8M0 exponent byte of each token row's scale), straight into acc.
          int sb[NB];
#pragma unroll
          for (int b = 0; b < NB; ++b) sb[b] = (int)(__float_as_uint(sc[b]) >> 23);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            load_frags(0, 2 * j);
            load_frags(1, 2 * j + 1);
            if (kSpread && pend) issue_part(pbuf, pk, std::integral_constant<int, 2>{}, j);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int a = 0; a < L::NBN; ++a)
#pragma unroll
              for (int b = 0; b < NB; ++b)
                acc[a][b] = mma8_scale_b(wf[0][a], wf[1][a], af[0][b], af[1][b], acc[a][b], sb[b]);
          }
        }
      }
    }
  };
  if (ABS && awave)
    with_live<L::NBM>(live < 0 ? 0 : live, [&](auto nb_c) { main_loop(nb_c, std::integral_constant<bool, ABS>{}); });
  else
    with_live<L::NBM>(live < 0 ? 0 : live, [&](auto nb_c) { main_loop(nb_c, std::false_type{}); });

  // Epilogue.  Each lane's accumulators hold 4-feature runs of one token row,
  // so direct stores write 16 bytes of 32 rows per instruction.  Where the
  // output tile fits the ring, it is first assembled in LDS and then stored
  // as whole row segments, 16 bytes per lane (up to 512 bytes of one row per
  // 32 lanes).  In LDS, 16-byte chunk c of tile row r sits at chunk slot
  // c ^ (r & xm) (xm = chunks per row - 1, at most 15): the 16 rows one
  // 8-byte write instruction covers per half-wave land on 16 different slots,
  // and a row's chunks, read 16 at a time, on 16 different slots.
  constexpr int kTileBytes = 2 * BM * BN;  // BM x BN, or 2 BM x BN / 2 when paired, fp16
  constexpr bool kStaged = MOE_S2_STAGED_OUT != 0 && kTileBytes <= S * STAGE;
  const int pitch = 2 * rw;               // bytes per row of the staged tile
  const int xm = (rw / 8 - 1) & 15;
  if constexpr (kStaged) __syncthreads();  // every wave is done with the ring
  _Float16* o = reinterpret_cast<_Float16*>(p.out);
#pragma unroll
  for (int b = 0; b < L::NBM; ++b) {
    const int m = xr0 + 32 * b + (l & 31);
    const bool valid = m < actual;
    if (FUSED && !valid) continue;
#pragma unroll
    for (int a = 0; a < L::NBN; ++a)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int nl = wn * L::WTN + 32 * a + 8 * rg + 4 * (l >> 5);  // feature within the tile
        const int n = n0 + nl;
        f32x4 sd = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (I8) sd = *reinterpret_cast<const f32x4*>(p.sd + (int64_t)e * p.H + n);
        f16x4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float y = (float)acc[a][b][4 * rg + q];
          if constexpr (I8 && !F8) y = y * shv[b];  // int8: ((acc * s_h[row]) * s_d[n]) * w
          if constexpr (I8) y = y * sd[q];
          // select, never multiply, so NaN/Inf garbage in padding rows cannot leak
          v[q] = valid ? (_Float16)(y * wr[b]) : (_Float16)0.0f;
        }
        if constexpr (kStaged)
          *reinterpret_cast<f16x4*>(smem + m * pitch + 16 * ((nl >> 3) ^ (m & xm)) + 2 * (nl & 7)) = v;
        else if constexpr (FUSED && MOE_S2_SCATTER) atomic_add_f16x4(o + orow[b] * p.H + n, v);
        else *reinterpret_cast<f16x4*>(o + orow[b] * p.H + n) = v;
      }
  }
  if constexpr (kStaged) {
    __syncthreads();
    // fused: the item's valid rows (the first `actual`) to their unpadded
    // expert-sorted rows; pre-routed: all rows, padding rows as the zeros above
    const int shift = __builtin_ctz(rw / 8);  // 16-byte chunks per row: rw / 8, a power of two
    const int rows_out = FUSED ? actual : rx;
    for (int idx = threadIdx.x; idx < rows_out << shift; idx += 64 * NW) {
      const int r = idx >> shift, c = idx & ((1 << shift) - 1);
      const u32x4 v = *reinterpret_cast<const u32x4*>(smem + r * pitch + 16 * (c ^ (r & xm)));
      if constexpr (FUSED && MOE_S2_SCATTER) {
        _Float16* dst = o + (int64_t)(p.sorted_ids[row0 + r] / p.topk) * p.H + n0 + 8 * c;
        atomic_add_f16x4(dst, __builtin_bit_cast(f16x4, u32x2{v[0], v[1]}));
        atomic_add_f16x4(dst + 4, __builtin_bit_cast(f16x4, u32x2{v[2], v[3]}));
      } else {
        const int64_t orr = FUSED ? (int64_t)go_e + (row0 - gpo_e) + r : (int64_t)(row0 + r);
        *reinterpret_cast<u32x4*>(o + orr * p.H + n0 + 8 * c) = v;
      }
    }
  }
  if constexpr (ABS) {
    // absorbed rows: stored directly (fused: their unpadded expert-sorted
    // rows; pre-routed: their padded rows, and the rest of their block as 0)
    if (awave && (l & 31) < nar) {
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int n = n0 + wn * L::WTN + 32 * aj + 8 * rg + 4 * (l >> 5);
        f16x4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = (_Float16)(aa[4 * rg + q] * awr);
        if constexpr (FUSED && MOE_S2_SCATTER) atomic_add_f16x4(o + aorow * p.H + n, v);
        else *reinterpret_cast<f16x4*>(o + aorow * p.H + n) = v;
      }
    }
    if (!FUSED && nar > 0) {
      for (int idx = threadIdx.x; idx < (BM - nar) * (rw / 8); idx += 64 * NW) {
        const int r = nar + idx / (rw / 8), c = idx % (rw / 8);
        *reinterpret_cast<u32x4*>(o + (int64_t)(w.ar0 + r) * p.H + n0 + 8 * c) = u32x4{0, 0, 0, 0};
      }
    }
  }
}

// LDS ring depth per tile: as many stages as fit the CU's 160 KiB (one
// workgroup per CU for the wide tiles) -- the stages in flight are what keeps
// enough bytes outstanding to stream weights at HBM rate.
// Compile-time tunables (-D...) with the measured defaults.
#ifndef MOE_S1_STAGES_128
#define MOE_S1_STAGES_128 3
#endif
#ifndef MOE_S1_STAGES_64
#define MOE_S1_STAGES_64 3
#endif
#ifndef MOE_S1_STAGES_32
#define MOE_S1_STAGES_32 4
#endif
#ifndef MOE_S2_STAGES_128
#define MOE_S2_STAGES_128 3
#endif
#ifndef MOE_S2_BN_128
#define MOE_S2_BN_128 256
#endif
#ifndef MOE_S2_STAGES_64
#define MOE_S2_STAGES_64 4
#endif
#ifndef MOE_S2_STAGES_32
#define MOE_S2_STAGES_32 4
#endif
constexpr int s1_stages(int bm) {
  return bm == 256 ? 2 : bm == 128 ? MOE_S1_STAGES_128 : (bm == 64 ? MOE_S1_STAGES_64 : MOE_S1_STAGES_32);
}
constexpr int s2_stages(int bm) {
  return bm == 256 ? 2 : bm == 128 ? MOE_S2_STAGES_128 : (bm == 64 ? MOE_S2_STAGES_64 : MOE_S2_STAGES_32);
}

// Waves per workgroup of the 128-row tiles (4 = one wave per SIMD; 8 = two,
// so one wave's LDS / barrier latency hides behind the other's MFMAs).
#ifndef MOE_S1_WAVES_128
#define MOE_S1_WAVES_128 8
#endif
#ifndef MOE_S2_WAVES_128
#define MOE_S2_WAVES_128 8
#endif

// Pair the blocks of multi-block experts (one weight-tile read per two
// blocks) in the 128-row instances; 0 turns pairing off.
#ifndef MOE_PAIR
#define MOE_PAIR 1
#endif
// fp16 Stage 1 of 32-row tiles: gate / up tile width of the narrow kernel
// (64 or 32; 0 = the 128-wide tiles) and its ring depth.
#ifndef MOE_S1_NARROW32
#define MOE_S1_NARROW32 32
#endif
#ifndef MOE_S1N_STAGES
#define MOE_S1N_STAGES 6
#endif

template <int BM, int WM, int NW, int QT, bool GATHER, bool PAIR>
static hipError_t go1(const Stage1Params& p, int64_t grid, hipStream_t s) {
  constexpr int kS = s1_stages(BM);
  hipLaunchKernelGGL((stage1_kernel<BM, WM, kS, NW, QT, GATHER, PAIR>), dim3((unsigned)grid),
                     dim3(64 * NW), 0, s, p);
  return hipGetLastError();
}

// Stage 2's K loop is short (I / 64 steps), so its wide-M tiles take a
// 256-wide N tile when H allows: half the workgroups, half the re-reads of the
// intermediate, and twice the work behind each workgroup's pipeline fill and
// epilogue.  Paired items are then 256 x 128.
template <int BM, int WM, int BN, int NW, int QT, bool FUSED, bool PAIR>
static hipError_t go2(const Stage2Params& p, int64_t max_blocks, hipStream_t s) {
  constexpr int kS = s2_stages(BM);
  const int64_t grid = schedule_grid(max_blocks, p.H / BN);
  if (grid <= 0) return hipSuccess;
  constexpr bool kStream = BM == 32 || (MOE_W8_STREAM != 0 && QT != kQF16 && BM == 256);
  hipLaunchKernelGGL((stage2_kernel<BM, WM, BN, kS, NW, QT, FUSED, PAIR, kStream>), dim3((unsigned)grid),
                     dim3(64 * NW), 0, s, p);
  return hipGetLastError();
}
template <int QT, bool FUSED>
static hipError_t go2_128(const Stage2Params& p, int64_t mb, hipStream_t s) {
  constexpr int NW = MOE_S2_WAVES_128;
  if (MOE_S2_BN_128 == 256 && p.H % 256 == 0) return go2<128, 2, 256, NW, QT, FUSED, MOE_PAIR != 0>(p, mb, s);
  return go2<128, 2, 128, NW, QT, FUSED, false>(p, mb, s);
}

hipError_t launch_stage1(const Stage1Params& params, int block_m, int qt, bool gather,
                         int64_t max_blocks, hipStream_t s) {
  Stage1Params p = params;
  p.host_blocks = (int)max_blocks;
  if (p.w_ld == 0) p.w_ld = p.H * (qt != kQF16 ? 1 : 2);
  if (p.w_es == 0) p.w_es = p.I * p.w_ld;
  if (p.h_ld == 0) p.h_ld = p.I;
  const int64_t grid = schedule_grid(max_blocks, p.I / kBN);
  if (grid <= 0) return hipSuccess;
  constexpr int NW = MOE_S1_WAVES_128;
  constexpr bool kPair = MOE_PAIR != 0;
  if (!gather) {
    if (block_m == 128 && qt == kQF16) return go1<128, 2, NW, kQF16, false, kPair>(p, grid, s);
    return hipErrorInvalidValue;
  }
  switch (block_m) {
    case 32:
      if (qt == kQI8) return go1<32, 1, 4, kQI8, true, false>(p, grid, s);
      if (qt == kQF8) return go1<32, 1, 4, kQF8, true, false>(p, grid, s);
      if constexpr (MOE_S1_NARROW32 != 0) {
        constexpr int kW = MOE_S1_NARROW32;
        const int64_t gn = schedule_grid(max_blocks, p.I / kW);
        hipLaunchKernelGGL((stage1_narrow_kernel<kW, MOE_S1N_STAGES>), dim3((unsigned)gn), dim3(256), 0, s, p);
        return hipGetLastError();
      }
      return go1<32, 1, 4, kQF16, true, false>(p, grid, s);
    case 64:
      if (qt == kQI8) return go1<64, 1, 4, kQI8, true, false>(p, grid, s);
      if (qt == kQF8) return go1<64, 1, 4, kQF8, true, false>(p, grid, s);
      return go1<64, 1, 4, kQF16, true, false>(p, grid, s);
    case 128:
      if (qt == kQI8) return go1<128, 2, NW, kQI8, true, kPair>(p, grid, s);
      if (qt == kQF8) return go1<128, 2, NW, kQF8, true, false>(p, grid, s);
      return go1<128, 2, NW, kQF16, true, kPair>(p, grid, s);
    case 256:
      // 256 token rows x (128 gate + 128 up) rows: two 64 KiB stages
      if (qt == kQI8) return go1<256, 4, 8, kQI8, true, false>(p, grid, s);
      if (qt == kQF8) return go1<256, 4, 8, kQF8, true, false>(p, grid, s);
      return go1<256, 4, 8, kQF16, true, false>(p, grid, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_stage2(const Stage2Params& params, int block_m, int qt, bool fused,
                         int64_t max_blocks, hipStream_t s) {
  Stage2Params p = params;
  p.host_blocks = (int)max_blocks;
  if (p.a_ld == 0) p.a_ld = p.I * (qt != kQF16 ? 1 : 2);
  if (p.wd_ld == 0) p.wd_ld = p.I * (qt != kQF16 ? 1 : 2);
  if (p.wd_es == 0) p.wd_es = p.H * p.wd_ld;
  const int64_t mb = max_blocks;
  if (!fused) {
    if (block_m == 128 && qt == kQF16) return go2_128<kQF16, false>(p, mb, s);
    return hipErrorInvalidValue;
  }
  switch (block_m) {
    case 32:
      if (qt == kQI8) return go2<32, 1, kBN, 4, kQI8, true, false>(p, mb, s);
      if (qt == kQF8) return go2<32, 1, kBN, 4, kQF8, true, false>(p, mb, s);
      return go2<32, 1, kBN, 4, kQF16, true, false>(p, mb, s);
    case 64:
      if (qt == kQI8) return go2<64, 1, kBN, 4, kQI8, true, false>(p, mb, s);
      if (qt == kQF8) return go2<64, 1, kBN, 4, kQF8, true, false>(p, mb, s);
      return go2<64, 1, kBN, 4, kQF16, true, false>(p, mb, s);
    case 128:
      if (qt == kQI8) return go2_128<kQI8, true>(p, mb, s);
      if (qt == kQF8) return go2_128<kQF8, true>(p, mb, s);
      return go2_128<kQF16, true>(p, mb, s);
    case 256:
      // 256 token rows x 256 weight rows: two 64 KiB stages (fp16: with the
      // absorbed rows, two 68 KiB stages)
      if (qt == kQF8 && p.H % 256 == 0) return go2<256, 4, 256, 8, kQF8, true, false>(p, mb, s);
      if (qt == kQI8 && p.H % 256 == 0) return go2<256, 4, 256, 8, kQI8, true, false>(p, mb, s);
      if (qt == kQF16 && p.H % 256 == 0) return go2<256, 4, 256, 8, kQF16, true, false>(p, mb, s);
      return hipErrorInvalidValue;
  }
  return hipErrorInvalidValue;
}

}  // namespace moe
