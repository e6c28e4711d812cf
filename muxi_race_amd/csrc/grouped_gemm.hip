// Grouped expert GEMMs for gfx950: Stage 1 (gate/up + SiLU*up) and Stage 2
// (down projection * routing weight), fp16 MFMA (v_mfma_f32_32x32x16_f16) and
// int8 MFMA (v_mfma_i32_32x32x32_i8).
//
// Reference algorithm: 初审材料/源代码/submission.py Stage1 family (:136-247,
// :1391-1635) and Stage2 family (:655-795, :1132-1378); base form
// xpuoj_data/submission.py:31-129 and :253-331.  The tiling here is this
// build's own: a 256-thread workgroup computes a BM x 128 output tile (Stage 1:
// for gate and up at once, sharing the token tile); K advances 128 bytes per
// step through an S-stage ring of XOR-swizzled LDS tiles filled by direct
// global->LDS loads (global_load_lds_dwordx4), so S-2 steps of loads stay in
// flight behind the MFMAs of the current step, with one barrier per step.
#include "launch.h"
#include "moe_common.h"

#include <type_traits>

namespace moe {

template <int BM, int WAVES_M, int BN, int NW>
struct Layout {
  static constexpr int WAVES_N = NW / WAVES_M;
  static constexpr int WTM = BM / WAVES_M;   // tokens per wave
  static constexpr int WTN = BN / WAVES_N;   // output features per wave
  static constexpr int NBM = WTM / 32;
  static constexpr int NBN = WTN / 32;
  static_assert(NBM >= 1 && NBN >= 1, "wave tile must hold at least one 32x32 block");
};

template <int BM, int WAVES_M, int S, int NW, bool I8, bool GATHER>
__global__ __launch_bounds__(64 * NW) void stage1_kernel(Stage1Params p) {
  using L = Layout<BM, WAVES_M, kBN, NW>;
  using Acc = typename std::conditional<I8, i32x16, f32x16>::type;
  constexpr int XB = BM * kRowBytes;
  constexpr int WB = kBN * kRowBytes;
  constexpr int STAGE = XB + 2 * WB;
  static_assert(S >= 2 && S * STAGE <= 160 * 1024, "LDS ring exceeds the 160 KiB of a CU");
  __shared__ __attribute__((aligned(16))) char smem[S * STAGE];

  const int ntiles = (int)(p.I / kBN);
  Work w;
  if (!schedule(blockIdx.x, p.gpo, p.E, BM, ntiles, p.host_blocks, false, w)) return;
  const int e = w.e;
  const int gpo_e = p.gpo[e];
  const int row0 = w.m_block * BM;
  const int n0 = w.n_tile * kBN;
  int actual = p.gs[e] - (row0 - gpo_e);
  actual = actual < 0 ? 0 : (actual > BM ? BM : actual);
  if (actual == 0) return;  // empty block: intermediate rows left untouched

  const int64_t kbytes = p.H * (I8 ? 1 : 2);
  const int nk = (int)(kbytes / kRowBytes);

  DmaTile<BM, NW> xl;
  DmaTile<kBN, NW> gl, ul;
#pragma unroll
  for (int i = 0; i < DmaTile<BM, NW>::NI; ++i) {
    const int r = DmaTile<BM, NW>::row_of(i);
    int64_t src_row;
    if (GATHER) {
      const int pid = r < actual ? p.sorted_ids[row0 + r] : 0;
      src_row = pid / p.topk;
    } else {
      src_row = row0 + r;
    }
    xl.set(i, p.x + src_row * kbytes);
  }
  const char* gbase = p.wg + ((int64_t)e * p.I + n0) * kbytes;
  const char* ubase = p.wu + ((int64_t)e * p.I + n0) * kbytes;
#pragma unroll
  for (int i = 0; i < DmaTile<kBN, NW>::NI; ++i) {
    const int r = DmaTile<kBN, NW>::row_of(i);
    gl.set(i, gbase + r * kbytes);
    ul.set(i, ubase + r * kbytes);
  }

  const int wave = threadIdx.x >> 6;
  const int wm = wave / L::WAVES_N;
  const int wn = wave % L::WAVES_N;
  // 32-row token blocks of this wave that hold at least one routed row
  // (wave-uniform); padding-only blocks skip their LDS reads and MFMAs.
  // (Skipping costs L2 sharing between the M blocks of one expert -- a block
  // with less MFMA work runs ahead of its siblings -- but measured faster
  // overall than keeping siblings in step.)
  const int live = (actual - wm * L::WTM + 31) / 32;
  Acc ag[L::NBN][L::NBM], au[L::NBN][L::NBM];
#pragma unroll
  for (int a = 0; a < L::NBN; ++a)
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) {
      ag[a][b] = Acc{};
      au[a][b] = Acc{};
    }

  // S-stage ring: stages ks+1 .. ks+S-2 stay in flight while stage ks is used.
  constexpr int Q = DmaTile<BM, NW>::NI + 2 * DmaTile<kBN, NW>::NI;  // loads per wave per stage
  auto issue = [&](int buf, int k) {
    char* st = smem + buf * STAGE;
    xl.issue(st, k);
    gl.issue(st + XB, k);
    ul.issue(st + XB + WB, k);
  };
  // The K loop is instantiated per count NB of this wave's token blocks that
  // hold routed rows (chosen once, outside the loop: a branch inside it would
  // move the accumulators out of AGPRs every step); padding-only blocks get no
  // LDS reads and no MFMAs.  Every variant issues the same loads and barriers.
  auto main_loop = [&](auto nb_c) {
    constexpr int NB = decltype(nb_c)::value;
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
      if (s < nk) issue(s, s);
    int cur = 0;
    for (int ks = 0; ks < nk; ++ks) {
      wait_stages<Q, S - 2>(nk - 1 - ks);
      barrier_no_fence();
      if (ks + S - 1 < nk) issue(cur == 0 ? S - 1 : cur - 1, ks + S - 1);
      const char* cx = smem + cur * STAGE;
      const char* cg = cx + XB;
      const char* cu = cg + WB;
      cur = cur + 1 == S ? 0 : cur + 1;
      if constexpr (NB > 0) {
        // Fragments double-buffered across the 4 K sub-steps: the LDS reads of
        // sub-step s+1 are in flight while the MFMAs of sub-step s run.
        u32x4 xf[2][NB], gf[2][L::NBN], uf[2][L::NBN];
        auto load_frags = [&](int buf, int s) {
#pragma unroll
          for (int b = 0; b < NB; ++b) xf[buf][b] = frag(cx, wm * L::WTM + 32 * b, s);
#pragma unroll
          for (int a = 0; a < L::NBN; ++a) {
            gf[buf][a] = frag(cg, wn * L::WTN + 32 * a, s);
            uf[buf][a] = frag(cu, wn * L::WTN + 32 * a, s);
          }
        };
        load_frags(0, 0);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int fb = s & 1;
          if (s < 3) load_frags(fb ^ 1, s + 1);
          __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
          for (int a = 0; a < L::NBN; ++a)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              ag[a][b] = mma(gf[fb][a], xf[fb][b], ag[a][b]);
              au[a][b] = mma(uf[fb][a], xf[fb][b], au[a][b]);
            }
        }
      }
    }
  };
  if (live >= L::NBM) main_loop(std::integral_constant<int, L::NBM>{});
  else if (L::NBM > 1 && live >= 1) main_loop(std::integral_constant<int, 1>{});
  else main_loop(std::integral_constant<int, 0>{});
  __syncthreads();  // every wave is done with the ring before LDS is reused

  const int l = lane_id();
  if constexpr (!I8) {
    // h = silu(g) * u -> fp16, valid rows only (submission.py:1532-1542).
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) {
      const int m = wm * L::WTM + 32 * b + (l & 31);
      if (m < actual) {
        _Float16* hrow = reinterpret_cast<_Float16*>(p.h) + (int64_t)(row0 + m) * p.I;
#pragma unroll
        for (int a = 0; a < L::NBN; ++a)
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const int n = n0 + wn * L::WTN + 32 * a + 8 * rg + 4 * (l >> 5);
            f16x4 v;
#pragma unroll
            for (int q = 0; q < 4; ++q)
              v[q] = (_Float16)silu_mul(ag[a][b][4 * rg + q], au[a][b][4 * rg + q]);
            *reinterpret_cast<f16x4*>(hrow + n) = v;
          }
      }
    }
  } else {
    // Dequantise (acc * s_x[token]) * s_w[e, n], h = silu(g) * u, then quantise
    // h per (row, this 128-column tile): amax over the tile's columns, which
    // are spread over the lane pair (l, l^32) and the WAVES_N waves.
    float* red = reinterpret_cast<float*>(smem);  // [WAVES_N][BM]; loop ended with a barrier
    float hv[L::NBM][L::NBN][16];
    const float* sgrow = p.sg + (int64_t)e * p.I;
    const float* surow = p.su + (int64_t)e * p.I;
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) {
      const int m = wm * L::WTM + 32 * b + (l & 31);
      float sx = 0.0f;
      if (m < actual) sx = p.x_scale[p.sorted_ids[row0 + m] / p.topk];
      float amax = 0.0f;
#pragma unroll
      for (int a = 0; a < L::NBN; ++a)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const int n = n0 + wn * L::WTN + 32 * a + 8 * rg + 4 * (l >> 5);
          const f32x4 sgv = *reinterpret_cast<const f32x4*>(sgrow + n);
          const f32x4 suv = *reinterpret_cast<const f32x4*>(surow + n);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float g = ((float)ag[a][b][4 * rg + q] * sx) * sgv[q];
            const float u = ((float)au[a][b][4 * rg + q] * sx) * suv[q];
            const float h = silu_mul(g, u);
            hv[b][a][4 * rg + q] = h;
            amax = fmaxf(amax, fabsf(h));
          }
        }
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      if (l < 32) red[wn * BM + wm * L::WTM + 32 * b + l] = amax;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) {
      const int mrow = wm * L::WTM + 32 * b + (l & 31);
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < L::WAVES_N; ++j) amax = fmaxf(amax, red[j * BM + mrow]);
      const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
      if (mrow < actual) {
        const int64_t grow = row0 + mrow;
        int8_t* hrow = reinterpret_cast<int8_t*>(p.h) + grow * p.I;
#pragma unroll
        for (int a = 0; a < L::NBN; ++a)
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            const int n = n0 + wn * L::WTN + 32 * a + 8 * rg + 4 * (l >> 5);
            uint32_t packed = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int qv = quant_i8(hv[b][a][4 * rg + q], inv);
              packed |= (uint32_t)(qv & 0xff) << (8 * q);
            }
            *reinterpret_cast<uint32_t*>(hrow + n) = packed;
          }
        // scales are stored block-major: [I/128][hs_stride]
        if (wn == 0 && l < 32) p.h_scale[(int64_t)w.n_tile * p.hs_stride + grow] = amax / 127.0f;
      }
    }
  }
}

template <int BM, int WAVES_M, int BN, int S, int NW, bool I8, bool FUSED>
__global__ __launch_bounds__(64 * NW) void stage2_kernel(Stage2Params p) {
  using L = Layout<BM, WAVES_M, BN, NW>;
  constexpr int XB = BM * kRowBytes;
  constexpr int WB = BN * kRowBytes;
  constexpr int STAGE = XB + WB + (I8 ? 256 * NW : 0);  // int8: + row scales of the step
  static_assert(S >= 2 && S * STAGE <= 160 * 1024, "LDS ring exceeds the 160 KiB of a CU");
  __shared__ __attribute__((aligned(16))) char smem[S * STAGE];

  const int ntiles = (int)(p.H / BN);
  Work w;
  if (!schedule(blockIdx.x, p.gpo, p.E, BM, ntiles, p.host_blocks, !FUSED, w)) return;
  const int row0 = w.m_block * BM;
  const int n0 = w.n_tile * BN;
  int actual = 0, gpo_e = 0, go_e = 0;
  const int e = w.e;
  if (e >= 0) {
    gpo_e = p.gpo[e];
    go_e = FUSED ? 0 : p.go[e];
    actual = p.gs[e] - (row0 - gpo_e);
    actual = actual < 0 ? 0 : (actual > BM ? BM : actual);
  }
  if (actual == 0) {
    if (!FUSED) {
      // Rows owned by no valid token are written as 0 (problem_detail.json:50 note 4).
      _Float16* o = reinterpret_cast<_Float16*>(p.out);
      for (int idx = threadIdx.x; idx < BM * (BN / 8); idx += 64 * NW) {
        const int r = idx / (BN / 8), c = idx % (BN / 8);
        *reinterpret_cast<u32x4*>(o + (int64_t)(row0 + r) * p.H + n0 + 8 * c) = u32x4{0, 0, 0, 0};
      }
    }
    return;
  }

  const int64_t kbytes = p.I * (I8 ? 1 : 2);
  const int nk = (int)(kbytes / kRowBytes);
  DmaTile<BM, NW> al;
  DmaTile<BN, NW> wl;
#pragma unroll
  for (int i = 0; i < DmaTile<BM, NW>::NI; ++i)
    al.set(i, p.a + (int64_t)(row0 + DmaTile<BM, NW>::row_of(i)) * kbytes);
  const char* wbase = p.wd + ((int64_t)e * p.H + n0) * kbytes;
#pragma unroll
  for (int i = 0; i < DmaTile<BN, NW>::NI; ++i) wl.set(i, wbase + DmaTile<BN, NW>::row_of(i) * kbytes);

  const int wave = threadIdx.x >> 6;
  const int wm = wave / L::WAVES_N;
  const int wn = wave % L::WAVES_N;
  const int l = lane_id();
  const int live = (actual - wm * L::WTM + 31) / 32;  // see Stage 1
  f32x16 acc[L::NBN][L::NBM];
#pragma unroll
  for (int a = 0; a < L::NBN; ++a)
#pragma unroll
    for (int b = 0; b < L::NBM; ++b) acc[a][b] = f32x16{};

  // int8: the row scales of K step ks (block-major layout, so contiguous) ride
  // in the same stage: wave w loads rows 64w..64w+63 (clamped inside the tile)
  // with one dword DMA, so every wave issues the same number of loads.
  const float* scale_src = nullptr;
  if constexpr (I8) {
    const int r = 64 * wave_id() + l;
    scale_src = p.a_scale + row0 + (r < BM ? r : 0);
  }
  constexpr int Q = DmaTile<BM, NW>::NI + DmaTile<BN, NW>::NI + (I8 ? 1 : 0);
  auto issue = [&](int buf, int k) {
    char* st = smem + buf * STAGE;
    al.issue(st, k);
    wl.issue(st + XB, k);
    if constexpr (I8)
      dma_to_lds<4>(scale_src + (int64_t)k * p.as_stride, st + XB + WB + 256 * wave_id());
  };
  // K loop instantiated per count of live token blocks (see Stage 1).
  auto main_loop = [&](auto nb_c) {
    constexpr int NB = decltype(nb_c)::value;
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
      if (s < nk) issue(s, s);
    int cur = 0;
    for (int ks = 0; ks < nk; ++ks) {
      wait_stages<Q, S - 2>(nk - 1 - ks);
      barrier_no_fence();
      if (ks + S - 1 < nk) issue(cur == 0 ? S - 1 : cur - 1, ks + S - 1);
      const char* ca = smem + cur * STAGE;
      const char* cw = ca + XB;
      cur = cur + 1 == S ? 0 : cur + 1;
      if constexpr (NB > 0) {
        u32x4 af[2][NB], wf[2][L::NBN];
        auto load_frags = [&](int buf, int s) {
#pragma unroll
          for (int b = 0; b < NB; ++b) af[buf][b] = frag(ca, wm * L::WTM + 32 * b, s);
#pragma unroll
          for (int a = 0; a < L::NBN; ++a) wf[buf][a] = frag(cw, wn * L::WTN + 32 * a, s);
        };
        if constexpr (!I8) {
          load_frags(0, 0);
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int fb = s & 1;
            if (s < 3) load_frags(fb ^ 1, s + 1);
            __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
            for (int a = 0; a < L::NBN; ++a)
#pragma unroll
              for (int b = 0; b < NB; ++b) acc[a][b] = mma(wf[fb][a], af[fb][b], acc[a][b]);
          }
        } else {
          // One K step of int8 is one 128-column scale block of the
          // intermediate: exact int32 partial product, then
          // acc += partial * s_h[row, block].
          const float* scl = reinterpret_cast<const float*>(cw + WB);
          float sc[NB];
#pragma unroll
          for (int b = 0; b < NB; ++b) sc[b] = scl[wm * L::WTM + 32 * b + (l & 31)];
          i32x16 ia[L::NBN][NB];
#pragma unroll
          for (int a = 0; a < L::NBN; ++a)
#pragma unroll
            for (int b = 0; b < NB; ++b) ia[a][b] = i32x16{};
          load_frags(0, 0);
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int fb = s & 1;
            if (s < 3) load_frags(fb ^ 1, s + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int a = 0; a < L::NBN; ++a)
#pragma unroll
              for (int b = 0; b < NB; ++b) ia[a][b] = mma(wf[fb][a], af[fb][b], ia[a][b]);
          }
#pragma unroll
          for (int a = 0; a < L::NBN; ++a)
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
              for (int r = 0; r < 16; ++r) acc[a][b][r] += (float)ia[a][b][r] * sc[b];
        }
      }
    }
  };
  if (live >= L::NBM) main_loop(std::integral_constant<int, L::NBM>{});
  else if (L::NBM > 1 && live >= 1) main_loop(std::integral_constant<int, 1>{});
  else main_loop(std::integral_constant<int, 0>{});

  _Float16* o = reinterpret_cast<_Float16*>(p.out);
#pragma unroll
  for (int b = 0; b < L::NBM; ++b) {
    const int m = wm * L::WTM + 32 * b + (l & 31);
    const bool valid = m < actual;
    float wr = 0.0f;
    int64_t orow = row0 + m;
    if (valid) {
      if (FUSED) {
        const int pid = p.sorted_ids[row0 + m];
        wr = reinterpret_cast<const float*>(p.routed)[pid];
        orow = pid;
      } else {
        // raw-order index (problem_detail.json:50 note 2), clamped to the
        // buffer as submission.py:1286-1288 does
        int64_t ridx = (int64_t)go_e + (row0 - gpo_e) + m;
        ridx = ridx >= p.V ? p.V - 1 : ridx;
        ridx = ridx < 0 ? 0 : ridx;
        if (p.V > 0)
          wr = p.routed_f16 ? (float)reinterpret_cast<const _Float16*>(p.routed)[ridx]
                            : reinterpret_cast<const float*>(p.routed)[ridx];
      }
    }
    if (FUSED && !valid) continue;
#pragma unroll
    for (int a = 0; a < L::NBN; ++a)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int n = n0 + wn * L::WTN + 32 * a + 8 * rg + 4 * (l >> 5);
        f32x4 sd = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (I8) sd = *reinterpret_cast<const f32x4*>(p.sd + (int64_t)e * p.H + n);
        f16x4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float y = acc[a][b][4 * rg + q];
          if constexpr (I8) y = y * sd[q];
          // select, never multiply, so NaN/Inf garbage in padding rows cannot leak
          v[q] = valid ? (_Float16)(y * wr) : (_Float16)0.0f;
        }
        *reinterpret_cast<f16x4*>(o + orow * p.H + n) = v;
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
  return bm == 128 ? MOE_S1_STAGES_128 : (bm == 64 ? MOE_S1_STAGES_64 : MOE_S1_STAGES_32);
}
constexpr int s2_stages(int bm) {
  return bm == 128 ? MOE_S2_STAGES_128 : (bm == 64 ? MOE_S2_STAGES_64 : MOE_S2_STAGES_32);
}

// Waves per workgroup of the 128-row tiles (4 = one wave per SIMD; 8 = two,
// so one wave's LDS / barrier latency hides behind the other's MFMAs).
#ifndef MOE_S1_WAVES_128
#define MOE_S1_WAVES_128 8
#endif
#ifndef MOE_S2_WAVES_128
#define MOE_S2_WAVES_128 8
#endif

template <int BM, int WM, int NW, bool I8, bool GATHER>
static hipError_t go1(const Stage1Params& p, int64_t grid, hipStream_t s) {
  constexpr int kS = s1_stages(BM);
  hipLaunchKernelGGL((stage1_kernel<BM, WM, kS, NW, I8, GATHER>), dim3((unsigned)grid),
                     dim3(64 * NW), 0, s, p);
  return hipGetLastError();
}

// Stage 2's K loop is short (I / 64 steps), so its wide-M tiles take a
// 256-wide N tile when H allows: half the workgroups, half the re-reads of the
// intermediate, and twice the work behind each workgroup's pipeline fill and
// epilogue.
template <int BM, int WM, int BN, int NW, bool I8, bool FUSED>
static hipError_t go2(const Stage2Params& p, int64_t max_blocks, hipStream_t s) {
  constexpr int kS = s2_stages(BM);
  const int64_t grid = schedule_grid(max_blocks, p.H / BN);
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL((stage2_kernel<BM, WM, BN, kS, NW, I8, FUSED>), dim3((unsigned)grid),
                     dim3(64 * NW), 0, s, p);
  return hipGetLastError();
}
template <bool I8, bool FUSED>
static hipError_t go2_128(const Stage2Params& p, int64_t mb, hipStream_t s) {
  constexpr int NW = MOE_S2_WAVES_128;
  if (MOE_S2_BN_128 == 256 && p.H % 256 == 0) return go2<128, 2, 256, NW, I8, FUSED>(p, mb, s);
  return go2<128, 2, 128, NW, I8, FUSED>(p, mb, s);
}

hipError_t launch_stage1(const Stage1Params& params, int block_m, bool int8, bool gather,
                         int64_t max_blocks, hipStream_t s) {
  Stage1Params p = params;
  p.host_blocks = (int)max_blocks;
  const int64_t grid = schedule_grid(max_blocks, p.I / kBN);
  if (grid <= 0) return hipSuccess;
  constexpr int NW = MOE_S1_WAVES_128;
  if (!gather) {
    if (block_m == 128 && !int8) return go1<128, 2, NW, false, false>(p, grid, s);
    return hipErrorInvalidValue;
  }
  switch (block_m) {
    case 32: return int8 ? go1<32, 1, 4, true, true>(p, grid, s) : go1<32, 1, 4, false, true>(p, grid, s);
    case 64: return int8 ? go1<64, 1, 4, true, true>(p, grid, s) : go1<64, 1, 4, false, true>(p, grid, s);
    case 128: return int8 ? go1<128, 2, NW, true, true>(p, grid, s) : go1<128, 2, NW, false, true>(p, grid, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_stage2(const Stage2Params& params, int block_m, bool int8, bool fused,
                         int64_t max_blocks, hipStream_t s) {
  Stage2Params p = params;
  p.host_blocks = (int)max_blocks;
  const int64_t mb = max_blocks;
  if (!fused) {
    if (block_m == 128 && !int8) return go2_128<false, false>(p, mb, s);
    return hipErrorInvalidValue;
  }
  switch (block_m) {
    case 32: return int8 ? go2<32, 1, kBN, 4, true, true>(p, mb, s) : go2<32, 1, kBN, 4, false, true>(p, mb, s);
    case 64: return int8 ? go2<64, 1, kBN, 4, true, true>(p, mb, s) : go2<64, 1, kBN, 4, false, true>(p, mb, s);
    case 128: return int8 ? go2_128<true, true>(p, mb, s) : go2_128<false, true>(p, mb, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace moe
