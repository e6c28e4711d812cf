// Load-path probe and encoder check (measurement and verification only; not
// part of the operator library).  The load-path probe
// streams tile rows through the same direct-to-LDS ring as the GEMM stages --
// DmaTile's global_load_lds_dwordx4 with the row swizzle, wait_stages,
// barrier_no_fence -- and does no compute, so its rate is the ceiling the
// stages' load path reaches for a given tile shape, row pitch and mix of L2
// hits.  Built into its own libmoe_probe.so; bench.py --probe-ring drives it.
//
// Workgroup g streams a private region: tile row r >= hit_rows is row r of
// stream_base + g * ROWS * pitch; rows r < hit_rows are rows of one shared
// hit region that every workgroup reads (L2 hits after the first touch), as a
// Stage 1 item's token rows are shared by the expert's other items.  K steps
// of 128 bytes, nk of them, from the start of each row.
#include "../moe_common.h"

namespace moe {

template <int ROWS, int NW, int S, bool NT>
__global__ __launch_bounds__(64 * NW) void ring_probe_kernel(const char* __restrict__ stream_base,
                                                              const char* __restrict__ hit_base, int64_t pitch,
                                                              int nk, int hit_rows, int* __restrict__ sink) {
  using LD = DmaTile<ROWS, NW>;
  constexpr int STAGE = ROWS * kRowBytes;
  static_assert(S >= 2 && S * STAGE <= 160 * 1024, "LDS ring exceeds the 160 KiB of a CU");
  __shared__ __attribute__((aligned(16))) char smem[S * STAGE];
  LD ld;
  const char* own = stream_base + (int64_t)blockIdx.x * ROWS * pitch;
#pragma unroll
  for (int i = 0; i < LD::NI; ++i) {
    const int r = LD::row_of(i);
    ld.set(i, (r < hit_rows ? hit_base : own) + (int64_t)r * pitch);
  }
  auto issue = [&](int buf, int k) {
    if constexpr (NT) ld.issue(smem + buf * STAGE, k, hit_rows);  // streamed rows non-temporal
    else ld.issue(smem + buf * STAGE, k);
  };
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) issue(s, s);
  int cur = 0;
  for (int k = 0; k < nk; ++k) {
    wait_stages<LD::NI, S - 2>(nk - 1 - k);
    barrier_no_fence();
    if (k + S - 1 < nk) issue(cur == 0 ? S - 1 : cur - 1, k + S - 1);
    cur = cur + 1 == S ? 0 : cur + 1;
  }
  wait_vmcnt<0>();
  barrier_no_fence();
  if (threadIdx.x == 0) sink[blockIdx.x] = *reinterpret_cast<const int*>(smem + (cur == 0 ? S - 1 : cur - 1) * STAGE);
}


// As ring_probe_kernel (384 rows, 8 waves, 3 stages), with the hit rows and
// the streamed rows issued by different waves: waves 0..3 load the first HIT
// tile rows (the shared region), waves 4..7 the other 384 - HIT rows, each
// group in the DmaTile layout of its own rows.  A wave's loads retire in
// order; here no wave holds hits queued behind misses.
template <int HIT>
__global__ __launch_bounds__(512) void ring_probe_split_kernel(const char* __restrict__ stream_base,
                                                                const char* __restrict__ hit_base, int64_t pitch,
                                                                int nk, int* __restrict__ sink) {
  constexpr int ROWS = 384, NW = 8, S = 3, TW = 4;
  constexpr int QT = HIT / (8 * TW), QW = (ROWS - HIT) / (8 * (NW - TW));
  static_assert(QT * 8 * TW == HIT && QW * 8 * (NW - TW) == ROWS - HIT, "row groups per wave");
  constexpr int STAGE = ROWS * kRowBytes;
  __shared__ __attribute__((aligned(16))) char smem[S * STAGE];
  const int w = wave_id(), l = lane_id();
  const bool tok = w < TW;
  const int wr = tok ? w : w - TW;   // wave index within its group
  const int nw = tok ? TW : NW - TW; // waves of its group
  const int q = tok ? QT : QW;
  const char* own = stream_base + (int64_t)blockIdx.x * ROWS * pitch;
  const char* src[QW > QT ? QW : QT];
  int dst[QW > QT ? QW : QT];
#pragma unroll
  for (int i = 0; i < (QW > QT ? QW : QT); ++i) {
    const int g = (tok ? 0 : HIT / 8) + nw * i + wr;  // row group (8 rows, 1 KiB of LDS)
    const int r = 8 * g + (l >> 3);
    src[i] = (tok ? hit_base : own) + (int64_t)r * pitch + (((l & 7) ^ swz(r)) << 4);
    dst[i] = 1024 * g;
  }
  auto issue = [&](int buf, int k) {
#pragma unroll
    for (int i = 0; i < (QW > QT ? QW : QT); ++i)
      if (i < q) dma_to_lds<16>(src[i] + (size_t)k * kRowBytes, smem + buf * STAGE + dst[i]);
  };
  auto wait = [&](int ahead) {
    if (tok) wait_stages<QT, S - 2>(ahead);
    else wait_stages<QW, S - 2>(ahead);
  };
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) issue(s, s);
  int cur = 0;
  for (int k = 0; k < nk; ++k) {
    wait(nk - 1 - k);
    barrier_no_fence();
    if (k + S - 1 < nk) issue(cur == 0 ? S - 1 : cur - 1, k + S - 1);
    cur = cur + 1 == S ? 0 : cur + 1;
  }
  wait_vmcnt<0>();
  barrier_no_fence();
  if (threadIdx.x == 0) sink[blockIdx.x] = *reinterpret_cast<const int*>(smem + (cur == 0 ? S - 1 : cur - 1) * STAGE);
}
}  // namespace moe

// variant: 0 / 1 = 384-row stages (the 128-row kernels' 128 + 256 or 256 + 128
// rows), 8 waves, 3 stages, default / non-temporal streamed rows; 2 / 3 =
// 96-row stages (the 32-row decode kernels' shape), 4 waves, 6 stages; 4 / 5 =
// 512-row stages (256 + 256 rows), 8 waves, 2 stages; 6 / 7 = the 384-row ring
// with hit rows and streamed rows issued by different waves (ring_probe_split_kernel),
// hit_rows 128 / 256 (fixed by the variant).
// stream_bytes / hit_bytes: sizes of the two regions (groups * rows * pitch
// and hit_rows * pitch at least); sink holds `groups` ints.  Returns 0, -1 for
// bad arguments (nothing launched), or the HIP error.
extern "C" int moe_probe_ring(int variant, const void* stream_base, int64_t stream_bytes, const void* hit_base,
                              int64_t hit_bytes, int64_t pitch, int nk, int hit_rows, int groups, int* sink,
                              void* stream) {
  const int rows = variant < 2 || variant > 5 ? 384 : (variant < 4 ? 96 : 512);
  if (variant == 6 || variant == 7) hit_rows = variant == 6 ? 128 : 256;
  if (variant < 0 || variant > 7 || !stream_base || !sink || groups <= 0 || nk <= 0 || pitch % 16 != 0 ||
      (int64_t)nk * moe::kRowBytes > pitch || hit_rows < 0 || hit_rows > rows || hit_rows % 8 != 0 ||
      (int64_t)groups * rows * pitch > stream_bytes || (hit_rows > 0 && (!hit_base || (int64_t)hit_rows * pitch > hit_bytes)))
    return -1;
  const hipStream_t s = (hipStream_t)stream;
  const char* sb = (const char*)stream_base;
  const char* hb = (const char*)hit_base;
  switch (variant) {
    case 0: hipLaunchKernelGGL((moe::ring_probe_kernel<384, 8, 3, false>), dim3(groups), dim3(512), 0, s, sb, hb, pitch, nk, hit_rows, sink); break;
    case 1: hipLaunchKernelGGL((moe::ring_probe_kernel<384, 8, 3, true>), dim3(groups), dim3(512), 0, s, sb, hb, pitch, nk, hit_rows, sink); break;
    case 2: hipLaunchKernelGGL((moe::ring_probe_kernel<96, 4, 6, false>), dim3(groups), dim3(256), 0, s, sb, hb, pitch, nk, hit_rows, sink); break;
    case 3: hipLaunchKernelGGL((moe::ring_probe_kernel<96, 4, 6, true>), dim3(groups), dim3(256), 0, s, sb, hb, pitch, nk, hit_rows, sink); break;
    case 4: hipLaunchKernelGGL((moe::ring_probe_kernel<512, 8, 2, false>), dim3(groups), dim3(512), 0, s, sb, hb, pitch, nk, hit_rows, sink); break;
    case 5: hipLaunchKernelGGL((moe::ring_probe_kernel<512, 8, 2, true>), dim3(groups), dim3(512), 0, s, sb, hb, pitch, nk, hit_rows, sink); break;
    case 6: hipLaunchKernelGGL((moe::ring_probe_split_kernel<128>), dim3(groups), dim3(512), 0, s, sb, hb, pitch, nk, sink); break;
    default: hipLaunchKernelGGL((moe::ring_probe_split_kernel<256>), dim3(groups), dim3(512), 0, s, sb, hb, pitch, nk, sink); break;
  }
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// fp8 encoder check: the library's f8_e4m3 (the gfx950 conversion
// instruction) against a bit-level restatement of OCP e4m3 with round to
// nearest even, for every float of magnitude <= 448.  Normals (>= 2^-6): the
// fp32 mantissa rounded to 3 bits (add 0x7FFFF plus the kept lsb, drop 20
// bits), the carry running into the exponent, rebiased from 127 to 7;
// subnormals: the round-to-even multiple of 2^-9.
// ---------------------------------------------------------------------------
namespace moe {
__device__ __forceinline__ uint32_t f8_e4m3_bits(float v) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t sign = (u >> 24) & 0x80u;
  const float a = __builtin_fabsf(v);
  uint32_t code;
  if (a >= 0.015625f) {
    const uint32_t au = __float_as_uint(a);
    code = ((au + 0x7FFFFu + ((au >> 20) & 1u)) >> 20) - (120u << 3);
    code = code > 0x7Eu ? 0x7Eu : code;
  } else {
    code = (uint32_t)__builtin_rintf(a * 512.0f);
  }
  return sign | code;
}

// thread t checks the 256 bit patterns [256 t, 256 t + 256); 2^24 threads
__global__ __launch_bounds__(256) void f8_check_kernel(unsigned long long* __restrict__ mismatches,
                                                        unsigned long long* __restrict__ compared) {
  const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  unsigned long long bad = 0, seen = 0;
  for (uint32_t i = 0; i < 256; i += 4) {
    float v[4];
    bool in[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = __uint_as_float((uint32_t)(t * 256 + i + j));
      in[j] = __builtin_fabsf(v[j]) <= 448.0f;  // false for NaN
    }
    const uint32_t packed = f8_e4m3x4(v[0], v[1], v[2], v[3]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!in[j]) continue;
      ++seen;
      const uint32_t ref = f8_e4m3_bits(v[j]);
      if (f8_e4m3(v[j]) != ref || ((packed >> (8 * j)) & 0xffu) != ref) ++bad;
    }
  }
  atomicAdd(compared, seen);
  if (bad) atomicAdd(mismatches, bad);
}
}  // namespace moe

// Counts, over every float of magnitude <= 448 (2 * (0x43E00000 + 1) of
// them), the values whose code from f8_e4m3 or from the packed f8_e4m3x4
// differs from the bit-level restatement.  Both counters are added to (the
// caller zeroes them).  Returns 0 or the HIP error.
extern "C" int moe_probe_f8_encoder(unsigned long long* mismatches, unsigned long long* compared, void* stream) {
  if (!mismatches || !compared) return -1;
  hipLaunchKernelGGL(moe::f8_check_kernel, dim3(1u << 16), dim3(256), 0, (hipStream_t)stream, mismatches, compared);
  return (int)hipGetLastError();
}
