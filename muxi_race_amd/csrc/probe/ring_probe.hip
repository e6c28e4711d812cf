// Load-path probe (measurement only; not part of the operator library): it
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

}  // namespace moe

// variant: 0 / 1 = 384-row stages (the 128-row kernels' 128 + 256 or 256 + 128
// rows), 8 waves, 3 stages, default / non-temporal streamed rows; 2 / 3 =
// 96-row stages (the 32-row decode kernels' shape), 4 waves, 6 stages; 4 / 5 =
// 512-row stages (256 + 256 rows), 8 waves, 2 stages.
// stream_bytes / hit_bytes: sizes of the two regions (groups * rows * pitch
// and hit_rows * pitch at least); sink holds `groups` ints.  Returns 0, -1 for
// bad arguments (nothing launched), or the HIP error.
extern "C" int moe_probe_ring(int variant, const void* stream_base, int64_t stream_bytes, const void* hit_base,
                              int64_t hit_bytes, int64_t pitch, int nk, int hit_rows, int groups, int* sink,
                              void* stream) {
  const int rows = variant < 2 ? 384 : (variant < 4 ? 96 : 512);
  if (variant < 0 || variant > 5 || !stream_base || !sink || groups <= 0 || nk <= 0 || pitch % 16 != 0 ||
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
    default: hipLaunchKernelGGL((moe::ring_probe_kernel<512, 8, 2, true>), dim3(groups), dim3(512), 0, s, sb, hb, pitch, nk, hit_rows, sink); break;
  }
  return (int)hipGetLastError();
}
