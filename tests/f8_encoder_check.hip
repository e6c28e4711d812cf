// Test infrastructure (not part of the operator library): the fp8 encoder of
// the kernels, f8_e4m3 / f8_e4m3x4 in muxi_race_amd/csrc/moe_common.h (the
// gfx950 conversion instruction v_cvt_pk_fp8_f32 on the input clamped to
// +-448), checked against a bit-level restatement of OCP e4m3 with round to
// nearest even, for every float of magnitude <= 448.  Built into
// tests/libf8check.so by tests/_native.py; tests/test_gpu_fp8.py runs it.
//
// Restatement.  Normals (>= 2^-6): the fp32 mantissa rounded to 3 bits (add
// 0x7FFFF plus the kept lsb, drop 20 bits), the carry running into the
// exponent, rebiased from 127 to 7, saturating at code 0x7E (448).
// Subnormals: the round-to-even multiple of 2^-9.
#include "../muxi_race_amd/csrc/moe_common.h"

namespace {

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
// cover all 2^32 patterns
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
    const uint32_t packed = moe::f8_e4m3x4(v[0], v[1], v[2], v[3]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!in[j]) continue;
      ++seen;
      const uint32_t ref = f8_e4m3_bits(v[j]);
      if (moe::f8_e4m3(v[j]) != ref || ((packed >> (8 * j)) & 0xffu) != ref) ++bad;
    }
  }
  atomicAdd(compared, seen);
  if (bad) atomicAdd(mismatches, bad);
}

}  // namespace

// Counts, over every float of magnitude <= 448 (2 * (0x43E00000 + 1) of
// them), the values whose code from f8_e4m3 or from the packed f8_e4m3x4
// differs from the bit-level restatement.  Both counters are added to (the
// caller zeroes them).  Returns 0 or the HIP error.
extern "C" int f8_encoder_check(unsigned long long* mismatches, unsigned long long* compared, void* stream) {
  if (!mismatches || !compared) return -1;
  hipLaunchKernelGGL(f8_check_kernel, dim3(1u << 16), dim3(256), 0, (hipStream_t)stream, mismatches, compared);
  return (int)hipGetLastError();
}
