// Exhaustive check of the library's paired f32 -> bf16 conversion (f32x2_to_bf16x2_bits, gfx950's
// v_cvt_pk_bf16_f32) against its integer rounding (f32_to_bf16_bits: nearest even, NaN kept quiet
// with its sign and top payload bits) over all 2^32 f32 bit patterns, both halves of the pair.
// Prints the mismatch counts (non-NaN inputs, NaN inputs) and one example; exit status 0 when both
// are zero.  Built by burn-extended_amd/build.py (build_checks) into lib/checks/; run by
// tests/test_gpu_convert.py.
#include <hip/hip_runtime.h>

#include <cstdio>

#include "../../burn-extended_amd/csrc/mx_device.hpp"

namespace {

__global__ void check_kernel(uint64_t base, unsigned long long *cnt, uint32_t *ex) {
  const uint64_t i = base + ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 2u;
  const uint32_t u[2] = {(uint32_t)i, (uint32_t)(i + 1u)};
  const uint32_t hw = burnext::f32x2_to_bf16x2_bits(__uint_as_float(u[0]), __uint_as_float(u[1]));
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint16_t got = (uint16_t)(hw >> (16 * h)), want = burnext::f32_to_bf16_bits(__uint_as_float(u[h]));
    if (got != want) {
      const bool nan = (u[h] & 0x7FFFFFFFu) > 0x7F800000u;
      atomicAdd(&cnt[nan ? 1 : 0], 1ull);
      ex[0] = u[h];
      ex[1] = ((uint32_t)got << 16) | want;
    }
  }
}

bool ok(hipError_t e, const char *what) {
  if (e != hipSuccess) std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return e == hipSuccess;
}

}  // namespace

int main() {
  unsigned long long *cnt = nullptr;
  uint32_t *ex = nullptr;
  if (!ok(hipMalloc(&cnt, 2 * sizeof(unsigned long long)), "hipMalloc") || !ok(hipMalloc(&ex, 8), "hipMalloc") ||
      !ok(hipMemset(cnt, 0, 2 * sizeof(unsigned long long)), "hipMemset") || !ok(hipMemset(ex, 0, 8), "hipMemset"))
    return 2;
  const uint64_t per = 1ull << 28;  // f32 patterns per launch: 2^27 threads of two
  for (uint64_t b = 0; b < (1ull << 32); b += per) {
    hipLaunchKernelGGL(check_kernel, dim3((unsigned)(per / 2 / 256)), dim3(256), 0, 0, b, cnt, ex);
    if (!ok(hipGetLastError(), "launch")) return 2;
  }
  unsigned long long h[2];
  uint32_t e[2];
  if (!ok(hipMemcpy(h, cnt, sizeof(h), hipMemcpyDeviceToHost), "hipMemcpy") ||
      !ok(hipMemcpy(e, ex, sizeof(e), hipMemcpyDeviceToHost), "hipMemcpy"))
    return 2;
  std::printf("bf16 pair convert vs integer rounding over 2^32 inputs: mismatches non-NaN %llu NaN %llu (example "
              "input %08x: got %04x want %04x)\n",
              h[0], h[1], e[0], e[1] >> 16, e[1] & 0xFFFFu);
  hipFree(cnt);
  hipFree(ex);
  return (h[0] == 0 && h[1] == 0) ? 0 : 1;
}
