// mfma_clock_probe.hip — the bf16 matrix-core rate this MI355X sustains, and
// the shader clock it runs at, as a function of the operand data.
//
// A measurement aid for the attention kernels' roofline, not part of the
// library: four 4-wave workgroups per CU (four waves per SIMD) each issue
// back-to-back v_mfma_f32_32x32x16_bf16 on four independent accumulators.
// The operands are either one constant bf16 value or random bf16 values
// (random sign and mantissa, exponents in [2^-7, 2^0)) rotated every
// iteration.  Every workgroup records s_memtime (shader clock) and
// s_memrealtime (100 MHz) around its loop, so the run reports the average
// shader clock beside the TFLOP/s.
//
// Built by `make probe` (the library's flags) into _build/mfma_clock_probe.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                            \
  do {                                                                      \
    hipError_t e_ = (x);                                                    \
    if (e_ != hipSuccess) {                                                 \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));          \
      std::exit(1);                                                         \
    }                                                                       \
  } while (0)

namespace {

constexpr int kThreads = 256;
constexpr int kMfmaPerIter = 16;

// Two random bf16 values in one word (a linear congruential step per call).
__device__ unsigned random_bf16x2(unsigned& state) {
  state = state * 1664525u + 1013904223u;
  const unsigned lo = ((state >> 8) & 0x807fu) | ((120u + ((state >> 4) & 7u)) << 7);
  const unsigned hi = ((state >> 16) & 0x807fu) | ((120u + ((state >> 24) & 7u)) << 7);
  return lo | (hi << 16);
}

template <bool RANDOM>
__global__ __launch_bounds__(kThreads) void mfma_loop(float* sink, unsigned long long* stamps,
                                                      int iters) {
  unsigned state = (blockIdx.x * kThreads + threadIdx.x) * 2654435761u + 12345u;
  u32x4 a[4], b[4];
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) {
      a[i][j] = RANDOM ? random_bf16x2(state) : 0x3f803f80u;  // 1.0 when constant
      b[i][j] = RANDOM ? random_bf16x2(state) : 0x3f803f80u;
    }
  f32x16 acc[4] = {f32x16{}, f32x16{}, f32x16{}, f32x16{}};
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // opaque to the optimiser, so that no MFMA is hoisted out of the loop
      asm volatile("" : "+v"(a[i]), "+v"(b[i]));
      if (RANDOM) a[i] = u32x4{a[i][1], a[i][2], a[i][3], a[i][0]};
    }
#pragma unroll
    for (int j = 0; j < kMfmaPerIter; ++j)
      acc[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          __builtin_bit_cast(bf16x8, a[j & 3]), __builtin_bit_cast(bf16x8, b[(j >> 2) & 3]),
          acc[j & 3], 0, 0, 0);
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  float t = 0.f;
  for (int j = 0; j < 4; ++j)
    for (int r = 0; r < 16; ++r) t += acc[j][r];
  sink[blockIdx.x * kThreads + threadIdx.x] = t;
  if (threadIdx.x == 0) {
    stamps[2 * blockIdx.x] = c1 - c0;
    stamps[2 * blockIdx.x + 1] = r1 - r0;
  }
}

}  // namespace

int main() {
  int dev = 0, cus = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int grid = 4 * cus;  // four waves per SIMD
  const int iters = 20000;
  float* sink = nullptr;
  unsigned long long* stamps = nullptr;
  CHECK(hipMalloc(&sink, sizeof(float) * grid * kThreads));
  CHECK(hipMalloc(&stamps, sizeof(unsigned long long) * 2 * grid));
  unsigned long long* host = (unsigned long long*)std::malloc(sizeof(unsigned long long) * 2 * grid);
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  const double flop = 2.0 * 32 * 32 * 16 * kMfmaPerIter * (double)iters * grid * (kThreads / 64);
  auto run = [&](auto kernel, const char* name) {
    for (int w = 0; w < 3; ++w) hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), 0, 0, sink, stamps, iters);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(e0));
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), 0, 0, sink, stamps, iters);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    CHECK(hipMemcpy(host, stamps, sizeof(unsigned long long) * 2 * grid, hipMemcpyDeviceToHost));
    double cycles = 0.0, ticks = 0.0;
    for (int i = 0; i < grid; ++i) {
      cycles += (double)host[2 * i];
      ticks += (double)host[2 * i + 1];
    }
    const double ghz = cycles / (ticks / 100e6) / 1e9;
    std::printf("%-9s operands: %8.3f ms  %6.0f TFLOP/s  shader clock %.3f GHz\n", name, ms,
                flop / (ms * 1e-3) / 1e12, ghz);
    std::fflush(stdout);
  };
  for (int rep = 0; rep < 2; ++rep) {
    run(mfma_loop<false>, "constant");
    run(mfma_loop<true>, "random");
  }
  std::free(host);
  CHECK(hipFree(sink));
  CHECK(hipFree(stamps));
  return 0;
}
