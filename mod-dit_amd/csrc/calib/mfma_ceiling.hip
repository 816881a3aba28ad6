// MFMA throughput ceiling on random operands: a measurement aid for bench.py's roofline,
// built into its own library (libmoddit_calib.so) and not part of the drop-in C ABI.
//
// MI355X draws more power per MFMA when the operands toggle many bits, and under a
// sustained MFMA load the shader clock settles where the board's power limit holds; the
// published dense peaks assume the top clock. This kernel issues nothing but back-to-back
// MFMAs of one kind (the 32x32 shapes the attention kernels use, and the 16x16 shapes of
// the same data types, which the part sustains at a higher clock), at two waves per SIMD,
// on random operands, and reports the rate and the shader clock it ran at (s_memtime over
// s_memrealtime, a 100 MHz counter). Every wave writes only its own output slot; the loop
// count is fixed.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <mutex>
#include <vector>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 512;  // 8 waves: two per SIMD
constexpr int kRegs = 8;       // operand registers cycled through the loop

__device__ __forceinline__ uint32_t mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// kind 0: bf16 32x32x16 (32768 flop); 1: int8 32x32x32 (65536 op); 2: fp8 e4m3 32x32x64
// with unit scales (131072 flop); 3-5: the 16x16 shapes of the same types (bf16 16x16x32,
// int8 16x16x64, fp8 16x16x128: half the work per MFMA, twice the MFMAs per trip).
// zeros != 0 runs the same loop on all-zero operands.
template <int kKind>
__global__ __launch_bounds__(kThreads) void mfma_ceiling_kernel(int iters, int zeros, float* out,
                                                                unsigned long long* clk) {
  const uint32_t gid = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t keep = zeros ? 0u : 0xffffffffu;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  unsigned long long t0 = 0, r0 = 0;
  float acc_sum = 0.f;
  if constexpr (kKind == 0) {
    bf16x8 a[kRegs], b[kRegs];
#pragma unroll
    for (int r = 0; r < kRegs; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t h1 = mix(gid * 131u + r * 8 + i);
        const uint32_t h2 = mix(h1 ^ 0x9e3779b9u);
        a[r][i] = static_cast<__bf16>((static_cast<int>(h1 & 0xffff) - 32768) / 16384.f * (keep & 1));
        b[r][i] = static_cast<__bf16>((static_cast<int>(h2 & 0xffff) - 32768) / 16384.f * (keep & 1));
      }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int r = 0; r < kRegs; r += 2) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r], b[r], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r + 1], b[r], c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r], b[r + 1], c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r + 1], b[r + 1], c3, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) acc_sum += c0[i] + c1[i] + c2[i] + c3[i];
  } else if constexpr (kKind == 3) {
    bf16x8 a[kRegs], b[kRegs];
#pragma unroll
    for (int r = 0; r < kRegs; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t h1 = mix(gid * 131u + r * 8 + i);
        const uint32_t h2 = mix(h1 ^ 0x9e3779b9u);
        a[r][i] = static_cast<__bf16>((static_cast<int>(h1 & 0xffff) - 32768) / 16384.f * (keep & 1));
        b[r][i] = static_cast<__bf16>((static_cast<int>(h2 & 0xffff) - 32768) / 16384.f * (keep & 1));
      }
    f32x4 c[8] = {};
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int r = 0; r < kRegs; r += 2)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          c[4 * h + 0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[r], b[r], c[4 * h + 0], 0, 0, 0);
          c[4 * h + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[r + 1], b[r], c[4 * h + 1], 0, 0, 0);
          c[4 * h + 2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[r], b[r + 1], c[4 * h + 2], 0, 0, 0);
          c[4 * h + 3] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[r + 1], b[r + 1], c[4 * h + 3], 0, 0, 0);
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) acc_sum += c[k][0] + c[k][1] + c[k][2] + c[k][3];
  } else if constexpr (kKind == 4) {
    i32x4 a[kRegs], b[kRegs];
#pragma unroll
    for (int r = 0; r < kRegs; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t h1 = mix(gid * 131u + r * 8 + i);
        a[r][i] = static_cast<int>(h1 & keep);
        b[r][i] = static_cast<int>(mix(h1 ^ 0x9e3779b9u) & keep);
      }
    i32x4 c[8] = {};
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int r = 0; r < kRegs; r += 2)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          c[4 * h + 0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[r], b[r], c[4 * h + 0], 0, 0, 0);
          c[4 * h + 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[r + 1], b[r], c[4 * h + 1], 0, 0, 0);
          c[4 * h + 2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[r], b[r + 1], c[4 * h + 2], 0, 0, 0);
          c[4 * h + 3] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[r + 1], b[r + 1], c[4 * h + 3], 0, 0, 0);
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) acc_sum += static_cast<float>(c[k][0] ^ c[k][1] ^ c[k][2] ^ c[k][3]);
  } else if constexpr (kKind == 5) {
    i32x8 a[kRegs], b[kRegs];
#pragma unroll
    for (int r = 0; r < kRegs; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t h1 = mix(gid * 131u + r * 8 + i) & 0xb7b7b7b7u & keep;
        a[r][i] = static_cast<int>(h1);
        b[r][i] = static_cast<int>(mix(h1 ^ 0x9e3779b9u) & 0xb7b7b7b7u & keep);
      }
    f32x4 c[8] = {};
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int r = 0; r < kRegs; r += 2)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          c[4 * h + 0] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[r], b[r], c[4 * h + 0], 0, 0, 0, 127, 0, 127);
          c[4 * h + 1] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[r + 1], b[r], c[4 * h + 1], 0, 0, 0, 127, 0, 127);
          c[4 * h + 2] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[r], b[r + 1], c[4 * h + 2], 0, 0, 0, 127, 0, 127);
          c[4 * h + 3] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[r + 1], b[r + 1], c[4 * h + 3], 0, 0, 0, 127, 0, 127);
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) acc_sum += c[k][0] + c[k][1] + c[k][2] + c[k][3];
  } else if constexpr (kKind == 1) {
    i32x4 a[kRegs], b[kRegs];
#pragma unroll
    for (int r = 0; r < kRegs; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t h1 = mix(gid * 131u + r * 8 + i);
        a[r][i] = static_cast<int>(h1 & keep);
        b[r][i] = static_cast<int>(mix(h1 ^ 0x9e3779b9u) & keep);
      }
    i32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int r = 0; r < kRegs; r += 2) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[r], b[r], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[r + 1], b[r], c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[r], b[r + 1], c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[r + 1], b[r + 1], c3, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) acc_sum += static_cast<float>(c0[i] ^ c1[i] ^ c2[i] ^ c3[i]);
  } else {
    i32x8 a[kRegs], b[kRegs];
#pragma unroll
    for (int r = 0; r < kRegs; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        // random e4m3 bytes with the exponent kept below the NaN encodings
        const uint32_t h1 = mix(gid * 131u + r * 8 + i) & 0xb7b7b7b7u & keep;
        a[r][i] = static_cast<int>(h1);
        b[r][i] = static_cast<int>(mix(h1 ^ 0x9e3779b9u) & 0xb7b7b7b7u & keep);
      }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int r = 0; r < kRegs; r += 2) {
        c0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[r], b[r], c0, 0, 0, 0, 127, 0, 127);
        c1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[r + 1], b[r], c1, 0, 0, 0, 127, 0, 127);
        c2 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[r], b[r + 1], c2, 0, 0, 0, 127, 0, 127);
        c3 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[r + 1], b[r + 1], c3, 0, 0, 0, 127, 0, 127);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) acc_sum += c0[i] + c1[i] + c2[i] + c3[i];
  }
  out[(blockIdx.x * (kThreads / 64) + wave) * 64 + lane] = acc_sum;
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = t1 - t0;
    clk[2 * blockIdx.x + 1] = r1 - r0;
  }
}

constexpr double kFlopPerMfma[6] = {32768.0, 65536.0, 131072.0, 16384.0, 32768.0, 65536.0};
constexpr int kMfmaPerTrip[6] = {16, 16, 16, 32, 32, 32};  // per wave per loop trip
// Dynamic LDS per workgroup that keeps the dispatcher from placing two workgroups on
// one CU (the kernel itself uses none): one 8-wave workgroup per CU for every kind.
constexpr int kOneGroupLds = 96 * 1024;

template <int kKind>
hipError_t launch_kind(int cus, int iters, int zeros, float* out, unsigned long long* clk) {
  static std::once_flag once;
  static hipError_t set = hipSuccess;
  std::call_once(once, [] {
    set = hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_ceiling_kernel<kKind>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kOneGroupLds);
  });
  if (set != hipSuccess) return set;
  hipLaunchKernelGGL(mfma_ceiling_kernel<kKind>, dim3(cus), dim3(kThreads), kOneGroupLds, nullptr, iters,
                     zeros, out, clk);
  return hipGetLastError();
}

#define CALIB_CHECK(x)                                                      \
  do {                                                                      \
    const hipError_t e_ = (x);                                              \
    if (e_ != hipSuccess) {                                                 \
      std::fprintf(stderr, "moddit_calib: %s: %s\n", #x, hipGetErrorString(e_)); \
      rc = 1;                                                               \
      goto done;                                                            \
    }                                                                       \
  } while (0)

}  // namespace

extern "C" {

// Runs `reps` timed launches of `iters` loop trips (16 MFMAs of a 32x32 kind or 32 of a
// 16x16 kind per wave per trip) on the current device, one 8-wave workgroup per CU,
// random operands (or all-zero ones when `zeros` is set), and reports the sustained rate
// over those launches in TFLOP/s (TOP/s for int8), their mean shader clock in MHz, and
// the shader cycles per MFMA per SIMD.
// The board's power control settles over tens of milliseconds, so a few hundred launches
// (~1 s) give the rate the part holds under load. Returns 0, or 1 on a HIP error (message
// on stderr), or 2 for a bad argument.
int moddit_calib_mfma(int kind, int zeros, int iters, int reps, double* rate, double* clock_mhz,
                      double* cycles_per_mfma) {
  if (kind < 0 || kind > 5 || iters <= 0 || reps <= 0 || rate == nullptr ||
      clock_mhz == nullptr || cycles_per_mfma == nullptr)
    return 2;
  int rc = 0;
  int dev = 0, cus = 0;
  float* out = nullptr;
  unsigned long long* clk = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  std::vector<unsigned long long> host;
  double total_ms = 0.0, mhz_sum = 0.0;
  int mhz_n = 0;
  CALIB_CHECK(hipGetDevice(&dev));
  CALIB_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  CALIB_CHECK(hipMalloc(&out, static_cast<size_t>(cus) * kThreads * sizeof(float)));
  CALIB_CHECK(hipMalloc(&clk, static_cast<size_t>(cus) * 2 * sizeof(unsigned long long)));
  CALIB_CHECK(hipEventCreate(&e0));
  CALIB_CHECK(hipEventCreate(&e1));
  host.resize(static_cast<size_t>(cus) * 2);
  for (int rep = 0; rep <= reps; ++rep) {  // the first launch warms up and is not counted
    CALIB_CHECK(hipEventRecord(e0, nullptr));
    switch (kind) {
      case 0: CALIB_CHECK(launch_kind<0>(cus, iters, zeros, out, clk)); break;
      case 1: CALIB_CHECK(launch_kind<1>(cus, iters, zeros, out, clk)); break;
      case 2: CALIB_CHECK(launch_kind<2>(cus, iters, zeros, out, clk)); break;
      case 3: CALIB_CHECK(launch_kind<3>(cus, iters, zeros, out, clk)); break;
      case 4: CALIB_CHECK(launch_kind<4>(cus, iters, zeros, out, clk)); break;
      default: CALIB_CHECK(launch_kind<5>(cus, iters, zeros, out, clk)); break;
    }
    CALIB_CHECK(hipEventRecord(e1, nullptr));
    CALIB_CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CALIB_CHECK(hipEventElapsedTime(&ms, e0, e1));
    if (rep == 0) continue;
    total_ms += ms;
    CALIB_CHECK(hipMemcpy(host.data(), clk, host.size() * sizeof(unsigned long long),
                          hipMemcpyDeviceToHost));
    double sum = 0.0;
    int n = 0;
    for (int w = 0; w < cus; ++w)
      if (host[2 * w + 1] != 0) {
        sum += static_cast<double>(host[2 * w]) / static_cast<double>(host[2 * w + 1]) * 100.0;
        ++n;
      }
    if (n > 0) {
      mhz_sum += sum / n;
      ++mhz_n;
    }
  }
  {
    const double mfmas = static_cast<double>(cus) * (kThreads / 64) * iters * kMfmaPerTrip[kind] * reps;
    const double mhz = mhz_n > 0 ? mhz_sum / mhz_n : 0.0;
    *rate = mfmas * kFlopPerMfma[kind] / (total_ms * 1e-3) / 1e12;
    *clock_mhz = mhz;
    *cycles_per_mfma = total_ms * 1e-3 * mhz * 1e6 / (mfmas / (cus * 4.0));
  }
done:
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (out) (void)hipFree(out);
  if (clk) (void)hipFree(clk);
  return rc;
}

}  // extern "C"
