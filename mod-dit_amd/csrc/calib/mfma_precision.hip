// Accumulation precision of single MFMA instructions: a characterisation aid for the
// accuracy contracts of the attention kernels, built into libmoddit_calib.so beside the
// throughput ceiling; not part of the drop-in C ABI.
//
// Each wave loads one A and one B operand fragment and one C input from global memory,
// issues ONE MFMA and stores the result. The operands are laid out as the attention
// kernels use them: A lane (m, h) and B lane (n, h) hold the same k positions in byte
// (element) order, m = n = lane % 32, h = lane / 32, so
//   C[m][n] = C_in[m][n] + sum_{h, j} A[(m, h)][j] * B[(n, h)][j],
// and the C fragment of lane l element i is row 8 (i / 4) + 4 (l / 32) + i % 4, column
// l % 32 (the 32x32 accumulator layout). The caller compares C with the exact sum.
//   kind 0: v_mfma_f32_32x32x16_bf16        (8 bf16 per lane, 16 bytes)
//   kind 2: v_mfma_scale_f32_32x32x64_f8f6f4 with e4m3 A and B and unit scales
//           (32 e4m3 bytes per lane)
// Buffers, per wave w: A and B 64 lanes x 32 bytes at w * 2048 bytes; C_in and C_out 64
// lanes x 16 floats at w * 1024 floats. One wave per workgroup; every wave reads and
// writes only its own slots.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int kKind>
__global__ __launch_bounds__(64) void mfma_precision_kernel(const uint8_t* a, const uint8_t* b,
                                                            const float* c_in, float* c_out) {
  const int w = blockIdx.x;
  const int lane = threadIdx.x;
  const uint8_t* pa = a + static_cast<int64_t>(w) * 2048 + lane * 32;
  const uint8_t* pb = b + static_cast<int64_t>(w) * 2048 + lane * 32;
  const float* pc = c_in + static_cast<int64_t>(w) * 1024 + lane * 16;
  f32x16 c;
#pragma unroll
  for (int i = 0; i < 16; ++i) c[i] = pc[i];
  if constexpr (kKind == 0) {
    const bf16x8 av = *reinterpret_cast<const bf16x8*>(pa);
    const bf16x8 bv = *reinterpret_cast<const bf16x8*>(pb);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c, 0, 0, 0);
  } else {
    const i32x8 av = *reinterpret_cast<const i32x8*>(pa);
    const i32x8 bv = *reinterpret_cast<const i32x8*>(pb);
    c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 0, 0, 0, 127, 0, 127);
  }
  float* po = c_out + static_cast<int64_t>(w) * 1024 + lane * 16;
#pragma unroll
  for (int i = 0; i < 16; ++i) po[i] = c[i];
}

}  // namespace

// Returns 0 on success, 2 for an argument error, 1 for a HIP error. Synchronous.
extern "C" int moddit_calib_mfma_precision(int kind, int waves, const void* a, const void* b,
                                           const float* c_in, float* c_out) {
  if ((kind != 0 && kind != 2) || waves <= 0 || !a || !b || !c_in || !c_out) return 2;
  const auto* pa = static_cast<const uint8_t*>(a);
  const auto* pb = static_cast<const uint8_t*>(b);
  if (kind == 0)
    hipLaunchKernelGGL(mfma_precision_kernel<0>, dim3(waves), dim3(64), 0, 0, pa, pb, c_in, c_out);
  else
    hipLaunchKernelGGL(mfma_precision_kernel<2>, dim3(waves), dim3(64), 0, 0, pa, pb, c_in, c_out);
  if (hipGetLastError() != hipSuccess) return 1;
  return hipDeviceSynchronize() == hipSuccess ? 0 : 1;
}
