// Shared device/host helpers for the gfx950 kernels of the MOD-DiT hot path.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/moddit.h"

namespace moddit {

// ---------------------------------------------------------------------------------
// Error reporting: a thread-local message behind integer status codes.
// ---------------------------------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define MODDIT_CHECK_ARG(cond, ...)          \
  do {                                       \
    if (!(cond)) {                           \
      ::moddit::set_error(__VA_ARGS__);      \
      return MODDIT_EINVAL;                  \
    }                                        \
  } while (0)

#define MODDIT_CHECK_LAUNCH(what)                                                   \
  do {                                                                              \
    hipError_t err_ = hipGetLastError();                                            \
    if (err_ != hipSuccess) {                                                       \
      ::moddit::set_error("%s: launch failed: %s", what, hipGetErrorString(err_)); \
      return MODDIT_EHIP;                                                           \
    }                                                                               \
  } while (0)

inline hipStream_t as_stream(moddit_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------------------------
// One-time launch setup. A kernel's dynamic-LDS limit (hipFuncSetAttribute) is set on
// the current device, so it is set once per device. Concurrent first launches from
// several host threads wait for the one that performs it (std::call_once), and every
// caller sees its status. Declare one `static LaunchSetup` per kernel.
// ---------------------------------------------------------------------------------
constexpr int kMaxDevices = 64;

struct LaunchSetup {
  std::once_flag flag[kMaxDevices];
  hipError_t status[kMaxDevices] = {};
};

inline hipError_t set_dynamic_lds_once(LaunchSetup& once, const void* kernel, int bytes) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  auto setup = [&] {
    return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  };
  if (dev < 0 || dev >= kMaxDevices) return setup();  // outside the table: every call
  std::call_once(once.flag[dev], [&] { once.status[dev] = setup(); });
  return once.status[dev];
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------------
// Vector types for MFMA operands and 16-byte moves.
// ---------------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8 __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
// Native vectors for raw 16/8-byte moves (HIP's uint4 struct defeats register promotion).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Storage element traits: both 16-bit types are moved as raw uint16_t.
struct Bf16 {
  typedef bf16x8 vec8;
  typedef __bf16 elem;
  static __device__ __forceinline__ f32x16 mma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_float(uint16_t u) {
    return __uint_as_float(static_cast<uint32_t>(u) << 16);
  }
  // Round-to-nearest-even; NaN stays a quiet NaN.
  static __device__ __forceinline__ uint16_t from_float(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
  }
};

struct Fp16 {
  typedef f16x8 vec8;
  typedef _Float16 elem;
  static __device__ __forceinline__ f32x16 mma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_float(uint16_t u) {
    _Float16 h;
    __builtin_memcpy(&h, &u, 2);
    return static_cast<float>(h);
  }
  static __device__ __forceinline__ uint16_t from_float(float f) {
    _Float16 h = static_cast<_Float16>(f);  // round-to-nearest-even
    uint16_t u;
    __builtin_memcpy(&u, &h, 2);
    return u;
  }
};

// Max / sum of x over lanes l and l ^ 32, in both lanes. v_permlane32_swap exchanges
// the two 32-lane halves of a register pair in the VALU (no LDS round trip, unlike the
// ds_bpermute behind __shfl_xor); both lanes of a pair get bit-identical results.
__device__ __forceinline__ float max_over_halves(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float sum_over_halves(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

template <typename V>
__device__ __forceinline__ V as_vec8(u32x4 x) {
  return __builtin_bit_cast(V, x);
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

__device__ __forceinline__ uint16_t u16_at(const u32x4& v, int i) {
  const uint32_t w = v[i >> 1];
  return static_cast<uint16_t>((i & 1) ? (w >> 16) : (w & 0xffffu));
}

// ---------------------------------------------------------------------------------
// Buffer loads. A raw buffer resource covers one tensor slice; offsets are 32-bit
// bytes. The VGPR offset (plus the instruction offset) is range-checked against
// `bytes`: out-of-range 16-byte loads return zeros instead of touching memory. The
// SGPR offset is not range-checked, so it may only carry offsets known to be in range.
// ---------------------------------------------------------------------------------
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                            uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                       r, static_cast<int>(voff), static_cast<int>(soff), 0));
}

// ---------------------------------------------------------------------------------
// Workgroup -> tile mapping. The dispatcher hands workgroup w to XCD (w % 8) whatever
// the XCDs' progress, so each XCD gets a fixed eighth of the grid, and each XCD has its
// own 4 MB L2. Two orders, chosen per launch by the bytes one head's key sweep reads:
//  - run == 0: XCD x owns one contiguous eighth of the tiles. When a head's K/V fits
//    in about two L2s, the XCD's resident workgroups all sit in one head and every
//    K/V tile is fetched from beyond L2 about once per head (a 4.5 MB CogVideoX head:
//    8 % faster than dealt runs).
//  - run > 0: runs of `run` consecutive tiles are dealt to the XCDs in turn. A larger
//    head does not fit anyway, and what L2 keeps is the tiles that neighbouring query
//    tiles share, which a run preserves; dealing spreads every head over all XCDs, so
//    block-sparse heads that differ in work by up to 1.6x no longer pile up on one XCD
//    (a 24-head grid gives each XCD three whole heads): 8-10 % faster at the headline.
//    Tiles past the last whole round of runs keep the dispatcher's order.
// ---------------------------------------------------------------------------------
constexpr int kNumXcd = 8;
constexpr int kXcdRun = 32;
constexpr int64_t kXcdHeadBytes = int64_t{8} << 20;

// Host side: the run length for a launch whose key sweep reads `head_bytes` per head.
inline int xcd_run_for(int64_t head_bytes) { return head_bytes > kXcdHeadBytes ? kXcdRun : 0; }

__device__ __forceinline__ int xcd_remap(int wg, int total, int run) {
  const int xcd = wg % kNumXcd;
  const int local = wg / kNumXcd;  // position in this XCD's dispatch order
  if (run == 0) {
    const int base = total / kNumXcd;
    const int rem = total % kNumXcd;
    return xcd * base + (xcd < rem ? xcd : rem) + local;
  }
  const int whole = total / (kNumXcd * run) * (kNumXcd * run);
  if (wg >= whole) return wg;
  return ((local / run) * kNumXcd + xcd) * run + local % run;
}

}  // namespace moddit
