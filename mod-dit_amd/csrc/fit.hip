// Ridge fit of the MOD-DiT line model through its Schur complement (gfx950).
//
// The fit solves (M^T M + lambda I) X = M^T S per head (MoD/mod/cuda_lstsq.py:189-264;
// the reference factors the whole F x F matrix, F = 3n, with Cholesky in fp32). With the
// columns of M ordered [2n-1 diagonals][n columns][1 frame block], M^T M + lambda I is
//
//     [ A    W  ]      A  = diag(a),  a_o = n - |o| + lambda        (diagonal x diagonal)
//     [ W^T  C  ]      W  = [B | db],  B[o][c] = 1 iff diagonal o crosses column c,
//                                       db[o] = (n/bpf) (bpf - |o|) for |o| < bpf
//                      C  = [[(n+lambda) I, vb], [vb^T, (n/bpf) bpf^2 + lambda]]
//
// Two cells share a diagonal only if they are the same diagonal, so A is diagonal, and
// diagonal o crosses exactly the columns c in [o, n-1+o] ∩ [0, n): every product with B
// or B^T is a difference of two prefix sums. Eliminating A leaves the (n+1) x (n+1)
// Schur complement S = C - W^T A^-1 W, whose inverse is formed once per shape (fp64,
// cached by the caller):
//
//     y     = m_cb - W^T (A^-1 m_d)                 prefix sums          (fit_rhs_kernel)
//     x_cb  = S^-1 y                                (n+1)^2 GEMV, fp64  (fit_gemv_kernel)
//     x_d   = A^-1 (m_d - B x_c - db x_b)           prefix sums          (fit_diag_kernel)
//
// All arithmetic is fp64 in a fixed order (deterministic); X is rounded to fp32 once.
// At n = 1800 the matrix read per fit is (n+1)^2 * 8 B = 26 MB, against 117 MB for the
// fp32 F x F inverse, and X agrees with the fp64 ridge solution to fp32 rounding.
#include <vector>

#include "common.h"

namespace moddit {
namespace {

constexpr int kFitThreads = 1024;

__device__ __forceinline__ double a_of(int k, int n, double lam) {
  const int o = k - (n - 1);
  return static_cast<double>(n - (o < 0 ? -o : o)) + lam;
}

__device__ __forceinline__ double db_of(int k, int n, int bpf) {
  const int o = k - (n - 1);
  const int ao = o < 0 ? -o : o;
  return ao < bpf ? static_cast<double>(n / bpf) * (bpf - ao) : 0.0;
}

// Exclusive prefix sums of v[0..len) into pre[0..len], pre[len] = total, by one
// 1024-thread workgroup: each thread sums a contiguous chunk, the chunk sums are scanned
// across the workgroup, then each thread rescans its chunk. Fixed order, deterministic.
__device__ void block_prefix_f64(const double* v, double* pre, int len, double* s_part) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int chunk = (len + kFitThreads - 1) / kFitThreads;
  const int i0 = tid * chunk;
  const int i1 = i0 + chunk < len ? i0 + chunk : len;
  double local = 0.0;
  for (int i = i0; i < i1; ++i) local += v[i];
  // inclusive scan of the chunk sums within each wave
  double incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  if (lane == 63) s_part[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    const double w = lane < kFitThreads / 64 ? s_part[lane] : 0.0;
    double wi = w;
#pragma unroll
    for (int o = 1; o < kFitThreads / 64; o <<= 1) {
      const double t = __shfl_up(wi, o);
      if (lane >= o) wi += t;
    }
    if (lane < kFitThreads / 64) s_part[lane] = wi - w;  // exclusive per wave
    if (lane == kFitThreads / 64 - 1) s_part[kFitThreads / 64] = wi;
  }
  __syncthreads();
  double run = s_part[wave] + incl - local;
  for (int i = i0; i < i1; ++i) {
    pre[i] = run;
    run += v[i];
  }
  if (tid == 0) pre[len] = s_part[kFitThreads / 64];
  __syncthreads();
}

// Deterministic workgroup sum of one value per thread (tree over a fixed order).
__device__ double block_sum_f64(double v, double* s_part) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  if (lane == 0) s_part[wave] = v;
  __syncthreads();
  double tot = 0.0;
  for (int w = 0; w < kFitThreads / 64; ++w) tot += s_part[w];
  __syncthreads();
  return tot;
}

// One workgroup per head: y = m_cb - W^T A^-1 m_d.
__global__ __launch_bounds__(kFitThreads) void fit_rhs_kernel(const float* __restrict__ mts,
                                                              double* __restrict__ y, int n,
                                                              int bpf, double lam) {
  extern __shared__ __align__(16) double fit_smem[];
  __shared__ double s_part[kFitThreads / 64 + 1];
  const int nd = 2 * n - 1;
  double* z = fit_smem;           // nd
  double* pre = fit_smem + nd;    // nd + 1
  const int h = blockIdx.x;
  const int F = 3 * n;
  const float* m = mts + static_cast<int64_t>(h) * F;
  double dbz = 0.0;
  for (int k = threadIdx.x; k < nd; k += kFitThreads) {
    const double zk = static_cast<double>(m[k]) / a_of(k, n, lam);
    z[k] = zk;
    dbz += db_of(k, n, bpf) * zk;
  }
  __syncthreads();
  block_prefix_f64(z, pre, nd, s_part);
  const double wb = block_sum_f64(dbz, s_part);
  double* yh = y + static_cast<int64_t>(h) * (n + 1);
  // column c is crossed by diagonals k = c .. c+n-1 (offset o = k-(n-1) in [c-n+1, c])
  for (int c = threadIdx.x; c < n; c += kFitThreads)
    yh[c] = static_cast<double>(m[nd + c]) - (pre[c + n] - pre[c]);
  if (threadIdx.x == 0) yh[n] = static_cast<double>(m[F - 1]) - wb;
}

// x_cb[h] = S^-1 y[h] for all heads. Workgroup = 8 rows of S^-1 x up to 16 heads; 32
// threads per row stride the reduction, and y chunks are staged in LDS and shared by the
// rows (measured at n = 1800 and 1080, H = 24 and 40: the fastest of the row x head
// blockings tried, 4 to 32 rows and 16 or 24 heads).
constexpr int kGemvThreads = 256;
constexpr int kGemvRows = 8;
constexpr int kGemvLanes = kGemvThreads / kGemvRows;  // threads per row
constexpr int kGemvHeads = 16;
constexpr int kGemvChunk = 128;

__global__ __launch_bounds__(kGemvThreads) void fit_gemv_kernel(const double* __restrict__ sinv,
                                                                const double* __restrict__ y,
                                                                double* __restrict__ xcb,
                                                                int heads, int m) {
  // y chunks are double-buffered in LDS; the next chunk's y values and this lane's S^-1
  // elements of it are loaded before the current chunk's products, so one barrier per
  // chunk separates the products from the next chunk's LDS writes
  __shared__ double s_y[2][kGemvHeads][kGemvChunk];
  constexpr int kPer = kGemvChunk / kGemvLanes;                 // S^-1 elements per lane
  constexpr int kStage = kGemvHeads * kGemvChunk / kGemvThreads;  // y values per thread
  static_assert(kGemvHeads * kGemvChunk % kGemvThreads == 0, "y chunk staging");
  const int tid = threadIdx.x;
  const int r = tid / kGemvLanes;
  const int j = tid % kGemvLanes;
  const int row = blockIdx.x * kGemvRows + r;
  const int h0 = blockIdx.y * kGemvHeads;
  const int nh = heads - h0 < kGemvHeads ? heads - h0 : kGemvHeads;
  double acc[kGemvHeads];
#pragma unroll
  for (int hh = 0; hh < kGemvHeads; ++hh) acc[hh] = 0.0;
  const double* srow = sinv + static_cast<int64_t>(row < m ? row : m - 1) * m;
  auto load_y = [&](int k0, double* v) {
#pragma unroll
    for (int q = 0; q < kStage; ++q) {
      const int i = tid + q * kGemvThreads;
      const int hh = i / kGemvChunk;
      const int g = k0 + i % kGemvChunk;
      v[q] = (hh < nh && g < m) ? y[static_cast<int64_t>(h0 + hh) * m + g] : 0.0;
    }
  };
  auto store_y = [&](int buf, const double* v) {
#pragma unroll
    for (int q = 0; q < kStage; ++q) {
      const int i = tid + q * kGemvThreads;
      s_y[buf][i / kGemvChunk][i % kGemvChunk] = v[q];
    }
  };
  auto load_a = [&](int k0, double* a) {
#pragma unroll
    for (int t = 0; t < kPer; ++t) {
      const int g = k0 + j + kGemvLanes * t;
      a[t] = g < m ? srow[g] : 0.0;
    }
  };
  double a_cur[kPer], yv[kStage];
  load_y(0, yv);
  load_a(0, a_cur);
  store_y(0, yv);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < m; k0 += kGemvChunk) {
    const bool more = k0 + kGemvChunk < m;
    double a_nxt[kPer];
    if (more) {
      load_y(k0 + kGemvChunk, yv);
      load_a(k0 + kGemvChunk, a_nxt);
    }
#pragma unroll
    for (int t = 0; t < kPer; ++t) {
#pragma unroll
      for (int hh = 0; hh < kGemvHeads; ++hh)
        acc[hh] = __builtin_fma(a_cur[t], s_y[buf][hh][j + kGemvLanes * t], acc[hh]);
    }
    if (more) {
      store_y(buf ^ 1, yv);
#pragma unroll
      for (int t = 0; t < kPer; ++t) a_cur[t] = a_nxt[t];
    }
    __syncthreads();
    buf ^= 1;
  }
#pragma unroll
  for (int hh = 0; hh < kGemvHeads; ++hh) {
    double v = acc[hh];
#pragma unroll
    for (int o = kGemvLanes / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    acc[hh] = v;
  }
  if (j == 0 && row < m) {
#pragma unroll
    for (int hh = 0; hh < kGemvHeads; ++hh)
      if (hh < nh) xcb[static_cast<int64_t>(h0 + hh) * m + row] = acc[hh];
  }
}

// One workgroup per head: x_d = A^-1 (m_d - B x_c - db x_b), X = [x_d, x_c, x_b] in fp32.
__global__ __launch_bounds__(kFitThreads) void fit_diag_kernel(const float* __restrict__ mts,
                                                               const double* __restrict__ xcb,
                                                               float* __restrict__ x, int n,
                                                               int bpf, double lam) {
  extern __shared__ __align__(16) double fit_smem[];
  __shared__ double s_part[kFitThreads / 64 + 1];
  double* xc = fit_smem;        // n
  double* pre = fit_smem + n;   // n + 1
  const int h = blockIdx.x;
  const int F = 3 * n;
  const int nd = 2 * n - 1;
  const float* m = mts + static_cast<int64_t>(h) * F;
  const double* xh = xcb + static_cast<int64_t>(h) * (n + 1);
  float* out = x + static_cast<int64_t>(h) * F;
  for (int c = threadIdx.x; c < n; c += kFitThreads) {
    const double v = xh[c];
    xc[c] = v;
    out[nd + c] = static_cast<float>(v);
  }
  const double xb = xh[n];
  if (threadIdx.x == 0) out[F - 1] = static_cast<float>(xb);
  __syncthreads();
  block_prefix_f64(xc, pre, n, s_part);
  // diagonal o crosses columns c in [max(o, 0), min(n-1, n-1+o)]
  for (int k = threadIdx.x; k < nd; k += kFitThreads) {
    const int o = k - (n - 1);
    const int c0 = o > 0 ? o : 0;
    const int c1 = o < 0 ? n + o : n;  // exclusive
    const double bx = pre[c1] - pre[c0];
    out[k] = static_cast<float>((static_cast<double>(m[k]) - bx - db_of(k, n, bpf) * xb) /
                                a_of(k, n, lam));
  }
}

constexpr int kFitMaxN = 4096;  // LDS: 4n-1 doubles per workgroup (128 KB at the limit)

// Scratch of the allocation-free entry point moddit_fit_lines_noalloc: room for the
// workspace of up to 64 heads at n <= 2048 (2 * 64 * 2049 doubles = 2.1 MB per device,
// held until the process ends). Host code never uses this name as an address: it
// resolves the device address once per device with hipGetSymbolAddress.
constexpr int64_t kNoAllocDoubles = 2 * int64_t{64} * 2049;
__device__ __align__(256) double scratch[kNoAllocDoubles];

struct ScratchAddr {
  std::once_flag flag[kMaxDevices];
  hipError_t status[kMaxDevices] = {};
  double* ptr[kMaxDevices] = {};
};

}  // namespace
}  // namespace moddit

// Closed form of the Schur complement S = C - W^T A^-1 W (see the top of this file):
//   S[c][c'] = (n + lambda) [c == c'] - sum_{k = max(c,c')}^{min(c,c')+n-1} 1/a_k
//   S[c][n]  = vb_c - sum_{k = c}^{c+n-1} db_k / a_k,   vb_c = bpf if c < (n/bpf) bpf else 0
//   S[n][n]  = (n/bpf) bpf^2 + lambda - sum_k db_k^2 / a_k
// with diagonal index k = o + n - 1. The band sums are differences of prefix sums formed
// in long double.
extern "C" int moddit_fit_schur_host(int n, int blocks_per_frame, double regularization,
                                     double* schur_out) {
  using namespace moddit;
  clear_error();
  MODDIT_CHECK_ARG(schur_out != nullptr, "fit_schur: null output");
  MODDIT_CHECK_ARG(n > 0 && blocks_per_frame > 0, "fit_schur: invalid n=%d bpf=%d", n,
                   blocks_per_frame);
  MODDIT_CHECK_ARG(regularization >= 0.0, "fit_schur: regularization must be >= 0");
  const int nd = 2 * n - 1;
  const int bpf = blocks_per_frame;
  const int nbk = n / bpf;
  std::vector<long double> q(nd + 1), rr(nd + 1);  // prefix sums of 1/a and db/a
  q[0] = 0.0L;
  rr[0] = 0.0L;
  long double dd = 0.0L;
  for (int k = 0; k < nd; ++k) {
    const int o = k - (n - 1);
    const int ao = o < 0 ? -o : o;
    const long double a = static_cast<long double>(n - ao) + regularization;
    const long double db = ao < bpf ? static_cast<long double>(nbk) * (bpf - ao) : 0.0L;
    q[k + 1] = q[k] + 1.0L / a;
    rr[k + 1] = rr[k] + db / a;
    dd += db * db / a;
  }
  const int64_t m = static_cast<int64_t>(n) + 1;
  for (int c = 0; c < n; ++c) {
    for (int c2 = c; c2 < n; ++c2) {
      // diagonals crossing both columns: k in [c2, c + n - 1]
      long double v = -(q[c + n] - q[c2]);
      if (c2 == c) v += static_cast<long double>(n) + regularization;
      schur_out[c * m + c2] = static_cast<double>(v);
      schur_out[c2 * m + c] = static_cast<double>(v);
    }
    const long double vb = c < nbk * bpf ? static_cast<long double>(bpf) : 0.0L;
    const double sb = static_cast<double>(vb - (rr[c + n] - rr[c]));
    schur_out[c * m + n] = sb;
    schur_out[static_cast<int64_t>(n) * m + c] = sb;
  }
  schur_out[static_cast<int64_t>(n) * m + n] =
      static_cast<double>(static_cast<long double>(nbk) * bpf * bpf + regularization - dd);
  return MODDIT_OK;
}

extern "C" int64_t moddit_fit_workspace_doubles(int heads, int n) {
  if (heads <= 0 || n <= 0) return 0;
  return 2 * static_cast<int64_t>(heads) * (static_cast<int64_t>(n) + 1);
}

namespace moddit {
namespace {

int check_fit_args(const double* schur_inv, const float* mts, float* x, int heads, int n,
                   int blocks_per_frame, double regularization) {
  MODDIT_CHECK_ARG(schur_inv && mts && x, "fit_lines: null pointer argument");
  MODDIT_CHECK_ARG(heads >= 0 && n > 0 && blocks_per_frame > 0,
                   "fit_lines: invalid shape heads=%d n=%d bpf=%d", heads, n, blocks_per_frame);
  MODDIT_CHECK_ARG(n <= kFitMaxN, "fit_lines: n=%d exceeds %d", n, kFitMaxN);
  MODDIT_CHECK_ARG(regularization >= 0.0, "fit_lines: regularization must be >= 0");
  return MODDIT_OK;
}

int launch_fit(const double* schur_inv, const float* mts, float* x, double* workspace, int heads,
               int n, int blocks_per_frame, double regularization, hipStream_t st) {
  const int m = n + 1;
  double* y = workspace;
  double* xcb = workspace + static_cast<int64_t>(heads) * m;
  const size_t lds_rhs = static_cast<size_t>(4 * n - 1) * sizeof(double);  // z (nd) + pre (nd+1)
  const size_t lds_diag = static_cast<size_t>(2 * n + 1) * sizeof(double);  // x_c (n) + pre (n+1)
  static LaunchSetup once_rhs, once_diag;
  if (set_dynamic_lds_once(once_rhs, reinterpret_cast<const void*>(fit_rhs_kernel),
                           static_cast<int>((4 * kFitMaxN - 1) * sizeof(double))) != hipSuccess ||
      set_dynamic_lds_once(once_diag, reinterpret_cast<const void*>(fit_diag_kernel),
                           static_cast<int>((2 * kFitMaxN + 1) * sizeof(double))) != hipSuccess) {
    set_error("fit_lines: cannot reserve LDS");
    return MODDIT_EHIP;
  }
  hipLaunchKernelGGL(fit_rhs_kernel, dim3(heads), dim3(kFitThreads), lds_rhs, st, mts, y, n,
                     blocks_per_frame, regularization);
  MODDIT_CHECK_LAUNCH("fit_lines (rhs)");
  dim3 grid((m + kGemvRows - 1) / kGemvRows, (heads + kGemvHeads - 1) / kGemvHeads);
  hipLaunchKernelGGL(fit_gemv_kernel, grid, dim3(kGemvThreads), 0, st, schur_inv, y, xcb, heads, m);
  MODDIT_CHECK_LAUNCH("fit_lines (gemv)");
  hipLaunchKernelGGL(fit_diag_kernel, dim3(heads), dim3(kFitThreads), lds_diag, st, mts, xcb, x, n,
                     blocks_per_frame, regularization);
  MODDIT_CHECK_LAUNCH("fit_lines (diag)");
  return MODDIT_OK;
}

}  // namespace
}  // namespace moddit

extern "C" int moddit_fit_lines(const double* schur_inv, const float* mts, float* x,
                                double* workspace, int heads, int n, int blocks_per_frame,
                                double regularization, moddit_stream_t stream) {
  using namespace moddit;
  clear_error();
  int rc = check_fit_args(schur_inv, mts, x, heads, n, blocks_per_frame, regularization);
  if (rc) return rc;
  MODDIT_CHECK_ARG(workspace != nullptr, "fit_lines: null workspace");
  if (heads == 0) return MODDIT_OK;
  return launch_fit(schur_inv, mts, x, workspace, heads, n, blocks_per_frame, regularization,
                    as_stream(stream));
}

// The same fit with its workspace in the library's device array `scratch` instead of a
// caller buffer: no allocation of any kind. The array's device address is looked up once
// per device (with that device current) and kept; calls that overlap on one device share
// the array and race. Nothing in it needs to start at zero: every call writes the whole
// workspace it reads.
extern "C" int moddit_fit_lines_noalloc(const double* schur_inv, const float* mts, float* x,
                                        int heads, int n, int blocks_per_frame,
                                        double regularization, moddit_stream_t stream) {
  using namespace moddit;
  clear_error();
  int rc = check_fit_args(schur_inv, mts, x, heads, n, blocks_per_frame, regularization);
  if (rc) return rc;
  const int64_t need = moddit_fit_workspace_doubles(heads, n);
  MODDIT_CHECK_ARG(need <= kNoAllocDoubles,
                   "fit_lines_noalloc: %d heads at n=%d need %lld doubles of scratch, the "
                   "fixed array holds %lld (e.g. 64 heads at n <= 2048)",
                   heads, n, static_cast<long long>(need), static_cast<long long>(kNoAllocDoubles));
  if (heads == 0) return MODDIT_OK;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("fit_lines_noalloc: no usable current device");
    return MODDIT_EHIP;
  }
  static ScratchAddr addr;
  std::call_once(addr.flag[dev], [&] {
    void* p = nullptr;
    addr.status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    addr.ptr[dev] = static_cast<double*>(p);
  });
  if (addr.status[dev] != hipSuccess || addr.ptr[dev] == nullptr) {
    set_error("fit_lines_noalloc: hipGetSymbolAddress failed: %s",
              hipGetErrorString(addr.status[dev]));
    return MODDIT_EHIP;
  }
  return launch_fit(schur_inv, mts, x, addr.ptr[dev], heads, n, blocks_per_frame, regularization,
                    as_stream(stream));
}
