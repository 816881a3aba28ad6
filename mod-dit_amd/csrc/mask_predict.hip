// Mask prediction for gfx950: M^T S line statistics, line prediction/selection,
// block-diagonal mode, block mask + attention tile lists, and the refresh merge (the
// ridge solve between M^T S and the selection is in fit.hip). All of it is HBM-bound
// integer/byte work; none of it is reshaped onto MFMA.
//
// Floating-point contraction is disabled in this file: the prediction
// cur + (cur - last) / T must round exactly like the reference's separate fp32 ops.
#pragma clang fp contract(off)

#include "common.h"

namespace moddit {
namespace {

// =====================================================================================
// M^T S (MoD/mod/cuda_lstsq_kernel.cu:17-162, 421-482; torch twin cuda_lstsq.py:91-139)
// =====================================================================================
//
// Three workgroup roles over one launch, all reading the map with 128-byte rows per
// wave:
//   diagonal bands  : 64 diagonals per workgroup, lane = diagonal, waves stride rows
//   column strips   : 64 columns per workgroup, lane = column, waves stride rows
//   frame blocks    : one workgroup per head sums the n/bpf diagonal bpf x bpf blocks
// fp16 inputs accumulate exactly as int64 multiples of 2^-24 (every fp16 value is one),
// so each output is the correctly rounded fp32 of the exact sum whatever the order;
// infinities/NaN are carried separately with float semantics. fp32 inputs accumulate
// in fp64.

constexpr int kMtsThreads = 256;

struct MtsParams {
  const void* map;
  int fp16;
  int heads;
  int n;
  int bpf;
  int n_bands;   // ceil((2n-1)/64)
  int n_strips;  // ceil(n/64)
  float* out;    // (H, 3n)
};

struct Acc {
  long long fixed;  // fp16 inputs: sum in units of 2^-24
  double wide;      // fp32 inputs
  float special;    // sum of the non-finite fp16 inputs (inf/NaN semantics)
};

__device__ __forceinline__ void acc_add_fp16(Acc& a, uint16_t u) {
  const int e = (u >> 10) & 31;
  const int m = u & 1023;
  if (e == 31) {
    a.special += Fp16::to_float(u);
    return;
  }
  long long mag = e == 0 ? static_cast<long long>(m)
                         : static_cast<long long>(1024 + m) << (e - 1);
  a.fixed += (u & 0x8000u) ? -mag : mag;
}

__device__ __forceinline__ void acc_merge(Acc& a, const Acc& b) {
  a.fixed += b.fixed;
  a.wide += b.wide;
  a.special += b.special;
}

__device__ __forceinline__ float acc_result(const Acc& a, bool fp16) {
  if (!fp16) return static_cast<float>(a.wide);
  if (a.special != 0.f || a.special != a.special) return a.special;
  return static_cast<float>(a.fixed) * 0x1p-24f;
}

__device__ __forceinline__ void acc_load(Acc& a, const MtsParams& p, int64_t idx) {
  if (p.fp16)
    acc_add_fp16(a, static_cast<const uint16_t*>(p.map)[idx]);
  else
    a.wide += static_cast<double>(static_cast<const float*>(p.map)[idx]);
}

__global__ __launch_bounds__(kMtsThreads) void mts_kernel(MtsParams p) {
  __shared__ long long s_fixed[kMtsThreads];
  __shared__ double s_wide[kMtsThreads];
  __shared__ float s_special[kMtsThreads];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = p.n;
  const int nd = 2 * n - 1;
  const int F = 3 * n;

  int role_id = blockIdx.x;
  Acc acc{0, 0.0, 0.f};

  if (role_id < p.heads * p.n_bands) {
    // ---- diagonal band ----
    const int h = role_id / p.n_bands;
    const int band = role_id % p.n_bands;
    const int dk = band * 64 + lane;  // diagonal index, offset = dk - (n-1)
    const int off = dk - (n - 1);
    const int off_lo = band * 64 - (n - 1);
    const int off_hi = band * 64 + 63 - (n - 1);
    const int r_lo = off_hi < 0 ? -off_hi : 0;
    const int r_hi = off_lo > 0 ? n - off_lo : n;
    const int64_t base = static_cast<int64_t>(h) * n * n;
    if (dk < nd) {
#pragma unroll 4
      for (int r = r_lo + wave; r < r_hi; r += 4) {
        const int c = r + off;
        if (c >= 0 && c < n) acc_load(acc, p, base + static_cast<int64_t>(r) * n + c);
      }
    }
    s_fixed[tid] = acc.fixed;
    s_wide[tid] = acc.wide;
    s_special[tid] = acc.special;
    __syncthreads();
    if (wave == 0 && dk < nd) {
      for (int w = 1; w < 4; ++w) {
        Acc o{s_fixed[w * 64 + lane], s_wide[w * 64 + lane], s_special[w * 64 + lane]};
        acc_merge(acc, o);
      }
      p.out[static_cast<int64_t>(h) * F + dk] = acc_result(acc, p.fp16);
    }
    return;
  }
  role_id -= p.heads * p.n_bands;

  if (role_id < p.heads * p.n_strips) {
    // ---- column strip ----
    const int h = role_id / p.n_strips;
    const int strip = role_id % p.n_strips;
    const int c = strip * 64 + lane;
    const int64_t base = static_cast<int64_t>(h) * n * n;
    if (c < n) {
#pragma unroll 4
      for (int r = wave; r < n; r += 4) acc_load(acc, p, base + static_cast<int64_t>(r) * n + c);
    }
    s_fixed[tid] = acc.fixed;
    s_wide[tid] = acc.wide;
    s_special[tid] = acc.special;
    __syncthreads();
    if (wave == 0 && c < n) {
      for (int w = 1; w < 4; ++w) {
        Acc o{s_fixed[w * 64 + lane], s_wide[w * 64 + lane], s_special[w * 64 + lane]};
        acc_merge(acc, o);
      }
      p.out[static_cast<int64_t>(h) * F + nd + c] = acc_result(acc, p.fp16);
    }
    return;
  }
  role_id -= p.heads * p.n_strips;

  // ---- frame-diagonal blocks ----
  const int h = role_id;
  const int bpf = p.bpf;
  const int nb = n / bpf;
  const int per = bpf * bpf;
  const int64_t total = static_cast<int64_t>(nb) * per;
  const int64_t base = static_cast<int64_t>(h) * n * n;
  for (int64_t idx = tid; idx < total; idx += kMtsThreads) {
    const int f = static_cast<int>(idx / per);
    const int rem = static_cast<int>(idx % per);
    const int i = rem / bpf;
    const int j = rem % bpf;
    acc_load(acc, p, base + static_cast<int64_t>(f * bpf + i) * n + (f * bpf + j));
  }
  s_fixed[tid] = acc.fixed;
  s_wide[tid] = acc.wide;
  s_special[tid] = acc.special;
  __syncthreads();
  for (int s = kMtsThreads / 2; s > 0; s >>= 1) {
    if (tid < s) {
      s_fixed[tid] += s_fixed[tid + s];
      s_wide[tid] += s_wide[tid + s];
      s_special[tid] += s_special[tid + s];
    }
    __syncthreads();
  }
  if (tid == 0) {
    Acc tot{s_fixed[0], s_wide[0], s_special[0]};
    p.out[static_cast<int64_t>(h) * F + F - 1] = acc_result(tot, p.fp16);
  }
}

// =====================================================================================
// Line prediction + k-smallest selection (MoD/mod/attn_mask.py:351-370)
// =====================================================================================
//
// One workgroup per head. Keys are (ordered(pred) << 14 | index) — unique, so the k-th
// smallest key is found exactly by a 6-pass 8-bit radix select (48 bits), and the k
// selected indices are compacted in ascending index order.

constexpr int kSelThreads = 1024;
constexpr int kSelMaxItems = 16384;  // 3n-1 <= 16384
constexpr int kIdxBits = 14;

__device__ __forceinline__ uint32_t ordered_bits(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // NaN orders last
  if (u == 0x80000000u) u = 0;                              // -0 == +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ int block_exclusive_scan(int v, int* s_wave, int* total) {
  // 1024 threads = 16 wave64s.
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  if (lane == 63) s_wave[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int w = lane < 16 ? s_wave[lane] : 0;
    int wincl = w;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int t = __shfl_up(wincl, o);
      if (lane >= o) wincl += t;
    }
    if (lane < 16) s_wave[lane] = wincl - w;  // exclusive per wave
    if (lane == 15) s_wave[16] = wincl;
  }
  __syncthreads();
  const int res = s_wave[wave] + incl - v;
  *total = s_wave[16];
  __syncthreads();
  return res;
}

__global__ __launch_bounds__(kSelThreads) void select_kernel(const float* __restrict__ x_cur,
                                                             const float* __restrict__ x_last,
                                                             int n, float inv_T_unused, int T,
                                                             int k, int32_t* __restrict__ sel) {
  extern __shared__ __align__(16) unsigned char sel_smem[];
  unsigned long long* keys = reinterpret_cast<unsigned long long*>(sel_smem);
  __shared__ int hist[256];
  __shared__ int s_wave[17];
  __shared__ unsigned long long s_prefix;
  __shared__ int s_kk;

  const int h = blockIdx.x;
  const int tid = threadIdx.x;
  const int F = 3 * n;
  const int items = 3 * n - 1;
  const int nd = 2 * n - 1;
  const float Tf = static_cast<float>(T);
  const float* xc = x_cur + static_cast<int64_t>(h) * F;
  const float* xl = x_last + static_cast<int64_t>(h) * F;

  for (int i = tid; i < items; i += kSelThreads) {
    float cur, last;
    if (i < n) {  // column line i: c = X[:, 2n-1+i] / 2
      cur = xc[nd + i] / 2.0f;
      last = xl[nd + i] / 2.0f;
    } else {  // diagonal line i-n: d = X[:, i-n]
      cur = xc[i - n];
      last = xl[i - n];
    }
    const float step = (cur - last) / Tf;
    const float pred = cur + step;
    keys[i] = (static_cast<unsigned long long>(ordered_bits(pred)) << kIdxBits) |
              static_cast<unsigned long long>(i);
  }
  if (tid == 0) {
    s_prefix = 0ull;
    s_kk = k;
  }
  __syncthreads();

  unsigned long long mask_hi = 0ull;
  for (int shift = 40; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    const unsigned long long prefix = s_prefix;
    for (int i = tid; i < items; i += kSelThreads) {
      const unsigned long long key = keys[i];
      if ((key & mask_hi) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
    }
    __syncthreads();
    if (tid < 64) {
      const int h0 = hist[4 * tid], h1 = hist[4 * tid + 1], h2 = hist[4 * tid + 2],
                h3 = hist[4 * tid + 3];
      const int local = h0 + h1 + h2 + h3;
      int incl = local;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o);
        if (tid >= o) incl += t;
      }
      const int excl = incl - local;
      const int kk = s_kk;
      if (excl < kk && kk <= incl) {
        int before = excl;
        int digit = 4 * tid;
        if (kk > before + h0) {
          before += h0;
          digit++;
          if (kk > before + h1) {
            before += h1;
            digit++;
            if (kk > before + h2) {
              before += h2;
              digit++;
            }
          }
        }
        s_prefix = prefix | (static_cast<unsigned long long>(digit) << shift);
        s_kk = kk - before;
      }
    }
    mask_hi |= 255ull << shift;
    __syncthreads();
  }
  const unsigned long long kth = s_prefix;

  // Ordered compaction of {key <= kth} by index.
  const int chunk = (items + kSelThreads - 1) / kSelThreads;
  const int i0 = tid * chunk;
  int cnt = 0;
  for (int i = i0; i < i0 + chunk && i < items; ++i) cnt += keys[i] <= kth ? 1 : 0;
  int total = 0;
  int pos = block_exclusive_scan(cnt, s_wave, &total);
  int32_t* out = sel + static_cast<int64_t>(h) * k;
  for (int i = i0; i < i0 + chunk && i < items; ++i) {
    if (keys[i] <= kth) {
      if (pos < k) out[pos] = i;
      ++pos;
    }
  }
}

__global__ void check_bd_kernel(const float* __restrict__ x, int heads, int F, float thr,
                                uint8_t* __restrict__ mode) {
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h < heads && mode[h] == MODDIT_MODE_SPARSE) {
    if (x[static_cast<int64_t>(h) * F + F - 1] <= thr) mode[h] = MODDIT_MODE_BLOCK_DIAGONAL;
  }
}

// =====================================================================================
// Block mask + attention tile lists (MoD/mod/attn_mask.py:440-559, 296-311)
// =====================================================================================
//
// One workgroup per (head, 128-row query tile). The selected lines of the head are
// expanded into column / diagonal byte maps in LDS, each thread evaluates the mask for a
// contiguous run of key blocks in both query block rows of the tile, writes the bool
// mask bytes, and an ordered block scan turns active key blocks into ascending tile
// entries (key_tile << 2 | row bits).

constexpr int kMaskThreads = 256;

struct MaskParams {
  const int32_t* sel;      // (H, k) or null when from_mask
  int k;
  const uint8_t* mode;     // (H)
  int n;                   // video blocks per side
  int bpf;
  int layout;
  int nb;                  // mask blocks per side
  int text_blocks;
  int block;               // 64 or 128
  int union_rows;
  const uint8_t* mask_in;  // (H, n_rows, nb) addressed with the strides below (from_mask)
  int64_t in_head_stride;
  int64_t in_row_stride;
  int n_rows;              // mask rows (query blocks); == nb when built from lines
  uint8_t* mask_out;       // (H, nb, nb) or null
  int32_t* counts;         // (H, n_qtiles) or null
  int32_t* entries;        // (H, n_qtiles, cap) or null
  int n_qtiles;
  int cap;
  int kv_tiles;            // key tiles at or beyond are dropped (from_mask only)
};

__device__ __forceinline__ bool video_cell(const uint8_t* colsel, const uint8_t* diagsel,
                                           int mode, int n, int bpf, int i, int j) {
  if (mode == MODDIT_MODE_FULL) return true;
  if (colsel[j] | diagsel[j - i + n - 1]) return true;
  return mode == MODDIT_MODE_BLOCK_DIAGONAL && (i / bpf) == (j / bpf);
}

template <bool kFromMask>
__global__ __launch_bounds__(kMaskThreads) void mask_tiles_kernel(MaskParams p) {
  extern __shared__ __align__(16) unsigned char mk_smem[];
  uint8_t* colsel = mk_smem;          // n bytes
  uint8_t* diagsel = mk_smem + p.n;   // 2n-1 bytes
  __shared__ int s_wave[8];
  __shared__ int s_total;

  const int tid = threadIdx.x;
  const int h = blockIdx.x / p.n_qtiles;
  const int t = blockIdx.x % p.n_qtiles;
  const int n = p.n;
  const int nb = p.nb;
  int mode = 0;

  if (!kFromMask) {
    mode = p.mode ? p.mode[h] : MODDIT_MODE_SPARSE;
    for (int i = tid; i < 3 * n - 1; i += kMaskThreads) mk_smem[i] = 0;
    __syncthreads();
    const int32_t* s = p.sel + static_cast<int64_t>(h) * p.k;
    for (int i = tid; i < p.k; i += kMaskThreads) {
      const int idx = s[i];
      if (idx >= 0 && idx < n) colsel[idx] = 1;
      else if (idx >= n && idx < 3 * n - 1) diagsel[idx - n] = 1;
    }
    __syncthreads();
  }

  // Mask rows covered by this query tile.
  const int rows_per_tile = p.block == 64 ? 2 : 1;
  const int r0 = t * rows_per_tile;
  const int r1 = r0 + 1;
  const int n_rows = p.n_rows;
  const bool has_r1 = rows_per_tile == 2 && r1 < n_rows;

  auto cell = [&](int i, int j) -> bool {
    if (kFromMask) return p.mask_in[h * p.in_head_stride + i * p.in_row_stride + j] != 0;
    switch (p.layout) {
      case MODDIT_LAYOUT_WAN:
        return video_cell(colsel, diagsel, mode, n, p.bpf, i, j);
      case MODDIT_LAYOUT_HUNYUAN:
        if (i < n && j < n) return video_cell(colsel, diagsel, mode, n, p.bpf, i, j);
        return true;
      case MODDIT_LAYOUT_COGVIDEOX: {
        const int tb = p.text_blocks;
        if (i >= tb && j >= tb) return video_cell(colsel, diagsel, mode, n, p.bpf, i - tb, j - tb);
        return true;
      }
      default:
        return true;
    }
  };

  const int chunk = (nb + kMaskThreads - 1) / kMaskThreads;
  const int j0 = tid * chunk;
  const int j1 = j0 + chunk < nb ? j0 + chunk : nb;
  const int tiles_per_col = p.block == 64 ? 1 : 2;

  // pass 1: mask bytes + entry count
  int cnt = 0;
  for (int j = j0; j < j1; ++j) {
    const bool m0 = r0 < n_rows && cell(r0, j);
    const bool m1 = has_r1 && cell(r1, j);
    if (!kFromMask && p.mask_out) {
      if (r0 < n_rows) p.mask_out[(static_cast<int64_t>(h) * nb + r0) * nb + j] = m0;
      if (has_r1) p.mask_out[(static_cast<int64_t>(h) * nb + r1) * nb + j] = m1;
    }
    if (m0 || m1) {
      for (int s = 0; s < tiles_per_col; ++s)
        if (j * tiles_per_col + s < p.kv_tiles) ++cnt;
    }
  }
  if (p.counts == nullptr) return;

  // block exclusive scan of cnt (256 threads = 4 waves)
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  if (lane == 63) s_wave[wave] = incl;
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int w = 0; w < kMaskThreads / 64; ++w) {
      const int v = s_wave[w];
      s_wave[w] = run;
      run += v;
    }
    s_total = run;
  }
  __syncthreads();
  int pos = s_wave[wave] + incl - cnt;

  const int64_t slot = static_cast<int64_t>(h) * p.n_qtiles + t;
  int32_t* out = p.entries + slot * p.cap;
  for (int j = j0; j < j1; ++j) {
    const bool m0 = r0 < n_rows && cell(r0, j);
    const bool m1 = has_r1 && cell(r1, j);
    if (!(m0 || m1)) continue;
    int bits;
    if (p.block == 128 || p.union_rows) bits = 3;
    else bits = (m0 ? 1 : 0) | (m1 ? 2 : 0);
    for (int s = 0; s < tiles_per_col; ++s) {
      const int kt = j * tiles_per_col + s;
      if (kt < p.kv_tiles) {
        if (pos < p.cap) out[pos] = (kt << 2) | bits;
        ++pos;
      }
    }
  }
  if (tid == 0) p.counts[slot] = s_total < p.cap ? s_total : p.cap;
}

// =====================================================================================
// Refresh merge (MoD/mod/attn_mask.py:671-675)
// =====================================================================================
__global__ void refresh_merge_kernel(const uint16_t* __restrict__ prev,
                                     const uint16_t* __restrict__ cur,
                                     const uint8_t* __restrict__ mask, int64_t mhs, int64_t mrs,
                                     int heads, int n, uint16_t* out) {
  const int64_t total = static_cast<int64_t>(heads) * n * n;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t h = idx / (static_cast<int64_t>(n) * n);
    const int64_t rem = idx - h * n * n;
    const int64_t i = rem / n;
    const int64_t j = rem - i * n;
    const bool m = mask[h * mhs + i * mrs + j] != 0;
    out[idx] = m ? cur[idx] : prev[idx];
  }
}

}  // namespace
}  // namespace moddit

using namespace moddit;

extern "C" int moddit_mts(const void* map, int map_dtype, int heads, int n, int blocks_per_frame,
                          float* mts_out, moddit_stream_t stream) {
  clear_error();
  MODDIT_CHECK_ARG(map && mts_out, "mts: null pointer argument");
  MODDIT_CHECK_ARG(map_dtype == MODDIT_FP16 || map_dtype == MODDIT_FP32,
                   "mts: map dtype must be fp16 or fp32");
  MODDIT_CHECK_ARG(heads >= 0 && n > 0, "mts: invalid shape heads=%d n=%d", heads, n);
  MODDIT_CHECK_ARG(blocks_per_frame > 0, "mts: blocks_per_frame must be positive, got %d",
                   blocks_per_frame);
  if (heads == 0) return MODDIT_OK;
  MtsParams p;
  p.map = map;
  p.fp16 = map_dtype == MODDIT_FP16;
  p.heads = heads;
  p.n = n;
  p.bpf = blocks_per_frame;
  p.n_bands = (2 * n - 1 + 63) / 64;
  p.n_strips = (n + 63) / 64;
  p.out = mts_out;
  const int64_t grid = static_cast<int64_t>(heads) * (p.n_bands + p.n_strips + 1);
  MODDIT_CHECK_ARG(grid < 0x7fffffff, "mts: shape too large");
  hipLaunchKernelGGL(mts_kernel, dim3(static_cast<unsigned>(grid)), dim3(kMtsThreads), 0,
                     as_stream(stream), p);
  MODDIT_CHECK_LAUNCH("mts");
  return MODDIT_OK;
}

// Closed form of M^T M + lambda I (MoD/mod/cuda_lstsq.py:42-89). Column order of M:
// [2n-1 diagonals by offset -(n-1)..n-1][n columns][1 frame-block-diagonal].
extern "C" int moddit_mtm_host(int n, int blocks_per_frame, double regularization,
                               double* mtm_out) {
  clear_error();
  MODDIT_CHECK_ARG(mtm_out != nullptr, "mtm: null output");
  MODDIT_CHECK_ARG(n > 0 && blocks_per_frame > 0, "mtm: invalid n=%d bpf=%d", n, blocks_per_frame);
  const int nd = 2 * n - 1;
  const int64_t F = 3 * static_cast<int64_t>(n);
  for (int64_t i = 0; i < F * F; ++i) mtm_out[i] = 0.0;
  const int bpf = blocks_per_frame;
  const int nbk = n / bpf;
  for (int kd = 0; kd < nd; ++kd) {
    const int off = kd - (n - 1);
    const int aoff = off < 0 ? -off : off;
    mtm_out[kd * F + kd] = static_cast<double>(n - aoff);
    for (int c = 0; c < n; ++c) {
      // diagonal with col-row = off crosses column c iff row = c - off is in [0, n)
      const bool hit = off >= 0 ? (c >= off) : (c < n + off);
      if (hit) {
        mtm_out[kd * F + nd + c] = 1.0;
        mtm_out[(nd + c) * F + kd] = 1.0;
      }
    }
    const double db = aoff < bpf ? static_cast<double>(nbk) * (bpf - aoff) : 0.0;
    mtm_out[kd * F + (F - 1)] = db;
    mtm_out[(F - 1) * F + kd] = db;
  }
  for (int c = 0; c < n; ++c) {
    mtm_out[(nd + c) * F + nd + c] = static_cast<double>(n);
    const double vb = c < nbk * bpf ? static_cast<double>(bpf) : 0.0;
    mtm_out[(nd + c) * F + (F - 1)] = vb;
    mtm_out[(F - 1) * F + nd + c] = vb;
  }
  mtm_out[(F - 1) * F + (F - 1)] = static_cast<double>(nbk) * bpf * bpf;
  for (int64_t i = 0; i < F; ++i) mtm_out[i * F + i] += regularization;
  return MODDIT_OK;
}

extern "C" int moddit_select_lines(const float* x_cur, const float* x_last, int heads, int n,
                                   int predict_T, int top_k, int32_t* sel_out,
                                   moddit_stream_t stream) {
  clear_error();
  MODDIT_CHECK_ARG(x_cur && x_last && sel_out, "select_lines: null pointer argument");
  MODDIT_CHECK_ARG(n > 0 && heads >= 0, "select_lines: invalid shape");
  MODDIT_CHECK_ARG(predict_T != 0, "select_lines: predict_T must be nonzero");
  const int items = 3 * n - 1;
  MODDIT_CHECK_ARG(items <= kSelMaxItems, "select_lines: 3n-1=%d exceeds %d", items, kSelMaxItems);
  MODDIT_CHECK_ARG(top_k > 0, "select_lines: top_k must be positive, got %d", top_k);
  const int k = top_k < items ? top_k : items;
  if (heads == 0) return MODDIT_OK;
  const size_t lds = static_cast<size_t>(items) * sizeof(unsigned long long);
  static LaunchSetup once;
  if (set_dynamic_lds_once(once, reinterpret_cast<const void*>(select_kernel),
                           kSelMaxItems * 8) != hipSuccess) {
    set_error("select_lines: cannot reserve LDS");
    return MODDIT_EHIP;
  }
  hipLaunchKernelGGL(select_kernel, dim3(heads), dim3(kSelThreads), lds, as_stream(stream), x_cur,
                     x_last, n, 0.f, predict_T, k, sel_out);
  MODDIT_CHECK_LAUNCH("select_lines");
  return MODDIT_OK;
}

extern "C" int moddit_check_bd(const float* x, int heads, int features, float threshold,
                               uint8_t* mode, moddit_stream_t stream) {
  clear_error();
  MODDIT_CHECK_ARG(x && mode, "check_bd: null pointer argument");
  MODDIT_CHECK_ARG(heads >= 0 && features > 0, "check_bd: invalid shape");
  if (heads == 0) return MODDIT_OK;
  hipLaunchKernelGGL(check_bd_kernel, dim3((heads + 63) / 64), dim3(64), 0, as_stream(stream), x,
                     heads, features, threshold, mode);
  MODDIT_CHECK_LAUNCH("check_bd");
  return MODDIT_OK;
}

static int check_tile_outputs(int n_rows, int nb, int block_size, int n_qtiles, int cap) {
  const int64_t tokens = static_cast<int64_t>(n_rows) * block_size;
  const int64_t need_q = (tokens + 127) / 128;
  MODDIT_CHECK_ARG(n_qtiles == need_q, "mask tiles: n_qtiles=%d but %lld mask tokens need %lld",
                   n_qtiles, static_cast<long long>(tokens), static_cast<long long>(need_q));
  MODDIT_CHECK_ARG(cap >= nb * (block_size / 64), "mask tiles: cap=%d below %d key tiles", cap,
                   nb * (block_size / 64));
  return MODDIT_OK;
}

extern "C" int moddit_mask_from_lines(const int32_t* sel, int heads, int k, const uint8_t* mode,
                                      int n, int blocks_per_frame, int layout, int nb,
                                      int text_blocks, int block_size, int union_rows,
                                      uint8_t* mask_out, int32_t* counts, int32_t* entries,
                                      int n_qtiles, int cap, moddit_stream_t stream) {
  clear_error();
  MODDIT_CHECK_ARG(sel != nullptr || k == 0, "mask_from_lines: null selection");
  MODDIT_CHECK_ARG(heads >= 0 && n > 0 && nb > 0 && k >= 0, "mask_from_lines: invalid shape");
  MODDIT_CHECK_ARG(blocks_per_frame > 0, "mask_from_lines: blocks_per_frame must be positive");
  MODDIT_CHECK_ARG(block_size == 64 || block_size == 128, "mask_from_lines: block_size must be 64 or 128");
  MODDIT_CHECK_ARG(layout >= 0 && layout <= MODDIT_LAYOUT_OTHER, "mask_from_lines: bad layout");
  MODDIT_CHECK_ARG((counts == nullptr) == (entries == nullptr),
                   "mask_from_lines: counts and entries go together");
  if (layout == MODDIT_LAYOUT_WAN) MODDIT_CHECK_ARG(nb == n, "mask_from_lines: wan layout needs nb == n");
  if (layout == MODDIT_LAYOUT_HUNYUAN) MODDIT_CHECK_ARG(nb >= n, "mask_from_lines: hunyuan layout needs nb >= n");
  if (layout == MODDIT_LAYOUT_COGVIDEOX)
    MODDIT_CHECK_ARG(text_blocks >= 0 && nb - text_blocks == n,
                     "mask_from_lines: cogvideox layout needs nb - text_blocks == n");
  if (counts) {
    int rc = check_tile_outputs(nb, nb, block_size, n_qtiles, cap);
    if (rc) return rc;
  } else {
    n_qtiles = static_cast<int>((static_cast<int64_t>(nb) * block_size + 127) / 128);
  }
  if (heads == 0) return MODDIT_OK;
  MaskParams p{};
  p.sel = sel;
  p.k = k;
  p.mode = mode;
  p.n = n;
  p.bpf = blocks_per_frame;
  p.layout = layout;
  p.nb = nb;
  p.text_blocks = text_blocks;
  p.block = block_size;
  p.union_rows = union_rows;
  p.mask_out = mask_out;
  p.n_rows = nb;
  p.counts = counts;
  p.entries = entries;
  p.n_qtiles = n_qtiles;
  p.cap = cap;
  p.kv_tiles = 0x7fffffff;
  const size_t lds = static_cast<size_t>(3 * n);
  MODDIT_CHECK_ARG(lds <= 65536, "mask_from_lines: n=%d too large", n);
  const int64_t grid = static_cast<int64_t>(heads) * n_qtiles;
  hipLaunchKernelGGL(mask_tiles_kernel<false>, dim3(static_cast<unsigned>(grid)),
                     dim3(kMaskThreads), lds, as_stream(stream), p);
  MODDIT_CHECK_LAUNCH("mask_from_lines");
  return MODDIT_OK;
}

extern "C" int moddit_mask_to_tiles(const uint8_t* mask, int heads, int n_rows, int n_cols,
                                    int64_t mask_head_stride, int64_t mask_row_stride,
                                    int block_size, int union_rows, int kv_tiles,
                                    int32_t* counts, int32_t* entries, int n_qtiles, int cap,
                                    moddit_stream_t stream) {
  clear_error();
  MODDIT_CHECK_ARG(mask && counts && entries, "mask_to_tiles: null pointer argument");
  MODDIT_CHECK_ARG(heads >= 0 && n_rows > 0 && n_cols > 0, "mask_to_tiles: invalid shape");
  MODDIT_CHECK_ARG(mask_head_stride >= 0 && mask_row_stride >= n_cols,
                   "mask_to_tiles: invalid mask strides");
  MODDIT_CHECK_ARG(block_size == 64 || block_size == 128, "mask_to_tiles: block_size must be 64 or 128");
  int rc = check_tile_outputs(n_rows, n_cols, block_size, n_qtiles, cap);
  if (rc) return rc;
  if (heads == 0) return MODDIT_OK;
  MaskParams p{};
  p.n = 1;
  p.bpf = 1;
  p.nb = n_cols;
  p.n_rows = n_rows;
  p.block = block_size;
  p.union_rows = union_rows;
  p.mask_in = mask;
  p.in_head_stride = mask_head_stride;
  p.in_row_stride = mask_row_stride;
  p.counts = counts;
  p.entries = entries;
  p.n_qtiles = n_qtiles;
  p.cap = cap;
  p.kv_tiles = kv_tiles < 0 ? 0 : kv_tiles;
  const int64_t grid = static_cast<int64_t>(heads) * n_qtiles;
  hipLaunchKernelGGL(mask_tiles_kernel<true>, dim3(static_cast<unsigned>(grid)),
                     dim3(kMaskThreads), 16, as_stream(stream), p);
  MODDIT_CHECK_LAUNCH("mask_to_tiles");
  return MODDIT_OK;
}

extern "C" int moddit_refresh_merge(const void* prev, const void* cur, const uint8_t* mask,
                                    int64_t mask_head_stride, int64_t mask_row_stride, int heads,
                                    int n, void* out, moddit_stream_t stream) {
  clear_error();
  MODDIT_CHECK_ARG(prev && cur && mask && out, "refresh_merge: null pointer argument");
  MODDIT_CHECK_ARG(heads >= 0 && n >= 0, "refresh_merge: invalid shape");
  const int64_t total = static_cast<int64_t>(heads) * n * n;
  if (total == 0) return MODDIT_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(refresh_merge_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     as_stream(stream), static_cast<const uint16_t*>(prev),
                     static_cast<const uint16_t*>(cur), mask, mask_head_stride, mask_row_stride,
                     heads, n, static_cast<uint16_t*>(out));
  MODDIT_CHECK_LAUNCH("refresh_merge");
  return MODDIT_OK;
}
