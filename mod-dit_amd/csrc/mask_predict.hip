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
// fp32 maps: three workgroup roles over one launch, all reading the map with 128-byte
// rows per wave:
//   diagonal bands  : 64 diagonals per workgroup, lane = diagonal, waves stride rows
//   column strips   : 64 columns per workgroup, lane = column, waves stride rows
//   frame blocks    : one workgroup per head sums the n/bpf diagonal bpf x bpf blocks
// Sums accumulate in fp64 and are rounded once (deterministic: fixed order).

constexpr int kMtsThreads = 256;

struct MtsParams {
  const float* map;
  int heads;
  int n;
  int bpf;
  int n_bands;   // ceil((2n-1)/64)
  int n_strips;  // ceil(n/64)
  float* out;    // (H, 3n)
};

__global__ __launch_bounds__(kMtsThreads) void mts_kernel(MtsParams p) {
  __shared__ double s_wide[kMtsThreads];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = p.n;
  const int nd = 2 * n - 1;
  const int F = 3 * n;

  int role_id = blockIdx.x;
  double acc = 0.0;

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
        if (c >= 0 && c < n) acc += static_cast<double>(p.map[base + static_cast<int64_t>(r) * n + c]);
      }
    }
    s_wide[tid] = acc;
    __syncthreads();
    if (wave == 0 && dk < nd) {
      for (int w = 1; w < 4; ++w) acc += s_wide[w * 64 + lane];
      p.out[static_cast<int64_t>(h) * F + dk] = static_cast<float>(acc);
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
      for (int r = wave; r < n; r += 4) acc += static_cast<double>(p.map[base + static_cast<int64_t>(r) * n + c]);
    }
    s_wide[tid] = acc;
    __syncthreads();
    if (wave == 0 && c < n) {
      for (int w = 1; w < 4; ++w) acc += s_wide[w * 64 + lane];
      p.out[static_cast<int64_t>(h) * F + nd + c] = static_cast<float>(acc);
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
    acc += static_cast<double>(p.map[base + static_cast<int64_t>(f * bpf + i) * n + (f * bpf + j)]);
  }
  s_wide[tid] = acc;
  __syncthreads();
  for (int s = kMtsThreads / 2; s > 0; s >>= 1) {
    if (tid < s) s_wide[tid] += s_wide[tid + s];
    __syncthreads();
  }
  if (tid == 0) p.out[static_cast<int64_t>(h) * F + F - 1] = static_cast<float>(s_wide[0]);
}

// -------------------------------------------------------------------------------------
// Single pass over an fp16 map (the product path). One workgroup per (head, 512-row x
// 256-column tile) reads its cells once with 16-byte loads. Each thread owns 8 consecutive
// columns of one 64-row slab of the tile and keeps its column sums and, per 16-row
// sub-block, the sums of the 23 diagonals its 8 x 16 cells lie on in fp64 registers.
// Every finite fp16 value is a multiple of 2^-24 below 2^16, so any sum of at most 8192 of
// them needs at most 53 significant bits and is exact in fp64 in any order; a tile's
// share of one line is at most 512 cells. The eight slabs' column sums and the threads'
// overlapping diagonal sums are combined in LDS (still exact), and each workgroup adds
// its column, diagonal and frame-block partials into an int64 accumulator per output
// (units of 2^-24) with global integer atomics: exact and order-independent, so every
// output is the correctly rounded fp32 of the exact sum in any workgroup order
// (deterministic), and the map is read once (155.5 MB at the headline). A partial that is
// not finite (inf/NaN inputs) goes into a float side accumulator instead (inf/NaN
// semantics only, also order-independent). The tile shape minimises the global atomics
// per cell for its area (256 column + 767 diagonal partials per 131,072 cells): contended
// atomics, not the loads, were what bounded the 64-row-block version of this pass.
constexpr int kMts1Threads = 256;
constexpr int kMts1Cols = 8;         // columns per thread
constexpr int kMts1Sub = 16;         // rows per register sub-block
constexpr int kMts1Slab = 64;        // rows per thread
constexpr int kMts1ColThreads = 32;  // threads across a tile's columns
constexpr int kMts1Slabs = kMts1Threads / kMts1ColThreads;   // 8
constexpr int kMts1TileC = kMts1ColThreads * kMts1Cols;      // 256
constexpr int kMts1TileR = kMts1Slabs * kMts1Slab;           // 512
constexpr int kMts1Diag = kMts1Cols + kMts1Sub - 1;          // 23
constexpr int kMts1TileDiag = kMts1TileC + kMts1TileR - 1;   // 767
// Exactness of the int64 accumulators: an fp16 value is below 2^16, i.e. 2^40 units of
// 2^-24, so a sum over c cells stays below 2^63 while c <= 2^23. Diagonal and column
// outputs sum n cells; the frame-block output sums (n / bpf) * bpf^2 = n * min(bpf, n)
// cells, which the entry point bounds (kMts1MaxFrameCells).
constexpr int kMts1MaxN = 1 << 20;
constexpr int64_t kMts1MaxFrameCells = int64_t{1} << 23;

struct Mts1Params {
  const uint16_t* map;
  int heads;
  int n;
  int bpf;
  int n_rt;  // row tiles per head
  int n_ct;  // column tiles per head
  unsigned long long* acc;  // (H, 3n) int64 units of 2^-24 (two's complement)
  float* special;           // (H, 3n) sums of the non-finite partials
  float* out;               // (H, 3n)
};

// Adds an exact fp64 partial (a multiple of 2^-24, |x| < 2^25) to an output.
__device__ __forceinline__ void mts1_flush(const Mts1Params& p, int64_t idx, double x) {
  if (x == 0.0) return;
  if (__builtin_isfinite(x)) {
    atomicAdd(&p.acc[idx], static_cast<unsigned long long>(static_cast<long long>(x * 0x1p24)));
  } else {
    atomicAdd(&p.special[idx], static_cast<float>(x));
  }
}

__global__ void mts1_zero_kernel(Mts1Params p) {
  const int64_t total = static_cast<int64_t>(p.heads) * 3 * p.n;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    p.acc[i] = 0ull;
    p.special[i] = 0.f;
  }
}

template <bool kVec>
__global__ __launch_bounds__(kMts1Threads) void mts1_kernel(Mts1Params p) {
  __shared__ double s_diag[kMts1TileDiag];
  __shared__ double s_col[kMts1Slabs][kMts1TileC];
  __shared__ long long s_frame[kMts1Threads / 64];
  const int tid = threadIdx.x;
  const int tc = tid % kMts1ColThreads;
  const int tr = tid / kMts1ColThreads;
  const int tiles = p.n_rt * p.n_ct;
  const int h = blockIdx.x / tiles;
  const int t = blockIdx.x - h * tiles;
  const int R0 = (t / p.n_ct) * kMts1TileR;
  const int C0 = (t % p.n_ct) * kMts1TileC;
  const int n = p.n;
  const int nd = 2 * n - 1;
  const int64_t F = 3 * static_cast<int64_t>(n);
  const int frame_end = (n / p.bpf) * p.bpf;
  for (int i = tid; i < kMts1TileDiag; i += kMts1Threads) s_diag[i] = 0.0;
  __syncthreads();

  const int c0 = C0 + tc * kMts1Cols;   // this thread's first column
  const int rs = R0 + tr * kMts1Slab;   // this thread's first row
  const uint16_t* base = p.map + static_cast<int64_t>(h) * n * n;
  const int64_t out0 = static_cast<int64_t>(h) * F;
  // frames of the first and last owned columns inside the frame blocks (-1: none)
  const int c_last = (c0 + kMts1Cols - 1 < frame_end ? c0 + kMts1Cols - 1 : frame_end - 1);
  const int cf_lo = c0 < frame_end ? c0 / p.bpf : -1;
  const int cf_hi = c0 < frame_end ? c_last / p.bpf : -1;
  double cacc[kMts1Cols];
#pragma unroll
  for (int j = 0; j < kMts1Cols; ++j) cacc[j] = 0.0;
  double fsum = 0.0;
  if (c0 < n) {
    for (int s0 = 0; s0 < kMts1Slab; s0 += kMts1Sub) {
      if (rs + s0 >= n) break;
      double dacc[kMts1Diag];
#pragma unroll
      for (int d = 0; d < kMts1Diag; ++d) dacc[d] = 0.0;
#pragma unroll
      for (int rr = 0; rr < kMts1Sub; ++rr) {
        const int r = rs + s0 + rr;
        if (r < n) {
          const uint16_t* row = base + static_cast<int64_t>(r) * n;
          uint16_t v[kMts1Cols];
          if constexpr (kVec) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(row + c0);
#pragma unroll
            for (int j = 0; j < kMts1Cols; ++j) v[j] = u16_at(w, j);
          } else {
#pragma unroll
            for (int j = 0; j < kMts1Cols; ++j) v[j] = c0 + j < n ? row[c0 + j] : 0;
          }
          double x[kMts1Cols];
#pragma unroll
          for (int j = 0; j < kMts1Cols; ++j) {
            x[j] = static_cast<double>(Fp16::to_float(v[j]));
            cacc[j] += x[j];
            dacc[j - rr + kMts1Sub - 1] += x[j];
          }
          // frame-block cells: only rows whose frame meets the owned columns
          const int rframe = r < frame_end ? r / p.bpf : -2;
          if (rframe >= cf_lo && rframe <= cf_hi) {
#pragma unroll
            for (int j = 0; j < kMts1Cols; ++j)
              if (c0 + j < frame_end && (c0 + j) / p.bpf == rframe) fsum += x[j];
          }
        }
      }
      // local diagonal kl = (c - C0) - (r - R0) + 511 of accumulator d
#pragma unroll
      for (int d = 0; d < kMts1Diag; ++d) {
        const int kl = (c0 - C0) + d - (kMts1Sub - 1) - (rs - R0) - s0 + (kMts1TileR - 1);
        if (dacc[d] != 0.0) atomicAdd(&s_diag[kl], dacc[d]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kMts1Cols; ++j) s_col[tr][tc * kMts1Cols + j] = cacc[j];
  // frame-block partial of the workgroup: each thread's sum (at most 512 cells) is exact in
  // fp64 and converts exactly to int64 units; the workgroup adds them as integers
  long long fq = 0;
  if (__builtin_isfinite(fsum))
    fq = static_cast<long long>(fsum * 0x1p24);
  else
    atomicAdd(&p.special[out0 + F - 1], static_cast<float>(fsum));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) fq += __shfl_xor(fq, o);
  if ((tid & 63) == 0) s_frame[tid >> 6] = fq;
  __syncthreads();
  if (tid == 0) {
    long long tot = 0;
    for (int w = 0; w < kMts1Threads / 64; ++w) tot += s_frame[w];
    if (tot != 0) atomicAdd(&p.acc[out0 + F - 1], static_cast<unsigned long long>(tot));
  }
  // column partials: the eight slabs' sums of one column (at most 512 cells, exact)
  for (int c = tid; c < kMts1TileC; c += kMts1Threads) {
    double sum = 0.0;
#pragma unroll
    for (int sl = 0; sl < kMts1Slabs; ++sl) sum += s_col[sl][c];
    if (C0 + c < n) mts1_flush(p, out0 + nd + C0 + c, sum);
  }
  // diagonal partials: global index k = (c - r) + n - 1 = kl - 511 + C0 - R0 + n - 1
  for (int kl = tid; kl < kMts1TileDiag; kl += kMts1Threads) {
    const int k = kl - (kMts1TileR - 1) + C0 - R0 + n - 1;
    if (k >= 0 && k < nd) mts1_flush(p, out0 + k, s_diag[kl]);
  }
}

__global__ void mts1_finalize_kernel(Mts1Params p) {
  const int64_t total = static_cast<int64_t>(p.heads) * 3 * p.n;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const float sp = p.special[i];
    p.out[i] = (sp != 0.f || sp != sp)
                   ? sp
                   : static_cast<float>(static_cast<long long>(p.acc[i])) * 0x1p-24f;
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

// LDS of the line-based mask kernel: column bytes, then the diagonal bytes at an 8-byte
// aligned offset plus 8 bytes of zero padding for the unaligned 8-byte windows.
__host__ __device__ inline int mask_diag_offset(int n) { return (n + 7) & ~7; }
__host__ __device__ inline int mask_lds_bytes(int n) {
  return mask_diag_offset(n) + ((2 * n - 1 + 7) & ~7) + 8;
}

// Tiles per workgroup: the selected-line byte maps are built in LDS once per workgroup
// and serve this many consecutive query tiles of the head.
constexpr int kMaskTilesPerWg = 8;
static_assert(kMaskTilesPerWg % 4 == 0, "the batched path packs four tiles per 64-bit word");
constexpr int kMaskCols = 8;  // mask columns per thread and pass
static_assert(kMaskThreads * kMaskCols * 2 < 65536, "a tile's entry count fits 16 bits");

template <bool kFromMask>
__global__ __launch_bounds__(kMaskThreads) void mask_tiles_kernel(MaskParams p) {
  extern __shared__ __align__(16) unsigned char mk_smem[];
  // colsel: n bytes; diagsel: 2n-1 bytes at an 8-byte aligned offset, followed by zero
  // padding so that the 8-byte windows read below stay inside the allocation
  const int diag_off = mask_diag_offset(p.n);
  uint8_t* colsel = mk_smem;
  uint8_t* diagsel = mk_smem + diag_off;
  __shared__ int s_wave[8];
  __shared__ int s_total;
  __shared__ int s_wpack[kMaskThreads / 64][kMaskTilesPerWg / 2];

  const int tid = threadIdx.x;
  const int wg_per_head = (p.n_qtiles + kMaskTilesPerWg - 1) / kMaskTilesPerWg;
  const int h = blockIdx.x / wg_per_head;
  const int t_begin = (blockIdx.x % wg_per_head) * kMaskTilesPerWg;
  const int t_end = t_begin + kMaskTilesPerWg < p.n_qtiles ? t_begin + kMaskTilesPerWg : p.n_qtiles;
  const int n = p.n;
  const int nb = p.nb;
  int mode = 0;

  if (!kFromMask) {
    mode = p.mode ? p.mode[h] : MODDIT_MODE_SPARSE;
    for (int i = tid; i < mask_lds_bytes(n) / 8; i += kMaskThreads)
      reinterpret_cast<uint64_t*>(mk_smem)[i] = 0;
    __syncthreads();
    const int32_t* s = p.sel + static_cast<int64_t>(h) * p.k;
    for (int i = tid; i < p.k; i += kMaskThreads) {
      const int idx = s[i];
      if (idx >= 0 && idx < n) colsel[idx] = 1;
      else if (idx >= n && idx < 3 * n - 1) diagsel[idx - n] = 1;
    }
    __syncthreads();
  }
  // Video block index of mask row/column q (-1 outside the video: all-true text rows and
  // columns of the hunyuan / cogvideox layouts; every cell of the 'other' layout).
  auto video_index = [&](int q) -> int {
    switch (p.layout) {
      case MODDIT_LAYOUT_WAN: return q;
      case MODDIT_LAYOUT_HUNYUAN: return q < n ? q : -1;
      case MODDIT_LAYOUT_COGVIDEOX: return q >= p.text_blocks ? q - p.text_blocks : -1;
      default: return -1;
    }
  };
  const bool full = mode == MODDIT_MODE_FULL;
  const bool bd = mode == MODDIT_MODE_BLOCK_DIAGONAL;
  const int rows_per_tile = p.block == 64 ? 2 : 1;
  const int tiles_per_col = p.block == 64 ? 1 : 2;
  const int n_rows = p.n_rows;
  const bool vec_mask = (nb % kMaskCols) == 0 && p.mask_out != nullptr &&
                        (reinterpret_cast<uintptr_t>(p.mask_out) & 7) == 0;

  // Per-column values do not depend on the query tile: computed once per workgroup for
  // this thread's columns of the first pass (the only pass while nb <= 2048), and on the
  // fly for the columns of later passes.
  // Rows are evaluated as 8 bytes (0/1), one per owned column: the selected-column and
  // text-column bytes are fixed per workgroup, and when the 8 columns are consecutive video
  // blocks their diagonal bytes for video row iv are the 8 consecutive diagsel bytes from
  // jv0 - iv + n - 1, read as one unaligned window.
  int jv_h[kMaskCols], jf_h[kMaskCols];
  uint64_t col_bytes = 0, text_bytes = 0, valid_bytes = 0;
  bool all_video = !kFromMask && tid * kMaskCols + kMaskCols <= nb;
  if (!kFromMask) {
#pragma unroll
    for (int c = 0; c < kMaskCols; ++c) {
      const int j = tid * kMaskCols + c;
      const int jv = j < nb ? video_index(j) : -1;
      jv_h[c] = jv;
      jf_h[c] = (bd && jv >= 0) ? jv / p.bpf : -3;
      if (j < nb) valid_bytes |= 1ull << (8 * c);
      if (j < nb && jv < 0) text_bytes |= 1ull << (8 * c);
      if (jv >= 0 && colsel[jv]) col_bytes |= 1ull << (8 * c);
      if (jv < 0 || jv != jv_h[0] + c) all_video = false;
    }
  }
  auto row_bytes = [&](bool has, int iv, int ifr) -> uint64_t {
    if (!has) return 0;
    if (iv < 0 || full) return valid_bytes;
    uint64_t r = col_bytes | text_bytes;
    if (all_video) {
      const int d0 = jv_h[0] - iv + n - 1;  // in [0, 2n-9]
      const uint64_t* w = reinterpret_cast<const uint64_t*>(diagsel) + (d0 >> 3);
      const int sh = (d0 & 7) * 8;
      const uint64_t lo = w[0];
      r |= sh ? (lo >> sh) | (w[1] << (64 - sh)) : lo;
    } else {
#pragma unroll
      for (int c = 0; c < kMaskCols; ++c)
        if (jv_h[c] >= 0 && diagsel[jv_h[c] - iv + n - 1]) r |= 1ull << (8 * c);
    }
    if (bd) {
#pragma unroll
      for (int c = 0; c < kMaskCols; ++c)
        if (jf_h[c] == ifr) r |= 1ull << (8 * c);
    }
    return r & valid_bytes;
  };
  // bit c of the result = byte c (0 or 1) of v; no partial product carries into the top byte
  auto byte_bits = [](uint64_t v) -> unsigned {
    return static_cast<unsigned>((v * 0x0102040810204080ull) >> 56);
  };

  if (!kFromMask && nb <= kMaskThreads * kMaskCols) {
    // One pass covers every column: evaluate all of the workgroup's tiles first, then place
    // all of their entries with one scan of the per-thread counts. Row bits and counts of
    // the tiles sit in 16-bit fields of 64-bit registers, four tiles per register (a
    // workgroup's count per tile is at most 4096), so the loops stay rolled. Entries here never reach kv_tiles
    // (line-based masks have no key-tile limit).
    const int j0 = tid * kMaskCols;
    uint64_t bits_w[kMaskTilesPerWg / 4];  // tile tt: m0 | m1 << 8 at bits 16 * (tt & 3) of word tt >> 2
    uint64_t cnt_w[kMaskTilesPerWg / 4];   // tile tt: entry count, same place
#pragma unroll
    for (int i = 0; i < kMaskTilesPerWg / 4; ++i) bits_w[i] = cnt_w[i] = 0;
#pragma unroll 1
    for (int tt = 0; tt < t_end - t_begin; ++tt) {
      const int t = t_begin + tt;
      const int r0 = t * rows_per_tile;
      const int r1 = r0 + 1;
      const bool has_r0 = r0 < n_rows;
      const bool has_r1 = rows_per_tile == 2 && r1 < n_rows;
      const int iv0 = video_index(r0);
      const int iv1 = video_index(r1);
      const uint64_t b0 = row_bytes(has_r0, iv0, iv0 >= 0 ? iv0 / p.bpf : -2);
      const uint64_t b1 = row_bytes(has_r1, iv1, iv1 >= 0 ? iv1 / p.bpf : -2);
      const unsigned m0 = byte_bits(b0);
      const unsigned m1 = byte_bits(b1);
      if (p.mask_out && j0 < nb) {
        uint8_t* row0 = p.mask_out + (static_cast<int64_t>(h) * nb + r0) * nb + j0;
        if (vec_mask) {
          if (has_r0) *reinterpret_cast<uint64_t*>(row0) = b0;
          if (has_r1) *reinterpret_cast<uint64_t*>(row0 + nb) = b1;
        } else {
          for (int c = 0; c < kMaskCols && j0 + c < nb; ++c) {
            if (has_r0) row0[c] = (m0 >> c) & 1;
            if (has_r1) row0[nb + c] = (m1 >> c) & 1;
          }
        }
      }
      const int sh = 16 * (tt & 3);
      const uint64_t cnt = static_cast<uint64_t>(__builtin_popcount(m0 | m1) * tiles_per_col);
#pragma unroll
      for (int i = 0; i < kMaskTilesPerWg / 4; ++i) {
        if (i == (tt >> 2)) {
          bits_w[i] |= static_cast<uint64_t>(m0 | (m1 << 8)) << sh;
          cnt_w[i] |= cnt << sh;
        }
      }
    }
    if (p.counts == nullptr) return;
    // inclusive scan of the packed counts (four 32-bit words) within the wave, then across
    // the four waves
    const int lane = tid & 63;
    const int wave = tid >> 6;
    constexpr int kWords = kMaskTilesPerWg / 2;
    int own[kWords], incl[kWords];
#pragma unroll
    for (int i = 0; i < kWords; ++i) {
      own[i] = static_cast<int>(cnt_w[i >> 1] >> (32 * (i & 1)));
      incl[i] = own[i];
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
#pragma unroll
      for (int i = 0; i < kWords; ++i) {
        const int v = __shfl_up(incl[i], o);
        if (lane >= o) incl[i] += v;
      }
    }
    if (lane == 63) {
#pragma unroll
      for (int i = 0; i < kWords; ++i) s_wpack[wave][i] = incl[i];
    }
    __syncthreads();
    int start[kWords], total[kWords];
#pragma unroll
    for (int i = 0; i < kWords; ++i) {
      int before = 0, all = 0;
      for (int w = 0; w < kMaskThreads / 64; ++w) {
        const int v = s_wpack[w][i];
        if (w < wave) before += v;
        all += v;
      }
      start[i] = before + incl[i] - own[i];
      total[i] = all;
    }
    const bool both = p.block == 128 || p.union_rows;
#pragma unroll 1
    for (int tt = 0; tt < t_end - t_begin; ++tt) {
      const int sh = 16 * (tt & 1);
      int st = 0, tl = 0;
#pragma unroll
      for (int i = 0; i < kWords; ++i)
        if (i == (tt >> 1)) {
          st = start[i];
          tl = total[i];
        }
      int pos = (st >> sh) & 0xffff;
      const int tot = (tl >> sh) & 0xffff;
      const int64_t slot = static_cast<int64_t>(h) * p.n_qtiles + t_begin + tt;
      int32_t* out = p.entries + slot * p.cap;
      uint64_t bw = 0;
#pragma unroll
      for (int i = 0; i < kMaskTilesPerWg / 4; ++i)
        if (i == (tt >> 2)) bw = bits_w[i];
      const unsigned rb = static_cast<unsigned>(bw >> (16 * (tt & 3))) & 0xffffu;
      const unsigned m0 = rb & 0xffu;
      const unsigned m1 = rb >> 8;
      unsigned rem = m0 | m1;
      while (rem != 0u) {
        const int c = __builtin_ctz(rem);
        rem &= rem - 1u;
        const int rbits = both ? 3 : static_cast<int>((m0 >> c) & 1u) | (static_cast<int>((m1 >> c) & 1u) << 1);
        for (int s2 = 0; s2 < tiles_per_col; ++s2) {
          if (pos < p.cap) out[pos] = ((((j0 + c) * tiles_per_col + s2)) << 2) | rbits;
          ++pos;
        }
      }
      if (tid == 0) p.counts[slot] = tot < p.cap ? tot : p.cap;
    }
    return;
  }

  for (int t = t_begin; t < t_end; ++t) {
    const int r0 = t * rows_per_tile;
    const int r1 = r0 + 1;
    const bool has_r0 = r0 < n_rows;
    const bool has_r1 = rows_per_tile == 2 && r1 < n_rows;
    const int iv0 = kFromMask ? 0 : video_index(r0);
    const int iv1 = kFromMask ? 0 : video_index(r1);
    const int if0 = iv0 >= 0 ? iv0 / p.bpf : -2;
    const int if1 = iv1 >= 0 ? iv1 / p.bpf : -2;
    const int64_t slot = static_cast<int64_t>(h) * p.n_qtiles + t;
    int32_t* out = p.counts ? p.entries + slot * p.cap : nullptr;
    int written = 0;
    for (int jb = 0; jb < nb; jb += kMaskThreads * kMaskCols) {
      const int j0 = jb + tid * kMaskCols;
      unsigned m0 = 0, m1 = 0;  // bit c: column j0 + c is active in row r0 / r1
      uint64_t b0 = 0, b1 = 0;  // byte c: the same as 0/1 (mask output)
      const bool fast = !kFromMask && jb == 0;
      if (fast) {
        b0 = row_bytes(has_r0, iv0, if0);
        b1 = row_bytes(has_r1, iv1, if1);
        m0 = byte_bits(b0);
        m1 = byte_bits(b1);
      }
#pragma unroll
      for (int c = 0; c < kMaskCols && !fast; ++c) {
        const int j = j0 + c;
        if (j >= nb) break;
        bool a0, a1;
        if (kFromMask) {
          const uint8_t* col = p.mask_in + h * p.in_head_stride + j;
          a0 = has_r0 && col[r0 * p.in_row_stride] != 0;
          a1 = has_r1 && col[r1 * p.in_row_stride] != 0;
        } else {
          // columns of later passes (nb > 2048)
          const int jv = video_index(j);
          const int jf = (bd && jv >= 0) ? jv / p.bpf : -3;
          const bool colj = jv >= 0 && colsel[jv];
          a0 = has_r0 && (iv0 < 0 || jv < 0 || full || colj || diagsel[jv - iv0 + n - 1] ||
                          (bd && if0 == jf));
          a1 = has_r1 && (iv1 < 0 || jv < 0 || full || colj || diagsel[jv - iv1 + n - 1] ||
                          (bd && if1 == jf));
        }
        m0 |= static_cast<unsigned>(a0) << c;
        m1 |= static_cast<unsigned>(a1) << c;
      }
      if (!kFromMask && p.mask_out && j0 < nb) {
        uint8_t* row0 = p.mask_out + (static_cast<int64_t>(h) * nb + r0) * nb + j0;
        if (!fast) {
#pragma unroll
          for (int c = 0; c < kMaskCols; ++c) {
            b0 |= static_cast<uint64_t>((m0 >> c) & 1u) << (8 * c);
            b1 |= static_cast<uint64_t>((m1 >> c) & 1u) << (8 * c);
          }
        }
        if (vec_mask) {
          if (has_r0) *reinterpret_cast<uint64_t*>(row0) = b0;
          if (has_r1) *reinterpret_cast<uint64_t*>(row0 + nb) = b1;
        } else {
          for (int c = 0; c < kMaskCols && j0 + c < nb; ++c) {
            if (has_r0) row0[c] = (m0 >> c) & 1;
            if (has_r1) row0[nb + c] = (m1 >> c) & 1;
          }
        }
      }
      if (out == nullptr) continue;
      // entries: ascending key tiles, counted then placed by an ordered block scan
      int cnt = 0;
      const unsigned any = m0 | m1;
#pragma unroll
      for (int c = 0; c < kMaskCols; ++c) {
        if ((any >> c) & 1) {
          for (int s2 = 0; s2 < tiles_per_col; ++s2)
            if ((j0 + c) * tiles_per_col + s2 < p.kv_tiles) ++cnt;
        }
      }
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
      int pos = written + s_wave[wave] + incl - cnt;
      const int total = s_total;
      __syncthreads();  // s_wave / s_total are rewritten by the next pass
#pragma unroll
      for (int c = 0; c < kMaskCols; ++c) {
        if (!((any >> c) & 1)) continue;
        int bits;
        if (p.block == 128 || p.union_rows) bits = 3;
        else bits = static_cast<int>((m0 >> c) & 1) | (static_cast<int>((m1 >> c) & 1) << 1);
        for (int s2 = 0; s2 < tiles_per_col; ++s2) {
          const int kt = (j0 + c) * tiles_per_col + s2;
          if (kt < p.kv_tiles) {
            if (pos < p.cap) out[pos] = (kt << 2) | bits;
            ++pos;
          }
        }
      }
      written += total;
    }
    if (out != nullptr && tid == 0) p.counts[slot] = written < p.cap ? written : p.cap;
  }
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

extern "C" int64_t moddit_mts_workspace_bytes(int heads, int n) {
  if (heads <= 0 || n <= 0) return 0;
  return static_cast<int64_t>(heads) * 3 * n * (sizeof(unsigned long long) + sizeof(float));
}

extern "C" int moddit_mts(const void* map, int map_dtype, int heads, int n, int blocks_per_frame,
                          void* workspace, float* mts_out, moddit_stream_t stream) {
  clear_error();
  MODDIT_CHECK_ARG(map && mts_out, "mts: null pointer argument");
  MODDIT_CHECK_ARG(map_dtype == MODDIT_FP16 || map_dtype == MODDIT_FP32,
                   "mts: map dtype must be fp16 or fp32");
  MODDIT_CHECK_ARG(heads >= 0 && n > 0, "mts: invalid shape heads=%d n=%d", heads, n);
  MODDIT_CHECK_ARG(blocks_per_frame > 0, "mts: blocks_per_frame must be positive, got %d",
                   blocks_per_frame);
  if (heads == 0) return MODDIT_OK;
  hipStream_t st = as_stream(stream);
  if (map_dtype == MODDIT_FP16) {
    MODDIT_CHECK_ARG(workspace != nullptr, "mts: fp16 maps need a workspace of "
                     "moddit_mts_workspace_bytes(heads, n) bytes");
    MODDIT_CHECK_ARG(aligned16(workspace), "mts: workspace must be 16-byte aligned");
    MODDIT_CHECK_ARG(n <= kMts1MaxN, "mts: n=%d exceeds %d", n, kMts1MaxN);
    MODDIT_CHECK_ARG(static_cast<int64_t>(n) * (blocks_per_frame < n ? blocks_per_frame : n) <=
                         kMts1MaxFrameCells,
                     "mts: n * min(blocks_per_frame, n) = %lld frame-block cells exceed %lld "
                     "(the exact fp16 sum's int64 range)",
                     static_cast<long long>(n) * (blocks_per_frame < n ? blocks_per_frame : n),
                     static_cast<long long>(kMts1MaxFrameCells));
    Mts1Params q;
    q.map = static_cast<const uint16_t*>(map);
    q.heads = heads;
    q.n = n;
    q.bpf = blocks_per_frame;
    q.n_rt = (n + kMts1TileR - 1) / kMts1TileR;
    q.n_ct = (n + kMts1TileC - 1) / kMts1TileC;
    const int64_t total = static_cast<int64_t>(heads) * 3 * n;
    q.acc = static_cast<unsigned long long*>(workspace);
    q.special = reinterpret_cast<float*>(q.acc + total);
    q.out = mts_out;
    const int64_t grid = static_cast<int64_t>(heads) * q.n_rt * q.n_ct;
    MODDIT_CHECK_ARG(grid < 0x7fffffff, "mts: shape too large");
    int64_t fill = (total + 255) / 256;
    if (fill > 4096) fill = 4096;
    hipLaunchKernelGGL(mts1_zero_kernel, dim3(static_cast<unsigned>(fill)), dim3(256), 0, st, q);
    MODDIT_CHECK_LAUNCH("mts (zero)");
    const bool vec = n % 8 == 0 && aligned16(map);
    auto kernel = vec ? mts1_kernel<true> : mts1_kernel<false>;
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(kMts1Threads), 0, st, q);
    MODDIT_CHECK_LAUNCH("mts");
    hipLaunchKernelGGL(mts1_finalize_kernel, dim3(static_cast<unsigned>(fill)), dim3(256), 0, st, q);
    MODDIT_CHECK_LAUNCH("mts (finalize)");
    return MODDIT_OK;
  }
  MtsParams p;
  p.map = static_cast<const float*>(map);
  p.heads = heads;
  p.n = n;
  p.bpf = blocks_per_frame;
  p.n_bands = (2 * n - 1 + 63) / 64;
  p.n_strips = (n + 63) / 64;
  p.out = mts_out;
  const int64_t grid = static_cast<int64_t>(heads) * (p.n_bands + p.n_strips + 1);
  MODDIT_CHECK_ARG(grid < 0x7fffffff, "mts: shape too large");
  hipLaunchKernelGGL(mts_kernel, dim3(static_cast<unsigned>(grid)), dim3(kMtsThreads), 0, st, p);
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
  const size_t lds = static_cast<size_t>(mask_lds_bytes(n));
  MODDIT_CHECK_ARG(lds <= 65536, "mask_from_lines: n=%d too large", n);
  const int64_t grid = static_cast<int64_t>(heads) * ((n_qtiles + kMaskTilesPerWg - 1) / kMaskTilesPerWg);
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
  const int64_t grid = static_cast<int64_t>(heads) * ((n_qtiles + kMaskTilesPerWg - 1) / kMaskTilesPerWg);
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
