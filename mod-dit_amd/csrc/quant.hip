// Quantisation pre-pass of the int8/fp8 attention path (SageAttention2-style numerics:
// int8 Q.K^T with per-block scales and a smoothed K, fp8 e4m3 P.V with a per-channel V
// scale), for gfx950.
//
// Blocks and tiles lie on the attention kernel's grid, which starts at token
// `grid_origin` (-63..0; negative for a text-first CogVideoX layout): tile t holds tokens
// grid_origin + 64t .. +63, tokens outside [0, S) count as zero.
//   q8[bh][s][d]   = rne(q * 127/amax_q(block)),  block = 32 grid rows
//   k8[bh][s][d]   = rne((k - mean_k[d]) * 127/amax(tile)), tile = 64 grid keys
//   v8t[bh][d][c]  = e4m3_rne(v[grid_origin + c] * 448/amax_v[d])  (transposed: keys
//                    contiguous, column c = grid position, so every 64-key tile is a
//                    64-byte aligned run; zero outside the sequence)
//   q_scale = amax_q/127, k_scale = amax_k/127, v_scale = amax_v/448 (1 where amax is 0)
//   q_kmean[bh][s] = q . mean_k (fp32)
//
// Subtracting the per-channel mean of K over the sequence shifts every score of a row by
// the same amount (q . mean_k), which softmax ignores, and removes the channel offsets
// that would otherwise dominate the int8 range; the attention kernels add
// scale * q_kmean back to the log-sum-exp so that it is the LSE of the unsmoothed scores.
// Reference: the quantised engine the reference runs, block_sparse_sage2_attn_cuda
// (MoD/mod/attn_mask.py:306), and SageAttention2's published scheme; the exact kernel is a
// third-party dependency absent from the reference tree.
#include "common.h"

namespace moddit {
namespace {

constexpr int kQThreads = 256;
constexpr int kStatChunks = 64;  // row ranges per (b, h) with partial column statistics

struct StatParams {
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int heads;
  int seq_len;
  float* part;  // [bh][chunk][2][D]: sum of k, max |v|
  float* vinv;  // [bh][D]: 448 / max |v| (1 where the max is 0)
  float* k_mean;
  float* v_scale;
};

// Grid (B*H, kStatChunks): chunk c covers rows [c*S/kStatChunks, (c+1)*S/kStatChunks);
// each thread reads 16 bytes of a row (D/8 threads per row, kQThreads*8/D rows in flight),
// the row lanes are then combined in LDS in a fixed order, so the statistics are
// deterministic.
template <int D, typename E>
__global__ __launch_bounds__(kQThreads) void qkv_stats_kernel(StatParams p) {
  constexpr int kColThreads = D / 8;
  constexpr int kRowLanes = kQThreads / kColThreads;
  constexpr int kUnroll = 4;
  __shared__ float red[2][kRowLanes][D];
  const int bh = blockIdx.x;
  const int chunk = blockIdx.y;
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;
  const uint16_t* kb = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* vb = p.v + b * p.v_sb + h * p.v_sh;
  const int ct = threadIdx.x % kColThreads;
  const int rl = threadIdx.x / kColThreads;
  const int d0 = ct * 8;
  const int r_begin = static_cast<int>(static_cast<int64_t>(p.seq_len) * chunk / kStatChunks);
  const int r_end = static_cast<int>(static_cast<int64_t>(p.seq_len) * (chunk + 1) / kStatChunks);
  float ks[8], vm[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    ks[j] = 0.f;
    vm[j] = 0.f;
  }
  int s = r_begin + rl;
  for (; s + (kUnroll - 1) * kRowLanes < r_end; s += kUnroll * kRowLanes) {
    u32x4 kw[kUnroll], vw[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      kw[u] = *reinterpret_cast<const u32x4*>(kb + (s + u * kRowLanes) * p.k_ss + d0);
      vw[u] = *reinterpret_cast<const u32x4*>(vb + (s + u * kRowLanes) * p.v_ss + d0);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ks[j] += E::to_float(u16_at(kw[u], j));
        vm[j] = fmaxf(vm[j], fabsf(E::to_float(u16_at(vw[u], j))));
      }
  }
  for (; s < r_end; s += kRowLanes) {
    const u32x4 kw = *reinterpret_cast<const u32x4*>(kb + s * p.k_ss + d0);
    const u32x4 vw = *reinterpret_cast<const u32x4*>(vb + s * p.v_ss + d0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ks[j] += E::to_float(u16_at(kw, j));
      vm[j] = fmaxf(vm[j], fabsf(E::to_float(u16_at(vw, j))));
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    red[0][rl][d0 + j] = ks[j];
    red[1][rl][d0 + j] = vm[j];
  }
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += kQThreads) {
    float sum = 0.f, mx = 0.f;
    for (int r = 0; r < kRowLanes; ++r) {
      sum += red[0][r][d];
      mx = fmaxf(mx, red[1][r][d]);
    }
    float* out = p.part + (static_cast<int64_t>(bh) * kStatChunks + chunk) * 2 * D;
    out[d] = sum;
    out[D + d] = mx;
  }
}

// Grid (B*H): the chunks' partial statistics in a fixed order -> k_mean, v_scale, vinv.
template <int D>
__global__ __launch_bounds__(kQThreads) void qkv_stats_finalize_kernel(StatParams p) {
  const int bh = blockIdx.x;
  const float* part = p.part + static_cast<int64_t>(bh) * kStatChunks * 2 * D;
  for (int d = threadIdx.x; d < D; d += kQThreads) {
    float sum = 0.f, mx = 0.f;
    for (int c = 0; c < kStatChunks; ++c) {
      sum += part[c * 2 * D + d];
      mx = fmaxf(mx, part[c * 2 * D + D + d]);
    }
    const int64_t o = static_cast<int64_t>(bh) * D + d;
    p.k_mean[o] = sum / static_cast<float>(p.seq_len);
    p.v_scale[o] = mx > 0.f ? mx / 448.f : 1.f;
    p.vinv[o] = mx > 0.f ? 448.f / mx : 1.f;
  }
}

struct QuantParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int heads;
  int seq_len;
  int origin;  // first token of the grid (-63..0)
  int s_pad;   // v8t row length: grid tiles * 64
  const float* vinv;     // [bh][D]
  const float* k_mean_in;  // [bh][D]
  int8_t* q8;
  float* q_scale;  // [bh][ceil((S - origin)/32)]
  int8_t* k8;
  float* k_scale;  // [bh][ceil((S - origin)/64)]
  uint8_t* v8t;
  float* q_kmean;  // [bh][S]
};

__device__ __forceinline__ int8_t to_i8(float x) {
  const float r = __builtin_rintf(x);  // round half to even
  return static_cast<int8_t>(fminf(fmaxf(r, -127.f), 127.f));
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

// Grid (B*H, grid tiles): one 64-row tile of Q, K and V per workgroup.
template <int D, typename E>
__global__ __launch_bounds__(kQThreads) void quantize_kernel(QuantParams p) {
  constexpr int kChunks = D / 8;                       // 16-byte input chunks per row
  constexpr int kPerThread = 64 * kChunks / kQThreads;  // chunks per thread
  __shared__ float mean[D];
  __shared__ float vinv[D];
  __shared__ float wmax[4][3];  // per wave: Q block 0, Q block 1, K tile
  const int bh = blockIdx.x;
  const int tile = blockIdx.y;
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;

  for (int d = tid; d < D; d += kQThreads) {
    mean[d] = p.k_mean_in[static_cast<int64_t>(bh) * D + d];
    vinv[d] = p.vinv[static_cast<int64_t>(bh) * D + d];
  }
  __syncthreads();

  const uint16_t* qb = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* kb = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* vb = p.v + b * p.v_sb + h * p.v_sh;
  const int row0 = p.origin + tile * 64;  // token of the tile's first row

  // V for the transposed fp8 tile (written last) is loaded first, so that its reads
  // overlap the Q/K work: thread (g, c) = (tid % 16, tid / 16) takes keys 4g..4g+3 of the
  // tile at channels 8c..8c+7 (tokens outside the sequence load as zero)
  static_assert(16 * kChunks <= kQThreads, "one V group per thread");
  const int vg = tid % 16;
  const int vc = tid / 16;
  const bool v_thread = vc < kChunks;
  u32x4 vraw[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int s = row0 + 4 * vg + t;
    vraw[t] = u32x4{0u, 0u, 0u, 0u};
    if (v_thread && s >= 0 && s < p.seq_len)
      vraw[t] = *reinterpret_cast<const u32x4*>(vb + s * p.v_ss + vc * 8);
  }
  // thread chunk i covers row i*kQThreads/kChunks + tid/kChunks, 16-byte chunk tid%kChunks:
  // the kChunks threads of a row are consecutive lanes of one wave
  float qv[kPerThread][8], kv[kPerThread][8];
  float qmax0 = 0.f, qmax1 = 0.f, kmax = 0.f;
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int idx = i * kQThreads + tid;
    const int r = idx / kChunks;
    const int c = idx % kChunks;
    const int s = row0 + r;
    const bool ok = s >= 0 && s < p.seq_len;
    u32x4 qw = {0u, 0u, 0u, 0u}, kw = {0u, 0u, 0u, 0u};
    if (ok) {
      qw = *reinterpret_cast<const u32x4*>(qb + s * p.q_ss + c * 8);
      kw = *reinterpret_cast<const u32x4*>(kb + s * p.k_ss + c * 8);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      qv[i][j] = ok ? E::to_float(u16_at(qw, j)) : 0.f;
      kv[i][j] = ok ? E::to_float(u16_at(kw, j)) - mean[c * 8 + j] : 0.f;
      if (r < 32)
        qmax0 = fmaxf(qmax0, fabsf(qv[i][j]));
      else
        qmax1 = fmaxf(qmax1, fabsf(qv[i][j]));
      kmax = fmaxf(kmax, fabsf(kv[i][j]));
    }
  }
  qmax0 = wave_max(qmax0);
  qmax1 = wave_max(qmax1);
  kmax = wave_max(kmax);
  if (lane == 0) {
    wmax[wave][0] = qmax0;
    wmax[wave][1] = qmax1;
    wmax[wave][2] = kmax;
  }
  __syncthreads();
  float am[3];
#pragma unroll
  for (int t = 0; t < 3; ++t)
    am[t] = fmaxf(fmaxf(wmax[0][t], wmax[1][t]), fmaxf(wmax[2][t], wmax[3][t]));
  const float qinv0 = am[0] > 0.f ? 127.f / am[0] : 1.f;
  const float qinv1 = am[1] > 0.f ? 127.f / am[1] : 1.f;
  const float kinv = am[2] > 0.f ? 127.f / am[2] : 1.f;
  if (tid == 0) {
    const int nqb = (p.seq_len - p.origin + 31) / 32;
    float* qs = p.q_scale + static_cast<int64_t>(bh) * nqb;
    qs[2 * tile] = am[0] > 0.f ? am[0] / 127.f : 1.f;
    if (2 * tile + 1 < nqb) qs[2 * tile + 1] = am[1] > 0.f ? am[1] / 127.f : 1.f;
    p.k_scale[static_cast<int64_t>(bh) * gridDim.y + tile] = am[2] > 0.f ? am[2] / 127.f : 1.f;
  }
  int8_t* q8 = p.q8 + (static_cast<int64_t>(bh) * p.seq_len) * D;
  int8_t* k8 = p.k8 + (static_cast<int64_t>(bh) * p.seq_len) * D;
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int idx = i * kQThreads + tid;
    const int r = idx / kChunks;
    const int c = idx % kChunks;
    const int s = row0 + r;
    // q . mean_k: 8 products per chunk, then the row's chunks in a fixed butterfly
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) dot = __builtin_fmaf(qv[i][j], mean[c * 8 + j], dot);
#pragma unroll
    for (int o = kChunks / 2; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
    if (s >= 0 && s < p.seq_len) {
      if (c == 0) p.q_kmean[static_cast<int64_t>(bh) * p.seq_len + s] = dot;
      const float qi = r < 32 ? qinv0 : qinv1;
      uint32_t qw[2], kw[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        qw[j] = 0u;
        kw[j] = 0u;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          qw[j] |= static_cast<uint32_t>(static_cast<uint8_t>(to_i8(qv[i][4 * j + t] * qi))) << (8 * t);
          kw[j] |= static_cast<uint32_t>(static_cast<uint8_t>(to_i8(kv[i][4 * j + t] * kinv))) << (8 * t);
        }
      }
      *reinterpret_cast<u32x2*>(q8 + static_cast<int64_t>(s) * D + c * 8) = u32x2{qw[0], qw[1]};
      *reinterpret_cast<u32x2*>(k8 + static_cast<int64_t>(s) * D + c * 8) = u32x2{kw[0], kw[1]};
    }
  }
  // Transposed fp8 V tile, row d, 64 grid columns (zeros outside the sequence), without
  // LDS: thread (g, c) packs the four keys of each of its channels into one word (e4m3,
  // round to nearest even). Consecutive threads take consecutive key groups, so the 16
  // words of a channel row are 64 contiguous bytes.
  if (v_thread) {
    uint8_t* vrow = p.v8t + (static_cast<int64_t>(bh) * D) * p.s_pad + tile * 64;
    float vf[4][8];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int s = row0 + 4 * vg + t;
      const bool ok = s >= 0 && s < p.seq_len;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        vf[t][j] = ok ? E::to_float(u16_at(vraw[t], j)) * vinv[vc * 8 + j] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int w = __builtin_amdgcn_cvt_pk_fp8_f32(vf[0][j], vf[1][j], 0, false);
      w = __builtin_amdgcn_cvt_pk_fp8_f32(vf[2][j], vf[3][j], w, true);
      *reinterpret_cast<uint32_t*>(vrow + static_cast<int64_t>(vc * 8 + j) * p.s_pad + 4 * vg) =
          static_cast<uint32_t>(w);
    }
  }
}

template <int D, typename E>
int launch_quant(const StatParams& sp, const QuantParams& qp, int bhs, hipStream_t st) {
  hipLaunchKernelGGL((qkv_stats_kernel<D, E>), dim3(bhs, kStatChunks), dim3(kQThreads), 0, st, sp);
  MODDIT_CHECK_LAUNCH("quantize_qkv (statistics)");
  hipLaunchKernelGGL((qkv_stats_finalize_kernel<D>), dim3(bhs), dim3(kQThreads), 0, st, sp);
  MODDIT_CHECK_LAUNCH("quantize_qkv (statistics, final)");
  hipLaunchKernelGGL((quantize_kernel<D, E>), dim3(bhs, qp.s_pad / 64), dim3(kQThreads), 0, st,
                     qp);
  MODDIT_CHECK_LAUNCH("quantize_qkv");
  return MODDIT_OK;
}

}  // namespace
}  // namespace moddit

extern "C" int moddit_quantize_qkv(const void* q, const void* k, const void* v, int batch,
                                   int heads, int seq_len, int head_dim,
                                   const int64_t q_strides[3], const int64_t k_strides[3],
                                   const int64_t v_strides[3], int dtype, int grid_origin,
                                   float* workspace, int8_t* q8, float* q_scale, int8_t* k8,
                                   float* k_scale, uint8_t* v8t, float* v_scale, float* k_mean,
                                   float* q_kmean, moddit_stream_t stream) {
  using namespace moddit;
  clear_error();
  MODDIT_CHECK_ARG(q && k && v && q_strides && k_strides && v_strides,
                   "quantize_qkv: null input");
  MODDIT_CHECK_ARG(workspace && q8 && q_scale && k8 && k_scale && v8t && v_scale && k_mean &&
                       q_kmean,
                   "quantize_qkv: null output or workspace");
  if (head_dim != 64 && head_dim != 128) {
    set_error("quantize_qkv: head_dim must be 64 or 128, got %d", head_dim);
    return MODDIT_EUNSUPPORTED;
  }
  if (dtype != MODDIT_BF16 && dtype != MODDIT_FP16) {
    set_error("quantize_qkv: dtype must be bf16 or fp16");
    return MODDIT_EUNSUPPORTED;
  }
  MODDIT_CHECK_ARG(batch >= 0 && heads >= 0 && seq_len >= 0, "quantize_qkv: negative size");
  if (grid_origin > 0 || grid_origin <= -64) {
    set_error("quantize_qkv: grid_origin must lie in (-64, 0], got %d", grid_origin);
    return MODDIT_EINVAL;
  }
  MODDIT_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(q8) &&
                       aligned16(k8) && aligned16(v8t),
                   "quantize_qkv: tensors must be 16-byte aligned");
  const int64_t* all[3] = {q_strides, k_strides, v_strides};
  for (int t = 0; t < 3; ++t)
    for (int j = 0; j < 3; ++j)
      MODDIT_CHECK_ARG(all[t][j] >= 0 && all[t][j] % 8 == 0,
                       "quantize_qkv: strides must be non-negative multiples of 8 elements");
  if (batch == 0 || heads == 0 || seq_len == 0) return MODDIT_OK;
  StatParams sp;
  sp.k = static_cast<const uint16_t*>(k);
  sp.v = static_cast<const uint16_t*>(v);
  sp.k_sb = k_strides[0]; sp.k_sh = k_strides[1]; sp.k_ss = k_strides[2];
  sp.v_sb = v_strides[0]; sp.v_sh = v_strides[1]; sp.v_ss = v_strides[2];
  sp.heads = heads;
  sp.seq_len = seq_len;
  sp.part = workspace;
  sp.vinv = workspace + static_cast<int64_t>(batch) * heads * kStatChunks * 2 * head_dim;
  sp.k_mean = k_mean;
  sp.v_scale = v_scale;
  QuantParams qp;
  qp.q = static_cast<const uint16_t*>(q);
  qp.k = sp.k;
  qp.v = sp.v;
  qp.q_sb = q_strides[0]; qp.q_sh = q_strides[1]; qp.q_ss = q_strides[2];
  qp.k_sb = sp.k_sb; qp.k_sh = sp.k_sh; qp.k_ss = sp.k_ss;
  qp.v_sb = sp.v_sb; qp.v_sh = sp.v_sh; qp.v_ss = sp.v_ss;
  qp.heads = heads;
  qp.seq_len = seq_len;
  qp.origin = grid_origin;
  qp.s_pad = (seq_len - grid_origin + 63) / 64 * 64;
  qp.vinv = sp.vinv;
  qp.k_mean_in = k_mean;
  qp.q8 = q8;
  qp.q_scale = q_scale;
  qp.k8 = k8;
  qp.k_scale = k_scale;
  qp.v8t = v8t;
  qp.q_kmean = q_kmean;
  const int bhs = batch * heads;
  hipStream_t st = as_stream(stream);
  const bool bf = dtype == MODDIT_BF16;
  if (head_dim == 128)
    return bf ? launch_quant<128, Bf16>(sp, qp, bhs, st) : launch_quant<128, Fp16>(sp, qp, bhs, st);
  return bf ? launch_quant<64, Bf16>(sp, qp, bhs, st) : launch_quant<64, Fp16>(sp, qp, bhs, st);
}

extern "C" int moddit_quantize_workspace_floats(int batch, int heads, int head_dim) {
  return batch * heads * (moddit::kStatChunks * 2 + 1) * head_dim;
}
