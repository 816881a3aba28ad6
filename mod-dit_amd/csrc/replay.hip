// Replayed block sparsity map for gfx950.
//
// For each (batch*head, 128-row query tile of the video region) one workgroup of four
// wave64s sweeps every 64-key tile of the video region:
//   S^T (64 keys x 32 queries) = K . round(Q*scale)^T    bf16/fp16 MFMA 32x32x16, fp32
// and counts the scores strictly below lse[row] + log_threshold. Each comparison is a
// wave-wide ballot whose popcount lands in a scalar register, so the count per
// (wave, key tile) needs no vector reduction. Counts are staged in LDS and combined
// into (query block, key block) cells of 64x64 or 128x128 tokens, then written as
// fp16(count / block_size^2).
//
// Reference semantics: flash_sparsity_replay_kernel
// (MoD/mod/cuda_flash_sparsity_kernel.cu:41-169): Q scaled in fp32 and rounded to the
// input dtype (:86-92), fp32 products, strict '<' against lse + log_threshold (:138-143),
// __float2half_rn of count / block_size^2 (:158-163). The last video block may run past
// the sequence end; rows and keys at or beyond seq_len are then not counted.
#include "common.h"

namespace moddit {
namespace {

constexpr int kBM = 128;
constexpr int kBN = 64;
constexpr int kThreads = 256;
constexpr int kFlush = 64;  // key tiles per flush; the LDS count ring holds two flushes

template <int D>
struct ReplayLds {
  static constexpr int kPitchK = D * 2 + 16;
  static constexpr int kKBytes = kBN * kPitchK;
  static constexpr int kCounts = 4 * 2 * kFlush * 4;  // int per (wave, ring slot)
  static constexpr int kTotal = 2 * kKBytes + kCounts;
};

struct ReplayParams {
  const uint16_t* q;
  const uint16_t* k;
  const float* lse;
  uint16_t* out;  // fp16 (B*H, nblk, nblk)
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int heads;
  int seq_len;
  int q_off;
  int k_off;
  int nblk;      // video blocks per side
  int block;     // 64 or 128
  int valid_q;   // video rows that exist: min(nblk*block, seq_len - q_off)
  int valid_k;   // video keys that exist: min(nblk*block, seq_len - k_off)
  int n_qtiles;  // 128-row tiles of the video region
  int n_ktiles;  // 64-key tiles of the video region
  int xcd_run;   // workgroup -> tile order (xcd_remap)
  float scale;
  float log_thr;
  uint32_t k_bytes;  // byte span of one head's video K rows
};

template <int D, typename E, bool kRagged>
__global__ __launch_bounds__(kThreads, 2) void replay_map_kernel(ReplayParams p) {
  using L = ReplayLds<D>;
  using V8 = typename E::vec8;
  constexpr int kDChunks = D / 16;
  constexpr int kVecPerRow = D / 8;
  constexpr int kKVecs = kBN * kVecPerRow / kThreads;

  extern __shared__ __align__(16) unsigned char smem[];
  int* cnt = reinterpret_cast<int*>(smem + 2 * L::kKBytes);

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int half = lane >> 5;
  const int c32 = lane & 31;

  const int tile = xcd_remap(blockIdx.x, gridDim.x, p.xcd_run);
  const int qt = tile % p.n_qtiles;
  const int bh = tile / p.n_qtiles;
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;

  const uint16_t* qb = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* kb = p.k + b * p.k_sb + h * p.k_sh;

  // Rows of this wave inside the video region: video rows are [0, nblk*block).
  const int video_rows = p.nblk * p.block;
  const int vrow0 = qt * kBM + wave * 32;
  const bool wave_active = vrow0 < video_rows;  // blocks are multiples of 32 rows
  const int vrow = vrow0 + c32;

  V8 qf[kDChunks];
  float thr = -INFINITY;
  {
    const bool row_ok = wave_active && vrow < p.valid_q;
    const int r = p.q_off + (row_ok ? vrow : 0);
    const u32x4* src = reinterpret_cast<const u32x4*>(qb + r * p.q_ss);
#pragma unroll
    for (int c = 0; c < kDChunks; ++c) {
      const u32x4 raw = src[2 * c + half];
      uint16_t e[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) e[j] = E::from_float(E::to_float(u16_at(raw, j)) * p.scale);
      const u32x4 packed = {pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]),
                            pack2(e[6], e[7])};
      qf[c] = as_vec8<V8>(packed);
    }
    // rows past the sequence end count nothing (no score is below -inf)
    thr = row_ok ? p.lse[static_cast<int64_t>(bh) * p.seq_len + r] + p.log_thr : -INFINITY;
    // Retire these loads before the loop (see attention.hip).
    __builtin_amdgcn_s_waitcnt(0);
  }

  // K rows of the video region through a buffer resource (loop-invariant VGPR offsets,
  // tile offset in the SGPR offset when every tile is a full in-range tile; otherwise in
  // the range-checked VGPR offset, so rows past the last key load zeros).
  const int k_col = tid % kVecPerRow;
  const int k_row0 = tid / kVecPerRow;
  constexpr int kKRowStep = kThreads / kVecPerRow;
  const uint16_t* kvid = kb + static_cast<int64_t>(p.k_off) * p.k_ss;
  const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(kvid, p.k_bytes);
  const uint32_t k_voff = static_cast<uint32_t>((k_row0 * p.k_ss + k_col * 8) * 2);
  const uint32_t k_row_step = static_cast<uint32_t>(kKRowStep * p.k_ss * 2);
  const uint32_t k_tile_bytes = static_cast<uint32_t>(kBN * p.k_ss * 2);
  u32x4 kreg[kKVecs];
  auto load_tile = [&](int kt) {
    const uint32_t so = static_cast<uint32_t>(kt) * k_tile_bytes;
#pragma unroll
    for (int i = 0; i < kKVecs; ++i) {
      if constexpr (kRagged)
        kreg[i] = buf_load16(k_rsrc, k_voff + so + i * k_row_step, 0);
      else
        kreg[i] = buf_load16(k_rsrc, k_voff, so + i * k_row_step);
    }
  };
  auto store_tile = [&](int stage) {
    unsigned char* ks = smem + stage * L::kKBytes;
#pragma unroll
    for (int i = 0; i < kKVecs; ++i)
      *reinterpret_cast<u32x4*>(ks + (k_row0 + i * kKRowStep) * L::kPitchK + k_col * 16) = kreg[i];
  };

  load_tile(0);
  store_tile(0);
  __syncthreads();

  const float inv_area = 1.0f / static_cast<float>(p.block * p.block);
  uint16_t* out_bh = p.out + static_cast<int64_t>(bh) * p.nblk * p.nblk;

  for (int it = 0; it < p.n_ktiles; ++it) {
    const bool has_next = it + 1 < p.n_ktiles;
    if (has_next) load_tile(it + 1);

    if (wave_active) {
      const unsigned char* ks = smem + (it & 1) * L::kKBytes;
      f32x16 s0 = f32x16{};
      f32x16 s1 = f32x16{};
#pragma unroll
      for (int c = 0; c < kDChunks; ++c) {
        const V8 a0 = *reinterpret_cast<const V8*>(ks + c32 * L::kPitchK + c * 32 + half * 16);
        const V8 a1 =
            *reinterpret_cast<const V8*>(ks + (32 + c32) * L::kPitchK + c * 32 + half * 16);
        s0 = E::mma(a0, qf[c], s0);
        s1 = E::mma(a1, qf[c], s1);
      }
      int total = 0;
      if (kRagged && it * kBN + kBN > p.valid_k) {
        // keys at or past the sequence end are not counted
        const int key0 = it * kBN + 4 * half;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kr = key0 + 8 * (i >> 2) + (i & 3);
          total += __builtin_popcountll(__ballot(s0[i] < thr && kr < p.valid_k));
          total += __builtin_popcountll(__ballot(s1[i] < thr && kr + 32 < p.valid_k));
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          total += __builtin_popcountll(__ballot(s0[i] < thr));
          total += __builtin_popcountll(__ballot(s1[i] < thr));
        }
      }
      // two halves of kFlush slots: a flush reads one half while the next kFlush key
      // tiles (at least one barrier later) write the other
      if (lane == 0) cnt[wave * 2 * kFlush + (it % (2 * kFlush))] = total;
    }

    if (has_next) store_tile((it + 1) & 1);
    __syncthreads();

    const int slot_hi = it % kFlush;
    if (slot_hi == kFlush - 1 || !has_next) {
      const int it0 = it - slot_hi;  // first key tile of this flush
      const int hb = ((it / kFlush) & 1) * kFlush;  // ring half it was written to
      if (p.block == 64) {
        // two 64-row query blocks per tile; one key block per key tile
        if (tid < 2 * kFlush) {
          const int qsub = tid / kFlush;
          const int s = tid % kFlush;
          const int qblk = 2 * qt + qsub;
          if (s <= slot_hi && qblk < p.nblk) {
            const int c = cnt[(2 * qsub) * 2 * kFlush + hb + s] + cnt[(2 * qsub + 1) * 2 * kFlush + hb + s];
            const float ratio = static_cast<float>(c) * inv_area;
            out_bh[static_cast<int64_t>(qblk) * p.nblk + it0 + s] = Fp16::from_float(ratio);
          }
        }
      } else {
        // one 128-row query block per tile; two key tiles per key block
        if (tid < kFlush / 2) {
          const int s = tid;
          if (2 * s + 1 <= slot_hi) {
            int c = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w)
              c += cnt[w * 2 * kFlush + hb + 2 * s] + cnt[w * 2 * kFlush + hb + 2 * s + 1];
            const float ratio = static_cast<float>(c) * inv_area;
            out_bh[static_cast<int64_t>(qt) * p.nblk + it0 / 2 + s] = Fp16::from_float(ratio);
          }
        }
      }
    }
  }
}

template <int D, typename E, bool kRagged>
int launch_replay_impl(const ReplayParams& p, int batch, hipStream_t stream) {
  using L = ReplayLds<D>;
  auto kernel = replay_map_kernel<D, E, kRagged>;
  static LaunchSetup once;
  if (set_dynamic_lds_once(once, reinterpret_cast<const void*>(kernel), L::kTotal) != hipSuccess) {
    set_error("sparsity_map: cannot reserve %d bytes of LDS", L::kTotal);
    return MODDIT_EHIP;
  }
  const int64_t tiles = static_cast<int64_t>(batch) * p.heads * p.n_qtiles;
  if (tiles == 0) return MODDIT_OK;
  if (tiles > 0x7fffffff) {
    set_error("sparsity_map: too many tiles (%lld)", static_cast<long long>(tiles));
    return MODDIT_EINVAL;
  }
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), L::kTotal,
                     stream, p);
  MODDIT_CHECK_LAUNCH("sparsity_map");
  return MODDIT_OK;
}

template <int D, typename E>
int launch_replay(const ReplayParams& p, int batch, hipStream_t stream) {
  if (p.valid_k == p.n_ktiles * kBN) return launch_replay_impl<D, E, false>(p, batch, stream);
  return launch_replay_impl<D, E, true>(p, batch, stream);
}

}  // namespace
}  // namespace moddit

extern "C" int moddit_sparsity_map(const void* q, const void* k, const float* lse, void* map_out,
                                   int batch, int heads, int seq_len, int head_dim,
                                   const int64_t q_strides[3], const int64_t k_strides[3],
                                   float softmax_scale, float log_threshold, int q_video_offset,
                                   int k_video_offset, int video_blocks, int block_size,
                                   int dtype, moddit_stream_t stream) {
  using namespace moddit;
  clear_error();
  MODDIT_CHECK_ARG(q && k && lse && map_out && q_strides && k_strides,
                   "sparsity_map: null pointer argument");
  if (head_dim != 64 && head_dim != 128) {
    set_error("sparsity_map: head_dim must be 64 or 128, got %d", head_dim);
    return MODDIT_EUNSUPPORTED;
  }
  if (dtype != MODDIT_BF16 && dtype != MODDIT_FP16) {
    set_error("sparsity_map: dtype must be bf16 or fp16");
    return MODDIT_EUNSUPPORTED;
  }
  MODDIT_CHECK_ARG(block_size == 64 || block_size == 128, "sparsity_map: block_size must be 64 or 128, got %d", block_size);
  MODDIT_CHECK_ARG(video_blocks > 0, "sparsity_map: video_blocks must be positive");
  MODDIT_CHECK_ARG(q_video_offset >= 0 && k_video_offset >= 0,
                   "sparsity_map: video offsets must be non-negative");
  const int64_t vt = static_cast<int64_t>(video_blocks) * block_size;
  // the last block may be partial, but must hold at least one token
  MODDIT_CHECK_ARG(q_video_offset + vt - block_size < seq_len,
                   "sparsity_map: Q video region exceeds sequence length");
  MODDIT_CHECK_ARG(k_video_offset + vt - block_size < seq_len,
                   "sparsity_map: K video region exceeds sequence length");
  MODDIT_CHECK_ARG(batch >= 0 && heads >= 0, "sparsity_map: negative size");
  MODDIT_CHECK_ARG(aligned16(q) && aligned16(k), "sparsity_map: q/k must be 16-byte aligned");
  for (int j = 0; j < 3; ++j)
    MODDIT_CHECK_ARG(q_strides[j] >= 0 && q_strides[j] % 8 == 0 && k_strides[j] >= 0 &&
                         k_strides[j] % 8 == 0,
                     "sparsity_map: strides must be non-negative multiples of 8 elements");
  MODDIT_CHECK_ARG(!std::isnan(log_threshold) && !std::isnan(softmax_scale),
                   "sparsity_map: NaN scale or threshold");

  ReplayParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.lse = lse;
  p.out = static_cast<uint16_t*>(map_out);
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.heads = heads;
  p.seq_len = seq_len;
  p.q_off = q_video_offset;
  p.k_off = k_video_offset;
  p.nblk = video_blocks;
  p.block = block_size;
  p.valid_q = static_cast<int>(vt < seq_len - q_video_offset ? vt : seq_len - q_video_offset);
  p.valid_k = static_cast<int>(vt < seq_len - k_video_offset ? vt : seq_len - k_video_offset);
  p.n_qtiles = static_cast<int>((vt + kBM - 1) / kBM);
  p.n_ktiles = static_cast<int>(vt / kBN);
  p.xcd_run = xcd_run_for(vt * head_dim * 2);  // the video K rows a sweep reads
  p.scale = softmax_scale;
  p.log_thr = log_threshold;
  const int64_t k_span = (static_cast<int64_t>(p.valid_k) - 1) * k_strides[2] * 2 + head_dim * 2;
  const int64_t k_grid = vt * k_strides[2] * 2;  // largest offset a (ragged) tile forms
  if (k_span > 0x7fffffffLL || k_grid > 0x7fffffffLL) {
    set_error("sparsity_map: one head's K span exceeds 2 GiB of 32-bit offsets");
    return MODDIT_EUNSUPPORTED;
  }
  p.k_bytes = static_cast<uint32_t>(k_span);

  hipStream_t st = as_stream(stream);
  const bool bf = dtype == MODDIT_BF16;
  if (head_dim == 128)
    return bf ? launch_replay<128, Bf16>(p, batch, st) : launch_replay<128, Fp16>(p, batch, st);
  return bf ? launch_replay<64, Bf16>(p, batch, st) : launch_replay<64, Fp16>(p, batch, st);
}
