// Replayed block sparsity map for gfx950.
//
// For each (batch*head, 128-row query tile of the video region) one workgroup of four
// wave64s sweeps every 64-key tile of the video region. Each wave owns 32 query rows as
// two 16-row blocks and computes, on bf16/fp16 MFMA 16x16x32 with fp32 accumulation,
//   S^T (16 keys x 16 queries) = K . round(Q*scale)^T   for 4 key blocks x 2 query blocks
// (lane l: query 16qq + l%16, keys 16kb + 4(l/16) + j), and counts the scores strictly
// below lse[row] + log_threshold. Each comparison is a wave-wide ballot whose popcount
// lands in a scalar register, so the count per (wave, key tile) needs no vector
// reduction. Counts are staged in LDS and combined into (query block, key block) cells
// of 64x64 or 128x128 tokens, then written as fp16(count / block_size^2).
//
// K tiles go straight from HBM into LDS (buffer_load ... lds, no register staging) in an
// XOR-swizzled row-major layout, double-buffered, one barrier per tile. Under the
// board's power limit the 16x16 shape holds a higher clock than 32x32x16, and without
// register staging it needs no more cycles. Its maps match the 32x32x16 form's
// bit for bit on the tested layers (both accumulate the same products in fp32).
//
// The list mode (kList) replays only the (query block, key tile) pairs of per-(head, 128-row
// query tile) key-tile lists with row bits, the format of moddit_mask_to_tiles, and
// writes only those cells: the refresh step's merge (MoD/mod/attn_mask.py:663-675) keeps
// the new map only where the current mask is active, so the other cells need no replay.
//
// Reference semantics: flash_sparsity_replay_kernel
// (MoD/mod/cuda_flash_sparsity_kernel.cu:41-169): Q scaled in fp32 and rounded to the
// input dtype (:86-92), fp32 products, strict '<' against lse + log_threshold (:138-143),
// __float2half_rn of count / block_size^2 (:158-163). The last video block may run past
// the sequence end; rows and keys at or beyond seq_len are then not counted.
#include "common.h"
#include "lds_dma.h"

namespace moddit {
namespace {

constexpr int kBM = 128;
constexpr int kBN = 64;
constexpr int kThreads = 256;
constexpr int kFlush = 64;  // key tiles per flush; the LDS count ring holds two flushes

template <int D>
struct ReplayLds {
  static constexpr int kRowBytes = D * 2;              // one key row, no padding
  static constexpr int kKBytes = kBN * kRowBytes;      // one 64-key K tile
  static constexpr int kRowsPerWindow = 1024 / kRowBytes;
  static constexpr int kWindows = kKBytes / 1024;      // 1 KB DMA windows per tile
  static constexpr int kCounts = 4 * 2 * kFlush * 4;   // int per (wave, ring slot)
  static constexpr int kTotal = 2 * kKBytes + kCounts;
};
// 16-byte chunk swizzle of a K row (XOR on the chunk index): the 16 rows a 16-lane group
// reads at one logical chunk land in distinct bank groups.
template <int D>
__device__ __forceinline__ int replay_swz(int r) { return (r / (128 / D)) % (D / 8); }

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
  // list mode: entries[h][qt][i] = key_tile << 2 | row bits, i < counts[h][qt]
  const int32_t* counts;
  const int32_t* entries;
  int cap;
};

template <int D, typename E, bool kRagged, bool kList>
__global__ __launch_bounds__(kThreads, 2) void replay_map_kernel(ReplayParams p) {
  using L = ReplayLds<D>;
  using V8 = typename E::vec8;

  extern __shared__ __align__(16) unsigned char smem[];
  int* cnt = reinterpret_cast<int*>(smem + 2 * L::kKBytes);

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int c16 = lane & 15;
  const int g = lane >> 4;

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
  constexpr int kDC = D / 32;

  // qf[qq][dc]: query row vrow0 + 16qq + c16, dims 32dc + 8g .. +7 (B operand of the
  // 16x16x32 MFMA), rounded as bf16(q * scale) like the reference
  V8 qf[2][kDC];
  float thr[2];
#pragma unroll
  for (int qq = 0; qq < 2; ++qq) {
    const int vrow = vrow0 + 16 * qq + c16;
    const bool row_ok = wave_active && vrow < p.valid_q;
    const int r = p.q_off + (row_ok ? vrow : 0);
    const u32x4* src = reinterpret_cast<const u32x4*>(qb + r * p.q_ss);
#pragma unroll
    for (int c = 0; c < kDC; ++c) {
      const u32x4 raw = src[4 * c + g];
      uint16_t e[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) e[j] = E::from_float(E::to_float(u16_at(raw, j)) * p.scale);
      const u32x4 packed = {pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]),
                            pack2(e[6], e[7])};
      qf[qq][c] = as_vec8<V8>(packed);
    }
    // rows past the sequence end count nothing (no score is below -inf)
    thr[qq] = row_ok ? p.lse[static_cast<int64_t>(bh) * p.seq_len + r] + p.log_thr : -INFINITY;
  }
  // Retire these loads before the loop (see attention.hip).
  __builtin_amdgcn_s_waitcnt(0);

  // K tiles go straight from HBM to LDS (buffer_load ... lds): window w of a stage holds
  // rows [w*kRowsPerWindow, ...), lane l at byte l*16, each lane loading the logical
  // chunk its physical position holds under the swizzle. Ragged grids keep the tile
  // offset in the range-checked VGPR offset, so rows past the last key load zeros.
  constexpr int kWinPerWave = L::kWindows / 4;
  const uint16_t* kvid = kb + static_cast<int64_t>(p.k_off) * p.k_ss;
  const u32x4 k_rsrc = raw_rsrc(kvid, p.k_bytes);
  const uint32_t k_lds = lds_addr(smem);
  uint32_t k_src[kWinPerWave];
#pragma unroll
  for (int i = 0; i < kWinPerWave; ++i) {
    const int w = wave * kWinPerWave + i;
    const int r = w * L::kRowsPerWindow + (lane * 16) / L::kRowBytes;
    const int pch = ((lane * 16) % L::kRowBytes) / 16;
    k_src[i] = static_cast<uint32_t>((r * p.k_ss + (pch ^ replay_swz<D>(r)) * 8) * 2);
  }
  const uint32_t k_tile_bytes = static_cast<uint32_t>(kBN * p.k_ss * 2);
  auto dma_tile = [&](int kt, int stage) {
    const uint32_t to = static_cast<uint32_t>(kt) * k_tile_bytes;
#pragma unroll
    for (int i = 0; i < kWinPerWave; ++i) {
      const uint32_t dst = k_lds + stage * L::kKBytes + (wave * kWinPerWave + i) * 1024;
      if constexpr (kRagged)
        lds_dma16(k_rsrc, dst, k_src[i] + to, 0);
      else
        lds_dma16(k_rsrc, dst, k_src[i], to);
    }
  };
  // K (A operand): row 16kb + c16, logical chunk 4dc + g; the swizzle depends on c16 only
  uint32_t k_rd[kDC];
#pragma unroll
  for (int c = 0; c < kDC; ++c)
    k_rd[c] = static_cast<uint32_t>(c16 * L::kRowBytes + (((4 * c + g) ^ replay_swz<D>(c16)) * 16));

  // The key tiles to sweep: all of them, or (list mode) the entries of this query tile.
  // A list entry outside [0, n_ktiles) holds no key of the video region: it is executed
  // by no wave and written nowhere (its DMA loads tile 0).
  int n_iter = p.n_ktiles;
  const int32_t* list = nullptr;
  if constexpr (kList) {
    const int64_t slot = static_cast<int64_t>(h) * p.n_qtiles + qt;
    n_iter = p.counts[slot];
    n_iter = n_iter < 0 ? 0 : (n_iter < p.cap ? n_iter : p.cap);
    list = p.entries + slot * p.cap;
  }
  const int wbit = 1 << (wave >> 1);  // row bit of this wave's 64 rows (list mode)
  auto key_tile = [&](int i, int& flags) -> int {
    if constexpr (!kList) {
      flags = 3;
      return i;
    } else {
      const int e = __builtin_amdgcn_readfirstlane(list[i]);
      const int kt = e >> 2;
      const bool in = kt >= 0 && kt < p.n_ktiles;
      flags = in ? (e & 3) : 0;
      return in ? kt : 0;
    }
  };

  int flags_cur = 0;
  int kt_cur = n_iter > 0 ? key_tile(0, flags_cur) : 0;
  if (n_iter > 0) dma_tile(kt_cur, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const float inv_area = 1.0f / static_cast<float>(p.block * p.block);
  uint16_t* out_bh = p.out + static_cast<int64_t>(bh) * p.nblk * p.nblk;

  for (int it = 0; it < n_iter; ++it) {
    const bool has_next = it + 1 < n_iter;
    int flags_next = 0;
    const int kt_next = has_next ? key_tile(it + 1, flags_next) : 0;
    // the stage of tile it+1 held tile it-1, which every wave finished reading before
    // the previous iteration's barrier
    if (has_next) dma_tile(kt_next, (it + 1) & 1);

    if (wave_active && (flags_cur & wbit)) {
      const unsigned char* ks = smem + (it & 1) * L::kKBytes;
      // s[kb][qq]: keys 16kb + 4g + j of query vrow0 + 16qq + c16
      f32x4 s[4][2];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) s[kb][0] = s[kb][1] = f32x4{};
#pragma unroll
      for (int c = 0; c < kDC; ++c) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const V8 a = *reinterpret_cast<const V8*>(ks + k_rd[c] + 16 * kb * L::kRowBytes);
          s[kb][0] = E::mma16(a, qf[0][c], s[kb][0]);
          s[kb][1] = E::mma16(a, qf[1][c], s[kb][1]);
        }
      }
      int total = 0;
      if (kRagged && kt_cur * kBN + kBN > p.valid_k) {
        // keys at or past the sequence end are not counted
        const int key0 = kt_cur * kBN + 4 * g;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool kin = key0 + 16 * kb + j < p.valid_k;
            total += __builtin_popcountll(__ballot(s[kb][0][j] < thr[0] && kin));
            total += __builtin_popcountll(__ballot(s[kb][1][j] < thr[1] && kin));
          }
      } else {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            total += __builtin_popcountll(__ballot(s[kb][0][j] < thr[0]));
            total += __builtin_popcountll(__ballot(s[kb][1][j] < thr[1]));
          }
      }
      // two halves of kFlush slots: a flush reads one half while the next kFlush key
      // tiles (at least one barrier later) write the other
      if (lane == 0) cnt[wave * 2 * kFlush + (it % (2 * kFlush))] = total;
    }

    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    const int slot_hi = it % kFlush;
    if (kList && (slot_hi == kFlush - 1 || !has_next)) {
      // list mode: position s of the flush holds the entry it - slot_hi + s
      const int it0 = it - slot_hi;
      const int hb = ((it / kFlush) & 1) * kFlush;
      if (p.block == 64) {
        if (tid < 2 * kFlush) {
          const int qsub = tid / kFlush;
          const int s = tid % kFlush;
          const int qblk = 2 * qt + qsub;
          if (s <= slot_hi && qblk < p.nblk) {
            const int e = list[it0 + s];
            const int kt = e >> 2;
            if (((e >> qsub) & 1) && kt >= 0 && kt < p.n_ktiles) {
              const int c = cnt[(2 * qsub) * 2 * kFlush + hb + s] +
                            cnt[(2 * qsub + 1) * 2 * kFlush + hb + s];
              const float ratio = static_cast<float>(c) * inv_area;
              out_bh[static_cast<int64_t>(qblk) * p.nblk + kt] = Fp16::from_float(ratio);
            }
          }
        }
      } else {
        // one 128-row block per query tile; the entries come in pairs (2j, 2j+1), both
        // rows bits set, one pair per active key block j (the moddit_mask_to_tiles list
        // of a 128-token block mask), so a pair never straddles a flush (kFlush is even)
        if (tid < kFlush / 2) {
          const int u = tid;
          if (2 * u + 1 <= slot_hi) {
            const int e = list[it0 + 2 * u];
            const int kt = e >> 2;
            if ((e & 3) == 3 && kt >= 0 && kt + 1 < p.n_ktiles) {
              int c = 0;
#pragma unroll
              for (int w = 0; w < 4; ++w)
                c += cnt[w * 2 * kFlush + hb + 2 * u] + cnt[w * 2 * kFlush + hb + 2 * u + 1];
              const float ratio = static_cast<float>(c) * inv_area;
              out_bh[static_cast<int64_t>(qt) * p.nblk + kt / 2] = Fp16::from_float(ratio);
            }
          }
        }
      }
    } else if (!kList && (slot_hi == kFlush - 1 || !has_next)) {
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
    kt_cur = kt_next;
    flags_cur = flags_next;
  }
}

template <int D, typename E, bool kRagged, bool kList>
int launch_replay_impl(const ReplayParams& p, int batch, hipStream_t stream) {
  using L = ReplayLds<D>;
  auto kernel = replay_map_kernel<D, E, kRagged, kList>;
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
  const bool aligned = p.valid_k == p.n_ktiles * kBN;
  if (p.entries != nullptr)
    return aligned ? launch_replay_impl<D, E, false, true>(p, batch, stream)
                   : launch_replay_impl<D, E, true, true>(p, batch, stream);
  return aligned ? launch_replay_impl<D, E, false, false>(p, batch, stream)
                 : launch_replay_impl<D, E, true, false>(p, batch, stream);
}

}  // namespace
}  // namespace moddit

namespace moddit {
namespace {

int sparsity_map_common(const void* q, const void* k, const float* lse, void* map_out,
                        int batch, int heads, int seq_len, int head_dim,
                        const int64_t q_strides[3], const int64_t k_strides[3],
                        float softmax_scale, float log_threshold, int q_video_offset,
                        int k_video_offset, int video_blocks, int block_size, int dtype,
                        const int32_t* tile_counts, const int32_t* tile_entries, int n_qtiles,
                        int cap, moddit_stream_t stream) {
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
  p.counts = tile_counts;
  p.entries = tile_entries;
  p.cap = cap;
  if (tile_entries != nullptr) {
    MODDIT_CHECK_ARG(tile_counts != nullptr, "sparsity_map_merge: null tile counts");
    MODDIT_CHECK_ARG(n_qtiles == p.n_qtiles,
                     "sparsity_map_merge: the tile lists have %d query tiles, the video region "
                     "needs %d", n_qtiles, p.n_qtiles);
    MODDIT_CHECK_ARG(cap >= 0, "sparsity_map_merge: negative list capacity");
  }
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

}  // namespace
}  // namespace moddit

extern "C" int moddit_sparsity_map(const void* q, const void* k, const float* lse, void* map_out,
                                   int batch, int heads, int seq_len, int head_dim,
                                   const int64_t q_strides[3], const int64_t k_strides[3],
                                   float softmax_scale, float log_threshold, int q_video_offset,
                                   int k_video_offset, int video_blocks, int block_size,
                                   int dtype, moddit_stream_t stream) {
  moddit::clear_error();
  return moddit::sparsity_map_common(q, k, lse, map_out, batch, heads, seq_len, head_dim,
                                     q_strides, k_strides, softmax_scale, log_threshold,
                                     q_video_offset, k_video_offset, video_blocks, block_size,
                                     dtype, nullptr, nullptr, 0, 0, stream);
}

extern "C" int moddit_sparsity_map_merge(const void* q, const void* k, const float* lse,
                                         void* map_inout, int batch, int heads, int seq_len,
                                         int head_dim, const int64_t q_strides[3],
                                         const int64_t k_strides[3], float softmax_scale,
                                         float log_threshold, int q_video_offset,
                                         int k_video_offset, int video_blocks, int block_size,
                                         int dtype, const int32_t* tile_counts,
                                         const int32_t* tile_entries, int n_qtiles, int cap,
                                         moddit_stream_t stream) {
  moddit::clear_error();
  MODDIT_CHECK_ARG(tile_counts && tile_entries, "sparsity_map_merge: null tile lists");
  return moddit::sparsity_map_common(q, k, lse, map_inout, batch, heads, seq_len, head_dim,
                                     q_strides, k_strides, softmax_scale, log_threshold,
                                     q_video_offset, k_video_offset, video_blocks, block_size,
                                     dtype, tile_counts, tile_entries, n_qtiles, cap, stream);
}
