// Dense and block-sparse flash-attention forward for gfx950 (CDNA4).
//
// One workgroup = 4 wave64s = 128 query rows (each wave owns 32 rows); keys stream in
// tiles of 64 (the mask's key-block granularity). Per key tile each wave computes
//   S^T (64 keys x 32 queries) = K . Q^T      with 2 x 8 (d=128) bf16 MFMA 32x32x16
//   O^T (d x 32 queries)      += V^T . P^T    with (d/32) x 4 MFMA 32x32x16
// Computing the transposed products puts one query per lane column, so the running
// row max / row sum live in one lane (plus one exchange with the lane 32 apart) and
// the rescale of O is a per-lane multiply. The S^T accumulator layout is exactly the
// B-operand layout P^T needs, so P never leaves registers.
//
// LDS per stage: K row-major [64][d] (pitch 2d+16 B) and V transposed [d][64]
// (pitch 136 B); two stages double-buffer the tiles, filled from registers that were
// loaded from global memory during the previous tile's math.
//
// The sparse variant walks a per-(head, query tile) list of key tiles, each entry
// carrying two row bits (query rows 0-63 / 64-127 of the tile); a wave whose bit is
// clear skips the math but still helps stage the tile.
//
// Reference semantics: flash_attn_func (MoD/mod/triton_flash_sparsity.py:320-321) for
// the dense pass incl. its LSE; block_sparse_sage2_attn_cuda at 128q x 64k tiles
// (MoD/mod/attn_mask.py:296-317) for the sparse pass, computed here in bf16/fp16 with
// fp32 softmax instead of SageAttention's quantisation.
#include "common.h"

namespace moddit {
namespace {

constexpr int kBM = 128;  // query rows per workgroup
constexpr int kBN = 64;   // keys per tile
constexpr int kThreads = 256;

template <int D>
struct AttnLds {
  static constexpr int kPitchK = D * 2 + 16;  // bytes per K row (68 dwords for d=128: 4 mod 64 banks)
  static constexpr int kPitchV = kBN * 2 + 16;  // bytes per V^T row (36 dwords: 16 lanes hit 16 bank quads)
  static constexpr int kKBytes = kBN * kPitchK;
  static constexpr int kVBytes = D * kPitchV;
  static constexpr int kStage = kKBytes + kVBytes;
  static constexpr int kTotal = 2 * kStage;
};

struct AttnParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int heads;
  int q_len;
  int kv_len;
  int n_qtiles;
  int n_ktiles;
  float scale_log2;  // softmax_scale * log2(e)
  const int32_t* counts;
  const int32_t* entries;
  int cap;
  uint32_t k_bytes;  // byte span of one head's K rows [0, kv_len)
  uint32_t v_bytes;
};

// Rows of a 64-key tile are stored in LDS in the order pi(r): inside every 16-row chunk
// the row groups [4,8) and [8,12) are swapped. With that order the S^T accumulator of
// lane half h holds keys 8h..8h+7 of each 16-key chunk, in order, so the matching V^T
// operand is one 16-byte LDS read.
__device__ __forceinline__ int key_perm(int r) { return r ^ ((((r >> 2) ^ (r >> 3)) & 1) * 12); }

// The running row max is only moved when a tile's max exceeds it by more than this many
// log2 units; probabilities then stay <= 2^8 and the O rescale is skipped for whole
// waves on most tiles. Softmax is shift-invariant, so results do not depend on it.
constexpr float kRescaleSlack = 8.0f;

template <int D, typename E, bool kSparse, bool kRagged>
__global__ __launch_bounds__(kThreads, 2) void attention_fwd_kernel(AttnParams p) {
  using L = AttnLds<D>;
  using V8 = typename E::vec8;
  constexpr int kDChunks = D / 16;                       // MFMA k-steps over d for S^T
  constexpr int kDSub = D / 32;                          // 32-row blocks of O^T
  constexpr int kVecPerRow = D / 8;                      // 16-byte vectors per token row
  constexpr int kKVecs = kBN * kVecPerRow / kThreads;    // K vectors per thread
  constexpr int kKRowStep = kThreads / kVecPerRow;       // K rows between a thread's vectors
  constexpr int kKeysPerThr = D / 32;                    // V keys per thread (x 8 dims)
  constexpr int kKeyGroups = kBN / kKeysPerThr;          // V key groups per tile

  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int half = lane >> 5;
  const int c32 = lane & 31;

  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = tile % p.n_qtiles;
  const int bh = tile / p.n_qtiles;
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;

  const uint16_t* qb = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* kb = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* vb = p.v + b * p.v_sb + h * p.v_sh;

  // ---- tile list ----
  int n_iter;
  const int32_t* list = nullptr;
  if (kSparse) {
    const int64_t slot = static_cast<int64_t>(h) * p.n_qtiles + qt;
    n_iter = p.counts[slot];
    n_iter = n_iter < 0 ? 0 : (n_iter < p.cap ? n_iter : p.cap);
    list = p.entries + slot * p.cap;
  } else {
    n_iter = p.n_ktiles;
  }
  const int wbit = 1 << (wave >> 1);

  // ---- Q fragments (B operand of S^T = K Q^T): lane holds query c32, dims 8*half.. ----
  const int q_row = qt * kBM + wave * 32 + c32;
  V8 qf[kDChunks];
  {
    const int r = q_row < p.q_len ? q_row : p.q_len - 1;
    const u32x4* src = reinterpret_cast<const u32x4*>(qb + r * p.q_ss);
#pragma unroll
    for (int c = 0; c < kDChunks; ++c) qf[c] = as_vec8<V8>(src[2 * c + half]);
    // Sparse: retire the Q loads here, otherwise the waitcnt pass keeps them pending
    // across the loop back-edge and every tile's first MFMAs wait for the K/V prefetch.
    // Dense: measured faster without it (the in-order wait de-phases the two waves that
    // share a SIMD), so it is left to the compiler there.
    if constexpr (kSparse) __builtin_amdgcn_s_waitcnt(0);
  }

  // ---- global -> register staging of one K/V tile ----
  // K: thread owns column k_col of rows k_row0 + i*kKRowStep (row-major, 256 B rows).
  // V: thread owns keys v_kgrp*kKeysPerThr + j, dims v_dgrp*8.. (transposed into LDS).
  const int k_col = tid % kVecPerRow;
  const int k_row0 = tid / kVecPerRow;
  const int v_kgrp = tid % kKeyGroups;
  const int v_dgrp = tid / kKeyGroups;
  // Buffer resources over this head's K/V rows; the byte span was checked on the host.
  const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(kb, p.k_bytes);
  const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc(vb, p.v_bytes);
  const uint32_t k_voff = static_cast<uint32_t>((k_row0 * p.k_ss + k_col * 8) * 2);
  const uint32_t v_voff = static_cast<uint32_t>((v_kgrp * kKeysPerThr * p.v_ss + v_dgrp * 8) * 2);
  const uint32_t k_row_step = static_cast<uint32_t>(kKRowStep * p.k_ss * 2);
  const uint32_t k_tile_bytes = static_cast<uint32_t>(kBN * p.k_ss * 2);
  const uint32_t v_row_bytes = static_cast<uint32_t>(p.v_ss * 2);
  const uint32_t v_tile_bytes = static_cast<uint32_t>(kBN * p.v_ss * 2);
  u32x4 kreg[kKVecs];
  u32x4 vreg[kKeysPerThr];

  // Full tiles put the tile offset in the SGPR offset (loop-invariant VGPR offsets keep
  // the loads free of register reuse hazards); the ragged variant puts it in the
  // range-checked VGPR offset so rows past kv_len read as zeros.
#define MODDIT_LOAD_TILE(KT)                                                              \
  do {                                                                                    \
    if constexpr (!kRagged) {                                                             \
      const uint32_t kso_ = static_cast<uint32_t>(KT) * k_tile_bytes;                     \
      const uint32_t vso_ = static_cast<uint32_t>(KT) * v_tile_bytes;                     \
      _Pragma("unroll") for (int i_ = 0; i_ < kKVecs; ++i_)                               \
          kreg[i_] = buf_load16(k_rsrc, k_voff, kso_ + i_ * k_row_step);                  \
      _Pragma("unroll") for (int j_ = 0; j_ < kKeysPerThr; ++j_)                          \
          vreg[j_] = buf_load16(v_rsrc, v_voff, vso_ + j_ * v_row_bytes);                 \
    } else {                                                                              \
      const uint32_t kto_ = static_cast<uint32_t>(KT) * k_tile_bytes;                     \
      const uint32_t vto_ = static_cast<uint32_t>(KT) * v_tile_bytes;                     \
      _Pragma("unroll") for (int i_ = 0; i_ < kKVecs; ++i_)                               \
          kreg[i_] = buf_load16(k_rsrc, k_voff + kto_ + i_ * k_row_step, 0);              \
      _Pragma("unroll") for (int j_ = 0; j_ < kKeysPerThr; ++j_)                          \
          vreg[j_] = buf_load16(v_rsrc, v_voff + vto_ + j_ * v_row_bytes, 0);             \
    }                                                                                     \
  } while (0)

#define MODDIT_STORE_TILE(STAGE)                                                          \
  do {                                                                                    \
    unsigned char* ks_ = smem + (STAGE) * L::kStage;                                      \
    unsigned char* vs_ = ks_ + L::kKBytes;                                                \
    _Pragma("unroll") for (int i_ = 0; i_ < kKVecs; ++i_) {                               \
      const int row_ = key_perm(k_row0 + i_ * kKRowStep);                                 \
      *reinterpret_cast<u32x4*>(ks_ + row_ * L::kPitchK + k_col * 16) = kreg[i_];         \
    }                                                                                     \
    _Pragma("unroll") for (int dd_ = 0; dd_ < 8; ++dd_) {                                 \
      unsigned char* dst_ =                                                               \
          vs_ + (v_dgrp * 8 + dd_) * L::kPitchV + v_kgrp * kKeysPerThr * 2;               \
      const uint32_t sel_ = (dd_ & 1) ? 0x07060302u : 0x05040100u;                        \
      if constexpr (kKeysPerThr == 4) {                                                   \
        u32x2 w_;                                                                         \
        w_.x = __builtin_amdgcn_perm(vreg[1][dd_ >> 1], vreg[0][dd_ >> 1], sel_);         \
        w_.y = __builtin_amdgcn_perm(vreg[3][dd_ >> 1], vreg[2][dd_ >> 1], sel_);         \
        *reinterpret_cast<u32x2*>(dst_) = w_;                                             \
      } else {                                                                            \
        *reinterpret_cast<uint32_t*>(dst_) =                                              \
            __builtin_amdgcn_perm(vreg[1][dd_ >> 1], vreg[0][dd_ >> 1], sel_);            \
      }                                                                                   \
    }                                                                                     \
  } while (0)

  f32x16 oacc[kDSub];
#pragma unroll
  for (int i = 0; i < kDSub; ++i) oacc[i] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;

  // Tile-list entries are uniform; decode with a clamp so a corrupt list can only select
  // a wrong (in-bounds) tile, never address outside K/V.
  auto decode = [&](int e_raw, int& kt, int& flags) {
    const int e = __builtin_amdgcn_readfirstlane(e_raw);
    kt = e >> 2;
    kt = kt < 0 ? 0 : (kt < p.n_ktiles ? kt : p.n_ktiles - 1);
    flags = e & 3;
  };
  auto entry = [&](int i) -> int {
    return kSparse ? list[i] : ((i << 2) | 3);
  };

  int e_cur = 0, e_next = 0;
  if (n_iter > 0) {
    e_cur = entry(0);
    if (n_iter > 1) e_next = entry(1);
    int kt0, fl0;
    decode(e_cur, kt0, fl0);
    MODDIT_LOAD_TILE(kt0);
    MODDIT_STORE_TILE(0);
  }
  __syncthreads();

  for (int it = 0; it < n_iter; ++it) {
    int kt, flags;
    decode(e_cur, kt, flags);
    const bool has_next = it + 1 < n_iter;
    int e_after = 0;
    if (has_next) {
      // The entry two tiles ahead is requested before this tile's K/V loads, so waiting
      // for it later never waits for those loads.
      if (it + 2 < n_iter) e_after = entry(it + 2);
      int kn, fn;
      decode(e_next, kn, fn);
      MODDIT_LOAD_TILE(kn);
    }

    if (flags & wbit) {
      const unsigned char* ks = smem + (it & 1) * L::kStage;
      const unsigned char* vs = ks + L::kKBytes;

      // S^T = K . Q^T, two 32-key halves (rows in key_perm order).
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

      if constexpr (kRagged) {
        const int key0 = kt * kBN;
        if (key0 + kBN > p.kv_len) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int kr = (i >> 3) * 16 + 8 * half + (i & 7);  // actual key of acc row i
            if (key0 + kr >= p.kv_len) s0[i] = -INFINITY;
            if (key0 + 32 + kr >= p.kv_len) s1[i] = -INFINITY;
          }
        }
      }

      float mx = s0[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s0[i]);
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s1[i]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mxs = mx * p.scale_log2;

      const bool need = mxs > m_run + kRescaleSlack;
      if (__ballot(need) != 0ull) {
        const float m_new = need ? mxs : m_run;
        const float alpha = need ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
        l_run *= alpha;
#pragma unroll
        for (int dsub = 0; dsub < kDSub; ++dsub) oacc[dsub] *= alpha;
        m_run = m_new;
      }
      const float m_use = (m_run == -INFINITY) ? 0.f : m_run;

      V8 pb[4];
      float rs = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[i], p.scale_log2, -m_use));
        const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[i], p.scale_log2, -m_use));
        rs += e0 + e1;
        pb[i >> 3][i & 7] = static_cast<typename E::elem>(e0);
        pb[2 + (i >> 3)][i & 7] = static_cast<typename E::elem>(e1);
      }
      l_run += rs;

      // O^T += V^T . P^T: lane half h supplies keys 8h..8h+7 of each 16-key chunk.
#pragma unroll
      for (int dsub = 0; dsub < kDSub; ++dsub) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const V8 a = *reinterpret_cast<const V8*>(vs + (dsub * 32 + c32) * L::kPitchV + c * 32 +
                                                    half * 16);
          oacc[dsub] = E::mma(a, pb[c], oacc[dsub]);
        }
      }
    }

    if (has_next) MODDIT_STORE_TILE((it + 1) & 1);
    __syncthreads();
    e_cur = e_next;
    e_next = e_after;
  }

  // ---- epilogue ----
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (q_row < p.q_len) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    uint16_t* orow = p.o + b * p.o_sb + h * p.o_sh + q_row * p.o_ss;
#pragma unroll
    for (int dsub = 0; dsub < kDSub; ++dsub) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = dsub * 32 + 8 * g + 4 * half;
        u32x2 w;
        w.x = pack2(E::from_float(oacc[dsub][4 * g + 0] * inv),
                    E::from_float(oacc[dsub][4 * g + 1] * inv));
        w.y = pack2(E::from_float(oacc[dsub][4 * g + 2] * inv),
                    E::from_float(oacc[dsub][4 * g + 3] * inv));
        *reinterpret_cast<u32x2*>(orow + d) = w;
      }
    }
    if (p.lse != nullptr && half == 0) {
      const int64_t li = static_cast<int64_t>(bh) * p.q_len + q_row;
      p.lse[li] = l_tot > 0.f ? (m_run + log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
    }
  }
}

#undef MODDIT_LOAD_TILE
#undef MODDIT_STORE_TILE

template <int D, typename E, bool kSparse, bool kRagged>
int launch_attention_impl(const AttnParams& p, int batch, hipStream_t stream) {
  using L = AttnLds<D>;
  auto kernel = attention_fwd_kernel<D, E, kSparse, kRagged>;
  static bool configured = false;  // the attribute is per function, same on every device
  if (!configured) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, L::kTotal) != hipSuccess) {
      set_error("attention: cannot reserve %d bytes of LDS", L::kTotal);
      return MODDIT_EHIP;
    }
    configured = true;
  }
  const int64_t tiles = static_cast<int64_t>(batch) * p.heads * p.n_qtiles;
  if (tiles == 0) return MODDIT_OK;
  if (tiles > 0x7fffffff) {
    set_error("attention: too many tiles (%lld)", static_cast<long long>(tiles));
    return MODDIT_EINVAL;
  }
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), L::kTotal,
                     stream, p);
  MODDIT_CHECK_LAUNCH("attention");
  return MODDIT_OK;
}

template <int D, typename E, bool kSparse>
int launch_attention(const AttnParams& p, int batch, hipStream_t stream) {
  // Key counts that are a multiple of the tile need no clamping or masking at all.
  if (p.kv_len % kBN == 0) return launch_attention_impl<D, E, kSparse, false>(p, batch, stream);
  return launch_attention_impl<D, E, kSparse, true>(p, batch, stream);
}

int attention_entry(const void* q, const void* k, const void* v, void* o, float* lse, int batch,
                    int heads, int q_len, int kv_len, int head_dim, const int64_t* qs,
                    const int64_t* ks, const int64_t* vs, const int64_t* os, float scale,
                    int dtype, const int32_t* counts, const int32_t* entries, int n_qtiles,
                    int cap, moddit_stream_t stream) {
  clear_error();
  MODDIT_CHECK_ARG(q && k && v && o, "attention: null tensor pointer");
  MODDIT_CHECK_ARG(qs && ks && vs && os, "attention: null stride array");
  MODDIT_CHECK_ARG(scale > 0.f && std::isfinite(scale), "attention: softmax_scale must be positive");
  MODDIT_CHECK_ARG(batch >= 0 && heads >= 0 && q_len >= 0 && kv_len >= 0,
                   "attention: negative size");
  if (head_dim != 64 && head_dim != 128) {
    set_error("attention: head_dim must be 64 or 128, got %d", head_dim);
    return MODDIT_EUNSUPPORTED;
  }
  if (dtype != MODDIT_BF16 && dtype != MODDIT_FP16) {
    set_error("attention: dtype must be bf16 or fp16");
    return MODDIT_EUNSUPPORTED;
  }
  MODDIT_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o),
                   "attention: q/k/v/o must be 16-byte aligned");
  const int64_t* all[4] = {qs, ks, vs, os};
  for (int t = 0; t < 4; ++t)
    for (int j = 0; j < 3; ++j)
      MODDIT_CHECK_ARG(all[t][j] >= 0 && all[t][j] % 8 == 0,
                       "attention: strides must be non-negative multiples of 8 elements");
  const bool sparse = counts != nullptr;
  const int nq = (q_len + kBM - 1) / kBM;
  if (sparse) {
    MODDIT_CHECK_ARG(entries != nullptr, "attention: tile entries missing");
    MODDIT_CHECK_ARG(n_qtiles == nq, "attention: n_qtiles=%d but q_len=%d needs %d", n_qtiles,
                     q_len, nq);
    MODDIT_CHECK_ARG(cap > 0, "attention: cap must be positive");
  }
  if (q_len == 0 || batch == 0 || heads == 0) return MODDIT_OK;
  MODDIT_CHECK_ARG(kv_len > 0 || sparse, "attention: kv_len must be positive for dense attention");

  AttnParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<uint16_t*>(o);
  p.lse = lse;
  p.q_sb = qs[0]; p.q_sh = qs[1]; p.q_ss = qs[2];
  p.k_sb = ks[0]; p.k_sh = ks[1]; p.k_ss = ks[2];
  p.v_sb = vs[0]; p.v_sh = vs[1]; p.v_ss = vs[2];
  p.o_sb = os[0]; p.o_sh = os[1]; p.o_ss = os[2];
  p.heads = heads;
  p.q_len = q_len;
  p.kv_len = kv_len;
  p.n_qtiles = nq;
  p.n_ktiles = (kv_len + kBN - 1) / kBN;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.counts = counts;
  p.entries = entries;
  p.cap = cap;
  if (sparse && kv_len == 0) {
    set_error("attention: kv_len must be positive");
    return MODDIT_EINVAL;
  }
  // Per-head K/V spans are addressed with 32-bit buffer offsets; a whole 64-key tile past
  // the last row must also stay below 2^31.
  const int64_t k_span = (static_cast<int64_t>(kv_len) - 1) * ks[2] * 2 + head_dim * 2;
  const int64_t v_span = (static_cast<int64_t>(kv_len) - 1) * vs[2] * 2 + head_dim * 2;
  const int64_t max_off = (static_cast<int64_t>(p.n_ktiles) * kBN) * (ks[2] > vs[2] ? ks[2] : vs[2]) * 2;
  if (k_span > 0x7fffffffLL || v_span > 0x7fffffffLL || max_off > 0x7fffffffLL) {
    set_error("attention: one head's K/V span exceeds 2 GiB of 32-bit offsets");
    return MODDIT_EUNSUPPORTED;
  }
  p.k_bytes = static_cast<uint32_t>(k_span);
  p.v_bytes = static_cast<uint32_t>(v_span);

  hipStream_t st = as_stream(stream);
  const bool bf = dtype == MODDIT_BF16;
  if (head_dim == 128) {
    if (bf) return sparse ? launch_attention<128, Bf16, true>(p, batch, st)
                          : launch_attention<128, Bf16, false>(p, batch, st);
    return sparse ? launch_attention<128, Fp16, true>(p, batch, st)
                  : launch_attention<128, Fp16, false>(p, batch, st);
  }
  if (bf) return sparse ? launch_attention<64, Bf16, true>(p, batch, st)
                        : launch_attention<64, Bf16, false>(p, batch, st);
  return sparse ? launch_attention<64, Fp16, true>(p, batch, st)
                : launch_attention<64, Fp16, false>(p, batch, st);
}

}  // namespace
}  // namespace moddit

extern "C" int moddit_flash_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                                int batch, int heads, int q_len, int kv_len, int head_dim,
                                const int64_t q_strides[3], const int64_t k_strides[3],
                                const int64_t v_strides[3], const int64_t o_strides[3],
                                float softmax_scale, int dtype, moddit_stream_t stream) {
  return moddit::attention_entry(q, k, v, o, lse, batch, heads, q_len, kv_len, head_dim,
                                 q_strides, k_strides, v_strides, o_strides, softmax_scale, dtype,
                                 nullptr, nullptr, 0, 0, stream);
}

extern "C" int moddit_block_sparse_fwd(const void* q, const void* k, const void* v, void* o,
                                       float* lse, int batch, int heads, int q_len, int kv_len,
                                       int head_dim, const int64_t q_strides[3],
                                       const int64_t k_strides[3], const int64_t v_strides[3],
                                       const int64_t o_strides[3], float softmax_scale, int dtype,
                                       const int32_t* counts, const int32_t* entries,
                                       int n_qtiles, int cap, moddit_stream_t stream) {
  if (counts == nullptr) {
    moddit::set_error("block_sparse_fwd: counts must not be NULL");
    return MODDIT_EINVAL;
  }
  return moddit::attention_entry(q, k, v, o, lse, batch, heads, q_len, kv_len, head_dim,
                                 q_strides, k_strides, v_strides, o_strides, softmax_scale, dtype,
                                 counts, entries, n_qtiles, cap, stream);
}
