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
// K and V tiles go straight from HBM into LDS (buffer_load ... lds, no register
// staging), both row-major with an XOR swizzle on 16-byte chunks that keeps the operand
// reads bank-conflict free; V^T fragments come out of the row-major V tile through
// ds_read_b64_tr_b16. Two stages per operand. The loop is software pipelined:
// iteration j computes S_{j+1} and O += P_j V_j while K_{j+2} and V_{j+1} stream in, then
// the softmax of S_{j+1}; one barrier per tile.
//
// The sparse variant walks a per-(head, query tile) list of key tiles, each entry
// carrying two row bits (query rows 0-63 / 64-127 of the tile); a wave whose bit is
// clear skips the math but still issues its share of the tile's DMA.
//
// Reference semantics: flash_attn_func (MoD/mod/triton_flash_sparsity.py:320-321) for
// the dense pass incl. its LSE; block_sparse_sage2_attn_cuda at 128q x 64k tiles
// (MoD/mod/attn_mask.py:296-317) for the sparse pass, computed here in bf16/fp16 with
// fp32 softmax instead of SageAttention's quantisation.
#include "common.h"
#include "lds_dma.h"

namespace moddit {
namespace {

constexpr int kBM = 128;  // query rows per workgroup
constexpr int kBN = 64;   // keys per tile
constexpr int kThreads = 256;

template <int D>
struct AttnLds {
  static constexpr int kRowBytes = D * 2;                 // one token row, no padding
  static constexpr int kTileBytes = kBN * kRowBytes;      // one 64-key K or V tile
  static constexpr int kTotal = 4 * kTileBytes;           // K ring (2) + V ring (2)
  static constexpr int kChunks = D / 8;                   // 16-byte chunks per row
  static constexpr int kRowsPerWindow = 1024 / kRowBytes; // rows per 1 KB DMA window
  static constexpr int kWindows = kTileBytes / 1024;      // DMA windows per tile
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
  int origin;    // token index of grid row/column 0 (-63..0); see moddit_block_sparse_fwd
  int n_qtiles;
  int n_ktiles;
  int xcd_run;    // workgroup -> tile order (xcd_remap)
  float scale_log2;  // softmax_scale * log2(e)
  const int32_t* counts;
  const int32_t* entries;
  int cap;
  uint32_t k_bytes;  // byte span of one head's K rows [0, kv_len)
  uint32_t v_bytes;
  // fused sparsity map (map != nullptr only for the kMap kernels)
  uint16_t* map;     // fp16 (B*H, map_nblk, map_nblk)
  int map_q_off;     // token of video row 0 (== key offset)
  int map_kt0;       // grid key tile holding video key 0
  int map_nblk;      // video blocks per side
  int map_block;     // 64 or 128
  int map_valid;     // video tokens that exist: min(map_nblk*map_block, seq_len - map_q_off)
  float map_scale;   // softmax scale applied to q before rounding
  float map_log_thr; // ln(threshold)
};

// K rows are stored in LDS in the order pi(r): inside every 16-row chunk the row groups
// [4,8) and [8,12) are swapped, so the S^T accumulator of lane half h holds keys
// 8h..8h+7 of each 16-key chunk, in order (the P^T operand needs no shuffle).
__device__ __forceinline__ int key_perm(int r) { return r ^ ((((r >> 2) ^ (r >> 3)) & 1) * 12); }

// 16-byte chunk swizzles (XOR on the chunk index) that make the MFMA operand reads
// bank-conflict free: K rows are read one row per lane (A operand of S^T), V rows
// through ds_read_b64_tr_b16 (four keys x 32 dims per half-wave).
template <int D>
__device__ __forceinline__ int swz_k(int r) { return (r / (128 / D)) % (D / 8); }
template <int D>
__device__ __forceinline__ int swz_v(int key) { return 4 * ((key / (128 / D)) % (D / 32)); }

// The running row max is only moved when a tile's max exceeds it by more than this many
// log2 units; probabilities then stay <= 2^8 and the O rescale is skipped for whole
// waves on most tiles. Softmax is shift-invariant, so results do not depend on it.
constexpr float kRescaleSlack = 8.0f;

typedef short s16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i%4 of the
// 4-element rows addressed by lanes i/4, i/4+4, i/4+8, i/4+12.
__device__ __forceinline__ s16x4 lds_read_tr16(const unsigned char* a) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(a));
}

// Map flush granularity of the fused map pass (key tiles per flush; the LDS count ring
// holds two flushes so that a flush never races the next tiles' counts).
constexpr int kMapFlush = 64;
constexpr int kMapCountBytes = 4 * 2 * kMapFlush * 4;  // int per (wave, ring slot)

template <int D, typename E, bool kSparse, bool kRagged, bool kMap = false>
__global__ __launch_bounds__(kThreads, 2) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_fwd_kernel(AttnParams p) {
  using L = AttnLds<D>;
  using V8 = typename E::vec8;
  constexpr int kDChunks = D / 16;  // MFMA k-steps over d for S^T
  constexpr int kDSub = D / 32;     // 32-row blocks of O^T
  constexpr int kWinPerWave = L::kWindows / 4;

  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* const k_ring = smem;
  unsigned char* const v_ring = smem + 2 * L::kTileBytes;

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
  const uint16_t* vb = p.v + b * p.v_sb + h * p.v_sh;

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
  // Grid rows outside [0, q_len) are padding: they load a clamped row and store nothing.
  const int q_row = p.origin + qt * kBM + wave * 32 + c32;
  V8 qf[kDChunks];
  {
    const int r = q_row < 0 ? 0 : (q_row < p.q_len ? q_row : p.q_len - 1);
    const u32x4* src = reinterpret_cast<const u32x4*>(qb + r * p.q_ss);
#pragma unroll
    for (int c = 0; c < kDChunks; ++c) qf[c] = as_vec8<V8>(src[2 * c + half]);
    __builtin_amdgcn_s_waitcnt(0);
  }

  // ---- direct global -> LDS staging (buffer_load ... lds, 16 B per lane) ----
  // DMA window w writes LDS bytes [w*1024, w*1024+1024) of a stage, lane l at l*16. The
  // per-lane source is chosen so that the window holds the swizzled rows.
  const u32x4 k_rsrc = raw_rsrc(kb, p.k_bytes);
  const u32x4 v_rsrc = raw_rsrc(vb, p.v_bytes);
  const uint32_t k_lds = lds_addr(k_ring);
  const uint32_t v_lds = lds_addr(v_ring);
  uint32_t k_src[kWinPerWave];
  uint32_t v_src[kWinPerWave];
#pragma unroll
  for (int i = 0; i < kWinPerWave; ++i) {
    const int w = wave * kWinPerWave + i;
    const int r = w * L::kRowsPerWindow + (lane * 16) / L::kRowBytes;  // LDS row
    const int pch = ((lane * 16) % L::kRowBytes) / 16;                  // physical chunk
    const int kq = pch ^ swz_k<D>(r);                                   // logical chunk
    const int vq = pch ^ swz_v<D>(r);
    k_src[i] = static_cast<uint32_t>((key_perm(r) * p.k_ss + kq * 8) * 2);
    v_src[i] = static_cast<uint32_t>((r * p.v_ss + vq * 8) * 2);
  }
  const uint32_t k_tile_bytes = static_cast<uint32_t>(kBN * p.k_ss * 2);
  const uint32_t v_tile_bytes = static_cast<uint32_t>(kBN * p.v_ss * 2);
  // Grid origin in bytes (two's complement). Keys before token 0 get offsets that wrap
  // to >= 2^31, beyond every range the buffer descriptors admit, so they load zeros.
  const uint32_t k_org = static_cast<uint32_t>(p.origin * static_cast<int>(p.k_ss) * 2);
  const uint32_t v_org = static_cast<uint32_t>(p.origin * static_cast<int>(p.v_ss) * 2);

  auto dma_k = [&](int kt, int stage) {
    const uint32_t to = static_cast<uint32_t>(kt) * k_tile_bytes;
#pragma unroll
    for (int i = 0; i < kWinPerWave; ++i) {
      const uint32_t dst = k_lds + stage * L::kTileBytes + (wave * kWinPerWave + i) * 1024;
      if constexpr (kRagged)
        lds_dma16(k_rsrc, dst, k_src[i] + to + k_org, 0);
      else
        lds_dma16(k_rsrc, dst, k_src[i], to);
    }
  };
  auto dma_v = [&](int kt, int stage) {
    const uint32_t to = static_cast<uint32_t>(kt) * v_tile_bytes;
#pragma unroll
    for (int i = 0; i < kWinPerWave; ++i) {
      const uint32_t dst = v_lds + stage * L::kTileBytes + (wave * kWinPerWave + i) * 1024;
      if constexpr (kRagged)
        lds_dma16(v_rsrc, dst, v_src[i] + to + v_org, 0);
      else
        lds_dma16(v_rsrc, dst, v_src[i], to);
    }
  };

  // ---- LDS operand addressing ----
  // K (A operand of S^T): lane reads row c32 (+32), logical chunk 2c+half.
  uint32_t k_rd[kDChunks];
#pragma unroll
  for (int c = 0; c < kDChunks; ++c)
    k_rd[c] = static_cast<uint32_t>(c32 * L::kRowBytes + (((2 * c + half) ^ swz_k<D>(c32)) * 16));
  // V (A operand of O^T, via ds_read_b64_tr_b16): in 16-lane group g (dgrp = g&1,
  // hh = g>>1) lane t addresses key 8*hh + (t>>2) (+16c + 4s) and dims dsub*32 + 16*dgrp + 4*(t&3).
  const int g16 = lane >> 4;
  const int t16 = lane & 15;
  const int v_key0 = 8 * (g16 >> 1) + (t16 >> 2);  // key within a 16-key chunk, s = 0
  uint32_t v_rd[kDSub];
#pragma unroll
  for (int dsub = 0; dsub < kDSub; ++dsub) {
    const int d = dsub * 32 + 16 * (g16 & 1) + 4 * (t16 & 3);
    v_rd[dsub] = static_cast<uint32_t>(v_key0 * L::kRowBytes + (((d >> 3) ^ swz_v<D>(v_key0)) * 16) + (d & 7) * 2);
  }

  f32x16 oacc[kDSub];
#pragma unroll
  for (int i = 0; i < kDSub; ++i) oacc[i] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;

  auto decode = [&](int e_raw, int& kt, int& flags) {
    const int e = __builtin_amdgcn_readfirstlane(e_raw);
    kt = e >> 2;
    // An entry outside the grid's key tiles [0, n_ktiles) holds no key of the sequence
    // (a 128-token block mask on a sequence that ends in the first half of its last
    // block lists such a tile): it is executed by no wave; its DMA loads a tile in range.
    flags = (kt >= 0 && kt < p.n_ktiles) ? (e & 3) : 0;
    kt = kt < 0 ? 0 : (kt < p.n_ktiles ? kt : p.n_ktiles - 1);
  };
  auto entry = [&](int i) -> int { return kSparse ? list[i] : ((i << 2) | 3); };

  auto qk = [&](const unsigned char* ks, f32x16& s0, f32x16& s1) {
    s0 = f32x16{};
    s1 = f32x16{};
#pragma unroll
    for (int c = 0; c < kDChunks; ++c) {
      const V8 a0 = *reinterpret_cast<const V8*>(ks + k_rd[c]);
      const V8 a1 = *reinterpret_cast<const V8*>(ks + k_rd[c] + 32 * L::kRowBytes);
      s0 = E::mma(a0, qf[c], s0);
      s1 = E::mma(a1, qf[c], s1);
    }
  };
  auto pv = [&](const unsigned char* vs, const V8* pb) {
#pragma unroll
    for (int dsub = 0; dsub < kDSub; ++dsub) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const unsigned char* a = vs + v_rd[dsub] + c * 16 * L::kRowBytes;
        const s16x4 lo = lds_read_tr16(a);
        const s16x4 hi = lds_read_tr16(a + 4 * L::kRowBytes);
        const u32x4 w = {__builtin_bit_cast(u32x2, lo).x, __builtin_bit_cast(u32x2, lo).y,
                         __builtin_bit_cast(u32x2, hi).x, __builtin_bit_cast(u32x2, hi).y};
        oacc[dsub] = E::mma(as_vec8<V8>(w), pb[c], oacc[dsub]);
      }
    }
  };
  auto softmax = [&](f32x16& s0, f32x16& s1, int kt, V8* pb, float& alpha, bool& rescale) {
    if constexpr (kRagged) {
      const int key0 = p.origin + kt * kBN;
      if (key0 < 0 || key0 + kBN > p.kv_len) {
        // element i of s0 is key key0 + 8*half + c, c = 16*(i>>3) + (i&7) (s1: c + 32);
        // comparing the constant c against per-tile bounds keeps no per-element value live
        const int lo = -key0 - 8 * half;           // key >= 0       <=> c >= lo
        const int hi = p.kv_len - key0 - 8 * half; // key < kv_len   <=> c < hi
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int c = (i >> 3) * 16 + (i & 7);
          if (c < lo || c >= hi) s0[i] = -INFINITY;
          if (c + 32 < lo || c + 32 >= hi) s1[i] = -INFINITY;
        }
      }
    }
    float mx = s0[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s0[i]);
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s1[i]);
    mx = max_over_halves(mx);
    const float mxs = mx * p.scale_log2;
    const bool need = mxs > m_run + kRescaleSlack;
    rescale = __ballot(need) != 0ull;
    const float m_new = need ? mxs : m_run;
    // exp2(0) = 1 when the max is kept; fminf drops the NaN of -inf - -inf
    alpha = __builtin_amdgcn_exp2f(__builtin_fminf(m_run - m_new, 0.f));
    m_run = m_new;
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    float rs = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[i], p.scale_log2, -m_use));
      const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[i], p.scale_log2, -m_use));
      rs += e0 + e1;
      pb[i >> 3][i & 7] = static_cast<typename E::elem>(e0);
      pb[2 + (i >> 3)][i & 7] = static_cast<typename E::elem>(e1);
    }
    l_run = l_run * alpha + rs;
  };

  // ---- prologue: K_0, V_0 -> stage 0, K_1 -> K stage 1; S_0 -> P_0 ----
  V8 pb[4];
  bool act_cur = false;
  int e_n1 = 0, e_n2 = 0;
  if (n_iter > 0) {
    const int e0 = entry(0);
    if (n_iter > 1) e_n1 = entry(1);
    if (n_iter > 2) e_n2 = entry(2);
    int kt0, f0;
    decode(e0, kt0, f0);
    dma_k(kt0, 0);
    dma_v(kt0, 0);
    if (n_iter > 1) {
      int kt1, f1;
      decode(e_n1, kt1, f1);
      dma_k(kt1, 1);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    act_cur = (f0 & wbit) != 0;
    if (act_cur) {
      f32x16 s0, s1;
      qk(k_ring, s0, s1);
      float alpha;
      bool rescale;
      softmax(s0, s1, kt0, pb, alpha, rescale);
    }
    __syncthreads();  // K stage 0 is refilled by the first iteration
  }

  // Iteration j: S_{j+1} = K_{j+1} Q^T, O += P_j V_j, P_{j+1} = softmax(S_{j+1}); K_{j+2}
  // and V_{j+1} stream into the stages freed by iteration j-1.
  bool pend = false;
  float pend_alpha = 1.f;
  for (int j = 0; j < n_iter; ++j) {
    const bool has1 = j + 1 < n_iter;
    const bool has2 = j + 2 < n_iter;
    int kt1 = 0, f1 = 0, kt2 = 0, f2 = 0;
    if (has1) decode(e_n1, kt1, f1);
    if (has2) decode(e_n2, kt2, f2);
    int e_n3 = 0;
    if (j + 3 < n_iter) e_n3 = entry(j + 3);
    if (has2) dma_k(kt2, j & 1);
    if (has1) dma_v(kt1, (j + 1) & 1);
    __builtin_amdgcn_sched_barrier(0);

    if (pend) {
#pragma unroll
      for (int dsub = 0; dsub < kDSub; ++dsub) oacc[dsub] *= pend_alpha;
      pend = false;
    }
    const bool act_next = has1 && ((f1 & wbit) != 0);
    const unsigned char* vs = v_ring + (j & 1) * L::kTileBytes;
    const unsigned char* ks1 = k_ring + ((j + 1) & 1) * L::kTileBytes;
    if (act_cur && act_next) {
      f32x16 s0, s1;
      qk(ks1, s0, s1);
      pv(vs, pb);
      V8 pn[4];
      softmax(s0, s1, kt1, pn, pend_alpha, pend);
#pragma unroll
      for (int c = 0; c < 4; ++c) pb[c] = pn[c];
    } else {
      if (act_cur) pv(vs, pb);
      if (act_next) {
        f32x16 s0, s1;
        qk(ks1, s0, s1);
        softmax(s0, s1, kt1, pb, pend_alpha, pend);
      }
    }
    act_cur = act_next;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    e_n1 = e_n2;
    e_n2 = e_n3;
  }
  if (pend) {
#pragma unroll
    for (int dsub = 0; dsub < kDSub; ++dsub) oacc[dsub] *= pend_alpha;
  }

  // ---- epilogue ----
  const float l_tot = sum_over_halves(l_run);
  if (q_row >= 0 && q_row < p.q_len) {
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

  if constexpr (kMap) {
    // ---- fused sparsity map: with this tile's final LSE in registers, sweep the video
    // key tiles again with bf16(q*scale) and count the scores below lse + ln(threshold)
    // (MoD/mod/cuda_flash_sparsity_kernel.cu:82-163). The grid origin puts every video
    // block on this tile's 64/128-row boundaries, so the counts of waves (0,1) / (2,3)
    // (or all four, for 128-blocks) are whole map cells.
    const int vrow_tile = p.origin + qt * kBM - p.map_q_off;  // multiple of 128
    if (vrow_tile + kBM <= 0 || vrow_tile >= p.map_valid) return;  // uniform per workgroup
    const int vrow = vrow_tile + wave * 32 + c32;
    const bool row_ok = vrow >= 0 && vrow < p.map_valid;
    // the LSE exactly as stored above
    const float lse_row = l_tot > 0.f ? (m_run + log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
    const float thr = row_ok ? lse_row + p.map_log_thr : -INFINITY;
    {
      // q scaled in fp32 and rounded to the storage type (reference :86-92)
      const int r = q_row < 0 ? 0 : (q_row < p.q_len ? q_row : p.q_len - 1);
      const u32x4* src = reinterpret_cast<const u32x4*>(qb + r * p.q_ss);
#pragma unroll
      for (int c = 0; c < kDChunks; ++c) {
        const u32x4 raw = src[2 * c + half];
        uint16_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = E::from_float(E::to_float(u16_at(raw, j)) * p.map_scale);
        qf[c] = as_vec8<V8>(u32x4{pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]),
                                  pack2(e[6], e[7])});
      }
    }
    // K-only pass: all four 16 KB stages of the K and V rings form one K ring, filled
    // three tiles ahead; the count ring sits past them.
    int* cnt = reinterpret_cast<int*>(smem + 4 * L::kTileBytes);
    const int n_vt = p.map_nblk * p.map_block / kBN;
    uint16_t* out_bh = p.map + static_cast<int64_t>(bh) * p.map_nblk * p.map_nblk;
    const float inv_area = 1.0f / static_cast<float>(p.map_block * p.map_block);
#pragma unroll
    for (int t = 0; t < 3; ++t)
      if (t < n_vt) dma_k(p.map_kt0 + t, t);
    // Each wave issues kWinPerWave DMAs per K tile (4 at d=128, 2 at d=64), and vector
    // memory operations retire in issue order: tile 0 has landed once at most the two
    // later tiles' DMAs are outstanding.
    static_assert(3 * kWinPerWave < 16, "vmcnt immediate holds at most 15");
    if (n_vt >= 3)
      MODDIT_WAIT_VM_LGKM0(2 * kWinPerWave);
    else
      MODDIT_WAIT_VM_LGKM0(0);
    __syncthreads();
    for (int j = 0; j < n_vt; ++j) {
      // stage (j+3)%4 held tile j-1, read in the previous iteration (barrier since)
      if (j + 3 < n_vt) dma_k(p.map_kt0 + j + 3, (j + 3) & 3);
      __builtin_amdgcn_sched_barrier(0);
      f32x16 s0, s1;
      qk(k_ring + (j & 3) * L::kTileBytes, s0, s1);
      int total = 0;
      if (j * kBN + kBN > p.map_valid) {
        // keys past the sequence end are not counted
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kr = j * kBN + (i >> 3) * 16 + 8 * half + (i & 7);
          total += __builtin_popcountll(__ballot(s0[i] < thr && kr < p.map_valid));
          total += __builtin_popcountll(__ballot(s1[i] < thr && kr + 32 < p.map_valid));
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          total += __builtin_popcountll(__ballot(s0[i] < thr));
          total += __builtin_popcountll(__ballot(s1[i] < thr));
        }
      }
      if (lane == 0) cnt[wave * 2 * kMapFlush + (j % (2 * kMapFlush))] = total;
      // tile j+1 must have landed; the DMAs of tiles j+2 and j+3 (and any map stores,
      // which are younger than tile j+1's DMA) may stay outstanding
      if (j + 3 < n_vt)
        MODDIT_WAIT_VM_LGKM0(2 * kWinPerWave);
      else if (j + 2 < n_vt)
        MODDIT_WAIT_VM_LGKM0(kWinPerWave);
      else
        MODDIT_WAIT_VM_LGKM0(0);
      __syncthreads();
      const int slot_hi = j % kMapFlush;
      if (slot_hi == kMapFlush - 1 || j + 1 == n_vt) {
        const int j0 = j - slot_hi;
        const int hb = ((j / kMapFlush) & 1) * kMapFlush;
        if (p.map_block == 64) {
          if (tid < 2 * kMapFlush) {
            const int qsub = tid / kMapFlush;
            const int sl = tid % kMapFlush;
            const int qblk = vrow_tile / 64 + qsub;
            if (sl <= slot_hi && qblk >= 0 && qblk < p.map_nblk) {
              const int c = cnt[(2 * qsub) * 2 * kMapFlush + hb + sl] +
                            cnt[(2 * qsub + 1) * 2 * kMapFlush + hb + sl];
              out_bh[static_cast<int64_t>(qblk) * p.map_nblk + j0 + sl] =
                  Fp16::from_float(static_cast<float>(c) * inv_area);
            }
          }
        } else {
          if (tid < kMapFlush / 2) {
            const int sl = tid;
            const int qblk = vrow_tile / 128;
            if (2 * sl + 1 <= slot_hi && qblk < p.map_nblk) {
              int c = 0;
#pragma unroll
              for (int w = 0; w < 4; ++w)
                c += cnt[w * 2 * kMapFlush + hb + 2 * sl] + cnt[w * 2 * kMapFlush + hb + 2 * sl + 1];
              out_bh[static_cast<int64_t>(qblk) * p.map_nblk + j0 / 2 + sl] =
                  Fp16::from_float(static_cast<float>(c) * inv_area);
            }
          }
        }
      }
    }
  }
}

template <int D, typename E, bool kSparse, bool kRagged, bool kMap = false>
int launch_attention_impl(const AttnParams& p, int batch, hipStream_t stream) {
  using L = AttnLds<D>;
  auto kernel = attention_fwd_kernel<D, E, kSparse, kRagged, kMap>;
  constexpr int kLds = L::kTotal + (kMap ? kMapCountBytes : 0);
  static LaunchSetup once;
  if (set_dynamic_lds_once(once, reinterpret_cast<const void*>(kernel), kLds) != hipSuccess) {
    set_error("attention: cannot reserve %d bytes of LDS", kLds);
    return MODDIT_EHIP;
  }
  const int64_t tiles = static_cast<int64_t>(batch) * p.heads * p.n_qtiles;
  if (tiles == 0) return MODDIT_OK;
  if (tiles > 0x7fffffff) {
    set_error("attention: too many tiles (%lld)", static_cast<long long>(tiles));
    return MODDIT_EINVAL;
  }
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), kLds, stream, p);
  MODDIT_CHECK_LAUNCH("attention");
  return MODDIT_OK;
}

template <int D, typename E, bool kSparse>
int launch_attention(const AttnParams& p, int batch, hipStream_t stream) {
  // The fused map pass addresses video key tiles that may extend past the last key
  // (partial last block): always the range-checked path.
  if (p.map != nullptr) return launch_attention_impl<D, E, false, true, true>(p, batch, stream);
  // Key counts that are a multiple of the tile (on an unshifted grid) need no clamping
  // or masking at all.
  if (p.kv_len % kBN == 0 && p.origin == 0)
    return launch_attention_impl<D, E, kSparse, false>(p, batch, stream);
  return launch_attention_impl<D, E, kSparse, true>(p, batch, stream);
}

struct MapArgs {
  void* out;
  int q_off;
  int video_blocks;
  int block;
  float log_thr;
};

int attention_entry(const void* q, const void* k, const void* v, void* o, float* lse, int batch,
                    int heads, int q_len, int kv_len, int head_dim, const int64_t* qs,
                    const int64_t* ks, const int64_t* vs, const int64_t* os, float scale,
                    int dtype, const int32_t* counts, const int32_t* entries, int n_qtiles,
                    int cap, int origin, moddit_stream_t stream, const MapArgs* map = nullptr) {
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
  // the fused map pass aligns the grid to 128-row tiles itself
  MODDIT_CHECK_ARG(origin > (map ? -kBM : -kBN) && origin <= 0,
                   "attention: grid_origin must be in (-64, 0], got %d", origin);
  const bool sparse = counts != nullptr;
  const int nq = (q_len - origin + kBM - 1) / kBM;
  if (sparse) {
    MODDIT_CHECK_ARG(entries != nullptr, "attention: tile entries missing");
    MODDIT_CHECK_ARG(n_qtiles == nq, "attention: n_qtiles=%d but q_len=%d (grid origin %d) needs %d",
                     n_qtiles, q_len, origin, nq);
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
  p.origin = origin;
  p.n_qtiles = nq;
  p.n_ktiles = (kv_len - origin + kBN - 1) / kBN;
  p.xcd_run = xcd_run_for(static_cast<int64_t>(kv_len) * head_dim * 2 * 2);  // K and V
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
  p.map = nullptr;
  if (map != nullptr) {
    const int vt = map->video_blocks * map->block;
    p.map = static_cast<uint16_t*>(map->out);
    p.map_q_off = map->q_off;
    p.map_kt0 = (map->q_off - origin) / kBN;
    p.map_nblk = map->video_blocks;
    p.map_block = map->block;
    p.map_valid = vt < q_len - map->q_off ? vt : q_len - map->q_off;
    p.map_scale = scale;
    p.map_log_thr = map->log_thr;
    // largest byte offset a video key tile forms
    const int64_t map_off = (static_cast<int64_t>(map->q_off) - origin + vt) * ks[2] * 2;
    if (map_off > 0x7fffffffLL) {
      set_error("flash_fwd_map: one head's K span exceeds 2 GiB of 32-bit offsets");
      return MODDIT_EUNSUPPORTED;
    }
  }

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
                                 nullptr, nullptr, 0, 0, 0, stream);
}

extern "C" int moddit_flash_fwd_map(const void* q, const void* k, const void* v, void* o,
                                    float* lse, void* map_out, int batch, int heads, int seq_len,
                                    int head_dim, const int64_t q_strides[3],
                                    const int64_t k_strides[3], const int64_t v_strides[3],
                                    const int64_t o_strides[3], float softmax_scale,
                                    float log_threshold, int video_offset, int video_blocks,
                                    int block_size, int dtype, moddit_stream_t stream) {
  using namespace moddit;
  clear_error();
  MODDIT_CHECK_ARG(map_out != nullptr, "flash_fwd_map: map_out must not be NULL");
  MODDIT_CHECK_ARG(block_size == 64 || block_size == 128,
                   "flash_fwd_map: block_size must be 64 or 128, got %d", block_size);
  MODDIT_CHECK_ARG(video_blocks > 0, "flash_fwd_map: video_blocks must be positive");
  MODDIT_CHECK_ARG(video_offset >= 0, "flash_fwd_map: video offset must be non-negative");
  // the last block may be partial, but must hold at least one token
  MODDIT_CHECK_ARG(static_cast<int64_t>(video_offset) + static_cast<int64_t>(video_blocks - 1) * block_size < seq_len,
                   "flash_fwd_map: video region exceeds sequence length");
  MODDIT_CHECK_ARG(!std::isnan(log_threshold), "flash_fwd_map: NaN threshold");
  // grid shifted so that video row 0 starts a 128-row tile
  const int origin = video_offset - ((video_offset + kBM - 1) / kBM) * kBM;
  MapArgs m{map_out, video_offset, video_blocks, block_size, log_threshold};
  return attention_entry(q, k, v, o, lse, batch, heads, seq_len, seq_len, head_dim, q_strides,
                         k_strides, v_strides, o_strides, softmax_scale, dtype, nullptr, nullptr,
                         0, 0, origin, stream, &m);
}

extern "C" int moddit_block_sparse_fwd(const void* q, const void* k, const void* v, void* o,
                                       float* lse, int batch, int heads, int q_len, int kv_len,
                                       int head_dim, const int64_t q_strides[3],
                                       const int64_t k_strides[3], const int64_t v_strides[3],
                                       const int64_t o_strides[3], float softmax_scale, int dtype,
                                       const int32_t* counts, const int32_t* entries,
                                       int n_qtiles, int cap, int grid_origin,
                                       moddit_stream_t stream) {
  if (counts == nullptr) {
    moddit::set_error("block_sparse_fwd: counts must not be NULL");
    return MODDIT_EINVAL;
  }
  return moddit::attention_entry(q, k, v, o, lse, batch, heads, q_len, kv_len, head_dim,
                                 q_strides, k_strides, v_strides, o_strides, softmax_scale, dtype,
                                 counts, entries, n_qtiles, cap, grid_origin, stream);
}
