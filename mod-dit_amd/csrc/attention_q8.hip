// Quantised (int8 Q.K^T, fp8 e4m3 P.V) dense and block-sparse attention forward for
// gfx950, on the output of moddit_quantize_qkv.
//
// Same work decomposition as the bf16 kernels (128 query rows per workgroup of 4 wave64s,
// 64-key tiles, transposed products, per-(head, query tile) key-tile lists with row bits),
// with the operands of the two products at half the width:
//   S^T (64 keys x 32 queries) = K8 . Q8^T     mfma_i32_32x32x32_i8   (D/32 x 2 per tile)
//   O^T (D x 32 queries)      += V8^T . P8^T   mfma_f32_32x32x64 fp8  (D/32 per tile)
// A tile is D bytes per key for K and for V, so a 3-stage ring takes 48 KB of LDS at
// D=128: K tiles are fetched three tiles ahead, V tiles two, each into the stage its
// predecessor three tiles back left free at the previous barrier. 48 KB and 166 VGPRs
// let three workgroups share a CU (three waves per SIMD) in the aligned kernel. The
// ragged kernels convert the scores once and mask boundary tiles in place: 139 VGPRs at
// D=64 (three waves), 199 at D=128 (two; three would spill).
//
// Operand layouts. MFMA products are sums over k, so any assignment of (lane half, byte)
// to k works as long as both operands use the same one; the layouts below are chosen so
// that every operand is a plain 16-byte LDS read:
// - K rows sit in LDS in the order pi(r) = bit2(r)*32 + (r>>3)*4 + (r&3), which makes the
//   int32 S^T accumulator of lane half h hold keys 32h..32h+31 of the tile in order
//   (s0[i] = key 32h+i, s1[i] = key 32h+16+i), exactly the bytes of P8^T it packs into;
// - V is stored transposed (keys contiguous per channel) by the quantisation pass, so the
//   fp8 A operand of lane (d, h) is keys 32h..32h+31 of row d: two 16-byte reads.
// 16-byte chunks are XOR-swizzled per row so that all these reads are bank-conflict free.
//
// Scores: s = int32 * q_scale(row block) * k_scale(key tile); softmax in fp32 as in the
// bf16 kernel (lazy rescale, exp2 with the softmax scale folded in); P = exp2(s - m + 7)
// is rounded to e4m3 (see kPShift) and the row sum uses the fp32 values; O is scaled by
// v_scale[d] / l at the end.
#include "common.h"
#include "lds_dma.h"

namespace moddit {
namespace {

constexpr int kBM = 128;
constexpr int kBN = 64;
constexpr int kThreads = 256;
constexpr int kStages = 3;
// The row max is moved lazily (when a tile's max exceeds it by more than kRescaleSlack
// log2 units) and P is formed as exp2(s - m + kPShift): P <= 2^(kPShift + kRescaleSlack)
// = 2^8.5 stays inside e4m3's range (448) while small probabilities keep kPShift more
// octaves above e4m3's subnormals. The shift cancels between P.V and the row sum.
constexpr float kRescaleSlack = 1.5f;
constexpr float kPShift = 7.0f;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

template <int D>
struct Q8Lds {
  static constexpr int kKRow = D;           // bytes per K row
  static constexpr int kKTile = kBN * D;    // bytes per K tile
  static constexpr int kVRow = kBN;         // bytes per V^T row (64 keys)
  static constexpr int kVTile = D * kBN;    // bytes per V^T tile
  static constexpr int kKWin = kKTile / 1024;  // 1 KB DMA windows per K tile
  static constexpr int kVWin = kVTile / 1024;
  static constexpr int kTotal = kStages * (kKTile + kVTile);
};

struct Q8Params {
  const int8_t* q8;
  const float* q_scale;  // [bh][ceil((S - origin)/32)]: 32-row blocks of the grid
  const int8_t* k8;
  const float* k_scale;  // [bh][n_ktiles]: 64-key tiles of the grid
  const uint8_t* v8t;    // [bh][D][s_pad]: column c = token origin + c
  const float* v_scale;  // [bh][D]
  const float* q_kmean;  // [bh][S]: q . mean_k (LSE correction of the smoothed K)
  uint16_t* o;
  float* lse;
  int64_t o_sb, o_sh, o_ss;
  int heads;
  int seq_len;  // keys (and the quantised tensors' rows)
  int q_len;    // queries: rows 0..q_len-1 (a prefix of the quantised rows)
  int s_pad;
  int origin;
  int n_qtiles;
  int n_ktiles;
  int xcd_run;  // workgroup -> tile order (xcd_remap)
  float scale_log2;
  float scale;
  const int32_t* counts;
  const int32_t* entries;
  int cap;
  uint32_t k_bytes;  // per head: seq_len * D
  uint32_t v_bytes;  // per head: D * s_pad
};

__device__ __forceinline__ int kperm8(int r) { return ((r >> 2) & 1) * 32 + ((r >> 3) << 2) + (r & 3); }

// chunk swizzles: K rows of D bytes (D/16 chunks), V^T rows of 64 bytes (4 chunks)
template <int D>
__device__ __forceinline__ int swz_k8(int r) { return (r / (256 / D)) % (D / 16); }
__device__ __forceinline__ int swz_v8(int r) { return (r >> 2) & 3; }

template <int D, typename E, bool kSparse, bool kRagged>
__global__ __launch_bounds__(kThreads, (kRagged && D == 128) ? 2 : 3) __attribute__((amdgpu_waves_per_eu((kRagged && D == 128) ? 2 : 3, (kRagged && D == 128) ? 2 : 3))) void attention_q8_kernel(Q8Params p) {
  using L = Q8Lds<D>;
  constexpr int kKSteps = D / 32;                // int8 MFMA k-steps over d
  constexpr int kDSub = D / 32;                  // 32-row blocks of O^T
  constexpr int kKWinPerWave = L::kKWin / 4;
  constexpr int kVWinPerWave = L::kVWin / 4;
  constexpr int kKRowsPerWin = 1024 / L::kKRow;
  constexpr int kVRowsPerWin = 1024 / L::kVRow;  // 16

  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* const k_ring = smem;
  unsigned char* const v_ring = smem + kStages * L::kKTile;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int half = lane >> 5;
  const int c32 = lane & 31;

  const int tile = xcd_remap(blockIdx.x, gridDim.x, p.xcd_run);
  const int qt = tile % p.n_qtiles;
  const int bh = tile / p.n_qtiles;
  const int h = bh % p.heads;

  int n_iter;
  const __attribute__((address_space(4))) int32_t* clist = nullptr;
  if (kSparse) {
    const int64_t slot = static_cast<int64_t>(h) * p.n_qtiles + qt;
    n_iter = p.counts[slot];
    n_iter = n_iter < 0 ? 0 : (n_iter < p.cap ? n_iter : p.cap);
    clist = (const __attribute__((address_space(4))) int32_t*)(p.entries + slot * p.cap);
  } else {
    n_iter = p.n_ktiles;
  }
  const int wbit = 1 << (wave >> 1);
  const __attribute__((address_space(4))) float* kscale =
      (const __attribute__((address_space(4))) float*)(p.k_scale + static_cast<int64_t>(bh) * p.n_ktiles);

  // ---- Q8 fragments: lane holds query c32, bytes d = 32c + 16h .. +15 of each k-step;
  // the wave's 32 rows are one quantisation block of the grid ----
  const int q_row = p.origin + qt * kBM + wave * 32 + c32;
  const int q_clamp = q_row < 0 ? 0 : (q_row < p.seq_len ? q_row : p.seq_len - 1);
  i32x4 qf[kKSteps];
  float q_sc;
  {
    const int8_t* src = p.q8 + (static_cast<int64_t>(bh) * p.seq_len + q_clamp) * D;
#pragma unroll
    for (int c = 0; c < kKSteps; ++c)
      qf[c] = *reinterpret_cast<const i32x4*>(src + 32 * c + 16 * half);
    const int nqb = (p.seq_len - p.origin + 31) / 32;
    const int qb = qt * (kBM / 32) + wave;
    q_sc = p.q_scale[static_cast<int64_t>(bh) * nqb + (qb < nqb ? qb : nqb - 1)] * p.scale_log2;
    __builtin_amdgcn_s_waitcnt(0);
  }

  // ---- DMA sources ----
  const int8_t* kbase = p.k8 + static_cast<int64_t>(bh) * p.seq_len * D;
  const uint8_t* vbase = p.v8t + static_cast<int64_t>(bh) * D * p.s_pad;
  const u32x4 k_rsrc = raw_rsrc(kbase, p.k_bytes);
  const u32x4 v_rsrc = raw_rsrc(vbase, p.v_bytes);
  const uint32_t k_lds = lds_addr(k_ring);
  const uint32_t v_lds = lds_addr(v_ring);
  uint32_t k_src[kKWinPerWave];
  uint32_t v_src[kVWinPerWave];
#pragma unroll
  for (int i = 0; i < kKWinPerWave; ++i) {
    const int w = wave * kKWinPerWave + i;
    const int r = w * kKRowsPerWin + (lane * 16) / L::kKRow;
    const int pch = ((lane * 16) % L::kKRow) / 16;
    k_src[i] = static_cast<uint32_t>(kperm8(r) * D + (pch ^ swz_k8<D>(r)) * 16);
  }
#pragma unroll
  for (int i = 0; i < kVWinPerWave; ++i) {
    const int w = wave * kVWinPerWave + i;
    const int r = w * kVRowsPerWin + lane / 4;  // channel d
    const int pch = lane & 3;
    v_src[i] = static_cast<uint32_t>(r * p.s_pad + (pch ^ swz_v8(r)) * 16);
  }
  // origin shift of the K rows (two's complement: keys before token 0 wrap out of range and
  // load as zero); V^T columns are already grid positions
  const uint32_t k_org = static_cast<uint32_t>(p.origin * D);

  auto dma_k = [&](int kt, int stage) {
    const uint32_t to = static_cast<uint32_t>(kt) * static_cast<uint32_t>(L::kKTile);
#pragma unroll
    for (int i = 0; i < kKWinPerWave; ++i) {
      const uint32_t dst = k_lds + stage * L::kKTile + (wave * kKWinPerWave + i) * 1024;
      if constexpr (kRagged)
        lds_dma16(k_rsrc, dst, k_src[i] + to + k_org, 0);
      else
        lds_dma16(k_rsrc, dst, k_src[i], to);
    }
  };
  auto dma_v = [&](int kt, int stage) {
    const uint32_t to = static_cast<uint32_t>(kt) * kBN;
#pragma unroll
    for (int i = 0; i < kVWinPerWave; ++i) {
      const uint32_t dst = v_lds + stage * L::kVTile + (wave * kVWinPerWave + i) * 1024;
      lds_dma16(v_rsrc, dst, v_src[i], to);
    }
  };

  // ---- LDS operand addressing ----
  uint32_t k_rd[kKSteps];
#pragma unroll
  for (int c = 0; c < kKSteps; ++c)
    k_rd[c] = static_cast<uint32_t>(c32 * L::kKRow + (((2 * c + half) ^ swz_k8<D>(c32)) * 16));
  uint32_t v_rd[kDSub][2];
#pragma unroll
  for (int ds = 0; ds < kDSub; ++ds) {
    const int r = ds * 32 + c32;
#pragma unroll
    for (int t = 0; t < 2; ++t)
      v_rd[ds][t] = static_cast<uint32_t>(r * L::kVRow + (((2 * half + t) ^ swz_v8(r)) * 16));
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
  auto entry = [&](int i) -> int { return kSparse ? clist[i] : ((i << 2) | 3); };

  auto qk = [&](const unsigned char* ks, i32x16& s0, i32x16& s1) {
    s0 = i32x16{};
    s1 = i32x16{};
#pragma unroll
    for (int c = 0; c < kKSteps; ++c) {
      const i32x4 a0 = *reinterpret_cast<const i32x4*>(ks + k_rd[c]);
      const i32x4 a1 = *reinterpret_cast<const i32x4*>(ks + k_rd[c] + 32 * L::kKRow);
      s0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, qf[c], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, qf[c], s1, 0, 0, 0);
    }
  };
  auto pv = [&](const unsigned char* vs, const i32x8& pb) {
#pragma unroll
    for (int ds = 0; ds < kDSub; ++ds) {
      const i32x4 lo = *reinterpret_cast<const i32x4*>(vs + v_rd[ds][0]);
      const i32x4 hi = *reinterpret_cast<const i32x4*>(vs + v_rd[ds][1]);
      const i32x8 a = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      oacc[ds] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, pb, oacc[ds], 0, 0, 0, 127,
                                                                  0, 127);
    }
  };
  // scores of key tile kt: s = int32 * q_scale * k_scale[kt], in log2 units (the softmax
  // scale is folded into q_sc)
  auto softmax = [&](const i32x16& s0, const i32x16& s1, int kt, i32x8& pb, float& alpha,
                     bool& rescale) {
    const int key0 = p.origin + kt * kBN;
    float f0[16], f1[16];
    float mx;
    bool general = false;
    // tiles wholly inside the sequence share one K scale on any grid (the quantiser's
    // blocks lie on the attention grid), so only tiles that cross 0 or seq_len need masking
    if constexpr (kRagged) general = key0 < 0 || key0 + kBN > p.seq_len;
    const float sc = kscale[kt] * q_sc;  // one K scale per tile on any grid, q_sc > 0
    if constexpr (!kRagged) {
      // every tile inside the sequence: max over the raw integer scores
      int mi = s0[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mi = max(mi, s0[i]);
#pragma unroll
      for (int i = 0; i < 16; ++i) mi = max(mi, s1[i]);
      // exchanged as an integer: the conversion and the scale (sc > 0) are monotone, so
      // this is the max of the scaled halves, without the float max's NaN canonicalising
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(mi, mi, false, false);
        mi = max(static_cast<int>(sw[0]), static_cast<int>(sw[1]));
      }
      mx = static_cast<float>(mi) * sc;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        f0[i] = static_cast<float>(s0[i]);
        f1[i] = static_cast<float>(s1[i]);
      }
      const bool need = mx > m_run + kRescaleSlack;
      rescale = __ballot(need) != 0ull;
      const float m_new = need ? mx : m_run;
      alpha = __builtin_amdgcn_exp2f(__builtin_fminf(m_run - m_new, 0.f));
      m_run = m_new;
      const float m_sh = m_new - kPShift;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        f0[i] = __builtin_fmaf(f0[i], sc, -m_sh);
        f1[i] = __builtin_fmaf(f1[i], sc, -m_sh);
      }
    } else {
      // ragged grids: the scores are converted once and, on tiles that cross 0 or
      // seq_len, masked in place, so both paths share the same registers
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        f0[i] = static_cast<float>(s0[i]);
        f1[i] = static_cast<float>(s1[i]);
      }
      if (general) {
        // keys outside [0, seq_len) are padding of the grid: masked in place. Element i of
        // f0 is key key0 + 32*half + i (f1: + 16); comparing the constant i with per-tile
        // bounds keeps no per-element value live across the loop.
        const int lo = -key0 - 32 * half;            // key >= 0       <=> i >= lo
        const int hi = p.seq_len - key0 - 32 * half; // key < seq_len  <=> i < hi
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (i < lo || i >= hi) f0[i] = -INFINITY;
          if (i + 16 < lo || i + 16 >= hi) f1[i] = -INFINITY;
        }
        float mr = f0[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) mr = fmaxf(mr, f0[i]);
#pragma unroll
        for (int i = 0; i < 16; ++i) mr = fmaxf(mr, f1[i]);
        mx = mr * sc;
      } else {
        // whole tile inside the sequence: max over the raw integer scores
        int mi = s0[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) mi = max(mi, s0[i]);
#pragma unroll
        for (int i = 0; i < 16; ++i) mi = max(mi, s1[i]);
        mx = static_cast<float>(mi) * sc;
      }
      mx = max_over_halves(mx);
      const bool need = mx > m_run + kRescaleSlack;
      rescale = __ballot(need) != 0ull;
      const float m_new = need ? mx : m_run;
      // exp2(0) = 1 when the max is kept; fminf drops the NaN of -inf - -inf
      alpha = __builtin_amdgcn_exp2f(__builtin_fminf(m_run - m_new, 0.f));
      m_run = m_new;
      // a row whose keys so far are all masked keeps m = -inf: shift by 0 (P = 0 anyway)
      const float m_sh = ((m_new == -INFINITY) ? 0.f : m_new) - kPShift;
#pragma unroll
      for (int i = 0; i < 16; ++i) {  // -inf * sc - m_sh stays -inf (sc > 0)
        f0[i] = __builtin_fmaf(f0[i], sc, -m_sh);
        f1[i] = __builtin_fmaf(f1[i], sc, -m_sh);
      }
    }
    float rs = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float a0 = __builtin_amdgcn_exp2f(f0[4 * w]);
      const float a1 = __builtin_amdgcn_exp2f(f0[4 * w + 1]);
      const float a2 = __builtin_amdgcn_exp2f(f0[4 * w + 2]);
      const float a3 = __builtin_amdgcn_exp2f(f0[4 * w + 3]);
      const float b0 = __builtin_amdgcn_exp2f(f1[4 * w]);
      const float b1 = __builtin_amdgcn_exp2f(f1[4 * w + 1]);
      const float b2 = __builtin_amdgcn_exp2f(f1[4 * w + 2]);
      const float b3 = __builtin_amdgcn_exp2f(f1[4 * w + 3]);
      rs += ((a0 + a1) + (a2 + a3)) + ((b0 + b1) + (b2 + b3));
      // each packing writes one half of the word; the previous tile's P word (dead once
      // its P.V MFMA has issued) supplies the other half, so no register is zeroed first
      int wa = __builtin_amdgcn_cvt_pk_fp8_f32(a0, a1, pb[w], false);
      wa = __builtin_amdgcn_cvt_pk_fp8_f32(a2, a3, wa, true);
      int wb = __builtin_amdgcn_cvt_pk_fp8_f32(b0, b1, pb[4 + w], false);
      wb = __builtin_amdgcn_cvt_pk_fp8_f32(b2, b3, wb, true);
      pb[w] = wa;
      pb[4 + w] = wb;
    }
    l_run = l_run * alpha + rs;
  };

  // ---- prologue: K_0..K_2 -> K stages 0..2, V_0, V_1 -> V stages 0, 1; S_0 -> P_0 ----
  i32x8 pb = i32x8{};
  bool act_cur = false;
  int e_n1 = 0, e_n2 = 0, e_n3 = 0;
  if (n_iter > 0) {
    const int e0 = entry(0);
    if (n_iter > 1) e_n1 = entry(1);
    if (n_iter > 2) e_n2 = entry(2);
    if (n_iter > 3) e_n3 = entry(3);
    int kt0, f0;
    decode(e0, kt0, f0);
    dma_k(kt0, 0);
    dma_v(kt0, 0);
    if (n_iter > 1) {
      int kt1, f1;
      decode(e_n1, kt1, f1);
      dma_k(kt1, 1);
      dma_v(kt1, 1);
    }
    if (n_iter > 2) {
      int kt2, f2;
      decode(e_n2, kt2, f2);
      dma_k(kt2, 2);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    act_cur = (f0 & wbit) != 0;
    if (act_cur) {
      i32x16 s0, s1;
      qk(k_ring, s0, s1);
      float alpha;
      bool rescale;
      softmax(s0, s1, kt0, pb, alpha, rescale);
    }
    __syncthreads();  // K stage 0 is refilled by the first iteration
  }

  // Iteration j: S_{j+1} = K_{j+1} Q^T, O += P_j V_j, P_{j+1} = softmax(S_{j+1}); K_{j+3}
  // and V_{j+2} stream into the stages of K_j and V_{j-1}, which the previous iteration
  // finished reading before its closing barrier (each wave retires its LDS reads first).
  bool pend = false;
  float pend_alpha = 1.f;
  int st0 = 0, st1 = 1, st2 = 2;  // ring stages of tiles j, j+1, j+2; tile j+3 reuses st0
  for (int j = 0; j < n_iter; ++j) {
    const bool has1 = j + 1 < n_iter;
    const bool has2 = j + 2 < n_iter;
    const bool has3 = j + 3 < n_iter;
    int kt1 = 0, f1 = 0, kt2 = 0, f2 = 0, kt3 = 0, f3 = 0;
    if (has1) decode(e_n1, kt1, f1);
    if (has2) decode(e_n2, kt2, f2);
    if (has3) decode(e_n3, kt3, f3);
    int e_n4 = 0;
    if (j + 4 < n_iter) e_n4 = entry(j + 4);
    if (has3) dma_k(kt3, st0);
    if (has2) dma_v(kt2, st2);
    __builtin_amdgcn_sched_barrier(0);

    if (pend) {
#pragma unroll
      for (int ds = 0; ds < kDSub; ++ds) oacc[ds] *= pend_alpha;
      pend = false;
    }
    const bool act_next = has1 && ((f1 & wbit) != 0);
    const unsigned char* vs = v_ring + st0 * L::kVTile;
    const unsigned char* ks1 = k_ring + st1 * L::kKTile;
    if (act_cur && act_next) {
      i32x16 s0, s1;
      qk(ks1, s0, s1);
      pv(vs, pb);
      softmax(s0, s1, kt1, pb, pend_alpha, pend);  // P_{j+1} overwrites P_j after its MFMAs
    } else {
      if (act_cur) pv(vs, pb);
      if (act_next) {
        i32x16 s0, s1;
        qk(ks1, s0, s1);
        softmax(s0, s1, kt1, pb, pend_alpha, pend);
      }
    }
    act_cur = act_next;
    // K_{j+2} and V_{j+1} (issued one iteration ago) must have landed; this iteration's
    // DMAs may stay in flight (vector loads retire in issue order)
    if (has3 && has2)
      MODDIT_WAIT_VM_LGKM0(kKWinPerWave + kVWinPerWave);
    else if (has2)
      MODDIT_WAIT_VM_LGKM0(kVWinPerWave);
    else
      MODDIT_WAIT_VM_LGKM0(0);
    __syncthreads();
    e_n1 = e_n2;
    e_n2 = e_n3;
    e_n3 = e_n4;
    const int freed = st0;
    st0 = st1;
    st1 = st2;
    st2 = freed;
  }
  if (pend) {
#pragma unroll
    for (int ds = 0; ds < kDSub; ++ds) oacc[ds] *= pend_alpha;
  }

  // ---- epilogue: O = O^T * v_scale[d] / l ----
  const float l_tot = sum_over_halves(l_run);
  if (q_row >= 0 && q_row < p.q_len) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const float* vsc = p.v_scale + static_cast<int64_t>(bh) * D;
    const int b = bh / p.heads;
    uint16_t* orow = p.o + b * p.o_sb + h * p.o_sh + q_row * p.o_ss;
#pragma unroll
    for (int ds = 0; ds < kDSub; ++ds) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = ds * 32 + 8 * g + 4 * half;
        const f32x4 sv = *reinterpret_cast<const f32x4*>(vsc + d);
        u32x2 w;
        w.x = pack2(E::from_float(oacc[ds][4 * g + 0] * (sv[0] * inv)),
                    E::from_float(oacc[ds][4 * g + 1] * (sv[1] * inv)));
        w.y = pack2(E::from_float(oacc[ds][4 * g + 2] * (sv[2] * inv)),
                    E::from_float(oacc[ds][4 * g + 3] * (sv[3] * inv)));
        *reinterpret_cast<u32x2*>(orow + d) = w;
      }
    }
    if (p.lse != nullptr && half == 0) {
      // LSE of the unsmoothed scores: + scale * q . mean_k
      const int64_t li = static_cast<int64_t>(bh) * p.q_len + q_row;
      const float corr = p.q_kmean[static_cast<int64_t>(bh) * p.seq_len + q_row];
      p.lse[li] = l_tot > 0.f ? __builtin_fmaf(m_run - kPShift + log2f(l_tot), 0.69314718055994531f,
                                               p.scale * corr)
                              : -INFINITY;
    }
  }
}

template <int D, typename E, bool kSparse, bool kRagged>
int launch_q8_impl(const Q8Params& p, int batch, hipStream_t stream) {
  using L = Q8Lds<D>;
  auto kernel = attention_q8_kernel<D, E, kSparse, kRagged>;
  static LaunchSetup once;
  if (set_dynamic_lds_once(once, reinterpret_cast<const void*>(kernel), L::kTotal) != hipSuccess) {
    set_error("attention_q8: cannot reserve %d bytes of LDS", L::kTotal);
    return MODDIT_EHIP;
  }
  const int64_t tiles = static_cast<int64_t>(batch) * p.heads * p.n_qtiles;
  if (tiles == 0) return MODDIT_OK;
  if (tiles > 0x7fffffff) {
    set_error("attention_q8: too many tiles");
    return MODDIT_EINVAL;
  }
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), L::kTotal,
                     stream, p);
  MODDIT_CHECK_LAUNCH("attention_q8");
  return MODDIT_OK;
}

template <int D, typename E, bool kSparse>
int launch_q8(const Q8Params& p, int batch, hipStream_t stream) {
  if (p.seq_len % kBN == 0 && p.origin == 0)
    return launch_q8_impl<D, E, kSparse, false>(p, batch, stream);
  return launch_q8_impl<D, E, kSparse, true>(p, batch, stream);
}

int q8_entry(const int8_t* q8, const float* q_scale, const int8_t* k8, const float* k_scale,
             const uint8_t* v8t, const float* v_scale, const float* q_kmean, void* o, float* lse,
             int batch,
             int heads, int seq_len, int q_len, int head_dim, const int64_t* os, float scale,
             int dtype,
             const int32_t* counts, const int32_t* entries, int n_qtiles, int cap, int origin,
             moddit_stream_t stream) {
  clear_error();
  MODDIT_CHECK_ARG(q8 && q_scale && k8 && k_scale && v8t && v_scale && o && os,
                   "attention_q8: null pointer argument");
  MODDIT_CHECK_ARG(lse == nullptr || q_kmean != nullptr,
                   "attention_q8: the LSE needs q_kmean (the quantiser's q . mean_k)");
  MODDIT_CHECK_ARG(scale > 0.f && std::isfinite(scale), "attention_q8: softmax_scale must be positive");
  MODDIT_CHECK_ARG(batch >= 0 && heads >= 0 && seq_len >= 0, "attention_q8: negative size");
  MODDIT_CHECK_ARG(q_len >= 0 && q_len <= seq_len,
                   "attention_q8: q_len=%d must lie in [0, seq_len=%d]", q_len, seq_len);
  if (head_dim != 64 && head_dim != 128) {
    set_error("attention_q8: head_dim must be 64 or 128, got %d", head_dim);
    return MODDIT_EUNSUPPORTED;
  }
  if (dtype != MODDIT_BF16 && dtype != MODDIT_FP16) {
    set_error("attention_q8: output dtype must be bf16 or fp16");
    return MODDIT_EUNSUPPORTED;
  }
  MODDIT_CHECK_ARG(origin > -kBN && origin <= 0, "attention_q8: grid_origin must be in (-64, 0], got %d", origin);
  MODDIT_CHECK_ARG(aligned16(q8) && aligned16(k8) && aligned16(v8t) && aligned16(o) &&
                       aligned16(v_scale),
                   "attention_q8: tensors must be 16-byte aligned");
  for (int j = 0; j < 3; ++j)
    MODDIT_CHECK_ARG(os[j] >= 0 && os[j] % 8 == 0,
                     "attention_q8: output strides must be non-negative multiples of 8");
  const bool sparse = counts != nullptr;
  const int nq = (q_len - origin + kBM - 1) / kBM;
  if (sparse) {
    MODDIT_CHECK_ARG(entries != nullptr, "attention_q8: tile entries missing");
    MODDIT_CHECK_ARG(n_qtiles == nq, "attention_q8: n_qtiles=%d but the sequence needs %d",
                     n_qtiles, nq);
    MODDIT_CHECK_ARG(cap > 0, "attention_q8: cap must be positive");
  }
  if (q_len == 0 || batch == 0 || heads == 0) return MODDIT_OK;
  Q8Params p;
  p.q8 = q8;
  p.q_scale = q_scale;
  p.k8 = k8;
  p.k_scale = k_scale;
  p.v8t = v8t;
  p.v_scale = v_scale;
  p.q_kmean = q_kmean;
  p.o = static_cast<uint16_t*>(o);
  p.lse = lse;
  p.o_sb = os[0]; p.o_sh = os[1]; p.o_ss = os[2];
  p.heads = heads;
  p.seq_len = seq_len;
  p.q_len = q_len;
  p.s_pad = (seq_len - origin + kBN - 1) / kBN * kBN;
  p.origin = origin;
  p.n_qtiles = nq;
  p.n_ktiles = (seq_len - origin + kBN - 1) / kBN;
  p.xcd_run = xcd_run_for(static_cast<int64_t>(seq_len) * head_dim * 2);  // int8 K, fp8 V
  p.scale_log2 = scale * 1.4426950408889634f;
  p.scale = scale;
  p.counts = counts;
  p.entries = entries;
  p.cap = cap;
  const int64_t kb = static_cast<int64_t>(seq_len) * head_dim;
  const int64_t vb = static_cast<int64_t>(head_dim) * p.s_pad;
  if (kb > 0x7fffffffLL || vb > 0x7fffffffLL ||
      static_cast<int64_t>(p.n_ktiles) * kBN * head_dim > 0x7fffffffLL) {
    set_error("attention_q8: one head's K/V exceeds 2 GiB of 32-bit offsets");
    return MODDIT_EUNSUPPORTED;
  }
  p.k_bytes = static_cast<uint32_t>(kb);
  p.v_bytes = static_cast<uint32_t>(vb);
  hipStream_t st = as_stream(stream);
  const bool bf = dtype == MODDIT_BF16;
  if (head_dim == 128) {
    if (bf) return sparse ? launch_q8<128, Bf16, true>(p, batch, st) : launch_q8<128, Bf16, false>(p, batch, st);
    return sparse ? launch_q8<128, Fp16, true>(p, batch, st) : launch_q8<128, Fp16, false>(p, batch, st);
  }
  if (bf) return sparse ? launch_q8<64, Bf16, true>(p, batch, st) : launch_q8<64, Bf16, false>(p, batch, st);
  return sparse ? launch_q8<64, Fp16, true>(p, batch, st) : launch_q8<64, Fp16, false>(p, batch, st);
}

}  // namespace
}  // namespace moddit

extern "C" int moddit_flash_fwd_q8(const int8_t* q8, const float* q_scale, const int8_t* k8,
                                   const float* k_scale, const uint8_t* v8t,
                                   const float* v_scale, const float* q_kmean, void* o,
                                   float* lse, int batch, int heads, int seq_len, int head_dim,
                                   const int64_t o_strides[3], float softmax_scale, int dtype,
                                   moddit_stream_t stream) {
  return moddit::q8_entry(q8, q_scale, k8, k_scale, v8t, v_scale, q_kmean, o, lse, batch, heads, seq_len,
                          seq_len, head_dim, o_strides, softmax_scale, dtype, nullptr, nullptr, 0,
                          0, 0, stream);
}

extern "C" int moddit_block_sparse_fwd_q8(const int8_t* q8, const float* q_scale,
                                          const int8_t* k8, const float* k_scale,
                                          const uint8_t* v8t, const float* v_scale,
                                          const float* q_kmean, void* o, float* lse, int batch,
                                          int heads, int seq_len, int q_len, int head_dim, const int64_t o_strides[3],
                                          float softmax_scale, int dtype, const int32_t* counts,
                                          const int32_t* entries, int n_qtiles, int cap,
                                          int grid_origin, moddit_stream_t stream) {
  if (counts == nullptr) {
    moddit::set_error("block_sparse_fwd_q8: counts must not be NULL");
    return MODDIT_EINVAL;
  }
  return moddit::q8_entry(q8, q_scale, k8, k_scale, v8t, v_scale, q_kmean, o, lse, batch, heads, seq_len,
                          q_len, head_dim, o_strides, softmax_scale, dtype, counts, entries,
                          n_qtiles, cap, grid_origin, stream);
}
