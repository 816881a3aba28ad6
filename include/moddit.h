/*
 * moddit.h — C ABI of the MI355X (gfx950) MOD-DiT sparse-attention hot path.
 *
 * Every entry point:
 *   - takes raw device pointers, sizes and element strides (no framework types);
 *   - launches on the caller's HIP stream (passed as an opaque pointer, NULL means
 *     the null stream) and never synchronises the device;
 *   - returns MODDIT_OK (0) or a nonzero status; moddit_last_error() then returns a
 *     thread-local message describing the failure;
 *   - writes only into caller-allocated outputs, except where a workspace is named.
 *
 * Element strides are in elements, not bytes. Attention tensors are addressed as
 * [batch][head][token][dim] with an arbitrary (batch, head, token) stride triple and a
 * unit dim stride, which covers both contiguous (B,H,S,D) tensors and (B,S,H,D)
 * storage viewed as (B,H,S,D).
 *
 * Each declaration names the reference interface it replaces (path:line inside the
 * MOD-DiT source tree).
 */
#ifndef MODDIT_H_
#define MODDIT_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* moddit_stream_t; /* a hipStream_t */

enum moddit_status {
  MODDIT_OK = 0,
  MODDIT_EINVAL = 1,      /* invalid argument (shape, stride, alignment, range) */
  MODDIT_EUNSUPPORTED = 2,/* valid but unsupported combination (dtype, head_dim)   */
  MODDIT_EHIP = 3         /* a HIP runtime call failed                            */
};

enum moddit_dtype { MODDIT_BF16 = 0, MODDIT_FP16 = 1, MODDIT_FP32 = 2 };

/* Per-head mask mode, the reference's 'sparse' / 'block_diagonal' / 'full' strings. */
enum moddit_head_mode { MODDIT_MODE_SPARSE = 0, MODDIT_MODE_BLOCK_DIAGONAL = 1, MODDIT_MODE_FULL = 2 };

/* Token layouts of MoD/mod/triton_flash_sparsity.py:101-120 and attn_mask.py:541-557. */
enum moddit_layout { MODDIT_LAYOUT_WAN = 0, MODDIT_LAYOUT_HUNYUAN = 1, MODDIT_LAYOUT_COGVIDEOX = 2, MODDIT_LAYOUT_OTHER = 3 };

/* Thread-local text of the last failure on this thread ("" if none). */
const char* moddit_last_error(void);

/* Library version string. */
const char* moddit_version(void);

/*
 * Dense attention forward with a natural-log LSE output.
 *   O[b,h,r,:] = softmax_r(scale * Q[b,h,r,:] . K[b,h,c,:]) over c < kv_len, then . V
 *   LSE[b,h,r] = log(sum_c exp(scale * q.k))   (fp32, contiguous (B,H,S); may be NULL)
 * q/k/v/o: dtype elements, head_dim D in {64,128}; q_len rows of Q/O, kv_len rows of K/V.
 * Replaces flash_attn_func (MoD/mod/triton_flash_sparsity.py:320-321), sageattn
 * (MoD/mod/attn_mask.py:271-276), flashinfer.single_prefill_with_kv_cache
 * (attn_mask.py:283-289) and the processors' F.scaled_dot_product_attention
 * (MoD/models/hunyuan/attention_processor.py:122-124).
 */
int moddit_flash_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                     int batch, int heads, int q_len, int kv_len, int head_dim,
                     const int64_t q_strides[3], const int64_t k_strides[3],
                     const int64_t v_strides[3], const int64_t o_strides[3],
                     float softmax_scale, int dtype, moddit_stream_t stream);

/*
 * Block-sparse attention forward. Query rows are grouped in tiles of 128 (two
 * 64-row query blocks) and keys in tiles of 64. For head h and query tile t the
 * active key tiles are entries[(h*n_qtiles + t)*cap + i], i < counts[h*n_qtiles + t],
 * in ascending order, each encoded as (key_tile << 2) | rows, where bit 0 enables
 * the tile for query rows 0..63 of the query tile and bit 1 for rows 64..127.
 * Rows with no active key tile produce zeros and LSE = -inf.
 * The tiles live on a grid whose row/column 0 is token grid_origin (-63..0): query
 * tile t covers tokens grid_origin + 128t .. +127 and key tile j tokens
 * grid_origin + 64j .. +63. Grid positions outside [0, q_len) / [0, kv_len) are
 * padding: such keys are masked out and such query rows are not written. A negative
 * origin lets text-first sequences whose text is not block-aligned (CogVideoX: 226 text
 * tokens) start both text and video on block boundaries without copying; the
 * reference rejects such shapes (MoD/mod/triton_flash_sparsity.py:157-160). A grid of
 * 128-token blocks starting 64..127 tokens early is the 64-token grid 64 tokens later
 * whose first tile row and column are padding: pass that grid, with rows kept per
 * 64-row half. Entries naming a key tile outside [0, ceil((kv_len - grid_origin)/64))
 * hold no keys and are skipped.
 * n_qtiles must equal ceil((q_len - grid_origin) / 128).
 * Replaces block_sparse_sage2_attn_cuda (MoD/mod/attn_mask.py:306,312-317) as driven
 * by AttentionSparseEngine (attn_mask.py:266-331).
 */
int moddit_block_sparse_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                            int batch, int heads, int q_len, int kv_len, int head_dim,
                            const int64_t q_strides[3], const int64_t k_strides[3],
                            const int64_t v_strides[3], const int64_t o_strides[3],
                            float softmax_scale, int dtype,
                            const int32_t* counts, const int32_t* entries, int n_qtiles, int cap,
                            int grid_origin, moddit_stream_t stream);

/*
 * Dense attention and the replayed sparsity map in one kernel: every workgroup runs
 * the dense pass of moddit_flash_fwd for its 128 query rows (O, and LSE when lse is not
 * NULL), then, with the rows' final LSE still in registers, sweeps the video key tiles
 * again and writes the map cells of moddit_sparsity_map for those rows (same counts,
 * same fp16 rounding, same partial-last-block rule). Self-attention: q_len = kv_len =
 * seq_len, and the video region starts at video_offset for queries and keys alike.
 * Replaces the two passes of flash_attn_with_sparsity_map
 * (MoD/mod/triton_flash_sparsity.py:274-341: flash_attn_func, then sparsity_map).
 */
int moddit_flash_fwd_map(const void* q, const void* k, const void* v, void* o, float* lse,
                         void* map_out, int batch, int heads, int seq_len, int head_dim,
                         const int64_t q_strides[3], const int64_t k_strides[3],
                         const int64_t v_strides[3], const int64_t o_strides[3],
                         float softmax_scale, float log_threshold, int video_offset,
                         int video_blocks, int block_size, int dtype, moddit_stream_t stream);

/*
 * Quantisation pass of the int8/fp8 attention path (SageAttention2-style: int8 Q.K^T,
 * fp8 e4m3 P.V), for self-attention q/k/v of shape (B,H,S,D), D in {64,128}.
 * Blocks and tiles lie on the attention grid that starts at token grid_origin (-63..0, the
 * grid_origin later given to moddit_block_sparse_fwd_q8; 0 for the dense kernel): grid
 * position c is token grid_origin + c, tokens outside [0,S) count as zero, G = S - grid_origin.
 *   q8[bh][s][d]  = rne(q * 127/amax_q), amax_q over each 32-position block of the grid
 *   k8[bh][s][d]  = rne((k - k_mean[bh][d]) * 127/amax_k), amax_k over each 64-position
 *                   tile, k_mean = per-channel mean over the sequence
 *   v8t[bh][d][c] = e4m3_rne(v[grid_origin + c] * 448/amax_v[d]), amax_v per channel over
 *                   the sequence; grid positions contiguous, s_pad = ceil(G/64)*64 columns,
 *                   zero outside the sequence
 *   q_scale [bh][ceil(G/32)] = amax_q/127, k_scale [bh][ceil(G/64)] = amax_k/127,
 *   v_scale [bh][D] = amax_v/448 (each 1 where the amax is 0), k_mean [bh][D],
 *   q_kmean [bh][S] = q . k_mean in fp32 (the attention kernels add softmax_scale times it
 *                     to the LSE, which then is that of the unsmoothed scores).
 * workspace: moddit_quantize_workspace_floats(B,H,D) floats (deterministic partial
 * column statistics; contents are scratch). All buffers are caller-allocated.
 * No counterpart call in the reference: its quantised engine, block_sparse_sage2_attn_cuda
 * (MoD/mod/attn_mask.py:306), quantises internally (third-party, not in the tree).
 */
int moddit_quantize_qkv(const void* q, const void* k, const void* v, int batch, int heads,
                        int seq_len, int head_dim, const int64_t q_strides[3],
                        const int64_t k_strides[3], const int64_t v_strides[3], int dtype,
                        int grid_origin, float* workspace, int8_t* q8, float* q_scale,
                        int8_t* k8, float* k_scale, uint8_t* v8t, float* v_scale,
                        float* k_mean, float* q_kmean, moddit_stream_t stream);
int moddit_quantize_workspace_floats(int batch, int heads, int head_dim);

/*
 * Attention on the output of moddit_quantize_qkv: scores from the int8 product times
 * q_scale * k_scale, fp32 online softmax, P rounded to e4m3 for the fp8 P.V product,
 * O = (P.V8) * v_scale[d] / rowsum written as dtype (bf16/fp16) with the given strides,
 * natural-log LSE (may be NULL; needs q_kmean when not). moddit_block_sparse_fwd_q8 takes
 * the tile lists and grid origin of moddit_block_sparse_fwd (the quantisation must have
 * used the same grid_origin; the dense kernel: 0), and q_len <= seq_len: queries
 * 0..q_len-1 attend to all seq_len keys (the reference's video-query prefix against the
 * full key set, attn_mask.py:312-317); o and lse hold q_len rows, n_qtiles covers them.
 * Replaces block_sparse_sage2_attn_cuda (MoD/mod/attn_mask.py:306,312-317) and sageattn
 * (attn_mask.py:271-276) with their own quantised arithmetic (parity unpinned against
 * them; pinned against exact attention on the dequantised inputs).
 */
int moddit_flash_fwd_q8(const int8_t* q8, const float* q_scale, const int8_t* k8,
                        const float* k_scale, const uint8_t* v8t, const float* v_scale,
                        const float* q_kmean, void* o, float* lse, int batch, int heads,
                        int seq_len, int head_dim, const int64_t o_strides[3],
                        float softmax_scale, int dtype, moddit_stream_t stream);
int moddit_block_sparse_fwd_q8(const int8_t* q8, const float* q_scale, const int8_t* k8,
                               const float* k_scale, const uint8_t* v8t, const float* v_scale,
                               const float* q_kmean, void* o, float* lse, int batch, int heads,
                               int seq_len, int q_len, int head_dim, const int64_t o_strides[3],
                               float softmax_scale, int dtype, const int32_t* counts,
                               const int32_t* entries, int n_qtiles, int cap, int grid_origin,
                               moddit_stream_t stream);

/*
 * Replayed block sparsity map (video x video blocks), fp16 output (B,H,n,n):
 *   map[b,h,i,j] = fp16_rn( #{(r,c) in block (i,j) :
 *                   fp32(sum_d round(q[r,d]*scale) * k[c,d]) < lse[r] + log_threshold}
 *                   / block_size^2 )
 * where round() is round-to-nearest-even to the input dtype and r, c are offset by
 * q_video_offset / k_video_offset. log_threshold = -inf gives an all-zero map.
 * lse: fp32 contiguous (B,H,S). block_size in {64,128}.
 * The last block may extend past the sequence end (offset + (n-1)*block_size < seq_len):
 * rows and keys at or beyond seq_len are not counted; the cell is still normalised by
 * block_size^2. The reference requires whole blocks (cuda_flash_sparsity_kernel.cu:283).
 * Replaces the pybind `sparsity_map` (MoD/mod/cuda_flash_sparsity_kernel.cu:289-334)
 * and the Triton `_sparsity_kernel` (MoD/mod/triton_flash_sparsity.py:28-98).
 */
int moddit_sparsity_map(const void* q, const void* k, const float* lse, void* map_out,
                        int batch, int heads, int seq_len, int head_dim,
                        const int64_t q_strides[3], const int64_t k_strides[3],
                        float softmax_scale, float log_threshold,
                        int q_video_offset, int k_video_offset, int video_blocks, int block_size,
                        int dtype, moddit_stream_t stream);

/*
 * The refresh step's map update in one pass: the cells of moddit_sparsity_map listed in
 * tile lists (counts, entries: the moddit_mask_to_tiles format with exact rows, over the
 * video x video block mask: n_qtiles = ceil(video_blocks * block_size / 128) query tiles
 * of 128 rows, entries key_tile << 2 | row bits; with block_size 128 each active block
 * column j is the entry pair 2j, 2j+1 with both row bits) are computed as
 * moddit_sparsity_map computes them and written into map_inout; every other cell keeps
 * its value. With map_inout holding the previous map and the lists those of the current
 * mask, the result is the merged map of the refresh step,
 * where(mask == False, prev, current) (MoD/mod/attn_mask.py:659-675 over
 * flash_attn_with_sparsity_map, MoD/mod/triton_flash_sparsity.py:274-341), bit for bit,
 * at the cost of the active cells only.
 */
int moddit_sparsity_map_merge(const void* q, const void* k, const float* lse, void* map_inout,
                              int batch, int heads, int seq_len, int head_dim,
                              const int64_t q_strides[3], const int64_t k_strides[3],
                              float softmax_scale, float log_threshold, int q_video_offset,
                              int k_video_offset, int video_blocks, int block_size, int dtype,
                              const int32_t* tile_counts, const int32_t* tile_entries,
                              int n_qtiles, int cap, moddit_stream_t stream);

/*
 * M^T S for the line model, per head (H, 3n) fp32:
 *   [0, 2n-1)   diagonal sums, index k <-> offset k-(n-1) (col - row)
 *   [2n-1, 3n-1) column sums
 *   3n-1        sum over the n/bpf frame-diagonal bpf x bpf blocks
 * map: contiguous (H,n,n) of map_dtype.
 *   FP16 (n <= 2^20 and n * min(blocks_per_frame, n) <= 2^23, so that every sum of
 *        fp16 values stays inside int64): one pass over the map, summed exactly in
 *        int64 units of 2^-24 and rounded once to fp32 (deterministic); needs a workspace of
 *        moddit_mts_workspace_bytes(heads, n) bytes, 16-byte aligned (scratch);
 *   FP32: summed in fp64 and rounded once; workspace may be NULL.
 * Replaces compute_mts (MoD/mod/cuda_lstsq_kernel.cu:421-482, kernels :17-162).
 */
int moddit_mts(const void* map, int map_dtype, int heads, int n, int blocks_per_frame,
               void* workspace, float* mts_out, moddit_stream_t stream);
int64_t moddit_mts_workspace_bytes(int heads, int n);

/*
 * Closed-form M^T M + lambda*I (F = 3n) written as doubles into a HOST buffer of F*F.
 * Replaces compute_mtm (MoD/mod/cuda_lstsq_kernel.cu:319-418; torch twin
 * MoD/mod/cuda_lstsq.py:42-89).
 */
int moddit_mtm_host(int n, int blocks_per_frame, double regularization, double* mtm_out);

/*
 * Ridge fit of the line model, X = (M^T M + lambda I)^-1 M^T S per head, through the Schur
 * complement of M^T M's diagonal x diagonal block (which is diagonal). With A =
 * diag(n-|o|+lambda) over the 2n-1 diagonals and W = M^T M's diagonal x [columns, frame]
 * block, S = C - W^T A^-1 W is (n+1) x (n+1):
 *   moddit_fit_schur_host  writes S in closed form (fp64, row-major) into a HOST buffer
 *                          of (n+1)^2 doubles; the caller inverts it once per
 *                          (n, blocks_per_frame, lambda) and keeps the inverse on the device;
 *   moddit_fit_lines       with schur_inv = S^-1 (device, fp64 (n+1)^2), mts (H,3n) fp32
 *                          from moddit_mts, writes x (H,3n) fp32 in M's column order. Three
 *                          kernels, fp64 arithmetic in a fixed order, x rounded once;
 *                          workspace: moddit_fit_workspace_doubles(H, n) doubles (scratch).
 * n <= 4096.
 * Replaces the cached Cholesky factor and _solve_all_heads (MoD/mod/cuda_lstsq.py:141-208:
 * torch.linalg.cholesky of the whole 3n x 3n M^T M, then cholesky_solve per call).
 */
int moddit_fit_schur_host(int n, int blocks_per_frame, double regularization, double* schur_out);
int64_t moddit_fit_workspace_doubles(int heads, int n);
int moddit_fit_lines(const double* schur_inv, const float* mts, float* x, double* workspace,
                     int heads, int n, int blocks_per_frame, double regularization,
                     moddit_stream_t stream);

/*
 * moddit_fit_lines without a workspace argument and without any allocation: the
 * workspace lives in a fixed device array of the library (2 * 64 * 2049 doubles =
 * 2.1 MB per device, held until the process ends), so heads * (n + 1) <= 64 * 2049
 * (e.g. 64 heads at n <= 2048; the headline's 24 heads at n = 1800 fit); larger shapes
 * return MODDIT_EINVAL. Same kernels and results as moddit_fit_lines. Calls that overlap
 * on one device share the array and race; serialise them (one stream per device).
 * No counterpart in the reference: this entry point is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops).
 */
int moddit_fit_lines_noalloc(const double* schur_inv, const float* mts, float* x, int heads,
                             int n, int blocks_per_frame, double regularization,
                             moddit_stream_t stream);

/*
 * Line prediction and selection: with c = X[:,2n-1:3n-1]/2 and d = X[:,:2n-1] for the
 * current (x_cur) and previous (x_last) fits, pred = cur + (cur - last) / predict_T over
 * v = [pred_c (n), pred_d (2n-1)]; selects the k = min(top_k, 3n-1) smallest per head,
 * ties broken by lower index, NaN ordered last. Writes the selected indices in ascending
 * index order to sel_out (H,k) int32.
 * Replaces choose_topk_lines (MoD/mod/attn_mask.py:351-370).
 */
int moddit_select_lines(const float* x_cur, const float* x_last, int heads, int n,
                        int predict_T, int top_k, int32_t* sel_out, moddit_stream_t stream);

/*
 * Block-diagonal mode decision: for each head with mode[h] == SPARSE,
 * mode[h] = BLOCK_DIAGONAL if x[h, features-1] <= threshold.
 * Replaces check_bd_values (MoD/mod/attn_mask.py:336-349).
 */
int moddit_check_bd(const float* x, int heads, int features, float threshold, uint8_t* mode,
                    moddit_stream_t stream);

/*
 * Block mask from selected lines and the attention kernel's tile lists.
 *   video[h,i,j] = mode==FULL | col_sel[j] | diag_sel[j-i+n-1] | (mode==BD & i/bpf==j/bpf)
 *   mask (H,nb,nb) bool (1 byte) merged per layout (wan: nb=n; hunyuan: video first,
 *   text rows/cols true; cogvideox: text first; other: all true).
 * counts/entries receive the tile lists of moddit_block_sparse_fwd for the mask at
 * block_size granularity (64 or 128); union_rows=1 reproduces the reference engine's
 * 128-row union (both row bits set whenever either 64-row block is active).
 * mask_out, counts or entries may be NULL to skip that output.
 * Replaces generate_mask_from_lines (MoD/mod/attn_mask.py:440-559) and the mask
 * conversion of AttentionSparseEngine (attn_mask.py:296-304).
 */
int moddit_mask_from_lines(const int32_t* sel, int heads, int k, const uint8_t* mode,
                           int n, int blocks_per_frame, int layout, int nb, int text_blocks,
                           int block_size, int union_rows, uint8_t* mask_out,
                           int32_t* counts, int32_t* entries, int n_qtiles, int cap,
                           moddit_stream_t stream);

/*
 * Tile lists from an explicit bool block mask at block_size granularity, the same
 * encoding as moddit_mask_from_lines. The mask has n_rows query blocks and n_cols key
 * blocks per head and is addressed as mask[h*mask_head_stride + i*mask_row_stride + j]
 * (views such as the video rows of a larger mask need no copy); key tiles at or beyond
 * kv_tiles are dropped. n_qtiles = ceil(n_rows*block_size/128), cap >= n_cols*block_size/64.
 * Replaces the mask conversion of AttentionSparseEngine (MoD/mod/attn_mask.py:296-311).
 */
int moddit_mask_to_tiles(const uint8_t* mask, int heads, int n_rows, int n_cols,
                         int64_t mask_head_stride, int64_t mask_row_stride, int block_size,
                         int union_rows, int kv_tiles, int32_t* counts, int32_t* entries,
                         int n_qtiles, int cap, moddit_stream_t stream);

/*
 * Refresh merge: out[h,i,j] = mask[h,i,j] ? cur[h,i,j] : prev[h,i,j] over (H,n,n) fp16,
 * where mask is addressed as mask[h*mask_head_stride + i*mask_row_stride + j].
 * out may alias prev. Replaces the torch.where of MoD/mod/attn_mask.py:671-675.
 */
int moddit_refresh_merge(const void* prev, const void* cur, const uint8_t* mask,
                         int64_t mask_head_stride, int64_t mask_row_stride,
                         int heads, int n, void* out, moddit_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MODDIT_H_ */
