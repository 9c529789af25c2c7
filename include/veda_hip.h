/*
 * veda_hip.h -- C ABI of the MI355X (gfx950) Veda sparse-attention kernels.
 *
 * Plain pointers and sizes only: no torch or HIP types in the signatures.
 * Every pointer argument is a device pointer unless stated otherwise; every
 * entry point enqueues its kernels on `stream` (a hipStream_t passed as
 * void*, NULL = the null stream) and returns without synchronising.
 *
 * Return value: VEDA_OK (0) on success; VEDA_EINVAL when an argument is out
 * of range (nothing was launched), VEDA_ELAUNCH when HIP refused a launch.
 * veda_last_error() returns a message for the last failure of the calling
 * thread. No entry point allocates device memory; callers own all buffers.
 *
 * Element types: "bf16" buffers hold bfloat16 bit patterns (uint16), "bool"
 * buffers hold one byte per element (0 / 1), as torch.bool does. Strides are
 * in elements.
 *
 * Tile conventions (all from miowtion/veda/tiling.py): tiles hold 128 slots;
 * a tile-ordered tensor is [N = n_tiles * 128, H', D]; the real rows of every
 * tile are a prefix of length valid_count[tile] (tiling.py:9-16).
 */
#ifndef VEDA_HIP_H_
#define VEDA_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VEDA_OK 0
#define VEDA_EINVAL (-1)
#define VEDA_ELAUNCH (-2)

/* Message of the calling thread's last failure ("" if none). */
const char* veda_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int veda_abi_version(void);

/*
 * Gather rows into tile order, optionally pooling every tile.
 * Replaces miowtion/kernels/tile_gather_triton.py:156-209 (gather_tiles,
 * gather_and_pool; kernel at :73-115) and miowtion/veda/tiling.py:278-297.
 *
 *   out[s, h', :] = slot_valid[s] ? x[gather_index[s], heads[h'], :] : 0
 *   feats[h', t, :] = [mean | max | min] over the valid_count[t] real rows
 *     (mean = sum over the 128 slots / max(valid_count, 1); 0 for empty tiles)
 *   sq[h', t, :]  = E[x^2],  var[h', t, :] = centred Var(x) (two-pass form)
 *
 * x: bf16 [x_rows, H, D] with strides (x_stride_s, x_stride_h, 1).
 * out: bf16 [n_tiles*128, n_heads, D], strides (out_stride_s, out_stride_h, 1),
 *   or NULL to pool only (x is then usually already tile-ordered).
 * feats: fp32 [n_heads, n_tiles, 3D] contiguous, or NULL (no pooling).
 * sq, var: fp32 [n_heads, n_tiles, D] contiguous, both NULL or both set;
 *   only with feats.
 * head_dim: 64 or 128.
 */
int veda_gather_tiles(const void* x, int64_t x_rows, int64_t x_heads,
                      int64_t x_stride_s, int64_t x_stride_h,
                      const int64_t* gather_index, const int32_t* slot_valid,
                      const int32_t* valid_count, int64_t n_tiles,
                      const int64_t* heads, int64_t n_heads, int64_t head_dim,
                      void* out, int64_t out_stride_s, int64_t out_stride_h,
                      float* feats, float* sq, float* var, void* stream);

/*
 * Write tile-ordered rows back: out[scatter_index[s], heads[h'], :] =
 * tiled[s, h', :] for every slot with slot_valid[s] != 0 (padding slots are
 * dropped, so the result on rows [0, S) equals the reference's index write
 * into its [S + 1, H, D] buffer).
 * Replaces miowtion/kernels/tile_gather_triton.py:212-224 (kernel :117-131)
 * and miowtion/veda/tiling.py:300-312.
 */
int veda_scatter_tiles(const void* tiled, int64_t tiled_stride_s,
                       int64_t tiled_stride_h, const int64_t* scatter_index,
                       const int32_t* slot_valid, int64_t n_tiles,
                       const int64_t* heads, int64_t n_heads, int64_t head_dim,
                       void* out, int64_t out_rows, int64_t out_heads,
                       int64_t out_stride_s, int64_t out_stride_h,
                       void* stream);

/*
 * Dense LSE [rows, H] (fp32, strides) -> tile order [N, n_heads] contiguous,
 * 0 on padding slots. Replaces miowtion/veda/attention.py:299-305.
 */
int veda_gather_lse(const float* lse, int64_t lse_rows, int64_t lse_heads,
                    int64_t lse_stride_s, int64_t lse_stride_h,
                    const int64_t* gather_index, const int32_t* slot_valid,
                    int64_t n_slots, const int64_t* heads, int64_t n_heads,
                    float* out, void* stream);

/*
 * Top-k of one column block of the video quadrant (rule 'topk').
 * Replaces the per-block body of miowtion/veda/mask.py:251-284.
 *
 * For every head h and selection row r (video tile id rows[r]):
 *   s[c] = scores[h, r, block_start + c] for c in [0, n_cols),
 *   s[c] = -inf where kv_ok[block_start + c] == 0,
 *   s[rows[r] - block_start] = +inf when rows[r] lies in the block,
 *   index[h, r, col0 + t] = block_start + (t-th largest column),
 *   keep[h, r, col0 + t]  = t < k_lo + extra[rows[r]] && value > -inf,
 * for t in [0, k_hi). Equal scores are ordered lower column first.
 * scores: fp32 with strides (s_stride_h, s_stride_r, 1).
 * extra: bool [n_extra] Bresenham pattern indexed by tile id.
 * index (int64) and keep (bool) share strides (o_stride_h, o_stride_r, 1).
 */
int veda_select_topk(const float* scores, int64_t n_heads, int64_t n_rows,
                     int64_t s_stride_h, int64_t s_stride_r,
                     int64_t block_start, int64_t n_cols,
                     const uint8_t* kv_ok, const int64_t* rows,
                     int64_t k_lo, int64_t k_hi, const uint8_t* extra,
                     int64_t n_extra, int64_t* index, uint8_t* keep,
                     int64_t o_stride_h, int64_t o_stride_r, int64_t col0,
                     void* stream);

/*
 * Block mask of a selection. Replaces miowtion/veda/mask.py:288-317.
 * index/keep: [n_heads, n_sel, k_total] contiguous. mask: bool
 * [n_heads, global_rows ? n_tiles : n_sel, n_tiles] contiguous.
 * Video rows: the kept selection; global key columns [n_video, n_tiles)
 * follow kv_ok; with global_rows, rows [n_video, n_tiles) equal kv_ok.
 */
int veda_dense_block_mask(const int64_t* index, const uint8_t* keep,
                          int64_t n_heads, int64_t n_sel, int64_t k_total,
                          const uint8_t* kv_ok, int64_t n_tiles,
                          int64_t n_video, int global_rows, uint8_t* mask,
                          void* stream);

/*
 * Full / partial key-tile lists of a block mask [n_heads, n_rows, n_tiles].
 * Replaces miowtion/kernels/fa4.py:266-296 (index_lists, _pack_lists):
 *   member = mask & kv_ok; full = member & full_tile; part = member & ~full
 *   *_cnt[h, r] = |list|; *_idx[h, r, :] = list members ascending, then the
 *   non-members ascending (n_tiles entries per row, int32).
 */
int veda_index_lists(const uint8_t* block_mask, int64_t n_heads,
                     int64_t n_rows, int64_t n_tiles, const uint8_t* kv_ok,
                     const uint8_t* full_tile, int32_t* part_cnt,
                     int32_t* part_idx, int32_t* full_cnt, int32_t* full_idx,
                     void* stream);

/*
 * Block-sparse attention forward on tile-ordered rows.
 * Replaces miowtion/kernels/fa4.py:299-377 (the FA4 CuTe sparse forward,
 * fa4_sm8x/flash_fwd.py:1297-1443) with the semantics of
 * miowtion/kernels/reference.py:1-56:
 *   query tile r (rows r*128 .. r*128+127 of q) attends to the key tiles in
 *   full_idx[h, r, :full_cnt[h, r]] (all 128 keys) and
 *   part_idx[h, r, :part_cnt[h, r]] (keys with local index < valid_count[j]);
 *   out = softmax(q k^T * scale) v over those keys, 0 for a row with none;
 *   lse[h, row] = natural-log log-sum-exp over them (-inf for none).
 * q: bf16 [n_q_tiles*128, H', D]; k, v: bf16 [n_k_tiles*128, H', D]; all
 * with their own (row, head) strides. Lists: int32, cnt [H', n_q_tiles],
 * idx [H', n_q_tiles, list_ld]. lse: fp32 or NULL, element
 * lse[h * lse_stride_h + row * lse_stride_s]. head_dim: 128.
 * front_tiles (0 .. n_q_tiles): query tiles [n_q_tiles - front_tiles,
 * n_q_tiles) of every head are dispatched before all others. It changes no
 * value, only the order: pass the number of tiles the mask makes dense
 * (miowtion/veda/mask.py:288-317 keeps every key tile for the global rows,
 * which come last in tile order), so that their long walks do not end the
 * launch; 0 is the plain (head, tile) order. The same argument of
 * veda_compensated_attention and veda_block_sparse_bwd (there it also
 * orders the key tiles of the dK / dV kernel) means the same.
 */
int veda_block_sparse_fwd(const void* q, int64_t q_stride_s, int64_t q_stride_h,
                          const void* k, int64_t k_stride_s, int64_t k_stride_h,
                          const void* v, int64_t v_stride_s, int64_t v_stride_h,
                          int64_t n_heads, int64_t head_dim,
                          int64_t n_q_tiles, int64_t n_k_tiles,
                          const int32_t* full_cnt, const int32_t* full_idx,
                          const int32_t* part_cnt, const int32_t* part_idx,
                          int64_t list_ld, const int32_t* valid_count,
                          float scale, void* out, int64_t o_stride_s,
                          int64_t o_stride_h, float* lse, int64_t lse_stride_h,
                          int64_t lse_stride_s, int64_t front_tiles, void* stream);

/*
 * Block-sparse attention forward with the tile permutation of q and out
 * fused in: equal to veda_gather_tiles of q (gather_index, padding slots
 * zero), then veda_block_sparse_fwd, then veda_scatter_tiles of the result
 * into out (scatter_index, slots with slot_valid 0 not written). Replaces
 * that sequence inside the reference's SparseStudent._attend
 * (miowtion/veda/attention.py:760-788: gather_tiles of q,
 * fa4.block_sparse_attention, scatter_tiles_). q: bf16 [q_rows, seq_heads,
 * D] in sequence order; out: bf16 [out_rows, seq_heads, D] (the reference's
 * [S + 1, H, D] buffer, row S taking padding); heads: int64 [n_heads], head
 * h' of k, v and the lists is head heads[h'] of q and out. gather_index,
 * scatter_index: int64 [n_q_tiles * 128], slot_valid: int32 [n_q_tiles *
 * 128]. A slot whose index or head is outside q / out reads zeros and
 * writes nothing, as in the gather and scatter kernels. k, v, lists,
 * valid_count, scale and front_tiles as veda_block_sparse_fwd; no LSE.
 */
int veda_block_sparse_fwd_seq(const void* q, int64_t q_rows, int64_t seq_heads,
                              int64_t q_stride_s, int64_t q_stride_h,
                              const int64_t* gather_index, const int64_t* scatter_index,
                              const int32_t* slot_valid, const int64_t* heads,
                              int64_t n_heads, const void* k, int64_t k_stride_s,
                              int64_t k_stride_h, const void* v, int64_t v_stride_s,
                              int64_t v_stride_h, int64_t head_dim, int64_t n_q_tiles,
                              int64_t n_k_tiles, const int32_t* full_cnt,
                              const int32_t* full_idx, const int32_t* part_cnt,
                              const int32_t* part_idx, int64_t list_ld,
                              const int32_t* valid_count, float scale, void* out,
                              int64_t out_rows, int64_t o_stride_s, int64_t o_stride_h,
                              int64_t front_tiles, void* stream);

/*
 * veda_block_sparse_fwd_seq with the gather of the key tiles fused in as
 * well: k and v are in sequence order like q (bf16 [q_rows, seq_heads, D],
 * the three sharing stride_s / stride_h), and key tile row t is row
 * gather_index[t] of them; head h' of the lists reads head heads[h'] of k
 * and v. Equal to veda_gather_tiles of q, k and v (gather_index, padding
 * slots zero), then veda_block_sparse_fwd, then veda_scatter_tiles of the
 * result, for every finite input: a padding row of a key tile (masked, p =
 * 0) is read from that tile's first row instead of as zeros, so a
 * non-finite value there reaches only the query tiles that keep the block,
 * which that row already reaches. Replaces gather_tiles of q, k and v,
 * fa4.block_sparse_attention and scatter_tiles_ inside the reference's
 * SparseStudent._attend (miowtion/veda/attention.py:760-788). Lists,
 * valid_count, scale and front_tiles as veda_block_sparse_fwd; no LSE.
 * (q_rows - 1) * stride_s * 2 + 256 must be below 2^32.
 */
int veda_block_sparse_fwd_seq_kv(const void* q, const void* k, const void* v, int64_t q_rows,
                                 int64_t seq_heads, int64_t stride_s, int64_t stride_h,
                                 const int64_t* gather_index, const int64_t* scatter_index,
                                 const int32_t* slot_valid, const int64_t* heads,
                                 int64_t n_heads, int64_t head_dim, int64_t n_q_tiles,
                                 int64_t n_k_tiles, const int32_t* full_cnt,
                                 const int32_t* full_idx, const int32_t* part_cnt,
                                 const int32_t* part_idx, int64_t list_ld,
                                 const int32_t* valid_count, float scale, void* out,
                                 int64_t out_rows, int64_t o_stride_s, int64_t o_stride_h,
                                 int64_t front_tiles, void* stream);

/*
 * Dense attention of rows [0, used) among themselves on packed [S, H, D]
 * rows (the h3 dense path, miowtion/h3/attention.py:28-102): out rows
 * [used, S) are 0 and their lse is 0. lse: fp32 or NULL, element
 * lse[row * lse_stride_s + h * lse_stride_h] ([S, H] in the reference).
 */
int veda_dense_fwd(const void* q, int64_t q_stride_s, int64_t q_stride_h,
                   const void* k, int64_t k_stride_s, int64_t k_stride_h,
                   const void* v, int64_t v_stride_s, int64_t v_stride_h,
                   int64_t seq_len, int64_t used, int64_t n_heads,
                   int64_t head_dim, float scale, void* out,
                   int64_t o_stride_s, int64_t o_stride_h, float* lse,
                   int64_t lse_stride_s, int64_t lse_stride_h, void* stream);

/*
 * Teacher block heat. Replaces miowtion/kernels/block_heat_triton.py:141-173
 * (heat_kernel :97-137) with the semantics of
 * miowtion/veda/heatmap.py:36-99:
 *   reduce 0 ('sum'): heat[h, r, j] = sum over real rows i of tile
 *     q_tiles[r] and real keys c of tile j of exp(q_i.k_c * scale - lse_i);
 *   reduce 1 ('max'): exp(max_i(bf16(max_c q_i.k_c) * scale - lse_i)).
 * The real rows of tile t are its first valid_count[t] slots (the tile
 * layout's prefix rule, tiling.py:9-16); padding rows and keys contribute
 * nothing; a q_tiles entry outside [0, n_tiles) gets a zero row. Scores are
 * fp32 (MFMA accumulation).
 * q, k: bf16 [n_tiles * 128, H', D] with strides; lse: fp32 [N, H'] with
 * strides; valid_count: int32 [n_tiles]; heat: fp32 [n_heads, n_q, n_tiles]
 * contiguous. head_dim: 128; n_tiles <= 2048.
 */
int veda_block_heat(const void* q, int64_t q_stride_s, int64_t q_stride_h,
                    const void* k, int64_t k_stride_s, int64_t k_stride_h,
                    const float* lse, int64_t lse_stride_s,
                    int64_t lse_stride_h, const int32_t* valid_count,
                    const int64_t* q_tiles, int64_t n_q, int64_t n_tiles,
                    int64_t n_heads, int64_t head_dim, int reduce, float scale,
                    float* heat, void* stream);

/*
 * Teacher dense pass in tile order with the block-heat statistics: the
 * fused form of the dense LSE pass (miowtion/h3/attention.py:80-102, as
 * OracleStudent uses it, miowtion/veda/attention.py:549-553) and the heat
 * (miowtion/veda/heatmap.py:36-110), the plan of
 * docs/features/veda_kernel.md:285-289.
 *
 * Item r (of n_items) is query tile q_tiles[r] (NULL: tile r) of q, which
 * holds q_tiles_held tiles; it attends to every valid key (the first
 * valid_count[j] slots of key tile j) of n_k_tiles key tiles. Writes
 *   lse[h * lse_stride_h + (128 r + s) * lse_stride_s]  natural-log LSE,
 *   part[(h * n_k_tiles + j) * (128 n_items) + 128 r + s]  (fp32, log2
 *     units) the row's log-sum-exp ('sum', reduce 0) or max ('max', reduce
 *     1) of scale * q.k over the valid keys of tile j (-inf if none),
 * and, when out and v are both non-NULL, the attention output in tile order
 * out[128 r + s, h, :]. part is caller workspace of n_heads * n_k_tiles *
 * 128 n_items floats. Then veda_heat_combine gives the heat.
 */
int veda_dense_heat_fwd(const void* q, int64_t q_stride_s, int64_t q_stride_h,
                        int64_t q_tiles_held, const void* k, int64_t k_stride_s,
                        int64_t k_stride_h, const void* v, int64_t v_stride_s,
                        int64_t v_stride_h, int64_t n_heads, int64_t head_dim,
                        const int64_t* q_tiles, int64_t n_items, int64_t n_k_tiles,
                        const int32_t* valid_count, float scale, int reduce,
                        void* out, int64_t o_stride_s, int64_t o_stride_h,
                        float* lse, int64_t lse_stride_h, int64_t lse_stride_s,
                        float* part, void* stream);

/*
 * Block heat from veda_dense_heat_fwd's statistics
 * (miowtion/veda/heatmap.py:36-110 semantics; miowtion/kernels/
 * block_heat_triton.py:141-173 computes the same from a separate LSE):
 *   'sum' (0): heat[h, r, j] = sum over the valid rows s of 2^(part - lse log2 e)
 *   'max' (1): heat[h, r, j] = 2^(max over the valid rows of (part - lse log2 e))
 * heat: fp32 [n_heads, n_items, n_tiles] contiguous; rows with lse = -inf
 * and slots past valid_count[q_tiles[r]] count as absent.
 */
int veda_heat_combine(const float* part, const float* lse, int64_t lse_stride_h,
                      int64_t lse_stride_s, const int32_t* valid_count,
                      const int64_t* q_tiles, int64_t n_items, int64_t n_tiles,
                      int64_t n_heads, int reduce, float* heat, void* stream);

/*
 * Tile summaries of the zero-order compensation
 * (miowtion/kernels/compensation_triton.py:80-99, :150-170): for key tile t
 * and head h, kc[t, h, :] = mean of k over the tile's real rows (sum /
 * max(valid_count[t], 1)) and vc[t, h, :] = their sum of v, both bf16.
 * k, v: bf16 [n_tiles * 128, n_heads, 128]; kc, vc: bf16 [n_tiles, n_heads,
 * 128] with strides (c_stride_s, c_stride_h, 1).
 */
int veda_tile_summaries(const void* k, int64_t k_stride_s, int64_t k_stride_h,
                        const void* v, int64_t v_stride_s, int64_t v_stride_h,
                        const int32_t* valid_count, int64_t n_tiles,
                        int64_t n_heads, int64_t head_dim, void* kc, void* vc,
                        int64_t c_stride_s, int64_t c_stride_h, void* stream);

/*
 * Zero-order compensation (miowtion/veda/attention.py:591-689; the Triton
 * form miowtion/kernels/compensation_triton.py:102-147, :173-225): for row
 * r of query tile i and head h,
 *   p_j = exp(q[r] . kc[j] * scale - lse_kept[h, r])   (lse_kept -> 0 if not finite)
 *   out[r] = (o_kept[r] + sum_j p_j vc[j]) / (1 + sum_j p_j valid_count[j])
 * over the key tiles j with keep[h, i, j] == 0 and valid_count[j] > 0.
 * keep: bytes [n_heads, n_q_tiles, n_k_tiles]; o_kept, q, out: bf16
 * [n_q_tiles * 128, n_heads, 128]; kc, vc from veda_tile_summaries.
 */
int veda_zero_order_compensation(const void* o_kept, int64_t ok_stride_s,
                                 int64_t ok_stride_h, const float* lse_kept,
                                 int64_t lse_stride_h, int64_t lse_stride_s,
                                 const void* q, int64_t q_stride_s, int64_t q_stride_h,
                                 const void* kc, const void* vc, int64_t c_stride_s,
                                 int64_t c_stride_h, const uint8_t* keep,
                                 const int32_t* valid_count, int64_t n_heads,
                                 int64_t head_dim, int64_t n_q_tiles, int64_t n_k_tiles,
                                 float scale, void* out, int64_t o_stride_s,
                                 int64_t o_stride_h, void* stream);

/*
 * Compensated block-sparse attention in one pass
 * (miowtion/kernels/compensation_triton.py:228-258 attention: the FA4
 * forward over the kept blocks, then compensate): the listed blocks
 * (full_* / part_*, as for veda_block_sparse_fwd) and then, for every key
 * tile j with keep[h, i, j] == 0 and valid_count[j] > 0, one virtual key
 * kc[j] with value vc[j] and weight valid_count[j] (the tile summaries of
 * veda_tile_summaries), all inside one online softmax: out = (sum over
 * kept keys of p v + sum over dropped tiles of p vc) / (sum over kept keys
 * of p + sum of p valid_count). A row that kept nothing gets the
 * reference's unit mass at reference 0 (out = num / (1 + den)). keep:
 * bytes [n_heads, n_q_tiles, n_k_tiles], the kept-block mask with kv_ok
 * applied. Shapes and strides as veda_block_sparse_fwd and
 * veda_zero_order_compensation.
 */
int veda_compensated_attention(const void* q, int64_t q_stride_s, int64_t q_stride_h,
                               const void* k, int64_t k_stride_s, int64_t k_stride_h,
                               const void* v, int64_t v_stride_s, int64_t v_stride_h,
                               int64_t n_heads, int64_t head_dim, int64_t n_q_tiles,
                               int64_t n_k_tiles, const int32_t* full_cnt,
                               const int32_t* full_idx, const int32_t* part_cnt,
                               const int32_t* part_idx, int64_t list_ld, const void* kc,
                               const void* vc, int64_t c_stride_s, int64_t c_stride_h,
                               const uint8_t* keep, const int32_t* valid_count, float scale,
                               void* out, int64_t o_stride_s, int64_t o_stride_h,
                               int64_t front_tiles, void* stream);

/*
 * Block-sparse attention backward: the gradients of veda_block_sparse_fwd
 * (FA4's backward with the Q-direction lists, reached through
 * miowtion/kernels/fa4.py:340-373 -> fa4_sm8x/interface.py:3722-3790
 * FlashAttnFunc.backward -> :2099 _flash_attn_bwd; the block-sparse main
 * loop is fa4_sm8x/flash_bwd.py:1261-1340). With P the forward's softmax
 * over the kept key tiles' valid keys,
 *   D = rowsum(dout * out) - dlse,   dS = P * (dout V^T - D)
 *   dq = dS K * scale,  dk = dS^T Q * scale,  dv = P^T dout.
 * q, out, dout, dq: bf16 [n_q_tiles * 128, n_heads, 128]; k, v, dk, dv: bf16
 * [n_k_tiles * 128, n_heads, 128] (strides in elements, last dim 1). lse:
 * the forward's natural-log LSE, lse[h * lse_stride_h + row *
 * lse_stride_s]; dlse: its gradient in the same form, or NULL.
 * full_* / part_*: the forward lists (rows = query tiles, entries = key
 * tiles, row stride list_ld); full_*_t / part_*_t: the transposed lists
 * (rows = key tiles, entries = query tiles, row stride list_ld_t), as
 * fa4.py:275-296 index_lists(transpose=True) builds them. Every row of
 * dq, dk, dv is written (0 where no block reaches it). Rows whose dout is
 * zero (+-0) and whose D is 0 add exactly zero for finite inputs, so 64-row
 * halves (and 32-row groups) made of them are skipped: a layer's gradient
 * through the scatter is zero on padding rows. workspace: at least
 * n_heads * n_q_tiles * 2048 bytes of device memory, 16-byte aligned
 * (per-row statistics; contents on entry do not matter).
 */
int veda_block_sparse_bwd(const void* q, int64_t q_stride_s, int64_t q_stride_h,
                          const void* k, int64_t k_stride_s, int64_t k_stride_h,
                          const void* v, int64_t v_stride_s, int64_t v_stride_h,
                          const void* out, int64_t o_stride_s, int64_t o_stride_h,
                          const void* dout, int64_t do_stride_s, int64_t do_stride_h,
                          const float* lse, int64_t lse_stride_h, int64_t lse_stride_s,
                          const float* dlse, int64_t dlse_stride_h,
                          int64_t dlse_stride_s, int64_t n_heads, int64_t head_dim,
                          int64_t n_q_tiles, int64_t n_k_tiles,
                          const int32_t* full_cnt, const int32_t* full_idx,
                          const int32_t* part_cnt, const int32_t* part_idx,
                          int64_t list_ld, const int32_t* full_cnt_t,
                          const int32_t* full_idx_t, const int32_t* part_cnt_t,
                          const int32_t* part_idx_t, int64_t list_ld_t,
                          const int32_t* valid_count, float scale, void* dq,
                          int64_t dq_stride_s, int64_t dq_stride_h, void* dk,
                          int64_t dk_stride_s, int64_t dk_stride_h, void* dv,
                          int64_t dv_stride_s, int64_t dv_stride_h, void* workspace,
                          int64_t workspace_bytes, int64_t front_tiles, void* stream);

/*
 * veda_block_sparse_bwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference.
 *
 * Same arguments and results as veda_block_sparse_bwd minus workspace /
 * workspace_bytes: the per-row statistics go to a 64 MiB device array of the
 * library instead (one per device, held until the process ends), so
 * n_heads * n_q_tiles * 2048 bytes must not exceed 64 MiB (32,768
 * (head, query tile) pairs; BASELINE C2 at 48 heads needs 28,416); larger
 * calls return VEDA_EINVAL before any launch. The entry point allocates
 * nothing. The stream must belong to the current device; the first call on
 * a device looks the array up (hipGetSymbolAddress). Calls that overlap on
 * one device (different streams, or threads without ordering) share the
 * array and race: order them on one stream.
 */
int veda_block_sparse_bwd_noalloc(
    const void* q, int64_t q_stride_s, int64_t q_stride_h, const void* k, int64_t k_stride_s,
    int64_t k_stride_h, const void* v, int64_t v_stride_s, int64_t v_stride_h, const void* out,
    int64_t o_stride_s, int64_t o_stride_h, const void* dout, int64_t do_stride_s,
    int64_t do_stride_h, const float* lse, int64_t lse_stride_h, int64_t lse_stride_s,
    const float* dlse, int64_t dlse_stride_h, int64_t dlse_stride_s, int64_t n_heads,
    int64_t head_dim, int64_t n_q_tiles, int64_t n_k_tiles, const int32_t* full_cnt,
    const int32_t* full_idx, const int32_t* part_cnt, const int32_t* part_idx, int64_t list_ld,
    const int32_t* full_cnt_t, const int32_t* full_idx_t, const int32_t* part_cnt_t,
    const int32_t* part_idx_t, int64_t list_ld_t, const int32_t* valid_count, float scale,
    void* dq, int64_t dq_stride_s, int64_t dq_stride_h, void* dk, int64_t dk_stride_s,
    int64_t dk_stride_h, void* dv, int64_t dv_stride_s, int64_t dv_stride_h,
    int64_t front_tiles, void* stream);

/*
 * Predictor tile embedding, miowtion/veda/predictor.py:251-255:
 *   out[h', t, :] = feats[h', t, :] @ W[heads[h']] (+ feats[h', t, :n_out]
 *   when residual), fp32 accumulation.
 * feats: fp32 [n_heads, n_tiles, k_dim] contiguous; W: [w_heads, k_dim,
 * n_out] contiguous, w_dtype 0 = bf16, 1 = fp32, 2 = fp8 e4m3 with a
 * per-head fp32 scale w_scale[w_heads] (dequantised as
 * bf16(e4m3 * scale), the resident form of miowtion/veda/bundle.py:280-297).
 * out: fp32 [n_heads, n_tiles, n_out] contiguous.
 */
int veda_predictor_embed(const float* feats, int64_t n_heads, int64_t n_tiles,
                         int64_t k_dim, const void* w, int w_dtype,
                         const float* w_scale, int64_t w_heads,
                         const int64_t* heads, int64_t n_out, int residual,
                         float* out, void* stream);

/*
 * Predictor block logits, miowtion/veda/predictor.py:325-338:
 *   out[h', i, j] = (accumulate ? out[h', i, j] : 0) + scale * a[h', i].b[h', j]
 *                   + (gain ? gain[heads[h']] * log_count[j] : 0)
 * a: fp32 [n_heads, n_q, dim], b: fp32 [n_heads, n_k, dim], out: fp32
 * [n_heads, n_q, n_k], all contiguous. gain/heads/log_count may be NULL.
 */
int veda_predictor_logits(const float* a, const float* b, int64_t n_heads,
                          int64_t n_q, int64_t n_k, int64_t dim, float scale,
                          const float* gain, const int64_t* heads,
                          const float* log_count, int accumulate, float* out,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VEDA_HIP_H_ */
