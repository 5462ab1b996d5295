/*
 * sa_api.h -- C ABI of libsa_hip.so, the MI355X (gfx950) sparse-attention hot path.
 *
 * Every entry point is `extern "C"`, takes plain pointers, sizes and strides, and returns
 * an int status (SA_OK or a negative SA_ERR_* code; sa_last_error() gives the message of
 * the calling thread's last failure). Nothing here throws across the ABI.
 *
 * Conventions
 *  - Tensors of shape [B, H, L, D] are passed as a device pointer plus three element
 *    strides {stride_b, stride_h, stride_l}; the D axis must be contiguous (stride 1).
 *    Element type is bf16 (uint16_t bit patterns) unless stated otherwise.
 *  - Device buffers are owned by the caller (PyTorch's caching allocator in the Python
 *    package), including every workspace (sized by the *_workspace queries). The library
 *    allocates no device memory and changes no allocator or device setting; its one
 *    device-resident buffer is the fixed scratch array of sa_tome_match_noalloc, part of the
 *    loaded code object.
 *  - `stream` is a hipStream_t passed as void*; NULL means the default stream. All GPU
 *    work is enqueued asynchronously on it; no entry point synchronises the device.
 *  - Entry points documented as "host" run on the CPU only and touch no GPU state.
 *  - Block-index lists ("kv lists") are int32 arrays kv_idx[rows][max_cnt] with per-row
 *    counts kv_cnt[rows], rows = B*H*ceil(Lq/64), each list holding the key-block indices
 *    to visit for one 64-row query block, ascending.
 *
 * Each declaration names the reference interface (file:line in
 * xiaolong-li1/SparseAttnFunctions, package `special_attentions`) whose work it replaces.
 */
#ifndef SA_API_H
#define SA_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SA_OK 0
#define SA_ERR_INVALID (-1)     /* bad argument: null pointer, shape, stride, range */
#define SA_ERR_UNSUPPORTED (-2) /* valid but not implemented (e.g. head_dim != 64) */
#define SA_ERR_HIP (-3)         /* a HIP runtime call failed (launch, device query) */

#define SA_ABI_VERSION 3

/* Version of this ABI (SA_ABI_VERSION). */
int sa_abi_version(void);

/* Message of the calling thread's last failed call ("" if none). Never NULL. */
const char* sa_last_error(void);

/*
 * Dense block mask -> kv lists.
 * Replaces the per-program scan of the boolean block mask inside the Triton kernel
 * (utils/block_sparse_attn_kernel.py:69-70, 163-199): the list is built once per call
 * instead of each of the 278 x 60 programs loading every mask entry.
 *   mask      uint8/bool, logical shape [B, H, nqb, nkb], element strides mask_strides[4]
 *             (any strides, 0 for broadcast, as the reference accepts,
 *             block_sparse_attn_kernel.py:125,141,155).
 *   kv_idx    int32 [B*H*nqb][max_cnt], max_cnt >= nkb.  kv_cnt int32 [B*H*nqb].
 */
int sa_mask_to_kv_list(const uint8_t* mask, const int64_t mask_strides[4], int B, int H,
                       int nqb, int nkb, int32_t* kv_idx, int max_cnt, int32_t* kv_cnt,
                       void* stream);

/*
 * Block mask of another block shape -> 64 x 64 tile lists with token-level cuts.
 * Serves sparse_attention_factory(BLOCK_M, BLOCK_N) (utils/block_sparse_attn_kernel.py:
 * 283-291): mask row m covers query rows [m*BLOCK_M, (m+1)*BLOCK_M), column n keys
 * [n*BLOCK_N, (n+1)*BLOCK_N) (:139-155). block_m, block_n: powers of two in 16..1024.
 *   mask      uint8/bool [B, H, >= ceil(Lq/block_m), >= ceil(Lk/block_n)], element strides.
 *   kv_idx/kv_cnt  lists of the 64-row tiles (rows B*H*ceil(Lq/64), max_cnt >= ceil(Lk/64)):
 *             a 64-key tile is listed when a mask cell it covers is set (cells past Lq or Lk
 *             neither keep nor cut a tile).
 *   kv_slot   [rows][max_cnt]: -1 when every cell of the tile is set, else the pattern of set
 *             cells, an index into sa_cell_tile_masks(block_m, block_n); may be NULL when both
 *             block sizes are >= 64 (then every listed tile is whole).
 * The lists and slots go to sa_block_sparse_fwd_tilemask / _mapped(_f16) unchanged.
 */
int sa_mask_cells_to_kv_list(const uint8_t* mask, const int64_t mask_strides[4], int B, int H,
                             int Lq, int Lk, int block_m, int block_n, int32_t* kv_idx,
                             int32_t* kv_slot, int max_cnt, int32_t* kv_cnt, void* stream);

/*
 * Host. Token masks of every cell pattern of a 64 x 64 tile for sa_mask_cells_to_kv_list:
 * masks[p][r] bit k is set when the cell holding (query r, key k) of the tile is set in
 * pattern p. *n_patterns = 2^(cells per tile) (at most 65 536, for 16 x 16 blocks);
 * masks = NULL: count only.
 */
int sa_cell_tile_masks(int block_m, int block_n, uint64_t* masks, int64_t* n_patterns);

/*
 * Block-sparse attention forward: out = softmax(q k^T * sm_scale [+ key_bias]) v restricted,
 * for each 64-row query block, to the 64-key blocks in its kv list.
 * Replaces `block_sparse_triton_fn` / `_forward` / `_fwd_kernel`
 * (utils/block_sparse_attn_kernel.py:52-265, 293): same masking of the partial last key
 * block (:87-89), fp32 online softmax, P rounded to bf16 before P.V (:107), no causal
 * mask, query-block m uses mask row m (:155). A query block with an empty list writes 0
 * (the reference divides by l=0 and writes NaN, :201-203).
 *   q [B,H,Lq,D], k/v [B,H,Lk,D], out [B,H,Lq,D]: bf16, strides as above; D = 64 or 128,
 *             the head dims the reference accepts (:231).
 *   kv_idx/kv_cnt: lists for B*H*ceil(Lq/64) rows (row = (b*H + h)*nqb + m); entries
 *             outside [0, ceil(Lk/64)) are skipped, counts are clamped to [0, max_cnt].
 *   key_bias  nullable fp32, element [b*bias_strides[0] + h*bias_strides[1] + key]:
 *             added to the scaled scores (proportional attention, MergeAttention.py:33-48).
 *   sm_scale  > 0 and finite.
 *   work_order nullable int32 [n_slots] from sa_attn_work_order (device copy): dispatch
 *             slot -> list row, -1 = idle. NULL visits rows in index order.
 * One wave per query block, never split into key ranges (sa_block_sparse_fwd_split is the
 * variant for few query blocks over long lists).
 */
int sa_block_sparse_fwd(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                        const int64_t k_strides[3], const uint16_t* v,
                        const int64_t v_strides[3], uint16_t* out,
                        const int64_t out_strides[3], int B, int H, int Lq, int Lk, int D,
                        const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                        const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                        const int32_t* work_order, int64_t n_slots, void* stream);

/*
 * sa_block_sparse_fwd with the scores in fp16 (same block_sparse_attn_kernel.py:52-209 work,
 * bf16 q, k, v and out, head dim 64 with an optional key_bias as there, or head dim 128 without
 * one; other head dims, or 128 with a key_bias, return SA_ERR_UNSUPPORTED). The workspace
 * (sa_block_sparse_fwd_k16_workspace with the same D; sa_block_pool_k16 writes it for D = 64
 * only) holds an fp16 copy of k (round
 * to nearest even: exact for 2^-17 <= |k| < 65504, on fp16's subnormal grid below, an absolute
 * error of at most 2^-25) and the largest squared key-row norm of each 64-row key block,
 * written by sa_block_sparse_fwd_k16_prepare or sa_block_pool_k16 (or by this call first, with
 * prepared = 0). Each query block forms its operands fp16(q * sm_scale * log2(e)) in registers,
 * so that S = q k^T lands in the exp2 domain and the softmax takes no multiply per score. A
 * query block uses these operands when its largest row norm of q * sm_scale * log2(e) times the
 * head's largest key-row norm is at most 32, with both squared norms below 4e9: that bounds
 * every |S * sm_scale * log2(e)| by 32 (Cauchy-Schwarz), and the 2^-11 relative rounding of each
 * q element then moves a score by at most 2^-6 in the exp2 domain. Any other query block (or
 * one with a NaN norm) runs exactly as in sa_block_sparse_fwd. Row sums, P (bf16) and P.V are
 * as there. A key bias is first written to the workspace multiplied by log2(e) (the product the
 * bf16 path forms per tile), and the fp16 path's S MFMAs start from it. The fp16 operands have no counterpart in the reference, whose kernel scales the
 * fp32 scores (:84-85).
 *   workspace  256-byte aligned, >= sa_block_sparse_fwd_k16_workspace(B, H, Lk, 64, with_bias)
 *              bytes (with_bias: room for the scaled bias too); with prepared = 1 it must hold
 *              this k's preparation, done earlier in stream order (another stream: the caller
 *              orders the two).
 */
int sa_block_sparse_fwd_k16_workspace(int B, int H, int Lk, int D, int with_bias, int64_t* bytes);
int sa_block_sparse_fwd_k16_prepare(const uint16_t* k, const int64_t k_strides[3], int B, int H, int Lk,
                                    int D, void* workspace, int64_t workspace_bytes, void* stream);
int sa_block_sparse_fwd_k16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                            const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                            uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                            int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                            const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                            const int32_t* work_order, int64_t n_slots, int prepared, void* workspace,
                            int64_t workspace_bytes, void* stream);

/*
 * sa_block_sparse_fwd for fp16 q, k, v and out (the reference kernel runs on either 16-bit
 * type: P is rounded to v's dtype, :107): same arguments and contract, D = 64 or 128, with the
 * fp16 MFMA and P rounded to fp16. fp16 P has too little exponent range for the unshifted
 * exp2 that bf16 launches try first, so an item's first pass subtracts, from every score of a
 * row, the row's maximum over the item's first tile; an item in which a later score exceeds
 * that by 2^16 or more (P rounds to inf) is redone with the running row maximum.
 */
int sa_block_sparse_fwd_f16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                            const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                            uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                            int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                            const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                            const int32_t* work_order, int64_t n_slots, void* stream);

/*
 * sa_block_sparse_fwd (bf16, head dim 64) where only the first 32 columns of v enter P.V and
 * out has 32 columns: v [B,H,Lk,64] as there (its tiles are read whole), out [B,H,Lq,32].
 * For a v whose other columns are zero or unused: the segment-indicator v of the
 * frame-pattern masses (ParternAttentionColVersion_V2.get_weight_for_patch and the
 * first-frame softmax and its segment sums, partern_attention.py:321-358, 413, 430, 443) has
 * 1 + frames <= 32 nonzero columns. Same lists, key_bias, work order and error contract;
 * never split into key ranges.
 */
int sa_block_sparse_fwd_v32(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                            const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                            uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                            const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                            const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                            const int32_t* work_order, int64_t n_slots, void* stream);

/*
 * sa_block_sparse_fwd for fp32 q, k, v and out (the reference kernel also runs on fp32 tiles,
 * :52-209, with P cast to v's dtype, :107, so kept in fp32): same arguments and list contract,
 * head dim 64 or 128 (:231), key_bias must be NULL (SA_ERR_UNSUPPORTED otherwise). fp32 MFMA
 * (v_mfma_f32_16x16x4_f32), running row maximum, P and row sums in fp32. Strides in elements,
 * multiples of 4; bases 16-byte aligned.
 */
int sa_block_sparse_fwd_f32(const float* q, const int64_t q_strides[3], const float* k,
                            const int64_t k_strides[3], const float* v, const int64_t v_strides[3],
                            float* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                            int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                            const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                            const int32_t* work_order, int64_t n_slots, void* stream);

/*
 * Block-sparse attention with token-level masks inside cut blocks: as sa_block_sparse_fwd
 * (bf16, D = 64 or 128), plus kv_slot[row][i] = -1 (every pair of the tile attends) or the index of a 64x64
 * bitmask in tile_masks (uint64 [slots][64]: bit c of word r = query r of the block may
 * attend key c). Replaces flex_attention with a BlockMask built from a mask_mod
 * (SildingTileAttention.py:88-106, 146), which also masks element-wise inside partial blocks.
 * lists_shared != 0: one set of lists (nqb rows) is used by every (b, h), as the
 * reference's B=H=1 BlockMask broadcasts.
 */
int sa_block_sparse_fwd_tilemask(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                 const int64_t k_strides[3], const uint16_t* v,
                                 const int64_t v_strides[3], uint16_t* out,
                                 const int64_t out_strides[3], int B, int H, int Lq, int Lk, int D,
                                 const int32_t* kv_idx, const int32_t* kv_cnt, const int32_t* kv_slot,
                                 int max_cnt, int lists_shared, const uint64_t* tile_masks,
                                 float sm_scale, const int32_t* work_order, int64_t n_slots,
                                 void* stream);

/*
 * Block-sparse attention over a remapped token layout, with the layout transform done by
 * the kernel's own loads and stores instead of copies. Replaces the permute-attend-unpermute
 * sequences of the reference: the sliding-tile layout (SildingTileAttention.py:111-143), the
 * 1.5-5B rearranger/recover (combined_attn.py:17-41) and the per-frame pad/truncate of
 * preprocess_qkv/reverse_process_out (utils/mask_related.py:87-187) on the query side.
 * As sa_block_sparse_fwd_tilemask (kv_slot and tile_masks both NULL: plain lists) with an
 * optional key_bias as in sa_block_sparse_fwd (not together with tile masks), plus:
 *   q_rows    nullable int32 [Lq]: logical query i reads q row q_rows[i]; an entry outside
 *             [0, q_src_rows) reads zeros (padding). NULL: q row i (q_src_rows ignored).
 *   o_rows    nullable int32 [Lq]: logical query i is written to out row o_rows[i]; an entry
 *             outside [0, o_dst_rows) is not written. NULL: out row i.
 * Lq is the logical query count (the kv lists index its 64-row blocks); k/v are in the
 * logical key order. The caller must not map two queries to one out row.
 */
int sa_block_sparse_fwd_mapped(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                               const int64_t k_strides[3], const uint16_t* v,
                               const int64_t v_strides[3], uint16_t* out,
                               const int64_t out_strides[3], int B, int H, int Lq, int Lk, int D,
                               const int32_t* kv_idx, const int32_t* kv_cnt, const int32_t* kv_slot,
                               int max_cnt, int lists_shared, const uint64_t* tile_masks,
                               const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                               const int32_t* q_rows, int q_src_rows, const int32_t* o_rows,
                               int o_dst_rows, const int32_t* work_order, int64_t n_slots,
                               void* stream);

/*
 * sa_block_sparse_fwd_mapped for fp16 q, k, v and out: same arguments and contract, computed
 * as sa_block_sparse_fwd_f16 (fp16 MFMA, P rounded to fp16, first-tile row offsets).
 */
int sa_block_sparse_fwd_mapped_f16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                   const int64_t k_strides[3], const uint16_t* v,
                                   const int64_t v_strides[3], uint16_t* out,
                                   const int64_t out_strides[3], int B, int H, int Lq, int Lk, int D,
                                   const int32_t* kv_idx, const int32_t* kv_cnt, const int32_t* kv_slot,
                                   int max_cnt, int lists_shared, const uint64_t* tile_masks,
                                   const float* key_bias, const int64_t bias_strides[2], float sm_scale,
                                   const int32_t* q_rows, int q_src_rows, const int32_t* o_rows,
                                   int o_dst_rows, const int32_t* work_order, int64_t n_slots,
                                   void* stream);

/*
 * Dense or causal attention that also returns the 2-D max-pooled attention map, a block-score
 * source (attn_with_pooling = _attention_pooling.forward, utils/attn_pooling_kernel.py:18-289):
 *   out[b,h,r] = softmax_c(q[b,h,r] . k[b,h/(H/H_kv),c] * sm_scale) v[...]     bf16 [B,H,L,D]
 *                (causal: keys c <= r only)
 *   Po[b,h,i,j] = max over queries r of block i and keys c of block j of the softmax P[r][c],
 *                 then each row of Po divided by its sum                          fp32 [B,H,nd,nd]
 * with D = 64 or 128, blocks of block_size in {32, 64, 128} tokens, nd = ceil(L / block_size)
 * <= 8192, and
 * Po[i][j] = 0 for j > i when causal. k and v have H_kv heads (H_kv divides H). Po has
 * element strides po_strides (b, h, i) and unit stride over j. workspace: at least
 * sa_attn_pooling_workspace() bytes, 256-byte aligned (kv lists, per-row maxima of every
 * G-key column and log-sum-exps: about 4*B*H*L*L/G bytes, G = 32 for block_size 32, else 64).
 */
int sa_attn_pooling_workspace(int B, int H, int L, int block_size, int64_t* bytes);
int sa_attn_pooling_fwd(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                        const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                        uint16_t* out, const int64_t out_strides[3], int B, int H, int H_kv, int L,
                        int D, int causal, float sm_scale, int block_size, float* po,
                        const int64_t po_strides[3], void* workspace, int64_t workspace_bytes,
                        void* stream);

/*
 * sa_attn_pooling_fwd for fp32 q, k, v and out, in fp32 arithmetic as the reference computes
 * (:230-240 casts bf16 inputs to fp32 and runs the kernel on fp32 tiles, P kept in fp32):
 * the attention of sa_block_sparse_fwd_f32 (fp32 MFMA, running row maximum) over every key
 * block (causal: up to the diagonal, the diagonal tile masked to keys <= query), grouped key
 * heads as there; the rows' column maxima and log-sum-exps go to the workspace and a reduce
 * kernel forms Po for every block size. D = 64 or 128; same workspace
 * (sa_attn_pooling_workspace), strides in elements, multiples of 4.
 */
int sa_attn_pooling_fwd_f32(const float* q, const int64_t q_strides[3], const float* k,
                            const int64_t k_strides[3], const float* v, const int64_t v_strides[3],
                            float* out, const int64_t out_strides[3], int B, int H, int H_kv, int L,
                            int D, int causal, float sm_scale, int block_size, float* po,
                            const int64_t po_strides[3], void* workspace, int64_t workspace_bytes,
                            void* stream);

/*
 * sa_attn_pooling_fwd for fp16 q, k, v and out (the reference also takes fp16, :230-289):
 * same arguments and contract, the attention computed as sa_block_sparse_fwd_f16; Po and the
 * workspace stay fp32.
 */
int sa_attn_pooling_fwd_f16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                            const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                            uint16_t* out, const int64_t out_strides[3], int B, int H, int H_kv, int L,
                            int D, int causal, float sm_scale, int block_size, float* po,
                            const int64_t po_strides[3], void* workspace, int64_t workspace_bytes,
                            void* stream);

/*
 * (host) Dispatch order of the attention work items (one per list row) for a GPU whose
 * workgroups are dealt round-robin to n_xcd XCDs (8 on MI355X): each XCD gets a
 * contiguous range of (b, h) heads, so their K/V stay in that XCD's L2, and within it the
 * text block rows (longest lists) come first. No counterpart in the reference, whose grid
 * is (ceil(Lq/64), B*H) in launch order (block_sparse_attn_kernel.py:229).
 *   order     NULL to query *n_slots only; else int32 [*n_slots] filled on the host.
 */
int sa_attn_work_order(int B, int H, int nqb, int n_text_blocks, int n_xcd, int32_t* order,
                       int64_t* n_slots);

/*
 * Host. Suggested key-range parts per query block for sa_block_sparse_fwd_split: a launch of
 * n_items = B*H*ceil(Lq/64) query blocks with lists of width max_cnt, head dim D, on a device
 * of n_cus compute units (MI355X: 256). *parts = 1: no split. Parts are chosen to fill the
 * wave slots (n_cus x 8 waves at D = 64, x 4 at 128) once, with at least 32 list positions per
 * part at the list width, at most 16; lists narrower than 64 are never split, nor launches
 * whose blocks fill half the slots. A pure function of its arguments (no device query). No
 * counterpart in the reference (its Triton launch has one program per query block).
 */
int sa_attn_split_parts(int64_t n_items, int max_cnt, int D, int n_cus, int* parts);

/*
 * Host. Workspace bytes sa_block_sparse_fwd_split needs for n_items query blocks, head dim D
 * and `parts` key-range parts (1..16): n_items * parts * (64*D + 128) * 4 (fp32 acc, row
 * sums and row maxima per part); 0 for parts = 1.
 */
int sa_attn_split_workspace(int64_t n_items, int D, int parts, int64_t* bytes);

/*
 * Block-sparse attention with each query block's list split into `parts` key ranges: as
 * sa_block_sparse_fwd (bf16, D = 64 or 128, plain lists, no key_bias) with the optional row
 * maps of sa_block_sparse_fwd_mapped (NULL: identity), for launches with few query blocks
 * over long lists, where one wave per block would leave most of the GPU idle. Part p of a
 * block with c list entries visits positions [c*p/parts, c*(p+1)/parts) in one wave and stores
 * its unnormalised fp32 partial (acc, row sum, row maximum) to `workspace`; a second kernel
 * on the same stream rescales the partials by their row maxima, sums them in part order and
 * normalises once. The output is a deterministic function of the arguments (parts included)
 * and equals the unsplit launch up to the fp32 summation order (one bf16 rounding step);
 * parts = 1 is the unsplit launch itself.
 * Replaces the same reference work as sa_block_sparse_fwd
 * (utils/block_sparse_attn_kernel.py:52-265), one Triton program per query block there.
 *   parts      1..16 (sa_attn_split_parts suggests one).
 *   workspace  device memory of >= sa_attn_split_workspace(B*H*ceil(Lq/64), D, parts) bytes,
 *              16-byte aligned, owned by the caller; read and written by this call's kernels
 *              on `stream` only (free or reuse it after them in stream order). NULL only with
 *              parts = 1.
 */
int sa_block_sparse_fwd_split(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                              const int64_t k_strides[3], const uint16_t* v, const int64_t v_strides[3],
                              uint16_t* out, const int64_t out_strides[3], int B, int H, int Lq, int Lk,
                              int D, const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                              float sm_scale, const int32_t* q_rows, int q_src_rows,
                              const int32_t* o_rows, int o_dst_rows, int parts, void* workspace,
                              int64_t workspace_bytes, void* stream);

/* sa_block_sparse_fwd_split for fp16 q, k, v and out (P rounded to fp16; each part offsets its
 * rows by their maxima over the part's first tile, as sa_block_sparse_fwd_f16). */
int sa_block_sparse_fwd_split_f16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                                  const int64_t k_strides[3], const uint16_t* v,
                                  const int64_t v_strides[3], uint16_t* out,
                                  const int64_t out_strides[3], int B, int H, int Lq, int Lk, int D,
                                  const int32_t* kv_idx, const int32_t* kv_cnt, int max_cnt,
                                  float sm_scale, const int32_t* q_rows, int q_src_rows,
                                  const int32_t* o_rows, int o_dst_rows, int parts, void* workspace,
                                  int64_t workspace_bytes, void* stream);

/*
 * Block means of q and k: pooled[(b*H + h)*nb + blk][d] = mean over the block's tokens,
 * nb = ceil(L/block), the last block averaging its L - (nb-1)*block tokens.
 * Replaces the pooling half of the block-score estimator calc_attn_block_sum_efficient
 * (utils/mask_related.py:40-81: replicate-pad, 8 random tokens per block, conv2d sum-pool)
 * with the deterministic mean-pool of the top-k mask rule. Bit-exact contract: fp32 sum of
 * the block's tokens in ascending order, then one IEEE division by the token count.
 *   q, k      bf16 [B,H,L,64] (k may be NULL to pool q only); pooled outputs fp32
 *             contiguous [B*H][nb][64].
 */
int sa_block_pool(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                  const int64_t k_strides[3], int B, int H, int L, int D, int block,
                  float* q_pooled, float* k_pooled, void* stream);

/*
 * sa_block_pool with block = 64 whose k pass also writes the workspace of
 * sa_block_sparse_fwd_k16 for this k (the fp16 copy and the per-block key norms, the same
 * bits as sa_block_sparse_fwd_k16_prepare), so that the attention call can pass prepared = 1
 * (this pass reads k anyway). No counterpart in the reference.
 *   workspace  256-byte aligned, >= sa_block_sparse_fwd_k16_workspace(B, H, L, 64) bytes.
 */
int sa_block_pool_k16(const uint16_t* q, const int64_t q_strides[3], const uint16_t* k,
                      const int64_t k_strides[3], int B, int H, int L, int D, float* q_pooled,
                      float* k_pooled, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Per-row top-k block selection -> kv lists.
 * Replaces get_sparse_attn_mask_from_topk (utils/block_sparse_attn_kernel.py:31-39:
 * torch.topk + scatter) and the top-k/scatter of transfer_attn_to_mask with text rows and
 * columns forced dense (SparseGen_Plus.py:28-50, 81-82); `local_bitmap` adds the static
 * local-window part of the combined mask (union, as LocalGlobalAttention.py:227-237).
 * For row r of head bh, the scores are score[c] = sum_d q_pooled[bh][r][d] *
 * k_pooled[bh][c][d] (fmaf chain, d ascending) or scores_in[bh][r][c]; the kept set is the
 * first `topk` columns in (score descending, column ascending) order, united with columns
 * < n_text_blocks, all columns when r < n_text_blocks, and local_bitmap[r][c] != 0.
 *   q_pooled [BH][nqb][D], k_pooled [BH][nkb][D] fp32 (D = 64), or scores_in fp32
 *             [BH][nqb][nkb] (then the pooled inputs may be NULL). nkb <= 1024.
 *   kv_idx    int32 [BH*nqb][max_cnt] (max_cnt >= nkb), kv_cnt int32 [BH*nqb].
 *   mask_out  nullable uint8 [BH][nqb][nkb] (1 = kept); scores_out nullable fp32, same shape.
 */
int sa_block_topk_kv_list(const float* q_pooled, const float* k_pooled, const float* scores_in,
                          int BH, int nqb, int nkb, int D, int topk, int n_text_blocks,
                          const uint8_t* local_bitmap, int32_t* kv_idx, int max_cnt,
                          int32_t* kv_cnt, uint8_t* mask_out, float* scores_out, void* stream);

/*
 * Sampled tokens of the adaptive estimator.
 * Replaces random_sample_tokens + pad_to_multiple (utils/mask_related.py:2-37): for every
 * 64-token block of q (and of k), the tokens at the num_keep largest of the block's 64
 * uniform draws, in (draw descending, position ascending) order -- torch.topk(sorted=True)
 * -- where positions past L stand for token L-1 (the reference's replicate padding).
 *   rand_q, rand_k  fp32 contiguous [B*H][nb][64] draws, nb = ceil(L/64) (rand_k, k,
 *             k_strides, tok_k, k_sampled NULL: sample q only).
 *   tok_q/tok_k nullable int32 [B*H][nb*num_keep] token ids.
 *   q_sampled, k_sampled  bf16 [B*H][ns_pad][64] (rows >= nb*num_keep are not written).
 *   1 <= num_keep <= 64, ns_pad >= nb*num_keep, D = 64.
 */
int sa_sample_block_tokens(const float* rand_q, const uint16_t* q, const int64_t q_strides[3],
                           const float* rand_k, const uint16_t* k, const int64_t k_strides[3],
                           int B, int H, int L, int D, int num_keep, int32_t* tok_q, int32_t* tok_k,
                           uint16_t* q_sampled, uint16_t* k_sampled, int ns_pad, void* stream);

/*
 * Sampled block scores of the adaptive estimator.
 * Replaces the attention-and-pool part of calc_attn_block_sum_efficient
 * (utils/mask_related.py:62-81): with ns = nb*num_keep sampled rows per head,
 * a = softmax_j(sq_i . sk_j / 8) and pooled[bh][I][J] = sum of a over the num_keep x
 * num_keep cell (I, J) (the conv2d with a ones kernel and stride num_keep). fp32 throughout
 * (the reference rounds scores, softmax and sums to bf16).
 *   q_sampled, k_sampled from sa_sample_block_tokens; num_keep 8 or 16; ns_pad = ns rounded
 *             up to a multiple of 32.
 *   pooled    fp32 [B*H][nb][nb].
 */
int sa_sampled_block_scores(const uint16_t* q_sampled, const uint16_t* k_sampled, int BH, int nb,
                            int num_keep, int ns_pad, float* pooled, void* stream);

/*
 * Energy-threshold / adaptive top-k block selection -> kv lists.
 * Replaces transfer_attn_to_mask (SparseGen_Plus.py:12-84). Per score row (n = nkb columns):
 * ranks in (score descending, column ascending) order and sequential fp32 prefix sums cum[]
 * in rank order, total = cum[n-1]; keeps the columns of rank < k with
 *   mode 0 ("energy"): k = n if total < threshold*total, else the first j with
 *             cum[j] >= threshold*total; then k = min(max(k, min_keep), max_keep)
 *             (:57-73: the crossing column itself is not kept before clamping);
 *   mode 1 ("topk"): k = init_k; if cum[init_k-1] < 0.6*total and init_k < n, k = min(3k, n);
 *             then if cum[init_k-1] < 0.9*total and init_k < n, k = min(k/3*2, n) (:31-46);
 *   mode 2 ("inclusive"): k = 1 + the first j with cum[j] >= threshold*total (k = n when
 *             none), then clamped to [min_keep, max_keep]: the frame-scope and row-scope
 *             energy cuts of generate_attention_mask_frame_scope / get_inner_frame_mask
 *             (utils/mask_related.py:224-232, 366-376: crossing column kept, last forced);
 *   mode 3 ("cumulative <="): the ranks j with cum[j] <= threshold*total, plus rank n-1
 *             (the head-scope cut of get_inner_frame_mask, utils/mask_related.py:378-391);
 * united with columns < n_text_blocks and every column of rows < n_text_blocks (:81-82).
 *   scores    fp32 [BH][nqb][nkb], nkb <= 1024; kv_idx int32 [BH*nqb][max_cnt >= nkb],
 *             kv_cnt int32 [BH*nqb]; mask_out nullable uint8 [BH][nqb][nkb].
 *   min_keep/max_keep/init_k are the reference's integers (max(1, int(seq*ratio)), ...).
 */
int sa_energy_kv_list(const float* scores, int BH, int nqb, int nkb, int mode, float threshold,
                      int min_keep, int max_keep, int init_k, int n_text_blocks, int32_t* kv_idx,
                      int max_cnt, int32_t* kv_cnt, uint8_t* mask_out, void* stream);

/*
 * Per-head token gather out[b,h,j] = x[b,h, idx[(b*H + h)*L_out + j]] (zero row outside
 * [0, L_in)). Replaces the per-head query-frame gather gather_q_chunk of the pattern
 * attention (partern_attention.py:378-384, torch.gather with per-head frame indices).
 */
int sa_gather_tokens_heads(const uint16_t* x, const int64_t x_strides[3], int B, int H, int L_in,
                           int D, const int32_t* idx, int L_out, uint16_t* out,
                           const int64_t out_strides[3], void* stream);

/*
 * Frame maps of the pattern attention (get_weight_for_patch, partern_attention.py:321-358)
 * from the sampled attention's segment masses map_mass [B,H,F*ns,>=F+1] (bf16; row = sampled
 * video query, column 0 = mass on the text keys, 1 + f = mass on frame f's samples):
 *   img2text[bh][f] = sum of column 0 over frame f's ns rows / ns      (fp32 [B*H][F])
 *   img2img[bh][f1][f2] = sum of column 1 + f2 over frame f1's rows / ns (fp32 [B*H][F][F])
 */
int sa_pattern_maps(const uint16_t* map_mass, const int64_t map_strides[3], int B, int H, int F,
                    int ns, float* img2text, float* img2img, void* stream);

/*
 * Per-head plan of the pattern attention (partern_attention.py:262-315, 412-435) from the
 * first-frame masses ff_mass [B,H,S,>=F+1] (bf16; column 0 text, 1 + i frame i) and img2img:
 *   stats   fp32 [B*H][F+1][3]: sum, min, max of each mass column over the S rows;
 *   fac     fp32 [B*H][F+1][4]: the modify factor x -> constrained_mod_factor(x / mean(x))
 *           as {1/mean, alpha, beta, mode} (mode 0 unchanged, 1 clamp, 2 clamp(alpha x + beta)),
 *           bounds [lo_text, hi_text] for column 0 and [lo_frame, hi_frame] for the frames,
 *           the "any head out of range" decision taken over all B*H heads per column;
 *   frame_case int32 [B*H][F]: 1 if img2img[0][i] >= map_thr (first-frame masses are used
 *           for key frame i), else 0 (queries of frame argmax_f img2img[f][i]);
 *   inv_map0 fp32 [B*H][F]: 1 / img2img[0][i];
 *   q_idx   int32 [B*H][F*S]: query token T + frame*S + r of selected row i*S + r.
 */
int sa_pattern_plan(const uint16_t* ff_mass, const int64_t ff_strides[3], const float* img2img,
                    int B, int H, int F, int S, int T, float lo_text, float hi_text,
                    float lo_frame, float hi_frame, float map_thr, float* stats, float* fac,
                    int32_t* frame_case, float* inv_map0, int32_t* q_idx, void* stream);

/*
 * Final mix of the pattern attention (partern_attention.py:447-452): for video row f1*S + r,
 *   out[T + f1*S + r] = sum_i img2img[f1][i] * s_i(r) * o_frames[i*S + r]
 *                       + img2text[f1] * mft(r) * o_text[f1*S + r]
 * with s_i(r) the frame-i modify factor (frame_case 0) or ff_mass[r][1+i] * inv_map0[i]
 * (frame_case 1) and mft(r) the text modify factor, both from fac. Rows < T of out are not
 * touched. o_frames/o_text [B,H,F*S,64], out [B,H,T+F*S,64] bf16; F <= 16.
 */
int sa_pattern_combine(const uint16_t* o_frames, const int64_t of_strides[3], const uint16_t* o_text,
                       const int64_t ot_strides[3], const uint16_t* ff_mass,
                       const int64_t ff_strides[3], const float* img2text, const float* img2img,
                       const float* fac, const int32_t* frame_case, const float* inv_map0, int B,
                       int H, int F, int S, int T, float lo_text, float hi_text, float lo_frame,
                       float hi_frame, uint16_t* out, const int64_t out_strides[3], void* stream);

/*
 * constrained_mod_factor (partern_attention.py:262-315) of a factor tensor x fp32 [BH][L]
 * (the reference's [B, H, L, 1]): unchanged when every head lies within [lo, hi]; otherwise each
 * head (range >= 1e-6) is mapped affinely from [min, max] onto [max(min, lo), min(max, hi)],
 * rescaled to its original sum, and every value is clamped to [lo, hi]. stats fp32 [BH][3]
 * receives each head's sum, min and max (caller buffer). BH <= 4096.
 */
int sa_constrained_mod_factor(const float* x, int BH, int64_t L, float lo, float hi, float* stats,
                              float* out, void* stream);

/*
 * Softmax probabilities of sampled queries over sampled keys, for the head-routing judges
 * (judge_sparsity / judge_similarity, partern_attention.py:468-514):
 *   P[bh][r][c - c_lo] = softmax_c(q_rows[bh][r] . k_rows[bh][c] * sm_scale + (c < n_bias ? bias : 0))
 * over all `keys` keys, written for c in [c_lo, c_hi) and r < rows.
 *   q_rows [BH][rows_pad][64], k_rows [BH][keys_pad][64] bf16 contiguous (pads: multiples of
 *   32; padded rows are not read as keys); P fp32 with strides p_bh_stride, p_row_stride.
 */
int sa_sampled_probs(const uint16_t* q_rows, const uint16_t* k_rows, int BH, int rows, int rows_pad,
                     int keys, int keys_pad, float sm_scale, int n_bias, float bias, int c_lo,
                     int c_hi, float* P, int64_t p_bh_stride, int64_t p_row_stride, void* stream);

/*
 * Per row of P (n >= 0 entries, n <= 16384): the sum of its K largest entries, 1 <= K <= n
 * (judge_sparsity's sorted-prefix share, partern_attention.py:474-475). share fp32 [BH][rows].
 */
int sa_topk_share(const float* P, int64_t p_bh_stride, int64_t p_row_stride, int BH, int rows,
                  int n, int K, float* share, void* stream);

/*
 * Gram matrices of the sampled frame-pair attention patterns (judge_similarity,
 * partern_attention.py:502-512): with P the [F*ns x F*ns] video part of the sampled
 * probabilities, G[bh][f2][chunk][pair(f1,f3)] = sum over s1 in the chunk (8 positions)
 * and all s2 of P[f1*ns + s1][f2*ns + s2] * P[f3*ns + s1][f2*ns + s2], f1 <= f3 (pairs in
 * row-major upper-triangle order). F <= 12, ns <= 512.
 */
int sa_pattern_gram(const float* P, int64_t p_bh_stride, int64_t p_row_stride, int BH, int F,
                    int ns, float* G, void* stream);

/*
 * The Gram partials of sa_pattern_gram computed straight from the sampled rows, without
 * writing the probabilities (judge_similarity, partern_attention.py:477-514): q_rows
 * [BH][rows_pad][64] holds the F*ns sampled video queries (row f*ns + s), k_rows
 * [BH][keys_pad][64] the T text keys then the F*ns sampled keys (bf16 contiguous, pads:
 * multiples of 32); the probabilities are softmax over all T + F*ns keys of
 * q . k * sm_scale (+ bias on the T text keys). G as sa_pattern_gram; F <= 12.
 */
int sa_pattern_sim_gram(const uint16_t* q_rows, const uint16_t* k_rows, int BH, int F, int ns,
                        int T, int rows_pad, int keys_pad, float sm_scale, float bias, float* G,
                        void* stream);

/*
 * Routing decision of unified_judge (partern_attention.py:516-521) per head:
 * share_mean = mean of share over rows (NULL: 0), col = mean over key frames f2 of the mean
 * over (f1, f3) of the cosine G[f1][f3] / sqrt(G[f1][f1] G[f3][f3]) from the Gram partials
 * (G1/G2 NULL: 0), use = share_mean <= sparse_thr && col1 > sim_thr && col2 > sim_thr.
 */
int sa_pattern_judge_finish(const float* share, const float* G1, const float* G2, int BH,
                            int rows, int F, int ns, float sparse_thr, float sim_thr,
                            float* share_mean, float* col1, float* col2, int32_t* use,
                            void* stream);

/*
 * Row-group sums: out[b*H + h][g][c] = sum over rows r in [g*R, min(L, g*R + R)) of
 * x[b, h, r, col0 + c] (fp32, rows ascending), c < ncols, col0 + ncols <= 64, g < ceil(L/R).
 * With x the key-block masses of a frame's attention (the attention of the frame's queries
 * over its keys with a 0/1 key-block indicator as v), these are the 64 x 64 cell sums of
 * get_inner_frame_mask (utils/mask_related.py:352-361: calc_attn, then the (s1 s2) sum).
 */
int sa_row_group_sums(const uint16_t* x, const int64_t x_strides[3], int B, int H, int L,
                      int rows_per_group, int col0, int ncols, float* out, void* stream);

/*
 * Kronecker fusion of get_block_mask (utils/mask_related.py:397-404): for each of BH heads,
 * out[i][j] (fp32 0/1, [F*Ri + pad][F*Ci + pad]) = frame_mask[i / Ri][j / Ci] &&
 * inner_mask[i % Ri][j % Ci] for i < F*Ri and j < F*Ci, and 1 on the `pad` trailing (text)
 * rows and columns, as the reference's pad(value=1). frame_mask uint8 [BH][F][F],
 * inner_mask uint8 [BH][Ri][Ci].
 */
int sa_kron_block_mask(const uint8_t* frame_mask, const uint8_t* inner_mask, int BH, int F, int Ri,
                       int Ci, int pad, float* out, void* stream);

/*
 * (host) Static local 3-D window of the combined mask, one byte per (query block, key
 * block): 1 iff both blocks are video blocks and their centre tokens (index
 * block*qb + block/2, clamped to L-1) lie within +-dt latent frames, +-dh patch rows and
 * +-dw patch columns of each other. Text rows/columns are 0 here (the top-k kernel adds
 * them). Plays the role of the static local-window masks of the reference: the 3-D tile
 * window of generate_sta_mask (SildingTileAttention.py:18-87), the +-1-frame tridiagonal
 * of SmartAttention.py:56-67 and the local part of LocalGlobalAttention.py:114-179.
 *   bitmap    uint8 [nb][nb], nb = ceil(L/block); L must equal text_len + T*Hp*Wp.
 */
int sa_local_window_bitmap(int L, int block, int text_len, int T, int Hp, int Wp, int dt, int dh,
                           int dw, uint8_t* bitmap);

/*
 * (host) The local window of sa_local_window_bitmap for a permuted token layout: position j
 * holds natural token perm[j] (text first, then row-major (t, h, w)); block b's centre token is
 * perm[min(b*block + block/2, L-1)], and two video centres are in the window as above. Every
 * row and column of a block holding any text token is set (the layout may put the text
 * anywhere, e.g. last in the 1.5-5B rearranger of combined_attn.py:17-31, so the top-k
 * kernel's leading n_text_blocks cannot express it). bitmap uint8 [nb][nb].
 */
int sa_local_window_bitmap_perm(int L, int block, int text_len, int T, int Hp, int Wp, int dt, int dh,
                                int dw, const int32_t* perm, uint8_t* bitmap);

/*
 * (host) Tile-major token order of sliding-tile attention (SildingTileAttention.py:111-131):
 * perm[j] = natural token at position j; text tokens stay first, video tokens are grouped
 * "(nt tt nh th nw tw) -> (nt nh nw tt th tw)" for tile = {tt, th, tw} dividing (T, Hp, Wp).
 */
int sa_sta_permutation(int text_len, int T, int Hp, int Wp, const int tile[3], int32_t* perm);

/*
 * (host) The sliding-tile mask (sta_mask_3d, SildingTileAttention.py:18-87: video pairs
 * within the kernel-sized window of tiles around the query tile, the centre clamped to the
 * canvas; video->text; text->all), on the tile-major layout, as 64x64 block lists: kv_idx /
 * kv_cnt / kv_slot [nb][nb] per query block (non-empty key blocks ascending; slot -1 for a
 * full block) and the bitmasks of the partial blocks. kv_idx = NULL: count *n_slots only.
 */
int sa_sta_block_masks(int text_len, int T, int Hp, int Wp, const int tile[3], const int kernel[3],
                       int32_t* kv_idx, int32_t* kv_cnt, int32_t* kv_slot, uint64_t* masks,
                       int* n_slots);

/*
 * Token gather out[b,h,j] = x[b,h,idx[j]] for j < L_out (16-bit elements, D a multiple of 8);
 * an index outside [0, L_in) gives a zero row. Serves the layout transforms that are copies: the sliding-tile order of k and v
 * (SildingTileAttention.py:111-131), the 1.5-5B rearranger/recover (combined_attn.py:17-41),
 * replicate padding (utils/mask_related.py:2-13) and preprocess_qkv/reverse_process_out
 * (utils/mask_related.py:87-187).
 */
int sa_gather_tokens(const uint16_t* x, const int64_t x_strides[3], int B, int H, int L_in, int D,
                     const int32_t* idx, int L_out, uint16_t* out, const int64_t out_strides[3],
                     void* stream);

/* ---- Token merging (ToMe bipartite soft matching) ----------------------------------- */

/*
 * Matching maps of one call, all caller-owned device buffers; G matching groups (one per
 * batch item for the head-averaged metric, one per (b, h) for the per-head metric), N
 * video tokens after text_len text tokens, L = text_len + N, Lm = L - r merged rows laid
 * out [text | unm (edge order) | dst (partition order)] as in merge_unmerge.py:128.
 */
typedef struct sa_tome_maps {
  int G, N, text_len, n_src, n_dst, r, L, Lm;
  const int32_t* a_idx;  /* [n_src] video-token index of each src (partition, all groups) */
  const int32_t* b_idx;  /* [n_dst] video-token index of each dst */
  int32_t* node_idx;     /* [G][n_src] best dst of each src (merge_unmerge.py:108) */
  float* node_max;       /* [G][n_src] its cosine score */
  int32_t* rank;         /* [G][n_src] position of each src in the edge order */
  int32_t* edge;         /* [G][n_src] edge order: src_idx = edge[:r], unm_idx = edge[r:] (:109-111) */
  int32_t* dst_idx;      /* [G][r] dst of the e-th merged src (:112) */
  int32_t* dst_cnt;      /* [G][n_dst] srcs merged into each dst (size - 1, :113-116) */
  int32_t* dst_cursor;   /* [G][n_dst] scratch */
  int32_t* dst_ptr;      /* [G][n_dst + 1] CSR offsets of the members of each dst */
  int32_t* members;      /* [G][r] edge positions grouped by dst, ascending */
  int32_t* row_of_token; /* [G][L] merged row holding each token (the unmerge map, :137-154) */
  float* key_bias;       /* [G][Lm] log(size) rounded to bf16, 0 for text/unm (MergeAttention.py:163-167) */
  int32_t* merged_src;   /* [G][Lm] token row that merged row j starts from: text j, unm its token, dst the dst token */
  int32_t* member_rows;  /* [G][r] token row of each entry of members (the flat gather list of the dst means) */
} sa_tome_maps;

/*
 * (host) src/dst partition of the video tokens of bipartite_soft_matching_video
 * (utils/merge_unmerge.py:62-92): every token of the first frame is dst; frames 1..T-1
 * are cut into (st, sy, sx) cells with one dst per cell at offset cell_choice[cell]
 * (cells [ (T-1)/st ][ Hp/sy ][ Wp/sx ], offset = (dt*sy + dy)*sx + dx; NULL = 0, the
 * reference's no_rand top-left); tokens outside whole cells are src. Within each class
 * tokens are in ascending order (the reference's argsort of the {-1, 0} buffer, made
 * stable). With a_idx = b_idx = NULL only the counts are returned.
 */
int sa_tome_partition(int T, int Hp, int Wp, int sx, int sy, int st, const int32_t* cell_choice,
                      int32_t* a_idx, int32_t* b_idx, int* n_src, int* n_dst);

/*
 * Cosine-normalised matching metric of the video tokens (tokens >= text_len).
 *   mode 0: per batch item, the sum over heads of k (the head mean up to 1/H) -> [B][N][64];
 *   mode 1: per head, (k, |k|, v, |v|) of MergeAttention.py:26-31 -> [B*H][N][130].
 * Each row is divided by its L2 norm (merge_unmerge.py:100). fp32 output, contiguous.
 */
int sa_tome_metric(const uint16_t* k, const int64_t k_strides[3], const uint16_t* v,
                   const int64_t v_strides[3], int B, int H, int L, int D, int text_len, int mode,
                   float* metric, void* stream);

/* Row-wise L2 normalisation of a caller-supplied metric [rows][C] fp32 (merge_unmerge.py:100),
 * the same arithmetic as sa_tome_metric's last step. */
int sa_tome_normalize(const float* metric, int64_t rows, int C, float* out, void* stream);

/* Workspace bytes needed by sa_tome_match (the workspace must be 16-byte aligned). */
int sa_tome_match_workspace(int G, int n_src, int n_dst, int64_t* bytes);

/*
 * Bipartite matching and all merge/unmerge maps (merge_unmerge.py:99-116): per src the dst
 * of highest cosine score (scores never materialised; ties -> lowest dst), edge order by
 * score descending then src position (stable), the top r merged. metric [G][N][C] fp32,
 * C <= 130. Fills every buffer of *maps except a_idx/b_idx, which it reads.
 */
int sa_tome_match(const float* metric, int C, sa_tome_maps* maps, void* workspace,
                  int64_t workspace_bytes, void* stream);

/*
 * sa_tome_match without a workspace argument and without any allocation. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops). The match's split partials and the rank's sorted key tiles
 * live in a device array inside the library (one 16 MiB copy per GPU, held until the process
 * ends); calls that need more than that -- max(G * splits * max(n_src, 1), G * n_src rounded
 * up to 1024) * 8 bytes with splits <= 16, the figure sa_tome_match_workspace returns -- fail
 * with SA_ERR_INVALID. Every call on one GPU shares that array: calls that overlap on
 * one GPU (on different streams or host threads) race and must be serialised by the caller.
 * Results are identical to sa_tome_match's.
 */
int sa_tome_match_noalloc(const float* metric, int C, sa_tome_maps* maps, void* stream);

/*
 * merge closure for a 4-D [B,H,L,64] tensor (merge_unmerge.py:119-128): out [B,H,Lm,64] =
 * [text | unm | dst], each dst row the mean of the dst token and its merged srcs (fp32 sum
 * in edge order, one division, bf16 rounding). Group of head (b, h) = (b*H + h) /
 * heads_per_group (H for the head-averaged metric, 1 for per-head maps).
 */
int sa_tome_merge(const uint16_t* x, const int64_t x_strides[3], int B, int H, int D,
                  int heads_per_group, const sa_tome_maps* maps, uint16_t* out,
                  const int64_t out_strides[3], void* stream);

/*
 * The merge closure applied to n (1..3) tensors of the same [B,H,L,64] shape in one launch,
 * as MergeAttention merges q, k and v with one set of maps (MergeAttention.py:33-38; the
 * merges of merge_unmerge.py:119-128): out[i] = merge(x[i]), each exactly as sa_tome_merge.
 * x_strides / out_strides hold n consecutive {stride_b, stride_h, stride_l} triples.
 */
int sa_tome_merge_multi(int n, const uint16_t* const* x, const int64_t* x_strides, int B, int H, int D,
                        int heads_per_group, const sa_tome_maps* maps, uint16_t* const* out,
                        const int64_t* out_strides, void* stream);

/* unmerge closure (merge_unmerge.py:137-154): out[b,h,t] = xm[b,h,row_of_token[t]]. */
int sa_tome_unmerge(const uint16_t* xm, const int64_t xm_strides[3], int B, int H, int D,
                    int heads_per_group, const sa_tome_maps* maps, uint16_t* out,
                    const int64_t out_strides[3], void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SA_API_H */
