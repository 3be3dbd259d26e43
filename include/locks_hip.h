/*
 * locks_hip.h -- C ABI of liblocks_hip.so, the MI355X (gfx950) LOCKS decode
 * hot path: rki4 page scoring, GQA combine + exact top-b page selection,
 * split-K sparse paged decode with LSE merge.
 *
 * Conventions (same contract as the reference's kernels):
 *   - every pointer is a device pointer; every buffer (outputs, partials,
 *     workspace) is caller-owned and persistent; no entry point allocates;
 *   - bf16 tensors are passed as uint16_t bit patterns;
 *   - `stream` is a hipStream_t (NULL = the default stream); launches are
 *     asynchronous and never synchronize the host, so every entry is safe
 *     inside HIP graph capture;
 *   - strides are in ELEMENTS of the pointed-to type;
 *   - return 0 on success, <0 on a rejected argument (-1) or a failed launch
 *     (-2); locks_last_error() then describes the failure (thread-local).
 *
 * Geometry contract of this build: summary rank 8, int4 basis, 1 <= G <= 16
 * query heads per kv head; the decode entries (split, fused, merge, dense)
 * take head_dim in {64, 128, 256} and page in {16, 32, 64}, the reference's
 * domain (src/locks/selection/rki4_state.py:288-334: d in {64,128,256},
 * page in {16,32,64}, G <= 8; G up to 16 is needed by the GLM-4-9B
 * 32q/2kv geometry); the summary entries (build, score) the same domain
 * (locks_pack_rki4: 128 / 16); MLA: kv_lora_rank 512 + 64 RoPE dims, <= 16
 * query heads.
 *
 * Summary slabs: the six rki4 slabs of one layer are passed as six base
 * pointers plus `slab_row_bytes`, the byte stride between consecutive
 * (block, kv head) rows of each (v4, vs, c8, cs, mu8, mus, in that order).
 * NULL means contiguous slabs of the shapes below (strides 8 d/2, 16, 8 P,
 * 2 P, d and 2 bytes); a state that keeps all six fields of a row together
 * (this package's Rki4State, and the reference's AoS record
 * selection/rki4_state.py:93-110: one record of 5d + 10P + 18 bytes rounded
 * up to 64, fields in the order v4, mu8, c8, cs, vs, mus) passes that record
 * size six times; the scorer then reads each page's record as one stream.  Bases and strides of v4, vs, c8, cs, mu8 are 16-byte aligned, mus
 * 2-byte aligned.
 *
 * Reference interfaces each entry replaces (paths under src/locks/):
 */
#ifndef LOCKS_HIP_H_
#define LOCKS_HIP_H_

#include <stdint.h>

#define LOCKS_ABI_VERSION 10

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version of the loaded library (LOCKS_ABI_VERSION). */
int32_t locks_abi_version(void);

/* Message of the last failed call on this host thread. */
const char* locks_last_error(void);

/*
 * Per-request page parameters for this step.
 * Replaces the Triton _derive_params_kernel / derive_page_params
 * (selection/select.py:28-58):
 *   n_pages = ceil(seq_len / page), n_sel_hi = n_pages - window_pages,
 *   S = n_sel_hi - sink_pages,
 *   b = budget_abs > 0 ? max(min(budget_abs, max(S, 1)), 1)
 *                      : min(max(ceil(S * budget), 1), max(S, 1))   (fp64 ceil)
 */
int32_t locks_derive_params(const int32_t* seq_lens, int32_t n_req, int32_t page,
                            int32_t window_pages, int32_t sink_pages, int32_t budget_abs,
                            double budget, int32_t* n_pages, int32_t* n_sel_hi,
                            int32_t* b_fix, void* stream);

/*
 * Scorer launch shape: pages per workgroup (a multiple of 8) for a state
 * with `max_pages` logical pages, and the resulting number of chunks, which
 * sizes the page-max buffer (n_req, n_kv, chunks, 16) fp32.  Host-only
 * integer math (the reference's auto_zsplit, selection/rki4_score_cuda.py:3161).
 */
int32_t locks_score_auto_chunk(int32_t n_req, int32_t n_kv, int32_t max_pages);
int32_t locks_score_num_chunks(int32_t max_pages, int32_t chunk);

/*
 * rki4 per-head page LSE scores.
 * Replaces rki4_score_bt(q, v4, vs, c8, cs, mu8, mus, bt, nsh, S, sm_scale,
 * zsplit, n_req) (selection/rki4_score_cuda.py:2518-2619; math :653-722).
 *   (d = head_dim in {64, 128, 256}, P = page in {16, 32, 64})
 *   q          (n_req, n_kv*G, d) bf16, strides (q_stride_req, q_stride_head, 1)
 *   v4         (num_blocks, n_kv, 8, d/2) u8  int4 column-major basis
 *   vs         (num_blocks, n_kv, 8)     bf16 per-column scales
 *   c8         (num_blocks, n_kv, P, 8)  i8   per-token coefficients
 *   cs         (num_blocks, n_kv, P)     bf16 per-token scales
 *   mu8        (num_blocks, n_kv, d)     i8   page centroid
 *   mus        (num_blocks, n_kv)        bf16 centroid scale
 *   slab_row_bytes  NULL or the six row strides (see above)
 *   block_table (n_req, bt_cols) i32, row stride bt_stride; page p -> block
 *   n_sel_hi   (n_req,) i32: pages [0, n_sel_hi) are scored
 *   score_h    (n_req, n_kv, G, max_pages) f32 -- written for p < n_sel_hi only
 *   page_max   (n_req, n_kv, 16, chunks) f32 -- per-head per-chunk maxima
 *              (head-major: one head's chunk maxima are contiguous)
 *   chunk      pages per workgroup (locks_score_auto_chunk); one workgroup
 *              scores its chunk for one kv head (grid: chunks x n_kv x n_req)
 * Block ids are clamped to [0, num_blocks) and page ids to [0, bt_cols).
 */
int32_t locks_score_rki4(const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
                         const uint8_t* v4, const uint16_t* vs, const int8_t* c8,
                         const uint16_t* cs, const int8_t* mu8, const uint16_t* mus,
                         const int64_t* slab_row_bytes,
                         int32_t num_blocks, const int32_t* block_table, int64_t bt_stride,
                         int32_t bt_cols, const int32_t* n_sel_hi, float* score_h,
                         int32_t max_pages, float* page_max, int32_t chunk, int32_t n_req,
                         int32_t n_kv, int32_t G, int32_t head_dim, int32_t page,
                         float sm_scale, void* stream);

/* Workspace bytes locks_select_nrm_topb needs for this geometry. */
int64_t locks_select_workspace_bytes(int32_t n_req, int32_t n_kv, int32_t max_pages);

/*
 * GQA combine + exact top-b page selection (sink + recent window always kept).
 * Replaces nrmtopb_select_cuda(score_h, hmax, npg, nsh, bfix, score,
 * page_table, page_cnt, n_req, n_kv, G, n_sink, mp, P_PAD, blk, has_hm, pdl)
 * (selection/select_cuda.py:834-938) including its page-parallel split chain
 * (:3528-3611), and for combine=1 the amax combine + topb_select_cuda
 * (selection/rki4_score_cuda.py:3494-3497, selection/select_cuda.py:3734).
 *   combine    0 = "nrm": score[p] = sum_g exp(score_h[g][p] - max_p score_h[g]),
 *              1 = "max": score[p] = max_g score_h[g][p]
 *   page_max / score_chunks: the scorer's per-chunk maxima (nrm only)
 *   score      (n_req, n_kv, max_pages) f32, written for p < n_sel_hi
 *   page_table (n_req, n_kv, max_pages) i32: kept pages ascending, -1 after
 *   page_cnt   (n_req, n_kv) i32
 *   workspace  >= locks_select_workspace_bytes(...) bytes, zero-filled once
 *              before its first use (every call leaves its histogram part
 *              zero again; unused when max_pages <= 2048); calls that
 *              overlap on one workspace race.  Its layout is derived from
 *              workspace_bytes (rows it can hold), not from n_req, so pass
 *              the same workspace_bytes on every call with that workspace
 *              whatever the batch size.
 *   b_max      host-side upper bound of b_fix (0 = unknown).  Only picks the
 *              route for rows above 8192 pages: when b_max * chunks exceeds
 *              4096 candidates, the 2048-page chunks build a row key
 *              histogram and a second pass emits the pages at or above the
 *              b-th largest key's bin (one more launch) instead of per-chunk
 *              top-b lists.  Either route gives the same page tables.
 * Launches: one kernel for rows of <= 8192 pages; otherwise a chunk kernel
 * (+ the band pass on the histogram route) and one finishing kernel.
 */
int32_t locks_select_nrm_topb(const float* score_h, const float* page_max, int32_t score_chunks,
                              const int32_t* n_pages, const int32_t* n_sel_hi,
                              const int32_t* b_fix, float* score, int32_t* page_table,
                              int32_t* page_cnt, void* workspace, int64_t workspace_bytes,
                              int32_t n_req, int32_t n_kv, int32_t G, int32_t n_sink,
                              int32_t max_pages, int32_t combine, int32_t b_max, void* stream);

/*
 * Split-K sparse paged decode over the selected pages.
 * Replaces sparse_decode_split_kernel (attention/decode.py:209-322) and the
 * CUDA decode_split(q, k, v, bt, tab, cnt, sl, m_part, l_part, acc_part,
 * scale, n_req, n_kv, G, split, pps_min, ...) (attention/decode_cuda.py:960-965).
 *   k_cache / v_cache: element strides of (block, token, kv head); d contiguous
 *   (vLLM kv_cache (NB, 2, page, n_kv, d) halves, attention/decode.py:64-73)
 *   page_table (n_req, n_kv, pt_cols) i32; page_cnt (n_req, n_kv) i32
 *   m_part, l_part (n_req, n_kv, split, G) f32; acc_part (..., G, head_dim) f32
 *   head_dim 64 / 128 / 256; page 16 / 32 / 64 tokens (a page runs as
 *   page / 16 steps of 16 tokens)
 *   max_cnt: the caller's upper bound of page_cnt (b_max + sink + window
 *   for a selection; 0 = none).  min(split, ceil(max_cnt / pps_min)) splits
 *   are launched ("nsplit"); pps = max(ceil(cnt / nsplit), pps_min), so a
 *   count above the bound is still decoded in full.  split remains the
 *   partial buffers' stride.  Inactive splits store nothing.
 */
int32_t locks_decode_splitk(const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
                            const uint16_t* k_cache, int64_t k_stride_block,
                            int64_t k_stride_tok, int64_t k_stride_head,
                            const uint16_t* v_cache, int64_t v_stride_block,
                            int64_t v_stride_tok, int64_t v_stride_head, int32_t num_blocks,
                            const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                            const int32_t* page_table, int64_t pt_stride_req,
                            int64_t pt_stride_head, int32_t pt_cols, const int32_t* page_cnt,
                            int64_t cnt_stride, const int32_t* seq_lens, float* m_part,
                            float* l_part, float* acc_part, int32_t n_req, int32_t n_kv,
                            int32_t G, int32_t head_dim, int32_t page, int32_t split,
                            int32_t pps_min, int32_t max_cnt, float sm_scale, void* stream);

/*
 * DRAM-tier V source of the split decode (the mem tier's data plane).
 * Replaces decode_split(..., v_src = 1, tier_pack) (attention/decode_cuda.py:
 * 960-1031, tier select :178-222, pack :1043-1070).  Per (selected page pt,
 * kv head kh) with physical block blk, one source is chosen:
 *   hot      complete page ((pt + 1) * page <= seq_len) and
 *            page2slot[kh * num_blocks + blk] = slot in [0, hot_slots):
 *            hot_v + (kh * hot_slots + slot) * page * head_dim, token stride head_dim;
 *   staged   else vbo[blk] = b in [0, stage_blocks): stage_v + b * stage_stride_block +
 *            kh * stage_stride_head, token stride stage_stride_tok;
 *   pinned   else pool_v + ((layer * num_blocks + blk) * n_kv + kh) * page * head_dim,
 *            token stride head_dim (pinned host memory through its device
 *            address, locks_host_device_pointer).
 * With k_tier (mem-kv) K follows the same select from hot_k / stage_k / pool_k
 * (same layouts); otherwise K is read from the paged cache.  On tier bytes
 * equal to the cache's, the partials equal locks_decode_splitk's bit for bit.
 * All pointers are device-visible and stay valid (graph-safe); the tier's
 * control plane (residency, staging, offload) is the caller's.
 */
typedef struct locks_tier_src {
    const uint16_t* hot_v;        /* (n_kv, hot_slots, page, head_dim) bf16, this layer */
    const uint16_t* stage_v;      /* staging pool of this layer, element strides below */
    const uint16_t* pool_v;       /* (layers, num_blocks, n_kv, page, head_dim) bf16, device address */
    const uint16_t* hot_k;        /* k_tier only, as hot_v */
    const uint16_t* stage_k;      /* k_tier only, as stage_v (same strides) */
    const uint16_t* pool_k;       /* k_tier only, as pool_v */
    const int32_t* page2slot;     /* (n_kv, num_blocks) hot slot of (kv head, block), -1 = none */
    const int32_t* vbo;           /* (num_blocks,) staging block of a block, -1 = none */
    int64_t stage_stride_block, stage_stride_tok, stage_stride_head;
    int32_t num_blocks;           /* must equal the call's num_blocks */
    int32_t hot_slots;            /* slots per (layer, kv head); page2slot values >= it are ignored */
    int32_t stage_blocks;         /* staging blocks; vbo values >= it are ignored */
    int32_t layer;                /* layer index into the pinned pools, in [0, num_layers) */
    int32_t k_tier;
    /* geometry the tier's buffers were laid out for; each must equal the
     * call's (the kernel derives every hot / pool offset from the call's) */
    int32_t n_kv, page, head_dim;
    int32_t num_layers;           /* layers in the pinned pools */
} locks_tier_src;

int32_t locks_decode_splitk_tier(const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
                                 const uint16_t* k_cache, int64_t k_stride_block,
                                 int64_t k_stride_tok, int64_t k_stride_head,
                                 const uint16_t* v_cache, int64_t v_stride_block,
                                 int64_t v_stride_tok, int64_t v_stride_head, int32_t num_blocks,
                                 const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                                 const int32_t* page_table, int64_t pt_stride_req,
                                 int64_t pt_stride_head, int32_t pt_cols, const int32_t* page_cnt,
                                 int64_t cnt_stride, const int32_t* seq_lens, float* m_part,
                                 float* l_part, float* acc_part, int32_t n_req, int32_t n_kv,
                                 int32_t G, int32_t head_dim, int32_t page, int32_t split,
                                 int32_t pps_min, int32_t max_cnt, float sm_scale,
                                 const locks_tier_src* tier, void* stream);

/* Device address of pinned (hipHostMalloc'd) host memory, for pool_v / pool_k. */
int32_t locks_host_device_pointer(void* host, void** dev);

/*
 * DRAM tier control plane (the reference's staging lifecycle and exact-LRU
 * residency, src/locks/tier/staging.py, tier/residency.py).  Every buffer is
 * caller-owned device memory (pool_v / pool_k: the pinned pools' device
 * addresses); launches go on `stream`, no host sync, graph-safe.
 * Layouts: page2slot / pool_valid (layers, n_kv, num_blocks), slot2page / lru
 * (layers, n_kv, hot_slots), clock (layers, n_kv); the per-layer entries take
 * one layer's slice.  Staging pools (layers, stage_blocks, page, n_kv,
 * head_dim) with the element strides given; vbo / v_flushed (num_blocks,).
 */

/* Replaces Residency.invalidate_written (residency.py:271-307, :389-419):
 * every page written this step ((seq_len - q_len) / page .. (seq_len - 1) /
 * page of each request with seq_len > 0) loses its hot slot and its pool
 * validity in every layer and kv head. */
int32_t locks_tier_invalidate(const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                              const int32_t* seq_lens, const int32_t* query_start_loc,
                              int32_t n_req, int32_t* page2slot, int32_t* slot2page,
                              int8_t* pool_valid, int32_t num_layers, int32_t n_kv,
                              int32_t num_blocks, int32_t hot_slots, int32_t page, void* stream);

/* Replaces Staging.begin_step's bookkeeping (staging.py:373-442: vflush_clear
 * :125-138, flush_collect :141-191, valloc :194-221, vslot :224-244): one
 * workgroup, requests in order.  Writes flush_list (max_flush, 2) = (block,
 * staging block) pairs to copy and *flush_cnt, frees collected staging blocks
 * onto free_stack, allocates one for every written page lacking one (stack
 * underflow sets *overflow), and fills v_slot_mapping (max_tokens,) int64
 * (staging block * page + offset, -1 = none).  Follow with
 * locks_tier_flush_copy before this step's locks_tier_scatter. */
int32_t locks_tier_stage_begin(const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                               const int32_t* seq_lens, const int32_t* query_start_loc,
                               int32_t n_req, int32_t* vbo, int32_t* v_flushed,
                               int32_t* free_stack, int32_t* free_top, int32_t* flush_list,
                               int32_t* flush_cnt, int32_t max_flush, int64_t* v_slot_mapping,
                               int32_t max_tokens, int32_t* overflow, int32_t num_blocks,
                               int32_t stage_blocks, int32_t page, void* stream);

/* Replaces _flush_copy_kernel (staging.py:247-277): every flush-list page of
 * every layer and kv head from the staging pool(s) to the pinned pool(s)
 * (layers, num_blocks, n_kv, page, head_dim), setting pool_valid. */
int32_t locks_tier_flush_copy(const int32_t* flush_list, const int32_t* flush_cnt,
                              int32_t max_flush, const uint16_t* stage_v, const uint16_t* stage_k,
                              int64_t stage_stride_layer, int64_t stage_stride_block,
                              int64_t stage_stride_tok, int64_t stage_stride_head,
                              uint16_t* pool_v, uint16_t* pool_k, int8_t* pool_valid,
                              int32_t num_layers, int32_t n_kv, int32_t num_blocks, int32_t page,
                              int32_t head_dim, int32_t k_tier, void* stream);

/* Replaces Staging.scatter_kv (staging.py:57-82, :444-460): token t's V (and,
 * k_tier, K) (n_kv, head_dim) into one layer's staging pool(s) at
 * v_slot_mapping[t] (skipped when negative). */
int32_t locks_tier_scatter(const uint16_t* value, int64_t v_stride_tok, int64_t v_stride_head,
                           const uint16_t* key, int64_t k_stride_tok, int64_t k_stride_head,
                           int32_t n_tokens, const int64_t* v_slot_mapping, uint16_t* stage_v,
                           uint16_t* stage_k, int64_t stage_stride_block, int64_t stage_stride_tok,
                           int64_t stage_stride_head, int32_t n_kv, int32_t head_dim, int32_t page,
                           int32_t stage_blocks, int32_t k_tier, void* stream);

/* Replaces Residency.gather_plan (residency.py:437-459: the clock advance,
 * _miss_diff_kernel :51-88, _select_victims_kernel :91-145) for one layer:
 * the selected complete pages of each (request, kv head) that have a hot
 * slot are touched; the others are misses (miss_pages (n_req, n_kv, pt_cols),
 * miss_cnt (n_req, n_kv)); each block's first miss takes the least recently
 * used slot not touched in this call (ties: lowest slot), evicting its page
 * (victims: the slot, -1 for later occurrences or when no slot is left,
 * which sets *overflow).  fetch_list (n_kv, fetch_cap, 2) = (block, slot) of
 * every install, fetch_cnt (n_kv,).  clock: this layer's (n_kv,) slice. */
int32_t locks_tier_plan(const int32_t* page_table, int64_t pt_stride_req, int64_t pt_stride_head,
                        int32_t pt_cols, const int32_t* page_cnt, int64_t cnt_stride,
                        const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                        const int32_t* seq_lens, int32_t n_req, int32_t* page2slot,
                        int32_t* slot2page, int32_t* lru, int32_t* clock, int32_t* miss_pages,
                        int32_t* miss_cnt, int32_t* victims, int32_t* fetch_list,
                        int32_t* fetch_cnt, int32_t fetch_cap, int32_t* overflow, int32_t n_kv,
                        int32_t num_blocks, int32_t hot_slots, int32_t page, void* stream);

/* Replaces Residency.gather_fetch (residency.py:216-268, :461-488) for one
 * layer: each fetch-list page's V (and K) into its hot slot, from the pinned
 * pool when pool_valid, else from the staging pool (vbo) with write-through
 * to the pinned pool (sets pool_valid), else from the pinned pool. */
int32_t locks_tier_fetch(const int32_t* fetch_list, const int32_t* fetch_cnt, int32_t fetch_cap,
                         uint16_t* hot_v, uint16_t* hot_k, uint16_t* pool_v, uint16_t* pool_k,
                         const uint16_t* stage_v, const uint16_t* stage_k,
                         int64_t stage_stride_block, int64_t stage_stride_tok,
                         int64_t stage_stride_head, const int32_t* vbo, int8_t* pool_valid,
                         int32_t layer, int32_t num_layers, int32_t n_kv, int32_t num_blocks,
                         int32_t hot_slots, int32_t stage_blocks, int32_t page, int32_t head_dim,
                         int32_t k_tier, void* stream);

/*
 * LSE merge of the split-K partials into the attention output.
 * Replaces merge_splits_kernel (attention/merge.py:105-152).  One workgroup
 * per (request, kv head, query head), so a row's partials are read by G
 * CUs in parallel.
 *   out (n_req, n_kv*G, head_dim) bf16 (out_is_f32 = 0) or f32 (out_is_f32 = 1),
 *   strides (out_stride_req, out_stride_head, 1), multiples of 4 elements;
 *   rows with page_cnt 0 get 0.
 *   pt_cols, max_cnt: as given to locks_decode_splitk (page_cnt is clamped
 *   to pt_cols and the split count derived from max_cnt exactly as there),
 *   so both derive the same pages per split and active split count.
 */
int32_t locks_decode_merge(const float* m_part, const float* l_part, const float* acc_part,
                           const int32_t* page_cnt, int64_t cnt_stride, int32_t pt_cols, void* out,
                           int64_t out_stride_req, int64_t out_stride_head, int32_t out_is_f32,
                           int32_t n_req, int32_t n_kv, int32_t G, int32_t head_dim,
                           int32_t split, int32_t pps_min, int32_t max_cnt, void* stream);

/*
 * locks_decode_splitk and locks_decode_merge in one launch: the last split
 * workgroup of each (request, kv head) row to finish merges that row into
 * out.  Replaces the same pair of launches
 * (attention/decode.py:328-387 -> attention/merge.py:105-152); same
 * arguments plus
 *   counters (n_req * n_kv * LOCKS_DECODE_COUNTER_STRIDE) i32 arrival
 *     counts, one per row at a stride of LOCKS_DECODE_COUNTER_STRIDE ints
 *     (256 B: rows never share a cache line): zero before the first call,
 *     left zero by every call; calls that share counters must not overlap;
 *   out / out_stride_* / out_is_f32 as locks_decode_merge.
 * Same values as locks_decode_splitk + locks_decode_merge up to fp32
 * reassociation (the last split merges the whole row in one workgroup).
 */
#define LOCKS_DECODE_COUNTER_STRIDE 64
int32_t locks_decode_fused(const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
                           const uint16_t* k_cache, int64_t k_stride_block, int64_t k_stride_tok,
                           int64_t k_stride_head, const uint16_t* v_cache, int64_t v_stride_block,
                           int64_t v_stride_tok, int64_t v_stride_head, int32_t num_blocks,
                           const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                           const int32_t* page_table, int64_t pt_stride_req,
                           int64_t pt_stride_head, int32_t pt_cols, const int32_t* page_cnt,
                           int64_t cnt_stride, const int32_t* seq_lens, float* m_part,
                           float* l_part, float* acc_part, int32_t* counters, void* out,
                           int64_t out_stride_req, int64_t out_stride_head, int32_t out_is_f32,
                           int32_t n_req, int32_t n_kv, int32_t G, int32_t head_dim,
                           int32_t page, int32_t split, int32_t pps_min, int32_t max_cnt,
                           float sm_scale,
                           void* stream);

/*
 * locks_decode_fused without caller buffers, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference: its
 * decode always takes caller-owned partials (attention/decode_cuda.py:960-965).
 * Same arguments as locks_decode_fused minus m_part / l_part / acc_part /
 * counters: those live in a file-scope device array of
 * LOCKS_NOALLOC_SCRATCH_BYTES (one copy per GPU, held until the process
 * ends), laid out as the arrival counters (n_req * n_kv *
 * LOCKS_DECODE_COUNTER_STRIDE i32) followed by the m, l (n_req * n_kv * split * G f32 each) and acc
 * (n_req * n_kv * split * G * head_dim f32) partials.  Calls needing more scratch
 * fail with -1 and a message.  Each call clears the counters (a fill kernel)
 * and launches the fused decode; nothing is allocated or freed.  Every call
 * on one GPU shares the array, so calls that overlap on one GPU (other
 * streams, other host threads) race.  Writes the same bits as
 * locks_decode_fused on the same inputs.
 */
#define LOCKS_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int32_t locks_decode_fused_noalloc(const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
                                   const uint16_t* k_cache, int64_t k_stride_block,
                                   int64_t k_stride_tok, int64_t k_stride_head,
                                   const uint16_t* v_cache, int64_t v_stride_block,
                                   int64_t v_stride_tok, int64_t v_stride_head, int32_t num_blocks,
                                   const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                                   const int32_t* page_table, int64_t pt_stride_req,
                                   int64_t pt_stride_head, int32_t pt_cols,
                                   const int32_t* page_cnt, int64_t cnt_stride,
                                   const int32_t* seq_lens, void* out, int64_t out_stride_req,
                                   int64_t out_stride_head, int32_t out_is_f32, int32_t n_req,
                                   int32_t n_kv, int32_t G, int32_t head_dim, int32_t page,
                                   int32_t split, int32_t pps_min, int32_t max_cnt,
                                   float sm_scale, void* stream);

/*
 * Dense full-KV decode: attention of each (request, kv head) group over
 * EVERY page of the row (pages 0 .. ceil(seq_len / page) - 1, no selection),
 * the dense comparator the sparse step is measured against.  No reference
 * kernel is replaced: the reference compares against FlashAttention-3 /
 * FlashInfer decode (README.md:80-90), which are not part of LOCKS.
 * Two launches: the split kernel in its dense form (page ids implicit, four
 * page stages per wave) writes the split partials, then one merge workgroup
 * per query head folds them.  Argument meanings as locks_decode_splitk and
 * locks_decode_merge; the partial buffers hold (n_req, n_kv, split, G[, head_dim]).
 */
int32_t locks_decode_dense(const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
                           const uint16_t* k_cache, int64_t k_stride_block, int64_t k_stride_tok,
                           int64_t k_stride_head, const uint16_t* v_cache, int64_t v_stride_block,
                           int64_t v_stride_tok, int64_t v_stride_head, int32_t num_blocks,
                           const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                           const int32_t* seq_lens, float* m_part, float* l_part, float* acc_part,
                           void* out, int64_t out_stride_req, int64_t out_stride_head,
                           int32_t out_is_f32, int32_t n_req, int32_t n_kv, int32_t G,
                           int32_t head_dim, int32_t page, int32_t split, float sm_scale,
                           void* stream);

/*
 * rki4 summary build on the GPU for the listed physical blocks of ONE layer
 * (head_dim 64 / 128 / 256 with page 16, 32 or 64: GQA K heads; head_dim
 * 512 with page 16: the MLA latent, n_kv 1).
 * Replaces the reference build chain _write_pre -> _eigh_chunked ->
 * _write_post (selection/rki4_build.py:147-158, :93-129, :178-225, the
 * `rki4_build_{tail,bulk,delta,refresh}` producers :264-364 call it):
 * gram on the matrix core, page x page parallel Jacobi eigensolver,
 * quantize/pack.
 *   k_cache   K half of one layer, element strides of (block, token, kv head)
 *   blocks    (n_blocks,) i32 physical block ids; ids outside [0, num_blocks)
 *             are skipped (rki4_build.py:133-144)
 *   outputs   the layer's six slabs with their row strides slab_row_bytes
 *             (as in locks_score_rki4) and the tag (num_blocks, n_kv, 8)
 *             bf16 = K[page-1, kh, 0:8]
 * Eigenvectors agree with any other eigensolver up to sign / rotation inside
 * degenerate eigenspaces, so bytes are comparable only through the score.
 */
int32_t locks_build_rki4(const uint16_t* k_cache, int64_t k_stride_block, int64_t k_stride_tok,
                         int64_t k_stride_head, int32_t num_blocks, const int32_t* blocks,
                         int32_t n_blocks, int32_t n_kv, int32_t head_dim, int32_t page,
                         uint8_t* v4, uint16_t* vs, int8_t* c8, uint16_t* cs, int8_t* mu8,
                         uint16_t* mus, const int64_t* slab_row_bytes, uint16_t* tag,
                         void* stream);

/*
 * Quantize + pack from a given eigen decomposition (the _write_post half,
 * selection/rki4_build.py:178-225 with the int4 pack :161-175), bit-exact to
 * the reference op order.  Inputs per page i < n: mu (n, 128) f32, dc
 * (n, 16, 128) f32, S2 (n, 16) f32 ascending, U (n, 16, 16) f32 (columns =
 * eigenvectors); rows (n,) i32 = slab row (block * n_kv + kv head);
 * slab_row_bytes as in locks_score_rki4.
 */
int32_t locks_pack_rki4(const float* mu, const float* dc, const float* S2, const float* U,
                        const int32_t* rows, int32_t n, int32_t head_dim, int32_t page,
                        uint8_t* v4, uint16_t* vs, int8_t* c8, uint16_t* cs, int8_t* mu8,
                        uint16_t* mus, const int64_t* slab_row_bytes, void* stream);

/*
 * Summary refresh lifecycle, step 1: the physical blocks to (re)build, as a
 * device list `blocks` plus a device count `count` (no host sync; entries
 * are distinct, in no particular order).  Replaces the block producers of
 * the reference's batched refreshes (selection/build.py:372-384
 * _tail_blocks, :415-427 _bulk_blocks, :472-488 _delta_select, called by
 * rki4_build_tail / _bulk / _delta, selection/rki4_build.py:264-315):
 *   LOCKS_REFRESH_TAIL   the last finalized page (max(sl/page - 1, 0)) of
 *                        rows[0..n_rows) (rows NULL: rows 0..n_rows-1)
 *   LOCKS_REFRESH_BULK   every finalized page p < sl/page, p < max_fin
 *   LOCKS_REFRESH_DELTA  the finalized pages whose content tag
 *                        K[page-1, kh, 0:8] differs (as bf16 numbers; the
 *                        NaN initial tag always does) from the stored tag in
 *                        ANY layer or kv head
 *   seq_lens    (n_req,) i32 SETTLED token counts (written K only)
 *   num_blocks  bound of valid block ids: min(state blocks, K blocks); ids
 *               outside [0, num_blocks) are skipped (rki4_build.py:133-144)
 *   k_layers    (n_layers,) device array of per-layer K base addresses with
 *               common element strides (DELTA only; NULL otherwise)
 *   tag         the state's (n_layers, tag_blocks, n_kv, 8) bf16 tag slab
 *   mark        (num_blocks,) u8, zero-filled once; every call leaves it zero
 *   blocks      (num_blocks,) i32 output list; count (1,) i32 output
 * The reference's bulk path clamps invalid slots to block 0 and rebuilds it;
 * here they are skipped (a non-finalized block's summary is never scored).
 */
#define LOCKS_REFRESH_TAIL 0
#define LOCKS_REFRESH_BULK 1
#define LOCKS_REFRESH_DELTA 2
int32_t locks_refresh_blocks(int32_t mode, const int32_t* block_table, int64_t bt_stride,
                             const int32_t* seq_lens, int32_t n_req, const int32_t* rows,
                             int32_t n_rows, int32_t max_fin, int32_t page, int32_t num_blocks,
                             const uint64_t* k_layers, int32_t n_layers, int64_t k_stride_block,
                             int64_t k_stride_tok, int64_t k_stride_head, int32_t n_kv,
                             const uint16_t* tag, int64_t tag_blocks, uint8_t* mark,
                             int32_t* blocks, int32_t* count, void* stream);

/*
 * Summary refresh lifecycle, step 2: locks_build_rki4 over ALL layers in one
 * launch (the reference loops layers / layer groups through torch ops,
 * selection/build.py:430-453 _build_blocks).  Layer l reads K from
 * k_layers[l] and writes the slabs at layer offset l * slab_blocks * n_kv
 * rows (slabs laid out (n_layers, slab_blocks, n_kv, ...) with row strides
 * slab_row_bytes, pointers to layer 0).  count (nullable) is a device count of valid `blocks` entries, at most
 * n_blocks, as written by locks_refresh_blocks.
 */
int32_t locks_build_rki4_layers(const uint64_t* k_layers, int32_t n_layers,
                                int64_t k_stride_block, int64_t k_stride_tok,
                                int64_t k_stride_head, int32_t num_blocks, const int32_t* blocks,
                                const int32_t* count, int32_t n_blocks, int32_t n_kv,
                                int32_t head_dim, int32_t page, int64_t slab_blocks, uint8_t* v4,
                                uint16_t* vs, int8_t* c8, uint16_t* cs, int8_t* mu8,
                                uint16_t* mus, const int64_t* slab_row_bytes, uint16_t* tag,
                                void* stream);


/*
 * Measurement helper (no counterpart in the reference): one streaming read of
 * `bytes` (a multiple of 16) from `src`, 2048 workgroups; `sink` receives a
 * store only in a practically impossible case.  Benchmarks time it beside a
 * kernel that moves the same bytes, as the practical read ceiling of a
 * launch of that size.
 */
int32_t locks_calib_read(const void* src, int64_t bytes, uint32_t* sink, void* stream);


/* ---------------------------------------------------------------------------
 * MLA (one latent KV head shared by all query heads; DeepSeek-V2-Lite:
 * kv_lora_rank 512 + 64 RoPE dims, 16 heads).  The cache is the engine's
 * latent cache (num_blocks, page, 576) bf16.  Summaries are the rki4 record
 * of the latent block built by locks_build_rki4 with head_dim 512, n_kv 1
 * (v4 (NB,1,8,256), vs (NB,1,8), c8 (NB,1,16,8), cs (NB,1,16), mu8 (NB,1,512),
 * mus (NB,1)).  The RoPE term reads either the exact bf16 keys from the
 * cache or the int8 RoPE summary built by locks_mla_build_rope (rk8
 * (NB,16,64) int8, rks (NB,16) bf16: 1056 B per page instead of 2048 B).
 * Selection reuses
 * locks_derive_params (budget_abs = budget_pages - sink - window) and
 * locks_select_nrm_topb (n_kv 1, G 1, combine 1 = max), which together
 * equal the reference's topb_middle (selection/mla_score_torch.py:51-73).
 * ------------------------------------------------------------------------- */

/*
 * Latent page score.  Replaces mla_page_score_factored_batched /
 * mla_page_score_ref (selection/mla_score_triton.py:97-151,
 * selection/mla_score_torch.py:27-48):
 *   score[r][p] = scale * max_{h < n_heads, t} (q_c8[h] . khat_t + q_rope[h] . k_rope_t)
 * for pages p < n_sel_hi[r] (full pages; written there only), where q_c is
 * int8-quantized per head and khat_t = mu + C_t V^T is the summary's
 * reconstruction of token t.  With rk8 / rks (both non-NULL) the RoPE term
 * is (qr8[h] . rk8_t) qrs[h] rks_t, q_rope int8-quantized per head like q_c
 * (absmax / 127), and the cache is not read (it may be NULL); with both NULL
 * it is q_rope[h] . k_rope_t on the cache's exact bf16 keys.
 *   q      (n_req, n_heads, 576) bf16, strides (q_stride_req, q_stride_head, 1)
 *   score  (n_req, score_stride) f32
 *   chunk  pages per workgroup (even, <= 1024; locks_mla_score_auto_chunk)
 */
int32_t locks_mla_score(const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
                        const uint8_t* v4, const uint16_t* vs, const int8_t* c8,
                        const uint16_t* cs, const int8_t* mu8, const uint16_t* mus,
                        const int8_t* rk8, const uint16_t* rks,
                        const uint16_t* cache, int64_t c_stride_block, int64_t c_stride_tok,
                        int32_t num_blocks, const int32_t* block_table, int64_t bt_stride,
                        int32_t bt_cols, const int32_t* n_sel_hi, float* score,
                        int64_t score_stride, int32_t max_pages, int32_t chunk, int32_t n_req,
                        int32_t n_heads, int32_t kv_lora_rank, int32_t rope_dim, int32_t page,
                        float scale, void* stream);
int32_t locks_mla_score_auto_chunk(int32_t n_req, int32_t max_pages);

/*
 * int8 RoPE summary of the listed physical blocks (ids outside
 * [0, num_blocks) are skipped; with n_blocks_dev non-NULL only the first
 * min(n_blocks, *n_blocks_dev) ids, read on the device): per token t of block b,
 *   rks[b][t] = bf16(max(max_d |k_rope[t][d]| / 127, 1e-8))
 *   rk8[b][t][d] = clamp(rint(k_rope[t][d] / that scale before rounding), +-127)
 * (the rki4 token-scale rule).  No reference counterpart: the reference
 * scores MLA pages with the exact RoPE keys (selection/mla_score_torch.py:41);
 * this summary halves the scorer's RoPE bytes.
 *   cache (num_blocks, 16, 576) bf16; rk8 (num_blocks, 16, 64) int8, contiguous;
 *   rks (num_blocks, 16) bf16, contiguous
 */
int32_t locks_mla_build_rope(const uint16_t* cache, int64_t c_stride_block, int64_t c_stride_tok,
                             int32_t num_blocks, const int32_t* blocks, int32_t n_blocks,
                             const int32_t* n_blocks_dev, int8_t* rk8, uint16_t* rks, void* stream);

/*
 * Split-K sparse decode over the selected latent pages.  Replaces the
 * gathered fp32 attention of LocksMLAImpl.forward_mqa
 * (backend/mla_attn.py:178-201): per request, softmax over the tokens of the
 * selected pages (position < seq_len) of q . [latent | rope] * scale;
 * values = the latent.  bf16 products, fp32 softmax, fp16 P . V with fp32
 * accumulation.
 *   page_table (n_req, pt_stride) i32 ascending; page_cnt (n_req,) i32
 *   m_part, l_part (n_req, split, 16) f32; acc_part (n_req, split, 16, 512) f32
 */
int32_t locks_mla_decode_splitk(const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
                                const uint16_t* cache, int64_t c_stride_block,
                                int64_t c_stride_tok, int32_t num_blocks,
                                const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                                const int32_t* page_table, int64_t pt_stride, int32_t pt_cols,
                                const int32_t* page_cnt, const int32_t* seq_lens, float* m_part,
                                float* l_part, float* acc_part, int32_t n_req, int32_t n_heads,
                                int32_t kv_lora_rank, int32_t rope_dim, int32_t page,
                                int32_t split, int32_t pps_min, float scale, void* stream);

/*
 * LSE merge of the MLA split partials (the attention/merge.py:105-152 rule)
 * into o (n_req, n_heads, 512) bf16 (out_is_f32 = 0) or f32, and lse
 * (n_req, lse_stride_req) f32 (may be NULL).  Rows with page_cnt 0 get 0
 * and lse -inf.
 */
int32_t locks_mla_decode_merge(const float* m_part, const float* l_part, const float* acc_part,
                               const int32_t* page_cnt, int32_t pt_cols, void* out,
                               int64_t out_stride_req, int64_t out_stride_head,
                               int32_t out_is_f32, float* lse, int64_t lse_stride_req,
                               int32_t n_req, int32_t n_heads, int32_t kv_lora_rank,
                               int32_t split, int32_t pps_min, void* stream);

/*
 * Dense full-cache MLA decode (the comparator of the sparse step): every
 * page of each request's row, in logical order (page count from seq_len,
 * no page table), split-K over `split` workgroups per request with three
 * page stages in flight and non-temporal page DMA, then the same LSE merge
 * into out (n_req, H, 512) and lse (n_req, H) (lse may be NULL).  Partials
 * as for locks_mla_decode_splitk (split <= 512).  No counterpart kernel in
 * the reference, whose dense baseline is FlashMLA (backend/mla_attn.py);
 * it exists so the sparse step is compared with a dense decode of the same
 * quality on the same GPU.
 */
int32_t locks_mla_decode_dense(const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
                               const uint16_t* cache, int64_t c_stride_block, int64_t c_stride_tok,
                               int32_t num_blocks, const int32_t* block_table, int64_t bt_stride,
                               int32_t bt_cols, const int32_t* seq_lens, float* m_part,
                               float* l_part, float* acc_part, void* out, int64_t out_stride_req,
                               int64_t out_stride_head, int32_t out_is_f32, float* lse,
                               int64_t lse_stride_req, int32_t n_req, int32_t n_heads,
                               int32_t kv_lora_rank, int32_t rope_dim, int32_t page,
                               int32_t split, float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOCKS_HIP_H_ */
