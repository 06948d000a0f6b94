/*
 * compactattn for MI355X (gfx950): C-ABI of libcompactattn_hip.so.
 *
 * This library replaces the reference's pybind11 torch extension
 * `compact_attn._C_compactattn` (compact_attn/csrc/compactattn/cache_fill.cpp:969-1021)
 * and the third-party / Triton kernels the compactattn prefill path calls around it.
 *
 * Conventions
 *  - Plain pointers to device memory, int sizes and strides (in elements), hipStream_t.
 *  - Every entry point validates its arguments on the host before any launch and
 *    returns CA_OK or a negative CA_ERR_* code; ca_last_error() gives the message
 *    (thread-local).  Nothing allocates device memory; scratch is caller-provided.
 *  - All launches go to the caller's stream; no entry point synchronises the host.
 *  - head_dim is 128 and the block (page) size is 64 tokens.
 *  - bf16 means IEEE bfloat16; summaries and scores are fp32.
 *
 * KV addressing.  Element (b, kv_head, logical block kb, token t in block, d) of a K or V
 * tensor lives at
 *     data + b*stride_b + kv_head*stride_h + phys(kb)*stride_blk + t*stride_tok + d
 * with phys(kb) = page_table ? page_table[(b*num_kv_heads + kv_head)*page_table_stride + kb]
 *                            : kb.
 * stride_tok must be below 2^24 elements (a 64-token block spans < 2^31 bytes; CA_ERR_LIMIT
 * otherwise).  A page table holds page ids in [0, num_pages); an id outside is clamped into
 * the pool, so a corrupt table cannot address memory outside it.
 * This covers the reference's seq-first [B, K, Hkv, D] tensors, its heads-first
 * k_hf/v_hf [B, Hkv, K, D] cache (compact_attn/prefill_sparse/llama/
 * modeling_llama_seerattn_chunked_dense_hf.py:59-82, viewed as 64-token pages by
 * compact_attn/kernels/varlen/flashinfer_zero_copy_prefill.py:1192-1193) and a global
 * page pool [num_pages, 64, 128] with a per-row page table.
 */
#ifndef COMPACTATTN_H
#define COMPACTATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CA_ABI_VERSION 2
#define CA_HEAD_DIM 128
#define CA_BLOCK 64
#define CA_MAX_BATCH 64

enum {
    CA_OK = 0,
    CA_ERR_INVALID = -1,   /* bad argument (shape, stride, alignment, null pointer) */
    CA_ERR_LIMIT = -2,     /* a size is beyond what this build supports */
    CA_ERR_WORKSPACE = -3, /* workspace missing or too small */
    CA_ERR_HIP = -4        /* a HIP runtime call failed */
};

/* Selection-rule flags. */
#define CA_RULE_TOPK 1      /* keep the top-k past blocks by (score desc, block id asc)   */
#define CA_RULE_ALPHA 2     /* keep score >= alpha * row max                              */
#define CA_RULE_THRESHOLD 4 /* keep score > threshold (strict)                           */
/* With CA_RULE_TOPK: rank every column kb < P + Qb instead of the past blocks only, each by
 * its value in the zeroed row (non-causal and non-finite entries read as 0), and keep the
 * picks that are causal -- the reference's min_budget (torch.topk over the zeroed row,
 * compact_attn/modules/flashprefill_prefill.py:633-647).  Ties go to the lower block id. */
#define CA_RULE_TOPK_ALLCOLS 8

/* The alpha rule's row max is the max over all P + Qb columns of the zeroed row, as in
 * flashprefill_prefill.py:633-645 (0 whenever a non-causal or non-finite column exists). */

typedef struct {
    int32_t batch;        /* requests in the launch, <= CA_MAX_BATCH                 */
    int32_t q_len;        /* chunk tokens per request; the chunk starts at a block
                             boundary and covers Qb = ceil(q_len/64) blocks, the last
                             holding q_len - 64 (Qb - 1) tokens                      */
    int32_t num_q_heads;  /* Hq                                                      */
    int32_t num_kv_heads; /* Hkv; Hq % Hkv == 0, group G = Hq / Hkv <= 16            */
    int32_t kv_cap;       /* per-row capacity in blocks of tables and summaries;
                             >= past_blocks[b] + Qb for every request                */
} ca_dims;

typedef struct {
    void* data; /* bf16 */
    int64_t stride_b;
    int64_t stride_h;
    int64_t stride_blk;
    int64_t stride_tok;
    const int32_t* page_table; /* optional (NULL: physical block = logical block) */
    int64_t page_table_stride;
    int64_t num_pages; /* with a page table: pages in the pool; page ids read from the table
                          are clamped into [0, num_pages) (ignored without a table)          */
} ca_kv_layout;

typedef struct {
    void* data; /* bf16, element (b, t, h, d) at data + b*stride_b + t*stride_t + h*stride_h + d */
    int64_t stride_b;
    int64_t stride_t;
    int64_t stride_h;
} ca_seq_layout;

typedef struct {
    int32_t flags;         /* CA_RULE_* bits                                          */
    int32_t topk;          /* blocks per (head, query block) row, over past blocks     */
    float alpha;           /* CA_RULE_ALPHA factor                                     */
    float threshold;       /* CA_RULE_THRESHOLD value                                  */
    int32_t sink_blocks;   /* always keep blocks kb < sink_blocks                      */
    int32_t window_blocks; /* keep 0 <= (P + qb) - kb < window_blocks                  */
    int32_t local_blocks;  /* keep the local_blocks past blocks right before the chunk */
    int32_t last_n_block;  /* leave the last n query blocks out of the union           */
} ca_select_rule;

/* Library identity and last error (thread-local, valid until the next call). */
int ca_abi_version(void);
const char* ca_last_error(void);

/*
 * Partial blocks.  A chunk whose q_len is not a multiple of 64 ends in a block of
 * n = q_len - 64 (Qb - 1) tokens: its rows are the only ones read from the chunk's tensors
 * and written to the cache (the cache rows past them keep what they held), and its
 * summaries pool those n tokens -- max and min over them, avg = their sequential sum
 * divided by n (the reference's mean over the valid tokens of a block,
 * compact_attn/flashprefill_vendor/flashprefill_native_forward.py:44-95; the pooling of
 * AttnGate's ceil_mode pools, compact_attn/prefill_sparse/attn_gate.py:113-130).
 *
 * Cache fill.  Appends one chunk of K/V per request into the cache at logical blocks
 * [past_blocks[b], past_blocks[b] + Qb) and writes, for each new block, the fp32
 * mean of its K rows into kmean[(b*Hkv + h)*kv_cap + kb][128] (sequential sum over the
 * block's tokens divided by their count, 64 except in a partial last block).  If gate_wk is given ([Hkv, 128, 128], in x out) it also writes
 * kgate = RoPE(W_k[h]^T mean) (rope_cos/rope_sin: [rope_rows, 128] indexed by absolute
 * block id, may be NULL for no RoPE) into kgate with the kmean layout.  With k_cache and
 * v_cache both NULL nothing is copied and only the summaries are written (v_new unused).
 * Replaces: transformers DynamicCache.update concatenation
 * (compact_attn/prefill_sparse/llama/modeling_llama_seerattn_chunked_dense.py:518-536),
 * compute_mean_vector / flash_prefill_compute_mean_k
 * (compact_attn/flashprefill_vendor/flashprefill_native_forward.py:44-95,505-538),
 * the gate K-block cache append (modeling_llama_seerattn.py:407-435 with
 * compact_attn/prefill_sparse/attn_gate.py:124-171) and cache_fill_current_tail
 * (compact_attn/csrc/compactattn/cache_fill.cpp, cache_fill_kernel.cu:665-719).
 */
int ca_cache_fill(const ca_dims* dims, const ca_seq_layout* k_new, const ca_seq_layout* v_new,
                  const ca_kv_layout* k_cache, const ca_kv_layout* v_cache,
                  const int32_t* past_blocks_host, float* kmean, const float* gate_wk,
                  const float* rope_cos, const float* rope_sin, int64_t rope_rows, float* kgate,
                  void* stream);

/*
 * Pooled query summaries: qhat[(b*Hq + h)*Qb + qb][128] = mean of the query rows of
 * block qb (sequential sum divided by the block's token count), optionally projected by gate_wq [Hq, 128, 128]
 * and rotated at absolute block id past_blocks[b] + qb.
 * Replaces: AttnGate.compress_query_blocks + block RoPE (attn_gate.py:113-171) and the
 * query-side mean of compute_block_score_chunked (flashprefill_native_forward.py:98-207).
 */
int ca_pool_query(const ca_dims* dims, const ca_seq_layout* q, const int32_t* past_blocks_host,
                  const float* gate_wq, const float* rope_cos, const float* rope_sin,
                  int64_t rope_rows, float* qhat, void* stream);

/*
 * ca_cache_fill (append + mean-K, no gate) and ca_pool_query (query-block means, no
 * projection) of one chunk in a single launch: dims->num_kv_heads sizes the cache side,
 * num_q_heads the query side; k_new/v_new [B, q_len, Hkv, 128], q [B, q_len, Hq, 128].
 * Results equal the two separate calls bit for bit.
 * Replaces: the FlashPrefill model's per-chunk cache update + mean-K cache
 * (modeling_llama_flashprefill_compactattn.py:121-150,205-246) and the query-side means of
 * compute_block_score_chunked (flashprefill_native_forward.py:98-207).
 */
int ca_cache_fill_pool_query(const ca_dims* dims, const ca_seq_layout* k_new, const ca_seq_layout* v_new,
                             const ca_kv_layout* k_cache, const ca_kv_layout* v_cache,
                             const int32_t* past_blocks_host, float* kmean, const ca_seq_layout* q, float* qhat,
                             void* stream);

/*
 * AttnGate block summaries for every gate type of the reference (compact_attn/prefill_sparse/
 * attn_gate.py:37-130,233-278: the Q{pools}_K{pools} classes, force_double, the
 * kv_group_aware_query form).  pools is a set of CA_POOL_* bits; the pooled vectors of a
 * block (max and min of the bf16 values, avg = sequential sum divided by the token count) are
 * concatenated in the order max, min, avg into an input of in = C*128 values (C pools), then
 * projected, y[o] = sum_{i < in} x[i] W[i][o] (sequential fma over i), and rotated at the
 * block's absolute id (rope_cos/rope_sin [rope_rows, 128], may be NULL).
 *
 * ca_gate_key_summaries: the new blocks of k_new ([B, q_len, Hkv, 128]) -> kgate rows
 * (b*gate_heads + j)*kv_cap + past_blocks[b] + n.  gate_heads = num_kv_heads: W_k
 * [Hkv, in, 128] per KV head; gate_heads = num_q_heads: the block is repeated to the G Q
 * heads of its group (head hk*G + j) and projected per Q head with W_k [Hq, in, 128] -- the
 * reference's single-linear gate (attn_gate.py:84-86 with MultiHeadLinear's repeat, :30-33).
 * ca_gate_query_summaries: the query blocks of q ([B, q_len, Hq, 128]) -> qhat
 * [B, gate_heads, Qb, 128].  gate_wq NULL: no projection (one pool only, gate_heads =
 * num_q_heads; the pooled vector is still rotated when rope tables are given, as the
 * reference rotates its unprojected query blocks).  gate_heads = num_q_heads: W_q
 * [Hq, in, 128] per Q head.  gate_heads =
 * num_kv_heads (kv_group_aware_query): the G heads of a KV group are pooled and concatenated
 * head-major into G*in values and projected with W_q [Hkv, G*in, 128].
 * Replaces: AttnGate.compress_query_blocks / compress_key_blocks / MultiHeadLinear /
 * apply_block_position_embeddings (attn_gate.py:20-34,113-171) and the gate K-block cache
 * append (compact_attn/prefill_sparse/llama/modeling_llama_seerattn.py:407-435).
 */
#define CA_POOL_MAX 1
#define CA_POOL_MIN 2
#define CA_POOL_AVG 4
int ca_gate_key_summaries(const ca_dims* dims, const ca_seq_layout* k_new, const int32_t* past_blocks_host,
                          int32_t pools, const float* gate_wk, int32_t gate_heads, const float* rope_cos,
                          const float* rope_sin, int64_t rope_rows, float* kgate, void* stream);
int ca_gate_query_summaries(const ca_dims* dims, const ca_seq_layout* q, const int32_t* past_blocks_host,
                            int32_t pools, const float* gate_wq, int32_t gate_heads, const float* rope_cos,
                            const float* rope_sin, int64_t rope_rows, float* qhat, void* stream);

/*
 * 128-token block summaries from 64-token ones, for FlashPrefill scoring with 128-token
 * blocks (the reference's default block_size, compact_attn/prefill_sparse/llama/
 * modeling_llama_flashprefill_compactattn.py:253; compact_attn/load_attention_replacement.py:
 * 255), while pages, tables and attention stay in 64-token blocks.  For each of `rows` rows of
 * n_blocks 64-token summaries (src [rows, src_stride, 128] fp32, the last block holding
 * last_tokens tokens, 1..64) it writes ceil(n_blocks/2) summaries (dst [rows, dst_stride, 128]):
 *     dst[j] = (c0 * src[2j] + c1 * src[2j+1]) / (c0 + c1)
 * in fp32 (two products, their sum, one correctly rounded division), c the blocks' token
 * counts, and dst[j] = src[2j] when 2j is the last block.  For block means this is the mean
 * over the pair's tokens (compute_mean_vector's per-block mean at block_size 128,
 * compact_attn/flashprefill_vendor/flashprefill_native_forward.py:44-95) up to rounding.
 * No counterpart in _C_compactattn.
 */
int ca_pair_block_summaries(const float* src, int64_t src_stride, float* dst, int64_t dst_stride, int64_t rows,
                            int32_t n_blocks, int32_t last_tokens, void* stream);

/*
 * Block scoring and per-row selection.  For every (b, h, qb) row it computes
 * logits[kb] = dot(qhat[b,h,qb], khat[b, h/G, kb]) * scale for kb <= P_b + qb (sequential
 * fma over d), the softmax over those kb (fixed evaluation order), applies the rule and
 * writes the row's keep bitmask rowmask[((b*Hq + h)*Qb + qb)*words + w],
 * words = ceil(kv_cap / 32), bit kb%32 of word kb/32.  scores ([B, Hq, Qb, kv_cap] fp32,
 * required) receives the normalised scores (non-causal entries 0); it doubles as the
 * logits scratch between the two kernels of this call.  khat is a kmean/kgate summary array.
 * Replaces: compute_block_score_chunked + normalize_scores (flashprefill_native_forward.py:
 * 98-207,365-374), AttnGate.score_compressed_blocks (attn_gate.py:173-204) and the per-row
 * rules of _flashprefill_keep_block_from_scores_rowwise (compact_attn/modules/
 * flashprefill_prefill.py:596-666).
 */
int ca_score_select(const ca_dims* dims, const float* qhat, const float* khat, float scale,
                    const ca_select_rule* rule, const int32_t* past_blocks_host, uint32_t* rowmask,
                    float* scores, void* stream);

/*
 * FlashPrefill block scores in the reference's per-token form: for every request b, Q head h,
 * query block qb and key block kb, the exp2 mass over the block's token slots t of
 *     s = dot(q_t, bf16(khat[b, h/G, kb])) * scale * log2(e)
 * taken where the whole key block precedes the token (64 P_b + block_size qb + t >=
 * block_size (kb + 1) - 1), shifted by its maximum over t, then normalised over the row:
 *     score = mass * exp2(max - rowmax) / (sum_kb of that + 1e-9).
 * Blocks here are block_size (64 or 128) tokens: past_blocks_host and dims->kv_cap count
 * block_size blocks (the chunk starts at past_blocks * block_size); the row's key blocks are
 * nk = P_b + ceil(q_len / block_size) <= kv_cap, and the chunk's last block keeps the slots
 * past q_len as zero queries, as the reference does.  q has the ca_seq_layout of the chunk's
 * queries; khat [B*Hkv, khat_stride, 128] fp32 block means (rounded to bf16 for the products,
 * as the reference stores them); scores [B, Hq, ceil(q_len/block_size), kv_cap] fp32 receives
 * the scores (0 past nk).  Products on bf16 MFMAs with fp32 accumulation: the scores agree
 * with an fp64 evaluation of the same formula to a few ulps, not bit for bit.  The pooled
 * scores of ca_score_select remain the bit-reproducible form; these feed ca_select_scores.
 * Replaces: compute_block_score_chunked (K_STRIDE = block_size) + normalize_scores
 * (compact_attn/flashprefill_vendor/flashprefill_native_forward.py:98-207,365-374) as
 * flash_prefill_score_chunked_from_mean_k runs them (:562-582).
 */
int ca_score_token_mass(const ca_dims* dims, const ca_seq_layout* q, const float* khat, int64_t khat_stride,
                        int32_t block_size, float scale, const int32_t* past_blocks_host, float* scores,
                        void* stream);

/*
 * Per-row selection from caller-provided scores, element (b, h, qb, kb) at
 * scores + b*stride_b + h*stride_h + qb*stride_q + kb (dtype 0 = fp32, 1 = bf16).  The score
 * columns cover kb in [0, P_b + Qb); causal as above.  Output as ca_score_select.
 * Replaces: build_keep_past_fast / build_keep_curr_fast (cache_fill_kernel.cu:274-326,
 * cache_fill.cpp:1124-1190) and _build_keep_block_mask (compact_attn/modules/
 * attention_forward_chunked_dense.py:352-403,559-638).
 */
int ca_select_scores(const ca_dims* dims, const void* scores, int32_t dtype, int64_t stride_b,
                     int64_t stride_h, int64_t stride_q, const ca_select_rule* rule,
                     const int32_t* past_blocks_host, uint32_t* rowmask, void* stream);

/*
 * Block-Union: Q-block union (OR over query blocks qb < Qb - last_n_block), GQA
 * intra-group union (OR over the G heads of a KV group), current-chunk blocks always kept,
 * then ascending compaction.  Writes table[row*table_stride + i] (i < counts[row]) with the
 * selected logical block ids of row = b*Hkv + kv_head, counts[row], and optionally
 * keep_block [B, Hq, kv_cap] u8 and keep_kv [B, Hkv, kv_cap] u8 (0/1, zero beyond the row).
 * Entries of table at i >= counts[row] are set to -1 up to kv_cap.
 * Replaces: _build_kv_head_union_keep_block_mask (attention_forward_chunked_dense.py:
 * 641-683), build_past_indices_and_metadata_from_keep_block / build_block_table /
 * build_selected_indices_from_kv_keep_block / build_flashinfer_kv_indices
 * (cache_fill_kernel.cu:163-190,328-483; the CSR form is ca_table_to_csr) and the Triton union kernel
 * (flashprefill_prefill.py:307-376).
 */
int ca_union_compact(const ca_dims* dims, const uint32_t* rowmask, int32_t last_n_block,
                     const int32_t* past_blocks_host, uint8_t* keep_block, uint8_t* keep_kv,
                     int32_t* table, int64_t table_stride, int32_t* counts, void* stream);

/*
 * Union + compaction from a caller-provided per-KV-group keep mask keep_kv
 * [B, Hkv, kv_cap] (u8, any nonzero = keep; current-chunk blocks are always kept).
 * Replaces: build_selected_indices_from_kv_keep_block_out (cache_fill_kernel.cu:449-483)
 * as used by chunked_prefill_column_dense_attention_from_keep_block
 * (attention_forward_chunked_dense.py:2147) with keep_block_kv_preprojected.
 */
int ca_compact_keep_kv(const ca_dims* dims, const uint8_t* keep_kv, const int32_t* past_blocks_host,
                       int32_t* table, int64_t table_stride, int32_t* counts, void* stream);

/*
 * Block tables -> CSR page lists for FlashInfer-style paged-KV consumers: kv_indptr
 * [B*Hkv + 1] (exclusive prefix sum of counts), kv_indices (kv_indices[kv_indptr[r] + i] =
 * r * kv_cap + table[r][i], the global page id of row r's block in the heads-first cache;
 * room for B*Hkv*kv_cap entries since the counts are device data), and optionally
 * kv_last_page_len [B*Hkv] (= 64, every page is full).  Uses dims->batch, num_kv_heads and
 * kv_cap only.  At most 8192 rows.
 * Replaces: the pages_per_row / kv_indptr / kv_indices construction of
 * build_flashinfer_kv_indices (compact_attn/csrc/compactattn/cache_fill_kernel.cu:485-505) and
 * its torch spec _build_index_metadata_reference_from_keep_block_kv
 * (compact_attn/kernels/varlen/flashinfer_zero_copy_prefill.py:482-510).
 */
int ca_table_to_csr(const ca_dims* dims, const int32_t* table, int64_t table_stride, const int32_t* counts,
                    int32_t* kv_indptr, int32_t* kv_indices, int64_t indices_capacity, int32_t* kv_last_page_len,
                    void* stream);

/* Identity tables (every block 0..P_b+Qb-1): the dense full-KV comparator's input. */
int ca_dense_table(const ca_dims* dims, const int32_t* past_blocks_host, int32_t* table,
                   int64_t table_stride, int32_t* counts, void* stream);

/*
 * Indexed attention prefill over the selected blocks (bf16 in, fp32 accumulate, bf16 out).
 * Query token t of request b (absolute position 64*P_b + t) and Q head h attend over the
 * keys of the blocks table[row][0..counts[row]) of row = b*Hkv + h/G with bottom-right
 * causal masking (key position j visible iff j <= 64*P_b + t).  out has q's layout;
 * lse (optional, [B, Hq, q_len] fp32, natural log) receives the log-sum-exp.
 * Each table row must hold strictly ascending block ids (no duplicates), as
 * ca_union_compact, ca_compact_keep_kv and ca_dense_table write them: the kernel drops
 * the trailing blocks past a query tile's causal edge and applies the causal mask only to
 * the trailing run of blocks that reach past the tile's first query, so an out-of-order
 * row could let a query see later keys.
 * num_splits >= 1 splits every row's block list that many ways; num_splits = 0 picks one
 * count for the launch (ca_attn_pick_splits) with at least ~16 blocks per split: at most 256
 * work items (row tiles x splits, one per CU) when all requests have one length, 1 when
 * their row tiles alone fill three quarters of the 256 CUs, and about 512 for ragged
 * batches (a ragged launch whose row tiles fill three quarters of the CUs runs unsplit when
 * its rows' selected counts are within 1.5x of their mean: the kernel decides from counts).  The work is placed on the 8 XCDs in units: whole KV rows (longest first) when
 * the requests have one length and the rows divide over the XCDs, otherwise single splits
 * of each row dealt round-robin request by request.  More than one split needs a workspace
 * of ca_attn_workspace_size(dims, past, num_splits) bytes.
 * Replaces: flash_attn_with_kvcache / FlashInfer paged prefill as driven by
 * flash_attn_indexed_prefill_from_paged_kv (compact_attn/kernels/varlen/
 * indexed_dense_prefill_varlen.py:1473-1613) and flashinfer_prefill_zero_copy
 * (flashinfer_zero_copy_prefill.py:1139-1353), plus pack_q_for_indexed_prefill
 * (cache_fill_kernel.cu:130-161) and the selected-KV gathers it needed
 * (cache_fill_kernel.cu:595-719).
 */
int ca_attn_fwd(const ca_dims* dims, const ca_seq_layout* q, const ca_kv_layout* k,
                const ca_kv_layout* v, const int32_t* table, int64_t table_stride,
                const int32_t* counts, const int32_t* past_blocks_host, float scale,
                const ca_seq_layout* out, float* lse, int32_t num_splits, void* workspace,
                int64_t workspace_bytes, void* stream);

/*
 * ca_attn_fwd without any allocation: no workspace argument, no hipMalloc/hipFree or allocating
 * library call.  No counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid allocation).
 * The split partials live in a library-owned device array of CA_STATIC_SCRATCH_BYTES that
 * each GPU the library runs on holds until the process ends (looked up on a device's first
 * call; the current device must be the stream's).  num_splits = 0 runs exactly as ca_attn_fwd
 * with num_splits = 0 when the automatic count's partials fit the array; otherwise that count
 * is lowered until they fit and used as a fixed count.  A positive count whose partials
 * (ca_attn_workspace_size) exceed the array fails with CA_ERR_LIMIT.  All calls on one GPU
 * share its array: calls that overlap on one GPU (other streams, other threads) race.
 */
#define CA_STATIC_SCRATCH_BYTES (48u << 20)
int ca_attn_fwd_noalloc(const ca_dims* dims, const ca_seq_layout* q, const ca_kv_layout* k,
                        const ca_kv_layout* v, const int32_t* table, int64_t table_stride,
                        const int32_t* counts, const int32_t* past_blocks_host, float scale,
                        const ca_seq_layout* out, float* lse, int32_t num_splits, void* stream);

/* Workspace bytes ca_attn_fwd needs for num_splits (0 = the automatic count). */
int64_t ca_attn_workspace_size(const ca_dims* dims, const int32_t* past_blocks_host,
                               int32_t num_splits);

/* The split count ca_attn_fwd uses for num_splits = 0. */
int32_t ca_attn_pick_splits(const ca_dims* dims, const int32_t* past_blocks_host);

/*
 * Dense decode attention over the whole cache (bf16 in, fp32 accumulate, bf16 out).
 * dims.q_len (1..64) query rows per request are the last q_len positions of its
 * kv_len_host[b] tokens: row t attends to keys j <= kv_len - q_len + t, read through the
 * K/V layouts (blocks 0 .. ceil(kv_len/64)-1, page table if given; kv_len need not be a
 * multiple of 64).  q/out [B, q_len, Hq, 128], lse as ca_attn_fwd.  The block lists are
 * split KV-wise (num_splits 1..64, or 0 for a per-request plan: about 256 work items, at
 * least 4 blocks per split, at most 32 splits) and merged by LSE; more than one split needs
 * ca_attn_decode_workspace_size() bytes of workspace.
 * Replaces: the q_len == 1 branch of LlamaSeerAttentionChunkedDense.forward
 * (compact_attn/prefill_sparse/llama/modeling_llama_seerattn_chunked_dense.py:878-894), i.e.
 * _dense_prefill_full_kv / flash_attn_with_kvcache over the updated cache.
 */
int ca_attn_decode(const ca_dims* dims, const ca_seq_layout* q, const ca_kv_layout* k,
                   const ca_kv_layout* v, const int32_t* kv_len_host, float scale,
                   const ca_seq_layout* out, float* lse, int32_t num_splits, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* Workspace bytes ca_attn_decode needs for num_splits (0 = its per-request plan). */
int64_t ca_attn_decode_workspace_size(const ca_dims* dims, const int32_t* kv_len_host,
                                      int32_t num_splits);

/*
 * Model plumbing.  Fused element-wise kernels of the Llama integration; they have no
 * counterpart in _C_compactattn and replace chains of PyTorch element-wise kernels around
 * the compactattn layers (bf16 in and out, fp32 math).
 *
 * ca_rope_apply: y = bf16(x * cos + rotate_half(x) * sin) for x, y [B, len, heads, 128]
 * (seq layouts that must not overlap; batch * len < 2^31), cos/sin fp32 [len, 128]
 * contiguous and 16-byte aligned (the rows of the len positions); bit-identical to
 * apply_rotary_pos_emb evaluated in fp32.
 * ca_rmsnorm: y = bf16(w * bf16(s * rsqrt(mean(s^2) + eps))) per row of n (multiple of 8),
 * s = x; with a residual (residual and sum_out both non-NULL) s = bf16(x + residual) is
 * written to sum_out first (the decoder's residual add fused into the following norm;
 * sum_out may alias x or residual, y must not overlap them).
 * ca_swiglu: y = bf16(bf16(silu(gate)) * up) per row of n (multiple of 8).
 */
int ca_rope_apply(const ca_seq_layout* x, const ca_seq_layout* y, int32_t batch, int32_t len, int32_t heads,
                  const float* cos, const float* sin, void* stream);
int ca_rmsnorm(const uint16_t* x, int64_t x_stride, const uint16_t* residual, int64_t r_stride, uint16_t* sum_out,
               int64_t s_stride, const uint16_t* w, uint16_t* y, int64_t y_stride, int64_t rows, int32_t n, float eps,
               void* stream);
int ca_swiglu(const uint16_t* gate, int64_t g_stride, const uint16_t* up, int64_t u_stride, uint16_t* y,
              int64_t y_stride, int64_t rows, int32_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* COMPACTATTN_H */
