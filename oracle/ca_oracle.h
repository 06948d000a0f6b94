/*
 * CPU oracle for the compactattn chunked-prefill path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product path (compactattention_amd) never
 * links, imports or calls it.
 *
 * Every routine restates the reference algorithm in plain C with a fixed
 * floating-point evaluation order (the same order the HIP kernels use), so
 * fp32 scores, selection masks and block tables can be compared bit for bit.
 * All tensors are host arrays in the canonical contiguous layouts given per
 * function; bf16 values are passed as their uint16 bit patterns.
 */
#ifndef CA_ORACLE_H
#define CA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_D 128
#define ORC_BLOCK 64

/* Selection-rule flags (same meaning as the product's CA_RULE_* flags). */
#define ORC_RULE_TOPK 1
#define ORC_RULE_ALPHA 2
#define ORC_RULE_THRESHOLD 4
#define ORC_RULE_TOPK_ALLCOLS 8 /* with ORC_RULE_TOPK: rank all Kb columns (the reference's min_budget) */

typedef struct {
    int32_t flags;
    int32_t topk;
    float alpha;
    float threshold;
    int32_t sink_blocks;
    int32_t window_blocks;
    int32_t local_blocks;
    int32_t last_n_block;
} orc_rule;

int orc_version(void);

float orc_exp(float x);
float orc_bf16_to_f32(uint16_t v);
uint16_t orc_f32_to_bf16(float v);

/* x: [B, L, H, 128] bf16 -> out: [B, H, ceil(L/64), 128] fp32 block means: the sequential
 * sum over a block's tokens divided by their count (64, or L % 64 for a partial last block). */
void orc_block_mean(const uint16_t* x, int B, int L, int H, float* out);

/* Gate pooling set (AttnGate pooling functions, compact_attn/prefill_sparse/attn_gate.py:
 * 233-237): the pooled vectors are concatenated in the order max, min, avg. */
#define ORC_POOL_MAX 1
#define ORC_POOL_MIN 2
#define ORC_POOL_AVG 4

/* Block pooling: x [B, L, H, 128] bf16 -> out [B, H, ceil(L/64), C*128] fp32 with
 * C = popcount(pools), over each block's tokens (a partial last block's valid ones); max and
 * min keep the bf16 values, avg is as orc_block_mean.  max/min are strict compares from token 0 (the first of equal values
 * stays). */
void orc_block_pool(const uint16_t* x, int B, int L, int H, int pools, float* out);

/* 128-token summaries from 64-token ones (FlashPrefill with 128-token score blocks): src
 * [rows, n_blocks, 128] (the last block holds last_tokens tokens) -> dst [rows,
 * ceil(n_blocks/2), 128], dst[j] = (c0*src[2j] + c1*src[2j+1]) / (c0 + c1) (fp32: two products,
 * their sum, one division; c = 64 or last_tokens), an unpaired last block copied. */
void orc_pair_block_means(const float* src, int rows, int n_blocks, int last_tokens, float* dst);

/* Per-head gate projection followed by block RoPE.
 * x: [B, H, N, 128] fp32, W: [H, 128, 128] (in, out), cos/sin: [rope_rows, 128]
 * indexed by absolute block id; block n of request b has id first_block[b] + n.
 * cos/sin may be NULL (projection only).  y: [B, H, N, 128]. */
void orc_gate_project(const float* x, int B, int H, int N, const float* W,
                      const float* cos_t, const float* sin_t, int64_t rope_rows,
                      const int32_t* first_block, float* y);

/* The same with an input width `in` (x [B, H, N, in], W [H, in, 128]); the sum over the
 * input runs i = 0 .. in-1 in order. */
void orc_gate_project_n(const float* x, int B, int H, int N, int in, const float* W,
                        const float* cos_t, const float* sin_t, int64_t rope_rows,
                        const int32_t* first_block, float* y);

/* Softmax-normalised block scores.
 * qhat: [B, Hq, Qb, 128], khat: [B, Hkv, cap, 128]; scores: [B, Hq, Qb, cap].
 * Row (b,h,qb) covers kb in [0, P_b + qb] (causal); other entries are 0. */
void orc_block_scores(const float* qhat, const float* khat, int B, int Hq, int Hkv, int Qb,
                      int cap, const int32_t* past_blocks, float scale, float* scores);

/* Per-row selection. scores: [B, Hq, Qb, cap] fp32 -> rowkeep [B, Hq, Qb, cap] u8. */
void orc_select_rows(const float* scores, int B, int Hq, int Qb, int cap,
                     const int32_t* past_blocks, const orc_rule* rule, uint8_t* rowkeep);

/* Q-block union, GQA union and compaction.
 * rowkeep: [B, Hq, Qb, cap] u8 -> keep_block [B, Hq, cap] u8, keep_kv [B, Hkv, cap] u8,
 * table [B*Hkv, cap] int32 (ascending ids, -1 padded), counts [B*Hkv]. */
void orc_union_compact(const uint8_t* rowkeep, int B, int Hq, int Hkv, int Qb, int cap,
                       const int32_t* past_blocks, int last_n_block, uint8_t* keep_block,
                       uint8_t* keep_kv, int32_t* table, int32_t* counts);

/* Attention over the blocks listed in the table (fp64 accumulation).
 * q: [B, Lq, Hq, 128] bf16; k, v: [B, Hkv, cap*64, 128] bf16 heads-first;
 * table [B*Hkv, cap], counts [B*Hkv]; out: [B, Lq, Hq, 128] fp32, lse: [B, Hq, Lq] (natural log,
 * may be NULL).  Query token t of request b sits at absolute position 64*P_b + t and sees
 * key position j iff j <= 64*P_b + t.  q_begin/q_end restrict the query tokens computed
 * (the rest of out is left untouched); head_begin/head_end restrict the Q heads. */
void orc_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, int B, int Lq, int Hq,
                   int Hkv, int cap, const int32_t* past_blocks, const int32_t* table,
                   const int32_t* counts, float scale, int q_begin, int q_end, int head_begin,
                   int head_end, float* out, float* lse);

/* Full path for one chunk (cache-fill mean + pooled scores + selection + union + table),
 * used as the timed CPU baseline.  Inputs as the functions above. */
int orc_num_threads(void);

#ifdef __cplusplus
}
#endif

#endif
