// Internal launch interface between the C-ABI layer (ca_api.cpp) and the kernels.
// Shapes reaching these launchers have already been validated on the host.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/compactattn.h"

namespace ca {

struct PastBlocks {
    int32_t p[CA_MAX_BATCH];
};

struct KvAddr {
    uint16_t* data;
    int64_t sb, sh, sblk, stok;
    const int32_t* page_table;
    int64_t pts;
    int32_t max_page;  // pages in the pool - 1 (page ids read from the table are clamped to it)
};

// Physical page of logical block kb of a row: the page table entry clamped into the pool, or
// kb itself without a page table (a corrupt table cannot address outside the pool).
__device__ __forceinline__ int64_t clamp_page(int32_t id, int32_t max_page) {
    return id < 0 ? 0 : (id > max_page ? max_page : id);
}

struct SeqAddr {
    uint16_t* data;
    int64_t sb, st, sh;
};

struct Shape {
    int B, Lq, Hq, Hkv, G, Qb, cap, words;
};

// pools: CA_POOL_* set of the gate-K summary; gk: gate heads per KV head (1 or G)
hipError_t launch_cache_fill(const Shape& s, const SeqAddr& k_new, const SeqAddr& v_new,
                             const KvAddr& k_cache, const KvAddr& v_cache, const PastBlocks& pb,
                             float* kmean, const float* wk, const float* rope_cos,
                             const float* rope_sin, float* kgate, int pools, int gk, hipStream_t stream);

// Cache append + mean-K (rows b*Hkv + h) and the query-block means (rows b*Hq + h) in one
// launch: the FlashPrefill summaries of a chunk.
hipError_t launch_chunk_summaries(const Shape& s, const SeqAddr& k_new, const SeqAddr& v_new, const KvAddr& k_cache,
                                  const KvAddr& v_cache, const PastBlocks& pb, float* kmean, const SeqAddr& q,
                                  float* qhat, hipStream_t stream);

// pools: CA_POOL_* set; kv_aware: one output per KV head from its G heads' pooled vectors
hipError_t launch_pool_query(const Shape& s, const SeqAddr& q, const PastBlocks& pb, const float* wq,
                             const float* rope_cos, const float* rope_sin, float* qhat, int pools,
                             bool kv_aware, hipStream_t stream);

// LDS bytes the score/select kernel needs for this shape (0 if unsupported).
size_t score_select_lds_bytes(const Shape& s, bool compute);

// 128-token block summaries from pairs of 64-token ones (rows of n_blocks source blocks, the last
// holding last_tokens tokens)
hipError_t launch_pair_summaries(const float* src, int64_t src_stride, float* dst, int64_t dst_stride,
                                 int64_t rows, int n_blocks, int last_tokens, hipStream_t stream);

hipError_t launch_score_select(const Shape& s, const float* qhat, const float* khat, float scale,
                               const void* scores_in, int dtype, int64_t ssb, int64_t ssh,
                               int64_t ssq, const ca_select_rule& rule, const PastBlocks& pb,
                               uint32_t* rowmask, float* scores_out, hipStream_t stream);

size_t union_lds_bytes(const Shape& s);

// FlashPrefill per-token block scores (the reference's compute_block_score_chunked +
// normalize_scores) in block_size (64 or 128) token blocks; s.cap = key blocks per row of the
// scores, khat rows hold khat_stride block means.
size_t token_mass_lds_bytes(const Shape& s, int bs);
hipError_t launch_token_mass(const Shape& s, const SeqAddr& q, const float* khat, int64_t khat_stride, int bs,
                             float scale, const PastBlocks& pb, float* scores, hipStream_t stream);
constexpr int kCsrRowsMax = 8192;
hipError_t launch_table_csr(const int32_t* table, int64_t table_stride, const int32_t* counts, int rows, int cap,
                            int32_t* indptr, int32_t* indices, int32_t* last_page_len, hipStream_t stream);

hipError_t launch_union_compact(const Shape& s, const uint32_t* rowmask, int last_n_block,
                                const uint8_t* keep_kv_in, const PastBlocks& pb, uint8_t* keep_block,
                                uint8_t* keep_kv, int32_t* table, int64_t table_stride,
                                int32_t* counts, bool dense, hipStream_t stream);

struct AttnArgs {
    Shape s;
    SeqAddr q;
    KvAddr k, v;
    const int32_t* table;
    int64_t table_stride;
    const int32_t* counts;
    PastBlocks pb;
    float scale;
    SeqAddr out;
    float* lse;
    int num_splits;  // > 0: every request uses this many splits; 0: per-request plan
    void* workspace;
    const int32_t* kv_len;  // decode: host array of per-request KV lengths (tokens); else null
};

constexpr int kMaxPrefillSplits = 16;
constexpr int kMaxDecodeSplits = 64;

// Split-KV plan.  Request b's block lists are cut into s[b] pieces (max = the largest,
// which sizes the workspace).  Work placement: with at most kPlanRows KV rows, whole rows
// go to XCDs (longest first, each to the least-loaded XCD), so a row's items share one L2
// and the XCDs carry equal work: entries xoff[x] .. xoff[x+1] list XCD x's units in order,
// each a row (xrow) and a range of its splits (xlo, xcnt).  When the rows do not divide
// evenly over the XCDs, each split of a row is a unit of its own, so the XCDs' loads even
// out; its items stream a disjoint part of the row's block list.
// Otherwise items are numbered request by request (off[b]) and dealt to XCDs in
// contiguous ranges.
constexpr int kPlanRows = 512;
struct SplitPlan {
    int32_t s[CA_MAX_BATCH];
    int32_t off[CA_MAX_BATCH + 1];
    int max;
    int use_rows;
    int per_xcd;      // work items per XCD (grid = 8 * per_xcd)
    int may_unsplit;  // the kernel drops the splits when the rows' selected counts are even
    uint16_t xrow[kPlanRows];  // placement units: a row and a range of its splits
    uint8_t xlo[kPlanRows];    // first split of the unit
    uint8_t xcnt[kPlanRows];   // splits in the unit
    int32_t xoff[9];
};

// dense = identity block lists over kv_len tokens (decode); otherwise per-row tables
void attn_plan(const Shape& s, const int32_t* nkb, int forced, bool dense, SplitPlan* plan);
bool attn_uses_decode_kernel(const Shape& s, bool dense);
void attn_positions(const Shape& s, const PastBlocks& pb, const int32_t* kv_len, int32_t* qpos0, int32_t* nkb);
int attn_pick_splits(const Shape& s, const PastBlocks& pb, const int32_t* kv_len);
int64_t attn_workspace_bytes(const Shape& s, int num_splits);
hipError_t launch_attn(const AttnArgs& a, hipStream_t stream);

// model plumbing (ca_model.hip)
hipError_t launch_rope(const SeqAddr& x, const SeqAddr& y, const float* cos, const float* sin, int B, int L, int H,
                       hipStream_t stream);
hipError_t launch_rmsnorm(const uint16_t* x, int64_t x_stride, const uint16_t* r, int64_t r_stride, uint16_t* s,
                          int64_t s_stride, const uint16_t* w, uint16_t* y, int64_t y_stride, int64_t rows, int n,
                          float eps, hipStream_t stream);
hipError_t launch_swiglu(const uint16_t* g, int64_t g_stride, const uint16_t* u, int64_t u_stride, uint16_t* y,
                         int64_t y_stride, int64_t rows, int n, hipStream_t stream);

}  // namespace ca
