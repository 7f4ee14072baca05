// Device-side view of a KV cache (contiguous or block-paged) and the host
// conversion from the public supersonic_kv_cache struct.
#pragma once

#include "common.hpp"
#include "../../include/supersonic_attn.h"

namespace ssa {

struct KvView {
    uint8_t* k;
    uint8_t* v;
    float* ks;
    float* vs;
    const int32_t* bt;
    int64_t seq_stride;
    int64_t head_stride;
    int64_t page_stride;
    int page_size;
    int max_pages;
    int64_t s_seq;
    int64_t s_head;
    int64_t s_page;

    // Element offset of the row of token t (sequence b, kv head h).
    __device__ __forceinline__ int64_t row(int b, int h, int t, int D) const {
        if (bt) {
            const int pg = bt[static_cast<int64_t>(b) * max_pages + t / page_size];
            return static_cast<int64_t>(pg) * page_stride + h * head_stride +
                   static_cast<int64_t>(t % page_size) * D;
        }
        return b * seq_stride + h * head_stride + static_cast<int64_t>(t) * D;
    }
    // row() for a wave-uniform (b, h, t): the block-table entry comes through
    // the scalar cache (the table is read-only while a kernel runs), so the
    // load is counted by lgkmcnt and waiting for it never drains the wave's
    // outstanding vector loads.
    __device__ __forceinline__ int64_t row_uniform(int b, int h, int t, int D) const {
        if (bt) {
            typedef const __attribute__((address_space(4))) int32_t* cptr;
            const cptr cbt = reinterpret_cast<cptr>(reinterpret_cast<uintptr_t>(bt));
            const int pg = cbt[static_cast<int64_t>(b) * max_pages + t / page_size];
            return static_cast<int64_t>(pg) * page_stride + h * head_stride +
                   static_cast<int64_t>(t % page_size) * D;
        }
        return b * seq_stride + h * head_stride + static_cast<int64_t>(t) * D;
    }
    // srow() for a wave-uniform (b, h, t), through the scalar cache as row_uniform().
    __device__ __forceinline__ int64_t srow_uniform(int b, int h, int t) const {
        if (bt) {
            typedef const __attribute__((address_space(4))) int32_t* cptr;
            const cptr cbt = reinterpret_cast<cptr>(reinterpret_cast<uintptr_t>(bt));
            const int pg = cbt[static_cast<int64_t>(b) * max_pages + t / page_size];
            return static_cast<int64_t>(pg) * s_page + h * s_head + (t % page_size);
        }
        return b * s_seq + h * s_head + t;
    }
    // Offset of token t's fp8 scale.
    __device__ __forceinline__ int64_t srow(int b, int h, int t) const {
        if (bt) {
            const int pg = bt[static_cast<int64_t>(b) * max_pages + t / page_size];
            return static_cast<int64_t>(pg) * s_page + h * s_head + (t % page_size);
        }
        return b * s_seq + h * s_head + t;
    }
};

// Validates the view for a kernel that walks 16-token blocks.  Returns 0 or
// SUPERSONIC_ERR_CACHE.
inline int make_view(const supersonic_kv_cache* c, bool fp8, KvView* out) {
    if (!c || !c->k || !c->v) return SUPERSONIC_ERR_NULL;
    if (fp8 && (!c->k_scale || !c->v_scale)) return SUPERSONIC_ERR_NULL;
    if (c->block_table) {
        if (c->page_size <= 0 || (c->page_size % 16) != 0 || c->max_pages_per_seq <= 0)
            return SUPERSONIC_ERR_CACHE;
    }
    out->k = static_cast<uint8_t*>(c->k);
    out->v = static_cast<uint8_t*>(c->v);
    out->ks = c->k_scale;
    out->vs = c->v_scale;
    out->bt = c->block_table;
    out->seq_stride = c->seq_stride;
    out->head_stride = c->head_stride;
    out->page_stride = c->page_stride;
    out->page_size = c->block_table ? c->page_size : 1;
    out->max_pages = c->max_pages_per_seq;
    out->s_seq = c->scale_seq_stride;
    out->s_head = c->scale_head_stride;
    out->s_page = c->scale_page_stride;
    return 0;
}

}  // namespace ssa
