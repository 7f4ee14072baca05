// Mixed step: one prefill chunk and a batch of decodes of the same layer in
// one call.
//
// Default: the decode, then the chunk, on the caller's stream.  Optional
// (SUPERSONIC_MIXED_DECODE_WGS = c > 0): the two on disjoint compute units at
// the same time.  Neither kernel fits beside the other on a CU (the prefill
// workgroup takes 133 KB of LDS and three waves a SIMD at ~168 registers; a
// decode wave up to 256 registers), so the split is by CU:
//   1. the decode goes first on the caller's stream, planned for c
//      workgroups, and occupies about c CUs;
//   2. the chunk's staging kernel and the prefill kernel go on a library
//      stream forked from the caller's; the prefill grid is the whole GPU on
//      the dynamic item schedule (items claimed longest first from a
//      counter), so the workgroups that find a free CU start at once and the
//      rest as the decode's CUs free up, taking only what is left;
//   3. the caller's stream waits for the library stream.
// Launch order keeps the decode's CUs its own: its workgroups are dispatched
// before the prefill's are enqueued.  Measured at config 5 (8192-token chunk,
// 32 decodes of U[512, 65536] tokens) the split is no faster than the
// default (c = 128-384: 0.82-0.85 ms against 0.83 ms; c = 32-96: 0.94-1.75
// ms): a 4-wave decode workgroup streams only 20-40 GB/s, so the decode
// needs nearly every CU's loads in flight to reach its HBM rate.
#include <algorithm>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "supersonic_attn.h"

namespace ssa {
namespace {

struct MixedStreams {
    hipStream_t aux = nullptr;
    hipEvent_t fork = nullptr;
    hipEvent_t join = nullptr;
};
std::mutex g_mixed_mu;
std::vector<MixedStreams> g_mixed;

// The library stream and fork/join events of the current device (created on
// first use, default priority), returned by value: the table may grow while
// another device's call is using its entry.  False if they cannot be created.
bool mixed_streams(int device, MixedStreams* out) {
    std::lock_guard<std::mutex> lock(g_mixed_mu);
    if (device < 0) return false;
    if (static_cast<size_t>(device) >= g_mixed.size()) g_mixed.resize(device + 1);
    MixedStreams& m = g_mixed[device];
    if (!m.aux) {
        if (hipStreamCreateWithFlags(&m.aux, hipStreamNonBlocking) != hipSuccess) {
            m.aux = nullptr;
            return false;
        }
    }
    if (!m.fork && hipEventCreateWithFlags(&m.fork, hipEventDisableTiming) != hipSuccess) m.fork = nullptr;
    if (!m.join && hipEventCreateWithFlags(&m.join, hipEventDisableTiming) != hipSuccess) m.join = nullptr;
    if (!m.fork || !m.join) return false;
    *out = m;
    return true;
}

int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }


}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" size_t supersonic_attn_gfx950_mixed_workspace_size(int kv_dtype, size_t q_heads, size_t kv_heads,
                                                             size_t head_dim, const supersonic_prefill_chunk* chunk,
                                                             const supersonic_decode_batch* decode) {
    size_t n = kClaimBytes;
    if (decode && decode->batch)
        n += align256(supersonic_attn_gfx950_decode_workspace_size(decode->batch, q_heads, kv_heads, head_dim,
                                                                   decode->max_kv_len));
    if (chunk && chunk->chunk_len)
        n += align256(supersonic_attn_gfx950_prefill_workspace_size(kv_dtype, kv_heads, head_dim, chunk->chunk_len,
                                                                    chunk->chunk_start));
    return n;
}

extern "C" int supersonic_attn_gfx950_mixed(size_t device_ordinal, void* stream, int kv_dtype, size_t q_heads,
                                            size_t kv_heads, size_t head_dim, size_t rotary_dim, float eps,
                                            float scale, const void* q_norm_w, const void* k_norm_w,
                                            const void* cos_table, const void* sin_table,
                                            const supersonic_prefill_chunk* chunk,
                                            const supersonic_decode_batch* decode, void* workspace,
                                            size_t workspace_bytes) {
    if (kv_dtype != SUPERSONIC_KV_BF16 && kv_dtype != SUPERSONIC_KV_FP8_E4M3) return SUPERSONIC_ERR_DTYPE;
    const bool has_c = chunk && chunk->chunk_len > 0;
    const bool has_d = decode && decode->batch > 0;
    const int dev = static_cast<int>(device_ordinal);
    // Workspace: [claim counters][decode][prefill], or the library's buffers.
    unsigned* claims = nullptr;
    void* dws = nullptr;
    void* pws = nullptr;
    size_t dbytes = 0, pbytes = 0;
    if (workspace) {
        const size_t need =
            supersonic_attn_gfx950_mixed_workspace_size(kv_dtype, q_heads, kv_heads, head_dim, chunk, decode);
        if (workspace_bytes < need) return SUPERSONIC_ERR_WORKSPACE;
        uint8_t* w = static_cast<uint8_t*>(workspace);
        claims = reinterpret_cast<unsigned*>(w);
        size_t o = kClaimBytes;
        if (has_d) {
            dbytes = align256(supersonic_attn_gfx950_decode_workspace_size(decode->batch, q_heads, kv_heads,
                                                                           head_dim, decode->max_kv_len));
            dws = w + o;
            o += dbytes;
        }
        if (has_c) {
            pws = w + o;
            pbytes = workspace_bytes - o;
        }
    }
    if (!has_c && !has_d) return 0;
    const int wgs = env_int("SUPERSONIC_MIXED_DECODE_WGS", 0);  // 0: one after the other
    if (has_c && has_d && wgs <= 0) {
        const int rc = decode_native(device_ordinal, stream, kv_dtype, decode->batch, q_heads, kv_heads, head_dim,
                                     rotary_dim, decode->max_kv_len, eps, scale, decode->q_proj, decode->k_new,
                                     decode->v_new, q_norm_w, k_norm_w, cos_table, sin_table, decode->positions,
                                     decode->cache, decode->out, dws, dbytes, 0);
        if (rc) return rc;
        return prefill_native(device_ordinal, stream, kv_dtype, q_heads, kv_heads, head_dim, rotary_dim,
                              chunk->chunk_len, chunk->chunk_start, eps, scale, chunk->q_proj, chunk->k_new,
                              chunk->v_new, q_norm_w, k_norm_w, cos_table, sin_table, chunk->cache, chunk->out, pws,
                              pbytes, nullptr);
    }
    if (!has_c)
        return decode_native(device_ordinal, stream, kv_dtype, decode->batch, q_heads, kv_heads, head_dim, rotary_dim,
                             decode->max_kv_len, eps, scale, decode->q_proj, decode->k_new, decode->v_new, q_norm_w,
                             k_norm_w, cos_table, sin_table, decode->positions, decode->cache, decode->out, dws,
                             dbytes, 0);
    if (!has_d)
        return prefill_native(device_ordinal, stream, kv_dtype, q_heads, kv_heads, head_dim, rotary_dim,
                              chunk->chunk_len, chunk->chunk_start, eps, scale, chunk->q_proj, chunk->k_new,
                              chunk->v_new, q_norm_w, k_norm_w, cos_table, sin_table, chunk->cache, chunk->out, pws,
                              pbytes, nullptr);

    ScopedDevice scoped(dev);
    if (!workspace) {
        claims = static_cast<unsigned*>(device_workspace(dev, kClaimBytes, kWorkspaceMixed));
        if (!claims) return SUPERSONIC_ERR_WORKSPACE;
    }
    MixedStreams streams;
    if (!mixed_streams(dev, &streams)) return SUPERSONIC_ERR_LAUNCH;
    const MixedStreams* ms = &streams;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // The library stream starts after the work queued on `stream` so far.
    if (hipEventRecord(ms->fork, st) != hipSuccess || hipStreamWaitEvent(ms->aux, ms->fork, 0) != hipSuccess)
        return SUPERSONIC_ERR_LAUNCH;
    int rc = decode_native(device_ordinal, stream, kv_dtype, decode->batch, q_heads, kv_heads, head_dim, rotary_dim,
                           decode->max_kv_len, eps, scale, decode->q_proj, decode->k_new, decode->v_new, q_norm_w,
                           k_norm_w, cos_table, sin_table, decode->positions, decode->cache, decode->out, dws, dbytes,
                           wgs);
    if (rc == 0)
        rc = prefill_native(device_ordinal, ms->aux, kv_dtype, q_heads, kv_heads, head_dim, rotary_dim,
                            chunk->chunk_len, chunk->chunk_start, eps, scale, chunk->q_proj, chunk->k_new,
                            chunk->v_new, q_norm_w, k_norm_w, cos_table, sin_table, chunk->cache, chunk->out, pws,
                            pbytes, claims);
    // Join even after an error, so `stream` never runs ahead of work already
    // queued on the library stream.
    if (hipEventRecord(ms->join, ms->aux) != hipSuccess || hipStreamWaitEvent(st, ms->join, 0) != hipSuccess)
        return rc ? rc : SUPERSONIC_ERR_LAUNCH;
    return rc;
}
