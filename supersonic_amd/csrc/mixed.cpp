// Mixed step: one prefill chunk and a batch of decodes of the same layer in
// one call, run at the same time on disjoint compute units.
//
// The decode is HBM-bound and the chunk MFMA-bound, so back to back each
// leaves the other's resource idle.  Neither kernel fits beside the other on
// a CU (the prefill workgroup takes 133 KB of LDS and three waves a SIMD at
// ~168 registers; a decode wave up to 256 registers), so the split is by CU:
//   1. the decode goes first on the caller's stream, planned for c
//      workgroups (one a CU), and occupies about c CUs;
//   2. the chunk's staging kernel and the prefill kernel go on a library
//      stream forked from the caller's; the prefill grid is the whole GPU on
//      the dynamic item schedule (items claimed longest first, each as the
//      previous one nears its end), so the workgroups that find a free CU
//      start at once and the rest as the decode's CUs free up, taking only
//      what is left;
//   3. the caller's stream waits for the library stream.
// Launch order keeps the decode's CUs its own: its workgroups are dispatched
// before the prefill's are enqueued.  c comes from the two parts' estimated
// times (mixed_decode_wgs); SUPERSONIC_MIXED_DECODE_WGS sets it (0: the two
// one after the other on the caller's stream).
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

// Decode workgroups of the CU split: c = n_cu * clamp(0.25 + 0.9 r, 0.5,
// 0.875) rounded to a multiple of 32, r = t_d / (t_d + t_p), with the decode's
// time t_d estimated as its K/V bytes at 6.4 TB/s (sequence lengths taken as
// max_kv_len / 2 on average; the lengths themselves are in device memory) and
// the chunk's t_p as its causal flops at 1.0 PF/s.  The decode on c CUs runs
// slower than its share of the GPU would suggest (each workgroup's loads in
// flight bound its rate), so c sits above the time share.  Fitted on config-5
// shapes, 16/2 heads, D 256 (one MI355X; c = 96..224 swept): 32 decodes of
// U[512, 65536] + an 8192-token chunk best at 160, 16 decodes + 8192 at 128,
// 8 + 8192 at 128, 32 + a 4096-token chunk at 224, the values this picks.
int mixed_decode_wgs(int n_cu, bool fp8, size_t Hq, size_t Hkv, size_t D, const supersonic_prefill_chunk* c,
                     const supersonic_decode_batch* d) {
    const double esz = fp8 ? 1.0 + 4.0 / static_cast<double>(D) : 2.0;  // + the per-token scales
    const double bytes = static_cast<double>(d->batch) * (0.5 * static_cast<double>(d->max_kv_len)) * 2.0 *
                         static_cast<double>(Hkv) * static_cast<double>(D) * esz;
    const double S = static_cast<double>(c->chunk_len), L0 = static_cast<double>(c->chunk_start);
    const double flops = 4.0 * static_cast<double>(Hq) * static_cast<double>(D) * S * (L0 + 0.5 * (S + 1.0));
    const double td = bytes / 6.4e12, tp = flops / 1.0e15;
    const double r = td / std::max(td + tp, 1e-12);
    const double f = std::min(0.875, std::max(0.5, 0.25 + 0.9 * r));
    const int w = (static_cast<int>(f * n_cu + 16.0) / 32) * 32;
    return std::max(32, std::min(w, n_cu));
}


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
    int wgs = env_int("SUPERSONIC_MIXED_DECODE_WGS", -1);  // unset: from the estimate; 0: one after the other
    if (has_c && has_d && wgs < 0) {
        int n_cu = device_cu_count(dev);
        if (n_cu <= 0) n_cu = 256;
        wgs = mixed_decode_wgs(n_cu, kv_dtype == SUPERSONIC_KV_FP8_E4M3, q_heads, kv_heads, head_dim, chunk, decode);
    }
    if (has_c && has_d && wgs == 0) {
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
