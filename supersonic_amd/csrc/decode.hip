// Split-K GQA decode attention for gfx950.
//
// Replaces the reference's decode attention cores:
//   * pfx_full_attention_decode_flat_kernel  kernels/prefill_helpers.hip:319-404
//     (one 32-lane block per query head, K read twice, serial over tokens);
//   * the megakernel attention phase        kernels/full_attention_4b.hip:5109-5470
//     (QK-norm, RoPE, KV append, FP8 quantise, online softmax, gate; block 0
//     of the whole grid, two barriers per token).
//
// Design (HBM-bound; every K/V byte is read exactly once):
//   grid  = (split, kv_head, batch); a workgroup owns `chunk` consecutive tokens
//           of one kv head and serves all G = Hq/Hkv query heads that share it.
//   block = 4 wave64s; wave w takes the 16-token blocks w, w+4, ... of the chunk,
//           with the next block's K/V loads in flight (two register sets)
//           while the current one is computed; two workgroups per CU.
//   loads : buffer loads against a resource bound to the block's live rows
//           (rows past kv_len read as zero), one per-lane offset per operand.
//   QK^T  : v_mfma_f32_16x16x32_{bf16,f16}.  A = the G query heads (rows, zero
//           padded to 16, kept in LDS), B = 16 tokens of K loaded straight from
//           HBM in the B-operand layout (16 B per lane per k-step).  The score tile lands
//           with one token per lane of each 16-lane DPP row, so softmax row
//           statistics are 4 DPP row_ror steps.
//   softmax: online, base 2, per head; per-lane partial sums reduced once.
//   PV    : VALU; each lane owns 8 dims of one token (128-bit loads), P is
//           broadcast through a per-wave LDS tile.
//   merge : the 4 waves merge through LDS; the last split of each (b, kv head)
//           to arrive (device-scope counter) merges the splits (log-sum-exp)
//           and applies the sigmoid gate, so one kernel does the whole step.
//   FP8   : e4m3 bytes -> bf16 with the hardware OCP converter; the per-token
//           K scale multiplies the score, the V scale multiplies p.
//   Fused prologue: the workgroup normalises + rotates its q heads; the split
//           that owns the new token also normalises + rotates k, writes K/V
//           (or fp8 codes + scales) into the cache and, after its cached
//           blocks, processes the new token as a one-token block read from LDS,
//           unquantised (as full_attention_4b.hip:5351-5353 does).
#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "common.hpp"
#include "kv_view.hpp"

#include "decode_split.hpp"

namespace ssa {

// The 4-wave kernels (head groups of 8 and 16) are held to two waves a SIMD
// (235 registers instead of 300): two workgroups a CU, so the ragged plan's
// target of 512 workgroups is resident at once (config 5's decodes 338.6 ->
// 331 us).
template <typename QT, bool FP8, int D, int GP>
__global__ __launch_bounds__(64 * decode_waves(GP)) __attribute__((amdgpu_waves_per_eu(GP >= 8 ? 2 : 1, 2)))
void decode_split_kernel(DecodeParams p) {
    __shared__ DecodeLds<D, GP> lds;
    decode_split_body<QT, FP8, D, GP>(p, blockIdx.x, blockIdx.y, blockIdx.z, lds);
}

// ----------------------------------------------------------------------------
// Host launch
// ----------------------------------------------------------------------------
struct SplitPlan {
    int chunk;
    int nsplit;
};

static int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    if (!v || !*v) return dflt;
    return atoi(v);
}

// Chunk of tokens per workgroup: enough workgroups to fill 256 CUs a few
// times over, but chunks of at least 64 tokens (4 waves x 16).
static int decode_target(int waves) {
    // 2048 resident waves: one 8-wave or two 4-wave workgroups per CU
    return std::max(1, env_int("SUPERSONIC_DECODE_TARGET_WGS", 2048 / waves));
}
static int decode_deterministic() { return env_int("SUPERSONIC_DECODE_DETERMINISTIC", 0) != 0; }
static int decode_min_chunk() { return std::max(64, env_int("SUPERSONIC_DECODE_MIN_CHUNK", 128)); }

// Uniform plan (one length for the whole batch): the same split count for
// every sequence.
static SplitPlan plan_splits(int B, int Hkv, int max_len, int waves) {
    const int target = decode_target(waves);
    const int min_chunk = decode_min_chunk();
    const int pairs = B * Hkv;
    int want = (target + pairs - 1) / pairs;
    if (want < 1) want = 1;
    int chunk = (max_len + want - 1) / want;
    chunk = ((chunk + 63) / 64) * 64;
    if (chunk < min_chunk) chunk = min_chunk;
    int nsplit = (max_len + chunk - 1) / chunk;
    if (nsplit < 1) nsplit = 1;
    return {chunk, nsplit};
}

// Partial rows of a call: the uniform plan needs B * Hq * nsplit; the ragged
// plan at most (ceil(target / Hkv) + B) * Hq (sum over b of ceil(len_b /
// chunk) <= total / chunk + B, and chunk >= total * Hkv / target).  Sized for
// the larger so that either plan fits.
static size_t decode_rows(int B, int Hq, int Hkv, int max_len, int waves) {
    const SplitPlan sp = plan_splits(B, Hkv, max_len, waves);
    const size_t uni = static_cast<size_t>(B) * Hq * sp.nsplit;
    const int target = decode_target(waves);
    const size_t rag = (static_cast<size_t>((target + Hkv - 1) / Hkv) + B) * Hq;
    return std::max(uni, rag);
}

static size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Workspace: [arrival counters, kArrivalBytes][part_o][part_ml].  The
// counters sit at a fixed offset so they never overlap partials of a call
// with another shape; they are zero before the first call (a fresh library
// workspace is zero-filled) and every call leaves them zero.
constexpr size_t kArrivalBytes = 64 * 1024;
constexpr int kMaxArrivals = static_cast<int>(kArrivalBytes / sizeof(unsigned));

static size_t workspace_bytes_for(size_t rows, int D) {
    return kArrivalBytes + align256(rows * D * sizeof(float)) + align256(rows * 2 * sizeof(float));
}

template <typename QT, bool FP8, int D>
static hipError_t launch_split(dim3 grid, hipStream_t st, int GP, const DecodeParams& p) {
    switch (GP) {
    case 4: hipLaunchKernelGGL((decode_split_kernel<QT, FP8, D, 4>), grid, dim3(64 * decode_waves(4)), 0, st, p); break;
    case 8: hipLaunchKernelGGL((decode_split_kernel<QT, FP8, D, 8>), grid, dim3(64 * decode_waves(8)), 0, st, p); break;
    default: hipLaunchKernelGGL((decode_split_kernel<QT, FP8, D, 16>), grid, dim3(64 * decode_waves(16)), 0, st, p); break;
    }
    return hipGetLastError();
}

template <typename QT, bool FP8>
static hipError_t launch_split_d(int D, dim3 grid, hipStream_t st, int GP, const DecodeParams& p) {
    switch (D) {
    case 64: return launch_split<QT, FP8, 64>(grid, st, GP, p);
    case 128: return launch_split<QT, FP8, 128>(grid, st, GP, p);
    case 256: return launch_split<QT, FP8, 256>(grid, st, GP, p);
    default: return hipErrorInvalidValue;
    }
}

struct DecodeRequest {
    int qdtype;       // 0 f16, 2 bf16
    bool fp8;
    int B, Hq, Hkv, D;
    int max_len;
    float scale;
    DecodeParams prm;         // q/lens/fused fields filled by the caller
    const uint16_t* gate;
    int64_t g_bstride, g_hstride;
    void* out;
    void* workspace;
    size_t workspace_bytes;
    int device;
    hipStream_t stream;
    bool ragged;      // per-sequence lengths: plan on the device from the lengths
    int target;       // ragged plan: workgroups to plan for (0: one round on the whole GPU)
};

// Returns 0, or a SUPERSONIC_ERR_* status.
static int run_decode(DecodeRequest& r) {
    if (r.D != 64 && r.D != 128 && r.D != 256) return SUPERSONIC_ERR_HEAD_DIM;
    if (r.Hkv <= 0 || r.Hq % r.Hkv != 0) return SUPERSONIC_ERR_HEADS;
    const int G = r.Hq / r.Hkv;
    if (G > 16) return SUPERSONIC_ERR_HEADS;
    const int GP = G <= 4 ? 4 : (G <= 8 ? 8 : 16);
    if (r.B <= 0) return 0;
    if (static_cast<int64_t>(r.B) * r.Hkv > kMaxArrivals) return SUPERSONIC_ERR_RANGE;
    if (r.max_len <= 0) r.max_len = 1;
    const int waves = decode_waves(GP);
    const SplitPlan sp = plan_splits(r.B, r.Hkv, r.max_len, waves);
    const size_t rows = decode_rows(r.B, r.Hq, r.Hkv, r.max_len, waves);
    const size_t need = workspace_bytes_for(rows, r.D);
    void* ws = r.workspace;
    if (ws) {
        if (r.workspace_bytes < need) return SUPERSONIC_ERR_WORKSPACE;
    } else {
        ws = device_workspace(r.device, need, kWorkspaceDecode);
        if (!ws) return SUPERSONIC_ERR_WORKSPACE;
    }
    DecodeParams& p = r.prm;
    p.Hq = r.Hq;
    p.Hkv = r.Hkv;
    p.G = G;
    p.chunk = sp.chunk;
    p.nsplit = sp.nsplit;
    p.ragged = r.ragged ? 1 : 0;
    p.B = r.B;
    p.target = r.ragged && r.target > 0 ? std::min(r.target, decode_target(waves)) : decode_target(waves);
    p.min_chunk = decode_min_chunk();
    p.det = decode_deterministic();
    p.scale_log2 = r.scale * kLog2e;
    p.arrivals = static_cast<unsigned*>(ws);
    p.arr_stride = arrival_stride(static_cast<long long>(r.B) * r.Hkv, kMaxArrivals);
    p.merge_polls = wait_polls(kMergePoll);
    p.part_o = reinterpret_cast<float*>(static_cast<char*>(ws) + kArrivalBytes);
    p.part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + kArrivalBytes + align256(rows * r.D * sizeof(float)));
    p.gate = r.gate;
    p.g_bstride = r.g_bstride;
    p.g_hstride = r.g_hstride;
    p.out = r.out;

    // ragged: one workgroup per item, at most target + B * Hkv items
    const dim3 grid = r.ragged ? dim3(static_cast<unsigned>(p.target + r.B * r.Hkv), 1, 1)
                               : dim3(sp.nsplit, r.Hkv, r.B);
    const ProfileEvents prof = take_profile_events();
    if (prof.before) (void)hipEventRecord(prof.before, r.stream);
    hipError_t e;
    if (r.fp8) e = launch_split_d<bf16_t, true>(r.D, grid, r.stream, GP, p);
    else if (r.qdtype == 0) e = launch_split_d<f16_t, false>(r.D, grid, r.stream, GP, p);
    else e = launch_split_d<bf16_t, false>(r.D, grid, r.stream, GP, p);
    if (e != hipSuccess) return SUPERSONIC_ERR_LAUNCH;
    if (prof.after) (void)hipEventRecord(prof.after, r.stream);

    return 0;
}

// Uniform kv_len for the drop-in entry points: a device array of B copies,
// kept per device and refreshed only when the value or batch changes.
static const int32_t* uniform_lens(int device, int B, int kv_len, hipStream_t st, size_t ws_need) {
    (void)ws_need;
    static std::mutex mu;
    std::lock_guard<std::mutex> lock(mu);
    static std::vector<int32_t*> bufs;
    static std::vector<std::pair<int, int>> keys;
    if (static_cast<size_t>(device) >= bufs.size()) {
        bufs.resize(device + 1, nullptr);
        keys.resize(device + 1, {-1, -1});
    }
    if (keys[device].first < B) {
        if (bufs[device]) (void)hipFree(bufs[device]);
        bufs[device] = nullptr;
        int cap = B < 64 ? 64 : B;
        if (hipMalloc(&bufs[device], cap * sizeof(int32_t)) != hipSuccess) return nullptr;
        keys[device] = {cap, -1};
    }
    if (keys[device].second != kv_len) {
        std::vector<int32_t> h(keys[device].first, kv_len);
        if (hipMemcpy(bufs[device], h.data(), h.size() * sizeof(int32_t), hipMemcpyHostToDevice) != hipSuccess)
            return nullptr;
        keys[device].second = kv_len;
    }
    (void)st;
    return bufs[device];
}

int prefill_dropin(int dtype, size_t device, size_t B, size_t Hq, size_t Hkv, size_t q_len, size_t kv_len, size_t D,
                   size_t groups, float scale, size_t off, const void* q, const void* k, const void* v, void* out);

static int decode_flat_common(int dtype, size_t device, size_t B, size_t Hq, size_t Hkv, size_t kv_len,
                              size_t kv_stride, size_t D, size_t groups, float scale, const void* q,
                              const void* k, const void* v, void* out) {
    if (dtype != 0 && dtype != 2) return 400;
    if (D == 0 || D > 256) return 401;
    if (Hkv == 0 || groups == 0 || Hq != Hkv * groups) return 401;
    if ((D != 64 && D != 128 && D != 256) || groups > 16) {
        // General shape (the reference takes any D <= 256 and any group
        // size): with at most 16 query heads per kv head, the split-K kernel
        // on copies zero-padded to the next native head size (zero dims add
        // nothing to q.k; the padded output dims are dropped); with more, the
        // f32 prefill kernel as a one-row prefill over all kv_len keys.
        ScopedDevice scoped(static_cast<int>(device));
        if (B == 0 || Hq == 0) return hipDeviceSynchronize() == hipSuccess ? 0 : 403;
        const int64_t nq = static_cast<int64_t>(B * Hq), nkv = static_cast<int64_t>(B * Hkv);
        const int64_t nk = nkv * static_cast<int64_t>(kv_len);
        const int d = static_cast<int>(D);
        const int64_t so = static_cast<int64_t>(kv_stride) * d;  // source (sequence, kv head) stride
        ScratchBuffers sb;
        int rc;
        if (groups <= 16) {
            const int dp = D <= 64 ? 64 : (D <= 128 ? 128 : 256);
            void* qp = sb.get(nq * dp * 2);
            void* kp = sb.get(nk * dp * 2);
            void* vp = sb.get(nk * dp * 2);
            void* op = sb.get(nq * dp * 2);
            if (!qp || !kp || !vp || !op) return 402;
            if (repack_rows(dtype, dtype, q, qp, nq, 1, d, 0, d, dp, nullptr) != hipSuccess ||
                repack_rows(dtype, dtype, k, kp, nkv, kv_len, so, d, d, dp, nullptr) != hipSuccess ||
                repack_rows(dtype, dtype, v, vp, nkv, kv_len, so, d, d, dp, nullptr) != hipSuccess)
                return 402;
            rc = decode_flat_common(dtype, device, B, Hq, Hkv, kv_len, kv_len, dp, groups, scale, qp, kp, vp, op);
            if (rc == 0 && repack_rows(dtype, dtype, op, out, nq, 1, dp, 0, d, d, nullptr) != hipSuccess) rc = 402;
        } else {
            void* qf = sb.get(nq * d * 4);
            void* kf = sb.get(nk * d * 4);
            void* vf = sb.get(nk * d * 4);
            void* of = sb.get(nq * d * 4);
            if (!qf || !kf || !vf || !of) return 402;
            if (repack_rows(dtype, 1, q, qf, nq, 1, d, 0, d, d, nullptr) != hipSuccess ||
                repack_rows(dtype, 1, k, kf, nkv, kv_len, so, d, d, d, nullptr) != hipSuccess ||
                repack_rows(dtype, 1, v, vf, nkv, kv_len, so, d, d, d, nullptr) != hipSuccess)
                return 402;
            rc = prefill_dropin(1, device, B, Hq, Hkv, 1, kv_len, D, groups, scale, kv_len > 0 ? kv_len - 1 : 0, qf,
                                kf, vf, of);
            rc = rc == 0 ? 0 : (rc == 12 ? 403 : 402);
            if (rc == 0 && repack_rows(1, dtype, of, out, nq, 1, d, 0, d, d, nullptr) != hipSuccess) rc = 402;
        }
        if (hipDeviceSynchronize() != hipSuccess && rc == 0) rc = 403;
        return rc;
    }
    ScopedDevice scoped(static_cast<int>(device));
    const int dev = static_cast<int>(device);
    const int32_t* lens = uniform_lens(dev, static_cast<int>(B), static_cast<int>(kv_len), nullptr, 0);
    if (!lens) return 402;
    DecodeRequest r{};
    r.qdtype = dtype;
    r.fp8 = false;
    r.B = static_cast<int>(B);
    r.Hq = static_cast<int>(Hq);
    r.Hkv = static_cast<int>(Hkv);
    r.D = static_cast<int>(D);
    r.max_len = static_cast<int>(kv_len);
    r.scale = scale;
    r.device = dev;
    r.stream = nullptr;
    r.out = out;
    DecodeParams& p = r.prm;
    p.kv.k = static_cast<uint8_t*>(const_cast<void*>(k));
    p.kv.v = static_cast<uint8_t*>(const_cast<void*>(v));
    p.kv.ks = p.kv.vs = nullptr;
    p.kv.bt = nullptr;
    p.kv.page_size = 1;
    p.kv.head_stride = static_cast<int64_t>(kv_stride) * D;
    p.kv.seq_stride = static_cast<int64_t>(Hkv) * kv_stride * D;
    p.q = static_cast<const uint16_t*>(q);
    p.q_bstride = static_cast<int64_t>(Hq) * D;
    p.q_hstride = static_cast<int64_t>(D);
    p.lens = lens;
    p.len_plus = 0;
    p.fused = 0;
    // kv_len == 0: split 0 of every (b, kv head) writes zeros.
    const int rc = run_decode(r);
    if (rc == SUPERSONIC_ERR_LAUNCH || rc == SUPERSONIC_ERR_WORKSPACE) return 402;
    if (rc != 0) return 401;
    if (hipDeviceSynchronize() != hipSuccess) return 403;
    // a merge that gave up on a partial (workspace not in its between-calls
    // state) wrote a wrong row: report it as the sync failure
    unsigned werr = 0;
    if (take_wait_error(&werr) != hipSuccess || werr != 0) return 403;
    return 0;
}

hipError_t take_wait_error_decode(unsigned* bits) { return take_wait_error(bits); }

}  // namespace ssa

using namespace ssa;

extern "C" int supersonic_qwen35_hip_full_attention_decode_flat(
    int dtype, size_t device_ordinal, size_t batch_size, size_t q_heads, size_t kv_heads,
    size_t kv_len, size_t head_dim, size_t num_kv_groups, float scale,
    const void* query, const void* key, const void* value, void* out) {
    return decode_flat_common(dtype, device_ordinal, batch_size, q_heads, kv_heads, kv_len, kv_len,
                              head_dim, num_kv_groups, scale, query, key, value, out);
}

extern "C" int supersonic_qwen35_hip_full_attention_decode_flat_strided(
    int dtype, size_t device_ordinal, size_t batch_size, size_t q_heads, size_t kv_heads,
    size_t kv_len, size_t kv_stride, size_t head_dim, size_t num_kv_groups, float scale,
    const void* query, const void* key, const void* value, void* out) {
    if (kv_stride < kv_len) return 401;
    return decode_flat_common(dtype, device_ordinal, batch_size, q_heads, kv_heads, kv_len, kv_stride,
                              head_dim, num_kv_groups, scale, query, key, value, out);
}

extern "C" size_t supersonic_attn_gfx950_decode_workspace_size(
    size_t batch, size_t q_heads, size_t kv_heads, size_t head_dim, size_t max_kv_len) {
    if (kv_heads == 0) return 0;
    const size_t G = q_heads / kv_heads;
    const int GP = G <= 4 ? 4 : (G <= 8 ? 8 : 16);
    const size_t rows = decode_rows(static_cast<int>(batch), static_cast<int>(q_heads), static_cast<int>(kv_heads),
                                    max_kv_len ? static_cast<int>(max_kv_len) : 1, decode_waves(GP));
    return workspace_bytes_for(rows, static_cast<int>(head_dim));
}

static int check_sizes(size_t a, size_t b, size_t c, size_t d, size_t e) {
    const size_t lim = 0x7FFFFFFF;
    return (a > lim || b > lim || c > lim || d > lim || e > lim) ? SUPERSONIC_ERR_RANGE : 0;
}

// The fused decode planned for `target_wgs` workgroups (0: the whole GPU);
// supersonic_attn_gfx950_decode is the whole-GPU one.
int ssa::decode_native(size_t device_ordinal, void* stream, int kv_dtype, size_t batch, size_t q_heads,
                  size_t kv_heads, size_t head_dim, size_t rotary_dim, size_t max_kv_len, float eps, float scale,
                  const void* q_proj, const void* k_new, const void* v_new, const void* q_norm_w,
                  const void* k_norm_w, const void* cos_table, const void* sin_table, const int32_t* positions,
                  const supersonic_kv_cache* cache, void* out, void* workspace, size_t workspace_bytes,
                  int target_wgs) {
    if (kv_dtype != SUPERSONIC_KV_BF16 && kv_dtype != SUPERSONIC_KV_FP8_E4M3) return SUPERSONIC_ERR_DTYPE;
    if (int rc = check_sizes(batch, q_heads, kv_heads, head_dim, max_kv_len)) return rc;
    if (!q_proj || !k_new || !v_new || !q_norm_w || !k_norm_w || !positions || !out) return SUPERSONIC_ERR_NULL;
    if (rotary_dim % 2 != 0 || rotary_dim > head_dim) return SUPERSONIC_ERR_ROTARY;
    if (rotary_dim > 0 && (!cos_table || !sin_table)) return SUPERSONIC_ERR_NULL;
    const bool fp8 = kv_dtype == SUPERSONIC_KV_FP8_E4M3;
    DecodeRequest r{};
    if (int rc = make_view(cache, fp8, &r.prm.kv)) return rc;
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return SUPERSONIC_ERR_HEAD_DIM;
    ScopedDevice scoped(static_cast<int>(device_ordinal));
    r.qdtype = 2;
    r.fp8 = fp8;
    r.B = static_cast<int>(batch);
    r.Hq = static_cast<int>(q_heads);
    r.Hkv = static_cast<int>(kv_heads);
    r.D = static_cast<int>(head_dim);
    r.max_len = static_cast<int>(max_kv_len);
    r.ragged = true;
    r.scale = scale;
    r.device = static_cast<int>(device_ordinal);
    r.stream = static_cast<hipStream_t>(stream);
    r.out = out;
    r.workspace = workspace;
    r.workspace_bytes = workspace_bytes;
    r.gate = static_cast<const uint16_t*>(q_proj) + head_dim;  // per head [q | gate]
    r.g_bstride = static_cast<int64_t>(q_heads) * 2 * head_dim;
    r.g_hstride = 2 * static_cast<int64_t>(head_dim);
    DecodeParams& p = r.prm;
    p.q = static_cast<const uint16_t*>(q_proj);
    p.q_bstride = static_cast<int64_t>(q_heads) * 2 * head_dim;
    p.q_hstride = 2 * static_cast<int64_t>(head_dim);
    p.lens = positions;
    p.len_plus = 1;
    p.fused = 1;
    p.k_new = static_cast<const uint16_t*>(k_new);
    p.v_new = static_cast<const uint16_t*>(v_new);
    p.q_norm_w = static_cast<const uint16_t*>(q_norm_w);
    p.k_norm_w = static_cast<const uint16_t*>(k_norm_w);
    p.cos_t = static_cast<const uint16_t*>(cos_table);
    p.sin_t = static_cast<const uint16_t*>(sin_table);
    p.half_rot = static_cast<int>(rotary_dim / 2);
    p.eps = eps;
    r.target = target_wgs;
    return run_decode(r);
}

extern "C" int supersonic_attn_gfx950_decode(
    size_t device_ordinal, void* stream, int kv_dtype,
    size_t batch, size_t q_heads, size_t kv_heads, size_t head_dim, size_t rotary_dim,
    size_t max_kv_len, float eps, float scale,
    const void* q_proj, const void* k_new, const void* v_new,
    const void* q_norm_w, const void* k_norm_w, const void* cos_table, const void* sin_table,
    const int32_t* positions, const supersonic_kv_cache* cache, void* out,
    void* workspace, size_t workspace_bytes) {
    return decode_native(device_ordinal, stream, kv_dtype, batch, q_heads, kv_heads, head_dim, rotary_dim, max_kv_len,
                         eps, scale, q_proj, k_new, v_new, q_norm_w, k_norm_w, cos_table, sin_table, positions, cache,
                         out, workspace, workspace_bytes, 0);
}

// ----------------------------------------------------------------------------
// Allocation-free decode: the split partials and arrival counters live in a
// file-scope device array (one copy per GPU, held until the process ends)
// instead of a caller or library workspace.
// ----------------------------------------------------------------------------
constexpr size_t kScratchBytes = 8u << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // device address of `scratch`, per device
}  // namespace

// Device address of this device's `scratch` (the current device must be
// `device`), looked up once per device.  The array is zero when the code
// object is loaded (static device storage), which is the state the kernels
// need (arrival counters and partial slots at zero) and every call leaves it
// in, so no clearing work is enqueued: a first call under stream capture
// records nothing extra.  NULL if the lookup fails.
static void* scratch_for(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0) return nullptr;
    if (static_cast<size_t>(device) >= g_scratch_ptr.size()) g_scratch_ptr.resize(device + 1, nullptr);
    if (!g_scratch_ptr[device]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        g_scratch_ptr[device] = ptr;
    }
    return g_scratch_ptr[device];
}

extern "C" int supersonic_attn_gfx950_decode_noalloc(
    size_t device_ordinal, void* stream, int kv_dtype,
    size_t batch, size_t q_heads, size_t kv_heads, size_t head_dim, size_t rotary_dim,
    size_t max_kv_len, float eps, float scale,
    const void* q_proj, const void* k_new, const void* v_new,
    const void* q_norm_w, const void* k_norm_w, const void* cos_table, const void* sin_table,
    const int32_t* positions, const supersonic_kv_cache* cache, void* out) {
    if (kv_dtype != SUPERSONIC_KV_BF16 && kv_dtype != SUPERSONIC_KV_FP8_E4M3) return SUPERSONIC_ERR_DTYPE;
    if (int rc = check_sizes(batch, q_heads, kv_heads, head_dim, max_kv_len)) return rc;
    if (kv_heads == 0) return SUPERSONIC_ERR_HEADS;
    // shapes whose partials do not fit the scratch array are rejected up front
    if (supersonic_attn_gfx950_decode_workspace_size(batch, q_heads, kv_heads, head_dim, max_kv_len) > kScratchBytes)
        return SUPERSONIC_ERR_WORKSPACE;
    void* ws;
    {
        ScopedDevice scoped(static_cast<int>(device_ordinal));
        ws = scratch_for(static_cast<int>(device_ordinal));
    }
    if (!ws) return SUPERSONIC_ERR_WORKSPACE;
    return supersonic_attn_gfx950_decode(device_ordinal, stream, kv_dtype, batch, q_heads, kv_heads, head_dim,
                                         rotary_dim, max_kv_len, eps, scale, q_proj, k_new, v_new, q_norm_w,
                                         k_norm_w, cos_table, sin_table, positions, cache, out, ws, kScratchBytes);
}

extern "C" int supersonic_attn_gfx950_decode_attend(
    size_t device_ordinal, void* stream, int kv_dtype,
    size_t batch, size_t q_heads, size_t kv_heads, size_t head_dim, size_t max_kv_len,
    float scale, const void* q, const int32_t* kv_lens, const supersonic_kv_cache* cache,
    const void* gate, void* out, void* workspace, size_t workspace_bytes) {
    if (kv_dtype != SUPERSONIC_KV_BF16 && kv_dtype != SUPERSONIC_KV_FP8_E4M3) return SUPERSONIC_ERR_DTYPE;
    if (int rc = check_sizes(batch, q_heads, kv_heads, head_dim, max_kv_len)) return rc;
    if (!q || !kv_lens || !out) return SUPERSONIC_ERR_NULL;
    const bool fp8 = kv_dtype == SUPERSONIC_KV_FP8_E4M3;
    DecodeRequest r{};
    if (int rc = make_view(cache, fp8, &r.prm.kv)) return rc;
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return SUPERSONIC_ERR_HEAD_DIM;
    ScopedDevice scoped(static_cast<int>(device_ordinal));
    r.qdtype = 2;
    r.fp8 = fp8;
    r.B = static_cast<int>(batch);
    r.Hq = static_cast<int>(q_heads);
    r.Hkv = static_cast<int>(kv_heads);
    r.D = static_cast<int>(head_dim);
    r.max_len = static_cast<int>(max_kv_len);
    r.ragged = true;
    r.scale = scale;
    r.device = static_cast<int>(device_ordinal);
    r.stream = static_cast<hipStream_t>(stream);
    r.out = out;
    r.workspace = workspace;
    r.workspace_bytes = workspace_bytes;
    r.gate = static_cast<const uint16_t*>(gate);
    r.g_bstride = static_cast<int64_t>(q_heads) * head_dim;
    r.g_hstride = static_cast<int64_t>(head_dim);
    DecodeParams& p = r.prm;
    p.q = static_cast<const uint16_t*>(q);
    p.q_bstride = static_cast<int64_t>(q_heads) * head_dim;
    p.q_hstride = static_cast<int64_t>(head_dim);
    p.lens = kv_lens;
    p.len_plus = 0;
    p.fused = 0;
    return run_decode(r);
}
