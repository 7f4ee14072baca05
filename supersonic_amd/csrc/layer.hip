// Persistent decode layer: the whole attention layer of a decode step in one
// kernel, the attention phase as a device function between the projections
// (the reference's persistent megakernel pattern,
// kernels/qwen36_moe_persistent/full_attn_phase.cuh:1-20, and the HIP
// megakernel's steps A-G, kernels/full_attention_4b.hip:4842-5577).
//
// One workgroup per compute unit (all of them resident at once: a cooperative
// launch), three phases
// separated by device-wide barriers:
//   1. input RMSNorm (applied while each workgroup stages the rows in LDS) and
//      the Q/K/V weight stream, 16 output columns per workgroup task;
//   2. the split-K attention step (QK RMSNorm, partial RoPE, KV append, online
//      softmax, last-arriver log-sum-exp merge, sigmoid gate): work item w of
//      the ragged plan on workgroup w;
//   3. the output projection with the residual add, in place on the hidden rows.
// Every value one phase hands to the next is stored and loaded with
// device-coherent accesses, so a barrier is: each wave waits for its own
// stores, one lane bumps a counter, the last to arrive raises a flag, and only
// the workgroups that read the previous phase's output wait (bounded) for the
// flag.  Launch fill and drain are paid once per layer instead of once per
// kernel.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "decode_split.hpp"
#include "kv_view.hpp"
#include "skinny.hpp"
#include "supersonic_attn.h"

namespace ssa {

struct LayerParams {
    SkinnyLdsParams qkv;  // phase 1: three segments, NORM staging from the hidden rows
    DecodeParams dec;     // phase 2: fused decode step, ragged plan over the grid
    SkinnyLdsParams op;   // phase 3: attn -> hidden (residual in place)
    unsigned* bar;        // barrier counters [0..2] and flags [32], [48] (another cache line), zero between calls
    int polls;            // bound of a barrier wait (kLayerSpin)
    // > 0: the decode step is expected to have this many work items (one
    // sequence of length max_kv_len); the last `hint` workgroups then take
    // them and skip phase 1, which the others share.
    int hint;
    int layer_len;        // host: the expected sequence length (max_kv_len), for the hint
};

constexpr int kLayerThreads = 64 * kSkinnyWaves;  // = 64 * decode_waves(4)
constexpr int kLayerSpin = 1 << 20;               // bounded barrier wait

// Every value one phase hands to the next is written and read with
// device-coherent (sc1) accesses, so the barrier needs no cache writeback or
// invalidate: each wave waits for its own stores to complete, then one lane
// counts the workgroup in; the last to arrive raises a flag on another cache
// line, which the waiting workgroups poll (polls on the counter's own line
// measured to hold back the arrivals' atomics).  The arriving lane is the
// last wave's first: it waits for the count to come back, and wave 0 goes on.
// Split form: arrive (after this workgroup's stores are complete), do
// independent work, then wait.
//
// Ordering: the producer's data stores are sc1 (written through to the
// device coherence point); `s_waitcnt vmcnt(0)` makes each wave wait until
// they are acknowledged there, the workgroup barrier orders every wave's wait
// before the counting atomic, and the compiler fences keep the stores above
// the wait.  A consumer issues its sc1 loads only after its poll has returned
// the flag (the poll result is waited for before the branch, and the
// workgroup barrier after the poll orders the other waves' loads after it),
// and sc1 loads are served from the coherence point, not from a stale
// per-XCD cache line.  This is what an agent-scope release / acquire pair
// provides, without the L2 writeback and invalidate those emit.
//
// The launch is cooperative (every workgroup co-resident, or the launch is
// refused), so a wait can only expire on a workspace whose counters were not
// zero: it then sets kWaitLayerBarrier in the error word and carries on, so
// that the kernel still exits.
constexpr int kArriveThread = kLayerThreads - 64;
__device__ __forceinline__ void grid_arrive(unsigned* ctr, unsigned* flag, unsigned n) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores are complete
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == kArriveThread) {
        const unsigned prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == n - 1) __hip_atomic_store(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}
__device__ __forceinline__ void grid_wait(unsigned* flag, int polls) {
    if (threadIdx.x == 0) {
        for (int it = 0;; ++it) {
            if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) break;
            if (it >= polls) {
                wait_expired(kWaitLayerBarrier);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

template <typename HT, bool FP8, int D>
__global__ __launch_bounds__(kLayerThreads) void decode_layer_kernel(LayerParams P) {
    static_assert(decode_waves(4) * 64 == kLayerThreads, "one workgroup shape for every phase");
    __shared__ union Lds {
        DecodeLds<D, 4> d;
        SkinnyLds s;
    } lds;
    const int w = blockIdx.x;
    const unsigned nwg = gridDim.x;
    const int ncb_qkv = P.qkv.cb_end[2], ncb_op = P.op.cb_end[2];
    // 1. input norm + Q/K/V projections on the first nq workgroups: column
    // blocks w, w + nq, ...; a workgroup with two left takes them together
    // (one staging of the rows, both weight streams in flight)
    const int nq = static_cast<int>(nwg) - P.hint;
    for (int cb = w; cb < ncb_qkv && w < nq;) {
        if (cb + nq < ncb_qkv) {
            skinny_lds_body<bf16_t, false, false, true, HT, false, true, SkinnyLds, true>(P.qkv, RopeEpi{}, cb, 0,
                                                                                           lds.s, cb + nq);
            cb += 2 * nq;
        } else {
            skinny_lds_body<bf16_t, false, false, true, HT, false, true>(P.qkv, RopeEpi{}, cb, 0, lds.s);
            cb += nq;
        }
        __syncthreads();
    }
    // 2. attention step (every workgroup plans the same ragged split).  The
    // work items go first to the workgroups that ran one phase-1 task (the
    // first ncb_qkv - nwg ran two), so the items start with their plan and
    // first K/V block (the cache does not depend on phase 1) while phase 1
    // finishes.  The workgroup arrives at barrier 0 first, then plans its item
    // and fetches its first block, and only then waits; a workgroup without
    // an item does not wait (only the readers of phase 1's output do).
    // With a hint the expected items sit on the workgroups without phase-1
    // work (any further item on the others).
    const int shift = min(max(ncb_qkv - static_cast<int>(nwg), 0), static_cast<int>(nwg));
    const int item = P.hint > 0 ? (w >= nq ? w - nq : P.hint + w)
                                : (w - shift + static_cast<int>(nwg)) % static_cast<int>(nwg);
    grid_arrive(&P.bar[0], &P.bar[32], nwg);
    bool had_item = false;
    decode_split_body<bf16_t, FP8, D, 4, true>(P.dec, item, 0, 0, lds.d, [&]() {
        grid_wait(&P.bar[32], P.polls);
        had_item = true;
    });
    if (!had_item && w < ncb_op) {
        // An output-projection workgroup without a decode item copies its
        // first task's weight rows into an LDS sink while the items run, so
        // that phase 3 finds them in this XCD's L2.  (The copies complete
        // before it arrives at barrier 1, which waits for its loads.)
        const int k = P.op.k;
        const int bytes = min(kSkinnyCols, P.op.n_seg[0] - w * kSkinnyCols) * k * 2;
        const __amdgpu_buffer_rsrc_t r =
            uniform_rsrc(reinterpret_cast<const uint8_t*>(P.op.w[0] + static_cast<int64_t>(w) * kSkinnyCols * k), bytes);
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        for (int off = wave * 1024; off < bytes; off += kSkinnyWaves * 1024)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds.s.xs, 16,
                                                     off + lane * 16, 0, 0, 0);
    }
    // Barrier 1: every workgroup arrives; those with an output-projection
    // task wait for all of them.
    grid_arrive(&P.bar[1], &P.bar[48], nwg);
    if (w < ncb_op) grid_wait(&P.bar[48], P.polls);
    // 3. output projection + residual
    for (int cb = w; cb < ncb_op; cb += nwg) {
        skinny_lds_body<HT, true, false, false, bf16_t, true, false>(P.op, RopeEpi{}, cb, 0, lds.s);
        __syncthreads();
    }
    // The last workgroup to finish resets every counter and flag: each
    // workgroup counts itself in here after its last arrival and its last
    // poll, so nothing reads or bumps them any more in this call, whether or
    // not a wait gave up.
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(&P.bar[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == nwg - 1) {
            __hip_atomic_store(&P.bar[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&P.bar[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&P.bar[32], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&P.bar[48], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&P.bar[2], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Workgroups of one layer-kernel instance resident at once, per device.
template <typename HT, bool FP8, int D>
static int layer_grid(int device) {
    static std::mutex mu;
    static std::vector<int> cap;
    std::lock_guard<std::mutex> lock(mu);
    if (device < 0) return 0;
    if (static_cast<size_t>(device) >= cap.size()) cap.resize(device + 1, -1);
    if (cap[device] < 0) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_layer_kernel<HT, FP8, D>, kLayerThreads, 0) !=
            hipSuccess)
            per_cu = 0;
        cap[device] = per_cu * device_cu_count(device);
    }
    return cap[device];
}

constexpr int kLayerMaxGrid = 1024;           // workspace bound on the grid (partial rows)
constexpr size_t kLayerBarBytes = 256;
constexpr size_t kLayerArrivalBytes = 64 << 10;

inline size_t al256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

struct LayerWs {
    size_t bar, arrivals, part_o, part_ml, q_proj, k_new, v_new, attn, total;
};

inline LayerWs layer_ws(int B, int Hq, int Hkv, int D, int max_len) {
    (void)max_len;
    // ragged plan: at most (ceil(target / Hkv) + B) * Hq partial rows
    const size_t rows = (static_cast<size_t>((kLayerMaxGrid + Hkv - 1) / Hkv) + B) * Hq;
    LayerWs w{};
    w.bar = 0;
    w.arrivals = kLayerBarBytes;
    w.part_o = w.arrivals + kLayerArrivalBytes;
    w.part_ml = w.part_o + al256(rows * D * 4);
    w.q_proj = w.part_ml + al256(rows * 2 * 4);
    w.k_new = w.q_proj + al256(static_cast<size_t>(B) * Hq * 2 * D * 2);
    w.v_new = w.k_new + al256(static_cast<size_t>(B) * Hkv * D * 2);
    w.attn = w.v_new + al256(static_cast<size_t>(B) * Hkv * D * 2);
    w.total = w.attn + al256(static_cast<size_t>(B) * Hq * D * 2);
    return w;
}

static bool plain_launch() {
    const char* v = getenv("SUPERSONIC_LAYER_LAUNCH");
    return v && std::strcmp(v, "plain") == 0;
}

template <typename HT, bool FP8, int D>
static int launch_layer(int device, hipStream_t st, LayerParams& P) {
    const int grid = std::min(layer_grid<HT, FP8, D>(device), kLayerMaxGrid);
    if (grid <= 0) return SUPERSONIC_ERR_LAUNCH;
    // one workgroup per item: every (sequence, kv head) needs one
    if (P.dec.B * P.dec.Hkv > grid) return SUPERSONIC_ERR_RANGE;
    P.dec.target = grid;
    P.dec.strict = 1;
    P.hint = 0;
    if (P.dec.B == 1 && P.layer_len > 0) {
        // the device plan for one sequence of the expected length
        const int64_t l = P.layer_len, Hkv = P.dec.Hkv;
        int64_t c = (l * Hkv + grid - 1) / grid;
        c = std::max((c + 15) / 16 * 16, static_cast<int64_t>(P.dec.min_chunk));
        for (int pass = 0; pass < 4; ++pass) {
            const int64_t items = std::max<int64_t>(1, (l + c - 1) / c) * Hkv;
            if (items <= grid) break;
            c = (c * items + grid - 1) / grid;
            c = (c + 15) / 16 * 16;
        }
        const int64_t items = std::max<int64_t>(1, (l + c - 1) / c) * Hkv;
        if (2 * items <= grid) P.hint = static_cast<int>(items);
    }
    P.polls = wait_polls(kLayerSpin);
    P.dec.merge_polls = wait_polls(kMergePoll);
    // Cooperative launch: the runtime refuses a grid whose workgroups cannot
    // all be resident at once, which the barriers need (as the reference's
    // persistent kernel does, kernels/full_attention_bridge_4b.cpp:4918-4927, :4963).
    // SUPERSONIC_LAYER_LAUNCH=plain: an ordinary launch (no co-residency
    // guarantee; a barrier that gives up is reported by the error word).
    if (plain_launch()) {
        hipLaunchKernelGGL((decode_layer_kernel<HT, FP8, D>), dim3(grid), dim3(kLayerThreads), 0, st, P);
        return hipGetLastError() == hipSuccess ? 0 : SUPERSONIC_ERR_LAUNCH;
    }
    void* args[] = {&P};
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&decode_layer_kernel<HT, FP8, D>),
                                                    dim3(grid), dim3(kLayerThreads), args, 0, st);
    if (e == hipErrorCooperativeLaunchTooLarge) return SUPERSONIC_ERR_COOPERATIVE;
    return e == hipSuccess ? 0 : SUPERSONIC_ERR_LAUNCH;
}

// Whether `device` runs cooperative launches (cached per device).
static bool cooperative_ok(int device) {
    static std::mutex mu;
    static std::vector<int> ok;
    std::lock_guard<std::mutex> lock(mu);
    if (device < 0) return false;
    if (static_cast<size_t>(device) >= ok.size()) ok.resize(device + 1, -1);
    if (ok[device] < 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeCooperativeLaunch, device) != hipSuccess) v = 0;
        ok[device] = v != 0;
    }
    return ok[device] != 0;
}

hipError_t take_wait_error_layer(unsigned* bits) { return take_wait_error(bits); }

}  // namespace ssa

using namespace ssa;

extern "C" size_t supersonic_attn_gfx950_decode_layer_workspace_size(size_t batch, size_t hidden_dim, size_t q_heads,
                                                                     size_t kv_heads, size_t head_dim,
                                                                     size_t max_kv_len) {
    (void)hidden_dim;
    if (batch == 0 || batch > 64 || kv_heads == 0 || q_heads > 4096 || head_dim > 512 || max_kv_len > 0x7FFFFFFF)
        return 0;
    return layer_ws(static_cast<int>(batch), static_cast<int>(q_heads), static_cast<int>(kv_heads),
                    static_cast<int>(head_dim), static_cast<int>(max_kv_len)).total;
}

extern "C" int supersonic_attn_gfx950_decode_layer(
    size_t device_ordinal, void* stream, int hidden_dtype, int kv_dtype, size_t batch, size_t hidden_dim,
    size_t q_heads, size_t kv_heads, size_t head_dim, size_t rotary_dim, size_t max_kv_len, float eps, float qk_eps,
    float scale, void* hidden, const void* input_norm_w, const void* q_proj_w, const void* k_proj_w,
    const void* v_proj_w, const void* q_norm_w, const void* k_norm_w, const void* o_proj_w, const void* cos_table,
    const void* sin_table, const int32_t* positions, const supersonic_kv_cache* cache, void* workspace,
    size_t workspace_bytes) {
    if (hidden_dtype != SUPERSONIC_DTYPE_BF16 && hidden_dtype != SUPERSONIC_DTYPE_F32) return SUPERSONIC_ERR_DTYPE;
    if (kv_dtype != SUPERSONIC_KV_BF16 && kv_dtype != SUPERSONIC_KV_FP8_E4M3) return SUPERSONIC_ERR_DTYPE;
    if (head_dim != 128 && head_dim != 256) return SUPERSONIC_ERR_HEAD_DIM;
    if (kv_heads == 0 || q_heads % kv_heads != 0 || q_heads / kv_heads > 4) return SUPERSONIC_ERR_HEADS;
    if (rotary_dim % 2 != 0 || rotary_dim > head_dim) return SUPERSONIC_ERR_ROTARY;
    if (batch == 0) return 0;
    const size_t B = batch, Hq = q_heads, Hkv = kv_heads, D = head_dim, hid = hidden_dim;
    const size_t nq = Hq * 2 * D, nkv = Hkv * D, adim = Hq * D;
    // both projections take the LDS-staged weight stream: rows * width <= 32768 elements
    if (B > 16 || hid == 0 || hid % 16 != 0 || B * hid > static_cast<size_t>(kXsMax) ||
        B * adim > static_cast<size_t>(kXsMax) || max_kv_len == 0 || max_kv_len > 0x7FFFFFFF ||
        B * Hkv > kLayerArrivalBytes / 4)
        return SUPERSONIC_ERR_RANGE;
    if (!hidden || !input_norm_w || !q_proj_w || !k_proj_w || !v_proj_w || !q_norm_w || !k_norm_w || !o_proj_w ||
        !positions || !workspace)
        return SUPERSONIC_ERR_NULL;
    if (rotary_dim > 0 && (!cos_table || !sin_table)) return SUPERSONIC_ERR_NULL;
    const uintptr_t al = reinterpret_cast<uintptr_t>(hidden) | reinterpret_cast<uintptr_t>(input_norm_w) |
                         reinterpret_cast<uintptr_t>(q_proj_w) | reinterpret_cast<uintptr_t>(k_proj_w) |
                         reinterpret_cast<uintptr_t>(v_proj_w) | reinterpret_cast<uintptr_t>(o_proj_w);
    if (al & 15) return SUPERSONIC_ERR_RANGE;
    const bool fp8 = kv_dtype == SUPERSONIC_KV_FP8_E4M3;
    const LayerWs L = layer_ws(static_cast<int>(B), static_cast<int>(Hq), static_cast<int>(Hkv), static_cast<int>(D),
                               static_cast<int>(max_kv_len));
    if (workspace_bytes < L.total) return SUPERSONIC_ERR_WORKSPACE;
    LayerParams P{};
    if (int rc = make_view(cache, fp8, &P.dec.kv)) return rc;
    ScopedDevice scoped(static_cast<int>(device_ordinal));
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    uint16_t* q_proj = reinterpret_cast<uint16_t*>(ws + L.q_proj);
    uint16_t* k_new = reinterpret_cast<uint16_t*>(ws + L.k_new);
    uint16_t* v_new = reinterpret_cast<uint16_t*>(ws + L.v_new);
    uint16_t* attn = reinterpret_cast<uint16_t*>(ws + L.attn);
    P.bar = reinterpret_cast<unsigned*>(ws + L.bar);
    P.layer_len = static_cast<int>(max_kv_len);
    // phase 1
    SkinnyLdsParams& q = P.qkv;
    q.xn = hidden;
    q.norm_w = static_cast<const uint16_t*>(input_norm_w);
    q.norm_eps = eps;
    q.w[0] = static_cast<const uint16_t*>(q_proj_w);
    q.w[1] = static_cast<const uint16_t*>(k_proj_w);
    q.w[2] = static_cast<const uint16_t*>(v_proj_w);
    q.out[0] = q_proj;
    q.out[1] = k_new;
    q.out[2] = v_new;
    q.n_seg[0] = static_cast<int>(nq);
    q.n_seg[1] = q.n_seg[2] = static_cast<int>(nkv);
    q.cb_end[0] = static_cast<int>(nq / kSkinnyCols);
    q.cb_end[1] = q.cb_end[0] + static_cast<int>(nkv / kSkinnyCols);
    q.cb_end[2] = q.cb_end[1] + static_cast<int>(nkv / kSkinnyCols);
    q.m = static_cast<int>(B);
    q.k = static_cast<int>(hid);
    // phase 2: the fused decode step's parameters (supersonic_attn_gfx950_decode)
    DecodeParams& p = P.dec;
    p.q = q_proj;
    p.q_bstride = static_cast<int64_t>(nq);
    p.q_hstride = 2 * static_cast<int64_t>(D);
    p.lens = positions;
    p.len_plus = 1;
    p.Hq = static_cast<int>(Hq);
    p.Hkv = static_cast<int>(Hkv);
    p.G = static_cast<int>(Hq / Hkv);
    p.ragged = 1;
    p.B = static_cast<int>(B);
    p.min_chunk = std::max(64, []() {
        const char* v = getenv("SUPERSONIC_DECODE_MIN_CHUNK");
        return (v && *v) ? atoi(v) : 128;
    }());
    p.det = []() {
        const char* v = getenv("SUPERSONIC_DECODE_DETERMINISTIC");
        return (v && *v) ? (atoi(v) != 0) : 0;
    }();
    p.scale_log2 = scale * kLog2e;
    p.fused = 1;
    p.k_new = k_new;
    p.v_new = v_new;
    p.q_norm_w = static_cast<const uint16_t*>(q_norm_w);
    p.k_norm_w = static_cast<const uint16_t*>(k_norm_w);
    p.cos_t = static_cast<const uint16_t*>(cos_table);
    p.sin_t = static_cast<const uint16_t*>(sin_table);
    p.half_rot = static_cast<int>(rotary_dim / 2);
    p.eps = qk_eps;
    p.part_o = reinterpret_cast<float*>(ws + L.part_o);
    p.part_ml = reinterpret_cast<float*>(ws + L.part_ml);
    p.arrivals = reinterpret_cast<unsigned*>(ws + L.arrivals);
    p.arr_stride = arrival_stride(static_cast<long long>(B) * Hkv, static_cast<long long>(kLayerArrivalBytes / 4));
    p.gate = q_proj + D;
    p.g_bstride = static_cast<int64_t>(nq);
    p.g_hstride = 2 * static_cast<int64_t>(D);
    p.out = attn;
    // phase 3
    SkinnyLdsParams& o = P.op;
    o.x = attn;
    o.w[0] = o.w[1] = o.w[2] = static_cast<const uint16_t*>(o_proj_w);
    o.out[0] = o.out[1] = o.out[2] = hidden;
    o.res = hidden;
    o.n_seg[0] = o.n_seg[1] = o.n_seg[2] = static_cast<int>(hid);
    o.cb_end[0] = o.cb_end[1] = o.cb_end[2] = static_cast<int>(hid / kSkinnyCols);
    o.m = static_cast<int>(B);
    o.k = static_cast<int>(adim);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int dev = static_cast<int>(device_ordinal);
    if (!plain_launch() && !cooperative_ok(dev)) return SUPERSONIC_ERR_COOPERATIVE;
    const ProfileEvents ev = take_profile_events();
    if (ev.before) (void)hipEventRecord(ev.before, st);
    int rc;
    const bool f32 = hidden_dtype == SUPERSONIC_DTYPE_F32;
    if (D == 256) {
        if (f32) rc = fp8 ? launch_layer<float, true, 256>(dev, st, P) : launch_layer<float, false, 256>(dev, st, P);
        else rc = fp8 ? launch_layer<bf16_t, true, 256>(dev, st, P) : launch_layer<bf16_t, false, 256>(dev, st, P);
    } else {
        if (f32) rc = fp8 ? launch_layer<float, true, 128>(dev, st, P) : launch_layer<float, false, 128>(dev, st, P);
        else rc = fp8 ? launch_layer<bf16_t, true, 128>(dev, st, P) : launch_layer<bf16_t, false, 128>(dev, st, P);
    }
    if (rc) return rc;
    if (ev.after) (void)hipEventRecord(ev.after, st);
    return 0;
}
