// Output projection after the gated attention, with the residual add.
//
//   decode:  hidden[r] = bf16(hidden[r] + bf16(attn[r] . W_o^T))
//            (megakernel step G, kernels/full_attention_4b.hip:5481-5577, bf16
//            weight branch :5551-5574)
//   prefill: out = bf16(lhs . rhs^T) then hidden = bf16(hidden + out)
//            (matmul_proj + residual_add, crates/runner/src/prefill_engine.rs:2308-2334,
//            kernels full_attention_4b.hip:2513-2575 and prefill_helpers.hip:59-68)
//
// Few rows (decode batches, <= 12 by default) make a weight stream: W [n, k]
// bf16 is read once from HBM and the kernel is HBM-bound.  A workgroup owns 16
// output columns (16 rows of W); its 8 waves split k and load W straight into
// the B-operand layout of v_mfma_f32_16x16x32_bf16 (lane l: W row n0 + l%16, 8
// consecutive k at 8*(l/16)), with the activation rows as the A operand (16
// rows per MFMA, zero past m).  8 k-steps (8 x 16 B per lane) are in flight per
// load batch, which keeps a wave under 128 VGPRs so two workgroups share a CU.
// The waves' partial sums meet in LDS; the epilogue rounds to bf16 and adds the
// residual with the reference's second rounding.  When there are fewer column
// blocks than CUs, k is also split over workgroups: each stores its fp32 partial
// block with device-coherent stores and the last to arrive adds the slices in
// slice order (deterministic) and runs the epilogue.
//
// When the rows fit (m * k <= 32768 elements) and there are enough column
// blocks that k is not split, skinny_lds_kernel runs instead: the workgroup
// stages its activation rows in LDS once (a coalesced copy issued ahead of the
// first W batch) and reads the A operand from there, rather than every wave
// loading its k range of the rows with the lanes past m masked off (measured:
// o_proj 13.6 -> 12.6 us, Q/K/V 29.1 -> 26.6 us at the config-2 decode shape).
//
// More rows are plain GEMMs and go to the hand-written MFMA GEMM (gemm.hip).
// SUPERSONIC_PROJ_GEMM=hipblaslt sends them to hipBLASLt instead, for
// comparison; the library then opens libhipblaslt at run time (dlopen), so the
// product library does not link it and integrators do not inherit it.
#include <dlfcn.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <map>
#include <mutex>
#include <tuple>

#include "common.hpp"
#include "kv_view.hpp"
#include "skinny.hpp"
#include "gemm.hpp"
#include "supersonic_attn.h"

namespace ssa {

// Up to three weight matrices side by side in one column space (the Q/K/V
// projections); segment i holds column blocks [cb_end[i-1], cb_end[i]).
struct SkinnyParams {
    const uint16_t* x;    // [batch][m][k] bf16
    const uint16_t* w[3]; // [batch][n_i][k] bf16
    void* out[3];         // [batch][m][n_i] (OT)
    const void* res;      // residual [batch][m][n_0] (OT), may alias out[0] (one segment)
    int n_seg[3];
    int cb_end[3];
    float* part;          // split k: [batch * column blocks][ks_count][MB*16*64] partial sums
    unsigned* arrivals;   // split k: [batch * column blocks] counters, zero between calls
    int m, k;
    int ks_count, slice;  // k split over ks_count workgroups of `slice` 32-wide k-steps
    int64_t x_bs, w_bs, o_bs;  // batch strides in elements
};

template <typename OT, bool RES, bool ROPE = false>
__global__ __launch_bounds__(64 * kSkinnyWaves) __attribute__((amdgpu_waves_per_eu(4))) void skinny_lds_kernel(SkinnyLdsParams p, RopeEpi e) {
    __shared__ SkinnyLdsBase lds;  // no NORM staging here: two workgroups a CU
    skinny_lds_body<OT, RES, ROPE, false, bf16_t, false, false, SkinnyLdsBase, false, kSkinnyLdsSteps>(p, e, blockIdx.x, blockIdx.z, lds);
}

constexpr int kSkinnyCB = 1;                        // 16-column blocks per workgroup
constexpr int kSkinnyKP = kSkinnyWaves / kSkinnyCB;  // k parts per workgroup (one per wave group)
constexpr int kSkinnyMaxM = 64;                     // hard limit (4 row blocks)
constexpr int kSkinnyDefaultM = 12;                 // measured crossover with hipBLASLt
constexpr size_t kSkinnyArrivalBytes = 64 << 10;  // counters at a fixed offset, ahead of the partials


template <typename OT, bool RES>
__device__ __forceinline__ void skinny_store(const SkinnyParams& p, int seg, int b, int row, int col, float s) {
    const int n = pick3(p.n_seg, seg);
    if (row >= p.m || col >= n) return;
    float y = bf16_round(s);
    const int64_t o = b * p.o_bs + static_cast<int64_t>(row) * n + col;
    if constexpr (RES) y = bf16_round(load_f32<OT>(static_cast<const OT*>(p.res), o) + y);
    store_f32<OT>(static_cast<OT*>(pick3(p.out, seg)), o, y);
}

// Workgroup (column block cb, k slice ks, batch b): 64 W rows x `slice` k-steps.
// Wave w: columns cb*64 + 16*(w&3) .. +16, half (w>>2) of the slice.  The four
// waves of a half read the same activation addresses, so the activations cross
// L2 once per workgroup; splitting k over workgroups keeps that at
// m*k*2*(column blocks) bytes in all, not per 16 columns.
template <typename OT, bool RES, int MB>
__global__ __launch_bounds__(64 * kSkinnyWaves) void skinny_kernel(SkinnyParams p) {
    __shared__ float red[kSkinnyKP][kSkinnyCB][MB][256];
    __shared__ int last_s;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int cbw = wave % kSkinnyCB, kh = wave / kSkinnyCB;
    const int cb = blockIdx.x, ks = blockIdx.y, b = blockIdx.z;
    const int seg = cb < p.cb_end[0] ? 0 : (cb < p.cb_end[1] ? 1 : 2);
    const int cbs = cb - (seg == 0 ? 0 : (seg == 1 ? p.cb_end[0] : p.cb_end[1]));  // column block inside the segment
    const int n = pick3(p.n_seg, seg);
    const uint16_t* x = p.x + b * p.x_bs;
    const uint16_t* w = pick3(p.w, seg) + b * p.w_bs;
    const int T = (p.k + 31) / 32;
    const int sb0 = ks * p.slice;
    const int sb1 = min(sb0 + p.slice, T);
    const int half = (max(sb1 - sb0, 0) + kSkinnyKP - 1) / kSkinnyKP;
    const int s0 = sb0 + kh * half;
    const int s1 = min(s0 + half, sb1);
    const int col = lane & 15;
    const int kq = (lane >> 4) * 8;
    const int n_w = cbs * kSkinnyCols + cbw * 16 + col;
    const bool nvalid = n_w < n;
    const uint16_t* wrow = w + static_cast<int64_t>(min(n_w, n - 1)) * p.k + kq;
    const uint16_t* xrow[MB];
    bool mvalid[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int r = mb * 16 + col;
        mvalid[mb] = r < p.m;
        xrow[mb] = x + static_cast<int64_t>(min(r, p.m - 1)) * p.k + kq;
    }
    f32x4_v acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4_v{0.f, 0.f, 0.f, 0.f};
    const u32x4_v zero = {0u, 0u, 0u, 0u};
    for (int sb = s0; sb < s1; sb += kSkinnySteps) {
        u32x4_v wv[kSkinnySteps];
#pragma unroll
        for (int j = 0; j < kSkinnySteps; ++j) {
            const int s = sb + j;
            wv[j] = (s < s1 && nvalid && s * 32 + kq < p.k) ? ld16(wrow + s * 32) : zero;
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            u32x4_v xv[kSkinnySteps];
#pragma unroll
            for (int j = 0; j < kSkinnySteps; ++j) {
                const int s = sb + j;
                xv[j] = (s < s1 && mvalid[mb] && s * 32 + kq < p.k) ? ld16(xrow[mb] + s * 32) : zero;
            }
#pragma unroll
            for (int j = 0; j < kSkinnySteps; ++j)
                acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xv[j]), as_bf16x8(wv[j]), acc[mb], 0, 0, 0);
        }
    }
    // accumulator layout: lane l, element i -> row 4*(l/16)+i, column l%16
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[kh][cbw][mb][(4 * (lane >> 4) + i) * 16 + col] = acc[mb][i];
    __syncthreads();
    // element e of the workgroup's block: column block c = e / (MB*256), row block, 16x16 entry
    constexpr int NE = kSkinnyCB * MB * 256;
    const bool split = p.ks_count > 1;
    const int64_t blk = static_cast<int64_t>(b) * gridDim.x + cb;
    for (int e = tid; e < NE; e += 64 * kSkinnyWaves) {
        const int c = e / (MB * 256), mb = (e / 256) % MB, r = e & 255;
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < kSkinnyKP; ++q) sum += red[q][c][mb][r];
        if (split)
            store_agent(p.part + (blk * p.ks_count + ks) * NE + e, sum);
        else
            skinny_store<OT, RES>(p, seg, b, mb * 16 + (r >> 4), cbs * kSkinnyCols + c * 16 + (r & 15), sum);
    }
    if (!split) return;
    // The last workgroup of the column block to arrive adds the k slices in
    // slice order (the result does not depend on arrival order) and stores.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores are complete
    __syncthreads();
    if (tid == 0) last_s = atomicAdd(&p.arrivals[blk], 1u) == static_cast<unsigned>(p.ks_count - 1);
    __syncthreads();
    if (!last_s) return;
    const float* base = p.part + blk * p.ks_count * NE;
    for (int e = tid; e < NE; e += 64 * kSkinnyWaves) {
        const int c = e / (MB * 256), mb = (e / 256) % MB, r = e & 255;
        float sum = 0.f;
        for (int q = 0; q < p.ks_count; ++q) sum += load_agent(base + q * NE + e);
        skinny_store<OT, RES>(p, seg, b, mb * 16 + (r >> 4), cbs * kSkinnyCols + c * 16 + (r & 15), sum);
    }
    if (tid == 0) p.arrivals[blk] = 0u;  // every slice has arrived: ready for the next call
}

// Input RMSNorm ahead of the Q/K/V projections (decode megakernel
// full_attention_4b.hip:4942-4967; prefill rms_norm_rows_model):
// normed = bf16(x * rsqrt(mean(x^2) + eps) * (1 + w)): one 256-thread
// workgroup per row, 8 elements (16 or 32 bytes) per thread and chunk, every
// chunk's load issued before the reduction (k <= 8192 in one pass of
// registers; longer rows re-read their chunks from cache).
template <typename XT>
__global__ __launch_bounds__(256) void input_norm_kernel(int rows, int k, float eps, const XT* x, const uint16_t* w,
                                                         uint16_t* out) {
    __shared__ float part[4];
    constexpr int CH = 4;  // chunks of 8 held per thread
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const XT* xr = x + static_cast<int64_t>(row) * k;
    const int nch = k / 8;
    float v[CH][8];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int ch = tid + 256 * c;
        if (ch < nch) load8f<XT>(xr + 8 * ch, v[c]);
        else
#pragma unroll
            for (int e = 0; e < 8; ++e) v[c][e] = 0.f;
    }
    for (int ch = tid + 256 * CH; ch < nch; ch += 256) {
        float f[8];
        load8f<XT>(xr + 8 * ch, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    }
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += v[c][e] * v[c][e];
    ss = wave_sum(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    const float inv = rsqrtf((part[0] + part[1] + part[2] + part[3]) / static_cast<float>(k) + eps);
    uint16_t* orow = out + static_cast<int64_t>(row) * k;
    for (int ch = tid; ch < nch; ch += 256) {
        const int c = (ch - tid) / 256;
        float f[8], g[8];
        if (c < CH) {
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = v[c < CH ? c : 0][e];
        } else {
            load8f<XT>(xr + 8 * ch, f);
        }
        unpack8<bf16_t>(ld16(w + 8 * ch), g);
        u32x4_v o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = f32_to_bf16_bits(f[2 * e] * inv * (g[2 * e] + 1.0f)) |
                   (f32_to_bf16_bits(f[2 * e + 1] * inv * (g[2 * e + 1] + 1.0f)) << 16);
        st16(orow + 8 * ch, o);
    }
}

// ---------------------------------------------------------------------------
// The same weight stream with the activation rows staged in LDS once per
// workgroup (<= 16 rows, m * k <= kXsMax): a coalesced copy instead of every
// wave loading its k range with the rows past m masked off.  Program order
// keeps the activation loads ahead of the first W batch, so waiting for them
// (vmcnt drains in issue order) never waits for W; the LDS hand-offs wait for
// lgkmcnt only.  (Applying the input RMSNorm while staging, in every
// workgroup, measured slower than the separate norm kernel: 30.9 vs 29.2 us
// for the config-2 Q/K/V step.)
// ---------------------------------------------------------------------------
// Unfused path of the same epilogue (rows past the LDS-staged kernel, head
// dims other than 128/256): one wave per (row, head) over the plain
// projection outputs.  Blocks 0 .. Hq-1 of a row: q head (q_proj [m, Hq*2D]
// -> q_out, gate_out); blocks Hq .. Hq+Hkv-1: kv head (k_in -> k_out
// normalised + rotated, v_in -> v_out, cache append).
__global__ __launch_bounds__(64) void qk_norm_rope_kernel(const uint16_t* q_proj, const uint16_t* k_in,
                                                          const uint16_t* v_in, RopeEpi e) {
    __shared__ float rowbuf[512];
    const int row = blockIdx.x, hh = blockIdx.y, lane = threadIdx.x;
    const int D = e.D, pos = e.pos[row];
    const bool qh = hh < e.Hq;
    const int h = qh ? hh : hh - e.Hq;
    const uint16_t* src = qh ? q_proj + (static_cast<int64_t>(row) * e.Hq + h) * 2 * D
                             : k_in + (static_cast<int64_t>(row) * e.Hkv + h) * D;
    uint16_t* dst = qh ? e.q_out + (static_cast<int64_t>(row) * e.Hq + h) * D
                       : e.k_out + (static_cast<int64_t>(row) * e.Hkv + h) * D;
    constexpr int EPL = 8;  // D <= 512: lane holds dims lane * 8 .. (lanes past D/8 idle)
    const int active = D / 8;
    float x[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) x[j] = lane < active ? bf16_bits_to_f32(src[lane * EPL + j]) : 0.f;
    // norm_rope_row over D dims with lane-contiguous groups of 8
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) ss += x[j] * x[j];
    ss = wave_sum(ss);
    const float inv = rsqrtf(ss / static_cast<float>(D) + e.eps);
    const uint16_t* w = qh ? e.q_norm_w : e.k_norm_w;
#pragma unroll
    for (int j = 0; j < EPL; ++j)
        if (lane < active) x[j] = bf16_round(x[j] * inv * (bf16_bits_to_f32(w[lane * EPL + j]) + 1.0f));
    const int hr = e.half_rot;
    if (hr > 0) {
#pragma unroll
        for (int j = 0; j < EPL; ++j)
            if (lane < active) rowbuf[lane * EPL + j] = x[j];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int d = lane * EPL + j;
            if (lane < active && d < 2 * hr) {
                const int ti = d < hr ? d : d - hr;
                const float c = bf16_bits_to_f32(e.cos_t[static_cast<int64_t>(pos) * hr + ti]);
                const float sn = bf16_bits_to_f32(e.sin_t[static_cast<int64_t>(pos) * hr + ti]);
                const float other = rowbuf[d < hr ? d + hr : d - hr];
                x[j] = d < hr ? bf16_round(x[j] * c - other * sn) : bf16_round(other * sn + x[j] * c);
            }
        }
    }
    if (lane >= active) return;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const int d = lane * EPL + j;
        dst[d] = static_cast<uint16_t>(f32_to_bf16_bits(x[j]));
        if (qh) {
            e.gate_out[(static_cast<int64_t>(row) * e.Hq + h) * D + d] = src[D + d];
        } else {
            const uint16_t vv = v_in[(static_cast<int64_t>(row) * e.Hkv + h) * D + d];
            e.v_out[(static_cast<int64_t>(row) * e.Hkv + h) * D + d] = vv;
            if (e.kv.k) {
                const int64_t o = e.kv.row(row, h, pos, D) + d;
                reinterpret_cast<uint16_t*>(e.kv.k)[o] = static_cast<uint16_t>(f32_to_bf16_bits(x[j]));
                reinterpret_cast<uint16_t*>(e.kv.v)[o] = vv;
            }
        }
    }
}

// Zero fill (a kernel rather than hipMemsetAsync, so the call can be captured
// into a HIP graph without a memset node).
__global__ void fill_u16_kernel(size_t total, uint16_t* y) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        y[i] = 0;
}

// hidden = bf16(hidden + y) over `total` elements (y bf16).
template <typename OT>
__global__ void residual_add_kernel(size_t total, const uint16_t* y, OT* hidden) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        store_f32<OT>(hidden, i, bf16_round(load_f32<OT>(hidden, i) + bf16_bits_to_f32(y[i])));
}

// out = T(float(lhs) + float(rhs)): pfx_element_add_kernel (prefill_helpers.hip:59-68).
template <typename T>
__global__ void element_add_kernel(size_t total, const T* lhs, const T* rhs, T* out) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        store_f32<T>(out, i, load_f32<T>(lhs, i) + load_f32<T>(rhs, i));
}

// One weight matrix as the whole column space.
inline void one_segment(SkinnyParams& p, const void* w, void* out, int n) {
    p.w[0] = p.w[1] = p.w[2] = static_cast<const uint16_t*>(w);
    p.out[0] = p.out[1] = p.out[2] = out;
    p.n_seg[0] = p.n_seg[1] = p.n_seg[2] = n;
    p.cb_end[0] = p.cb_end[1] = p.cb_end[2] = (n + kSkinnyCols - 1) / kSkinnyCols;
}

inline unsigned stride_blocks(size_t n) {
    const size_t b = (n + 255) / 256;
    return static_cast<unsigned>(b < 8192 ? (b ? b : 1) : 8192);
}

// Largest row count the streaming kernel takes (SUPERSONIC_PROJ_SKINNY_MAX_M,
// default 12, at most 64, read per call); more rows go to hipBLASLt.
int skinny_max_m() {
    const char* e = getenv("SUPERSONIC_PROJ_SKINNY_MAX_M");
    const int x = e ? atoi(e) : kSkinnyDefaultM;
    return x < 0 ? 0 : (x > kSkinnyMaxM ? kSkinnyMaxM : x);
}

bool skinny_fits(int m, int k, const void* x, const void* w) {
    return m >= 1 && m <= skinny_max_m() && k % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(w) & 15) == 0;
}

// Plans the k split (enough workgroups to cover the CUs, at least 8 k-steps
// per wave) and launches.  Returns a SUPERSONIC status (0 = ok).
// The staged-activation kernel takes <= 16 rows with m * k <= kXsMax when the
// plain kernel would not split k (enough column blocks to fill the CUs);
// SUPERSONIC_PROJ_LDS=0 (read per call) turns it off.
bool lds_path(int dev, int m, int k, int batch, int ncb) {
    const char* e = getenv("SUPERSONIC_PROJ_LDS");
    if (e && atoi(e) == 0) return false;
    const int cus = device_cu_count(dev) > 0 ? device_cu_count(dev) : 256;
    return m >= 1 && m <= 16 && static_cast<int64_t>(m) * k <= kXsMax && k % 8 == 0 &&
           static_cast<int64_t>(ncb) * batch * 2 > cus;
}

SkinnyLdsParams lds_params(const SkinnyParams& q) {
    SkinnyLdsParams p{};
    p.x = q.x;
    for (int i = 0; i < 3; ++i) {
        p.w[i] = q.w[i];
        p.out[i] = q.out[i];
        p.n_seg[i] = q.n_seg[i];
        p.cb_end[i] = q.cb_end[i];
    }
    p.res = q.res;
    p.m = q.m;
    p.k = q.k;
    p.x_bs = q.x_bs;
    p.w_bs = q.w_bs;
    p.o_bs = q.o_bs;
    return p;
}

template <typename OT, bool RES>
int launch_skinny_lds(hipStream_t st, int batch, const SkinnyLdsParams& p) {
    const dim3 grid(p.cb_end[2], 1, batch), blk(64 * kSkinnyWaves);
    hipLaunchKernelGGL((skinny_lds_kernel<OT, RES, false>), grid, blk, 0, st, p, RopeEpi{});
    return hipGetLastError() == hipSuccess ? 0 : SUPERSONIC_ERR_LAUNCH;
}

// k split of the streaming kernel: enough workgroups to cover the CUs, at
// least 8 k-steps per wave, and a counter per column block.
int skinny_k_split(int cus, int64_t wgs, int k) {
    const int T = (k + 31) / 32;
    int ks = 1;
    while (wgs * ks * 2 <= cus && T / (ks * 2) >= kSkinnyKP * 8) ks *= 2;
    if (wgs > static_cast<int64_t>(kSkinnyArrivalBytes / 4)) ks = 1;
    return ks;
}

// Bytes of [arrival counters | k-split partials] the streaming kernel needs for
// this shape on any device (the split is bounded by the k-step count alone).
size_t skinny_ws_bytes(int m, int k, int64_t wgs) {
    const int T = (k + 31) / 32;
    int ks = 1;
    while (T / (ks * 2) >= kSkinnyKP * 8) ks *= 2;
    if (ks == 1 || wgs > static_cast<int64_t>(kSkinnyArrivalBytes / 4)) return 0;
    const int MB = (m + 15) / 16;
    return kSkinnyArrivalBytes + static_cast<size_t>(wgs) * ks * kSkinnyCB * MB * 256 * sizeof(float);
}

// ws: the skinny_ws_bytes() region (arrival counters zero between calls), or
// NULL for the library's own.
template <typename OT, bool RES>
int launch_skinny(int dev, hipStream_t st, int batch, SkinnyParams p, uint8_t* ws = nullptr, size_t ws_bytes = 0) {
    const int ncb = p.cb_end[2];
    const int T = (p.k + 31) / 32;
    const int MB = (p.m + 15) / 16;
    const int64_t wgs = static_cast<int64_t>(ncb) * batch;
    const int cus = device_cu_count(dev) > 0 ? device_cu_count(dev) : 256;
    const int ks = skinny_k_split(cus, wgs, p.k);
    p.ks_count = ks;
    p.slice = (T + ks - 1) / ks;
    if (ks > 1) {
        const size_t need = kSkinnyArrivalBytes + static_cast<size_t>(wgs) * ks * kSkinnyCB * MB * 256 * sizeof(float);
        if (!ws) ws = static_cast<uint8_t*>(device_workspace(dev, need, kWorkspaceSkinny));
        else if (ws_bytes < need) return SUPERSONIC_ERR_WORKSPACE;
        if (!ws) return SUPERSONIC_ERR_WORKSPACE;
        p.arrivals = reinterpret_cast<unsigned*>(ws);
        p.part = reinterpret_cast<float*>(ws + kSkinnyArrivalBytes);
    }
    const dim3 grid(ncb, ks, batch), blk(64 * kSkinnyWaves);
    switch (MB) {
    case 1: hipLaunchKernelGGL((skinny_kernel<OT, RES, 1>), grid, blk, 0, st, p); break;
    case 2: hipLaunchKernelGGL((skinny_kernel<OT, RES, 2>), grid, blk, 0, st, p); break;
    case 3: hipLaunchKernelGGL((skinny_kernel<OT, RES, 3>), grid, blk, 0, st, p); break;
    default: hipLaunchKernelGGL((skinny_kernel<OT, RES, 4>), grid, blk, 0, st, p); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : SUPERSONIC_ERR_LAUNCH;
}

// ---------------------------------------------------------------------------
// hipBLASLt for the GEMM-sized calls: out[b] (m x n, row-major) = lhs[b] . rhs[b]^T.
// In hipBLASLt's column-major terms that is D (n x m, ld n) = op_T(A: k x n, ld k) . B (k x m, ld k).
// ---------------------------------------------------------------------------
namespace {
// hipBLASLt entry points resolved with dlsym on first use (types from its header only).
struct LtApi {
    bool tried = false, ok = false;
#define SSA_LT_FN(name) decltype(&::name) name = nullptr;
    SSA_LT_FN(hipblasLtCreate)
    SSA_LT_FN(hipblasLtMatrixLayoutCreate)
    SSA_LT_FN(hipblasLtMatrixLayoutSetAttribute)
    SSA_LT_FN(hipblasLtMatmulDescCreate)
    SSA_LT_FN(hipblasLtMatmulDescSetAttribute)
    SSA_LT_FN(hipblasLtMatmulPreferenceCreate)
    SSA_LT_FN(hipblasLtMatmulPreferenceSetAttribute)
    SSA_LT_FN(hipblasLtMatmulPreferenceDestroy)
    SSA_LT_FN(hipblasLtMatmulAlgoGetHeuristic)
    SSA_LT_FN(hipblasLtMatmul)
#undef SSA_LT_FN
    bool load() {
        if (tried) return ok;
        tried = true;
        void* h = dlopen("libhipblaslt.so.1", RTLD_NOW | RTLD_LOCAL);
        if (!h) h = dlopen("/opt/rocm/lib/libhipblaslt.so.1", RTLD_NOW | RTLD_LOCAL);
        if (!h) return false;
        bool all = true;
#define SSA_LT_SYM(name) \
    name = reinterpret_cast<decltype(name)>(dlsym(h, #name)); \
    all = all && name != nullptr;
        SSA_LT_SYM(hipblasLtCreate)
        SSA_LT_SYM(hipblasLtMatrixLayoutCreate)
        SSA_LT_SYM(hipblasLtMatrixLayoutSetAttribute)
        SSA_LT_SYM(hipblasLtMatmulDescCreate)
        SSA_LT_SYM(hipblasLtMatmulDescSetAttribute)
        SSA_LT_SYM(hipblasLtMatmulPreferenceCreate)
        SSA_LT_SYM(hipblasLtMatmulPreferenceSetAttribute)
        SSA_LT_SYM(hipblasLtMatmulPreferenceDestroy)
        SSA_LT_SYM(hipblasLtMatmulAlgoGetHeuristic)
        SSA_LT_SYM(hipblasLtMatmul)
#undef SSA_LT_SYM
        ok = all;
        return ok;
    }
};
LtApi g_lt_api;  // guarded by g_lt_mutex

struct LtPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};
struct LtDevice {
    hipblasLtHandle_t handle = nullptr;
    std::map<std::tuple<int, int, int, int>, LtPlan> plans;
};
std::mutex g_lt_mutex;
std::map<int, LtDevice> g_lt;
constexpr size_t kLtWorkspace = 32u << 20;
// SUPERSONIC_PROJ_GEMM=hipblaslt routes the GEMM-sized projections to
// hipBLASLt instead of the hand-written kernel (for comparison).
bool use_hipblaslt() {
    const char* v = getenv("SUPERSONIC_PROJ_GEMM");
    return v && std::strcmp(v, "hipblaslt") == 0;
}
size_t lt_ws_bytes() { return use_hipblaslt() ? kLtWorkspace : 0; }
// The three projections (or one) as one hand-written GEMM launch.  ws: the
// caller's region for the tail split (gemm_ws_bytes()), or null for the
// library's own.
int gemm_segments(int dev, hipStream_t st, int m, int k, const void* a, int nseg, const void* const* w,
                  void* const* out, const int* n, int epilogue, uint8_t* ws, size_t ws_bytes) {
    GemmArgs g;
    g.m = m;
    g.k = k;
    g.a = static_cast<const uint16_t*>(a);
    g.lda = k;
    g.nseg = nseg;
    for (int i = 0; i < nseg; ++i) {
        g.w[i] = static_cast<const uint16_t*>(w[i]);
        g.out[i] = out[i];
        g.n[i] = n[i];
    }
    g.epilogue = epilogue;
    const size_t need = gemm_ws_bytes(m, nseg, n);
    if (need > 0) {
        if (ws) {
            if (ws_bytes < need) return 1;
            g.ws = ws;
        } else {
            g.ws = device_workspace(dev, need, kWorkspaceGemm);  // zero-filled once; each call leaves the tail counts equal
        }
        g.ws_bytes = g.ws ? need : 0;
    }
    return gemm_bt(st, g);
}

bool make_layout(hipblasLtMatrixLayout_t* l, uint64_t rows, uint64_t cols, int64_t ld, int batch, int64_t stride) {
    if (g_lt_api.hipblasLtMatrixLayoutCreate(l, HIP_R_16BF, rows, cols, ld) != HIPBLAS_STATUS_SUCCESS) return false;
    if (batch > 1) {
        const int32_t bc = batch;
        if (g_lt_api.hipblasLtMatrixLayoutSetAttribute(*l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc, sizeof(bc)) !=
                HIPBLAS_STATUS_SUCCESS ||
            g_lt_api.hipblasLtMatrixLayoutSetAttribute(*l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &stride,
                                              sizeof(stride)) != HIPBLAS_STATUS_SUCCESS)
            return false;
    }
    return true;
}
}  // namespace

// 0 on success, 1 when hipBLASLt has no plan for the shape, 2 on a launch error.
// ws: kLtWorkspace bytes of caller memory, or NULL for the library's own.
int lt_gemm(int dev, hipStream_t st, int batch, int m, int n, int k, const void* lhs, const void* rhs, void* out,
            void* ws = nullptr) {
    std::lock_guard<std::mutex> lock(g_lt_mutex);
    if (!g_lt_api.load()) return 1;
    LtDevice& D = g_lt[dev];
    if (!D.handle && g_lt_api.hipblasLtCreate(&D.handle) != HIPBLAS_STATUS_SUCCESS) {
        D.handle = nullptr;
        return 1;
    }
    if (!ws) ws = device_workspace(dev, kLtWorkspace, kWorkspaceProjLt);
    if (!ws) return 2;
    const auto key = std::make_tuple(batch, m, n, k);
    auto it = D.plans.find(key);
    if (it == D.plans.end()) {
        LtPlan P;
        const hipblasOperation_t opA = HIPBLAS_OP_T, opB = HIPBLAS_OP_N;
        if (g_lt_api.hipblasLtMatmulDescCreate(&P.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS ||
            g_lt_api.hipblasLtMatmulDescSetAttribute(P.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opA, sizeof(opA)) !=
                HIPBLAS_STATUS_SUCCESS ||
            g_lt_api.hipblasLtMatmulDescSetAttribute(P.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opB, sizeof(opB)) !=
                HIPBLAS_STATUS_SUCCESS ||
            !make_layout(&P.a, k, n, k, batch, static_cast<int64_t>(n) * k) ||
            !make_layout(&P.b, k, m, k, batch, static_cast<int64_t>(m) * k) ||
            !make_layout(&P.d, n, m, n, batch, static_cast<int64_t>(m) * n))
            return 1;
        hipblasLtMatmulPreference_t pref;
        if (g_lt_api.hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return 1;
        const uint64_t wsb = kLtWorkspace;
        g_lt_api.hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb));
        hipblasLtMatmulHeuristicResult_t res[1];
        int found = 0;
        const hipblasStatus_t hs =
            g_lt_api.hipblasLtMatmulAlgoGetHeuristic(D.handle, P.desc, P.a, P.b, P.d, P.d, pref, 1, res, &found);
        g_lt_api.hipblasLtMatmulPreferenceDestroy(pref);
        if (hs != HIPBLAS_STATUS_SUCCESS || found < 1) return 1;
        P.algo = res[0].algo;
        it = D.plans.emplace(key, P).first;
    }
    const LtPlan& P = it->second;
    const float alpha = 1.f, beta = 0.f;
    if (g_lt_api.hipblasLtMatmul(D.handle, P.desc, &alpha, rhs, P.a, lhs, P.b, &beta, out, P.d, out, P.d, &P.algo, ws,
                        kLtWorkspace, st) != HIPBLAS_STATUS_SUCCESS)
        return 2;
    return 0;
}

}  // namespace ssa

using namespace ssa;

// Drop-in for kernels/full_attention_bridge_4b.cpp:3683-3704 (kernel
// full_attention_4b.hip:2513-2575), bound at crates/kernel-ffi/src/prefill_ffi.rs:782-792.
extern "C" int supersonic_qwen35_4b_hip_matmul_rhs_transposed_tiled(int dtype, size_t device_ordinal,
                                                                    size_t batch_elems, int m, int n, int k,
                                                                    const void* lhs, const void* rhs, void* out) {
    if (dtype != SUPERSONIC_DTYPE_BF16) return 272;
    const int dev = static_cast<int>(device_ordinal);
    ScopedDevice scoped(dev);
    if (batch_elems > 0 && m > 0 && n > 0) {
        const int batch = static_cast<int>(batch_elems);
        if (k <= 0 || skinny_fits(m, k, lhs, rhs)) {
            SkinnyParams p{};
            p.x = static_cast<const uint16_t*>(lhs);
            one_segment(p, rhs, out, n);
            p.m = m;
            p.k = k > 0 ? k : 0;
            p.x_bs = static_cast<int64_t>(m) * p.k;
            p.w_bs = static_cast<int64_t>(n) * p.k;
            p.o_bs = static_cast<int64_t>(m) * n;
            if (m > skinny_max_m()) {  // k == 0 with many rows: the product is zero
                if (hipMemsetAsync(out, 0, batch_elems * m * n * 2, nullptr) != hipSuccess) return 270;
            } else if (k > 0 && lds_path(dev, m, k, batch, p.cb_end[2])) {
                if (launch_skinny_lds<bf16_t, false>(nullptr, batch, lds_params(p)) != 0) return 270;
            } else if (launch_skinny<bf16_t, false>(dev, nullptr, batch, p) != 0) {
                return 270;  // the reference's launch-failure code covers a workspace failure too
            }
        } else if (use_hipblaslt()) {
            if (lt_gemm(dev, nullptr, batch, m, n, k, lhs, rhs, out) != 0) return 270;
        } else {
            GemmArgs g;
            g.batch = batch;
            g.m = m;
            g.k = k;
            g.a = static_cast<const uint16_t*>(lhs);
            g.lda = k;
            g.a_bs = static_cast<int64_t>(m) * k;
            g.w[0] = static_cast<const uint16_t*>(rhs);
            g.out[0] = out;
            g.n[0] = n;
            g.w_bs = static_cast<int64_t>(n) * k;
            g.o_bs = static_cast<int64_t>(m) * n;
            if (batch == 1) {
                g.ws_bytes = gemm_ws_bytes(m, 1, &n);
                if (g.ws_bytes > 0) g.ws = device_workspace(dev, g.ws_bytes, kWorkspaceGemm);
                if (!g.ws) g.ws_bytes = 0;
            }
            if (gemm_bt(nullptr, g) != 0) return 270;
        }
    }
    if (hipDeviceSynchronize() != hipSuccess) return 271;
    return 0;
}

// Drop-in for kernels/prefill_helpers_bridge.cpp:281-290, bound at prefill_ffi.rs:661-668.
extern "C" int supersonic_qwen35_hip_element_add(int dtype, size_t device_ordinal, size_t total_elems,
                                                 const void* lhs, const void* rhs, void* out) {
    if (dtype < 0 || dtype > 2) return 300;
    ScopedDevice scoped(static_cast<int>(device_ordinal));
    if (total_elems) {
        const dim3 grid(stride_blocks(total_elems)), blk(256);
        switch (dtype) {
        case 0:
            hipLaunchKernelGGL((element_add_kernel<f16_t>), grid, blk, 0, nullptr, total_elems,
                               static_cast<const f16_t*>(lhs), static_cast<const f16_t*>(rhs), static_cast<f16_t*>(out));
            break;
        case 1:
            hipLaunchKernelGGL((element_add_kernel<float>), grid, blk, 0, nullptr, total_elems,
                               static_cast<const float*>(lhs), static_cast<const float*>(rhs), static_cast<float*>(out));
            break;
        default:
            hipLaunchKernelGGL((element_add_kernel<bf16_t>), grid, blk, 0, nullptr, total_elems,
                               static_cast<const bf16_t*>(lhs), static_cast<const bf16_t*>(rhs),
                               static_cast<bf16_t*>(out));
            break;
        }
        if (hipGetLastError() != hipSuccess) return 301;
    }
    if (hipDeviceSynchronize() != hipSuccess) return 302;
    return 0;
}

namespace ssa {
inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Workspace of the o_proj entry point: the streaming kernel's [counters |
// partials] (rows <= the streaming limit), or the GEMM output rows followed by
// the hipBLASLt workspace.
size_t o_proj_ws_bytes(int m, int n, int k) {
    if (m <= skinny_max_m()) return skinny_ws_bytes(m, k, (n + kSkinnyCols - 1) / kSkinnyCols);
    if (!use_hipblaslt()) return 256 + gemm_ws_bytes(m, 1, &n);  // the GEMM adds into the hidden rows in place
    return align256(static_cast<size_t>(m) * n * 2) + kLtWorkspace;
}
// Workspace of the qkv entry point: the normed rows, then the streaming
// kernel's [counters | partials] or the hipBLASLt workspace.
size_t qkv_ws_bytes(int m, int k, int nq, int nkv) {
    const size_t normed = align256(static_cast<size_t>(m) * k * 2);
    if (m <= skinny_max_m()) return normed + skinny_ws_bytes(m, k, nq / kSkinnyCols + 2 * (nkv / kSkinnyCols));
    const int ns[3] = {nq, nkv, nkv};
    return normed + (use_hipblaslt() ? lt_ws_bytes() : gemm_ws_bytes(m, 3, ns));
}
}  // namespace ssa

extern "C" size_t supersonic_attn_gfx950_o_proj_workspace_size(size_t rows, size_t hidden_dim, size_t attn_dim) {
    if (rows == 0 || hidden_dim == 0 || rows > 0x7FFFFFFF || hidden_dim > 0x7FFFFFFF || attn_dim > 0x7FFFFFFF)
        return 0;
    return o_proj_ws_bytes(static_cast<int>(rows), static_cast<int>(hidden_dim), static_cast<int>(attn_dim));
}

extern "C" size_t supersonic_attn_gfx950_qkv_proj_workspace_size(size_t rows, size_t hidden_dim, size_t q_out_dim,
                                                                 size_t kv_out_dim) {
    if (rows == 0 || rows > 0x7FFFFFFF || hidden_dim > 0x7FFFFFFF || q_out_dim > 0x7FFFFFFF ||
        kv_out_dim > 0x7FFFFFFF)
        return 0;
    return qkv_ws_bytes(static_cast<int>(rows), static_cast<int>(hidden_dim), static_cast<int>(q_out_dim),
                        static_cast<int>(kv_out_dim));
}

extern "C" int supersonic_attn_gfx950_o_proj_residual(size_t device_ordinal, void* stream, int hidden_dtype,
                                                      size_t rows, size_t hidden_dim, size_t attn_dim,
                                                      const void* attn, const void* o_proj_w, void* hidden,
                                                      void* workspace, size_t workspace_bytes) {
    if (hidden_dtype != SUPERSONIC_DTYPE_BF16 && hidden_dtype != SUPERSONIC_DTYPE_F32) return SUPERSONIC_ERR_DTYPE;
    if (rows > 0x7FFFFFFF || hidden_dim > 0x7FFFFFFF || attn_dim > 0x7FFFFFFF) return SUPERSONIC_ERR_RANGE;
    if (rows == 0 || hidden_dim == 0) return 0;
    if (!hidden || (attn_dim && (!attn || !o_proj_w))) return SUPERSONIC_ERR_NULL;
    const int dev = static_cast<int>(device_ordinal);
    ScopedDevice scoped(dev);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int m = static_cast<int>(rows), n = static_cast<int>(hidden_dim), k = static_cast<int>(attn_dim);
    const bool f32 = hidden_dtype == SUPERSONIC_DTYPE_F32;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    const ProfileEvents ev = take_profile_events();
    if (ev.before) (void)hipEventRecord(ev.before, st);
    if (skinny_fits(m, k, attn, o_proj_w)) {
        SkinnyParams p{};
        p.x = static_cast<const uint16_t*>(attn);
        one_segment(p, o_proj_w, hidden, n);
        p.res = hidden;
        p.m = m;
        p.k = k;
        int rc;
        if (k > 0 && lds_path(dev, m, k, 1, p.cb_end[2]))
            rc = f32 ? launch_skinny_lds<float, true>(st, 1, lds_params(p))
                     : launch_skinny_lds<bf16_t, true>(st, 1, lds_params(p));
        else
            rc = f32 ? launch_skinny<float, true>(dev, st, 1, p, ws, workspace_bytes)
                     : launch_skinny<bf16_t, true>(dev, st, 1, p, ws, workspace_bytes);
        if (rc) return rc;
    } else if (!use_hipblaslt()) {
        if (k == 0) return 0;  // nothing to add
        const void* w1[1] = {o_proj_w};
        void* o1[1] = {hidden};
        const int n1[1] = {n};
        if (gemm_segments(dev, st, m, k, attn, 1, w1, o1, n1, f32 ? kGemmResidualF32 : kGemmResidualBf16, ws,
                          workspace_bytes) != 0)
            return SUPERSONIC_ERR_LAUNCH;
    } else {
        const size_t total = rows * hidden_dim;
        void* y;
        void* lt_ws = nullptr;
        if (ws) {
            if (workspace_bytes < align256(total * 2) + kLtWorkspace) return SUPERSONIC_ERR_WORKSPACE;
            y = ws;
            lt_ws = ws + align256(total * 2);
        } else {
            y = device_workspace(dev, total * 2, kWorkspaceProj);
        }
        if (!y) return SUPERSONIC_ERR_WORKSPACE;
        if (k == 0) {
            hipLaunchKernelGGL(fill_u16_kernel, dim3(stride_blocks(total)), dim3(256), 0, st, total,
                               static_cast<uint16_t*>(y));
            if (hipGetLastError() != hipSuccess) return SUPERSONIC_ERR_LAUNCH;
        } else if (lt_gemm(dev, st, 1, m, n, k, attn, o_proj_w, y, lt_ws) != 0) {
            return SUPERSONIC_ERR_LAUNCH;
        }
        const dim3 grid(stride_blocks(total)), blk(256);
        if (f32)
            hipLaunchKernelGGL((residual_add_kernel<float>), grid, blk, 0, st, total, static_cast<const uint16_t*>(y),
                               static_cast<float*>(hidden));
        else
            hipLaunchKernelGGL((residual_add_kernel<bf16_t>), grid, blk, 0, st, total,
                               static_cast<const uint16_t*>(y), static_cast<bf16_t*>(hidden));
        if (hipGetLastError() != hipSuccess) return SUPERSONIC_ERR_LAUNCH;
    }
    if (ev.after) (void)hipEventRecord(ev.after, st);
    return 0;
}

extern "C" int supersonic_attn_gfx950_qkv_proj(size_t device_ordinal, void* stream, int hidden_dtype, size_t rows,
                                               size_t hidden_dim, size_t q_out_dim, size_t kv_out_dim, float eps,
                                               const void* hidden, const void* input_norm_w, const void* q_proj_w,
                                               const void* k_proj_w, const void* v_proj_w, void* q_proj_out,
                                               void* k_out, void* v_out, void* workspace, size_t workspace_bytes) {
    if (hidden_dtype != SUPERSONIC_DTYPE_BF16 && hidden_dtype != SUPERSONIC_DTYPE_F32) return SUPERSONIC_ERR_DTYPE;
    if (rows > 0x7FFFFFFF || hidden_dim > 0x7FFFFFFF || q_out_dim > 0x7FFFFFFF || kv_out_dim > 0x7FFFFFFF)
        return SUPERSONIC_ERR_RANGE;
    if (rows == 0) return 0;
    if (!hidden || !input_norm_w || !q_proj_w || !q_proj_out || (kv_out_dim && (!k_proj_w || !v_proj_w || !k_out || !v_out)))
        return SUPERSONIC_ERR_NULL;
    if (hidden_dim == 0 || hidden_dim % 8 != 0) return SUPERSONIC_ERR_RANGE;
    const int dev = static_cast<int>(device_ordinal);
    ScopedDevice scoped(dev);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int m = static_cast<int>(rows), k = static_cast<int>(hidden_dim);
    const int nq = static_cast<int>(q_out_dim), nkv = static_cast<int>(kv_out_dim);
    const bool f32 = hidden_dtype == SUPERSONIC_DTYPE_F32;
    const bool aligned = ((reinterpret_cast<uintptr_t>(hidden) | reinterpret_cast<uintptr_t>(input_norm_w) |
                           reinterpret_cast<uintptr_t>(q_proj_w) | reinterpret_cast<uintptr_t>(k_proj_w) |
                           reinterpret_cast<uintptr_t>(v_proj_w)) & 15) == 0;
    // the normed rows go to the workspace once (bf16 [rows, hidden_dim]),
    // followed by the projection's own workspace
    const size_t normed_bytes = align256(static_cast<size_t>(m) * k * 2);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    uint16_t* normed;
    uint8_t* rest = nullptr;
    size_t rest_bytes = 0;
    if (ws) {
        if (workspace_bytes < normed_bytes) return SUPERSONIC_ERR_WORKSPACE;
        normed = reinterpret_cast<uint16_t*>(ws);
        rest = ws + normed_bytes;
        rest_bytes = workspace_bytes - normed_bytes;
    } else {
        normed = static_cast<uint16_t*>(device_workspace(dev, static_cast<size_t>(m) * k * 2, kWorkspaceProj));
    }
    if (!normed) return SUPERSONIC_ERR_WORKSPACE;
    const ProfileEvents ev = take_profile_events();
    if (ev.before) (void)hipEventRecord(ev.before, st);
    {
        const dim3 grid(m), blk(256);
        if (f32)
            hipLaunchKernelGGL((input_norm_kernel<float>), grid, blk, 0, st, m, k, eps, static_cast<const float*>(hidden),
                               static_cast<const uint16_t*>(input_norm_w), normed);
        else
            hipLaunchKernelGGL((input_norm_kernel<bf16_t>), grid, blk, 0, st, m, k, eps,
                               static_cast<const bf16_t*>(hidden), static_cast<const uint16_t*>(input_norm_w), normed);
        if (hipGetLastError() != hipSuccess) return SUPERSONIC_ERR_LAUNCH;
    }
    if (skinny_fits(m, k, normed, q_proj_w) && aligned && nq % kSkinnyCols == 0 && nkv % kSkinnyCols == 0) {
        // the three matrices as one column space of the weight-streaming kernel
        SkinnyParams p{};
        p.x = normed;
        p.w[0] = static_cast<const uint16_t*>(q_proj_w);
        p.w[1] = static_cast<const uint16_t*>(k_proj_w);
        p.w[2] = static_cast<const uint16_t*>(v_proj_w);
        p.out[0] = q_proj_out;
        p.out[1] = k_out;
        p.out[2] = v_out;
        p.n_seg[0] = nq;
        p.n_seg[1] = p.n_seg[2] = nkv;
        p.cb_end[0] = nq / kSkinnyCols;
        p.cb_end[1] = p.cb_end[0] + nkv / kSkinnyCols;
        p.cb_end[2] = p.cb_end[1] + nkv / kSkinnyCols;
        p.m = m;
        p.k = k;
        if (p.cb_end[2] > 0) {
            const int rc = lds_path(dev, m, k, 1, p.cb_end[2])
                               ? launch_skinny_lds<bf16_t, false>(st, 1, lds_params(p))
                               : launch_skinny<bf16_t, false>(dev, st, 1, p, rest, rest_bytes);
            if (rc) return rc;
        }
    } else {
        // GEMM-sized: the three matrices as column segments of one GEMM
        const void* wts[3] = {q_proj_w, k_proj_w, v_proj_w};
        void* os[3] = {q_proj_out, k_out, v_out};
        const int ns[3] = {nq, nkv, nkv};
        if (!use_hipblaslt()) {
            if (gemm_segments(dev, st, m, k, normed, 3, wts, os, ns, kGemmStore, ws ? rest : nullptr, rest_bytes) != 0)
                return SUPERSONIC_ERR_LAUNCH;
        } else {
            if (ws && rest_bytes < kLtWorkspace) return SUPERSONIC_ERR_WORKSPACE;
            for (int i = 0; i < 3; ++i) {
                if (ns[i] == 0) continue;
                if (lt_gemm(dev, st, 1, m, ns[i], k, normed, wts[i], os[i], rest) != 0) return SUPERSONIC_ERR_LAUNCH;
            }
        }
    }
    if (ev.after) (void)hipEventRecord(ev.after, st);
    return 0;
}

// ---------------------------------------------------------------------------
// Input RMSNorm + Q/K/V projections + per-head QK RMSNorm + partial RoPE
// (+ bf16 KV-cache append): the megakernel's steps A-D
// (full_attention_4b.hip:4942-5101 feeding :5142-5224, :5282-5294) in one
// weight-streaming launch after the input norm.
// ---------------------------------------------------------------------------
namespace ssa {
constexpr size_t kRopeCounterBytes = 64 << 10;  // per-head arrival counters (Hq + Hkv <= 16384)

size_t qkv_rope_ws_bytes(int m, int k, int Hq, int Hkv, int D) {
    const size_t normed = align256(static_cast<size_t>(m) * k * 2);
    // unfused path: q_proj and the raw k / v rows, then the projection's own workspace
    const size_t raw = align256(static_cast<size_t>(m) * Hq * 2 * D * 2) + 2 * align256(static_cast<size_t>(m) * Hkv * D * 2);
    return kRopeCounterBytes + normed + raw + qkv_ws_bytes(m, k, Hq * 2 * D, Hkv * D) - align256(static_cast<size_t>(m) * k * 2);
}
}  // namespace ssa

extern "C" size_t supersonic_attn_gfx950_qkv_proj_rope_workspace_size(size_t rows, size_t hidden_dim, size_t q_heads,
                                                                      size_t kv_heads, size_t head_dim) {
    if (rows == 0 || rows > 0x7FFFFFFF || hidden_dim > 0x7FFFFFFF || q_heads > 4096 || kv_heads > 4096 ||
        head_dim > 512)
        return 0;
    return qkv_rope_ws_bytes(static_cast<int>(rows), static_cast<int>(hidden_dim), static_cast<int>(q_heads),
                             static_cast<int>(kv_heads), static_cast<int>(head_dim));
}

extern "C" int supersonic_attn_gfx950_qkv_proj_rope(
    size_t device_ordinal, void* stream, int hidden_dtype, size_t rows, size_t hidden_dim, size_t q_heads,
    size_t kv_heads, size_t head_dim, size_t rotary_dim, float eps, float qk_eps, const void* hidden,
    const void* input_norm_w, const void* q_proj_w, const void* k_proj_w, const void* v_proj_w,
    const void* q_norm_w, const void* k_norm_w, const void* cos_table, const void* sin_table,
    const int32_t* positions, void* q_out, void* gate_out, void* k_out, void* v_out,
    const supersonic_kv_cache* cache, void* workspace, size_t workspace_bytes) {
    if (hidden_dtype != SUPERSONIC_DTYPE_BF16 && hidden_dtype != SUPERSONIC_DTYPE_F32) return SUPERSONIC_ERR_DTYPE;
    if (rows > 0x7FFFFFFF || hidden_dim > 0x7FFFFFFF || q_heads > 4096 || kv_heads > 4096) return SUPERSONIC_ERR_RANGE;
    if (head_dim == 0 || head_dim > 512 || head_dim % 16 != 0) return SUPERSONIC_ERR_HEAD_DIM;
    if (kv_heads == 0 || q_heads % kv_heads != 0) return SUPERSONIC_ERR_HEADS;
    if (rotary_dim % 2 != 0 || rotary_dim > head_dim) return SUPERSONIC_ERR_ROTARY;
    if (rows == 0) return 0;
    if (!hidden || !input_norm_w || !q_proj_w || !k_proj_w || !v_proj_w || !q_norm_w || !k_norm_w || !positions ||
        !q_out || !gate_out || !k_out || !v_out)
        return SUPERSONIC_ERR_NULL;
    if (rotary_dim > 0 && (!cos_table || !sin_table)) return SUPERSONIC_ERR_NULL;
    if (hidden_dim == 0 || hidden_dim % 8 != 0) return SUPERSONIC_ERR_RANGE;
    KvView kv{};
    if (cache) {
        if (cache->k_scale || cache->v_scale) return SUPERSONIC_ERR_CACHE;  // bf16 caches only
        if (int rc = make_view(cache, false, &kv)) return rc;
    }
    const int dev = static_cast<int>(device_ordinal);
    ScopedDevice scoped(dev);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int m = static_cast<int>(rows), k = static_cast<int>(hidden_dim);
    const int Hq = static_cast<int>(q_heads), Hkv = static_cast<int>(kv_heads), D = static_cast<int>(head_dim);
    const int nq = Hq * 2 * D, nkv = Hkv * D;
    const size_t need = qkv_rope_ws_bytes(m, k, Hq, Hkv, D);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    if (ws) {
        if (workspace_bytes < need) return SUPERSONIC_ERR_WORKSPACE;
    } else {
        // zero-filled once; every call leaves the counters at zero
        ws = static_cast<uint8_t*>(device_workspace(dev, need, kWorkspaceRope));
        if (!ws) return SUPERSONIC_ERR_WORKSPACE;
    }
    RopeEpi e{};
    e.q_out = static_cast<uint16_t*>(q_out);
    e.gate_out = static_cast<uint16_t*>(gate_out);
    e.k_out = static_cast<uint16_t*>(k_out);
    e.v_out = static_cast<uint16_t*>(v_out);
    e.q_norm_w = static_cast<const uint16_t*>(q_norm_w);
    e.k_norm_w = static_cast<const uint16_t*>(k_norm_w);
    e.cos_t = static_cast<const uint16_t*>(cos_table);
    e.sin_t = static_cast<const uint16_t*>(sin_table);
    e.pos = positions;
    e.kv = kv;
    e.counters = reinterpret_cast<unsigned*>(ws);
    e.Hq = Hq;
    e.Hkv = Hkv;
    e.D = D;
    e.half_rot = static_cast<int>(rotary_dim / 2);
    e.eps = qk_eps;
    uint16_t* normed = reinterpret_cast<uint16_t*>(ws + kRopeCounterBytes);
    uint8_t* rest = ws + kRopeCounterBytes + align256(static_cast<size_t>(m) * k * 2);
    const bool f32 = hidden_dtype == SUPERSONIC_DTYPE_F32;
    const bool aligned = ((reinterpret_cast<uintptr_t>(hidden) | reinterpret_cast<uintptr_t>(input_norm_w) |
                           reinterpret_cast<uintptr_t>(q_proj_w) | reinterpret_cast<uintptr_t>(k_proj_w) |
                           reinterpret_cast<uintptr_t>(v_proj_w) | reinterpret_cast<uintptr_t>(q_out) |
                           reinterpret_cast<uintptr_t>(k_out)) & 15) == 0;
    const ProfileEvents ev = take_profile_events();
    if (ev.before) (void)hipEventRecord(ev.before, st);
    {
        const dim3 grid(m), blk(256);
        if (f32)
            hipLaunchKernelGGL((input_norm_kernel<float>), grid, blk, 0, st, m, k, eps, static_cast<const float*>(hidden),
                               static_cast<const uint16_t*>(input_norm_w), normed);
        else
            hipLaunchKernelGGL((input_norm_kernel<bf16_t>), grid, blk, 0, st, m, k, eps,
                               static_cast<const bf16_t*>(hidden), static_cast<const uint16_t*>(input_norm_w), normed);
        if (hipGetLastError() != hipSuccess) return SUPERSONIC_ERR_LAUNCH;
    }
    const int ncb = (nq + 2 * nkv) / kSkinnyCols;
    if (aligned && (D == 128 || D == 256) && lds_path(dev, m, k, 1, ncb) && m <= skinny_max_m() &&
        Hq + Hkv <= static_cast<int>(kRopeCounterBytes / 4)) {
        SkinnyLdsParams p{};
        p.x = normed;
        p.w[0] = static_cast<const uint16_t*>(q_proj_w);
        p.w[1] = static_cast<const uint16_t*>(k_proj_w);
        p.w[2] = static_cast<const uint16_t*>(v_proj_w);
        p.n_seg[0] = nq;
        p.n_seg[1] = p.n_seg[2] = nkv;
        p.cb_end[0] = nq / kSkinnyCols;
        p.cb_end[1] = p.cb_end[0] + nkv / kSkinnyCols;
        p.cb_end[2] = p.cb_end[1] + nkv / kSkinnyCols;
        p.m = m;
        p.k = k;
        hipLaunchKernelGGL((skinny_lds_kernel<bf16_t, false, true>), dim3(ncb, 1, 1), dim3(64 * kSkinnyWaves), 0, st,
                           p, e);
        if (hipGetLastError() != hipSuccess) return SUPERSONIC_ERR_LAUNCH;
    } else {
        // plain projections into the workspace, then one wave per (row, head)
        uint16_t* qp = reinterpret_cast<uint16_t*>(rest);
        uint16_t* kr = reinterpret_cast<uint16_t*>(rest + align256(static_cast<size_t>(m) * nq * 2));
        uint16_t* vr = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(kr) + align256(static_cast<size_t>(m) * nkv * 2));
        uint8_t* pws = reinterpret_cast<uint8_t*>(vr) + align256(static_cast<size_t>(m) * nkv * 2);
        const size_t pws_bytes = ws + need > pws ? static_cast<size_t>(ws + need - pws) : 0;
        if (skinny_fits(m, k, normed, q_proj_w) && aligned && nq % kSkinnyCols == 0 && nkv % kSkinnyCols == 0) {
            SkinnyParams p{};
            p.x = normed;
            p.w[0] = static_cast<const uint16_t*>(q_proj_w);
            p.w[1] = static_cast<const uint16_t*>(k_proj_w);
            p.w[2] = static_cast<const uint16_t*>(v_proj_w);
            p.out[0] = qp;
            p.out[1] = kr;
            p.out[2] = vr;
            p.n_seg[0] = nq;
            p.n_seg[1] = p.n_seg[2] = nkv;
            p.cb_end[0] = nq / kSkinnyCols;
            p.cb_end[1] = p.cb_end[0] + nkv / kSkinnyCols;
            p.cb_end[2] = p.cb_end[1] + nkv / kSkinnyCols;
            p.m = m;
            p.k = k;
            const int rc = lds_path(dev, m, k, 1, p.cb_end[2]) ? launch_skinny_lds<bf16_t, false>(st, 1, lds_params(p))
                                                               : launch_skinny<bf16_t, false>(dev, st, 1, p, pws, pws_bytes);
            if (rc) return rc;
        } else {
            const void* wts[3] = {q_proj_w, k_proj_w, v_proj_w};
            void* os[3] = {qp, kr, vr};
            const int ns[3] = {nq, nkv, nkv};
            if (!use_hipblaslt()) {
                if (gemm_segments(dev, st, m, k, normed, 3, wts, os, ns, kGemmStore, workspace ? pws : nullptr,
                                  pws_bytes) != 0)
                    return SUPERSONIC_ERR_LAUNCH;
            } else {
                if (workspace && pws_bytes < kLtWorkspace) return SUPERSONIC_ERR_WORKSPACE;
                for (int i = 0; i < 3; ++i)
                    if (lt_gemm(dev, st, 1, m, ns[i], k, normed, wts[i], os[i], workspace ? pws : nullptr) != 0)
                        return SUPERSONIC_ERR_LAUNCH;
            }
        }
        hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(m, Hq + Hkv), dim3(64), 0, st, qp, kr, vr, e);
        if (hipGetLastError() != hipSuccess) return SUPERSONIC_ERR_LAUNCH;
    }
    if (ev.after) (void)hipEventRecord(ev.after, st);
    return 0;
}
