// The LDS-staged weight-streaming projection (decode rows): parameters, the
// QK-norm / RoPE epilogue and the workgroup body as a device function, shared
// by the projection kernels (proj.hip) and the persistent decode layer
// (layer.hip).
#pragma once

#include "common.hpp"
#include "kv_view.hpp"

namespace ssa {

constexpr int kSkinnyWaves = 8;
constexpr int kSkinnySteps = 8;                     // 32-wide k-steps per load batch (<= 128 VGPRs)
constexpr int kSkinnyLdsSteps = 16;                 // ... of the standalone LDS-staged kernel (k = 4096 in one batch; 2-3% faster)
constexpr int kSkinnyCols = 16;                     // W rows (output columns) per workgroup

__device__ __forceinline__ bf16x8_v as_bf16x8(const u32x4_v& v) { return __builtin_bit_cast(bf16x8_v, v); }

template <typename XT>
__device__ __forceinline__ void load8f(const XT* p, float (&f)[8]);
template <>
__device__ __forceinline__ void load8f<bf16_t>(const bf16_t* p, float (&f)[8]) { unpack8<bf16_t>(ld16(p), f); }
template <>
__device__ __forceinline__ void load8f<float>(const float* p, float (&f)[8]) {
    const f32x4_v a = *reinterpret_cast<const f32x4_v*>(p);
    const f32x4_v b = *reinterpret_cast<const f32x4_v*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f[e] = a[e];
        f[4 + e] = b[e];
    }
}


constexpr int kXsMax = 32768;  // staged elements (64 KB): two workgroups per CU
constexpr int kXsChunks = kXsMax / 8 / 512;  // 16-byte chunks per thread at most
constexpr int kXsDummy = kXsMax + 120;        // 16-byte slot for the chunks past the rows

// Per-head QK RMSNorm + partial RoPE (+ KV-cache append) applied to the
// Q/K projection outputs (the fused projection of the decode step).
struct RopeEpi {
    uint16_t* q_out;      // [m, Hq*D]   normalised + rotated q
    uint16_t* gate_out;   // [m, Hq*D]   raw gate half of each q_proj head
    uint16_t* k_out;      // [m, Hkv*D]  normalised + rotated k
    uint16_t* v_out;      // [m, Hkv*D]
    const uint16_t* q_norm_w;
    const uint16_t* k_norm_w;
    const uint16_t* cos_t;  // [max_pos, half_rot]
    const uint16_t* sin_t;
    const int32_t* pos;     // [m] position of each row (RoPE angle, cache slot)
    KvView kv;              // bf16 cache the new k / v are appended to (kv.k == NULL: none)
    unsigned* counters;     // [Hq + Hkv] column-block arrivals per head, zero between calls
    int Hq, Hkv, D, half_rot;
    float eps;
};

// One head row of D bf16 values, lane holding the EPL = D / 64 consecutive
// dims lane * EPL ..: RMSNorm with (1 + w) (bf16 result), then rotate-half
// RoPE on dims [0, 2 hr) at position pos (bf16 result), the megakernel's
// steps B-C (full_attention_4b.hip:5142-5224).  rowbuf: D floats of LDS
// private to the wave (RoPE partners).
template <int EPL>
__device__ __forceinline__ void norm_rope_row(float (&x)[EPL], const uint16_t* w, const uint16_t* cos_t,
                                              const uint16_t* sin_t, int pos, int hr, float eps, int D,
                                              float* rowbuf) {
    const int lane = threadIdx.x & 63;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) ss += x[j] * x[j];
    ss = wave_sum(ss);
    const float inv = rsqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
    for (int j = 0; j < EPL; ++j)
        x[j] = bf16_round(x[j] * inv * (bf16_bits_to_f32(w[lane * EPL + j]) + 1.0f));
    if (hr > 0) {
#pragma unroll
        for (int j = 0; j < EPL; ++j) rowbuf[lane * EPL + j] = x[j];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int d = lane * EPL + j;
            if (d < 2 * hr) {
                const int ti = d < hr ? d : d - hr;
                const float c = bf16_bits_to_f32(cos_t[static_cast<int64_t>(pos) * hr + ti]);
                const float sn = bf16_bits_to_f32(sin_t[static_cast<int64_t>(pos) * hr + ti]);
                const float other = rowbuf[d < hr ? d + hr : d - hr];
                x[j] = d < hr ? bf16_round(x[j] * c - other * sn) : bf16_round(other * sn + x[j] * c);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

struct SkinnyLdsParams {
    const uint16_t* x;      // [batch][m][k] bf16
    // NORM staging: the activation rows are bf16(xn * rsqrt(mean(xn^2) + norm_eps)
    // * (1 + norm_w)) of xn [batch][m][k] (bf16 or f32), computed while staging
    const void* xn;
    const uint16_t* norm_w;
    float norm_eps;
    const uint16_t* w[3];
    void* out[3];
    const void* res;
    int n_seg[3];
    int cb_end[3];
    int m, k;
    int64_t x_bs, w_bs, o_bs;
};

// LDS of one weight-streaming workgroup (SkinnyLdsBase without the NORM
// staging array: 74 KB, so two workgroups share a CU).
struct SkinnyLdsBase {
    __attribute__((aligned(16))) uint16_t xs[kXsMax + 16 * 8];
    __attribute__((aligned(16))) float red[kSkinnyWaves][256];
    int last_s;
};
struct SkinnyLds : SkinnyLdsBase {
    float part[kXsMax / 8];   // NORM staging: sum of squares of each 8-element chunk
};

// One workgroup of the weight stream: column block cb of batch element b.
// NORM: the rows are normalised while staged (XT: element type of p.xn).
// COH_IN / COH_OUT: the activation rows are read / the outputs written with
// device-coherent accesses (data exchanged with other workgroups of the same
// kernel).  PAIR (plain store epilogue only): a second column block cb2 (or
// none when cb2 < 0) shares the staged rows, and both blocks' weight loads are
// in flight together, so two blocks cost little more than one.
template <typename OT, bool RES, bool ROPE, bool NORM = false, typename XT = bf16_t, bool COH_IN = false,
          bool COH_OUT = false, typename LdsT = SkinnyLds, bool PAIR = false, int STEPS = kSkinnySteps>
__device__ __forceinline__ void skinny_lds_body(const SkinnyLdsParams& p, const RopeEpi& e, int cb, int b,
                                                LdsT& L, int cb2 = -1) {
    static_assert(!PAIR || (!RES && !ROPE), "pairs take the plain store epilogue");
    uint16_t (&xs)[kXsMax + 16 * 8] = L.xs;
    float (&red)[kSkinnyWaves][256] = L.red;
    // opaque: when several bodies are inlined into one kernel, lane-derived
    // values are not shared between them (and kept live across other phases)
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int seg = cb < p.cb_end[0] ? 0 : (cb < p.cb_end[1] ? 1 : 2);
    const int cbs = cb - (seg == 0 ? 0 : (seg == 1 ? p.cb_end[0] : p.cb_end[1]));
    const int n = pick3(p.n_seg, seg);
    const int k = p.k, m = p.m;
    const int ldx = k + 8;  // padded LDS row: the 16 rows of an A operand read hit distinct banks
    const int cpr = k / 8;  // 16-byte chunks per row
    const uint16_t* x = p.x + b * p.x_bs;
    const u32x4_v zero = {0u, 0u, 0u, 0u};

    // 1. the activation rows (and norm weights), ahead of any W load
    // Branch-free (clamped addresses, values selected afterwards): conditional
    // loads and stores would sit in blocks where the wait for these loads
    // falls back to vmcnt(0), which would also wait for the W batch.
    const int nch = m * cpr;
    u32x4_v xr[kXsChunks];
    // NORM: the rows' chunks as floats and the norm weights, loaded before the W batch
    float xf[NORM ? kXsChunks : 1][8];
    u32x4_v nwr[NORM ? kXsChunks : 1];
    if constexpr (!NORM) {
#pragma unroll
        for (int j = 0; j < kXsChunks; ++j) {
            const int c = min(tid + 512 * j, nch - 1);
            const uint16_t* src = x + static_cast<int64_t>(c / cpr) * k + 8 * (c % cpr);
            xr[j] = COH_IN ? ld16_agent(src) : ld16(src);
        }
    } else {
        const XT* xin = static_cast<const XT*>(p.xn) + b * p.x_bs;
#pragma unroll
        for (int j = 0; j < kXsChunks; ++j) {
            const int c = min(tid + 512 * j, nch - 1);
            load8f<XT>(xin + static_cast<int64_t>(c / cpr) * k + 8 * (c % cpr), xf[j]);
            nwr[j] = ld16(p.norm_w + 8 * (c % cpr));
        }
    }
    asm volatile("" ::: "memory");

    // 2. the first W batch
    const int T = (k + 31) / 32;
    const int per = (T + kSkinnyWaves - 1) / kSkinnyWaves;
    const int s0 = wave * per;
    const int s1 = min(s0 + per, T);
    const int col = lane & 15;
    const int kq = (lane >> 4) * 8;
    const int n_w = cbs * 16 + col;
    const uint16_t* wrow = pick3(p.w, seg) + b * p.w_bs + static_cast<int64_t>(min(n_w, n - 1)) * k + kq;
    // Unconditional W loads at a clamped, always in-range address: a step
    // outside this wave's range (or past k) meets a zero A operand instead.
    // (A load under a condition would sit in its own block, where waiting for
    // the activation loads issued before it falls back to vmcnt(0).)
    const uint16_t* wrow0 = wrow - kq;
    auto wload = [&](int s) { return ld16(wrow0 + min(s * 32 + kq, k - 8)); };
    u32x4_v wv[STEPS];
#pragma unroll
    for (int j = 0; j < STEPS; ++j) wv[j] = wload(s0 + j);
    // PAIR: the second block's column segment, weight row and first batch
    const bool two = PAIR && cb2 >= 0;
    const int cb2c = two ? cb2 : cb;
    const int seg2 = cb2c < p.cb_end[0] ? 0 : (cb2c < p.cb_end[1] ? 1 : 2);
    const int cbs2 = cb2c - (seg2 == 0 ? 0 : (seg2 == 1 ? p.cb_end[0] : p.cb_end[1]));
    const int n2 = pick3(p.n_seg, seg2);
    const uint16_t* wrow20 = pick3(p.w, seg2) + b * p.w_bs + static_cast<int64_t>(min(cbs2 * 16 + col, n2 - 1)) * k;
    auto wload2 = [&](int s) { return ld16(wrow20 + min(s * 32 + kq, k - 8)); };
    u32x4_v wv2[PAIR ? STEPS : 1];
    if constexpr (PAIR) {
#pragma unroll
        for (int j = 0; j < STEPS; ++j) wv2[j] = wload2(s0 + j);
    }
    // RES: the residual element this thread adds in the epilogue, loaded now so
    // that its round trip overlaps the weight stream (clamped, branch-free)
    float res_v = 0.f;
    if constexpr (RES && !ROPE) {
        const int row = min(tid >> 4, m - 1), c = min(cbs * 16 + (tid & 15), n - 1);
        res_v = load_f32<OT>(static_cast<const OT*>(p.res), b * p.o_bs + static_cast<int64_t>(row) * n + c);
    }

    // 3. stage the rows in LDS; chunks past the rows go to a dummy slot at the
    // end of the padding.  The padded rows end at m * ldx - 8 = m * k + 8 (m - 1)
    // <= kXsMax + 120 elements (m <= 16, m * k <= kXsMax), so the slot
    // [kXsMax + 120, kXsMax + 128) never overlaps a row.
    if constexpr (!NORM) {
#pragma unroll
        for (int j = 0; j < kXsChunks; ++j) {
            const int c = tid + 512 * j;
            st16(c < nch ? xs + (c / cpr) * ldx + 8 * (c % cpr) : xs + kXsDummy, xr[j]);
        }
    } else {
        // RMSNorm with (1 + w) of each row (input_norm_kernel's arithmetic): the
        // chunks' sums of squares go to LDS, one wave adds each row's (a fixed
        // order), then the normalised bf16 chunks are staged
        float (&part)[kXsMax / 8] = L.part;
#pragma unroll
        for (int j = 0; j < kXsChunks; ++j) {
            const int c = tid + 512 * j;
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += xf[j][i] * xf[j][i];
            if (c < nch) part[c] = ss;
        }
        lds_barrier();
        for (int row = wave; row < m; row += kSkinnyWaves) {
            float ss = 0.f;
            for (int c = lane; c < cpr; c += 64) ss += part[row * cpr + c];
            ss = wave_sum(ss);
            if (lane == 0) part[row * cpr] = rsqrtf(ss / static_cast<float>(k) + p.norm_eps);
        }
        lds_barrier();
#pragma unroll
        for (int j = 0; j < kXsChunks; ++j) {
            const int c = tid + 512 * j;
            if (c < nch) {
                const float inv = part[(c / cpr) * cpr];
                float g[8];
                unpack8<bf16_t>(nwr[j], g);
                u32x4_v o;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[i] = f32_to_bf16_bits(xf[j][2 * i] * inv * (g[2 * i] + 1.0f)) |
                           (f32_to_bf16_bits(xf[j][2 * i + 1] * inv * (g[2 * i + 1] + 1.0f)) << 16);
                st16(xs + (c / cpr) * ldx + 8 * (c % cpr), o);
            }
        }
    }
    lds_barrier();

    // 4. the weight stream, A operand from LDS
    const bool mvalid = col < m;
    const uint16_t* xrow = xs + col * ldx + kq;
    f32x4_v acc = {0.f, 0.f, 0.f, 0.f}, acc2 = {0.f, 0.f, 0.f, 0.f};
    for (int sb = s0; sb < s1; sb += STEPS) {
        if (sb > s0) {
#pragma unroll
            for (int j = 0; j < STEPS; ++j) wv[j] = wload(sb + j);
            if constexpr (PAIR) {
#pragma unroll
                for (int j = 0; j < STEPS; ++j) wv2[j] = wload2(sb + j);
            }
        }
#pragma unroll
        for (int j = 0; j < STEPS; ++j) {
            const int s = sb + j;
            const u32x4_v a = (s < s1 && mvalid && s * 32 + kq < k)
                                  ? *reinterpret_cast<const u32x4_v*>(xrow + s * 32) : zero;
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(wv[j]), acc, 0, 0, 0);
            if constexpr (PAIR) acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(wv2[j]), acc2, 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][(4 * (lane >> 4) + i) * 16 + col] = acc[i];
    __syncthreads();
    if constexpr (!ROPE) {
        if (tid < 256) {
            const int row = tid >> 4, c = cbs * 16 + (tid & 15);
            if (row < m && c < n) {
                float sum = 0.f;
#pragma unroll
                for (int v = 0; v < kSkinnyWaves; ++v) sum += red[v][tid];
                float y = bf16_round(sum);
                const int64_t o = b * p.o_bs + static_cast<int64_t>(row) * n + c;
                if constexpr (RES) y = bf16_round(res_v + y);
                if constexpr (COH_OUT) store_f32_agent<OT>(static_cast<OT*>(pick3(p.out, seg)), o, y);
                else store_f32<OT>(static_cast<OT*>(pick3(p.out, seg)), o, y);
            }
        }
        if constexpr (PAIR) {
            if (two) {
                __syncthreads();  // every thread has read red for the first block
#pragma unroll
                for (int i = 0; i < 4; ++i) red[wave][(4 * (lane >> 4) + i) * 16 + col] = acc2[i];
                __syncthreads();
                if (tid < 256) {
                    const int row = tid >> 4, c = cbs2 * 16 + (tid & 15);
                    if (row < m && c < n2) {
                        float sum = 0.f;
#pragma unroll
                        for (int v = 0; v < kSkinnyWaves; ++v) sum += red[v][tid];
                        const float y = bf16_round(sum);
                        const int64_t o = b * p.o_bs + static_cast<int64_t>(row) * n2 + c;
                        if constexpr (COH_OUT) store_f32_agent<OT>(static_cast<OT*>(pick3(p.out, seg2)), o, y);
                        else store_f32<OT>(static_cast<OT*>(pick3(p.out, seg2)), o, y);
                    }
                }
            }
        }
    } else {
        // Segments: 0 = W_q (per head [q | gate], 2D columns), 1 = W_k, 2 = W_v.
        // A 16-column block lies inside one head and one half of it.
        const int D = e.D;
        const int c0 = cbs * 16;
        const int hq = seg == 0 ? c0 / (2 * D) : c0 / D;   // head of the block
        const bool is_q = seg == 0 && (c0 % (2 * D)) < D;
        const bool is_gate = seg == 0 && !is_q;
        const bool norm_block = is_q || seg == 1;           // its head is normalised once complete
        if (tid < 256) {
            const int row = tid >> 4, cc = tid & 15;
            float sum = 0.f;
#pragma unroll
            for (int v = 0; v < kSkinnyWaves; ++v) sum += red[v][tid];
            const uint32_t yb = f32_to_bf16_bits(sum);          // the projection's bf16 rounding
            const uint32_t pair = yb | (static_cast<uint32_t>(__shfl_xor(static_cast<int>(yb), 1)) << 16);
            if (row < m) {
                const int d = (seg == 0 ? c0 % (2 * D) : c0 % D) + cc - (is_gate ? D : 0);
                const int64_t hd = static_cast<int64_t>(row) * (seg == 0 ? e.Hq : e.Hkv) * D + hq * D + d;
                if (norm_block) {
                    // pre-norm values, device-coherent: the head's last block reads them back
                    uint16_t* dst = seg == 0 ? e.q_out : e.k_out;
                    if ((cc & 1) == 0) store_agent_u32(reinterpret_cast<uint32_t*>(dst + hd), pair);
                } else if (is_gate) {
                    e.gate_out[hd] = static_cast<uint16_t>(yb);
                } else {
                    e.v_out[hd] = static_cast<uint16_t>(yb);
                    if (e.kv.k) {
                        const int64_t o = e.kv.row(row, hq, e.pos[row], D) + d;
                        reinterpret_cast<uint16_t*>(e.kv.v)[o] = static_cast<uint16_t>(yb);
                    }
                }
            }
        }
        if (!norm_block) return;
        // the head's last column block to arrive normalises and rotates it
        int& last_s = L.last_s;
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores are complete
        __syncthreads();
        const int ctr = seg == 0 ? hq : e.Hq + hq;
        if (tid == 0) {
            const unsigned prev = atomicAdd(&e.counters[ctr], 1u);
            last_s = prev == static_cast<unsigned>(D / 16 - 1);
            if (last_s) e.counters[ctr] = 0u;  // every block of the head has arrived
        }
        __syncthreads();
        if (!last_s) return;
        float* rowbuf = reinterpret_cast<float*>(xs) + wave * D;  // the activations are no longer read
        uint16_t* dst = seg == 0 ? e.q_out : e.k_out;
        const uint16_t* nw = seg == 0 ? e.q_norm_w : e.k_norm_w;
        const int H = seg == 0 ? e.Hq : e.Hkv;
        for (int row = wave; row < m; row += kSkinnyWaves) {
            uint16_t* rp = dst + static_cast<int64_t>(row) * H * D + hq * D;
            const int pos = e.pos[row];
            auto run = [&](auto epl_tag) {
                constexpr int EPL = decltype(epl_tag)::value;
                float x[EPL];
                if constexpr (EPL == 4) {
                    const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t*>(rp) + lane, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                    for (int j = 0; j < 4; ++j) x[j] = bf16_bits_to_f32(static_cast<uint32_t>(v >> (16 * j)) & 0xFFFFu);
                } else {
                    const uint32_t v = __hip_atomic_load(reinterpret_cast<uint32_t*>(rp) + lane, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
                    x[0] = bf16_bits_to_f32(v & 0xFFFFu);
                    x[1] = bf16_bits_to_f32(v >> 16);
                }
                norm_rope_row<EPL>(x, nw, e.cos_t, e.sin_t, pos, e.half_rot, e.eps, D, rowbuf);
#pragma unroll
                for (int j = 0; j < EPL; ++j) {
                    rp[lane * EPL + j] = static_cast<uint16_t>(f32_to_bf16_bits(x[j]));
                    if (seg == 1 && e.kv.k) {
                        const int64_t o = e.kv.row(row, hq, pos, D) + lane * EPL + j;
                        reinterpret_cast<uint16_t*>(e.kv.k)[o] = static_cast<uint16_t>(f32_to_bf16_bits(x[j]));
                    }
                }
            };
            if (D == 256) run(std::integral_constant<int, 4>{});
            else run(std::integral_constant<int, 2>{});
        }
    }
}

}  // namespace ssa
