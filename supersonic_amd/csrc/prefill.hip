// Causal GQA prefill attention on gfx950 MFMA.
//
// Replaces the reference's prefill attention
//   supersonic_qwen35_full_attention_prefill_kernel  kernels/full_attention.hip:246-361
//   (one wave per query row, scalar dot per key, two passes, per-key barriers)
// and, in the fused entry point, the chain around it
//   crates/runner/src/prefill_engine.rs:1951-2308
//   (split q/gate, QK RMSNorm, RoPE, transposes, cache copies, cast, gate).
//
// Kernel design (flash attention forward, fp32 accumulation):
//   workgroup = 4 wave64s, 128 query rows of one head (32 rows per wave);
//   keys in tiles of 64 staged through LDS: K row-major (16 B padded rows),
//   V transposed (V^T[dim][token]) with a token permutation inside every
//   16-token group so each MFMA operand fetch is one 16-byte ds_read.
//   S^T = K Q^T   v_mfma_f32_32x32x16_{bf16,f16}: A = K rows, B = Q^T held in
//                 registers for the whole kernel.  The C layout gives every
//                 lane one query row and 16 keys of each 32-key block.
//   O^T += V^T P^T: the B operand (P^T) is exactly the lane's own 8 softmax
//                 weights per 16-key step: no shuffles between the two GEMMs.
//   online softmax in base 2; one cross-lane max per tile (lane ^ 32).
//   causal: key tiles past the workgroup's last row are never loaded; a wave
//   skips the MFMA work of tiles past its own last row; only tiles that cross
//   the diagonal or the kv_len edge are masked.  Query tiles are scheduled
//   longest first.
//   Global -> register prefetch of the next K/V tile overlaps the MFMA work.
#include <cstdlib>

#include "common.hpp"
#include "kv_view.hpp"

namespace ssa {

struct PrefillParams {
    const uint16_t* q;   // element (b, h, row, d) at b*q_bs + h*q_hs + row*q_rs + d
    int64_t q_bs, q_hs, q_rs;
    KvView kv;           // K/V rows of (b, kv head, token)
    int Hq, G, S, L, off;
    float scale_log2;
    int nqt;             // query tiles of 128 rows
    // drop-in output: f32, element (b, h, row, d) at b*o_bs + h*o_hs + row*o_rs + d
    float* out_f32;
    int64_t o_bs, o_hs, o_rs;
    // fused: bf16 output [S, Hq*D] with the sigmoid gate; Q prologue
    uint16_t* out_bf16;
    const uint16_t* gate;  // element (h, row, d) at h*q_hs + row*q_rs + d (b = 0)
    const uint16_t* q_norm_w;
    const uint16_t* cos_t;
    const uint16_t* sin_t;
    int half_rot;
    float eps;
};

template <typename QT> struct Mfma32;
template <> struct Mfma32<bf16_t> {
    typedef bf16x8_v op;
    static __device__ __forceinline__ f32x16_v mma(const op& a, const op& b, const f32x16_v& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma32<f16_t> {
    typedef f16x8_v op;
    static __device__ __forceinline__ f32x16_v mma(const op& a, const op& b, const f32x16_v& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

template <typename OP>
__device__ __forceinline__ OP to_op(const u32x4_v& w) {
    OP r;
    __builtin_memcpy(&r, &w, 16);
    return r;
}

template <typename QT>
__device__ __forceinline__ uint32_t pk2(float a, float b) {
    return Elem<QT>::from_f32(a) | (Elem<QT>::from_f32(b) << 16);
}

// Position of key w (0..15) inside its 16-key group of the V^T tile: keys
// {0-3, 8-11} first, then {4-7, 12-15}, matching which keys the two lane
// halves hold in the 32x32 C layout.
__device__ __forceinline__ int vperm16(int w) {
    return (w & 3) + 4 * ((w >> 3) & 1) + 8 * ((w >> 2) & 1);
}

template <typename QT, int D, bool FUSED>
__global__ __launch_bounds__(256, 1) void prefill_kernel(PrefillParams p) {
    typedef typename Mfma32<QT>::op op_t;
    constexpr int KS = D / 16;        // QK^T k-steps
    constexpr int DB = D / 32;        // 32-dim output blocks
    constexpr int KROW = D + 8;       // K tile row stride (elements), 16 B pad
    constexpr int VROW = 64 + 8;      // V^T tile row stride (elements)
    constexpr int CPR = D / 8;        // 16-byte chunks per row
    constexpr int LPT = D / 32;       // 16-byte chunks per thread per tile (K and V each)

    __shared__ __attribute__((aligned(16))) uint16_t k_s[64 * KROW];
    __shared__ __attribute__((aligned(16))) uint16_t vt_s[D * VROW];

    const int qt = p.nqt - 1 - static_cast<int>(blockIdx.x);
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / p.G;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5;
    const int q0 = qt * 128;
    const int row_w0 = q0 + 32 * wave;
    const int myrow = row_w0 + (lane & 31);
    const bool row_ok = myrow < p.S;
    const int S = p.S, L = p.L, off = p.off;

    const int lim_wg = min(L, off + min(q0 + 128, S));
    const int ntiles = lim_wg > 0 ? (lim_wg + 63) / 64 : 0;
    const int lim_wave = min(L, off + min(row_w0 + 32, S));
    const int lim_row = min(L, off + myrow + 1);

    // ------------------------------------------------ Q^T operand (registers)
    op_t qb[KS];
    {
        const uint16_t* qrow = p.q + b * p.q_bs + h * p.q_hs + static_cast<int64_t>(row_ok ? myrow : 0) * p.q_rs;
        u32x4_v raw[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            raw[s] = row_ok ? ld16(qrow + 16 * s + 8 * g) : u32x4_v{0u, 0u, 0u, 0u};
        }
        if constexpr (FUSED) {
            // RMSNorm with (1 + w) and rotate-half RoPE at position off + row,
            // bf16 after each step (prefill_engine.rs:2025-2096).  Values stay
            // packed in `raw` between the steps to keep register pressure low.
            float ss = 0.f;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                float x[8];
                unpack8<bf16_t>(raw[s], x);
#pragma unroll
                for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
            }
            ss += __shfl_xor(ss, 32);
            const float inv = rsqrtf(ss / static_cast<float>(D) + p.eps);
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                float x[8], w[8];
                unpack8<bf16_t>(raw[s], x);
                unpack8<bf16_t>(ld16(p.q_norm_w + 16 * s + 8 * g), w);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    raw[s][j] = pk2<bf16_t>(x[2 * j] * inv * (w[2 * j] + 1.0f),
                                            x[2 * j + 1] * inv * (w[2 * j + 1] + 1.0f));
            }
            const int hr = p.half_rot;  // multiple of 16 (checked on the host)
            if (hr > 0 && row_ok) {
                const int pos = off + myrow;
                const int sh = hr / 16;
#pragma unroll
                for (int s = 0; s < KS / 2; ++s) {
                    if (s < sh) {
                        float c[8], sn[8], x0[8], x1[8];
                        unpack8<bf16_t>(ld16(p.cos_t + static_cast<int64_t>(pos) * hr + 16 * s + 8 * g), c);
                        unpack8<bf16_t>(ld16(p.sin_t + static_cast<int64_t>(pos) * hr + 16 * s + 8 * g), sn);
                        unpack8<bf16_t>(raw[s], x0);
                        u32x4_v hi = raw[0];
#pragma unroll
                        for (int s2 = 0; s2 < KS; ++s2)
                            if (s2 == s + sh) hi = raw[s2];
                        unpack8<bf16_t>(hi, x1);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            raw[s][j] = pk2<bf16_t>(x0[2 * j] * c[2 * j] - x1[2 * j] * sn[2 * j],
                                                    x0[2 * j + 1] * c[2 * j + 1] - x1[2 * j + 1] * sn[2 * j + 1]);
                            hi[j] = pk2<bf16_t>(x0[2 * j] * sn[2 * j] + x1[2 * j] * c[2 * j],
                                                x0[2 * j + 1] * sn[2 * j + 1] + x1[2 * j + 1] * c[2 * j + 1]);
                        }
#pragma unroll
                        for (int s2 = 0; s2 < KS; ++s2)
                            if (s2 == s + sh) raw[s2] = hi;
                    }
                }
            }
#pragma unroll
            for (int s = 0; s < KS; ++s) qb[s] = to_op<op_t>(raw[s]);
        } else {
#pragma unroll
            for (int s = 0; s < KS; ++s) qb[s] = to_op<op_t>(raw[s]);
        }
    }

    f32x16_v oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] = 0.f;
    float m_run = -1e30f, l_part = 0.f;

    // ------------------------------------------------ tile loads
    u32x4_v kreg[LPT], vreg[LPT];
    auto load_tile = [&](int k0) {
        const int64_t base = p.kv.row(b, kvh, k0, D);  // tile lies inside one page
        const int last = L - 1 - k0;
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int ci = tid + 256 * i;
            const int tok = min(ci / CPR, last);
            const int c = ci % CPR;
            kreg[i] = ld16(p.kv.k + (base + static_cast<int64_t>(tok) * D + 8 * c) * 2);
        }
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int tok = min(tid & 63, last);
            const int c = (tid >> 6) + 4 * i;
            vreg[i] = ld16(p.kv.v + (base + static_cast<int64_t>(tok) * D + 8 * c) * 2);
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int ci = tid + 256 * i;
            const int tok = ci / CPR;
            const int c = ci % CPR;
            st16(&k_s[tok * KROW + 8 * c], kreg[i]);
        }
        const int tok = tid & 63;
        const int vp = (tok & ~15) + vperm16(tok & 15);
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int c = (tid >> 6) + 4 * i;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vt_s[(8 * c + 2 * e) * VROW + vp] = static_cast<uint16_t>(vreg[i][e] & 0xFFFFu);
                vt_s[(8 * c + 2 * e + 1) * VROW + vp] = static_cast<uint16_t>(vreg[i][e] >> 16);
            }
        }
    };

    if (ntiles > 0) load_tile(0);
    for (int it = 0; it < ntiles; ++it) {
        const int k0 = it * 64;
        __syncthreads();
        store_tile();
        __syncthreads();
        if (it + 1 < ntiles) load_tile(k0 + 64);
        if (k0 >= lim_wave) continue;  // the whole tile is past this wave's rows

        // S^T = K Q^T for the two 32-key blocks.
        f32x16_v sacc[2];
#pragma unroll
        for (int bt = 0; bt < 2; ++bt) {
#pragma unroll
            for (int i = 0; i < 16; ++i) sacc[bt][i] = 0.f;
            const uint16_t* kr = &k_s[(32 * bt + (lane & 31)) * KROW + 8 * g];
#pragma unroll
            for (int s = 0; s < KS; ++s) sacc[bt] = Mfma32<QT>::mma(to_op<op_t>(ld16(kr + 16 * s)), qb[s], sacc[bt]);
        }

        // Online softmax (base 2).  Lane holds row myrow, keys
        // k0 + 32 bt + 8 (i>>2) + 4 g + (i&3).
        const bool need_mask = (k0 + 64 > off + row_w0 + 1) || (k0 + 64 > L);
        float mx = -INFINITY;
#pragma unroll
        for (int bt = 0; bt < 2; ++bt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float v = sacc[bt][i] * p.scale_log2;
                if (need_mask) {
                    const int t = k0 + 32 * bt + 8 * (i >> 2) + 4 * g + (i & 3);
                    if (t >= lim_row) v = -INFINITY;
                }
                sacc[bt][i] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = exp2f(m_run - m_new);
        m_run = m_new;
        float psum = 0.f;
        op_t pk[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            u32x4_v w;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float a = exp2f(sacc[u >> 1][8 * (u & 1) + 2 * j] - m_new);
                const float c = exp2f(sacc[u >> 1][8 * (u & 1) + 2 * j + 1] - m_new);
                psum += a + c;
                w[j] = pk2<QT>(a, c);
            }
            pk[u] = to_op<op_t>(w);
        }
        l_part = l_part * alpha + psum;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;

        // O^T += V^T P^T.
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const uint16_t* vr = &vt_s[(32 * db + (lane & 31)) * VROW + 8 * g];
#pragma unroll
            for (int u = 0; u < 4; ++u) oacc[db] = Mfma32<QT>::mma(to_op<op_t>(ld16(vr + 16 * u)), pk[u], oacc[db]);
        }
    }

    // ------------------------------------------------ epilogue
    const float l_tot = l_part + __shfl_xor(l_part, 32);
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    if (!row_ok) return;
    if constexpr (!FUSED) {
        float* orow = p.out_f32 + b * p.o_bs + h * p.o_hs + static_cast<int64_t>(myrow) * p.o_rs;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int d = 32 * db + 8 * q4 + 4 * g;
                f32x4_v o = {oacc[db][4 * q4] * inv, oacc[db][4 * q4 + 1] * inv, oacc[db][4 * q4 + 2] * inv,
                             oacc[db][4 * q4 + 3] * inv};
                *reinterpret_cast<f32x4_v*>(orow + d) = o;
            }
    } else {
        // bf16(attn) * sigmoid(gate), bf16 out [S, Hq*D] (prefill_engine.rs:2263-2308).
        uint16_t* orow = p.out_bf16 + static_cast<int64_t>(myrow) * p.Hq * D + h * D;
        const uint16_t* grow = p.gate + h * p.q_hs + static_cast<int64_t>(myrow) * p.q_rs;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int d = 32 * db + 8 * q4 + 4 * g;
                const u32x2_v gw = *reinterpret_cast<const u32x2_v*>(grow + d);
                float gv[4] = {bf16_bits_to_f32(gw[0] & 0xFFFFu), bf16_bits_to_f32(gw[0] >> 16),
                               bf16_bits_to_f32(gw[1] & 0xFFFFu), bf16_bits_to_f32(gw[1] >> 16)};
                uint32_t r[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = bf16_round(oacc[db][4 * q4 + e] * inv);
                    r[e] = f32_to_bf16_bits(a * (1.0f / (1.0f + expf(-gv[e]))));
                }
                u32x2_v o = {r[0] | (r[1] << 16), r[2] | (r[3] << 16)};
                *reinterpret_cast<u32x2_v*>(orow + d) = o;
            }
    }
}

// ----------------------------------------------------------------------------
// fp32 prefill (drop-in dtype 1): one wave per query row, online softmax.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prefill_f32_kernel(const float* q, const float* k, const float* v, float* out,
                                                          int B, int Hq, int Hkv, int S, int L, int D, int G,
                                                          float scale, int off) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= B * Hq * S) return;
    const int qp = row % S, h = (row / S) % Hq, b = row / (S * Hq);
    const int kvh = h / G;
    const int lim = min(L, off + qp + 1);
    const float* qr = q + static_cast<int64_t>(row) * D;
    const float* kb = k + (static_cast<int64_t>(b) * Hkv + kvh) * L * D;
    const float* vb = v + (static_cast<int64_t>(b) * Hkv + kvh) * L * D;
    float qv[8], acc[8];
    for (int e = 0; e < 8; ++e) {
        const int d = lane + 64 * e;
        qv[e] = d < D ? qr[d] : 0.f;
        acc[e] = 0.f;
    }
    float m = -1e30f, l = 0.f;
    for (int t = 0; t < lim; ++t) {
        float part = 0.f;
        for (int e = 0; e < 8; ++e) {
            const int d = lane + 64 * e;
            if (d < D) part += qv[e] * kb[static_cast<int64_t>(t) * D + d];
        }
        const float s = wave_sum(part) * scale;
        const float mn = fmaxf(m, s);
        const float a = expf(m - mn), w = expf(s - mn);
        l = l * a + w;
        for (int e = 0; e < 8; ++e) {
            const int d = lane + 64 * e;
            acc[e] = acc[e] * a + (d < D ? w * vb[static_cast<int64_t>(t) * D + d] : 0.f);
        }
        m = mn;
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    for (int e = 0; e < 8; ++e) {
        const int d = lane + 64 * e;
        if (d < D) out[static_cast<int64_t>(row) * D + d] = acc[e] * inv;
    }
}

// ----------------------------------------------------------------------------
// Fused prefill: K RMSNorm + RoPE and the cache write for the chunk's tokens.
// One wave per (token, kv head); the row is staged in a per-wave LDS slot so
// RoPE pairs (i, i + half_rot) can be any distance apart.
// ----------------------------------------------------------------------------
struct KvPrepParams {
    const uint16_t* k_new;  // [S, Hkv*D]
    const uint16_t* v_new;
    const uint16_t* k_norm_w;
    const uint16_t* cos_t;
    const uint16_t* sin_t;
    KvView kv;
    int S, Hkv, D, off, half_rot, fp8;
    float eps;
};

__global__ __launch_bounds__(256) void kv_prep_kernel(KvPrepParams p) {
    __shared__ float rows_s[4][2][512];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + wave;
    if (row >= p.S * p.Hkv) return;
    const int s = row / p.Hkv, h = row % p.Hkv;
    const int D = p.D;
    float* kr = rows_s[wave][0];
    float* vr = rows_s[wave][1];
    const uint16_t* ksrc = p.k_new + static_cast<int64_t>(row) * D;
    const uint16_t* vsrc = p.v_new + static_cast<int64_t>(row) * D;
    float ss = 0.f;
    for (int d = lane; d < D; d += 64) {
        const float x = bf16_bits_to_f32(ksrc[d]);
        kr[d] = x;
        ss += x * x;
        vr[d] = bf16_bits_to_f32(vsrc[d]);
    }
    ss = wave_sum(ss);
    const float inv = rsqrtf(ss / static_cast<float>(D) + p.eps);
    for (int d = lane; d < D; d += 64) kr[d] = bf16_round(kr[d] * inv * (bf16_bits_to_f32(p.k_norm_w[d]) + 1.0f));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int pos = p.off + s;
    const int hr = p.half_rot;
    float r0[4], r1[4];
    int nr = 0;
    for (int i = lane; i < hr; i += 64) {
        const float c = bf16_bits_to_f32(p.cos_t[static_cast<int64_t>(pos) * hr + i]);
        const float sn = bf16_bits_to_f32(p.sin_t[static_cast<int64_t>(pos) * hr + i]);
        const float x0 = kr[i], x1 = kr[i + hr];
        r0[nr] = bf16_round(x0 * c - x1 * sn);
        r1[nr] = bf16_round(x0 * sn + x1 * c);
        ++nr;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    nr = 0;
    for (int i = lane; i < hr; i += 64) {
        kr[i] = r0[nr];
        kr[i + hr] = r1[nr];
        ++nr;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int64_t o = p.kv.row(0, h, pos, D);
    if (!p.fp8) {
        uint16_t* kc = reinterpret_cast<uint16_t*>(p.kv.k) + o;
        uint16_t* vc = reinterpret_cast<uint16_t*>(p.kv.v) + o;
        for (int d = lane; d < D; d += 64) {
            kc[d] = static_cast<uint16_t>(f32_to_bf16_bits(kr[d]));
            vc[d] = static_cast<uint16_t>(f32_to_bf16_bits(vr[d]));
        }
    } else {
        for (int which = 0; which < 2; ++which) {
            const float* src = which ? vr : kr;
            uint8_t* dst = (which ? p.kv.v : p.kv.k) + o;
            float am = 0.f;
            for (int d = lane; d < D; d += 64) am = fmaxf(am, fabsf(src[d]));
            am = wave_max(am);
            const float sc = fmaxf(am / 448.0f, 1e-12f);
            const float iv = 1.0f / sc;
            for (int d = lane * 4; d < D; d += 256) {
                *reinterpret_cast<uint32_t*>(dst + d) =
                    f32x4_to_fp8x4(src[d] * iv, src[d + 1] * iv, src[d + 2] * iv, src[d + 3] * iv);
            }
            if (lane == 0) (which ? p.kv.vs : p.kv.ks)[p.kv.srow(0, h, pos)] = sc;
        }
    }
}

// ----------------------------------------------------------------------------
// Host side
// ----------------------------------------------------------------------------
template <typename QT, bool FUSED>
static hipError_t launch_prefill(int D, dim3 grid, hipStream_t st, const PrefillParams& p) {
    switch (D) {
    case 64: hipLaunchKernelGGL((prefill_kernel<QT, 64, FUSED>), grid, dim3(256), 0, st, p); break;
    case 128: hipLaunchKernelGGL((prefill_kernel<QT, 128, FUSED>), grid, dim3(256), 0, st, p); break;
    case 256: hipLaunchKernelGGL((prefill_kernel<QT, 256, FUSED>), grid, dim3(256), 0, st, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

static int prefill_dropin(int dtype, size_t device, size_t B, size_t Hq, size_t Hkv, size_t q_len, size_t kv_len,
                          size_t D, size_t groups, float scale, size_t off, const void* q, const void* k,
                          const void* v, void* out) {
    if (dtype != 0 && dtype != 1 && dtype != 2) return 64;
    if (D == 0 || D > 512 || Hkv == 0 || groups == 0 || Hq != Hkv * groups) return 14;
    if (dtype != 1 && D != 64 && D != 128 && D != 256) return 14;
    ScopedDevice scoped(static_cast<int>(device));
    if (B == 0 || Hq == 0 || q_len == 0) return hipDeviceSynchronize() == hipSuccess ? 0 : 12;
    if (dtype == 1) {
        const size_t rows = B * Hq * q_len;
        hipLaunchKernelGGL(prefill_f32_kernel, dim3(grid1d(rows, 4)), dim3(256), 0, 0,
                           static_cast<const float*>(q), static_cast<const float*>(k), static_cast<const float*>(v),
                           static_cast<float*>(out), static_cast<int>(B), static_cast<int>(Hq),
                           static_cast<int>(Hkv), static_cast<int>(q_len), static_cast<int>(kv_len),
                           static_cast<int>(D), static_cast<int>(groups), scale, static_cast<int>(off));
        if (hipGetLastError() != hipSuccess) return 11;
        if (hipDeviceSynchronize() != hipSuccess) return 12;
        return 0;
    }
    PrefillParams p{};
    p.q = static_cast<const uint16_t*>(q);
    p.q_rs = static_cast<int64_t>(D);
    p.q_hs = static_cast<int64_t>(q_len) * D;
    p.q_bs = static_cast<int64_t>(Hq) * q_len * D;
    p.kv.k = static_cast<uint8_t*>(const_cast<void*>(k));
    p.kv.v = static_cast<uint8_t*>(const_cast<void*>(v));
    p.kv.page_size = 1;
    p.kv.head_stride = static_cast<int64_t>(kv_len) * D;
    p.kv.seq_stride = static_cast<int64_t>(Hkv) * kv_len * D;
    p.Hq = static_cast<int>(Hq);
    p.G = static_cast<int>(groups);
    p.S = static_cast<int>(q_len);
    p.L = static_cast<int>(kv_len);
    p.off = static_cast<int>(off);
    p.scale_log2 = scale * kLog2e;
    p.nqt = static_cast<int>((q_len + 127) / 128);
    p.out_f32 = static_cast<float*>(out);
    p.o_rs = p.q_rs;
    p.o_hs = p.q_hs;
    p.o_bs = p.q_bs;
    dim3 grid(p.nqt, static_cast<unsigned>(Hq), static_cast<unsigned>(B));
    const hipError_t e = dtype == 0 ? launch_prefill<f16_t, false>(static_cast<int>(D), grid, nullptr, p)
                                    : launch_prefill<bf16_t, false>(static_cast<int>(D), grid, nullptr, p);
    if (e != hipSuccess) return 11;
    if (hipDeviceSynchronize() != hipSuccess) return 12;
    return 0;
}

}  // namespace ssa

using namespace ssa;

extern "C" int supersonic_qwen35_hip_full_attention_prefill(
    int dtype, size_t device_ordinal, size_t batch_size, size_t q_heads, size_t kv_heads, size_t q_len,
    size_t kv_len, size_t head_dim, size_t num_kv_groups, float scale, size_t seqlen_offset, const void* query,
    const void* key, const void* value, void* out) {
    return prefill_dropin(dtype, device_ordinal, batch_size, q_heads, kv_heads, q_len, kv_len, head_dim,
                          num_kv_groups, scale, seqlen_offset, query, key, value, out);
}

extern "C" int supersonic_qwen35_4b_hip_full_attention_prefill(
    int dtype, size_t device_ordinal, size_t batch_size, size_t q_heads, size_t kv_heads, size_t q_len,
    size_t kv_len, size_t head_dim, size_t num_kv_groups, float scale, size_t seqlen_offset, const void* query,
    const void* key, const void* value, void* out) {
    return prefill_dropin(dtype, device_ordinal, batch_size, q_heads, kv_heads, q_len, kv_len, head_dim,
                          num_kv_groups, scale, seqlen_offset, query, key, value, out);
}

extern "C" int supersonic_attn_gfx950_prefill(
    size_t device_ordinal, void* stream, int kv_dtype, size_t q_heads, size_t kv_heads, size_t head_dim,
    size_t rotary_dim, size_t chunk_len, size_t chunk_start, float eps, float scale, const void* q_proj,
    const void* k_new, const void* v_new, const void* q_norm_w, const void* k_norm_w, const void* cos_table,
    const void* sin_table, const supersonic_kv_cache* cache, void* out) {
    if (kv_dtype != SUPERSONIC_KV_BF16) return SUPERSONIC_ERR_DTYPE;  // fp8 lane: not yet
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return SUPERSONIC_ERR_HEAD_DIM;
    if (kv_heads == 0 || q_heads % kv_heads != 0) return SUPERSONIC_ERR_HEADS;
    if (rotary_dim > head_dim || (rotary_dim / 2) % 16 != 0) return SUPERSONIC_ERR_ROTARY;
    if (!q_proj || !k_new || !v_new || !q_norm_w || !k_norm_w || !out) return SUPERSONIC_ERR_NULL;
    if (rotary_dim > 0 && (!cos_table || !sin_table)) return SUPERSONIC_ERR_NULL;
    if (chunk_len + chunk_start > 0x7FFFFFFF || q_heads > 4096) return SUPERSONIC_ERR_RANGE;
    KvView kv;
    if (int rc = make_view(cache, false, &kv)) return rc;
    if (kv.bt && kv.page_size % 64 != 0) return SUPERSONIC_ERR_CACHE;
    if (chunk_len == 0) return 0;
    ScopedDevice scoped(static_cast<int>(device_ordinal));
    hipStream_t st = static_cast<hipStream_t>(stream);

    KvPrepParams kp{};
    kp.k_new = static_cast<const uint16_t*>(k_new);
    kp.v_new = static_cast<const uint16_t*>(v_new);
    kp.k_norm_w = static_cast<const uint16_t*>(k_norm_w);
    kp.cos_t = static_cast<const uint16_t*>(cos_table);
    kp.sin_t = static_cast<const uint16_t*>(sin_table);
    kp.kv = kv;
    kp.S = static_cast<int>(chunk_len);
    kp.Hkv = static_cast<int>(kv_heads);
    kp.D = static_cast<int>(head_dim);
    kp.off = static_cast<int>(chunk_start);
    kp.half_rot = static_cast<int>(rotary_dim / 2);
    kp.fp8 = 0;
    kp.eps = eps;
    hipLaunchKernelGGL(kv_prep_kernel, dim3(grid1d(chunk_len * kv_heads, 4)), dim3(256), 0, st, kp);
    if (hipGetLastError() != hipSuccess) return SUPERSONIC_ERR_LAUNCH;

    PrefillParams p{};
    p.q = static_cast<const uint16_t*>(q_proj);
    p.q_bs = 0;
    p.q_hs = 2 * static_cast<int64_t>(head_dim);
    p.q_rs = static_cast<int64_t>(q_heads) * 2 * head_dim;
    p.kv = kv;
    p.Hq = static_cast<int>(q_heads);
    p.G = static_cast<int>(q_heads / kv_heads);
    p.S = static_cast<int>(chunk_len);
    p.L = static_cast<int>(chunk_start + chunk_len);
    p.off = static_cast<int>(chunk_start);
    p.scale_log2 = scale * kLog2e;
    p.nqt = static_cast<int>((chunk_len + 127) / 128);
    p.out_bf16 = static_cast<uint16_t*>(out);
    p.gate = static_cast<const uint16_t*>(q_proj) + head_dim;
    p.q_norm_w = static_cast<const uint16_t*>(q_norm_w);
    p.cos_t = static_cast<const uint16_t*>(cos_table);
    p.sin_t = static_cast<const uint16_t*>(sin_table);
    p.half_rot = static_cast<int>(rotary_dim / 2);
    p.eps = eps;
    dim3 grid(p.nqt, static_cast<unsigned>(q_heads), 1);
    const ProfileEvents prof = take_profile_events();
    if (prof.before) (void)hipEventRecord(prof.before, st);
    if (launch_prefill<bf16_t, true>(static_cast<int>(head_dim), grid, st, p) != hipSuccess)
        return SUPERSONIC_ERR_LAUNCH;
    if (prof.after) (void)hipEventRecord(prof.after, st);
    return 0;
}
