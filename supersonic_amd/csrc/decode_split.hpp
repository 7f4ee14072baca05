// Split-K decode attention: parameters, device helpers and the kernel body as
// a device function, shared by the standalone split kernel (decode.hip) and
// the persistent decode layer (layer.hip).
#pragma once

#include <type_traits>
#include <utility>

#include "common.hpp"
#include "kv_view.hpp"

namespace ssa {

struct DecodeParams {
    KvView kv;
    const uint16_t* q;        // attend: q [B, Hq, D]; fused: q_proj [B, Hq*2D]
    int64_t q_bstride;        // elements between batch rows of q
    int64_t q_hstride;        // elements between heads of q
    const int32_t* lens;      // kv_lens [B] (attend) or positions [B] (fused)
    int len_plus;             // 0 (attend) or 1 (fused: len = position + 1)
    int Hq, Hkv, G, chunk, nsplit;
    // Ragged plan (ragged != 0): the workgroups of a 1-D grid split the batch's
    // total length into chunks of about total * Hkv / target tokens, so every
    // workgroup gets about the same number of tokens whatever the lengths;
    // chunk and nsplit are then unused.
    int ragged, B, target, min_chunk;
    // 1: the grid has exactly `target` workgroups (the persistent layer), so
    // the plan must not exceed target items: if the chunk growth below has
    // not got there, every sequence takes one split (B * Hkv <= target is
    // checked on the host).  0: the grid holds target + B * Hkv workgroups.
    int strict;
    int det;                  // 1: static block order (bit-reproducible), 0: blocks claimed from an LDS counter
    float scale_log2;         // softmax scale * log2(e)
    int fused;
    const uint16_t* k_new;    // [B, Hkv*D] bf16
    const uint16_t* v_new;
    const uint16_t* q_norm_w; // [D] bf16
    const uint16_t* k_norm_w;
    const uint16_t* cos_t;    // [max_pos, half_rot] bf16
    const uint16_t* sin_t;
    int half_rot;
    float eps;
    float* part_o;            // [rows, D], row of (b, h, split) = pre_b * Hq + h * n_b + split
    float* part_ml;           // [rows, 2] (max in log2 units, sum)
    unsigned* arrivals;       // [B, Hkv] split arrival counters, zero between calls
    int arr_stride;           // words between two counters (each on its own cache line when it fits)
    int merge_polls;          // bound of the merge's poll for partials in flight (kMergePoll)
    const uint16_t* gate;     // NULL, or gate element (b, h, d) at b*g_bstride + h*g_hstride + d
    int64_t g_bstride, g_hstride;
    void* out;                // [B, Hq*D] of QT
};

template <typename QT> struct Mfma;
template <> struct Mfma<bf16_t> {
    typedef bf16x8_v op;
    static __device__ __forceinline__ f32x4_v mma(const op& a, const op& b, const f32x4_v& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4_v mma16(const s16x4_v& a, const s16x4_v& b, const f32x4_v& c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<f16_t> {
    typedef f16x8_v op;
    static __device__ __forceinline__ f32x4_v mma(const op& a, const op& b, const f32x4_v& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4_v mma16(const s16x4_v& a, const s16x4_v& b, const f32x4_v& c) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, a), __builtin_bit_cast(h4, b), c, 0, 0, 0);
    }
};

template <typename OP>
__device__ __forceinline__ OP as_op(const u32x4_v& w) {
    OP r;
    __builtin_memcpy(&r, &w, 16);
    return r;
}

// 8 e4m3 bytes -> 8 bf16 (exact: every e4m3 value is a bf16 value), two
// bytes per gfx950 v_cvt_scalef32_pk_bf16_fp8 at scale 1.
__device__ __forceinline__ u32x4_v fp8x8_to_bf16x8(u32x2_v w) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    u32x4_v r;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        r[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[i], 1.0f, false));
        r[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[i], 1.0f, true));
    }
    return r;
}

// First of the 8 consecutive dims that lane group g (= lane >> 4) holds in
// QK^T k-step s, for Q (A operand) and K (B operand) alike: 32 s + 8 g for
// 16-bit K; for e4m3 K a lane loads 16 dims (16 bytes) at once, so k-steps
// 2 ss and 2 ss + 1 take the two halves: 64 ss + 16 g + 8 (s & 1).
template <bool FP8>
__device__ __forceinline__ constexpr int kdim(int s, int g) {
    return FP8 ? 64 * (s >> 1) + 16 * g + 8 * (s & 1) : 32 * s + 8 * g;
}

// Buffer resource for a base that is uniform across the wave (forced into
// SGPRs: it can come from a block-table load the compiler cannot prove
// uniform).  Reads at or past `bytes` return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const uint8_t* base, int bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
    void* u = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, static_cast<short>(0), bytes, 0x00020000);
}

template <typename QT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return Elem<QT>::from_f32(a) | (Elem<QT>::from_f32(b) << 16);
}

// Waves per workgroup: 8 for head groups up to 4 (one workgroup per CU, two
// waves per SIMD at up to 256 registers); the larger groups need more
// registers and run 4 (two workgroups per CU for 8, one for 16).
__host__ __device__ constexpr int decode_waves(int GP) { return GP <= 4 ? 8 : 4; }

// LDS of one split workgroup (a caller that runs other phases in the same
// workgroup overlays it with theirs).
template <int D, int GP>
struct DecodeLds {
    static constexpr int NW = decode_waves(GP);
    float smem[NW * GP * D];        // q staging, then the wave merge
    float kn_s[D], vn_s[D];         // the new token (fused owner split)
    float ml_s[NW][GP][2];
    u32x4_v qop_s[(D / 32) * 64];   // Q as the MFMA A operand
    int next_blk;                   // next 16-token block to claim
    int plan_s[8];
    int last_s;
};

// One split workgroup: work item (vbx, vby, vbz) = (split, kv head, sequence)
// in the uniform plan, or item vbx of the ragged plan.  COH: q / k_new / v_new
// / gate are read and the output written with device-coherent accesses (they
// are exchanged with other workgroups of the same kernel).
struct NoMid {
    __device__ void operator()() const {}
};

// mid: called by every thread once, after the work item is planned and its
// first K/V block fetched, before q / k_new / v_new / gate are read (not
// called when the workgroup has no work item).
template <typename QT, bool FP8, int D, int GP, bool COH = false, typename Mid = NoMid>
__device__ __forceinline__ void decode_split_body(const DecodeParams& p, int vbx, int vby, int vbz,
                                                  DecodeLds<D, GP>& L, const Mid& mid = Mid()) {
    constexpr bool kMid = !std::is_same<Mid, NoMid>::value;
    static_assert(D % 64 == 0 && D <= 512, "head_dim");
    static_assert(GP == 4 || GP == 8 || GP == 16, "padded group");
    static_assert(decode_waves(GP) * GP >= 16, "smem holds the 16 padded Q rows");
    typedef typename Mfma<QT>::op op_t;
    constexpr int KSTEPS = D / 32;
    constexpr int ESZ = FP8 ? 1 : 2;
    constexpr int VQD = D / 16;      // V dims per lane and token (PV A operand)
    constexpr int VQW = VQD * ESZ / 4;  // ... in 32-bit words
    constexpr int VCE = 16 / ESZ;       // elements of a 16-byte chunk
    auto vdim = [](int w, int q, int m) {
        if constexpr (VQW >= 4) return (w / (VCE / 4)) * 16 * VCE + VCE * m + 4 * (w % (VCE / 4)) + q;
        else return VQD * m + 4 * w + q;
    };

    constexpr int NW = decode_waves(GP);
    constexpr int NT = 64 * NW;
    float (&smem)[NW * GP * D] = L.smem;
    float (&kn_s)[D] = L.kn_s;
    float (&vn_s)[D] = L.vn_s;
    float (&ml_s)[NW][GP][2] = L.ml_s;
    int& next_blk = L.next_blk;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Work item (b, kv head, split), chunk length, and the partial rows of
    // sequence b: pre_b splits before it, n_b of its own per head.
    int split, kvh, b, chunk, n_b, len;
    int64_t pre_b;
    if (p.ragged) {
        // Every workgroup plans the same way from the lengths: chunk =
        // ceil(total * Hkv / target) rounded up to 16 (at least min_chunk),
        // sequence b gets n_b = max(1, ceil(len_b / chunk)) splits per kv
        // head, each of them ceil(len_b / n_b) tokens (rounded up to 16), items
        // are ordered (b, kv head, split), and workgroup i takes item i (past
        // the last item it has nothing to do).
        int (&plan_s)[8] = L.plan_s;
        if (wave == 0) {
            // Up to 64 sequences (the usual case) the lengths are loaded once
            // and kept in a register: every pass below would otherwise be
            // another dependent load.
            const bool one = p.B <= 64;
            const int l0 = lane < p.B ? max(p.lens[lane] + p.len_plus, 0) : 0;
            auto len_of = [&](int bi) { return one ? l0 : (bi < p.B ? max(p.lens[bi] + p.len_plus, 0) : 0); };
            int64_t tot = 0;
            for (int b0 = 0; b0 < p.B; b0 += 64) tot += len_of(b0 + lane);
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) tot += __shfl_xor(tot, o);
            // Per-sequence rounding can push the item count past the target
            // (a second, mostly idle round): grow the chunk in proportion
            // until the items fit (a few passes; uniform lengths need none).
            int64_t c = (tot * p.Hkv + p.target - 1) / p.target;
            c = max((c + 15) / 16 * 16, static_cast<int64_t>(p.min_chunk));
            bool fits = false;
            for (int pass = 0; pass < 5; ++pass) {
                int64_t items = 0;
                for (int b0 = 0; b0 < p.B; b0 += 64) {
                    const int bi = b0 + lane;
                    const int64_t l = len_of(bi);
                    items += bi < p.B ? max(static_cast<int64_t>(1), (l + c - 1) / c) : 0;
                }
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) items += __shfl_xor(items, o);
                items *= p.Hkv;
                fits = items <= p.target;
                if (fits || pass == 4) break;
                c = (c * items + p.target - 1) / p.target;
                c = (c + 15) / 16 * 16;
            }
            if (p.strict && !fits) {
                // four growth steps did not get there: one split per sequence
                int64_t mx = 0;
                for (int b0 = 0; b0 < p.B; b0 += 64) mx = max(mx, static_cast<int64_t>(len_of(b0 + lane)));
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) mx = max(mx, __shfl_xor(mx, o));
                c = max(c, (mx + 15) / 16 * 16);
            }
            const int ch = static_cast<int>(c);
            if (lane == 0) plan_s[0] = -1;
            const int w = vbx;
            int run = 0, run_n = 0;  // items and splits of the sequences before b0
            for (int b0 = 0; b0 < p.B; b0 += 64) {
                const int bi = b0 + lane;
                const int l = len_of(bi);
                const int n = bi < p.B ? max(1, (l + ch - 1) / ch) : 0;
                int incl = n;        // inclusive scan of the split counts
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const int t = __shfl_up(incl, o);
                    if (lane >= o) incl += t;
                }
                const int first = run + (incl - n) * p.Hkv;  // first item of sequence bi
                if (bi < p.B && w >= first && w < first + n * p.Hkv) {
                    plan_s[0] = bi;
                    plan_s[1] = (w - first) / n;
                    plan_s[2] = (w - first) % n;
                    plan_s[3] = n;
                    plan_s[4] = run_n + incl - n;
                    // the sequence's n splits share its length equally (16-token
                    // blocks), so no split is left with a short remainder
                    plan_s[5] = l > 0 ? ((l + n - 1) / n + 15) / 16 * 16 : ch;
                    plan_s[6] = l;
                }
                const int tot_n = __shfl(incl, 63);
                run += tot_n * p.Hkv;
                run_n += tot_n;
            }
        }
        __syncthreads();
        b = plan_s[0];
        if (b < 0) return;  // uniform
        kvh = plan_s[1];
        split = plan_s[2];
        n_b = plan_s[3];
        pre_b = plan_s[4];
        chunk = plan_s[5];
        len = plan_s[6];
    } else {
        split = vbx;
        kvh = vby;
        b = vbz;
        chunk = p.chunk;
        n_b = p.nsplit;
        pre_b = static_cast<int64_t>(b) * p.nsplit;
        len = p.lens[b] + p.len_plus;
    }
    const int t_begin = split * chunk;
    if (t_begin >= len) {  // uniform: ragged batch, nothing to do
        if (len <= 0 && split == 0) {
            // No tokens at all: the output is zero (what the merge of no splits gives).
            for (int idx = tid; idx < p.G * D; idx += NT) {
                const int h = kvh * p.G + idx / D;
                if constexpr (COH) store_f32_agent(static_cast<QT*>(p.out), (static_cast<int64_t>(b) * p.Hq + h) * D + idx % D, 0.f);
                else store_f32(static_cast<QT*>(p.out), (static_cast<int64_t>(b) * p.Hq + h) * D + idx % D, 0.f);
            }
        }
        return;
    }
    const int t_end = min(len, t_begin + chunk);
    const int ns = (len + chunk - 1) / chunk;  // splits that hold tokens (<= n_b)
    const int G = p.G;
    const int pos = len - 1;
    const bool owner = p.fused && pos >= t_begin && pos < t_end;
    // This split's partial slots go to zero before any of its loads is
    // issued: a slot may still hold a partial of an earlier call, and the
    // merge polls for non-zero words.  A wave waits for its own row loads
    // (issued after these stores; vmcnt drains in issue order) before the
    // split can arrive, so the zeros have landed by then.  Wave hh owns head
    // row hh (the wave that stores the partial later), wave 0 the (M, L) words.
    {
        constexpr int DVz = D / 64;
        for (int hh = wave; hh < G; hh += NW)
            st_coh<DVz>(p.part_o + (pre_b * p.Hq + static_cast<int64_t>(kvh * G + hh) * n_b + split) * D,
                        lane * DVz * 4, typename U32N<DVz>::t{});
        if (wave == 0 && lane < G)
            __hip_atomic_store(reinterpret_cast<uint64_t*>(
                                   &p.part_ml[2 * (pre_b * p.Hq + static_cast<int64_t>(kvh * G + lane) * n_b + split)]),
                               uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    const int n_s = lane & 15;           // score lane: token within the block
    // Cached tokens of this split; the owner's new token (the last one) is
    // handled after the loop.
    const int t_main = owner ? pos : t_end;
    const int nblk = (t_main - t_begin + 15) >> 4;
    const uint8_t* kbase = p.kv.k;
    const uint8_t* vbase = p.kv.v;

    // Block data of one 16-token block, loaded one block ahead (registers).
    struct Blk {
        op_t kb[FP8 ? 1 : KSTEPS];
        u32x4_v kr8[FP8 ? KSTEPS / 2 : 1];  // raw e4m3 K, 16 dims a load: converted when the block is processed
        uint32_t vq[4][VQW];                // V of token 4(lane>>4)+j, the dims vdim(., ., lane&15)
        float ksc, vsc;
    };
    // Buffer resources bound to the block's live rows (a block lies inside one
    // page): rows past kv_len read as zeros, so every load is one per-lane
    // offset plus a constant, with no per-load clamping.
    const int k_lane_off = n_s * D * ESZ + kdim<FP8>(0, lane >> 4) * ESZ;
    // Cache policy of the K/V loads: nontemporal for 16-bit caches (every
    // byte is read once; 6.0 -> 7.1 TB/s for the 8-wave kernel's access
    // pattern on MI355X; the 4-wave kernels measured the same either way);
    // the e4m3 kernel measured faster without it (59.5 against 63 us at
    // config 4).
    constexpr int kStream = FP8 ? 0 : 2;
    // V as the PV MFMA's A operand: a lane's V bytes of a token are 16-byte chunks, chunk c
    // at 16 (lane & 15) + 256 c, so each load instruction reads 256
    // consecutive bytes of the row across 16 lanes; vdim maps (4-dim group w,
    // q, row m) of the A operand to the dim the lane holds there.
    const int vq_lane_off = 4 * (lane >> 4) * D * ESZ + (VQW >= 4 ? 16 : VQD * ESZ) * (lane & 15);
    auto fetch = [&](int blk, Blk& B) {
        const int t0 = t_begin + blk * 16;
        // The page comes through the scalar cache (lgkmcnt): waiting for it
        // does not wait for the other block's vector loads still in flight.
        const int ub = __builtin_amdgcn_readfirstlane(b), uk = __builtin_amdgcn_readfirstlane(kvh);
        const int ut = __builtin_amdgcn_readfirstlane(t0);
        const int64_t base = p.kv.row_uniform(ub, uk, ut, D);
        const int nvalid = __builtin_amdgcn_readfirstlane(max(0, min(16, t_main - t0)));  // wave-uniform
        const __amdgpu_buffer_rsrc_t kr = uniform_rsrc(kbase + base * ESZ, nvalid * D * ESZ);
        const __amdgpu_buffer_rsrc_t vr = uniform_rsrc(vbase + base * ESZ, nvalid * D * ESZ);
        // K as the QK^T MFMA's A operand: row = token n_s, k = dims kdim(s, lane>>4) + j.
        if constexpr (!FP8) {
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s)
                B.kb[s] = as_op<op_t>(__builtin_bit_cast(u32x4_v, __builtin_amdgcn_raw_buffer_load_b128(kr, k_lane_off + 64 * s, 0, kStream)));
        } else {
            // raw bytes only, 16 per lane: converted when the block is processed
#pragma unroll
            for (int ss = 0; ss < KSTEPS / 2; ++ss)
                B.kr8[ss] = __builtin_bit_cast(u32x4_v, __builtin_amdgcn_raw_buffer_load_b128(kr, k_lane_off + 64 * ss, 0, kStream));
        }
        {
            // the lane's four token rows 4(lane>>4) .. +3, VQD dims each;
            // 16 lanes cover a row
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (VQW >= 4) {
#pragma unroll
                    for (int c = 0; c < VQW / 4; ++c) {
                        const u32x4_v w = __builtin_bit_cast(u32x4_v, __builtin_amdgcn_raw_buffer_load_b128(vr, vq_lane_off + 256 * c, j * D * ESZ, kStream));
#pragma unroll
                        for (int e = 0; e < 4; ++e) B.vq[j][4 * c + e] = w[e];
                    }
                } else if constexpr (VQW == 2) {
                    const u32x2_v w = __builtin_bit_cast(u32x2_v, __builtin_amdgcn_raw_buffer_load_b64(vr, vq_lane_off, j * D * ESZ, kStream));
                    B.vq[j][0] = w[0];
                    B.vq[j][1] = w[1];
                } else {
                    B.vq[j][0] = __builtin_amdgcn_raw_buffer_load_b32(vr, vq_lane_off, j * D * ESZ, kStream);
                }
            }
        }
        B.ksc = 1.f;
        B.vsc = 1.f;
        if constexpr (FP8) {
            const int64_t sb = p.kv.srow_uniform(ub, uk, ut);
            const int kn = max(0, min(n_s, nvalid - 1));  // nvalid is 0 when a split holds only the new token
            B.ksc = p.kv.ks[sb + kn];
            B.vsc = p.kv.vs[sb + kn];
        }
    };

    Blk A, Bn;  // the block register sets (A's first fetch is issued in the prologue)
    // ---------------------------------------------------------------- prologue
    if (tid == 0) next_blk = NW;  // blocks 0 .. NW-1 are the waves' first
    // One wave per row: rows 0 .. G-1 are the q heads, row G (owner split of
    // the fused step) is the new k (with v alongside).  Lane l holds dims
    // l + 64 k.  All global loads of a row go out before any arithmetic, so the
    // prologue costs one memory round trip.
    {
        constexpr int EPL = D / 64;
        const int hr = p.fused ? p.half_rot : 0;
        const int rows = G + (owner ? 1 : 0);
        // A row's global loads (q head, or the new k with v), clamped to a real
        // row so they need no branch.
        auto row_loads = [&](const int r, float (&x)[EPL], float (&vx)[EPL], float (&w)[EPL], float (&cs)[EPL],
                             float (&sn)[EPL]) {
            // Branch-free: every pointer is chosen per wave (an absent input is
            // replaced by the row itself, a valid address whose value is then
            // ignored) and every index is clamped, so the row's loads go out
            // back to back and one wait covers them all.
            const bool is_k = r == G;
            const uint16_t* qrow = reinterpret_cast<const uint16_t*>(p.q) + b * p.q_bstride +
                                   static_cast<int64_t>(kvh * G + min(r, G - 1)) * p.q_hstride;
            const int64_t ko = (static_cast<int64_t>(b) * p.Hkv + kvh) * D;
            const uint16_t* xsrc = is_k ? p.k_new + ko : qrow;
            const uint16_t* vsrc = is_k ? p.v_new + ko : qrow;
            const uint16_t* wsrc = p.fused ? (is_k ? p.k_norm_w : p.q_norm_w) : qrow;
            const uint16_t* ctab = hr > 0 ? p.cos_t + static_cast<int64_t>(pos) * hr : qrow;
            const uint16_t* stab = hr > 0 ? p.sin_t + static_cast<int64_t>(pos) * hr : qrow;
            uint32_t xr[EPL], vr[EPL], wr[EPL], cr[EPL], sr[EPL];
#pragma unroll
            for (int k = 0; k < EPL; ++k) {
                const int d = lane + 64 * k;
                const int ti = d < hr ? d : (d < 2 * hr ? d - hr : 0);
                xr[k] = COH ? load_agent_u16(xsrc + d) : xsrc[d];
                vr[k] = COH ? load_agent_u16(vsrc + d) : vsrc[d];
                wr[k] = wsrc[d];
                cr[k] = ctab[ti];
                sr[k] = stab[ti];
            }
#pragma unroll
            for (int k = 0; k < EPL; ++k) {
                const int d = lane + 64 * k;
                x[k] = is_k ? bf16_bits_to_f32(xr[k]) : Elem<QT>::to_f32(xr[k]);
                vx[k] = bf16_bits_to_f32(vr[k]);
                w[k] = bf16_bits_to_f32(wr[k]);
                const bool rot = d < 2 * hr;
                cs[k] = rot ? bf16_bits_to_f32(cr[k]) : 0.f;
                sn[k] = rot ? bf16_bits_to_f32(sr[k]) : 0.f;
            }
        };
        auto row_compute = [&](const int r, float (&x)[EPL], float (&vx)[EPL], float (&w)[EPL], float (&cs)[EPL],
                               float (&sn)[EPL]) {
            const bool is_k = r == G;
            float* row = is_k ? kn_s : &smem[r * D];
            if (p.fused) {
                // Per-head RMSNorm with (1 + w), bf16 result (full_attention_4b.hip:5142-5191).
                float ss = 0.f;
#pragma unroll
                for (int k = 0; k < EPL; ++k) ss += x[k] * x[k];
                ss = wave_sum(ss);
                const float inv = rsqrtf(ss / static_cast<float>(D) + p.eps);
#pragma unroll
                for (int k = 0; k < EPL; ++k) x[k] = bf16_round(x[k] * inv * (w[k] + 1.0f));
                // Rotate-half partial RoPE at the new token's position (:5193-5224);
                // the partner of dim d < 2 hr is d +- hr, read from the row in LDS.
                if (hr > 0) {
#pragma unroll
                    for (int k = 0; k < EPL; ++k) row[lane + 64 * k] = x[k];
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                    for (int k = 0; k < EPL; ++k) {
                        const int d = lane + 64 * k;
                        if (d < 2 * hr) {
                            const float other = row[d < hr ? d + hr : d - hr];
                            x[k] = d < hr ? bf16_round(x[k] * cs[k] - other * sn[k])
                                          : bf16_round(other * sn[k] + x[k] * cs[k]);
                        }
                    }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                }
            }
#pragma unroll
            for (int k = 0; k < EPL; ++k) {
                row[lane + 64 * k] = x[k];
                if (is_k) vn_s[lane + 64 * k] = vx[k];
            }
        };
        // Rows past the first NW (large head groups) first, then this wave's
        // first row, then the wave's first K/V block: waiting for the row
        // (vmcnt drains in issue order) does not wait for the block, whose
        // round trip overlaps the norm and RoPE.  No load may follow the
        // block's before its use: a later load whose register is reused
        // would make the compiler wait for the block too.
        // With a mid hook (the persistent layer), the first K/V block is
        // fetched and the hook (a grid barrier: q, k_new and v_new are
        // written by another phase) runs before any of the rows is read.
        if constexpr (kMid) {
            fetch(max(0, min(wave, nblk - 1)), A);
            mid();
        }
        for (int r = wave + NW; r < rows; r += NW) {
            float x[EPL], vx[EPL], w[EPL], cs[EPL], sn[EPL];
            row_loads(r, x, vx, w, cs, sn);
            row_compute(r, x, vx, w, cs, sn);
        }
        if constexpr (!kMid) {
            float x[EPL], vx[EPL], w[EPL], cs[EPL], sn[EPL];
            row_loads(min(wave, rows - 1), x, vx, w, cs, sn);
            fetch(max(0, min(wave, nblk - 1)), A);
            if (wave < rows) row_compute(wave, x, vx, w, cs, sn);
        } else {
            float x[EPL], vx[EPL], w[EPL], cs[EPL], sn[EPL];
            row_loads(min(wave, rows - 1), x, vx, w, cs, sn);
            if (wave < rows) row_compute(wave, x, vx, w, cs, sn);
        }
        // heads G .. 15 are zero rows of the padded MFMA operand (smem holds
        // at least 16 rows)
        for (int idx = G * D + tid; idx < 16 * D; idx += NT) smem[idx] = 0.f;
    }
    lds_barrier();
    if (p.fused && owner) {
        // KV append at slot pos (:5226-5296); FP8 uses the absmax scale and OCP e4m3.
        // uniform indices: the table entry comes through the scalar cache and
        // the wait for it leaves the first K/V block's loads in flight
        const int ub = __builtin_amdgcn_readfirstlane(b), uk = __builtin_amdgcn_readfirstlane(kvh);
        const int up = __builtin_amdgcn_readfirstlane(pos);
        const int64_t off = p.kv.row_uniform(ub, uk, up, D);
        if constexpr (!FP8) {
            uint16_t* kc = reinterpret_cast<uint16_t*>(p.kv.k) + off;
            uint16_t* vc = reinterpret_cast<uint16_t*>(p.kv.v) + off;
            for (int d = tid; d < D; d += NT) {
                kc[d] = static_cast<uint16_t>(f32_to_bf16_bits(kn_s[d]));
                vc[d] = static_cast<uint16_t>(f32_to_bf16_bits(vn_s[d]));
            }
        } else {
            if (wave < 2) {
                const float* src = wave == 0 ? kn_s : vn_s;
                uint8_t* dst = (wave == 0 ? p.kv.k : p.kv.v) + off;
                float am = 0.f;
                for (int d = lane; d < D; d += 64) am = fmaxf(am, fabsf(src[d]));
                am = wave_max(am);
                const float sc = fmaxf(am / 448.0f, 1e-12f);
                const float inv = 1.0f / sc;
                for (int d = lane * 4; d < D; d += 256) {
                    const uint32_t c4 = f32x4_to_fp8x4(src[d] * inv, src[d + 1] * inv,
                                                       src[d + 2] * inv, src[d + 3] * inv);
                    *reinterpret_cast<uint32_t*>(dst + d) = c4;
                }
                if (lane == 0) (wave == 0 ? p.kv.ks : p.kv.vs)[p.kv.srow_uniform(ub, uk, up)] = sc;
            }
        }
    }

    // Q as the MFMA A operand: row = head (lane & 15), k = dims 32s + 8(lane>>4) + j.
    // Kept in LDS (one copy for the 4 waves) and read back per block, which
    // leaves registers for the next block's loads.
    u32x4_v (&qop_s)[KSTEPS * 64] = L.qop_s;
    if (wave == 0) {
        const int hh = lane & 15;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            u32x4_v w;
            const int dk = kdim<FP8>(s, lane >> 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = pack2<QT>(smem[hh * D + dk + 2 * j], smem[hh * D + dk + 2 * j + 1]);
            qop_s[s * 64 + lane] = w;
        }
    }
    lds_barrier();  // smem is reused by the merge below

    // ---------------------------------------------------------------- main loop
    // One 16-token block, both products on the MFMA pipe.  The scores come
    // out transposed (S^T = K Q^T: lane = head lane&15, tokens 4(lane>>4) + i),
    // which is already the layout of the probabilities as the B operand of
    // the PV MFMA (16x16x16: k = tokens 4(lane>>4) .. +3, n = head).  V^T is
    // its A operand (m = dim, k = token): the lane's four token rows are
    // interleaved by byte permutes (vpairs; e4m3 then takes an exact convert
    // to bf16).  acc[4w + q] holds, for head lane&15, the dims
    // vdim(w, q, 4(lane>>4) + i).  The softmax state (m_run, l_run) belongs to
    // the lane's head; l_run sums only the lane's tokens until the end.  FP8:
    // the V scale goes on p (per token, along the contraction), the K scale
    // on the score.  Tokens >= nv are masked.
    constexpr int NS = D / 16;
    f32x4_v acc[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) acc[s] = f32x4_v{0.f, 0.f, 0.f, 0.f};
    float m_run = -1e30f, l_run = 0.f;
    auto process = [&](int nv, const op_t (&kb)[KSTEPS], float ksc, float vsc, auto&& vpairs) {
        f32x4_v sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) sc = Mfma<QT>::mma(kb[s], as_op<op_t>(qop_s[s * 64 + lane]), sc);
        // the scales of tokens 4(lane>>4) + i, from the lanes that loaded them
        const int t4 = 4 * (lane >> 4);
        float s2[4], ps[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float ks = FP8 ? __shfl(ksc, (lane & 48) + t4 + i) : 1.f;
            s2[i] = t4 + i < nv ? sc[i] * (p.scale_log2 * ks) : -INFINITY;
        }
        float bm = max3_raw(s2[0], s2[1], fmaxf(s2[2], s2[3]));
        bm = xor32_max(xor16_max(bm));
        const float mn = fmaxf(m_run, bm);
        const float al = __builtin_amdgcn_exp2f(m_run - mn);
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float pe = __builtin_amdgcn_exp2f(s2[i] - mn);
            sum += pe;
            ps[i] = FP8 ? pe * __shfl(vsc, (lane & 48) + t4 + i) : pe;
        }
        l_run = l_run * al + sum;
        m_run = mn;
        // rescale only when some head's running max moved (a scalar branch)
        if (__builtin_amdgcn_ballot_w64(al != 1.0f) != 0) {
#pragma unroll
            for (int s = 0; s < NS; ++s) acc[s] *= al;
        }
        const u32x2_v pw = {pack2<QT>(ps[0], ps[1]), pack2<QT>(ps[2], ps[3])};
        const s16x4_v pop = __builtin_bit_cast(s16x4_v, pw);
#pragma unroll
        for (int w = 0; w < VQD / 4; ++w) {
            uint32_t vp[4][2];  // bf16 pairs (tokens 2h, 2h+1) of dim 4w + q
            vpairs(w, vp);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u32x2_v a = {vp[q][0], vp[q][1]};
                acc[4 * w + q] = Mfma<QT>::mma16(__builtin_bit_cast(s16x4_v, a), pop, acc[4 * w + q]);
            }
        }
    };
    auto process_blk = [&](int blk, Blk& B) {
        const int t0 = t_begin + blk * 16;
        if constexpr (!FP8) {
            // words 2w, 2w+1 of the lane's four token rows (dims 4w .. 4w+3)
            // -> the pairs (tokens 2h, 2h+1) of each dim: one v_perm_b32 each
            process(min(16, t_main - t0), B.kb, 1.f, 1.f, [&](int w, uint32_t (&vp)[4][2]) {
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const uint32_t a0 = B.vq[2 * h][2 * w + c], a1 = B.vq[2 * h + 1][2 * w + c];
                        vp[2 * c][h] = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
                        vp[2 * c + 1][h] = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
                    }
            });
        } else {
            op_t kb[KSTEPS];
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
                const u32x4_v& w = B.kr8[s >> 1];
                kb[s] = as_op<op_t>(fp8x8_to_bf16x8((s & 1) ? u32x2_v{w[2], w[3]} : u32x2_v{w[0], w[1]}));
            }
            // word w of the lane's four token rows -> the bf16 pairs of dims
            // 4w .. 4w+3: v_perm_b32 takes byte q of tokens 0 and 1 (2 and 3)
            // side by side, one convert per pair
            auto vpairs = [&](int w, uint32_t (&vp)[4][2]) {
                uint32_t r[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) r[j] = B.vq[j][w];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t lo = __builtin_amdgcn_perm(r[2 * h + 1], r[2 * h], 0x05010400u);  // bytes 0, 1
                    const uint32_t hi = __builtin_amdgcn_perm(r[2 * h + 1], r[2 * h], 0x07030602u);  // bytes 2, 3
                    vp[0][h] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false));
                    vp[1][h] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true));
                    vp[2][h] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false));
                    vp[3][h] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true));
                }
            };
            process(min(16, t_main - t0), kb, B.ksc, B.vsc, vpairs);
        }
    };

    // Software pipeline: the next block's loads are in flight while the
    // current block is computed (two register sets, unrolled by two).
    // Blocks are claimed from an LDS counter (wave w starts with block w), so
    // a wave whose loads are served more slowly simply takes fewer blocks and
    // the waves of the workgroup finish together (about 3% faster at config 2
    // and 4 than a static order).  The claim order changes the fp32 summation
    // order from run to run; p.det selects the static order (wave w takes
    // blocks w, w + NW, ...), whose results are identical run to run.
    int nxt = wave + NW;
    auto take = [&]() {
        int v = 0;
        if (p.det) {
            v = nxt;
            nxt += NW;
        } else {
            if (lane == 0) v = atomicAdd(&next_blk, 1);
            v = __builtin_amdgcn_readfirstlane(v);
        }
        return v;
    };
    {
        int c0 = wave, c1 = nblk;
        if (c0 < nblk) {
            c1 = take();
            if (c1 < nblk) fetch(c1, Bn);
        }
        while (c0 < nblk) {
            process_blk(c0, A);
            if (c1 >= nblk) break;
            c0 = take();
            if (c0 < nblk) fetch(c0, A);
            process_blk(c1, Bn);
            if (c0 >= nblk) break;
            c1 = take();
            if (c1 < nblk) fetch(c1, Bn);
        }
    }
    // The new token (fused owner split): one more block of one token, read
    // from LDS unquantised (as full_attention_4b.hip:5351-5353 does), on wave 0.
    if (owner && wave == 0) {
        op_t kbn[KSTEPS];
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            u32x4_v w;
            const int d0 = kdim<FP8>(s, lane >> 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = pack2<QT>(kn_s[d0 + 2 * j], kn_s[d0 + 2 * j + 1]);
            kbn[s] = as_op<op_t>(w);
        }
        // token 0 of the block is k = 0 of lanes 0..15
        process(1, kbn, 1.f, 1.f, [&](int w, uint32_t (&vp)[4][2]) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                vp[q][0] = lane < 16 ? Elem<QT>::from_f32(vn_s[vdim(w, q, lane)]) : 0u;
                vp[q][1] = 0u;
            }
        });
    }

    // ---------------------------------------------------------------- merge
    // Arrival: every split of (b, kv head) that holds tokens counts itself in
    // as its main loop ends (the last wave; its round trip overlaps the
    // workgroup's reduction below); the last one to arrive keeps its partial
    // in LDS and merges them all, polling for the others' partials, which are
    // stored or on their way.
    unsigned arrival = 0;
    if (wave == NW - 1 && lane == 0) arrival = atomicAdd(&p.arrivals[(b * p.Hkv + kvh) * p.arr_stride], 1u);
    // One LDS round: the lane's head has its running max (the same in the
    // four rows) and its sum over all its tokens; every wave parks its sums,
    // scaled to the workgroup's max, in its own slot, and the split's partial
    // is then the sum of the NW slots.
    int& last_s = L.last_s;
    const float lt = xor32_sum(xor16_sum(l_run));
    const int hl = lane & 15;
    if (lane < GP) {
        ml_s[wave][lane][0] = m_run;
        ml_s[wave][lane][1] = lt;
    }
    __syncthreads();
    const int hc = min(hl, GP - 1);
    float mw = ml_s[0][hc][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) mw = fmaxf(mw, ml_s[w][hc][0]);
    const float f = exp2f(ml_s[wave][hc][0] - mw);
    if (wave == NW - 1 && lane == 0) last_s = arrival == static_cast<unsigned>(ns - 1);
    if (hl < GP) {
        float* const row = &smem[(wave * GP + hl) * D];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int s4 = 0; s4 < NS / 4; ++s4) {
                const f32x4_v v = {acc[4 * s4][i] * f, acc[4 * s4 + 1][i] * f, acc[4 * s4 + 2][i] * f, acc[4 * s4 + 3][i] * f};
                *reinterpret_cast<f32x4_v*>(row + vdim(s4, 0, 4 * (lane >> 4) + i)) = v;
            }
    }
    __syncthreads();
    // (M, L) of head hh of this split, from the waves' (m, l)
    auto own_ml = [&](int hh, float& M, float& Lsum) {
        M = -1e30f;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, ml_s[w][hh][0]);
        Lsum = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) Lsum += exp2f(ml_s[w][hh][0] - M) * ml_s[w][hh][1];
    };
    // Partials: part_o rows of D floats, part_ml rows of (M, L), both as
    // part_enc words (zero = not written yet), written and read with
    // device-coherent (sc1) vector accesses, so no device-wide fence (an L2
    // writeback and invalidate on this GPU) is needed and no writer waits for
    // its stores to complete.  A lane holds DV consecutive dims of a row.
    constexpr int DV = D / 64;
    typedef typename U32N<DV>::t dv_t;
    auto row_of = [&](int hh, int sp) { return pre_b * p.Hq + static_cast<int64_t>(kvh * G + hh) * n_b + sp; };
    if (!last_s) {
        for (int hh = wave; hh < G; hh += NW) {
            dv_t w;
#pragma unroll
            for (int j = 0; j < DV; ++j) {
                float o = 0.f;
#pragma unroll
                for (int ww = 0; ww < NW; ++ww) o += smem[(ww * GP + hh) * D + lane * DV + j];
                if constexpr (DV == 1) w = part_enc(o);
                else w[j] = part_enc(o);
            }
            st_coh<DV>(p.part_o + row_of(hh, split) * D, lane * DV * 4, w);
        }
        if (wave == 0 && lane < G) {
            float M, Lsum;
            own_ml(lane, M, Lsum);
            const uint64_t v = part_enc(M) | (static_cast<uint64_t>(part_enc(Lsum)) << 32);
            __hip_atomic_store(reinterpret_cast<uint64_t*>(&p.part_ml[2 * row_of(lane, split)]), v, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }

    // ---------------------------------------------------------------- split merge
    // The last split of (b, kv head) merges all of them (log-sum-exp), its own
    // partial straight from LDS, and applies the gate.  With at least twice as
    // many waves as heads, two waves share a head, each taking half of the
    // splits, and combine through LDS.  A wave takes MCH splits a round: one
    // load for their (M, L) (lane c holds split c's) and one per split for the
    // dims, polled until no word reads zero (every split zeroed its own slots
    // as it started).  The gate goes out with the first round.
    constexpr int MCH = 16;  // splits a round (32 measured slower: the merge then spills)
    const int WPH = 2 * G <= NW ? 2 : 1;                 // waves per head
    const int part = WPH == 2 ? wave % 2 : 0;
    const int half = WPH == 2 ? (ns + 1) / 2 : ns;
    const int sp_lo = part * half, sp_hi = min(ns, sp_lo + half);
    const bool has_gate = p.gate != nullptr;
    float Mr = -1e30f, Lr = 0.f, orr[DV];               // this wave's running merge
    int my_h = -1;
    for (int hh = wave / WPH; hh < G; hh += NW / WPH) {
        my_h = hh;
        const int h = kvh * G + hh;
        // branch-free: without a gate the load reads the output row (a valid
        // address) and the values are ignored
        const uint16_t* grow = has_gate ? p.gate + b * p.g_bstride + h * p.g_hstride
                                        : static_cast<const uint16_t*>(p.out) + (static_cast<int64_t>(b) * p.Hq + h) * D;
        uint16_t graw[DV];
#pragma unroll
        for (int j = 0; j < DV; ++j) graw[j] = COH ? load_agent_u16(grow + lane * DV + j) : grow[lane * DV + j];
        float M = -1e30f, Ls = 0.f;
#pragma unroll
        for (int j = 0; j < DV; ++j) orr[j] = 0.f;
        // this split's own partial, from LDS, merged at its place in split
        // order (the result does not depend on which split arrives last)
        float own_m, own_l, own_o[DV];
        own_ml(hh, own_m, own_l);
#pragma unroll
        for (int j = 0; j < DV; ++j) {
            float o = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ++ww) o += smem[(ww * GP + hh) * D + lane * DV + j];
            own_o[j] = o;
        }
        const int64_t row0 = row_of(hh, 0);
        uint32_t* const pml = reinterpret_cast<uint32_t*>(p.part_ml) + 2 * row0;
        uint32_t* const po = reinterpret_cast<uint32_t*>(p.part_o) + row0 * D;
        for (int s0 = sp_lo; s0 < sp_hi; s0 += MCH) {
            u32x2_v mlw;
            dv_t os[MCH];
            const int cl = min(lane, MCH - 1);
            const bool want_l = s0 + cl < sp_hi && s0 + cl != split && lane < MCH;
            for (int it = 0;; ++it) {
                mlw = ld_coh<2>(pml, 8 * min(s0 + cl, sp_hi - 1));
#pragma unroll
                for (int c = 0; c < MCH; ++c) os[c] = ld_coh<DV>(po + static_cast<int64_t>(min(s0 + c, sp_hi - 1)) * D, lane * DV * 4);
                bool miss = want_l & ((mlw[0] == 0u) | (mlw[1] == 0u));
#pragma unroll
                for (int c = 0; c < MCH; ++c) {
                    const bool want = s0 + c < sp_hi && s0 + c != split;
                    bool z = false;
                    if constexpr (DV == 1) z = os[c] == 0u;
                    else {
#pragma unroll
                        for (int j = 0; j < DV; ++j) z |= os[c][j] == 0u;
                    }
                    miss |= want & z;
                }
                // every split has arrived, so its partial is stored or on its
                // way (the cap only guards against a workspace that was not
                // zero-filled)
                if (!__builtin_amdgcn_ballot_w64(miss)) break;
                if (it >= p.merge_polls) {
                    if (lane == 0) wait_expired(kWaitDecodeMerge);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            const bool own_lane = lane < MCH && s0 + lane == split && split < sp_hi;  // inside this wave's range
            const float m_l = want_l ? part_dec(mlw[0]) : (own_lane ? own_m : -1e30f);
            const float l_l = want_l ? part_dec(mlw[1]) : (own_lane ? own_l : 0.f);
            float mc = M;
#pragma unroll
            for (int c = 0; c < MCH; ++c) mc = fmaxf(mc, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m_l), c)));
            const float a = __builtin_amdgcn_exp2f(M - mc);
            Ls *= a;
#pragma unroll
            for (int j = 0; j < DV; ++j) orr[j] *= a;
            const float f_l = want_l || own_lane ? __builtin_amdgcn_exp2f(m_l - mc) : 0.f;
            Ls += wave_sum(f_l * l_l);
#pragma unroll
            for (int c = 0; c < MCH; ++c) {
                const bool want = s0 + c < sp_hi && s0 + c != split;
                const bool own = s0 + c == split && split < sp_hi;
                const float f = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f_l), c));
                if constexpr (DV == 1) orr[0] = fmaf(f, want ? part_dec(os[c]) : (own ? own_o[0] : 0.f), orr[0]);
                else {
#pragma unroll
                    for (int j = 0; j < DV; ++j)
                        orr[j] = fmaf(f, want ? part_dec(os[c][j]) : (own ? own_o[j] : 0.f), orr[j]);
                }
            }
            M = mc;
        }
        Mr = M;
        Lr = Ls;
        auto finish = [&]() {
            const float inv = Lr > 0.f ? 1.0f / Lr : 0.f;
            float r[DV];
#pragma unroll
            for (int j = 0; j < DV; ++j) {
                r[j] = orr[j] * inv;
                if (has_gate) {
                    // bf16(bf16(attn) * sigmoid(gate)) (full_attention_4b.hip:5464-5470)
                    r[j] = bf16_round(bf16_round(r[j]) * (1.0f / (1.0f + expf(-bf16_bits_to_f32(graw[j])))));
                }
            }
            const int64_t ob = (static_cast<int64_t>(b) * p.Hq + h) * D + lane * DV;
            uint16_t* const op = reinterpret_cast<uint16_t*>(static_cast<QT*>(p.out)) + ob;
            if constexpr (DV == 4) {
                if ((reinterpret_cast<uintptr_t>(op) & 7) == 0) {  // one 8-byte store of the lane's 4 dims
                    const uint64_t v = static_cast<uint64_t>(pack2<QT>(r[0], r[1])) |
                                       (static_cast<uint64_t>(pack2<QT>(r[2], r[3])) << 32);
                    if constexpr (COH) __hip_atomic_store(reinterpret_cast<uint64_t*>(op), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    else *reinterpret_cast<uint64_t*>(op) = v;
                    return;
                }
            }
#pragma unroll
            for (int j = 0; j < DV; ++j) {
                if constexpr (COH) store_f32_agent(static_cast<QT*>(p.out), ob + j, r[j]);
                else store_f32(static_cast<QT*>(p.out), ob + j, r[j]);
            }
        };
        if (WPH == 1) {
            finish();
        } else {
            // two waves per head: the second parks (M, L, o) in LDS (smem is
            // free once every wave has read its own partial), the first
            // combines and writes the head
            lds_barrier();
            float* park = &smem[hh * (D + 2)];
            if (part == 1) {
#pragma unroll
                for (int j = 0; j < DV; ++j) park[lane * DV + j] = orr[j];
                if (lane == 0) {
                    park[D] = Mr;
                    park[D + 1] = Lr;
                }
            }
            lds_barrier();
            if (part == 0) {
                const float M2 = park[D], L2 = park[D + 1];
                const float mm = fmaxf(Mr, M2);
                const float a1 = __builtin_amdgcn_exp2f(Mr - mm), a2 = __builtin_amdgcn_exp2f(M2 - mm);
                Lr = Lr * a1 + L2 * a2;
#pragma unroll
                for (int j = 0; j < DV; ++j) orr[j] = orr[j] * a1 + park[lane * DV + j] * a2;
                finish();
            }
        }
    }
    if (WPH == 2 && my_h < 0) {  // waves without a head still take part in the two barriers
        lds_barrier();
        lds_barrier();
    }
    if (tid == 0) p.arrivals[(b * p.Hkv + kvh) * p.arr_stride] = 0u;  // every split has arrived: ready for the next call
}

}  // namespace ssa
