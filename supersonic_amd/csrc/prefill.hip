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
//   workgroup = 128 query rows of one head: 8 compute wave64s of 16 rows and
//   4 copy waves; keys in tiles of 64, double-buffered in LDS and copied
//   global->LDS directly (buffer_load ... lds).  K is copied row-major into
//   padded blocks; V comes from a transposed staging copy (vt_stage_kernel)
//   so the PV operand is one conflict-free ds_read_b128 per MFMA.
//   S^T = K Q^T     v_mfma_f32_16x16x32: A = 16 key rows (LDS), B = Q^T held
//                   in registers for the whole kernel.
//   O^T += V^T P^T  the B operand (P^T) is the lane's own softmax weights.
//   Online softmax in base 2 with a lazy running max (O is rescaled only
//   when a row max grows by more than 2^8); the row sums add the 16-bit
//   weights exactly as the MFMA uses them.
//   Causal: key tiles past the workgroup's last row are never loaded; a wave
//   skips the MFMA work of tiles past its own last row; only tiles that cross
//   the diagonal or the kv_len edge are masked.  Query tiles run longest
//   first, the heads of one kv head on one XCD.
#include <cstdlib>

#include <type_traits>

#include "common.hpp"
#include "kv_view.hpp"

namespace ssa {

struct PrefillParams {
    const uint16_t* q;   // element (b, h, row, d) at b*q_bs + h*q_hs + row*q_rs + d
    int64_t q_bs, q_hs, q_rs;
    KvView kv;           // K/V rows of (b, kv head, token)
    // V^T staging (vt_stage_kernel): element (b, kv head, dim, position) at
    // ((b * Hkv + h) * D + dim) * vt_ld + position
    const uint16_t* vt;
    int vt_ld;
    int Hq, Hkv, G, S, L, off;
    float scale_log2;
    int nqt;             // query tiles of 128 rows
    int B;               // sequences
    int n_wg;            // workgroups of the persistent grid
    // Dynamic schedule (NULL: the static one).  Per item list x (an XCD's, or
    // the single list) a claim counter at claims[32 x] and a finished-workgroup
    // counter at claims[32 (8 + x)], each on its own 128-byte line; both are
    // zero before a launch and the list's last workgroup to finish zeroes them.
    unsigned* claims;
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
    float rescale_slack;  // lazy-rescale slack in log2 units (0 = exact running max)
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

typedef short s16x4_v __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_v __attribute__((ext_vector_type(2)));

// Two f32 -> packed 16-bit pair with the hardware RNE converters.
template <typename QT> __device__ __forceinline__ uint32_t cvt_pk(float a, float b);
template <> __device__ __forceinline__ uint32_t cvt_pk<bf16_t>(float a, float b) {
    f32x2_v v = {a, b};
    bf16x2_v r = __builtin_convertvector(v, bf16x2_v);
    return __builtin_bit_cast(uint32_t, r);
}
template <> __device__ __forceinline__ uint32_t cvt_pk<f16_t>(float a, float b) {
    f32x2_v v = {a, b};
    f16x2_v r = __builtin_convertvector(v, f16x2_v);
    return __builtin_bit_cast(uint32_t, r);
}

// Two 16-bit ones packed in a word (the A operand of the row-sum MFMA).
template <typename QT> constexpr uint32_t kOnePair = 0x3F803F80u;  // bf16 1.0, 1.0
template <> constexpr uint32_t kOnePair<f16_t> = 0x3C003C00u;       // f16 1.0, 1.0

// Tile geometry.  A K tile is 64 keys x D in LDS.  Copy instruction i
// (i < NR = D/8) of a tile moves rows i, i + NR, i + 2 NR, ... (64/NR rows,
// one 1 KB run) into LDS block i.  K blocks are padded by 8 words so the
// 16-row ds_read_b128 K reads hit distinct banks (SQ_LDS_BANK_CONFLICT is 0
// on gfx950).  Row r lives at (r % NR) * KBLK + (r / NR) * ROWB, so every
// inner-loop LDS offset is an immediate on one per-lane base.
//
// A V tile arrives transposed: D rows (dims) of 64 keys, 128 B each, copy
// instruction i moving dims 8i .. 8i + 7 into block i (1 KB, unpadded).  Dims
// 16 P .. 16 P + 15 fill the 2 KB pair P; inside a pair dim r's 16-byte chunk
// c (keys 8c .. 8c + 7 in staging order) sits at granule 8 r + (c ^ (r >> 1)),
// which spreads the 16 dims one ds_read_b128 of the PV loop touches over all
// 16 granule slots of a 256-byte bank row.
template <int D> struct Tile {
    static constexpr int ROWB = 2 * D;        // bytes per key row
    static constexpr int NR = D / 8;          // copy instructions (= 1 KB blocks) per tile
    static constexpr int KBLK = 1024 + 32;
    static constexpr int KBYTES = NR * KBLK;
    static constexpr int VBYTES = NR * 1024;
    static constexpr int STAGE = KBYTES + VBYTES;
    static constexpr int NI = NR / 4;         // copy instructions per copy wave (K and V each)
    static __device__ __forceinline__ constexpr int koff(int r) { return (r % NR) * KBLK + (r / NR) * ROWB; }
};

// Buffer resource for a tile base that is uniform across the wave (forced
// into SGPRs: the base can come from a block-table load the compiler cannot
// prove uniform).  Reads past `bytes` return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const uint8_t* base, int bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
    void* u = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, static_cast<short>(0), bytes, 0x00020000);
}

template <typename QT> struct Mfma16;
template <> struct Mfma16<bf16_t> {
    typedef bf16x8_v op;
    static __device__ __forceinline__ f32x4_v mma(const op& a, const op& b, const f32x4_v& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma16<f16_t> {
    typedef f16x8_v op;
    static __device__ __forceinline__ f32x4_v mma(const op& a, const op& b, const f32x4_v& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

// LDS read lookahead of the K-operand (reads) and V-operand (MFMAs) pipelines
constexpr int kKLA = 8;
constexpr int kVLA = 6;

constexpr int kPrefillWaves = 8;   // compute waves: 8 x 16 query rows = 128 rows
constexpr int kCopyWaves = 4;      // waves that only move K / V^T tiles into LDS
constexpr int kPrefillThreads = 64 * (kPrefillWaves + kCopyWaves);


// One workgroup = 128 query rows of one head: 8 compute waves of 16 rows each
// plus 4 copy waves that only issue the global->LDS tile copies (the copy
// path runs at about 48 B/clk per CU, and a wave that issues copies stalls
// until they are accepted, so compute waves never issue any).  Three waves
// share a SIMD (about 150 registers each); one wave's softmax VALU work
// overlaps another's MFMA chains.
//
//   S^T = K Q^T      v_mfma_f32_16x16x32: A = 16 key rows (LDS), B = Q^T (16
//                    query rows, registers).  C: lane l holds query row l & 15
//                    and keys 16 kb + 4 (l >> 4) + i of key block kb.
//   O^T += V^T P^T   per 32-key step the B operand (P^T) is the lane's own 8
//                    weights (keys 4 g + i of the two 16-key blocks), and the A
//                    operand (V^T) comes from two transposing LDS reads, each
//                    giving a lane 4 consecutive keys of dim (l & 15).
template <typename QT, int D, bool FUSED>
__global__ __launch_bounds__(kPrefillThreads) void prefill_kernel(PrefillParams p) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass only needs the launch stub
    typedef typename Mfma16<QT>::op op_t;
    typedef Tile<D> T;
    constexpr int KS = D / 32;        // QK^T k-steps (32 dims each)
    constexpr int DBK = D / 16;       // 16-dim output blocks
    // [stage][K | V] tiles; the fused prologue stages the query rows in one stage
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * T::STAGE];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: copy offsets stay in SGPRs
    // Persistent grid (one workgroup per CU), items longest first.  When the
    // heads split evenly over the 8 XCDs (workgroup i runs on XCD i % 8), each
    // XCD has its own item list holding the heads that share its kv heads, so
    // its L2 keeps their K/V.  Workgroup j of a list of W takes items j,
    // 2W-1-j, 2W+j, ...: a long item pairs with a short one and every
    // workgroup gets about the same number of key tiles.
    const int bid = blockIdx.x;
    const int hpx = p.Hq / 8;
    const bool by_xcd = hpx > 0 && (p.Hq % 8) == 0 && (p.n_wg % 8) == 0;
    const int j = by_xcd ? (bid >> 3) : bid;
    const int W = by_xcd ? (p.n_wg >> 3) : p.n_wg;
    const int hpi = by_xcd ? hpx : p.Hq;     // heads per item list
    const int n_items = p.nqt * hpi * p.B;
    // Dynamic schedule: the list's items are claimed one at a time from a
    // counter in list order (longest first), so workgroups that start late
    // (their CUs busy with other work when the grid was dispatched) take only
    // what is left.  The first copy wave claims item r + 1 during item r and
    // leaves it in claimed[(r + 1) & 1]; every reader is at least one
    // workgroup barrier behind the write.
    __shared__ int claimed[2];
    const bool dyn = p.claims != nullptr;
    unsigned* const ctr = dyn ? p.claims + 32 * (by_xcd ? (bid & 7) : 0) : nullptr;
    auto claim_next = [&](const int slot) {
        if (wave == kPrefillWaves && (tid & 63) == 0) {
            claimed[slot] = static_cast<int>(__hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the write is in LDS before the next barrier
        }
    };
    // Item r of this workgroup (false past the last): 128 query rows `qt` of
    // head h of sequence b.  The sequence of m is increasing (static schedule).
    auto item_at = [&](const int r, int& qt, int& h, int& b) -> bool {
        const int m = dyn ? claimed[r & 1] : ((r & 1) ? (r + 1) * W - 1 - j : r * W + j);
        if (m >= n_items) return false;
        qt = p.nqt - 1 - m / (hpi * p.B);
        const int rem = m % (hpi * p.B);
        h = (by_xcd ? (bid & 7) * hpx : 0) + rem % hpi;
        b = rem / hpi;
        return true;
    };
    // 64-key tiles of query block qt: keys below the block's last row (causal).
    auto tiles_of = [&](const int qt) -> int {
        const int lim = min(p.L, p.off + min(qt * 128 + 128, p.S));
        return lim > 0 ? (lim + 63) / 64 : 0;
    };
    // Tiles alternate between the two LDS stages across items: tile `it` of
    // an item that follows gt tiles goes to stage (gt + it + 1) & 1, so the
    // next item's first tile can be copied while this item's last tile is
    // computed, and the fused query staging of an item uses stage gt & 1 (its
    // previous item's last tile, read by then).
    //
    // Copy waves: the next tile is issued once every wave has passed the
    // barrier of tile it (the stage it goes to was last read by tile it - 1)
    // and has landed by the next barrier.  Same barrier count per item as the
    // compute waves (one per tile plus the item end).
    auto copy_items = [&]() {
        const int lane = tid & 63;
        const int dma_lane = (lane / (D / 8)) * T::NR * T::ROWB + (lane % (D / 8)) * 16;
        const int vt_rowb = 2 * p.vt_ld;
        const int vt_lane0 = (lane >> 3) * vt_rowb + 16 * ((lane & 7) ^ (lane >> 4));
        const int vt_lane1 = (lane >> 3) * vt_rowb + 16 * ((lane & 7) ^ (4 + (lane >> 4)));
        // Direct global->LDS copy of key tile `it` of (h, b) into stage `st`
        // (asynchronous, counted by vmcnt).  K: lane l of copy instruction i
        // moves 16 bytes of row i + NR (l / (D/8)); rows past kv_len fall
        // outside the buffer range and read as zeros (masked later; never
        // stale cache contents).  V^T: lane l of instruction i moves chunk
        // c = (l & 7) ^ (4 (i & 1) + (l >> 4)) of dim 8 i + (l >> 3) (the
        // swizzle of the tile geometry); the staging buffer is zero past kv_len.
        auto issue_tile = [&](const int h, const int b, const int it, const int st) {
            const int kvh = h / p.G;
            const uint16_t* vt_head = p.vt + (static_cast<int64_t>(b) * p.Hkv + kvh) * D * p.vt_ld;
            const int k0 = it * 64;
            const int64_t base = p.kv.row_uniform(b, kvh, k0, D) * 2;  // a tile lies inside one page
            const __amdgpu_buffer_rsrc_t kr = tile_rsrc(p.kv.k + base, min(64, p.L - k0) * T::ROWB);
            const __amdgpu_buffer_rsrc_t vr = tile_rsrc(reinterpret_cast<const uint8_t*>(vt_head + k0),
                                                        D * vt_rowb - 2 * k0);
            const int cw = wave - kPrefillWaves;
            const int lbase = __builtin_amdgcn_readfirstlane(st * T::STAGE + cw * T::NI * T::KBLK);
            const int vbase = __builtin_amdgcn_readfirstlane(st * T::STAGE + T::KBYTES + cw * T::NI * 1024);
#pragma unroll
            for (int jj = 0; jj < T::NI; ++jj) {
                const int i = cw * T::NI + jj;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (__attribute__((address_space(3))) void*)(lds + lbase + jj * T::KBLK),
                                                         16, dma_lane, i * T::ROWB, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (__attribute__((address_space(3))) void*)(lds + vbase + jj * 1024),
                                                         16, (i & 1) ? vt_lane1 : vt_lane0, 8 * i * vt_rowb, 0, 0);
            }
        };
        // s_waitcnt vmcnt(0) alone (the other counters are not waited for)
        auto wait_vm0 = []() { __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8)); };
        // first tile of the first item that has keys at all
        auto issue_first = [&](int r, const int st) {
            int qt, h, b;
            for (; item_at(r, qt, h, b); ++r) {
                if (tiles_of(qt) > 0) {
                    issue_tile(h, b, 0, st);
                    return;
                }
                if (dyn) return;  // only item r is claimed yet (and every item has tiles)
            }
        };
        issue_first(0, 1);
        int gt = 0, qt, h, b;
        for (int r = 0; item_at(r, qt, h, b); ++r) {
            const int nt = tiles_of(qt);
            // The next item is claimed as this one nears its end (at the
            // barrier of tile nt - 3, two barriers before the other copy
            // waves read the claim), so workgroups claim in the order they
            // finish: longest-processing-time-first.  Items of fewer than 3
            // tiles claim at their start.
            if (dyn && nt < 3) claim_next((r + 1) & 1);
            for (int it = 0; it < nt; ++it) {
                // Tile `it` has landed.  The compute waves' barrier also
                // orders their LDS reads; these waves read no LDS, so a bare
                // barrier (no implied wait for every load in flight) is enough.
                wait_vm0();
                __builtin_amdgcn_s_barrier();
                if (dyn && nt >= 3 && it == nt - 3) claim_next((r + 1) & 1);
                if (it + 1 < nt) issue_tile(h, b, it + 1, (gt + it + 2) & 1);
                else issue_first(r + 1, (gt + nt + 1) & 1);
            }
            __builtin_amdgcn_s_barrier();  // item end (the next tile needs no wait yet)
            gt += nt;
        }
        wait_vm0();  // no LDS write in flight when the workgroup ends
        if (dyn && wave == kPrefillWaves && (tid & 63) == 0) {
            // This workgroup's claims are over (its last one failed); the
            // list's last workgroup to get here leaves both counters at zero.
            unsigned* const done = ctr + 32 * 8;
            const unsigned wl = by_xcd ? static_cast<unsigned>(p.n_wg >> 3) : static_cast<unsigned>(p.n_wg);
            if (__hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 == wl) {
                __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    };
    // One work item = 128 query rows of one head of one sequence, run by the
    // compute waves; gt = tiles of the workgroup's items before it.  A
    // `return` inside ends the item, not the workgroup.
    auto run_item = [&](const int qt, const int h, const int b, const int gt) {
    // Opaque per item, so the compiler does not hoist lane-derived values and
    // loads (norm weights, offsets) out of the item loop, where they would
    // stay live through the key loop.
    int lane = tid & 63;
    asm volatile("" : "+v"(lane));
    const int kvh = h / p.G;
    const int g4 = lane >> 4;
    const int q0 = qt * 128;
    const int row_w0 = q0 + 16 * wave;
    const int myrow = row_w0 + (lane & 15);
    const bool row_ok = myrow < p.S;
    const int S = p.S, L = p.L, off = p.off;

    const int ntiles = tiles_of(qt);
    const int lim_wave = min(L, off + min(row_w0 + 16, S));
    const int lim_row = min(L, off + myrow + 1);

    // ------------------------------------------------ Q^T operand (registers)
    // B operand of S^T = K Q^T: lane holds query row (lane & 15), dims 32 s + 8 g4 + j.
    op_t qb[KS];
    if constexpr (!FUSED) {
        const uint16_t* qrow = p.q + b * p.q_bs + h * p.q_hs + static_cast<int64_t>(row_ok ? myrow : 0) * p.q_rs;
#pragma unroll
        for (int s = 0; s < KS; ++s)
            qb[s] = to_op<op_t>(row_ok ? ld16(qrow + 32 * s + 8 * g4) : u32x4_v{0u, 0u, 0u, 0u});
    } else if (p.half_rot % 32 == 0 || p.half_rot == 16) {
        // This wave's 16 query rows normed and rotated in the operand layout
        // itself: lane holds row myrow, dims 32 s + 8 g4 + j (64 of the row's
        // dims), RMSNorm with (1 + w) over the row (the four lanes l, l ^ 16,
        // l ^ 32, l ^ 48 hold it), then rotate-half RoPE at position off + row,
        // bf16 after each step (prefill_engine.rs:2025-2096).  A RoPE partner
        // (dim d +- half_rot) is in the same lane, chunk s +- half_rot / 32,
        // when half_rot is a multiple of 32, or in lane ^ 32, same chunk, when
        // it is 16.  Every global load is issued before any arithmetic.
        const int hr = p.half_rot;
        const int hs = hr / 32;                  // rotary chunks per half (0 for half_rot 16)
        const int pos = off + (row_ok ? myrow : 0);
        const uint16_t* qrow = p.q + h * p.q_hs + static_cast<int64_t>(row_ok ? myrow : 0) * p.q_rs;
        u32x4_v raw[KS], wv[KS], cw[KS / 2], sw[KS / 2];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            raw[s] = row_ok ? ld16(qrow + 32 * s + 8 * g4) : u32x4_v{0u, 0u, 0u, 0u};
            wv[s] = ld16(p.q_norm_w + 32 * s + 8 * g4);
        }
#pragma unroll
        for (int c = 0; c < KS / 2; ++c) {
            cw[c] = sw[c] = u32x4_v{0u, 0u, 0u, 0u};
            const int ci = hr == 16 ? 8 * (g4 & 1) : 32 * c + 8 * g4;  // table column of the chunk
            if (c < (hr == 16 ? 1 : hs)) {
                cw[c] = ld16(p.cos_t + static_cast<int64_t>(pos) * hr + ci);
                sw[c] = ld16(p.sin_t + static_cast<int64_t>(pos) * hr + ci);
            }
        }
        float ss = 0.f;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            float x[8];
            unpack8<bf16_t>(raw[s], x);
#pragma unroll
            for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
        }
        ss = xor32_sum(xor16_sum(ss));
        const float inv = rsqrtf(ss / static_cast<float>(D) + p.eps);
        u32x4_v nq[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            float x[8], w[8];
            unpack8<bf16_t>(raw[s], x);
            unpack8<bf16_t>(wv[s], w);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                nq[s][j] = cvt_pk<bf16_t>(x[2 * j] * inv * (w[2 * j] + 1.0f), x[2 * j + 1] * inv * (w[2 * j + 1] + 1.0f));
        }
        // out = x cos + sg y sin on the normed bf16 values (sg = -1 in the first half)
        auto rot8 = [&](const u32x4_v& xv, const u32x4_v& yv, const u32x4_v& cv, const u32x4_v& sv, const float sg) {
            float x[8], y[8], cs[8], sn[8];
            unpack8<bf16_t>(xv, x);
            unpack8<bf16_t>(yv, y);
            unpack8<bf16_t>(cv, cs);
            unpack8<bf16_t>(sv, sn);
            u32x4_v o;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o[j] = cvt_pk<bf16_t>(x[2 * j] * cs[2 * j] + sg * y[2 * j] * sn[2 * j],
                                      x[2 * j + 1] * cs[2 * j + 1] + sg * y[2 * j + 1] * sn[2 * j + 1]);
            return o;
        };
        // chunks s < 2 HS rotate with partner chunk s +- HS (a compile-time
        // index for each HS, so the arrays stay in registers)
        auto rope_hs = [&](auto hs_c) {
            constexpr int HS = decltype(hs_c)::value;
            u32x4_v o[2 * HS];
#pragma unroll
            for (int s = 0; s < 2 * HS; ++s)
                o[s] = s < HS ? rot8(nq[s], nq[s + HS], cw[s], sw[s], -1.0f)
                              : rot8(nq[s], nq[s - HS], cw[s - HS], sw[s - HS], 1.0f);
#pragma unroll
            for (int s = 0; s < 2 * HS; ++s) nq[s] = o[s];
        };
        if (hr == 16) {
            u32x4_v y;
#pragma unroll
            for (int j = 0; j < 4; ++j) y[j] = static_cast<uint32_t>(__shfl_xor(static_cast<int>(nq[0][j]), 32));
            nq[0] = rot8(nq[0], y, cw[0], sw[0], g4 < 2 ? -1.0f : 1.0f);
        } else {
            static_assert(KS / 2 <= 4, "head_dim up to 256");
            switch (hs) {
            case 1: rope_hs(std::integral_constant<int, 1>{}); break;
            case 2: if constexpr (KS / 2 >= 2) rope_hs(std::integral_constant<int, 2>{}); break;
            case 3: if constexpr (KS / 2 >= 3) rope_hs(std::integral_constant<int, 3>{}); break;
            case 4: if constexpr (KS / 2 >= 4) rope_hs(std::integral_constant<int, 4>{}); break;
            default: break;
            }
        }
#pragma unroll
        for (int s = 0; s < KS; ++s) qb[s] = to_op<op_t>(nq[s]);
    } else {
            // This wave's 16 query rows: RMSNorm with (1 + w) and rotate-half RoPE
            // at position off + row, bf16 after each step (prefill_engine.rs:2025-2096),
            // (lane c of a row holds dims 8c .. 8c+7); every global load is issued
            // before any arithmetic.  The rows are staged in LDS (stage 0), where
            // the RoPE partner dims are read back and the operand is read
            // transposed.
            uint16_t* qs = reinterpret_cast<uint16_t*>(lds + (gt & 1) * T::STAGE) + wave * 16 * D;
            constexpr int LPR = D / 8;              // lanes per row, 16 B each
            constexpr int RPI = 64 / LPR;           // rows per instruction
            constexpr int NIN = 16 / RPI;           // instructions per wave
            const int c = lane % LPR, rr = lane / LPR;
            const int hr = p.half_rot;              // a multiple of 16 (checked on the host)
            const bool rot = 8 * c < 2 * hr;
            const u32x4_v wtw = ld16(p.q_norm_w + 8 * c);
            u32x4_v qw[NIN], cw[NIN], sw[NIN];
    #pragma unroll
            for (int k = 0; k < NIN; ++k) {
                const int row = row_w0 + k * RPI + rr;
                qw[k] = cw[k] = sw[k] = u32x4_v{0u, 0u, 0u, 0u};
                if (row < S) {
                    qw[k] = ld16(p.q + h * p.q_hs + static_cast<int64_t>(row) * p.q_rs + 8 * c);
                    if (rot) {
                        const int64_t ti = static_cast<int64_t>(off + row) * hr + (8 * c < hr ? 8 * c : 8 * c - hr);
                        cw[k] = ld16(p.cos_t + ti);
                        sw[k] = ld16(p.sin_t + ti);
                    }
                }
            }
            float wt[8];
            unpack8<bf16_t>(wtw, wt);
            // RMSNorm: the row's sum of squares over its LPR lanes on the VALU
            // (DPP within 16 lanes, a permlane swap across 16), no LDS traffic.
            u32x4_v nq[NIN];
    #pragma unroll
            for (int k = 0; k < NIN; ++k) {
                float x[8];
                unpack8<bf16_t>(qw[k], x);
                float ss = 0.f;
    #pragma unroll
                for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
                if constexpr (LPR >= 16) {
                    ss = row16_sum(ss);
                    if constexpr (LPR == 32) ss = xor16_sum(ss);
                } else {
    #pragma unroll
                    for (int o = 1; o < LPR; o <<= 1) ss += __shfl_xor(ss, o);
                }
                const float inv = rsqrtf(ss / static_cast<float>(D) + p.eps);
    #pragma unroll
                for (int j = 0; j < 4; ++j)
                    nq[k][j] = cvt_pk<bf16_t>(x[2 * j] * inv * (wt[2 * j] + 1.0f), x[2 * j + 1] * inv * (wt[2 * j + 1] + 1.0f));
                st16(qs + (k * RPI + rr) * D + 8 * c, nq[k]);
            }
            if (hr > 0) {
                // RoPE: the rotating lanes read their partner's 8 normed dims back
                // (all reads are issued before any write; LDS is in order per wave).
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const int pc = 8 * c < hr ? 8 * c + hr : 8 * c - hr;
                u32x4_v yq[NIN];
    #pragma unroll
                for (int k = 0; k < NIN; ++k)
                    yq[k] = rot ? ld16(qs + (k * RPI + rr) * D + pc) : u32x4_v{0u, 0u, 0u, 0u};
                if (rot) {
    #pragma unroll
                    for (int k = 0; k < NIN; ++k) {
                        float x[8], y[8], cs[8], sn[8];
                        unpack8<bf16_t>(nq[k], x);
                        unpack8<bf16_t>(yq[k], y);
                        unpack8<bf16_t>(cw[k], cs);
                        unpack8<bf16_t>(sw[k], sn);
                        const float sg = 8 * c < hr ? -1.0f : 1.0f;
                        u32x4_v o;
    #pragma unroll
                        for (int j = 0; j < 4; ++j)
                            o[j] = cvt_pk<bf16_t>(x[2 * j] * cs[2 * j] + sg * y[2 * j] * sn[2 * j],
                                               x[2 * j + 1] * cs[2 * j + 1] + sg * y[2 * j + 1] * sn[2 * j + 1]);
                        st16(qs + (k * RPI + rr) * D + 8 * c, o);
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    #pragma unroll
            for (int s = 0; s < KS; ++s) qb[s] = to_op<op_t>(ld16(qs + (lane & 15) * D + 32 * s + 8 * g4));
    }

    f32x4_v oacc[DBK];
#pragma unroll
    for (int d = 0; d < DBK; ++d) oacc[d] = f32x4_v{0.f, 0.f, 0.f, 0.f};
    float m_run = -1e30f;
    // Row sums on the MFMA pipe: lacc += ones * P^T sums each query's 16-bit
    // weights exactly as the PV product uses them (every lane ends up with
    // its own row's total in lacc[0]; the four entries are equal).
    f32x4_v lacc = {0.f, 0.f, 0.f, 0.f};
    const op_t ones = to_op<op_t>(u32x4_v{kOnePair<QT>, kOnePair<QT>, kOnePair<QT>, kOnePair<QT>});
    const float c2 = p.scale_log2;

    // Per-lane LDS bases: K row (lane & 15), dims 8 g4 (for r < 16,
    // koff(r + 16 m) - koff(r) does not depend on r, so the other rows are the
    // compile-time offsets koff(16 m)).  V^T: dim (lane & 15) of each pair,
    // chunk 4 u + g4 of 32-key step u (swizzled granule).
    const int kbase_off = T::koff(lane & 15) + 16 * g4;
    const int vx = (lane & 15) >> 1;
    const int vrd0 = T::KBYTES + 16 * (8 * (lane & 15) + (g4 ^ vx));
    const int vrd1 = T::KBYTES + 16 * (8 * (lane & 15) + ((4 + g4) ^ vx));
    for (int it = 0; it < ntiles; ++it) {
        const int k0 = it * 64;
        const int st = (gt + it + 1) & 1;
        __syncthreads();                // the copy waves' tile `it` has landed; stage st^1 is free again
        if (k0 >= lim_wave) continue;   // the whole tile is past this wave's rows

        const uint8_t* kl = lds + st * T::STAGE + kbase_off;
        const uint8_t* vl0 = lds + st * T::STAGE + vrd0;
        const uint8_t* vl1 = lds + st * T::STAGE + vrd1;

        // S^T = K Q^T, four 16-key blocks.
        f32x4_v sacc[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) sacc[kb] = f32x4_v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const op_t ka = to_op<op_t>(ld16(kl + T::koff(16 * kb) + 64 * s));
                sacc[kb] = Mfma16<QT>::mma(ka, qb[s], sacc[kb]);
            }
        }
        __builtin_amdgcn_sched_group_barrier(0x100, kKLA, 0);
#pragma unroll
        for (int i = 0; i < 4 * KS - kKLA; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kKLA, 0);
        __builtin_amdgcn_sched_barrier(0);

        // Online softmax, base 2, exact running max.  Lane holds row myrow and
        // keys k0 + 16 kb + 4 g4 + i.
        const bool need_mask = (k0 + 64 > off + row_w0 + 1) || (k0 + 64 > L);
        if (need_mask) {
            // Only tiles crossing the diagonal or kv_len: a real branch (the
            // empty volatile asm keeps the compiler from if-converting it).
            asm volatile("" ::: "memory");
            const int rem = lim_row - (k0 + 4 * g4);  // key 16 kb + i is valid iff < rem
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (16 * kb + i >= rem) sacc[kb][i] = -INFINITY;
        }
        float mx = max3_raw(sacc[0][0], sacc[0][1], sacc[0][2]);
        mx = max3_raw(mx, sacc[0][3], sacc[1][0]);
        mx = max3_raw(mx, sacc[1][1], sacc[1][2]);
        mx = max3_raw(mx, sacc[1][3], sacc[2][0]);
        mx = max3_raw(mx, sacc[2][1], sacc[2][2]);
        mx = max3_raw(mx, sacc[2][3], sacc[3][0]);
        mx = max3_raw(mx, sacc[3][1], sacc[3][2]);
        mx = max3_raw(mx, sacc[3][3], sacc[3][3]);
        mx = xor16_max(mx);
        mx = xor32_max(mx) * c2;
        if (__any(mx > m_run + p.rescale_slack)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
#pragma unroll
            for (int i = 0; i < 4; ++i) lacc[i] *= alpha;
#pragma unroll
            for (int d = 0; d < DBK; ++d)
#pragma unroll
                for (int i = 0; i < 4; ++i) oacc[d][i] *= alpha;
        }
        const float m_use = m_run;
        op_t pk[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            u32x4_v w;
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float a = __builtin_amdgcn_exp2f(fmaf(sacc[2 * u + hb][2 * j], c2, -m_use));
                    const float c = __builtin_amdgcn_exp2f(fmaf(sacc[2 * u + hb][2 * j + 1], c2, -m_use));
                    w[2 * hb + j] = cvt_pk<QT>(a, c);
                }
            pk[u] = to_op<op_t>(w);
        }
        __builtin_amdgcn_sched_barrier(0);

        // O^T += V^T P^T: two 32-key steps.  A operand: dims 16 d + (lane & 15),
        // the 8 keys of staging chunk 4 u + g4, which are exactly the keys
        // 32 u + 4 g4 + {0..3} and 32 u + 16 + 4 g4 + {0..3} that the lane's
        // B operand (P^T) carries.
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int d = 0; d < DBK; ++d) {
                const op_t va = to_op<op_t>(ld16((u ? vl1 : vl0) + 2048 * d));
                oacc[d] = Mfma16<QT>::mma(va, pk[u], oacc[d]);
            }
            lacc = Mfma16<QT>::mma(ones, pk[u], lacc);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, kVLA, 1);
#pragma unroll
        for (int i = 0; i < 2 * DBK - kVLA; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kVLA, 1);
    }

    __syncthreads();                    // item end (the copy waves' last barrier)
    // ------------------------------------------------ epilogue
    // O^T C layout: lane holds row myrow, dims 16 d + 4 g4 + i.
    const float l_tot = lacc[0];
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    if constexpr (!FUSED) {
        if (!row_ok) return;
        float* orow = p.out_f32 + b * p.o_bs + h * p.o_hs + static_cast<int64_t>(myrow) * p.o_rs;
#pragma unroll
        for (int d = 0; d < DBK; ++d) {
            f32x4_v o = {oacc[d][0] * inv, oacc[d][1] * inv, oacc[d][2] * inv, oacc[d][3] * inv};
            *reinterpret_cast<f32x4_v*>(orow + 16 * d + 4 * g4) = o;
        }
    } else {
        // bf16(attn) * sigmoid(gate), bf16 out [S, Hq*D] (prefill_engine.rs:2263-2308).
        // The accumulator layout gives a lane 8 bytes of each of 16 rows, so
        // the rows go through the wave's own LDS rows (the stage the next
        // item stages its queries in; its tiles are read by now) and the gate
        // loads and output stores move 16 contiguous bytes a lane: row
        // k RPI + rr, dims 8c .. 8c+7.  16-byte chunks are XOR-swizzled by
        // row, so the 16 rows of a write land in different banks.
        constexpr int LPR = D / 8, RPI = 64 / LPR, NIN = 16 / RPI, CM = LPR - 1;
        // the lane index afresh (mbcnt), so that no new value stays live
        // through the key loop, which runs at the register limit
        const int ln = static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
        const int c = ln % LPR, rr = ln / LPR, g4e = ln >> 4;
        u32x4_v gq[NIN];
#pragma unroll
        for (int k = 0; k < NIN; ++k) {
            const int row = min(row_w0 + k * RPI + rr, S - 1);
            gq[k] = ld16(p.gate + h * p.q_hs + static_cast<int64_t>(row) * p.q_rs + 8 * c);
        }
        uint8_t* const os = lds + ((gt + ntiles) & 1) * T::STAGE + wave * 16 * D * 2;
        const int r16 = ln & 15;
#pragma unroll
        for (int d = 0; d < DBK; ++d) {
            const int ch = 2 * d + (g4e >> 1);
            const u32x2_v a = {cvt_pk<bf16_t>(oacc[d][0] * inv, oacc[d][1] * inv),
                               cvt_pk<bf16_t>(oacc[d][2] * inv, oacc[d][3] * inv)};
            *reinterpret_cast<u32x2_v*>(os + r16 * D * 2 + ((ch ^ (r16 & CM)) * 16) + (g4e & 1) * 8) = a;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int k = 0; k < NIN; ++k) {
            const int rl = k * RPI + rr, row = row_w0 + rl;
            const u32x4_v av = ld16(os + rl * D * 2 + ((c ^ (rl & CM)) * 16));
            u32x4_v o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float r2[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const float a = bf16_bits_to_f32(hh ? av[e] >> 16 : av[e] & 0xFFFFu);
                    const float g = bf16_bits_to_f32(hh ? gq[k][e] >> 16 : gq[k][e] & 0xFFFFu);
                    // sigmoid(g) = 1 / (1 + 2^(-g log2 e)), hardware exp2 and reciprocal
                    r2[hh] = a * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * kLog2e));
                }
                o[e] = cvt_pk<bf16_t>(r2[0], r2[1]);
            }
            if (row < S) st16(p.out_bf16 + static_cast<int64_t>(row) * p.Hq * D + h * D + 8 * c, o);
        }
    }
    };

    // Separate loops for the copy and the compute waves (same items, same
    // barrier count per item), so neither keeps the other's registers live.
    if (dyn) {
        claim_next(0);
        __builtin_amdgcn_s_barrier();  // item 0's claim is visible to every wave
    }
    if (wave >= kPrefillWaves) {
        copy_items();
    } else {
        int gt = 0, qt, h, b;
        for (int r = 0; item_at(r, qt, h, b); ++r) {
            run_item(qt, h, b, gt);
            gt += tiles_of(qt);
        }
    }
#endif
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
// V^T staging for the prefill kernel.  The PV product needs, per lane, 8
// consecutive keys of one dim; the cache stores token rows.  This pass writes
// each kv head's V transposed, dims as rows of vt_ld positions (kv_len rounded
// up to 64, zero past kv_len), with the keys of every 32-key group stored in
// the order the S^T accumulator hands them to the PV MFMA: position
// 8 g + j holds key 4 g + j for j < 4 and key 16 + 4 g + (j - 4) for j >= 4.
// One workgroup per (64-key tile, kv head, sequence).
// ----------------------------------------------------------------------------
__device__ __forceinline__ constexpr int vt_key_of_position(int p) {
    return (p & ~31) + ((p & 4) ? 16 : 0) + 4 * ((p & 31) >> 3) + (p & 3);
}

template <int D>
__global__ __launch_bounds__(256) void vt_stage_kernel(KvView kv, uint16_t* vt, int Hkv, int L, int ld) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[64][D + 8];
    const int t0 = blockIdx.x * 64, h = blockIdx.y, b = blockIdx.z;
    for (int idx = threadIdx.x; idx < 64 * (D / 8); idx += 256) {
        const int r = idx / (D / 8), c = idx % (D / 8);
        const int t = t0 + r;
        u32x4_v w = {0u, 0u, 0u, 0u};
        if (t < L) w = ld16(reinterpret_cast<const uint16_t*>(kv.v) + kv.row(b, h, t, D) + 8 * c);
        *reinterpret_cast<u32x4_v*>(&tile[r][8 * c]) = w;
    }
    __syncthreads();
    uint16_t* dst = vt + (static_cast<int64_t>(b) * Hkv + h) * D * ld + t0;
    for (int idx = threadIdx.x; idx < D * 8; idx += 256) {
        const int d = idx >> 3, c = idx & 7;
        u32x4_v w;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            w[j] = static_cast<uint32_t>(tile[vt_key_of_position(8 * c + 2 * j)][d]) |
                   (static_cast<uint32_t>(tile[vt_key_of_position(8 * c + 2 * j + 1)][d]) << 16);
        st16(dst + static_cast<int64_t>(d) * ld + 8 * c, w);
    }
}

// Fused prefill, bf16 cache: one pass that appends the chunk's new tokens to
// the cache and does vt_stage_kernel's work for every position.  One
// workgroup per (64-position tile, kv head); lane c of a row holds dims
// 8c .. 8c + 7 (16-byte accesses).  New tokens (position >= off): K gets
// RMSNorm with (1 + w) and rotate-half RoPE (bf16 after each step, RoPE
// partners read back through an LDS row), K and V go to the cache, and V to
// the LDS tile; prefix positions read V back from the cache; the tile is then
// written out transposed in the PV operand's key order.
struct KvStageParams {
    const uint16_t* k_new;  // [S, Hkv*D]
    const uint16_t* v_new;
    const uint16_t* k_norm_w;
    const uint16_t* cos_t;
    const uint16_t* sin_t;
    KvView kv;
    uint16_t* vt;           // [Hkv, D, ld]
    uint16_t* kst;          // fp8 cache: bf16 K rows [Hkv, ld, D] for the attention kernel
    int S, Hkv, off, L, ld, half_rot;
    float eps;
};

constexpr int kKvStageWaves = 16;  // 4 per SIMD: the rows' memory round trips overlap

// One row's e4m3 codes with the per-(token, head) absmax scale, as the fused
// decode append writes them (full_attention_4b.hip:5228-5281, OCP codec): the
// row's LPR lanes hold 8 values each; returns the lane's 8 codes, sets sc.
template <int LPR>
__device__ __forceinline__ u32x2_v quantize_row8(const float (&x)[8], float& sc) {
    float am = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(x[e]));
#pragma unroll
    for (int m = 1; m < LPR; m <<= 1) am = fmaxf(am, __shfl_xor(am, m));
    sc = fmaxf(am / 448.0f, 1e-12f);
    const float inv = 1.0f / sc;
    return u32x2_v{f32x4_to_fp8x4(x[0] * inv, x[1] * inv, x[2] * inv, x[3] * inv),
                   f32x4_to_fp8x4(x[4] * inv, x[5] * inv, x[6] * inv, x[7] * inv)};
}

// 8 e4m3 codes times their row scale, rounded to bf16.
__device__ __forceinline__ u32x4_v dequant8_bf16(u32x2_v w, float sc) {
    u32x4_v r;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const f32x2_v lo = fp8x2_to_f32(w[i], false);
        const f32x2_v hi = fp8x2_to_f32(w[i], true);
        r[2 * i] = pk2<bf16_t>(lo[0] * sc, lo[1] * sc);
        r[2 * i + 1] = pk2<bf16_t>(hi[0] * sc, hi[1] * sc);
    }
    return r;
}

template <int D, bool FP8>
__global__ __launch_bounds__(64 * kKvStageWaves) void kv_stage_kernel(KvStageParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t vtile[64][D + 8];
    constexpr int LPR = D / 8;          // lanes per row
    constexpr int RPI = 64 / LPR;       // rows per wave instruction
    __shared__ __attribute__((aligned(16))) uint16_t krow[kKvStageWaves][RPI][D];  // per-wave RoPE exchange
    const int t0 = blockIdx.x * 64, h = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = lane % LPR;
    const int hr = p.half_rot;
    const bool rot = 8 * c < 2 * hr;
    float wt[8];
    unpack8<bf16_t>(ld16(p.k_norm_w + 8 * c), wt);
    for (int r0 = wave * RPI; r0 < 64; r0 += kKvStageWaves * RPI) {
        const int r = r0 + lane / LPR;
        const int pos = t0 + r;
        u32x4_v vw = {0u, 0u, 0u, 0u};
        if (pos < p.L) {
            const int64_t o = p.kv.row(0, h, pos, D) + 8 * c;
            if (pos >= p.off) {
                const int64_t src = (static_cast<int64_t>(pos - p.off) * p.Hkv + h) * D + 8 * c;
                const u32x4_v kw = ld16(p.k_new + src);
                vw = ld16(p.v_new + src);
                u32x4_v cw4 = {0u, 0u, 0u, 0u}, sw4 = {0u, 0u, 0u, 0u};
                if (rot) {
                    const int64_t ti = static_cast<int64_t>(pos) * hr + (8 * c < hr ? 8 * c : 8 * c - hr);
                    cw4 = ld16(p.cos_t + ti);
                    sw4 = ld16(p.sin_t + ti);
                }
                float x[8];
                unpack8<bf16_t>(kw, x);
                float ss = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
                // the row's LPR lanes are aligned groups of the wave
#pragma unroll
                for (int m = 1; m < LPR; m <<= 1) ss += __shfl_xor(ss, m);
                const float inv = rsqrtf(ss / static_cast<float>(D) + p.eps);
                u32x4_v nq;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    nq[e] = pk2<bf16_t>(x[2 * e] * inv * (wt[2 * e] + 1.0f), x[2 * e + 1] * inv * (wt[2 * e + 1] + 1.0f));
                st16(&krow[wave][lane / LPR][8 * c], nq);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (rot) {
                    const int pc = 8 * c < hr ? 8 * c + hr : 8 * c - hr;
                    float xn[8], y[8], cs[8], sn[8];
                    unpack8<bf16_t>(nq, xn);
                    unpack8<bf16_t>(ld16(&krow[wave][lane / LPR][pc]), y);
                    unpack8<bf16_t>(cw4, cs);
                    unpack8<bf16_t>(sw4, sn);
                    const float sg = 8 * c < hr ? -1.0f : 1.0f;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        nq[e] = pk2<bf16_t>(xn[2 * e] * cs[2 * e] + sg * y[2 * e] * sn[2 * e],
                                            xn[2 * e + 1] * cs[2 * e + 1] + sg * y[2 * e + 1] * sn[2 * e + 1]);
                }
                if constexpr (!FP8) {
                    st16(reinterpret_cast<uint16_t*>(p.kv.k) + o, nq);
                    st16(reinterpret_cast<uint16_t*>(p.kv.v) + o, vw);
                } else {
                    // the attention reads this chunk's K and V unquantised (the
                    // reference runs prefill in bf16 and quantises the cache
                    // afterwards); the cache gets the e4m3 codes and scales
                    st16(p.kst + (static_cast<int64_t>(h) * p.ld + pos) * D + 8 * c, nq);
                    float xk[8], xv[8], sk, sv;
                    unpack8<bf16_t>(nq, xk);
                    unpack8<bf16_t>(vw, xv);
                    const u32x2_v qk8 = quantize_row8<LPR>(xk, sk);
                    const u32x2_v qv8 = quantize_row8<LPR>(xv, sv);
                    *reinterpret_cast<u32x2_v*>(p.kv.k + o) = qk8;
                    *reinterpret_cast<u32x2_v*>(p.kv.v + o) = qv8;
                    if (c == 0) {
                        const int64_t so = p.kv.srow(0, h, pos);
                        p.kv.ks[so] = sk;
                        p.kv.vs[so] = sv;
                    }
                }
            } else if constexpr (!FP8) {
                vw = ld16(reinterpret_cast<const uint16_t*>(p.kv.v) + o);
            } else {
                // prefix from the fp8 cache: codes times scale, as bf16
                const int64_t so = p.kv.srow(0, h, pos);
                st16(p.kst + (static_cast<int64_t>(h) * p.ld + pos) * D + 8 * c,
                     dequant8_bf16(*reinterpret_cast<const u32x2_v*>(p.kv.k + o), p.kv.ks[so]));
                vw = dequant8_bf16(*reinterpret_cast<const u32x2_v*>(p.kv.v + o), p.kv.vs[so]);
            }
        }
        st16(&vtile[r][8 * c], vw);
    }
    __syncthreads();
    uint16_t* dst = p.vt + static_cast<int64_t>(h) * D * p.ld + t0;
    for (int idx = threadIdx.x; idx < D * 8; idx += 64 * kKvStageWaves) {
        const int d = idx >> 3, cc = idx & 7;
        u32x4_v w;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            w[j] = static_cast<uint32_t>(vtile[vt_key_of_position(8 * cc + 2 * j)][d]) |
                   (static_cast<uint32_t>(vtile[vt_key_of_position(8 * cc + 2 * j + 1)][d]) << 16);
        st16(dst + static_cast<int64_t>(d) * p.ld + 8 * cc, w);
    }
}

// Stages V^T for `B` sequences of `L` keys into the prefill workspace slot of
// `device` and points `p` at it.  Returns hipSuccess or the failing error.
static hipError_t stage_vt(int device, hipStream_t st, const KvView& kv, int B, int Hkv, int L, int D,
                           PrefillParams& p) {
    const int ld = (L + 63) / 64 * 64;
    const size_t bytes = static_cast<size_t>(B) * Hkv * D * ld * 2;
    void* ws = device_workspace(device, bytes, kWorkspacePrefill);
    if (!ws) return hipErrorOutOfMemory;
    p.vt = static_cast<const uint16_t*>(ws);
    p.vt_ld = ld;
    const dim3 grid(ld / 64, Hkv, B);
    uint16_t* vt = static_cast<uint16_t*>(ws);
    switch (D) {
    case 64: hipLaunchKernelGGL(vt_stage_kernel<64>, grid, dim3(256), 0, st, kv, vt, Hkv, L, ld); break;
    case 128: hipLaunchKernelGGL(vt_stage_kernel<128>, grid, dim3(256), 0, st, kv, vt, Hkv, L, ld); break;
    case 256: hipLaunchKernelGGL(vt_stage_kernel<256>, grid, dim3(256), 0, st, kv, vt, Hkv, L, ld); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ----------------------------------------------------------------------------
// Host side
// ----------------------------------------------------------------------------
// Persistent grid: one workgroup per CU (a workgroup's LDS allows no second
// one), a multiple of 8 so the XCD-aware item lists stay aligned, and never
// more workgroups than items.
template <typename QT, bool FUSED>
static hipError_t launch_prefill(int device, int D, hipStream_t st, PrefillParams& p) {
    const int items = p.nqt * p.Hq * p.B;
    int n = device_cu_count(device);
    if (n <= 0) n = 256;
    n = n >= 8 ? n & ~7 : n;
    p.n_wg = items < n ? items : n;
    const dim3 grid(static_cast<unsigned>(p.n_wg));
    switch (D) {
    case 64: hipLaunchKernelGGL((prefill_kernel<QT, 64, FUSED>), grid, dim3(kPrefillThreads), 0, st, p); break;
    case 128: hipLaunchKernelGGL((prefill_kernel<QT, 128, FUSED>), grid, dim3(kPrefillThreads), 0, st, p); break;
    case 256: hipLaunchKernelGGL((prefill_kernel<QT, 256, FUSED>), grid, dim3(kPrefillThreads), 0, st, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

static float rescale_slack() {
    const char* v = getenv("SUPERSONIC_PREFILL_RESCALE_SLACK");
    return (v && *v) ? static_cast<float>(atof(v)) : 8.0f;
}

int prefill_dropin(int dtype, size_t device, size_t B, size_t Hq, size_t Hkv, size_t q_len, size_t kv_len, size_t D,
                   size_t groups, float scale, size_t off, const void* q, const void* k, const void* v, void* out) {
    if (dtype != 0 && dtype != 1 && dtype != 2) return 64;
    if (D == 0 || D > 512 || Hkv == 0 || groups == 0 || Hq != Hkv * groups) return 14;
    if (dtype != 1 && D != 64 && D != 128 && D != 256) {
        // General head size (the reference takes any D <= 512): D <= 256 runs
        // the MFMA kernel on copies zero-padded to the next native tile (the
        // zero dims add nothing to q.k, and the padded output dims are dropped);
        // larger D runs the f32 kernel on f32 copies.
        ScopedDevice scoped(static_cast<int>(device));
        if (B == 0 || Hq == 0 || q_len == 0) return hipDeviceSynchronize() == hipSuccess ? 0 : 12;
        const int64_t nq = static_cast<int64_t>(B * Hq * q_len), nk = static_cast<int64_t>(B * Hkv * kv_len);
        const int d = static_cast<int>(D);
        ScratchBuffers sb;
        int rc;
        if (D <= 256) {
            const int dp = D <= 64 ? 64 : (D <= 128 ? 128 : 256);
            void* qp = sb.get(nq * dp * 2);
            void* kp = sb.get(nk * dp * 2);
            void* vp = sb.get(nk * dp * 2);
            void* op = sb.get(nq * dp * 4);
            if (!qp || !kp || !vp || !op) return 2;
            if (repack_rows(dtype, dtype, q, qp, nq, 1, d, 0, d, dp, nullptr) != hipSuccess ||
                repack_rows(dtype, dtype, k, kp, nk, 1, d, 0, d, dp, nullptr) != hipSuccess ||
                repack_rows(dtype, dtype, v, vp, nk, 1, d, 0, d, dp, nullptr) != hipSuccess)
                return 11;
            rc = prefill_dropin(dtype, device, B, Hq, Hkv, q_len, kv_len, dp, groups, scale, off, qp, kp, vp, op);
            if (rc == 0 && repack_rows(1, 1, op, out, nq, 1, dp, 0, d, d, nullptr) != hipSuccess) rc = 11;
        } else {
            void* qf = sb.get(nq * d * 4);
            void* kf = sb.get(nk * d * 4);
            void* vf = sb.get(nk * d * 4);
            if (!qf || !kf || !vf) return 2;
            if (repack_rows(dtype, 1, q, qf, nq, 1, d, 0, d, d, nullptr) != hipSuccess ||
                repack_rows(dtype, 1, k, kf, nk, 1, d, 0, d, d, nullptr) != hipSuccess ||
                repack_rows(dtype, 1, v, vf, nk, 1, d, 0, d, d, nullptr) != hipSuccess)
                return 11;
            rc = prefill_dropin(1, device, B, Hq, Hkv, q_len, kv_len, D, groups, scale, off, qf, kf, vf, out);
        }
        if (hipDeviceSynchronize() != hipSuccess && rc == 0) rc = 12;
        return rc;
    }
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
    p.Hkv = static_cast<int>(Hkv);
    p.G = static_cast<int>(groups);
    p.S = static_cast<int>(q_len);
    p.L = static_cast<int>(kv_len);
    p.off = static_cast<int>(off);
    p.scale_log2 = scale * kLog2e;
    p.rescale_slack = rescale_slack();
    p.nqt = static_cast<int>((q_len + 127) / 128);
    p.out_f32 = static_cast<float*>(out);
    p.o_rs = p.q_rs;
    p.o_hs = p.q_hs;
    p.o_bs = p.q_bs;
    p.B = static_cast<int>(B);
    if (kv_len > 0 && stage_vt(static_cast<int>(device), nullptr, p.kv, static_cast<int>(B), static_cast<int>(Hkv),
                               static_cast<int>(kv_len), static_cast<int>(D), p) != hipSuccess)
        return 11;
    const int dev = static_cast<int>(device);
    const hipError_t e = dtype == 0 ? launch_prefill<f16_t, false>(dev, static_cast<int>(D), nullptr, p)
                                    : launch_prefill<bf16_t, false>(dev, static_cast<int>(D), nullptr, p);
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

extern "C" size_t supersonic_attn_gfx950_prefill_workspace_size(int kv_dtype, size_t kv_heads, size_t head_dim,
                                                                size_t chunk_len, size_t chunk_start) {
    const size_t L = chunk_start + chunk_len;
    if (L > 0x7FFFFFFF || kv_heads > 4096 || head_dim > 512) return 0;
    const size_t ld = (L + 63) / 64 * 64;
    const size_t stage = kv_heads * head_dim * ld * 2;  // V^T staging
    return kv_dtype == SUPERSONIC_KV_FP8_E4M3 ? 2 * stage : stage;  // + the bf16 K rows of an fp8 cache
}

namespace ssa {
// The fused prefill with an optional dynamic schedule (claims: zeroed claim
// counters, PrefillParams::claims); supersonic_attn_gfx950_prefill is the
// static one.
int prefill_native(size_t device_ordinal, void* stream, int kv_dtype, size_t q_heads, size_t kv_heads,
                   size_t head_dim, size_t rotary_dim, size_t chunk_len, size_t chunk_start, float eps, float scale,
                   const void* q_proj, const void* k_new, const void* v_new, const void* q_norm_w,
                   const void* k_norm_w, const void* cos_table, const void* sin_table,
                   const supersonic_kv_cache* cache, void* out, void* workspace, size_t workspace_bytes,
                   unsigned* claims) {
    if (kv_dtype != SUPERSONIC_KV_BF16 && kv_dtype != SUPERSONIC_KV_FP8_E4M3) return SUPERSONIC_ERR_DTYPE;
    const bool fp8 = kv_dtype == SUPERSONIC_KV_FP8_E4M3;
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return SUPERSONIC_ERR_HEAD_DIM;
    if (kv_heads == 0 || q_heads % kv_heads != 0) return SUPERSONIC_ERR_HEADS;
    if (rotary_dim > head_dim || (rotary_dim / 2) % 16 != 0) return SUPERSONIC_ERR_ROTARY;
    if (!q_proj || !k_new || !v_new || !q_norm_w || !k_norm_w || !out) return SUPERSONIC_ERR_NULL;
    if (rotary_dim > 0 && (!cos_table || !sin_table)) return SUPERSONIC_ERR_NULL;
    if (chunk_len + chunk_start > 0x7FFFFFFF || q_heads > 4096) return SUPERSONIC_ERR_RANGE;
    KvView kv;
    if (int rc = make_view(cache, fp8, &kv)) return rc;
    if (kv.bt && kv.page_size % 64 != 0) return SUPERSONIC_ERR_CACHE;
    if (chunk_len == 0) return 0;
    ScopedDevice scoped(static_cast<int>(device_ordinal));
    hipStream_t st = static_cast<hipStream_t>(stream);


    PrefillParams p{};
    p.q = static_cast<const uint16_t*>(q_proj);
    p.q_bs = 0;
    p.q_hs = 2 * static_cast<int64_t>(head_dim);
    p.q_rs = static_cast<int64_t>(q_heads) * 2 * head_dim;
    p.kv = kv;
    p.Hq = static_cast<int>(q_heads);
    p.Hkv = static_cast<int>(kv_heads);
    p.G = static_cast<int>(q_heads / kv_heads);
    p.S = static_cast<int>(chunk_len);
    p.L = static_cast<int>(chunk_start + chunk_len);
    p.off = static_cast<int>(chunk_start);
    p.scale_log2 = scale * kLog2e;
    p.rescale_slack = rescale_slack();
    p.nqt = static_cast<int>((chunk_len + 127) / 128);
    p.out_bf16 = static_cast<uint16_t*>(out);
    p.gate = static_cast<const uint16_t*>(q_proj) + head_dim;
    p.q_norm_w = static_cast<const uint16_t*>(q_norm_w);
    p.cos_t = static_cast<const uint16_t*>(cos_table);
    p.sin_t = static_cast<const uint16_t*>(sin_table);
    p.half_rot = static_cast<int>(rotary_dim / 2);
    p.eps = eps;
    p.B = 1;
    p.claims = claims;
    // K norm + RoPE + cache append for the chunk and the V^T staging of every
    // position, in one pass
    {
        const int ld = (p.L + 63) / 64 * 64;
        // V^T staging, then (fp8 cache) the bf16 K rows the attention reads
        const size_t stage_bytes = static_cast<size_t>(p.Hkv) * head_dim * ld * 2;
        const size_t need = fp8 ? 2 * stage_bytes : stage_bytes;
        void* ws = workspace;
        if (ws) {
            if (workspace_bytes < need) return SUPERSONIC_ERR_WORKSPACE;
        } else {
            ws = device_workspace(static_cast<int>(device_ordinal), need, kWorkspacePrefill);
        }
        if (!ws) return SUPERSONIC_ERR_WORKSPACE;
        p.vt = static_cast<const uint16_t*>(ws);
        p.vt_ld = ld;
        uint16_t* kst = fp8 ? reinterpret_cast<uint16_t*>(static_cast<uint8_t*>(ws) + stage_bytes) : nullptr;
        if (fp8) {
            // the attention kernel's K: the contiguous staging rows
            KvView ks{};
            ks.k = reinterpret_cast<uint8_t*>(kst);
            ks.head_stride = static_cast<int64_t>(ld) * head_dim;
            ks.seq_stride = static_cast<int64_t>(p.Hkv) * ld * head_dim;
            ks.page_size = 1;
            p.kv = ks;
        }
        KvStageParams kp{};
        kp.k_new = static_cast<const uint16_t*>(k_new);
        kp.v_new = static_cast<const uint16_t*>(v_new);
        kp.k_norm_w = static_cast<const uint16_t*>(k_norm_w);
        kp.cos_t = static_cast<const uint16_t*>(cos_table);
        kp.sin_t = static_cast<const uint16_t*>(sin_table);
        kp.kv = kv;
        kp.vt = static_cast<uint16_t*>(ws);
        kp.kst = kst;
        kp.S = static_cast<int>(chunk_len);
        kp.Hkv = static_cast<int>(kv_heads);
        kp.off = static_cast<int>(chunk_start);
        kp.L = p.L;
        kp.ld = ld;
        kp.half_rot = static_cast<int>(rotary_dim / 2);
        kp.eps = eps;
        const dim3 grid(ld / 64, kp.Hkv);
        const dim3 blk(64 * kKvStageWaves);
        switch (head_dim * 2 + (fp8 ? 1 : 0)) {
        case 128: hipLaunchKernelGGL((kv_stage_kernel<64, false>), grid, blk, 0, st, kp); break;
        case 129: hipLaunchKernelGGL((kv_stage_kernel<64, true>), grid, blk, 0, st, kp); break;
        case 256: hipLaunchKernelGGL((kv_stage_kernel<128, false>), grid, blk, 0, st, kp); break;
        case 257: hipLaunchKernelGGL((kv_stage_kernel<128, true>), grid, blk, 0, st, kp); break;
        case 512: hipLaunchKernelGGL((kv_stage_kernel<256, false>), grid, blk, 0, st, kp); break;
        default: hipLaunchKernelGGL((kv_stage_kernel<256, true>), grid, blk, 0, st, kp); break;
        }
        if (hipGetLastError() != hipSuccess) return SUPERSONIC_ERR_LAUNCH;
    }
    const ProfileEvents prof = take_profile_events();
    if (prof.before) (void)hipEventRecord(prof.before, st);
    if (launch_prefill<bf16_t, true>(static_cast<int>(device_ordinal), static_cast<int>(head_dim), st, p) != hipSuccess)
        return SUPERSONIC_ERR_LAUNCH;
    if (prof.after) (void)hipEventRecord(prof.after, st);
    return 0;
}
}  // namespace ssa

extern "C" int supersonic_attn_gfx950_prefill(
    size_t device_ordinal, void* stream, int kv_dtype, size_t q_heads, size_t kv_heads, size_t head_dim,
    size_t rotary_dim, size_t chunk_len, size_t chunk_start, float eps, float scale, const void* q_proj,
    const void* k_new, const void* v_new, const void* q_norm_w, const void* k_norm_w, const void* cos_table,
    const void* sin_table, const supersonic_kv_cache* cache, void* out, void* workspace, size_t workspace_bytes) {
    return ssa::prefill_native(device_ordinal, stream, kv_dtype, q_heads, kv_heads, head_dim, rotary_dim, chunk_len,
                               chunk_start, eps, scale, q_proj, k_new, v_new, q_norm_w, k_norm_w, cos_table,
                               sin_table, cache, out, workspace, workspace_bytes, nullptr);
}
