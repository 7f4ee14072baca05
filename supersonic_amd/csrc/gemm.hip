// bf16 GEMM out = a . w^T for the prefill-sized projections (rows > the
// weight-streaming limit): the reference's matmul_rhs_transposed_tiled
// (kernels/full_attention_4b.hip:2513-2575) and the hipBLASLt calls the
// projection entry points used before, as one MFMA kernel for gfx950.
//
// Workgroup tile 256 x 256, eight waves in a 2 x 4 grid (two a SIMD, so one
// wave's MFMAs run while the other waits), each wave 128 x 64 on
// v_mfma_f32_32x32x16_bf16 (4 x 2 blocks of 32 x 32, 128 fp32 accumulators
// per lane).  k advances 64 at a time through two LDS stages (64 KB a
// stage: a 256 x 64 tile of a and of w) filled by direct global->LDS copies
// one tile ahead, so the copies of the next tile overlap the MFMAs of the
// current one (a depth of 32 with four stages measured 5% slower: twice the
// barriers).  LDS rows are 128 bytes; the 16-byte chunk c of row r is stored
// at c ^ ((r >> 1) & 7): the 16 lanes a 16-byte read serves at once (rows
// r .. r + 15, one chunk) then cover all 64 banks.  Out-of-range rows and k-chunks read as zeros
// (buffer range / offset checks), so any m, n and k % 8 == 0 work.
// Workgroups are mapped to tiles XCD by XCD: consecutive tiles of the order
// (bands of 4 m-tiles, n-major within a band) go to one XCD, whose L2 then
// serves the shared rows of a and w.  One workgroup fits a CU (144 KB of LDS),
// so the tiles run in rounds of one per CU; when the last round would occupy at
// most half the CUs, its tiles run as two workgroups each, over the two halves
// of k, the first handing its fp32 accumulators to the second through the
// caller's workspace.
#include <algorithm>

#include "common.hpp"
#include "gemm.hpp"

namespace ssa {

constexpr int kGBM = 256, kGBN = 256, kGBK = 64, kGStages = kGBK == 32 ? 4 : 2;
constexpr int kGRowB = kGBK * 2;                    // LDS row bytes
constexpr int kGCpr = kGBK / 8;                     // 16-byte chunks a row
constexpr int kGRowsPer256 = 256 / kGRowB;          // rows that share the 64 banks
constexpr int kGSwzShift = kGRowsPer256 == 4 ? 2 : 1;
constexpr int kGCopyRows = 1024 / kGRowB;           // rows one copy instruction moves
#ifndef SSA_GEMM_WAVES
#define SSA_GEMM_WAVES 8
#endif
constexpr int kGWaves = SSA_GEMM_WAVES;             // 8: 2 x 4 waves of 128 x 64; 4: 2 x 2 waves of 128 x 128
constexpr int kGWN = kGWaves / 2;                   // waves along n
constexpr int kGWTN = kGBN / kGWN;                  // wave tile columns
constexpr int kGJB = kGWTN / 32;                    // 32-column blocks a wave
constexpr int kGCopies = kGBM / kGCopyRows / kGWaves;  // copy instructions a wave issues per operand tile
constexpr int kGThreads = 64 * kGWaves;
constexpr int kGTileBytes = kGBM * kGBK * 2;        // 16 KB: one operand tile
constexpr int kGStageBytes = 2 * kGTileBytes;       // a + w
constexpr int kGBand = 4;                           // m-tiles per band of the tile order (4: o_proj +2.5% over 8)
constexpr int kGEpiRow = 2 * kGWTN + 16;            // epilogue LDS row: a wave tile row of bf16 + 16 bytes
constexpr int kGLds = kGStages * kGStageBytes > kGWaves * 128 * kGEpiRow ? kGStages * kGStageBytes : kGWaves * 128 * kGEpiRow;

struct GemmKParams {
    const uint16_t* a;
    int64_t lda, a_bs;
    const uint16_t* w[3];
    void* out[3];
    int n[3];
    int nt_end[3];  // cumulative n-tiles of the segments
    int64_t w_bs, o_bs;
    int m, k, mt, nt, tiles;
    int vec_mask;   // bit s: segment s takes 16-byte output chunks
    // Tail split: the first `full` tiles of the order run whole; each of the
    // remaining `tail` tiles runs as two workgroups over the two halves of k
    // (k-tiles [0, khalf) and [khalf, KT)), the first handing its fp32
    // accumulators to the second through `part` and a pair of counts.
    int full, tail, khalf;
    uint32_t* part;      // [tail][8 waves][32][64 lanes] x 16 bytes
    unsigned* flags;     // [tail][produced, consumed], equal between calls
    int tail_polls;      // bound of the second half's wait
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemm_rsrc(const uint16_t* base, int64_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
    void* u = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
    const int nb = static_cast<int>(min(bytes, static_cast<int64_t>(0x7ffffff0)));
    return __builtin_amdgcn_make_buffer_rsrc(u, static_cast<short>(0), __builtin_amdgcn_readfirstlane(nb), 0x00020000);
}

template <int EPI>
__global__ __launch_bounds__(kGThreads) void gemm_bt_kernel(GemmKParams p) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kGLds];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b = blockIdx.y;

    // ---- tile of this workgroup (XCD-contiguous ranges of the tile order;
    // the tail tiles, two workgroups each, follow the whole ones)
    const int i = blockIdx.x;
    const int T = p.full;
    const bool is_tail = i >= T;
    const int tj = i - T;               // tail: workgroup index within the tail
    const int half = tj & 1;            // tail: which half of k
    const int q = T / 8, r = T % 8;
    const int xcd = i % 8, slot = i / 8;
    const int t = is_tail ? T + (tj >> 1) : (xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot);
    const int band = t / (kGBand * p.nt);
    const int gm = min(kGBand, p.mt - band * kGBand);
    const int tin = t - band * kGBand * p.nt;
    const int tm = band * kGBand + tin % gm;
    const int tn = tin / gm;
    const int seg = tn < p.nt_end[0] ? 0 : (tn < p.nt_end[1] ? 1 : 2);
    const int tn_s = tn - (seg == 0 ? 0 : (seg == 1 ? p.nt_end[0] : p.nt_end[1]));
    const int ns = pick3(p.n, seg);
    const int m0 = tm * kGBM, n0 = tn_s * kGBN;
    const int k = p.k;

    const uint16_t* abase = p.a + b * p.a_bs + static_cast<int64_t>(m0) * p.lda;
    const uint16_t* wbase = pick3(p.w, seg) + b * p.w_bs + static_cast<int64_t>(n0) * k;
    const __amdgpu_buffer_rsrc_t ar = gemm_rsrc(abase, static_cast<int64_t>(p.m - m0) * p.lda * 2);
    const __amdgpu_buffer_rsrc_t wr = gemm_rsrc(wbase, static_cast<int64_t>(ns - n0) * k * 2);

    // k-tiles kt0 .. KT-1 of this workgroup; k-tile kt goes to stage
    // (kt - kt0) % kGStages
    const int KT_all = (k + kGBK - 1) / kGBK;
    const int kt0 = is_tail && half ? p.khalf : 0;
    const int KT = is_tail && !half ? p.khalf : KT_all;
    // ---- direct global->LDS copies: instruction j of a wave moves rows
    // rr = kGCopyRows (kGCopies wave + j) .. of a tile; lane l takes row
    // rr + l / kGCpr and physical chunk l % kGCpr, i.e. the logical chunk
    // (l % kGCpr) ^ swz(row), swz(row) = (row >> kGSwzShift) % kGCpr.
    const int crow = lane / kGCpr;
    // The whole offset goes in the per-lane operand (the range check does
    // not cover the scalar offset).
    constexpr int kOOB = 0x7ffffff0;  // offset past any range: reads zero
    auto issue = [&](int kt) {
        const int k0 = kt * kGBK;
        const int st = (kt - kt0) % kGStages;
        uint8_t* sa = lds + st * kGStageBytes;
        uint8_t* sw = sa + kGTileBytes;
#pragma unroll
        for (int j = 0; j < kGCopies; ++j) {
            const int rr = kGCopyRows * (kGCopies * wave + j);
            const int cchunk = (lane % kGCpr) ^ (((rr + crow) >> kGSwzShift) % kGCpr);
            const bool kin = k0 + 8 * cchunk < k;  // the chunk lies inside k (k % 8 == 0)
            const int ab = __builtin_amdgcn_readfirstlane(rr * kGRowB);
            const int ao = kin ? (rr + crow) * static_cast<int>(p.lda) * 2 + (k0 + 8 * cchunk) * 2 : kOOB;
            const int wo = kin ? (rr + crow) * k * 2 + (k0 + 8 * cchunk) * 2 : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (__attribute__((address_space(3))) void*)(sa + ab), 16, ao, 0,
                                                     0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (__attribute__((address_space(3))) void*)(sw + ab), 16, wo, 0,
                                                     0, 0);
        }
    };

    // ---- accumulators: block (ib, jb) of this wave's 128 x 64
    const int wm = wave / kGWN, wn = wave % kGWN;
    f32x16_v acc[4][kGJB];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int jb = 0; jb < kGJB; ++jb)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[ib][jb][e] = 0.f;

    // operand reads: row (lane % 32) of a 32-row block, logical chunk
    // 2 s + lane / 32 of k16 step s, stored at chunk ^ swz(row)
    const int orow = lane & 31;
    const int sw_x = (orow >> kGSwzShift) % kGCpr;
    const int a_rd = (wm * 128 + orow) * kGRowB;
    const int w_rd = (wn * kGWTN + orow) * kGRowB;

    // Wait until tile kt has landed in LDS (this wave's copies, then every
    // wave's through the barrier); tile kt + 3 then goes to the stage of tile
    // kt - 1, which every wave has finished reading.  A wave issues
    // 2 kGCopies copy instructions a tile.
    auto arrive_tile = [&](int kt) {
        const int ahead = min(KT - 1 - kt, kGStages - 2);
        static_assert(kGStages == 2 || 2 * kGCopies == 4, "vmcnt counts");
        if (ahead >= 2) __builtin_amdgcn_s_waitcnt(0x0F78);        // vmcnt(8): two tiles of 4 in flight
        else if (ahead == 1) __builtin_amdgcn_s_waitcnt(0x0F74);   // vmcnt(4)
        else __builtin_amdgcn_s_waitcnt(0x0F70);                    // vmcnt(0)
        lds_barrier();
        if (kt + kGStages - 1 < KT) issue(kt + kGStages - 1);
    };
    // Fragments of k16 step s of tile kt, and the 16 MFMAs of one step.
    auto read_frags = [&](int kt, int s, bf16x8_v (&af)[4], bf16x8_v (&bfr)[kGJB]) {
        const uint8_t* sa = lds + ((kt - kt0) % kGStages) * kGStageBytes;
        const uint8_t* sw = sa + kGTileBytes;
        const int ck = (2 * s + (lane >> 5)) ^ sw_x;
#pragma unroll
        for (int ib = 0; ib < 4; ++ib)
            af[ib] = *reinterpret_cast<const bf16x8_v*>(sa + a_rd + ib * 32 * kGRowB + ck * 16);
#pragma unroll
        for (int jb = 0; jb < kGJB; ++jb)
            bfr[jb] = *reinterpret_cast<const bf16x8_v*>(sw + w_rd + jb * 32 * kGRowB + ck * 16);
    };
    auto mma_step = [&](const bf16x8_v (&af)[4], const bf16x8_v (&bfr)[kGJB]) {
#pragma unroll
        for (int ib = 0; ib < 4; ++ib)
#pragma unroll
            for (int jb = 0; jb < kGJB; ++jb)
                acc[ib][jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ib], bfr[jb], acc[ib][jb], 0, 0, 0);
    };
#pragma unroll
    for (int u = 0; u < kGStages - 1; ++u)
        if (kt0 + u < KT) issue(kt0 + u);
    // Software pipeline over the k16 steps: the fragments of the next step
    // are read while the MFMAs of the current one run (two register sets).
    bf16x8_v a0[4], b0[kGJB], a1[4], b1[kGJB];
    if (kt0 < KT) {
        arrive_tile(kt0);
        read_frags(kt0, 0, a0, b0);
    }
    constexpr int NS = kGBK / 16;  // k16 steps a tile (even)
    for (int kt = kt0; kt < KT; ++kt) {
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            bf16x8_v(&ca)[4] = (st & 1) ? a1 : a0;
            bf16x8_v(&cb)[kGJB] = (st & 1) ? b1 : b0;
            bf16x8_v(&na)[4] = (st & 1) ? a0 : a1;
            bf16x8_v(&nb)[kGJB] = (st & 1) ? b0 : b1;
            if (st + 1 < NS) {
                read_frags(kt, st + 1, na, nb);
            } else if (kt + 1 < KT) {
                arrive_tile(kt + 1);  // (waits for this wave's outstanding reads too)
                read_frags(kt + 1, 0, na, nb);
            }
            mma_step(ca, cb);
            // the compiler's MFMA / LDS-read interleave strategy 0 (+2-3% on
            // both projection GEMMs against its default schedule)
            __builtin_amdgcn_iglp_opt(0);
        }
    }

    // ---- tail hand-over: the first half stores its accumulators
    // (device-coherent 16-byte stores, lane-contiguous) and, once every
    // wave's stores have completed, bumps the tile's produced count; the
    // second half waits (bounded: both halves run in the same last round of
    // workgroups) until the produced count is ahead of its own consumed
    // count, adds them and bumps the consumed count.  The two counts only
    // grow and each has one writer, so a hand-over that gave up (recorded in
    // the error word; the output then lacks the first half) is absorbed: the
    // late producer's bump evens the counts, and the next call waits for its
    // own producer again.
    if (is_tail) {
        uint32_t* pt = p.part + ((static_cast<int64_t>(tj >> 1) * kGWaves + wave) * (16 * kGJB)) * 64 * 4;
        unsigned* produced = p.flags + 2 * (tj >> 1);
        unsigned* consumed = produced + 1;
        if (!half) {
#pragma unroll
            for (int ib = 0; ib < 4; ++ib)
#pragma unroll
                for (int jb = 0; jb < kGJB; ++jb)
#pragma unroll
                    for (int qd = 0; qd < 4; ++qd) {
                        const int rr = (ib * kGJB + jb) * 4 + qd;
                        u32x4_v v;
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = __float_as_uint(acc[ib][jb][4 * qd + e]);
                        st_coh<4>(pt + rr * 64 * 4, lane * 16, v);
                    }
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores are complete
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __syncthreads();
            if (tid == 0) __hip_atomic_fetch_add(produced, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        // the ready bit travels through the first LDS word once every wave is
        // done with the operand stages (a separate __shared__ variable would
        // take the kernel past 144 KB of LDS, measured 12% slower)
        int& tail_ready = *reinterpret_cast<int*>(lds);
        lds_barrier();
        if (tid == 0) {
            const unsigned c = __hip_atomic_load(consumed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            int ready = 0;
            for (int it = 0;; ++it) {
                const unsigned pr = __hip_atomic_load(produced, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (static_cast<int>(pr - c) > 0) {
                    ready = 1;
                    break;
                }
                if (it >= p.tail_polls) {
                    wait_expired(kWaitGemmTail);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            __hip_atomic_store(consumed, c + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            tail_ready = ready;
        }
        __syncthreads();
        if (tail_ready) {
#pragma unroll
            for (int ib = 0; ib < 4; ++ib)
#pragma unroll
                for (int jb = 0; jb < kGJB; ++jb)
#pragma unroll
                    for (int qd = 0; qd < 4; ++qd) {
                        const int rr = (ib * kGJB + jb) * 4 + qd;
                        const u32x4_v v = ld_coh<4>(pt + rr * 64 * 4, lane * 16);
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[ib][jb][4 * qd + e] += __uint_as_float(v[e]);
                    }
        }
    }

    // ---- epilogue, through LDS: lane holds column wn 64 + jb 32 + lane % 32
    // and rows wm 128 + ib 32 + 8 (e / 4) + 4 (lane / 32) + e % 4 of the tile;
    // each wave parks its 128 x 64 bf16 block (rows of 144 bytes: the two
    // lane halves, 4 rows apart, hit different banks), then writes it out as
    // 16-byte row chunks (one store instruction per 8 rows instead of one
    // per value).
    lds_barrier();  // every wave is done with the operand stages
    uint8_t* blk = lds + wave * (128 * kGEpiRow);
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int jb = 0; jb < kGJB; ++jb)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = ib * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                *reinterpret_cast<uint16_t*>(blk + r * kGEpiRow + (jb * 32 + (lane & 31)) * 2) =
                    static_cast<uint16_t>(f32_to_bf16_bits(acc[ib][jb][e]));
            }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    void* outp = pick3(p.out, seg);
    const bool vec = (p.vec_mask >> seg) & 1;  // ns % 8 == 0 and 16-byte aligned rows
    const int64_t obase = b * p.o_bs;
    constexpr int kCpr = kGWTN / 8;  // 16-byte chunks of a wave tile row
#pragma unroll 4
    for (int it = 0; it < 128 * kCpr / 64; ++it) {
        const int qd = it * 64 + lane;
        const int r = qd / kCpr, c = qd % kCpr;
        const int row = m0 + wm * 128 + r, col = n0 + wn * kGWTN + 8 * c;
        if (row >= p.m || col >= ns) continue;
        const u32x4_v v = *reinterpret_cast<const u32x4_v*>(blk + r * kGEpiRow + c * 16);
        const int64_t o = obase + static_cast<int64_t>(row) * ns + col;
        float y[8];
        unpack8<bf16_t>(v, y);
        if (vec) {
            if constexpr (EPI == kGemmStore) {
                *reinterpret_cast<u32x4_v*>(static_cast<uint16_t*>(outp) + o) = v;
            } else if constexpr (EPI == kGemmResidualBf16) {
                uint16_t* h = static_cast<uint16_t*>(outp) + o;
                float hv[8];
                unpack8<bf16_t>(*reinterpret_cast<const u32x4_v*>(h), hv);
                u32x4_v w;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    w[i] = f32_to_bf16_bits(hv[2 * i] + y[2 * i]) | (f32_to_bf16_bits(hv[2 * i + 1] + y[2 * i + 1]) << 16);
                *reinterpret_cast<u32x4_v*>(h) = w;
            } else {
                float* h = static_cast<float*>(outp) + o;
                f32x4_v h0 = *reinterpret_cast<const f32x4_v*>(h), h1 = *reinterpret_cast<const f32x4_v*>(h + 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    h0[i] = bf16_round(h0[i] + y[i]);
                    h1[i] = bf16_round(h1[i] + y[4 + i]);
                }
                *reinterpret_cast<f32x4_v*>(h) = h0;
                *reinterpret_cast<f32x4_v*>(h + 4) = h1;
            }
        } else {
            for (int i = 0; i < 8 && col + i < ns; ++i) {
                if constexpr (EPI == kGemmStore) {
                    static_cast<uint16_t*>(outp)[o + i] = static_cast<uint16_t>(f32_to_bf16_bits(y[i]));
                } else if constexpr (EPI == kGemmResidualBf16) {
                    uint16_t* h = static_cast<uint16_t*>(outp);
                    h[o + i] = static_cast<uint16_t>(f32_to_bf16_bits(bf16_bits_to_f32(h[o + i]) + y[i]));
                } else {
                    float* h = static_cast<float*>(outp);
                    h[o + i] = bf16_round(h[o + i] + y[i]);
                }
            }
        }
    }
}

// Shapes the tiled kernel does not take (k or the row stride not a multiple
// of 8): one thread per output element, fp32 sum in k order.
template <int EPI>
__global__ void gemm_bt_simple_kernel(GemmKParams p) {
    const int b = blockIdx.y;
    const int64_t total = static_cast<int64_t>(p.m) * (p.n[0] + p.n[1] + p.n[2]);
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int ntot = p.n[0] + p.n[1] + p.n[2];
        const int row = static_cast<int>(i / ntot);
        int col = static_cast<int>(i % ntot);
        const int seg = col < p.n[0] ? 0 : (col < p.n[0] + p.n[1] ? 1 : 2);
        col -= seg == 0 ? 0 : (seg == 1 ? p.n[0] : p.n[0] + p.n[1]);
        const int ns = pick3(p.n, seg);
        const uint16_t* ar = p.a + b * p.a_bs + static_cast<int64_t>(row) * p.lda;
        const uint16_t* wr = pick3(p.w, seg) + b * p.w_bs + static_cast<int64_t>(col) * p.k;
        float sum = 0.f;
        for (int kk = 0; kk < p.k; ++kk) sum = fmaf(bf16_bits_to_f32(ar[kk]), bf16_bits_to_f32(wr[kk]), sum);
        const int64_t o = b * p.o_bs + static_cast<int64_t>(row) * ns + col;
        const float y = bf16_round(sum);
        void* outp = pick3(p.out, seg);
        if constexpr (EPI == kGemmStore) {
            static_cast<uint16_t*>(outp)[o] = static_cast<uint16_t>(f32_to_bf16_bits(y));
        } else if constexpr (EPI == kGemmResidualBf16) {
            uint16_t* h = static_cast<uint16_t*>(outp);
            h[o] = static_cast<uint16_t>(f32_to_bf16_bits(bf16_bits_to_f32(h[o]) + y));
        } else {
            float* h = static_cast<float*>(outp);
            h[o] = bf16_round(h[o] + y);
        }
    }
}

int gemm_bt(hipStream_t st, const GemmArgs& g) {
    if (g.batch <= 0 || g.m <= 0 || g.k < 0 || g.nseg < 1 || g.nseg > 3) return 1;
    if (g.lda < g.k || g.batch > 65535) return 1;
    // 32-bit per-lane copy offsets: 256 rows of lda elements stay below the
    // buffer range (2^31 - 16 bytes)
    const bool tiled = g.k % 8 == 0 && g.lda % 8 == 0 && g.lda < (1 << 22);
    GemmKParams p{};
    p.a = g.a;
    p.lda = g.lda;
    p.a_bs = g.a_bs;
    p.w_bs = g.w_bs;
    p.o_bs = g.o_bs;
    p.m = g.m;
    p.k = g.k;
    p.mt = (g.m + kGBM - 1) / kGBM;
    int nt = 0;
    for (int s = 0; s < 3; ++s) {
        const int n = s < g.nseg ? g.n[s] : 0;
        p.w[s] = s < g.nseg ? g.w[s] : g.w[0];
        p.out[s] = s < g.nseg ? g.out[s] : g.out[0];
        p.n[s] = n;
        const uintptr_t op = reinterpret_cast<uintptr_t>(p.out[s]);
        if (n % 8 == 0 && op % 16 == 0 && (g.o_bs % 8) == 0) p.vec_mask |= 1 << s;
        nt += (n + kGBN - 1) / kGBN;
        p.nt_end[s] = nt;
    }
    p.nt = nt;
    if (nt == 0) return 0;
    const int64_t tiles = static_cast<int64_t>(p.mt) * nt;
    if (tiles > 0x7fffffff) return 1;
    p.tiles = static_cast<int>(tiles);
    p.full = p.tiles;
    {
        // Tail split: with whole rounds of one workgroup a CU, the last
        // partial round's tiles run as two half-k workgroups each.
        int dev = 0;
        (void)hipGetDevice(&dev);
        const int cus = device_cu_count(dev) > 0 ? device_cu_count(dev) : 256;
        const int tail = p.tiles % cus;
        const int KT = (g.k + kGBK - 1) / kGBK;
        if (g.batch == 1 && p.tiles > cus && tail > 0 && 2 * tail <= cus && KT >= 4 &&
            g.ws && g.ws_bytes >= gemm_tail_bytes(tail)) {
            p.full = p.tiles - tail;
            p.tail = tail;
            p.khalf = KT / 2;
            p.flags = static_cast<unsigned*>(g.ws);
            p.tail_polls = wait_polls(1 << 22);
            p.part = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(g.ws) + kGemmFlagBytes);
        }
    }
    if (!tiled) {
        const int64_t total = static_cast<int64_t>(g.m) * (p.n[0] + p.n[1] + p.n[2]);
        const dim3 sgrid(static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65536)),
                         static_cast<unsigned>(g.batch));
        switch (g.epilogue) {
        case kGemmResidualBf16: hipLaunchKernelGGL(gemm_bt_simple_kernel<kGemmResidualBf16>, sgrid, dim3(256), 0, st, p); break;
        case kGemmResidualF32: hipLaunchKernelGGL(gemm_bt_simple_kernel<kGemmResidualF32>, sgrid, dim3(256), 0, st, p); break;
        default: hipLaunchKernelGGL(gemm_bt_simple_kernel<kGemmStore>, sgrid, dim3(256), 0, st, p); break;
        }
        return hipGetLastError() == hipSuccess ? 0 : 1;
    }
    const dim3 grid(static_cast<unsigned>(p.full + 2 * p.tail), static_cast<unsigned>(g.batch)), blk(kGThreads);
    switch (g.epilogue) {
    case kGemmResidualBf16: hipLaunchKernelGGL(gemm_bt_kernel<kGemmResidualBf16>, grid, blk, 0, st, p); break;
    case kGemmResidualF32: hipLaunchKernelGGL(gemm_bt_kernel<kGemmResidualF32>, grid, blk, 0, st, p); break;
    default: hipLaunchKernelGGL(gemm_bt_kernel<kGemmStore>, grid, blk, 0, st, p); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

hipError_t take_wait_error_gemm(unsigned* bits) { return take_wait_error(bits); }

}  // namespace ssa
