// Hand-written bf16 GEMM with a transposed right-hand side for the
// prefill-sized projections: out[m][n] = a[m][k] . w[n][k]^T, fp32
// accumulation, up to three column segments (separate weights and outputs) in
// one launch, optionally batched, with a plain bf16 store or a residual add
// in the epilogue.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ssa {

enum GemmEpilogue { kGemmStore = 0, kGemmResidualBf16 = 1, kGemmResidualF32 = 2 };

struct GemmArgs {
    int batch = 1, m = 0, k = 0;
    const uint16_t* a = nullptr;  // [batch][m][lda]
    int64_t lda = 0, a_bs = 0;
    int nseg = 1;
    const uint16_t* w[3] = {nullptr, nullptr, nullptr};  // [n_s][k] per segment
    void* out[3] = {nullptr, nullptr, nullptr};          // [m][n_s] per segment
    int n[3] = {0, 0, 0};
    int64_t w_bs = 0, o_bs = 0;  // batch strides (elements) of w and out (segment 0 only when batched)
    int epilogue = kGemmStore;   // residual: out = bf16(out + bf16(a.w^T)), in place (one segment)
    // Optional workspace (zero-filled before its first use; every call leaves
    // each tile's two hand-over counts equal) for splitting the last partial round of tiles along
    // k; without one (or too small) the tail runs whole.
    void* ws = nullptr;
    size_t ws_bytes = 0;
};

constexpr size_t kGemmFlagBytes = 8192;  // tail counts, two per tile (<= 1024 tail tiles)
// Workspace bytes of the tail split for `tail` tiles.
inline size_t gemm_tail_bytes(int tail) { return kGemmFlagBytes + static_cast<size_t>(tail) * 8 * 32 * 64 * 16; }
// Workspace bytes for the tail split of a GEMM of m rows and the given
// column segments on a GPU of `cus` CUs (256 on MI355X); 0 when it has no
// tail to split.
inline size_t gemm_ws_bytes(int m, int nseg, const int* n, int cus = 256) {
    int64_t nt = 0;
    for (int s = 0; s < nseg; ++s) nt += (n[s] + 255) / 256;
    const int64_t tiles = static_cast<int64_t>((m + 255) / 256) * nt;
    const int tail = static_cast<int>(tiles % cus);
    return tiles > cus && tail > 0 && 2 * tail <= cus ? gemm_tail_bytes(tail) : 0;
}

// Launches on `st`; 0 on success.  Requires k % 8 == 0 and 16-byte aligned
// rows (lda % 8 == 0).
int gemm_bt(hipStream_t st, const GemmArgs& g);

}  // namespace ssa
