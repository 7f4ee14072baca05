// Drop-in replacements for the reference's prefill-chain helpers and the
// BF16 -> FP8 KV quantiser.  All are HBM-bound elementwise/row kernels: one
// wave64 per row for the row reductions (DPP + cross-row shuffles), plain
// coalesced grid-stride loops for the rest.  The fused entry points do not use
// them; they exist so the reference's chain keeps working when linked against
// this library.
#include "common.hpp"
#include "../../include/supersonic_attn.h"

namespace ssa {

// ---------------------------------------------------------------- RMSNorm
// full_attention.hip:2507-2560: x * rsqrt(mean(x^2) + eps) * (w [+ 1]).
template <typename T, bool UNIT>
__global__ __launch_bounds__(256) void rms_norm_kernel(int n_rows, int n_cols, float eps, const T* xs,
                                                       const T* w, T* out) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n_rows) return;
    const T* x = xs + static_cast<size_t>(row) * n_cols;
    T* o = out + static_cast<size_t>(row) * n_cols;
    float ss = 0.f;
    for (int c = lane; c < n_cols; c += 64) {
        const float v = load_f32(x, c);
        ss += v * v;
    }
    ss = wave_sum(ss);
    const float inv = rsqrtf(ss / static_cast<float>(n_cols) + eps);
    for (int c = lane; c < n_cols; c += 64) {
        const float wv = load_f32(w, c) + (UNIT ? 1.0f : 0.0f);
        store_f32(o, c, load_f32(x, c) * inv * wv);
    }
}

// ---------------------------------------------------------------- cast
template <typename I, typename O>
__global__ __launch_bounds__(256) void cast_kernel(size_t n, const I* in, O* out) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * 256)
        store_f32(out, i, load_f32(in, i));
}

// ---------------------------------------------------------------- RoPE
// prefill_helpers.hip:79-108: rotate-half over dims [0, 2*half_rot) in place.
template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(int seq_len, int num_heads, int head_dim, int half_rot,
                                                   const T* cos_t, const T* sin_t, T* data) {
    const size_t total = static_cast<size_t>(seq_len) * num_heads * half_rot;
    for (size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
         idx += static_cast<size_t>(gridDim.x) * 256) {
        const int i = static_cast<int>(idx % half_rot);
        const size_t hp = idx / half_rot;
        const int h = static_cast<int>(hp % num_heads);
        const size_t pos = hp / num_heads;
        const float c = load_f32(cos_t, pos * half_rot + i);
        const float s = load_f32(sin_t, pos * half_rot + i);
        const size_t base = (pos * num_heads + h) * head_dim;
        const float x0 = load_f32(data, base + i);
        const float x1 = load_f32(data, base + half_rot + i);
        store_f32(data, base + i, x0 * c - x1 * s);
        store_f32(data, base + half_rot + i, x0 * s + x1 * c);
    }
}

// ---------------------------------------------------------------- transpose
// prefill_helpers.hip:114-130: [S, H, D] -> [H, S, D]; one block per (s, h) row.
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(int S, int H, int D, const T* src, T* dst) {
    const size_t row = blockIdx.x;  // s * H + h
    const int s = static_cast<int>(row / H), h = static_cast<int>(row % H);
    const T* in = src + row * D;
    T* o = dst + (static_cast<size_t>(h) * S + s) * D;
    for (int d = threadIdx.x; d < D; d += 256) o[d] = in[d];
}

// ---------------------------------------------------------------- sigmoid gate
// prefill_helpers.hip:183-195.
template <typename T>
__global__ __launch_bounds__(256) void sigmoid_mul_kernel(size_t n, const T* data, const T* gate, T* out) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * 256) {
        const float g = load_f32(gate, i);
        store_f32(out, i, load_f32(data, i) * (1.0f / (1.0f + expf(-g))));
    }
}

// ---------------------------------------------------------------- split q/gate
// prefill_helpers.hip:239-257: per head [q (D) | gate (D)].
template <typename T>
__global__ __launch_bounds__(256) void split_qgate_kernel(int S, int H, int D, const T* src, T* q, T* g) {
    const size_t row = blockIdx.x;  // s * H + h
    const T* in = src + row * 2 * D;
    for (int d = threadIdx.x; d < D; d += 256) {
        q[row * D + d] = in[d];
        g[row * D + d] = in[D + d];
    }
}

// ---------------------------------------------------------------- FP8 quantiser
// The reference encoder float_to_fp8_e4m3 (full_attention_4b.hip:205-232),
// restated with exact exponent extraction.  floor(log2f(v)) differs from the
// exact exponent only within an ulp below a power of two, where both branches
// round to that power of two, so the bytes are identical.
__device__ __forceinline__ uint32_t ref_fp8_encode(float val) {
    uint32_t sign = 0;
    if (val < 0.0f) {
        sign = 0x80;
        val = -val;
    }
    const float kSub = 1.52587890625e-2f;
    if (val >= 448.0f) return sign | 0x7E;
    if (val < kSub * 0.125f) return sign;
    if (val < 0.015625f) {
        int m = static_cast<int>(rintf(val / kSub * 8.0f));
        if (m < 0) m = 0;
        if (m >= 8) return sign | 0x08;
        return sign | static_cast<uint32_t>(m);
    }
    int e = static_cast<int>((__float_as_uint(val) >> 23) & 0xFF) - 127 + 7;  // floor(log2) + 7
    if (e < 1) e = 1;
    if (e > 14) e = 14;
    const float pow2 = __uint_as_float(static_cast<uint32_t>(e - 7 + 127) << 23);
    int m = static_cast<int>(rintf((val / pow2 - 1.0f) * 8.0f));
    if (m < 0) m = 0;
    if (m >= 8) {
        m = 0;
        e += 1;
        if (e > 14) return sign | 0x7E;
    }
    return sign | (static_cast<uint32_t>(e) << 3) | static_cast<uint32_t>(m);
}

// One wave per (head, position) row: absmax -> scale -> codes
// (quantize_kv_to_fp8_kernel, full_attention_4b.hip:4786-4829).
template <bool REF_CODEC>
__global__ __launch_bounds__(256) void quantize_kv_kernel(const uint16_t* src, uint8_t* dst, float* dst_scale,
                                                          int Hkv, int S, int D, int max_T, int pos_offset) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= Hkv * S) return;
    const int h = row / S, t = row % S;
    const uint16_t* x = src + (static_cast<size_t>(h) * S + t) * D;
    float am = 0.f;
    for (int d = lane; d < D; d += 64) am = fmaxf(am, fabsf(bf16_bits_to_f32(x[d])));
    am = wave_max(am);
    const float scale = fmaxf(am / 448.0f, 1e-12f);
    const float inv = 1.0f / scale;
    const size_t orow = static_cast<size_t>(h) * max_T + pos_offset + t;
    if (lane == 0) dst_scale[orow] = scale;
    uint8_t* o = dst + orow * D;
    for (int d = lane; d < D; d += 64) {
        const float v = bf16_bits_to_f32(x[d]) * inv;
        uint32_t c;
        if (REF_CODEC) {
            c = ref_fp8_encode(v);
        } else {
            c = f32x4_to_fp8x4(v, 0.f, 0.f, 0.f) & 0xFFu;
        }
        o[d] = static_cast<uint8_t>(c);
    }
}

// ---------------------------------------------------------------- row repack
// dst row r = (o, i), o < n_outer, i < n_inner, holds dout elements: the
// first din come from src[o * so + i * si + c] (cast I -> O), the rest are
// zero.  The general head-size paths of the drop-ins pad head dims to a
// native tile (or cast to f32) and compact the results back with it.
template <typename I, typename O>
__global__ __launch_bounds__(256) void repack_rows_kernel(const I* src, O* dst, int64_t n_inner, int64_t so,
                                                          int64_t si, int din, int dout, int64_t total) {
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t r = e / dout;
        const int c = static_cast<int>(e - r * dout);
        const int64_t o = r / n_inner, i = r - o * n_inner;
        store_f32(dst, e, c < din ? load_f32(src, o * so + i * si + c) : 0.f);
    }
}

template <typename I, typename O>
static hipError_t repack_as(const void* src, void* dst, int64_t n_outer, int64_t n_inner, int64_t so, int64_t si,
                            int din, int dout, hipStream_t st) {
    const int64_t total = n_outer * n_inner * dout;
    if (total <= 0) return hipSuccess;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL((repack_rows_kernel<I, O>), dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536)),
                       dim3(256), 0, st, static_cast<const I*>(src), static_cast<O*>(dst), n_inner, so, si, din, dout,
                       total);
    return hipGetLastError();
}

template <typename I>
static hipError_t repack_to(int tout, const void* src, void* dst, int64_t n_outer, int64_t n_inner, int64_t so,
                            int64_t si, int din, int dout, hipStream_t st) {
    switch (tout) {
    case 0: return repack_as<I, f16_t>(src, dst, n_outer, n_inner, so, si, din, dout, st);
    case 1: return repack_as<I, float>(src, dst, n_outer, n_inner, so, si, din, dout, st);
    case 2: return repack_as<I, bf16_t>(src, dst, n_outer, n_inner, so, si, din, dout, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t repack_rows(int tin, int tout, const void* src, void* dst, int64_t n_outer, int64_t n_inner, int64_t so,
                       int64_t si, int din, int dout, hipStream_t st) {
    switch (tin) {
    case 0: return repack_to<f16_t>(tout, src, dst, n_outer, n_inner, so, si, din, dout, st);
    case 1: return repack_to<float>(tout, src, dst, n_outer, n_inner, so, si, din, dout, st);
    case 2: return repack_to<bf16_t>(tout, src, dst, n_outer, n_inner, so, si, din, dout, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace ssa

using namespace ssa;

namespace {

template <typename T>
int rms_norm_device(int dev, int rows, int cols, float eps, int unit, const void* x, const void* w, void* o) {
    ScopedDevice scoped(dev);
    const unsigned grid = grid1d(static_cast<size_t>(rows), 4);
    if (rows > 0) {
        if (unit)
            hipLaunchKernelGGL((rms_norm_kernel<T, true>), dim3(grid), dim3(256), 0, 0, rows, cols, eps,
                               static_cast<const T*>(x), static_cast<const T*>(w), static_cast<T*>(o));
        else
            hipLaunchKernelGGL((rms_norm_kernel<T, false>), dim3(grid), dim3(256), 0, 0, rows, cols, eps,
                               static_cast<const T*>(x), static_cast<const T*>(w), static_cast<T*>(o));
        if (hipGetLastError() != hipSuccess) return 71;
    }
    if (hipDeviceSynchronize() != hipSuccess) return 72;
    return 0;
}

unsigned stride_grid(size_t n) {
    size_t g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    return static_cast<unsigned>(g ? g : 1);
}

template <typename I, typename O>
int cast_device(int dev, size_t n, const void* x, void* o) {
    ScopedDevice scoped(dev);
    if (n) {
        hipLaunchKernelGGL((cast_kernel<I, O>), dim3(stride_grid(n)), dim3(256), 0, 0, n,
                           static_cast<const I*>(x), static_cast<O*>(o));
        if (hipGetLastError() != hipSuccess) return 135;
    }
    if (hipDeviceSynchronize() != hipSuccess) return 136;
    return 0;
}

template <typename I>
int cast_out(int out_dtype, int dev, size_t n, const void* x, void* o) {
    switch (out_dtype) {
    case 0: return cast_device<I, f16_t>(dev, n, x, o);
    case 1: return cast_device<I, float>(dev, n, x, o);
    case 2: return cast_device<I, bf16_t>(dev, n, x, o);
    default: return 137;
    }
}

template <typename T>
int rope_device(int dev, size_t S, size_t H, size_t D, size_t hr, const void* c, const void* s, void* data) {
    ScopedDevice scoped(dev);
    const size_t n = S * H * hr;
    if (n) {
        hipLaunchKernelGGL((rope_kernel<T>), dim3(stride_grid(n)), dim3(256), 0, 0, static_cast<int>(S),
                           static_cast<int>(H), static_cast<int>(D), static_cast<int>(hr),
                           static_cast<const T*>(c), static_cast<const T*>(s), static_cast<T*>(data));
        if (hipGetLastError() != hipSuccess) return 311;
    }
    if (hipDeviceSynchronize() != hipSuccess) return 312;
    return 0;
}

template <typename T>
int transpose_device(int dev, size_t S, size_t H, size_t D, const void* src, void* dst) {
    ScopedDevice scoped(dev);
    if (S * H && D) {
        hipLaunchKernelGGL((transpose_kernel<T>), dim3(static_cast<unsigned>(S * H)), dim3(256), 0, 0,
                           static_cast<int>(S), static_cast<int>(H), static_cast<int>(D),
                           static_cast<const T*>(src), static_cast<T*>(dst));
        if (hipGetLastError() != hipSuccess) return 321;
    }
    if (hipDeviceSynchronize() != hipSuccess) return 322;
    return 0;
}

template <typename T>
int sigmoid_mul_device(int dev, size_t n, const void* d, const void* g, void* o) {
    ScopedDevice scoped(dev);
    if (n) {
        hipLaunchKernelGGL((sigmoid_mul_kernel<T>), dim3(stride_grid(n)), dim3(256), 0, 0, n,
                           static_cast<const T*>(d), static_cast<const T*>(g), static_cast<T*>(o));
        if (hipGetLastError() != hipSuccess) return 351;
    }
    if (hipDeviceSynchronize() != hipSuccess) return 352;
    return 0;
}

template <typename T>
int split_qgate_device(int dev, size_t S, size_t H, size_t D, const void* src, void* q, void* g) {
    ScopedDevice scoped(dev);
    if (S * H && D) {
        hipLaunchKernelGGL((split_qgate_kernel<T>), dim3(static_cast<unsigned>(S * H)), dim3(256), 0, 0,
                           static_cast<int>(S), static_cast<int>(H), static_cast<int>(D),
                           static_cast<const T*>(src), static_cast<T*>(q), static_cast<T*>(g));
        if (hipGetLastError() != hipSuccess) return 371;
    }
    if (hipDeviceSynchronize() != hipSuccess) return 372;
    return 0;
}

}  // namespace

extern "C" int supersonic_qwen35_hip_rms_norm(int dtype, size_t device_ordinal, size_t n_rows, size_t n_cols,
                                              float eps, int add_unit_offset, const void* xs,
                                              const void* weight, void* out) {
    const int dev = static_cast<int>(device_ordinal);
    const int r = static_cast<int>(n_rows), c = static_cast<int>(n_cols);
    switch (dtype) {
    case 0: return rms_norm_device<f16_t>(dev, r, c, eps, add_unit_offset, xs, weight, out);
    case 1: return rms_norm_device<float>(dev, r, c, eps, add_unit_offset, xs, weight, out);
    case 2: return rms_norm_device<bf16_t>(dev, r, c, eps, add_unit_offset, xs, weight, out);
    default: return 74;
    }
}

extern "C" int supersonic_qwen35_hip_cast(int input_dtype, int output_dtype, size_t device_ordinal,
                                          size_t total_elems, const void* xs, void* out) {
    const int dev = static_cast<int>(device_ordinal);
    switch (input_dtype) {
    case 0: return cast_out<f16_t>(output_dtype, dev, total_elems, xs, out);
    case 1: return cast_out<float>(output_dtype, dev, total_elems, xs, out);
    case 2: return cast_out<bf16_t>(output_dtype, dev, total_elems, xs, out);
    default: return 137;
    }
}

extern "C" int supersonic_qwen35_hip_apply_rope_prefill(int dtype, size_t device_ordinal, size_t seq_len,
                                                        size_t num_heads, size_t head_dim, size_t half_rot,
                                                        const void* cos_table, const void* sin_table,
                                                        void* data) {
    const int dev = static_cast<int>(device_ordinal);
    switch (dtype) {
    case 0: return rope_device<f16_t>(dev, seq_len, num_heads, head_dim, half_rot, cos_table, sin_table, data);
    case 1: return rope_device<float>(dev, seq_len, num_heads, head_dim, half_rot, cos_table, sin_table, data);
    case 2: return rope_device<bf16_t>(dev, seq_len, num_heads, head_dim, half_rot, cos_table, sin_table, data);
    default: return 310;
    }
}

extern "C" int supersonic_qwen35_hip_transpose_shd_hsd(int dtype, size_t device_ordinal, size_t s, size_t h,
                                                       size_t d, const void* src, void* dst) {
    const int dev = static_cast<int>(device_ordinal);
    switch (dtype) {
    case 0: return transpose_device<uint16_t>(dev, s, h, d, src, dst);
    case 1: return transpose_device<uint32_t>(dev, s, h, d, src, dst);
    case 2: return transpose_device<uint16_t>(dev, s, h, d, src, dst);
    default: return 320;
    }
}

extern "C" int supersonic_qwen35_hip_sigmoid_mul(int dtype, size_t device_ordinal, size_t total_elems,
                                                 const void* data, const void* gate, void* out) {
    const int dev = static_cast<int>(device_ordinal);
    switch (dtype) {
    case 0: return sigmoid_mul_device<f16_t>(dev, total_elems, data, gate, out);
    case 1: return sigmoid_mul_device<float>(dev, total_elems, data, gate, out);
    case 2: return sigmoid_mul_device<bf16_t>(dev, total_elems, data, gate, out);
    default: return 350;
    }
}

extern "C" int supersonic_qwen35_hip_split_qgate(int dtype, size_t device_ordinal, size_t s, size_t num_heads,
                                                 size_t head_dim, const void* src, void* query_out,
                                                 void* gate_out) {
    const int dev = static_cast<int>(device_ordinal);
    switch (dtype) {
    case 0: return split_qgate_device<uint16_t>(dev, s, num_heads, head_dim, src, query_out, gate_out);
    case 1: return split_qgate_device<uint32_t>(dev, s, num_heads, head_dim, src, query_out, gate_out);
    case 2: return split_qgate_device<uint16_t>(dev, s, num_heads, head_dim, src, query_out, gate_out);
    default: return 370;
    }
}

extern "C" int supersonic_qwen35_4b_hip_quantize_kv_to_fp8(int dtype, size_t device_ordinal, const void* src,
                                                           void* dst_fp8, float* dst_scale, int num_kv_heads,
                                                           int seq_len, int head_dim, int max_T,
                                                           int pos_offset) {
    if (dtype != 2) return 256;
    ScopedDevice scoped(static_cast<int>(device_ordinal));
    const int rows = num_kv_heads * seq_len;
    if (rows > 0) {
        hipLaunchKernelGGL((quantize_kv_kernel<true>), dim3(grid1d(static_cast<size_t>(rows), 4)), dim3(256), 0,
                           0, static_cast<const uint16_t*>(src), static_cast<uint8_t*>(dst_fp8), dst_scale,
                           num_kv_heads, seq_len, head_dim, max_T, pos_offset);
    }
    const hipError_t le = hipGetLastError();
    const hipError_t se = hipDeviceSynchronize();
    if (le != hipSuccess) return 254;
    if (se != hipSuccess) return 255;
    return 0;
}

// OCP-codec variant of the quantiser (same layout and scale rule); the codec
// of the native fused entry points.
extern "C" int supersonic_attn_gfx950_quantize_kv_fp8_ocp(size_t device_ordinal, void* stream, const void* src,
                                                          void* dst_fp8, float* dst_scale, int num_kv_heads,
                                                          int seq_len, int head_dim, int max_T, int pos_offset) {
    if (!src || !dst_fp8 || !dst_scale) return SUPERSONIC_ERR_NULL;
    ScopedDevice scoped(static_cast<int>(device_ordinal));
    const int rows = num_kv_heads * seq_len;
    if (rows > 0) {
        hipLaunchKernelGGL((quantize_kv_kernel<false>), dim3(grid1d(static_cast<size_t>(rows), 4)), dim3(256), 0,
                           static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(src),
                           static_cast<uint8_t*>(dst_fp8), dst_scale, num_kv_heads, seq_len, head_dim, max_T,
                           pos_offset);
        if (hipGetLastError() != hipSuccess) return SUPERSONIC_ERR_LAUNCH;
    }
    return 0;
}
