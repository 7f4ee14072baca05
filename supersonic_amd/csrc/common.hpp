// Shared device/host helpers for the gfx950 full-attention library.
// CDNA4 only: wave64, MFMA, OCP e4m3 hardware converts.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <cstdlib>

#include "supersonic_attn.h"

namespace ssa {

// ----------------------------------------------------------------------------
// Scalar element types.  bf16 / f16 are carried as raw 16-bit patterns so the
// kernels control every rounding step themselves.
// ----------------------------------------------------------------------------
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_v __attribute__((ext_vector_type(8)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));
typedef float f32x16_v __attribute__((ext_vector_type(16)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));
typedef short s16x4_v __attribute__((ext_vector_type(4)));  // 4 x 16-bit MFMA operand (16x16x16)

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Round-to-nearest-even f32 -> bf16 bits with the hardware converter
// (v_cvt_pk_bf16_f32; a NaN stays a quiet NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}
__device__ __forceinline__ float bf16_round(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
    _Float16 h;
    uint16_t s = static_cast<uint16_t>(b);
    __builtin_memcpy(&h, &s, 2);
    return static_cast<float>(h);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float x) {
    _Float16 h = static_cast<_Float16>(x);
    uint16_t s;
    __builtin_memcpy(&s, &h, 2);
    return s;
}

template <typename T> struct Elem;
template <> struct Elem<bf16_t> {
    static __device__ __forceinline__ float to_f32(uint32_t b) { return bf16_bits_to_f32(b); }
    static __device__ __forceinline__ uint32_t from_f32(float x) { return f32_to_bf16_bits(x); }
};
template <> struct Elem<f16_t> {
    static __device__ __forceinline__ float to_f32(uint32_t b) { return f16_bits_to_f32(b); }
    static __device__ __forceinline__ uint32_t from_f32(float x) { return f32_to_f16_bits(x); }
};

template <typename T> __device__ __forceinline__ float load_f32(const T* p, size_t i);
template <> __device__ __forceinline__ float load_f32<float>(const float* p, size_t i) { return p[i]; }
template <> __device__ __forceinline__ float load_f32<bf16_t>(const bf16_t* p, size_t i) { return bf16_bits_to_f32(p[i].bits); }
template <> __device__ __forceinline__ float load_f32<f16_t>(const f16_t* p, size_t i) { return f16_bits_to_f32(p[i].bits); }

template <typename T> __device__ __forceinline__ void store_f32(T* p, size_t i, float x);
template <> __device__ __forceinline__ void store_f32<float>(float* p, size_t i, float x) { p[i] = x; }
template <> __device__ __forceinline__ void store_f32<bf16_t>(bf16_t* p, size_t i, float x) { p[i].bits = static_cast<uint16_t>(f32_to_bf16_bits(x)); }
template <> __device__ __forceinline__ void store_f32<f16_t>(f16_t* p, size_t i, float x) { p[i].bits = static_cast<uint16_t>(f32_to_f16_bits(x)); }

// Unpack 8 packed 16-bit values (a 16-byte load) to f32.
template <typename T>
__device__ __forceinline__ void unpack8(const u32x4_v& w, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = Elem<T>::to_f32(w[i] & 0xFFFFu);
        f[2 * i + 1] = Elem<T>::to_f32(w[i] >> 16);
    }
}
template <>
__device__ __forceinline__ void unpack8<bf16_t>(const u32x4_v& w, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(w[i] << 16);
        f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
}

// ----------------------------------------------------------------------------
// OCP e4m3 through the gfx950 converters.
// ----------------------------------------------------------------------------
// Two e4m3 bytes (selected by word_hi: bytes 0-1 or 2-3 of v) -> 2 floats.
__device__ __forceinline__ f32x2_v fp8x2_to_f32(uint32_t v, bool word_hi) {
    return word_hi ? __builtin_amdgcn_cvt_pk_f32_fp8(v, true) : __builtin_amdgcn_cvt_pk_f32_fp8(v, false);
}
// Four floats -> four e4m3 bytes, round-to-nearest-even, saturated to +-448.
__device__ __forceinline__ uint32_t f32x4_to_fp8x4(float a, float b, float c, float d) {
    a = fminf(fmaxf(a, -448.f), 448.f);
    b = fminf(fmaxf(b, -448.f), 448.f);
    c = fminf(fmaxf(c, -448.f), 448.f);
    d = fminf(fmaxf(d, -448.f), 448.f);
    uint32_t r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0u, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
    return r;
}

// ----------------------------------------------------------------------------
// Cross-lane reductions.  DPP row rotates stay inside 16-lane rows.
// ----------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// Reduce across the 16 lanes of each DPP row; every lane gets the result.
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp_f32<0x128>(x));  // row_ror:8
    x = fmaxf(x, dpp_f32<0x124>(x));  // row_ror:4
    x = fmaxf(x, dpp_f32<0x122>(x));  // row_ror:2
    x = fmaxf(x, dpp_f32<0x121>(x));  // row_ror:1
    return x;
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f32<0x128>(x);
    x += dpp_f32<0x124>(x);
    x += dpp_f32<0x122>(x);
    x += dpp_f32<0x121>(x);
    return x;
}
// Reductions over lanes l ^ 16 and l ^ 32 with the gfx950 permlane swaps
// (VALU, no LDS round trip).  Each swap returns the lane's own value and its
// partner's in some order, which is all a max or a sum needs.
// max of three MFMA results as one v_max3_f32.  fmaxf would first quiet
// every operand (a v_max_f32 x, x per value) because MFMA outputs are not
// known to be canonical; scores are never signalling NaNs.
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float xor16_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return max3_raw(__uint_as_float(r[0]), __uint_as_float(r[1]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return max3_raw(__uint_as_float(r[0]), __uint_as_float(r[1]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float wave_sum(float x) {
    x = row16_sum(x);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}
__device__ __forceinline__ float wave_max(float x) {
    x = row16_max(x);
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

__device__ __forceinline__ u32x4_v ld16(const void* p) {
    return *reinterpret_cast<const u32x4_v*>(p);
}
__device__ __forceinline__ void st16(void* p, const u32x4_v& v) {
    *reinterpret_cast<u32x4_v*>(p) = v;
}

constexpr float kLog2e = 1.4426950408889634f;

// Device-coherent (sc1) relaxed accesses: visible across the XCDs' L2s without
// a device-wide fence.
__device__ __forceinline__ void store_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Device-coherent accesses of data another workgroup of the same kernel wrote
// (agent-scope relaxed atomics: sc1 loads and write-through stores).
__device__ __forceinline__ uint16_t load_agent_u16(const uint16_t* p) {
    return __hip_atomic_load(const_cast<uint16_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent_u16(uint16_t* p, uint16_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent_u32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_agent_u32(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split partials travel as the bitwise complement of the float's bits (a NaN
// made canonical first), so a word of zero means "not written yet": a reader
// polls for its data instead of every writer waiting for its stores to
// complete before it signals.  Readers set the words back to zero.
__device__ __forceinline__ uint32_t part_enc(float v) { return ~(v != v ? 0x7fc00000u : __float_as_uint(v)); }
__device__ __forceinline__ float part_dec(uint32_t w) { return __uint_as_float(~w); }
__device__ __forceinline__ void store_part(float* p, float v) { store_agent_u32(reinterpret_cast<uint32_t*>(p), part_enc(v)); }
constexpr int kMergePoll = 1 << 16;

// Words between the split arrival counters of a call with `pairs` (sequence,
// kv head) pairs in a region of `words` counters: 32 (one 128-byte line each,
// so the atomics of different pairs do not queue on one line) or, for many
// pairs, the largest power of two that fits.
__host__ __device__ constexpr int arrival_stride(long long pairs, long long words) {
    int s = 32;
    while (s > 1 && pairs * s > words) s >>= 1;
    return s;
}

// Sticky error word of this code object (each translation unit holds its own
// copy on every GPU): a bounded wait that gives up sets its bit and the kernel
// carries on to a normal exit.  The host reads and clears it with
// take_wait_error(); supersonic_attn_gfx950_wait_status() reports the OR of
// every translation unit's word.
enum : unsigned { kWaitLayerBarrier = 1u, kWaitDecodeMerge = 2u, kWaitGemmTail = 4u };
static __device__ unsigned g_wait_error;
__device__ __forceinline__ void wait_expired(unsigned bit) {
    __hip_atomic_fetch_or(&g_wait_error, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Device-coherent (sc1) vector accesses of 4 << L2B bytes per lane through a
// buffer resource on a wave-uniform base: one instruction for a lane's
// 4-16 bytes (coherent accesses cost about as much per instruction as per
// dword, so wide ones pay).
template <int N> struct U32N { typedef uint32_t t __attribute__((ext_vector_type(N))); };
template <> struct U32N<1> { typedef uint32_t t; };
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coh_rsrc(const void* uniform_base) {
    const uint64_t a = reinterpret_cast<uint64_t>(uniform_base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
    void* u = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, static_cast<short>(0), 0x7fffffff, 0x00020000);
}
constexpr int kSc1 = 0x10;  // cache-policy bit: device-coherent access
template <int N>
__device__ __forceinline__ typename U32N<N>::t ld_coh(const void* uniform_base, int byte_off) {
    const __amdgpu_buffer_rsrc_t r = coh_rsrc(uniform_base);
    if constexpr (N == 4) return __builtin_bit_cast(typename U32N<N>::t, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSc1));
    else if constexpr (N == 2) return __builtin_bit_cast(typename U32N<N>::t, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, kSc1));
    else return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, kSc1);
}
template <int N>
__device__ __forceinline__ void st_coh(void* uniform_base, int byte_off, typename U32N<N>::t v) {
    const __amdgpu_buffer_rsrc_t r = coh_rsrc(uniform_base);
    if constexpr (N == 4) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_v, v), r, byte_off, 0, kSc1);
    else if constexpr (N == 2) __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_v, v), r, byte_off, 0, kSc1);
    else __builtin_amdgcn_raw_buffer_store_b32(v, r, byte_off, 0, kSc1);
}  // bounded poll of a merge for partials in flight

__device__ __forceinline__ u32x4_v ld16_agent(const void* p) {
    uint64_t* q = reinterpret_cast<uint64_t*>(const_cast<void*>(p));
    const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return u32x4_v{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32), static_cast<uint32_t>(b),
                   static_cast<uint32_t>(b >> 32)};
}
// store_f32 through the coherent path (bf16 / f16 / f32 elements)
template <typename T> __device__ __forceinline__ void store_f32_agent(T* p, size_t i, float x);
template <> __device__ __forceinline__ void store_f32_agent<float>(float* p, size_t i, float x) { store_agent(p + i, x); }
template <> __device__ __forceinline__ void store_f32_agent<bf16_t>(bf16_t* p, size_t i, float x) {
    store_agent_u16(reinterpret_cast<uint16_t*>(p) + i, static_cast<uint16_t>(f32_to_bf16_bits(x)));
}
template <> __device__ __forceinline__ void store_f32_agent<f16_t>(f16_t* p, size_t i, float x) {
    store_agent_u16(reinterpret_cast<uint16_t*>(p) + i, static_cast<uint16_t>(f32_to_f16_bits(x)));
}

// Element seg (0..2) of a 3-entry parameter array by selects: indexing a kernel
// parameter's array with a run-time index would copy the parameters to
// private (scratch) memory.
template <typename T>
__device__ __forceinline__ T pick3(const T (&a)[3], int seg) {
    return seg == 0 ? a[0] : (seg == 1 ? a[1] : a[2]);
}

// Workgroup barrier that waits only for LDS traffic: unlike __syncthreads it
// leaves outstanding global loads in flight.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

}  // namespace ssa

// ----------------------------------------------------------------------------
// Host side
// ----------------------------------------------------------------------------
namespace ssa {

// Saves, sets and restores the current device around a bridge call, the
// reference bridges' ScopedHipDevice (kernels/prefill_helpers_bridge.cpp:11-19).
struct ScopedDevice {
    int previous = -1;
    bool changed = false;
    explicit ScopedDevice(int target) {
        if (hipGetDevice(&previous) != hipSuccess) previous = -1;
        if (previous != target) {
            if (hipSetDevice(target) == hipSuccess) changed = true;
        }
    }
    ~ScopedDevice() {
        if (changed && previous >= 0) (void)hipSetDevice(previous);
    }
};

// Per-device scratch owned by the library: grown on demand, never shrunk,
// released at process exit.  Used for split-K partials of the entry points
// that have no workspace argument.
// Slots: one cached buffer per (device, slot) so the decode partials and the
// prefill V^T staging never share memory.
constexpr int kWorkspaceDecode = 0;
constexpr int kWorkspacePrefill = 1;
constexpr int kWorkspaceProj = 2;    // scratch rows: the o_proj GEMM output (hipBLASLt path), qkv_proj normed rows
constexpr int kWorkspaceProjLt = 3;  // hipBLASLt workspace
constexpr int kWorkspaceSkinny = 4;  // split-k partials and arrival counters of the o_proj kernel
constexpr int kWorkspaceGemm = 5;    // tail-split partials and flags of the hand-written GEMM
constexpr int kWorkspaceRope = 6;    // qkv_proj_rope: per-head counters (zero between calls), then rows
constexpr int kWorkspaceMixed = 7;   // mixed step: the prefill's claim counters (zero between calls)
constexpr int kWorkspaceSlots = 8;
void* device_workspace(int device, size_t bytes, int slot);

// Compute units of `device` (cached; 256 on MI355X), 0 if the query fails.
int device_cu_count(int device);

// Optional pair of events recorded on the launch stream immediately before and
// after the dominant kernel of the next entry-point call (benchmarks time that
// kernel on its own stream with them).  Cleared after use.
struct ProfileEvents {
    hipEvent_t before = nullptr;
    hipEvent_t after = nullptr;
};
ProfileEvents take_profile_events();

// Poll budget of a bounded wait: SUPERSONIC_WAIT_POLLS when set (read per
// call; a small value lets a test force the give-up path), else `dflt`.
inline int wait_polls(int dflt) {
    const char* v = getenv("SUPERSONIC_WAIT_POLLS");
    if (!v || !*v) return dflt;
    const long n = strtol(v, nullptr, 10);
    return n < 0 ? 0 : (n > (1L << 30) ? (1 << 30) : static_cast<int>(n));
}

// Reads and clears this translation unit's error word on the current device
// (synchronous; the caller has synchronised the work it asks about).
static inline hipError_t take_wait_error(unsigned* bits) {
    unsigned v = 0;
    hipError_t e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_wait_error), sizeof(v), 0, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return e;
    if (v) {
        const unsigned zero = 0;
        e = hipMemcpyToSymbol(HIP_SYMBOL(g_wait_error), &zero, sizeof(zero), 0, hipMemcpyHostToDevice);
    }
    *bits |= v;
    return e;
}
// Per translation unit readers (decode.hip, layer.hip, gemm.hip).
hipError_t take_wait_error_decode(unsigned* bits);
hipError_t take_wait_error_layer(unsigned* bits);
hipError_t take_wait_error_gemm(unsigned* bits);

// The fused entry points with their scheduling knobs (decode.hip,
// prefill.hip): decode planned for target_wgs workgroups (0: the whole GPU),
// prefill on the dynamic schedule when claims is not NULL (16 zeroed
// 128-byte counter lines).
int decode_native(size_t device_ordinal, void* stream, int kv_dtype, size_t batch, size_t q_heads,
                  size_t kv_heads, size_t head_dim, size_t rotary_dim, size_t max_kv_len, float eps, float scale,
                  const void* q_proj, const void* k_new, const void* v_new, const void* q_norm_w,
                  const void* k_norm_w, const void* cos_table, const void* sin_table, const int32_t* positions,
                  const supersonic_kv_cache* cache, void* out, void* workspace, size_t workspace_bytes,
                  int target_wgs);
int prefill_native(size_t device_ordinal, void* stream, int kv_dtype, size_t q_heads, size_t kv_heads,
                   size_t head_dim, size_t rotary_dim, size_t chunk_len, size_t chunk_start, float eps, float scale,
                   const void* q_proj, const void* k_new, const void* v_new, const void* q_norm_w,
                   const void* k_norm_w, const void* cos_table, const void* sin_table,
                   const supersonic_kv_cache* cache, void* out, void* workspace, size_t workspace_bytes,
                   unsigned* claims);
constexpr size_t kClaimBytes = 16 * 128;

// Row repack with cast and zero padding (elementwise.hip): dst row
// (o, i) of dout elements = src[o * so + i * si + 0 .. din) cast from dtype
// code tin to tout (0 f16, 1 f32, 2 bf16), zero past din.  Asynchronous on st.
hipError_t repack_rows(int tin, int tout, const void* src, void* dst, int64_t n_outer, int64_t n_inner, int64_t so,
                       int64_t si, int din, int dout, hipStream_t st);

// Device buffers of one drop-in call (released when it returns).
struct ScratchBuffers {
    void* p[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    int n = 0;
    void* get(size_t bytes) {
        void* q = nullptr;
        if (n >= 6 || hipMalloc(&q, bytes ? bytes : 16) != hipSuccess) return nullptr;
        p[n++] = q;
        return q;
    }
    ~ScratchBuffers() {
        for (int i = 0; i < n; ++i) (void)hipFree(p[i]);
    }
};

inline unsigned grid1d(size_t n, int block) {
    return static_cast<unsigned>((n + block - 1) / block);
}

}  // namespace ssa
