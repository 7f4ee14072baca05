// Host runtime pieces shared by the bridges: the per-device workspace cache.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "supersonic_attn.h"

namespace ssa {

namespace {
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::vector<Workspace> g_ws;  // index device * kWorkspaceSlots + slot
}  // namespace

// Returns a device buffer of at least `bytes` for (`device`, `slot`), growing
// the cached one when needed.  The buffer is reused by every call on that
// device that uses the slot, so such calls that overlap on one device race.
void* device_workspace(int device, size_t bytes, int slot) {
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if (device < 0 || slot < 0 || slot >= kWorkspaceSlots) return nullptr;
    const size_t idx = static_cast<size_t>(device) * kWorkspaceSlots + slot;
    if (idx >= g_ws.size()) g_ws.resize(idx + 1);
    Workspace& w = g_ws[idx];
    if (w.bytes >= bytes && w.ptr) return w.ptr;
    if (w.ptr) {
        (void)hipDeviceSynchronize();
        (void)hipFree(w.ptr);
        w.ptr = nullptr;
        w.bytes = 0;
    }
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    if (hipMalloc(&w.ptr, want) != hipSuccess) {
        w.ptr = nullptr;
        return nullptr;
    }
    // Zero-filled once: kernels that keep counters in the workspace rely on
    // it and leave them zero after every call.
    if (hipMemset(w.ptr, 0, want) != hipSuccess) {
        (void)hipFree(w.ptr);
        w.ptr = nullptr;
        return nullptr;
    }
    w.bytes = want;
    return w.ptr;
}

int device_cu_count(int device) {
    static std::mutex m;
    static std::vector<int> counts;
    std::lock_guard<std::mutex> lock(m);
    if (device < 0) return 0;
    if (static_cast<size_t>(device) >= counts.size()) counts.resize(device + 1, -1);
    if (counts[device] < 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) n = 0;
        counts[device] = n;
    }
    return counts[device];
}

namespace {
std::mutex g_prof_mutex;
ProfileEvents g_prof;
}  // namespace

ProfileEvents take_profile_events() {
    std::lock_guard<std::mutex> lock(g_prof_mutex);
    ProfileEvents e = g_prof;
    g_prof = ProfileEvents{};
    return e;
}

}  // namespace ssa

extern "C" void supersonic_attn_gfx950_set_profile_events(void* before, void* after) {
    std::lock_guard<std::mutex> lock(ssa::g_prof_mutex);
    ssa::g_prof.before = static_cast<hipEvent_t>(before);
    ssa::g_prof.after = static_cast<hipEvent_t>(after);
}

// Waits for `stream`, then reads and clears the error words of the code
// objects that hold bounded waits on this device.
extern "C" int supersonic_attn_gfx950_wait_status(size_t device_ordinal, void* stream, uint32_t* bits) {
    if (!bits) return SUPERSONIC_ERR_NULL;
    *bits = 0;
    ssa::ScopedDevice scoped(static_cast<int>(device_ordinal));
    if (hipStreamSynchronize(static_cast<hipStream_t>(stream)) != hipSuccess) return SUPERSONIC_ERR_SYNC;
    unsigned v = 0;
    if (ssa::take_wait_error_decode(&v) != hipSuccess || ssa::take_wait_error_layer(&v) != hipSuccess ||
        ssa::take_wait_error_gemm(&v) != hipSuccess)
        return SUPERSONIC_ERR_SYNC;
    *bits = v;
    return 0;
}

extern "C" const char* supersonic_attn_version(void) { return "supersonic-attn-gfx950 0.1.0"; }

// RoPE tables on the host, RotaryTables::build (crates/qwen35/src/rotary.rs:15-46):
// inv_freq_i = theta^(-2i / rotary_dim) and the angle pos * inv_freq_i in
// double precision; each cos / sin is rounded to float, then to bf16
// (round-to-nearest-even), the conversion chain of a double tensor cast to
// bf16.  cos_out / sin_out are host arrays of max_pos * rotary_dim / 2 bf16
// bit patterns, row pos holding the rotary_dim / 2 pair angles.
static uint16_t f32_to_bf16_rne_host(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);  // quiet NaN
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

extern "C" int supersonic_attn_rope_tables(size_t rotary_dim, size_t max_pos, double theta, uint16_t* cos_out,
                                           uint16_t* sin_out) {
    if (rotary_dim % 2 != 0 || !(theta > 0.0)) return SUPERSONIC_ERR_ROTARY;
    const size_t half = rotary_dim / 2;
    if (half == 0 || max_pos == 0) return 0;
    if (!cos_out || !sin_out) return SUPERSONIC_ERR_NULL;
    for (size_t i = 0; i < half; ++i) {
        const double freq = 1.0 / std::pow(theta, 2.0 * static_cast<double>(i) / static_cast<double>(rotary_dim));
        for (size_t p = 0; p < max_pos; ++p) {
            const double ang = static_cast<double>(p) * freq;
            cos_out[p * half + i] = f32_to_bf16_rne_host(static_cast<float>(std::cos(ang)));
            sin_out[p * half + i] = f32_to_bf16_rne_host(static_cast<float>(std::sin(ang)));
        }
    }
    return 0;
}
