/*
 * supersonic_attn.h — C ABI of the gfx950 (MI355X) full-attention library.
 *
 * Two groups of entry points:
 *
 *  1. Drop-in replacements for the reference bridge symbols the Rust crate
 *     `kernel-ffi` binds (crates/kernel-ffi/src/prefill_ffi.rs:635-950).  Same
 *     names, argument order and meaning, dtype codes, status codes, null
 *     stream and synchronise-before-return behaviour.
 *  2. Native fused entry points (`supersonic_attn_gfx950_*`): QK RMSNorm +
 *     partial RoPE + KV append (bf16 or fp8 e4m3) + split-K / MFMA attention +
 *     sigmoid gate in one call, asynchronous on a caller stream, over a
 *     contiguous or block-paged KV cache.
 *
 * All pointers are caller-owned device memory unless stated otherwise.  Every
 * function returns 0 on success and a non-zero status otherwise.
 */
#ifndef SUPERSONIC_ATTN_H
#define SUPERSONIC_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes of ScalarType::kernel_dtype_code (crates/gpu-hal/src/scalar_type.rs:25-32). */
#define SUPERSONIC_DTYPE_F16 0
#define SUPERSONIC_DTYPE_F32 1
#define SUPERSONIC_DTYPE_BF16 2
/* KV-cache element codes of the native entry points. */
#define SUPERSONIC_KV_BF16 2
#define SUPERSONIC_KV_FP8_E4M3 3

/* Status codes of the native entry points (the drop-ins keep the reference's). */
#define SUPERSONIC_ERR_DTYPE 1001
#define SUPERSONIC_ERR_HEAD_DIM 1002
#define SUPERSONIC_ERR_HEADS 1003
#define SUPERSONIC_ERR_NULL 1004
#define SUPERSONIC_ERR_ROTARY 1005
#define SUPERSONIC_ERR_WORKSPACE 1006
#define SUPERSONIC_ERR_LAUNCH 1007
#define SUPERSONIC_ERR_SYNC 1008
#define SUPERSONIC_ERR_RANGE 1009
#define SUPERSONIC_ERR_CACHE 1010
/* The device cannot co-schedule the persistent layer's grid (no cooperative
 * launch, or the grid does not fit at once). */
#define SUPERSONIC_ERR_COOPERATIVE 1011
/* Bits of supersonic_attn_gfx950_wait_status(): a bounded wait gave up. */
#define SUPERSONIC_WAIT_LAYER_BARRIER 1u /* persistent layer: grid barrier */
#define SUPERSONIC_WAIT_DECODE_MERGE 2u  /* split-K merge: a partial never arrived */
#define SUPERSONIC_WAIT_GEMM_TAIL 4u     /* prefill GEMM: a tail tile's first k half never arrived */

/* ------------------------------------------------------------------------- */
/* 1. Drop-in reference symbols                                              */
/* ------------------------------------------------------------------------- */

/* Causal GQA prefill attention.  Replaces
 * kernels/full_attention_bridge.cpp:1887 (kernel full_attention.hip:246-361),
 * bound at crates/kernel-ffi/src/prefill_ffi.rs:899-915.
 * query [B, Hq, q_len, D], key/value [B, Hkv, kv_len, D] (dtype), out f32
 * [B, Hq, q_len, D].  Row p attends keys t < min(kv_len, seqlen_offset + p + 1).
 * dtype 0/1/2, any head_dim 1..512 (as the reference on wave64): 64, 128 and
 * 256 run the MFMA kernel directly, other sizes up to 256 run it on copies
 * zero-padded to the next of those, larger ones the f32 kernel on f32 copies.
 * Status: 64 bad dtype, 14 unsupported head_dim (0 or > 512) or heads,
 * 2 workspace allocation, 11 launch, 12 sync. */
int supersonic_qwen35_hip_full_attention_prefill(
    int dtype, size_t device_ordinal, size_t batch_size, size_t q_heads, size_t kv_heads,
    size_t q_len, size_t kv_len, size_t head_dim, size_t num_kv_groups, float scale,
    size_t seqlen_offset, const void* query, const void* key, const void* value, void* out);

/* Same contract; replaces kernels/full_attention_bridge_4b.cpp:1906 (no Rust caller). */
int supersonic_qwen35_4b_hip_full_attention_prefill(
    int dtype, size_t device_ordinal, size_t batch_size, size_t q_heads, size_t kv_heads,
    size_t q_len, size_t kv_len, size_t head_dim, size_t num_kv_groups, float scale,
    size_t seqlen_offset, const void* query, const void* key, const void* value, void* out);

/* Single-token decode attention.  Replaces kernels/prefill_helpers_bridge.cpp:444-470
 * (kernel prefill_helpers.hip:319-404), bound at prefill_ffi.rs:917-931.
 * query [B, Hq, D], key/value [B, Hkv, kv_len, D], out [B, Hq*D] (dtype).
 * dtype 0/2, any head_dim 1..256 and Hq = Hkv * num_kv_groups: head_dim 64,
 * 128, 256 with up to 16 groups run the split-K kernel directly, other head
 * sizes on copies zero-padded to the next of those, more groups as a one-row
 * f32 prefill.  Status: 400 bad dtype, 401 head_dim 0 or > 256 (or heads),
 * 402 launch or allocation, 403 sync (or a split merge that gave up). */
int supersonic_qwen35_hip_full_attention_decode_flat(
    int dtype, size_t device_ordinal, size_t batch_size, size_t q_heads, size_t kv_heads,
    size_t kv_len, size_t head_dim, size_t num_kv_groups, float scale,
    const void* query, const void* key, const void* value, void* out);

/* As decode_flat over a cache whose token capacity kv_stride >= kv_len:
 * key/value [B, Hkv, kv_stride, D].  Declared at prefill_ffi.rs:934-949; the
 * reference implements it for CUDA only (full_attention_cuda.cuh:579-680). */
int supersonic_qwen35_hip_full_attention_decode_flat_strided(
    int dtype, size_t device_ordinal, size_t batch_size, size_t q_heads, size_t kv_heads,
    size_t kv_len, size_t kv_stride, size_t head_dim, size_t num_kv_groups, float scale,
    const void* query, const void* key, const void* value, void* out);

/* BF16 -> FP8 KV quantiser.  Replaces kernels/full_attention_bridge_4b.cpp:5071-5111
 * (kernel full_attention_4b.hip:4786-4829), bound at prefill_ffi.rs:856-867.
 * src [Hkv, seq_len, D] bf16; dst_fp8 [Hkv, max_T, D] u8 and dst_scale
 * [Hkv, max_T] f32 written at positions pos_offset..pos_offset+seq_len.
 * Bytes are bit-identical to the reference encoder (float_to_fp8_e4m3,
 * full_attention_4b.hip:205-232).  dtype 2 only.  Status: 256 bad dtype,
 * 254 launch, 255 sync. */
int supersonic_qwen35_4b_hip_quantize_kv_to_fp8(
    int dtype, size_t device_ordinal, const void* src, void* dst_fp8, float* dst_scale,
    int num_kv_heads, int seq_len, int head_dim, int max_T, int pos_offset);

/* Row RMSNorm, x * rsqrt(mean(x^2) + eps) * (w [+ 1]).  Replaces
 * kernels/full_attention_bridge.cpp:3946 (kernel full_attention.hip:2507-2560),
 * bound at prefill_ffi.rs:638-648.  Status: 74 bad dtype, 71 launch, 72 sync. */
int supersonic_qwen35_hip_rms_norm(
    int dtype, size_t device_ordinal, size_t n_rows, size_t n_cols, float eps,
    int add_unit_offset, const void* xs, const void* weight, void* out);

/* Element cast.  Replaces kernels/full_attention_bridge.cpp:3563, bound at
 * prefill_ffi.rs:650-657.  Status: 137 bad dtype, 135 launch, 136 sync. */
int supersonic_qwen35_hip_cast(
    int input_dtype, int output_dtype, size_t device_ordinal, size_t total_elems,
    const void* xs, void* out);

/* In-place partial RoPE on [seq_len, num_heads, head_dim]; cos/sin tables
 * [*, half_rot] already offset to the chunk's first position.  Replaces
 * kernels/prefill_helpers_bridge.cpp:293 (kernel prefill_helpers.hip:79-108),
 * bound at prefill_ffi.rs:670-680.  Status: 310 bad dtype, 311 launch, 312 sync. */
int supersonic_qwen35_hip_apply_rope_prefill(
    int dtype, size_t device_ordinal, size_t seq_len, size_t num_heads, size_t head_dim,
    size_t half_rot, const void* cos_table, const void* sin_table, void* data);

/* [S, H, D] -> [H, S, D].  Replaces kernels/prefill_helpers_bridge.cpp:315
 * (kernel prefill_helpers.hip:114-130), bound at prefill_ffi.rs:682-690.
 * Status: 320 bad dtype, 321 launch, 322 sync. */
int supersonic_qwen35_hip_transpose_shd_hsd(
    int dtype, size_t device_ordinal, size_t s, size_t h, size_t d, const void* src, void* dst);

/* out = data * sigmoid(gate).  Replaces kernels/prefill_helpers_bridge.cpp:363
 * (kernel prefill_helpers.hip:183-195), bound at prefill_ffi.rs:692-699.
 * Status: 350 bad dtype, 351 launch, 352 sync. */
int supersonic_qwen35_hip_sigmoid_mul(
    int dtype, size_t device_ordinal, size_t total_elems, const void* data, const void* gate,
    void* out);

/* [S, H, 2D] per-head [q | gate] -> query [S, H, D], gate [S, H, D].  Replaces
 * kernels/prefill_helpers_bridge.cpp:393 (kernel prefill_helpers.hip:239-257), bound
 * at prefill_ffi.rs:714-723.  Status: 370 bad dtype, 371 launch, 372 sync. */
int supersonic_qwen35_hip_split_qgate(
    int dtype, size_t device_ordinal, size_t s, size_t num_heads, size_t head_dim,
    const void* src, void* query_out, void* gate_out);

/* out[b] = bf16(lhs[b] . rhs[b]^T) with fp32 accumulation: lhs [batch, m, k],
 * rhs [batch, n, k], out [batch, m, n], bf16 only (the projections, o_proj
 * included, of prefill_engine.rs:356-414).  Replaces
 * kernels/full_attention_bridge_4b.cpp:3683-3704 (kernel full_attention_4b.hip:2513-2575),
 * bound at prefill_ffi.rs:782-792.  m <= 12 (SUPERSONIC_PROJ_SKINNY_MAX_M): HBM-streaming MFMA kernel; larger m:
 * the hand-written tiled MFMA GEMM (SUPERSONIC_PROJ_GEMM=hipblaslt: hipBLASLt).
 * Status: 272 bad dtype, 270 launch, 271 sync. */
int supersonic_qwen35_4b_hip_matmul_rhs_transposed_tiled(
    int dtype, size_t device_ordinal, size_t batch_elems, int m, int n, int k,
    const void* lhs, const void* rhs, void* out);

/* out = lhs + rhs elementwise (fp32 add, one rounding): the residual add of
 * prefill_engine.rs:419-429.  Replaces kernels/prefill_helpers_bridge.cpp:281-290
 * (kernel prefill_helpers.hip:59-68), bound at prefill_ffi.rs:661-668.
 * dtype 0/1/2.  Status: 300 bad dtype, 301 launch, 302 sync. */
int supersonic_qwen35_hip_element_add(
    int dtype, size_t device_ordinal, size_t total_elems, const void* lhs, const void* rhs,
    void* out);

/* ------------------------------------------------------------------------- */
/* 2. Native fused entry points (no reference counterpart; they replace the  */
/*    a1-a9 chain of prefill_engine.rs:1951-2308 and the megakernel's        */
/*    attention phase full_attention_4b.hip:5109-5470)                       */
/* ------------------------------------------------------------------------- */

/* KV cache view.  Token t of sequence b, kv head h lives at element offset
 *   contiguous (block_table == NULL):  b*seq_stride + h*head_stride + t*D
 *   paged:  block_table[b*max_pages_per_seq + t/page_size]*page_stride
 *           + h*head_stride + (t % page_size)*D
 * and its fp8 scale (kv_dtype FP8) at the same formula with D = 1 and the
 * scale_* strides.  The qwen35 crate's [1, Hkv, cap, D] cache per sequence is
 * contiguous mode with head_stride = cap*D. */
typedef struct supersonic_kv_cache {
    void* k;
    void* v;
    float* k_scale;
    float* v_scale;
    const int32_t* block_table;
    int64_t seq_stride;
    int64_t head_stride;
    int64_t page_stride;
    int32_t page_size;
    int32_t max_pages_per_seq;
    int64_t scale_seq_stride;
    int64_t scale_head_stride;
    int64_t scale_page_stride;
} supersonic_kv_cache;

/* Bytes of workspace supersonic_attn_gfx950_decode needs for this shape.
 * A caller-owned workspace must be zero-filled before its first use and not
 * written by the caller between calls: its first 64 KiB hold per-(sequence,
 * kv head) split counters that every call leaves at zero, the rest the split
 * partials (a zero word marks a partial not yet written; each split zeroes its
 * own slots before it writes them).  Calls that share a
 * workspace must not overlap.  batch * kv_heads <= 16384. */
size_t supersonic_attn_gfx950_decode_workspace_size(
    size_t batch, size_t q_heads, size_t kv_heads, size_t head_dim, size_t max_kv_len);

/* One decode step for `batch` sequences: per-head Q/K RMSNorm ((1+w), eps),
 * partial RoPE at positions[b], append K/V at slot positions[b] (fp8: per
 * (token, head) absmax scale, OCP e4m3), split-K attention over slots
 * 0..positions[b] (the new token read unquantised), sigmoid gate.
 * q_proj [batch, Hq*2D] bf16 (per head [q | gate]); k_new, v_new [batch, Hkv*D]
 * bf16; q_norm_w, k_norm_w [D] bf16; cos/sin [max_pos, rotary_dim/2] bf16;
 * positions [batch] int32 device; out [batch, Hq*D] bf16.  max_kv_len >=
 * max(positions)+1.  workspace may be NULL (library-owned).  Asynchronous on
 * `stream` (hipStream_t; NULL = null stream). */
int supersonic_attn_gfx950_decode(
    size_t device_ordinal, void* stream, int kv_dtype,
    size_t batch, size_t q_heads, size_t kv_heads, size_t head_dim, size_t rotary_dim,
    size_t max_kv_len, float eps, float scale,
    const void* q_proj, const void* k_new, const void* v_new,
    const void* q_norm_w, const void* k_norm_w, const void* cos_table, const void* sin_table,
    const int32_t* positions, const supersonic_kv_cache* cache, void* out,
    void* workspace, size_t workspace_bytes);

/* supersonic_attn_gfx950_decode without a workspace and without any allocation
 * (no reference counterpart: for callers that cannot allocate device memory,
 * e.g. code under HIP graph capture or serving loops that forbid hipMalloc).
 * The split partials and arrival counters live in a file-scope device array of
 * 8 MiB per GPU (held until the process ends); shapes whose
 * supersonic_attn_gfx950_decode_workspace_size() exceeds 8 MiB return
 * SUPERSONIC_ERR_WORKSPACE.  Every call on a GPU shares that array, so calls
 * that overlap on one GPU (different streams, or threads) race.  Same
 * arguments and results as supersonic_attn_gfx950_decode. */
int supersonic_attn_gfx950_decode_noalloc(
    size_t device_ordinal, void* stream, int kv_dtype,
    size_t batch, size_t q_heads, size_t kv_heads, size_t head_dim, size_t rotary_dim,
    size_t max_kv_len, float eps, float scale,
    const void* q_proj, const void* k_new, const void* v_new,
    const void* q_norm_w, const void* k_norm_w, const void* cos_table, const void* sin_table,
    const int32_t* positions, const supersonic_kv_cache* cache, void* out);

/* Attention-only decode over an existing cache: q [batch, Hq, D] bf16 (already
 * normalised and rotated), kv_lens [batch] int32 device, optional gate
 * [batch, Hq*D] bf16 (NULL = no gate), out [batch, Hq*D] bf16. */
int supersonic_attn_gfx950_decode_attend(
    size_t device_ordinal, void* stream, int kv_dtype,
    size_t batch, size_t q_heads, size_t kv_heads, size_t head_dim, size_t max_kv_len,
    float scale, const void* q, const int32_t* kv_lens, const supersonic_kv_cache* cache,
    const void* gate, void* out, void* workspace, size_t workspace_bytes);

/* Bytes of workspace supersonic_attn_gfx950_prefill needs for a chunk of
 * chunk_len tokens starting at chunk_start (the staged V^T rows of every
 * position, and for an fp8 cache the bf16 K rows the attention reads).  No
 * GPU call. */
size_t supersonic_attn_gfx950_prefill_workspace_size(
    int kv_dtype, size_t kv_heads, size_t head_dim, size_t chunk_len, size_t chunk_start);

/* One prefill chunk of one sequence (cache sequence index 0): tokens at
 * positions chunk_start .. chunk_start+chunk_len-1.  Q/K RMSNorm + RoPE, K/V
 * written to the cache (bf16, or fp8 with scales), causal MFMA attention over
 * the cached prefix plus the chunk, sigmoid gate.  q_proj [S, Hq*2D],
 * k_new/v_new [S, Hkv*D], out [S, Hq*D], all bf16.  Asynchronous on `stream`.
 * workspace: caller device memory of at least
 * supersonic_attn_gfx950_prefill_workspace_size() bytes (no allocation, no
 * synchronisation: the call can be captured into a HIP graph; calls sharing a
 * workspace must not overlap), or NULL for a library-owned buffer per device
 * (grown on demand with a device synchronisation; overlapping calls on one
 * device then race). */
int supersonic_attn_gfx950_prefill(
    size_t device_ordinal, void* stream, int kv_dtype,
    size_t q_heads, size_t kv_heads, size_t head_dim, size_t rotary_dim,
    size_t chunk_len, size_t chunk_start, float eps, float scale,
    const void* q_proj, const void* k_new, const void* v_new,
    const void* q_norm_w, const void* k_norm_w, const void* cos_table, const void* sin_table,
    const supersonic_kv_cache* cache, void* out, void* workspace, size_t workspace_bytes);

/* A mixed step: one prefill chunk and a batch of decode sequences of the same
 * layer in one call (no reference counterpart: the reference runs prefill and
 * decode as separate engine steps, prefill_engine.rs / decode_engine.rs; this
 * serves chunked-prefill batching).  The two run at the same time on disjoint
 * CUs: the decode first on `stream`, planned for c workgroups (one a CU), the
 * chunk on a library stream forked from `stream` (same priority) with a
 * dynamic item schedule, so its workgroups take the CUs the decode leaves and
 * the decode's as they free up; `stream` then waits for both.  c comes from
 * the two parts' estimated times; SUPERSONIC_MIXED_DECODE_WGS sets it, and 0
 * runs the decode, then the chunk, on `stream`.  Results are those of
 * supersonic_attn_gfx950_decode and supersonic_attn_gfx950_prefill with the
 * same arguments (the layer arguments are shared).  Either part may be empty
 * (batch 0 / chunk_len 0).  The chunk's and the decodes' cache views may
 * share one block-paged cache (different sequences).  workspace: NULL
 * (library-owned) or caller device memory of at least
 * supersonic_attn_gfx950_mixed_workspace_size() bytes, zero-filled before its
 * first use and not written between calls.  Calls sharing the library
 * stream of a device must not overlap.  The library stream and its two events
 * are created by the first CU-split call on a device: make that call outside
 * stream capture (later calls can be captured with a caller workspace). */
typedef struct supersonic_prefill_chunk {
    size_t chunk_len;
    size_t chunk_start;
    const void* q_proj;     /* [chunk_len, Hq*2D] bf16 */
    const void* k_new;      /* [chunk_len, Hkv*D] bf16 */
    const void* v_new;
    const supersonic_kv_cache* cache;  /* the chunk's sequence is cache sequence 0 */
    void* out;              /* [chunk_len, Hq*D] bf16 */
} supersonic_prefill_chunk;

typedef struct supersonic_decode_batch {
    size_t batch;
    size_t max_kv_len;      /* >= max(positions) + 1 */
    const void* q_proj;     /* [batch, Hq*2D] bf16 */
    const void* k_new;      /* [batch, Hkv*D] bf16 */
    const void* v_new;
    const int32_t* positions;  /* [batch] int32, device */
    const supersonic_kv_cache* cache;
    void* out;              /* [batch, Hq*D] bf16 */
} supersonic_decode_batch;

size_t supersonic_attn_gfx950_mixed_workspace_size(
    int kv_dtype, size_t q_heads, size_t kv_heads, size_t head_dim,
    const supersonic_prefill_chunk* chunk, const supersonic_decode_batch* decode);

int supersonic_attn_gfx950_mixed(
    size_t device_ordinal, void* stream, int kv_dtype,
    size_t q_heads, size_t kv_heads, size_t head_dim, size_t rotary_dim, float eps, float scale,
    const void* q_norm_w, const void* k_norm_w, const void* cos_table, const void* sin_table,
    const supersonic_prefill_chunk* chunk, const supersonic_decode_batch* decode,
    void* workspace, size_t workspace_bytes);

/* Input RMSNorm + Q/K/V projections, before the attention:
 *   normed = bf16(hidden * rsqrt(mean(hidden^2) + eps) * (1 + input_norm_w))
 *   q_proj_out = bf16(normed . q_proj_w^T), k_out = bf16(normed . k_proj_w^T),
 *   v_out = bf16(normed . v_proj_w^T)
 * hidden [rows, hidden_dim] bf16 (hidden_dtype 2) or f32 holding bf16 values
 * (hidden_dtype 1); input_norm_w [hidden_dim]; q_proj_w [q_out_dim, hidden_dim],
 * k/v_proj_w [kv_out_dim, hidden_dim]; outputs [rows, q_out_dim] / [rows,
 * kv_out_dim], all bf16 -- the q_proj / k_new / v_new of
 * supersonic_attn_gfx950_decode (q_out_dim = q_heads * 2 * head_dim).  Replaces
 * the megakernel's input norm and projections (full_attention_4b.hip:4942-4967,
 * :5019-5101) and rms_norm_rows_model + matmul_proj of prefill_engine.rs:1951-2117.
 * A norm kernel writes the normed rows once (workspace), then rows <= 12
 * (SUPERSONIC_PROJ_SKINNY_MAX_M) with q/kv_out_dim % 16 == 0 take one
 * weight-streaming launch over the three matrices; otherwise one launch of the
 * hand-written MFMA GEMM over the three matrices as column segments
 * (SUPERSONIC_PROJ_GEMM=hipblaslt: one hipBLASLt GEMM per matrix instead).
 * hidden_dim % 8 == 0.  Asynchronous on `stream`.  workspace: caller device
 * memory of at least supersonic_attn_gfx950_qkv_proj_workspace_size() bytes,
 * zero-filled before its first use and not written by the caller between calls
 * (split-k arrival counters, which every call leaves at zero, and the GEMM's
 * tail hand-over counts, which every call leaves pairwise equal);
 * calls sharing it must not overlap.  NULL: library-owned buffers per device
 * (grown on demand; overlapping calls on one device then race). */
size_t supersonic_attn_gfx950_qkv_proj_workspace_size(
    size_t rows, size_t hidden_dim, size_t q_out_dim, size_t kv_out_dim);
int supersonic_attn_gfx950_qkv_proj(
    size_t device_ordinal, void* stream, int hidden_dtype, size_t rows, size_t hidden_dim,
    size_t q_out_dim, size_t kv_out_dim, float eps, const void* hidden, const void* input_norm_w,
    const void* q_proj_w, const void* k_proj_w, const void* v_proj_w, void* q_proj_out,
    void* k_out, void* v_out, void* workspace, size_t workspace_bytes);

/* Input RMSNorm + Q/K/V projections + per-head Q/K RMSNorm ((1+w), qk_eps) +
 * partial RoPE at positions[r] (+ KV-cache append), the megakernel's steps A-D
 * (full_attention_4b.hip:4942-5101 feeding :5142-5224 and the append
 * :5282-5294), and rms_norm_rows_model + matmul_proj + the norm/RoPE chain of
 * prefill_engine.rs:1951-2096 for one position per row:
 *   q_out [rows, q_heads*D]  normalised + rotated q of each head,
 *   gate_out [rows, q_heads*D] the raw gate half of each q_proj head,
 *   k_out [rows, kv_heads*D] normalised + rotated k, v_out [rows, kv_heads*D] v,
 * all bf16; cache (NULL: none) is a bf16 cache view that receives k_out / v_out
 * of row r at slot positions[r] of sequence r.  The outputs feed
 * supersonic_attn_gfx950_decode_attend (q, gate, kv_lens = positions + 1).
 * Rows <= 12 with rows * hidden_dim <= 32768 and head_dim 128/256: one
 * weight-streaming launch whose epilogue normalises and rotates each head as
 * its last column block completes; otherwise the projections, then one wave
 * per (row, head).  workspace: at least
 * supersonic_attn_gfx950_qkv_proj_rope_workspace_size() bytes, zero-filled
 * before first use (per-head arrival counters left at zero by every call),
 * or NULL for a library-owned buffer.  Status: SUPERSONIC_ERR_CACHE for an
 * fp8 cache. */
size_t supersonic_attn_gfx950_qkv_proj_rope_workspace_size(
    size_t rows, size_t hidden_dim, size_t q_heads, size_t kv_heads, size_t head_dim);
int supersonic_attn_gfx950_qkv_proj_rope(
    size_t device_ordinal, void* stream, int hidden_dtype, size_t rows, size_t hidden_dim,
    size_t q_heads, size_t kv_heads, size_t head_dim, size_t rotary_dim, float eps, float qk_eps,
    const void* hidden, const void* input_norm_w, const void* q_proj_w, const void* k_proj_w,
    const void* v_proj_w, const void* q_norm_w, const void* k_norm_w, const void* cos_table,
    const void* sin_table, const int32_t* positions, void* q_out, void* gate_out, void* k_out,
    void* v_out, const supersonic_kv_cache* cache, void* workspace, size_t workspace_bytes);

/* One whole attention layer of a decode step in a single persistent kernel
 * (the attention phase as a device function between the projections, as the
 * reference's persistent megakernel runs it: qwen36_moe_persistent/
 * full_attn_phase.cuh:1-20, full_attention_4b.hip:4842-5577):
 *   normed = RMSNorm(hidden) (1 + input_norm_w, eps)
 *   q_proj, k, v = normed . W_q^T, W_k^T, W_v^T               (bf16)
 *   attn = supersonic_attn_gfx950_decode(q_proj, k, v, ...)  (QK norm with
 *          qk_eps, RoPE, KV append at positions[b], attention, gate)
 *   hidden = bf16(hidden + bf16(attn . W_o^T))                (in place)
 * hidden [batch, hidden_dim] bf16 (hidden_dtype 2) or f32 holding bf16 values
 * (1); weights as supersonic_attn_gfx950_qkv_proj / _o_proj_residual; cache,
 * positions, tables as supersonic_attn_gfx950_decode.  One workgroup per
 * compute unit, three phases separated by device-wide barriers, launched
 * cooperatively so that every workgroup of the grid is resident at once
 * (SUPERSONIC_ERR_COOPERATIVE when the device cannot do that).  Limits: batch <= 16,
 * batch * hidden_dim <= 32768 and batch * q_heads * head_dim <= 32768,
 * hidden_dim % 16 == 0, head_dim 128/256, q_heads / kv_heads <= 4, 16-byte
 * aligned hidden and weights (otherwise SUPERSONIC_ERR_RANGE: use the
 * separate entry points).  workspace (required): at least
 * supersonic_attn_gfx950_decode_layer_workspace_size() bytes, zero-filled
 * before its first use (barrier and split counters that every call leaves at
 * zero); calls sharing it must not overlap.  Asynchronous on `stream`. */
size_t supersonic_attn_gfx950_decode_layer_workspace_size(
    size_t batch, size_t hidden_dim, size_t q_heads, size_t kv_heads, size_t head_dim, size_t max_kv_len);
int supersonic_attn_gfx950_decode_layer(
    size_t device_ordinal, void* stream, int hidden_dtype, int kv_dtype, size_t batch, size_t hidden_dim,
    size_t q_heads, size_t kv_heads, size_t head_dim, size_t rotary_dim, size_t max_kv_len, float eps,
    float qk_eps, float scale, void* hidden, const void* input_norm_w, const void* q_proj_w,
    const void* k_proj_w, const void* v_proj_w, const void* q_norm_w, const void* k_norm_w,
    const void* o_proj_w, const void* cos_table, const void* sin_table, const int32_t* positions,
    const supersonic_kv_cache* cache, void* workspace, size_t workspace_bytes);

/* Output projection with the residual add, after the gated attention:
 *   hidden[r, j] = bf16(hidden[r, j] + bf16(sum_c attn[r, c] * o_proj_w[j, c]))
 * attn [rows, attn_dim] bf16 (the fused decode/prefill `out`), o_proj_w
 * [hidden_dim, attn_dim] bf16, hidden [rows, hidden_dim] updated in place, bf16
 * (hidden_dtype 2, the prefill engine's hidden) or f32 holding bf16 values
 * (hidden_dtype 1, the megakernel's hidden_f32).  Replaces the megakernel's
 * step G (full_attention_4b.hip:5481-5577) and matmul_proj + residual_add of
 * prefill_engine.rs:2308-2334.  rows <= 12 (SUPERSONIC_PROJ_SKINNY_MAX_M, at most 64) with attn_dim % 8 == 0: one
 * HBM-streaming MFMA kernel with the residual fused; otherwise the hand-written
 * MFMA GEMM with the residual add in its epilogue, in place
 * (SUPERSONIC_PROJ_GEMM=hipblaslt: hipBLASLt and a residual kernel).
 * Asynchronous on `stream`.  workspace: split-k partials and arrival counters,
 * the GEMM's tail-split flags and partials, or (hipBLASLt) the GEMM output rows; caller device memory of at
 * least supersonic_attn_gfx950_o_proj_workspace_size() bytes under the same
 * rules as supersonic_attn_gfx950_qkv_proj's, or NULL for library-owned
 * buffers per device. */
size_t supersonic_attn_gfx950_o_proj_workspace_size(size_t rows, size_t hidden_dim, size_t attn_dim);
int supersonic_attn_gfx950_o_proj_residual(
    size_t device_ordinal, void* stream, int hidden_dtype, size_t rows, size_t hidden_dim,
    size_t attn_dim, const void* attn, const void* o_proj_w, void* hidden,
    void* workspace, size_t workspace_bytes);

/* OCP e4m3 variant of supersonic_qwen35_4b_hip_quantize_kv_to_fp8: same
 * layout and scale rule (scale = max(absmax/448, 1e-12)), hardware OCP
 * round-to-nearest-even codes, the codec the fused entry points write.
 * Asynchronous on `stream`. */
int supersonic_attn_gfx950_quantize_kv_fp8_ocp(
    size_t device_ordinal, void* stream, const void* src, void* dst_fp8, float* dst_scale,
    int num_kv_heads, int seq_len, int head_dim, int max_T, int pos_offset);

/* Benchmark hook (no reference counterpart): two hipEvent_t recorded on the
 * launch stream right before and right after the dominant kernel (split-K
 * decode kernel, MFMA prefill kernel, o_proj kernel) of the next fused-entry call on any
 * thread; the pair is consumed by that call.  NULL, NULL clears it. */
void supersonic_attn_gfx950_set_profile_events(void* before, void* after);

/* RoPE cos / sin tables on the host, as RotaryTables::build
 * (crates/qwen35/src/rotary.rs:15-46) builds them: inv_freq_i =
 * theta^(-2i/rotary_dim), angle pos * inv_freq_i in double precision, each
 * value rounded to float and then to bf16 (RNE).  cos_out / sin_out: host
 * arrays of max_pos * rotary_dim/2 bf16 bit patterns, [max_pos, rotary_dim/2],
 * the layout the fused entry points read (after a copy to the device).
 * No GPU call.  Status: SUPERSONIC_ERR_ROTARY (odd rotary_dim or theta <= 0),
 * SUPERSONIC_ERR_NULL. */
int supersonic_attn_rope_tables(size_t rotary_dim, size_t max_pos, double theta, uint16_t* cos_out,
                                uint16_t* sin_out);

/* Bounded waits (no reference counterpart).  Waits that depend on another
 * workgroup (the persistent layer's grid barriers, the split-K merge's poll
 * for partials in flight, the prefill GEMM's tail hand-over) give up after a bounded number of polls, set a bit
 * in a sticky per-device error word and let the kernel exit normally.  This
 * call synchronises `stream`, returns the OR of the SUPERSONIC_WAIT_* bits
 * set since the last call in *bits and clears them.  A set bit means some
 * output since then is wrong, and the workspace of the call that set it must be
 * zero-filled again before reuse.  Under the documented preconditions
 * (cooperative launch, zero-filled workspaces) no wait gives up.  The
 * synchronous drop-ins check the word themselves and return their sync-failure
 * status.  SUPERSONIC_WAIT_POLLS (environment) overrides the poll bound, for
 * tests that force the give-up path. */
int supersonic_attn_gfx950_wait_status(size_t device_ordinal, void* stream, uint32_t* bits);

/* Library version string. */
const char* supersonic_attn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SUPERSONIC_ATTN_H */
