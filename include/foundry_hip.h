/*
 * foundry_hip.h: the C-ABI of libfoundry_hip.so, the MI355X (gfx950) backend
 * for Foundry's 4-bit quantized weight path.
 *
 * This is the one boundary a host binds. It is what the reference's `Device`
 * trait (src/nn/primitive.rs:70-120) needs from a backend, flattened to plain
 * pointers and sizes: a device owns one HIP stream; storage is device memory
 * the device allocated; every op returns a fresh output the caller allocated
 * and passes in. A Rust `src/hip` backend binds these through a thin FFI crate
 * (see INTEGRATION.md); the Python package foundry_amd binds them with ctypes.
 *
 * Conventions
 * - Every function returns an fh_status (0 = FH_OK). On error, fh_last_error()
 *   returns a thread-local message naming the function and the cause.
 * - Failure is sticky, as the reference's command stream is
 *   (src/metal/stream.rs:109-115, :201-212): once a launch or a
 *   synchronisation reports a device error, every later call on that device
 *   returns FH_ERR_FAILED.
 * - Ops validate shapes and dtypes before any launch (the reference does so in
 *   `primitive::output`, src/nn/primitive.rs:146-289) and check that every
 *   operand lies inside a live allocation of this device (the reference's
 *   ForeignStorage check, src/metal/mod.rs:187-200). A rejected call launches
 *   nothing.
 * - Ops are asynchronous on the device's stream. fh_download synchronises
 *   first (src/metal/mod.rs:614), fh_synchronize waits for everything.
 * - One host thread per device, as in the reference (Rc-based, !Send
 *   tensors). No internal locking.
 *
 * bf16 values are passed as their uint16_t bit patterns.
 */
#ifndef FOUNDRY_HIP_H
#define FOUNDRY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FH_ABI_VERSION 2

typedef struct fh_device fh_device;
typedef struct fh_graph fh_graph;

/* Error kinds. Mirrors MetalError (src/metal/error.rs:7-58) where a HIP
 * counterpart exists, plus the Tensor-level validation errors
 * (src/nn/error.rs) that the reference raises before the device call. */
typedef enum fh_status {
    FH_OK = 0,
    FH_ERR_INVALID_ARGUMENT = 1,  /* shapes, sizes or null pointers do not fit the op */
    FH_ERR_DEVICE_UNAVAILABLE = 2,/* MetalError::DeviceUnavailable */
    FH_ERR_ALLOCATION = 3,        /* MetalError::BufferAllocation */
    FH_ERR_FOREIGN_STORAGE = 4,   /* MetalError::ForeignStorage */
    FH_ERR_OUT_OF_BOUNDS = 5,     /* MetalError::ToBytesOutOfBounds; operand past its allocation */
    FH_ERR_LAUNCH = 6,            /* a kernel launch was refused */
    FH_ERR_FAILED = 7,            /* MetalError::CommandBufferFailed (sticky) */
    FH_ERR_INDEX_TOO_LARGE = 8,   /* MetalError::KernelIndexTooLarge */
    FH_ERR_DTYPE = 9,             /* MetalError::DTypeNotFloat; TensorError::IndicesNotU32 */
    FH_ERR_UNSUPPORTED = 10,      /* valid request the kernels do not implement (e.g. group != 64) */
    FH_ERR_CAPTURE = 11           /* graph capture misuse */
} fh_status;

/* src/nn/dtype.rs:6-10 */
typedef enum fh_dtype { FH_F32 = 0, FH_BF16 = 1, FH_U32 = 2 } fh_dtype;

/* src/nn/profile.rs:7-13. STEPS keeps normal batching and times the span of
 * work; KERNELS brackets every dispatch with events (per-kernel GPU time). */
typedef enum fh_profile_mode {
    FH_PROFILE_OFF = 0,
    FH_PROFILE_STEPS = 1,
    FH_PROFILE_KERNELS = 2
} fh_profile_mode;

/* src/nn/memory.rs:1-5 */
typedef struct fh_allocated_memory {
    uint64_t bytes;
    const char *source; /* static string */
} fh_allocated_memory;

/* src/nn/profile.rs:15-21 (DeviceProfile) */
typedef struct fh_profile {
    uint64_t dispatches;      /* kernels launched since the last take */
    uint64_t allocations;     /* fh_alloc calls since the last take */
    uint64_t allocated_bytes; /* bytes they requested */
    uint64_t gpu_busy_ns;     /* union of timed GPU intervals (0 when unavailable) */
} fh_profile;

/* ---- errors and version ---- */
const char *fh_last_error(void);
int fh_abi_version(void);

/* ---- device lifecycle: MetalDevice::new / ::profiled (src/metal/mod.rs:108-149) ---- */
int fh_device_count(int *count);
int fh_device_create(int ordinal, fh_device **out);
int fh_device_create_profiled(int ordinal, int mode, fh_device **out);
/* Synchronises, frees every allocation the device still owns, destroys it. */
int fh_device_destroy(fh_device *dev);
/* Device::device_name (src/nn/primitive.rs:74) */
int fh_device_name(const fh_device *dev, char *buf, size_t len);
/* Device::synchronize (src/nn/primitive.rs:86) */
int fh_synchronize(fh_device *dev);
/* The device's HIP stream (hipStream_t), for callers that time with events. */
int fh_device_stream(fh_device *dev, void **stream);

/* ---- storage: Device::{zeros, storage_from_bytes, storage_to_bytes}
 *      (src/nn/primitive.rs:88-103; src/metal/mod.rs:565-637) ---- */
/* Allocates nbytes (at least 1) of device memory, 256-byte aligned. With
 * zero_fill != 0 the memory is cleared before any later op on the stream
 * reads it (Device::zeros). */
int fh_alloc(fh_device *dev, size_t nbytes, int zero_fill, void **out);
/* Frees an allocation of this device after the work queued on it ends.
 * A live graph retains every allocation its captured ops touched, as a
 * Metal command buffer retains its buffers (src/metal/mod.rs:280-282): the
 * allocation is then no longer usable by ops but stays allocated until the
 * last graph that uses it is destroyed. A free asked for while capturing is
 * carried out at fh_capture_end, on the same rule. */
int fh_free(fh_device *dev, void *ptr);
/* Host -> device copy into an owned range; ordered on the stream. */
int fh_upload(fh_device *dev, void *dst, const void *src, size_t nbytes);
/* Device -> host copy of an owned range; synchronises first. */
int fh_download(fh_device *dev, void *dst, const void *src, size_t nbytes);

/* ---- memory and profile counters (src/nn/primitive.rs:75-83) ----
 * Bytes counted: every live allocation (including retired ones a graph still
 * holds) plus the device's own work areas (the 33 MB of GEMV/GEMM partial
 * sums and the batched GEMV's x image), allocated at creation. */
int fh_max_memory_allocated(const fh_device *dev, fh_allocated_memory *out);
int fh_reset_run_memory_peak(fh_device *dev);
int fh_run_memory_peak(const fh_device *dev, fh_allocated_memory *out);
/* Counters since the previous take, then reset. Returns FH_ERR_UNSUPPORTED
 * (and leaves *out zeroed) when the device was not created profiled, as the
 * reference returns None (src/nn/primitive.rs:83). */
int fh_take_profile(fh_device *dev, fh_profile *out);

/* ---- batching: the HIP counterpart of the reference's CommandStream
 * (src/metal/stream.rs:29-215), which encodes many dispatches and commits
 * them at once. Between begin and end, ops are validated and recorded, not
 * run; fh_graph_launch replays the recording on the device's stream. ---- */
int fh_capture_begin(fh_device *dev);
/* Ends the capture; the graph retains the allocations its ops touched. */
int fh_capture_end(fh_device *dev, fh_graph **out);
/* FH_ERR_FOREIGN_STORAGE for a graph of another (or a destroyed) device. */
int fh_graph_launch(fh_device *dev, fh_graph *graph);
/* Waits for the device's queued work (a replay may still be running), then
 * destroys the graph and releases its allocations; any the caller already
 * freed are freed now. A graph may outlive its device (it can then only be
 * destroyed). */
int fh_graph_destroy(fh_graph *graph);

/* ---- event timing on the device's stream ---- */
/* Records a start event now, in stream order. */
int fh_timer_begin(fh_device *dev);
/* Records an end event, waits for it, writes the milliseconds between the two. */
int fh_timer_end(fh_device *dev, double *elapsed_ms);

/* ---- the HBM read ceiling, for measurement: one launch that reads nbytes
 * (16-byte aligned, a multiple of 16) in 16-byte loads, 32 KB per block,
 * and writes one XOR word per wavefront to out (fh_read_probe_blocks gives
 * the number of words). No counterpart in the reference (it is the
 * roofline's measured read rate beside the quoted peak). ---- */
int fh_read_probe_blocks(uint64_t nbytes, uint64_t *blocks);
int fh_read_probe(fh_device *dev, const void *src, uint64_t nbytes, uint32_t *out);

/* ======================================================================
 * q4 ops. Weight format (affine group quantisation):
 *   wq     u32 [rows, k/8]   element j of a row = nibble j%8 (bits 4*(j%8)..+3)
 *                            of word j/8, little-endian nibble order
 *   scales bf16[rows, k/group]
 *   biases bf16[rows, k/group]
 *   w[r, j] = f32(scales[r, j/group]) * q[r, j] + f32(biases[r, j/group])
 * The kernels implement group = 64 and k a multiple of 64.
 * ====================================================================== */

/* q4 Embedding::forward (src/nn/linear.rs:53-69) -> Op::IndexSelect{dim 0}
 * (src/nn/primitive.rs:258-289; src/metal/mod.rs:483-500;
 * src/metal/kernels/index_select.metal:11-29) over a q4 table.
 * out bf16[n_ids, k]: out[i, :] = RNE_bf16(w[ids[i], :]); an id >= rows
 * writes a zero row. Bit-exact. n_ids may be 0. */
int fh_q4_embed(fh_device *dev, const uint32_t *wq, const uint16_t *scales,
                const uint16_t *biases, int64_t rows, int64_t k, int64_t group,
                const uint32_t *ids, int64_t n_ids, uint16_t *out);

/* q4 Linear::forward (src/nn/linear.rs:22-35) -> Op::Matmul
 * (src/nn/primitive.rs:234-256; src/metal/mod.rs:434-481;
 * src/metal/kernels/matmul.metal:29-65) with a q4 right operand:
 *   y[i, r] = sum_j x[i, j] * w[r, j]       (fp32 accumulation)
 * x bf16[m, k] with row stride x_ld (elements, >= k); y [m, n] contiguous,
 * y_dtype FH_BF16 (RNE of the fp32 sum, the reference's output rounding) or
 * FH_F32 (the fp32 sum itself). m <= 8 runs the decode GEMV, larger m the
 * prefill GEMM. m may be 0. */
int fh_q4_matmul(fh_device *dev, const uint16_t *x, int64_t m, int64_t k,
                 int64_t x_ld, const uint32_t *wq, const uint16_t *scales,
                 const uint16_t *biases, int64_t n, int64_t group, void *y,
                 int y_dtype);

/* Materialised dequantisation: out bf16[rows, k] = RNE_bf16(w). Bit-exact.
 * The value the prefill GEMM feeds to the matrix cores. */
int fh_q4_dequant(fh_device *dev, const uint32_t *wq, const uint16_t *scales,
                  const uint16_t *biases, int64_t rows, int64_t k, int64_t group,
                  uint16_t *out);

/* ======================================================================
 * Strided ops: the reference's non-quantized Ops (src/nn/primitive.rs:48-68)
 * over strided views, so that a backend can run every Op of the unchanged
 * model code (Device::run and Device::run_in_place, src/metal/mod.rs:639-
 * 725). Each entry point is one plain kernel of the Metal kernel it replaces
 * (src/metal/kernels/{copy,unary,binary,reduce,matmul,index_select,
 * slice_scatter}.metal) with the same arithmetic: fp32 math on values
 * decoded from the dtype, the output rounded once (RNE for bf16).
 *
 * A view is the reference's Layout flattened as StridedArgs is
 * (src/metal/args.rs:22-29): element offset, rank 0..4, sizes and strides in
 * elements (strides >= 0; a broadcast dim has stride 0). The pointer passed
 * beside a view is the storage base; the view addresses base + offset + sum
 * i_d * stride_d. Every element a view addresses must lie in one live
 * allocation of the device. Outputs are fresh and contiguous, as
 * Device::run returns them; shape rules are those of primitive::output
 * (src/nn/primitive.rs:146-289). dtype is an fh_dtype.
 * ====================================================================== */

typedef struct fh_view {
    int64_t offset;
    int32_t ndim;
    int64_t dims[4];
    int64_t strides[4];
} fh_view;

/* UnaryOp, BinaryOp, ReduceOp (src/nn/primitive.rs:14-46) */
typedef enum fh_unary_op { FH_NEG = 0, FH_EXP = 1, FH_SQRT = 2, FH_RECIPROCAL = 3 } fh_unary_op;
typedef enum fh_binary_op { FH_ADD = 0, FH_SUB = 1, FH_MUL = 2, FH_DIV = 3 } fh_binary_op;
typedef enum fh_reduce_op { FH_SUM = 0, FH_AMAX = 1, FH_ARGMAX = 2 } fh_reduce_op;

/* Op::Copy (copy_strided, copy.metal:1-13): dst = the view's elements in
 * row-major order. Any dtype. */
int fh_copy_strided(fh_device *dev, int dtype, const void *src, const fh_view *view, void *dst);

/* Op::ToDtype (to_dtype_strided, copy.metal:15-36): F32 <-> BF16 (RNE with
 * the quiet-NaN rule); the same float dtype is a copy. */
int fh_to_dtype(fh_device *dev, int from, const void *src, const fh_view *view, int to, void *dst);

/* Op::Unary (unary_strided, unary.metal:1-40) on F32 or BF16. */
int fh_unary(fh_device *dev, int op, int dtype, const void *src, const fh_view *view, void *dst);

/* Op::Binary (binary_strided, binary.metal:1-44). Both views have the
 * output's dims: a caller broadcasts first by expanding (stride 0), as
 * Tensor::binary does (src/nn/tensor.rs:332-343). */
int fh_binary(fh_device *dev, int op, int dtype, const void *lhs, const fh_view *lhs_view,
              const void *rhs, const fh_view *rhs_view, void *dst);

/* Op::Reduce{op, dim} (reduce_rows / argmax_rows, reduce.metal:1-93): one
 * block of 256 threads per output element; thread t folds k = t, t + 256,
 * ..., then a halving tree, the reference's order (its sums are bit-equal).
 * Output dims = the view's with dims[dim] = 1, contiguous; SUM/AMAX keep the
 * dtype, ARGMAX writes u32 (first index on ties). AMAX/ARGMAX over an empty
 * dim are refused (TensorError::EmptyReduction); an empty SUM is 0. */
int fh_reduce(fh_device *dev, int op, int dtype, const void *src, const fh_view *view, int32_t dim,
              void *dst);

/* Op::Matmul (MetalDevice::matmul, src/metal/mod.rs:434-481; matmul_tiled,
 * matmul.metal:29-65): lhs [..., m, k] x rhs [..., k, n] with equal batch
 * dims, out [..., m, n]; fp32 sums in order of k, output rounded once.
 * Any strides are read in place (no operand copy). */
int fh_matmul(fh_device *dev, int dtype, const void *lhs, const fh_view *lhs_view, const void *rhs,
              const fh_view *rhs_view, void *dst);

/* Op::IndexSelect{dim 0} (index_select_rows, index_select.metal:11-29):
 * table 2-D [rows, cols] (F32 or BF16), ids U32 1-D [n] -> dst [n, cols];
 * an id >= rows gives a zero row. */
int fh_index_select(fh_device *dev, int dtype, const void *table, const fh_view *table_view,
                    const uint32_t *ids, const fh_view *ids_view, void *dst);

/* Op::Cat{dim} (MetalDevice::cat, src/metal/mod.rs:502-524): dst = lhs then
 * rhs along dim; all other dims equal. */
int fh_cat(fh_device *dev, int dtype, int32_t dim, const void *lhs, const fh_view *lhs_view,
           const void *rhs, const fh_view *rhs_view, void *dst);

/* Device::run_in_place(Op::SliceScatter{dim, start}) (src/metal/mod.rs:697-
 * 725; slice_scatter_strided, slice_scatter.metal:1-21): writes src into
 * target[..., start : start + src.dims[dim], ...] in place. The target view
 * is contiguous (Tensor::slice_scatter requires it, src/nn/tensor.rs:
 * 307-316) and src may be strided. */
int fh_slice_scatter(fh_device *dev, int dtype, int32_t dim, int64_t start, void *target,
                     const fh_view *target_view, const void *src, const fh_view *src_view);

/* ======================================================================
 * Decoder-step ops: the plumbing around the q4 linears that a Llama decode
 * step needs, each one kernel where the reference runs several dispatches.
 * All tensors are bf16 (uint16_t bits) unless stated; every op rounds where
 * the reference's op sequence rounds (its tensors are bf16).
 * `positions` are device u32 arrays, so a captured decode step can be
 * replayed with the position advanced on the device (fh_advance_positions).
 * ====================================================================== */

/* RmsNorm::forward (src/nn/norm.rs:32-50), optionally fused with the
 * residual add before it (src/models/llama/model.rs:254-279):
 *   h = residual ? RNE(x + residual) : x   (h written to residual_out)
 *   y = RNE(RNE(h * 1/sqrt(sum(h^2)/dim + eps)) * weight)
 * x, residual, residual_out, y: [rows, dim]; weight: [dim]. dim is a multiple
 * of 8, at most 8192; operands are 16-byte aligned. residual_out may alias
 * residual (an in-place residual stream). */
int fh_rms_norm(fh_device *dev, const uint16_t *x, const uint16_t *residual,
                uint16_t *residual_out, const uint16_t *weight, int64_t rows, int64_t dim,
                float eps, uint16_t *y);

/* KV caches of the attention entry points below. One (sequence, KV head)
 * owns max_len * head_dim elements of each cache. V is [max_len][head_dim].
 * K holds the same keys in groups of 16: group g (keys 16 g .. 16 g + n_g -
 * 1, n_g = min(16, max_len - 16 g)) is n_g * head_dim contiguous elements
 * laid out [head_dim / 32][n_g][32], i.e. dim d of key j is element
 * 16 g * head_dim + (d / 32) * n_g * 32 + (j % 16) * 32 + d % 32 of the
 * region. The reference's StaticCache (src/nn/kv_cache.rs:41-80) keeps K as
 * [max_len][head_dim]; the regrouping lets a matrix-core fragment of 16 keys
 * x 32 dims be read as one 1 KB run. Sizes are unchanged. */

/* apply_rotary_pos_emb (src/models/llama/rotary_emb.rs:62-85) on q and k of
 * each token, then StaticCache::update (src/nn/kv_cache.rs:41-80) of k and v
 * at the token's position. qkv: [tokens, (n_heads + 2 n_kv) * head_dim] (q
 * heads, then k heads, then v heads); cos_tab/sin_tab: [table_len, head_dim];
 * positions: device u32 [tokens]; k_cache/v_cache: n_kv regions of max_len *
 * head_dim (K grouped as above); q_out: [tokens, n_heads, head_dim]. head_dim is a multiple of 16 and every
 * operand 16-byte aligned. A position >= max_len or >= table_len writes
 * nothing. */
int fh_rope_kv(fh_device *dev, const uint16_t *qkv, int64_t tokens, int64_t n_heads,
               int64_t n_kv, int64_t head_dim, const uint16_t *cos_tab, const uint16_t *sin_tab,
               int64_t table_len, const uint32_t *positions, uint16_t *k_cache,
               uint16_t *v_cache, int64_t max_len, uint16_t *q_out);

/* Bytes of device workspace fh_attention needs for these sizes (the scores
 * and per-chunk softmax statistics of every row). */
int fh_attention_workspace(int64_t tokens, int64_t n_heads, int64_t n_kv, int64_t head_dim,
                           int64_t max_len, uint64_t *bytes);

/* scaled_dot_product_attention (src/nn/attention.rs:23-60) with the causal
 * mask (src/nn/masking.rs:11-32): query token t attends keys 0..positions[t]
 * of its KV head (grouped-query: head h uses KV head h / (n_heads/n_kv)).
 * Scores RNE(q.k) (fp32 sums), times scale in fp32, softmax in fp32,
 * probabilities RNE to bf16 from the row's global max and sum, out =
 * RNE(sum p v). q, out: [tokens, n_heads * head_dim]; caches: n_kv regions of
 * max_len * head_dim (K grouped as above). head_dim is 64, 128 or 256 and n_heads/n_kv at most 8; tokens at
 * most 65535. The context is split into chunks of 64 keys scored in
 * parallel, and P.V is split over head_dim, so a long context fills the
 * device. workspace: at least fh_attention_workspace() bytes of device
 * memory, 16-byte aligned, no initial contents; calls that share a workspace
 * must not run concurrently. */
int fh_attention(fh_device *dev, const uint16_t *q, const uint16_t *k_cache,
                 const uint16_t *v_cache, const uint32_t *positions, int64_t tokens,
                 int64_t n_heads, int64_t n_kv, int64_t head_dim, int64_t max_len, float scale,
                 void *workspace, uint64_t workspace_bytes, uint16_t *out);

/* Bytes of device workspace fh_decode_attention needs for these sizes. */
int fh_decode_attention_workspace(int64_t batch, int64_t n_heads, int64_t n_kv, int64_t head_dim,
                                  int64_t max_len, uint64_t *bytes);

/* The decode step's attention for a batch of sequences that each add one
 * token: fh_rope_kv's RoPE of the token's q and k and its cache write at
 * positions[b], then fh_attention over keys 0..positions[b] of sequence b --
 * the same rounding points, in two kernel launches instead of three, or in
 * one when max_len <= 1024 and head_dim is 64 or 128 (the workspace is then
 * not touched, but is still checked and required). qkv:
 * [batch, (n_heads + 2 n_kv) * head_dim]; cos_tab/sin_tab: [table_len,
 * head_dim]; positions: device u32 [batch]; k_cache/v_cache: batch x n_kv
 * regions of max_len * head_dim (one cache per sequence, K grouped as above);
 * out: [batch, n_heads *
 * head_dim]. A position >= max_len or >= table_len writes nothing to the
 * caches and zeros to out. head_dim is 64, 128 or 256, n_heads/n_kv at most
 * 8, batch at most 65535, operands 16-byte aligned. workspace: as for
 * fh_attention, at least fh_decode_attention_workspace() bytes. */
int fh_decode_attention(fh_device *dev, const uint16_t *qkv, int64_t batch, int64_t n_heads,
                        int64_t n_kv, int64_t head_dim, const uint16_t *cos_tab,
                        const uint16_t *sin_tab, int64_t table_len, const uint32_t *positions,
                        uint16_t *k_cache, uint16_t *v_cache, int64_t max_len, float scale,
                        void *workspace, uint64_t workspace_bytes, uint16_t *out);

/* fh_decode_attention without a workspace argument, for callers that cannot
 * allocate (code under graph capture, tight serving loops, harnesses that
 * forbid allocation). No counterpart in the reference. The workspace is a
 * static array of FH_DECODE_SCRATCH_BYTES in device memory, one per GPU,
 * held from the library's first use on that GPU until the process ends; this
 * call allocates nothing (on a profiled device it records only pooled
 * events). Sizes whose workspace (fh_decode_attention_workspace) exceeds it
 * return FH_ERR_UNSUPPORTED. Every call on one GPU shares the array: calls
 * that overlap on one GPU (from two fh_devices' streams) race. The workspace
 * needs no initial contents, so nothing is cleared between calls. */
#define FH_DECODE_SCRATCH_BYTES (32ull << 20)
int fh_decode_attention_noalloc(fh_device *dev, const uint16_t *qkv, int64_t batch, int64_t n_heads,
                                int64_t n_kv, int64_t head_dim, const uint16_t *cos_tab,
                                const uint16_t *sin_tab, int64_t table_len, const uint32_t *positions,
                                uint16_t *k_cache, uint16_t *v_cache, int64_t max_len, float scale,
                                uint16_t *out);

/* Decode-step fusions of the q4 Linear (m <= 8 rows, the GEMV; larger m
 * returns FH_ERR_UNSUPPORTED -- use the unfused ops -- except
 * fh_q4_gate_up_silu without a norm weight, below). Same arithmetic as the
 * unfused sequence, with no intermediate tensor in memory:
 *   fh_q4_matmul_rmsnorm: y = fh_rms_norm(x, residual, residual_out,
 *     norm_weight, eps) @ W^T (src/nn/norm.rs:32-50 then src/nn/linear.rs:
 *     22-35). x, residual, residual_out: [m, k] (row stride k); residual and
 *     residual_out may be null; residual_out (the updated residual stream h)
 *     must not overlap x or residual. The sum of squares runs in another
 *     order than fh_rms_norm's (a normalised value can differ by one bf16 ulp).
 *   fh_q4_gate_up_silu: act = fh_silu_mul(x' @ W^T) for W = [gate; up] rows
 *     (n = 2f): act[:, j] = RNE(RNE(g_j / (exp(-g_j) + 1)) * u_j) with g, u
 *     the bf16 outputs of the linear (src/models/llama/mlp.rs:49-58); act:
 *     [m, f] bf16. x' = x, or with norm_weight, the RMSNorm above (residual
 *     arguments as for fh_q4_matmul_rmsnorm). Above 8 rows, without a norm
 *     weight or residual: the prompt GEMM with the activation in its
 *     epilogue, when its tiles of 256 rows x 128 gate/up pairs fill the GPU
 *     (f % 128 == 0, k % 512 == 0; x and act 16-byte aligned, act not
 *     overlapping x); other shapes return FH_ERR_UNSUPPORTED. Bit-identical
 *     to fh_q4_matmul then fh_silu_mul.
 * The q4 operands follow fh_q4_matmul (group 64); x 16-byte aligned. */
int fh_q4_matmul_rmsnorm(fh_device *dev, const uint16_t *x, const uint16_t *residual,
                         uint16_t *residual_out, const uint16_t *norm_weight, float eps, int64_t m,
                         int64_t k, const uint32_t *wq, const uint16_t *scales,
                         const uint16_t *biases, int64_t n, int64_t group, void *y, int y_dtype);
int fh_q4_gate_up_silu(fh_device *dev, const uint16_t *x, const uint16_t *residual,
                       uint16_t *residual_out, const uint16_t *norm_weight, float eps, int64_t m,
                       int64_t k, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                       int64_t n, int64_t group, uint16_t *act);

/* A load-time copy of a q4 weight's scales and biases, interleaved per group
 * pair: sb (u32 [n, k / 64], 16-byte aligned) gets at dword 2p of row r the
 * scales of groups 2p and 2p + 1 (group 2p in the low half) and at dword
 * 2p + 1 their biases. fh_q4_weight.sb takes it; the 2..8-row decode GEMV of
 * fh_llama_forward then reads a chunk's scales and biases with one load
 * instead of two (the same values: results are unchanged). No counterpart in
 * the reference (its Linear reads the separate scales / biases tensors,
 * src/nn/linear.rs:22-35); a data layout of this library's decoder.
 * group = 64, k a multiple of 128. */
int fh_q4_interleave(fh_device *dev, const uint16_t *scales, const uint16_t *biases, int64_t n,
                     int64_t k, int64_t group, uint32_t *sb);

/* A load-time copy of a q4 weight's packed words in the batched decode
 * GEMV's task order: wt (u32, n * k / 8 words, 16-byte aligned) holds, for
 * task tile t, group pair p and column c < 16, the 16 words of pair p of
 * weight row r(t, c) at words ((t * k / 128 + p) * 16 + c) * 16. r(t, c) =
 * 16 t + c, or with silu_pairs (a [gate; up] weight of n = 2f rows) the gate
 * row 8 t + c for c < 8 and the up row f + 8 t + c - 8. fh_q4_weight.wt
 * takes it (silu_pairs = 1 for the gate/up weight, 0 for the others); the
 * 2..8-row GEMVs of fh_llama_forward then read one contiguous KiB per
 * wavefront load instead of 16 rows x 64 bytes (the same values: results
 * are unchanged). No counterpart in the reference (its Linear reads the
 * packed tensor as stored, src/nn/linear.rs:22-35); a data layout of this
 * library's decoder. group = 64; n a multiple of 16 (32 with silu_pairs),
 * k of 128; wt must not overlap wq. */
int fh_q4_tile(fh_device *dev, const uint32_t *wq, int64_t n, int64_t k, int64_t group, int silu_pairs,
               uint32_t *wt);

/* LlamaMlp's act_fn(gate) * up (src/models/llama/mlp.rs:49-58, Silu at
 * src/nn/activation.rs:19-28): gate_up row = [gate (f) | up (f)],
 * out = RNE(RNE(g / (1 + exp(-g))) * u), out: [rows, f]. */
int fh_silu_mul(fh_device *dev, const uint16_t *gate_up, int64_t rows, int64_t f, uint16_t *out);

/* Greedy next token (src/generate/mod.rs:192-204): row argmax of bf16
 * values, ties to the lowest index (src/metal/kernels/reduce.metal:42-78).
 * x: [rows, n]; out: u32 [rows]. */
int fh_argmax(fh_device *dev, const uint16_t *x, int64_t rows, int64_t n, uint32_t *out);

/* For each sequence r < rows: log[r * capacity + position[r] - base] =
 * token[r] when 0 <= position[r] - base < capacity. The greedy loop's token
 * record (token_ids per batch row, src/bench/mod.rs:250-300), kept on the
 * device so a captured step can be replayed without reading back each
 * token. token, position: u32 [rows]; log: u32 [rows, capacity]. */
int fh_append_token(fh_device *dev, const uint32_t *token, int64_t rows, uint32_t *log,
                    const uint32_t *position, int64_t base, int64_t capacity);

/* positions[i] += by for i < n, on the device's stream. */
int fh_advance_positions(fh_device *dev, uint32_t *positions, int64_t n, int64_t by);

/* fh_append_token(dev, token, rows, log, position, base, capacity), then
 * fh_advance_positions(dev, position, rows, by), as one launch: the decode
 * step's token record and position bump (src/generate/mod.rs:45-90), one
 * dispatch fewer per replayed step. With capacity 0 nothing is logged and
 * log may be null. token and position may share memory. */
int fh_append_token_advance(fh_device *dev, const uint32_t *token, int64_t rows, uint32_t *log,
                            uint32_t *position, int64_t base, int64_t capacity, int64_t by);

/* ======================================================================
 * The decoder forward issued from native code: the layer loop that a
 * caller would otherwise drive op by op, so an eager prefill is not bound
 * by per-call host overhead.
 * ====================================================================== */

/* A q4 weight: n rows of k columns (group 64), as fh_q4_matmul takes it.
 * sb: null, or fh_q4_interleave's copy of scales / biases, which the
 * batched decode GEMVs (2..8 rows) then read instead. wt: null, or (with sb)
 * fh_q4_tile's copy of the words, built with silu_pairs = 1 for gate_up and
 * 0 for the other weights, which the batched decode GEMVs read instead of
 * wq. */
typedef struct fh_q4_weight {
    const uint32_t *wq;
    const uint16_t *scales;
    const uint16_t *biases;
    int64_t n;
    int64_t k;
    const uint32_t *sb;
    const uint32_t *wt;
} fh_q4_weight;

/* One decoder layer (LlamaDecoderLayer, src/models/llama/model.rs:47, :254-280):
 * qkv = [Wq; Wk; Wv] and gate_up = [Wgate; Wup] rows; bf16 norm weights
 * [hidden]; caches: batch x n_kv regions of max_len * head_dim (K grouped
 * as for fh_rope_kv). */
typedef struct fh_llama_layer {
    fh_q4_weight qkv, o, gate_up, down;
    const uint16_t *input_norm;
    const uint16_t *post_norm;
    uint16_t *k_cache;
    uint16_t *v_cache;
} fh_llama_layer;

/* A Llama model on one device and the buffers of one forward. rows =
 * batch * max_tokens: h, h2, x, o [rows, hidden]; qkv [rows, (n_heads +
 * 2 n_kv) * head_dim]; q, attn [rows, n_heads * head_dim]; gate_up
 * [rows, 2 ffn]; act [rows, ffn]; logits [batch, vocab]. cos_tab/sin_tab:
 * [max_len, head_dim]. Workspaces: at least fh_attention_workspace(
 * max_tokens, ...) and fh_decode_attention_workspace(batch, ...) bytes.
 * `layers` is a host array of n_layers entries. */
typedef struct fh_llama_model {
    int64_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab;
    int64_t batch, max_len, max_tokens;
    float rms_norm_eps;
    float scale;
    const fh_llama_layer *layers;
    fh_q4_weight embed;
    const uint16_t *final_norm;
    const uint16_t *cos_tab;
    const uint16_t *sin_tab;
    uint16_t *h, *h2, *x, *qkv, *q, *attn, *o, *gate_up, *act, *logits;
    void *attn_workspace;
    uint64_t attn_workspace_bytes;
    void *decode_workspace;
    uint64_t decode_workspace_bytes;
} fh_llama_model;

/* LlamaModel::forward (src/models/llama/model.rs:92-121) and the greedy
 * pick of Decoder::step (src/generate/mod.rs:150-204): ids and positions
 * (device u32 [batch, seq_tokens], sequence-major) run through the embedding,
 * every layer and the tied LM head of each sequence's last row; next (device
 * u32 [batch]) gets each sequence's argmax. The same op sequence as calling
 * the ops above one by one: up to 8 rows the RMSNorms, residual adds and SiLU
 * go inside the GEMVs and one new token's RoPE and cache write inside
 * fh_decode_attention; above 8 rows the unfused ops run, and prefill
 * attention runs one sequence at a time. Above 8 rows a GEMM that splits K
 * passes its f32 partials (the device's partial area) to the RoPE, RMSNorm
 * or SiLU after it, which adds them in the order of the GEMM's own reduce:
 * the results are bit-identical to the op sequence, but the buffers o,
 * gate_up and (seq_tokens > 1) qkv are then not written. The weight shapes
 * are checked against the config before any work is issued; every op checks
 * its own ranges as it runs. May be captured (fh_capture_begin).
 * 1 <= seq_tokens <= max_tokens. */
int fh_llama_forward(fh_device *dev, const fh_llama_model *model, int64_t seq_tokens,
                     const uint32_t *ids, const uint32_t *positions, uint32_t *next);

#ifdef __cplusplus
}
#endif

#endif
