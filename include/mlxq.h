/*
 * mlxq.h -- C ABI of libmlxq, the MI355X (gfx950) implementation of
 * mlx-bun's quantized-inference hot path.
 *
 * The TypeScript decode loop binds these symbols with bun:ffi dlopen the same
 * way it binds libmlxc today (src/mlx/ffi.ts:26-41): plain pointers, sizes
 * and ints, an int status per call (0 = OK), and a last-error string read on
 * failure (the reference routes mlx-c errors through a recording handler and
 * throws a JS Error carrying the message, src/mlx/ffi.ts:277-294, :338-348).
 *
 * Conventions
 *  - Device buffers are raw device pointers (u64 in bun:ffi).  The caller
 *    owns every buffer (mlxq_malloc / mlxq_free); array handles and their
 *    dispose()/FinalizationRegistry lifetime stay on the TypeScript side
 *    (src/mlx/array.ts:45-57).
 *  - Every compute call is asynchronous on `stream` (a hipStream_t; NULL is
 *    the library's default stream).  mlxq_synchronize is the only call that
 *    blocks on device work (apart from the explicit host<->device copies).
 *  - dtype codes are mlx_dtype enum values (src/mlx/ffi.ts:297-300), so the
 *    TS layer passes MlxArray.dtype through unchanged.
 *  - Quantized tensors use MLX's affine layout: codes packed little-endian
 *    into uint32 (element j at bits [j*bits, (j+1)*bits)), groups of
 *    `group_size` consecutive elements along the last axis, one T scale and
 *    one T bias per group.
 *  - Errors: a non-zero status leaves a message retrievable with
 *    mlxq_last_error() (thread-local, valid until the next failing call on
 *    the same thread).
 */
#ifndef MLXQ_H
#define MLXQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLXQ_ABI_VERSION 1

/* dtype codes (mlx_dtype) */
enum {
  MLXQ_UINT32 = 3,
  MLXQ_INT32 = 7,
  MLXQ_FLOAT16 = 9,
  MLXQ_FLOAT32 = 10,
  MLXQ_BFLOAT16 = 12
};

/* status codes */
enum {
  MLXQ_OK = 0,
  MLXQ_ERR_ARGUMENT = 1,    /* shape / dtype / size rejected */
  MLXQ_ERR_UNSUPPORTED = 2, /* valid request this build does not implement */
  MLXQ_ERR_HIP = 3,         /* HIP runtime error */
  MLXQ_ERR_STATE = 4        /* library not initialised */
};

/* SDPA mask modes: the reference's Mask.mode (src/model/gemma4-base.ts:21-32)
 * restricted to what the quantized path dispatches: "" (attend everything),
 * "causal" (bottom-right aligned, createCausalMask :1595-1615).  An "array"
 * mask with causalEquivalent=true is passed as MLXQ_MASK_CAUSAL; a sliding
 * window mask as MLXQ_MASK_CAUSAL with window > 0. */
enum { MLXQ_MASK_NONE = 0, MLXQ_MASK_CAUSAL = 1 };

/* ---------------------------------------------------------------- runtime */

/* Selects `device`, creates the default stream.  Replaces the implicit
 * libmlxc load + default GPU stream (src/mlx/array.ts:9-10). */
int mlxq_init(int device);
int mlxq_abi_version(void);
const char* mlxq_last_error(void);
int mlxq_device_count(int* count);
/* Name of the device code object arch this build targets ("gfx950"). */
const char* mlxq_target_arch(void);

int mlxq_malloc(void** ptr, uint64_t nbytes);
int mlxq_free(void* ptr);
int mlxq_memcpy_htod(void* dst, const void* src, uint64_t nbytes, void* stream);
int mlxq_memcpy_dtoh(void* dst, const void* src, uint64_t nbytes, void* stream);
int mlxq_memcpy_dtod(void* dst, const void* src, uint64_t nbytes, void* stream);
/* Zero-fill by kernel (safe inside a captured HIP graph). */
int mlxq_fill_zero(void* dst, uint64_t nbytes, void* stream);
/* Strided 2-D copy: `rows` rows of `row_bytes`, pitches in bytes.  Used by
 * the host cache classes for the ring reorder / trim steps. */
int mlxq_copy_2d(void* dst, uint64_t dst_pitch, const void* src, uint64_t src_pitch,
                 uint64_t row_bytes, uint64_t rows, void* stream);
int mlxq_stream_create(void** stream);
int mlxq_stream_destroy(void* stream);
int mlxq_synchronize(void* stream);
int mlxq_event_create(void** event);
int mlxq_event_destroy(void* event);
int mlxq_event_record(void* event, void* stream);
int mlxq_event_elapsed_ms(void* start, void* stop, float* ms);
/* HIP graph capture of the calls issued on `stream` between begin and end
 * (the analogue of the reference's compiled decode closures,
 * src/model/compiled-decode.ts, for launch-bound loops).
 * Workspace: decode split-K partials, the qmm split-K partials and the
 * sorted gather's work list live in one library-owned block per device.  A
 * call that needs the block to grow fails (MLXQ_ERR_STATE) while its stream
 * is being captured: run the call once, or reserve, before capture.  While
 * any exec made by mlxq_graph_end exists, a later eager call that grows the
 * block leaves the old one allocated (a replay keeps reading and writing
 * it); replaced blocks are freed when the last such exec is destroyed.
 * Graphs captured by other means are not tracked: reserve enough before
 * capturing them.  Replays and calls that overlap on one device race on the
 * block (serialise them on one stream). */
int mlxq_graph_begin(void* stream);
int mlxq_graph_end(void* stream, void** graph_exec);
int mlxq_graph_launch(void* graph_exec, void* stream);
int mlxq_graph_destroy(void* graph_exec);
/* Grow the current device's workspace to at least `nbytes` now (not while
 * `stream` is being captured); its current size. */
int mlxq_workspace_reserve(uint64_t nbytes, void* stream);
int mlxq_workspace_size(uint64_t* nbytes);

/* -------------------------------------------------------------- quantize */

/* mx.quantize(w, group_size, bits, "affine") -- replaces mlx_quantize as
 * bound by ops.quantize (src/mlx/ops.ts:615-641, src/mlx/ffi.ts:100).
 * w: [rows, dim] T; packed: [rows, dim*bits/32] u32; scales/biases:
 * [rows, dim/group_size] T.  bits in {2,4,8}, group_size in {32,64,128},
 * T in {float16, bfloat16, float32}. */
int mlxq_quantize(const void* w, int dtype, int64_t rows, int64_t dim, int group_size, int bits,
                  uint32_t* packed, void* scales, void* biases, void* stream);

/* Quantize `rows_per_head` new rows of each of `heads` [B*H] heads straight
 * into a KV cache laid out [heads, capacity, .] at slot
 * (write_pos + r) mod capacity.  One launch replaces the quantize + six
 * slice_update calls of QuantizedKVCache.updateAndFetchQuantized
 * (src/model/gemma4-base.ts:452-507) and of RotatingQuantizedKVCache's
 * in-place ring write (:1026-1094). */
int mlxq_kv_append(const void* x, int dtype, int64_t heads, int64_t rows_per_head, int64_t dim,
                   int group_size, int bits, uint32_t* packed, void* scales, void* biases,
                   int64_t capacity, int64_t write_pos, void* stream);

/* mx.dequantize -- replaces mlx_dequantize (src/mlx/ops.ts:212-225,
 * src/mlx/ffi.ts:163).  out: [rows, dim] T = T(scale*code + bias). */
int mlxq_dequantize(const uint32_t* packed, const void* scales, const void* biases, int dtype,
                    int64_t rows, int64_t dim, int group_size, int bits, void* out, void* stream);

/* QuantizedEmbedding.encode -- replaces its three takeAxis gathers of the
 * packed table, scales and biases plus ops.dequantize
 * (src/model/gemma4-base.ts:185-194; src/mlx/ops.ts:227-231, :212-225) with
 * one pass.  ids: [n] uint32 token ids on the device (int32 ids of the same
 * value are the same bits); table: packed [vocab, dim*bits/32] u32,
 * scales/biases [vocab, dim/group_size] T.  out: [n, dim] T, row i =
 * T(scale*code + bias) of table row ids[i]; an id outside [0, vocab) gives a
 * zero row.  The tied head (QuantizedEmbedding.asLinear, :197-200) is
 * mlxq_quantized_matmul on the same table. */
int mlxq_embedding_gather(const uint32_t* ids, int64_t n, const uint32_t* packed, const void* scales,
                          const void* biases, int dtype, int64_t vocab, int64_t dim, int group_size, int bits,
                          void* out, void* stream);

/* --------------------------------------------------------- quantized mm */

/* mx.quantized_matmul -- replaces mlx_quantized_matmul as bound by
 * ops.quantizedMatmul / quantizedMatmulQT (src/mlx/ops.ts:171-184,
 * :760-775; src/mlx/ffi.ts:164).
 * x: [batch, M, K] T.  transpose=1: w [w_batch, N, K*bits/32], scales/biases
 * [w_batch, N, K/group_size] (QuantizedLinear.forward,
 * src/model/gemma4-base.ts:120-158).  transpose=0: w [w_batch, K,
 * N*bits/32], scales/biases [w_batch, K, N/group_size].  x batch b uses w
 * batch b / (batch / w_batch) (MLX broadcasting of a size-1 batch axis, as
 * quantizedSdpaUnfused's expand_dims does, :1291-1303).
 * y: [batch, M, N] T, fp32 accumulation. */
int mlxq_quantized_matmul(const void* x, int dtype, int64_t batch, int64_t M, int64_t K,
                          const uint32_t* w, const void* scales, const void* biases, int64_t w_batch,
                          int64_t N, int group_size, int bits, int transpose, void* y, void* stream);

/* mx.gather_qmm with rhs_indices and no lhs_indices -- replaces
 * mlx_gather_qmm as bound by ops.gatherQmm (src/mlx/ops.ts:186-204,
 * src/mlx/ffi.ts:167) for QuantizedSwitchLinear.forward (MoE experts,
 * src/model/gemma4-base.ts:1615-1645).
 * Output batch element i < batch computes y[i] = x[x_map[i]] @ W[e]^T with
 * e = rhs_indices[i] (transpose=1; transpose=0: x[..] @ W[e]).
 * x: [x_batch, M, K] T.  w: [n_experts, N, K*bits/32] (transpose=1) or
 * [n_experts, K, N*bits/32], scales/biases per expert as in
 * mlxq_quantized_matmul.  x_map: [batch] int32 on the device, the x batch
 * element of each output element -- the broadcast of x's batch dims against
 * rhs_indices' shape, computed by the caller (SwitchGLU's
 * expand_dims(x, (-2, -3)) against indices [B, L, k] gives x_map[i] = i / k,
 * src/model/gemma4.ts:434-438); NULL means x_map[i] = i (x_batch == batch).
 * rhs_indices: [batch] uint32 on the device.  An index outside [0, x_batch)
 * or [0, n_experts) yields a zero output row (MLX leaves it undefined).
 * sorted_indices (a scheduling hint in MLX) is mlxq_gather_qmm_sorted
 * below; results do not depend on it.  y: [batch, M, N] T, fp32
 * accumulation. */
int mlxq_gather_qmm(const void* x, int dtype, int64_t x_batch, int64_t batch, int64_t M, int64_t K,
                    const int32_t* x_map, const uint32_t* rhs_indices, const uint32_t* w, const void* scales,
                    const void* biases, int64_t n_experts, int64_t N, int group_size, int bits, int transpose,
                    void* y, void* stream);

/* gatherQmm(x, w, scales, biases, rhsIndices, spec, sortedIndices = true)
 * -- the call of src/mlx/ops.ts:186-204 with sorted_indices set, as
 * SwitchGLU makes it once a batch has 64 or more (row, expert) pairs: rows
 * gathered in expert order first (_gather_sort, src/model/gemma4.ts:441-464),
 * so x is [rows, 1, K] with row i using expert rhs_indices[i] (transpose=1,
 * no x map).  Rows with equal consecutive indices run as one GEMM block, so
 * an expert's weights stream once per block rather than once per row.
 * Results equal mlxq_gather_qmm's over the same rows (up to fp32 summation
 * order) whatever the index order; unsorted indices are only slower.  Index
 * range and zero rows as mlxq_gather_qmm.  Uses the library's workspace
 * (1 + 3 rows int32) on `stream`.  y: [rows, 1, N] T. */
int mlxq_gather_qmm_sorted(const void* x, int dtype, int64_t rows, int64_t K, const uint32_t* rhs_indices,
                           const uint32_t* w, const void* scales, const void* biases, int64_t n_experts,
                           int64_t N, int group_size, int bits, void* y, void* stream);

/* ------------------------------------------------------------------ sdpa */

/* quantizedSdpa(q, kq, vq, scale, mask, groupSize, bits) -- replaces the
 * dispatch of src/model/gemma4-base.ts:1560-1578 (unfused decode :1273-1340,
 * N-tiled prefill :1356-1521, Metal flash-decoding kernel
 * src/model/fused-decode-kernel.ts:274-312) with one entry point.
 * q: [B, Hq, Lq, D] T; out: [B, Hq, Lq, D] T; GQA: q head h reads kv head
 * h / (Hq/Hkv).  K/V triples are cache buffers [B, Hkv, kv_capacity, .]
 * (the reference's fetch views read in place, no contiguous copy).
 * Row b attends `valid` logical positions j = 0..valid-1:
 *   valid = valid_len ? min(valid_len[b], kv_capacity) : n_kv
 *   slot(j) = ring_offset ? (ring_offset[b] - valid + j) mod kv_capacity : j
 * valid_len / ring_offset are device int32 [B] arrays or NULL (ring_offset
 * is the ring write index, the rotating caches' ringIdx).  Query i is at
 * logical position valid - Lq + i; MLXQ_MASK_CAUSAL allows j <= pos and,
 * with window > 0, pos < j + window.
 * Queries are scaled as the reference does (T(q * T(scale)), skipped when
 * scale == 1); scores, softmax and both contractions accumulate in fp32. */
int mlxq_quantized_sdpa(const void* q, int dtype, int B, int Hq, int Hkv, int Lq, int D,
                        const uint32_t* k_packed, const void* k_scales, const void* k_biases,
                        const uint32_t* v_packed, const void* v_scales, const void* v_biases,
                        int64_t kv_capacity, int64_t n_kv, const int32_t* valid_len,
                        const int32_t* ring_offset, int mask_mode, int window, float scale,
                        int group_size, int bits, void* out, void* stream);

/* quantizedSdpa under an "array" mask that is neither the causal matrix nor a
 * causal sliding window -- replaces the where(mask, scores, FINFO_MIN) of the
 * unfused path, src/model/gemma4-base.ts:1320-1327, where the dispatch sends
 * every such mask (:1543-1545, :1577).  mask: device uint8, nonzero = attend:
 * query i of row b attends logical key j (0 <= j < valid, slot(j) as above)
 * iff mask[b * mask_batch_stride + i * mask_row_stride + j] != 0; a batch
 * stride of 0 shares one [Lq, .] mask across the batch, and mask_row_stride
 * must be >= n_kv (>= kv_capacity with valid_len).  A query with no attended
 * key averages V over its valid keys, as the reference's softmax over
 * all-FINFO_MIN scores does.  Other arguments and rounding as
 * mlxq_quantized_sdpa (no mask_mode / window); runs the generic VALU kernel,
 * no device allocation. */
int mlxq_quantized_sdpa_array_mask(const void* q, int dtype, int B, int Hq, int Hkv, int Lq, int D,
                                   const uint32_t* k_packed, const void* k_scales, const void* k_biases,
                                   const uint32_t* v_packed, const void* v_scales, const void* v_biases,
                                   int64_t kv_capacity, int64_t n_kv, const int32_t* valid_len,
                                   const int32_t* ring_offset, const uint8_t* mask, int64_t mask_batch_stride,
                                   int64_t mask_row_stride, float scale, int group_size, int bits, void* out,
                                   void* stream);

/* mlxq_quantized_sdpa without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory -- code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Same arguments, kernels and results as mlxq_quantized_sdpa;
 * its scratch (the split-K partials of decode and of the split wide
 * prefill) is a fixed block of MLXQ_NOALLOC_SCRATCH_BYTES per device, held
 * from mlxq_init until the process ends, instead of the growable workspace.
 * A request whose partials need more fails with MLXQ_ERR_UNSUPPORTED before
 * any launch (a 32k-context decode needs about 0.5 MB; the 32-row, 4096-slot
 * D 256 ring decode 2.7 MB; a split D 512 prefill chunk of 512 queries
 * 33 MB).  Every call on a device shares that device's block and nothing in
 * it needs to start at zero (partials are written before they are read);
 * calls that overlap on one device (two streams, or this call beside a
 * replay of a graph that captured it) race on it. */
#define MLXQ_NOALLOC_SCRATCH_BYTES (8u << 20)
int mlxq_quantized_sdpa_noalloc(const void* q, int dtype, int B, int Hq, int Hkv, int Lq, int D,
                                const uint32_t* k_packed, const void* k_scales, const void* k_biases,
                                const uint32_t* v_packed, const void* v_scales, const void* v_biases,
                                int64_t kv_capacity, int64_t n_kv, const int32_t* valid_len,
                                const int32_t* ring_offset, int mask_mode, int window, float scale,
                                int group_size, int bits, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLXQ_H */
