/*
 * pocketlm_hip.h - C ABI of libpocketlm_hip.so, the MI355X (gfx950) backend
 * for PocketLM's quantized-decode hot path.
 *
 * Every entry point keeps the name, argument order and return codes of the
 * reference export it replaces (cited as file:line under
 * src/pcketlm/native/ of the reference tree), so the reference's ctypes
 * argtypes bind unchanged.  What differs is where the data lives:
 *
 *   - Tensor arguments are DEVICE pointers (HBM, e.g. torch CUDA tensors).
 *   - The per-expert address tables of the MoE entry points
 *     (const uint64_t* / const T** arrays) are HOST arrays whose entries
 *     are device addresses, exactly as the reference passes host arrays of
 *     host addresses.  Their contents are captured at call time.
 *   - Calls are asynchronous on the stream set by pocketlm_set_stream()
 *     for the calling thread (default: the null stream).  Outputs are
 *     valid once that stream reaches the work.
 *   - Failures of the HIP runtime return -(1000 + hipError_t) from every
 *     int-returning entry point; the reference's own codes are unchanged.
 *   - A scale grid with fewer columns than ceil(cols/128) is rejected with
 *     the entry point's bad-dimension code instead of being read past its
 *     end (the reference leaves that check to its Python wrapper).
 *
 * Library-owned device scratch (MLP activations, split results) comes from
 * a per-(device, stream) arena that grows on demand and is kept for reuse;
 * calls on one stream are ordered, calls on different streams each get
 * their own arena.
 */
#ifndef POCKETLM_HIP_H_
#define POCKETLM_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ runtime */

/* New (no reference counterpart): set the HIP stream used by this thread's
 * subsequent calls.  NULL selects the null stream.  Returns 0. */
int pocketlm_set_stream(void* hip_stream);

/* New: human-readable text of the last failure on this thread ("" if none). */
const char* pocketlm_last_error(void);

/* New, no counterpart in the reference (whose CPU kernels need no device
 * scratch).  Each host thread keeps device scratch per (device, stream) it
 * calls on: an arena at its high-water size (growth at least doubles it and
 * keeps the block it replaced, for work still queued or graphs captured
 * earlier) and 64 stream words.  pocketlm_scratch_bytes: the calling
 * thread's bytes held.  pocketlm_release_scratch: waits for the calling
 * thread's streams and frees its scratch; graphs it captured must not be
 * replayed afterwards.  Returns 0, or a negative code with nothing freed when
 * a stream wait fails. */
int64_t pocketlm_scratch_bytes(void);
int pocketlm_release_scratch(void);

/* New: 1 when a HIP device of architecture gfx950 is visible, else 0. */
int pocketlm_device_available(void);

/* Feature probes the reference loaders require to return 1 before they
 * accept a library (src/pcketlm/native/__init__.py:291-293, 462-466,
 * 160-195).  Here they report pocketlm_device_available(). */
int fp8_dequant_cpu_has_avx2_f16c(void);      /* fp8_dequant.cpp:67 */
int fp8_linear_avx512_cpu_has_avx512(void);   /* fp8_linear_avx512.cpp:63 */
int q4_cpu_has_avx2_f16c(void);               /* q4_dequant.cpp:116 */
int ds_cpu_has_avx2(void);                    /* ds_forward.cpp:182 */

/* ------------------------------------------------------- FP8 block dequant */
/* W e4m3fn bytes [rows, cols] row-major, scale_inv fp32
 * [ceil(rows/128), scale_cols]; out[r,c] = cvt(dec(W[r,c]) * scale).
 * NaN bytes decode to NaN (fp32 bits 0x7FF00000 / 0xFFF00000).
 * Codes: -1 null pointer, -2 rows/cols/scale_cols <= 0,
 *        -3 scale_cols != ceil(cols/128). */

/* fp8_dequant.cpp:119-164: fp16 out, round-to-nearest-even, NaN -> 0x7F80/0xFF80 */
int fp8_e4m3_dequant_to_fp16(const uint8_t* fp8_weight, const float* scale_inv,
                             uint16_t* out_fp16, int64_t rows, int64_t cols,
                             int64_t scale_cols);

/* fp8_dequant.cpp:166-204: bf16 out via bits + 0x7FFF + lsb, NaN -> 0xFFFF */
int fp8_e4m3_dequant_to_bf16(const uint8_t* fp8_weight, const float* scale_inv,
                             uint16_t* out_bf16, int64_t rows, int64_t cols,
                             int64_t scale_cols);

/* New export for the fp32 branch of dequantize_fp8_block_scaled
 * (src/pcketlm/core/runtime/fp8_source.py:852-858), which the reference
 * computes with torch: out = dec(W) * scale in fp32. */
int fp8_e4m3_dequant_to_f32(const uint8_t* fp8_weight, const float* scale_inv,
                            float* out_f32, int64_t rows, int64_t cols,
                            int64_t scale_cols);

/* ------------------------------------------------- FP8 block-scaled GEMV */
/* hidden fp32 [batch, in_cols]; out fp32 [batch, out_rows];
 * out[b,n] = sum_kb scale[n/128,kb] * sum_{k in kb} hidden[b,k]*dec(W[n,k]),
 * NaN weight bytes contribute 0.  Each weight byte is read from HBM once per
 * call for all batch rows.  Codes: -1 null pointer, -2 bad dims. */

/* fp8_linear.cpp:50-117 */
int fp8_e4m3_block_linear_f32(const uint8_t* fp8_weight, const float* scale_inv,
                              const float* hidden, float* out, int64_t batch,
                              int64_t out_rows, int64_t in_cols, int64_t scale_cols);

/* fp8_linear.cpp:119-210: two same-shape weights sharing hidden */
int fp8_e4m3_block_dual_linear_f32(const uint8_t* fp8_weight_a, const float* scale_inv_a,
                                   const uint8_t* fp8_weight_b, const float* scale_inv_b,
                                   const float* hidden, float* out_a, float* out_b,
                                   int64_t batch, int64_t out_rows, int64_t in_cols,
                                   int64_t scale_cols);

/* fp8_linear.cpp:212-362: out = down . (silu(gate . x) * (up . x)),
 * silu(g) = g / (1 + exp(-g)).  gate/up [I, H], down [H, I].
 * Code -3 when the activation scratch cannot be allocated. */
int fp8_e4m3_block_mlp_f32(const uint8_t* gate_weight, const float* gate_scale_inv,
                           const uint8_t* up_weight, const float* up_scale_inv,
                           const uint8_t* down_weight, const float* down_scale_inv,
                           const float* hidden, float* out, int64_t batch,
                           int64_t intermediate_rows, int64_t hidden_cols,
                           int64_t gate_scale_cols, int64_t down_scale_cols);

/* fp8_linear_avx512.cpp:157-250: same kernel as fp8_e4m3_block_mlp_f32 */
int fp8_e4m3_block_mlp_avx512_f32(const uint8_t* gate_weight, const float* gate_scale_inv,
                                  const uint8_t* up_weight, const float* up_scale_inv,
                                  const uint8_t* down_weight, const float* down_scale_inv,
                                  const float* hidden, float* out, int64_t batch,
                                  int64_t intermediate_rows, int64_t hidden_cols,
                                  int64_t gate_scale_cols, int64_t down_scale_cols);

/* fp8_linear.cpp:364-473: E experts, unweighted; out [E, batch, hidden].
 * An expert whose gate/up pointers are null gets a zero activation; one
 * whose down pointers are null leaves its output rows untouched. */
int fp8_e4m3_block_mlp_many_f32(const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
                                const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
                                const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs,
                                const float* hidden, float* out, int64_t expert_count,
                                int64_t batch, int64_t intermediate_rows, int64_t hidden_cols,
                                int64_t gate_scale_cols, int64_t down_scale_cols);

/* fp8_linear.cpp:475-589: out[b,h] = sum_e route[e] * expert_e(x_b)[h];
 * route_weights fp32 [E] (device).  Each expert matrix is read once. */
int fp8_e4m3_block_mlp_many_weighted_f32(
    const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
    const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
    const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs, const float* hidden,
    const float* route_weights, float* out, int64_t expert_count, int64_t batch,
    int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
    int64_t down_scale_cols);

/* No single reference counterpart: the pair of calls run_fp8_moe makes at
 * one token (fp8_source.py:1643-1646 -> fp8_linear.cpp:475-589 for the
 * routed experts, fp8_source.py:1849-1859 -> fp8_linear.cpp:212-362 for the
 * shared expert) in two launches instead of four.  The six tables hold
 * expert_count routed experts followed by the shared expert (same shapes);
 * out gets the routed sum as fp8_e4m3_block_mlp_many_weighted_f32 computes
 * it, out_shared the shared expert's MLP as fp8_e4m3_block_mlp_f32 computes
 * it (the same per-row arithmetic, so the same values).  Returns -2 for more
 * than 63 routed experts. */
int fp8_e4m3_block_mlp_many_weighted_shared_f32(
    const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
    const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
    const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs, const float* hidden,
    const float* route_weights, float* out, float* out_shared, int64_t expert_count, int64_t batch,
    int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
    int64_t down_scale_cols);

/* fp8_linear_avx512.cpp:252-371: same kernel as the weighted entry point */
int fp8_e4m3_block_mlp_many_weighted_avx512_f32(
    const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
    const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
    const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs, const float* hidden,
    const float* route_weights, float* out, int64_t expert_count, int64_t batch,
    int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
    int64_t down_scale_cols);

/* fp8_linear.cpp:591-831: route_weights fp32 [E, batch] (device); (e, b)
 * pairs with weight exactly 0 contribute nothing.  Each expert matrix is
 * read once per call for all its active rows. */
int fp8_e4m3_block_mlp_many_row_weighted_f32(
    const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
    const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
    const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs, const float* hidden,
    const float* route_weights, float* out, int64_t expert_count, int64_t batch,
    int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
    int64_t down_scale_cols);

/* fp8_linear.cpp:833-980: sparse (item, row, weight) pairs (device arrays,
 * int64 / int64 / fp32, length pair_count).  out is zeroed first; -4 when
 * a pair index is out of range (checked before any kernel runs; this reads
 * the two index arrays back to the host and so waits for the stream). */
int fp8_e4m3_block_mlp_many_pair_weighted_f32(
    const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
    const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
    const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs, const float* hidden,
    const int64_t* pair_item_indices, const int64_t* pair_row_indices,
    const float* pair_weights, float* out, int64_t expert_count, int64_t pair_count,
    int64_t batch, int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
    int64_t down_scale_cols);

/* No single reference counterpart: several FP8 linears sharing one hidden
 * (fp8_linear.cpp:50-117 each), such as the q_a and kv_a projections that
 * the DeepSeek attention computes from the same hidden state
 * (fp8_source.py:1943-1945 and 1967-1969), in one launch.  count
 * (1..8) weights of out_rows[i] x in_cols with their scale grids; output i
 * is fp32 [batch, out_rows[i]] at out_ptrs[i].  The three address arrays are
 * host arrays of device addresses, as in the MoE entry points.  Each output
 * has the values of fp8_e4m3_block_linear_f32 on that weight.  Codes as
 * fp8_e4m3_block_linear_f32 (-2 also for count outside 1..8). */
int fp8_e4m3_block_linear_many_f32(const uint64_t* weight_ptrs, const uint64_t* scale_ptrs,
                                   const float* hidden, const uint64_t* out_ptrs,
                                   const int64_t* out_rows, int64_t count, int64_t batch,
                                   int64_t in_cols, int64_t scale_cols);

/* bf16-activation twins.  The reference wrappers cast the activations to
 * fp32 before these calls (native/__init__.py:3451 linear, 3500 dual, 3568
 * MLP, 3760 weighted, 3834 row-weighted, 3910 pair-weighted; the routed +
 * shared call has no reference wrapper); the twins take bf16
 * activations [batch, hidden] as they are and widen them on the device.  The
 * widening is exact, so each twin returns exactly the values of its fp32
 * entry point for the widened activations; they only read half the
 * activation bytes, which matters at 2..8 activation rows.  Arguments and
 * codes are otherwise those of the fp32 entry point. */
int fp8_e4m3_block_linear_bf16x_f32(const uint8_t* fp8_weight, const float* scale_inv,
                                    const uint16_t* hidden_bf16, float* out, int64_t batch,
                                    int64_t out_rows, int64_t in_cols, int64_t scale_cols);
/* FP8 weights in 8-row tiles (no counterpart in the reference, whose FP8
 * linears read the row-major [out_rows, in_cols] e4m3 matrix of
 * fp8_linear.cpp:79-210; for callers that keep a weight resident and run it
 * on batches of 2..8 rows, e.g. a speculative verifier).  The packed weight
 * holds ceil(rows / 8) x ceil(cols / 128) tiles of 1 KB, tile (t, b) at
 * (t * ceil(cols / 128) + b) * 1024, row r of the tile at r * 128 within it,
 * columns b * 128 .. b * 128 + 127; rows and columns past the matrix are
 * zero.  Every wave load of the linear then reads one contiguous KB.
 * fp8_e4m3_tiles8_bytes returns the packed size (-2 for bad dimensions);
 * fp8_e4m3_pack_tiles8 packs a row-major weight into a 16-byte aligned
 * buffer of that size on the current stream.  The tiles8 linears return
 * exactly the values of fp8_e4m3_block_linear_f32 / _bf16x_f32 for the
 * row-major weight (same kernel, schedule and arithmetic; only the weight
 * addresses differ); they need in_cols % 16 == 0 and 16-byte aligned
 * activations (code -2 otherwise). */
int64_t fp8_e4m3_tiles8_bytes(int64_t rows, int64_t cols);
int fp8_e4m3_pack_tiles8(const uint8_t* fp8_weight, uint8_t* out_tiles, int64_t rows, int64_t cols);
int fp8_e4m3_block_linear_tiles8_f32(const uint8_t* fp8_tiles, const float* scale_inv, const float* hidden,
                                     float* out, int64_t batch, int64_t out_rows, int64_t in_cols,
                                     int64_t scale_cols);
int fp8_e4m3_block_linear_tiles8_bf16x_f32(const uint8_t* fp8_tiles, const float* scale_inv,
                                           const uint16_t* hidden_bf16, float* out, int64_t batch,
                                           int64_t out_rows, int64_t in_cols, int64_t scale_cols);
int fp8_e4m3_block_linear_many_bf16x_f32(const uint64_t* weight_ptrs, const uint64_t* scale_ptrs,
                                         const uint16_t* hidden_bf16, const uint64_t* out_ptrs,
                                         const int64_t* out_rows, int64_t count, int64_t batch,
                                         int64_t in_cols, int64_t scale_cols);
int fp8_e4m3_block_dual_linear_bf16x_f32(const uint8_t* weight_a, const float* scale_inv_a,
                                         const uint8_t* weight_b, const float* scale_inv_b,
                                         const uint16_t* hidden_bf16, float* out_a, float* out_b,
                                         int64_t batch, int64_t out_rows, int64_t in_cols,
                                         int64_t scale_cols);
int fp8_e4m3_block_mlp_bf16x_f32(const uint8_t* gate_weight, const float* gate_scale_inv,
                                 const uint8_t* up_weight, const float* up_scale_inv,
                                 const uint8_t* down_weight, const float* down_scale_inv,
                                 const uint16_t* hidden_bf16, float* out, int64_t batch,
                                 int64_t intermediate_rows, int64_t hidden_cols,
                                 int64_t gate_scale_cols, int64_t down_scale_cols);
int fp8_e4m3_block_mlp_many_weighted_bf16x_f32(
    const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
    const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
    const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs, const uint16_t* hidden_bf16,
    const float* route_weights, float* out, int64_t expert_count, int64_t batch,
    int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
    int64_t down_scale_cols);
int fp8_e4m3_block_mlp_many_weighted_shared_bf16x_f32(
    const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
    const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
    const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs, const uint16_t* hidden_bf16,
    const float* route_weights, float* out, float* out_shared, int64_t expert_count, int64_t batch,
    int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
    int64_t down_scale_cols);
int fp8_e4m3_block_mlp_many_row_weighted_bf16x_f32(
    const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
    const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
    const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs, const uint16_t* hidden_bf16,
    const float* route_weights, float* out, int64_t expert_count, int64_t batch,
    int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
    int64_t down_scale_cols);
int fp8_e4m3_block_mlp_many_pair_weighted_bf16x_f32(
    const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
    const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
    const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs, const uint16_t* hidden_bf16,
    const int64_t* pair_item_indices, const int64_t* pair_row_indices,
    const float* pair_weights, float* out, int64_t expert_count, int64_t pair_count,
    int64_t batch, int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
    int64_t down_scale_cols);
/* No counterpart in the reference: the pair-weighted MoE above (fp32 or
 * bf16 activations) without the host read-back of the pair indices, for
 * callers that must not wait on the stream (HIP graph capture, the verifier
 * batch).  Pairs with an index out of range are left out, and their number
 * is written to *bad_pairs (device memory) instead of returning -4; the
 * route weights are summed per (expert, row) in pair order, as above.
 * Codes -1 null, -2 bad dims, -3 workspace. */
int fp8_e4m3_block_mlp_many_pair_weighted_nosync_f32(
    const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
    const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
    const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs, const float* hidden,
    const int64_t* pair_item_indices, const int64_t* pair_row_indices,
    const float* pair_weights, float* out, int* bad_pairs, int64_t expert_count, int64_t pair_count,
    int64_t batch, int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
    int64_t down_scale_cols);
int fp8_e4m3_block_mlp_many_pair_weighted_nosync_bf16x_f32(
    const uint64_t* gate_weight_ptrs, const uint64_t* gate_scale_ptrs,
    const uint64_t* up_weight_ptrs, const uint64_t* up_scale_ptrs,
    const uint64_t* down_weight_ptrs, const uint64_t* down_scale_ptrs, const uint16_t* hidden_bf16,
    const int64_t* pair_item_indices, const int64_t* pair_row_indices,
    const float* pair_weights, float* out, int* bad_pairs, int64_t expert_count, int64_t pair_count,
    int64_t batch, int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
    int64_t down_scale_cols);

/* --------------------------------------------------------------------- Q4 */
/* Per-row symmetric Q4 (src/pcketlm/core/model_import/q4_quantize.py:48-71):
 * two's-complement nibbles flat over the whole tensor, element 2i in the low
 * nibble of byte i; one fp16 scale per channel (row). */

/* q4_dequant.cpp:171-208: out[c*cs+i] = fp16(q * f32(scale[c])), RNE.
 * Returns nothing, as the reference; failures are reported by
 * pocketlm_last_error(). */
void q4_dequant_to_fp16(const uint8_t* packed, const uint16_t* scales, uint16_t* out_fp16,
                        int64_t num_channels, int64_t channel_size);

/* q4_dequant.cpp:210-286: host arrays of device pointers / sizes.  Codes:
 * 1 null array, 2 tensor_count <= 0.  Entries with a null pointer or a
 * non-positive size are skipped. */
int q4_dequant_many_to_fp16(const uint8_t** packed_ptrs, const uint16_t** scale_ptrs,
                            uint16_t** out_ptrs, const int64_t* num_channels,
                            const int64_t* channel_sizes, int64_t tensor_count);

/* q4_dequant.cpp:357-476: one token through S selected Q4 SwiGLU experts,
 * combined with route weights, fp16 out.  hidden fp16 [H], route fp32 [S]
 * and out are device pointers; the six arrays are host arrays of device
 * pointers.  Codes: 1 null/bad size, 3 null expert pointer. */
int q4_moe_selected_forward_u16(const uint16_t* hidden, const uint8_t** gate_packed_ptrs,
                                const uint16_t** gate_scale_ptrs, const uint8_t** up_packed_ptrs,
                                const uint16_t** up_scale_ptrs, const uint8_t** down_packed_ptrs,
                                const uint16_t** down_scale_ptrs, const float* route_weights,
                                uint16_t* out_fp16, int64_t hidden_size,
                                int64_t intermediate_size, int64_t selected_count);

/* New export: one Q4 matrix [rows, cols] times one fp16 vector [cols],
 * fp32 out [rows]: the per-row dot of q4_moe_selected_forward_u16
 * (q4_dequant.cpp:314-355) on its own.  Codes: 1 null, 2 bad dims. */
int q4_gemv_f16_f32(const uint8_t* packed, const uint16_t* scales, const uint16_t* hidden,
                    float* out, int64_t rows, int64_t cols);

/* ------------------------------------------------------------------- row8 */
/* fp16_packed_gemv.cpp:52-77: packed[blk][col][lane] = W[8*blk+lane][col],
 * rows past the end zero.  Codes: 1 null, 2 negative dims. */
int native_pack_u16_rows8(const uint16_t* weight, uint16_t* packed, int64_t rows, int64_t cols);

/* fp16_packed_gemv.cpp:79-116: out[n] = sum_k hidden[k] * W[n,k], fp32
 * fused multiply-add; hidden and W share dtype_code (0 fp16, 1 bf16).
 * Codes: 1 null, 2 negative dims or bad dtype_code. */
int native_packed_gemv_rows8(const uint16_t* hidden, const uint16_t* packed, float* out,
                             int64_t rows, int64_t cols, int dtype_code);

/* New export covering the biased and fused variants of
 * fp16_kv_cache.cpp:117-298: `count` row8 GEMVs that share one hidden
 * vector (q/k/v or gate/up) in a single launch.  Arrays are host arrays of
 * device pointers; bias_ptrs may be NULL or hold NULL entries. */
int native_packed_gemv_rows8_many(const uint16_t* hidden, const uint16_t* const* packed_ptrs,
                                  const uint16_t* const* bias_ptrs, float* const* out_ptrs,
                                  const int64_t* rows, int64_t count, int64_t cols,
                                  int dtype_code);

/* The fp32-activation row8 GEMV of the dense decode's o and down projections
 * (packed_rows8_gemv_float_hidden, fp16_kv_cache.cpp:146-174; a static helper
 * there, called at 1045 and 1515): y[r] = sum_k hidden[k] * W[r, k] as one fma
 * chain per row, no bias.  hidden is fp32 [cols]; packed as
 * native_packed_gemv_rows8 (dtype_code 0 fp16, 1 bf16).  Codes 1 null, 2 bad
 * dimensions or dtype. */
int native_packed_gemv_rows8_f32_hidden(const float* hidden, const uint16_t* packed, float* out, int64_t rows,
                                        int64_t cols, int dtype_code);

/* ------------------------------------------------------ DeepSeek session */
typedef int (*pocketlm_ds_tensor_callback)(int64_t layer_idx, int64_t layer_kind,
                                           int64_t weight_role, const void** out_ptr,
                                           int64_t* out_nbytes);

/* ds_forward.cpp:192-219: opaque session with call counters */
void* ds_session_create(int64_t num_layers, int64_t hidden_dim, int64_t num_experts,
                        int64_t top_k, void* fp8_pack_callback, void* kv_session_handle);
void ds_session_destroy(void* handle);
/* ds_forward.cpp:221-263: codes 1 bad handle/layer, 2 null callback,
 * 10+k / 20+k callback failures */
int ds_session_register_layer(void* handle, int64_t layer_idx, int64_t layer_kind,
                              int64_t weight_role, pocketlm_ds_tensor_callback fp8_ptr_callback,
                              pocketlm_ds_tensor_callback scale_ptr_callback);
/* ds_forward.cpp:265-335: -1 on a null handle / bad index */
int64_t ds_monolithic_call_counter(void* handle);
int64_t ds_callback_invocation_count(void* handle);
int64_t ds_expert_invocation_count(void* handle);
int64_t ds_attention_invocation_count(void* handle);
int64_t ds_fused_attention_invocation_count(void* handle);
int64_t ds_layers_executed_count(void* handle);
int64_t ds_registered_layer_count(void* handle);
int64_t ds_registered_fp8_nbytes(void* handle, int64_t index);
int64_t ds_registered_scale_nbytes(void* handle, int64_t index);

/* ds_forward.cpp:337-367: hidden_out = sum_e route[e] * expert_outputs[e]
 * (device pointers).  Codes 1 null, 2 bad dims.  Bumps monolithic_calls by
 * one and expert_invocations by selected_count. */
int ds_moe_layer_forward_f32(void* handle, const float* expert_outputs, const float* route_weights,
                             int64_t selected_count, int64_t batch, int64_t hidden_dim,
                             float* hidden_out);

/* ds_forward.cpp:784-877: the routed-expert FP8 MoE of one layer through
 * the weighted kernel (route fp32 [selected], device).  Codes 1 null,
 * 2 bad dims, 100+k when the kernel returns k. */
int ds_moe_layer_forward_fp8_f32(void* handle, const uint64_t* gate_weight_ptrs,
                                 const uint64_t* gate_scale_ptrs, const uint64_t* up_weight_ptrs,
                                 const uint64_t* up_scale_ptrs, const uint64_t* down_weight_ptrs,
                                 const uint64_t* down_scale_ptrs, const float* hidden,
                                 const float* route_weights, int64_t selected_count, int64_t batch,
                                 int64_t intermediate_rows, int64_t hidden_dim,
                                 int64_t gate_scale_cols, int64_t down_scale_cols,
                                 float* hidden_out);

/* Callback bridges of the session (ds_forward.cpp:369-512), with the
 * reference's callback types (ds_forward.cpp:20-43).  Each calls its
 * callback once, checks the element count it reports (code 20 when it
 * differs), copies that many fp32 values from the callback's buffer (host
 * or device memory) to the output (host or device memory) on the calling
 * thread's stream and waits for the copy, since the callback's buffer is
 * only guaranteed for the duration of the call.  Codes 1 null handle /
 * pointer / callback, 2 bad dims (bad layer index for the attention
 * bridge), 10+k when the callback returns k or a null buffer, 20 count
 * mismatch, -(1000+err) copy failure.  Counters as in the reference:
 * callback_invocations += 1 per callback; on success monolithic_calls += 1
 * and attention_invocations += 1 (attention), layers_executed += num_layers
 * (decode), num_layers * n_tokens (prefill), num_layers * k (verify). */
typedef int (*pocketlm_ds_attention_callback)(int64_t layer_idx, const float* hidden_in, int64_t batch,
                                              int64_t hidden_dim, const float** out, int64_t* out_count);
typedef int (*pocketlm_ds_decode_callback)(int64_t input_token_id, const float** out, int64_t* out_count);
typedef int (*pocketlm_ds_prefill_callback)(const int64_t* input_token_ids, int64_t n_tokens, const float** out,
                                            int64_t* out_count);
typedef int (*pocketlm_ds_verify_callback)(const int64_t* candidate_token_ids, int64_t k, const float** out,
                                           int64_t* out_count);
int ds_attention_layer_forward_f32(void* handle, int64_t layer_idx, const float* hidden_in, int64_t batch,
                                   int64_t hidden_dim, pocketlm_ds_attention_callback attention_callback,
                                   float* hidden_out);
int ds_forward_decode_f32(void* handle, int64_t input_token_id, pocketlm_ds_decode_callback decode_callback,
                          float* output_logits, int64_t vocab_size);
int ds_forward_prefill_f32(void* handle, const int64_t* input_token_ids, int64_t n_tokens,
                           pocketlm_ds_prefill_callback prefill_callback, float* output_final_logits,
                           int64_t vocab_size);
int ds_forward_verify_f32(void* handle, const int64_t* candidate_token_ids, int64_t k,
                          pocketlm_ds_verify_callback verify_callback, float* output_logits_per_position,
                          int64_t vocab_size);

/* ds_forward.cpp:517-597: MLA attention of one decode token over the latent
 * cache (device fp32): q_nope [H][nope], q_pe [H][rope], kv_cache [L][R],
 * pe_cache [L][rope], wkv_b [H][nope + v][R] -> output_heads [H][v].
 * Codes: 1 null pointer, 2 bad dimensions (also R > 1024 or rope > 256, the
 * device kernel's limits), -3 workspace. */
int ds_mla_attention_flash_forward(const float* q_nope, const float* q_pe, const float* kv_cache,
                                   const float* pe_cache, const float* wkv_b, float* output_heads,
                                   int64_t num_heads, int64_t cache_len, int64_t qk_nope_dim, int64_t qk_rope_dim,
                                   int64_t kv_lora_rank, int64_t v_head_dim, float softmax_scale);

/* ds_forward.cpp:647-782: one-token DeepSeek attention block (device fp32
 * weights and caches): q_a -> RMSNorm -> q_b -> RoPE, kv_a -> RMSNorm /
 * RoPE into row previous_len of next_kv_cache / next_pe_cache (after the
 * previous rows, copied unless the buffers are the same), the MLA above,
 * then o.  Codes: 1 null pointer or handle, 2 bad dimensions, 3 null
 * previous caches with previous_len > 0, 100 + the MLA call's code. */
int ds_attention_block_forward_f32(
    void* handle, const float* hidden_in, const float* q_a_weight, const float* q_b_weight, const float* kv_a_weight,
    const float* kv_b_weight, const float* o_weight, const float* q_norm_weight, const float* kv_norm_weight,
    const float* previous_kv_cache, const float* previous_pe_cache, const float* rope_cos, const float* rope_sin,
    float* next_kv_cache, float* next_pe_cache, float* hidden_out, int64_t hidden_dim, int64_t q_lora_rank,
    int64_t kv_lora_rank, int64_t num_heads, int64_t qk_nope_dim, int64_t qk_rope_dim, int64_t v_head_dim,
    int64_t previous_len, float rms_eps, float softmax_scale);

/* No single reference counterpart: the FP8 model's one-token attention,
 * fp8_source.py:6337-6454 (`_run_fp8_single_token_attention_native_linear`
 * at one token), which the reference runs as native FP8 linears plus torch.
 * The steps and arguments of ds_attention_block_forward_f32 (without the
 * session handle), with the projections FP8 block-scaled: q_a [q_rank,
 * hidden] and kv_a [R + rope, hidden] on the bf16 hidden state in one launch,
 * q_b [H (nope + rope), q_rank] and o [hidden, H v] on fp32 activations (the
 * reference's FP8 linear takes fp32), each with its scale_inv grid
 * [ceil(rows/128)][ceil(cols/128)]; kv_b fp32 [H (nope + v), R] (the
 * reference dequantizes it to fp32 before the attention).  hidden_out fp32
 * [hidden].  Codes as ds_attention_block_forward_f32, and -1 / -2 from an FP8
 * linear. */
int ds_fp8_attention_block_bf16x_f32(
    const uint16_t* hidden_bf16, const uint8_t* q_a_weight, const float* q_a_scale_inv, const uint8_t* q_b_weight,
    const float* q_b_scale_inv, const uint8_t* kv_a_weight, const float* kv_a_scale_inv, const float* kv_b_weight,
    const uint8_t* o_weight, const float* o_scale_inv, const float* q_norm_weight, const float* kv_norm_weight,
    const float* previous_kv_cache, const float* previous_pe_cache, const float* rope_cos, const float* rope_sin,
    float* next_kv_cache, float* next_pe_cache, float* hidden_out, int64_t hidden_dim, int64_t q_lora_rank,
    int64_t kv_lora_rank, int64_t num_heads, int64_t qk_nope_dim, int64_t qk_rope_dim, int64_t v_head_dim,
    int64_t previous_len, float rms_eps, float softmax_scale);

/* ds_forward.cpp:879-955: softmax top-k router over u16 (fp16/bf16) hidden
 * [hidden_dim] and router weights [num_experts, hidden_dim] (device);
 * output_expert_ids int64 [k] and output_weights fp32 [k] (device).
 * Codes 1 null, 2 bad dims. */
int ds_router_topk_u16(const uint16_t* hidden_u16, const uint16_t* router_weights_u16,
                       int64_t hidden_dim, int64_t num_experts, int64_t k, int64_t dtype_code,
                       int64_t* output_expert_ids, float* output_weights);
/* No counterpart in the reference: ds_router_topk_u16 without the status
 * read-back (for callers that must not wait on the stream, e.g. under HIP
 * graph capture).  The status the synchronous call would return (0, or 3 / 4
 * for a degenerate softmax sum) is written to *status (device memory); the
 * return value covers only the argument checks (1 null, 2 bad dims) and the
 * launch. */
int ds_router_topk_u16_nosync(const uint16_t* hidden_u16, const uint16_t* router_weights_u16, int64_t hidden_dim,
                              int64_t num_experts, int64_t k, int64_t dtype_code, int64_t* output_expert_ids,
                              float* output_weights, int* status);

/* New export for DeepSeek-V3 routing, the torch code of run_fp8_router
 * (src/pcketlm/core/runtime/fp8_source.py:1527-1547) with the group mask of
 * _mask_deepseek_route_groups (5125-5140), from router logits fp32
 * [batch, num_experts] (device).  scoring: 0 sigmoid, 1 softmax.  bias may
 * be NULL.  Writes indices int64 [batch, top_k] and weights fp32
 * [batch, top_k] rounded to bf16 (device).  Codes 1 null, 2 bad dims. */
int ds_route_topk_f32(const float* logits, const float* bias, int64_t batch, int64_t num_experts,
                      int64_t top_k, int64_t n_groups, int64_t topk_groups, int scoring,
                      float route_scale, int64_t* out_indices, float* out_weights);

/* ------------------------------------------------------------------ lm_head */

/* fp16_matmul.cpp:155-204 (native_lm_head_topk_u16): the logits of hidden
 * (u16 [hidden_size], fp16 dtype_code 0 / bf16 1) against every row of weight
 * (u16 [rows][hidden_size], same type), fp32 accumulation, and the top_k
 * (row + token_offset, logit) pairs, written in descending order to
 * out_ids int64 [top_k] / out_logits fp32 [top_k] (all device).  Ties go to
 * the lower row; NaN logits rank as -inf; with fewer rows than top_k the
 * remaining slots are -1 / -inf.  top_k <= 64 and ceil(rows / 4096) * top_k
 * <= 4096 (vocabularies up to 262144 rows at top_k 16).  Codes 1 null,
 * 2 bad dims, -3 workspace. */
int native_lm_head_topk_u16(const uint16_t* hidden, const uint16_t* weight, int64_t* out_ids, float* out_logits,
                            int64_t rows, int64_t hidden_size, int64_t top_k, int dtype_code, int64_t token_offset);

/* fp16_matmul.cpp:344-396 (native_fp16_matmul): c = a @ b for fp16 (u16
 * storage) a [m][k], b [k][n], c [m][n] (all device, row-major), fp32
 * accumulation, c rounded to fp16 to nearest even.  The reference widens to
 * fp32 and calls sgemm; the sums here run in another order (within 1 fp16
 * ulp of the fp32 product rounded).  m or n = 0 writes nothing, k = 0 writes
 * zeros.  Codes 1 null, 2 negative dims. */
int native_fp16_matmul(const uint16_t* a, const uint16_t* b, uint16_t* c, int64_t m, int64_t n, int64_t k);

/* ---------------------------------------------------------------- weight files to HBM */

/* New export: byte ranges of a file copied into device memory (current
 * device), for the reference's on-disk artifacts that it reads into host
 * memory (FP8 pack spans, src/pcketlm/core/runtime/fp8_pack.py:54-241; row8
 * artifacts, src/pcketlm/native/row8_artifact_cache.cpp:20-147; Q4
 * safetensors shards, src/pcketlm/core/model_import/q4_quantize.py:92-168).
 * Span i is file bytes [file_offsets[i], file_offsets[i] + byte_lengths[i])
 * to device address device_dsts[i].  Reader threads fill pinned staging
 * buffers and overlap their reads with the copies; the copies start after
 * the work queued on the library's stream, and the call returns when the
 * bytes are in device memory.  Codes -1 null, -2 a span outside the file,
 * -5 open/read failure, -(1000 + hipError_t). */
int pocketlm_file_spans_to_device(const char* path, const uint64_t* file_offsets, const uint64_t* byte_lengths,
                                  const uint64_t* device_dsts, int64_t count);

/* row8_artifact_cache.cpp:20-43: nbytes at offset of a row8 artifact file
 * (nbytes even and non-zero) loaded into a device buffer the handle owns;
 * NULL on failure.  Here the bytes land in device memory. */
void* row8_artifact_load_tensor(const char* path, uint64_t offset, uint64_t nbytes);
/* row8_artifact_cache.cpp:45-48: frees the handle and its device buffer. */
void row8_artifact_free_tensor(void* handle);
/* row8_artifact_cache.cpp:50-56: the handle's data, a device pointer here
 * (every tensor pointer of this library is one), ready for
 * native_packed_gemv_rows8. */
const uint16_t* row8_artifact_tensor_data(void* handle);
/* row8_artifact_cache.cpp:58-64. */
uint64_t row8_artifact_tensor_nbytes(void* handle);
/* row8_artifact_cache.cpp:66-102: a read-only mapping of the whole file
 * (host memory), NULL on failure. */
void* row8_artifact_map_file(const char* path);
/* row8_artifact_cache.cpp:104-120. */
void row8_artifact_unmap_file(void* handle);
/* row8_artifact_cache.cpp:122-138: host pointer to [offset, offset + nbytes)
 * of the mapping, NULL for an odd or out-of-range request. */
const uint16_t* row8_artifact_mapped_data(void* handle, uint64_t offset, uint64_t nbytes);
/* row8_artifact_cache.cpp:140-147. */
uint64_t row8_artifact_mapped_nbytes(void* handle);

/* New export: run_fp8_moe (src/pcketlm/core/runtime/fp8_source.py:1569-1884)
 * with the experts chosen on the device.  The reference reads the router's
 * indices on the host (sorted unique experts, 1600) before it calls the
 * weighted (M == 1, fp8_linear.cpp:475-589) or row-weighted (M > 1,
 * 591-831) kernel, adds the shared expert's MLP (1849-1859) and sums in
 * bf16 (1762, 1861-1862).  Here the router's outputs stay in HBM:
 *   expert_table   device uint64 [6][num_experts]: gate, gate scale_inv, up,
 *                  up scale_inv, down, down scale_inv addresses of every
 *                  expert (0 = absent: contributes nothing when chosen);
 *   route_indices  device int64 [batch][top_k], route_weights device fp32
 *                  [batch][top_k] (ds_route_topk_f32's outputs);
 *   shared_ptrs    host uint64 [6] of the shared expert, or NULL;
 *   out            device fp32 [batch][hidden_dim], the route-weighted sum
 *                  over the distinct chosen experts in ascending order;
 *   out_shared     device fp32 [batch][hidden_dim] (required with a shared
 *                  expert);
 *   out_bf16       device bf16 [batch][hidden_dim] = bf16(bf16(out) +
 *                  bf16(out_shared)), NaN as 0x7FC0, or NULL;
 *   rejected       device int32, or NULL: receives the number of choices
 *                  outside [0, num_experts) (left out) plus those of an
 *                  expert whose weight addresses are not 16-byte aligned
 *                  (scales: 4), which contributes nothing.
 * Same values as the host-routed calls given the same experts.  Three
 * launches' worth of work in two: the gate/up launch finds each expert
 * among the choices, the down launch computes the shared expert and the
 * bf16 tail beside the routed sum.  batch 1..8, batch * top_k <= 64,
 * hidden_dim and intermediate_rows multiples of 16, hidden 16-byte
 * aligned.  Codes -1 null, -2 bad dims, -3 workspace. */
int fp8_e4m3_block_moe_device_routed_f32(const uint64_t* expert_table, int64_t num_experts,
                                         const int64_t* route_indices, const float* route_weights,
                                         int64_t top_k, const uint64_t* shared_ptrs, const float* hidden,
                                         float* out, float* out_shared, uint16_t* out_bf16, int* rejected,
                                         int64_t batch, int64_t intermediate_rows, int64_t hidden_dim,
                                         int64_t gate_scale_cols, int64_t down_scale_cols);
/* The same with bf16 activations (the decode path's), widened exactly. */
int fp8_e4m3_block_moe_device_routed_bf16x_f32(const uint64_t* expert_table, int64_t num_experts,
                                               const int64_t* route_indices, const float* route_weights,
                                               int64_t top_k, const uint64_t* shared_ptrs,
                                               const uint16_t* hidden_bf16, float* out, float* out_shared,
                                               uint16_t* out_bf16, int* rejected, int64_t batch,
                                               int64_t intermediate_rows, int64_t hidden_dim,
                                               int64_t gate_scale_cols, int64_t down_scale_cols);
/* New export: one DeepSeek-V3 MoE layer from the router's logits, the work
 * of run_fp8_router followed by run_fp8_moe (src/pcketlm/core/runtime/
 * fp8_source.py:1500-1566, 1569-1884) with no host round trip: the routing
 * of ds_route_topk_f32 (logits fp32 [batch, num_experts], bias or NULL,
 * n_groups / topk_groups / scoring / route_scale as there) and the plan of
 * fp8_e4m3_block_moe_device_routed_bf16x_f32 run as one launch, then the
 * same gate/up and down launches.  out_indices int64 [batch, top_k] and
 * out_weights fp32 [batch, top_k] receive the router's choices and weights
 * (both NULL to skip).  Results equal ds_route_topk_f32 followed by
 * fp8_e4m3_block_moe_device_routed_bf16x_f32, bit for bit.  Codes -1 null,
 * -2 bad dims (as both), -3 workspace. */
int fp8_e4m3_block_moe_from_logits_bf16x_f32(const float* router_logits, const float* router_bias, int64_t n_groups,
                                             int64_t topk_groups, int scoring, float route_scale,
                                             const uint64_t* expert_table, int64_t num_experts, int64_t top_k,
                                             const uint64_t* shared_ptrs, const uint16_t* hidden_bf16, float* out,
                                             float* out_shared, uint16_t* out_bf16, int64_t* out_indices,
                                             float* out_weights, int* rejected, int64_t batch,
                                             int64_t intermediate_rows, int64_t hidden_dim, int64_t gate_scale_cols,
                                             int64_t down_scale_cols);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): fp8_e4m3_block_moe_device_routed_bf16x_f32 with its
 * scratch (the fp32 activations [groups][batch][intermediate_rows], 256-byte
 * aligned, then the expert plan) in a fixed 8 MiB device array of the
 * library instead of its workspace.  It calls no hipMalloc or hipFree: the
 * array's address is looked up once per device, on the first call made with
 * that device current.  Same arguments, results and codes, plus -2 when a
 * call needs more than the 8 MiB (groups = batch * top_k + 1 with a shared
 * expert: batch 8, top_k 8 and intermediate_rows 2048 need 4.3 MB).  Every
 * call on a device shares its array, so calls that overlap on one device
 * (two streams, or two threads) race; nothing in it needs to start at zero. */
int fp8_e4m3_block_moe_device_routed_bf16x_f32_noalloc(const uint64_t* expert_table, int64_t num_experts,
                                                       const int64_t* route_indices, const float* route_weights,
                                                       int64_t top_k, const uint64_t* shared_ptrs,
                                                       const uint16_t* hidden_bf16, float* out, float* out_shared,
                                                       uint16_t* out_bf16, int* rejected, int64_t batch,
                                                       int64_t intermediate_rows, int64_t hidden_dim,
                                                       int64_t gate_scale_cols, int64_t down_scale_cols);

/* ---------------------------------------------------------------------------
 * KV session and dense decoder layer decode (src/pcketlm/native/
 * fp16_kv_cache.cpp).  The cache lives in device memory on the device that
 * is current at init: [layer][K|V][max_seq_len][kv_width] fp16 (dtype_code 0)
 * or bf16 (1), committed rows followed by tentative rows.  Lengths are kept
 * on the host, so commit and rollback move no data.  Row pointers given to
 * append/copy may be device or host memory; copies run on the library's
 * stream (pocketlm_set_stream).  Same return codes as the reference. */

/* fp16_kv_cache.cpp:594-611.  NULL on bad arguments or allocation failure. */
void* kv_prefill_init_typed(int64_t layer_count, int64_t max_seq_len, int64_t kv_width, int dtype_code);
/* fp16_kv_cache.cpp:613-619 (fp16). */
void* kv_prefill_init(int64_t layer_count, int64_t max_seq_len, int64_t kv_width);
/* fp16_kv_cache.cpp:621-624.  Waits for the device before freeing the cache. */
void kv_free(void* handle);
/* fp16_kv_cache.cpp:661-669: count rows of kv_width values after the
 * committed rows (tentative rows move back).  1 bad args, 2 full. */
int kv_append_committed(void* handle, int64_t layer, const uint16_t* k_new, const uint16_t* v_new, int64_t count);
/* fp16_kv_cache.cpp:671-679: count rows after the tentative rows. */
int kv_append_tentative(void* handle, int64_t layer, const uint16_t* k_new, const uint16_t* v_new, int64_t count);
/* fp16_kv_cache.cpp:681-715: the first min(count, tentative) tentative rows
 * of every layer become committed. */
int kv_commit(void* handle, int64_t count);
/* fp16_kv_cache.cpp:717-728: drop every layer's tentative rows. */
int kv_rollback(void* handle);
/* fp16_kv_cache.cpp:730-744.  -1 for a bad layer. */
int64_t kv_committed_length(void* handle, int64_t layer);
int64_t kv_tentative_length(void* handle, int64_t layer);
/* fp16_kv_cache.cpp:746-778: committed (+ tentative) rows into k_out/v_out.
 * 1 bad args, 2 more rows than max_count. */
int kv_copy_layer(void* handle, int64_t layer, uint16_t* k_out, uint16_t* v_out, int64_t max_count,
                  int include_tentative);
/* fp16_kv_cache.cpp:1533-1589 (with 1398-1531 and the attention decode
 * 920-1060): one decode step of a dense decoder layer with row8-packed
 * weights (native_pack_u16_rows8).  Input RMSNorm, q/k/v (+ biases), optional
 * per-head q/k RMSNorm, RoPE at position committed + tentative, the new k/v
 * appended as a tentative row, attention over every row of the layer, o
 * projection, residual, post RMSNorm, SiLU MLP, residual -> out (hidden_size
 * values of the session's type).  head_dim = hidden_size / num_heads.  All
 * pointers are device pointers; packed weights 16-byte aligned; biases and
 * q/k norm weights may be NULL.  Codes: 1 null, 2 bad sizes, 100 + the
 * attention decode's (1 layer, 2 heads, 3 divisibility, 4 kv_width, 5 cache
 * full), and 106 for more than 16 query heads per kv head or head_dim > 256
 * (limits of this build's attention kernel). */
int kv_dense_layer_decode_u16_ext_packed_rows8(
    void* handle, int64_t layer, const uint16_t* hidden, const uint16_t* input_norm_weight,
    const uint16_t* post_norm_weight, const uint16_t* q_weight_packed, const uint16_t* k_weight_packed,
    const uint16_t* v_weight_packed, const uint16_t* o_weight_packed, const uint16_t* gate_weight_packed,
    const uint16_t* up_weight_packed, const uint16_t* down_weight_packed, const uint16_t* q_bias,
    const uint16_t* k_bias, const uint16_t* v_bias, const uint16_t* q_norm_weight, const uint16_t* k_norm_weight,
    uint16_t* out, int64_t hidden_size, int64_t intermediate_size, int64_t num_heads, int64_t num_kv_heads,
    float rms_eps, float rope_theta);

/* The entry points over row-major (unpacked) weights that the reference's
 * KV loader binds unconditionally (native/__init__.py:2615-2745):
 * kv_attention_decode_fp16 (fp16_kv_cache.cpp:780-918),
 * kv_attention_decode_u16_ext (920-1060), kv_dense_layer_decode_fp16
 * (1206-1260) and kv_dense_layer_decode_u16_ext (1398-1531).  Same
 * arguments.  They are not implemented by this library: after the
 * reference's argument checks (code 1 for a bad handle, layer or null
 * pointer, 2 for non-positive sizes) they return 90, with the reason in
 * pocketlm_last_error().  A caller packs each weight once with
 * native_pack_u16_rows8 and calls kv_dense_layer_decode_u16_ext_packed_rows8,
 * which runs the same layer. */
int kv_attention_decode_fp16(void* handle, int64_t layer, const uint16_t* hidden, const uint16_t* q_weight,
                             const uint16_t* k_weight, const uint16_t* v_weight, const uint16_t* o_weight,
                             uint16_t* out, int64_t hidden_size, int64_t num_attention_heads,
                             int64_t num_key_value_heads, float rope_theta);
int kv_attention_decode_u16_ext(void* handle, int64_t layer, const uint16_t* hidden, const uint16_t* q_weight,
                                const uint16_t* k_weight, const uint16_t* v_weight, const uint16_t* o_weight,
                                const uint16_t* q_bias, const uint16_t* k_bias, const uint16_t* v_bias,
                                const uint16_t* q_norm_weight, const uint16_t* k_norm_weight, uint16_t* out,
                                int64_t hidden_size, int64_t num_attention_heads, int64_t num_key_value_heads,
                                float rope_theta, float rms_eps);
int kv_dense_layer_decode_fp16(void* handle, int64_t layer, const uint16_t* hidden,
                               const uint16_t* input_norm_weight, const uint16_t* post_norm_weight,
                               const uint16_t* q_weight, const uint16_t* k_weight, const uint16_t* v_weight,
                               const uint16_t* o_weight, const uint16_t* gate_weight, const uint16_t* up_weight,
                               const uint16_t* down_weight, uint16_t* out, int64_t hidden_size,
                               int64_t intermediate_size, int64_t num_heads, int64_t num_kv_heads, float rms_eps,
                               float rope_theta);
int kv_dense_layer_decode_u16_ext(void* handle, int64_t layer, const uint16_t* hidden,
                                  const uint16_t* input_norm_weight, const uint16_t* post_norm_weight,
                                  const uint16_t* q_weight, const uint16_t* k_weight, const uint16_t* v_weight,
                                  const uint16_t* o_weight, const uint16_t* gate_weight, const uint16_t* up_weight,
                                  const uint16_t* down_weight, const uint16_t* q_bias, const uint16_t* k_bias,
                                  const uint16_t* v_bias, const uint16_t* q_norm_weight,
                                  const uint16_t* k_norm_weight, uint16_t* out, int64_t hidden_size,
                                  int64_t intermediate_size, int64_t num_heads, int64_t num_kv_heads, float rms_eps,
                                  float rope_theta);

#ifdef __cplusplus
}
#endif

#endif /* POCKETLM_HIP_H_ */
