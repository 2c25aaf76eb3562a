/*
 * jeeves_fp8.h -- C ABI of the MI355X (gfx950) FP8 linear-layer library
 * (libjeeves_fp8.so).
 *
 * The reference's FP8 path (PostHog/jeeves, `--precision fp8`) is Python over
 * Triton kernels; these entry points are what its Python layer would bind in
 * their place (ctypes, see the wrapper in jeeves_amd/_lib.py). Each
 * declaration names the reference interface it replaces.
 *
 * Conventions for every entry point:
 *   - pointers are device pointers (HBM) unless stated; bf16 tensors are
 *     passed as raw 16-bit storage, e4m3fn codes as bytes;
 *   - `stream` is a hipStream_t (NULL = the legacy default stream);
 *   - calls only enqueue work on `stream`: no allocation, no host
 *     synchronisation, so they may be captured into a HIP graph;
 *   - the return value is a JV_* status; on failure jv_fp8_last_error()
 *     returns a message for the calling thread;
 *   - row strides (`ld*`) are in elements; rows of bf16 and e4m3 operands
 *     must start on 16-byte boundaries (ld*elem_size % 16 == 0, base 16-byte
 *     aligned).
 */
#ifndef JEEVES_FP8_H
#define JEEVES_FP8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JV_OK 0
#define JV_ERR_VALUE 1   /* invalid argument (the reference raises ValueError) */
#define JV_ERR_RUNTIME 2 /* invalid state (the reference raises RuntimeError) */
#define JV_ERR_HIP 3     /* a HIP launch or runtime call failed */

/* K granularity of the GEMM (BLOCK_K, inference/fp8.py:26). */
#define JV_FP8_BLOCK_K 128
/* Rows at or below which the GEMM takes the HBM-bound decode kernel
 * (the counterpart of SPLIT_K_MAX_ROWS's regime split, inference/fp8.py:20). */
#define JV_FP8_DECODE_MAX_ROWS 64
/* Tile counters a stream needs at most (TILE_COUNTER_SLOTS, inference/fp8.py:27). */
#define JV_FP8_TILE_COUNTER_SLOTS 65536

/* Message for the last failed call on this thread ("" if none). */
const char* jv_fp8_last_error(void);

/* Compute units of HIP device `device` (-1 = current device).
 * Replaces sm_count (model/triton_kernels.py:18-20). Returns <= 0 on error. */
int jv_device_cu_count(int device);

/* quantize_rows (inference/fp8_weights.py:16-19) on the device, for bf16 rows:
 *   scales[r] = max(max_c |x[r,c]|, 1e-12) * fp32(1/448)
 *   codes[r,c] = e4m3fn(x[r,c] / scales[r])   (IEEE quotient, RNE, NaN on overflow)
 * x: [rows, cols] bf16, row stride ldx; codes: [rows, cols] bytes, row stride
 * ldc; scales: [rows] fp32. cols must be a positive multiple of 8.
 * ldc = 0 writes the codes in the GEMMs' packed fragment order instead (the
 * tiled weight layout below applied to token rows, rows padded to a multiple
 * of 16 with zero codes; cols a multiple of 128 up to 16384; the buffer holds
 * jv_fp8_packed_codes_bytes(rows, cols) bytes), for jv_fp8_gemm with
 * ldxq = 0. Both the decode and the prefill GEMMs read that order fastest, and
 * jv_fp8_linear uses it for its own codes.
 * Used for per-token activation quantization and for FP8Linear.load_weight
 * (inference/fp8.py:164-166). */
int jv_fp8_quantize_rows_bf16(const void* x, int64_t ldx, int64_t rows, int64_t cols, void* codes, int64_t ldc,
                              float* scales, void* stream);

/* Bytes of rows x cols activation codes in the packed fragment order (rows
 * padded to a multiple of 16), or -1 when the layout does not apply. The
 * counterpart of the fp16 row copies fp8_matmul allocates
 * (inference/fp8.py:142-143). */
int64_t jv_fp8_packed_codes_bytes(int64_t rows, int64_t cols);

/* Same for float32 rows (FP8Linear.load_weight given fp32 weights). cols must be a
 * positive multiple of 4. */
int jv_fp8_quantize_rows_f32(const float* x, int64_t ldx, int64_t rows, int64_t cols, void* codes, int64_t ldc,
                             float* scales, void* stream);

/* quantize_rows on the host CPU (inference/fp8_weights.py:16-19), for the
 * exporter's quantize_row_blocks_on_cpu (inference/fp8_weights.py:22-26) on
 * a machine without a GPU: float32 rows in, e4m3 codes [rows, cols] (row
 * stride ldc) and float32 scales [rows] out, bitwise equal to the device
 * quantizer. Runs on `threads` host threads (0: all hardware threads); makes
 * no HIP call. */
int jv_fp8_quantize_rows_host(const float* w, int64_t ldw, int64_t rows, int64_t cols, void* codes, int64_t ldc,
                              float* scales, int threads);

/* Workspace bytes jv_fp8_linear needs for these sizes (activation codes and
 * scales, LoRA low-rank activations, split-K partials). */
int64_t jv_fp8_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t lora_rank);

/* fp8_matmul (inference/fp8.py:112-148) plus FP8Linear.forward's bias
 * (inference/fp8.py:183-184) and an optional LoRA adapter
 * (model/lora.py:122-133), as one call:
 *   per-token quantization of x (quantize_rows semantics), then
 *   v[m,n] = acc[m,n] * sx[m] * w_scale[n] + lora_scaling * sum_r (x A^T)[m,r] * B[n,r],
 *   y[m,n] = bf16(v[m,n]), or with a bias bf16( bf16(v[m,n]) + bias[n] )
 *   (the bias added to the bf16 GEMM output in bf16, as FP8Linear.forward does),
 *   acc[m,n] = sum_k xq[m,k] * w[n,k]  (e4m3 x e4m3, fp32 accumulation).
 * x: [M,K] bf16 (row stride ldx); w: [N,K] e4m3fn (row stride ldw, or
 * ldw = 0: the tiled layout below);
 * w_scale: [N] fp32; bias: [N] bf16 or NULL; lora_a: [rank,K] bf16 and
 * lora_b: [N,rank] bf16, or NULL with lora_rank 0 (rank 16 supported);
 * y: [M,N] bf16 (row stride ldy).
 * K must be a positive multiple of 128 (JV_ERR_VALUE otherwise, the
 * ValueError of inference/fp8.py:115-117). workspace must hold
 * jv_fp8_linear_workspace_bytes(M,N,K,rank) bytes (256-byte aligned).
 * tile_counters: n_counters int32 slots, zero before first use, owned by one
 * stream (launches on different streams must not share them); kernels leave
 * them zero. Results are deterministic for a given device CU count. */
int jv_fp8_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* w_scale, const void* bias,
                  const void* lora_a, const void* lora_b, int64_t lora_rank, float lora_scaling, void* y, int64_t ldy,
                  int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, int32_t* tile_counters,
                  int64_t n_counters, void* stream);

/* Bytes of device memory jv_fp8_linear_noalloc keeps per GPU for the rest of
 * the process (its tile counters and workspace). */
#define JV_FP8_NOALLOC_SCRATCH_BYTES (32 << 20)

/* jv_fp8_linear without a workspace or tile counters, for callers that cannot
 * allocate device memory (code under HIP graph capture that must not touch
 * the allocator, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. It allocates nothing: the quantized
 * activations, scales, LoRA low-rank activations, split-K partials and tile
 * counters live in a library-owned device array of
 * JV_FP8_NOALLOC_SCRATCH_BYTES per GPU (minus 16 KiB of counters for the
 * workspace: every decode call, M <= 64 and K <= 16384, and on the 9B
 * projection shapes prefill batches up to 8176 tokens at K = 4096 or 2720 at
 * K = 12288 fit; the split-K partials of the prefill plans, up to 16 MiB,
 * share the space, so other shapes can reach the limit sooner).
 * Sizes whose jv_fp8_linear_workspace_bytes exceed it return JV_ERR_VALUE. Same results
 * as jv_fp8_linear, bit for bit. Every call on a GPU shares that GPU's
 * scratch: calls that overlap on one GPU (concurrent streams, or host threads
 * on one device without ordering) race; calls ordered on one stream do not.
 * Arguments as jv_fp8_linear. */
int jv_fp8_linear_noalloc(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* w_scale, const void* bias,
                          const void* lora_a, const void* lora_b, int64_t lora_rank, float lora_scaling, void* y,
                          int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream);

/* W8A16 parity mode: the arithmetic of the reference's FP8Linear.forward
 * (inference/fp8.py:62-99 with its bias at :183-184, stated as
 * ((x.float() @ w8.float().t()) * scale).to(bf16) in model/metal_test.py:213):
 *   y[m,n] = bf16( sum_k x[m,k] * w[n,k] * w_scale[n] )   (bf16 x e4m3, fp32 sums)
 *   then, with a bias, y[m,n] = bf16( y[m,n] + bias[n] ).
 * No activation quantization: the bf16 activations enter the GEMM as they
 * are. Arguments as jv_fp8_linear (no LoRA); K a positive multiple of 128.
 * workspace: jv_w8a16_workspace_bytes(M,N,K) bytes (split-K partials of the
 * decode kernel or of the prefill kernel's 64x64 tiles, 0 for most shapes);
 * tile_counters as jv_fp8_linear, needed whenever that size is not 0 (the
 * call checks that the split's tiles fit n_counters). */
int64_t jv_w8a16_workspace_bytes(int64_t M, int64_t N, int64_t K);
int jv_w8a16_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* w_scale, const void* bias,
                    void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                    int32_t* tile_counters, int64_t n_counters, void* stream);

/* Workspace bytes jv_fp8_gemm needs (split-K partials only). */
int64_t jv_fp8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* The GEMM and epilogue alone on already-quantized activations
 * (_fp8_matmul, inference/fp8.py:62-99, with FP8 x FP8 operands):
 * xq: [M,K] e4m3fn (row stride ldxq; ldxq = 0: the packed fragment order of
 * jv_fp8_quantize_rows_bf16 with ldc = 0);
 * x_scale: [M] fp32; lora_t: [M,rank] fp32 low-rank activations or NULL;
 * other arguments as jv_fp8_linear. */
int jv_fp8_gemm(const void* xq, int64_t ldxq, const float* x_scale, const void* w, int64_t ldw, const float* w_scale,
                const void* bias, const float* lora_t, const void* lora_b, int64_t lora_rank, float lora_scaling, void* y,
                int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                int32_t* tile_counters, int64_t n_counters, void* stream);

/* SwiGLU between the gate/up and down projections (SwiGLU.forward,
 * model/model.py:581-584) fused with the down projection's per-token
 * quantization: h = bf16(bf16(silu(gate)) * up), then quantize_rows(h).
 * gate, up: [M,I] bf16 (may be the two halves of one fused gate+up output);
 * codes: [M,I] with row stride ldc (ldc = 0: packed fragment order, as for
 * jv_fp8_quantize_rows_bf16); scales: [M]; h_out: [M,I] bf16 copy of h or NULL; lora_a:
 * [rank,I] bf16 with lora_t: [M,rank] fp32 output (h A^T), or NULL/0.
 * I must be a positive multiple of 8 and at most 16384. */
int jv_fp8_swiglu_quantize(const void* gate, int64_t ldg, const void* up, int64_t ldu, int64_t M, int64_t I, void* codes,
                           int64_t ldc, float* scales, void* h_out, int64_t ldh, const void* lora_a, int64_t lora_rank,
                           float* lora_t, void* stream);

/* SwiGLU.forward's gate and up projections (model/model.py:581-584) as one
 * fused FP8 linear with SwiGLU in the GEMM epilogue:
 *   h[m,i] = bf16( bf16(silu(g[m,i])) * u[m,i] ),
 * g and u being what jv_fp8_linear would output for the gate rows [0, I) and
 * the up rows [I, 2I) of w (bias and LoRA included), so h is bitwise the
 * result of running the two projections and then F.silu(gate) * up on bf16.
 * w: [2I, K] e4m3fn, gate rows then up rows (row stride ldw, or ldw = 0: the
 * tiled layout); w_scale, bias: [2I]; lora_b: [2I, rank]; h: [M, I] bf16 with
 * row stride ldh >= I; h_amax: NULL or [M, I/16] uint16 receiving, per token
 * and 16 channels of h, the largest |h| as a bf16 magnitude pattern (NaN
 * sorts above inf). I a positive multiple of 16, K <= 16384. workspace:
 * jv_fp8_linear_workspace_bytes(M, 2I, K, rank) bytes; tile_counters as for
 * jv_fp8_linear: the fused GEMM takes the plain GEMM's plan for the same
 * weight, a K split across workgroups included (the last workgroup of a
 * tile applies SwiGLU to the summed tile). The gate+up output [M, 2I] never
 * reaches memory.
 * h follows the reference's F.silu(gate) * up branch (two bf16 roundings);
 * its fla branch (_fla_swiglu, one rounding) is not matched, and parity with
 * it is unpinned. */
int jv_fp8_linear_swiglu(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* w_scale, const void* bias,
                         const void* lora_a, const void* lora_b, int64_t lora_rank, float lora_scaling, void* h,
                         int64_t ldh, uint16_t* h_amax, int64_t M, int64_t I, int64_t K, void* workspace,
                         int64_t workspace_bytes, int32_t* tile_counters, int64_t n_counters, void* stream);

/* The down projection's per-token quantization of h (quantize_rows
 * semantics, as jv_fp8_quantize_rows_bf16), for jv_fp8_gemm: codes in the
 * packed fragment order when ldc = 0, scales [M]; with lora_a [rank, I] bf16
 * also lora_t [M, rank] = h A^T in fp32. h_amax: the maxima
 * jv_fp8_linear_swiglu wrote for this h, or NULL. Decode batches (M <= 128)
 * in the packed layout without LoRA take each row's maximum from h_amax when
 * it is 8-byte aligned, so a row splits over several workgroups; h_amax must
 * then be exactly what jv_fp8_linear_swiglu stored with this h. Otherwise it
 * is not read, and each row's maximum is taken from h itself in the one pass
 * that encodes it (the row stays in registers). Either way the codes and
 * scales are the same bits. I a multiple of 16 (of 128 when packed), at most
 * 16384. */
int jv_fp8_quantize_swiglu_output(const void* h, int64_t ldh, const uint16_t* h_amax, int64_t M, int64_t I, void* codes,
                                  int64_t ldc, float* scales, const void* lora_a, int64_t lora_rank, float* lora_t,
                                  void* stream);

/* Tiled weight layout. Every GEMM entry point takes ldw = 0 to mean that w
 * holds the codes in the decode MFMA's fragment order instead of row-major:
 * for 16-row tile t = n/16 and 128-deep step s = k/128, a 2 KB fragment of
 * two 1 KB halves (h = (k%32)/16), each 64 lanes x 16 bytes with
 * lane = n%16 + 16*((k%128)/32); byte offset
 *   ((t*(K/128) + s)*2 + h)*1024 + lane*16 + k%16.
 * It needs N % 16 == 0, K % 128 == 0 and N*K < 64 GiB, and holds N*K bytes; decode waves
 * read it as one contiguous 1 KB per load. No counterpart in the reference's
 * CUDA path; its Metal path stores its weights tiled for its own kernel in
 * the same way (MetalFP8Linear.tiled_codes, inference/fp8_metal.py:13-34;
 * tile_fp8_codes, model/metal.py:705). These convert codes (row stride ldc)
 * to and from it, asynchronously on `stream`; not in place. */
int jv_fp8_tile_weight(const void* codes, int64_t ldc, int64_t N, int64_t K, void* tiled, void* stream);
int jv_fp8_untile_weight(const void* tiled, int64_t N, int64_t K, void* codes, int64_t ldc, void* stream);

/* Dispatch introspection (the role of split_for, inference/fp8.py:105-109):
 * the number of K splits across workgroups the GEMM uses for these sizes on a
 * device with cu_count compute units (1 = no cross-workgroup split; the
 * decode kernel splits narrow weights, the prefill tiles split K when too few
 * of them fill the CUs, as the reference splits below 256 rows,
 * inference/fp8.py:118-123), and the tile counters it needs. */
int jv_fp8_split_for(int64_t M, int64_t N, int64_t K, int cu_count);
int64_t jv_fp8_counters_needed(int64_t M, int64_t N, int64_t K, int cu_count);

/* The same introspection for the whole launch: shape[0] = the GEMM kernel
 * (0 decode, 1 prefill lockstep tiles, 2 prefill ping-pong tiles, 3 batch-decode
 * kernel: 17-128 tokens, no K split, no counters), shape[1] =
 * its workgroups (K splits included), shape[2] = threads per workgroup,
 * shape[3] = K splits across workgroups. For measurement tools that
 * compare a GEMM with other launches of its shape. */
int jv_fp8_launch_shape(int64_t M, int64_t N, int64_t K, int cu_count, int32_t* shape);

#ifdef __cplusplus
}
#endif

#endif /* JEEVES_FP8_H */
