/*
 * gs_gemv.h -- C ABI of the gfx950 quantized GEMV that produces the logits.
 *
 * The step before the sampler in gguf-rs-cli's decode (src/model/llama.rs:333-334):
 * the output projection `gpu.cmd_gemv(output, &xn, &logits)`, one f32 logit per
 * row of the quantized output matrix.  The reference uploads a GGUF tensor with
 *
 *   pub fn upload(&mut self, wt: &QuantTensor) -> Option<GpuTensor>   src/gpu/mod.rs:222-238
 *
 * (repacking the blocks with pack_q4_0_for_gpu / pack_q4_1_for_gpu /
 * pack_q3k_for_gpu / pack_q4k_for_gpu / pack_q5k_for_gpu / pack_q6k_for_gpu /
 * pack_q8_0_for_gpu, src/tensor/dequant.rs:319-480) and runs
 *
 *   pub fn cmd_gemv(&mut self, wt: &GpuTensor, inp: &ActBuf, out: &ActBuf)   src/gpu/mod.rs:438-443
 *
 * with the block type's shader (src/gpu/q*_gemv.glsl).
 * Its CPU path is QuantTensor::matvec / row_dot (src/tensor/dequant.rs:277-318).
 *
 * Weights are the GGUF tensor's raw blocks (what QuantTensor::data() returns,
 * src/tensor/dequant.rs:265-267): Q4_0 = 18 bytes per 32 weights (f16 d, 16 bytes
 * of nibbles: byte l holds weights l and l + 16), Q4_1 = 20 (f16 d, f16 m, the
 * same nibbles), Q8_0 = 34 bytes per 32 weights (f16 d, 32 int8),
 * Q3_K = 110 bytes per 256 weights (hmask[32], qs[64], 12 bytes of 6-bit scales,
 * f16 d),
 * Q6_K = 210 bytes per 256 weights (ql[128], qh[64], int8 scales[16], f16 d),
 * Q4_K = 144 bytes (f16 d, f16 dmin, 12 bytes of 6-bit scales and mins,
 * qs[128]), Q5_K = 176 bytes (the same with qh[32] before qs).
 * The result is out[r] = sum_c W[r][c] * x[c], W dequantized as the reference
 * does it (Q4_0: (q - 8) * d; Q4_1: q * d + m; Q8_0: q * d; Q3_K / Q6_K:
 * (d * scale) * q; Q4_K / Q5_K: (d * sc) * q - dmin * m; dq40 / dq41 / dq4k /
 * dq5k, src/tensor/dequant.rs:26-54, 141-196); the summation order
 * is the kernel's own, so results agree with the reference's to f32 rounding,
 * not bit for bit.  Q5_K follows the GGUF format where the reference's two
 * paths cannot: its CPU dq5k indexes qh[32 + l] in a 32-byte slice from the
 * third step on (a panic, :177,192) and its shader decodes the scales of
 * sub-blocks 4-7 with another bit layout (q5k_gemv.glsl get_scale_min); here
 * qh[l] serves every step and the scales are get_scale_min_k4's, as in dq4k.
 * Q3_K follows the GGUF format too: the reference's dq3k reads the low bits of
 * weight i from qs[i / 4] (:134) and unpacks the 6-bit scales with another bit
 * layout (:126-131), and its shader with a third one; here weight
 * 128 n + 32 j + l takes bits 2j..2j+1 of qs[32 n + l] and bit 4n + j of
 * hmask[l], and the scales are GGUF's (low nibbles in bytes 0-7, top bits in
 * bytes 8-11).  Q4_0 follows dq40 / row_dot: the reference's Q4_0 shader
 * decodes its scale word as f16 bits, but pack_q4_0_for_gpu stores the f32
 * bits of the scale (dequant.rs:328, q4_0_gemv.glsl), so its GPU results
 * differ from its CPU results.
 * Same status codes as gs_sampler.h.
 */
#ifndef GS_GEMV_H
#define GS_GEMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Block types, numbered as GgmlType (src/gguf/types.rs:43-48). */
#define GS_QTYPE_Q4_0  2u
#define GS_QTYPE_Q4_1  3u
#define GS_QTYPE_Q8_0  8u
#define GS_QTYPE_Q3_K  11u
#define GS_QTYPE_Q4_K  12u
#define GS_QTYPE_Q5_K  13u
#define GS_QTYPE_Q6_K  14u

typedef struct gs_qmatrix gs_qmatrix;

/* Replaces Gpu::upload (src/gpu/mod.rs:222-238) for the seven block types above.
 * `blocks` is a host pointer to rows*cols weights in GGUF block order
 * (row-major, dims[0] = cols as in QuantTensor::new, src/tensor/dequant.rs:256-263).
 * The blocks are split into the device layout (bit planes, int8 scales, f16 d)
 * and copied to the current HIP device; synchronous.  cols must be a multiple
 * of the block size (32 / 256) -- where the reference's upload returns None
 * and falls back to the CPU, this returns GS_ERR_UNSUPPORTED (for Q4_0 and Q4_1
 * the reference has no such check and would read misaligned blocks) -- and at
 * most 16384.  Other block types return GS_ERR_UNSUPPORTED, as the
 * reference's upload returns None for them. */
int gs_qmatrix_upload(uint32_t qtype, const void *blocks, size_t rows, size_t cols, gs_qmatrix **out);
int gs_qmatrix_destroy(gs_qmatrix *m);
int gs_qmatrix_shape(const gs_qmatrix *m, uint32_t *qtype, size_t *rows, size_t *cols);

/* Replaces Gpu::cmd_gemv (src/gpu/mod.rs:438-443): for b < B,
 * d_out[b*rows + r] = sum_c W[r][c] * d_x[b*cols + c].  Device pointers;
 * asynchronous on `stream` (NULL = default stream).  B = 1 is the reference's
 * decode step; each further vector is another full pass over the weights (a
 * GEMV per vector, not a GEMM), so this entry is meant for small B: a
 * batch of hundreds of vectors should bring its own GEMM and hand the logits
 * to the sampler. */
int gs_gemv(const gs_qmatrix *m, const float *d_x, size_t B, float *d_out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GS_GEMV_H */
