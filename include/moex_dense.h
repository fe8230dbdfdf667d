/*
 * moex_dense.h -- C ABI of the MI355X (gfx950) dense int8 projections on either side of moex's attention: the fused
 * qkv projection that writes the q / gate / k / v rows attn_decode reads (moex.cu:1084,1395; [LQ = 9216][D = 2048])
 * and the o projection of its output (moex.cu:1086,1399; [D = 2048][AH*AHD = 4096]).
 *
 * The weights are the reference's default form of these matrices (struct Mat with q and s, kernels.cuh:186-196):
 * int8 [O][I] row-major plus one fp32 scale per row, y = s[o] * (q[o,:] . x). Every entry point replaces one function
 * of src/kernels.cuh, cited on its declaration, with the reference's argument order. All pointers are device pointers;
 * stream is an opaque hipStream_t (NULL = the default stream). Nothing allocates or synchronizes, except moex_gemm_i8
 * with S > 8: it rounds X to fp16 into a per-(device, stream) workspace of S * I * 2 bytes, allocated on first use
 * and grown (after waiting for the stream) for a larger S * I, kept until the process ends. Errors are reported
 * as in moex_attn.h (print and exit(1), or the soft-error slot).
 */
#ifndef MOEX_DENSE_H
#define MOEX_DENSE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* quantize_rows_i8_k<<<O, 256>>>(W, q, s, I) (kernels.cuh:144-156): fp16 rows W [O][I] (binary16 bit patterns) ->
 * q int8 [O][I], s f32 [O] = absmax/127 of the row (1 for a zero row), q = round-half-even(w / s). Bit-exact. */
void moex_quantize_rows_i8(const uint16_t* W, int8_t* q, float* s, int O, int I, void* stream);

/* gemv(Mat{q, s}, x, y, I, O, st) for an int8 Mat (kernels.cuh:214-219 -> gemv_i8, :98-141):
 * y [O] = s * (q . x), fp32 sums. I % 512 == 0 (as the reference requires). */
void moex_gemv_i8(const int8_t* q, const float* s, const float* x, float* y, int I, int O, void* stream);

/* gemm(Mat{q, s}, X, Y, S, I, O, st) for an int8 Mat (kernels.cuh:339-350): Y [S][O] = X [S][I] . q^T * s.
 * S <= 8 (MTP / draft rounds): one GEMV pass that reads the weights once for all S rows; each row is bit-identical
 * to moex_gemv_i8 of that row alone. S > 8 (prefill): a tiled fp16 MFMA GEMM (activations rounded to fp16, int8
 * weights exact, fp32 accumulation, the row scale applied last), as gemm_i8_k (kernels.cuh:250-337).
 * I % 512 == 0 for S <= 8, I % 32 == 0 for S > 8. */
void moex_gemm_i8(const int8_t* q, const float* s, const float* X, float* Y, int S, int I, int O, void* stream);

#ifdef __cplusplus
}
#endif
#endif
