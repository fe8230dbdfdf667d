/*
 * moex_dense.h -- C ABI of the MI355X (gfx950) dense projections on either side of moex's attention: the fused
 * qkv projection that writes the q / gate / k / v rows attn_decode reads (moex.cu:1084,1395; [LQ = 9216][D = 2048])
 * and the o projection of its output (moex.cu:1086,1399; [D = 2048][AH*AHD = 4096]).
 *
 * The weights are the reference's default form of these matrices (struct Mat with q and s, kernels.cuh:186-196):
 * int8 [O][I] row-major plus one fp32 scale per row, y = s[o] * (q[o,:] . x); moex_gemv / moex_gemm take the
 * matrix in any of the reference's forms (int8, int4 gs64, int6 gs64, fp16). Every entry point replaces one function
 * of src/kernels.cuh, cited on its declaration, with the reference's argument order. All pointers are device pointers;
 * stream is an opaque hipStream_t (NULL = the default stream). Nothing allocates or synchronizes, except the MFMA
 * GEMM (moex_gemm_i8 with S > 8, moex_gemm when it takes the GEMM): it rounds X to fp16 into a per-(device, stream)
 * workspace of S * I * 2 bytes and, when its tile grid is short of one workgroup per CU, splits K and keeps the fp32
 * partial sums in a second one (nks * S * O * 4 bytes, nks <= 512 / tiles). Both are allocated on first use and
 * grown (after waiting for the stream) for larger sizes, kept until the process ends. Errors are reported as in
 * moex_attn.h (print and exit(1), or the soft-error slot).
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

/* ---- the other weight forms of a dense matrix (struct Mat, kernels.cuh:186-196) ----
 * A matrix is held in exactly one form, the first non-NULL of q4, q6, q, f16 (the reference's order of tests):
 *   f16       fp16 [O][I] (binary16 bit patterns);
 *   q, s      int8 [O][I] + fp32 row scales [O] (as above);
 *   q4, s     int4 gs64: [O][I/2] bytes, weight i of a row in bits 4 (i % 2) of byte i / 2 (low nibble first), two's
 *             complement, and fp32 scales [O][I/64], one per 64 inputs: w = q * s;
 *   q6, q6h, s  int6 gs64: the low 4 bits in q6 as q4's nibbles, the high 2 bits in q6h [O][I/4] at bits 2 (i % 4) of
 *             byte i / 4, u = low | high << 4 in [0, 63], w = (u - 32) * s, s [O][I/64]. */
typedef struct moex_mat {
    const uint16_t* f16;
    const int8_t* q;
    const float* s;
    const uint8_t* q4;
    const uint8_t* q6;
    const uint8_t* q6h;
} moex_mat;

/* quantize_rows_q4_k<<<O, 64>>>(W, q4, s, I) (kernels.cuh:576-590): per 64-input group scale = absmax / 7 (1 for a
 * zero group), q = round-half-even(w / scale) clamped to [-8, 7]. I % 64 == 0. Bit-exact. */
void moex_quantize_rows_q4(const uint16_t* W, uint8_t* q4, float* s, int O, int I, void* stream);

/* quantize_rows_q6_k<<<O, 64>>>(W, q6, q6h, s, I) (kernels.cuh:552-573): scale = group absmax / 31 (1 for a zero
 * group), u = round-half-even(w / scale) clamped to [-32, 31], + 32. I % 64 == 0. Bit-exact. */
void moex_quantize_rows_q6(const uint16_t* W, uint8_t* q6, uint8_t* q6h, float* s, int O, int I, void* stream);

/* gemv(m, x, y, I, O, st) (kernels.cuh:214-219): y [O] = W . x with fp32 sums for any form of m (int8 as
 * moex_gemv_i8; int4 and int6 sum each 32-input unit, then scale it, as gemv_q4_k / gemv_q6_k, :486-550; fp16 as
 * gemv_f16_k, :68-93). I % 64 == 0 (int4, int6), I % 32 == 0 (fp16), int8 as moex_gemv_i8. */
void moex_gemv(const moex_mat* m, const float* x, float* y, int I, int O, void* stream);

/* gemm(m, X, Y, S, I, O, st) (kernels.cuh:339-369): Y [S][O] = X [S][I] . W^T with the reference's choice of path:
 *   int8: moex_gemm_i8;
 *   int6 with S <= 8: one GEMV pass for all S rows, each row bit-identical to moex_gemv of that row;
 *   int4 and fp16 with S <= 2: moex_gemv row by row;
 *   otherwise the fp16 MFMA GEMM: activations rounded to fp16, int4 / int6 weights times their group scale rounded
 *   to fp16 (fp16 weights as stored), fp32 accumulation (gemm_wmma_k :225-248, gemm_i8_k<true> :250-337).
 * The GEMM takes the per-stream workspaces of moex_gemm_i8 (see the top of this file). */
void moex_gemm(const moex_mat* m, const float* X, float* Y, int S, int I, int O, void* stream);

#ifdef __cplusplus
}
#endif
#endif
