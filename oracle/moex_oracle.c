/*
 * moex_oracle.c -- CPU restatement of moex's attention hot path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library, and only as the
 * checker or as the timed CPU baseline. The product (moex_amd/, libmoex_attn.so) never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference repository).
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math: SSE single precision is IEEE binary32,
 * so float / and sqrtf are correctly rounded, like nvcc's defaults -prec-div=true -prec-sqrt=true).
 *
 * Parity status of each function:
 *   orc_int8_quant_row     pinned: closed form (max |x| is order-free, IEEE divide, round-half-even),
 *                          checked against numpy and brute force in tests/test_oracle.py.
 *   orc_tq_tables          pinned: centroids recomputed by a Lloyd-Max iteration for N(0,1/128), codes
 *                          round(127 c / c_max), thresholds = midpoints (tests/test_oracle.py).
 *   orc_tq_wht             pinned: H.H = 128 I, inverse(forward(x)) = x, orthonormality, Sylvester order
 *                          against scipy.linalg.hadamard (tests/test_oracle.py).
 *   orc_tq_half_sum        pinned by construction against a brute-force 32-lane butterfly simulation; the
 *                          FMA-contraction question of the CUDA build (x*x fused into the first
 *                          shuffle-add) is parity unpinned: no CUDA run is possible here; this oracle
 *                          assumes no contraction.
 *   orc_tq_quant/pack      pinned: nearest-centroid brute force, packing round trip, norm invariant.
 *   orc_attn_row_f64       pinned: tiny cases against a dense numpy softmax and against closed forms
 *                          (one key, equal keys, V constant) in tests/test_oracle.py.
 *   orc_attn_row_fa_emul   not a parity target: it models the rounding points of attn_fa_k
 *                          (kernels.cuh:1508,1513,1656-1661) to estimate the reference kernel's error.
 *   orc_qk_norm_rope_row   tolerance only (rsqrtf/powf/sinf/cosf bits are parity unpinned).
 *   orc_quantize_rows_i8   pinned: closed form (max |w| is order-free, IEEE divide, round-half-even), checked
 *                          against numpy on random and edge rows in tests/test_oracle.py.
 *   orc_dense_i8_f64       pinned: the exact product of the int8 rows with fp32 inputs in fp64, checked against
 *                          numpy's float64 matmul in tests/test_oracle.py.
 *   orc_dense_i8_fp16x     not a parity target: the precision model of the prefill GEMM (activations rounded to
 *                          fp16, kernels.cuh:250,306-307), used to bound the reference kernel's error.
 *   orc_quantize_rows_q4/q6  pinned: closed form (group absmax, IEEE divide, round-half-even, clamp, packing),
 *                          checked in tests/test_oracle.py on constructed ties and known packed bytes, and against
 *                          numpy's rint on random rows.
 *   orc_dense_mat_f64      pinned: the exact product of the dequantized weights (q * scale, fp16 as stored) in fp64,
 *                          checked against numpy's float64 matmul of independently unpacked weights.
 *   orc_dense_mat_fp16x    not a parity target: the precision model of the int4 / int6 / fp16 GEMMs (weights
 *                          fp16(fp32(q * scale)), activations fp16, kernels.cuh:276-279,306-307,313-317).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#define AHD 256
#define TQ_KB 128
#define TQ_VB 96

/* ---- turbo constants: kernels.cuh:1123-1139 (values restated; the tables are data fixed by the format) ---- */
static const float S1[128] = {
    -1, 1, 1,-1,-1, 1,-1, 1,-1,-1, 1, 1, 1, 1, 1, 1, 1,-1, 1,-1, 1,-1,-1, 1, 1, 1,-1, 1, 1,-1,-1,-1,
    -1, 1, 1,-1, 1, 1,-1, 1,-1, 1, 1,-1,-1, 1,-1, 1, 1, 1, 1,-1,-1,-1,-1,-1, 1,-1, 1, 1, 1, 1,-1, 1,
    -1,-1, 1,-1,-1,-1, 1,-1,-1,-1, 1,-1,-1,-1, 1, 1, 1,-1,-1, 1, 1, 1,-1,-1, 1, 1,-1, 1, 1,-1, 1,-1,
    -1, 1, 1,-1, 1,-1, 1,-1, 1, 1, 1, 1,-1, 1,-1, 1, 1,-1, 1, 1,-1,-1,-1,-1,-1, 1, 1,-1, 1, 1,-1, 1};
static const float S2[128] = {
     1, 1, 1, 1,-1, 1, 1,-1, 1,-1,-1,-1, 1,-1,-1,-1, 1, 1,-1,-1, 1,-1, 1,-1, 1,-1,-1, 1,-1, 1, 1, 1,
     1, 1,-1,-1,-1, 1,-1,-1,-1,-1,-1,-1, 1, 1, 1,-1, 1,-1, 1, 1, 1,-1,-1, 1,-1,-1,-1,-1,-1,-1, 1, 1,
     1,-1, 1,-1,-1,-1,-1, 1,-1, 1,-1, 1,-1,-1, 1, 1,-1, 1,-1, 1, 1,-1, 1,-1,-1,-1,-1, 1,-1,-1, 1,-1,
     1,-1, 1, 1, 1,-1,-1, 1,-1, 1,-1, 1, 1,-1,-1, 1,-1, 1,-1, 1, 1,-1, 1,-1, 1,-1,-1,-1,-1,-1, 1,-1};
static const int8_t I4[16] = {-127, -96, -75, -58, -44, -31, -18, -6, 6, 18, 31, 44, 58, 75, 96, 127};
static const int8_t I3[8] = {-127, -79, -45, -14, 14, 45, 79, 127};
static const float M4[15] = {-0.212203f, -0.162947f, -0.127026f, -0.097164f, -0.070671f, -0.046174f, -0.022824f, 0.f,
                             0.022824f, 0.046174f, 0.070671f, 0.097164f, 0.127026f, 0.162947f, 0.212203f};
static const float M3[7] = {-0.154496f, -0.092804f, -0.044243f, 0.f, 0.044243f, 0.092804f, 0.154496f};
/* kernels.cuh:1135: float / float, evaluated in binary32 */
static float K4(void) { volatile float a = 0.241529f, b = 127.f; return a / b; }
static float K3(void) { volatile float a = 0.190207f, b = 127.f; return a / b; }

void orc_tq_tables(float* s1, float* s2, int8_t* i4, int8_t* i3, float* k43, float* m4, float* m3) {
    memcpy(s1, S1, sizeof S1); memcpy(s2, S2, sizeof S2);
    memcpy(i4, I4, sizeof I4); memcpy(i3, I3, sizeof I3);
    k43[0] = K4(); k43[1] = K3();
    memcpy(m4, M4, sizeof M4); memcpy(m3, M3, sizeof M3);
}

/* ---- fp16 rounding (IEEE binary16, round to nearest even), used by the precision model ---- */
static uint16_t f2h_bits(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);                  /* rounds to >= 65520: inf */
    if (ax < 0x38800000u) {                                                    /* result subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;                           /* < 2^-25: rounds to 0 */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        int e = (int)(ax >> 23);                                               /* 102..112 */
        int sh = 126 - e;                                                      /* value = m * 2^(e-150); unit 2^-24 */
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 112, m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13), rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}
static float h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff, x;
    if (e == 0) {
        if (!m) x = sign;
        else { float v = (float)m * (1.0f / 16777216.0f); return sign ? -v : v; }
    } else if (e == 31) x = sign | 0x7f800000u | (m << 13);
    else x = sign | ((e + 112) << 23) | (m << 13);
    float f; memcpy(&f, &x, 4); return f;
}
float orc_round_f16(float x) { return h2f(f2h_bits(x)); }
void orc_round_f16_array(const float* x, float* y, long n) { for (long i = 0; i < n; i++) y[i] = orc_round_f16(x[i]); }

/* ---- int8 quantize-append: kernels.cuh:1227-1235 ----
 * mk = max|x| over the row; sk = mk > 0 ? mk/127 : 1; q = round-half-even(x / sk). */
void orc_int8_quant_row(const float* x, int8_t* q, float* scale) {
    float mk = 0.f;
    for (int d = 0; d < AHD; d++) { float a = fabsf(x[d]); if (a > mk) mk = a; }
    const float sk = mk > 0.f ? mk / 127.f : 1.f;
    for (int d = 0; d < AHD; d++) q[d] = (int8_t)(int)rintf(x[d] / sk);
    *scale = sk;
}

/* ---- 32-lane xor butterfly sum (kernels.cuh:13-16, warp_sum), simulated lane by lane ---- */
static float warp_sum32(const float* v32) {
    float a[32], b[32];
    memcpy(a, v32, sizeof a);
    for (int o = 16; o; o >>= 1) {
        for (int i = 0; i < 32; i++) b[i] = a[i] + a[i ^ o];
        memcpy(a, b, sizeof a);
    }
    return a[0];
}
/* ---- tq_half_sum: kernels.cuh:1161-1169: four 32-lane sums, then ((s0 + s1) + s2) + s3 ---- */
float orc_tq_half_sum(const float* v128) {
    float s[4];
    for (int w = 0; w < 4; w++) s[w] = warp_sum32(v128 + 32 * w);
    return s[0] + s[1] + s[2] + s[3];
}

/* ---- tq_wht: kernels.cuh:1143-1159. One 128-value half: signs, butterfly stages h = 1..16 within each group of
 * 32 (lane with bit h set: partner - own; else own + partner), stages 32 and 64 (a+b, a-b), times 1/sqrt(128)
 * as a float constant, times the second sign table. dir 0 forward (S1 then S2), 1 inverse (S2 then S1). */
static void wht_half(const float* x, float* y, int dir) {
    float v[128], t[128];
    const float *sa = dir ? S2 : S1, *sb = dir ? S1 : S2;
    for (int j = 0; j < 128; j++) v[j] = x[j] * sa[j];
    for (int h = 1; h < 32; h <<= 1) {
        for (int j = 0; j < 128; j++) {
            const float o = v[j ^ h];
            t[j] = (j & h) ? o - v[j] : v[j] + o;
        }
        memcpy(v, t, sizeof v);
    }
    for (int h = 32; h < 128; h <<= 1)
        for (int j = 0; j < 128; j++)
            if (!(j & h)) { const float a = v[j], b = v[j + h]; v[j] = a + b; v[j + h] = a - b; }
    for (int j = 0; j < 128; j++) { const float s = v[j] * 0.08838834764831845f; y[j] = s * sb[j]; }
}
void orc_tq_wht(const float* x, float* y, int dir) { wht_half(x, y, dir); wht_half(x + 128, y + 128, dir); }

/* ---- tq_quant<BITS>: kernels.cuh:1172-1183 (per 128-value half) ---- */
static void tq_quant_half(const float* x, int bits, int* idx, float* norm_out) {
    float sq[128], xn[128], r[128], c[128];
    for (int j = 0; j < 128; j++) sq[j] = x[j] * x[j];
    const float n = sqrtf(orc_tq_half_sum(sq));
    for (int j = 0; j < 128; j++) xn[j] = n > 1e-20f ? x[j] / n : 0.f;
    wht_half(xn, r, 0);
    const float kq = bits == 4 ? K4() : K3();
    for (int j = 0; j < 128; j++) {
        int k = 0;
        if (bits == 4) { for (int i = 0; i < 15; i++) k += r[j] >= M4[i]; }
        else           { for (int i = 0; i < 7; i++)  k += r[j] >= M3[i]; }
        idx[j] = k;
        c[j] = (float)(bits == 4 ? I4[k] : I3[k]) * kq;
    }
    for (int j = 0; j < 128; j++) sq[j] = c[j] * c[j];
    const float rn = sqrtf(orc_tq_half_sum(sq));
    *norm_out = rn > 1e-20f ? n / rn : n;
}
void orc_tq_quant(const float* x, int bits, int* idx, float* norms) {
    tq_quant_half(x, bits, idx, norms);
    tq_quant_half(x + 128, bits, idx + 128, norms + 1);
}

/* ---- turbo packing: kernels.cuh:1210-1226 ----
 * K: byte b*64 + j/2 = idx[j] | idx[j+1] << 4 (j even, within half b).
 * V: low 2 bits of dim j of half b at byte b*32 + j/4, bit 2(j&3); high bit at byte 64 + b*16 + j/8, bit j&7. */
void orc_turbo_pack(const int* ik, const int* iv, uint8_t* kb, uint8_t* vb) {
    memset(kb, 0, TQ_KB); memset(vb, 0, TQ_VB);
    for (int b = 0; b < 2; b++)
        for (int j = 0; j < 128; j++) {
            const int d = b * 128 + j;
            kb[b * 64 + j / 2] |= (uint8_t)((ik[d] & 15) << (4 * (j & 1)));
            vb[b * 32 + j / 4] |= (uint8_t)((iv[d] & 3) << (2 * (j & 3)));
            vb[64 + b * 16 + j / 8] |= (uint8_t)(((iv[d] >> 2) & 1) << (j & 7));
        }
}
void orc_turbo_unpack(const uint8_t* kb, const uint8_t* vb, int* ik, int* iv) {
    for (int b = 0; b < 2; b++)
        for (int j = 0; j < 128; j++) {
            const int d = b * 128 + j;
            ik[d] = (kb[b * 64 + j / 2] >> (4 * (j & 1))) & 15;
            iv[d] = ((vb[b * 32 + j / 4] >> (2 * (j & 3))) & 3) | (((vb[64 + b * 16 + j / 8] >> (j & 7)) & 1) << 2);
        }
}
/* One (kv head, position) row: post-RoPE k and raw v -> codes + norms (kernels.cuh:1210-1226). */
void orc_turbo_quant_row(const float* k, const float* v, uint8_t* kb, uint8_t* vb, float* kn, float* vn) {
    int ik[AHD], iv[AHD];
    orc_tq_quant(k, 4, ik, kn);
    orc_tq_quant(v, 3, iv, vn);
    orc_turbo_pack(ik, iv, kb, vb);
}

/* ---- KV append of T tokens (kernels.cuh:1185-1236, the KV-head blocks): row kvh*max_t + pos0 + t.
 * k, v: post-RoPE keys and raw values, token stride ld floats, head kvh at offset kvh*AHD. */
void orc_kv_append(const float* k, const float* v, long ld, int T, int KV, int pos0, int max_t, int turbo,
                   int8_t* ck, int8_t* cv, float* cks, float* cvs) {
    for (int t = 0; t < T; t++)
        for (int h = 0; h < KV; h++) {
            const float *kr = k + (size_t)t * ld + h * AHD, *vr = v + (size_t)t * ld + h * AHD;
            const size_t row = (size_t)h * max_t + pos0 + t;
            if (turbo) orc_turbo_quant_row(kr, vr, (uint8_t*)ck + row * TQ_KB, (uint8_t*)cv + row * TQ_VB, cks + row * 2, cvs + row * 2);
            else { orc_int8_quant_row(kr, ck + row * AHD, cks + row); orc_int8_quant_row(vr, cv + row * AHD, cvs + row); }
        }
}

/* ---- dequantized cache rows in double (the value the kernels' arithmetic approximates) ----
 * int8: k = q * ks (the scale applied to the score, kernels.cuh:1273,1779); turbo: code * K * half norm
 * (kernels.cuh:1265-1268, 1303-1306). */
static void key_row(const int8_t* ck, const float* cks, size_t row, int turbo, double* out) {
    if (!turbo) { for (int d = 0; d < AHD; d++) out[d] = (double)ck[row * AHD + d] * (double)cks[row]; return; }
    const uint8_t* kb = (const uint8_t*)ck + row * TQ_KB;
    const double kq = K4();
    for (int d = 0; d < AHD; d++) {
        const int b = d >> 7, j = d & 127;
        const int ix = (kb[b * 64 + j / 2] >> (4 * (j & 1))) & 15;
        out[d] = (double)I4[ix] * kq * (double)cks[row * 2 + b];
    }
}
static void val_row(const int8_t* cv, const float* cvs, size_t row, int turbo, double* out) {
    if (!turbo) { for (int d = 0; d < AHD; d++) out[d] = (double)cv[row * AHD + d] * (double)cvs[row]; return; }
    const uint8_t* vb = (const uint8_t*)cv + row * TQ_VB;
    const double kq = K3();
    for (int d = 0; d < AHD; d++) {
        const int b = d >> 7, j = d & 127;
        const int ix = ((vb[b * 32 + j / 4] >> (2 * (j & 3))) & 3) | (((vb[64 + b * 16 + j / 8] >> (j & 7)) & 1) << 2);
        out[d] = (double)I3[ix] * kq * (double)cvs[row * 2 + b];
    }
}
/* exact (double) inverse rotation of one 256-row: S1 . H . S2 / sqrt(128) per half */
static void wht_inv_f64(const double* x, double* y) {
    for (int b = 0; b < 2; b++) {
        double v[128];
        for (int j = 0; j < 128; j++) v[j] = x[b * 128 + j] * S2[j];
        for (int h = 1; h < 128; h <<= 1)
            for (int j = 0; j < 128; j++)
                if (!(j & h)) { const double a = v[j], c = v[j + h]; v[j] = a + c; v[j + h] = a - c; }
        for (int j = 0; j < 128; j++) y[b * 128 + j] = v[j] / sqrt(128.0) * S1[j];
    }
}

/* ---- fp64 reference attention for one output row (token t, query head h).
 * tests/test_fa.cu:59-80: s_j = q.k_j * ks_j / sqrt(256), softmax over keys 0..pos0+t, sum of e_j v_j vs_j,
 * divided by l, times sigmoid(gate). Turbo (kernels.cuh:1238-1315, 1730-1738): dequantized codes, the output
 * rotated back (inverse WHT) before the gate. gate == NULL: no gate (and for turbo no inverse rotation:
 * the raw attention output in the rotated domain, what attn_fa writes when q_gate is null). */
void orc_attn_row_f64(const float* qo, const float* gate, long ld, int H, int KV,
                      const int8_t* ck, const int8_t* cv, const float* cks, const float* cvs, int max_t, int turbo,
                      int pos0, int t, int h, double* out) {
    const int kvh = h / (H / KV), p = pos0 + t;
    const float* q = qo + ((size_t)t * H + h) * AHD;
    double* s = (double*)malloc(sizeof(double) * (size_t)(p + 1));
    double kr[AHD], vr[AHD], acc[AHD];
    double m = -1e300;
    for (int j = 0; j <= p; j++) {
        key_row(ck, cks, (size_t)kvh * max_t + j, turbo, kr);
        double d = 0;
        for (int i = 0; i < AHD; i++) d += (double)q[i] * kr[i];
        s[j] = d / 16.0;
        if (s[j] > m) m = s[j];
    }
    double l = 0;
    for (int i = 0; i < AHD; i++) acc[i] = 0;
    for (int j = 0; j <= p; j++) {
        const double e = exp(s[j] - m);
        l += e;
        val_row(cv, cvs, (size_t)kvh * max_t + j, turbo, vr);
        for (int i = 0; i < AHD; i++) acc[i] += e * vr[i];
    }
    free(s);
    for (int i = 0; i < AHD; i++) acc[i] /= l;
    if (gate == NULL) { memcpy(out, acc, sizeof acc); return; }
    if (turbo) { double r[AHD]; wht_inv_f64(acc, r); memcpy(acc, r, sizeof acc); }
    for (int i = 0; i < AHD; i++) {
        const double g = gate[(size_t)t * ld + h * 2 * AHD + AHD + i];
        out[i] = acc[i] / (1.0 + exp(-g));
    }
}
/* many rows: rows[2*i] = token, rows[2*i+1] = head; out: nrows x 256 */
void orc_attn_rows_f64(const float* qo, const float* gate, long ld, int H, int KV,
                       const int8_t* ck, const int8_t* cv, const float* cks, const float* cvs, int max_t, int turbo,
                       int pos0, const int* rows, int nrows, double* out) {
    for (int r = 0; r < nrows; r++)
        orc_attn_row_f64(qo, gate, ld, H, KV, ck, cv, cks, cvs, max_t, turbo, pos0, rows[2 * r], rows[2 * r + 1], out + (size_t)r * AHD);
}

/* ---- precision model of attn_fa_k (int8 and turbo), one output row. Not a parity target.
 * kernels.cuh:1508 Q rounded to fp16; :1513 sl2 = rsqrtf(256) * log2(e); :1620-1632 S scaled by K scale * sl2,
 * causal mask; base-2 online softmax over 64-key tiles; :1656-1661 P * V scale rounded to fp16; P.V and Q.K
 * accumulated in fp32 (here: exactly, in double, then rounded per tile), :1680-1690 O / l * sigmoid(g).
 * Turbo (:1587-1612): S = (S0 * n0 / n1 + S1) * n1 * K4 * sl2, P carries V's half norm * K3. */
void orc_attn_row_fa_emul(const float* qo, const float* gate, long ld, int H, int KV,
                          const int8_t* ck, const int8_t* cv, const float* cks, const float* cvs, int max_t, int turbo,
                          int pos0, int t, int h, double* out) {
    const int kvh = h / (H / KV), p = pos0 + t;
    const float* q = qo + ((size_t)t * H + h) * AHD;
    float q16[AHD];
    for (int i = 0; i < AHD; i++) q16[i] = orc_round_f16(q[i]);
    const float sl2 = (1.0f / 16.0f) * 1.4426950408889634f;
    const float k4 = K4(), k3 = K3();
    float m = -INFINITY, l = 0.f;
    double o[AHD];
    for (int i = 0; i < AHD; i++) o[i] = 0;
    for (int k0 = 0; k0 <= p; k0 += 64) {
        const int n = (p + 1 - k0) < 64 ? p + 1 - k0 : 64;
        float s[64], mx = -INFINITY;
        for (int j = 0; j < n; j++) {
            const size_t row = (size_t)kvh * max_t + k0 + j;
            if (!turbo) {
                double d = 0;
                for (int i = 0; i < AHD; i++) d += (double)q16[i] * (double)ck[row * AHD + i];
                s[j] = (float)d * (cks[row] * sl2);
            } else {
                const uint8_t* kb = (const uint8_t*)ck + row * TQ_KB;
                double d0 = 0, d1 = 0;
                for (int i = 0; i < AHD; i++) {
                    const int b = i >> 7, jj = i & 127;
                    const int ix = (kb[b * 64 + jj / 2] >> (4 * (jj & 1))) & 15;
                    const double pr = (double)q16[i] * (double)I4[ix];
                    if (b) d1 += pr; else d0 += pr;
                }
                const float n0 = cks[row * 2], n1 = fmaxf(cks[row * 2 + 1], 1e-30f);
                s[j] = ((float)d0 * (n0 / n1) + (float)d1) * (n1 * k4 * sl2);
            }
            if (s[j] > mx) mx = s[j];
        }
        const float mn = fmaxf(m, mx), c = exp2f(m - mn);
        m = mn; l *= c;
        for (int i = 0; i < AHD; i++) o[i] *= c;
        for (int j = 0; j < n; j++) {
            const size_t row = (size_t)kvh * max_t + k0 + j;
            const float e = exp2f(s[j] - mn);
            l += e;
            if (!turbo) {
                const float pv = orc_round_f16(e * cvs[row]);
                for (int i = 0; i < AHD; i++) o[i] += (double)pv * (double)cv[row * AHD + i];
            } else {
                const uint8_t* vb = (const uint8_t*)cv + row * TQ_VB;
                const float p0 = orc_round_f16(e * (cvs[row * 2] * k3)), p1 = orc_round_f16(e * (cvs[row * 2 + 1] * k3));
                for (int i = 0; i < AHD; i++) {
                    const int b = i >> 7, jj = i & 127;
                    const int ix = ((vb[b * 32 + jj / 4] >> (2 * (jj & 3))) & 3) | (((vb[64 + b * 16 + jj / 8] >> (jj & 7)) & 1) << 2);
                    o[i] += (double)(b ? p1 : p0) * (double)I3[ix];
                }
            }
        }
        for (int i = 0; i < AHD; i++) o[i] = (float)o[i];  /* fp32 accumulators between tiles */
    }
    double acc[AHD];
    for (int i = 0; i < AHD; i++) acc[i] = o[i] / l;
    if (gate == NULL) { memcpy(out, acc, sizeof acc); return; }
    if (turbo) { double r[AHD]; wht_inv_f64(acc, r); memcpy(acc, r, sizeof acc); }
    for (int i = 0; i < AHD; i++) out[i] = acc[i] / (1.0 + exp(-(double)gate[(size_t)t * ld + h * 2 * AHD + AHD + i]));
}
void orc_attn_rows_fa_emul(const float* qo, const float* gate, long ld, int H, int KV,
                           const int8_t* ck, const int8_t* cv, const float* cks, const float* cvs, int max_t, int turbo,
                           int pos0, const int* rows, int nrows, double* out) {
    for (int r = 0; r < nrows; r++)
        orc_attn_row_fa_emul(qo, gate, ld, H, KV, ck, cv, cks, cvs, max_t, turbo, pos0, rows[2 * r], rows[2 * r + 1], out + (size_t)r * AHD);
}

/* ---- query/key front (kernels.cuh:1185-1209; ref/qwen36_ref.py:62-76): RMSNorm(1 + w) then partial RoPE on
 * dims < rot (rotate-half pairs d, d + rot/2), angle pos * theta^(-2j/rot). Double precision; turbo queries are then
 * rotated forward (tq_wht). Tolerance parity only. w: fp16 bits of the norm weight. */
void orc_qk_norm_rope_row(const float* x, const uint16_t* w, int pos, int rot, float theta, float eps, int wht_fwd, float* out) {
    double ss = 0, y[AHD], z[AHD];
    for (int d = 0; d < AHD; d++) ss += (double)x[d] * x[d];
    const double r = 1.0 / sqrt(ss / AHD + (double)eps);
    for (int d = 0; d < AHD; d++) y[d] = x[d] * r * (1.0 + (double)h2f(w[d]));
    memcpy(z, y, sizeof y);
    const int h2 = rot / 2;
    for (int j = 0; j < h2; j++) {
        const double ang = (double)pos * pow((double)theta, -2.0 * j / rot), cs = cos(ang), sn = sin(ang);
        z[j] = y[j] * cs - y[j + h2] * sn;
        z[j + h2] = y[j + h2] * cs + y[j] * sn;
    }
    if (!wht_fwd) { for (int d = 0; d < AHD; d++) out[d] = (float)z[d]; return; }
    for (int b = 0; b < 2; b++) {  /* exact forward rotation S2 . H . S1 / sqrt(128) */
        double v[128];
        for (int j = 0; j < 128; j++) v[j] = z[b * 128 + j] * S1[j];
        for (int h = 1; h < 128; h <<= 1)
            for (int j = 0; j < 128; j++)
                if (!(j & h)) { const double a = v[j], c = v[j + h]; v[j] = a + c; v[j + h] = a - c; }
        for (int j = 0; j < 128; j++) out[b * 128 + j] = (float)(v[j] / sqrt(128.0) * S2[j]);
    }
}

/* ---- dense int8 projections (the attention's qkv and o projections: kernels.cuh:186-196 Mat, :98-141 gemv_i8,
 * :143-156 quantize_rows_i8_k, :250-337 gemm) ---- */

/* quantize_rows_i8_k (kernels.cuh:144-156): fp16 rows [O][I] -> int8 [O][I] + a scale per row, absmax / 127
 * (1 for an all-zero row), q = round-half-even(w / scale) with the IEEE binary32 quotient. */
void orc_quantize_rows_i8(const uint16_t* W, long O, long I, int8_t* q, float* s) {
    for (long o = 0; o < O; o++) {
        const uint16_t* wr = W + o * I;
        float m = 0.f;
        for (long i = 0; i < I; i++) { const float a = fabsf(h2f(wr[i])); if (a > m) m = a; }
        const float sc = m > 0.f ? m / 127.f : 1.f;
        for (long i = 0; i < I; i++) q[o * I + i] = (int8_t)(int)rintf(h2f(wr[i]) / sc);
        s[o] = sc;
    }
}

/* The exact product y[t][o] = s[o] * sum_i q[o][i] * x[t][i], summed in fp64 and rounded once
 * (tests/test_kernels.cu:373: the reference's "exact int8 reference" of gemv_i8). */
void orc_dense_i8_f64(const int8_t* q, const float* s, const float* x, long S, long I, long O, double* y) {
    for (long t = 0; t < S; t++)
        for (long o = 0; o < O; o++) {
            double a = 0;
            for (long i = 0; i < I; i++) a += (double)q[o * I + i] * x[t * I + i];
            y[t * O + o] = a * s[o];
        }
}

/* The prefill GEMM's rounding points (kernels.cuh:306-307: activations to fp16; the int8 weights are exact in
 * fp16; fp32 accumulation, here exact in fp64): y = s[o] * sum_i q[o][i] * fp16(x[t][i]). */
void orc_dense_i8_fp16x(const int8_t* q, const float* s, const float* x, long S, long I, long O, double* y) {
    for (long t = 0; t < S; t++)
        for (long o = 0; o < O; o++) {
            double a = 0;
            for (long i = 0; i < I; i++) a += (double)q[o * I + i] * orc_round_f16(x[t * I + i]);
            y[t * O + o] = a * s[o];
        }
}

/* ---- the other dense forms (struct Mat, kernels.cuh:186-196): int4 gs64, int6 gs64, fp16 ---- */

/* quantize_rows_q4_k (kernels.cuh:576-590): per 64-input group scale = absmax / 7 (1 for a zero group),
 * q = clamp(round-half-even(w / scale), -8, 7); weight i in bits 4 (i % 2) of byte i / 2 (low nibble first). */
void orc_quantize_rows_q4(const uint16_t* W, long O, long I, uint8_t* q, float* s) {
    memset(q, 0, (size_t)O * (I / 2));
    for (long o = 0; o < O; o++)
        for (long g = 0; g < I / 64; g++) {
            const uint16_t* w = W + o * I + g * 64;
            float m = 0.f;
            for (int i = 0; i < 64; i++) { const float a = fabsf(h2f(w[i])); if (a > m) m = a; }
            const float sc = m > 0.f ? m / 7.f : 1.f;
            for (int i = 0; i < 64; i++) {
                int v = (int)rintf(h2f(w[i]) / sc);
                v = v < -8 ? -8 : v > 7 ? 7 : v;
                q[o * (I / 2) + (g * 64 + i) / 2] |= (uint8_t)((v & 15) << (4 * (i & 1)));
            }
            s[o * (I / 64) + g] = sc;
        }
}

/* quantize_rows_q6_k (kernels.cuh:552-573): scale = group absmax / 31 (1 for a zero group), u = clamp(round-half-
 * even(w / scale), -32, 31) + 32; the low 4 bits in q as q4's nibbles, the high 2 bits at bits 2 (i % 4) of byte
 * i / 4 of qh. */
void orc_quantize_rows_q6(const uint16_t* W, long O, long I, uint8_t* q, uint8_t* qh, float* s) {
    memset(q, 0, (size_t)O * (I / 2));
    memset(qh, 0, (size_t)O * (I / 4));
    for (long o = 0; o < O; o++)
        for (long g = 0; g < I / 64; g++) {
            const uint16_t* w = W + o * I + g * 64;
            float m = 0.f;
            for (int i = 0; i < 64; i++) { const float a = fabsf(h2f(w[i])); if (a > m) m = a; }
            const float sc = m > 0.f ? m / 31.f : 1.f;
            for (int i = 0; i < 64; i++) {
                const int u = (int)fminf(31.f, fmaxf(-32.f, rintf(h2f(w[i]) / sc))) + 32;
                const long k = g * 64 + i;
                q[o * (I / 2) + k / 2] |= (uint8_t)((u & 15) << (4 * (i & 1)));
                qh[o * (I / 4) + k / 4] |= (uint8_t)((u >> 4) << (2 * (i & 3)));
            }
            s[o * (I / 64) + g] = sc;
        }
}

/* weight i of row o of a matrix in form fmt (1: int4 gs64, 2: int6 gs64, 3: fp16) as its integer code times the
 * group scale (the exact value, fp64) */
static double mat_w(int fmt, const void* w, const uint8_t* wh, const float* s, long I, long o, long i) {
    if (fmt == 3) return h2f(((const uint16_t*)w)[o * I + i]);
    const uint8_t b = ((const uint8_t*)w)[o * (I / 2) + i / 2];
    const int nib = (b >> (4 * (i & 1))) & 15;
    int v;
    if (fmt == 1) v = nib >= 8 ? nib - 16 : nib;
    else v = (nib | (((wh[o * (I / 4) + i / 4] >> (2 * (i & 3))) & 3) << 4)) - 32;
    return (double)v * (double)s[o * (I / 64) + i / 64];
}

/* y[t][o] = sum_i w[o][i] * x[t][i] with the exact weights, fp64 (tests/test_kernels.cu:415-423: the reference's
 * "exact int4 math" of gemv_q4). */
void orc_dense_mat_f64(int fmt, const void* w, const uint8_t* wh, const float* s, const float* x, long S, long I,
                       long O, double* y) {
    for (long t = 0; t < S; t++)
        for (long o = 0; o < O; o++) {
            double a = 0;
            for (long i = 0; i < I; i++) a += mat_w(fmt, w, wh, s, I, o, i) * x[t * I + i];
            y[t * O + o] = a;
        }
}

/* The GEMMs' rounding points: an int4 / int6 weight is q * scale in fp32, then fp16 (kernels.cuh:276-279,
 * 313-317); fp16 weights as stored; activations rounded to fp16 (:306-307); exact sums in fp64. */
void orc_dense_mat_fp16x(int fmt, const void* w, const uint8_t* wh, const float* s, const float* x, long S, long I,
                         long O, double* y) {
    for (long t = 0; t < S; t++)
        for (long o = 0; o < O; o++) {
            double a = 0;
            for (long i = 0; i < I; i++) {
                const float wf = fmt == 3 ? (float)mat_w(fmt, w, wh, s, I, o, i) : orc_round_f16((float)mat_w(fmt, w, wh, s, I, o, i));
                a += (double)wf * orc_round_f16(x[t * I + i]);
            }
            y[t * O + o] = a;
        }
}
