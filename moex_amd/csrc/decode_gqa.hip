// Split-K GQA decode / MTP-verify attention on gfx950 (replaces attn_gqa_k, kernels.cuh:1740-1844).
//
// One workgroup = (kv head, key split, query token), 4 wavefronts. The 8 query heads of the group share every K/V
// read. Each wavefront takes 32-key steps of the split (step j -> wavefront j % 4), reads K and V rows straight from
// HBM into registers (no LDS staging), widens them to fp16 and runs both products on v_mfma_f32_16x16x32_f16:
//
//   S[key][c] = K[key][:] . Qx[c][:]   16 keys x 16 columns; column c = (head c/2, part c&1) where Q = Qhi + Qlo,
//                                      Qhi = fp16(q), Qlo = fp16(q - Qhi): the two parts are added after the MFMA,
//                                      so the score keeps ~22 mantissa bits (the reference decode is fp32).
//   O[c][dim] += Px[c][key] . V[key][dim]   with Px the same hi/lo split of p * vscale (scaled by a power of two so
//                                      the largest value of the split is in [1, 2): no fp16 underflow).
//
// The MFMA contraction index is permuted consistently on both operands (the sums do not care):
//   S MFMA s (0..7), lane group g = lane/16, slot j: dim = 128*(s/4) + 32*g + 8*(s%4) + j  (each MFMA within one
//     128-half, so the turbo half norms apply per MFMA);
//   S output (16x16 D layout): lane holds keys 16*grp + 4*g + i (i = 0..3, grp = two 16-key groups) for column
//     lane%16, which is exactly the key order of the P.V A operand slots j = 4*grp + i;
//   P.V MFMA c (0..15): output column m = lane%16 is dim 128*(c/8) + 8*m + c%8 (one 128-half per MFMA).
// Softmax is base 2; the partial written per (token, head, split) is {m (log2 units), l, acc[256]}.
#include "common.hpp"

namespace moex {

namespace {

constexpr float SL2 = 0.0625f * 1.4426950408889634f;  // 1/sqrt(256) * log2(e)
constexpr float TK4 = 0.241529f / 127.f, TK3 = 0.190207f / 127.f;

// biased (code + 128) TurboQuant centroid codes, 4 per dword: K (16 entries), V (8 entries)
// I4 = {-127,-96,-75,-58,-44,-31,-18,-6,6,18,31,44,58,75,96,127}, I3 = {-127,-79,-45,-14,14,45,79,127}
constexpr uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a + 128) | ((uint32_t)(b + 128) << 8) | ((uint32_t)(c + 128) << 16) | ((uint32_t)(d + 128) << 24);
}
constexpr uint32_t K4T0 = pack4(-127, -96, -75, -58), K4T1 = pack4(-44, -31, -18, -6);
constexpr uint32_t K4T2 = pack4(6, 18, 31, 44), K4T3 = pack4(58, 75, 96, 127);
constexpr uint32_t V3T0 = pack4(-127, -79, -45, -14), V3T1 = pack4(14, 45, 79, 127);

// 4 nibble indices (one per byte, values 0..15) -> 4 biased K codes
__device__ __forceinline__ uint32_t lut16(uint32_t idx) {
    const uint32_t s = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(K4T1, K4T0, s), hi = __builtin_amdgcn_perm(K4T3, K4T2, s);
    const uint32_t mask = ((idx >> 3) & 0x01010101u) * 0xffu;
    return (hi & mask) | (lo & ~mask);
}
// 8 nibbles of a dword -> two half8 halves: dims 0..7 as fp16 (biased-code magic)
__device__ __forceinline__ half8_t nib8_to_h8(uint32_t x) {
    const uint32_t even = x & 0x0f0f0f0fu, odd = (x >> 4) & 0x0f0f0f0fu;  // dims 0,2,4,6 / 1,3,5,7
    const uint32_t be = lut16(even), bo = lut16(odd);
    // interleave to dims order: bytes (e0 o0 e1 o1) (e2 o2 e3 o3)
    const uint32_t d01 = __builtin_amdgcn_perm(bo, be, 0x05010400u), d23 = __builtin_amdgcn_perm(bo, be, 0x07030602u);
    uint32_t r0, r1, r2, r3;
    biased4_to_h4(d01, r0, r1);
    biased4_to_h4(d23, r2, r3);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 u = {r0, r1, r2, r3};
    return __builtin_bit_cast(half8_t, u);
}

__device__ __forceinline__ half8_t q_part8(const float* q, int part) {  // 8 floats -> hi or lo fp16 parts
    half8_t r;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const _Float16 hi = (_Float16)q[j];
        r[j] = part ? (_Float16)(q[j] - (float)hi) : hi;
    }
    return r;
}

// ---- work-item mapping: blocks are dispatched round-robin over the 8 XCDs (block b -> XCD b % 8); renumber so
// that consecutive work items (the T tokens of a split, then neighbouring splits) land on the same XCD and share
// its L2.
__device__ __forceinline__ int xcd_work_id(int b, int nb) {
    const int q = nb >> 3, r = nb & 7, x = b & 7, i = b >> 3;
    return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + i;
}
}  // namespace

template <bool TB>
__global__ void __launch_bounds__(256, 2) gqa_decode_kernel(const float* __restrict__ qo, moex_kv_cache kv, int H,
                                                            const int* __restrict__ pos_d, int max_t,
                                                            float* __restrict__ part, int T, int ns) {
    __shared__ float red[8];
    __shared__ __align__(16) float ow[4][GQ][AHD];  // per-wavefront partial O, merged at the end
    __shared__ float mw[4][GQ], lw[4][GQ];
    const int nb = gridDim.x, w_id = xcd_work_id(blockIdx.x, nb);
    const int tok = w_id % T, s = (w_id / T) % ns, kvh = w_id / (T * ns);
    const int pos0 = *pos_d, Tk = pos0 + tok + 1, Tmax = pos0 + T;
    const int L = (Tmax + ns - 1) / ns, lo = s * L, hi = min(Tk, lo + L);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 4, m16 = lane & 15;
    const size_t rbase = (size_t)kvh * max_t;

    // V scale normalizer: a power of two putting the split's largest V scale in [1, 2)
    float vmax = 0.f;
    for (int t = lo + tid; t < hi; t += 256) {
        if (TB) vmax = fmaxf(vmax, fmaxf(kv.vs[(rbase + t) * 2], kv.vs[(rbase + t) * 2 + 1]) * TK3);
        else vmax = fmaxf(vmax, kv.vs[rbase + t]);
    }
#pragma unroll
    for (int o = 32; o; o >>= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, o));
    if (lane == 0) red[wv] = vmax;
    __syncthreads();
    vmax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int ex = 0;
    if (vmax > 0.f) (void)frexpf(vmax, &ex);  // vmax = f * 2^ex, f in [0.5, 1)
    const float vnorm = ldexpf(1.f, 1 - ex), vdenorm = ldexpf(1.f, ex - 1);

    // Q operands: column c = lane%16 -> head hq = c/2, part c&1; MFMA s reads dims 128*(s/4) + 32*g + 8*(s%4) + 0..7
    const int hq = m16 >> 1, qpart = m16 & 1;
    half8_t qf[8];
    {
        const float* qrow = qo + ((size_t)tok * H + kvh * GQ + hq) * AHD;
#pragma unroll
        for (int sidx = 0; sidx < 8; sidx++) {
            const float4* p4 = reinterpret_cast<const float4*>(qrow + 128 * (sidx >> 2) + 32 * g + 8 * (sidx & 3));
            const float4 a = p4[0], b = p4[1];
            const float qv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            qf[sidx] = q_part8(qv, qpart);
        }
    }

    float4_t o[16];
#pragma unroll
    for (int c = 0; c < 16; c++) o[c] = float4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;  // head hq's running max (log2) and this lane's part of the sum

    const int nsteps = hi > lo ? (hi - lo + 31) >> 5 : 0;
    for (int step = wv; step < nsteps; step += 4) {
        const int k0 = lo + step * 32;
        // ---- loads: K for the two 16-key groups (key k0 + 16*grp + m16), V and scales for the 8 slot keys ----
        uint4 kr[2][4];
#pragma unroll
        for (int grp = 0; grp < 2; grp++) {
            const size_t row = rbase + min(k0 + 16 * grp + m16, hi - 1);
            if (TB) {
                const uint4* kp = reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(kv.k) + row * TQ_KB);
                kr[grp][0] = kp[g];      // half 0: bytes 16g .. 16g+15 = dims 32g .. 32g+31
                kr[grp][1] = kp[4 + g];  // half 1
            } else {
                const uint4* kp = reinterpret_cast<const uint4*>(kv.k + row * AHD);
                kr[grp][0] = kp[2 * g]; kr[grp][1] = kp[2 * g + 1];
                kr[grp][2] = kp[8 + 2 * g]; kr[grp][3] = kp[8 + 2 * g + 1];
            }
        }
        int skey[8];
#pragma unroll
        for (int j = 0; j < 8; j++) skey[j] = k0 + 16 * (j >> 2) + 4 * g + (j & 3);
        uint2 vr[8][2];   // int8: dims 8*m16 .. +7 of each half; turbo: [0] = (low-bit u16 of half 0, of half 1),
                          // [1] = (high-bit byte of half 0, of half 1)
        float ksc[8], vsc0[8], vsc1[8];
        float kn0[8], kn1[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const size_t row = rbase + min(skey[j], hi - 1);
            if (TB) {
                const uint8_t* vp = reinterpret_cast<const uint8_t*>(kv.v) + row * TQ_VB;
                const uint32_t l0 = *reinterpret_cast<const uint16_t*>(vp + 2 * m16);
                const uint32_t l1 = *reinterpret_cast<const uint16_t*>(vp + 32 + 2 * m16);
                vr[j][0] = make_uint2(l0, l1);
                vr[j][1] = make_uint2(vp[64 + m16], vp[80 + m16]);
                const float2 kn = *reinterpret_cast<const float2*>(kv.ks + row * 2);
                const float2 vn = *reinterpret_cast<const float2*>(kv.vs + row * 2);
                kn0[j] = kn.x; kn1[j] = kn.y;
                vsc0[j] = vn.x; vsc1[j] = vn.y;
            } else {
                const int8_t* vp = kv.v + row * AHD;
                vr[j][0] = *reinterpret_cast<const uint2*>(vp + 8 * m16);
                vr[j][1] = *reinterpret_cast<const uint2*>(vp + 128 + 8 * m16);
                ksc[j] = kv.ks[row];
                vsc0[j] = kv.vs[row];
            }
        }
        // ---- S = K . Qx: 2 groups x 8 MFMAs (turbo: halves accumulated separately) ----
        float sc[8];
#pragma unroll
        for (int grp = 0; grp < 2; grp++) {
            float4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int sidx = 0; sidx < 8; sidx++) {
                half8_t a;
                if (TB) {
                    const uint4 u = kr[grp][sidx >> 2];
                    const uint32_t wsel = (sidx & 3) == 0 ? u.x : (sidx & 3) == 1 ? u.y : (sidx & 3) == 2 ? u.z : u.w;
                    a = nib8_to_h8(wsel);
                } else {
                    const uint4 u = kr[grp][2 * (sidx >> 2) + ((sidx & 3) >> 1)];
                    a = (sidx & 1) ? i8x8_to_h8(u.z, u.w) : i8x8_to_h8(u.x, u.y);
                }
                if (TB && sidx >= 4) s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[sidx], s1, 0, 0, 0);
                else s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[sidx], s0, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int j = 4 * grp + i;
                if (TB) {
                    const float a0 = s0[i] + __shfl_xor(s0[i], 1), a1 = s1[i] + __shfl_xor(s1[i], 1);
                    sc[j] = (a0 * kn0[j] + a1 * kn1[j]) * (TK4 * SL2);
                } else {
                    sc[j] = (s0[i] + __shfl_xor(s0[i], 1)) * (ksc[j] * SL2);
                }
                if (skey[j] >= hi) sc[j] = -INFINITY;
            }
        }
        // ---- online softmax of head hq over this step's 32 keys ----
        float mt = sc[0];
#pragma unroll
        for (int j = 1; j < 8; j++) mt = fmaxf(mt, sc[j]);
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float m_new = fmaxf(m_run, mt);  // finite: every step holds at least one key < hi
        const float cfac = fast_exp2(m_run - m_new);
        m_run = m_new;
        float pv0[8], pv1[8], psum = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float p = fast_exp2(sc[j] - m_new);
            psum += p;
            if (TB) { pv0[j] = p * (vsc0[j] * TK3 * vnorm); pv1[j] = p * (vsc1[j] * TK3 * vnorm); }
            else pv0[j] = p * (vsc0[j] * vnorm);
        }
        l_run = l_run * cfac + psum;
        // rescale O rows: row 4g+i belongs to head 2g + i/2; its factor lives in lane 20g + 2*(i/2)
        if (__builtin_amdgcn_read_exec() && __ballot(cfac != 1.f)) {
            const float c0 = __shfl(cfac, 20 * g), c1 = __shfl(cfac, 20 * g + 2);
#pragma unroll
            for (int c = 0; c < 16; c++) { o[c][0] *= c0; o[c][1] *= c0; o[c][2] *= c1; o[c][3] *= c1; }
        }
        // P operands (row = column c of S: head hq, part qpart): hi / lo fp16 split
        half8_t pa0, pa1;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const _Float16 h0 = (_Float16)pv0[j];
            pa0[j] = qpart ? (_Float16)(pv0[j] - (float)h0) : h0;
            if (TB) {
                const _Float16 h1 = (_Float16)pv1[j];
                pa1[j] = qpart ? (_Float16)(pv1[j] - (float)h1) : h1;
            }
        }
        // ---- O += Px . V: 16 MFMAs, MFMA c -> dims 128*(c/8) + 8*m16 + c%8 ----
        if (TB) {
            // decode 3-bit codes of the 8 slot keys for both halves: biased bytes per (key, 4 dims)
            uint32_t vb[8][2][2];  // [key][half][dims 0..3 / 4..7]
#pragma unroll
            for (int j = 0; j < 8; j++)
#pragma unroll
                for (int hb = 0; hb < 2; hb++) {
                    const uint32_t lo16 = hb ? vr[j][0].y : vr[j][0].x, hi8 = hb ? vr[j][1].y : vr[j][1].x;
#pragma unroll
                    for (int q4 = 0; q4 < 2; q4++) {
                        uint32_t idx = 0;
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const int dd = 4 * q4 + e;
                            idx |= (((lo16 >> (2 * dd)) & 3u) | (((hi8 >> dd) & 1u) << 2)) << (8 * e);
                        }
                        vb[j][hb][q4] = __builtin_amdgcn_perm(V3T1, V3T0, idx);
                    }
                }
#pragma unroll
            for (int c = 0; c < 16; c++) {
                const int hb = c >> 3, bp = c & 7, q4 = bp >> 2, sh = 8 * (bp & 3);
                // gather byte bp of the 8 keys into biased pairs, then widen
                uint32_t w[4];
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const uint32_t a = (vb[2 * jj][hb][q4] >> sh) & 0xffu, b = (vb[2 * jj + 1][hb][q4] >> sh) & 0xffu;
                    const half2_t off = u2h2(0x64806480u);
                    w[jj] = h22u(u2h2(0x64006400u | a | (b << 16)) - off);
                }
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                const u32x4 u = {w[0], w[1], w[2], w[3]};
                o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(hb ? pa1 : pa0, __builtin_bit_cast(half8_t, u), o[c], 0, 0, 0);
            }
        } else {
            // widen each key's 2 x 8 bytes to fp16 pairs (dims 2k, 2k+1), then pick dim bp for the 8 keys
            uint32_t vh[8][2][4];
#pragma unroll
            for (int j = 0; j < 8; j++)
#pragma unroll
                for (int hb = 0; hb < 2; hb++) {
                    const uint2 u = vr[j][hb];
                    i8x4_to_h4(u.x, vh[j][hb][0], vh[j][hb][1]);
                    i8x4_to_h4(u.y, vh[j][hb][2], vh[j][hb][3]);
                }
#pragma unroll
            for (int c = 0; c < 16; c++) {
                const int hb = c >> 3, bp = c & 7, wd = bp >> 1;
                const uint32_t sel = (bp & 1) ? 0x07060302u : 0x05040100u;  // high or low halves of two dwords
                uint32_t w[4];
#pragma unroll
                for (int jj = 0; jj < 4; jj++) w[jj] = __builtin_amdgcn_perm(vh[2 * jj + 1][hb][wd], vh[2 * jj][hb][wd], sel);
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                const u32x4 u = {w[0], w[1], w[2], w[3]};
                o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa0, __builtin_bit_cast(half8_t, u), o[c], 0, 0, 0);
            }
        }
    }
    // ---- this wavefront's partial -> LDS: l summed over the 4 lane groups (same column), hi+lo rows added ----
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (g == 0 && qpart == 0) { mw[wv][hq] = m_run; lw[wv][hq] = l_run; }
#pragma unroll
    for (int c = 0; c < 16; c++) {
        const int dim = 128 * (c >> 3) + 8 * m16 + (c & 7);
        ow[wv][2 * g][dim] = o[c][0] + o[c][1];
        ow[wv][2 * g + 1][dim] = o[c][2] + o[c][3];
    }
    __syncthreads();
    // ---- merge the 4 wavefronts; thread = dim, all 8 heads ----
    const int d = tid;
#pragma unroll
    for (int h = 0; h < GQ; h++) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) if (lw[w][h] > 0.f) M = fmaxf(M, mw[w][h]);
        float l = 0.f, acc = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float f = lw[w][h] > 0.f ? fast_exp2(mw[w][h] - M) : 0.f;
            l += lw[w][h] * f;
            acc += ow[w][h][d] * f;
        }
        part_acc(part, tok, kvh * GQ + h, s, H, ns)[d] = acc * vdenorm;
        if (d == 0) {  // empty split: m = -inf, l = 0, acc = 0
            float* ml = part_ml(part, tok, kvh * GQ + h, s, H, ns, T);
            ml[0] = M; ml[1] = l;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// int8 KV (gqa_x_kernel below). Q.K runs on v_mfma_i32_16x16x64_i8 with the raw int8 K bytes as operands: the fp32
// query enters as 24-bit fixed point in three signed base-256 digits (x = d2*2^16 + d1*2^8 + d0, each digit in
// [-128, 127]), every digit product is accumulated exactly in int32 and the digits are recombined in fp32, so the
// scores keep fp32-level precision (the reference decode is fp32).
//   Q.K:  16 keys x 16 columns per MFMA; column m < 8 = digit 2 of head m, m >= 8 = digit 1 of head m-8, a second
//         MFMA holds digit 0 of the 8 heads. Lane (g = lane/16, m = lane%16) receives keys 4g + i of the group for
//         column m; the digits of a head are brought together with two row_ror:8 DPP moves.
// P.V runs on fp16 MFMA (see gqa_x_kernel). Each chunk first computes all its scores and their maximum (pass 1), then
// forms P (pass 1.5) and accumulates P.V (pass 2).
constexpr int ICH = 128;                           // keys per chunk: 32 keys (two 16-key groups) per wavefront
typedef int int4_t_ __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int dpp_ror8(int x) { return __builtin_amdgcn_update_dpp(0, x, 0x128, 0xf, 0xf, false); }

// three signed base-256 digits of n, |n| <= 2^22 + 2^15: n = d2*65536 + d1*256 + d0
__device__ __forceinline__ void digits3(int n, int& d2, int& d1, int& d0) {
    d2 = (n + 32896) >> 16;
    const int r = n - (d2 << 16);
    d1 = (r + 128) >> 8;
    d0 = r - (d1 << 8);
}
__device__ __forceinline__ uint32_t pack_bytes(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) | ((uint32_t)d << 24);
}
__device__ __forceinline__ void tr4x4_(const uint32_t r0, const uint32_t r1, const uint32_t r2, const uint32_t r3, uint32_t c[4]) {
    const uint32_t t0 = __builtin_amdgcn_perm(r1, r0, 0x05010400u), t1 = __builtin_amdgcn_perm(r1, r0, 0x07030602u);
    const uint32_t t2 = __builtin_amdgcn_perm(r3, r2, 0x05010400u), t3 = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
    c[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u); c[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    c[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u); c[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}
typedef __attribute__((address_space(1))) const void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

// One workgroup per (kv head, split, group of TT query tokens), walking the split in chunks of ICH keys with the
// loads of chunk c+1 in flight while chunk c is computed: the V rows go straight to LDS (global_load_lds_dwordx4,
// double buffered, 16-byte pieces XOR-swizzled by key/4 so the pass-2 reads of the four lane groups hit disjoint
// banks), the K rows and the scales to registers (two buffers that swap roles every chunk). Every K/V byte of the
// chunk serves all TT tokens of the group (MTP verify windows): per token only the MFMAs, the scores and P are
// repeated. TT = 1 runs two workgroups per CU; TT > 1 holds TT tokens' scores and accumulators (and reads the query
// digits from LDS) and runs one workgroup per CU.
constexpr int I8_VBUF = ICH * AHD;                 // 32 KB per V buffer
constexpr int I8_QL = 2 * 4 * 64 * 16;             // Q digit operands of one token
static_assert(I8_QL <= I8_VBUF, "query digits of one token stage in V buffer 1");
// 2^(a - b) with 2^(-inf - -inf) = 1 (a running maximum that has not moved, also while it is still -inf)
__device__ __forceinline__ float ex2d(float a, float b) { return a == b ? 1.f : fast_exp2(a - b); }

// ---- gqa_x_kernel: Q.K on the int8 MFMA (as gqa_i8_kernel: exact int32 products of the int8 K rows with the
// query's three base-256 digits), P.V on v_mfma_f32_16x16x32_f16 with fp32 accumulation:
//   P.V:  A = P, 16 rows (hi parts of the 8 heads, then lo parts: p * vs * 2^sig = hi + lo in fp16, ~22 bits) x 32
//         keys (a wavefront's keys; lane group g takes keys 4g..4g+3 of both 16-key groups, which is where the Q.K
//         output layout left them); B = V widened exactly to fp16; output column n of tile j is dim 64*wv + 4n + j,
//         so each lane reads one dword (4 dims) per key.
// O stays in the MFMA accumulators across chunks (rescaled by 2^(m_old - m_new) times the change of the per-chunk power
// of two 2^sig), so a chunk costs no int32 -> fp32 fold and the per-token work is only the MFMAs, the scores and P.
constexpr int X_PL = 4 * 64 * 16;  // P operands of one token per chunk: [step = wavefront][lane] half8
template <int TT>
constexpr int x_lds() { return 2 * I8_VBUF + TT * X_PL + (TT > 1 ? TT * I8_QL : 0); }

template <int TT>
__global__ void __launch_bounds__(256, TT == 1 ? 2 : 1) gqa_x_kernel(const float* __restrict__ qo, moex_kv_cache kv,
                                                                     int H, const int* __restrict__ pos_d, int max_t,
                                                                     float* __restrict__ part, int T, int ns) {
    extern __shared__ __align__(16) unsigned char smem[];
    half8_t* Pl = reinterpret_cast<half8_t*>(smem + 2 * I8_VBUF);  // [TT][4][64]
    // query digits: [TT][2][4][64]; TT = 1 holds them in registers and only stages them in V buffer 1
    int4_t_* Ql = reinterpret_cast<int4_t_*>(TT == 1 ? smem + I8_VBUF : smem + 2 * I8_VBUF + TT * X_PL);
    __shared__ float mxw[TT][4][GQ], lsum[TT][4][GQ], vmw[4], qsc_s[TT][GQ];
    const int nb = gridDim.x, w_id = xcd_work_id(blockIdx.x, nb);
    const int ngr = (T + TT - 1) / TT;
    const int tg = w_id % ngr, s = (w_id / ngr) % ns, kvh = w_id / (ngr * ns);
    const int tb = tg * TT, ntok = min(TT, T - tb);
    const int pos0 = *pos_d, Tmax = pos0 + T;
    const int L = (Tmax + ns - 1) / ns, lo = s * L;
    const int hi = min(pos0 + tb + ntok, lo + L);  // keys of the group's last token; token t sees [lo, hit[t])
    int hit[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) hit[t] = min(pos0 + tb + min(t, ntok - 1) + 1, lo + L);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 4, m16 = lane & 15, hq = m16 & 7;
    const bool lo8 = m16 < 8;
    const size_t rbase = (size_t)kvh * max_t;
    const int8_t* Kg = kv.k + rbase * AHD;
    const int8_t* Vg = kv.v + rbase * AHD;
    const float* ksg = kv.ks + rbase;
    const float* vsg = kv.vs + rbase;
    const int nch = hi > lo ? (hi - lo + ICH - 1) / ICH : 0;

    // ---- loaders. V: thread tid moves 16-byte piece (tid%16) ^ (4*wv) of key 16*it + tid/16 into LDS slot tid%16
    // (the swizzle depends on (key/4)%4 = wv only). K: this wavefront's keys c0 + 32*wv + 16*grp + m16, dims
    // 64*ks + 16g + 0..15; scales of the keys 16*grp + 4g + i its lane scores. ----
    const int8_t* vsrc = Vg + 16 * ((tid & 15) ^ (4 * wv));
    auto issue_v = [&](unsigned char* buf, int c0) {
        const int nk = min(ICH, hi - c0);
        if (nk == ICH) {
            const int8_t* p = vsrc + (size_t)(c0 + (tid >> 4)) * AHD;
#pragma unroll
            for (int it = 0; it < ICH / 16; it++)
                __builtin_amdgcn_global_load_lds((gptr_t)(p + it * 16 * AHD), (lptr_t)(buf + (it * 256 + 64 * wv) * 16), 16, 0, 0);
        } else {
            const int nit = (nk + 15) >> 4;
            for (int it = 0; it < nit; it++) {
                const int t = min(c0 + 16 * it + (tid >> 4), hi - 1);
                __builtin_amdgcn_global_load_lds((gptr_t)(vsrc + (size_t)t * AHD), (lptr_t)(buf + (it * 256 + 64 * wv) * 16), 16, 0, 0);
            }
        }
    };
    auto issue_k = [&](int4_t_ (&kd)[2][4], float (&ksd)[8], float (&vsd)[8], int c0) {
        const int k0 = c0 + 32 * wv;
        if (k0 >= hi) return;
        if (k0 + 32 <= hi) {
            const int8_t* kp = Kg + (size_t)(k0 + m16) * AHD + 16 * g;
#pragma unroll
            for (int grp = 0; grp < 2; grp++)
#pragma unroll
                for (int ks = 0; ks < 4; ks++) kd[grp][ks] = *reinterpret_cast<const int4_t_*>(kp + grp * 16 * AHD + 64 * ks);
#pragma unroll
            for (int grp = 0; grp < 2; grp++) {
                const float4 a = *reinterpret_cast<const float4*>(ksg + k0 + 16 * grp + 4 * g);
                const float4 b = *reinterpret_cast<const float4*>(vsg + k0 + 16 * grp + 4 * g);
                ksd[4 * grp] = a.x; ksd[4 * grp + 1] = a.y; ksd[4 * grp + 2] = a.z; ksd[4 * grp + 3] = a.w;
                vsd[4 * grp] = b.x; vsd[4 * grp + 1] = b.y; vsd[4 * grp + 2] = b.z; vsd[4 * grp + 3] = b.w;
            }
        } else {
#pragma unroll
            for (int grp = 0; grp < 2; grp++) {
                const int8_t* kp = Kg + (size_t)min(k0 + 16 * grp + m16, hi - 1) * AHD + 16 * g;
#pragma unroll
                for (int ks = 0; ks < 4; ks++) kd[grp][ks] = *reinterpret_cast<const int4_t_*>(kp + 64 * ks);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int t = min(k0 + 16 * (j >> 2) + 4 * g + (j & 3), hi - 1);
                ksd[j] = ksg[t]; vsd[j] = vsg[t];
            }
        }
    };
    int4_t_ kA[2][4], kB[2][4];
    float ksA[8], vsA[8], ksB[8], vsB[8];
    if (nch > 0) {
        issue_k(kA, ksA, vsA, lo);
        issue_v(smem, lo);
    }

    // ---- query digits, once per workgroup: thread = (head tid/32, dims 8*(tid%32) .. +7), per token ----
#pragma unroll
    for (int t = 0; t < TT; t++) {
        const int h = tid >> 5, d0 = (tid & 31) * 8;
        const float* qrow = qo + ((size_t)(tb + min(t, ntok - 1)) * H + kvh * GQ + h) * AHD + d0;
        const float4 x0 = reinterpret_cast<const float4*>(qrow)[0], x1 = reinterpret_cast<const float4*>(qrow)[1];
        const float qv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        float qm = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) qm = fmaxf(qm, fabsf(qv[j]));
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) qm = fmaxf(qm, __shfl_xor(qm, o));
        int e = 0;
        if (qm > 0.f) (void)frexpf(qm, &e);  // qm < 2^e
        const float up = ldexpf(1.f, 22 - e);
        if ((tid & 31) == 0) qsc_s[t][h] = ldexpf(1.f, e - 22) * SL2;
        int d2[8], d1[8], dz[8];
#pragma unroll
        for (int j = 0; j < 8; j++) digits3((int)__builtin_rintf(qv[j] * up), d2[j], d1[j], dz[j]);
        // B operand of Q.K: MFMA ks, lane 16g + m holds dims 64ks + 16g + 0..15 of column m
        const int ks = d0 >> 6, gg = (d0 >> 4) & 3, jb = d0 & 15;
        unsigned char* qa_b = reinterpret_cast<unsigned char*>(Ql + ((t * 2 + 0) * 4 + ks) * 64);
        unsigned char* qb_b = reinterpret_cast<unsigned char*>(Ql + ((t * 2 + 1) * 4 + ks) * 64);
        *reinterpret_cast<uint2*>(qa_b + (16 * gg + h) * 16 + jb) =
            make_uint2(pack_bytes(d2[0], d2[1], d2[2], d2[3]), pack_bytes(d2[4], d2[5], d2[6], d2[7]));
        *reinterpret_cast<uint2*>(qa_b + (16 * gg + h + 8) * 16 + jb) =
            make_uint2(pack_bytes(d1[0], d1[1], d1[2], d1[3]), pack_bytes(d1[4], d1[5], d1[6], d1[7]));
        *reinterpret_cast<uint2*>(qb_b + (16 * gg + h) * 16 + jb) =
            make_uint2(pack_bytes(dz[0], dz[1], dz[2], dz[3]), pack_bytes(dz[4], dz[5], dz[6], dz[7]));
        *reinterpret_cast<uint2*>(qb_b + (16 * gg + h + 8) * 16 + jb) = make_uint2(0u, 0u);
    }
    __syncthreads();
    int4_t_ qa[4], qb[4];  // TT = 1 only
    float qs[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) qs[t] = qsc_s[t][hq];
    if (TT == 1) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) { qa[ks] = Ql[ks * 64 + lane]; qb[ks] = Ql[(4 + ks) * 64 + lane]; }
    }

    float4_t o[TT][4];                    // O^T tiles j: lane (g, m16) holds rows 4g + i, column m16
    float m4[TT][4], mo[TT], lacc[TT];    // running max of heads 4(g&1)+i and of head hq; head hq's partial sum
#pragma unroll
    for (int t = 0; t < TT; t++) {
        mo[t] = -INFINITY; lacc[t] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) { m4[t][i] = -INFINITY; o[t][i] = float4_t{0.f, 0.f, 0.f, 0.f}; }
    }
    int sig_ref = 0;  // O is held times 2^sig_ref
    const int rd = 16 * ((4 * wv + (m16 >> 2)) ^ (4 * g)) + 4 * (m16 & 3);  // swizzled byte offset of my V dims

    auto chunk = [&](int c, const int4_t_ (&kr)[2][4], const float (&ksv)[8], const float (&vv)[8],
                     int4_t_ (&kn)[2][4], float (&ksn)[8], float (&vn)[8]) __attribute__((always_inline)) {
        const int c0 = lo + c * ICH, nk = min(ICH, hi - c0), nsteps = (nk + 31) >> 5;
        const int k0 = c0 + 32 * wv;
        const bool has = k0 < hi;
        const unsigned char* Vs = smem + (c & 1) * I8_VBUF;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // chunk c's K, scales and V rows have landed
        __syncthreads();                                   // ... for every wavefront; chunk c-1 is done with LDS
        if (c + 1 < nch) {                                 // all loads of chunk c+1 go out now
            issue_k(kn, ksn, vn, c0 + ICH);
            issue_v(smem + ((c + 1) & 1) * I8_VBUF, c0 + ICH);
        }
        // ---- pass 1: scores of this wavefront's 32 keys (int8 MFMA on the query digits) ----
        float sc[TT][8];
        float vm = 0.f;
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int j = 0; j < 8; j++) sc[t][j] = -INFINITY;
        if (has) {
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (k0 + 16 * (j >> 2) + 4 * g + (j & 3) < hi) vm = fmaxf(vm, vv[j]);
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int grp = 0; grp < 2; grp++) {
                    int4_t_ da = {0, 0, 0, 0}, db = {0, 0, 0, 0};
#pragma unroll
                    for (int ks = 0; ks < 4; ks++) {
                        const int4_t_ a = TT == 1 ? qa[ks] : Ql[(t * 8 + ks) * 64 + lane];
                        const int4_t_ b = TT == 1 ? qb[ks] : Ql[(t * 8 + 4 + ks) * 64 + lane];
                        da = __builtin_amdgcn_mfma_i32_16x16x64_i8(kr[grp][ks], a, da, 0, 0, 0);
                        db = __builtin_amdgcn_mfma_i32_16x16x64_i8(kr[grp][ks], b, db, 0, 0, 0);
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int x = dpp_ror8(da[i]), y = dpp_ror8(db[i]);
                        const int a2 = lo8 ? da[i] : x, a1 = lo8 ? x : da[i], a0 = lo8 ? db[i] : y;
                        const float raw = ((float)a2 * 65536.f + (float)a1 * 256.f) + (float)a0;
                        const int j = 4 * grp + i, key = k0 + 16 * grp + 4 * g + i;
                        sc[t][j] = key < hit[t] ? raw * (ksv[j] * qs[t]) : -INFINITY;
                    }
                }
        }
#pragma unroll
        for (int t = 0; t < TT; t++) {
            float mx = sc[t][0];
#pragma unroll
            for (int j = 1; j < 8; j++) mx = fmaxf(mx, sc[t][j]);
            mx = fmaxf(mx, __shfl_xor(mx, 16)); mx = fmaxf(mx, __shfl_xor(mx, 32));
            if (g == 0 && lo8) mxw[t][wv][m16] = mx;
        }
#pragma unroll
        for (int o2 = 1; o2 < 64; o2 <<= 1) vm = fmaxf(vm, __shfl_xor(vm, o2));
        if (lane == 0) vmw[wv] = vm;
        __syncthreads();
        const float VM = fmaxf(fmaxf(vmw[0], vmw[1]), fmaxf(vmw[2], vmw[3]));
        int ev = 0;
        if (VM > 0.f) (void)frexpf(VM, &ev);  // VM < 2^ev: p * vs * 2^(10 - ev) < 2^10
        const int sig = 10 - ev;
        const float vsc = ldexpf(1.f, sig);
        const float sfac = c == 0 ? 1.f : ldexpf(1.f, sig - sig_ref);  // O re-expressed at the new power of two
        sig_ref = sig;
        // ---- pass 1.5: probabilities (hi/lo fp16 operands to LDS), running maxima, O rescale ----
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const float M = fmaxf(fmaxf(mxw[t][0][hq], mxw[t][1][hq]), fmaxf(mxw[t][2][hq], mxw[t][3][hq]));
            const float mn = fmaxf(mo[t], M);
            float ls = 0.f;
            if (has) {
                half8_t pv;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float p = mn == -INFINITY ? 0.f : fast_exp2(sc[t][j] - mn);  // 0 for masked keys
                    ls += p;
                    const float x = p * (vv[j] * vsc);
                    const _Float16 h = (_Float16)x;
                    pv[j] = lo8 ? h : (_Float16)(x - (float)h);
                }
                Pl[(t * 4 + wv) * 64 + lane] = pv;
            }
            lacc[t] = lacc[t] * ex2d(mo[t], mn) + ls;
            mo[t] = mn;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int h = 4 * (g & 1) + i;
                const float Mh = fmaxf(fmaxf(mxw[t][0][h], mxw[t][1][h]), fmaxf(mxw[t][2][h], mxw[t][3][h]));
                const float mnh = fmaxf(m4[t][i], Mh);
                const float f = ex2d(m4[t][i], mnh) * sfac;
                m4[t][i] = mnh;
#pragma unroll
                for (int jt = 0; jt < 4; jt++) o[t][jt][i] *= f;
            }
        }
        __syncthreads();
        // ---- pass 2: O^T += P . V over the chunk's steps (one per wavefront that had keys), this wavefront's dims ----
        for (int st = 0; st < nsteps; st++) {
            uint32_t r[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int key = 32 * st + 16 * (j >> 2) + 4 * g + (j & 3);
                r[j] = *reinterpret_cast<const uint32_t*>(Vs + key * AHD + rd);
            }
            uint32_t c0v[4], c1v[4];
            tr4x4_(r[0], r[1], r[2], r[3], c0v);
            tr4x4_(r[4], r[5], r[6], r[7], c1v);
            half8_t vb[4];
#pragma unroll
            for (int jt = 0; jt < 4; jt++) vb[jt] = i8x8_to_h8(c0v[jt], c1v[jt]);
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const half8_t pa = Pl[(t * 4 + st) * 64 + lane];
#pragma unroll
                for (int jt = 0; jt < 4; jt++) o[t][jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb[jt], o[t][jt], 0, 0, 0);
            }
        }
    };
    for (int c = 0; c < nch; c += 2) {  // two chunks per trip: the K/scale register buffers swap roles
        chunk(c, kA, ksA, vsA, kB, ksB, vsB);
        if (c + 1 < nch) chunk(c + 1, kB, ksB, vsB, kA, ksA, vsA);
    }
    // ---- partials: rows 4g+i of the O^T tiles are the hi parts (g < 2) of head 4(g&1)+i, the lo parts (g >= 2) ----
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TT; t++) {
        float l = lo8 ? lacc[t] : 0.f;
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        if (g == 0 && lo8) lsum[t][wv][m16] = l;
    }
    __syncthreads();
    const float unscale = ldexpf(1.f, -sig_ref);
#pragma unroll
    for (int t = 0; t < TT; t++) {
        float ov[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int jt = 0; jt < 4; jt++) ov[i][jt] = (o[t][jt][i] + __shfl_xor(o[t][jt][i], 32)) * unscale;
        if (g < 2 && t < ntok) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int h = 4 * g + i;
                float* p = part_acc(part, tb + t, kvh * GQ + h, s, H, ns);
                *reinterpret_cast<float4*>(p + 64 * wv + 4 * m16) = make_float4(ov[i][0], ov[i][1], ov[i][2], ov[i][3]);
                if (wv == 0 && m16 == 0) {
                    float* ml = part_ml(part, tb + t, kvh * GQ + h, s, H, ns, T);
                    ml[0] = m4[t][i];  // -inf when the token has no key in this split
                    ml[1] = lsum[t][0][h] + lsum[t][1][h] + lsum[t][2][h] + lsum[t][3][h];
                }
            }
        }
    }
}

template <int TT>
static void launch_x(const float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, float* part,
                     int T, int ns, hipStream_t st) {
    static bool once = [] {
        MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(gqa_x_kernel<TT>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, x_lds<TT>()));
        return true;
    }();
    (void)once;
    const int nb = KV * ns * ((T + TT - 1) / TT);
    hipLaunchKernelGGL(gqa_x_kernel<TT>, dim3(nb), dim3(256), x_lds<TT>(), st, qo, kv, H, pos_d, max_t, part, T, ns);
}

void launch_gqa(const float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, float* part, int T,
                int ns, hipStream_t st) {
    if (kv.turbo) {
        const int nb = KV * ns * T;
        hipLaunchKernelGGL(gqa_decode_kernel<true>, dim3(nb), dim3(256), 0, st, qo, kv, H, pos_d, max_t, part, T, ns);
    } else {
        if (T == 1) launch_x<1>(qo, kv, H, KV, pos_d, max_t, part, T, ns, st);
        else if (T == 2) launch_x<2>(qo, kv, H, KV, pos_d, max_t, part, T, ns, st);
        else launch_x<4>(qo, kv, H, KV, pos_d, max_t, part, T, ns, st);
    }
    MOEX_LAUNCHED();
}

}  // namespace moex
