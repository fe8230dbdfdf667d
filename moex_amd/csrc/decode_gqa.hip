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
        float* p = part + (((size_t)tok * H + kvh * GQ + h) * ns + s) * (AHD + 2);
        p[2 + d] = acc * vdenorm;
        if (d == 0) { p[0] = M; p[1] = l; }  // empty split: m = -inf, l = 0, acc = 0
    }
}

// ---------------------------------------------------------------------------------------------------------------
// int8 KV: the same split-K decode on v_mfma_i32_16x16x64_i8, with the raw int8 K and V bytes as MFMA operands (no
// widening at all). The fp32 query and the probabilities enter as 24-bit fixed point written in three signed base-256
// digits (x = d2*2^16 + d1*2^8 + d0, each digit in [-128, 127]); every digit product is accumulated exactly in int32
// and the digits are recombined in fp32, so both products keep fp32-level precision (the reference decode is fp32).
// Two passes over each chunk of keys make the int32 accumulation possible: pass 1 computes all scores of the chunk
// and their exact maximum (no online rescaling), pass 2 forms P = 2^(s - max) and accumulates P.V.
//   Q.K:  16 keys x 16 columns per MFMA; column m < 8 = digit 2 of head m, m >= 8 = digit 1 of head m-8, a second
//         MFMA holds digit 0 of the 8 heads. Lane (g = lane/16, m = lane%16) receives keys 4g + i of the group for
//         column m; the digits of a head are brought together with two row_ror:8 DPP moves.
//   P.V:  rows = the same digit/head layout for P; the four wavefronts split the 256 dims (64 each) and all of them
//         walk every key of the chunk, reading the P operands that pass 1 left in LDS. Each lane loads 4 bytes (dims
//         64w + 4m .. +3) of 16 key rows and a 4x4 byte transpose turns them into the B operands.
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

// One workgroup per split, walking it in chunks of 256 keys with the loads of chunk c+1 in flight while chunk c is
// computed: the V rows go straight to LDS (global_load_lds_dwordx4, double buffered, 64-byte blocks XOR-swizzled by
// key/4 so the pass-2 reads of the four lane groups hit disjoint banks), the K rows and the scales to registers.
// The query digits are computed once per workgroup and shared through LDS.
constexpr int I8_VBUF = ICH * AHD;                                       // 64 KB per V buffer
constexpr int I8_LDS_ALL = 2 * I8_VBUF + 2 * (ICH / 64) * 64 * 16 + 2 * 4 * 64 * 16;  // + P operands + Q operands

__device__ __forceinline__ void issue_v_chunk(const int8_t* Vg, unsigned char* buf, int c0, int nk, int hi, int tid,
                                              int wv) {
    const int nit = (nk + 15) >> 4;  // 16 keys (256 16-byte pieces) per workgroup-wide instruction
    for (int it = 0; it < nit; it++) {
        const int q = it * 256 + tid, key = q >> 4, pc = (q & 15) ^ (4 * ((key >> 2) & 3));
        const int t = min(c0 + key, hi - 1);
        __builtin_amdgcn_global_load_lds((gptr_t)(Vg + (size_t)t * AHD + 16 * pc),
                                         (lptr_t)(buf + (size_t)(it * 256 + 64 * wv) * 16), 16, 0, 0);
    }
}

__global__ void __launch_bounds__(256, 2) gqa_i8_kernel(const float* __restrict__ qo, moex_kv_cache kv, int H,
                                                        const int* __restrict__ pos_d, int max_t,
                                                        float* __restrict__ part, int T, int ns) {
    extern __shared__ __align__(16) unsigned char smem[];
    int4_t_* Pl = reinterpret_cast<int4_t_*>(smem + 2 * I8_VBUF);             // [ICH/64][2][64]
    int4_t_* Ql = Pl + (ICH / 64) * 2 * 64;                                   // [2][4][64]
    __shared__ float mxw[4][GQ], lsum[4][GQ], vmw[4], qsc[GQ];
    const int nb = gridDim.x, w_id = xcd_work_id(blockIdx.x, nb);
    const int tok = w_id % T, s = (w_id / T) % ns, kvh = w_id / (T * ns);
    const int pos0 = *pos_d, Tk = pos0 + tok + 1, Tmax = pos0 + T;
    const int L = (Tmax + ns - 1) / ns, lo = s * L, hi = min(Tk, lo + L);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 4, m16 = lane & 15, hq = m16 & 7;
    const bool lo8 = m16 < 8;
    const size_t rbase = (size_t)kvh * max_t;
    const int8_t* Kg = kv.k + rbase * AHD;
    const int8_t* Vg = kv.v + rbase * AHD;
    const float* ksg = kv.ks + rbase;
    const float* vsg = kv.vs + rbase;
    const int nch = hi > lo ? (hi - lo + ICH - 1) / ICH : 0;

    // ---- loads of chunk 0 (registers: this wavefront's K step and scales; LDS: all V rows) ----
    int4_t_ kr[2][4];
    float ksn[8], vvn[8];  // scales of the next chunk to compute
    const int stw = wv >> 1, gq0 = 2 * (wv & 1);  // this wavefront's Q.K step and first 16-key group
    int4_t_ krn[2][4];  // K rows of the next chunk (double buffer)
    auto issue_kr = [&](int k0) {
#pragma unroll
        for (int grp = 0; grp < 2; grp++) {
            const int4_t_* kp = reinterpret_cast<const int4_t_*>(Kg + (size_t)min(k0 + 16 * grp + m16, hi - 1) * AHD + 16 * g);
#pragma unroll
            for (int ks = 0; ks < 4; ks++) krn[grp][ks] = kp[4 * ks];
        }
    };
    auto issue_scales = [&](int k0) {
        if (k0 + 32 <= hi) {
#pragma unroll
            for (int grp = 0; grp < 2; grp++) {
                const float4 a = *reinterpret_cast<const float4*>(ksg + k0 + 16 * grp + 4 * g);
                const float4 b = *reinterpret_cast<const float4*>(vsg + k0 + 16 * grp + 4 * g);
                ksn[4 * grp] = a.x; ksn[4 * grp + 1] = a.y; ksn[4 * grp + 2] = a.z; ksn[4 * grp + 3] = a.w;
                vvn[4 * grp] = b.x; vvn[4 * grp + 1] = b.y; vvn[4 * grp + 2] = b.z; vvn[4 * grp + 3] = b.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int t = min(k0 + 16 * (j >> 2) + 4 * g + (j & 3), hi - 1);
                ksn[j] = ksg[t]; vvn[j] = vsg[t];
            }
        }
    };
    if (nch > 0) {
        const int k0 = lo + 64 * stw + 16 * gq0;
        if (k0 < hi) { issue_kr(k0); issue_scales(k0); }
        issue_v_chunk(Vg, smem, lo, min(ICH, hi - lo), hi, tid, wv);
    }

    // ---- query digits, once per workgroup: thread = (head tid/32, dims 8*(tid%32) .. +7) ----
    {
        const int h = tid >> 5, d0 = (tid & 31) * 8;
        const float* qrow = qo + ((size_t)tok * H + kvh * GQ + h) * AHD + d0;
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
        if ((tid & 31) == 0) qsc[h] = ldexpf(1.f, e - 22);
        int d2[8], d1[8], dz[8];
#pragma unroll
        for (int j = 0; j < 8; j++) digits3((int)__builtin_rintf(qv[j] * up), d2[j], d1[j], dz[j]);
        // B operand of Q.K: MFMA ks, lane 16g + m holds dims 64ks + 16g + 0..15 of column m
        const int ks = d0 >> 6, gg = (d0 >> 4) & 3, jb = d0 & 15;
        unsigned char* qa_b = reinterpret_cast<unsigned char*>(Ql + (0 * 4 + ks) * 64);
        unsigned char* qb_b = reinterpret_cast<unsigned char*>(Ql + (1 * 4 + ks) * 64);
        *reinterpret_cast<uint2*>(qa_b + (16 * gg + h) * 16 + jb) =
            make_uint2(pack_bytes(d2[0], d2[1], d2[2], d2[3]), pack_bytes(d2[4], d2[5], d2[6], d2[7]));
        *reinterpret_cast<uint2*>(qa_b + (16 * gg + h + 8) * 16 + jb) =
            make_uint2(pack_bytes(d1[0], d1[1], d1[2], d1[3]), pack_bytes(d1[4], d1[5], d1[6], d1[7]));
        *reinterpret_cast<uint2*>(qb_b + (16 * gg + h) * 16 + jb) =
            make_uint2(pack_bytes(dz[0], dz[1], dz[2], dz[3]), pack_bytes(dz[4], dz[5], dz[6], dz[7]));
        *reinterpret_cast<uint2*>(qb_b + (16 * gg + h + 8) * 16 + jb) = make_uint2(0u, 0u);
    }
    __syncthreads();
    int4_t_ qa[4], qb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) { qa[ks] = Ql[ks * 64 + lane]; qb[ks] = Ql[(4 + ks) * 64 + lane]; }
    const float qscale = qsc[hq];

    float of[4][4];                 // fp32 result: [MFMA c][row i]; lanes g < 2: head 4g + i, dim 64*wv + 4*m16 + c
    float m_run[4];                 // running max of heads 4*(g&1) + i
    float lw_acc = 0.f, mh_run = -INFINITY;  // this lane's share of head hq's sum, head hq's running max
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) of[c][i] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) m_run[i] = -INFINITY;
    const int rd = 16 * ((4 * wv + (m16 >> 2)) ^ (4 * g)) + 4 * (m16 & 3);  // swizzled byte offset of my V dims

    for (int c = 0; c < nch; c++) {
        const int c0 = lo + c * ICH, nk = min(ICH, hi - c0), nsteps = (nk + 63) >> 6;
        const int k0 = c0 + 64 * stw + 16 * gq0;
        const bool has = k0 < hi;
        unsigned char* Vs = smem + (c & 1) * I8_VBUF;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // chunk c's K, scales and V rows have landed
        __syncthreads();                                   // ... for every wavefront; chunk c-1 is done with LDS
        float ksv[8], vv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) { ksv[j] = ksn[j]; vv[j] = vvn[j]; }
#pragma unroll
        for (int grp = 0; grp < 2; grp++)
#pragma unroll
            for (int ks = 0; ks < 4; ks++) kr[grp][ks] = krn[grp][ks];
        const int c1 = c0 + ICH;  // the next chunk: all its loads go out now
        if (c + 1 < nch) {
            const int k1 = c1 + 64 * stw + 16 * gq0;
            if (k1 < hi) { issue_kr(k1); issue_scales(k1); }
            issue_v_chunk(Vg, smem + ((c + 1) & 1) * I8_VBUF, c1, min(ICH, hi - c1), hi, tid, wv);
        }
        // ---- pass 1: scores of this wavefront's 32 keys ----
        float sc[8];
        float mx = -INFINITY, vm = 0.f;
        if (has) {
#pragma unroll
            for (int grp = 0; grp < 2; grp++) {
                int4_t_ da = {0, 0, 0, 0}, db = {0, 0, 0, 0};
#pragma unroll
                for (int ks = 0; ks < 4; ks++) {
                    da = __builtin_amdgcn_mfma_i32_16x16x64_i8(kr[grp][ks], qa[ks], da, 0, 0, 0);
                    db = __builtin_amdgcn_mfma_i32_16x16x64_i8(kr[grp][ks], qb[ks], db, 0, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int x = dpp_ror8(da[i]), y = dpp_ror8(db[i]);
                    const int a2 = lo8 ? da[i] : x, a1 = lo8 ? x : da[i], a0 = lo8 ? db[i] : y;
                    const float raw = ((float)a2 * 65536.f + (float)a1 * 256.f) + (float)a0;
                    const int j = 4 * grp + i, key = k0 + 16 * grp + 4 * g + i;
                    const float v = key < hi ? raw * (ksv[j] * (SL2 * qscale)) : -INFINITY;
                    sc[j] = v;
                    mx = fmaxf(mx, v);
                    if (key < hi) vm = fmaxf(vm, vv[j]);
                }
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16)); mx = fmaxf(mx, __shfl_xor(mx, 32));
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) vm = fmaxf(vm, __shfl_xor(vm, o));
        if (g == 0 && lo8) mxw[wv][m16] = mx;
        if (lane == 0) vmw[wv] = vm;
        __syncthreads();
        const float M = fmaxf(fmaxf(mxw[0][hq], mxw[1][hq]), fmaxf(mxw[2][hq], mxw[3][hq]));  // head hq, this chunk
        float VM = fmaxf(fmaxf(vmw[0], vmw[1]), fmaxf(vmw[2], vmw[3]));
        VM = VM > 0.f ? VM : 1.f;
        const float iv = 4194304.f / VM;  // P' = p * vs / VM in 22-bit fixed point
        // ---- pass 1.5: P digits of this wavefront's 32 keys -> LDS (dwords gq0, gq0+1 of the step's operands) ----
        float lc = 0.f;
        if (has) {
            uint32_t wa[2], wb[2];
#pragma unroll
            for (int q4 = 0; q4 < 2; q4++) {
                int da[4], db[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int j = 4 * q4 + u;
                    const float p = fast_exp2(sc[j] - M);  // 0 for masked keys
                    lc += p;
                    int d2, d1, d0;
                    digits3((int)(p * (vv[j] * iv) + 0.5f), d2, d1, d0);
                    da[u] = lo8 ? d2 : d1;
                    db[u] = lo8 ? d0 : 0;
                }
                wa[q4] = pack_bytes(da[0], da[1], da[2], da[3]);
                wb[q4] = pack_bytes(db[0], db[1], db[2], db[3]);
            }
            *(reinterpret_cast<uint2*>(Pl + (stw * 2 + 0) * 64 + lane) + (wv & 1)) = make_uint2(wa[0], wa[1]);
            *(reinterpret_cast<uint2*>(Pl + (stw * 2 + 1) * 64 + lane) + (wv & 1)) = make_uint2(wb[0], wb[1]);
        } else if (stw < nsteps) {  // the step exists but none of its keys is mine: zero probabilities
            *(reinterpret_cast<uint2*>(Pl + (stw * 2 + 0) * 64 + lane) + (wv & 1)) = make_uint2(0u, 0u);
            *(reinterpret_cast<uint2*>(Pl + (stw * 2 + 1) * 64 + lane) + (wv & 1)) = make_uint2(0u, 0u);
        }
        {   // chunk bookkeeping of head hq (identical in every wavefront)
            const float mh_new = fmaxf(mh_run, M);
            lw_acc = lw_acc * fast_exp2(mh_run - mh_new) + (lo8 ? lc : 0.f) * fast_exp2(M - mh_new);
            mh_run = mh_new;
        }
        __syncthreads();
        // ---- pass 2: P.V for this wavefront's 64 dims over every step of the chunk ----
        int4_t_ oa[4], ob[4];
#pragma unroll
        for (int cc = 0; cc < 4; cc++) { oa[cc] = int4_t_{0, 0, 0, 0}; ob[cc] = int4_t_{0, 0, 0, 0}; }
        for (int st = 0; st < nsteps; st++) {
            uint32_t r[16];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int key = 64 * st + 16 * (j >> 2) + 4 * g + (j & 3);
                r[j] = *reinterpret_cast<const uint32_t*>(Vs + key * AHD + rd);
            }
            const int4_t_ pa = Pl[(st * 2 + 0) * 64 + lane], pb = Pl[(st * 2 + 1) * 64 + lane];
            uint32_t tq[4][4];
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) tr4x4_(r[4 * q4], r[4 * q4 + 1], r[4 * q4 + 2], r[4 * q4 + 3], tq[q4]);
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                const int4_t_ vb = {(int)tq[0][cc], (int)tq[1][cc], (int)tq[2][cc], (int)tq[3][cc]};
                oa[cc] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb, oa[cc], 0, 0, 0);
                ob[cc] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pb, vb, ob[cc], 0, 0, 0);
            }
        }
        // ---- fold the chunk into fp32: rows 4g+i (g < 2) = digit 2 of head 4g+i, its digit 1 in lane + 32 ----
        const float vs_scale = VM * (1.f / 4194304.f);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int h = 4 * (g & 1) + i;
            const float Mh = fmaxf(fmaxf(mxw[0][h], mxw[1][h]), fmaxf(mxw[2][h], mxw[3][h]));
            const float mn = fmaxf(m_run[i], Mh);
            const float f_old = fast_exp2(m_run[i] - mn), f_new = fast_exp2(Mh - mn) * vs_scale;
            m_run[i] = mn;
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                const int d1 = __shfl_xor(oa[cc][i], 32);
                const float x = ((float)oa[cc][i] * 65536.f + (float)d1 * 256.f) + (float)ob[cc][i];
                of[cc][i] = of[cc][i] * f_old + x * f_new;
            }
        }
    }
    // ---- head sums: lanes m16 < 8 of every group and wavefront hold parts of head m16's sum ----
    float l_run = lw_acc;
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    __syncthreads();  // the last chunk's readers of mxw are done
    if (g == 0 && lo8) lsum[wv][m16] = l_run;
    __syncthreads();
    if (g < 2) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int h = 4 * g + i;
            float* p = part + (((size_t)tok * H + kvh * GQ + h) * ns + s) * (AHD + 2);
            float2* dst = reinterpret_cast<float2*>(p + 2 + 64 * wv + 4 * m16);  // rows are 8-byte aligned
            dst[0] = make_float2(of[0][i], of[1][i]);
            dst[1] = make_float2(of[2][i], of[3][i]);
            if (wv == 0 && m16 == 0) {
                p[0] = nch ? m_run[i] : -INFINITY;
                p[1] = nch ? lsum[0][h] + lsum[1][h] + lsum[2][h] + lsum[3][h] : 0.f;
            }
        }
    }
}

void launch_gqa(const float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, float* part, int T,
                int ns, hipStream_t st) {
    const int nb = KV * ns * T;
    if (kv.turbo)
        hipLaunchKernelGGL(gqa_decode_kernel<true>, dim3(nb), dim3(256), 0, st, qo, kv, H, pos_d, max_t, part, T, ns);
    else {
        static bool once = [] {
            MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(gqa_i8_kernel),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, I8_LDS_ALL));
            return true;
        }();
        (void)once;
        hipLaunchKernelGGL(gqa_i8_kernel, dim3(nb), dim3(256), I8_LDS_ALL, st, qo, kv, H, pos_d, max_t, part, T, ns);
    }
    MOEX_LAUNCHED();
}

}  // namespace moex
