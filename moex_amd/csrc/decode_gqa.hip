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

void launch_gqa(const float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, float* part, int T,
                int ns, hipStream_t st) {
    const int nb = KV * ns * T;
    if (kv.turbo)
        hipLaunchKernelGGL(gqa_decode_kernel<true>, dim3(nb), dim3(256), 0, st, qo, kv, H, pos_d, max_t, part, T, ns);
    else
        hipLaunchKernelGGL(gqa_decode_kernel<false>, dim3(nb), dim3(256), 0, st, qo, kv, H, pos_d, max_t, part, T, ns);
    MOEX_LAUNCHED();
}

}  // namespace moex
