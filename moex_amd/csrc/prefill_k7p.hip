// int8-only prefill fallback (replaces attn_prefill_k, kernels.cuh:1331-1441): the path taken when MOEX_FA=0.
//
// Workgroup = (kv head, 4 tokens) = 32 query rows (token r/8, head r%8), 4 wavefronts, keys in tiles of 32. Q, K
// (row-major) and V (transposed) are fp16 in LDS. S = Q.K^T on v_mfma_f32_16x16x32_f16 (one 16x16 tile per
// wavefront), written to LDS; 8 threads per row run a natural-base online softmax (__expf, as the reference) and
// write P * vscale as fp16; O += P.V on the same MFMA with the 2 x 16 output tiles split 8 per wavefront and held
// in registers. A deliberately simple, independent formulation: it cross-checks the FA kernel.
#include "common.hpp"

namespace moex {

namespace {
constexpr int PR = 32, PK = 32, PLD = AHD + 8, VTS = PK + 8, SLD = PK + 4;
constexpr int K7P_SMEM = PR * PLD * 2 + PK * PLD * 2 + AHD * VTS * 2 + PR * SLD * 4 + PR * VTS * 2 + 3 * PR * 4 + 2 * PK * 4;
}

__global__ void __launch_bounds__(256) k7p_prefill_kernel(const float* __restrict__ qo, const float* __restrict__ q_gate,
                                                          moex_kv_cache kv, float* __restrict__ out, int H, int KV,
                                                          const int* __restrict__ pos_d, int max_t, int ld, int T) {
    extern __shared__ __align__(16) unsigned char smem[];
    _Float16* Qs = reinterpret_cast<_Float16*>(smem);   // [PR][PLD]
    _Float16* Ks = Qs + PR * PLD;                         // [PK][PLD]
    _Float16* Vt = Ks + PK * PLD;                         // [AHD][VTS]
    float* Ss = reinterpret_cast<float*>(Vt + AHD * VTS);  // [PR][SLD]
    _Float16* Ps = reinterpret_cast<_Float16*>(Ss + PR * SLD);  // [PR][VTS]
    float* mrow = reinterpret_cast<float*>(Ps + PR * VTS);
    float *lrow = mrow + PR, *crow = lrow + PR, *ksc = crow + PR, *vsc = ksc + PK;
    const int G = GQ, TT = PR / G, kvh = blockIdx.x, t0 = blockIdx.y * TT, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, g = lane >> 4, c16 = lane & 15;
    const int pos0 = *pos_d, nt = min(TT, T - t0), hi = pos0 + t0 + nt;
    for (int e = tid; e < PR * AHD; e += 256) {
        const int r = e / AHD, d = e % AHD, tl = r / G;
        Qs[r * PLD + d] = (_Float16)(tl < nt ? qo[((size_t)(t0 + tl) * H + kvh * G + r % G) * AHD + d] : 0.f);
    }
    if (tid < PR) { mrow[tid] = -INFINITY; lrow[tid] = 0.f; }
    const size_t rbase = (size_t)kvh * max_t;
    const float scale = 0.0625f;
    const int r_sm = tid >> 3, q_sm = tid & 7;
    const int rpos = pos0 + t0 + min(r_sm / G, nt - 1);
    // output tiles of this wavefront: row tile w & 1, dim tiles 8*(w >> 1) .. +7
    const int rt = w & 1, ct0 = 8 * (w >> 1);
    float4_t oacc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) oacc[i] = float4_t{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < hi; k0 += PK) {
        __syncthreads();  // previous tile's readers are done
        {   // K rows (fp16, row-major) and V^T
            const int key = tid >> 3, c = (tid & 7) * 32, t = k0 + key;
            uint4 a[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
            if (t < hi) {
                const uint4* p = reinterpret_cast<const uint4*>(kv.k + (rbase + t) * AHD + c);
                a[0] = p[0]; a[1] = p[1];
            }
            const uint32_t in[8] = {a[0].x, a[0].y, a[0].z, a[0].w, a[1].x, a[1].y, a[1].z, a[1].w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                uint32_t lo, hi2;
                i8x4_to_h4(in[i], lo, hi2);
                *reinterpret_cast<uint2*>(Ks + key * PLD + c + 4 * i) = make_uint2(lo, hi2);
            }
            const int dg = tid & 63, kb = (tid >> 6) * 8;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int tt = k0 + kb + i;
                const uint32_t x = tt < hi ? *reinterpret_cast<const uint32_t*>(kv.v + (rbase + tt) * AHD + 4 * dg) : 0u;
#pragma unroll
                for (int e = 0; e < 4; e++) Vt[(4 * dg + e) * VTS + kb + i] = (_Float16)(float)(int8_t)(x >> (8 * e));
            }
            if (tid < PK) {
                ksc[tid] = k0 + tid < hi ? kv.ks[rbase + k0 + tid] : 0.f;
                vsc[tid] = k0 + tid < hi ? kv.vs[rbase + k0 + tid] : 0.f;
            }
        }
        __syncthreads();
        {   // S: wavefront w computes rows 16*(w&1) .., keys 16*(w>>1) ..
            const int sr = 16 * (w & 1), sk = 16 * (w >> 1);
            float4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < AHD; kk += 32) {
                const half8_t a = *reinterpret_cast<const half8_t*>(Qs + (sr + c16) * PLD + kk + 8 * g);
                const half8_t b = *reinterpret_cast<const half8_t*>(Ks + (sk + c16) * PLD + kk + 8 * g);
                s = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, s, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) Ss[(sr + 4 * g + i) * SLD + sk + c16] = s[i];
        }
        __syncthreads();
        {   // softmax: 8 threads per row, 4 keys each
            float sv[4], mx = -INFINITY;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int kk = q_sm * 4 + u, t = k0 + kk;
                sv[u] = t <= rpos ? Ss[r_sm * SLD + kk] * ksc[kk] * scale : -INFINITY;
                mx = fmaxf(mx, sv[u]);
            }
#pragma unroll
            for (int o = 1; o < 8; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
            const float mo = mrow[r_sm], mn = fmaxf(mo, mx), c = __expf(mo - mn);
            float sum = 0.f;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int kk = q_sm * 4 + u;
                const float p = __expf(sv[u] - mn);
                sum += p;
                Ps[r_sm * VTS + kk] = (_Float16)(p * vsc[kk]);
            }
#pragma unroll
            for (int o = 1; o < 8; o <<= 1) sum += __shfl_xor(sum, o);
            __syncthreads();  // every thread has read mrow before it changes
            if (q_sm == 0) { mrow[r_sm] = mn; lrow[r_sm] = lrow[r_sm] * c + sum; crow[r_sm] = c; }
        }
        __syncthreads();
        {   // O = O * c + P . V
            float cr[4];
#pragma unroll
            for (int i = 0; i < 4; i++) cr[i] = crow[16 * rt + 4 * g + i];
            const half8_t a = *reinterpret_cast<const half8_t*>(Ps + (16 * rt + c16) * VTS + 8 * g);
#pragma unroll
            for (int j = 0; j < 8; j++) {
#pragma unroll
                for (int i = 0; i < 4; i++) oacc[j][i] *= cr[i];
                const int dim = 16 * (ct0 + j) + c16;
                const half8_t b = *reinterpret_cast<const half8_t*>(Vt + dim * VTS + 8 * g);
                oacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, oacc[j], 0, 0, 0);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 16 * rt + 4 * g + i, tl = r / G, h = kvh * G + r % G;
        if (tl >= nt) continue;
        const size_t t = (size_t)(t0 + tl);
        const float il = 1.f / lrow[r];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int d = 16 * (ct0 + j) + c16;
            float x = oacc[j][i] * il;
            if (q_gate) x = x / (1.f + __expf(-q_gate[t * ld + h * 2 * AHD + AHD + d]));
            out[(t * H + h) * AHD + d] = x;
        }
    }
}

void launch_prefill_k7p(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                        const int* pos_d, int max_t, int ld, int T, hipStream_t st) {
    static bool once = [] {
        MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(k7p_prefill_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, K7P_SMEM));
        return true;
    }();
    (void)once;
    const int tt = PR / GQ;
    hipLaunchKernelGGL(k7p_prefill_kernel, dim3(KV, (T + tt - 1) / tt), dim3(256), K7P_SMEM, st, qo, q_gate, kv, out, H,
                       KV, pos_d, max_t, ld, T);
    MOEX_LAUNCHED();
}

}  // namespace moex
