// int8-only prefill fallback (replaces attn_prefill_k, kernels.cuh:1331-1441): the path taken when MOEX_FA=0, and
// for GQA groups other than 8 query heads per kv head (any G that divides 32).
//
// Workgroup = (kv head, 32 query rows): row r is token r / G, head r % G of the group. Keys come in tiles of 128,
// staged once in LDS for the 4 wavefronts (K widened to fp16 as [key][dim], V widened to fp16 as V^T [dim][key]).
// Wavefront w owns keys 32w .. 32w + 31 of every tile and runs its own online softmax over them, so there is no
// exchange between wavefronts inside the key loop:
//   - S^T = K_w . Q^T on v_mfma_f32_32x32x16_f16, with Q (fp16) in registers: lane L holds query row L % 32 and
//     16 of the 32 keys, so a row's maximum and sum are in-lane plus one exchange with lane L ^ 32;
//   - P * vscale is rounded to fp16 in the lane that formed it and is used there as the B operand of
//     O^T += V^T . P^T (same MFMA), which works because V^T's keys are stored in the order the S^T accumulators
//     hold them (bits 2 and 3 of the key index swapped within each 16-key group);
//   - O^T (256 dims x 32 rows) stays in the wavefront's registers and is rescaled only when a row maximum moves.
// After the last tile the four wavefronts' {m, l, O} merge through LDS (reusing the tile buffers), and the output is
// divided by l and gated. Base-2 softmax with the reference's scale log2(e) / 16.
#include "common.hpp"

namespace moex {

namespace {
constexpr int KR = 32;            // query rows per workgroup
constexpr int KB = 128;           // keys per tile (32 per wavefront)
constexpr int KS = AHD + 8;       // K row stride in halves
constexpr int VS = KB + 8;        // V^T row stride in halves
constexpr int K_BYTES = KB * KS * 2, V_BYTES = AHD * VS * 2;
constexpr int MERGE_BYTES = 4 * KR * AHD * 4 + 2 * 4 * KR * 4;  // the wavefronts' O and {m, l}
constexpr int SC_OFF = K_BYTES + V_BYTES;                        // per-key K and V scales, KB each
constexpr int K7P_LDS_TILES = SC_OFF + 2 * KB * 4;
constexpr int K7P_LDS = K7P_LDS_TILES > MERGE_BYTES ? K7P_LDS_TILES : MERGE_BYTES;
constexpr float K7P_SL2 = 0.0625f * 1.4426950408889634f;

__device__ __forceinline__ int swap23(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }
}  // namespace

__global__ void __launch_bounds__(256, 1) k7p_prefill_kernel(const float* __restrict__ qo, const float* __restrict__ q_gate,
                                                             moex_kv_cache kv, float* __restrict__ out, int H, int KV,
                                                             const int* __restrict__ pos_d, int max_t, int ld, int T) {
    extern __shared__ __align__(16) unsigned char lds[];
    _Float16* Kl = reinterpret_cast<_Float16*>(lds);
    _Float16* Vl = reinterpret_cast<_Float16*>(lds + K_BYTES);
    float* ksl = reinterpret_cast<float*>(lds + SC_OFF);
    float* vsl = ksl + KB;
    const int G = H / KV, tpb = KR / G;  // tokens per workgroup
    const int kvh = blockIdx.x, t0 = blockIdx.y * tpb, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int pos0 = *pos_d, nt = min(tpb, T - t0), hi = pos0 + t0 + nt;
    // this lane's query row (rows past the chunk repeat its last token; they are never written)
    const int tl = min(col / G, nt - 1), hd = kvh * G + col % G, rpos = pos0 + t0 + tl;
    half8_t q[16];  // Q^T operand: dims 16c + 8 half .. + 7
    {
        const float* qr = qo + ((size_t)(t0 + tl) * H + hd) * AHD + 8 * half;
#pragma unroll
        for (int c = 0; c < 16; c++) {
            const float4 a = *reinterpret_cast<const float4*>(qr + 16 * c);
            const float4 b = *reinterpret_cast<const float4*>(qr + 16 * c + 4);
            q[c] = half8_t{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                           (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
        }
    }
    float16_t o[8];  // O^T, dim tile j: query row lane % 32, dims 32j + 8(i/4) + 4 half + i % 4
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = float16_t{};
    float m = -INFINITY, l = 0.f;  // running max (log2 units) and sum of row `col` over this wavefront's keys
    const size_t rbase = (size_t)kvh * max_t;
    for (int k0 = 0; k0 < hi; k0 += KB) {
        __syncthreads();  // the previous tile is consumed
        {   // K: thread t widens dims 128 (t % 2) .. +127 of key t / 2
            const int key = tid >> 1, d0 = 128 * (tid & 1), t = k0 + key;
            const uint4* src = reinterpret_cast<const uint4*>(kv.k + (rbase + min(t, hi - 1)) * AHD + d0);
            uint4 u[8];
#pragma unroll
            for (int i = 0; i < 8; i++) u[i] = t < hi ? src[i] : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                uint32_t a0, a1, a2, a3, b0, b1, b2, b3;
                i8x4_to_h4(u[i].x, a0, a1); i8x4_to_h4(u[i].y, a2, a3);
                i8x4_to_h4(u[i].z, b0, b1); i8x4_to_h4(u[i].w, b2, b3);
                uint4* dst = reinterpret_cast<uint4*>(Kl + key * KS + d0 + 16 * i);
                dst[0] = make_uint4(a0, a1, a2, a3);
                dst[1] = make_uint4(b0, b1, b2, b3);
            }
            // V: thread t widens dims 4 (t % 64) .. +3 of keys 32 (t / 64) .. +31 into V^T, keys in accumulator order
            const int dg = tid & 63, kg = 32 * (tid >> 6);
            uint32_t r[32];
#pragma unroll
            for (int i = 0; i < 32; i++) {
                const int tt = k0 + kg + i;
                r[i] = tt < hi ? *reinterpret_cast<const uint32_t*>(kv.v + (rbase + tt) * AHD + 4 * dg) : 0u;
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                _Float16* vrow = Vl + (4 * dg + e) * VS + kg;
#pragma unroll
                for (int g8 = 0; g8 < 4; g8++) {  // slots 8 g8 .. +7 hold keys swap23(slot)
                    half8_t x;
#pragma unroll
                    for (int p = 0; p < 8; p++) {
                        const int sl = 8 * g8 + p, key = (sl & 16) + swap23(sl & 15);
                        x[p] = (_Float16)(float)(int8_t)(r[key] >> (8 * e));
                    }
                    *reinterpret_cast<half8_t*>(vrow + 8 * g8) = x;
                }
            }
            if (tid < KB) {
                const int tt = min(k0 + tid, hi - 1);
                ksl[tid] = kv.ks[rbase + tt] * K7P_SL2;
                vsl[tid] = kv.vs[rbase + tt];
            }
        }
        __syncthreads();
        const int kw = 32 * w;  // this wavefront's keys in the tile
        if (k0 + kw >= hi) continue;  // no key of this wavefront's sub-tile exists
        float16_t s = {};
#pragma unroll
        for (int c = 0; c < 16; c++) {
            const half8_t a = *reinterpret_cast<const half8_t*>(Kl + (kw + col) * KS + 16 * c + 8 * half);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, q[c], s, 0, 0, 0);
        }
        // scores -> log2 units, causal mask (key <= the row's position), tile maximum
        float mx = -INFINITY;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 sc = *reinterpret_cast<const float4*>(ksl + kw + 8 * g + 4 * half);
            const float scv[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = k0 + kw + 8 * g + 4 * half + i;
                const float v = key <= rpos ? s[4 * g + i] * scv[i] : -INFINITY;
                s[4 * g + i] = v;
                mx = fmaxf(mx, v);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        const float c = mn == -INFINITY ? 1.f : fast_exp2(m - mn);  // 0 on the first keys (m = -inf)
        // P * vscale -> fp16 B operands (keys of accumulators 8h .. 8h + 7)
        float sum = 0.f;
        half8_t pb[2];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 vs = *reinterpret_cast<const float4*>(vsl + kw + 8 * g + 4 * half);
            const float vsv[4] = {vs.x, vs.y, vs.z, vs.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float p = mn == -INFINITY ? 0.f : fast_exp2(s[4 * g + i] - mn);
                sum += p;
                pb[g >> 1][4 * (g & 1) + i] = (_Float16)(p * vsv[i]);
            }
        }
        sum += __shfl_xor(sum, 32);
        l = l * c + sum;
        m = mn;
        if (__ballot(c != 1.f)) {  // the lane's O accumulators all belong to its own row
#pragma unroll
            for (int j = 0; j < 8; j++)
#pragma unroll
                for (int i = 0; i < 16; i++) o[j][i] *= c;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
#pragma unroll
            for (int h2 = 0; h2 < 2; h2++) {
                const half8_t a = *reinterpret_cast<const half8_t*>(Vl + (32 * j + col) * VS + kw + 16 * h2 + 8 * half);
                o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[h2], o[j], 0, 0, 0);
            }
        }
    }
    // merge the four wavefronts: M = max m_w, l = sum l_w 2^(m_w - M), O = sum O_w 2^(m_w - M)
    __syncthreads();
    float* Om = reinterpret_cast<float*>(lds);          // [w][row][dim]
    float* mm = Om + 4 * KR * AHD;                      // [w][row]
    float* lm = mm + 4 * KR;
    if (half == 0) { mm[w * KR + col] = m; lm[w * KR + col] = l; }
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; v++) M = fmaxf(M, mm[v * KR + col]);  // wavefront 0 holds key 0 of every row: finite
    float L = 0.f;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const float mv = mm[v * KR + col];
        L += mv == -INFINITY ? 0.f : lm[v * KR + col] * fast_exp2(mv - M);
    }
    const float f = m == -INFINITY ? 0.f : fast_exp2(m - M) / L;  // this wavefront's weight for row `col`
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            Om[(w * KR + col) * AHD + 32 * j + 8 * (i >> 2) + 4 * half + (i & 3)] = o[j][i] * f;
    __syncthreads();
    // thread t: row t / 8, dims 32 (t % 8) .. +31
    const int row = tid >> 3, dd = 32 * (tid & 7), trow = row / G;
    if (trow >= nt) return;
    const size_t tok = (size_t)(t0 + trow);
    const int h = kvh * G + row % G;
    float* dst = out + (tok * H + h) * AHD + dd;
    const float* gate = q_gate ? q_gate + tok * ld + h * 2 * AHD + AHD + dd : nullptr;
#pragma unroll
    for (int d = 0; d < 32; d += 4) {
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float4 y = *reinterpret_cast<const float4*>(Om + (v * KR + row) * AHD + dd + d);
            x.x += y.x; x.y += y.y; x.z += y.z; x.w += y.w;
        }
        if (gate) {
            const float4 g = *reinterpret_cast<const float4*>(gate + d);
            x.x /= 1.f + __expf(-g.x); x.y /= 1.f + __expf(-g.y);
            x.z /= 1.f + __expf(-g.z); x.w /= 1.f + __expf(-g.w);
        }
        *reinterpret_cast<float4*>(dst + d) = x;
    }
}

void launch_prefill_k7p(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                        const int* pos_d, int max_t, int ld, int T, hipStream_t st) {
    static bool once = [] {
        MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(k7p_prefill_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, K7P_LDS));
        return true;
    }();
    (void)once;
    const int tpb = KR / (H / KV);
    hipLaunchKernelGGL(k7p_prefill_kernel, dim3(KV, (T + tpb - 1) / tpb), dim3(256), K7P_LDS, st, qo, q_gate, kv, out, H,
                       KV, pos_d, max_t, ld, T);
    MOEX_LAUNCHED();
}

}  // namespace moex
