// Dense int8 projections on gfx950: the attention's qkv and o projections in their default form, int8 weights with a
// per-row scale (replaces quantize_rows_i8_k, gemv_i8 and gemm_i8_k / gemm(), kernels.cuh:98-156,250-337).
//
//   quantize_rows_kernel   fp16 [O][I] -> int8 [O][I] + scale absmax/127 per row (bit-exact: IEEE divide, rint).
//   gemv_kernel<NT>        y[t][o] = s[o] * sum_i q[o][i] x[t][i] for NT <= 8 rows of x, fp32 sums. HBM-bound on the
//                          weights, which are read once for all NT rows. The NT input rows sit in LDS; a wavefront
//                          takes 8 weight rows at a time, its lanes walking I in dwords (256 contiguous bytes per row
//                          and instruction), and reduces each sum across the wavefront. The assignment of rows and of
//                          the sum order to lanes does not depend on NT, so any row of a multi-row call is
//                          bit-identical to the same row alone.
//   gemm_kernel            S > 8 rows (prefill): Y = X . W^T * s on v_mfma_f32_32x32x16_f16. Weights are widened to
//                          fp16 exactly (integers), activations rounded to fp16 as the reference does
//                          (kernels.cuh:306-307), fp32 accumulation, the row scale applied last. Workgroup tile 128
//                          weight rows x 128 tokens, 4 wavefronts of 64 x 64, K steps of 32 double-buffered in LDS.
#include "common.hpp"

namespace moex {

namespace {

__device__ __forceinline__ float wave_sum(float v) {
    v += __shfl_xor(v, 32);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 1);
    return v;
}

__global__ void __launch_bounds__(256) quantize_rows_kernel(const uint16_t* __restrict__ W, int8_t* __restrict__ q,
                                                            float* __restrict__ s, int I) {
    __shared__ float red[4];
    const size_t row = blockIdx.x;
    const _Float16* wr = reinterpret_cast<const _Float16*>(W) + row * I;
    float m = 0.f;
    for (int i = threadIdx.x; i < I; i += 256) m = fmaxf(m, fabsf((float)wr[i]));
#pragma unroll
    for (int o = 32; o; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = m > 0.f ? m / 127.f : 1.f;
    for (int i = threadIdx.x; i < I; i += 256) q[row * I + i] = (int8_t)(int)__builtin_rintf((float)wr[i] / sc);
    if (threadIdx.x == 0) s[row] = sc;
}

constexpr int GV_R = 8;       // weight rows a wavefront takes at a time
constexpr int GV_WAVES = 4;   // wavefronts per workgroup

// Workgroup b takes row groups b, b + nb, .. (GV_R rows each), its wavefronts one group at a time.
template <int NT>
__global__ void __launch_bounds__(64 * GV_WAVES) gemv_kernel(const int8_t* __restrict__ q, const float* __restrict__ s,
                                                             const float* __restrict__ x, float* __restrict__ y, int I,
                                                             int O) {
    extern __shared__ __align__(16) float xs[];  // [NT][I]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int e = tid; e < NT * I / 4; e += 64 * GV_WAVES)
        reinterpret_cast<float4*>(xs)[e] = reinterpret_cast<const float4*>(x)[e];
    __syncthreads();
    const int ngroups = (O + GV_R - 1) / GV_R;
    for (int g = blockIdx.x * GV_WAVES + wv; g < ngroups; g += gridDim.x * GV_WAVES) {
        const int r0 = g * GV_R;
        float acc[NT][GV_R];
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int r = 0; r < GV_R; r++) acc[t][r] = 0.f;
        const uint32_t* qr[GV_R];
#pragma unroll
        for (int r = 0; r < GV_R; r++) qr[r] = reinterpret_cast<const uint32_t*>(q + (size_t)min(r0 + r, O - 1) * I);
        for (int c = lane; c < I / 4; c += 64) {
            uint32_t w[GV_R];
#pragma unroll
            for (int r = 0; r < GV_R; r++) w[r] = __builtin_nontemporal_load(qr[r] + c);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float4 xv = reinterpret_cast<const float4*>(xs + t * I)[c];
#pragma unroll
                for (int r = 0; r < GV_R; r++) {
                    acc[t][r] += (float)(int8_t)(w[r]) * xv.x;
                    acc[t][r] += (float)(int8_t)(w[r] >> 8) * xv.y;
                    acc[t][r] += (float)(int8_t)(w[r] >> 16) * xv.z;
                    acc[t][r] += (float)(int8_t)(w[r] >> 24) * xv.w;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int r = 0; r < GV_R; r++) {
                const float v = wave_sum(acc[t][r]);
                if (lane == 0 && r0 + r < O) y[(size_t)t * O + r0 + r] = v * s[r0 + r];
            }
    }
}

// ---- prefill GEMM ----
constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 32;
constexpr int GM_LD = GM_BK + 8;  // halves per LDS row (80 B: conflict-free 16-byte operand reads)

__global__ void __launch_bounds__(256) gemm_kernel(const int8_t* __restrict__ W, const float* __restrict__ s,
                                                   const float* __restrict__ X, float* __restrict__ Y, int S, int I,
                                                   int O) {
    __shared__ __align__(16) _Float16 lds[2][2][GM_BM * GM_LD];  // [buffer][W, X][row][k]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, r = lane & 31, h32 = lane >> 5;
    const int o0 = blockIdx.x * GM_BM, s0 = blockIdx.y * GM_BN;
    const int wo = (wv >> 1) * 64, ws = (wv & 1) * 64;  // this wavefront's 64 x 64 block of the tile
    // staging: thread tid owns 16 weights (row tid/2, k 16*(tid%2)) and 16 activations (token tid/2, same k)
    const int sr = tid >> 1, sk = (tid & 1) * 16;
    const bool wok = o0 + sr < O, xok = s0 + sr < S;
    const int8_t* wp = W + (size_t)min(o0 + sr, O - 1) * I + sk;
    const float* xp = X + (size_t)min(s0 + sr, S - 1) * I + sk;
    uint4 wreg;
    float4 xreg[4];
    auto load = [&](int k0) {
        wreg = *reinterpret_cast<const uint4*>(wp + k0);
#pragma unroll
        for (int j = 0; j < 4; j++) xreg[j] = reinterpret_cast<const float4*>(xp + k0)[j];
    };
    auto store = [&](int b) {
        uint32_t h[8];
        i8x4_to_h4(wok ? wreg.x : 0u, h[0], h[1]);
        i8x4_to_h4(wok ? wreg.y : 0u, h[2], h[3]);
        i8x4_to_h4(wok ? wreg.z : 0u, h[4], h[5]);
        i8x4_to_h4(wok ? wreg.w : 0u, h[6], h[7]);
        uint4* wd = reinterpret_cast<uint4*>(&lds[b][0][sr * GM_LD + sk]);
        wd[0] = make_uint4(h[0], h[1], h[2], h[3]);
        wd[1] = make_uint4(h[4], h[5], h[6], h[7]);
        uint32_t xh[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float4 v = xok ? xreg[j] : make_float4(0.f, 0.f, 0.f, 0.f);
            xh[2 * j] = h22u(half2_t{(_Float16)v.x, (_Float16)v.y});
            xh[2 * j + 1] = h22u(half2_t{(_Float16)v.z, (_Float16)v.w});
        }
        uint4* xd = reinterpret_cast<uint4*>(&lds[b][1][sr * GM_LD + sk]);
        xd[0] = make_uint4(xh[0], xh[1], xh[2], xh[3]);
        xd[1] = make_uint4(xh[4], xh[5], xh[6], xh[7]);
    };
    float16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;
    const int nk = I / GM_BK;
    load(0);
    store(0);
    if (nk > 1) load(GM_BK);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int b = kt & 1;
        if (kt + 1 < nk) {
            store(b ^ 1);                                  // tile kt + 1, loaded during the previous step
            if (kt + 2 < nk) load((kt + 2) * GM_BK);
        }
        // D^T (tokens x rows per 32x32 block) = X . W^T: A = activation rows, B = weight rows, both [row][k]
#pragma unroll
        for (int kk = 0; kk < GM_BK; kk += 16) {
            half8_t a[2], bw[2];
#pragma unroll
            for (int j = 0; j < 2; j++)
                a[j] = *reinterpret_cast<const half8_t*>(&lds[b][1][(ws + 32 * j + r) * GM_LD + kk + 8 * h32]);
#pragma unroll
            for (int i = 0; i < 2; i++)
                bw[i] = *reinterpret_cast<const half8_t*>(&lds[b][0][(wo + 32 * i + r) * GM_LD + kk + 8 * h32]);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j], bw[i], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    // acc[i][j] element e: weight row wo + 32i + r (the lane's column), token ws + 32j + 8*(e/4) + 4*h32 + e%4
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int o = o0 + wo + 32 * i + r;
        if (o >= O) continue;
        const float so = s[o];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int t = s0 + ws + 32 * j + 8 * (e >> 2) + 4 * h32 + (e & 3);
                if (t < S) Y[(size_t)t * O + o] = acc[i][j][e] * so;
            }
    }
}

template <int NT>
void launch_gemv_t(const int8_t* q, const float* s, const float* x, float* y, int I, int O, hipStream_t st) {
    static bool once = [] {
        MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(gemv_kernel<NT>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        return true;
    }();
    (void)once;
    static const int cus = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            return v;
        return 256;
    }();
    const int groups = (O + GV_R - 1) / GV_R;
    const int nb = std::min(cus, (groups + GV_WAVES - 1) / GV_WAVES);
    hipLaunchKernelGGL(gemv_kernel<NT>, dim3(nb), dim3(64 * GV_WAVES), NT * I * 4, st, q, s, x, y, I, O);
    MOEX_LAUNCHED();
}

}  // namespace

void launch_quantize_rows_i8(const uint16_t* W, int8_t* q, float* s, int O, int I, hipStream_t st) {
    hipLaunchKernelGGL(quantize_rows_kernel, dim3(O), dim3(256), 0, st, W, q, s, I);
    MOEX_LAUNCHED();
}

void launch_gemv_i8(const int8_t* q, const float* s, const float* x, float* y, int NT, int I, int O, hipStream_t st) {
    switch (NT) {
        case 1: launch_gemv_t<1>(q, s, x, y, I, O, st); break;
        case 2: launch_gemv_t<2>(q, s, x, y, I, O, st); break;
        case 3: launch_gemv_t<3>(q, s, x, y, I, O, st); break;
        case 4: launch_gemv_t<4>(q, s, x, y, I, O, st); break;
        case 5: launch_gemv_t<5>(q, s, x, y, I, O, st); break;
        case 6: launch_gemv_t<6>(q, s, x, y, I, O, st); break;
        case 7: launch_gemv_t<7>(q, s, x, y, I, O, st); break;
        default: launch_gemv_t<8>(q, s, x, y, I, O, st); break;
    }
}

void launch_gemm_i8(const int8_t* q, const float* s, const float* X, float* Y, int S, int I, int O, hipStream_t st) {
    hipLaunchKernelGGL(gemm_kernel, dim3((O + GM_BM - 1) / GM_BM, (S + GM_BN - 1) / GM_BN), dim3(256), 0, st, q, s,
                       X, Y, S, I, O);
    MOEX_LAUNCHED();
}

}  // namespace moex
