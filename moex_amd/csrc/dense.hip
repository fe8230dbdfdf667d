// Dense projections on gfx950: the attention's qkv and o projections in their default form, int8 weights with a
// per-row scale (replaces quantize_rows_i8_k, gemv_i8 and gemm_i8_k / gemm(), kernels.cuh:98-156,250-337), and the
// reference's other matrix forms, int4 / int6 with a scale per 64 inputs and fp16 (quantize_rows_q4_k / _q6_k,
// gemv_q4_k / gemv_q6_k / gemv_f16_k, gemm_wmma_k, gemm_i8_k<true>: kernels.cuh:68-93,225-337,486-590).
//
//   quantize_rows_kernel   fp16 [O][I] -> int8 [O][I] + scale absmax/127 per row (bit-exact: IEEE divide, rint).
//   gemv_kernel<NT>        y[t][o] = s[o] * sum_i q[o][i] x[t][i] for NT <= 8 rows of x, fp32 sums. HBM-bound on the
//                          weights, which are read once for all NT rows. The NT input rows sit in LDS; a wavefront
//                          takes 8 weight rows over 1/KS of I, its lanes walking it in 16-byte chunks (1 KB contiguous
//                          per row and instruction, 16 KB per wavefront issued before any product), reduces each
//                          sum across the wavefront, and the KS parts of a row are added in LDS. KS and the sum order
//                          depend on O and I only, so any row of a multi-row call is bit-identical to the same row
//                          alone.
//   gemm_kernel            S > 8 rows (prefill): Y = X . W^T * s on v_mfma_f32_32x32x16_f16. Weights are widened to
//                          fp16 exactly (integers), activations rounded to fp16 as the reference does
//                          (kernels.cuh:306-307), fp32 accumulation, the row scale applied last. Workgroup tile 128
//                          weight rows x 128 tokens, 4 wavefronts of 64 x 64, K steps of 32 double-buffered in LDS,
//                          up to three workgroups per CU; the blocks of a token tile run on one XCD (its activations
//                          are read into one L2).
//   gemm_ws_kernel         The same product and sum order with split roles: 4 wavefronts widen the next K step into
//                          LDS while 4 run the MFMAs of this one. Used when the grid fits the chip in one pass.
//   quantize_gs64_kernel   fp16 rows -> int4 / int6 codes + a scale per 64-input group (bit-exact).
//   gemv_mat_kernel        the GEMV of the int4 / int6 / fp16 forms: a lane per 16-weight unit of R rows, each unit
//                          summed in order and scaled, wavefront and part sums as gemv_kernel.
//   gemm_kernel<form>      the same tiled MFMA GEMM for every form: the staging widens int4 / int6 weights times
//                          their group scale to fp16 (or copies fp16 weights) where int8 is widened exactly.
#include <algorithm>
#include <cstdlib>
#include "common.hpp"

namespace moex {

namespace {

// sum over the wavefront, every lane receives it: DPP within each 16-lane row (rotate by 8 and 4, then the quad
// swaps), then the 16- and 32-lane swaps (v_permlane16/32_swap). All VALU: the ds_bpermute round trips of __shfl_xor
// were most of a GEMV's time after its loads had landed (o_proj, 2 rows: 9.0 -> 6.2 us without them)
template <int CTRL> __device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0x128>(v);  // row_ror:8
    v += dpp_f<0x124>(v);  // row_ror:4
    v += dpp_f<0x4e>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_f<0xb1>(v);   // quad_perm [1, 0, 3, 2]
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
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

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int GV_R = 8;       // weight rows of a row group
// 16-byte chunks per lane and row loaded before any is used: 16 KB per wavefront in flight, 8 KB from NT = 5 on
// (registers)
template <int NT> constexpr int gv_u() { return NT <= 4 ? 2 : 1; }
constexpr int GV_WAVES = 8;   // wavefronts per workgroup

// A grid of nb workgroups; in round j, wavefront wv of workgroup b takes row group b + nb * (wv / KS + j * 8 / KS)
// over the KS-th part wv % KS of I, and the KS partial sums of a group are added in LDS in part order. KS (1, 2, 4
// or 8) depends on O and I only, so the sum order of a row never depends on NT.
template <int NT>
__global__ void __launch_bounds__(64 * GV_WAVES) gemv_kernel(const int8_t* __restrict__ q, const float* __restrict__ s,
                                                             const float* __restrict__ x, float* __restrict__ y, int I,
                                                             int O, int KS) {
    constexpr int GV_U = gv_u<NT>();
    extern __shared__ __align__(16) float xs[];  // [NT][I], then the partial sums [GV_WAVES][NT][GV_R]
    float* red = xs + NT * I;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nb = gridDim.x;
    const int ngroups = (O + GV_R - 1) / GV_R, gpr = GV_WAVES / KS;  // groups per workgroup and round
    const int rounds = (ngroups + nb * gpr - 1) / (nb * gpr);
    const int part = wv % KS, slice = I / 16 / KS, cb = part * slice, ce = cb + slice;  // 16-byte chunks of a row
    u32x4 w[GV_U][GV_R];
#define GV_LOAD(g_, c0_)                                                                                         \
    do {                                                                                                         \
        _Pragma("unroll") for (int u = 0; u < GV_U; u++)                                                         \
        _Pragma("unroll") for (int r = 0; r < GV_R; r++) {                                                       \
            const u32x4* row_ = reinterpret_cast<const u32x4*>(q + (size_t)min((g_) * GV_R + r, O - 1) * I);     \
            const int c_ = (c0_) + 64 * u + lane;                                                                \
            w[u][r] = c_ < ce ? __builtin_nontemporal_load(row_ + c_) : u32x4{0u, 0u, 0u, 0u};                  \
        }                                                                                                        \
    } while (0)
    for (int e = tid; e < NT * I / 4; e += 64 * GV_WAVES)
        reinterpret_cast<float4*>(xs)[e] = reinterpret_cast<const float4*>(x)[e];
    __syncthreads();
    for (int j = 0; j < rounds; j++) {
        const int g = blockIdx.x + nb * (wv / KS + j * gpr);
        if (g < ngroups) {
            float acc[NT][GV_R];
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int r = 0; r < GV_R; r++) acc[t][r] = 0.f;
            for (int c0 = cb; c0 < ce; c0 += 64 * GV_U) {
                GV_LOAD(g, c0);
#pragma unroll
                for (int u = 0; u < GV_U; u++) {
                    const int c = c0 + 64 * u + lane;
                    if (c >= ce) continue;  // only when a part is shorter than 64 chunks (I % 1024 != 0)
#pragma unroll
                    for (int t = 0; t < NT; t++) {
#pragma unroll
                        for (int d = 0; d < 4; d++) {
                            const float4 xv = reinterpret_cast<const float4*>(xs + t * I)[4 * c + d];
#pragma unroll
                            for (int r = 0; r < GV_R; r++) {
                                const uint32_t wd = w[u][r][d];
                                acc[t][r] += (float)(int8_t)(wd) * xv.x;
                                acc[t][r] += (float)(int8_t)(wd >> 8) * xv.y;
                                acc[t][r] += (float)(int8_t)(wd >> 16) * xv.z;
                                acc[t][r] += (float)(int8_t)(wd >> 24) * xv.w;
                            }
                        }
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int r = 0; r < GV_R; r++) {
                    const float v = wave_sum(acc[t][r]);
                    if (lane == 0) red[(wv * NT + t) * GV_R + r] = v;
                }
        }
        __syncthreads();
        if (g < ngroups && part == 0 && lane < NT * GV_R) {
            const int t = lane / GV_R, r = lane % GV_R, o = g * GV_R + r;
            float v = red[(wv * NT + t) * GV_R + r];
            for (int p = 1; p < KS; p++) v += red[((wv + p) * NT + t) * GV_R + r];
            if (o < O) y[(size_t)t * O + o] = v * s[o];
        }
        __syncthreads();  // the partial sums are read before the next round writes them
    }
#undef GV_LOAD
}

// The same product when every wavefront has at most one row group and one load step (rounds = 1, a part of at most
// 64 * GV_U chunks: the attention's qkv and o shapes). Without loops every load goes out at the start; each lane reads
// its inputs straight from L2, so the products wait only for their own rows. Same sum order as gemv_kernel.
template <int NT, int R>
__global__ void __launch_bounds__(64 * GV_WAVES) gemv1_kernel(const int8_t* __restrict__ q, const float* __restrict__ s,
                                                              const float* __restrict__ x, float* __restrict__ y, int I,
                                                              int O, int KS) {
    constexpr int GV_U = gv_u<NT>();
    extern __shared__ __align__(16) float red[];  // the partial sums [GV_WAVES][NT][R] (R weight rows a group)
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nb = gridDim.x;
    const int ngroups = (O + R - 1) / R;
    const int part = wv % KS, slice = I / 16 / KS, cb = part * slice, ce = cb + slice;
    const int g = blockIdx.x + nb * (wv / KS);
    const bool on = g < ngroups;
    // the lane's 16 inputs of each row of x first (read from L2 by every wavefront of this part; no LDS copy and no
    // barrier before the products), then the weights, so the products of the first weight rows start while the
    // later rows are still arriving
    float4 xv[GV_U][NT][4];
#pragma unroll
    for (int u = 0; u < GV_U; u++) {
        if (cb + 64 * u >= ce) continue;  // a step past the part (wave-uniform): nothing to load
        const int c = min(cb + 64 * u + lane, I / 16 - 1);
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int d = 0; d < 4; d++) xv[u][t][d] = reinterpret_cast<const float4*>(x + (size_t)t * I)[4 * c + d];
    }
    u32x4 w[GV_U][R];
#pragma unroll
    for (int u = 0; u < GV_U; u++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            const u32x4* row = reinterpret_cast<const u32x4*>(q + (size_t)min(min(g, ngroups - 1) * R + r, O - 1) * I);
            const int c = cb + 64 * u + lane;
            w[u][r] = on && c < ce ? __builtin_nontemporal_load(row + c) : u32x4{0u, 0u, 0u, 0u};
        }
    // the row scale of this lane's output, loaded now so that its round trip overlaps the weights'
    const float so = s[min(min(g, ngroups - 1) * R + lane % R, O - 1)];
    float acc[NT][R];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[t][r] = 0.f;
#pragma unroll
    for (int u = 0; u < GV_U; u++) {
        const int c = cb + 64 * u + lane;
        if (c >= ce) continue;
#pragma unroll
        for (int t = 0; t < NT; t++) {
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const float4 xq = xv[u][t][d];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t wd = w[u][r][d];
                    acc[t][r] += (float)(int8_t)(wd) * xq.x;
                    acc[t][r] += (float)(int8_t)(wd >> 8) * xq.y;
                    acc[t][r] += (float)(int8_t)(wd >> 16) * xq.z;
                    acc[t][r] += (float)(int8_t)(wd >> 24) * xq.w;
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float v = wave_sum(acc[t][r]);
            if (lane == 0) red[(wv * NT + t) * R + r] = v;
        }
    __syncthreads();
    if (on && part == 0 && lane < NT * R) {
        const int t = lane / R, r = lane % R, o = g * R + r;
        float v = red[(wv * NT + t) * R + r];
        for (int p = 1; p < KS; p++) v += red[((wv + p) * NT + t) * R + r];
        if (o < O) y[(size_t)t * O + o] = v * so;
    }
}

// ---- prefill GEMM ----
constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 32;
constexpr int GM_LD = GM_BK + 8;  // halves per LDS row (80 B: conflict-free 16-byte operand reads)

// The weight forms of a dense matrix (struct Mat, kernels.cuh:186-196): int8 with a row scale, int4 and int6 with a
// scale per 64 inputs (gs64), fp16.
enum { MF_I8 = 0, MF_Q4 = 1, MF_Q6 = 2, MF_F16 = 3 };

// A product rounded to fp32 before anything else rounds it: without the barrier the compiler may fuse a multiply
// with its fp16 conversion (v_fma_mix*), one rounding instead of the reference's two.
__device__ __forceinline__ float r32(float x) {
    asm volatile("" : "+v"(x));
    return x;
}
// 16 weights of one row at k .. k + 15 (k % 16 == 0) -> 8 dwords of fp16 pairs, as the reference's GEMMs widen them:
// int8 exactly (row scale applied after the sums); int4 / int6 times the group scale in fp32, then rounded to fp16
// (kernels.cuh:276-279, 313-317: __float2half / __floats2half2_rn of (float)v * s); fp16 as stored.
struct WStage {
    uint4 a;      // int8: 16 codes; int4 / int6: .x, .y the 16 low nibbles; fp16: halves 0-7
    uint4 b;      // fp16: halves 8-15
    uint32_t h;   // int6: the 16 high 2-bit fields
    float sc;     // int4 / int6: the group scale
};
template <int FMT>
__device__ __forceinline__ void wstage_load(WStage& w, const void* W, const uint8_t* Wh, const float* s, size_t row,
                                            int I, int k) {
    if constexpr (FMT == MF_I8) {
        w.a = *reinterpret_cast<const uint4*>(reinterpret_cast<const int8_t*>(W) + row * I + k);
    } else if constexpr (FMT == MF_F16) {
        const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(W) + row * I + k);
        w.a = p[0];
        w.b = p[1];
    } else {
        const uint2 lo = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(W) + row * (I / 2) + k / 2);
        w.a = make_uint4(lo.x, lo.y, 0u, 0u);
        if constexpr (FMT == MF_Q6) w.h = *reinterpret_cast<const uint32_t*>(Wh + row * (I / 4) + k / 4);
        w.sc = s[row * (I / 64) + k / 64];
    }
}
template <int FMT>
__device__ __forceinline__ void wstage_widen(const WStage& w, bool ok, uint32_t (&h)[8]) {
    if constexpr (FMT == MF_I8) {
        i8x4_to_h4(ok ? w.a.x : 0u, h[0], h[1]);
        i8x4_to_h4(ok ? w.a.y : 0u, h[2], h[3]);
        i8x4_to_h4(ok ? w.a.z : 0u, h[4], h[5]);
        i8x4_to_h4(ok ? w.a.w : 0u, h[6], h[7]);
    } else if constexpr (FMT == MF_F16) {
        h[0] = ok ? w.a.x : 0u; h[1] = ok ? w.a.y : 0u; h[2] = ok ? w.a.z : 0u; h[3] = ok ? w.a.w : 0u;
        h[4] = ok ? w.b.x : 0u; h[5] = ok ? w.b.y : 0u; h[6] = ok ? w.b.z : 0u; h[7] = ok ? w.b.w : 0u;
    } else {
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const uint32_t nib = ((e < 8 ? w.a.x : w.a.y) >> (4 * (e & 7))) & 15u;
            int q;
            if constexpr (FMT == MF_Q4) q = (int)nib - (int)((nib & 8u) << 1);       // two's complement nibble
            else q = (int)(nib | (((w.h >> (2 * e)) & 3u) << 4)) - 32;               // 6-bit code, offset 32
            v[e] = r32((float)q * w.sc);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = ok ? h22u(half2_t{(_Float16)v[2 * i], (_Float16)v[2 * i + 1]}) : 0u;
    }
}

template <int FMT>
__global__ void __launch_bounds__(256, 3) gemm_kernel(const void* __restrict__ W, const uint8_t* __restrict__ Wh,
                                                   const float* __restrict__ s, const _Float16* __restrict__ X,
                                                   float* __restrict__ Y, int S, int I, int O) {
    __shared__ __align__(16) _Float16 lds[2][2][GM_BM * GM_LD];  // [buffer][W, X][row][k]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, r = lane & 31, h32 = lane >> 5;
    // XCD-aware order (block b runs on XCD b % 8): with the token tiles a multiple of 8, XCD x takes token tiles
    // x * spx .. x * spx + spx - 1 against every weight tile, so each token tile is read into one L2 only
    const int nO = (O + GM_BM - 1) / GM_BM, nS = (S + GM_BN - 1) / GM_BN, bid = blockIdx.x;
    int ot, stl;
    if (nS % 8 == 0) {
        const int spx = nS / 8, i = bid >> 3;
        ot = i / spx;
        stl = (bid & 7) * spx + i % spx;
    } else {
        ot = bid % nO;
        stl = bid / nO;
    }
    const int o0 = ot * GM_BM, s0 = stl * GM_BN;
    const int wo = (wv >> 1) * 64, ws = (wv & 1) * 64;  // this wavefront's 64 x 64 block of the tile
    // staging: thread tid owns 16 weights (row tid/2, k 16*(tid%2)) and 16 activations (token tid/2, same k)
    const int sr = tid >> 1, sk = (tid & 1) * 16;
    const bool wok = o0 + sr < O, xok = s0 + sr < S;
    const size_t wrow = (size_t)min(o0 + sr, O - 1);
    const _Float16* xp = X + (size_t)min(s0 + sr, S - 1) * I + sk;
    WStage wreg;
    uint4 xreg[2];
    auto load = [&](int k0) {
        wstage_load<FMT>(wreg, W, Wh, s, wrow, I, k0 + sk);
#pragma unroll
        for (int j = 0; j < 2; j++) xreg[j] = reinterpret_cast<const uint4*>(xp + k0)[j];
    };
    auto store = [&](int b) {
        uint32_t h[8];
        wstage_widen<FMT>(wreg, wok, h);
        uint4* wd = reinterpret_cast<uint4*>(&lds[b][0][sr * GM_LD + sk]);
        wd[0] = make_uint4(h[0], h[1], h[2], h[3]);
        wd[1] = make_uint4(h[4], h[5], h[6], h[7]);
        uint4* xd = reinterpret_cast<uint4*>(&lds[b][1][sr * GM_LD + sk]);
        xd[0] = xok ? xreg[0] : make_uint4(0u, 0u, 0u, 0u);
        xd[1] = xok ? xreg[1] : make_uint4(0u, 0u, 0u, 0u);
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
        const float so = FMT == MF_I8 ? s[o] : 1.f;  // the group scales are in the widened weights
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int t = s0 + ws + 32 * j + 8 * (e >> 2) + 4 * h32 + (e & 3);
                if (t < S) Y[(size_t)t * O + o] = FMT == MF_I8 ? acc[i][j][e] * so : acc[i][j][e];
            }
    }
}

// Activations rounded to fp16 once (round to nearest even, as kernels.cuh:306-307 rounds them inside gemm_i8_k): the
// GEMM tiles re-read them once per weight tile, so fp16 halves that traffic and takes the rounding off the staging.
__global__ void __launch_bounds__(256) round_f16_kernel(const float4* __restrict__ X, uint2* __restrict__ Xh, size_t n4) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        const float4 v = X[i];
        Xh[i] = make_uint2(h22u(half2_t{(_Float16)v.x, (_Float16)v.y}), h22u(half2_t{(_Float16)v.z, (_Float16)v.w}));
    }
}

constexpr int GEMM_WS_MAX_BLOCKS = 512;  // 2 workgroups x 256 CUs
constexpr int GEMM_MIN_KSTEPS = 16;        // K steps of a split, at least

// Sum of the K splits of gemm_ws_kernel, in split order (deterministic), times the row scale (int8; s = nullptr: none).
__global__ void __launch_bounds__(256) gemm_reduce_kernel(const float* __restrict__ part, const float* __restrict__ s,
                                                          float* __restrict__ Y, int S, int O, int nks) {
    const size_t n = (size_t)S * O;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        float a = 0.f;
        for (int k = 0; k < nks; k++) a += part[k * n + i];
        Y[i] = s ? a * s[i % O] : a;  // no row scale for the group-scaled forms
    }
}

// Warp-specialised variant: wavefronts 4-7 load and widen the next K step into the other LDS buffer while
// wavefronts 0-3 run the MFMAs of this one (one barrier per K step), so the staging VALU work runs beside the MFMAs.
template <int FMT>
__global__ void __launch_bounds__(512, 2) gemm_ws_kernel(const void* __restrict__ W, const uint8_t* __restrict__ Wh,
                                                         const float* __restrict__ s, const _Float16* __restrict__ X,
                                                         float* __restrict__ Y, int S, int I, int O, int nks,
                                                         float* __restrict__ part) {
    __shared__ __align__(16) _Float16 lds[2][2][GM_BM * GM_LD];  // [buffer][W, X][row][k]
    const int nO = (O + GM_BM - 1) / GM_BM, nS = (S + GM_BN - 1) / GM_BN, tiles = nO * nS;
    const int ks = blockIdx.x / tiles, bid = blockIdx.x % tiles;  // K split ks of tile bid (nks = 1: no split)
    const int kb = ks * (I / GM_BK) / nks, nk = (ks + 1) * (I / GM_BK) / nks - kb;
    int ot, stl;
    if (nS % 8 == 0) {
        const int spx = nS / 8, i = bid >> 3;
        ot = i / spx;
        stl = (bid & 7) * spx + i % spx;
    } else {
        ot = bid % nO;
        stl = bid / nO;
    }
    const int o0 = ot * GM_BM, s0 = stl * GM_BN;
    if (threadIdx.x >= 256) {
        // ---- staging: thread t owns 16 weights (row t/2, k 16*(t%2)) and 16 activations (token t/2, same k) ----
        const int tid = threadIdx.x - 256, sr = tid >> 1, sk = (tid & 1) * 16;
        const bool wok = o0 + sr < O, xok = s0 + sr < S;
        const size_t wrow = (size_t)min(o0 + sr, O - 1);
        const _Float16* xp = X + (size_t)min(s0 + sr, S - 1) * I + kb * GM_BK + sk;
        WStage wreg;
        uint4 xreg[2];
        auto load = [&](int k0) {
            wstage_load<FMT>(wreg, W, Wh, s, wrow, I, kb * GM_BK + k0 + sk);
#pragma unroll
            for (int j = 0; j < 2; j++) xreg[j] = reinterpret_cast<const uint4*>(xp + k0)[j];
        };
        auto store = [&](int b) {
            uint32_t h[8];
            wstage_widen<FMT>(wreg, wok, h);
            uint4* wd = reinterpret_cast<uint4*>(&lds[b][0][sr * GM_LD + sk]);
            wd[0] = make_uint4(h[0], h[1], h[2], h[3]);
            wd[1] = make_uint4(h[4], h[5], h[6], h[7]);
            uint4* xd = reinterpret_cast<uint4*>(&lds[b][1][sr * GM_LD + sk]);
            xd[0] = xok ? xreg[0] : make_uint4(0u, 0u, 0u, 0u);
            xd[1] = xok ? xreg[1] : make_uint4(0u, 0u, 0u, 0u);
        };
        load(0);
        store(0);
        if (nk > 1) load(GM_BK);
        __syncthreads();
        for (int kt = 0; kt < nk; kt++) {
            if (kt + 1 < nk) {
                store((kt + 1) & 1);  // the buffer the computing wavefronts finished at the last barrier
                if (kt + 2 < nk) load((kt + 2) * GM_BK);
            }
            __syncthreads();
        }
        return;
    }
    // ---- computing wavefronts ----
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, r = lane & 31, h32 = lane >> 5;
    const int wo = (wv >> 1) * 64, ws = (wv & 1) * 64;  // this wavefront's 64 x 64 block of the tile
    float16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int b = kt & 1;
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
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int o = o0 + wo + 32 * i + r;
        if (o >= O) continue;
        const float so = nks > 1 || FMT != MF_I8 ? 1.f : s[o];  // a K split leaves the scale to the reduction
        float* Yo = nks > 1 ? part + (size_t)ks * S * O : Y;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int t = s0 + ws + 32 * j + 8 * (e >> 2) + 4 * h32 + (e & 3);
                if (t < S) Yo[(size_t)t * O + o] = acc[i][j][e] * so;
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
    const int groups = (O + GV_R - 1) / GV_R;
    int ks = 1;  // split each row over up to 8 wavefronts until ~4 wavefronts per CU have work
    while (ks < GV_WAVES && groups * ks < 1024 && (I / 16) % (128 * ks) == 0) ks *= 2;
    static const int cus = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            return v;
        return 256;
    }();
    const int nb = std::min(cus, groups * ks);
    const size_t lds = (size_t)NT * I * 4 + GV_WAVES * NT * GV_R * 4;
    const bool one = groups <= nb * (GV_WAVES / ks) && I / 16 / ks <= 64 * gv_u<NT>();
    if (one) {
        // groups of 4 rows when groups of 8 would leave half the wavefronts without work (o_proj): every wavefront
        // then has work, half as much, and the sums are the same (a row's sum order does not depend on the group)
        if ((O + 3) / 4 * ks <= nb * GV_WAVES && groups * ks * 2 <= nb * GV_WAVES)
            hipLaunchKernelGGL((gemv1_kernel<NT, 4>), dim3(nb), dim3(64 * GV_WAVES), (size_t)GV_WAVES * NT * 4 * 4, st,
                               q, s, x, y, I, O, ks);
        else
            hipLaunchKernelGGL((gemv1_kernel<NT, GV_R>), dim3(nb), dim3(64 * GV_WAVES), (size_t)GV_WAVES * NT * GV_R * 4,
                               st, q, s, x, y, I, O, ks);
    } else {
        hipLaunchKernelGGL(gemv_kernel<NT>, dim3(nb), dim3(64 * GV_WAVES), lds, st, q, s, x, y, I, O, ks);
    }
    MOEX_LAUNCHED();
}

// ---- int4 / int6 gs64 quantizers (quantize_rows_q4_k, quantize_rows_q6_k: kernels.cuh:552-590) ----
// A workgroup per row; each wavefront takes 64-weight groups g = w, w + 4, .., a lane per weight. Scale = group absmax
// / 7 (int4) or / 31 (int6), 1 for an all-zero group; codes round-half-even(w / scale) clamped to [-8, 7] /
// [-32, 31] (int6 stored + 32). Packing: weight i's nibble at bits 4 (i % 2) of byte i / 2 of the row's low plane
// (low nibble first); int6 adds its high 2 bits at bits 2 (i % 4) of byte i / 4 of the high plane. The lanes OR their
// fields together across 8 (nibbles) or 16 (2-bit fields) lanes and one lane writes the dword.
template <bool SIX>
__global__ void __launch_bounds__(256) quantize_gs64_kernel(const uint16_t* __restrict__ W, uint8_t* __restrict__ q,
                                                            uint8_t* __restrict__ qh, float* __restrict__ s, int I) {
    const size_t row = blockIdx.x;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, G = I / 64;
    const _Float16* wr = reinterpret_cast<const _Float16*>(W) + row * I;
    for (int g = wv; g < G; g += 4) {
        const float w = (float)wr[g * 64 + lane];
        float m = fabsf(w);
#pragma unroll
        for (int o = 32; o; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float sc = m > 0.f ? m / (SIX ? 31.f : 7.f) : 1.f;
        uint32_t lo, hi = 0;
        if (SIX) {
            const uint32_t u = (uint32_t)((int)fminf(31.f, fmaxf(-32.f, __builtin_rintf(w / sc))) + 32);
            lo = (u & 15u) << (4 * (lane & 7));
            hi = (u >> 4) << (2 * (lane & 15));
        } else {
            const int v = max(-8, min(7, (int)__builtin_rintf(w / sc)));
            lo = ((uint32_t)v & 15u) << (4 * (lane & 7));
        }
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) lo |= __shfl_xor(lo, o);
        if ((lane & 7) == 0) reinterpret_cast<uint32_t*>(q + row * (I / 2) + g * 32)[lane >> 3] = lo;
        if (SIX) {
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) hi |= __shfl_xor(hi, o);
            if ((lane & 15) == 0) reinterpret_cast<uint32_t*>(qh + row * (I / 4) + g * 16)[lane >> 4] = hi;
        }
        if (lane == 0) s[row * G + g] = sc;
    }
}

// ---- GEMV of the int4 / int6 / fp16 forms (gemv_q4_k, gemv_q6_k, gemv_f16_k: kernels.cuh:68-93,486-550) ----
// y[t][o] = sum over the row's 16-weight units c of (sum_k w[o][16c + k] x[t][16c + k]) * scale[o][c / 4] (fp16: no
// scale), fp32 sums. Layout as gemv_kernel: a wavefront takes R rows over the KS-th part of the row's units, a lane
// per unit (8 B of int4, 8 + 4 B of int6, 32 B of fp16 a row), reads its 16 inputs per row of x from L2, sums the
// unit in k order, and the KS parts of a row are added in LDS in part order. KS and R depend on O, I and the form
// only, so every row of a multi-row call is bit-identical to the same row alone.
template <int FMT>
struct MatUnit {
    uint4 a[FMT == MF_F16 ? 2 : 1];  // int4 / int6: .x, .y the 16 low nibbles; fp16: 16 halves
    uint32_t h;                      // int6: the 16 high 2-bit fields
    float sc;
};
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <int FMT>
__device__ __forceinline__ void mat_unit_load(MatUnit<FMT>& u, const uint8_t* W, const uint8_t* Wh, const float* s,
                                              size_t row, int I, int c) {
    if constexpr (FMT == MF_F16) {
        const u32x4* p = reinterpret_cast<const u32x4*>(W + (row * I + 16 * (size_t)c) * 2);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const u32x4 v = __builtin_nontemporal_load(p + i);
            u.a[i] = make_uint4(v[0], v[1], v[2], v[3]);
        }
    } else {
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(W + row * (I / 2)) + c);
        u.a[0] = make_uint4(v[0], v[1], 0u, 0u);
        if constexpr (FMT == MF_Q6) u.h = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(Wh + row * (I / 4)) + c);
        u.sc = s[row * (I / 64) + c / 4];
    }
}
template <int FMT>
__device__ __forceinline__ float mat_unit_dot(const MatUnit<FMT>& u, const float4 (&x)[4]) {
    float d = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float xv[4] = {x[j].x, x[j].y, x[j].z, x[j].w};
#pragma unroll
        for (int n = 0; n < 4; n++) {
            const int k = 4 * j + n;
            float w;
            if constexpr (FMT == MF_F16) {
                const uint4& q = u.a[k / 8];
                const uint32_t d2 = ((k / 2) & 3) == 0 ? q.x : ((k / 2) & 3) == 1 ? q.y : ((k / 2) & 3) == 2 ? q.z : q.w;
                w = (float)u2h2(d2)[k & 1];
            } else {
                const uint32_t dw = k < 8 ? u.a[0].x : u.a[0].y;
                if constexpr (FMT == MF_Q4) {
                    w = (float)(int)__builtin_amdgcn_sbfe(dw, 4 * (k & 7), 4);  // the signed nibble (the builtin returns it as unsigned)
                } else {
                    const uint32_t hb = (u.h >> (2 * k)) & 3u;
                    w = (float)((int)(((dw >> (4 * (k & 7))) & 15u) | (hb << 4)) - 32);
                }
            }
            d = fmaf(w, xv[n], d);
        }
    }
    return FMT == MF_F16 ? d : d * u.sc;
}
constexpr int GM_WAVES = 8;
template <int FMT, int NT, int R>
__global__ void __launch_bounds__(64 * GM_WAVES) gemv_mat_kernel(const uint8_t* __restrict__ W,
                                                                 const uint8_t* __restrict__ Wh,
                                                                 const float* __restrict__ s,
                                                                 const float* __restrict__ x, float* __restrict__ y,
                                                                 int I, int O, int KS) {
    __shared__ float red[GM_WAVES][NT][R];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nb = gridDim.x;
    const int U = I / 16, ngroups = (O + R - 1) / R, gpr = GM_WAVES / KS;
    const int rounds = (ngroups + nb * gpr - 1) / (nb * gpr);
    const int part = wv % KS, slice = U / KS, cb = part * slice, ce = cb + slice;
    for (int j = 0; j < rounds; j++) {
        const int g = blockIdx.x + nb * (wv / KS + j * gpr);
        if (g < ngroups) {
            float acc[NT][R];
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int r = 0; r < R; r++) acc[t][r] = 0.f;
            for (int c = cb + lane; c < ce; c += 64) {
                MatUnit<FMT> u[R];
#pragma unroll
                for (int r = 0; r < R; r++) mat_unit_load<FMT>(u[r], W, Wh, s, (size_t)min(g * R + r, O - 1), I, c);
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    float4 xv[4];
                    const float4* xp = reinterpret_cast<const float4*>(x + (size_t)t * I + 16 * (size_t)c);
#pragma unroll
                    for (int i = 0; i < 4; i++) xv[i] = xp[i];
#pragma unroll
                    for (int r = 0; r < R; r++) acc[t][r] += mat_unit_dot<FMT>(u[r], xv);
                }
            }
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const float v = wave_sum(acc[t][r]);
                    if (lane == 0) red[wv][t][r] = v;
                }
        }
        __syncthreads();
        if (g < ngroups && part == 0 && lane < NT * R) {
            const int t = lane / R, r = lane % R, o = g * R + r;
            float v = red[wv][t][r];
            for (int p = 1; p < KS; p++) v += red[wv + p][t][r];
            if (o < O) y[(size_t)t * O + o] = v;
        }
        __syncthreads();  // the partial sums are read before the next round writes them
    }
}

int dense_cus() {
    static const int cus = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            return v;
        return 256;
    }();
    return cus;
}

template <int FMT, int NT>
void launch_gemv_mat_t(const uint8_t* W, const uint8_t* Wh, const float* s, const float* x, float* y, int I, int O,
                       hipStream_t st) {
    // parts of at least 64 units (one load step a lane wherever I allows: a second, dependent step cost the qkv
    // shape 8.4 -> 6.4 us for int4); rows per wavefront: 4, fewer while the grid would leave CUs without a
    // workgroup; up to two workgroups per CU at once before the kernel loops over further rounds
    const int U = I / 16, cus = dense_cus();
    int ks = 1;
    while (ks < GM_WAVES && U % (2 * ks) == 0 && U / (2 * ks) >= 64) ks *= 2;
    const int gpr = GM_WAVES / ks;
    int R = 4;
    while (R > 1 && ((O + R - 1) / R + gpr - 1) / gpr < cus) R /= 2;
    const int nb = std::min(2 * cus, ((O + R - 1) / R + gpr - 1) / gpr);
    if (R == 4)
        hipLaunchKernelGGL((gemv_mat_kernel<FMT, NT, 4>), dim3(nb), dim3(64 * GM_WAVES), 0, st, W, Wh, s, x, y, I, O, ks);
    else if (R == 2)
        hipLaunchKernelGGL((gemv_mat_kernel<FMT, NT, 2>), dim3(nb), dim3(64 * GM_WAVES), 0, st, W, Wh, s, x, y, I, O, ks);
    else
        hipLaunchKernelGGL((gemv_mat_kernel<FMT, NT, 1>), dim3(nb), dim3(64 * GM_WAVES), 0, st, W, Wh, s, x, y, I, O, ks);
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
    // Both kernels sum in the same order (identical results). A grid that fits the chip in one pass of two
    // workgroups per CU runs the warp-specialised kernel; a larger one the 4-wavefront kernel, whose extra
    // workgroups in flight hide the staging better than the split roles do (measured on the qkv/o_proj shapes).
    const size_t n4 = (size_t)S * I / 4;  // I % 32 == 0
    _Float16* Xh = reinterpret_cast<_Float16*>(stream_workspace(n4 * 8, st, 2));
    if (!Xh) {
        report(hipErrorOutOfMemory, __FILE__, __LINE__);
        return;
    }
    hipLaunchKernelGGL(round_f16_kernel, dim3((unsigned)std::min<size_t>((n4 + 255) / 256, 4096)), dim3(256), 0, st,
                       reinterpret_cast<const float4*>(X), reinterpret_cast<uint2*>(Xh), n4);
    MOEX_LAUNCHED();
    const int blocks = ((O + GM_BM - 1) / GM_BM) * ((S + GM_BN - 1) / GM_BN);
    if (blocks <= GEMM_WS_MAX_BLOCKS) {
        // a grid short of one workgroup per CU splits K (each split at least GEMM_MIN_KSTEPS steps), summed by a
        // second kernel; at one per CU and above, the partials' traffic cost more than the extra workgroups gained
        int nks = 2 * blocks >= GEMM_WS_MAX_BLOCKS ? 1 : std::max(1, std::min(GEMM_WS_MAX_BLOCKS / blocks, I / GM_BK / GEMM_MIN_KSTEPS));
        float* part = nullptr;
        if (nks > 1) {
            part = reinterpret_cast<float*>(stream_workspace((size_t)nks * S * O * sizeof(float), st, 3));
            if (!part) nks = 1;
        }
        hipLaunchKernelGGL(gemm_ws_kernel<MF_I8>, dim3(blocks * nks), dim3(512), 0, st, q, nullptr, s, Xh, Y, S, I, O, nks,
                           part);
        if (nks > 1) {
            MOEX_LAUNCHED();
            hipLaunchKernelGGL(gemm_reduce_kernel, dim3(1024), dim3(256), 0, st, part, s, Y, S, O, nks);
        }
    } else
        hipLaunchKernelGGL(gemm_kernel<MF_I8>, dim3(blocks), dim3(256), 0, st, q, nullptr, s, Xh, Y, S, I, O);
    MOEX_LAUNCHED();
}

void launch_quantize_rows_gs64(const uint16_t* W, uint8_t* q, uint8_t* qh, float* s, int O, int I, bool six,
                               hipStream_t st) {
    if (six) hipLaunchKernelGGL(quantize_gs64_kernel<true>, dim3(O), dim3(256), 0, st, W, q, qh, s, I);
    else hipLaunchKernelGGL(quantize_gs64_kernel<false>, dim3(O), dim3(256), 0, st, W, q, qh, s, I);
    MOEX_LAUNCHED();
}

void launch_gemv_mat(const moex_mat& m, const float* x, float* y, int NT, int I, int O, hipStream_t st) {
    if (m.q4) {
        for (int t = 0; t < NT; t++)
            launch_gemv_mat_t<MF_Q4, 1>(m.q4, nullptr, m.s, x + (size_t)t * I, y + (size_t)t * O, I, O, st);
    } else if (m.q6) {
        switch (NT) {
            case 1: launch_gemv_mat_t<MF_Q6, 1>(m.q6, m.q6h, m.s, x, y, I, O, st); break;
            case 2: launch_gemv_mat_t<MF_Q6, 2>(m.q6, m.q6h, m.s, x, y, I, O, st); break;
            case 3: launch_gemv_mat_t<MF_Q6, 3>(m.q6, m.q6h, m.s, x, y, I, O, st); break;
            case 4: launch_gemv_mat_t<MF_Q6, 4>(m.q6, m.q6h, m.s, x, y, I, O, st); break;
            case 5: launch_gemv_mat_t<MF_Q6, 5>(m.q6, m.q6h, m.s, x, y, I, O, st); break;
            case 6: launch_gemv_mat_t<MF_Q6, 6>(m.q6, m.q6h, m.s, x, y, I, O, st); break;
            case 7: launch_gemv_mat_t<MF_Q6, 7>(m.q6, m.q6h, m.s, x, y, I, O, st); break;
            default: launch_gemv_mat_t<MF_Q6, 8>(m.q6, m.q6h, m.s, x, y, I, O, st); break;
        }
    } else {
        const uint8_t* W = reinterpret_cast<const uint8_t*>(m.f16);
        for (int t = 0; t < NT; t++)
            launch_gemv_mat_t<MF_F16, 1>(W, nullptr, nullptr, x + (size_t)t * I, y + (size_t)t * O, I, O, st);
    }
}

void launch_gemm_mat(const moex_mat& m, const float* X, float* Y, int S, int I, int O, hipStream_t st) {
    const size_t n4 = (size_t)S * I / 4;  // I % 32 == 0
    _Float16* Xh = reinterpret_cast<_Float16*>(stream_workspace(n4 * 8, st, 2));
    if (!Xh) {
        report(hipErrorOutOfMemory, __FILE__, __LINE__);
        return;
    }
    hipLaunchKernelGGL(round_f16_kernel, dim3((unsigned)std::min<size_t>((n4 + 255) / 256, 4096)), dim3(256), 0, st,
                       reinterpret_cast<const float4*>(X), reinterpret_cast<uint2*>(Xh), n4);
    MOEX_LAUNCHED();
    // the int8 GEMM's choice of kernel and K split (launch_gemm_i8); the group scales are in the widened weights, so
    // the split's reduction applies none
    const int blocks = ((O + GM_BM - 1) / GM_BM) * ((S + GM_BN - 1) / GM_BN);
    const void* W = m.q4 ? static_cast<const void*>(m.q4) : m.q6 ? static_cast<const void*>(m.q6)
                                                                 : static_cast<const void*>(m.f16);
    const uint8_t* Wh = m.q4 ? nullptr : m.q6h;
    const float* sg = m.q4 || m.q6 ? m.s : nullptr;
    if (blocks <= GEMM_WS_MAX_BLOCKS) {
        int nks = 2 * blocks >= GEMM_WS_MAX_BLOCKS ? 1 : std::max(1, std::min(GEMM_WS_MAX_BLOCKS / blocks, I / GM_BK / GEMM_MIN_KSTEPS));
        float* part = nullptr;
        if (nks > 1) {
            part = reinterpret_cast<float*>(stream_workspace((size_t)nks * S * O * sizeof(float), st, 3));
            if (!part) nks = 1;
        }
        if (m.q4) hipLaunchKernelGGL(gemm_ws_kernel<MF_Q4>, dim3(blocks * nks), dim3(512), 0, st, W, Wh, sg, Xh, Y, S, I, O, nks, part);
        else if (m.q6) hipLaunchKernelGGL(gemm_ws_kernel<MF_Q6>, dim3(blocks * nks), dim3(512), 0, st, W, Wh, sg, Xh, Y, S, I, O, nks, part);
        else hipLaunchKernelGGL(gemm_ws_kernel<MF_F16>, dim3(blocks * nks), dim3(512), 0, st, W, Wh, sg, Xh, Y, S, I, O, nks, part);
        if (nks > 1) {
            MOEX_LAUNCHED();
            hipLaunchKernelGGL(gemm_reduce_kernel, dim3(1024), dim3(256), 0, st, part, nullptr, Y, S, O, nks);
        }
    } else if (m.q4) {
        hipLaunchKernelGGL(gemm_kernel<MF_Q4>, dim3(blocks), dim3(256), 0, st, W, Wh, sg, Xh, Y, S, I, O);
    } else if (m.q6) {
        hipLaunchKernelGGL(gemm_kernel<MF_Q6>, dim3(blocks), dim3(256), 0, st, W, Wh, sg, Xh, Y, S, I, O);
    } else {
        hipLaunchKernelGGL(gemm_kernel<MF_F16>, dim3(blocks), dim3(256), 0, st, W, Wh, sg, Xh, Y, S, I, O);
    }
    MOEX_LAUNCHED();
}

}  // namespace moex
