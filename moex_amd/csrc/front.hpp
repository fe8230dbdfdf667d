// The q/k front's arithmetic (RMSNorm(1 + w), partial RoPE, the int8 quantizer) over a group of 256 threads in which
// thread d owns dim d of one head row (kernels.cuh:13-41,1185-1236). qk_norm_rope_kernel runs it as a whole block;
// the int8 T = 1 decode kernel runs it in its prologue as two groups of 256 (both calling the same barriers), so the
// rows it appends and the query it scores are bit-identical to the front kernel's. The reductions keep the
// reference's orders: the 32-lane xor tree of warp_sum and the second xor tree over the 8 partials of block_sum (an
// xor-shuffle with offset <= 16 never leaves its 32-lane half of a 64-wide wavefront). Every function turns FP
// contraction off for its own body (the including file may allow it).
#pragma once
#include "common.hpp"

namespace moex {
namespace front {

// The group barrier: __syncthreads(), or (BARE) s_barrier after the wavefront's LDS operations, which leaves vector
// memory operations in flight (a decode kernel's DMA transfers issued before its prologue)
template <bool BARE>
__device__ __forceinline__ void sync() {
    if (BARE) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else __syncthreads();
}

__device__ __forceinline__ float sum32(float v) {  // 32-lane xor tree (kernels.cuh:13-16)
#pragma clang fp contract(off)
#pragma unroll
    for (int o = 16; o; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float max32(float v) {
#pragma clang fp contract(off)
#pragma unroll
    for (int o = 16; o; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
// sum over the group (d = 0..255): 32-lane trees, then the reference's xor tree over the 8 partials (kernels.cuh:19-28)
template <bool BARE = false>
__device__ __forceinline__ float block_sum(float v, float* sh8, int d) {
#pragma clang fp contract(off)
    v = sum32(v);
    sync<BARE>();
    if ((d & 31) == 0) sh8[d >> 5] = v;
    sync<BARE>();
    return ((sh8[0] + sh8[4]) + (sh8[2] + sh8[6])) + ((sh8[1] + sh8[5]) + (sh8[3] + sh8[7]));
}
template <bool BARE = false>
__device__ __forceinline__ float block_max(float v, float* sh8, int d) {
#pragma clang fp contract(off)
    v = max32(v);
    sync<BARE>();
    if ((d & 31) == 0) sh8[d >> 5] = v;
    sync<BARE>();
    float m = sh8[0];
#pragma unroll
    for (int i = 1; i < 8; i++) m = fmaxf(m, sh8[i]);
    return m;
}

// RMSNorm(1 + w) of a head row, then the partial RoPE on dims < rot (kernels.cuh:1197-1209); t: the group's 256-float
// LDS row. Returns dim d of the result.
template <bool BARE = false>
__device__ __forceinline__ float norm_rope(float x, const uint16_t* w, int d, int pos, int rot, float theta, float eps,
                                           float* t, float* sh8) {
#pragma clang fp contract(off)
    const float r = rsqrtf(block_sum<BARE>(x * x, sh8, d) / AHD + eps);
    const float wd = (float)__builtin_bit_cast(_Float16, w[d]);
    x = x * r * (1.f + wd);
    t[d] = x;
    sync<BARE>();
    const int h2 = rot / 2;
    if (d < rot) {
        const int j = d < h2 ? d : d - h2;
        const float ang = (float)pos * powf(theta, -2.f * j / rot);
        const float cs = cosf(ang), sn = sinf(ang);
        x = d < h2 ? t[d] * cs - t[d + h2] * sn : t[d] * cs + t[d - h2] * sn;
    }
    return x;
}

// norm_rope of N rows at once (row i with weights w[i]; t: N LDS rows of 256, sh8: 8 N floats): one set of barriers
// and one angle per dim for all of them, each row's arithmetic that of norm_rope
template <int N, bool BARE>
__device__ __forceinline__ void norm_rope_n(float (&x)[N], const uint16_t* const (&w)[N], int d, int pos, int rot,
                                            float theta, float eps, float* t, float* sh8) {
#pragma clang fp contract(off)
    float v[N];
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = sum32(x[i] * x[i]);
    sync<BARE>();
    if ((d & 31) == 0) {
#pragma unroll
        for (int i = 0; i < N; i++) sh8[8 * i + (d >> 5)] = v[i];
    }
    sync<BARE>();
#pragma unroll
    for (int i = 0; i < N; i++) {
        const float* s8 = sh8 + 8 * i;
        const float r = rsqrtf((((s8[0] + s8[4]) + (s8[2] + s8[6])) + ((s8[1] + s8[5]) + (s8[3] + s8[7]))) / AHD + eps);
        const float wd = (float)__builtin_bit_cast(_Float16, w[i][d]);
        x[i] = x[i] * r * (1.f + wd);
        t[i * AHD + d] = x[i];
    }
    sync<BARE>();
    const int h2 = rot / 2;
    if (d < rot) {
        const int j = d < h2 ? d : d - h2;
        const float ang = (float)pos * powf(theta, -2.f * j / rot);
        const float cs = cosf(ang), sn = sinf(ang);
#pragma unroll
        for (int i = 0; i < N; i++) {
            const float* ti = t + i * AHD;
            x[i] = d < h2 ? ti[d] * cs - ti[d + h2] * sn : ti[d] * cs + ti[d - h2] * sn;
        }
    }
}

// int8 quantizer of a k and a v row (kernels.cuh:1227-1235): absmax / 127 per row, round-half-even of the IEEE
// quotient
template <bool BARE = false>
__device__ __forceinline__ void quant_i8(float x, float vv, float* sh8, int d, int8_t& ck, int8_t& cv, float& sk,
                                         float& sv) {
#pragma clang fp contract(off)
    const float mk = block_max<BARE>(fabsf(x), sh8, d), mv = block_max<BARE>(fabsf(vv), sh8 + 8, d);
    sk = mk > 0.f ? mk / 127.f : 1.f;
    sv = mv > 0.f ? mv / 127.f : 1.f;
    ck = (int8_t)__builtin_rintf(x / sk);
    cv = (int8_t)__builtin_rintf(vv / sv);
}

}  // namespace front
}  // namespace moex
