// The q/k front's arithmetic (RMSNorm(1 + w), partial RoPE, the int8 and TurboQuant quantizers, the WHT) over a group
// of 256 threads in which thread d owns dim d of one head row (kernels.cuh:13-41,1141-1236). qk_norm_rope_kernel
// runs it as a whole block; the T = 1 decode kernels (int8 and turbo) run it in their prologues as two groups of 256
// (both calling the same barriers), so the rows they append and the queries they score are bit-identical to the
// front kernel's. The reductions keep the reference's orders: the 32-lane xor tree of warp_sum, the second xor tree
// over the 8 partials of block_sum and the in-order sum of the four 32-lane partials of each 128-value half (an
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


// TurboQuant constants (kernels.cuh:1123-1139): sign tables, centroid codes, decision thresholds.
static __constant__ float c_S1[128] = {
    -1, 1, 1,-1,-1, 1,-1, 1,-1,-1, 1, 1, 1, 1, 1, 1, 1,-1, 1,-1, 1,-1,-1, 1, 1, 1,-1, 1, 1,-1,-1,-1,
    -1, 1, 1,-1, 1, 1,-1, 1,-1, 1, 1,-1,-1, 1,-1, 1, 1, 1, 1,-1,-1,-1,-1,-1, 1,-1, 1, 1, 1, 1,-1, 1,
    -1,-1, 1,-1,-1,-1, 1,-1,-1,-1, 1,-1,-1,-1, 1, 1, 1,-1,-1, 1, 1, 1,-1,-1, 1, 1,-1, 1, 1,-1, 1,-1,
    -1, 1, 1,-1, 1,-1, 1,-1, 1, 1, 1, 1,-1, 1,-1, 1, 1,-1, 1, 1,-1,-1,-1,-1,-1, 1, 1,-1, 1, 1,-1, 1};
static __constant__ float c_S2[128] = {
     1, 1, 1, 1,-1, 1, 1,-1, 1,-1,-1,-1, 1,-1,-1,-1, 1, 1,-1,-1, 1,-1, 1,-1, 1,-1,-1, 1,-1, 1, 1, 1,
     1, 1,-1,-1,-1, 1,-1,-1,-1,-1,-1,-1, 1, 1, 1,-1, 1,-1, 1, 1, 1,-1,-1, 1,-1,-1,-1,-1,-1,-1, 1, 1,
     1,-1, 1,-1,-1,-1,-1, 1,-1, 1,-1, 1,-1,-1, 1, 1,-1, 1,-1, 1, 1,-1, 1,-1,-1,-1,-1, 1,-1,-1, 1,-1,
     1,-1, 1, 1, 1,-1,-1, 1,-1, 1,-1, 1, 1,-1,-1, 1,-1, 1,-1, 1, 1,-1, 1,-1, 1,-1,-1,-1,-1,-1, 1,-1};
static __constant__ int8_t c_I4[16] = {-127, -96, -75, -58, -44, -31, -18, -6, 6, 18, 31, 44, 58, 75, 96, 127};
static __constant__ int8_t c_I3[8] = {-127, -79, -45, -14, 14, 45, 79, 127};
static __constant__ float c_M4[15] = {-0.212203f, -0.162947f, -0.127026f, -0.097164f, -0.070671f, -0.046174f, -0.022824f, 0.f,
                               0.022824f, 0.046174f, 0.070671f, 0.097164f, 0.127026f, 0.162947f, 0.212203f};
static __constant__ float c_M3[7] = {-0.154496f, -0.092804f, -0.044243f, 0.f, 0.044243f, 0.092804f, 0.154496f};
constexpr float K4 = 0.241529f / 127.f, K3 = 0.190207f / 127.f;  // code scales (kernels.cuh:1135)


// sum over the thread's 128-value half: 32-lane trees, then ((s0 + s1) + s2) + s3 (kernels.cuh:1161-1169)
template <bool BARE = false>
__device__ __forceinline__ float half_sum(float v, float* sh8, int d) {
#pragma clang fp contract(off)
    v = sum32(v);
    const int g = d >> 5;
    sync<BARE>();
    if ((d & 31) == 0) sh8[g] = v;
    sync<BARE>();
    const int b = g & ~3;
    return ((sh8[b] + sh8[b + 1]) + sh8[b + 2]) + sh8[b + 3];
}

// WHT of both 128-value halves of the group's row (kernels.cuh:1143-1159); dir 0 forward, 1 inverse. Stages 1..32
// are xor-shuffles within the wavefront; stage 64 (dims j and j ^ 64, different wavefronts) goes through sh.
template <bool BARE = false>
__device__ __forceinline__ float wht(float x, float* sh, int dir, int d) {
#pragma clang fp contract(off)
    const int j = d & 127;
    float v = x * (dir ? c_S2[j] : c_S1[j]);
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) {
        const float o = __shfl_xor(v, h);
        v = (d & h) ? o - v : v + o;
    }
    sync<BARE>();
    sh[d] = v;
    sync<BARE>();
    const float a = sh[d & ~64], b = sh[d | 64];
    v = (j & 64) ? a - b : a + b;
    return v * 0.08838834764831845f * (dir ? c_S1[j] : c_S2[j]);
}

// wht of N rows at once (row i in x[i], its stage-64 exchange in sh + i AHD): one pair of barriers for all of them,
// each row's arithmetic that of wht
template <int N, bool BARE>
__device__ __forceinline__ void wht_n(float (&x)[N], float* sh, int dir, int d) {
#pragma clang fp contract(off)
    const int j = d & 127;
    float v[N];
#pragma unroll
    for (int i = 0; i < N; i++) {
        v[i] = x[i] * (dir ? c_S2[j] : c_S1[j]);
#pragma unroll
        for (int h = 1; h < 64; h <<= 1) {
            const float o = __shfl_xor(v[i], h);
            v[i] = (d & h) ? o - v[i] : v[i] + o;
        }
    }
    sync<BARE>();
#pragma unroll
    for (int i = 0; i < N; i++) sh[i * AHD + d] = v[i];
    sync<BARE>();
#pragma unroll
    for (int i = 0; i < N; i++) {
        const float a = sh[i * AHD + (d & ~64)], b = sh[i * AHD + (d | 64)];
        x[i] = ((j & 64) ? a - b : a + b) * 0.08838834764831845f * (dir ? c_S1[j] : c_S2[j]);
    }
}

// TurboQuant code of x (thread d of the row); norm_out = the half's corrected norm (kernels.cuh:1172-1183)
template <int BITS, bool BARE = false>
__device__ __forceinline__ int tq_quant(float x, float* sh, float* sh8, int d, float& norm_out) {
#pragma clang fp contract(off)
    const float n = sqrtf(half_sum<BARE>(x * x, sh8, d));
    const float r = wht<BARE>(n > 1e-20f ? x / n : 0.f, sh, 0, d);
    int idx = 0;
    if (BITS == 4) {
#pragma unroll
        for (int i = 0; i < 15; i++) idx += r >= c_M4[i];
    } else {
#pragma unroll
        for (int i = 0; i < 7; i++) idx += r >= c_M3[i];
    }
    const float c = BITS == 4 ? (float)c_I4[idx] * K4 : (float)c_I3[idx] * K3;
    const float rn = sqrtf(half_sum<BARE>(c * c, sh8, d));
    norm_out = rn > 1e-20f ? n / rn : n;
    return idx;
}

// TurboQuant quantize-append of one row (kernels.cuh:1210-1226): x = post-RoPE k of dim d, vv = raw v of dim d; K
// 4-bit, V 3-bit codes packed as the reference packs them. Every thread of the group computes; store: this group
// writes the cache row.
template <bool BARE = false>
__device__ __forceinline__ void append_turbo(float x, float vv, moex_kv_cache kv, size_t row, float* sh, float* sh8,
                                             int d, bool store) {
#pragma clang fp contract(off)
    const int j = d & 127, b = d >> 7;
    float nk, nv;
    const int ik = tq_quant<4, BARE>(x, sh, sh8, d, nk);
    const int iv = tq_quant<3, BARE>(vv, sh, sh8, d, nv);
    uint8_t* K = reinterpret_cast<uint8_t*>(kv.k) + row * TQ_KB;
    uint8_t* V = reinterpret_cast<uint8_t*>(kv.v) + row * TQ_VB;
    const int ik1 = __shfl_down(ik, 1);
    const int lo = iv & 3;
    const int q4 = lo | (__shfl_down(lo, 1) << 2) | (__shfl_down(lo, 2) << 4) | (__shfl_down(lo, 3) << 6);
    const unsigned long long hb = __ballot(iv & 4);
    if (!store) return;
    if (!(j & 1)) K[b * 64 + j / 2] = (uint8_t)(ik | (ik1 << 4));
    if (!(j & 3)) V[b * 32 + j / 4] = (uint8_t)q4;
    if (!(j & 7)) V[64 + b * 16 + j / 8] = (uint8_t)(hb >> (d & 63));
    if (j == 0) { kv.ks[row * 2 + b] = nk; kv.vs[row * 2 + b] = nv; }
}

// ---- The same arithmetic on one wavefront per head row: lane l owns dims 4l .. 4l + 3 (x[i] = dim 4l + i), so a
// workgroup of 256 threads serves four rows and needs no barrier. The reductions and the WHT reproduce the orders of
// the 256-thread functions above exactly: a 32-lane warp of the reference (dims 32w .. 32w + 31) is lanes 8w .. 8w+7;
// its xor tree pairs dims d and d ^ 16, ^ 8, ^ 4 across lanes (lane ^ 4, ^ 2, ^ 1) and d ^ 2, d ^ 1 inside the lane.
namespace wave {

// every dim gets its reference warp's sum (the 32-lane xor tree: offsets 16, 8, 4, 2, 1)
__device__ __forceinline__ void sum32(float (&v)[4]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int o = 4; o >= 1; o >>= 1)
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] += __shfl_xor(v[i], o);
    float a[4];
#pragma unroll
    for (int i = 0; i < 4; i++) a[i] = v[i] + v[i ^ 2];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = a[i] + a[i ^ 1];
}
// the 8 warp sums (warp w: lane 8w), wave-uniform
__device__ __forceinline__ void warp_sums(const float (&v)[4], float (&s)[8]) {
#pragma unroll
    for (int w = 0; w < 8; w++) s[w] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[0]), 8 * w));
}
// block_sum over the row's 256 dims of v (per dim): the reference's second xor tree over the 8 warp sums
__device__ __forceinline__ float block_sum(float (&v)[4]) {
#pragma clang fp contract(off)
    sum32(v);
    float s[8];
    warp_sums(v, s);
    return ((s[0] + s[4]) + (s[2] + s[6])) + ((s[1] + s[5]) + (s[3] + s[7]));
}
// half_sum of the lane's 128-value half: ((s0 + s1) + s2) + s3 over the half's four warps
__device__ __forceinline__ float half_sum(float (&v)[4], int lane) {
#pragma clang fp contract(off)
    sum32(v);
    float s[8];
    warp_sums(v, s);
    const float h0 = ((s[0] + s[1]) + s[2]) + s[3], h1 = ((s[4] + s[5]) + s[6]) + s[7];
    return lane < 32 ? h0 : h1;
}
__device__ __forceinline__ float row_max(const float (&v)[4]) {
    float m = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    return m;
}

// The RoPE factors of the lane's 4 dims at one position: they depend on the position and the dim only, so the rows
// of one token (every head, and its key row) share them
struct Rope {
    float cs[4], sn[4];
};
__device__ __forceinline__ Rope rope_angles(int lane, int pos, int rot, float theta) {
#pragma clang fp contract(off)
    const int h2 = rot / 2, d0 = 4 * lane;
    // the angles depend on j = d mod h2 only: lane t computes those of j = t and t + 64 (the same expression as the
    // 256-thread function), the rotating lanes take theirs by shuffle
    float ca = 1.f, sa = 0.f, cb = 1.f, sb = 0.f;
    if (lane < h2) {
        const float ang = (float)pos * powf(theta, -2.f * lane / rot);
        ca = cosf(ang);
        sa = sinf(ang);
    }
    if (lane + 64 < h2) {
        const float ang = (float)pos * powf(theta, -2.f * (lane + 64) / rot);
        cb = cosf(ang);
        sb = sinf(ang);
    }
    Rope rp;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int d = d0 + i, j = d < h2 ? d : d - h2;
        const float c0 = __shfl(ca, j & 63), c1 = __shfl(cb, j & 63);  // every lane takes part in every shuffle
        const float s0 = __shfl(sa, j & 63), s1 = __shfl(sb, j & 63);
        rp.cs[i] = j < 64 ? c0 : c1;
        rp.sn[i] = j < 64 ? s0 : s1;
    }
    return rp;
}
// norm_rope on the lane's 4 dims (rot % 8 == 0: a RoPE partner is 4 dims per lane away, same slot); wb: the lane's 4
// fp16 norm weights (w + 4 lane), loaded by the caller. In two steps: the RMSNorm(1 + w) and the partner values,
// then the rotation by rp = rope_angles of the row's position
__device__ __forceinline__ void norm_partner(float (&x)[4], float (&px)[4], uint2 wb, int lane, int rot, float eps) {
#pragma clang fp contract(off)
    float sq[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sq[i] = x[i] * x[i];
    const float r = rsqrtf(block_sum(sq) / AHD + eps);
    const uint16_t wh[4] = {(uint16_t)(wb.x & 0xffffu), (uint16_t)(wb.x >> 16), (uint16_t)(wb.y & 0xffffu),
                            (uint16_t)(wb.y >> 16)};
#pragma unroll
    for (int i = 0; i < 4; i++) x[i] = x[i] * r * (1.f + (float)__builtin_bit_cast(_Float16, wh[i]));
    const int h2 = rot / 2, d0 = 4 * lane;
    const int partner = d0 < h2 ? lane + h2 / 4 : lane - h2 / 4;
#pragma unroll
    for (int i = 0; i < 4; i++) px[i] = __shfl(x[i], partner & 63);
}
__device__ __forceinline__ void rotate(float (&x)[4], const float (&px)[4], const Rope& rp, int lane, int rot) {
#pragma clang fp contract(off)
    const int h2 = rot / 2, d0 = 4 * lane;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int d = d0 + i;
        if (d < rot) x[i] = d < h2 ? x[i] * rp.cs[i] - px[i] * rp.sn[i] : x[i] * rp.cs[i] + px[i] * rp.sn[i];
    }
}
__device__ __forceinline__ void norm_rope(float (&x)[4], uint2 wb, int lane, const Rope& rp, int rot, float eps) {
    float px[4];
    norm_partner(x, px, wb, lane, rot, eps);
    rotate(x, px, rp, lane, rot);
}
__device__ __forceinline__ void norm_rope(float (&x)[4], uint2 wb, int lane, int pos, int rot, float theta, float eps) {
    float px[4];
    norm_partner(x, px, wb, lane, rot, eps);
    rotate(x, px, rope_angles(lane, pos, rot, theta), lane, rot);
}
__device__ __forceinline__ void norm_rope(float (&x)[4], const uint16_t* w, int lane, int pos, int rot, float theta,
                                          float eps) {
    norm_rope(x, *reinterpret_cast<const uint2*>(w + 4 * lane), lane, pos, rot, theta, eps);
}

// wht of both 128-value halves of the row (dir 0 forward, 1 inverse)
__device__ __forceinline__ void wht(float (&x)[4], int dir, int lane) {
#pragma clang fp contract(off)
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int j = (4 * lane + i) & 127;
        v[i] = x[i] * (dir ? c_S2[j] : c_S1[j]);
    }
#pragma unroll
    for (int h = 1; h <= 2; h <<= 1) {  // stages 1, 2: inside the lane
        float a[4];
#pragma unroll
        for (int i = 0; i < 4; i++) a[i] = (i & h) ? v[i ^ h] - v[i] : v[i] + v[i ^ h];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = a[i];
    }
#pragma unroll
    for (int h = 4; h <= 64; h <<= 1) {  // stages 4 .. 64: lane ^ h / 4
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float o = __shfl_xor(v[i], h / 4);
            v[i] = ((4 * lane) & h) ? o - v[i] : v[i] + o;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int j = (4 * lane + i) & 127;
        x[i] = v[i] * 0.08838834764831845f * (dir ? c_S1[j] : c_S2[j]);
    }
}

// TurboQuant codes of the lane's 4 dims; norm_out = the lane's half's corrected norm
template <int BITS>
__device__ __forceinline__ void tq_quant(const float (&x)[4], int lane, int (&idx)[4], float& norm_out) {
#pragma clang fp contract(off)
    float sq[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sq[i] = x[i] * x[i];
    const float n = sqrtf(half_sum(sq, lane));
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; i++) r[i] = n > 1e-20f ? x[i] / n : 0.f;
    wht(r, 0, lane);
    float cc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int k = 0;
        if (BITS == 4) {
#pragma unroll
            for (int t = 0; t < 15; t++) k += r[i] >= c_M4[t];
        } else {
#pragma unroll
            for (int t = 0; t < 7; t++) k += r[i] >= c_M3[t];
        }
        idx[i] = k;
        const float c = BITS == 4 ? (float)c_I4[k] * K4 : (float)c_I3[k] * K3;
        cc[i] = c * c;
    }
    const float rn = sqrtf(half_sum(cc, lane));
    norm_out = rn > 1e-20f ? n / rn : n;
}

// int8 codes of the lane's 4 dims of a k and a v row (byte i = dim 4l + i) and the rows' scales
__device__ __forceinline__ void quant_i8(const float (&x)[4], const float (&vv)[4], uint32_t& ck, uint32_t& cv,
                                         float& sk, float& sv) {
#pragma clang fp contract(off)
    float ak[4], av[4];
#pragma unroll
    for (int i = 0; i < 4; i++) { ak[i] = fabsf(x[i]); av[i] = fabsf(vv[i]); }
    const float mk = row_max(ak), mv = row_max(av);
    sk = mk > 0.f ? mk / 127.f : 1.f;
    sv = mv > 0.f ? mv / 127.f : 1.f;
    ck = cv = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        ck |= (uint32_t)(uint8_t)(int8_t)__builtin_rintf(x[i] / sk) << (8 * i);
        cv |= (uint32_t)(uint8_t)(int8_t)__builtin_rintf(vv[i] / sv) << (8 * i);
    }
}

// quantize-append of one row (x: post-RoPE k, vv: raw v, the lane's 4 dims each), int8 or TurboQuant
__device__ __forceinline__ void append(const float (&x)[4], const float (&vv)[4], moex_kv_cache kv, size_t row,
                                       int lane) {
#pragma clang fp contract(off)
    if (kv.turbo) {
        int ik[4], iv[4];
        float nk, nv;
        tq_quant<4>(x, lane, ik, nk);
        tq_quant<3>(vv, lane, iv, nv);
        const int b = lane >> 5, l = lane & 31;  // half, lane within it: dims 4l .. 4l + 3 of the half
        uint8_t* K = reinterpret_cast<uint8_t*>(kv.k) + row * TQ_KB;
        uint8_t* V = reinterpret_cast<uint8_t*>(kv.v) + row * TQ_VB;
        const uint32_t kb = (uint32_t)(ik[0] | (ik[1] << 4)) | ((uint32_t)(ik[2] | (ik[3] << 4)) << 8);
        *reinterpret_cast<uint16_t*>(K + b * 64 + 2 * l) = (uint16_t)kb;
        V[b * 32 + l] = (uint8_t)((iv[0] & 3) | ((iv[1] & 3) << 2) | ((iv[2] & 3) << 4) | ((iv[3] & 3) << 6));
        const int hb = ((iv[0] >> 2) & 1) | (((iv[1] >> 2) & 1) << 1) | (((iv[2] >> 2) & 1) << 2) | (((iv[3] >> 2) & 1) << 3);
        const int hb1 = __shfl_down(hb, 1);
        if (!(l & 1)) V[64 + b * 16 + l / 2] = (uint8_t)(hb | (hb1 << 4));
        if (l == 0) { kv.ks[row * 2 + b] = nk; kv.vs[row * 2 + b] = nv; }
    } else {
        uint32_t ck, cv;
        float sk, sv;
        quant_i8(x, vv, ck, cv, sk, sv);
        *reinterpret_cast<uint32_t*>(kv.k + row * AHD + 4 * lane) = ck;
        *reinterpret_cast<uint32_t*>(kv.v + row * AHD + 4 * lane) = cv;
        if (lane == 0) { kv.ks[row] = sk; kv.vs[row] = sv; }
    }
}

}  // namespace wave

}  // namespace front
}  // namespace moex
