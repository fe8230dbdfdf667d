// Small kernels of the attention step: q/k RMSNorm + partial RoPE + KV quantize-append (int8 and TurboQuant),
// the per-query-head decode kernel, the split combine (+ gate, + turbo inverse rotation) and turbo_out.
//
// The quantizer arithmetic must reproduce the reference's bits (kernels.cuh:1141-1236): no FMA contraction,
// correctly rounded divide and square root, the 32-lane butterfly order of warp_sum and the in-order sum of the
// four 32-lane partials of each 128-value half (tq_half_sum). A 256-thread block holds one head row, thread d
// owns dim d; on a 64-wide wavefront an xor-shuffle with offset <= 16 never leaves its 32-lane half, so the
// reference's warp tree is reproduced exactly. The WHT's stage 32 is a shuffle too (dims d and d^32 share a
// wavefront); only stage 64 crosses wavefronts and goes through LDS.
#pragma clang fp contract(off)
#include <cstdlib>
#include <mutex>
#include "front.hpp"

namespace moex {

// graph-fallback flag (kernels.cuh:46, g_skip): nonzero -> qk_norm_rope / turbo_out return at once
__device__ int g_skip;

// ---- the front's helpers over a 256-thread block (thread d = threadIdx.x owns dim d of the row) ----
using front::c_I3;
using front::c_I4;
using front::K3;
using front::K4;
__device__ __forceinline__ float block_sum(float v, float* sh8) { return front::block_sum(v, sh8, threadIdx.x); }
__device__ __forceinline__ float wht(float x, float* sh, int dir) { return front::wht(x, sh, dir, threadIdx.x); }

// Quantize-append of one (kv head, position) row: x = post-RoPE k of dim d, vv = raw v of dim d.
__device__ __forceinline__ void append_row(float x, float vv, moex_kv_cache kv, size_t row, float* sh, float* sh8) {
    const int d = threadIdx.x;
    if (kv.turbo) {  // K 4-bit, V 3-bit (kernels.cuh:1210-1226)
        front::append_turbo(x, vv, kv, row, sh, sh8, d, true);
    } else {  // int8 per row (kernels.cuh:1227-1235)
        int8_t ck, cv;
        float sk, sv;
        front::quant_i8(x, vv, sh8, d, ck, cv, sk, sv);
        const size_t o = row * AHD + d;
        kv.k[o] = ck;
        kv.v[o] = cv;
        if (d == 0) { kv.ks[row] = sk; kv.vs[row] = sv; }
    }
}

// qk_norm_rope_k (kernels.cuh:1185-1236): grid (H + KV, T), 256 threads. Blocks [0, H): query heads -> qo;
// [H, H+KV): key heads -> quantize-append of k and v at position *pos_d + token.
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ kn, float* __restrict__ qo, moex_kv_cache kv,
    int H, int KV, const int* __restrict__ pos_d, int max_t, int rot, float theta, float eps, int ld) {
    if (g_skip) return;
    __shared__ float t[AHD];
    __shared__ float sh[AHD];
    __shared__ float sh8[16];
    const int tok = blockIdx.y, pos = *pos_d + tok, hh = blockIdx.x, d = threadIdx.x;
    q += (size_t)tok * ld; k += (size_t)tok * ld; v += (size_t)tok * ld; qo += (size_t)tok * H * AHD;
    const bool isq = hh < H;
    float x = isq ? q[hh * 2 * AHD + d] : k[(hh - H) * AHD + d];
    x = front::norm_rope(x, isq ? qn : kn, d, pos, rot, theta, eps, t, sh8);
    if (isq) {
        const float y = kv.turbo ? wht(x, sh, 0) : x;  // turbo: the keys' rotation (the block is uniform)
        qo[hh * AHD + d] = y;
    } else {
        append_row(x, v[(hh - H) * AHD + d], kv, (size_t)(hh - H) * max_t + pos, sh, sh8);
    }
}

// The same front on wavefronts of RPW rows of one token each (front::wave, the same bits): a token's H + KV rows go
// to ceil((H + KV) / RPW) wavefronts, four to a workgroup, no barrier. A wavefront issues all of its row reads first
// and computes the token's RoPE angles once for its rows (powf, sinf and cosf of arguments up to the position: most
// of a row's arithmetic). KV rows append (k normalized and rotated; v raw). Needs rot % 8 == 0.
template <int RPW>
__global__ void __launch_bounds__(256) front_rows_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ kn, float* __restrict__ qo, moex_kv_cache kv,
    int H, int KV, const int* __restrict__ pos_d, int max_t, int rot, float theta, float eps, int ld, int T) {
    if (g_skip) return;
    const int R = H + KV, wpt = (R + RPW - 1) / RPW;
    const int w = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (w >= T * wpt) return;
    const int tok = w / wpt, r0 = (w - tok * wpt) * RPW, pos = *pos_d + tok;
    q += (size_t)tok * ld; k += (size_t)tok * ld; v += (size_t)tok * ld;
    float4 x4[RPW], v4[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
        const int hh = r0 + i;
        if (hh < H) {
            x4[i] = *reinterpret_cast<const float4*>(q + hh * 2 * AHD + 4 * lane);
        } else if (hh < R) {
            x4[i] = *reinterpret_cast<const float4*>(k + (hh - H) * AHD + 4 * lane);
            v4[i] = *reinterpret_cast<const float4*>(v + (hh - H) * AHD + 4 * lane);
        }
    }
    const uint2 wq = *reinterpret_cast<const uint2*>(qn + 4 * lane), wk = *reinterpret_cast<const uint2*>(kn + 4 * lane);
    const front::wave::Rope rp = front::wave::rope_angles(lane, pos, rot, theta);
#pragma unroll
    for (int i = 0; i < RPW; i++) {
        const int hh = r0 + i;
        if (hh >= R) break;
        const bool isq = hh < H;
        float x[4] = {x4[i].x, x4[i].y, x4[i].z, x4[i].w};
        front::wave::norm_rope(x, isq ? wq : wk, lane, rp, rot, eps);
        if (isq) {
            if (kv.turbo) front::wave::wht(x, 0, lane);  // the keys' rotation
            *reinterpret_cast<float4*>(qo + ((size_t)tok * H + hh) * AHD + 4 * lane) = make_float4(x[0], x[1], x[2], x[3]);
        } else {
            const float vv[4] = {v4[i].x, v4[i].y, v4[i].z, v4[i].w};
            front::wave::append(x, vv, kv, (size_t)(hh - H) * max_t + pos, lane);
        }
    }
}
// Quantize-append only, one wavefront per row (rows r = token KV + kv head)
__global__ void __launch_bounds__(256) append_rows_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                          moex_kv_cache kv, int KV, const int* __restrict__ pos_d,
                                                          int max_t, int ld, int T) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= T * KV) return;
    const int tok = r / KV, kvh = r - tok * KV;
    const size_t o = (size_t)tok * ld + kvh * AHD + 4 * lane;
    const float4 k4 = *reinterpret_cast<const float4*>(k + o), v4 = *reinterpret_cast<const float4*>(v + o);
    const float x[4] = {k4.x, k4.y, k4.z, k4.w}, vv[4] = {v4.x, v4.y, v4.z, v4.w};
    front::wave::append(x, vv, kv, (size_t)kvh * max_t + *pos_d + tok, lane);
}

// Quantize-append only: grid (KV, T); k already normalized and rotated.
__global__ void __launch_bounds__(256) kv_append_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                        moex_kv_cache kv, const int* __restrict__ pos_d, int max_t,
                                                        int ld) {
    __shared__ float sh[AHD];
    __shared__ float sh8[16];
    const int tok = blockIdx.y, kvh = blockIdx.x, d = threadIdx.x;
    const size_t o = (size_t)tok * ld + kvh * AHD + d;
    append_row(k[o], v[o], kv, (size_t)kvh * max_t + *pos_d + tok, sh, sh8);
}

// turbo_out_k (kernels.cuh:1730-1738): out = WHT_inv(out) / (1 + e^-g), in place. Grid (H, T).
__global__ void __launch_bounds__(256) turbo_out_kernel(float* __restrict__ out, const float* __restrict__ q_gate,
                                                        int H, int ld) {
    if (g_skip) return;
    __shared__ float sh[AHD];
    const int h = blockIdx.x, tok = blockIdx.y, d = threadIdx.x;
    float* o = out + ((size_t)tok * H + h) * AHD;
    const float x = wht(o[d], sh, 1);
    o[d] = x / (1.f + __expf(-q_gate[(size_t)tok * ld + h * 2 * AHD + AHD + d]));
}

// turbo_out_kernel on one wavefront per (token, head) row, four rows a workgroup (front::wave::wht: the same bits)
__global__ void __launch_bounds__(256) turbo_out_rows_kernel(float* __restrict__ out, const float* __restrict__ q_gate,
                                                             int H, int ld, int T) {
    if (g_skip) return;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= T * H) return;
    const int tok = r / H, h = r - tok * H;
    float4* o4 = reinterpret_cast<float4*>(out + (size_t)r * AHD + 4 * lane);
    const float4 a = *o4;
    float x[4] = {a.x, a.y, a.z, a.w};
    front::wave::wht(x, 1, lane);
    const float4 g = *reinterpret_cast<const float4*>(q_gate + (size_t)tok * ld + h * 2 * AHD + AHD + 4 * lane);
    *o4 = make_float4(x[0] / (1.f + __expf(-g.x)), x[1] / (1.f + __expf(-g.y)), x[2] / (1.f + __expf(-g.z)),
                      x[3] / (1.f + __expf(-g.w)));
}

// attn_combine_k (kernels.cuh:1317-1329): merge ns partials {m (log2 units), l, acc[256]}.
// Grid (H, T, CDC): block (h, t, c) owns dims [64 c, 64 c + 64); its 256 threads are 16 dim quads (one float4 of acc
// per split) x 16 split groups. A thread loads 8 of its splits at once, takes their maximum, then weighs them with
// independent exponentials (no serial online chain); m and l are the same for the 16 threads of a group, so only
// the group's acc goes through LDS. One pass over the partials.
constexpr int CDC = AHD / 64, CNG = 16, CSB = 8;
__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ part, const float* __restrict__ q_gate,
                                                      float* __restrict__ out, int H, int ns, int ld) {
    __shared__ float sm[CNG], sl[CNG];
    __shared__ float4 sa[CNG][16];
    const int tok = blockIdx.y, h = blockIdx.x, tid = threadIdx.x, T = gridDim.y;
    float* pp = const_cast<float*>(part);
    const float4* acc_rows = reinterpret_cast<const float4*>(part_acc(pp, tok, h, 0, H, ns) + 64 * blockIdx.z);
    const float2* ml = reinterpret_cast<const float2*>(part_ml(pp, tok, h, 0, H, ns, T));
    const int dq = tid & 15, gi = tid >> 4;
    // the gate goes out with the partials rather than after the merge
    const float gt = (q_gate && tid < 64) ? q_gate[(size_t)tok * ld + h * 2 * AHD + AHD + 64 * blockIdx.z + tid] : 0.f;
    float mt = -INFINITY, lt = 0.f;
    float4 at = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = gi; s0 < ns; s0 += CSB * CNG) {
        float2 q[CSB];
        float4 a[CSB];
#pragma unroll
        for (int u = 0; u < CSB; u++) {
            const int s = s0 + u * CNG;
            if (s < ns) {
                q[u] = ml[s];
                a[u] = acc_rows[(size_t)s * (AHD / 4) + dq];
            } else {
                q[u] = make_float2(-INFINITY, 0.f);
                a[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        float mb = mt;
#pragma unroll
        for (int u = 0; u < CSB; u++)
            if (q[u].y > 0.f) mb = fmaxf(mb, q[u].x);  // empty splits (l = 0, m = -inf) contribute nothing
        if (mb == -INFINITY) continue;                  // nothing yet
        const float f = fast_exp2(mt - mb);             // 0 while mt = -inf
        lt *= f;
        at.x *= f; at.y *= f; at.z *= f; at.w *= f;
#pragma unroll
        for (int u = 0; u < CSB; u++) {
            const float g = q[u].y > 0.f ? fast_exp2(q[u].x - mb) : 0.f;
            lt = fmaf(q[u].y, g, lt);
            at.x = fmaf(a[u].x, g, at.x); at.y = fmaf(a[u].y, g, at.y);
            at.z = fmaf(a[u].z, g, at.z); at.w = fmaf(a[u].w, g, at.w);
        }
        mt = mb;
    }
    if (dq == 0) { sm[gi] = mt; sl[gi] = lt; }
    sa[gi][dq] = at;
    __syncthreads();
    if (tid >= 64) return;
    float M = -INFINITY;
#pragma unroll
    for (int g = 0; g < CNG; g++) M = fmaxf(M, sm[g]);  // split 0 is never empty: M is finite
    float l = 0.f, acc = 0.f;
    const float* saf = reinterpret_cast<const float*>(&sa[0][0]);
#pragma unroll
    for (int g = 0; g < CNG; g++) {
        const float f = fast_exp2(sm[g] - M);
        l += sl[g] * f;
        acc += saf[g * 64 + tid] * f;
    }
    float x = acc / l;
    if (q_gate) x = x / (1.f + __expf(-gt));
    out[((size_t)tok * H + h) * AHD + 64 * blockIdx.z + tid] = x;
}

// Per-query-head decode (the contract of attn_decode_k, kernels.cuh:1238-1315): any H / KV, int8 or turbo.
// Workgroup = (query head, token, split), 4 wavefronts. Wavefront w walks the split's keys in chunks of 64 taken
// round-robin (chunk c goes to wavefront c % 4) and keeps its own online softmax state:
//   - lane i scores key i of the chunk alone, over the whole row (the query sits in LDS and every lane reads the
//     same word, a broadcast);
//   - the chunk's maximum and sum are wavefront reductions, the probabilities (times the key's V scale) stay in the
//     lane of their key;
//   - lane i then accumulates dims 4i .. 4i+3 over the chunk's keys, reading each V row with one coalesced 256-byte
//     wavefront load and taking the key's probability by a wavefront broadcast.
// The four states {m, l, acc} merge through LDS at the end. Base-2 softmax with the scale log2(e) / 16.
// ns == 1: the gated output (no gate if q_gate is NULL); else partials for combine_kernel.
constexpr int DH_CH = 64;  // keys per wavefront chunk
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__global__ void __launch_bounds__(256) decode_heads_kernel(const float* __restrict__ qo, const float* __restrict__ q_gate,
                                                           moex_kv_cache kv, float* __restrict__ out, int H, int KV,
                                                           const int* __restrict__ pos_d, int max_t, int ld,
                                                           float* __restrict__ part) {
    __shared__ __align__(16) float qv[AHD];
    __shared__ float klut[16], vlut[8];
    __shared__ float wm[4], wl[4];
    __shared__ __align__(16) float wacc[4][AHD];
    const int h = blockIdx.x, tok = blockIdx.y, sp = blockIdx.z, ns = gridDim.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nk = *pos_d + tok + 1, per = (nk + ns - 1) / ns, lo = sp * per, hi = min(nk, lo + per);
    const int kvh = h / (H / KV);
    const bool tb = kv.turbo;
    qv[tid] = qo[((size_t)tok * H + h) * AHD + tid];
    if (tid < 16) klut[tid] = (float)c_I4[tid] * K4;
    if (tid < 8) vlut[tid] = (float)c_I3[tid] * K3;
    __syncthreads();
    const float sl2 = 0.0625f * 1.4426950408889634f;
    const size_t rbase = (size_t)kvh * max_t;
    // turbo V fields of this lane's dims 4 lane .. +3 (half hb, in-half dims j0 .. j0 + 3): the low 2-bit codes are
    // one byte, the high bits a nibble of another
    const int hb = lane >> 5, j0 = 4 * (lane & 31);
    const int vlo = hb * 32 + (j0 >> 2), vhi = 64 + hb * 16 + (j0 >> 3), vsh = j0 & 7;
    float m = -INFINITY, l = 0.f;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    for (int c0 = lo + DH_CH * w; c0 < hi; c0 += 4 * DH_CH) {
        const int n = min(DH_CH, hi - c0), key = c0 + min(lane, n - 1);
        const size_t row = rbase + key;
        float sc;
        if (tb) {  // two half sums over 4-bit codes, each times its half norm
            const uint4* kp = reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(kv.k) + row * TQ_KB);
            float d[2] = {0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint4 x = kp[u];
                const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                for (int b = 0; b < 4; b++)
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        d[u >> 2] += klut[(xw[b] >> (4 * e)) & 15] * qv[32 * u + 8 * b + e];
            }
            sc = (d[0] * kv.ks[row * 2] + d[1] * kv.ks[row * 2 + 1]) * sl2;
        } else {
            const uint4* kp = reinterpret_cast<const uint4*>(kv.k + row * AHD);
            float d = 0.f;
#pragma unroll 4
            for (int u = 0; u < 16; u++) {
                const uint4 x = kp[u];
                const float4* q4 = reinterpret_cast<const float4*>(qv + 16 * u);
                const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const float4 qq = q4[b];
                    d += (float)(int8_t)(xw[b]) * qq.x + (float)(int8_t)(xw[b] >> 8) * qq.y +
                         (float)(int8_t)(xw[b] >> 16) * qq.z + (float)(int8_t)(xw[b] >> 24) * qq.w;
                }
            }
            sc = d * kv.ks[row] * sl2;
        }
        if (lane >= n) sc = -INFINITY;
        const float mn = fmaxf(m, wave_max(sc));  // finite: every chunk has a key
        const float cr = fast_exp2(m - mn);       // 0 while m = -inf
        const float p = lane < n ? fast_exp2(sc - mn) : 0.f;
        l = l * cr + wave_sum(p);
        m = mn;
        a0 *= cr; a1 *= cr; a2 *= cr; a3 *= cr;
        float pv0, pv1 = 0.f;  // p times the V scale (turbo: of each half)
        if (tb) { pv0 = p * kv.vs[row * 2]; pv1 = p * kv.vs[row * 2 + 1]; }
        else pv0 = p * kv.vs[row];
        if (tb) {
            const uint8_t* vr = reinterpret_cast<const uint8_t*>(kv.v) + (rbase + c0) * TQ_VB;
            for (int i = 0; i < n; i++) {
                const float p0 = __shfl(pv0, i), p1 = __shfl(pv1, i), pk = hb ? p1 : p0;
                const uint32_t lo2 = vr[(size_t)i * TQ_VB + vlo], hi1 = vr[(size_t)i * TQ_VB + vhi] >> vsh;
                a0 += pk * vlut[(lo2 & 3) | ((hi1 & 1) << 2)];
                a1 += pk * vlut[((lo2 >> 2) & 3) | ((hi1 & 2) << 1)];
                a2 += pk * vlut[((lo2 >> 4) & 3) | (hi1 & 4)];
                a3 += pk * vlut[((lo2 >> 6) & 3) | ((hi1 & 8) >> 1)];
            }
        } else {
            const int8_t* vr = kv.v + (rbase + c0) * AHD + 4 * lane;
            for (int i = 0; i < n; i++) {
                const float pk = __shfl(pv0, i);
                const uint32_t x = *reinterpret_cast<const uint32_t*>(vr + (size_t)i * AHD);
                a0 += pk * (float)(int8_t)x; a1 += pk * (float)(int8_t)(x >> 8);
                a2 += pk * (float)(int8_t)(x >> 16); a3 += pk * (float)(int8_t)(x >> 24);
            }
        }
    }
    if (lane == 0) { wm[w] = m; wl[w] = l; }
    *reinterpret_cast<float4*>(&wacc[w][4 * lane]) = make_float4(a0, a1, a2, a3);
    __syncthreads();
    // thread d: dim d of the merged state (a wavefront without keys has m = -inf and weighs nothing)
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; v++) M = fmaxf(M, wm[v]);
    float L = 0.f, A = 0.f;
    if (M != -INFINITY) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float f = fast_exp2(wm[v] - M);
            L += wl[v] * f;
            A += wacc[v][tid] * f;
        }
    }
    if (ns == 1) {
        const float x = A / L;
        out[((size_t)tok * H + h) * AHD + tid] =
            q_gate ? x / (1.f + __expf(-q_gate[(size_t)tok * ld + h * 2 * AHD + AHD + tid])) : x;
        return;
    }
    part_acc(part, tok, h, sp, H, ns)[tid] = A;  // an empty split: m = -inf, l = 0, acc = 0
    if (tid == 0) {
        float* ml = part_ml(part, tok, h, sp, H, ns, gridDim.y);
        ml[0] = M; ml[1] = L;
    }
}

const int* skip_flag() {
    static std::mutex mu;
    static const int* ptr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lk(mu);
    if (!ptr[dev]) {  // first use on this device, which is current here
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_skip)) != hipSuccess) return nullptr;
        ptr[dev] = static_cast<const int*>(p);
    }
    return ptr[dev];
}

__global__ void set_int_kernel(int* p, int v) { *p = v; }
__global__ void set_skip_kernel(int v) { g_skip = v; }

// ---- launchers ----
void launch_qk_norm_rope(const float* q, const float* k, const float* v, const uint16_t* qn, const uint16_t* kn,
                         float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, int rot,
                         float theta, float eps, int ld, int T, hipStream_t st) {
    // the 16-byte row loads and the wavefront layout need 4-float aligned rows
    const bool al = ld % 4 == 0 && ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)qo) % 16 == 0 &&
                    ((uintptr_t)qn | (uintptr_t)kn) % 8 == 0;
    // rows per wavefront: 3 (a 2048-token chunk at 32768: int8 26.7-29.3 -> 20.1-22.0 us, turbo 33.4-34.4 -> 32.4;
    // 6 and 9 no better, turbo slower at 6); MOEX_FRONT_RPW=1, 3, 6 or 9 for comparisons (read on every call)
    int rpw = 3;
    if (const char* e = std::getenv("MOEX_FRONT_RPW")) rpw = std::atoi(e);
    const int waves = T * ((H + KV + rpw - 1) / std::max(rpw, 1));
    const dim3 grid((waves + 3) / 4);
    if (rot % 8 == 0 && al) {
        if (rpw == 1)
            hipLaunchKernelGGL(front_rows_kernel<1>, grid, dim3(256), 0, st, q, k, v, qn, kn, qo, kv, H, KV, pos_d, max_t,
                               rot, theta, eps, ld, T);
        else if (rpw == 9)
            hipLaunchKernelGGL(front_rows_kernel<9>, grid, dim3(256), 0, st, q, k, v, qn, kn, qo, kv, H, KV, pos_d, max_t,
                               rot, theta, eps, ld, T);
        else if (rpw == 6)
            hipLaunchKernelGGL(front_rows_kernel<6>, grid, dim3(256), 0, st, q, k, v, qn, kn, qo, kv, H, KV, pos_d, max_t,
                               rot, theta, eps, ld, T);
        else
            hipLaunchKernelGGL(front_rows_kernel<3>, dim3((T * ((H + KV + 2) / 3) + 3) / 4), dim3(256), 0, st, q, k, v, qn,
                               kn, qo, kv, H, KV, pos_d, max_t, rot, theta, eps, ld, T);
    } else
        hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(H + KV, T), dim3(256), 0, st, q, k, v, qn, kn, qo, kv, H, KV,
                           pos_d, max_t, rot, theta, eps, ld);
    MOEX_LAUNCHED();
}
void launch_kv_append(const float* k, const float* v, moex_kv_cache kv, int KV, const int* pos_d, int max_t, int ld,
                      int T, hipStream_t st) {
    if (ld % 4 == 0 && ((uintptr_t)k | (uintptr_t)v) % 16 == 0)
        hipLaunchKernelGGL(append_rows_kernel, dim3((T * KV + 3) / 4), dim3(256), 0, st, k, v, kv, KV, pos_d, max_t, ld,
                           T);
    else
        hipLaunchKernelGGL(kv_append_kernel, dim3(KV, T), dim3(256), 0, st, k, v, kv, pos_d, max_t, ld);
    MOEX_LAUNCHED();
}
void launch_turbo_out(float* out, const float* q_gate, int H, int ld, int T, hipStream_t st) {
    if (ld % 4 == 0 && ((uintptr_t)out | (uintptr_t)q_gate) % 16 == 0)
        hipLaunchKernelGGL(turbo_out_rows_kernel, dim3((T * H + 3) / 4), dim3(256), 0, st, out, q_gate, H, ld, T);
    else
        hipLaunchKernelGGL(turbo_out_kernel, dim3(H, T), dim3(256), 0, st, out, q_gate, H, ld);
    MOEX_LAUNCHED();
}
void launch_combine(const float* part, const float* q_gate, float* out, int H, int ns, int ld, int T, hipStream_t st) {
    hipLaunchKernelGGL(combine_kernel, dim3(H, T, CDC), dim3(256), 0, st, part, q_gate, out, H, ns, ld);
    MOEX_LAUNCHED();
}
void launch_decode_heads(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                         const int* pos_d, int max_t, int ld, float* part, int T, int ns, hipStream_t st) {
    hipLaunchKernelGGL(decode_heads_kernel, dim3(H, T, ns), dim3(256), 0, st, qo, q_gate, kv, out, H, KV, pos_d, max_t,
                       ld, part);
    MOEX_LAUNCHED();
}
void launch_set_int(int* p, int v, hipStream_t st) {
    hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, st, p, v);
    MOEX_LAUNCHED();
}
void launch_set_skip(int v, hipStream_t st) {
    hipLaunchKernelGGL(set_skip_kernel, dim3(1), dim3(1), 0, st, v);
    MOEX_LAUNCHED();
}

}  // namespace moex
