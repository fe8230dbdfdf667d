// FlashAttention-2 chunked causal GQA prefill on gfx950 (replaces attn_fa_k<TB>, kernels.cuh:1443-1728).
//
// Workgroup = (kv head, 16 query tokens) = 128 query rows (8 heads x 16 tokens), 4 wavefronts of 32 rows;
// wavefront w owns tokens 4w .. 4w+3, row r = (token 4w + r/8, head r%8). Keys in tiles of 32:
//   - the block stages each K/V tile once: int8 (or turbo codes) from HBM -> fp16 in LDS, K as [key][dim]
//     (16-byte chunks XOR-swizzled by key), V transposed as [dim][key] (row stride 72 B: conflict-free reads);
//     the next tile's global loads are in flight while the current one is computed (double-buffered LDS);
//   - S^T = K . Q^T on v_mfma_f32_32x32x16_f16 (Q fp16 in registers): the 32x32 D layout gives every lane ONE
//     query row (lane % 32) and 16 keys, so the row max / row sum are in-lane plus one cross-half exchange;
//   - P^T (fp16, times V's row scale) stays in registers and is directly the B operand of O^T += V^T . P^T;
//     O^T (256 dims x 32 rows per wavefront, 128 fp32 per lane) lives in registers for the whole key loop.
// Softmax in base 2 with the K scale, 1/sqrt(256) and log2(e) folded into one factor per key (kernels.cuh:1513).
// Rounding points follow the reference kernel: Q and P * vscale rounded to fp16, fp32 accumulate (:1508,:1656).
// Turbo: K codes decoded to the centroids' int8 codes, S accumulated per 128-half and combined with the half norms;
// V's two half norms give two P operands (dims < 128 / >= 128). No gate when q_gate is null.
#include "common.hpp"

namespace moex {

namespace {
constexpr int FT = 16;               // tokens per workgroup
constexpr int BK = 32;               // keys per tile
constexpr int VST = BK + 4;          // V^T row stride in halves (72 B)
constexpr int KT_BYTES = BK * AHD * 2;      // 16 KB
constexpr int VT_BYTES = AHD * VST * 2;     // 18 KB
constexpr int BUF_BYTES = KT_BYTES + VT_BYTES + 4 * BK * 4;  // + ks, vs (turbo: kn0, kn1 / vs0, vs1)
constexpr float SL2 = 0.0625f * 1.4426950408889634f;
constexpr float TK4 = 0.241529f / 127.f, TK3 = 0.190207f / 127.f;

constexpr uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a + 128) | ((uint32_t)(b + 128) << 8) | ((uint32_t)(c + 128) << 16) | ((uint32_t)(d + 128) << 24);
}
constexpr uint32_t K4T0 = pack4(-127, -96, -75, -58), K4T1 = pack4(-44, -31, -18, -6);
constexpr uint32_t K4T2 = pack4(6, 18, 31, 44), K4T3 = pack4(58, 75, 96, 127);
constexpr uint32_t V3T0 = pack4(-127, -79, -45, -14), V3T1 = pack4(14, 45, 79, 127);

__device__ __forceinline__ uint32_t lut16(uint32_t idx) {
    const uint32_t s = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(K4T1, K4T0, s), hi = __builtin_amdgcn_perm(K4T3, K4T2, s);
    const uint32_t mask = ((idx >> 3) & 0x01010101u) * 0xffu;
    return (hi & mask) | (lo & ~mask);
}

// 4x4 byte transpose: r[k] = 4 bytes (dims) of key k -> c[d] = 4 bytes (keys) of dim d
__device__ __forceinline__ void tr4x4(const uint32_t r[4], uint32_t c[4]) {
    const uint32_t t0 = __builtin_amdgcn_perm(r[1], r[0], 0x05010400u), t1 = __builtin_amdgcn_perm(r[1], r[0], 0x07030602u);
    const uint32_t t2 = __builtin_amdgcn_perm(r[3], r[2], 0x05010400u), t3 = __builtin_amdgcn_perm(r[3], r[2], 0x07030602u);
    c[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u); c[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    c[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u); c[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

__device__ __forceinline__ int kchunk(int key, int c) { return c ^ (key & 15); }  // swizzled 16-byte chunk

// raw global data of one tile held by a thread between the load and the LDS write
struct Stage {
    uint4 k[2];      // int8: 32 bytes of key t/8 (dims 32*(t%8) ..); turbo: k[0] = 16 nibble bytes
    uint32_t v[8];   // int8: 4 bytes (dims 4*(t%64) ..) of keys 8*(t/64) .. +7; turbo: (low byte | high byte << 8)
    float sa, sb, sc, sd;  // thread < BK: scales of key t
};

template <bool TB>
__device__ __forceinline__ void stage_load(Stage& S, moex_kv_cache kv, size_t rbase, int k0, int hi, int tid) {
    {
        const int key = tid >> 3, c = tid & 7, t = k0 + key;
        const size_t row = rbase + (t < hi ? t : hi - 1);
        if (TB) {
            S.k[0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(kv.k) + row * TQ_KB + c * 16);
        } else {
            const uint4* p = reinterpret_cast<const uint4*>(kv.k + row * AHD + c * 32);
            S.k[0] = p[0]; S.k[1] = p[1];
        }
    }
    {
        const int dg = tid & 63, kb = (tid >> 6) * 8;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int t = k0 + kb + i;
            const size_t row = rbase + (t < hi ? t : hi - 1);
            if (TB) {
                const uint8_t* vp = reinterpret_cast<const uint8_t*>(kv.v) + row * TQ_VB;
                const int b = dg >> 5;
                S.v[i] = (uint32_t)vp[b * 32 + (dg & 31)] | ((uint32_t)vp[64 + b * 16 + ((dg & 31) >> 1)] << 8);
            } else {
                S.v[i] = *reinterpret_cast<const uint32_t*>(kv.v + row * AHD + dg * 4);
            }
        }
    }
    if (tid < BK) {
        const int t = k0 + tid;
        const size_t row = rbase + (t < hi ? t : hi - 1);
        if (TB) {
            const float2 kn = *reinterpret_cast<const float2*>(kv.ks + row * 2);
            const float2 vn = *reinterpret_cast<const float2*>(kv.vs + row * 2);
            S.sa = kn.x; S.sb = kn.y; S.sc = vn.x; S.sd = vn.y;
        } else {
            S.sa = kv.ks[row]; S.sc = kv.vs[row];
        }
    }
}

template <bool TB>
__device__ __forceinline__ void stage_store(const Stage& S, unsigned char* buf, int k0, int hi, int tid) {
    _Float16* Kt = reinterpret_cast<_Float16*>(buf);
    _Float16* Vt = reinterpret_cast<_Float16*>(buf + KT_BYTES);
    float* sc = reinterpret_cast<float*>(buf + KT_BYTES + VT_BYTES);
    {
        const int key = tid >> 3, c = tid & 7;
        const bool ok = k0 + key < hi;
        uint32_t w[16];
        if (TB) {
            const uint32_t in[4] = {S.k[0].x, S.k[0].y, S.k[0].z, S.k[0].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {  // 8 nibbles -> dims 8i .. 8i+7 (biased codes), widened
                const uint32_t e = lut16(in[i] & 0x0f0f0f0fu), o = lut16((in[i] >> 4) & 0x0f0f0f0fu);
                const uint32_t d01 = __builtin_amdgcn_perm(o, e, 0x05010400u), d23 = __builtin_amdgcn_perm(o, e, 0x07030602u);
                biased4_to_h4(d01, w[4 * i], w[4 * i + 1]);
                biased4_to_h4(d23, w[4 * i + 2], w[4 * i + 3]);
            }
        } else {
            const uint32_t in[8] = {S.k[0].x, S.k[0].y, S.k[0].z, S.k[0].w, S.k[1].x, S.k[1].y, S.k[1].z, S.k[1].w};
#pragma unroll
            for (int i = 0; i < 8; i++) i8x4_to_h4(in[i], w[2 * i], w[2 * i + 1]);
        }
        if (!ok) {
#pragma unroll
            for (int i = 0; i < 16; i++) w[i] = 0u;
        }
#pragma unroll
        for (int q = 0; q < 4; q++)  // 4 chunks of 8 halves: dims 32c + 8q
            *reinterpret_cast<uint4*>(Kt + key * AHD + kchunk(key, 4 * c + q) * 8) = make_uint4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
    }
    {
        const int dg = tid & 63, kb = (tid >> 6) * 8;
        uint32_t r[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t x;
            if (TB) {  // 4 dims: 3-bit codes from the low-bit byte and a nibble of the high-bit byte -> biased codes
                const uint32_t lo8 = S.v[i] & 0xffu, hb4 = (S.v[i] >> (8 + 4 * (dg & 1))) & 15u;
                uint32_t idx = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) idx |= (((lo8 >> (2 * e)) & 3u) | (((hb4 >> e) & 1u) << 2)) << (8 * e);
                x = __builtin_amdgcn_perm(V3T1, V3T0, idx);
            } else {
                x = S.v[i] ^ 0x80808080u;  // biased
            }
            r[i] = k0 + kb + i < hi ? x : 0x80808080u;  // zero codes past the end
        }
        uint32_t ca[4], cb[4];
        tr4x4(r, ca);
        tr4x4(r + 4, cb);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            uint32_t h0, h1, h2, h3;
            biased4_to_h4(ca[e], h0, h1);
            biased4_to_h4(cb[e], h2, h3);
            _Float16* dst = Vt + (4 * dg + e) * VST + kb;
            *reinterpret_cast<uint2*>(dst) = make_uint2(h0, h1);
            *reinterpret_cast<uint2*>(dst + 4) = make_uint2(h2, h3);
        }
    }
    if (tid < BK) {
        const bool ok = k0 + tid < hi;
        if (TB) {
            sc[tid] = ok ? S.sa : 0.f;
            sc[BK + tid] = ok ? S.sb : 0.f;
            sc[2 * BK + tid] = ok ? S.sc * TK3 : 0.f;
            sc[3 * BK + tid] = ok ? S.sd * TK3 : 0.f;
        } else {
            sc[tid] = ok ? S.sa * SL2 : 0.f;
            sc[2 * BK + tid] = ok ? S.sc : 0.f;
        }
    }
}

// XCD-aware block order: blocks b, b+8, ... run on one XCD. Each kv head gets 8/KV XCDs (its K/V stays in their L2),
// and the heaviest (latest) token tiles are dispatched first on every XCD.
__device__ __forceinline__ bool map_block(int b, int KV, int NT, int& kvh, int& tile) {
    if (8 % KV == 0) {
        const int xpk = 8 / KV, x = b & 7, i = b >> 3;
        kvh = x / xpk;
        const int rank = i * xpk + (x % xpk);
        if (rank >= NT) return false;
        tile = NT - 1 - rank;
        return true;
    }
    kvh = b / NT; tile = NT - 1 - b % NT;
    return kvh < KV;
}
}  // namespace

int fa_grid(int KV, int T) {
    const int NT = (T + FT - 1) / FT;
    if (8 % KV == 0) { const int xpk = 8 / KV; return 8 * ((NT + xpk - 1) / xpk); }
    return KV * NT;
}

template <bool TB>
__global__ void __launch_bounds__(256, 1) fa_prefill_kernel(const float* __restrict__ qo, const float* __restrict__ q_gate,
                                                            moex_kv_cache kv, float* __restrict__ out, int H, int KV,
                                                            const int* __restrict__ pos_d, int max_t, int ld, int T) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int NT = (T + FT - 1) / FT;
    int kvh, tile;
    if (!map_block(blockIdx.x, KV, NT, kvh, tile)) return;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h32 = lane >> 5, r = lane & 31;
    const int t0 = tile * FT, pos0 = *pos_d, nt = min(FT, T - t0), hi = pos0 + t0 + nt;  // keys [0, hi)
    const int tokw = 4 * w + (r >> 3), head = kvh * GQ + (r & 7);                     // this lane's row
    const int prow = min(pos0 + t0 + tokw, hi - 1);                                     // its last visible key
    const int wmax = min(pos0 + t0 + 4 * w + 3, hi - 1);                                // the wavefront's last key
    const size_t rbase = (size_t)kvh * max_t;

    // Q row (fp16) as B operands: MFMA s covers dims 16s + 8*h32 + 0..7
    half8_t qf[16];
    {
        const float* qrow = qo + ((size_t)(t0 + min(tokw, nt - 1)) * H + head) * AHD;
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const float4* p4 = reinterpret_cast<const float4*>(qrow + 16 * s + 8 * h32);
            const float4 a = p4[0], b = p4[1];
            qf[s] = half8_t{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                            (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
        }
    }
    float16_t o[8];
#pragma unroll
    for (int db = 0; db < 8; db++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[db][i] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    const int ntiles = (hi + BK - 1) / BK;
    Stage S;
    stage_load<TB>(S, kv, rbase, 0, hi, tid);
    for (int kt = 0; kt < ntiles; kt++) {
        const int k0 = kt * BK;
        unsigned char* buf = smem + (kt & 1) * BUF_BYTES;
        stage_store<TB>(S, buf, k0, hi, tid);
        __syncthreads();
        if (kt + 1 < ntiles) stage_load<TB>(S, kv, rbase, k0 + BK, hi, tid);
        if (k0 > wmax) continue;  // every row of this wavefront is before the tile (causal)
        const _Float16* Kt = reinterpret_cast<const _Float16*>(buf);
        const _Float16* Vt = reinterpret_cast<const _Float16*>(buf + KT_BYTES);
        const float* scl = reinterpret_cast<const float*>(buf + KT_BYTES + VT_BYTES);
        // ---- S^T = K . Q^T ----
        float16_t s0, s1;
#pragma unroll
        for (int i = 0; i < 16; i++) { s0[i] = 0.f; s1[i] = 0.f; }
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const half8_t a = *reinterpret_cast<const half8_t*>(Kt + r * AHD + kchunk(r, 2 * s + h32) * 8);
            if (TB && s >= 8) s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[s], s1, 0, 0, 0);
            else s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[s], s0, 0, 0, 0);
        }
        // lane: row r, keys kk(i) = 8*(i/4) + 4*h32 + i%4
        float sv[16], mt = -INFINITY;
#pragma unroll
        for (int a4 = 0; a4 < 4; a4++) {
            const int kb = 8 * a4 + 4 * h32;
            const float4 ksc = *reinterpret_cast<const float4*>(scl + kb);
            const float kv4[4] = {ksc.x, ksc.y, ksc.z, ksc.w};
            float kv4b[4] = {0.f, 0.f, 0.f, 0.f};
            if (TB) {
                const float4 k1 = *reinterpret_cast<const float4*>(scl + BK + kb);
                kv4b[0] = k1.x; kv4b[1] = k1.y; kv4b[2] = k1.z; kv4b[3] = k1.w;
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int i = 4 * a4 + e;
                float x = TB ? (s0[i] * kv4[e] + s1[i] * kv4b[e]) * (TK4 * SL2) : s0[i] * kv4[e];
                if (k0 + kb + e > prow) x = -INFINITY;
                sv[i] = x;
                mt = fmaxf(mt, x);
            }
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float m_new = fmaxf(m_run, mt);  // key 0 is visible to every row: finite from the first tile
        const float cf = fast_exp2(m_run - m_new);
        m_run = m_new;
        if (__ballot(cf != 1.f)) {
#pragma unroll
            for (int db = 0; db < 8; db++)
#pragma unroll
                for (int i = 0; i < 16; i++) o[db][i] *= cf;
        }
        // ---- P^T (times V's scale) as B operands: MFMA m uses i = 8m .. 8m+7 ----
        half8_t pb0[2], pb1[2];
        float psum = 0.f;
#pragma unroll
        for (int a4 = 0; a4 < 4; a4++) {
            const int kb = 8 * a4 + 4 * h32;
            const float4 v4 = *reinterpret_cast<const float4*>(scl + 2 * BK + kb);
            const float va[4] = {v4.x, v4.y, v4.z, v4.w};
            float vb[4] = {0.f, 0.f, 0.f, 0.f};
            if (TB) {
                const float4 v5 = *reinterpret_cast<const float4*>(scl + 3 * BK + kb);
                vb[0] = v5.x; vb[1] = v5.y; vb[2] = v5.z; vb[3] = v5.w;
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int i = 4 * a4 + e;
                const float p = fast_exp2(sv[i] - m_new);
                psum += p;
                pb0[i >> 3][i & 7] = (_Float16)(p * va[e]);
                if (TB) pb1[i >> 3][i & 7] = (_Float16)(p * vb[e]);
            }
        }
        l_run = l_run * cf + psum;
        // ---- O^T += V^T . P^T: A = V^T rows dim 32db + r, keys 16m + 4*h32 + {0..3} and 16m + 8 + 4*h32 + {0..3}
#pragma unroll
        for (int db = 0; db < 8; db++) {
            const _Float16* vrow = Vt + (32 * db + r) * VST + 4 * h32;
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const half4_t x0 = *reinterpret_cast<const half4_t*>(vrow + 16 * m);
                const half4_t x1 = *reinterpret_cast<const half4_t*>(vrow + 16 * m + 8);
                const half8_t a = half8_t{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, (TB && db >= 4) ? pb1[m] : pb0[m], o[db], 0, 0, 0);
            }
        }
    }
    // ---- epilogue: O / l * sigmoid(gate) ----
    l_run += __shfl_xor(l_run, 32);
    if (tokw >= nt) return;
    const float il = 1.f / l_run;
    const size_t t = (size_t)(t0 + tokw);
    float* orow = out + (t * H + head) * AHD;
    const float* grow = q_gate ? q_gate + t * ld + head * 2 * AHD + AHD : nullptr;
#pragma unroll
    for (int db = 0; db < 8; db++)
#pragma unroll
        for (int a4 = 0; a4 < 4; a4++) {
            const int d = 32 * db + 8 * a4 + 4 * h32;
            float4 res = make_float4(o[db][4 * a4] * il, o[db][4 * a4 + 1] * il, o[db][4 * a4 + 2] * il, o[db][4 * a4 + 3] * il);
            if (grow) {
                const float4 g = *reinterpret_cast<const float4*>(grow + d);
                res.x /= 1.f + __expf(-g.x); res.y /= 1.f + __expf(-g.y);
                res.z /= 1.f + __expf(-g.z); res.w /= 1.f + __expf(-g.w);
            }
            *reinterpret_cast<float4*>(orow + d) = res;
        }
}

void launch_fa(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV, const int* pos_d,
               int max_t, int ld, int T, hipStream_t st) {
    static bool once = [] {
        MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(fa_prefill_kernel<false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 2 * BUF_BYTES));
        MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(fa_prefill_kernel<true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 2 * BUF_BYTES));
        return true;
    }();
    (void)once;
    const int nb = fa_grid(KV, T);
    if (kv.turbo)
        hipLaunchKernelGGL(fa_prefill_kernel<true>, dim3(nb), dim3(256), 2 * BUF_BYTES, st, qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T);
    else
        hipLaunchKernelGGL(fa_prefill_kernel<false>, dim3(nb), dim3(256), 2 * BUF_BYTES, st, qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T);
    MOEX_LAUNCHED();
}

}  // namespace moex
