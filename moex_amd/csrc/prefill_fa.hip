// FlashAttention-2 chunked causal GQA prefill on gfx950 (replaces attn_fa_k<TB>, kernels.cuh:1443-1728).
//
// Chunks of at most FA_GQA_MAXT tokens (turbo: a quarter) run on the split-K decode kernels instead (fa_plan).
// Workgroup = (kv head, 16 query tokens) = 128 query rows (8 heads x 16 tokens) and 8 wavefronts:
//   - wavefronts 4-7 fill LDS with key tiles of 32, widened to fp16: K as [key][dim] (row stride padded to 528 B:
//     conflict-free reads with immediate offsets), V transposed as [dim][key] and already multiplied by its row scale
//     (int8: vs; turbo: half norm * K3), so P enters the P.V product as plain fp16 probabilities. Turbo K is likewise
//     multiplied by its half norm * K4; int8 K stays exact and its scale is applied to the fp32 score. A pre-pass
//     (fa_image_kernel) widens every tile once into a workspace and the wavefronts copy the images by DMA; without
//     the workspace (MOEX_FA_IMAGES=0, an allocation that failed, the no-allocation entry point) they load and widen
//     each tile themselves;
//   - wavefronts 0-3 compute, 32 query rows each (wavefront w: tokens 4w .. 4w+3, row r = (token 4w + r/8,
//     head r%8)): S^T = K . Q^T and O^T += V^T . P^T on v_mfma_f32_32x32x16_f16 with Q fp16 in registers. The 32x32
//     D layout gives each lane one query row (lane % 32) and 16 keys. LDS operand reads are issued two MFMAs ahead
//     of their use.
// A SIMD holds one wavefront of each kind, so the filling runs beside the other's MFMAs; one barrier per tile (per
// pair of tiles on the image path). The DMA wavefronts' barrier is a bare s_barrier: __syncthreads() would make them
// wait for the images still in flight.
// Lazy rescale: O and l are only rescaled when a row's maximum grows by more than 8 (log2 units) over the value the
// probabilities are referenced to (m_ref, set by tile 0), so p <= 2^8 and the VALU touches O only then. A score
// enters the softmax as s * scale - m_ref in one fma. Each lane tests its own half of the row against the slack (a
// wavefront-wide ballot); only a rescale needs the row's full maximum, from the lane ^ 32 exchange.
// Softmax in base 2 (scale 1/sqrt(256) * log2(e), kernels.cuh:1513). Rounding: Q, P and the scaled V values are
// fp16 MFMA operands with fp32 accumulation; the reference rounds Q and P * vscale (kernels.cuh:1508,1656).
#include <algorithm>
#include <cstdlib>
#include <map>
#include <mutex>
#include <type_traits>
#include "common.hpp"

namespace moex {

namespace {
constexpr int FT = 16;                      // tokens per workgroup
constexpr int BK = 32;                      // keys per tile
constexpr int VST = BK + 8;                 // V^T row stride in halves (80 B: conflict-free A-operand reads)
constexpr int KST = AHD + 8;                // K row stride in halves (528 B: rows shift by 4 banks, conflict-free reads)
constexpr int KT_BYTES = BK * KST * 2;      // 16.5 KB
constexpr int VT_BYTES = AHD * VST * 2;     // 36 KB
constexpr int SC_BYTES = BK * 4;            // per-key score scale
// One tile buffer in LDS: widened K rows, scaled V^T, the score scales and a spare slot. A tile image in global memory
// (the pre-pass output) holds the same bytes, so a DMA copies it as is.
constexpr int TILE_BYTES = KT_BYTES + VT_BYTES + 2 * SC_BYTES;  // 37632 B
constexpr int FA_GQA_MAXT = 64;             // int8 chunks up to this many tokens (turbo: a quarter) run on the
                                            // split-K decode kernels
constexpr float SL2 = 0.0625f * 1.4426950408889634f;
constexpr float TK4 = 0.241529f / 127.f, TK3 = 0.190207f / 127.f;
constexpr int FA_KPF = 2;                   // LDS operand reads in flight ahead of the MFMAs
constexpr float RESCALE_LSUM = 256.f;       // p <= 2^8 between rescales: a lane's sum of p beyond it asks for the row max

constexpr uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a + 128) | ((uint32_t)(b + 128) << 8) | ((uint32_t)(c + 128) << 16) | ((uint32_t)(d + 128) << 24);
}
constexpr uint32_t K4T0 = pack4(-127, -96, -75, -58), K4T1 = pack4(-44, -31, -18, -6);
constexpr uint32_t K4T2 = pack4(6, 18, 31, 44), K4T3 = pack4(58, 75, 96, 127);
constexpr uint32_t V3T0 = pack4(-127, -79, -45, -14), V3T1 = pack4(14, 45, 79, 127);

__device__ __forceinline__ uint32_t lut16(uint32_t idx) {  // 4 nibble indices (one per byte) -> 4 biased K codes
    const uint32_t s = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(K4T1, K4T0, s), hi = __builtin_amdgcn_perm(K4T3, K4T2, s);
    // byte b from hi when bit 3 of index b is set: selector b + 4 picks byte b of the first perm operand
    return __builtin_amdgcn_perm(hi, lo, 0x03020100u | ((idx >> 1) & 0x04040404u));
}
// 4x4 byte transpose: r[k] = 4 bytes (dims) of key k -> c[d] = 4 bytes (keys) of dim d
__device__ __forceinline__ void tr4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3, uint32_t c[4]) {
    const uint32_t t0 = __builtin_amdgcn_perm(r1, r0, 0x05010400u), t1 = __builtin_amdgcn_perm(r1, r0, 0x07030602u);
    const uint32_t t2 = __builtin_amdgcn_perm(r3, r2, 0x05010400u), t3 = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
    c[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u); c[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    c[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u); c[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}
// V^T key positions within each 16-key group are [0..3, 8..11, 4..7, 12..15]: a P.V A operand (keys 16m + 4h + 0..3
// and 16m + 8 + 4h + 0..3) is the 8 contiguous halves at position 16m + 8h, and one staging thread writes them.

// raw global data of one tile held by a thread between the load and the LDS write
constexpr int TPK = 256 / BK;               // threads per K row; each owns BK dims (BK bytes of int8)
struct StageK {
    uint4 k[BK / 16];  // int8: BK bytes of key t/TPK (dims BK*(t%TPK) ..); turbo: the first BK/32 hold its nibbles
    float kn;          // turbo: the half norm of those dims
    float ks;          // int8: the row scale of key k0 + t % BK (times sl2 when stored); turbo: unused
};
// V: thread t stages dims 4*(t%64) .. +3 of the 8 keys 16m + 4h + {0..3, 8..11} with m = t/128, h = (t/64)%2
struct StageV {
    uint32_t v[8];     // int8: 4 bytes of each key; turbo: low byte | high byte << 8
    float vs[8];       // scales of those keys (turbo: the half norm of the thread's dims, times K3 when stored)
};
__device__ __forceinline__ int vkey(int tid, int i) { return 16 * (tid >> 7) + 4 * ((tid >> 6) & 1) + (i & 3) + 8 * (i >> 2); }

// A scale product that is converted to fp16 later goes through r32 (rounded to fp32 first, then to fp16): otherwise
// the compiler may fuse the product and the conversion into one v_fma_mixlo (one rounding) in one kernel and not in
// another, and the tile images and the in-kernel widening must hold the same bytes (measured: one turbo half norm in
// 8192 came out one fp16 ulp apart between two kernels that inline the same code)
__device__ __forceinline__ float r32(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

// FULL: every key of the tile exists (no clamping / masking)
template <bool TB, bool FULL = false>
__device__ __forceinline__ void load_k(StageK& S, moex_kv_cache kv, size_t rbase, int k0, int hi, int tid) {
    const int key = tid / TPK, c = tid % TPK, t = k0 + key;
    const size_t row = rbase + (FULL || t < hi ? t : hi - 1);
    if (TB) {  // dims BK*c .. +BK-1 are nibble bytes (BK/2)*c .. of the row (halves are contiguous in the layout)
        const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(kv.k) + row * TQ_KB + c * (BK / 2));
#pragma unroll
        for (int i = 0; i < BK / 32; i++) S.k[i] = p[i];
        S.kn = kv.ks[row * 2 + (BK * c) / 128];
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(kv.k + row * AHD + c * BK);
#pragma unroll
        for (int i = 0; i < BK / 16; i++) S.k[i] = p[i];
    }
    if (!TB) {  // every thread loads a scale (branch-free); threads < BK own key tid's. The loaded values are
                // only scaled when stored, so a load's first use is its store
        const int tt = k0 + (tid & (BK - 1));
        S.ks = kv.ks[rbase + (FULL || tt < hi ? tt : hi - 1)];
    }
}

template <bool TB, bool FULL = false>
__device__ __forceinline__ void load_v(StageV& S, moex_kv_cache kv, size_t rbase, int k0, int hi, int tid) {
    const int dg = tid & 63;
    if (FULL && !TB) {  // rows k0 + vkey(tid, 0) + {0..3, 8..11}: one base address, constant offsets
        const size_t row0 = rbase + k0 + vkey(tid, 0);
        const int8_t* vp = kv.v + row0 * AHD + dg * 4;
#pragma unroll
        for (int i = 0; i < 8; i++) S.v[i] = *reinterpret_cast<const uint32_t*>(vp + ((i & 3) + 8 * (i >> 2)) * AHD);
        const float4 a = *reinterpret_cast<const float4*>(kv.vs + row0), b = *reinterpret_cast<const float4*>(kv.vs + row0 + 8);
        S.vs[0] = a.x; S.vs[1] = a.y; S.vs[2] = a.z; S.vs[3] = a.w;
        S.vs[4] = b.x; S.vs[5] = b.y; S.vs[6] = b.z; S.vs[7] = b.w;
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int t = k0 + vkey(tid, i);
        const size_t row = rbase + (FULL || t < hi ? t : hi - 1);
        if (TB) {
            const uint8_t* vp = reinterpret_cast<const uint8_t*>(kv.v) + row * TQ_VB;
            const int b = dg >> 5;
            S.v[i] = (uint32_t)vp[b * 32 + (dg & 31)] | ((uint32_t)vp[64 + b * 16 + ((dg & 31) >> 1)] << 8);
            S.vs[i] = kv.vs[row * 2 + b];
        } else {
            S.v[i] = *reinterpret_cast<const uint32_t*>(kv.v + row * AHD + dg * 4);
            S.vs[i] = kv.vs[row];
        }
    }
}

template <bool TB, bool FULL = false>
__device__ __forceinline__ void store_k(const StageK& S, unsigned char* kbuf, float* sbuf, float* spare, int k0, int hi,
                                        int tid) {
    _Float16* Kt = reinterpret_cast<_Float16*>(kbuf);
    const int key = tid / TPK, c = tid % TPK;
    const bool ok = k0 + key < hi;
    uint32_t w[BK / 2];  // BK halves
    if (TB) {  // BK nibbles -> biased codes -> fp16, times the half norm * K4
        const _Float16 sch = (_Float16)r32(S.kn * TK4);
        const half2_t sc = half2_t{sch, sch};
#pragma unroll
        for (int i = 0; i < BK / 8; i++) {
            const uint4 u = S.k[i >> 2];
            const uint32_t x = (i & 3) == 0 ? u.x : (i & 3) == 1 ? u.y : (i & 3) == 2 ? u.z : u.w;
            const uint32_t e = lut16(x & 0x0f0f0f0fu), o = lut16((x >> 4) & 0x0f0f0f0fu);
            const uint32_t d01 = __builtin_amdgcn_perm(o, e, 0x05010400u), d23 = __builtin_amdgcn_perm(o, e, 0x07030602u);
            uint32_t a0, a1, a2, a3;
            biased4_to_h4(d01, a0, a1);
            biased4_to_h4(d23, a2, a3);
            w[4 * i] = h22u(u2h2(a0) * sc); w[4 * i + 1] = h22u(u2h2(a1) * sc);
            w[4 * i + 2] = h22u(u2h2(a2) * sc); w[4 * i + 3] = h22u(u2h2(a3) * sc);
        }
    } else {
#pragma unroll
        for (int i = 0; i < BK / 4; i++) {
            const uint4 u = S.k[i >> 2];
            const uint32_t x = (i & 3) == 0 ? u.x : (i & 3) == 1 ? u.y : (i & 3) == 2 ? u.z : u.w;
            i8x4_to_h4(x, w[2 * i], w[2 * i + 1]);
        }
    }
    if (!FULL && !ok) {
#pragma unroll
        for (int i = 0; i < BK / 2; i++) w[i] = 0u;
    }
#pragma unroll
    for (int q = 0; q < BK / 8; q++)  // chunks of 8 halves: dims BK*c + 8q
        *reinterpret_cast<uint4*>(Kt + key * KST + ((BK / 8) * c + q) * 8) = make_uint4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
    // threads >= BK write their copy to the spare slot (branch-free)
    float* dst = tid < BK ? sbuf + tid : spare + (tid & (BK - 1));
    *dst = FULL || k0 + (tid & (BK - 1)) < hi ? (TB ? SL2 : S.ks * SL2) : 0.f;
}

template <bool TB, bool FULL = false>
__device__ __forceinline__ void store_v(const StageV& S, unsigned char* vbuf, int k0, int hi, int tid) {
    _Float16* Vt = reinterpret_cast<_Float16*>(vbuf);
    const int dg = tid & 63;
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
        r[i] = FULL || k0 + vkey(tid, i) < hi ? x : 0x80808080u;  // zero past the end
    }
    // per dim e: the 8 keys -> fp16 times the key's scale, one 16-byte write at V^T position 16m + 8h
    half2_t vsc[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        vsc[i] = TB ? half2_t{(_Float16)r32(S.vs[2 * i] * TK3), (_Float16)r32(S.vs[2 * i + 1] * TK3)}
                    : half2_t{(_Float16)S.vs[2 * i], (_Float16)S.vs[2 * i + 1]};
    uint32_t ca[4], cb[4];
    tr4x4(r[0], r[1], r[2], r[3], ca);
    tr4x4(r[4], r[5], r[6], r[7], cb);
    _Float16* base = Vt + (4 * dg) * VST + 16 * (tid >> 7) + 8 * ((tid >> 6) & 1);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        uint32_t h0, h1, h2, h3;
        biased4_to_h4(ca[e], h0, h1);
        biased4_to_h4(cb[e], h2, h3);
        *reinterpret_cast<uint4*>(base + e * VST) = make_uint4(h22u(u2h2(h0) * vsc[0]), h22u(u2h2(h1) * vsc[1]),
                                                               h22u(u2h2(h2) * vsc[2]), h22u(u2h2(h3) * vsc[3]));
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
// Key pieces of token tile t (keys [0, pos0 + min(FT (t + 1), T))), for chunks whose token tiles leave the chip
// underfilled (KV x tiles < CUs; the host then passes nsf > 1). Computed on the device (pos0 is a device value), the
// same way by the FA kernel and the merge: a tile of n key tiles takes floor(n / w) pieces (1 to nsf), w = the chip's
// average share of the work, so the pieces of all tiles fill the chip about once; w is at least
// max(FA_MINW, 2 x token tiles), as each workgroup first loads its queries (more of them for a longer chunk) and
// each piece adds merge traffic. Piece s is tiles [s n / ns, (s + 1) n / ns): at least w >= 8 tiles, so its first key
// is below every row of the token tile (each row sees a key in every piece).
constexpr int FA_MINW = 8;
constexpr int FA_NSF_MAX = 32;
constexpr int FP_ROW = AHD + 4;  // a piece's partial row: O[256], m, l, 2 spare (16-byte aligned rows)
__host__ __device__ inline int fa_piece_w(int pos0, int T, int KV, int NT, int ncu) {
    const int total = (NT * ((2 * pos0 + T + FT) / 2) + NT * (BK - 1)) / BK;  // about the sum of n (split chunks: NT <= CUs)
    const int m = FA_MINW > 2 * NT ? FA_MINW : 2 * NT, v = (KV * total + ncu - 1) / ncu;
    return m > v ? m : v;
}
__host__ __device__ inline int fa_pieces(int t, int pos0, int T, int nsf, int w) {
    const int n = (pos0 + (FT * (t + 1) < T ? FT * (t + 1) : T) + BK - 1) / BK, k = n / w;
    return k < 1 ? 1 : k > nsf ? nsf : k;
}
int fa_grid(int KV, int T) {
    const int NT = (T + FT - 1) / FT;
    if (8 % KV == 0) { const int xpk = 8 / KV; return 8 * ((NT + xpk - 1) / xpk); }
    return KV * NT;
}
}  // namespace

// Tile images: a workgroup widens 32-key tiles j = blockIdx.x, + gridDim.x, .. of one kv head (keys past pos0 + T
// zeroed) into their images, with the staging wavefronts' arithmetic. The prefill kernel then copies images into LDS
// by DMA, so each tile is widened once instead of once per token tile. The stores go out in whole rows: the V^T part,
// which a staging thread holds as 16-byte pieces of rows 320 bytes apart, is assembled in LDS first, and int8 K rows
// are taken by 16-byte slots (two rows a wavefront instruction). The grid is sized from the cache (the chunk's end is
// a device value) but capped: a cache of 262 144 positions would otherwise launch 8 194 workgroups per kv head, most
// of them for tiles past the chunk's end, and their dispatch alone took microseconds.
template <bool TB>
__global__ void __launch_bounds__(256) fa_image_kernel(moex_kv_cache kv, const int* __restrict__ pos_d, int T, int max_t,
                                                       int ntmax, unsigned char* __restrict__ img) {
    const int kvh = blockIdx.y, hi = *pos_d + T, tid = threadIdx.x;
    const size_t rbase = (size_t)kvh * max_t;
    __shared__ __align__(16) unsigned char vl[VT_BYTES];  // the tile's V^T, written transposed, copied out in rows
    for (int j = blockIdx.x; j < ntmax && j * BK < hi; j += gridDim.x) {
        const int k0 = j * BK;
        unsigned char* t = img + ((size_t)kvh * ntmax + j) * TILE_BYTES;
        float* sc = reinterpret_cast<float*>(t + KT_BYTES + VT_BYTES);
        StageK sk;
        StageV sv;
        if (!TB) {
            // int8 K rows by 16-byte slots: thread t takes slots t + 256 u (row s / 32, dims 8 (s % 32) ..), so a
            // wavefront's loads read 2 whole rows and its stores write 2 whole rows of the image
            uint2 kr[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int sl = tid + 256 * u, r = sl >> 5;
                kr[u] = *reinterpret_cast<const uint2*>(kv.k + (rbase + min(k0 + r, hi - 1)) * AHD + 8 * (sl & 31));
            }
            const float ks = kv.ks[rbase + min(k0 + (tid & (BK - 1)), hi - 1)];
            if (k0 + BK <= hi) load_v<TB, true>(sv, kv, rbase, k0, hi, tid);
            else load_v<TB>(sv, kv, rbase, k0, hi, tid);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int sl = tid + 256 * u, r = sl >> 5;
                uint32_t h0, h1, h2, h3;
                i8x4_to_h4(kr[u].x, h0, h1);
                i8x4_to_h4(kr[u].y, h2, h3);
                const bool ok = k0 + r < hi;
                *reinterpret_cast<uint4*>(t + r * (KST * 2) + 16 * (sl & 31)) =
                    ok ? make_uint4(h0, h1, h2, h3) : make_uint4(0u, 0u, 0u, 0u);
            }
            if (tid < BK) sc[tid] = k0 + tid < hi ? ks * SL2 : 0.f;
            if (k0 + BK <= hi) store_v<TB, true>(sv, vl, k0, hi, tid);
            else store_v<TB>(sv, vl, k0, hi, tid);
        } else if (k0 + BK <= hi) {
            load_k<TB, true>(sk, kv, rbase, k0, hi, tid);
            load_v<TB, true>(sv, kv, rbase, k0, hi, tid);
            store_k<TB, true>(sk, t, sc, sc + BK, k0, hi, tid);
            store_v<TB, true>(sv, vl, k0, hi, tid);
        } else {
            load_k<TB>(sk, kv, rbase, k0, hi, tid);
            load_v<TB>(sv, kv, rbase, k0, hi, tid);
            store_k<TB>(sk, t, sc, sc + BK, k0, hi, tid);
            store_v<TB>(sv, vl, k0, hi, tid);
        }
        __syncthreads();
        // the 1024 data slots of V^T (rows of 5 16-byte slots, the fifth padding): slot d = row d / 4, piece d % 4
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int d = tid + 256 * u, off = (d >> 2) * (VST * 2) + 16 * (d & 3);
            *reinterpret_cast<uint4*>(t + KT_BYTES + off) = *reinterpret_cast<const uint4*>(vl + off);
        }
        __syncthreads();
    }
}

// Tile image j of a kv head (src: its first image) -> the LDS buffer buf, by DMA wavefront pw (0..3): 1 KB pieces
// pw, pw + 4, .. (10 for pw = 0, 9 for the others), leaving out the padding slots nobody reads.
__device__ __forceinline__ void fa_issue_img(const unsigned char* src, int j, unsigned char* buf, int pw, int lane) {
    constexpr int NP = (TILE_BYTES + 1023) / 1024;  // 37 pieces, the last one partial
    static_assert(NP == 37 && TILE_BYTES % 16 == 0, "image pieces");
    const unsigned char* g = src + (size_t)j * TILE_BYTES + 16 * lane;
#pragma unroll
    for (int u = 0; u < 10; u++) {
        const int i = pw + 4 * u, sl = 64 * i + lane;  // 16-byte slot of the image
        // padding: slot 32 of each 33-slot K row, slot 4 of each 5-slot V^T row, the spare scales, the end
        const bool pad = sl < KT_BYTES / 16 ? sl % 33 == 32
                         : sl < (KT_BYTES + VT_BYTES) / 16 ? (sl - KT_BYTES / 16) % 5 == 4
                                                           : sl >= (KT_BYTES + VT_BYTES + SC_BYTES) / 16;
        if (i < NP && !pad)
            __builtin_amdgcn_global_load_lds((gptr_t)(g + i * 1024), (lptr_t)(buf + i * 1024), 16, 0, 0);
    }
}
// The DMA wavefronts' wait for the first pair of a run of ntiles tiles issued back to back (the tiles after it are
// still in flight: 10 transfers a tile for pw = 0, 9 for the others)
__device__ __forceinline__ void fa_wait_first_pair(int ntiles, int pw) {
    if (ntiles >= 4) { if (pw == 0) wait_vm<20>(); else wait_vm<18>(); }
    else if (ntiles == 3) { if (pw == 0) wait_vm<10>(); else wait_vm<9>(); }
    else wait_vm<0>();
}

// One key tile of a computing wavefront (32 query rows): S^T = K . Q^T, the lazily rescaled softmax and O^T += V^T . P^T.
// Kt, Vt, scl: the tile's buffer in LDS; k0: its first key; first: the first tile this wavefront computes for its
// rows (it sets m_ref, and each of its rows sees the tile's first key); prow: the last key the lane's row sees; wmin:
// the last key the wavefront's first row sees (a tile reaching past it is a diagonal one).
__device__ __forceinline__ void fa_tile(const _Float16* Kt, const _Float16* Vt, const float* scl, int k0, bool first,
                                        int prow, int wmin, int r, int h32, const half8_t (&qf)[16],
                                        float16_t (&o)[8], float& m_ref, float& l_run) {
    const half2_t ones = half2_t{(_Float16)1.f, (_Float16)1.f};
    float16_t sc;
#pragma unroll
    for (int i = 0; i < 16; i++) sc[i] = 0.f;
    float4 kq[4];  // the score scales, read during the last Q.K MFMAs
    {   // K operands read FA_KPF MFMAs ahead of their use (LDS latency)
        const _Float16* krow = Kt + r * KST + 8 * h32;
        half8_t ka[FA_KPF];
#pragma unroll
        for (int s = 0; s < FA_KPF; s++) ka[s] = *reinterpret_cast<const half8_t*>(krow + 16 * s);
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const half8_t a = ka[s % FA_KPF];
            if (s + FA_KPF < 16)
                ka[s % FA_KPF] = *reinterpret_cast<const half8_t*>(krow + 16 * (s + FA_KPF));
            if (s == 16 - 2) {
#pragma unroll
                for (int a4 = 0; a4 < 4; a4++) kq[a4] = *reinterpret_cast<const float4*>(scl + 8 * a4 + 4 * h32);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep each read FA_KPF MFMAs ahead of its use
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[s], sc, 0, 0, 0);
        }
    }
    // scores relative to the row's reference maximum: t = s * scale - m_ref in one fma (tile 0 sets m_ref: key 0
    // is unmasked in every row, so it is finite)
    const float mneg = first ? 0.f : -m_ref;
#pragma unroll
    for (int a4 = 0; a4 < 4; a4++) {
        sc[4 * a4] = fmaf(sc[4 * a4], kq[a4].x, mneg); sc[4 * a4 + 1] = fmaf(sc[4 * a4 + 1], kq[a4].y, mneg);
        sc[4 * a4 + 2] = fmaf(sc[4 * a4 + 2], kq[a4].z, mneg); sc[4 * a4 + 3] = fmaf(sc[4 * a4 + 3], kq[a4].w, mneg);
    }
    if (k0 + BK - 1 > wmin) {  // a diagonal tile: causal mask per row
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (k0 + 8 * (i >> 2) + 4 * h32 + (i & 3) > prow) sc[i] = -INFINITY;
    }
    // ---- P^T (fp16) as B operands: MFMA m (keys 16m ..) takes S elements 8m .. 8m+7 ----
    half8_t pf[2];
    float ls = 0.f;
    auto make_p = [&]() {
        ls = 0.f;
#pragma unroll
        for (int m = 0; m < 2; m++)
#pragma unroll
            for (int jj = 0; jj < 8; jj += 2) {
                const float p0 = fast_exp2(sc[8 * m + jj]), p1 = fast_exp2(sc[8 * m + jj + 1]);
                const half2_t ph = half2_t{(_Float16)p0, (_Float16)p1};
                pf[m][jj] = ph[0]; pf[m][jj + 1] = ph[1];
                ls = __builtin_amdgcn_fdot2(ph, ones, ls, false);
            }
    };
    auto row_max = [&]() {  // this lane's half of the row; the other half is in lane ^ 32
        float mt = sc[0];
#pragma unroll
        for (int i = 1; i < 16; i++) mt = fmaxf(mt, sc[i]);
        return mt;
    };
    if (first) {
        float mt = row_max();
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        m_ref = mt;
#pragma unroll
        for (int i = 0; i < 16; i++) sc[i] -= mt;
        make_p();
    } else {
        // lazy rescale: O and l are referenced to m_ref and move only when a row's maximum passes it by the
        // slack. No score of a lane's half passes m_ref + slack while its probabilities sum to at most 2^slack,
        // so the row maximum is needed only when some lane's sum exceeds that (or overflowed)
        make_p();
        if (__ballot(!(ls <= RESCALE_LSUM))) {
            const float mt = row_max();
            const float d = fmaxf(fmaxf(mt, __shfl_xor(mt, 32)), 0.f);
            const float cf = fast_exp2(-d);
#pragma unroll
            for (int db = 0; db < 8; db++)
#pragma unroll
                for (int i = 0; i < 16; i++) o[db][i] *= cf;
            l_run *= cf;
            m_ref += d;
#pragma unroll
            for (int i = 0; i < 16; i++) sc[i] -= d;
            make_p();
        }
    }
    l_run += ls;
    // ---- O^T += V^T . P^T ----
    {   // V^T operands read FA_KPF MFMAs ahead (MFMA q: dims 32*(q/2) + r, keys 16*(q%2) ..)
        const _Float16* vrow = Vt + r * VST + 8 * h32;
        half8_t va[FA_KPF];
#pragma unroll
        for (int q = 0; q < FA_KPF; q++) va[q] = *reinterpret_cast<const half8_t*>(vrow + 32 * (q >> 1) * VST + 16 * (q & 1));
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const half8_t a = va[q % FA_KPF];
            if (q + FA_KPF < 16) {
                const int qn = q + FA_KPF;
                va[q % FA_KPF] = *reinterpret_cast<const half8_t*>(vrow + 32 * (qn >> 1) * VST + 16 * (qn & 1));
            }
            __builtin_amdgcn_sched_barrier(0);
            o[q >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[q & 1], o[q >> 1], 0, 0, 0);
        }
    }
}

// What a block does: up to two segments, each a token tile over key tiles [ja, ja + ntiles), and what its epilogue
// writes: the output rows, a piece's partial rows for fa_merge_kernel, or its half of a pair (merged in the kernel).
enum { FA_MODE_ONE = 0, FA_MODE_SPLIT = 1, FA_MODE_PAIR = 2 };
enum { FA_EPI_OUT = 0, FA_EPI_PIECE = 1, FA_EPI_PAIR = 2 };
struct FaSeg {
    int tile, ja, ntiles, epi;
};
__host__ __device__ inline int fa_ntiles(int t, int pos0, int T) {  // key tiles token tile t sees
    return (pos0 + (FT * (t + 1) < T ? FT * (t + 1) : T) + BK - 1) / BK;
}

// Pairs (full grids): token tile t's work grows with t, so one block per tile leaves the chip waiting for the last
// tiles (at pos0 = 0 the heaviest has twice the average). Pair q = tiles NT - 1 - q (heavy) and q (light), both of one
// kv head, goes to two blocks on one XCD: block 0 takes key tiles [0, s) of the heavy tile, block 1 key tiles [s, n) of
// the heavy one and then the light tile, s chosen so both take about as long (block 1 gives up FA_PAIR_EXTRA tiles for
// its second segment). The heavy tile's halves merge in
// the kernel (fa_pair_merge). A pair whose halves would differ by less than FA_PAIR_MIN tiles is not split; an odd
// tile count leaves the middle tile to one block.
constexpr int FA_PAIR_MIN = 4;
constexpr int FA_PAIR_EXTRA = 5;  // key tiles the second block of a pair gives up for its second segment (see fa_pair_segs)
constexpr int FA_PAIR_SLOT = 64 * 128 + 128;  // floats per wavefront half: O (lane-interleaved float4s), {m, l} per lane
__device__ __forceinline__ bool fa_pair_block(int b, int KV, int NT, int& kvh, int& q, int& role) {
    if (8 % KV == 0) {  // blocks b and b + 8 run on one XCD: the two blocks of a pair
        const int xpk = 8 / KV, x = b & 7, i = b >> 3;
        kvh = x / xpk;
        q = (i >> 1) * xpk + x % xpk;
        role = i & 1;
    } else {
        const int per = 2 * ((NT + 1) / 2);
        kvh = b / per;
        q = (b % per) >> 1;
        role = b & 1;
        if (kvh >= KV) return false;
    }
    return q < NT / 2 || (q == NT / 2 && (NT & 1) && role == 0);
}
__host__ inline int fa_pair_grid(int KV, int T) {
    const int nq = ((T + FT - 1) / FT + 1) / 2;
    if (8 % KV == 0) { const int xpk = 8 / KV; return 16 * ((nq + xpk - 1) / xpk); }
    return KV * 2 * nq;
}
// pk packs the pair parameters: bits 0-7 the minimum tiles of the heavy tile's second part, 8-15 the second block's
// extra cost in tiles (its second segment's queries, epilogue and output)
__device__ __forceinline__ int fa_pair_segs(int q, int role, int pos0, int T, int NT, int pk, FaSeg (&sg)[2]) {
    const int pmin = pk & 255, extra = (pk >> 8) & 255;
    if (q == NT / 2) {  // the middle tile of an odd count
        sg[0] = FaSeg{q, 0, fa_ntiles(q, pos0, T), FA_EPI_OUT};
        return 1;
    }
    const int tH = NT - 1 - q, nH = fa_ntiles(tH, pos0, T), nL = fa_ntiles(q, pos0, T);
    // block 1's part starts at or below every row's last key, so each row sees keys in both parts
    // equal time, not equal tiles: block 0 runs s tiles, block 1 the other nH + nL - s plus its extra
    const int s = min((nH + nL + extra + 1) / 2, (pos0 + FT * tH) / BK);
    if (s < 1 || nH - s < pmin) {
        sg[0] = role ? FaSeg{q, 0, nL, FA_EPI_OUT} : FaSeg{tH, 0, nH, FA_EPI_OUT};
        return 1;
    }
    if (role == 0) {
        sg[0] = FaSeg{tH, 0, s, FA_EPI_PAIR};
        return 1;
    }
    sg[0] = FaSeg{tH, s, nH - s, FA_EPI_PAIR};
    sg[1] = FaSeg{q, 0, nL, FA_EPI_OUT};
    return 2;
}

// The pair merge, per computing wavefront (32 rows, the same rows in both blocks). Its arrival counter pcnt[2 slot]
// is even when a launch starts (zeroed at allocation, +2 per launch); the first arrival stores its {O, m, l} with
// agent-scope stores, waits for them to complete and marks pcnt[2 slot + 1] with the count the second arrival will
// have seen. The second arrival waits for that mark (the first is past its arrival, so it is running and the wait
// ends; it is bounded all the same), loads the partner's half the same way and merges. The merge is symmetric in
// the two halves, so the bits do not depend on which block arrives first. Returns true in the merging wavefront.
__device__ __forceinline__ bool fa_pair_merge(float* __restrict__ pbuf, unsigned* __restrict__ pcnt, int slot, int lane,
                                              float16_t (&o)[8], float m_ref, float& l_run) {
    // products rounded before the sum (no fma contraction), so the merge is symmetric in the two halves
#pragma clang fp contract(off)
    unsigned* cnt = pcnt + 2 * slot;
    unsigned old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(pbuf + (size_t)slot * FA_PAIR_SLOT, 0, FA_PAIR_SLOT * 4, 0x00020000);
    constexpr int SC1 = 16;  // agent-scope accesses (the partner may run on another XCD)
    typedef float f4v __attribute__((ext_vector_type(4)));
    typedef float f2v __attribute__((ext_vector_type(2)));
    if (!(old & 1)) {
#pragma unroll
        for (int db = 0; db < 8; db++)
#pragma unroll
            for (int a4 = 0; a4 < 4; a4++)
                __builtin_amdgcn_raw_buffer_store_b128(
                    f4v{o[db][4 * a4], o[db][4 * a4 + 1], o[db][4 * a4 + 2], o[db][4 * a4 + 3]}, rs,
                    ((4 * db + a4) * 64 + lane) * 16, 0, SC1);
        __builtin_amdgcn_raw_buffer_store_b64(f2v{m_ref, l_run}, rs, 64 * 128 * 4 + lane * 8, 0, SC1);
        __builtin_amdgcn_s_waitcnt(0);  // the stores have completed
        if (lane == 0) __hip_atomic_store(cnt + 1, old + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    for (int it = 0; it < (1 << 22); it++) {
        const unsigned mark = __builtin_amdgcn_readfirstlane(__hip_atomic_load(cnt + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (mark == old) break;
        __builtin_amdgcn_s_sleep(4);
    }
    const f2v ml = __builtin_amdgcn_raw_buffer_load_b64(rs, 64 * 128 * 4 + lane * 8, 0, SC1);
    const float M = fmaxf(m_ref, ml.x), ca = fast_exp2(ml.x - M), cb = fast_exp2(m_ref - M);
    l_run = ml.y * ca + l_run * cb;
#pragma unroll
    for (int db = 0; db < 8; db++)
#pragma unroll
        for (int a4 = 0; a4 < 4; a4++) {
            const f4v pa = __builtin_amdgcn_raw_buffer_load_b128(rs, ((4 * db + a4) * 64 + lane) * 16, 0, SC1);
#pragma unroll
            for (int e = 0; e < 4; e++)
                o[db][4 * a4 + e] = pa[e] * ca + o[db][4 * a4 + e] * cb;
        }
    return true;
}

// The lane's output row: O / l * sigmoid(gate) (the gate by the hardware reciprocal: 1 ulp; the output's tolerance
// is fp16-level)
__device__ __forceinline__ void fa_write_out(const float16_t (&o)[8], float l_run, float* __restrict__ out,
                                             const float* __restrict__ q_gate, size_t t, int head, int H, int ld,
                                             int h32) {
    const float il = 1.f / l_run;
    float* orow = out + (t * H + head) * AHD;
    const float* grow = q_gate ? q_gate + t * ld + head * 2 * AHD + AHD : nullptr;
    // the gate row is loaded a dims block ahead of its use (loads issued one by one behind the stores would each
    // wait for the memory round trip)
    float4 gc[4], gn[4];
    if (grow)
#pragma unroll
        for (int a4 = 0; a4 < 4; a4++) gc[a4] = *reinterpret_cast<const float4*>(grow + 8 * a4 + 4 * h32);
#pragma unroll
    for (int db = 0; db < 8; db++) {
        if (grow && db + 1 < 8)
#pragma unroll
            for (int a4 = 0; a4 < 4; a4++)
                gn[a4] = *reinterpret_cast<const float4*>(grow + 32 * (db + 1) + 8 * a4 + 4 * h32);
#pragma unroll
        for (int a4 = 0; a4 < 4; a4++) {
            const int d = 32 * db + 8 * a4 + 4 * h32;
            float4 res = make_float4(o[db][4 * a4] * il, o[db][4 * a4 + 1] * il, o[db][4 * a4 + 2] * il, o[db][4 * a4 + 3] * il);
            if (grow) {
                const float4 g = gc[a4];
                res.x *= __builtin_amdgcn_rcpf(1.f + __expf(-g.x)); res.y *= __builtin_amdgcn_rcpf(1.f + __expf(-g.y));
                res.z *= __builtin_amdgcn_rcpf(1.f + __expf(-g.z)); res.w *= __builtin_amdgcn_rcpf(1.f + __expf(-g.w));
            }
            *reinterpret_cast<float4*>(orow + d) = res;
        }
#pragma unroll
        for (int a4 = 0; a4 < 4; a4++) gc[a4] = gn[a4];
    }
}

// Warp-specialised workgroup of 8 wavefronts. Wavefronts 0-3 compute (32 query rows each); wavefronts 4-7 fill the LDS
// tile buffers. Each SIMD holds one wavefront of each kind, so the filling runs beside the other wavefront's MFMAs.
//   IMG = false: the staging wavefronts load the next tiles' int8/turbo K and V and widen them (two buffers: during
//   tile j the computing wavefronts read buffer j%2 while the staging wavefronts fill buffer (j+1)%2; one barrier per
//   tile).
//   IMG = true: the tiles were widened by fa_image_kernel; the staging wavefronts only copy images by DMA into four
//   buffers (two pairs of tiles: one computed while the next lands, one barrier per pair), leaving out the padding
//   slots nobody reads.
template <bool TB, bool IMG, int MODE>
__global__ void __launch_bounds__(512, 1) fa_prefill_kernel(const float* __restrict__ qo, const float* __restrict__ q_gate,
                                                            moex_kv_cache kv, const unsigned char* __restrict__ img,
                                                            int ntmax, float* __restrict__ out, int H, int KV,
                                                            const int* __restrict__ pos_d, int max_t, int ld, int T,
                                                            float* __restrict__ fpart, int nsf, int ncu,
                                                            unsigned* __restrict__ pcnt) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int NB = IMG ? 4 : 2;
#define KBUF(i) (smem + (i) * TILE_BYTES)
#define VBUF(i) (smem + (i) * TILE_BYTES + KT_BYTES)
#define SBUF(i) (reinterpret_cast<float*>(smem + (i) * TILE_BYTES + KT_BYTES + VT_BYTES))
    const int NT = (T + FT - 1) / FT, pos0 = *pos_d;
    // the block's segments (at most two): token tile, key tiles [ja, ja + ntiles), what the epilogue does
    FaSeg sg[2];
    int kvh, nseg = 1, piece = 0, pslot = 0;
    if (MODE == FA_MODE_SPLIT) {
        // block b takes the b-th piece, pieces listed heaviest token tile first, so the blocks left without one are
        // the last ones dispatched (a queued block waits for a whole CU's LDS even when it has nothing to do)
        const int w = fa_piece_w(pos0, T, KV, NT, ncu);
        int b = blockIdx.x, tile, nsp = 1;
        for (tile = NT - 1; tile >= 0; tile--) {
            nsp = fa_pieces(tile, pos0, T, nsf, w);
            if (b < KV * nsp) break;
            b -= KV * nsp;
        }
        if (tile < 0) return;
        kvh = b % KV;
        piece = b / KV;
        const int nall = fa_ntiles(tile, pos0, T), ja = piece * nall / nsp;
        sg[0] = FaSeg{tile, ja, (piece + 1) * nall / nsp - ja, nsp > 1 ? FA_EPI_PIECE : FA_EPI_OUT};
    } else if (MODE == FA_MODE_PAIR) {
        int q, role;
        if (!fa_pair_block(blockIdx.x, KV, NT, kvh, q, role)) return;
        nseg = fa_pair_segs(q, role, pos0, T, NT, nsf, sg);  // nsf: the packed pair parameters
        pslot = (kvh * (NT / 2) + q) * 4;
    } else {
        int tile;
        if (!map_block(blockIdx.x, KV, NT, kvh, tile)) return;
        sg[0] = FaSeg{tile, 0, fa_ntiles(tile, pos0, T), FA_EPI_OUT};
    }
    const size_t rbase = (size_t)kvh * max_t;

    if (threadIdx.x >= 256 && IMG) {
        // ---------------- DMA wavefronts: image j -> buffer j % 4, 1 KB pieces i = pw, pw + 4, .. ----------------
        const int pw = (threadIdx.x >> 6) - 4, lane = threadIdx.x & 63;
        const unsigned char* src = img + (size_t)kvh * ntmax * TILE_BYTES;
        for (int g = 0; g < nseg; g++) {
            const int ja = __builtin_amdgcn_readfirstlane(sg[g].ja), ntiles = __builtin_amdgcn_readfirstlane(sg[g].ntiles);
            auto issue = [&](int j) { fa_issue_img(src, ja + j, smem + (j % NB) * TILE_BYTES, pw, lane); };
            // piece counts per wavefront: 10 for pw = 0 (pieces 0, 4, .., 36), 9 for the others
            // pairs of tiles: pair p = tiles 2p, 2p + 1 in buffers 2 (p % 2), + 1; one barrier per pair
            asm volatile("s_barrier" ::: "memory");  // the queries' reads are out ahead of the first images
            for (int j = 0; j < 4 && j < ntiles; j++) issue(j);
            fa_wait_first_pair(ntiles, pw);
            asm volatile("s_barrier" ::: "memory");  // pair 0 is in buffers 0, 1
            const int np = (ntiles + 1) / 2;
            for (int p = 0; p < np; p++) {
                wait_vm<0>();                            // pair p + 1 has landed
                asm volatile("s_barrier" ::: "memory");  // every computing wavefront is past pair p
                if (2 * p + 4 < ntiles) issue(2 * p + 4);
                if (2 * p + 5 < ntiles) issue(2 * p + 5);
            }
        }
        return;
    }
    if (threadIdx.x >= 256) {
        // ---------------- staging wavefronts ----------------
        const int tid = threadIdx.x - 256;
        for (int g = 0; g < nseg; g++) {
            const int ntiles = __builtin_amdgcn_readfirstlane(sg[g].ntiles), ka = __builtin_amdgcn_readfirstlane(sg[g].ja) * BK;
            const int hi = pos0 + min(FT * (__builtin_amdgcn_readfirstlane(sg[g].tile) + 1), T);
            StageK sk;
            StageV sv;
            load_k<TB>(sk, kv, rbase, ka, hi, tid);
            load_v<TB>(sv, kv, rbase, ka, hi, tid);
            store_k<TB>(sk, KBUF(0), SBUF(0), SBUF(0) + BK, ka, hi, tid);
            store_v<TB>(sv, VBUF(0), ka, hi, tid);
            if (ntiles > 1) {
                load_k<TB>(sk, kv, rbase, ka + BK, hi, tid);
                load_v<TB>(sv, kv, rbase, ka + BK, hi, tid);
            }
            __syncthreads();
            for (int j = 0; j < ntiles; j++) {
                const int k1 = ka + (j + 1) * BK, b = (j + 1) & 1;
                if (j + 1 < ntiles) {
                    if (k1 + BK <= hi) {
                        store_k<TB, true>(sk, KBUF(b), SBUF(b), SBUF(b) + BK, k1, hi, tid);
                        store_v<TB, true>(sv, VBUF(b), k1, hi, tid);
                    } else {
                        store_k<TB>(sk, KBUF(b), SBUF(b), SBUF(b) + BK, k1, hi, tid);
                        store_v<TB>(sv, VBUF(b), k1, hi, tid);
                    }
                }
                if (j + 2 < ntiles) {
                    const int k2 = k1 + BK;
                    if (k2 + BK <= hi) {
                        load_k<TB, true>(sk, kv, rbase, k2, hi, tid);
                        load_v<TB, true>(sv, kv, rbase, k2, hi, tid);
                    } else {
                        load_k<TB>(sk, kv, rbase, k2, hi, tid);
                        load_v<TB>(sv, kv, rbase, k2, hi, tid);
                    }
                }
                // tile j + 1 is in LDS; tile j + 2 stays in flight into registers (__syncthreads would wait for it)
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            }
        }
        return;
    }

    // ---------------- computing wavefronts ----------------
    __builtin_amdgcn_s_setprio(2);  // ahead of the staging wavefronts at the SIMD's issue arbiter
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), h32 = lane >> 5, r = lane & 31;
    constexpr bool PIECEWISE = MODE != FA_MODE_ONE;
    auto segment = [&](const FaSeg& sgc) {
        // wave-uniform (the segment table may sit in scratch; its values would otherwise be taken as divergent)
        const int tile = __builtin_amdgcn_readfirstlane(sgc.tile), ja = __builtin_amdgcn_readfirstlane(sgc.ja);
        const int epi = __builtin_amdgcn_readfirstlane(sgc.epi);
        int ntiles = __builtin_amdgcn_readfirstlane(sgc.ntiles);
        const int t0 = tile * FT, nt = min(FT, T - t0), hi = pos0 + t0 + nt;  // keys [0, hi)
        if (MODE == FA_MODE_ONE) ntiles = (hi + BK - 1) / BK;
        const int tokw = 4 * w + (r >> 3), head = kvh * GQ + (r & 7);                     // this lane's row
        const int prow = min(pos0 + t0 + tokw, hi - 1);                                     // its last visible key
        const int wmin = min(pos0 + t0 + 4 * w, hi - 1);                                    // the wavefront's first row
        const int wmax = min(pos0 + t0 + 4 * w + 3, hi - 1);                                // ... and its last key
        const int wtiles = wmax / BK + 1;  // tiles this wavefront computes

        // Q row (fp16) as B operands: MFMA s covers dims 16s + 8*h32 + 0..7
        half8_t qf[16];
        {
            const float* qrow = qo + ((size_t)(t0 + min(tokw, nt - 1)) * H + head) * AHD;
            float4 qa[32];
#pragma unroll
            for (int s = 0; s < 16; s++) {
                const float4* p4 = reinterpret_cast<const float4*>(qrow + 16 * s + 8 * h32);
                qa[2 * s] = p4[0];
                qa[2 * s + 1] = p4[1];
            }
            // with tile images, the DMA wavefronts send the first images once these reads are out
            if (IMG) asm volatile("s_barrier" ::: "memory");
#pragma unroll
            for (int s = 0; s < 16; s++) {
                const float4 a = qa[2 * s], b = qa[2 * s + 1];
                qf[s] = half8_t{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                                (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
            }
        }
        float16_t o[8];
#pragma unroll
        for (int db = 0; db < 8; db++)
#pragma unroll
            for (int i = 0; i < 16; i++) o[db][i] = 0.f;
        float m_ref = -INFINITY, l_run = 0.f;
        __syncthreads();

        // pieces: this wavefront's tiles of the piece, then barriers only while the others finish theirs (one loop
        // with a per-tile test makes the compiler spill once the trip count is not the tile count)
        const int wt = max(0, min(ntiles, wtiles - ja));
        for (int j = 0; j < (PIECEWISE ? wt : ntiles); j++) {
            if (PIECEWISE || j < wtiles) {
                fa_tile(reinterpret_cast<const _Float16*>(KBUF(j % NB)), reinterpret_cast<const _Float16*>(VBUF(j % NB)),
                        SBUF(j % NB), (ja + j) * BK, j == 0, prow, wmin, r, h32, qf, o, m_ref, l_run);
            }
            if (!IMG || (j & 1) || j + 1 == ntiles) __syncthreads();
        }
        if (PIECEWISE)
            for (int j = wt; j < ntiles; j++)
                if (!IMG || (j & 1) || j + 1 == ntiles) __syncthreads();

        // ---- epilogue: O / l * sigmoid(gate), this piece's {O, m, l} for the merge kernel, or the pair merge ----
        l_run += __shfl_xor(l_run, 32);
        const size_t t = (size_t)(t0 + tokw);
        if (MODE == FA_MODE_SPLIT && epi == FA_EPI_PIECE) {
            if (tokw < nt) {
                float* pr = fpart + ((t * H + head) * nsf + piece) * FP_ROW;
#pragma unroll
                for (int db = 0; db < 8; db++)
#pragma unroll
                    for (int a4 = 0; a4 < 4; a4++)
                        *reinterpret_cast<float4*>(pr + 32 * db + 8 * a4 + 4 * h32) =
                            make_float4(o[db][4 * a4], o[db][4 * a4 + 1], o[db][4 * a4 + 2], o[db][4 * a4 + 3]);
                if (h32 == 0) *reinterpret_cast<float2*>(pr + AHD) = make_float2(m_ref, l_run);
            }
            return;
        }
        if (MODE == FA_MODE_PAIR && epi == FA_EPI_PAIR) {
            // the two blocks of a pair hold keys [0, s) and [s, n) of this token tile for the same rows; the one that
            // finishes last merges, so neither waits for a block that may not have started
            if (!fa_pair_merge(fpart, pcnt, pslot + w, lane, o, m_ref, l_run)) return;
        }
        if (tokw < nt) fa_write_out(o, l_run, out, q_gate, t, head, H, ld, h32);
    };
    if (MODE == FA_MODE_PAIR) {  // one copy of the segment's code: a second inlined copy ran 1.5x slower per tile
#pragma nounroll
        for (int g = 0; g < nseg; g++) segment(sg[g]);
    } else {
        segment(sg[0]);
    }
#undef KBUF
#undef VBUF
#undef SBUF
}

// Merge of the key pieces of the token tiles that fa_prefill_kernel split: out = sum_s O_s 2^(m_s - M) /
// sum_s l_s 2^(m_s - M), times sigmoid(gate). Grid (ceil(T / 4), H): wavefront w merges token 4 blockIdx.x + w, lane
// l dims 4l .. 4l + 3 (lane s < pieces also holds piece s's m and l). Tiles with one piece were written by the FA
// kernel.
__global__ void __launch_bounds__(256) fa_merge_kernel(const float* __restrict__ fpart, const float* __restrict__ q_gate,
                                                       float* __restrict__ out, int H, int KV, const int* __restrict__ pos_d,
                                                       int ld, int T, int nsf, int ncu) {
    const int tok = 4 * blockIdx.x + (threadIdx.x >> 6), h = blockIdx.y, lane = threadIdx.x & 63, pos0 = *pos_d;
    if (tok >= T) return;
    const int nsp = fa_pieces(tok / FT, pos0, T, nsf, fa_piece_w(pos0, T, KV, (T + FT - 1) / FT, ncu));
    if (nsp <= 1) return;
    const float* pr = fpart + ((size_t)tok * H + h) * nsf * FP_ROW;
    const float2 ml = lane < nsp ? *reinterpret_cast<const float2*>(pr + lane * FP_ROW + AHD) : make_float2(-INFINITY, 0.f);
    float M = ml.x;  // finite: each piece holds keys of every row
#pragma unroll
    for (int x = 32; x >= 1; x >>= 1) M = fmaxf(M, __shfl_xor(M, x));
    const float f = lane < nsp ? fast_exp2(ml.x - M) : 0.f;
    float l = ml.y * f;
#pragma unroll
    for (int x = 32; x >= 1; x >>= 1) l += __shfl_xor(l, x);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
    for (int s = 0; s < nsp; s++) {
        const float fs = __shfl(f, s);
        const float4 q = *reinterpret_cast<const float4*>(pr + s * FP_ROW + 4 * lane);
        acc.x += q.x * fs; acc.y += q.y * fs; acc.z += q.z * fs; acc.w += q.w * fs;
    }
    const float il = 1.f / l;
    float4 res = make_float4(acc.x * il, acc.y * il, acc.z * il, acc.w * il);
    if (q_gate) {
        const float4 g = *reinterpret_cast<const float4*>(q_gate + (size_t)tok * ld + h * 2 * AHD + AHD + 4 * lane);
        res.x /= 1.f + __expf(-g.x); res.y /= 1.f + __expf(-g.y);
        res.z /= 1.f + __expf(-g.z); res.w /= 1.f + __expf(-g.w);
    }
    *reinterpret_cast<float4*>(out + ((size_t)tok * H + h) * AHD + 4 * lane) = res;
}

// Workspaces, one per (device, stream, kind), grown on demand. Calls on one stream are ordered, so they can share
// theirs. A buffer that is outgrown is never freed: a HIP graph captured earlier may still hold its address and
// replay into it, so it stays allocated until the process ends (growth goes to at least 1.5x, which bounds the
// retired bytes by twice the live ones). While the stream is being captured nothing is allocated: a workspace that
// would have to grow is reported as hipErrorStreamCaptureUnsupported and nullptr is returned (one eager call of the
// same shape on the stream before the capture avoids that).
namespace {
struct WsKey {
    int dev;
    hipStream_t st;
    int kind;  // 0: FA tile images, 1: FA partials of split token tiles, 2: fp16 GEMM activations,
               // 3: GEMM K-split partials, 4: decode-kernel partials of short FA chunks, 5: FA pair arrival
               // counters (zeroed when allocated)
    bool operator<(const WsKey& o) const {
        return dev != o.dev ? dev < o.dev : st != o.st ? st < o.st : kind < o.kind;
    }
};
std::mutex g_ws_mu;
std::map<WsKey, std::pair<unsigned char*, size_t>> g_ws;
size_t g_ws_retired = 0;  // bytes of outgrown buffers kept alive for captured graphs

}  // namespace

unsigned char* stream_workspace(size_t need, hipStream_t st, int kind, bool quiet) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    auto& w = g_ws[WsKey{dev, st, kind}];
    if (w.second >= need) return w.first;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
        if (!quiet) report(hipErrorStreamCaptureUnsupported, __FILE__, __LINE__);
        return nullptr;
    }
    const size_t want = std::max(need, w.second + w.second / 2);
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();  // out of memory: the caller takes a path without it, or reports the error
        return nullptr;
    }
    if (kind == 5 && hipMemsetAsync(p, 0, want, st) != hipSuccess) {  // counters start even (never during capture)
        (void)hipGetLastError();
        (void)hipFree(p);
        return nullptr;
    }
    if (w.first) g_ws_retired += w.second;  // kept, not freed (see above)
    w = {static_cast<unsigned char*>(p), want};
    return w.first;
}

size_t stream_workspace_bytes() {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    size_t b = g_ws_retired;
    for (auto& kv : g_ws) b += kv.second.second;
    return b;
}

namespace {
template <bool TB, bool IMG, int MODE>
void set_lds() {
    static bool once = [] {
        MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(fa_prefill_kernel<TB, IMG, MODE>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (IMG ? 4 : 2) * TILE_BYTES));
        return true;
    }();
    (void)once;
}

int fa_ncu() {
    // MOEX_FA_CUS=n plans the FA grids as for a chip of n CUs (read on every call; the grids stay correct for any n:
    // tests use it to reach layouts this chip's count does not, such as a pair grid with an odd number of tiles)
    if (const char* e = std::getenv("MOEX_FA_CUS")) return std::max(8, std::atoi(e));
    static const int ncu = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            return v;
        return 256;
    }();
    return ncu;
}

// What one attn_fa call of T tokens over a cache of max_t positions needs: the most key pieces per token tile
// (the device picks the actual count from pos0), the bytes of their partial rows, and the bytes of the tile images.
struct FaPlan {
    int NT, ntmax, nsf;
    bool pair;          // full grid: pairs of token tiles (fa_pair_segs), their halves merged in the kernel
    size_t part_bytes, img_bytes, cnt_bytes;
    int gns;            // > 0: a chunk this short runs on the split-K decode kernels with gns splits
    size_t gqa_bytes;   // their partials
};

// Chunks of at most this many tokens run on the decode kernels (int8: gqa_wsp_kernel per 4-token group; turbo:
// gqa_wst_kernel per token; then the combine) instead of the FA kernel, whose workgroups hold 16 tokens each and
// leave most of the chip idle on a short chunk. MOEX_FA_GQA_MAXT=n sets the int8 bound to n and the turbo bound to
// n / 4 (0: never); it is read on every call.
int fa_gqa_maxt(bool turbo) {
    int n = FA_GQA_MAXT;
    if (const char* e = std::getenv("MOEX_FA_GQA_MAXT")) n = std::max(0, std::atoi(e));
    return turbo ? n / 4 : n;
}

FaPlan fa_plan(int H, int KV, int max_t, int T, bool turbo) {
    const int ncu = fa_ncu();
    FaPlan p;
    p.NT = (T + FT - 1) / FT;
    p.ntmax = (max_t + BK - 1) / BK;
    const int NT = p.NT;
    // key pieces per token tile, at most (the device decides, from pos0): only when the token tiles leave the chip
    // underfilled. A full grid is not split: blocks queued behind a full chip were measured to start only after many
    // CUs had freed, so pieces of the heavy tiles gained little and the merge cost more. MOEX_FA_SPLIT=n caps the
    // pieces (1: no splitting).
    int nsf = KV * NT >= ncu ? 1 : std::min(FA_NSF_MAX, (2 * ncu + KV * NT - 1) / (KV * NT));
    if (const char* e = std::getenv("MOEX_FA_SPLIT")) nsf = std::max(1, std::min(nsf, std::atoi(e)));
    if (nsf > 1) {
        // pos0 <= max_t - T: if the heaviest token tile would not split at any of these positions, launch unsplit
        // (the split launch's extra blocks and merge cost a few microseconds even when nothing splits)
        const int pmax = std::max(0, max_t - T);
        bool any = false;
        for (int i = 0; i <= 32 && !any; i++) {
            const int p0 = (int)((long long)pmax * i / 32);
            any = fa_pieces(NT - 1, p0, T, nsf, fa_piece_w(p0, T, KV, NT, ncu)) > 1;
        }
        if (!any) nsf = 1;
    }
    p.nsf = nsf;
    p.part_bytes = nsf > 1 ? (size_t)T * H * nsf * FP_ROW * sizeof(float) : 0;
    // pairs: MOEX_FA_PAIR=0 turns them off (read on every call)
    const char* pe = std::getenv("MOEX_FA_PAIR");
    // (one wave of workgroups: with more, one tile per workgroup heaviest first already balances the waves and
    // measured faster, 4096 tokens at pos0 = 0: 158 against 178 us)
    p.pair = nsf == 1 && NT >= 2 && KV * NT <= ncu && !(pe && std::atoi(pe) == 0);
    p.cnt_bytes = 0;
    if (p.pair) {
        const size_t slots = (size_t)KV * (NT / 2) * 4;
        p.part_bytes = slots * FA_PAIR_SLOT * sizeof(float);
        p.cnt_bytes = slots * 2 * sizeof(unsigned);
    }
    // tile images for every chunk: measured faster than widening in the kernel at every chunk length and context
    // (a 3-token chunk over 90 000 keys: 159 against 388 us for turbo). MOEX_FA_IMAGES=0 turns them off (read on
    // every call), which saves the workspace and gives the same bits.
    const char* ie = std::getenv("MOEX_FA_IMAGES");
    p.img_bytes = !(ie && std::atoi(ie) == 0) ? (size_t)KV * p.ntmax * TILE_BYTES : 0;
    p.gns = 0;
    p.gqa_bytes = 0;
    if (T <= fa_gqa_maxt(turbo) && H == KV * GQ) {
        p.gns = gqa_splits(T, KV, moex_decode_splits(max_t), turbo);
        p.gqa_bytes = (size_t)T * H * p.gns * (AHD + 2) * sizeof(float);
    }
    return p;
}

// One attn_fa call on given buffers: img (tile images, or nullptr to widen in the kernel) and fpart (room for nsf
// pieces' partial rows when nsf > 1).
template <bool TB>
void launch_fa_bufs(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                    const int* pos_d, int max_t, int ld, int T, hipStream_t st, const FaPlan& p, unsigned char* img,
                    float* fpart, int nsf, unsigned* pcnt) {
    const int ncu = fa_ncu(), ntmax = p.ntmax;
    if (nsf > 1 && !fpart) nsf = 1;
    const bool pair = nsf == 1 && p.pair && fpart && pcnt;
    if (img) {
        // workgroups per kv head: every tile of the cache, at most 16 per CU over the kv heads (MOEX_FA_IMG_WG=n:
        // n per CU, read on every call)
        int wpc = 16;
        if (const char* e = std::getenv("MOEX_FA_IMG_WG")) wpc = std::max(1, std::atoi(e));
        const int gx = std::max(1, std::min(ntmax, wpc * ncu / KV));
        hipLaunchKernelGGL(fa_image_kernel<TB>, dim3(gx, KV), dim3(256), 0, st, kv, pos_d, T, max_t, ntmax, img);
        MOEX_LAUNCHED();
    }
    // a split launch has KV x tiles x nsf blocks: the pieces of every tile, the rest exit at once
    const int mode = nsf > 1 ? FA_MODE_SPLIT : pair ? FA_MODE_PAIR : FA_MODE_ONE;
    int pmin = FA_PAIR_MIN;  // MOEX_FA_PAIR_MIN=n: split a pair's heavy tile only when its second half has n tiles
    if (const char* e = std::getenv("MOEX_FA_PAIR_MIN")) pmin = std::max(1, std::min(255, std::atoi(e)));
    // the second block of a pair also loads its light tile's queries and writes its output: it takes FA_PAIR_EXTRA
    // fewer key tiles (MOEX_FA_PAIR_EXTRA=n overrides; measured on 2048-token chunks: at pos0 = 0 59.4 -> 58.2 us, at 32768 -0.4 %)
    int pextra = FA_PAIR_EXTRA;
    if (const char* e = std::getenv("MOEX_FA_PAIR_EXTRA")) pextra = std::max(0, std::min(255, std::atoi(e)));
    const int pk = pmin | (pextra << 8);
    const dim3 grid(mode == FA_MODE_SPLIT ? KV * p.NT * nsf : mode == FA_MODE_PAIR ? fa_pair_grid(KV, T) : fa_grid(KV, T));
    const size_t lds = (img ? 4 : 2) * TILE_BYTES;
#define FA_LAUNCH(IMG_, MODE_)                                                                                         \
    do {                                                                                                               \
        set_lds<TB, IMG_, MODE_>();                                                                                    \
        hipLaunchKernelGGL((fa_prefill_kernel<TB, IMG_, MODE_>), grid, dim3(512), lds, st, qo, q_gate, kv, img, ntmax,  \
                           out, H, KV, pos_d, max_t, ld, T, fpart, mode == FA_MODE_PAIR ? pk : nsf, ncu, pcnt);       \
    } while (0)
    if (img) {
        if (mode == FA_MODE_SPLIT) FA_LAUNCH(true, FA_MODE_SPLIT);
        else if (mode == FA_MODE_PAIR) FA_LAUNCH(true, FA_MODE_PAIR);
        else FA_LAUNCH(true, FA_MODE_ONE);
    } else {
        if (mode == FA_MODE_SPLIT) FA_LAUNCH(false, FA_MODE_SPLIT);
        else if (mode == FA_MODE_PAIR) FA_LAUNCH(false, FA_MODE_PAIR);
        else FA_LAUNCH(false, FA_MODE_ONE);
    }
#undef FA_LAUNCH
    MOEX_LAUNCHED();
    if (nsf > 1) {
        hipLaunchKernelGGL(fa_merge_kernel, dim3((T + 3) / 4, H), dim3(256), 0, st, fpart, q_gate, out, H, KV, pos_d, ld,
                           T, nsf, ncu);
        MOEX_LAUNCHED();
    }
}

template <bool TB>
void launch_fa_t(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV, const int* pos_d,
                 int max_t, int ld, int T, hipStream_t st) {
    const FaPlan p = fa_plan(H, KV, max_t, T, TB);
    if (p.gns > 0) {  // a short chunk: split-K decode kernels and the gated combine (turbo: in the rotated domain, as
                      // the FA kernel leaves it)
        float* part = reinterpret_cast<float*>(stream_workspace(p.gqa_bytes, st, 4));
        if (part) {
            launch_gqa(qo, kv, H, KV, pos_d, max_t, part, T, p.gns, st);
            launch_combine(part, q_gate, out, H, p.gns, ld, T, st);
            return;
        }
    }
    float* fpart = p.part_bytes ? reinterpret_cast<float*>(stream_workspace(p.part_bytes, st, 1)) : nullptr;
    unsigned* pcnt = p.cnt_bytes ? reinterpret_cast<unsigned*>(stream_workspace(p.cnt_bytes, st, 5)) : nullptr;
    unsigned char* img = p.img_bytes ? stream_workspace(p.img_bytes, st, 0) : nullptr;
    launch_fa_bufs<TB>(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T, st, p, img, fpart, fpart ? p.nsf : 1, pcnt);
}
}  // namespace

void launch_fa(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV, const int* pos_d,
               int max_t, int ld, int T, hipStream_t st) {
    if (kv.turbo) launch_fa_t<true>(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T, st);
    else launch_fa_t<false>(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T, st);
}

void launch_fa_scratch(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                       const int* pos_d, int max_t, int ld, int T, hipStream_t st, float* scratch, size_t bytes) {
    const FaPlan p = fa_plan(H, KV, max_t, T, kv.turbo != 0);
    if (p.gns > 0 && p.gqa_bytes <= bytes) {  // a short chunk, as in launch_fa_t
        launch_gqa(qo, kv, H, KV, pos_d, max_t, scratch, T, p.gns, st);
        launch_combine(scratch, q_gate, out, H, p.gns, ld, T, st);
        return;
    }
    // the pieces' partial rows must fit the scratch: fewer pieces when they do not (no tile images: the staging
    // wavefronts widen every tile, which gives the same bits)
    const size_t per = (size_t)T * H * FP_ROW * sizeof(float);
    int nsf = p.nsf;
    if (nsf > 1 && per * nsf > bytes) nsf = (int)std::min<size_t>(nsf, bytes / per);
    if (nsf < 2) nsf = 1;
    float* fpart = nsf > 1 ? scratch : nullptr;
    // full grids run one block per token tile here (pairs need arrival counters that persist across calls)
    if (kv.turbo) launch_fa_bufs<true>(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T, st, p, nullptr, fpart, nsf, nullptr);
    else launch_fa_bufs<false>(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T, st, p, nullptr, fpart, nsf, nullptr);
}

size_t fa_workspace_bytes(int H, int KV, int max_t, int T) {
    // the larger of the int8 and the turbo plan (the query does not name the cache format)
    size_t b = 0;
    for (bool tb : {false, true}) {
        const FaPlan p = fa_plan(H, KV, max_t, T, tb);
        b = std::max(b, p.gns > 0 ? p.gqa_bytes : p.part_bytes + p.img_bytes + p.cnt_bytes);
    }
    return b;
}

}  // namespace moex
