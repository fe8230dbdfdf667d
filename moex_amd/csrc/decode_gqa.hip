// Split-K GQA decode / MTP-verify attention on gfx950 (replaces attn_gqa_k, kernels.cuh:1740-1844).
//
// One workgroup = (kv head, key split, group of query tokens); the 8 query heads of the group share every K/V byte.
// int8 cache: gqa_ws1_kernel for a single query token (warp-specialised: producer wavefronts stream K/V into LDS,
// consumer wavefronts compute), gqa_wsp_kernel for MTP-verify windows (token pairs on the same pipeline).
// gqa_wst_kernel serves the TurboQuant cache, one token per workgroup, on eight symmetric wavefronts that each stream
// and decode their own keys. The partial written per (token, head, split) is {m (log2 units), l, acc[256]}.
#include "front.hpp"

namespace moex {

namespace {

constexpr float SL2 = 0.0625f * 1.4426950408889634f;  // 1/sqrt(256) * log2(e)
constexpr float TK4 = 0.241529f / 127.f, TK3 = 0.190207f / 127.f;

// ---- work-item mapping: blocks are dispatched round-robin over the 8 XCDs (block b -> XCD b % 8); renumber so
// that consecutive work items (the T tokens of a split, then neighbouring splits) land on the same XCD and share
// its L2.
__device__ __forceinline__ int xcd_work_id(int b, int nb) {
    const int q = nb >> 3, r = nb & 7, x = b & 7, i = b >> 3;
    return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + i;
}
}  // namespace

// ---------------------------------------------------------------------------------------------------------------
// Q.K runs on v_mfma_i32_16x16x64_i8 with the raw int8 K bytes (or the signed turbo K codes) as the A operand: the
// fp32 query enters as 24-bit fixed point in three signed base-256 digits (x = d2*2^16 + d1*2^8 + d0, each digit in
// [-128, 127]), every digit product accumulated exactly in int32 and the digits recombined in fp32, so the scores keep
// fp32-level precision (the reference decode is fp32). The int8 kernels give each digit its own MFMA per 64 dims with
// column m of the B operand one (token, head) of the query: the lane that receives the score of (key, column m)
// recombines it from its three accumulators. The turbo kernel packs digits 2 and 0 of the 8 heads into the 16 columns
// of one MFMA and digit 1 into a second, and brings a head's digits together with one row_ror:8 DPP move.
// P.V runs on v_mfma_f32_16x16x32_f16: P = p * vs * 2^sig is split into fp16 hi + lo (~22 bits), V widened exactly to
// fp16, fp32 accumulation.
typedef int int4_t_ __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int dpp_ror8(int x) { return __builtin_amdgcn_update_dpp(0, x, 0x128, 0xf, 0xf, false); }

// three signed base-256 digits of n, |n| <= 2^22 + 2^15: n = d2*65536 + d1*256 + d0
__device__ __forceinline__ void digits3(int n, int& d2, int& d1, int& d0) {
    d2 = (n + 32896) >> 16;
    const int r = n - (d2 << 16);
    d1 = (r + 128) >> 8;
    d0 = r - (d1 << 8);
}
__device__ __forceinline__ uint32_t pack_bytes(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) | ((uint32_t)d << 24);
}
__device__ __forceinline__ void tr4x4_(const uint32_t r0, const uint32_t r1, const uint32_t r2, const uint32_t r3, uint32_t c[4]) {
    const uint32_t t0 = __builtin_amdgcn_perm(r1, r0, 0x05010400u), t1 = __builtin_amdgcn_perm(r1, r0, 0x07030602u);
    const uint32_t t2 = __builtin_amdgcn_perm(r3, r2, 0x05010400u), t3 = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
    c[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u); c[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    c[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u); c[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// P.V takes V as biased bytes b = v + 128 (1 .. 255) read as the fp16 subnormal b * 2^-24: one v_perm per two codes
// builds the operand (MFMA takes fp16 subnormals exactly), and O = 2^24 o - 128 * sum(P) is restored once at the end.
constexpr int VBIAS = 128;
// fp16 operand of 8 keys of one dim from 8 key rows of biased codes: half k = byte j of r[k] as a subnormal
// (b * 2^-24; MFMA takes fp16 subnormals exactly)
__device__ __forceinline__ half8_t bsub8(const uint32_t r[8], int j) {
    const uint32_t sel = (uint32_t)j | 0x0c00u | ((uint32_t)(4 + j) << 16) | 0x0c000000u;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 u = {__builtin_amdgcn_perm(r[1], r[0], sel), __builtin_amdgcn_perm(r[3], r[2], sel),
               __builtin_amdgcn_perm(r[5], r[4], sel), __builtin_amdgcn_perm(r[7], r[6], sel)};
    return __builtin_bit_cast(half8_t, u);
}

// 2^(a - b) with 2^(-inf - -inf) = 1 (a running maximum that has not moved, also while it is still -inf)
__device__ __forceinline__ float ex2d(float a, float b) { return a == b ? 1.f : fast_exp2(a - b); }

// x combined with its partner lane l ^ 16 / l ^ 32 (v_permlane16/32_swap: both lanes of a pair receive both values)
__device__ __forceinline__ float max_x16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_x32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_x16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_x32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// x reduced over the 16 lanes of its DPP row (lanes 16r .. 16r + 15); every lane of the row receives the result
template <int CTRL> __device__ __forceinline__ float dppf(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float max_row16(float x) {
    x = fmaxf(x, dppf<0x128>(x));  // row_ror:8
    x = fmaxf(x, dppf<0x124>(x));  // row_ror:4
    x = fmaxf(x, dppf<0x4e>(x));   // quad_perm [2, 3, 0, 1]
    return fmaxf(x, dppf<0xb1>(x));  // quad_perm [1, 0, 3, 2]
}
__device__ __forceinline__ float sum_row16(float x) {
    x += dppf<0x128>(x);
    x += dppf<0x124>(x);
    x += dppf<0x4e>(x);
    return x + dppf<0xb1>(x);
}

// ---- The warp-specialised decode pipeline (gqa_ws1_kernel, gqa_wsp_kernel, gqa_wst_kernel). A vector-memory
// instruction waits at issue while the CU's request queue is full, which under the chip-wide K/V stream is most of
// the time; a wavefront that both loads and computes therefore cannot compute while its next chunk goes out. Here
// waves 4..7 only move rows (global_load_lds: K, V and the scales of a chunk into a ring of LDS stages) and waves
// 0..3 only compute, one per SIMD. Each consumer owns a fixed slice of the keys of every chunk and keeps its own
// running maximum, sum and O over all 256 dims, so the chunk loop needs no exchange between consumers: one barrier
// per chunk hands a landed stage to the consumers and a consumed one back to the producers. The four consumer states
// merge once at the end.
//   K stage: row r holds its 16-byte piece p in slot p ^ (r % 16), so the 16 lanes of a ds_read_b128 (16 rows, one
//            piece) hit 16 different slots.
//   V stage: row r holds its 16-byte piece p in slot p ^ 4 * ((r / 4) % 4), so the four lane groups of a pass-2 read
//            (keys 4g + i) hit disjoint banks.
//   O:       16 tiles; column n of tile 4 pc + j is dim 64 pc + 4 n + j, row 2h (2h + 1) is the hi (lo) part of
//            head h, so lane group g holds heads 2g and 2g + 1 whole. It is rescaled only when the reference maximum of a head moves by more
//            than WS_SLACK (log2 units; P then stays below 2^WS_SLACK) or the V scale exponent grows.
constexpr int WS_NC = 4;                              // consumer wavefronts (waves 0 .. WS_NC-1)
constexpr int WS_NP = 4;                              // producer wavefronts (the next WS_NP waves)
constexpr float WS_SLACK = 8.f;

// The producer side of gqa_ws1_kernel / gqa_wsp_kernel: chunks of CH keys (keys [clo(c), chi(c)), chunk 0 the short
// one) in a ring of NS LDS stages, NS - 1 chunks in flight. A stage holds the K rows, the V rows, then ks[CH] and
// vs[CH]. Producers 0, 1 move the K rows, 2, 3 the V rows (CH / 8 instructions of 4 rows each); with 128-key chunks
// each producer also moves 64 scales (ks for 0, 1, vs for 2, 3), with 64-key chunks producers 0 and 2 move all 64
// (4 bytes a lane). Rows past the chunk repeat its last row: their P is 0. Chunk c + NS - 1 is issued at the barrier
// that hands chunk c to the consumers (its stage held chunk c - 1, now consumed); the producers end each chunk with a
// bare s_barrier, as __syncthreads would also wait for the chunks still in flight. Takes part in the nch + 2
// barriers of the chunk loop and the consumer merge.
// LDS transfers of 16 (4) bytes per active lane, lane l to lds + 16 l (4 l), written in inline asm: the compiler cannot
// tell which LDS bytes a transfer writes and would make the wavefront's next LDS read wait for every transfer in
// flight; the kernel waits for its own transfers with vm_wait. dma16s: wave-uniform base + per-lane 32-bit offset.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved: every other use of it in this kernel sets it first
__device__ __forceinline__ void dma16(const void* g, const unsigned char* lds) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m) : "memory", "m0");
}
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, const unsigned char* lds) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, const unsigned char* lds) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(m) : "memory", "m0");
}
#pragma clang diagnostic pop
template <int N> __device__ __forceinline__ void vm_wait() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

template <int CH>
constexpr int ring_stage() { return 2 * CH * AHD + 2 * CH * 4; }

// chunk c of the ring into stage c % NS (the producers' transfers of it)
template <int CH, int NS>
__device__ __forceinline__ void ring_issue(unsigned char* smem, const moex_kv_cache& kv, size_t rbase, int pw, int lane,
                                           int lo, int first, int c) {
    static_assert((CH == 64 || CH == 128) && NS >= 2 && NS <= 4, "ring shape");
    constexpr int KB = CH * AHD, STAGE = ring_stage<CH>(), NI = CH / 8;
    constexpr bool SC_ALL = CH == 128;
    const bool sc = SC_ALL || !(pw & 1);
    const int8_t* src = (pw < 2 ? kv.k : kv.v) + rbase * AHD;
    const float* ssrc = (pw < 2 ? kv.ks : kv.vs) + rbase;
    const int r4 = lane >> 4, sl = lane & 15;
    const int c0 = c == 0 ? lo : lo + first + (c - 1) * CH, ce = c == 0 ? lo + first : lo + first + c * CH;
    unsigned char* st = smem + (c % NS) * STAGE;
    unsigned char* sb = st + (pw < 2 ? 0 : KB);
#pragma unroll
    for (int u = 0; u < NI; u++) {
        const int i = NI * (pw & 1) + u, r = 4 * i + r4;  // instruction i covers rows 4i .. 4i+3
        const int piece = pw < 2 ? sl ^ (r & 15) : sl ^ (4 * (i & 3));
        dma16(src + (size_t)min(c0 + r, ce - 1) * AHD + 16 * piece, sb + i * 1024);
    }
    if (sc) {
        const int k0 = SC_ALL ? 64 * (pw & 1) : 0;
        dma4(ssrc + min(c0 + k0 + lane, ce - 1), st + 2 * KB + (pw < 2 ? 0 : 4 * CH) + 4 * k0);
    }
}
// the first NS - 1 chunks
template <int CH, int NS>
__device__ __forceinline__ void ring_first(unsigned char* smem, const moex_kv_cache& kv, size_t rbase, int pw, int lane,
                                           int lo, int first, int nch) {
    for (int c = 0; c < NS - 1 && c < nch; c++) ring_issue<CH, NS>(smem, kv, rbase, pw, lane, lo, first, c);
}
// issued: the first chunks went out already (ring_first). ppos >= 0: the cache row at position ppos was just formed
// by this workgroup (patch: K row, V row, ks, vs in LDS) and may not have reached memory when its chunk was moved; the
// producer that moved each part of that row overwrites it in the stage once the chunk has landed.
template <int CH, int NS>
__device__ __forceinline__ void ring_producer(unsigned char* smem, const moex_kv_cache& kv, size_t rbase, int pw,
                                              int lane, int lo, int first, int nch, bool issued = false, int ppos = -1,
                                              const unsigned char* patch = nullptr) {
    constexpr int KB = CH * AHD, STAGE = ring_stage<CH>(), NI = CH / 8;
    constexpr bool SC_ALL = CH == 128;
    const bool sc = SC_ALL || !(pw & 1);
    if (!issued) ring_first<CH, NS>(smem, kv, rbase, pw, lane, lo, first, nch);
    for (int c = 0; c < nch; c++) {
        // chunk c has landed when at most the chunks issued after it are in flight (NI or NI + 1 instructions each)
        const int after = min(nch - 1 - c, NS - 2);
        if (after == 0) vm_wait<0>();
        else if (sc) { if (after == 1) vm_wait<NI + 1>(); else vm_wait<2 * (NI + 1)>(); }
        else { if (after == 1) vm_wait<NI>(); else vm_wait<2 * NI>(); }
        const int c0 = c == 0 ? lo : lo + first + (c - 1) * CH, ce = c == 0 ? lo + first : lo + first + c * CH;
        if (ppos >= c0 && ppos < ce) {
            const int r = ppos - c0;
            unsigned char* st = smem + (c % NS) * STAGE;
            if ((r >> 2) / NI == (pw & 1) && lane < 16) {  // this producer moved the row's K (V) bytes
                const int slot = pw < 2 ? lane ^ (r & 15) : lane ^ (4 * ((r >> 2) & 3));
                *reinterpret_cast<uint4*>(st + (pw < 2 ? 0 : KB) + r * AHD + 16 * slot) =
                    *reinterpret_cast<const uint4*>(patch + (pw < 2 ? 0 : AHD) + 16 * lane);
            }
            if (sc && lane == 0 && (SC_ALL ? r / 64 == (pw & 1) : true))
                *reinterpret_cast<float*>(st + 2 * KB + (pw < 2 ? 0 : 4 * CH) + 4 * r) =
                    reinterpret_cast<const float*>(patch + 2 * AHD)[pw < 2 ? 0 : 1];
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (c + NS - 1 < nch) ring_issue<CH, NS>(smem, kv, rbase, pw, lane, lo, first, c + NS - 1);
    }
    __syncthreads();
    __syncthreads();
}

// ---- gqa_ws1_kernel: one query token, chunks of 64 keys with three in flight. A pure DMA stream of the decode's size
// measured 5.35-5.46 TB/s with one 64 KB chunk in flight per CU and 5.7-5.8 TB/s with 96-128 KB in flight, and a
// smaller last chunk shortens the tail; so the chunk is 64 keys (33 KB) in a ring of four LDS stages, and consumer w
// owns keys 16w .. 16w + 15 of every chunk. The stage layouts, the Q.K fixed-point digits, the P hi / lo rows and the
// lazy rescale are those of the pipeline above; P.V runs on v_mfma_f32_16x16x16_f16, whose A operand is exactly the lane's
// 4 probabilities (keys 4g .. 4g + 3) and whose B operand is 4 keys of one dim (two v_perm of biased V bytes).
constexpr int W1_CH = 16 * WS_NC;                     // keys per chunk: 16 per consumer
constexpr int W1_NS = 4;                              // stages: three chunks in flight, one being computed
constexpr int W1_KB = W1_CH * AHD;                    // K rows of a stage; the V rows follow, then ks[64], vs[64]
constexpr int W1_STAGE = ring_stage<W1_CH>();
constexpr int W1_QT = W1_NS * W1_STAGE;              // query digit table: [digit 0, 1, 2][head][256] int8
constexpr int W1_QS = W1_QT + 3 * GQ * AHD;             // the heads' score scales
constexpr int W1_QO = W1_QS + GQ * 4;                   // the query rows formed in the prologue: [head][256] f32
constexpr int W1_PT = W1_QO + GQ * AHD * 4;              // the new cache row formed there: K, V codes, ks, vs
constexpr int W1_LDS = W1_PT + 2 * AHD + 16;
static_assert(WS_NC * GQ * AHD * 4 <= W1_LDS, "the consumer merge fits in the stages");
static_assert(W1_LDS <= 160 * 1024, "LDS");

// fr.q != nullptr: attn_decode's q/k front runs in the prologue (as qk_norm_rope_kernel would, bit for bit): the
// query rows of the group go to LDS (and to qo from split 0), and the split that holds position pos0 forms the new
// K/V row, writes it to the cache and patches it into its stage (its chunk may have been moved before the row
// reached memory). With the skip flag set it does neither and reads qo, as the attention kernels after a skipped
// front would.
// FR: launched with the front's arguments (a separate instance, so that the kernel without the front keeps its own
// code and registers)
template <bool FR>
__global__ void __launch_bounds__(64 * (WS_NC + WS_NP), 1) gqa_ws1_kernel(const float* __restrict__ qo, moex_kv_cache kv,
                                                                         int H, const int* __restrict__ pos_d,
                                                                         int max_t, float* __restrict__ part, int ns,
                                                                         FrontArgs fr) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float cm[WS_NC][GQ], cl[WS_NC][GQ];
    const int nb = gridDim.x, w_id = xcd_work_id(blockIdx.x, nb);
    const int s = w_id % ns, kvh = w_id / ns;
    const int pos0 = *pos_d, Tmax = pos0 + 1;
    const int L = (Tmax + ns - 1) / ns, lo = s * L;
    const int hi = min(Tmax, lo + L);  // keys [lo, hi) of this split
    const int nch = hi > lo ? (hi - lo + W1_CH - 1) / W1_CH : 0;
    const int first = hi > lo ? hi - lo - (nch - 1) * W1_CH : 0;  // chunk 0 is the short one
    auto clo = [&](int c) { return c == 0 ? lo : lo + first + (c - 1) * W1_CH; };
    auto chi = [&](int c) { return c == 0 ? lo + first : lo + first + c * W1_CH; };
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 4, m16 = lane & 15;
    const size_t rbase = (size_t)kvh * max_t;
    const bool fused = FR && fr.q && !(fr.skip && *fr.skip);
    // the producers' first chunks go out at once when the queries are read from qo. With the front in the prologue
    // the consumers form it, two query heads each (and wavefront 0 the new row), and the chunks go out once the
    // consumers have issued all of their row reads (a barrier between the two), so those reads are not queued behind
    // ~25 MB of chunk transfers while the front's arithmetic runs beside the chunks' flight
    if (wv >= WS_NC && !fused) ring_first<W1_CH, W1_NS>(smem, kv, rbase, wv - WS_NC, lane, lo, first, nch);
    const bool app = fused && hi == Tmax && hi > lo;  // this split holds the new row pos0
    const float* qtab = reinterpret_cast<const float*>(smem + W1_QO);
    unsigned char* patch = smem + W1_PT;
    if (fused) {
        float4 qa[2], ka, va;
        uint2 wq, wk;
        if (wv < WS_NC) {
#pragma unroll
            for (int j = 0; j < 2; j++)
                qa[j] = *reinterpret_cast<const float4*>(fr.q + (kvh * GQ + 2 * wv + j) * 2 * AHD + 4 * lane);
            wq = *reinterpret_cast<const uint2*>(fr.qn + 4 * lane);
            if (app && wv == 0) {
                ka = *reinterpret_cast<const float4*>(fr.k + kvh * AHD + 4 * lane);
                va = *reinterpret_cast<const float4*>(fr.v + kvh * AHD + 4 * lane);
                wk = *reinterpret_cast<const uint2*>(fr.kn + 4 * lane);
            }
        }
        asm volatile("s_barrier" ::: "memory");  // the consumers' row reads are issued
        if (wv >= WS_NC) {
            ring_first<W1_CH, W1_NS>(smem, kv, rbase, wv - WS_NC, lane, lo, first, nch);
        } else {
            // ---- the front (front::wave: the arithmetic of qk_norm_rope_kernel): consumer w forms query heads
            // 2w, 2w + 1; in the split that holds pos0, consumer 0 also forms the key row and the int8 codes of the
            // new row, which go to the cache and to the patch ----
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int h = 2 * wv + j;
                float x[4] = {qa[j].x, qa[j].y, qa[j].z, qa[j].w};
                front::wave::norm_rope(x, wq, lane, pos0, fr.rot, fr.theta, fr.eps);
                const float4 y = make_float4(x[0], x[1], x[2], x[3]);
                *reinterpret_cast<float4*>(smem + W1_QO + 4 * (h * AHD + 4 * lane)) = y;
                if (s == 0) *reinterpret_cast<float4*>(fr.qo + (kvh * GQ + h) * AHD + 4 * lane) = y;
            }
            if (app && wv == 0) {
                float x[4] = {ka.x, ka.y, ka.z, ka.w};
                const float vv[4] = {va.x, va.y, va.z, va.w};
                front::wave::norm_rope(x, wk, lane, pos0, fr.rot, fr.theta, fr.eps);
                uint32_t ck, cv;
                float sk, sv;
                front::wave::quant_i8(x, vv, ck, cv, sk, sv);
                const size_t row = rbase + pos0;
                *reinterpret_cast<uint32_t*>(kv.k + row * AHD + 4 * lane) = ck;
                *reinterpret_cast<uint32_t*>(kv.v + row * AHD + 4 * lane) = cv;
                reinterpret_cast<uint32_t*>(patch)[lane] = ck;
                reinterpret_cast<uint32_t*>(patch + AHD)[lane] = cv;
                if (lane == 0) {
                    kv.ks[row] = sk;
                    kv.vs[row] = sv;
                    reinterpret_cast<float*>(patch + 2 * AHD)[0] = sk;
                    reinterpret_cast<float*>(patch + 2 * AHD)[1] = sv;
                }
            }
        }
        front::sync<true>();
    }

    if (wv >= WS_NC) {
        ring_producer<W1_CH, W1_NS>(smem, kv, rbase, wv - WS_NC, lane, lo, first, nch, true, app ? pos0 : -1, patch);
    } else {
        // ---- consumers. The query digits, once per workgroup: consumer w turns heads 2w, 2w + 1 (lane l: head
        // 2w + l / 32, dims 8 (l % 32) .. + 7) into three signed base-256 digits of a 2^(22 - e) fixed point (|q| < 2^e
        // over the head) in the digit table; after the first barrier every consumer takes its operands from it ----
        {
            const int h = 2 * wv + (lane >> 5), d0 = 8 * (lane & 31);
            const float* qrow = fused ? qtab + h * AHD + d0 : qo + ((size_t)kvh * GQ + h) * AHD + d0;
            const float4 qa = *reinterpret_cast<const float4*>(qrow), qb = *reinterpret_cast<const float4*>(qrow + 4);
            float qm = fmaxf(fmaxf(fmaxf(fabsf(qa.x), fabsf(qa.y)), fmaxf(fabsf(qa.z), fabsf(qa.w))),
                             fmaxf(fmaxf(fabsf(qb.x), fabsf(qb.y)), fmaxf(fabsf(qb.z), fabsf(qb.w))));
            qm = max_x16(max_row16(qm));  // the 32 lanes of the head
            int e = 0;
            if (qm > 0.f) (void)frexpf(qm, &e);  // qm < 2^e
            const float up = ldexpf(1.f, 22 - e);
            const float xv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
            int d[3][8];
#pragma unroll
            for (int k = 0; k < 8; k++) digits3((int)__builtin_rintf(xv[k] * up), d[2][k], d[1][k], d[0][k]);
            unsigned char* qt = smem + W1_QT + h * AHD + d0;
#pragma unroll
            for (int dig = 0; dig < 3; dig++)
                *reinterpret_cast<uint2*>(qt + dig * GQ * AHD) =
                    make_uint2(pack_bytes(d[dig][0], d[dig][1], d[dig][2], d[dig][3]),
                               pack_bytes(d[dig][4], d[dig][5], d[dig][6], d[dig][7]));
            if ((lane & 31) == 0) reinterpret_cast<float*>(smem + W1_QS)[h] = ldexpf(1.f, e - 22) * SL2;
        }
        // column m16 of the Q.K MFMA is head m16 / 2 (every head twice); lane (g, m16) holds dims 64 ks + 16 g .. + 15
        int4_t_ qd[3][4];
        float qs = 0.f;
        float4_t o[16];
#pragma unroll
        for (int J = 0; J < 16; J++) o[J] = float4_t{0.f, 0.f, 0.f, 0.f};
        float mref = -INFINITY, lacc = 0.f, vmax = 0.f, xsum = 0.f;
        int sig = 0;
        const int kb = 16 * wv;  // this consumer's keys kb .. kb + 15 of every chunk
        for (int c = 0; c < nch; c++) {
            __syncthreads();  // chunk c is in stage c % 4 (and, at c = 0, the digit table is complete)
            if (c == 0) {
#pragma unroll
                for (int dig = 0; dig < 3; dig++)
#pragma unroll
                    for (int ks = 0; ks < 4; ks++)
                        qd[dig][ks] = *reinterpret_cast<const int4_t_*>(smem + W1_QT + (dig * GQ + (m16 >> 1)) * AHD +
                                                                        64 * ks + 16 * g);
                qs = reinterpret_cast<const float*>(smem + W1_QS)[m16 >> 1];
            }
            const int c0 = clo(c), ce = chi(c);
            if (c0 + kb >= ce) continue;
            const unsigned char* sb = smem + (c % W1_NS) * W1_STAGE;
            const float* sks = reinterpret_cast<const float*>(sb + 2 * W1_KB);
            const float* svs = sks + W1_CH;
            const float4 ksv = *reinterpret_cast<const float4*>(sks + kb + 4 * g);
            const float4 vv4 = *reinterpret_cast<const float4*>(svs + kb + 4 * g);
            float vv[4] = {vv4.x, vv4.y, vv4.z, vv4.w};
            // ---- scores of keys kb + 4 g + i for column m16: 12 MFMAs in 3 chains ----
            int4_t_ acc[3];
#pragma unroll
            for (int dig = 0; dig < 3; dig++) acc[dig] = int4_t_{0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const int4_t_ a = *reinterpret_cast<const int4_t_*>(sb + (kb + m16) * AHD + 16 * ((4 * ks + g) ^ m16));
#pragma unroll
                for (int dig = 0; dig < 3; dig++)
                    acc[dig] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qd[dig][ks], acc[dig], 0, 0, 0);
            }
            float sc[4];
            {
                const float kq[4] = {ksv.x, ksv.y, ksv.z, ksv.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float raw = ((float)acc[2][i] * 65536.f + (float)acc[1][i] * 256.f) + (float)acc[0][i];
                    sc[i] = raw * (kq[i] * qs);
                }
            }
            float vm;
            if (c0 + kb + 16 <= ce) {
                vm = fmaxf(fmaxf(vv[0], vv[1]), fmaxf(vv[2], vv[3]));
            } else {
                vm = 0.f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const bool ok = c0 + kb + 4 * g + i < ce;
                    sc[i] = ok ? sc[i] : -INFINITY;
                    vm = ok ? fmaxf(vm, vv[i]) : vm;
                }
            }
            float M = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            // the reductions over the lane groups only when some lane's own keys pass a bound (rare). A lane's own
            // maximum passes m_ref + slack exactly when its group's does, and V scales below 2^(7 - sig) cannot move
            // the exponent: the same decisions as with the reduced values, bit for bit
            if (__builtin_amdgcn_ballot_w64(M > mref + WS_SLACK || vm >= ldexpf(1.f, 7 - sig)) != 0) {
                M = max_x32(max_x16(M));
                vm = max_x32(max_x16(vm));
                const float nref = M > mref + WS_SLACK ? M : mref;
                const float fown = ex2d(mref, nref);
                vmax = fmaxf(vmax, vm);
                int ev = 0;
                if (vmax > 0.f) (void)frexpf(vmax, &ev);
                const int nsig = 7 - ev;
                if (__builtin_amdgcn_ballot_w64(fown != 1.f) != 0 || nsig != sig) {
                    const float sf = ldexpf(1.f, nsig - sig);
                    float fr[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) fr[i] = __shfl(fown, 2 * (2 * g + (i >> 1))) * sf;
#pragma unroll
                    for (int J = 0; J < 16; J++)
#pragma unroll
                        for (int i = 0; i < 4; i++) o[J][i] *= fr[i];
                    lacc *= fown;
                    xsum *= fown * sf;
                    mref = nref;
                    sig = nsig;
                }
            }
            // ---- P = 2^(s - mref) * vs * 2^sig: row m16 of the A operand (hi for even m16, lo for odd), keys 4g .. ----
            half4_t pa;
            {
                const float vsc = ldexpf(1.f, sig);
                float ls = 0.f, xs = 0.f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float p = fast_exp2(sc[i] - mref);
                    ls += p;
                    const float x = p * (vv[i] * vsc);
                    xs += x;
                    const _Float16 h = (_Float16)x;
                    pa[i] = (m16 & 1) ? (_Float16)(x - (float)h) : h;
                }
                lacc += ls;
                xsum += xs;
            }
            // ---- O^T += P . V: B operand = 4 keys of one dim, biased bytes as fp16 subnormals ----
            const unsigned char* Vs = sb + W1_KB;
#pragma unroll
            for (int pc = 0; pc < 4; pc++) {
                const int rd = 16 * ((4 * pc + (m16 >> 2)) ^ (4 * g)) + 4 * (m16 & 3);
                uint32_t r[4];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    r[j] = *reinterpret_cast<const uint32_t*>(Vs + (kb + 4 * g + j) * AHD + rd) ^ 0x80808080u;
#pragma unroll
                for (int jt = 0; jt < 4; jt++) {
                    const uint32_t sel = (uint32_t)jt | 0x0c00u | ((uint32_t)(4 + jt) << 16) | 0x0c000000u;
                    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                    const u32x2 u = {__builtin_amdgcn_perm(r[1], r[0], sel), __builtin_amdgcn_perm(r[3], r[2], sel)};
                    o[4 * pc + jt] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, u),
                                                                            o[4 * pc + jt], 0, 0, 0);
                }
            }
        }
        // ---- merge the four consumers: m, l per head, then O rows (hi + lo) scaled to the common maximum ----
        const float l = sum_x32(sum_x16(lacc));
        __syncthreads();  // every consumer is past its last chunk: the stages are free
        if (lane < 16 && !(lane & 1)) { cm[wv][lane >> 1] = mref; cl[wv][lane >> 1] = l; }
        __syncthreads();
        float* Ow = reinterpret_cast<float*>(smem);  // [consumer][head][256]
        const float un = ldexpf(1.f, -sig);
        const float xb = sum_x32(sum_x16(xsum)) * VBIAS;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int h = 2 * g + e;
            float Mh = cm[0][h];
#pragma unroll
            for (int w = 1; w < WS_NC; w++) Mh = fmaxf(Mh, cm[w][h]);
            const float f = ex2d(cm[wv][h], Mh) * un, b = __shfl(xb, 2 * h);
#pragma unroll
            for (int pc = 0; pc < 4; pc++) {
                float t[4];
#pragma unroll
                for (int jt = 0; jt < 4; jt++)
                    t[jt] = fmaf(o[4 * pc + jt][2 * e] + o[4 * pc + jt][2 * e + 1], 16777216.f, -b) * f;
                *reinterpret_cast<float4*>(Ow + (wv * GQ + h) * AHD + 64 * pc + 4 * m16) =
                    make_float4(t[0], t[1], t[2], t[3]);
            }
        }
    }
    __syncthreads();
    for (int it = tid; it < GQ * 64; it += 64 * (WS_NC + WS_NP)) {
        const float* Ow = reinterpret_cast<const float*>(smem);
        const int h = it >> 6, d4 = 4 * (it & 63);
        float4 a = *reinterpret_cast<const float4*>(Ow + h * AHD + d4);
#pragma unroll
        for (int w = 1; w < WS_NC; w++) {
            const float4 b = *reinterpret_cast<const float4*>(Ow + (w * GQ + h) * AHD + d4);
            a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
        }
        *reinterpret_cast<float4*>(part_acc(part, 0, kvh * GQ + h, s, H, ns) + d4) = a;
        if ((it & 63) == 0) {
            float Mh = cm[0][h], lh = 0.f;
#pragma unroll
            for (int w = 1; w < WS_NC; w++) Mh = fmaxf(Mh, cm[w][h]);
#pragma unroll
            for (int w = 0; w < WS_NC; w++) lh += cl[w][h] * ex2d(cm[w][h], Mh);
            float* ml = part_ml(part, 0, kvh * GQ + h, s, H, ns, 1);
            ml[0] = Mh;  // -inf when the split has no key
            ml[1] = lh;
        }
    }
}

// ---- gqa_wsp_kernel<NPR>: MTP-verify windows, NPR token pairs (up to 4 tokens) per workgroup, on the
// pipeline (same producers, stages and chunk order). Consumer w serves pair w % NPR and owns 32 NPR keys of every
// chunk (part w / NPR). Column m of the Q.K MFMA is (token m / 8 of the pair, head m % 8), so one set of MFMAs scores
// both tokens. P enters P.V as two A operands, its hi and lo fp16 parts (row = column), accumulated into the same O
// tiles against one widened V operand: V is widened once per pair, and O (rows = (token, head)) takes 64 registers.
// Chunks of 64 keys, three in flight, for two token pairs (each consumer then owns 32 keys of a chunk); chunks of 128
// keys, one in flight, for one pair (four consumers x 32 keys).
template <int NPR> constexpr int wsp_ch() { return NPR == 2 ? 64 : 128; }
template <int NPR> constexpr int wsp_ns() { return NPR == 2 ? 4 : 2; }
template <int NPR> constexpr int wsp_lds() { return wsp_ns<NPR>() * ring_stage<wsp_ch<NPR>()>(); }
static_assert(WS_NC * 16 * AHD * 4 <= wsp_lds<1>() && WS_NC * 16 * AHD * 4 <= wsp_lds<2>(), "the pair merge fits");
static_assert(wsp_lds<1>() <= 160 * 1024 && wsp_lds<2>() <= 160 * 1024, "LDS");

// FR (one token group, T <= 2 NPR, fr.q set, skip flag clear): attn_decode's q/k front runs in the prologue, as
// front_rows_kernel would, bit for bit. The consumers issue the reads of the group's 8 T query rows (a token's rows
// on one or two consumers, which share its RoPE angles) and of the split's new cache rows, a barrier lets the
// producers send the first chunks, and the consumers form the rows while those fly: the query rows into the last ring
// stage (its first chunk is issued only at the first chunk barrier, after the query digits are taken from it) and to
// qo from split 0, the
// new rows to the cache. The new rows sit at the split's end, so a chunk that holds them is moved after the first
// chunk barrier, which follows the stores; only a split whose new rows fall in its first NS - 1 chunks holds its
// first chunks back until the rows are stored.
template <int NPR, bool FR>
__global__ void __launch_bounds__(64 * (WS_NC + WS_NP), 1) gqa_wsp_kernel(const float* __restrict__ qo, moex_kv_cache kv,
                                                                         int H, const int* __restrict__ pos_d,
                                                                         int max_t, float* __restrict__ part, int T,
                                                                         int ns, FrontArgs fr) {
    constexpr int CH = wsp_ch<NPR>(), NS = wsp_ns<NPR>(), KB = CH * AHD, STAGE = ring_stage<CH>();
    constexpr int TT = 2 * NPR, KPC = CH * NPR / WS_NC;  // tokens per workgroup, keys per consumer per chunk
    static_assert(KPC == 32, "one 32-key block per consumer and chunk");
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float cm[WS_NC][16], cl[WS_NC][16];
    const int nb = gridDim.x, w_id = xcd_work_id(blockIdx.x, nb);
    const int ngr = (T + TT - 1) / TT;
    const int tg = w_id % ngr, s = (w_id / ngr) % ns, kvh = w_id / (ngr * ns);
    const int tb = tg * TT, ntok = min(TT, T - tb);
    const int pos0 = *pos_d, Tmax = pos0 + T;
    const int L = (Tmax + ns - 1) / ns, lo = s * L;
    const int hi = min(pos0 + tb + ntok, lo + L);  // keys [lo, hi) of this split that the group's last token sees
    const int nch = hi > lo ? (hi - lo + CH - 1) / CH : 0;
    const int first = hi > lo ? hi - lo - (nch - 1) * CH : 0;  // chunk 0 is the short one
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 4, m16 = lane & 15;
    const size_t rbase = (size_t)kvh * max_t;

    const bool fused = FR && ngr == 1 && fr.q && !(fr.skip && *fr.skip);
    const float* qtab = reinterpret_cast<const float*>(smem + (NS - 1) * STAGE);  // [token][head][256] when fused
    if (fused) {
        // this split's new cache rows: positions [nlo, hi)
        const int nlo = max(lo, pos0), nk = max(0, hi - nlo);
        const int cnew = nlo < lo + first ? 0 : 1 + (nlo - lo - first) / CH;  // the chunk of the first new row
        const bool late = nk > 0 && cnew < NS - 1;  // ... among the first chunks: they wait for the stores
        // consumer w takes token t = w / P, heads (w % P) 8 / P .. (P = 2 consumers a token for T <= 2, else 1), and
        // the token's new cache row when it is this split's (w % P == 0): one set of RoPE angles for all its rows
        constexpr int P = TT == 2 ? 2 : 1, HP = GQ / P;
        const int t = wv / P, h0 = (wv % P) * HP;
        const bool qrows = wv < WS_NC && t < T;
        const bool krow = qrows && wv % P == 0 && pos0 + t >= nlo && pos0 + t < hi;
        float4 qa[HP], ka, va;
        uint2 wq, wk;
        if (qrows) {
#pragma unroll
            for (int j = 0; j < HP; j++)
                qa[j] = *reinterpret_cast<const float4*>(fr.q + (size_t)t * fr.ld + (kvh * GQ + h0 + j) * 2 * AHD + 4 * lane);
            wq = *reinterpret_cast<const uint2*>(fr.qn + 4 * lane);
            if (krow) {
                const size_t o = (size_t)t * fr.ld + kvh * AHD + 4 * lane;
                ka = *reinterpret_cast<const float4*>(fr.k + o);
                va = *reinterpret_cast<const float4*>(fr.v + o);
                wk = *reinterpret_cast<const uint2*>(fr.kn + 4 * lane);
            }
        }
        asm volatile("s_barrier" ::: "memory");  // the consumers' row reads are issued
        if (wv >= WS_NC) {
            if (!late) ring_first<CH, NS>(smem, kv, rbase, wv - WS_NC, lane, lo, first, nch);
        } else {
            float* qt = reinterpret_cast<float*>(smem + (NS - 1) * STAGE);
            if (qrows) {
                const front::wave::Rope rp = front::wave::rope_angles(lane, pos0 + t, fr.rot, fr.theta);
#pragma unroll
                for (int j = 0; j < HP; j++) {
                    const int h = h0 + j;
                    float x[4] = {qa[j].x, qa[j].y, qa[j].z, qa[j].w};
                    front::wave::norm_rope(x, wq, lane, rp, fr.rot, fr.eps);
                    const float4 y = make_float4(x[0], x[1], x[2], x[3]);
                    *reinterpret_cast<float4*>(qt + (t * GQ + h) * AHD + 4 * lane) = y;
                    if (s == 0) *reinterpret_cast<float4*>(fr.qo + ((size_t)t * H + kvh * GQ + h) * AHD + 4 * lane) = y;
                }
                if (krow) {
                    float x[4] = {ka.x, ka.y, ka.z, ka.w};
                    const float vv[4] = {va.x, va.y, va.z, va.w};
                    front::wave::norm_rope(x, wk, lane, rp, fr.rot, fr.eps);
                    front::wave::append(x, vv, kv, rbase + pos0 + t, lane);
                }
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the new rows are in memory
        }
        front::sync<true>();
        if (wv >= WS_NC && late) ring_first<CH, NS>(smem, kv, rbase, wv - WS_NC, lane, lo, first, nch);
    }
    if (wv >= WS_NC) {
        ring_producer<CH, NS>(smem, kv, rbase, wv - WS_NC, lane, lo, first, nch, fused);
    } else {
        const int pr = wv % NPR;                                        // token pair
        const bool live = 2 * pr < ntok;
        const int tl = 2 * pr + (m16 >> 3);                             // this lane's token (column m16)
        const int htl = min(pos0 + tb + tl + 1, lo + L);                // ... sees keys below htl
        const int hlo = min(pos0 + tb + 2 * pr + 1, lo + L);            // keys below hlo: both tokens of the pair
        const int hhi = min(pos0 + tb + min(2 * pr + 2, ntok), lo + L);  // keys below hhi: some live token of it
        // ---- query digits: lane (g, m16) holds dims 64 ks + 16 g .. +15 of (token tl, head m16 % 8) ----
        int4_t_ qd[3][4];
        float qs;
        {
            const float* qrow = fused ? qtab + (min(tl, ntok - 1) * GQ + (m16 & 7)) * AHD + 16 * g
                                      : qo + ((size_t)(tb + min(tl, ntok - 1)) * H + kvh * GQ + (m16 & 7)) * AHD + 16 * g;
            float4 qv4[16];
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
#pragma unroll
                for (int u = 0; u < 4; u++) qv4[4 * ks + u] = *reinterpret_cast<const float4*>(qrow + 64 * ks + 4 * u);
            float qm = 0.f;
#pragma unroll
            for (int u = 0; u < 16; u++)
                qm = fmaxf(fmaxf(qm, fmaxf(fabsf(qv4[u].x), fabsf(qv4[u].y))), fmaxf(fabsf(qv4[u].z), fabsf(qv4[u].w)));
            qm = max_x32(max_x16(qm));
            int e = 0;
            if (qm > 0.f) (void)frexpf(qm, &e);  // qm < 2^e
            const float up = ldexpf(1.f, 22 - e);
            qs = ldexpf(1.f, e - 22) * SL2;
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float4 x = qv4[4 * ks + u];
                    int d[3][4];
                    digits3((int)__builtin_rintf(x.x * up), d[2][0], d[1][0], d[0][0]);
                    digits3((int)__builtin_rintf(x.y * up), d[2][1], d[1][1], d[0][1]);
                    digits3((int)__builtin_rintf(x.z * up), d[2][2], d[1][2], d[0][2]);
                    digits3((int)__builtin_rintf(x.w * up), d[2][3], d[1][3], d[0][3]);
#pragma unroll
                    for (int dig = 0; dig < 3; dig++)
                        qd[dig][ks][u] = (int)pack_bytes(d[dig][0], d[dig][1], d[dig][2], d[dig][3]);
                }
        }
        float4_t o[16];  // column n of tile 4 pc + j is dim 64 pc + 4 n + j; row r is column r of the Q.K MFMA
#pragma unroll
        for (int J = 0; J < 16; J++) o[J] = float4_t{0.f, 0.f, 0.f, 0.f};
        float mref = -INFINITY, lacc = 0.f, vmax = 0.f;  // reference maximum and sum of column m16, V-scale maximum
        float xsum = 0.f;                                 // sum of P * vs * 2^sig of this lane's keys: the V bias
        int sig = 0;                                      // O is held times 2^sig
        for (int c = 0; c < nch; c++) {
            __syncthreads();  // chunk c is in stage c % NS
            if (!live) continue;
            const int c0 = c == 0 ? lo : lo + first + (c - 1) * CH, ce = c == 0 ? lo + first : lo + first + c * CH;
            const int cmax = min(ce, hhi), cmin = min(ce, hlo), ctl = min(ce, htl);
            const unsigned char* sb = smem + (c % NS) * STAGE;
            const float* sks = reinterpret_cast<const float*>(sb + 2 * KB);
            const float* svs = sks + CH;
            const unsigned char* Vs = sb + KB;
#pragma unroll 1
            for (int kb = (wv / NPR) * KPC; kb < (wv / NPR + 1) * KPC; kb += 32) {  // keys kb .. kb+31 of the chunk
                if (c0 + kb >= cmax) break;
                float ksv[8], vv[8];
                {
                    const float4 a0 = *reinterpret_cast<const float4*>(sks + kb + 4 * g);
                    const float4 a1 = *reinterpret_cast<const float4*>(sks + kb + 16 + 4 * g);
                    const float4 b0 = *reinterpret_cast<const float4*>(svs + kb + 4 * g);
                    const float4 b1 = *reinterpret_cast<const float4*>(svs + kb + 16 + 4 * g);
                    ksv[0] = a0.x; ksv[1] = a0.y; ksv[2] = a0.z; ksv[3] = a0.w;
                    ksv[4] = a1.x; ksv[5] = a1.y; ksv[6] = a1.z; ksv[7] = a1.w;
                    vv[0] = b0.x; vv[1] = b0.y; vv[2] = b0.z; vv[3] = b0.w;
                    vv[4] = b1.x; vv[5] = b1.y; vv[6] = b1.z; vv[7] = b1.w;
                }
                int4_t_ acc[2][3];
#pragma unroll
                for (int grp = 0; grp < 2; grp++)
#pragma unroll
                    for (int dig = 0; dig < 3; dig++) acc[grp][dig] = int4_t_{0, 0, 0, 0};
#pragma unroll
                for (int ks = 0; ks < 4; ks++)
#pragma unroll
                    for (int grp = 0; grp < 2; grp++) {
                        const int4_t_ a =
                            *reinterpret_cast<const int4_t_*>(sb + (kb + 16 * grp + m16) * AHD + 16 * ((4 * ks + g) ^ m16));
#pragma unroll
                        for (int dig = 0; dig < 3; dig++)
                            acc[grp][dig] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qd[dig][ks], acc[grp][dig], 0, 0, 0);
                    }
                float sc[8];
#pragma unroll
                for (int grp = 0; grp < 2; grp++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float raw =
                            ((float)acc[grp][2][i] * 65536.f + (float)acc[grp][1][i] * 256.f) + (float)acc[grp][0][i];
                        sc[4 * grp + i] = raw * (ksv[4 * grp + i] * qs);
                    }
                float vm;
                if (c0 + kb + 32 <= cmin) {  // all 32 keys valid for both tokens
                    vm = fmaxf(fmaxf(fmaxf(vv[0], vv[1]), fmaxf(vv[2], vv[3])), fmaxf(fmaxf(vv[4], vv[5]), fmaxf(vv[6], vv[7])));
                } else {
                    vm = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const int key = c0 + kb + 16 * (j >> 2) + 4 * g + (j & 3);
                        sc[j] = key < ctl ? sc[j] : -INFINITY;
                        vm = key < cmax ? fmaxf(vm, vv[j]) : vm;
                    }
                }
                float M = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
                // the reductions over the lane groups only when some lane's own keys pass a bound (rare). A lane's
                // own maximum passes m_ref + slack exactly when its group's does, and V scales below 2^(7 - sig)
                // cannot move the exponent: the same decisions as with the reduced values, bit for bit
                if (__builtin_amdgcn_ballot_w64(M > mref + WS_SLACK || vm >= ldexpf(1.f, 7 - sig)) != 0) {
                    M = max_x32(max_x16(M));
                    vm = max_x32(max_x16(vm));
                    // ---- lazy rescale: new reference maximum of a column / V-scale exponent ----
                    const float nref = M > mref + WS_SLACK ? M : mref;
                    const float fown = ex2d(mref, nref);
                    vmax = fmaxf(vmax, vm);
                    int ev = 0;
                    if (vmax > 0.f) (void)frexpf(vmax, &ev);  // vmax < 2^ev: p * vs * 2^(7 - ev) < 2^(7 + WS_SLACK)
                    const int nsig = 7 - ev;
                    if (__builtin_amdgcn_ballot_w64(fown != 1.f) != 0 || nsig != sig) {
                        const float sf = ldexpf(1.f, nsig - sig);
                        float fr[4];
#pragma unroll
                        for (int i = 0; i < 4; i++) fr[i] = __shfl(fown, 4 * g + i) * sf;  // O row 4g + i = column 4g + i
#pragma unroll
                        for (int J = 0; J < 16; J++)
#pragma unroll
                            for (int i = 0; i < 4; i++) o[J][i] *= fr[i];
                        lacc *= fown;
                        xsum *= fown * sf;
                        mref = nref;
                        sig = nsig;
                    }
                }
                // ---- P = 2^(s - mref) * vs * 2^sig = hi + lo in fp16 (a column with no key yet has P = 0); each lane's
                // 8 keys are its own A operand ----
                half8_t pah, pal;
                {
                    const float vsc = ldexpf(1.f, sig), mr = mref == -INFINITY ? 0.f : mref;
                    half8_t ph, pl;
                    float ls = 0.f, xs = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const float p = fast_exp2(sc[j] - mr);
                        ls += p;
                        const float x = p * (vv[j] * vsc);
                        xs += x;
                        const _Float16 h = (_Float16)x;
                        ph[j] = h;
                        pl[j] = (_Float16)(x - (float)h);
                    }
                    lacc += ls;
                    xsum += xs;
                    pah = ph;
                    pal = pl;
                }
                // ---- O^T += (P_hi + P_lo) . V over these 32 keys, all 256 dims ----
#pragma unroll
                for (int pc = 0; pc < 4; pc++) {
                    const int rd = 16 * ((4 * pc + (m16 >> 2)) ^ (4 * g)) + 4 * (m16 & 3);
                    uint32_t r[8];
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        r[j] = *reinterpret_cast<const uint32_t*>(Vs + (kb + 16 * (j >> 2) + 4 * g + (j & 3)) * AHD + rd);
#pragma unroll
                    for (int j = 0; j < 8; j++) r[j] ^= 0x80808080u;  // biased codes
#pragma unroll
                    for (int jt = 0; jt < 4; jt++) {
                        const half8_t vb = bsub8(r, jt);
                        o[4 * pc + jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pah, vb, o[4 * pc + jt], 0, 0, 0);
                        o[4 * pc + jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pal, vb, o[4 * pc + jt], 0, 0, 0);
                    }
                }
            }
        }
        // ---- merge the consumers of each pair: m, l per column, then O rows scaled to the common maximum ----
        const float l = sum_x32(sum_x16(lacc));
        __syncthreads();  // every consumer is past its last chunk: stage 0 is free
        if (lane < 16) { cm[wv][lane] = mref; cl[wv][lane] = l; }
        __syncthreads();
        float* Ow = reinterpret_cast<float*>(smem);  // [consumer][column][256]
        const float un = ldexpf(1.f, -sig);
        // the V operands were (v + 128) * 2^-24: O = 2^24 o - 128 * sum(P * vs * 2^sig) per column
        const float xb = sum_x32(sum_x16(xsum)) * VBIAS;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int col = 4 * g + i;
            float Mc = cm[pr][col];
#pragma unroll
            for (int w = pr + NPR; w < WS_NC; w += NPR) Mc = fmaxf(Mc, cm[w][col]);
            const float f = ex2d(cm[wv][col], Mc) * un, b = __shfl(xb, col);
#pragma unroll
            for (int pc = 0; pc < 4; pc++)
                *reinterpret_cast<float4*>(Ow + (wv * 16 + col) * AHD + 64 * pc + 4 * m16) =
                    make_float4(fmaf(o[4 * pc][i], 16777216.f, -b) * f, fmaf(o[4 * pc + 1][i], 16777216.f, -b) * f,
                                fmaf(o[4 * pc + 2][i], 16777216.f, -b) * f, fmaf(o[4 * pc + 3][i], 16777216.f, -b) * f);
        }
    }
    __syncthreads();
    // ---- partials of the split: item = (token, head, dims 4 (item % 64) .. +3) ----
    for (int it = tid; it < ntok * GQ * 64; it += 64 * (WS_NC + WS_NP)) {
        const float* Ow = reinterpret_cast<const float*>(smem);
        const int t = it / (GQ * 64), h = (it >> 6) % GQ, d4 = 4 * (it & 63);
        const int pr = t >> 1, col = 8 * (t & 1) + h;
        float4 a = *reinterpret_cast<const float4*>(Ow + (pr * 16 + col) * AHD + d4);
#pragma unroll
        for (int w = pr + NPR; w < WS_NC; w += NPR) {
            const float4 b = *reinterpret_cast<const float4*>(Ow + (w * 16 + col) * AHD + d4);
            a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
        }
        *reinterpret_cast<float4*>(part_acc(part, tb + t, kvh * GQ + h, s, H, ns) + d4) = a;
        if ((it & 63) == 0) {
            float Mc = cm[pr][col], lc = 0.f;
#pragma unroll
            for (int w = pr + NPR; w < WS_NC; w += NPR) Mc = fmaxf(Mc, cm[w][col]);
#pragma unroll
            for (int w = pr; w < WS_NC; w += NPR) lc += cl[w][col] * ex2d(cm[w][col], Mc);
            float* ml = part_ml(part, tb + t, kvh * GQ + h, s, H, ns, T);
            ml[0] = Mc;  // -inf when the token has no key in this split
            ml[1] = lc;
        }
    }
}

template <int NPR>
static void launch_wsp(const float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, float* part,
                       int T, int ns, hipStream_t st, const FrontArgs* fr) {
    static bool once = [] {
        MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(gqa_wsp_kernel<NPR, false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, wsp_lds<NPR>()));
        MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(gqa_wsp_kernel<NPR, true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, wsp_lds<NPR>()));
        return true;
    }();
    (void)once;
    const dim3 grid(KV * ns * ((T + 2 * NPR - 1) / (2 * NPR))), block(64 * (WS_NC + WS_NP));
    if (fr && fr->q && T <= 2 * NPR)
        hipLaunchKernelGGL((gqa_wsp_kernel<NPR, true>), grid, block, wsp_lds<NPR>(), st, qo, kv, H, pos_d, max_t, part, T,
                           ns, *fr);
    else
        hipLaunchKernelGGL((gqa_wsp_kernel<NPR, false>), grid, block, wsp_lds<NPR>(), st, qo, kv, H, pos_d, max_t, part,
                           T, ns, FrontArgs{});
}

// TurboQuant codes -> signed int8 centroid codes (kernels.cuh:1122-1170 tables, scaled by 127 / max centroid):
//   K: 4-bit codes -> two v_perm LUT halves, a third v_perm picks per byte; the MFMA operand takes a lane's 16 codes
//      as (even nibbles, odd nibbles) of two dwords, and the query digits use the same dim order.
//   V: 3-bit codes, the low 2 bits and the high bit in separate planes of the row. For 16 codes (one 32-bit word of
//      low fields, 16 high bits): the four masks (w >> 2f) & 0x03030303 transposed as a 4 x 4 byte matrix put the
//      low field of code 4k + i in byte i of selector k; the high bits of codes 4k .. 4k + 3 go to bit 2 of those
//      bytes by one multiply (nibble * 0x810204: bit i lands at 8i + 2, the terms never overlap, so the product is
//      their OR); a v_perm LUT then maps each selector to 4 codes.
constexpr uint32_t spack(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) | ((uint32_t)(d & 0xff) << 24);
}
constexpr uint32_t SK0 = spack(-127, -96, -75, -58), SK1 = spack(-44, -31, -18, -6);
constexpr uint32_t SK2 = spack(6, 18, 31, 44), SK3 = spack(58, 75, 96, 127);
// V codes biased by 128 (1 .. 255), read by the consumers as fp16 subnormals (bsub8)
constexpr uint32_t SV0 = spack(1, 49, 83, 114), SV1 = spack(142, 173, 207, 255);
// 8 nibbles of x -> the 4 signed K codes of its even nibbles (ev) and of its odd nibbles (od). The low 3 bits of a
// nibble index a half-table (bytes 0-7 of the two v_perm sources); bit 3 moves the final pick to the upper half,
// selector byte b + 4. 13 VALU per 8 codes.
__device__ __forceinline__ void k_codes8(uint32_t x, int& ev, int& od) {
    const uint32_t t = x >> 4;
    const uint32_t se = x & 0x07070707u, so = t & 0x07070707u;
    uint32_t pe, po;  // (y & 0x04040404) | 0x03020100 in one v_and_or_b32 (the constants held in registers)
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(pe) : "v"(x >> 1), "v"(0x04040404u), "v"(0x03020100u));
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(po) : "v"(t >> 1), "v"(0x04040404u), "v"(0x03020100u));
    const uint32_t le = __builtin_amdgcn_perm(SK1, SK0, se), he = __builtin_amdgcn_perm(SK3, SK2, se);
    const uint32_t lo = __builtin_amdgcn_perm(SK1, SK0, so), ho = __builtin_amdgcn_perm(SK3, SK2, so);
    ev = (int)__builtin_amdgcn_perm(he, le, pe);
    od = (int)__builtin_amdgcn_perm(ho, lo, po);
}
__device__ __forceinline__ int4_t_ k_codes(uint2 x) {  // 16 nibbles -> the MFMA operand (even, odd, even, odd)
    int a, b, c, d;
    k_codes8(x.x, a, b);
    k_codes8(x.y, c, d);
    return int4_t_{a, b, c, d};
}

// ---- gqa_wst_kernel: TurboQuant cache, one query token per workgroup. Eight symmetric wavefronts with no roles:
// chunk c of the split (128 keys, chunk 0 the short one) gives keys 16w .. 16w + 15 to wavefront w, which streams
// them through a private ring of four LDS stages by its own DMA (K nibble rows, both half-norm pairs, raw V rows),
// decodes its own codes and keeps its own online softmax state; the eight states merge once, at the end. No barrier
// runs inside the key loop, the transfers are spread over all wavefronts, and the two wavefronts of a SIMD cover each
// other's stalls.
//   Q.K as S^T = Qd . K^T on v_mfma_i32_16x16x64_i8: the A operand holds query digits, row r = digit r % 4 (2, 1, 0,
//     then a zero row) of head r / 4 in the first MFMA and of head r / 4 + 4 in the second; the B operand holds the K
//     codes, column = key. Lane (g, m) then receives all three digits of heads g and g + 4 against key m and forms
//     both scores itself: every score is formed once.
//   P = 2^(s - m_ref) * vn * K3 * 2^sig per V half (the V half norm rides in P), split into fp16 hi + lo parts, goes
//     through a 1 KB LDS tile per wavefront into the P.V operand layout: row m = hi part of head m (m < 8) or lo part
//     of head m - 8, keys 4g .. 4g + 3 in lane (g, m).
//   V: P.V on v_mfma_f32_16x16x16_f16, one MFMA per V half h and slot b (0..7); column n is dim 128 h + 8 n + b, so
//     lane (g, n) decodes dims 8n .. 8n + 7 of both halves of keys 4g .. 4g + 3 straight from the raw rows (per key two
//     16-bit words of low fields and two bytes of high bits): one v_perm LUT per 4 codes gives the codes biased by
//     128, one v_perm per 2 codes the fp16-subnormal operand (as in the int8 kernels; the bias comes out at the end).
constexpr int WT_NW = 8;                         // wavefronts
constexpr int WT_K = 16;                         // keys per wavefront and chunk
constexpr int WT_CH = WT_K * WT_NW;              // keys per chunk
constexpr int WT_NS = 4;                         // stages per wavefront
constexpr int WT_NRM = WT_K * TQ_KB;             // stage: K nibble rows at 0, then the norms (K pairs, V pairs)
constexpr int WT_RV = WT_NRM + 2 * WT_K * 8;     // then the raw V rows, at a 112-byte stride: the four rows that a
constexpr int WT_VS = 112;                       // read spans (keys 4g + i, g = 0..3) start on distinct banks
constexpr int WT_STAGE = WT_RV + WT_K * WT_VS;   // 4096 B
constexpr int WT_PT = 2 * 16 * WT_K * 2;         // P tiles of a wavefront: two V halves of [16 rows][16 keys] fp16
constexpr int WT_P0 = WT_NW * WT_NS * WT_STAGE;
constexpr int WT_QT = WT_P0 + WT_NW * WT_PT;     // query digit table: [digit 2, 1, 0, zero][head][256] int8
constexpr int WT_QS = WT_QT + 4 * GQ * AHD;      // the heads' score scales
constexpr int WT_LDS = WT_QS + GQ * 4;
static_assert((WT_NW + 1) * GQ * AHD * 4 <= WT_P0, "the merge and the merged rows fit in the stages");
static_assert(WT_LDS <= 160 * 1024, "LDS");
static_assert(WT_NW == GQ, "one wavefront per head for the query digits and the inverse rotation");

// Sign tables of the inverse rotation (kernels.cuh:1123-1132, TQ_S1 / TQ_S2) as bit masks: bit j set = -1.
constexpr uint32_t WS1[4] = {0xe46a0359u, 0x42f85949u, 0xa4c63bbbu, 0x49f250a9u};
constexpr uint32_t WS2[4] = {0x16acee90u, 0x3f628fdcu, 0xb7a5357au, 0xbea56562u};
__device__ __forceinline__ float sgn(const uint32_t* m, int j, float x) {
    return (m[j >> 5] >> (j & 31)) & 1 ? -x : x;
}


// 16 V codes -> biased code bytes. w = 2-bit low fields (code c at bits 2c); x = high bits, codes 0-7 in bits 0-7 and
// codes 8-15 in bits 16-23. Word f of the result holds codes f, 4 + f, 8 + f, 12 + f in bytes 0..3: byte i of
// (w >> 2f) & 0x03030303 is the low field of code 4i + f; with the high-bit nibbles moved one per byte (nibble i's bits
// in the low half of byte i; the upper halves keep bits that the masks below drop), bit f of byte i is its high bit,
// brought to bit 2 by one shift; one v_perm LUT maps the 3-bit selectors to codes.
__device__ __forceinline__ void v_codes16(uint32_t w, uint32_t x, uint32_t cd[4]) {
    const uint32_t hs = (x & ~0x0f000f00u) | ((x << 4) & 0x0f000f00u);
    cd[0] = __builtin_amdgcn_perm(SV1, SV0, (w & 0x03030303u) | ((hs << 2) & 0x04040404u));
    cd[1] = __builtin_amdgcn_perm(SV1, SV0, ((w >> 2) & 0x03030303u) | ((hs << 1) & 0x04040404u));
    cd[2] = __builtin_amdgcn_perm(SV1, SV0, ((w >> 4) & 0x03030303u) | (hs & 0x04040404u));
    cd[3] = __builtin_amdgcn_perm(SV1, SV0, ((w >> 6) & 0x03030303u) | ((hs >> 1) & 0x04040404u));
}

// rot != 0: the partial's acc is rotated back (the inverse WHT of turbo_out_k, kernels.cuh:1730-1738, is linear, so
// it commutes with the combine's weighted sum): the combine then gates it directly and no turbo_out launch follows.
__global__ void __launch_bounds__(64 * WT_NW, 1) gqa_wst_kernel(const float* __restrict__ qo, moex_kv_cache kv, int H,
                                                                const int* __restrict__ pos_d, int max_t,
                                                                float* __restrict__ part, int T, int ns, int rot,
                                                                FrontArgs fr) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float cm[WT_NW][GQ], cl[WT_NW][GQ];
    const int nb = gridDim.x, w_id = xcd_work_id(blockIdx.x, nb);
    const int tok = w_id % T, s = (w_id / T) % ns, kvh = w_id / (T * ns);
    const int pos0 = *pos_d, Tmax = pos0 + T;
    const int L = (Tmax + ns - 1) / ns, lo = s * L;
    const int hi = min(pos0 + tok + 1, lo + L);  // keys [lo, hi) of this split that the token sees
    const int nch = hi > lo ? (hi - lo + WT_CH - 1) / WT_CH : 0;
    const int first = hi > lo ? hi - lo - (nch - 1) * WT_CH : 0;  // chunk 0 is the short one
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, m16 = lane & 15;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: the step addresses stay scalar
    const size_t rbase = (size_t)kvh * max_t;
    const uint8_t* Kg = reinterpret_cast<const uint8_t*>(kv.k) + rbase * TQ_KB;
    const uint8_t* Vg = reinterpret_cast<const uint8_t*>(kv.v) + rbase * TQ_VB;
    const float* kng = kv.ks + 2 * rbase;
    const float* vng = kv.vs + 2 * rbase;
    // this wavefront's steps: chunks cs .. nch - 1 (chunk 0 may hold none of its keys); step j uses stage j % WT_NS
    const int cs = (nch > 0 && WT_K * wv >= first) ? 1 : 0, nst = nch - cs;
    unsigned char* ring = smem + wv * WT_NS * WT_STAGE;
    auto keys = [&](int j, int& k0, int& ke) {  // the step's first key and the end of its chunk
        const int c = cs + j;
        k0 = (c == 0 ? lo : lo + first + (c - 1) * WT_CH) + WT_K * wv;
        ke = c == 0 ? lo + first : lo + first + c * WT_CH;
    };
    // five transfers per step: the 16 K rows (two of 8 rows; row r keeps 16-byte piece p in slot p ^ ((r / 2) % 8), so
    // the 8-byte reads of 16 rows at a 128-byte stride hit distinct banks), the norms (lanes 0-31 the K pairs, 32-63
    // the V pairs) and the raw V rows: 16-byte slot t (of 7 per row, the seventh a copy of the sixth) from row t / 7,
    // piece min(t % 7, 5), by all lanes and then lanes 0-47; past the chunk's end keys are clamped
    const int kr0 = lane >> 3, kr1 = 8 + (lane >> 3);
    const uint32_t ko0 = kr0 * TQ_KB + 16 * ((lane & 7) ^ ((kr0 >> 1) & 7));
    const uint32_t ko1 = kr1 * TQ_KB + 16 * ((lane & 7) ^ ((kr1 >> 1) & 7));
    const int vt1 = 64 + lane;
    const uint32_t vo0 = (lane / 7) * TQ_VB + 16 * min(lane % 7, 5), vo1 = (vt1 / 7) * TQ_VB + 16 * min(vt1 % 7, 5);
    auto issue = [&](int j) {
        int k0, ke;
        keys(j, k0, ke);
        unsigned char* st = ring + (j % WT_NS) * WT_STAGE;
        const float* nsrc = lane < 32 ? kng : vng;
        if (k0 + WT_K <= ke) {
            const uint8_t* kb = Kg + (size_t)k0 * TQ_KB;
            const uint8_t* vb = Vg + (size_t)k0 * TQ_VB;
            dma16s(kb, ko0, st);
            dma16s(kb, ko1, st + 1024);
            dma4(nsrc + 2 * (size_t)k0 + (lane & 31), st + WT_NRM);
            dma16s(vb, vo0, st + WT_RV);
            if (lane < 48) dma16s(vb, vo1, st + WT_RV + 1024);
        } else {
            dma16(Kg + (size_t)min(k0 + kr0, ke - 1) * TQ_KB + (ko0 - kr0 * TQ_KB), st);
            dma16(Kg + (size_t)min(k0 + kr1, ke - 1) * TQ_KB + (ko1 - kr1 * TQ_KB), st + 1024);
            dma4(nsrc + 2 * (size_t)min(k0 + ((lane & 31) >> 1), ke - 1) + (lane & 1), st + WT_NRM);
            dma16(Vg + (size_t)min(k0 + lane / 7, ke - 1) * TQ_VB + (vo0 - (lane / 7) * TQ_VB), st + WT_RV);
            if (lane < 48)
                dma16(Vg + (size_t)min(k0 + vt1 / 7, ke - 1) * TQ_VB + (vo1 - (vt1 / 7) * TQ_VB), st + WT_RV + 1024);
        }
    };
    // step j's operands from its stage into registers: the K nibbles of key m16 (per MFMA ks), its norm pairs, and
    // the raw V words of keys 4g .. 4g + 3 (dims 8 m16 .. 8 m16 + 7 of both halves)
    // v_perm selectors: low fields of dims 8 m16 .. 8 m16 + 7 (bytes 2 (m16 % 2), +1 of each half's dword) into the
    // two halves of vw; the high-bit byte m16 % 4 of each half's dword into bytes 0 and 2 of vx (bytes 1, 3 unused)
    const uint32_t ow = 2 * (m16 & 1), ox = m16 & 3;
    const uint32_t vsel_w = ow | (ow + 1) << 8 | (ow + 4) << 16 | (ow + 5) << 24, vsel_x = ox | (ox + 4) << 16;
    struct StepRegs {
        uint2 nib[4];
        float2 kn, vn;
        uint32_t vw[4], vx[4];
    };
    auto load_regs = [&](int j, StepRegs& r) {
        const unsigned char* st = ring + (j % WT_NS) * WT_STAGE;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int byte = 32 * ks + 8 * g;  // row m16
            r.nib[ks] = *reinterpret_cast<const uint2*>(st + m16 * TQ_KB + 16 * ((byte >> 4) ^ ((m16 >> 1) & 7)) +
                                                         (byte & 15));
        }
        r.kn = *reinterpret_cast<const float2*>(st + WT_NRM + 8 * m16);
        r.vn = *reinterpret_cast<const float2*>(st + WT_NRM + 8 * WT_K + 8 * m16);
        // whole dwords (two per read instruction), the lane's 16 bits / byte of each half picked by one v_perm
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t* row = reinterpret_cast<const uint32_t*>(st + WT_RV + (4 * g + i) * WT_VS);
            r.vw[i] = __builtin_amdgcn_perm(row[8 + (m16 >> 1)], row[m16 >> 1], vsel_w);
            r.vx[i] = __builtin_amdgcn_perm(row[20 + (m16 >> 2)], row[16 + (m16 >> 2)], vsel_x);
        }
    };
    // step j has landed once at most 5 * min(a, nst - 1 - j) transfers are in flight (a = steps issued past it)
    auto wait_step = [&](int j, int a) {
        const int ahead = min(a, nst - 1 - j);
        if (ahead >= 3) vm_wait<15>();
        else if (ahead == 2) vm_wait<10>();
        else if (ahead == 1) vm_wait<5>();
        else vm_wait<0>();
    };

    // ---- the front (T <= 4, fr.q set, skip flag clear), one wavefront per row (front::wave: the arithmetic of
    // front_rows_kernel, no barrier): wavefront w forms query head w of the workgroup's token (RMSNorm, RoPE, the
    // forward rotation) and keeps it for its query digits; wavefronts 0 .. nr - 1 form the new key rows this token sees
    // in this split, [na, hi), and append them (TurboQuant). The rows leave the queue (vmcnt) before a barrier that all
    // transfers follow. Workgroups of later tokens in the same split append the same rows again, with the same bytes:
    // every workgroup moves only rows it has written itself ----
    const bool fused = fr.q && !(fr.skip && *fr.skip);
    const int na = max(lo, pos0), nr = fused ? max(0, hi - na) : 0;  // nr <= tok + 1 <= 4 rows
    const bool app = nr > 0;
    float qf4[4];
    if (fused) {
        const float4 a =
            *reinterpret_cast<const float4*>(fr.q + (size_t)tok * fr.ld + (kvh * GQ + wv) * 2 * AHD + 4 * lane);
        qf4[0] = a.x; qf4[1] = a.y; qf4[2] = a.z; qf4[3] = a.w;
        front::wave::norm_rope(qf4, fr.qn, lane, pos0 + tok, fr.rot, fr.theta, fr.eps);
        front::wave::wht(qf4, 0, lane);
        if (s == 0)
            *reinterpret_cast<float4*>(fr.qo + ((size_t)tok * H + kvh * GQ + wv) * AHD + 4 * lane) =
                make_float4(qf4[0], qf4[1], qf4[2], qf4[3]);
        if (wv < nr) {
            const size_t o = (size_t)(na + wv - pos0) * fr.ld + kvh * AHD + 4 * lane;
            const float4 k4 = *reinterpret_cast<const float4*>(fr.k + o);
            const float4 v4 = *reinterpret_cast<const float4*>(fr.v + o);
            float x[4] = {k4.x, k4.y, k4.z, k4.w};
            const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
            front::wave::norm_rope(x, fr.kn, lane, na + wv, fr.rot, fr.theta, fr.eps);
            front::wave::append(x, vv, kv, rbase + na + wv, lane);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
    }
    // ---- query digits, once per workgroup: wavefront w turns head w (lane l: dims 4l .. 4l + 3) into three signed
    // base-256 digits of a 2^(22 - e) fixed point (|q| < 2^e over the head) and writes them to the digit table in
    // the operand order: dim d at byte 16 (d / 16) + pos(d % 16), pos = the K codes' order {0,2,4,6, 1,3,5,7, 8,..} ----
    {
        float4 q4;
        if (fused) q4 = make_float4(qf4[0], qf4[1], qf4[2], qf4[3]);
        else q4 = *reinterpret_cast<const float4*>(qo + ((size_t)tok * H + kvh * GQ + wv) * AHD + 4 * lane);
        float qm = fmaxf(fmaxf(fabsf(q4.x), fabsf(q4.y)), fmaxf(fabsf(q4.z), fabsf(q4.w)));
        qm = max_x32(max_x16(max_row16(qm)));
        int e = 0;
        if (qm > 0.f) (void)frexpf(qm, &e);  // qm < 2^e
        const float up = ldexpf(1.f, 22 - e);
        int8_t* qt = reinterpret_cast<int8_t*>(smem + WT_QT) + wv * AHD;
        const float xv[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            int d2, d1, d0;
            digits3((int)__builtin_rintf(xv[k] * up), d2, d1, d0);
            const int d = 4 * lane + k, dl = d & 15;
            const int at = 16 * (d >> 4) + 8 * (dl >> 3) + ((dl & 1) ? 4 : 0) + ((dl & 7) >> 1);
            qt[at] = (int8_t)d2;
            qt[GQ * AHD + at] = (int8_t)d1;
            qt[2 * GQ * AHD + at] = (int8_t)d0;
        }
        reinterpret_cast<uint32_t*>(qt + 3 * GQ * AHD)[lane] = 0u;  // the zero rows
        if (lane == 0) reinterpret_cast<float*>(smem + WT_QS)[wv] = ldexpf(1.f, e - 22) * (SL2 * TK4);
    }
    // the first steps' transfers (the compiler's wait for the query rows above does not cover them); after the new
    // row's stores, in the split that appends it
    if (app) __syncthreads();
#pragma unroll
    for (int j = 0; j < WT_NS - 1; j++)
        if (j < nst) issue(j);
    __syncthreads();
    // the A operand of MFMA ks: lane (g, m16) holds the 16 bytes of dims 64 ks + 16 g .. + 15 of its row, digit m16 % 4
    // of head m16 / 4 (qx) and of head m16 / 4 + 4 (qy)
    const int dg = m16 & 3, hr = m16 >> 2;
    // (kept in registers: re-reading them from LDS every step measured 4 us slower)
    const unsigned char* qtx = smem + WT_QT + (dg * GQ + hr) * AHD + 16 * g;  // head hr; head hr + 4 at + 4 * AHD
    int4_t_ qx[4], qy[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        qx[ks] = *reinterpret_cast<const int4_t_*>(qtx + 64 * ks);
        qy[ks] = *reinterpret_cast<const int4_t_*>(qtx + 4 * AHD + 64 * ks);
    }
    const float qsA = reinterpret_cast<const float*>(smem + WT_QS)[g];
    const float qsB = reinterpret_cast<const float*>(smem + WT_QS)[g + 4];  // the lane's score heads g and g + 4
    float4_t o[16];  // o[8 h + b]: rows 4g .. 4g + 3 (hi rows for g < 2, lo rows for g >= 2), column m16: dim 128h + 8 m16 + b
#pragma unroll
    for (int J = 0; J < 16; J++) o[J] = float4_t{0.f, 0.f, 0.f, 0.f};
    float mA = -INFINITY, mB = -INFINITY, lA = 0.f, lB = 0.f, vmax = 0.f;
    // sums of P * vn * K3 * 2^sig over the lane's keys per score head and V half: the bias taken out at the end
    float xA0 = 0.f, xA1 = 0.f, xB0 = 0.f, xB1 = 0.f;
    int sig = 0;
    unsigned char* Pt = smem + WT_P0 + wv * WT_PT;  // [V half][row 8 hl + h][16 keys] fp16
    // O += P . V of one step: block (h, b), operand half k = key 4g + k
    auto pv = [&](const uint32_t (&cd)[4][4], const half4_t& pa0, const half4_t& pa1) {
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const int f = b & 3, by = 2 * h + (b >> 2);  // dim 8 m16 + b of half h: code 8h + b, word f, byte by
                const uint32_t sel = (uint32_t)by | 0x0c00u | ((uint32_t)(4 + by) << 16) | 0x0c000000u;
                typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
                const u32x2_t vb = {__builtin_amdgcn_perm(cd[1][f], cd[0][f], sel),
                                    __builtin_amdgcn_perm(cd[3][f], cd[2][f], sel)};
                o[8 * h + b] = __builtin_amdgcn_mfma_f32_16x16x16f16(h ? pa1 : pa0, __builtin_bit_cast(half4_t, vb),
                                                                    o[8 * h + b], 0, 0, 0);
            }
    };
    // P.V runs one step behind: step j's runs among step j + 1's K decode and Q.K (MFMA and VALU work of one
    // wavefront overlap when interleaved), from its V codes and P kept in registers; before step 0 it adds zeros
    uint32_t cdp[4][4];
    half4_t pp0, pp1;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int f = 0; f < 4; f++) cdp[i][f] = 0x80808080u;
#pragma unroll
    for (int i = 0; i < 4; i++) pp0[i] = pp1[i] = (_Float16)0.f;
    for (int j = 0; j < nst; j++) {
        // step j + WT_NS - 1 goes to the stage of step j - 1, which this wavefront has read
        if (j + WT_NS - 1 < nst) issue(j + WT_NS - 1);
        wait_step(j, WT_NS - 1);
        StepRegs cur;
        load_regs(j, cur);
        int k0, ke;
        keys(j, k0, ke);
        // ---- K codes and Q.K: [128-dim half], heads g (sx) and g + 4 (sy) against key m16 ----
        int4_t_ sx[2], sy[2];
        sx[0] = sx[1] = sy[0] = sy[1] = int4_t_{0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int4_t_ b = k_codes(cur.nib[ks]);
            sx[ks >> 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qx[ks], b, sx[ks >> 1], 0, 0, 0);
            sy[ks >> 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qy[ks], b, sy[ks >> 1], 0, 0, 0);
        }
        pv(cdp, pp0, pp1);  // step j - 1
        const float2 kn = cur.kn, vn = cur.vn;
        // ---- scores: per half d2 * 65536 + (d1 * 256 + d0), the latter exact in int32 (|d1 * 256 + d0| < 2^30) ----
        float scA, scB;
        {
            const float a0 = fmaf((float)sx[0][0], 65536.f, (float)(sx[0][1] * 256 + sx[0][2]));
            const float a1 = fmaf((float)sx[1][0], 65536.f, (float)(sx[1][1] * 256 + sx[1][2]));
            const float b0 = fmaf((float)sy[0][0], 65536.f, (float)(sy[0][1] * 256 + sy[0][2]));
            const float b1 = fmaf((float)sy[1][0], 65536.f, (float)(sy[1][1] * 256 + sy[1][2]));
            scA = (a0 * kn.x + a1 * kn.y) * qsA;
            scB = (b0 * kn.x + b1 * kn.y) * qsB;
        }
        float vm = fmaxf(vn.x, vn.y);
        if (k0 + WT_K > ke && k0 + m16 >= ke) {
            scA = scB = -INFINITY;
            vm = 0.f;
        }
        // the reductions over a head's 16 lanes only when some lane's own key passes a bound (rare). A lane's own
        // score passes m_ref + slack exactly when its head's maximum does, and V scales below 2^(7 - sig) cannot move
        // the exponent: the same decisions as with the reduced values
        if (__builtin_amdgcn_ballot_w64(scA > mA + WS_SLACK || scB > mB + WS_SLACK || vm * TK3 >= ldexpf(1.f, 7 - sig)) !=
            0) {
            const float MA = max_row16(scA), MB = max_row16(scB);
            vm = max_row16(vm) * TK3;  // every lane group g holds the step's 16 keys: uniform over the wavefront
            // ---- lazy rescale ----
            const float nA = MA > mA + WS_SLACK ? MA : mA, nB = MB > mB + WS_SLACK ? MB : mB;
            const float fA = ex2d(mA, nA), fB = ex2d(mB, nB);
            vmax = fmaxf(vmax, vm);
            int ev = 0;
            if (vmax > 0.f) (void)frexpf(vmax, &ev);  // vmax < 2^ev: p * vn * K3 * 2^(7 - ev) < 2^(7 + WS_SLACK)
            const int nsig = 7 - ev;
            if (__builtin_amdgcn_ballot_w64(fA != 1.f || fB != 1.f) != 0 || nsig != sig) {
                const float sf = ldexpf(1.f, nsig - sig);
                float fr[4];  // O row 4g + i is head 4 (g & 1) + i: its factor from lane 16 i
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float a = __shfl(fA, 16 * i), b = __shfl(fB, 16 * i);
                    fr[i] = ((g & 1) ? b : a) * sf;
                }
#pragma unroll
                for (int J = 0; J < 16; J++)
#pragma unroll
                    for (int i = 0; i < 4; i++) o[J][i] *= fr[i];
                lA *= fA;
                lB *= fB;
                xA0 *= fA * sf; xA1 *= fA * sf; xB0 *= fB * sf; xB1 *= fB * sf;
                mA = nA;
                mB = nB;
                sig = nsig;
            }
        }
        // ---- P of both V halves, fp16 hi + lo, into the P tiles: row 8 hl + h, column = key ----
        {
            const float vs0 = vn.x * ldexpf(1.f, sig) * TK3, vs1 = vn.y * ldexpf(1.f, sig) * TK3;
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const float p = fast_exp2((hh ? scB : scA) - (hh ? mB : mA));
                const float x0 = p * vs0, x1 = p * vs1;
                if (hh) { lB += p; xB0 += x0; xB1 += x1; } else { lA += p; xA0 += x0; xA1 += x1; }
                const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
                _Float16* pr = reinterpret_cast<_Float16*>(Pt) + (g + 4 * hh) * WT_K + m16;
                pr[0] = h0;
                pr[8 * WT_K] = (_Float16)(x0 - (float)h0);
                pr[16 * WT_K] = h1;
                pr[24 * WT_K] = (_Float16)(x1 - (float)h1);
            }
        }
        // P operand rows m16, keys 4g .. 4g + 3, and the V codes of the 4 keys, for the next step's P.V
        pp0 = *reinterpret_cast<const half4_t*>(Pt + (m16 * WT_K + 4 * g) * 2);
        pp1 = *reinterpret_cast<const half4_t*>(Pt + ((16 + m16) * WT_K + 4 * g) * 2);
#pragma unroll
        for (int i = 0; i < 4; i++) v_codes16(cur.vw[i], cur.vx[i], cdp[i]);
    }
    pv(cdp, pp0, pp1);  // the last step
    // ---- merge the eight wavefronts: m, l per head, then O rows (hi + lo) scaled to the common maximum ----
    const float lAs = sum_row16(lA), lBs = sum_row16(lB);
    // the V operands were (code + 128) * 2^-24: O = 2^24 o - 128 * sum(P * vn * K3 * 2^sig), per head and V half
    const float bA0 = sum_row16(xA0) * VBIAS, bA1 = sum_row16(xA1) * VBIAS;
    const float bB0 = sum_row16(xB0) * VBIAS, bB1 = sum_row16(xB1) * VBIAS;
    if (m16 == 0) { cm[wv][g] = mA; cm[wv][g + 4] = mB; cl[wv][g] = lAs; cl[wv][g + 4] = lBs; }
    __syncthreads();  // every wavefront is past its last step: the rings are free
    float* Ow = reinterpret_cast<float*>(smem);  // [wavefront][head][256]
    const float un = ldexpf(1.f, -sig);
#pragma unroll
    for (int J = 0; J < 16; J++)
#pragma unroll
        for (int i = 0; i < 4; i++) o[J][i] += __shfl_xor(o[J][i], 32);  // lanes l, l + 32: the hi and lo rows
    float b0[4], b1[4];  // row 4g + i is head 4 (g & 1) + i: its sums from lane 16 i (all lanes take part)
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a0 = __shfl(bA0, 16 * i), a1 = __shfl(bA1, 16 * i);
        const float c0 = __shfl(bB0, 16 * i), c1 = __shfl(bB1, 16 * i);
        b0[i] = (g & 1) ? c0 : a0;
        b1[i] = (g & 1) ? c1 : a1;
    }
    if (g < 2) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int h = 4 * g + i;
            float Mh = cm[0][h];
#pragma unroll
            for (int w = 1; w < WT_NW; w++) Mh = fmaxf(Mh, cm[w][h]);
            const float f = ex2d(cm[wv][h], Mh) * un;
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const float b = hf ? b1[i] : b0[i];
                float* dst = Ow + (wv * GQ + h) * AHD + 128 * hf + 8 * m16;
                float r[8];
#pragma unroll
                for (int k = 0; k < 8; k++) r[k] = fmaf(o[8 * hf + k][i], 16777216.f, -b) * f;
                *reinterpret_cast<float4*>(dst) = make_float4(r[0], r[1], r[2], r[3]);
                *reinterpret_cast<float4*>(dst + 4) = make_float4(r[4], r[5], r[6], r[7]);
            }
        }
    }
    __syncthreads();
    float* Om = reinterpret_cast<float*>(smem) + WT_NW * GQ * AHD;  // [head][256]: the merged acc, when rotating back
    for (int it = tid; it < GQ * 64; it += 64 * WT_NW) {
        const int h = it >> 6, d4 = 4 * (it & 63);
        float4 a = *reinterpret_cast<const float4*>(Ow + h * AHD + d4);
#pragma unroll
        for (int w = 1; w < WT_NW; w++) {
            const float4 b = *reinterpret_cast<const float4*>(Ow + (w * GQ + h) * AHD + d4);
            a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
        }
        if (rot) *reinterpret_cast<float4*>(Om + h * AHD + d4) = a;
        else *reinterpret_cast<float4*>(part_acc(part, tok, kvh * GQ + h, s, H, ns) + d4) = a;
        if ((it & 63) == 0) {
            float Mh = cm[0][h];
#pragma unroll
            for (int w = 1; w < WT_NW; w++) Mh = fmaxf(Mh, cm[w][h]);
            float lsum = 0.f;
#pragma unroll
            for (int w = 0; w < WT_NW; w++) lsum += cl[w][h] * ex2d(cm[w][h], Mh);
            float* ml = part_ml(part, tok, kvh * GQ + h, s, H, ns, T);
            ml[0] = Mh;  // -inf when the token has no key in this split
            ml[1] = lsum;
        }
    }
    if (rot) {
        // wavefront w: head w, both halves; lane L holds in-half dims L and L + 64 (stages 1..32 by xor shuffles,
        // stage 64 in the lane), in the order of the reference's inverse: x S2, butterflies, / sqrt(128), x S1
        __syncthreads();
        const int h = wv;
        float* dst = part_acc(part, tok, kvh * GQ + h, s, H, ns);
#pragma unroll
        for (int b = 0; b < 2; b++) {
            float v0 = sgn(WS2, lane, Om[h * AHD + 128 * b + lane]);
            float v1 = sgn(WS2, lane + 64, Om[h * AHD + 128 * b + 64 + lane]);
#pragma unroll
            for (int st = 1; st < 64; st <<= 1) {
                const float o0 = __shfl_xor(v0, st), o1 = __shfl_xor(v1, st);
                v0 = (lane & st) ? o0 - v0 : v0 + o0;
                v1 = (lane & st) ? o1 - v1 : v1 + o1;
            }
            const float a0 = v0 + v1, a1 = v0 - v1;
            dst[128 * b + lane] = sgn(WS1, lane, a0 * 0.08838834764831845f);
            dst[128 * b + 64 + lane] = sgn(WS1, lane + 64, a1 * 0.08838834764831845f);
        }
    }
}

int gqa_splits(int T, int KV, int ns, bool turbo) {
    // the decode kernels run one workgroup per CU (int8: one token or a group of up to 4; turbo: one token): beyond one
    // workgroup per CU extra splits only add per-workgroup set-up and partials
    static const int cus = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            return v;
        return 256;
    }();
    const int fill = cus / (KV * (turbo ? T : T <= 2 ? 1 : (T + 3) / 4));
    return fill < 1 ? 1 : (fill < ns ? fill : ns);
}

void launch_gqa(const float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, float* part, int T,
                int ns, hipStream_t st, bool rot_out, const FrontArgs* fr) {
    if (kv.turbo) {
        static bool once = [] {
            MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(gqa_wst_kernel),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, WT_LDS));
            return true;
        }();
        (void)once;
        hipLaunchKernelGGL(gqa_wst_kernel, dim3(KV * ns * T), dim3(64 * WT_NW), WT_LDS, st, qo, kv, H, pos_d,
                           max_t, part, T, ns, rot_out ? 1 : 0, fr && T <= 4 ? *fr : FrontArgs{});
    } else {
        if (T == 1) {
            static bool once = [] {
                MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(gqa_ws1_kernel<true>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, W1_LDS));
                MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(gqa_ws1_kernel<false>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, W1_LDS));
                return true;
            }();
            (void)once;
            if (fr && fr->q)
                hipLaunchKernelGGL(gqa_ws1_kernel<true>, dim3(KV * ns), dim3(64 * (WS_NC + WS_NP)), W1_LDS, st, qo, kv, H,
                                   pos_d, max_t, part, ns, *fr);
            else
                hipLaunchKernelGGL(gqa_ws1_kernel<false>, dim3(KV * ns), dim3(64 * (WS_NC + WS_NP)), W1_LDS, st, qo, kv, H,
                                   pos_d, max_t, part, ns, FrontArgs{});
        }
        else if (T == 2) launch_wsp<1>(qo, kv, H, KV, pos_d, max_t, part, T, ns, st, fr);
        else launch_wsp<2>(qo, kv, H, KV, pos_d, max_t, part, T, ns, st, fr);
    }
    MOEX_LAUNCHED();
}

}  // namespace moex
