// Split-K GQA decode / MTP-verify attention on gfx950 (replaces attn_gqa_k, kernels.cuh:1740-1844).
//
// One workgroup = (kv head, key split, group of query tokens); the 8 query heads of the group share every K/V byte.
// int8 cache: gqa_ws1_kernel for a single query token (warp-specialised: producer wavefronts stream K/V into LDS,
// consumer wavefronts compute), gqa_wsp_kernel for MTP-verify windows (token pairs on the same pipeline).
// gqa_wst_kernel serves the TurboQuant cache, one token per workgroup on the same pipeline, the codes unpacked on the
// way. The partial written per (token, head, split) is {m (log2 units), l, acc[256]}.
#include "common.hpp"

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
constexpr int WS_CH = 32 * WS_NC;                     // keys per chunk of the turbo kernel: 32 per consumer
constexpr float WS_SLACK = 8.f;

// The producer side of gqa_ws1_kernel / gqa_wsp_kernel: chunks of CH keys (keys [clo(c), chi(c)), chunk 0 the short
// one) in a ring of NS LDS stages, NS - 1 chunks in flight. A stage holds the K rows, the V rows, then ks[CH] and
// vs[CH]. Producers 0, 1 move the K rows, 2, 3 the V rows (CH / 8 instructions of 4 rows each); with 128-key chunks
// each producer also moves 64 scales (ks for 0, 1, vs for 2, 3), with 64-key chunks producers 0 and 2 move all 64
// (4 bytes a lane). Rows past the chunk repeat its last row: their P is 0. Chunk c + NS - 1 is issued at the barrier
// that hands chunk c to the consumers (its stage held chunk c - 1, now consumed); the producers end each chunk with a
// bare s_barrier, as __syncthreads would also wait for the chunks still in flight. Takes part in the nch + 2
// barriers of the chunk loop and the consumer merge.
template <int CH>
constexpr int ring_stage() { return 2 * CH * AHD + 2 * CH * 4; }

template <int CH, int NS>
__device__ __forceinline__ void ring_producer(unsigned char* smem, const moex_kv_cache& kv, size_t rbase, int pw,
                                              int lane, int lo, int first, int nch) {
    static_assert((CH == 64 || CH == 128) && NS >= 2 && NS <= 4, "ring shape");
    constexpr int KB = CH * AHD, STAGE = ring_stage<CH>(), NI = CH / 8;
    constexpr bool SC_ALL = CH == 128;
    const bool sc = SC_ALL || !(pw & 1);
    const int8_t* src = (pw < 2 ? kv.k : kv.v) + rbase * AHD;
    const float* ssrc = (pw < 2 ? kv.ks : kv.vs) + rbase;
    const int r4 = lane >> 4, sl = lane & 15;
    auto issue = [&](int c) {
        const int c0 = c == 0 ? lo : lo + first + (c - 1) * CH, ce = c == 0 ? lo + first : lo + first + c * CH;
        unsigned char* st = smem + (c % NS) * STAGE;
        unsigned char* sb = st + (pw < 2 ? 0 : KB);
#pragma unroll
        for (int u = 0; u < NI; u++) {
            const int i = NI * (pw & 1) + u, r = 4 * i + r4;  // instruction i covers rows 4i .. 4i+3
            const int piece = pw < 2 ? sl ^ (r & 15) : sl ^ (4 * (i & 3));
            __builtin_amdgcn_global_load_lds((gptr_t)(src + (size_t)min(c0 + r, ce - 1) * AHD + 16 * piece),
                                             (lptr_t)(sb + i * 1024), 16, 0, 0);
        }
        if (sc) {
            const int k0 = SC_ALL ? 64 * (pw & 1) : 0;
            __builtin_amdgcn_global_load_lds((gptr_t)(ssrc + min(c0 + k0 + lane, ce - 1)),
                                             (lptr_t)(st + 2 * KB + (pw < 2 ? 0 : 4 * CH) + 4 * k0), 4, 0, 0);
        }
    };
    for (int c = 0; c < NS - 1 && c < nch; c++) issue(c);
    for (int c = 0; c < nch; c++) {
        // chunk c has landed when at most the chunks issued after it are in flight (NI or NI + 1 instructions each)
        const int after = min(nch - 1 - c, NS - 2);
        if (after == 0) wait_vm<0>();
        else if (sc) { if (after == 1) wait_vm<NI + 1>(); else wait_vm<2 * (NI + 1)>(); }
        else { if (after == 1) wait_vm<NI>(); else wait_vm<2 * NI>(); }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (c + NS - 1 < nch) issue(c + NS - 1);
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
constexpr int W1_LDS = W1_NS * W1_STAGE;
static_assert(WS_NC * GQ * AHD * 4 <= W1_LDS, "the consumer merge fits in the stages");
static_assert(W1_LDS <= 160 * 1024, "LDS");

__global__ void __launch_bounds__(64 * (WS_NC + WS_NP), 1) gqa_ws1_kernel(const float* __restrict__ qo, moex_kv_cache kv,
                                                                         int H, const int* __restrict__ pos_d,
                                                                         int max_t, float* __restrict__ part, int ns) {
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

    if (wv >= WS_NC) {
        ring_producer<W1_CH, W1_NS>(smem, kv, rbase, wv - WS_NC, lane, lo, first, nch);
    } else {
        // ---- consumers. Query digits in registers: column m16 of the Q.K MFMA is head m16 / 2 (every head twice);
        // lane (g, m16) holds dims 64 ks + 16 g .. +15 of it, the 4 lanes of a column together hold its 256 dims ----
        int4_t_ qd[3][4];
        float qs;
        {
            const float* qrow = qo + ((size_t)kvh * GQ + (m16 >> 1)) * AHD + 16 * g;
            float4 qv4[16];
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
#pragma unroll
                for (int u = 0; u < 4; u++) qv4[4 * ks + u] = *reinterpret_cast<const float4*>(qrow + 64 * ks + 4 * u);
            float qm = 0.f;
#pragma unroll
            for (int u = 0; u < 16; u++)
                qm = fmaxf(fmaxf(qm, fmaxf(fabsf(qv4[u].x), fabsf(qv4[u].y))), fmaxf(fabsf(qv4[u].z), fabsf(qv4[u].w)));
            qm = fmaxf(qm, __shfl_xor(qm, 16));
            qm = fmaxf(qm, __shfl_xor(qm, 32));
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
        float4_t o[16];
#pragma unroll
        for (int J = 0; J < 16; J++) o[J] = float4_t{0.f, 0.f, 0.f, 0.f};
        float mref = -INFINITY, lacc = 0.f, vmax = 0.f, xsum = 0.f;
        int sig = 0;
        const int kb = 16 * wv;  // this consumer's keys kb .. kb + 15 of every chunk
        for (int c = 0; c < nch; c++) {
            __syncthreads();  // chunk c is in stage c % 4
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

template <int NPR>
__global__ void __launch_bounds__(64 * (WS_NC + WS_NP), 1) gqa_wsp_kernel(const float* __restrict__ qo, moex_kv_cache kv,
                                                                         int H, const int* __restrict__ pos_d,
                                                                         int max_t, float* __restrict__ part, int T,
                                                                         int ns) {
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

    if (wv >= WS_NC) {
        ring_producer<CH, NS>(smem, kv, rbase, wv - WS_NC, lane, lo, first, nch);
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
            const float* qrow = qo + ((size_t)(tb + min(tl, ntok - 1)) * H + kvh * GQ + (m16 & 7)) * AHD + 16 * g;
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
                       int T, int ns, hipStream_t st) {
    static bool once = [] {
        MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(gqa_wsp_kernel<NPR>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, wsp_lds<NPR>()));
        return true;
    }();
    (void)once;
    hipLaunchKernelGGL(gqa_wsp_kernel<NPR>, dim3(KV * ns * ((T + 2 * NPR - 1) / (2 * NPR))),
                       dim3(64 * (WS_NC + WS_NP)), wsp_lds<NPR>(), st, qo, kv, H, pos_d, max_t, part, T, ns);
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
// 4 nibble indices (one per byte) -> 4 signed K codes
__device__ __forceinline__ int lut16s(uint32_t idx) {
    const uint32_t s3 = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(SK1, SK0, s3), hi = __builtin_amdgcn_perm(SK3, SK2, s3);
    // byte b from hi when bit 3 of index b is set: selector b + 4 picks byte b of the first perm operand
    return (int)__builtin_amdgcn_perm(hi, lo, 0x03020100u | ((idx >> 1) & 0x04040404u));
}
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

// ---- gqa_wst_kernel: TurboQuant cache, one query token per workgroup, on the warp-specialised pipeline.
// Producers move each 128-key chunk by DMA (36 transfers per chunk, 4-byte ones for the norms so every key index is
// clamped): the K nibble rows (row r keeps 16-byte piece p in slot p ^ ((r / 2) % 8), so the 8-byte fragment reads of
// 16 rows at a 128-byte stride hit distinct banks) and the K and V half norms into one of three K stages, the raw V
// rows (96 bytes, packed) into one of two raw V buffers. Producer j moves the raw V rows of keys 32j .. 32j + 31 and,
// once they have landed, unpacks their 3-bit codes into consumer j's int8 code area for that chunk (the int8
// kernels' V layout, two areas per consumer), so the unpacking runs beside the consumers' work on the previous chunk. Two
// chunks are in flight: chunk c + 2 is issued at the barrier that starts chunk c. Q.K puts digit 2 of the 8 heads
// (columns 0-7) and digit 0 (columns 8-15) into one MFMA and digit 1 (both halves) into a second, per 128-dim half;
// one row_ror:8 DPP move gives each lane of a head's pair the digit its partner holds, digits 1 and 0 are added
// exactly in int32 and digit 2 joins in one fma, in the same order in both lanes; P carries the V half norm. P rows are (hi / lo part, head), so the P.V key order being the
// Q.K output order, each lane's probabilities are its own A operand; the hi and lo rows of O are added across lanes at
// the end.
constexpr int WST_KB = 128 * TQ_KB;                      // K nibble rows of a stage
constexpr int WST_NS = 3;                                // K stages
constexpr int WST_STAGE = WST_KB + 2 * 128 * 8;          // K nibble rows + K norms + V norms
constexpr int WST_RV = 128 * TQ_VB;                      // raw V rows of a chunk (two buffers)
constexpr int WST_VC = 32 * AHD;                         // one consumer's unpacked V codes (two buffers)
constexpr int WST_VC0 = WST_NS * WST_STAGE + 2 * WST_RV;  // offset of the V code areas
constexpr int WST_LDS = WST_VC0 + 2 * WS_NC * WST_VC;
static_assert((WS_NC + 1) * GQ * AHD * 4 <= WST_NS * WST_STAGE, "the consumer merge and the merged rows fit in the stages");
static_assert(WST_LDS <= 160 * 1024, "LDS");

// Sign tables of the inverse rotation (kernels.cuh:1123-1132, TQ_S1 / TQ_S2) as bit masks: bit j set = -1.
constexpr uint32_t WS1[4] = {0xe46a0359u, 0x42f85949u, 0xa4c63bbbu, 0x49f250a9u};
constexpr uint32_t WS2[4] = {0x16acee90u, 0x3f628fdcu, 0xb7a5357au, 0xbea56562u};
__device__ __forceinline__ float sgn(const uint32_t* m, int j, float x) {
    return (m[j >> 5] >> (j & 31)) & 1 ? -x : x;
}

// rot != 0: the partial's acc is rotated back (the inverse WHT of turbo_out_k, kernels.cuh:1730-1738, is linear, so
// it commutes with the combine's weighted sum): the combine then gates it directly and no turbo_out launch follows.
__global__ void __launch_bounds__(64 * (WS_NC + WS_NP), 1) gqa_wst_kernel(const float* __restrict__ qo, moex_kv_cache kv,
                                                                         int H, const int* __restrict__ pos_d,
                                                                         int max_t, float* __restrict__ part, int T,
                                                                         int ns, int rot) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float cm[WS_NC][GQ], cl[WS_NC][GQ];
    const int nb = gridDim.x, w_id = xcd_work_id(blockIdx.x, nb);
    const int tok = w_id % T, s = (w_id / T) % ns, kvh = w_id / (T * ns);
    const int pos0 = *pos_d, Tmax = pos0 + T;
    const int L = (Tmax + ns - 1) / ns, lo = s * L;
    const int hi = min(pos0 + tok + 1, lo + L);  // keys [lo, hi) of this split that the token sees
    const int nch = hi > lo ? (hi - lo + WS_CH - 1) / WS_CH : 0;
    const int first = hi > lo ? hi - lo - (nch - 1) * WS_CH : 0;  // chunk 0 is the short one
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 4, m16 = lane & 15;
    const size_t rbase = (size_t)kvh * max_t;

    if (wv >= WS_NC) {
        // ---- producers: transfer i (0..35) of a chunk goes to producer i % 4: 0-15 K rows (8 rows each), 16-27 raw
        // V rows (1 KB of the packed rows each; producer j takes the 3 KB of keys 32j ..), 28-31 K norms, 32-35 V
        // norms (64 floats each): 9 per producer ----
        const int pw = wv - WS_NC;
        const uint8_t* Kg = reinterpret_cast<const uint8_t*>(kv.k) + rbase * TQ_KB;
        const uint8_t* Vg = reinterpret_cast<const uint8_t*>(kv.v) + rbase * TQ_VB;
        const float* kng = kv.ks + 2 * rbase;
        const float* vng = kv.vs + 2 * rbase;
        // a full chunk's sources sit at lane-constant byte offsets from its first row: computed once
        int offs[9];
#pragma unroll
        for (int u = 0; u < 9; u++) {
            const int i = pw + 4 * u;
            if (i < 16) {
                const int r = 8 * i + (lane >> 3);
                offs[u] = r * TQ_KB + 16 * ((lane & 7) ^ ((r >> 1) & 7));
            } else if (i < 28) {
                offs[u] = (3 * pw + (i - 16) / 4) * 1024 + 16 * lane;  // the chunk's raw V rows are contiguous
            } else {
                offs[u] = 4 * (64 * (i & 3) + lane);                   // two norms per key, contiguous
            }
        }
        auto issue = [&](int c) {
            const int c0 = c == 0 ? lo : lo + first + (c - 1) * WS_CH, ce = c == 0 ? lo + first : lo + first + c * WS_CH;
            unsigned char* st = smem + (c % WST_NS) * WST_STAGE;
            unsigned char* rv = smem + WST_NS * WST_STAGE + (c & 1) * WST_RV;
            if (ce - c0 == WS_CH) {
                const uint8_t* kb0 = Kg + (size_t)c0 * TQ_KB;
                const uint8_t* vb0 = Vg + (size_t)c0 * TQ_VB;
                const uint8_t* nk0 = reinterpret_cast<const uint8_t*>(kng + 2 * (size_t)c0);
                const uint8_t* nv0 = reinterpret_cast<const uint8_t*>(vng + 2 * (size_t)c0);
#pragma unroll
                for (int u = 0; u < 9; u++) {
                    const int i = pw + 4 * u;
                    if (i < 16)
                        __builtin_amdgcn_global_load_lds((gptr_t)(kb0 + offs[u]), (lptr_t)(st + i * 1024), 16, 0, 0);
                    else if (i < 28)
                        __builtin_amdgcn_global_load_lds((gptr_t)(vb0 + offs[u]),
                                                         (lptr_t)(rv + (3 * pw + (i - 16) / 4) * 1024), 16, 0, 0);
                    else
                        __builtin_amdgcn_global_load_lds((gptr_t)((i < 32 ? nk0 : nv0) + offs[u]),
                                                         (lptr_t)(st + WST_KB + (i < 32 ? 0 : 1024) + 256 * (i & 3)),
                                                         4, 0, 0);
                }
                return;
            }
#pragma unroll
            for (int u = 0; u < 9; u++) {
                const int i = pw + 4 * u;
                if (i < 16) {
                    const int r = 8 * i + (lane >> 3), piece = (lane & 7) ^ ((r >> 1) & 7);
                    __builtin_amdgcn_global_load_lds((gptr_t)(Kg + (size_t)min(c0 + r, ce - 1) * TQ_KB + 16 * piece),
                                                     (lptr_t)(st + i * 1024), 16, 0, 0);
                } else if (i < 28) {  // the raw V rows of keys 32 pw .. 32 pw + 31 (unpacked by this producer)
                    const int piece = 3 * pw + (i - 16) / 4, b = piece * 1024 + 16 * lane, r = b / TQ_VB;
                    __builtin_amdgcn_global_load_lds((gptr_t)(Vg + (size_t)min(c0 + r, ce - 1) * TQ_VB + (b - r * TQ_VB)),
                                                     (lptr_t)(rv + piece * 1024), 16, 0, 0);
                } else {
                    const int f = 64 * (i & 3) + lane, key = min(c0 + (f >> 1), ce - 1);
                    __builtin_amdgcn_global_load_lds((gptr_t)((i < 32 ? kng : vng) + 2 * (size_t)key + (f & 1)),
                                                     (lptr_t)(st + WST_KB + (i < 32 ? 0 : 1024) + 256 * (i & 3)),
                                                     4, 0, 0);
                }
            }
        };
        if (nch > 0) issue(0);
        if (nch > 1) issue(1);
        for (int c = 0; c < nch; c++) {
            if (c + 1 < nch) wait_vm<9>();  // chunk c has landed (chunk c + 1 may still be in flight)
            else wait_vm<0>();
            const int c0 = c == 0 ? lo : lo + first + (c - 1) * WS_CH, ce = c == 0 ? lo + first : lo + first + c * WS_CH;
            if (c0 + 32 * pw < ce) {
                // V codes of keys 32 pw + 0..31 into consumer pw's code area of chunk c (its chunk c - 2 user is done):
                // lane = (piece pc = lane % 16, keys lane / 16 + 4 it)
                unsigned char* Vc = smem + WST_VC0 + ((c & 1) * WS_NC + pw) * WST_VC;
                const int pc = lane & 15, hb = pc >> 3, q = pc & 7;
                const unsigned char* rw0 = smem + WST_NS * WST_STAGE + (c & 1) * WST_RV + (32 * pw + (lane >> 4)) * TQ_VB;
                uint32_t Lw[8], Hh[8];
#pragma unroll
                for (int it = 0; it < 8; it++) {
                    Lw[it] = *reinterpret_cast<const uint32_t*>(rw0 + it * 4 * TQ_VB + 32 * hb + 4 * q);
                    Hh[it] = *reinterpret_cast<const uint16_t*>(rw0 + it * 4 * TQ_VB + 64 + 16 * hb + 2 * q);
                }
#pragma unroll
                for (int it = 0; it < 8; it++) {
                    const int kk = (lane >> 4) + 4 * it;  // 0..31
                    uint32_t sel[4];
                    tr4x4_(Lw[it] & 0x03030303u, (Lw[it] >> 2) & 0x03030303u, (Lw[it] >> 4) & 0x03030303u,
                           (Lw[it] >> 6) & 0x03030303u, sel);
                    uint32_t cd[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const uint32_t idx = sel[k] | ((__builtin_amdgcn_ubfe(Hh[it], 4 * k, 4) * 0x810204u) & 0x04040404u);
                        cd[k] = __builtin_amdgcn_perm(SV1, SV0, idx);
                    }
                    // not a C++ store: the compiler would wait for every DMA in flight before it (it cannot tell that the
                    // code areas are none of their destinations)
                    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
                    const uint32_t la = (uint32_t)(uintptr_t)(Vc + kk * AHD + 16 * (pc ^ (4 * ((kk >> 2) & 3))));
                    asm volatile("ds_write_b128 %0, %1" ::"v"(la), "v"(u32x4_t{cd[0], cd[1], cd[2], cd[3]}) : "memory");
                }
            }
            // chunk c and its V codes are ready, and the consumers are done with chunk c - 1: its K stage takes chunk
            // c + 2, as does the raw V buffer of chunk c. Not __syncthreads: that waits for chunk c + 1 too.
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (c + 2 < nch) issue(c + 2);
        }
        __syncthreads();
        __syncthreads();
    } else {
        __builtin_amdgcn_s_setprio(2);  // consumers ahead of the unpacking producers at the SIMD's issue arbiter
        // (the other way round measured 3 us slower)
        // ---- consumers. Query digits in registers: MFMA ks, lane (g, m16) holds dims
        // 64 ks + 16 g + {0,2,4,6, 1,3,5,7, 8,10,12,14, 9,11,13,15} of head m16 % 8; qa = digit 2 (m16 < 8) or 0,
        // qb = digit 1 ----
        const int hq = m16 & 7;
        const bool lo8 = m16 < 8;
        int4_t_ qa[4], qb[4];
        float qs;
        {
            const float* qrow = qo + ((size_t)tok * H + kvh * GQ + hq) * AHD + 16 * g;
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
            qs = ldexpf(1.f, e - 22) * (SL2 * TK4);
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                int da[16], db[16];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float4 x = qv4[4 * ks + u];
                    const float xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        int d2, d1, d0;
                        digits3((int)__builtin_rintf(xv[k] * up), d2, d1, d0);
                        // dim 4u + k of the lane's 16 goes to operand byte: even dims of each 8 first, then odd
                        const int dl = 4 * u + k, pos = 8 * (dl >> 3) + ((dl & 1) ? 4 : 0) + ((dl & 7) >> 1);
                        da[pos] = lo8 ? d2 : d0;
                        db[pos] = d1;
                    }
                }
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    qa[ks][w] = (int)pack_bytes(da[4 * w], da[4 * w + 1], da[4 * w + 2], da[4 * w + 3]);
                    qb[ks][w] = (int)pack_bytes(db[4 * w], db[4 * w + 1], db[4 * w + 2], db[4 * w + 3]);
                }
            }
        }
        float4_t o[16];  // ws layout: row 2h (2h + 1) = hi (lo) part of head h
#pragma unroll
        for (int J = 0; J < 16; J++) o[J] = float4_t{0.f, 0.f, 0.f, 0.f};
        float mref = -INFINITY, lacc = 0.f, vmax = 0.f;
        float xsum0 = 0.f, xsum1 = 0.f;  // sum of P * vn * K3 * 2^sig of this lane's keys (V halves 0, 1): the bias
        int sig = 0;
        const int kb = 32 * wv;
        for (int c = 0; c < nch; c++) {
            __syncthreads();  // chunk c is in K stage c % WST_NS, its V codes in area c % 2
            const int c0 = c == 0 ? lo : lo + first + (c - 1) * WS_CH, ce = c == 0 ? lo + first : lo + first + c * WS_CH;
            if (c0 + kb >= ce) continue;
            const unsigned char* sb = smem + (c % WST_NS) * WST_STAGE;
            const unsigned char* Vc = smem + WST_VC0 + ((c & 1) * WS_NC + wv) * WST_VC;  // V codes (ws layout)
            const float2* skn = reinterpret_cast<const float2*>(sb + WST_KB);
            const float2* svn = skn + 128;
            float2 kn[8], vn[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                kn[j] = skn[kb + 16 * (j >> 2) + 4 * g + (j & 3)];
                vn[j] = svn[kb + 16 * (j >> 2) + 4 * g + (j & 3)];
            }
            // ---- K codes and the 16 Q.K MFMAs (halves in separate accumulators) ----
            int4_t_ da0[2], db0[2], da1[2], db1[2];
#pragma unroll
            for (int grp = 0; grp < 2; grp++) {
                da0[grp] = int4_t_{0, 0, 0, 0}; db0[grp] = int4_t_{0, 0, 0, 0};
                da1[grp] = int4_t_{0, 0, 0, 0}; db1[grp] = int4_t_{0, 0, 0, 0};
            }
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
#pragma unroll
                for (int grp = 0; grp < 2; grp++) {
                    const int byte = 64 * (ks >> 1) + 32 * (ks & 1) + 8 * g;  // row kb + 16 grp + m16
                    const uint2 nib = *reinterpret_cast<const uint2*>(sb + (kb + 16 * grp + m16) * TQ_KB +
                                                                      16 * ((byte >> 4) ^ ((m16 >> 1) & 7)) + (byte & 15));
                    const int4_t_ a = k_codes(nib);
                    if (ks < 2) {
                        da0[grp] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qa[ks], da0[grp], 0, 0, 0);
                        db0[grp] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qb[ks], db0[grp], 0, 0, 0);
                    } else {
                        da1[grp] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qa[ks], da1[grp], 0, 0, 0);
                        db1[grp] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qb[ks], db1[grp], 0, 0, 0);
                    }
                }
            // ---- scores: both lanes of a head (m16, m16 ^ 8) recombine its digits in the same order (|d1 * 256 + d0|
            // < 2^30: exact in int32) ----
            float sc[8];
#pragma unroll
            for (int grp = 0; grp < 2; grp++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int a0 = da0[grp][i], x0 = dpp_ror8(a0), a1 = da1[grp][i], x1 = dpp_ror8(a1);
                    const float r0 = fmaf((float)(lo8 ? a0 : x0), 65536.f, (float)(db0[grp][i] * 256 + (lo8 ? x0 : a0)));
                    const float r1 = fmaf((float)(lo8 ? a1 : x1), 65536.f, (float)(db1[grp][i] * 256 + (lo8 ? x1 : a1)));
                    sc[4 * grp + i] = (r0 * kn[4 * grp + i].x + r1 * kn[4 * grp + i].y) * qs;
                }
            float vm;
            if (c0 + kb + 32 <= ce) {
                vm = 0.f;
#pragma unroll
                for (int j = 0; j < 8; j++) vm = fmaxf(vm, fmaxf(vn[j].x, vn[j].y));
            } else {
                vm = 0.f;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const bool ok = c0 + kb + 16 * (j >> 2) + 4 * g + (j & 3) < ce;
                    sc[j] = ok ? sc[j] : -INFINITY;
                    vm = ok ? fmaxf(vm, fmaxf(vn[j].x, vn[j].y)) : vm;
                }
            }
            float M = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
            // the reductions over the lane groups only when some lane's own keys pass a bound (rare). A lane's
            // own maximum passes m_ref + slack exactly when its group's does, and V scales below 2^(7 - sig)
            // cannot move the exponent: the same decisions as with the reduced values, bit for bit
            if (__builtin_amdgcn_ballot_w64(M > mref + WS_SLACK || vm * TK3 >= ldexpf(1.f, 7 - sig)) != 0) {
                M = max_x32(max_x16(M));
                vm = max_x32(max_x16(vm)) * TK3;
                // ---- lazy rescale ----
                const float nref = M > mref + WS_SLACK ? M : mref;
                const float fown = ex2d(mref, nref);
                vmax = fmaxf(vmax, vm);
                int ev = 0;
                if (vmax > 0.f) (void)frexpf(vmax, &ev);  // vmax < 2^ev: p * vn * K3 * 2^(7 - ev) < 2^(7 + WS_SLACK)
                const int nsig = 7 - ev;
                if (__builtin_amdgcn_ballot_w64(fown != 1.f) != 0 || nsig != sig) {
                    const float sf = ldexpf(1.f, nsig - sig);
                    float fr[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) fr[i] = __shfl(fown, (4 * g + i) & 7) * sf;  // O row m: head m % 8
#pragma unroll
                    for (int J = 0; J < 16; J++)
#pragma unroll
                        for (int i = 0; i < 4; i++) o[J][i] *= fr[i];
                    lacc *= fown;
                    xsum0 *= fown * sf; xsum1 *= fown * sf;
                    mref = nref;
                    sig = nsig;
                }
            }
            // ---- P of both V halves = 2^(s - mref) * vn * K3 * 2^sig as fp16 hi (m16 < 8) / lo (m16 >= 8): row m16 of
            // the P operand (head m16 % 8), each lane's 8 keys its own A operand (the P.V key order is the Q.K
            // output order) ----
            half8_t pa0, pa1;
            {
                const float vsc = ldexpf(1.f, sig) * TK3;
                half8_t p0v, p1v;
                float ls = 0.f, xs0 = 0.f, xs1 = 0.f;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float p = fast_exp2(sc[j] - mref);
                    ls += p;
                    const float x0 = p * (vn[j].x * vsc), x1 = p * (vn[j].y * vsc);
                    xs0 += x0; xs1 += x1;
                    const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
                    p0v[j] = lo8 ? h0 : (_Float16)(x0 - (float)h0);
                    p1v[j] = lo8 ? h1 : (_Float16)(x1 - (float)h1);
                }
                lacc += lo8 ? ls : 0.f;
                xsum0 += xs0; xsum1 += xs1;
                pa0 = p0v;
                pa1 = p1v;
            }
            // ---- O^T += P . V over these 32 keys: dims < 128 (pc 0, 1) with the half-0 P, the rest with half 1 ----
#pragma unroll
            for (int pc = 0; pc < 4; pc++) {
                const int rd = 16 * ((4 * pc + (m16 >> 2)) ^ (4 * g)) + 4 * (m16 & 3);
                uint32_t r[8];
#pragma unroll
                for (int j = 0; j < 8; j++)
                    r[j] = *reinterpret_cast<const uint32_t*>(Vc + (16 * (j >> 2) + 4 * g + (j & 3)) * AHD + rd);
#pragma unroll
                for (int jt = 0; jt < 4; jt++)
                    o[4 * pc + jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pc < 2 ? pa0 : pa1, bsub8(r, jt),
                                                                         o[4 * pc + jt], 0, 0, 0);
            }
        }
        // ---- merge the four consumers: m, l per head, then O rows (hi + lo) scaled to the common maximum ----
        const float l = sum_x32(sum_x16(lacc));
        __syncthreads();  // every consumer is past its last chunk: the stages are free
        if (lane < 8) { cm[wv][lane] = mref; cl[wv][lane] = l; }
        __syncthreads();
        float* Ow = reinterpret_cast<float*>(smem);  // [consumer][head][256]
        const float un = ldexpf(1.f, -sig);
        // O rows 4g + i: head (4g + i) % 8, hi for g < 2 and lo for g >= 2: lanes l and l + 32 hold the two parts
#pragma unroll
        for (int J = 0; J < 16; J++)
#pragma unroll
            for (int i = 0; i < 4; i++) o[J][i] += __shfl_xor(o[J][i], 32);
        // the V operands were (code + 128) * 2^-24: O = 2^24 o - 128 * sum(P * vn * K3 * 2^sig), per head and V half
        const float xb0 = sum_x32(sum_x16(xsum0)) * VBIAS, xb1 = sum_x32(sum_x16(xsum1)) * VBIAS;
        if (g < 2) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int h = 4 * g + i;
                const float Mh = fmaxf(fmaxf(cm[0][h], cm[1][h]), fmaxf(cm[2][h], cm[3][h]));
                const float f = ex2d(cm[wv][h], Mh) * un;
                const float b0 = __shfl(xb0, h), b1 = __shfl(xb1, h);  // lane h: head h's sums (its hi lanes)
#pragma unroll
                for (int pc = 0; pc < 4; pc++) {
                    const float b = pc < 2 ? b0 : b1;
                    *reinterpret_cast<float4*>(Ow + (wv * GQ + h) * AHD + 64 * pc + 4 * m16) =
                        make_float4(fmaf(o[4 * pc][i], 16777216.f, -b) * f, fmaf(o[4 * pc + 1][i], 16777216.f, -b) * f,
                                    fmaf(o[4 * pc + 2][i], 16777216.f, -b) * f, fmaf(o[4 * pc + 3][i], 16777216.f, -b) * f);
                }
            }
        }
    }
    __syncthreads();
    float* Om = reinterpret_cast<float*>(smem) + WS_NC * GQ * AHD;  // [head][256]: the merged acc, when rotating back
    for (int it = tid; it < GQ * 64; it += 64 * (WS_NC + WS_NP)) {
        const float* Ow = reinterpret_cast<const float*>(smem);
        const int h = it >> 6, d4 = 4 * (it & 63);
        float4 a = *reinterpret_cast<const float4*>(Ow + h * AHD + d4);
#pragma unroll
        for (int w = 1; w < WS_NC; w++) {
            const float4 b = *reinterpret_cast<const float4*>(Ow + (w * GQ + h) * AHD + d4);
            a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
        }
        if (rot) *reinterpret_cast<float4*>(Om + h * AHD + d4) = a;
        else *reinterpret_cast<float4*>(part_acc(part, tok, kvh * GQ + h, s, H, ns) + d4) = a;
        if ((it & 63) == 0) {
            const float Mh = fmaxf(fmaxf(cm[0][h], cm[1][h]), fmaxf(cm[2][h], cm[3][h]));
            float* ml = part_ml(part, tok, kvh * GQ + h, s, H, ns, T);
            ml[0] = Mh;  // -inf when the token has no key in this split
            ml[1] = cl[0][h] * ex2d(cm[0][h], Mh) + cl[1][h] * ex2d(cm[1][h], Mh) + cl[2][h] * ex2d(cm[2][h], Mh) +
                    cl[3][h] * ex2d(cm[3][h], Mh);
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
                int ns, hipStream_t st, bool rot_out) {
    if (kv.turbo) {
        static bool once = [] {
            MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(gqa_wst_kernel),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, WST_LDS));
            return true;
        }();
        (void)once;
        hipLaunchKernelGGL(gqa_wst_kernel, dim3(KV * ns * T), dim3(64 * (WS_NC + WS_NP)), WST_LDS, st, qo, kv, H, pos_d,
                           max_t, part, T, ns, rot_out ? 1 : 0);
    } else {
        if (T == 1) {
            static bool once = [] {
                MOEX_CK(hipFuncSetAttribute(reinterpret_cast<const void*>(gqa_ws1_kernel),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, W1_LDS));
                return true;
            }();
            (void)once;
            hipLaunchKernelGGL(gqa_ws1_kernel, dim3(KV * ns), dim3(64 * (WS_NC + WS_NP)), W1_LDS, st, qo, kv, H, pos_d,
                               max_t, part, ns);
        }
        else if (T == 2) launch_wsp<1>(qo, kv, H, KV, pos_d, max_t, part, T, ns, st);
        else launch_wsp<2>(qo, kv, H, KV, pos_d, max_t, part, T, ns, st);
    }
    MOEX_LAUNCHED();
}

}  // namespace moex
