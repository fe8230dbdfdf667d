// extern "C" entry points of libmoex_attn (include/moex_attn.h): argument checks, the reference's dispatch
// (kernels.cuh:1846-1865) and error handling (kernels.cuh:8-11). Host code only; kernels are launched through the
// internal launchers of the .hip files.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include "common.hpp"

namespace moex {

static int* g_soft = nullptr;  // kernels.cuh:8 (g_soft_ck)

void report(hipError_t e, const char* file, int line) {
    if (g_soft) {
        if (!*g_soft) *g_soft = (int)e;
        return;
    }
    fprintf(stderr, "HIP %s at %s:%d\n", hipGetErrorString(e), file, line);
    exit(1);
}

static bool arg_fail(const char* what) {
    if (g_soft) {
        if (!*g_soft) *g_soft = (int)hipErrorInvalidValue;
        return true;
    }
    fprintf(stderr, "moex_attn: invalid argument: %s\n", what);
    exit(1);
}
#define MOEX_REQUIRE(cond, what) do { if (!(cond)) { arg_fail(what); return; } } while (0)

static inline hipStream_t S(void* st) { return reinterpret_cast<hipStream_t>(st); }

size_t decode_ns1_workspace_bytes(int H, int KV, int max_t, int T, bool turbo) {
    if (T > 2 || H != KV * GQ) return 0;
    const int n2 = gqa_splits(T, KV, moex_decode_splits(max_t), turbo);
    return n2 > 1 ? (size_t)T * H * n2 * (AHD + 2) * sizeof(float) : 0;
}

}  // namespace moex

using namespace moex;

extern "C" {

moex_kv_cache moex_kv_alloc(int KV, int max_t, int turbo) {
    moex_kv_cache c;
    memset(&c, 0, sizeof c);
    c.turbo = turbo ? 1 : 0;
    const size_t kb = turbo ? TQ_KB : AHD, vb = turbo ? TQ_VB : AHD, ns = turbo ? 2 : 1;
    MOEX_CK(hipMalloc(&c.k, (size_t)KV * max_t * kb));
    MOEX_CK(hipMalloc(&c.v, (size_t)KV * max_t * vb));
    MOEX_CK(hipMalloc(&c.ks, (size_t)KV * max_t * ns * 4));
    MOEX_CK(hipMalloc(&c.vs, (size_t)KV * max_t * ns * 4));
    return c;
}

size_t moex_kv_bytes(int KV, int max_t, int turbo) {
    return (size_t)KV * max_t * (turbo ? TQ_KB + TQ_VB + 16 : 2 * AHD + 8);
}

void moex_kv_free(moex_kv_cache kv) {
    if (kv.k) MOEX_CK(hipFree(kv.k));
    if (kv.v) MOEX_CK(hipFree(kv.v));
    if (kv.ks) MOEX_CK(hipFree(kv.ks));
    if (kv.vs) MOEX_CK(hipFree(kv.vs));
}

int moex_fa_on(void) {  // kernels.cuh:1699-1702
    static const int on = !(getenv("MOEX_FA") && atoi(getenv("MOEX_FA")) == 0);
    return on;
}

int moex_fa_supported(void) {  // kernels.cuh:1705-1712, asked per device
    static int arch[64] = {};  // 0 = not asked, 1 = gfx950, 2 = other
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (!arch[dev]) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) != hipSuccess) return 0;
        arch[dev] = strncmp(p.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
    }
    return arch[dev] == 1;
}

int moex_decode_splits(int n_ctx) {
    int dev = 0, cus = 256;  // MI355X
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
    }
    // two streaming workgroups per CU over both kv heads (each walks its split in 128-key chunks), but no split
    // shorter than 256 keys
    int ns = cus;
    if (ns > (n_ctx + 255) / 256) ns = (n_ctx + 255) / 256;
    return ns < 1 ? 1 : ns;
}

int moex_gqa_splits(int T, int KV, int ns, int turbo) {
    if (!(T > 0 && KV > 0 && ns > 0)) {
        arg_fail("T, KV, ns");
        return 1;
    }
    return gqa_splits(T, KV, ns, turbo != 0);
}

void moex_quantize_rows_i8(const uint16_t* W, int8_t* q, float* s, int O, int I, void* stream) {
    MOEX_REQUIRE(O > 0 && I > 0, "O, I");
    launch_quantize_rows_i8(W, q, s, O, I, S(stream));
}

void moex_gemv_i8(const int8_t* q, const float* s, const float* x, float* y, int I, int O, void* stream) {
    MOEX_REQUIRE(O > 0 && I > 0 && I % 512 == 0 && I <= 40448, "gemv_i8 needs I % 512 == 0 and I <= 40448");
    launch_gemv_i8(q, s, x, y, 1, I, O, S(stream));
}

void moex_gemm_i8(const int8_t* q, const float* s, const float* X, float* Y, int S_, int I, int O, void* stream) {
    MOEX_REQUIRE(O > 0 && I > 0 && S_ > 0, "S, I, O");
    if (S_ <= 8) {  // kernels.cuh:341-349: one GEMV pass for the MTP / draft rows
        MOEX_REQUIRE(I % 512 == 0 && I <= 40448, "gemm_i8 with S <= 8 needs I % 512 == 0 and I <= 40448");
        const int per = 40448 / I;  // input rows that fit in LDS (160 KB of fp32 less the partial sums) per pass
        for (int t0 = 0; t0 < S_;) {
            const int nt = S_ - t0 < per ? S_ - t0 : per;
            launch_gemv_i8(q, s, X + (size_t)t0 * I, Y + (size_t)t0 * O, nt, I, O, S(stream));
            t0 += nt;
        }
        return;
    }
    MOEX_REQUIRE(I % 32 == 0, "gemm_i8 needs I % 32 == 0");
    launch_gemm_i8(q, s, X, Y, S_, I, O, S(stream));
}

void moex_quantize_rows_q4(const uint16_t* W, uint8_t* q4, float* s, int O, int I, void* stream) {
    MOEX_REQUIRE(O > 0 && I > 0 && I % 64 == 0, "quantize_rows_q4 needs I % 64 == 0");
    launch_quantize_rows_gs64(W, q4, nullptr, s, O, I, false, S(stream));
}

void moex_quantize_rows_q6(const uint16_t* W, uint8_t* q6, uint8_t* q6h, float* s, int O, int I, void* stream) {
    MOEX_REQUIRE(O > 0 && I > 0 && I % 64 == 0, "quantize_rows_q6 needs I % 64 == 0");
    launch_quantize_rows_gs64(W, q6, q6h, s, O, I, true, S(stream));
}

namespace {
// the form a Mat is held in, tested in the reference's order (kernels.cuh:214-219): int4, int6, int8, fp16
bool mat_ok(const moex_mat* m, int I) {
    if (!m) return false;
    if (m->q4) return m->s && I % 64 == 0;
    if (m->q6) return m->q6h && m->s && I % 64 == 0;
    if (m->q) return m->s != nullptr;
    return m->f16 && I % 32 == 0;
}
}  // namespace

void moex_gemv(const moex_mat* m, const float* x, float* y, int I, int O, void* stream) {
    MOEX_REQUIRE(O > 0 && I > 0 && mat_ok(m, I), "gemv needs one form of the matrix (int4 / int6: I % 64 == 0 and "
                                                  "scales; fp16: I % 32 == 0)");
    if (!m->q4 && !m->q6 && m->q) {
        moex_gemv_i8(m->q, m->s, x, y, I, O, stream);
        return;
    }
    launch_gemv_mat(*m, x, y, 1, I, O, S(stream));
}

void moex_gemm(const moex_mat* m, const float* X, float* Y, int S_, int I, int O, void* stream) {
    MOEX_REQUIRE(O > 0 && I > 0 && S_ > 0 && mat_ok(m, I), "gemm needs one form of the matrix (int4 / int6: "
                                                            "I % 64 == 0 and scales; fp16: I % 32 == 0)");
    if (!m->q4 && !m->q6 && m->q) {  // kernels.cuh:340-349, 366
        moex_gemm_i8(m->q, m->s, X, Y, S_, I, O, stream);
        return;
    }
    if (m->q6 && !m->q4 && S_ <= 8) {  // :350-357, 360: one GEMV pass for the rows
        launch_gemv_mat(*m, X, Y, S_, I, O, S(stream));
        return;
    }
    if (S_ <= 2) {  // :358-362: the GEMV row by row
        launch_gemv_mat(*m, X, Y, S_, I, O, S(stream));
        return;
    }
    MOEX_REQUIRE(I % 32 == 0, "gemm needs I % 32 == 0");
    launch_gemm_mat(*m, X, Y, S_, I, O, S(stream));
}

size_t moex_attn_workspace_bytes(int H, int KV, int max_t, int T) {
    if (!(KV > 0 && H == KV * GQ && T > 0 && max_t > 0)) return 0;
    if (T <= 2)  // a one-split attn_decode step (attn_fa of T <= 2 takes the same workspace kind, never more)
        return std::max({fa_workspace_bytes(H, KV, max_t, T), decode_ns1_workspace_bytes(H, KV, max_t, T, false),
                         decode_ns1_workspace_bytes(H, KV, max_t, T, true)});
    return fa_workspace_bytes(H, KV, max_t, T);
}

size_t moex_workspace_held(void) { return stream_workspace_bytes(); }

const char* moex_version(void) { return "moex_attn gfx950 0.1"; }

void moex_set_soft_error(int* slot) { g_soft = slot; }

void moex_set_skip(int value, void* stream) { launch_set_skip(value, S(stream)); }

void moex_set_int(int* p, int v, void* stream) { launch_set_int(p, v, S(stream)); }

void moex_qk_norm_rope(const float* q, const float* k, const float* v, const uint16_t* qn, const uint16_t* kn,
                       float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, int rot, float theta,
                       float eps, int ld, int T, void* stream) {
    MOEX_REQUIRE(H > 0 && KV > 0 && H % KV == 0 && T > 0, "H, KV, T");
    MOEX_REQUIRE(rot >= 0 && rot <= AHD && rot % 2 == 0, "rot");
    launch_qk_norm_rope(q, k, v, qn, kn, qo, kv, H, KV, pos_d, max_t, rot, theta, eps, ld, T, S(stream));
}

void moex_kv_append(const float* k, const float* v, moex_kv_cache kv, int KV, const int* pos_d, int max_t, int ld,
                    int T, void* stream) {
    MOEX_REQUIRE(KV > 0 && T > 0, "KV, T");
    launch_kv_append(k, v, kv, KV, pos_d, max_t, ld, T, S(stream));
}

void moex_attn_gqa(const float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, float* part, int T,
                   int ns, void* stream) {
    MOEX_REQUIRE(KV > 0 && H == KV * GQ, "the GQA kernel needs H / KV == 8");
    MOEX_REQUIRE(T > 0 && ns > 0 && part, "T, ns, part");
    MOEX_REQUIRE(((uintptr_t)part & 15) == 0, "part must be 16-byte aligned");
    launch_gqa(qo, kv, H, KV, pos_d, max_t, part, T, ns, S(stream));
}

void moex_attn_gqa_out(const float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, float* part,
                       int T, int ns, void* stream) {
    MOEX_REQUIRE(KV > 0 && H == KV * GQ, "the GQA kernel needs H / KV == 8");
    MOEX_REQUIRE(T > 0 && ns > 0 && part, "T, ns, part");
    MOEX_REQUIRE(((uintptr_t)part & 15) == 0, "part must be 16-byte aligned");
    launch_gqa(qo, kv, H, KV, pos_d, max_t, part, T, ns, S(stream), kv.turbo != 0);
}

void moex_attn_combine(const float* part, const float* q_gate, float* out, int H, int ns, int ld, int T, void* stream) {
    MOEX_REQUIRE(H > 0 && T > 0 && ns > 0, "H, T, ns");
    launch_combine(part, q_gate, out, H, ns, ld, T, S(stream));
}

void moex_attn_decode_heads(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                            const int* pos_d, int max_t, int ld, float* part, int T, int ns, void* stream) {
    MOEX_REQUIRE(H > 0 && KV > 0 && H % KV == 0 && T > 0 && ns > 0, "H, KV, T, ns");
    MOEX_REQUIRE(ns == 1 || part, "part is needed when ns > 1");
    launch_decode_heads(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, part, T, ns, S(stream));
}

void moex_turbo_out(float* out, const float* q_gate, int H, int ld, int T, void* stream) {
    MOEX_REQUIRE(H > 0 && T > 0 && q_gate, "H, T, q_gate");
    launch_turbo_out(out, q_gate, H, ld, T, S(stream));
}

void moex_attn_fa(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV, const int* pos_d,
                  int max_t, int ld, int T, void* stream) {
    MOEX_REQUIRE(KV > 0 && H == KV * GQ, "attn_fa needs H / KV == 8");
    MOEX_REQUIRE(T > 0, "T");
    if (!moex_fa_supported()) {  // kernels.cuh:1715-1719: outside gfx950 keep the simpler kernels
        if (kv.turbo) launch_decode_heads(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, nullptr, T, 1, S(stream));
        else launch_prefill_k7p(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T, S(stream));
        return;
    }
    launch_fa(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T, S(stream));
}

void moex_attn_prefill(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                       const int* pos_d, int max_t, int ld, int T, void* stream) {
    MOEX_REQUIRE(KV > 0 && H % KV == 0 && 32 % (H / KV) == 0, "attn_prefill needs H / KV to divide 32");
    MOEX_REQUIRE(!kv.turbo, "attn_prefill reads int8 KV only");
    MOEX_REQUIRE(T > 0, "T");
    launch_prefill_k7p(qo, q_gate, kv, out, H, KV, pos_d, max_t, ld, T, S(stream));
}

}  // extern "C"

namespace {
// The step of moex_attn_decode after its argument checks. fa_scr: nullptr, or a scratch of fa_bytes for the prefill
// branch's key-piece partials (the no-allocation entry point).
void decode_step(const float* q, const float* k, const float* v, const uint16_t* qn, const uint16_t* kn, float* qo,
                 moex_kv_cache kv, float* out, int H, int KV, const int* pos_d, int max_t, int rot, float theta,
                 float eps, int T, int ld, hipStream_t st, float* part, int ns, float* fa_scr, size_t fa_bytes) {
    const int G = H / KV;
    if (ns == 1 && T <= 2 && G == GQ) {
        // the reference's one-split path (attn_decode_k per query head, no partials): one workgroup per head and
        // token leaves the chip idle (90 000 keys: 8.4 ms int8, 11.6 ms turbo). The split-K kernels take it with
        // partials of the library's own (a workspace, or the no-allocation scratch). The per-head kernel runs when
        // that is not available: one split, no allocation possible, or the stream is being captured before an eager
        // call made the workspace (quietly: the reference's path allocates nothing and captures first time).
        const size_t need = decode_ns1_workspace_bytes(H, KV, max_t, T, kv.turbo != 0);
        const int n2 = gqa_splits(T, KV, moex_decode_splits(max_t), kv.turbo != 0);
        float* w = !need ? nullptr
                   : fa_scr ? (need <= fa_bytes ? fa_scr : nullptr)
                            : reinterpret_cast<float*>(stream_workspace(need, st, 4, true));
        if (w) {
            part = w;
            ns = n2;
        }
    }
    if (ns > 1 && G == GQ && T <= 4) {
        // up to 4 tokens (a decode step or an MTP window): the split kernel runs the q/k front in its prologue (one
        // launch fewer per step); turbo: its partials rotated back, so the combine gates them and no turbo_out
        // follows
        const FrontArgs fr{q, k, v, qn, kn, qo, skip_flag(), rot, theta, eps, ld};
        ns = gqa_splits(T, KV, ns, kv.turbo != 0);
        launch_gqa(qo, kv, H, KV, pos_d, max_t, part, T, ns, st, kv.turbo != 0, &fr);
        launch_combine(part, q, out, H, ns, ld, T, st);
        return;
    }
    launch_qk_norm_rope(q, k, v, qn, kn, qo, kv, H, KV, pos_d, max_t, rot, theta, eps, ld, T, st);
    const float* gate = kv.turbo ? nullptr : q;  // turbo: gated after the inverse rotation
    if (T > 2 && ns == 1 && G == GQ && (moex_fa_on() || kv.turbo) && moex_fa_supported()) {
        if (fa_scr) launch_fa_scratch(qo, gate, kv, out, H, KV, pos_d, max_t, ld, T, st, fa_scr, fa_bytes);
        else launch_fa(qo, gate, kv, out, H, KV, pos_d, max_t, ld, T, st);
    } else if (T > 2 && ns == 1 && 32 % G == 0 && !kv.turbo) {  // kernels.cuh:1856: any G dividing 32
        launch_prefill_k7p(qo, q, kv, out, H, KV, pos_d, max_t, ld, T, st);
    } else if (ns > 1 && G == GQ) {
        ns = gqa_splits(T, KV, ns, kv.turbo != 0);
        // turbo: the split kernel rotates its partials back, so the combine gates them and turbo_out is not needed
        launch_gqa(qo, kv, H, KV, pos_d, max_t, part, T, ns, st, kv.turbo != 0);
        launch_combine(part, q, out, H, ns, ld, T, st);
        return;
    } else {
        launch_decode_heads(qo, gate, kv, out, H, KV, pos_d, max_t, ld, part, T, ns, st);
        if (ns > 1) launch_combine(part, gate, out, H, ns, ld, T, st);
    }
    if (kv.turbo) launch_turbo_out(out, q, H, ld, T, st);
}
}  // namespace

extern "C" {

void moex_attn_decode(const float* q, const float* k, const float* v, const uint16_t* qn, const uint16_t* kn, float* qo,
                      moex_kv_cache kv, float* out, int H, int KV, const int* pos_d, int max_t, int rot, float theta,
                      float eps, int T, int ld, void* stream, float* part, int ns) {
    MOEX_REQUIRE(H > 0 && KV > 0 && H % KV == 0 && T > 0 && ns > 0, "H, KV, T, ns");
    MOEX_REQUIRE(ns == 1 || part, "part is needed when ns > 1");
    MOEX_REQUIRE(((uintptr_t)part & 15) == 0, "part must be 16-byte aligned");
    MOEX_REQUIRE(rot >= 0 && rot <= AHD && rot % 2 == 0, "rot");
    decode_step(q, k, v, qn, kn, qo, kv, out, H, KV, pos_d, max_t, rot, theta, eps, T, ld, S(stream), part, ns, nullptr,
                0);
}

void moex_attn_decode_noalloc(const float* q, const float* k, const float* v, const uint16_t* qn, const uint16_t* kn,
                              float* qo, moex_kv_cache kv, float* out, int H, int KV, const int* pos_d, int max_t,
                              int rot, float theta, float eps, int T, int ld, void* stream, int ns) {
    MOEX_REQUIRE(H > 0 && KV > 0 && H % KV == 0 && T > 0 && ns > 0, "H, KV, T, ns");
    MOEX_REQUIRE(rot >= 0 && rot <= AHD && rot % 2 == 0, "rot");
    MOEX_REQUIRE(ns == 1 || (size_t)T * H * ns * (AHD + 2) * sizeof(float) <= MOEX_NOALLOC_SCRATCH_BYTES,
                 "attn_decode_noalloc: the split partials T*H*ns*1032 bytes exceed MOEX_NOALLOC_SCRATCH_BYTES");
    float* scr = noalloc_scratch();
    if (!scr) return;  // reported
    decode_step(q, k, v, qn, kn, qo, kv, out, H, KV, pos_d, max_t, rot, theta, eps, T, ld, S(stream),
                ns > 1 ? scr : nullptr, ns, scr, MOEX_NOALLOC_SCRATCH_BYTES);
}

}  // extern "C"
