// Shared constants, device helpers and internal launcher declarations of libmoex_attn (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/moex_attn.h"
#include "../../include/moex_dense.h"

namespace moex {

constexpr int AHD = 256;                  // head dim (kernels.cuh:1111)
constexpr int TQ_KB = 128, TQ_VB = 96;    // turbo bytes per row (kernels.cuh:1122)
constexpr int GQ = 8;                     // query heads per KV head on the GQA paths

// error plumbing (api.cpp): HIP errors abort like the reference's CK, or go to the soft slot
void report(hipError_t e, const char* file, int line);
#define MOEX_CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) ::moex::report(e_, __FILE__, __LINE__); } while (0)
#define MOEX_LAUNCHED() MOEX_CK(hipGetLastError())

// ---- int8 -> fp16 widening (exact) ----
// fp16 0x64XX = 1024 + XX. A signed byte b stored as (b ^ 0x80) = b + 128, so 0x64(b+128) - 1152 = b.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

// global_load_lds operands (a DMA from global memory into LDS, 16 bytes a lane) and a wait on the vector memory counter
typedef __attribute__((address_space(1))) const void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;
// s_waitcnt with only vmcnt = n (expcnt, lgkmcnt left at their no-wait maxima)
template <int n>
__device__ __forceinline__ void wait_vm() {
    static_assert(n >= 0 && n < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ half2_t u2h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t h22u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// Biased bytes (b + 128) in w -> two fp16 pairs: lo = bytes 0,1, hi = bytes 2,3.
__device__ __forceinline__ void biased4_to_h4(uint32_t u, uint32_t& lo, uint32_t& hi) {
    const half2_t off = u2h2(0x64806480u);  // {1152, 1152}
    const uint32_t l = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t h = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    lo = h22u(u2h2(l) - off);
    hi = h22u(u2h2(h) - off);
}
__device__ __forceinline__ void i8x4_to_h4(uint32_t w, uint32_t& lo, uint32_t& hi) { biased4_to_h4(w ^ 0x80808080u, lo, hi); }

// 8 int8 (two dwords) -> one MFMA operand of 8 fp16
__device__ __forceinline__ half8_t i8x8_to_h8(uint32_t a, uint32_t b) {
    uint32_t r0, r1, r2, r3;
    i8x4_to_h4(a, r0, r1);
    i8x4_to_h4(b, r2, r3);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 u = {r0, r1, r2, r3};
    return __builtin_bit_cast(half8_t, u);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Split-K partials in the caller's part buffer (T*H*ns*(AHD+2) floats, the reference's size): the acc rows
// [T][H][ns][AHD] first, then {m (log2 units), l} pairs [T][H][ns][2], so the combine reads every split's m and l
// contiguously and each acc row is 16-byte aligned.
__device__ __forceinline__ float* part_acc(float* part, int t, int h, int s, int H, int ns) {
    return part + (((size_t)t * H + h) * ns + s) * AHD;
}
__device__ __forceinline__ float* part_ml(float* part, int t, int h, int s, int H, int ns, int T) {
    return part + (size_t)T * H * ns * AHD + (((size_t)t * H + h) * ns + s) * 2;
}

// The q/k front's inputs (attn_decode's q, k, v, qn, kn, qo, rot, theta, eps, ld) when a decode kernel runs the front
// in its own prologue instead of after a separate qk_norm_rope launch, and the graph-fallback flag it honours.
struct FrontArgs {
    const float* q;
    const float* k;
    const float* v;
    const uint16_t* qn;
    const uint16_t* kn;
    float* qo;
    const int* skip;
    int rot;
    float theta;
    float eps;
    int ld;
};

}  // namespace moex

// ---- internal launchers (each defined in its .hip file; argument checks happen in api.cpp) ----
namespace moex {
void launch_qk_norm_rope(const float* q, const float* k, const float* v, const uint16_t* qn, const uint16_t* kn,
                         float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, int rot,
                         float theta, float eps, int ld, int T, hipStream_t st);
void launch_kv_append(const float* k, const float* v, moex_kv_cache kv, int KV, const int* pos_d, int max_t, int ld,
                      int T, hipStream_t st);
void launch_turbo_out(float* out, const float* q_gate, int H, int ld, int T, hipStream_t st);
void launch_combine(const float* part, const float* q_gate, float* out, int H, int ns, int ld, int T, hipStream_t st);
void launch_decode_heads(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                         const int* pos_d, int max_t, int ld, float* part, int T, int ns, hipStream_t st);
void launch_set_int(int* p, int v, hipStream_t st);
void launch_set_skip(int v, hipStream_t st);
// split count moex_attn_decode uses for the GQA kernel when the caller allows ns splits (never more than ns)
int gqa_splits(int T, int KV, int ns, bool turbo);
// rot_out (turbo caches): the partials come out rotated back to the output domain, for a gated combine with no
// turbo_out after it
// fr (T <= 4, int8 or turbo): the split kernel runs the q/k front itself (query rows, the new K/V rows appended to the
// cache) and writes qo; without it qo must hold the front's output already
void launch_gqa(const float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, float* part, int T,
                int ns, hipStream_t st, bool rot_out = false, const FrontArgs* fr = nullptr);
// this device's graph-fallback flag (g_skip, kernels.cuh:46), for kernels of other files; nullptr if unavailable
const int* skip_flag();
void launch_fa(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV, const int* pos_d,
               int max_t, int ld, int T, hipStream_t st);
// dense int8 projections (dense.hip)
void launch_quantize_rows_i8(const uint16_t* W, int8_t* q, float* s, int O, int I, hipStream_t st);
void launch_gemv_i8(const int8_t* q, const float* s, const float* x, float* y, int NT, int I, int O, hipStream_t st);
// Device memory kept per (device, stream, kind) until the process ends, grown on demand. nullptr if it cannot be
// allocated; during stream capture a workspace that would have to grow is not allocated and nullptr is returned,
// reported as hipErrorStreamCaptureUnsupported unless quiet (the caller then takes a path that needs none).
unsigned char* stream_workspace(size_t need, hipStream_t st, int kind, bool quiet = false);
// workspace bytes of a one-split attn_decode step of T <= 2 tokens (its split-K partials), 0 when it takes none
size_t decode_ns1_workspace_bytes(int H, int KV, int max_t, int T, bool turbo);
// bytes the workspaces hold on every device and stream, outgrown buffers included
size_t stream_workspace_bytes();
// attn_fa that allocates nothing: no tile images, the key pieces' partials in the given scratch (fewer pieces if they
// would not fit it)
void launch_fa_scratch(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                       const int* pos_d, int max_t, int ld, int T, hipStream_t st, float* scratch, size_t bytes);
// this device's copy of the no-allocation scratch (MOEX_NOALLOC_SCRATCH_BYTES), nullptr (error reported) if its
// address cannot be had
float* noalloc_scratch();
// the most workspace bytes one attn_fa call with these sizes takes on its stream
size_t fa_workspace_bytes(int H, int KV, int max_t, int T);
void launch_gemm_i8(const int8_t* q, const float* s, const float* X, float* Y, int S, int I, int O, hipStream_t st);
// the other weight forms (dense.hip): int4 / int6 gs64 quantizers, the GEMV (NT rows, int6 in one pass, the others a
// launch per row) and the fp16 MFMA GEMM
void launch_quantize_rows_gs64(const uint16_t* W, uint8_t* q, uint8_t* qh, float* s, int O, int I, bool six,
                               hipStream_t st);
void launch_gemv_mat(const moex_mat& m, const float* x, float* y, int NT, int I, int O, hipStream_t st);
void launch_gemm_mat(const moex_mat& m, const float* X, float* Y, int S, int I, int O, hipStream_t st);
void launch_prefill_k7p(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                        const int* pos_d, int max_t, int ld, int T, hipStream_t st);
}  // namespace moex
