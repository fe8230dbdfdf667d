/*
 * moex_attn.h -- C ABI of the MI355X (gfx950) attention hot path of moex (Qwen3.6-35B-A3B GQA layers:
 * 16 query heads, 2 KV heads, head_dim 256).
 *
 * Every entry point replaces one function or kernel launch of the reference header src/kernels.cuh; the
 * citation is on each declaration. Arguments keep the reference's order and meaning. Differences:
 *   - the stream is an opaque hipStream_t passed as void* (NULL = the default stream);
 *   - fp16 weight pointers (qn, kn) are raw binary16 bit patterns (uint16_t);
 *   - raw kernel launches take their grid-defining sizes (T, ns) explicitly instead of a <<<grid>>>.
 * All pointers are device pointers unless stated otherwise. Nothing allocates or synchronizes except
 * moex_kv_alloc / moex_kv_free and the per-stream workspaces below.
 *
 * Workspaces. moex_attn_fa widens the K/V tiles once into a tile-image workspace of KV * ceil(max_t / 32) * 37632
 * bytes (MOEX_FA_IMAGES=0: none, the kernel widens each tile itself, same results, slower). A chunk whose token
 * tiles leave the chip underfilled (KV * ceil(T / 16) < CUs) may split each token tile's keys over several
 * workgroups, with a second workspace for their partial results, T * H * pieces * 1040 bytes (at most 32 pieces;
 * MOEX_FA_SPLIT=n caps them, 1 turns splitting off). A chunk whose token tiles fill the chip once (KV * ceil(T / 16)
 * <= CUs, not split, e.g. 2048 tokens) runs its token tiles in heavy/light pairs on two workgroups each, the heavy
 * tile's two halves merged in the kernel: a workspace of KV * (ceil(T / 16) / 2) * 4 * 33280 bytes for one half's
 * partial rows and one of 8 bytes per such slot for arrival counters (zeroed when allocated; MOEX_FA_PAIR=0 turns
 * pairs off). A chunk of at most 64 tokens (turbo: 16; MOEX_FA_GQA_MAXT=n
 * sets the int8 bound to n and the turbo bound to n / 4, 0 turns it off) runs on the split-K decode kernels and the
 * combine instead, with a workspace of T * H * ns * 1032 bytes for their partials (ns = moex_gqa_splits(T, KV,
 * moex_decode_splits(max_t), turbo)). moex_attn_decode with ns == 1 and T <= 2 (the reference's one-split call) runs
 * the split-K kernels too, with its partials in a workspace of T * H * n2 * 1032 bytes (n2 = moex_gqa_splits(T, KV,
 * moex_decode_splits(max_t), turbo); none when n2 == 1). The dense GEMM (moex_dense.h) keeps two more. Each is one per (device, stream), allocated on first use with hipMalloc and grown
 * when a larger call comes. An outgrown buffer is not freed before the process ends, because a HIP graph captured
 * earlier may still replay into it. No workspace is allocated while the stream is being captured: a call that would
 * need to grow one reports hipErrorStreamCaptureUnsupported. So after one eager call of a given max_t and T on a
 * stream, the same call can be captured into a HIP graph. The one exception is the one-split decode step above: while
 * its workspace does not exist yet it is captured with the per-head kernel of the reference (no partials, no
 * allocation, no error), so it can be captured first time as the reference's can. A graph's replays use the capturing stream's workspaces:
 * replays and eager calls that overlap in time on different streams race on them. moex_attn_workspace_bytes gives
 * the bytes one call needs, moex_workspace_held the bytes held now (for a VRAM audit next to moex_kv_bytes).
 *
 * Errors (kernels.cuh:8-11, CK): a failing HIP call prints "HIP <error> at <file>:<line>" and exits(1),
 * unless a soft-error slot is installed (moex_set_soft_error), in which case the first error code is
 * stored there and the call returns. Argument errors (unsupported head_dim/group shapes) are reported
 * the same way with code hipErrorInvalidValue (1).
 */
#ifndef MOEX_ATTN_H
#define MOEX_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOEX_AHD 256   /* head dim (kernels.cuh:1111, AHD) */
#define MOEX_TQ_KB 128 /* turbo K bytes per (kv head, position) (kernels.cuh:1122, TQ_KB) */
#define MOEX_TQ_VB 96  /* turbo V bytes per (kv head, position) (kernels.cuh:1122, TQ_VB) */

/* KV cache (kernels.cuh:1121, struct KVCache): same fields, same order, same layout.
 * int8:  k, v int8 [KV][max_t][256]; ks, vs f32 [KV][max_t]          (520 B per kv head and position)
 * turbo: k u8 [KV][max_t][128] (4-bit codes), v u8 [KV][max_t][96] (3-bit codes),
 *        ks, vs f32 [KV][max_t][2] (one norm per 128-value half)      (240 B per kv head and position) */
typedef struct moex_kv_cache {
    int8_t* k;
    int8_t* v;
    float* ks;
    float* vs;
    int turbo;
} moex_kv_cache;

/* ---- cache storage (kernels.cuh:1867-1877) ---- */
/* kv_alloc (kernels.cuh:1867): hipMalloc of the four arrays. */
moex_kv_cache moex_kv_alloc(int KV, int max_t, int turbo);
/* kv_bytes (kernels.cuh:1875): bytes kv_alloc takes, KV * max_t * (turbo ? 240 : 520). */
size_t moex_kv_bytes(int KV, int max_t, int turbo);
/* no counterpart (the reference never frees its cache): hipFree of the four arrays. */
void moex_kv_free(moex_kv_cache kv);

/* ---- full attention step (kernels.cuh:1846-1865, attn_decode) ----
 * q: raw q_proj rows, token stride ld: query [h*512, +256), gate [h*512+256, +256). k, v: raw k/v rows, stride ld.
 * Per token blockIdx-equivalent t at position *pos_d + t: q/k RMSNorm(1+w) and partial RoPE (rot dims, theta),
 * all T K/V rows quantized into kv (int8, or turbo codes), the query written to qo [T][H][256] (turbo: rotated),
 * then attention over keys [0, pos+t] written gated to out [T][H][256].
 * Dispatch as the reference: T > 2 and ns == 1 -> prefill (FA; MOEX_FA=0 -> moex_attn_prefill for int8);
 * ns > 1 -> split-K GQA decode + combine (part: T*H*ns*(256+2) floats); ns == 1 with T <= 2 and H/KV == 8 -> the
 * same split-K kernels with partials in the library's per-stream workspace (the per-head kernel of the reference
 * only under a first-time capture or when one split would do); otherwise the per-head kernel.
 * ns > 1, H/KV == 8, T <= 4 (int8 or turbo): the front and the appends run inside the split kernel (two launches in
 * all), with qo, the cache rows and out bit-identical to the separate front's. */
void moex_attn_decode(const float* q, const float* k, const float* v, const uint16_t* qn, const uint16_t* kn,
                      float* qo, moex_kv_cache kv, float* out, int H, int KV, const int* pos_d, int max_t,
                      int rot, float theta, float eps, int T, int ld, void* stream, float* part, int ns);

/* No counterpart in the reference: moex_attn_decode for callers that cannot allocate (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc). Same arguments and result, without part: the split-K partials
 * (T*H*ns*(256+2) floats) live in a device array of the library, MOEX_NOALLOC_SCRATCH_BYTES per GPU, held from the
 * library's load until the process ends; a larger T*H*ns is rejected (argument error). The prefill branch (T > 2,
 * ns == 1) runs FA without tile images (the same bits) and puts its key pieces' partials in that array, with fewer
 * pieces when they would not fit (results then within the FA tolerance of moex_attn_decode, not bit-identical), and
 * runs full one-wave grids one token tile per workgroup, without the pairs of moex_attn_fa (within the FA tolerance
 * of moex_attn_decode there, not bit-identical).
 * Calls nothing that allocates. Every call on a GPU shares that GPU's array: calls that overlap in time on one GPU
 * (different streams, or a replayed graph beside an eager call) race on it. */
#define MOEX_NOALLOC_SCRATCH_BYTES (32u << 20)
void moex_attn_decode_noalloc(const float* q, const float* k, const float* v, const uint16_t* qn, const uint16_t* kn,
                              float* qo, moex_kv_cache kv, float* out, int H, int KV, const int* pos_d, int max_t,
                              int rot, float theta, float eps, int T, int ld, void* stream, int ns);

/* attn_fa (kernels.cuh:1713): FlashAttention-2 causal GQA prefill of T query tokens at *pos_d..*pos_d+T-1.
 * qo [T][H][256] f32 (rotated for turbo); q_gate: the q rows (gate at [t*ld + h*512 + 256]); NULL = no gate
 * (turbo, followed by moex_turbo_out). Needs H / KV == 8. */
void moex_attn_fa(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                  const int* pos_d, int max_t, int ld, int T, void* stream);

/* attn_prefill (kernels.cuh:1435): the int8-only prefill fallback (K7P), same arguments and result. Any GQA group
 * G = H / KV that divides 32 (kernels.cuh:1856); moex_attn_decode routes T > 2, ns == 1 int8 steps of such G here
 * when FA does not apply (MOEX_FA=0, or G != 8). */
void moex_attn_prefill(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                       const int* pos_d, int max_t, int ld, int T, void* stream);

/* ---- raw launches used by the reference's tests ---- */
/* qk_norm_rope_k (kernels.cuh:1185), grid (H+KV, T): norm + RoPE + quantize-append. */
void moex_qk_norm_rope(const float* q, const float* k, const float* v, const uint16_t* qn, const uint16_t* kn,
                       float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, int rot,
                       float theta, float eps, int ld, int T, void* stream);
/* The quantize-append half of qk_norm_rope_k (kernels.cuh:1210-1235) alone: k rows are already normalized and
 * rotated. Row kvh*max_t + *pos_d + t gets token t's k/v (token stride ld floats, kv head at kvh*256). */
void moex_kv_append(const float* k, const float* v, moex_kv_cache kv, int KV, const int* pos_d, int max_t,
                    int ld, int T, void* stream);
/* attn_gqa_k (kernels.cuh:1745), grid (KV, T, ns): split-K GQA decode, writes partials {m, l, acc[256]} into part
 * (T*H*ns*(256+2) floats, the reference's size): acc rows at part[((t*H + h)*ns + s)*256], then the {m, l} pairs at
 * part[T*H*ns*256 + ((t*H + h)*ns + s)*2]. m is the running max in log2 units (the combine below reads it so).
 * part must be 16-byte aligned (any hipMalloc / cudaMalloc pointer is). */
void moex_attn_gqa(const float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, float* part,
                   int T, int ns, void* stream);
/* No counterpart in the reference: moex_attn_gqa whose turbo partials come out rotated back to the output domain (the
 * inverse WHT of turbo_out_k applied per split, which the combine's weighted sum commutes with), so that
 * moex_attn_combine with the gate gives the final output and no moex_turbo_out follows. moex_attn_decode's split-K
 * branch runs this. For an int8 cache it is moex_attn_gqa. */
void moex_attn_gqa_out(const float* qo, moex_kv_cache kv, int H, int KV, const int* pos_d, int max_t, float* part,
                       int T, int ns, void* stream);
/* attn_combine_k (kernels.cuh:1317), grid (H, T): merges ns partials, out = acc/l * sigmoid(gate) (no gate if
 * q_gate is NULL). */
void moex_attn_combine(const float* part, const float* q_gate, float* out, int H, int ns, int ld, int T,
                       void* stream);
/* attn_decode_k (kernels.cuh:1244), grid (H, T, ns): per-query-head decode (any H/KV). ns == 1 writes the gated
 * output (no gate if q_gate is NULL), ns > 1 partials for moex_attn_combine. */
void moex_attn_decode_heads(const float* qo, const float* q_gate, moex_kv_cache kv, float* out, int H, int KV,
                            const int* pos_d, int max_t, int ld, float* part, int T, int ns, void* stream);
/* turbo_out_k (kernels.cuh:1731), grid (H, T): out = WHT_inverse(out) * sigmoid(gate), in place. */
void moex_turbo_out(float* out, const float* q_gate, int H, int ld, int T, void* stream);
/* set_int_k (kernels.cuh:1879): *p = v on the stream (graph-friendly position update). */
void moex_set_int(int* p, int v, void* stream);

/* ---- runtime switches ---- */
/* g_soft_ck (kernels.cuh:8): while slot != NULL, errors are recorded in *slot (first one wins) instead of exit. */
void moex_set_soft_error(int* slot);
/* g_skip (kernels.cuh:46): while the device flag is nonzero, moex_qk_norm_rope and moex_turbo_out return at once
 * (the graph fallback of the reference's decode step). Set on the stream. */
void moex_set_skip(int value, void* stream);
/* attn_fa_on (kernels.cuh:1699): 1 unless MOEX_FA=0 (read once). */
int moex_fa_on(void);
/* fa_supported (kernels.cuh:1705): 1 when the current device is gfx950. */
int moex_fa_supported(void);
/* Recommended ns for the split-K decode at n_ctx keys on the current device (the engine's ASPLIT). The part
 * buffer must hold T*H*ns*(256+2) floats. No counterpart in the reference (ASPLIT is a constant there). */
int moex_decode_splits(int n_ctx);
/* The split count moex_attn_decode runs its GQA kernel with when it is given ns splits for T query tokens of a
 * cache with KV heads (turbo != 0 for a turbo cache): at most ns. A caller that launches moex_attn_gqa and
 * moex_attn_combine itself passes this value to both. No counterpart in the reference. */
int moex_gqa_splits(int T, int KV, int ns, int turbo);
/* Workspace bytes one moex_attn_fa or moex_attn_decode call with these sizes takes on its stream: tile images plus
 * the partials of split token tiles, or for T <= 2 the partials of the one-split decode step. No counterpart in the reference (its attn_fa_k needs none); for the
 * engine's VRAM audit (moex.cu:960) beside moex_kv_bytes. */
size_t moex_attn_workspace_bytes(int H, int KV, int max_t, int T);
/* Bytes the library's per-stream workspaces hold now, on every device and stream, outgrown buffers included. No
 * counterpart in the reference. */
size_t moex_workspace_held(void);
/* Library build identifier. */
const char* moex_version(void);

#ifdef __cplusplus
}
#endif
#endif
