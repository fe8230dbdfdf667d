// Drives the reference-side shim of INTEGRATION.md (extracted verbatim into _gen/attn_moex_amd.h by the Makefile)
// with the reference's own types and signatures (kernels.cuh:1713,1850,1867,1875): kv_alloc, kv_bytes, attn_decode
// for a prefill chunk (T = T0, ns = 1 -> FA), attn_fa on the same queries, then attn_decode for one token with split
// partials (ns > 1). Inputs come from files the test wrote, outputs go to files the test checks against the oracle.
//   shim_driver <dir> <turbo> <T0> <ns>
// Dense mode drives the dense projections' shim with the reference's struct Mat (kernels.cuh:186-196): fp16 rows
// from a file, quantized to int4 and int6 through the library, then gemv and gemm (S rows) for each form.
//   shim_driver <dir> dense <O> <I> <S>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include "attn_moex_amd.h"
// the reference's dense matrix (kernels.cuh:186-196), which the dense shim converts
struct Mat {
    const half* f16 = nullptr;
    const int8_t* q = nullptr;
    const float* s = nullptr;
    const uint8_t* q4 = nullptr;
    const uint8_t *q6 = nullptr, *q6h = nullptr;
};
#include "dense_moex_amd.h"

#define HC(x) do { hipError_t e = (x); if (e != hipSuccess) { fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e)); exit(2); } } while (0)

static std::vector<char> slurp(const char* dir, const char* name) {
    char p[1024];
    snprintf(p, sizeof p, "%s/%s", dir, name);
    FILE* f = fopen(p, "rb");
    if (!f) { fprintf(stderr, "cannot open %s\n", p); exit(2); }
    fseek(f, 0, SEEK_END);
    std::vector<char> b(ftell(f));
    fseek(f, 0, SEEK_SET);
    if (fread(b.data(), 1, b.size(), f) != b.size()) exit(2);
    fclose(f);
    return b;
}
static void spit(const char* dir, const char* name, const void* d, size_t n) {
    char p[1024];
    snprintf(p, sizeof p, "%s/%s", dir, name);
    FILE* f = fopen(p, "wb");
    if (!f || fwrite(d, 1, n, f) != n) { fprintf(stderr, "cannot write %s\n", p); exit(2); }
    fclose(f);
}
template <class T> static T* to_dev(const std::vector<char>& h) {
    void* p = nullptr;
    HC(hipMalloc(&p, h.size()));
    HC(hipMemcpy(p, h.data(), h.size(), hipMemcpyHostToDevice));
    return static_cast<T*>(p);
}
static void from_dev(const char* dir, const char* name, const void* d, size_t n) {
    std::vector<char> h(n);
    HC(hipMemcpy(h.data(), d, n, hipMemcpyDeviceToHost));
    spit(dir, name, h.data(), n);
}

static int dense_main(const char* dir, int O, int I, int S) {
    std::vector<char> wh = slurp(dir, "w16.bin"), xh = slurp(dir, "x.bin");
    const half* w = to_dev<half>(wh);
    const float* X = to_dev<float>(xh);
    uint8_t *q4, *q6, *q6h;
    float *s4, *s6, *y, *Y;
    HC(hipMalloc(&q4, (size_t)O * I / 2));
    HC(hipMalloc(&q6, (size_t)O * I / 2));
    HC(hipMalloc(&q6h, (size_t)O * I / 4));
    HC(hipMalloc(&s4, (size_t)O * (I / 64) * 4));
    HC(hipMalloc(&s6, (size_t)O * (I / 64) * 4));
    HC(hipMalloc(&y, (size_t)O * 4));
    HC(hipMalloc(&Y, (size_t)S * O * 4));
    moex_quantize_rows_q4(reinterpret_cast<const uint16_t*>(w), q4, s4, O, I, nullptr);
    moex_quantize_rows_q6(reinterpret_cast<const uint16_t*>(w), q6, q6h, s6, O, I, nullptr);
    Mat m[3];
    m[0].q4 = q4; m[0].s = s4;
    m[1].q6 = q6; m[1].q6h = q6h; m[1].s = s6;
    m[2].f16 = w;
    const char* names[3] = {"q4", "q6", "f16"};
    for (int f = 0; f < 3; f++) {
        gemv(m[f], X, y, I, O);
        gemm(m[f], X, Y, S, I, O);
        HC(hipDeviceSynchronize());
        char n[64];
        snprintf(n, sizeof n, "y_%s.bin", names[f]);
        from_dev(dir, n, y, (size_t)O * 4);
        snprintf(n, sizeof n, "Y_%s.bin", names[f]);
        from_dev(dir, n, Y, (size_t)S * O * 4);
    }
    from_dev(dir, "q4.bin", q4, (size_t)O * I / 2);
    from_dev(dir, "s4.bin", s4, (size_t)O * (I / 64) * 4);
    from_dev(dir, "q6.bin", q6, (size_t)O * I / 2);
    from_dev(dir, "q6h.bin", q6h, (size_t)O * I / 4);
    from_dev(dir, "s6.bin", s6, (size_t)O * (I / 64) * 4);
    printf("dense shim ok\n");
    return 0;
}

int main(int argc, char** argv) {
    if (argc == 6 && !strcmp(argv[2], "dense")) return dense_main(argv[1], atoi(argv[3]), atoi(argv[4]), atoi(argv[5]));
    if (argc != 5) { fprintf(stderr, "usage: shim_driver dir turbo T0 ns\n"); return 2; }
    const char* dir = argv[1];
    const int turbo = atoi(argv[2]), T0 = atoi(argv[3]), ns = atoi(argv[4]);
    const int H = 16, KV = 2, LQ = H * 2 * AHD + 2 * KV * AHD, max_t = T0 + 8, rot = 64;
    const float theta = 1e7f, eps = 1e-6f;
    hipStream_t st;
    HC(hipStreamCreate(&st));
    KVCache kv = kv_alloc(KV, max_t, turbo);
    const size_t kb = kv_bytes(KV, max_t, turbo);
    if (kb != (size_t)KV * max_t * (turbo ? 240 : 520)) { fprintf(stderr, "kv_bytes %zu\n", kb); return 3; }
    // rows 0 .. T0-1 (the chunk), then row T0 (the decode token)
    std::vector<char> qkv_h = slurp(dir, "qkv.bin");
    float* qkv = to_dev<float>(qkv_h);
    std::vector<char> wn = slurp(dir, "norm.bin");  // fp16 q norm then k norm weights
    const half* qn = to_dev<half>(wn);
    const half* kn = qn + AHD;
    int* pos_d = nullptr;
    float *qo, *out, *out2, *part;
    HC(hipMalloc(&pos_d, sizeof(int)));
    HC(hipMalloc(&qo, (size_t)T0 * H * AHD * 4));
    HC(hipMalloc(&out, (size_t)T0 * H * AHD * 4));
    HC(hipMalloc(&out2, (size_t)T0 * H * AHD * 4));
    HC(hipMalloc(&part, (size_t)H * ns * (AHD + 2) * 4));
    HC(hipMemsetAsync(pos_d, 0, sizeof(int), st));
    attn_decode(qkv, qkv + H * 2 * AHD, qkv + H * 2 * AHD + KV * AHD, qn, kn, qo, kv, out, H, KV, pos_d, max_t, rot,
                theta, eps, T0, LQ, st, nullptr, 1);
    attn_fa(qo, turbo ? nullptr : qkv, kv, out2, H, KV, pos_d, max_t, LQ, T0, st);
    HC(hipStreamSynchronize(st));
    from_dev(dir, "chunk_qo.bin", qo, (size_t)T0 * H * AHD * 4);
    from_dev(dir, "chunk_out.bin", out, (size_t)T0 * H * AHD * 4);
    from_dev(dir, "chunk_fa.bin", out2, (size_t)T0 * H * AHD * 4);
    const float* row = qkv + (size_t)T0 * LQ;
    HC(hipMemcpyAsync(pos_d, &T0, sizeof(int), hipMemcpyHostToDevice, st));
    attn_decode(row, row + H * 2 * AHD, row + H * 2 * AHD + KV * AHD, qn, kn, qo, kv, out, H, KV, pos_d, max_t, rot,
                theta, eps, 1, LQ, st, part, ns);
    HC(hipStreamSynchronize(st));
    from_dev(dir, "dec_qo.bin", qo, (size_t)H * AHD * 4);
    from_dev(dir, "dec_out.bin", out, (size_t)H * AHD * 4);
    const size_t rb = turbo ? 128 : 256, vb = turbo ? 96 : 256, sn = turbo ? 2 : 1;
    from_dev(dir, "cache_k.bin", kv.k, (size_t)KV * max_t * rb);
    from_dev(dir, "cache_v.bin", kv.v, (size_t)KV * max_t * vb);
    from_dev(dir, "cache_ks.bin", kv.ks, (size_t)KV * max_t * sn * 4);
    from_dev(dir, "cache_vs.bin", kv.vs, (size_t)KV * max_t * sn * 4);
    printf("shim ok fa_on=%d fa_supported=%d\n", (int)attn_fa_on(), (int)fa_supported());
    return 0;
}
