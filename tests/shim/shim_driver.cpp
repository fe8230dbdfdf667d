// Drives the reference-side shim of INTEGRATION.md (extracted verbatim into _gen/attn_moex_amd.h by the Makefile)
// with the reference's own types and signatures (kernels.cuh:1713,1850,1867,1875): kv_alloc, kv_bytes, attn_decode
// for a prefill chunk (T = T0, ns = 1 -> FA), attn_fa on the same queries, then attn_decode for one token with split
// partials (ns > 1). Inputs come from files the test wrote, outputs go to files the test checks against the oracle.
//   shim_driver <dir> <turbo> <T0> <ns>
#include <cstdio>
#include <cstdlib>
#include <vector>
#include "attn_moex_amd.h"

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

int main(int argc, char** argv) {
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
