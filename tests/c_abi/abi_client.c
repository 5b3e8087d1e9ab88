/*
 * A C client of include/dtattn.h with no torch and no Python: the calls a DTorch maintainer's
 * SdpaOp::Compute branch would make (dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:
 * 107-109), on device buffers from hipMalloc and the null stream.  tests/test_gpu_c_abi_client.py writes
 * the inputs, runs this program and checks its outputs against the oracle.
 *
 *   abi_client prefill DIR   DIR/meta: B Hq Hkv Sq Sk D causal; DIR/q.bin k.bin v.bin (bf16 bits,
 *                            contiguous [B, H, S, D]) -> DIR/o.bin (bf16), DIR/lse.bin (fp32)
 *   abi_client decode DIR    DIR/meta: B Hq Hkv S_max D; DIR/q.bin [B, Hq, 1, D], k.bin v.bin
 *                            [B, Hkv, S_max, D] (bf16 bits), lengths.bin (int32 [B]) -> o.bin, lse.bin,
 *                            o_noalloc.bin, lse_noalloc.bin (the allocation-free entry point, same call)
 *
 * Exit status 0 on success; on any failure the dtattn or HIP error text goes to stderr.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "dtattn.h"

static int die(const char* what, const char* detail) {
    fprintf(stderr, "abi_client: %s: %s\n", what, detail ? detail : "");
    return 1;
}

#define HIP_OK(call)                                                                    \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess) return die(#call, hipGetErrorString(e_));                 \
    } while (0)

static void* read_file(const char* dir, const char* name, size_t bytes) {
    char path[1024];
    snprintf(path, sizeof(path), "%s/%s", dir, name);
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    void* buf = malloc(bytes ? bytes : 1);
    size_t got = fread(buf, 1, bytes, f);
    fclose(f);
    if (got != bytes) {
        free(buf);
        return NULL;
    }
    return buf;
}

static int write_file(const char* dir, const char* name, const void* buf, size_t bytes) {
    char path[1024];
    snprintf(path, sizeof(path), "%s/%s", dir, name);
    FILE* f = fopen(path, "wb");
    if (!f) return 1;
    size_t put = fwrite(buf, 1, bytes, f);
    fclose(f);
    return put == bytes ? 0 : 1;
}

/* host buffer -> new device buffer */
static int upload(const char* dir, const char* name, size_t bytes, void** dev) {
    void* h = read_file(dir, name, bytes);
    if (!h) return die("cannot read input", name);
    hipError_t e = hipMalloc(dev, bytes);
    if (e == hipSuccess) e = hipMemcpy(*dev, h, bytes, hipMemcpyHostToDevice);
    free(h);
    if (e != hipSuccess) return die("upload", hipGetErrorString(e));
    return 0;
}

static int download(const char* dir, const char* name, const void* dev, size_t bytes) {
    void* h = malloc(bytes ? bytes : 1);
    hipError_t e = hipMemcpy(h, dev, bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        free(h);
        return die("download", hipGetErrorString(e));
    }
    const int rc = write_file(dir, name, h, bytes);
    free(h);
    return rc ? die("cannot write output", name) : 0;
}

static int run_prefill(const char* dir) {
    long long B, Hq, Hkv, Sq, Sk, D, causal;
    char path[1024];
    snprintf(path, sizeof(path), "%s/meta", dir);
    FILE* f = fopen(path, "r");
    if (!f || fscanf(f, "%lld %lld %lld %lld %lld %lld %lld", &B, &Hq, &Hkv, &Sq, &Sk, &D, &causal) != 7)
        return die("bad meta", path);
    fclose(f);
    const size_t qb = (size_t)(B * Hq * Sq * D) * 2, kb = (size_t)(B * Hkv * Sk * D) * 2;
    void *q, *k, *v, *o, *lse;
    if (upload(dir, "q.bin", qb, &q) || upload(dir, "k.bin", kb, &k) || upload(dir, "v.bin", kb, &v)) return 1;
    HIP_OK(hipMalloc(&o, qb));
    HIP_OK(hipMalloc(&lse, (size_t)(B * Hq * Sq) * 4));

    dtattn_prefill_args a;
    memset(&a, 0, sizeof(a));
    a.q = q, a.k = k, a.v = v, a.o = o, a.lse = (float*)lse;
    a.B = B, a.Hq = Hq, a.Hkv = Hkv, a.Sq = Sq, a.Sk = Sk, a.D = D, a.Dv = D;
    a.q_stride[0] = Hq * Sq * D, a.q_stride[1] = Sq * D, a.q_stride[2] = D;
    a.k_stride[0] = Hkv * Sk * D, a.k_stride[1] = Sk * D, a.k_stride[2] = D;
    memcpy(a.v_stride, a.k_stride, sizeof(a.k_stride));
    memcpy(a.o_stride, a.q_stride, sizeof(a.q_stride));
    a.lse_stride[0] = Hq * Sq, a.lse_stride[1] = Sq;
    a.dtype = DTATTN_BF16, a.o_dtype = DTATTN_BF16;
    a.scale = nanf("");  /* the default 1/sqrt(D) */
    a.causal = (int32_t)causal;
    /* a head dim above 128 may split its keys when given the workspace this query names */
    const size_t ws_bytes = dtattn_prefill_workspace_size(&a);
    void* ws = NULL;
    if (ws_bytes > 0) {
        HIP_OK(hipMalloc(&ws, ws_bytes));
        a.workspace = ws, a.workspace_bytes = ws_bytes;
    }
    if (dtattn_prefill_fwd(&a, NULL) != DTATTN_OK) return die("dtattn_prefill_fwd", dtattn_last_error());
    HIP_OK(hipDeviceSynchronize());
    if (download(dir, "o.bin", o, qb) || download(dir, "lse.bin", lse, (size_t)(B * Hq * Sq) * 4)) return 1;
    hipFree(q), hipFree(k), hipFree(v), hipFree(o), hipFree(lse);
    if (ws) hipFree(ws);
    return 0;
}

static int run_decode(const char* dir) {
    long long B, Hq, Hkv, Smax, D;
    char path[1024];
    snprintf(path, sizeof(path), "%s/meta", dir);
    FILE* f = fopen(path, "r");
    if (!f || fscanf(f, "%lld %lld %lld %lld %lld", &B, &Hq, &Hkv, &Smax, &D) != 5) return die("bad meta", path);
    fclose(f);
    const size_t qb = (size_t)(B * Hq * D) * 2, kb = (size_t)(B * Hkv * Smax * D) * 2, lb = (size_t)(B * Hq) * 4;
    void *q, *k, *v, *len, *o, *lse;
    if (upload(dir, "q.bin", qb, &q) || upload(dir, "k.bin", kb, &k) || upload(dir, "v.bin", kb, &v) ||
        upload(dir, "lengths.bin", (size_t)B * 4, &len))
        return 1;
    HIP_OK(hipMalloc(&o, qb));
    HIP_OK(hipMalloc(&lse, lb));

    dtattn_decode_args a;
    memset(&a, 0, sizeof(a));
    a.q = q, a.k_cache = k, a.v_cache = v, a.lengths = (const int32_t*)len, a.o = o, a.lse = (float*)lse;
    a.B = B, a.Hq = Hq, a.Hkv = Hkv, a.S_max = Smax, a.D = D;
    a.q_stride[0] = Hq * D, a.q_stride[1] = D;
    a.k_stride[0] = Hkv * Smax * D, a.k_stride[1] = Smax * D, a.k_stride[2] = D;
    memcpy(a.v_stride, a.k_stride, sizeof(a.k_stride));
    memcpy(a.o_stride, a.q_stride, sizeof(a.q_stride));
    a.lse_stride[0] = Hq;
    a.dtype = DTATTN_BF16;
    a.scale = nanf("");
    a.chunk = 0;
    const size_t ws_bytes = dtattn_decode_workspace_size(B, Hq, Smax, D, 0);
    void* ws = NULL;
    HIP_OK(hipMalloc(&ws, ws_bytes));
    a.workspace = ws, a.workspace_bytes = ws_bytes;
    if (dtattn_decode_splitkv(&a, NULL) != DTATTN_OK) return die("dtattn_decode_splitkv", dtattn_last_error());
    HIP_OK(hipDeviceSynchronize());
    if (download(dir, "o.bin", o, qb) || download(dir, "lse.bin", lse, lb)) return 1;
    /* the allocation-free entry point: same arguments, its workspace fields ignored */
    a.workspace = NULL, a.workspace_bytes = 0;
    HIP_OK(hipMemset(o, 0, qb));
    if (dtattn_decode_splitkv_noalloc(&a, NULL) != DTATTN_OK)
        return die("dtattn_decode_splitkv_noalloc", dtattn_last_error());
    HIP_OK(hipDeviceSynchronize());
    if (download(dir, "o_noalloc.bin", o, qb) || download(dir, "lse_noalloc.bin", lse, lb)) return 1;
    hipFree(q), hipFree(k), hipFree(v), hipFree(len), hipFree(o), hipFree(lse), hipFree(ws);
    return 0;
}

int main(int argc, char** argv) {
    if (argc != 3) return die("usage", "abi_client {prefill|decode} DIR");
    if (dtattn_abi_version() != DTATTN_ABI_VERSION) return die("ABI version", "library and header differ");
    if (strcmp(argv[1], "prefill") == 0) return run_prefill(argv[2]);
    if (strcmp(argv[1], "decode") == 0) return run_decode(argv[2]);
    return die("unknown mode", argv[1]);
}
