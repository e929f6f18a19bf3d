// Probe: issue cost of matrix-core (MFMA) and vector-ALU instructions on
// gfx950, alone and interleaved, at W waves per SIMD (one workgroup of 4W
// waves per CU, every CU). Each wave runs `iters` iterations of NM MFMAs on
// eight independent accumulators and NV dependent-pair FP32 FMAs, NM/GRP
// groups of GRP MFMAs alternating with their share of the FMAs; the printed
// figure is SIMD cycles (clock64) per wave-iteration. FP32 MFMAs and VALU
// instructions add up (no co-execution); BF16/F16 4x4x4 overlap partly.
// Built and run by compressed-kv-attention_amd/probes.py.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_)); exit(1); } } while (0)
typedef float f4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// MK: 0 none, 1 f32 4x4x1, 2 bf16 4x4x4, 3 f16 4x4x4, 4 bf16 16x16x16 (f4 acc), 5 f32 16x16x4
template <int MK, int NM, int NV, int GRP>
__global__ void kern(long long *cyc, float *out, int iters) {
    float a = threadIdx.x * 1e-3f, b = blockIdx.x * 1e-3f;
    s4 sa = {1, 2, 3, 4}, sb = {5, 6, 7, 8};
    h4 ha = {1, 2, 3, 4}, hb = {5, 6, 7, 8};
    typedef short s8 __attribute__((ext_vector_type(8)));
    s8 ta = {1, 2, 3, 4, 5, 6, 7, 8};
    f4 acc[8];
    for (int j = 0; j < 8; ++j) acc[j] = f4{0, 0, 0, 0};
    float v[16];
    for (int j = 0; j < 16; ++j) v[j] = a + j;
    __syncthreads();
    long long t0 = clock64();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < NM; ++j) {
            if constexpr (MK == 1) acc[j % 8] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, acc[j % 8], 4, 0, 0);
            if constexpr (MK == 2) acc[j % 8] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(sa, sb, acc[j % 8], 4, 0, 0);
            if constexpr (MK == 3) acc[j % 8] = __builtin_amdgcn_mfma_f32_4x4x4f16(ha, hb, acc[j % 8], 4, 0, 0);
            if constexpr (MK == 4) acc[j % 8] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ta, ta, acc[j % 8], 0, 0, 0);
            if constexpr (MK == 5) acc[j % 8] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[j % 8], 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) v[j % 16] = fmaf(v[j % 16], (j & 1) ? b : a, (j & 1) ? a : b);
        if constexpr (NM > 0 && NV > 0) {
#pragma unroll
            for (int j = 0; j < NM / GRP; ++j) {
                __builtin_amdgcn_sched_group_barrier(0x008, GRP, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, NV * GRP / NM, 0);
            }
        }
    }
    long long t1 = clock64();
    __shared__ long long mx[16], mn[16];
    if (threadIdx.x % 64 == 0) { mx[threadIdx.x / 64] = t1; mn[threadIdx.x / 64] = t0; }
    __syncthreads();
    if (threadIdx.x == 0) {
        long long hi = mx[0], lo = mn[0];
        for (int w = 1; w < blockDim.x / 64; ++w) { hi = mx[w] > hi ? mx[w] : hi; lo = mn[w] < lo ? mn[w] : lo; }
        cyc[blockIdx.x] = hi - lo;
    }
    float s = 0;
    for (int j = 0; j < 16; ++j) s += v[j];
    for (int j = 0; j < 8; ++j) s += acc[j][0];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}
const char *mk[] = {"none", "f32 4x4x1", "bf16 4x4x4", "f16 4x4x4", "bf16 16x16x32", "f32 16x16x4"};
template <int MK, int NM, int NV, int GRP>
void run(long long *c, float *d, int W, int cus) {
    const int iters = 400;
    hipLaunchKernelGGL((kern<MK, NM, NV, GRP>), dim3(cus), dim3(256 * W), 0, 0, c, d, iters);
    hipLaunchKernelGGL((kern<MK, NM, NV, GRP>), dim3(cus), dim3(256 * W), 0, 0, c, d, iters);
    CK(hipGetLastError());
    static long long h[1024];
    CK(hipMemcpy(h, c, sizeof(long long) * cus, hipMemcpyDeviceToHost));
    double s = 0;
    for (int i = 0; i < cus; ++i) s += h[i];
    printf("%-14s %2d mfma + %2d valu (grp %d) W=%d: %7.1f SIMD cycles per wave-iteration\n", mk[MK], NM, NV, GRP, W,
           s / cus / iters / W);
}
template <int MK> void mix(long long *c, float *d, int cus) {
    for (int W : {2, 4}) {
        run<MK, 16, 0, 1>(c, d, W, cus);
        run<MK, 16, 32, 4>(c, d, W, cus);
        run<MK, 16, 32, 1>(c, d, W, cus);
    }
}
int main() {
    setvbuf(stdout, NULL, _IONBF, 0);
    int cus = 0;
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    if (cus > 1024) cus = 1024;
    long long *c; float *d;
    CK(hipMalloc(&c, sizeof(long long) * 1024));
    CK(hipMalloc(&d, sizeof(float) * 1024 * 1024));
    for (int W : {2, 4}) run<0, 0, 32, 1>(c, d, W, cus);
    mix<1>(c, d, cus); mix<2>(c, d, cus); mix<3>(c, d, cus); mix<5>(c, d, cus);
    for (int W : {2, 4}) { run<4, 4, 0, 1>(c, d, W, cus); run<4, 4, 32, 1>(c, d, W, cus); }
    return 0;
}
