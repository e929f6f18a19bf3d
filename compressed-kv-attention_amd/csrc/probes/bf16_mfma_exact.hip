// Probe: is v_mfma_f32_4x4x4_16b_bf16 with one live K slot (A's other
// slots 0) the same operation as fmaf(a, b, c) on the BF16 inputs widened to
// FP32? (It would let the score products run on the BF16 matrix path, which
// overlaps the vector ALU in part.) Inputs from files, outputs to files, the
// comparison in compressed-kv-attention_amd/probes.py.
//   bf16_mfma_exact DIR N_WAVES SLOT
// DIR/a.bin: N_WAVES*64*4 uint16 (A lanes), b.bin same (B lanes), c.bin N_WAVES*64*4 float (C, lane 4b+j reg i)
// writes DIR/mfma.bin and DIR/ref.bin (N_WAVES*64*4 float each)
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
typedef float f4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));

__global__ void k_mfma(const short *A, const short *B, const float *C, float *D, int n_waves) {
    const int w = blockIdx.x;
    if (w >= n_waves) return;
    const int l = threadIdx.x;
    const size_t o = (size_t(w) * 64 + l) * 4;
    s4 a = {A[o], A[o + 1], A[o + 2], A[o + 3]};
    s4 b = {B[o], B[o + 1], B[o + 2], B[o + 3]};
    f4 c = {C[o], C[o + 1], C[o + 2], C[o + 3]};
    f4 d = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 0, 0, 0);
    D[o] = d.x; D[o + 1] = d.y; D[o + 2] = d.z; D[o + 3] = d.w;
}

__device__ float bf(short s) { return __uint_as_float(uint32_t(uint16_t(s)) << 16); }

// reference: D[lane 4b+j][i] = fmaf(A[4b+i][s], B[4b+j][s], C[4b+j][i])
__global__ void k_ref(const short *A, const short *B, const float *C, float *D, int n_waves, int s) {
    const int w = blockIdx.x;
    if (w >= n_waves) return;
    const int l = threadIdx.x, b = l / 4, j = l % 4;
    for (int i = 0; i < 4; ++i) {
        const float a = bf(A[(size_t(w) * 64 + 4 * b + i) * 4 + s]);
        const float bb = bf(B[(size_t(w) * 64 + 4 * b + j) * 4 + s]);
        const float c = C[(size_t(w) * 64 + l) * 4 + i];
        D[(size_t(w) * 64 + l) * 4 + i] = fmaf(a, bb, c);
    }
}

template <class T> std::vector<T> rd(const char *dir, const char *name, size_t n) {
    char p[512]; snprintf(p, sizeof p, "%s/%s", dir, name);
    FILE *f = fopen(p, "rb"); if (!f) { perror(p); exit(2); }
    std::vector<T> v(n); if (fread(v.data(), sizeof(T), n, f) != n) { fprintf(stderr, "short %s\n", p); exit(2); }
    fclose(f); return v;
}
void wr(const char *dir, const char *name, const std::vector<float> &v) {
    char p[512]; snprintf(p, sizeof p, "%s/%s", dir, name);
    FILE *f = fopen(p, "wb"); fwrite(v.data(), 4, v.size(), f); fclose(f);
}
#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e)); exit(1); } } while (0)
int main(int argc, char **argv) {
    const char *dir = argv[1]; const int nw = atoi(argv[2]); const int s = atoi(argv[3]);
    const size_t n = size_t(nw) * 256;
    auto A = rd<short>(dir, "a.bin", n), B = rd<short>(dir, "b.bin", n);
    auto C = rd<float>(dir, "c.bin", n);
    short *dA, *dB; float *dC, *dD, *dR;
    CK(hipMalloc(&dA, n * 2)); CK(hipMalloc(&dB, n * 2)); CK(hipMalloc(&dC, n * 4));
    CK(hipMalloc(&dD, n * 4)); CK(hipMalloc(&dR, n * 4));
    CK(hipMemcpy(dA, A.data(), n * 2, hipMemcpyHostToDevice));
    CK(hipMemcpy(dB, B.data(), n * 2, hipMemcpyHostToDevice));
    CK(hipMemcpy(dC, C.data(), n * 4, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(k_mfma, dim3(nw), dim3(64), 0, 0, dA, dB, dC, dD, nw);
    hipLaunchKernelGGL(k_ref, dim3(nw), dim3(64), 0, 0, dA, dB, dC, dR, nw, s);
    CK(hipDeviceSynchronize());
    std::vector<float> D(n), R(n);
    CK(hipMemcpy(D.data(), dD, n * 4, hipMemcpyDeviceToHost));
    CK(hipMemcpy(R.data(), dR, n * 4, hipMemcpyDeviceToHost));
    wr(dir, "mfma.bin", D); wr(dir, "ref.bin", R);
    printf("bfexact: %d waves slot %d done\n", nw, s);
    return 0;
}
