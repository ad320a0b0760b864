// Does a wave's MFMA work overlap with another wave's VALU work on the same
// SIMD of a gfx950 CU?
//
// Each workgroup has 8 waves; waves 0-3 land on SIMDs 0-3 and run role A,
// waves 4-7 land on SIMDs 0-3 again and run role B.  One workgroup per CU.
// Roles:
//   mfma        2 independent chains of v_mfma_f32_32x32x16_bf16, 8 per iteration
//   mfma-agpr   the same with the accumulators in AGPRs (inline asm)
//   fma64       4 dependent chains of v_fma_f32, 64 per iteration
//   sel48       the scoring kernel's per-row-group energy work: 16 v_fma_f32,
//               16 v_exp_f32, 16 v_add_f32 per iteration
// If the pipes overlapped, "mfma + X" would take max(mfma, X); if they
// serialise it takes the sum.
//
// Measured on one MI355X (two runs, ms): mfma 0.574-0.587, mfma-agpr 0.624-0.688,
// fma64+fma64 0.739-0.768, mfma+fma64 0.981-1.078, mfma+sel48 0.846-0.869.
//
// Build and run (one GPU):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       flashprefillv2-mlx_amd/microbench/mfma_valu_overlap.hip -o /tmp/mfma_valu_overlap
//   /tmp/mfma_valu_overlap
#include <hip/hip_runtime.h>
#include <cstdio>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kIters = 4000;

#define CHECK(call)                                                     \
  do {                                                                  \
    hipError_t err_ = (call);                                           \
    if (err_ != hipSuccess) {                                           \
      fprintf(stderr, "%s: %s\n", #call, hipGetErrorString(err_));      \
      return 1;                                                         \
    }                                                                   \
  } while (0)

enum Role { kIdle = 0, kMfma = 1, kMfmaAgpr = 2, kFma64 = 3, kSel48 = 4 };

__device__ __forceinline__ void work(int role, float seed, float* out) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(seed * (lane + i));
    b[i] = (__bf16)(seed * (lane - i));
  }
  f32x16 acc0 = {}, acc1 = {};
  float x0 = seed * lane, x1 = x0 + 1.f, x2 = x0 + 2.f, x3 = x0 + 3.f, e0 = 0.f, e1 = 0.f;
  if (role == kMfma) {
    for (int it = 0; it < kIters; ++it)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, acc1, 0, 0, 0);
      }
  } else if (role == kMfmaAgpr) {
    for (int it = 0; it < kIters; ++it)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc0) : "v"(a), "v"(b));
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc1) : "v"(b), "v"(a));
      }
  } else if (role == kFma64) {
    for (int it = 0; it < kIters; ++it)
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x0) : "v"(x1), "v"(x2));
        asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x1) : "v"(x2), "v"(x3));
        asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x2) : "v"(x3), "v"(x0));
        asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x3) : "v"(x0), "v"(x1));
      }
  } else if (role == kSel48) {
    for (int it = 0; it < kIters; ++it)
#pragma unroll
      for (int j = 0; j < 16; j += 2) {
        float p0, p1;
        asm volatile("v_fma_f32 %0, %1, %2, %3" : "=v"(p0) : "v"(x1), "v"(x2), "v"(x3));
        asm volatile("v_fma_f32 %0, %1, %2, %3" : "=v"(p1) : "v"(x2), "v"(x3), "v"(x0));
        asm volatile("v_exp_f32 %0, %0" : "+v"(p0));
        asm volatile("v_exp_f32 %0, %0" : "+v"(p1));
        asm volatile("v_add_f32 %0, %0, %1" : "+v"(e0) : "v"(p0));
        asm volatile("v_add_f32 %0, %0, %1" : "+v"(e1) : "v"(p1));
      }
  }
  float r = x0 + x1 + x2 + x3 + e0 + e1;
  for (int i = 0; i < 16; ++i) r += acc0[i] + acc1[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = r;  // grid * 512 floats, allocated below
}

__global__ __launch_bounds__(512) void overlap_kernel(float* out, int role_a, int role_b, float seed) {
  work((threadIdx.x >> 6) < 4 ? role_a : role_b, seed, out);
}

int main() {
  int ncu = 0;
  CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, 0));
  float* out = nullptr;
  CHECK(hipMalloc(&out, size_t(ncu) * 512 * sizeof(float)));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  const char* names[] = {"idle", "mfma", "mfma-agpr", "fma64", "sel48"};
  const int pairs[][2] = {{kMfma, kIdle},  {kMfmaAgpr, kIdle},  {kFma64, kIdle},     {kSel48, kIdle},
                          {kFma64, kFma64}, {kSel48, kSel48},   {kMfma, kMfma},      {kMfma, kFma64},
                          {kMfmaAgpr, kFma64}, {kMfma, kSel48}, {kMfmaAgpr, kSel48}};
  for (const auto& p : pairs) {
    overlap_kernel<<<ncu, 512>>>(out, p[0], p[1], 1e-3f);  // warm-up
    CHECK(hipEventRecord(e0));
    overlap_kernel<<<ncu, 512>>>(out, p[0], p[1], 1e-3f);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    printf("%-10s + %-10s %.4f ms\n", names[p[0]], names[p[1]], ms);
  }
  CHECK(hipFree(out));
  return 0;
}
