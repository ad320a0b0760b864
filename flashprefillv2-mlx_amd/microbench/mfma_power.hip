// Sustained bf16 MFMA rate and shader clock of a gfx950 chip running nothing
// but MFMAs, for the two MFMA shapes an attention kernel can be built on:
//   32x32x16  v_mfma_f32_32x32x16_bf16 (16 accumulators per lane)
//   16x16x32  v_mfma_f32_16x16x32_bf16 (4 accumulators per lane)
// each with constant operands and with 8 operand pairs of random bf16 data
// (N(0,1)-like) cycled from MFMA to MFMA, so the inputs change like real data
// without any VALU work; then the random case with the attention slice's VALU
// work interleaved (29 VALU per 8 32x32x16 MFMAs or 16 16x16x32 MFMAs).  Two waves per SIMD (one 512-thread workgroup per
// CU), independent accumulator chains keeping the matrix pipe full, about
// 0.2 s per launch so the power management settles.
//
// The clock is s_memtime (shader cycles) over s_memrealtime (100 MHz) across
// each wave's loop, averaged over the waves.
//
// Measured on one MI355X (two runs; % of the 2.5 PFLOP/s dense bf16 peak):
//   32x32x16 constant / random           70-71 % at 1.74-1.78 GHz
//   16x16x32 constant / random           80-81 % at 1.98-2.01 GHz
//   32x32x16 random + the slice's VALU   58.2-58.5 % at 1.98 GHz
//   16x16x32 random + the slice's VALU   60.1-60.2 % at 2.30 GHz
//   32x32x16 f16 random                  68.1-68.2 % at 1.73-1.74 GHz
//   32x32x16 f16 random + slice VALU     55.5-55.7 % at 1.89-1.90 GHz
//     (bf16 in the same runs: 69.8-70.4 %, and 57.1 % at 1.94-1.95 GHz)
// The chip is power-limited with the matrix pipe full: the 16x16x32 shape
// draws less power per FLOP and runs 13 % faster, random operands cost
// about 1 %, and the f16 MFMA about 3 % more than the bf16 one (its
// operands here carry bf16's 8 significant bits).  With the VALU work interleaved the 16x16x32 loop runs at a
// higher clock but keeps the pipe busy for fewer of its cycles (63 % against
// 71 %), and the difference shrinks to 3 %.
//
// Build and run (one GPU):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       flashprefillv2-mlx_amd/microbench/mfma_power.hip -o /tmp/mfma_power
//   /tmp/mfma_power
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

#define CHECK(call)                                                     \
  do {                                                                  \
    hipError_t err_ = (call);                                           \
    if (err_ != hipSuccess) {                                           \
      fprintf(stderr, "%s: %s\n", #call, hipGetErrorString(err_));      \
      return 1;                                                         \
    }                                                                   \
  } while (0)

// A roughly N(0,1) value from a 32-bit hash (sum of four uniforms, centred).
__device__ __forceinline__ float hash_normal(uint32_t x) {
  float s = 0.f;
  for (int i = 0; i < 4; ++i) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    s += static_cast<float>(x >> 8) * (1.f / 16777216.f);
  }
  return (s - 2.f) * 1.732f;
}

// The attention kernel's VALU work per 16 of its 32x32x16 MFMAs (one 32-key
// slice of one wave), half of it per call: 8 v_fma_f32 + 8 v_exp_f32 (the
// exp2 of the logits), 4 v_cvt_pk_bf16_f32, 4 v_dot2c_f32_bf16 (the row sum
// of the packed P), 5 v_xor_b32 (LDS address swizzles).  Independent of the
// MFMA results, as the kernel's exps work on the previous slice.
__device__ __forceinline__ void slice_valu_half(float (&x)[8], uint32_t& w, float& l, uint32_t& adr, int k) {
  float p = x[k];
  asm volatile("v_fma_f32 %0, %1, %2, %3" : "=v"(p) : "v"(x[k]), "v"(x[(k + 1) & 7]), "v"(x[(k + 2) & 7]));
  asm volatile("v_exp_f32 %0, %0" : "+v"(p));
  x[k] = p;
  if (k & 1) {
    asm volatile("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(w) : "v"(x[k - 1]), "v"(x[k]));
    asm volatile("v_dot2c_f32_bf16 %0, %1, %2" : "+v"(l) : "v"(w), "v"(0x3f803f80u));
  }
  if (k < 5) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(adr) : "v"(x[k]));
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// SHAPE 0: 32x32x16 (4 chains), 1: 16x16x32 (8 chains), 2: 32x32x16 f16
// (v_mfma_f32_32x32x16_f16, operands converted from the same random data).  RANDOM: cycle 8
// operand pairs of random data, else one constant pair.  MIX: the attention
// slice's VALU work (slice_valu_half per 8 32x32x16-equivalents) interleaved
// with the MFMAs in the same wave.
template <int SHAPE, bool RANDOM, bool MIX = false>
__global__ __launch_bounds__(512) void mfma_loop(float* out, unsigned long long* ticks, int iters, uint32_t seed) {
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * 8 + (threadIdx.x >> 6);
  bf16x8 a[8], b[8];
  for (int p = 0; p < 8; ++p)
    for (int i = 0; i < 8; ++i) {
      const uint32_t h = seed + (gw * 64 + lane) * 131u + (RANDOM ? p : 0) * 17u + i;
      a[p][i] = (__bf16)hash_normal(h);
      b[p][i] = (__bf16)hash_normal(h ^ 0x9e3779b9u);
    }
  float r = 0.f;
  float x[8];
  for (int i = 0; i < 8; ++i) x[i] = 1e-3f * (lane + i);
  uint32_t w = 0, adr = lane;
  float l = 0.f;
  unsigned long long c0, c1, t0, t1;
  if constexpr (SHAPE == 0) {
    f32x16 acc[4] = {};
    t0 = __builtin_amdgcn_s_memrealtime();
    c0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        acc[k & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[k], b[k], acc[k & 3], 0, 0, 0);
        if constexpr (MIX) slice_valu_half(x, w, l, adr, k);
      }
    }
    c1 = __builtin_amdgcn_s_memtime();
    t1 = __builtin_amdgcn_s_memrealtime();
    for (int c = 0; c < 4; ++c)
      for (int i = 0; i < 16; ++i) r += acc[c][i];
  } else if constexpr (SHAPE == 2) {
    f16x8 ah[8], bh[8];
    for (int p = 0; p < 8; ++p)
      for (int i = 0; i < 8; ++i) {
        ah[p][i] = (_Float16)(float)a[p][i];
        bh[p][i] = (_Float16)(float)b[p][i];
      }
    f32x16 acc[4] = {};
    t0 = __builtin_amdgcn_s_memrealtime();
    c0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        acc[k & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[k], bh[k], acc[k & 3], 0, 0, 0);
        if constexpr (MIX) slice_valu_half(x, w, l, adr, k);
      }
    }
    c1 = __builtin_amdgcn_s_memtime();
    t1 = __builtin_amdgcn_s_memrealtime();
    for (int c = 0; c < 4; ++c)
      for (int i = 0; i < 16; ++i) r += acc[c][i];
  } else {
    f32x4 acc[8] = {};
    t0 = __builtin_amdgcn_s_memrealtime();
    c0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        acc[k & 7] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[k & 7], b[k & 7], acc[k & 7], 0, 0, 0);
        if constexpr (MIX) {
          if (k & 1) slice_valu_half(x, w, l, adr, k >> 1);
        }
      }
    }
    c1 = __builtin_amdgcn_s_memtime();
    t1 = __builtin_amdgcn_s_memrealtime();
    for (int c = 0; c < 8; ++c)
      for (int i = 0; i < 4; ++i) r += acc[c][i];
  }
  for (int i = 0; i < 8; ++i) r += x[i];
  r += l + static_cast<float>(w ^ adr);
  out[blockIdx.x * 512 + threadIdx.x] = r;  // grid * 512 floats
  if (lane == 0) {
    ticks[2 * gw] = c1 - c0;   // grid * 8 waves * 2 entries
    ticks[2 * gw + 1] = t1 - t0;
  }
}

template <int SHAPE, bool RANDOM, bool MIX = false>
int run(int ncu, float* out, unsigned long long* ticks, const char* name) {
  // FLOP per wave per iteration: 8 x 32x32x16 or 16 x 16x16x32 MFMAs, each
  // loop iteration 8 * 32768 = 16 * 16384 = 262144 FLOP.
  const int iters = 300000;
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  mfma_loop<SHAPE, RANDOM, MIX><<<ncu, 512>>>(out, ticks, iters / 8, 1u);  // warm-up
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(e0));
  mfma_loop<SHAPE, RANDOM, MIX><<<ncu, 512>>>(out, ticks, iters, 1u);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  std::vector<unsigned long long> h(size_t(ncu) * 16);
  CHECK(hipMemcpy(h.data(), ticks, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost));
  double ghz = 0.0;
  for (int w = 0; w < ncu * 8; ++w) ghz += double(h[2 * w]) / double(h[2 * w + 1]) * 0.1;
  ghz /= ncu * 8;
  const double flop = double(ncu) * 8 * iters * 262144.0;
  printf("%-22s %8.2f ms  %7.1f TFLOP/s  %5.1f %% of 2.5 PF  clock %.3f GHz\n", name, ms, flop / ms / 1e9,
         flop / ms / 1e9 / 2516.6 * 100, ghz);
  return 0;
}

int main() {
  int ncu = 0;
  CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, 0));
  float* out = nullptr;
  unsigned long long* ticks = nullptr;
  CHECK(hipMalloc(&out, size_t(ncu) * 512 * sizeof(float)));
  CHECK(hipMalloc(&ticks, size_t(ncu) * 16 * sizeof(unsigned long long)));
  for (int rep = 0; rep < 2; ++rep) {
    if (run<0, false>(ncu, out, ticks, "32x32x16 constant")) return 1;
    if (run<0, true>(ncu, out, ticks, "32x32x16 random")) return 1;
    if (run<1, false>(ncu, out, ticks, "16x16x32 constant")) return 1;
    if (run<1, true>(ncu, out, ticks, "16x16x32 random")) return 1;
    if (run<0, true, true>(ncu, out, ticks, "32x32x16 random + VALU")) return 1;
    if (run<1, true, true>(ncu, out, ticks, "16x16x32 random + VALU")) return 1;
    if (run<2, true>(ncu, out, ticks, "32x32x16 f16 random")) return 1;
    if (run<2, true, true>(ncu, out, ticks, "32x32x16 f16 rnd + VALU")) return 1;
  }
  CHECK(hipFree(out));
  CHECK(hipFree(ticks));
  return 0;
}
