// Shared device/host helpers for the gfx950 FPV2 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "fpv2.h"

namespace fpv2 {

// ---------------------------------------------------------------------------
// Host-side error reporting (thread-local message behind fpv2_last_error).
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int status, const char* fmt, ...);
int check_launch(const char* kernel);

// ---------------------------------------------------------------------------
// Vector types.  16-bit element types are carried as raw uint16 bits in
// memory; the MFMA operands are 8-element vectors of the element type.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

// Element traits: memory type, MFMA operand type and conversions.
template <typename T> struct Elem;

template <> struct Elem<bf16_t> {
  typedef bf16x8 vec8;
  static __device__ __forceinline__ float to_float(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
  }
  // float -> bf16, round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
  static __device__ __forceinline__ uint16_t from_float(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Elem<f16_t> {
  typedef f16x8 vec8;
  static __device__ __forceinline__ float to_float(uint16_t b) {
    _Float16 h = __builtin_bit_cast(_Float16, b);
    return static_cast<float>(h);
  }
  static __device__ __forceinline__ uint16_t from_float(float f) {
    _Float16 h = static_cast<_Float16>(f);  // round-to-nearest-even
    return __builtin_bit_cast(uint16_t, h);
  }
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Pack two floats into two 16-bit elements of T (low half = a), RNE.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b);
template <>
__device__ __forceinline__ uint32_t pack2<bf16_t>(float a, float b) {
  const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}
template <>
__device__ __forceinline__ uint32_t pack2<f16_t>(float a, float b) {
  const f16x2 v = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// acc + lo(w) + hi(w) for two packed 16-bit elements of T
// (v_dot2c_f32_bf16 / v_dot2_f32_f16 against (1, 1)).
template <typename T>
__device__ __forceinline__ float add_pair(uint32_t w, float acc);
template <>
__device__ __forceinline__ float add_pair<bf16_t>(uint32_t w, float acc) {
  const bf16x2 one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one, acc, false);
}
template <>
__device__ __forceinline__ float add_pair<f16_t>(uint32_t w, float acc) {
  const f16x2 one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one, acc, false);
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::vec8 as_vec8(u32x4 v) {
  return __builtin_bit_cast(typename Elem<T>::vec8, v);
}

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void store16(void* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

// Raw buffer access.  A resource descriptor covers [base, base + bytes);
// loads at offsets past the range return zeros (hardware range check), so
// masked rows are read branch-free with offset kOOB.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // gfx9-family raw buffer format
constexpr uint32_t kOOB = 0x80000000u;        // any offset >= range reads 0
constexpr int64_t kMaxRsrcBytes = 0x7fffffffLL;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), static_cast<int>(kRsrcWord3));
}
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

// Correct rounding of a double to the 16-bit formats: round to float with
// round-to-odd (sticky bit), then round-to-nearest-even to 16 bits.  The
// double -> float step keeps 13+ guard bits, so the result equals a single
// rounding of the double.
__device__ __forceinline__ float double_to_float_odd(double x) {
  float f = static_cast<float>(x);  // round-to-nearest-even
  double fd = static_cast<double>(f);
  if (__builtin_fabs(fd) > __builtin_fabs(x)) {
    f = __uint_as_float(__float_as_uint(f) - 1u);  // one step toward zero
    fd = static_cast<double>(f);
  }
  if (fd != x && __builtin_isfinite(x)) f = __uint_as_float(__float_as_uint(f) | 1u);
  return f;
}

// ---------------------------------------------------------------------------
// LDS access by inline asm.  The kernels that stream tiles into LDS with
// buffer_load ... lds read those tiles by inline asm.  The compiler cannot tell these
// reads from the asynchronous global->LDS fills of other stages and would
// otherwise wait for all outstanding fills before each stage's first read,
// which serialises the fill latency with the multiply.  Reads complete in
// order; a read's result is valid after lgkm_wait<N>() (s_waitcnt
// lgkmcnt(N)) with N no larger than the number of LDS reads issued after it.
// The wait takes the result registers as operands so that their uses cannot
// be scheduled before it.  A stage is read only after the vmcnt wait and
// the barrier that completed every wave's fills of it.
//
// With ASM = false (used where register pressure is high enough that the
// compiler might spill or copy a register between the asm read and its
// wait) the same reads are ordinary LDS loads and the transposing-read
// builtin, and the compiler places the waits; the waits below are then
// no-ops.
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
template <bool ASM, int OFF>
__device__ __forceinline__ u32x4 lds_read_b128(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field is 16 bits");
  if constexpr (ASM) {
    u32x4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
  } else {
    return *reinterpret_cast<const lds_u32x4*>(static_cast<uintptr_t>(addr + OFF));
  }
}
template <bool ASM, int N>
__device__ __forceinline__ void lgkm_wait(u32x4& r) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt is 4 bits");
  if constexpr (ASM) asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(r) : "i"(N));
}
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  // vmcnt(N) expcnt(7) lgkmcnt(15): vmcnt bits [3:0] and [15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)(p)));
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [0, N).
template <int I, int N>
struct StaticFor {
  template <typename F>
  static __device__ __forceinline__ void run(F&& f) {
    if constexpr (I < N) {
      f(std::integral_constant<int, I>{});
      StaticFor<I + 1, N>::run(f);
    }
  }
};

}  // namespace fpv2
