// Decoder-layer operations of the end-to-end prefill harness: residual add +
// RMSNorm, per-head Q/K RMSNorm + rotary embedding, SwiGLU gate.  They stand
// in for mlx-lm's fused mx.fast.rms_norm / mx.fast.rope kernels that the
// reference's end-to-end runs use (README.md:30-46, external dependency).
//
// All three are HBM-bound streaming kernels: each element is read once and
// written once (the norm re-reads its own row, which it has just touched, from
// cache).  16-byte vector accesses along rows; float32 arithmetic; one
// rounding to the storage type per stored value.
#include "fpv2_common.h"
#include "fpv2_decoder.h"

namespace fpv2 {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormVecs = FPV2_MAX_NORM_COLS / 8 / kNormThreads;  // 16-byte vectors per thread

template <typename T>
__device__ __forceinline__ float lo_f(uint32_t w) { return Elem<T>::to_float(w & 0xffffu); }
template <typename T>
__device__ __forceinline__ float hi_f(uint32_t w) { return Elem<T>::to_float(w >> 16); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

struct NormArgs {
  uint16_t* x;
  const uint16_t* delta;
  const uint16_t* weight;
  uint16_t* y;
  int64_t cols;
  int64_t x_stride, d_stride, y_stride;
  float eps;
};

// One workgroup per row.  Thread t owns the 16-byte vectors t, t + 256, ...
// of the row and keeps them in registers between the two passes.
template <typename T>
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(NormArgs a) {
  __shared__ float partial[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nvec = static_cast<int>(a.cols / 8);
  uint16_t* x = a.x + row * a.x_stride;
  const uint16_t* d = a.delta ? a.delta + row * a.d_stride : nullptr;
  u32x4 xv[kNormVecs];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kNormVecs; ++i) {
    const int c = tid + i * kNormThreads;
    if (c < nvec) {
      u32x4 v = *reinterpret_cast<const u32x4*>(x + 8 * c);
      if (d != nullptr) {
        const u32x4 dv = *reinterpret_cast<const u32x4*>(d + 8 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[j] = pack2<T>(lo_f<T>(v[j]) + lo_f<T>(dv[j]), hi_f<T>(v[j]) + hi_f<T>(dv[j]));
        *reinterpret_cast<u32x4*>(x + 8 * c) = v;
      }
      xv[i] = v;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float l = lo_f<T>(v[j]), h = hi_f<T>(v[j]);
        ss += l * l + h * h;
      }
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) partial[tid >> 6] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; ++w) total += partial[w];
  const float r = rsqrtf(total / static_cast<float>(a.cols) + a.eps);
  uint16_t* y = a.y + row * a.y_stride;
#pragma unroll
  for (int i = 0; i < kNormVecs; ++i) {
    const int c = tid + i * kNormThreads;
    if (c < nvec) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(a.weight + 8 * c);
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack2<T>(lo_f<T>(xv[i][j]) * r * lo_f<T>(w[j]),
                        hi_f<T>(xv[i][j]) * r * hi_f<T>(w[j]));
      *reinterpret_cast<u32x4*>(y + 8 * c) = o;
    }
  }
}

struct RopeArgs {
  const uint16_t* qkv;
  const uint16_t* qw;
  const uint16_t* kw;
  const float* cos;
  const float* sin;
  uint16_t* q_out;
  uint16_t* k_out;
  uint16_t* v_out;  // null: no V heads
  int64_t rows;
  int64_t qkv_stride;
  int64_t q_hs, q_rs;    // q_out head / row strides
  int64_t kv_hs, kv_rs;  // k_out and v_out head / row strides
  int qh, kh, d;
  float eps;
};

// Sixteen lanes per (row, head) item, four items per wave: the query and key
// heads are normalised and rotated, the value heads (when v_out is given) are
// copied.  Lane s of a group handles the element quads j = 4 (s + 16 p) of
// the first half and their rotation partners j + D/2 (8-byte loads of the
// head, 16-byte loads of the float32 tables).
template <typename T>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(RopeArgs a) {
  const int sub = threadIdx.x & 15;
  const int heads = a.qh + a.kh + (a.v_out != nullptr ? a.kh : 0);
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const bool valid = item < a.rows * heads;  // a group past the end computes nothing
  const int64_t row = valid ? item / heads : 0;
  const int h = valid ? static_cast<int>(item - row * heads) : 0;
  const int half = a.d / 2;
  const int quads = half / 4;
  const int kind = h < a.qh ? 0 : (h < a.qh + a.kh ? 1 : 2);  // q, k, v
  const uint16_t* src = a.qkv + row * a.qkv_stride + static_cast<int64_t>(h) * a.d;
  const uint16_t* w = kind == 0 ? a.qw : a.kw;
  uint16_t* dst = kind == 0 ? a.q_out + row * a.q_rs + h * a.q_hs
                : kind == 1 ? a.k_out + row * a.kv_rs + (h - a.qh) * a.kv_hs
                            : a.v_out + row * a.kv_rs + (h - a.qh - a.kh) * a.kv_hs;
  u32x2 x1[2] = {}, x2[2] = {};
  float ss = 0.f;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int qd = sub + 16 * p;
    if (valid && qd < quads) {
      x1[p] = *reinterpret_cast<const u32x2*>(src + 4 * qd);
      x2[p] = *reinterpret_cast<const u32x2*>(src + 4 * qd + half);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float a1 = lo_f<T>(x1[p][j]), b1 = hi_f<T>(x1[p][j]);
        const float a2 = lo_f<T>(x2[p][j]), b2 = hi_f<T>(x2[p][j]);
        ss += a1 * a1 + b1 * b1 + a2 * a2 + b2 * b2;
      }
    }
  }
  // the four groups of a wave reduce together; each keeps its own sum
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if (kind == 2) {  // value head: copy
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int qd = sub + 16 * p;
      if (valid && qd < quads) {
        *reinterpret_cast<u32x2*>(dst + 4 * qd) = x1[p];
        *reinterpret_cast<u32x2*>(dst + 4 * qd + half) = x2[p];
      }
    }
    return;
  }
  const float r = rsqrtf(ss / static_cast<float>(a.d) + a.eps);
  const float* cs = a.cos + row * a.d;
  const float* sn = a.sin + row * a.d;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int qd = sub + 16 * p;
    if (valid && qd < quads) {
      const int j0 = 4 * qd;
      const u32x2 w1 = *reinterpret_cast<const u32x2*>(w + j0);
      const u32x2 w2 = *reinterpret_cast<const u32x2*>(w + j0 + half);
      const f32x4 c1 = *reinterpret_cast<const f32x4*>(cs + j0);
      const f32x4 c2 = *reinterpret_cast<const f32x4*>(cs + j0 + half);
      const f32x4 s1 = *reinterpret_cast<const f32x4*>(sn + j0);
      const f32x4 s2 = *reinterpret_cast<const f32x4*>(sn + j0 + half);
      float n1[4], n2[4];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        // the norm's output is stored in T before the rotation reads it
        const uint32_t m1 = pack2<T>(lo_f<T>(x1[p][j]) * r * lo_f<T>(w1[j]),
                                     hi_f<T>(x1[p][j]) * r * hi_f<T>(w1[j]));
        const uint32_t m2 = pack2<T>(lo_f<T>(x2[p][j]) * r * lo_f<T>(w2[j]),
                                     hi_f<T>(x2[p][j]) * r * hi_f<T>(w2[j]));
        n1[2 * j] = lo_f<T>(m1);
        n1[2 * j + 1] = hi_f<T>(m1);
        n2[2 * j] = lo_f<T>(m2);
        n2[2 * j + 1] = hi_f<T>(m2);
      }
      u32x2 o1, o2;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int e = 2 * j;
        o1[j] = pack2<T>(n1[e] * c1[e] - n2[e] * s1[e], n1[e + 1] * c1[e + 1] - n2[e + 1] * s1[e + 1]);
        o2[j] = pack2<T>(n2[e] * c2[e] + n1[e] * s2[e], n2[e + 1] * c2[e + 1] + n1[e + 1] * s2[e + 1]);
      }
      *reinterpret_cast<u32x2*>(dst + j0) = o1;
      *reinterpret_cast<u32x2*>(dst + j0 + half) = o2;
    }
  }
}

struct SiluArgs {
  const uint16_t* gu;
  uint16_t* out;
  int64_t rows, nvec, cols;
  int64_t in_stride, out_stride;
};

__device__ __forceinline__ float silu(float g) { return g / (1.f + __expf(-g)); }

template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(SiluArgs a) {
  const int64_t total = a.rows * a.nvec;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t row = t / a.nvec;
    const int64_t c = t - row * a.nvec;
    const uint16_t* g = a.gu + row * a.in_stride + 8 * c;
    const u32x4 gv = *reinterpret_cast<const u32x4*>(g);
    const u32x4 uv = *reinterpret_cast<const u32x4*>(g + a.cols);
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack2<T>(silu(lo_f<T>(gv[j])) * lo_f<T>(uv[j]), silu(hi_f<T>(gv[j])) * hi_f<T>(uv[j]));
    *reinterpret_cast<u32x4*>(a.out + row * a.out_stride + 8 * c) = o;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace fpv2

extern "C" int fpv2_add_rms_norm(void* x, const void* delta, const void* weight, void* y,
                                 int dtype, int64_t rows, int64_t cols, int64_t x_row_stride,
                                 int64_t delta_row_stride, int64_t y_row_stride, float eps,
                                 void* stream) {
  using namespace fpv2;
  if (dtype != FPV2_BF16 && dtype != FPV2_F16)
    return fail(FPV2_ERR_UNSUPPORTED, "fpv2_add_rms_norm: dtype must be bf16 or f16");
  if (x == nullptr || weight == nullptr || y == nullptr)
    return fail(FPV2_ERR_ARGUMENT, "fpv2_add_rms_norm: null pointer");
  if (y == x || y == delta)
    return fail(FPV2_ERR_ARGUMENT, "fpv2_add_rms_norm: y must not alias x or delta");
  if (rows < 0 || cols <= 0 || cols % 8 || cols > FPV2_MAX_NORM_COLS)
    return fail(FPV2_ERR_ARGUMENT, "fpv2_add_rms_norm: cols must be a positive multiple of 8 "
                "and at most %d", FPV2_MAX_NORM_COLS);
  if (x_row_stride < cols || y_row_stride < cols || x_row_stride % 8 || y_row_stride % 8 ||
      (delta && (delta_row_stride < cols || delta_row_stride % 8)))
    return fail(FPV2_ERR_ARGUMENT, "fpv2_add_rms_norm: row strides must be multiples of 8 "
                "and at least cols");
  if (!aligned16(x) || !aligned16(weight) || !aligned16(y) || (delta && !aligned16(delta)))
    return fail(FPV2_ERR_ARGUMENT, "fpv2_add_rms_norm: pointers must be 16-byte aligned");
  if (rows == 0) return FPV2_OK;
  if (rows > 0x7fffffff) return fail(FPV2_ERR_ARGUMENT, "fpv2_add_rms_norm: too many rows");
  NormArgs a{static_cast<uint16_t*>(x), static_cast<const uint16_t*>(delta),
             static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(y), cols,
             x_row_stride, delta_row_stride, y_row_stride, eps};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == FPV2_BF16)
    hipLaunchKernelGGL(add_rms_norm_kernel<bf16_t>, dim3(rows), dim3(kNormThreads), 0, s, a);
  else
    hipLaunchKernelGGL(add_rms_norm_kernel<f16_t>, dim3(rows), dim3(kNormThreads), 0, s, a);
  return check_launch("add_rms_norm_kernel");
}

extern "C" int fpv2_qk_norm_rope(const void* qkv, const void* q_weight, const void* k_weight,
                                 const float* cos, const float* sin, void* q_out, void* k_out,
                                 void* v_out, int dtype, int64_t rows, int64_t query_heads,
                                 int64_t kv_heads, int64_t head_dim, int64_t qkv_row_stride,
                                 int64_t q_head_stride, int64_t q_row_stride,
                                 int64_t kv_head_stride, int64_t kv_row_stride, float eps,
                                 void* stream) {
  using namespace fpv2;
  const auto a8 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; };
  if (dtype != FPV2_BF16 && dtype != FPV2_F16)
    return fail(FPV2_ERR_UNSUPPORTED, "fpv2_qk_norm_rope: dtype must be bf16 or f16");
  if (!qkv || !q_weight || !k_weight || !cos || !sin || !q_out || !k_out)
    return fail(FPV2_ERR_ARGUMENT, "fpv2_qk_norm_rope: null pointer");
  if (head_dim <= 0 || head_dim % 8 || head_dim > 256)
    return fail(FPV2_ERR_ARGUMENT,
                "fpv2_qk_norm_rope: head_dim must be a multiple of 8 and at most 256");
  if (rows < 0 || query_heads <= 0 || kv_heads <= 0 || query_heads + 2 * kv_heads > 4096)
    return fail(FPV2_ERR_ARGUMENT, "fpv2_qk_norm_rope: bad rows or head counts");
  const int64_t in_heads = query_heads + kv_heads + (v_out ? kv_heads : 0);
  if (qkv_row_stride < in_heads * head_dim)
    return fail(FPV2_ERR_ARGUMENT, "fpv2_qk_norm_rope: qkv rows are shorter than the heads read");
  if (qkv_row_stride % 4 || q_head_stride % 4 || q_row_stride % 4 || kv_head_stride % 4 ||
      kv_row_stride % 4 || q_head_stride < head_dim || kv_head_stride < head_dim ||
      q_row_stride <= 0 || kv_row_stride <= 0)
    return fail(FPV2_ERR_ARGUMENT, "fpv2_qk_norm_rope: strides must be positive multiples of 4 "
                "and head strides at least head_dim");
  if (!a8(qkv) || !aligned16(cos) || !aligned16(sin) || !a8(q_weight) || !a8(k_weight) ||
      !a8(q_out) || !a8(k_out) || (v_out && !a8(v_out)))
    return fail(FPV2_ERR_ARGUMENT, "fpv2_qk_norm_rope: qkv, weights and outputs must be 8-byte "
                "aligned, cos and sin 16-byte aligned");
  if (rows == 0) return FPV2_OK;
  const int64_t items = rows * in_heads;
  const int64_t groups = (items + 15) / 16;  // 16 (row, head) items per workgroup
  if (groups > 0x7fffffff) return fail(FPV2_ERR_ARGUMENT, "fpv2_qk_norm_rope: too many rows");
  RopeArgs a{static_cast<const uint16_t*>(qkv), static_cast<const uint16_t*>(q_weight),
             static_cast<const uint16_t*>(k_weight), cos, sin, static_cast<uint16_t*>(q_out),
             static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(v_out), rows, qkv_row_stride,
             q_head_stride, q_row_stride, kv_head_stride, kv_row_stride,
             static_cast<int>(query_heads), static_cast<int>(kv_heads),
             static_cast<int>(head_dim), eps};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == FPV2_BF16)
    hipLaunchKernelGGL(qk_norm_rope_kernel<bf16_t>, dim3(groups), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(qk_norm_rope_kernel<f16_t>, dim3(groups), dim3(256), 0, s, a);
  return check_launch("qk_norm_rope_kernel");
}

extern "C" int fpv2_silu_mul(const void* gate_up, void* out, int dtype, int64_t rows,
                             int64_t cols, int64_t in_row_stride, int64_t out_row_stride,
                             void* stream) {
  using namespace fpv2;
  if (dtype != FPV2_BF16 && dtype != FPV2_F16)
    return fail(FPV2_ERR_UNSUPPORTED, "fpv2_silu_mul: dtype must be bf16 or f16");
  if (!gate_up || !out) return fail(FPV2_ERR_ARGUMENT, "fpv2_silu_mul: null pointer");
  if (rows < 0 || cols <= 0 || cols % 8 || in_row_stride < 2 * cols || out_row_stride < cols ||
      in_row_stride % 8 || out_row_stride % 8)
    return fail(FPV2_ERR_ARGUMENT, "fpv2_silu_mul: cols and row strides must be multiples of 8, "
                "in_row_stride >= 2 cols, out_row_stride >= cols");
  if (!aligned16(gate_up) || !aligned16(out))
    return fail(FPV2_ERR_ARGUMENT, "fpv2_silu_mul: pointers must be 16-byte aligned");
  if (rows == 0) return FPV2_OK;
  SiluArgs a{static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), rows, cols / 8,
             cols, in_row_stride, out_row_stride};
  const int64_t total = rows * (cols / 8);
  const int64_t want = (total + 255) / 256;
  const unsigned grid = static_cast<unsigned>(want < 8192 ? want : 8192);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == FPV2_BF16)
    hipLaunchKernelGGL(silu_mul_kernel<bf16_t>, dim3(grid), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(silu_mul_kernel<f16_t>, dim3(grid), dim3(256), 0, s, a);
  return check_launch("silu_mul_kernel");
}
