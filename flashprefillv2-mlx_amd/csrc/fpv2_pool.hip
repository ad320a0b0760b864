// Block mean pooling of K and V (fpv2/selection.py:68-80, called on the
// padded key/value tensors at fpv2/patch.py:137-138).
//
// HBM-bound: every element of K and V is read once, the pooled rows are
// written once.  One workgroup owns one (tensor, head, block) triple and
// reduces block_size rows x D columns.  Lanes read 16-byte vectors along D
// (coalesced rows); row groups accumulate in float64 and are combined through
// LDS.  float64 accumulation makes the block sum exact for bf16/f16 data (and
// for f32 data whose magnitudes span < 2^21), so the pooled value is the
// correctly rounded mean regardless of reduction order.
#include <stdarg.h>

#include "fpv2_common.h"

namespace fpv2 {
namespace {

constexpr int kPoolThreads = 256;

template <typename T> struct PoolIO;
template <> struct PoolIO<bf16_t> {
  static constexpr int kVec = 8;  // elements per 16-byte load
  static __device__ __forceinline__ void add(double* acc, u32x4 v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += static_cast<double>(Elem<bf16_t>::to_float(v[i] & 0xffffu));
      acc[2 * i + 1] += static_cast<double>(Elem<bf16_t>::to_float(v[i] >> 16));
    }
  }
  static __device__ __forceinline__ uint16_t round(double m) {
    return Elem<bf16_t>::from_float(double_to_float_odd(m));
  }
};
template <> struct PoolIO<f16_t> {
  static constexpr int kVec = 8;
  static __device__ __forceinline__ void add(double* acc, u32x4 v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += static_cast<double>(Elem<f16_t>::to_float(v[i] & 0xffffu));
      acc[2 * i + 1] += static_cast<double>(Elem<f16_t>::to_float(v[i] >> 16));
    }
  }
  static __device__ __forceinline__ uint16_t round(double m) {
    return Elem<f16_t>::from_float(double_to_float_odd(m));
  }
};

struct PoolArgs {
  const void* src[2];
  void* dst[2];
  int64_t batch;
  int64_t valid_rows;
  int64_t num_blocks;
  int64_t head_dim;
  int64_t block_size;
  int64_t batch_stride;
  int64_t row_stride;
  int64_t out_batch_stride;  // elements between batches of dst
};

// 16-bit element types: 16-byte vector loads.
template <typename T>
__global__ __launch_bounds__(kPoolThreads) void pool16_kernel(PoolArgs a) {
  constexpr int V = PoolIO<T>::kVec;
  __shared__ double red[kPoolThreads * V];
  const int64_t item = blockIdx.x;  // (batch, block)
  const int which = blockIdx.y;     // tensor 0 / 1
  const int64_t n = item / a.num_blocks;
  const int64_t b = item - n * a.num_blocks;
  const int cols = static_cast<int>(a.head_dim / V);
  const int groups = kPoolThreads / cols;  // row groups
  const int tid = threadIdx.x;
  const int col = tid % cols;
  const int grp = tid / cols;
  const uint16_t* src = static_cast<const uint16_t*>(a.src[which]) + n * a.batch_stride;
  const int64_t row0 = b * a.block_size;
  int64_t row_end = row0 + a.block_size;
  if (row_end > a.valid_rows) row_end = a.valid_rows;

  double acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0;
  if (grp < groups) {
    // Unrolled by 4 so several 16-byte loads are in flight per lane.
    int64_t r = row0 + grp;
    for (; r + 3 * groups < row_end; r += 4 * groups) {
      u32x4 v0 = load16(src + r * a.row_stride + col * V);
      u32x4 v1 = load16(src + (r + groups) * a.row_stride + col * V);
      u32x4 v2 = load16(src + (r + 2 * groups) * a.row_stride + col * V);
      u32x4 v3 = load16(src + (r + 3 * groups) * a.row_stride + col * V);
      PoolIO<T>::add(acc, v0);
      PoolIO<T>::add(acc, v1);
      PoolIO<T>::add(acc, v2);
      PoolIO<T>::add(acc, v3);
    }
    for (; r < row_end; r += groups) PoolIO<T>::add(acc, load16(src + r * a.row_stride + col * V));
  }
#pragma unroll
  for (int i = 0; i < V; ++i) red[tid * V + i] = acc[i];
  __syncthreads();
  // Combine row groups: thread (col, i) sums column element col*V+i.
  const int total = cols * V;
  uint16_t* dst = static_cast<uint16_t*>(a.dst[which]) + n * a.out_batch_stride + b * a.head_dim;
  for (int e = tid; e < total; e += kPoolThreads) {
    const int c = e / V;
    const int i = e - c * V;
    double s = 0.0;
    for (int g = 0; g < groups; ++g) s += red[(g * cols + c) * V + i];
    dst[e] = PoolIO<T>::round(s / static_cast<double>(a.block_size));
  }
}

// Generic path (float32 data, or head_dim not a multiple of 8).
template <typename T>
__device__ __forceinline__ double load_elem(const void* p, int64_t idx);
template <> __device__ __forceinline__ double load_elem<float>(const void* p, int64_t idx) {
  return static_cast<const float*>(p)[idx];
}
template <> __device__ __forceinline__ double load_elem<bf16_t>(const void* p, int64_t idx) {
  return Elem<bf16_t>::to_float(static_cast<const uint16_t*>(p)[idx]);
}
template <> __device__ __forceinline__ double load_elem<f16_t>(const void* p, int64_t idx) {
  return Elem<f16_t>::to_float(static_cast<const uint16_t*>(p)[idx]);
}
template <typename T>
__device__ __forceinline__ void store_elem(void* p, int64_t idx, double m);
template <> __device__ __forceinline__ void store_elem<float>(void* p, int64_t idx, double m) {
  static_cast<float*>(p)[idx] = static_cast<float>(m);
}
template <> __device__ __forceinline__ void store_elem<bf16_t>(void* p, int64_t idx, double m) {
  static_cast<uint16_t*>(p)[idx] = PoolIO<bf16_t>::round(m);
}
template <> __device__ __forceinline__ void store_elem<f16_t>(void* p, int64_t idx, double m) {
  static_cast<uint16_t*>(p)[idx] = PoolIO<f16_t>::round(m);
}

template <typename T>
__global__ __launch_bounds__(kPoolThreads) void pool_generic_kernel(PoolArgs a) {
  __shared__ double red[kPoolThreads];
  const int64_t item = blockIdx.x;
  const int which = blockIdx.y;
  const int64_t n = item / a.num_blocks;
  const int64_t b = item - n * a.num_blocks;
  const int64_t row0 = b * a.block_size;
  int64_t row_end = row0 + a.block_size;
  if (row_end > a.valid_rows) row_end = a.valid_rows;
  const int tid = threadIdx.x;
  // Columns in chunks of up to kPoolThreads; row groups split the rows.
  const int cols = a.head_dim < kPoolThreads ? static_cast<int>(a.head_dim) : kPoolThreads;
  const int groups = kPoolThreads / cols;
  const int col = tid % cols;
  const int grp = tid / cols;
  for (int64_t c0 = 0; c0 < a.head_dim; c0 += cols) {
    const int64_t c = c0 + col;
    double s = 0.0;
    if (grp < groups && c < a.head_dim) {
      for (int64_t r = row0 + grp; r < row_end; r += groups)
        s += load_elem<T>(a.src[which], n * a.batch_stride + r * a.row_stride + c);
    }
    red[tid] = s;
    __syncthreads();
    if (tid < cols && c0 + tid < a.head_dim) {
      double t = 0.0;
      for (int g = 0; g < groups; ++g) t += red[g * cols + tid];
      store_elem<T>(a.dst[which], n * a.out_batch_stride + b * a.head_dim + c0 + tid,
                    t / static_cast<double>(a.block_size));
    }
    __syncthreads();
  }
}

int launch_pool(const PoolArgs& a, int tensors, int dtype, hipStream_t stream) {
  if (a.batch <= 0 || a.num_blocks <= 0 || a.head_dim <= 0 || a.block_size <= 0)
    return fail(FPV2_ERR_ARGUMENT, "pool: batch, num_blocks, head_dim and block_size must be positive");
  if (a.valid_rows < 0 || a.valid_rows > a.num_blocks * a.block_size)
    return fail(FPV2_ERR_ARGUMENT, "pool: valid_rows must lie in [0, num_blocks*block_size]");
  for (int i = 0; i < tensors; ++i)
    if (!a.src[i] || !a.dst[i]) return fail(FPV2_ERR_ARGUMENT, "pool: null pointer");
  if (a.batch > 1 && a.out_batch_stride < a.num_blocks * a.head_dim)
    return fail(FPV2_ERR_ARGUMENT, "pool: out_batch_stride must be >= num_blocks*head_dim");
  const int64_t items = a.batch * a.num_blocks;
  if (items > 0x7fffffffLL) return fail(FPV2_ERR_UNSUPPORTED, "pool: too many blocks");
  dim3 grid(static_cast<unsigned>(items), tensors);
  const bool vec_ok = (a.head_dim % 8 == 0) && (a.head_dim / 8 <= kPoolThreads) &&
                      (a.row_stride % 8 == 0) && (a.batch_stride % 8 == 0);
  bool aligned = true;
  for (int i = 0; i < tensors; ++i)
    aligned = aligned && (reinterpret_cast<uintptr_t>(a.src[i]) % 16 == 0);
  switch (dtype) {
    case FPV2_BF16:
      if (vec_ok && aligned)
        hipLaunchKernelGGL(pool16_kernel<bf16_t>, grid, dim3(kPoolThreads), 0, stream, a);
      else
        hipLaunchKernelGGL(pool_generic_kernel<bf16_t>, grid, dim3(kPoolThreads), 0, stream, a);
      break;
    case FPV2_F16:
      if (vec_ok && aligned)
        hipLaunchKernelGGL(pool16_kernel<f16_t>, grid, dim3(kPoolThreads), 0, stream, a);
      else
        hipLaunchKernelGGL(pool_generic_kernel<f16_t>, grid, dim3(kPoolThreads), 0, stream, a);
      break;
    case FPV2_F32:
      hipLaunchKernelGGL(pool_generic_kernel<float>, grid, dim3(kPoolThreads), 0, stream, a);
      break;
    default:
      return fail(FPV2_ERR_UNSUPPORTED, "pool: unsupported dtype %d", dtype);
  }
  return check_launch("pool");
}

}  // namespace
}  // namespace fpv2

extern "C" int fpv2_pool_blocks(const void* x, void* out, int dtype, int64_t batch,
                                int64_t valid_rows, int64_t num_blocks, int64_t head_dim,
                                int64_t block_size, int64_t batch_stride, int64_t row_stride,
                                int64_t out_batch_stride, void* stream) {
  fpv2::PoolArgs a{};
  a.src[0] = x;
  a.dst[0] = out;
  a.batch = batch;
  a.valid_rows = valid_rows;
  a.num_blocks = num_blocks;
  a.head_dim = head_dim;
  a.block_size = block_size;
  a.batch_stride = batch_stride;
  a.row_stride = row_stride;
  a.out_batch_stride = out_batch_stride;
  return fpv2::launch_pool(a, 1, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int fpv2_pool_kv(const void* k, const void* v, void* pooled_k, void* pooled_v,
                            int dtype, int64_t kv_heads, int64_t valid_rows, int64_t num_blocks,
                            int64_t head_dim, int64_t block_size, int64_t head_stride,
                            int64_t row_stride, int64_t pooled_head_stride, void* stream) {
  fpv2::PoolArgs a{};
  a.src[0] = k;
  a.src[1] = v;
  a.dst[0] = pooled_k;
  a.dst[1] = pooled_v;
  a.batch = kv_heads;
  a.valid_rows = valid_rows;
  a.num_blocks = num_blocks;
  a.head_dim = head_dim;
  a.block_size = block_size;
  a.batch_stride = head_stride;
  a.row_stride = row_stride;
  a.out_batch_stride = pooled_head_stride;
  return fpv2::launch_pool(a, 2, dtype, static_cast<hipStream_t>(stream));
}
