// Block mean pooling of K and V (fpv2/selection.py:68-80, called on the
// padded key/value tensors at fpv2/patch.py:137-138).
//
// HBM-bound: every element of K and V is read once, the pooled rows are
// written once.  One workgroup owns one (tensor, head, block) triple and
// reduces block_size rows x D columns.  Lanes read 16-byte vectors along D
// (coalesced rows); row groups accumulate in float64 and are combined by
// lane exchanges within a wave, then through LDS across the four waves.
// float64 accumulation makes the block sum exact for bf16/f16 data (and for
// f32 data whose magnitudes span < 2^21), so the pooled value is the
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
//
// Lane layout: the D/8 16-byte columns of a row are padded to C = 64/R (a
// power of two), and a wave holds R row groups of every column: lane l loads
// column l/R of the rows of row group l%R (the wave's loads of one row step
// cover R whole rows, so they are as coalesced as a row-major lane order).
// The R partials of a column sit in R adjacent lanes and are combined by a
// butterfly that scatters as it reduces: at each step a lane keeps half of its
// live accumulators and adds the partner's copy of that half (DPP moves, no
// LDS), so after log2(R) steps lane l holds the wave's sums of elements
// 8/R * (l%R) .. of its column, which are the 8/R doubles at l * 8/R in
// column-major order: one contiguous, conflict-free LDS write per wave.  The
// four waves' sums are then added per element.
template <int M>
__device__ __forceinline__ double dpp_partner(double x) {
  // x of a lane whose bit log2(M) differs: quad_perm [1,0,3,2] (xor 1) and
  // [2,3,0,1] (xor 2); for M = 4 the half-row mirror (lane i <-> 7 - i), whose
  // pairs also differ in bit 2 (used only as the first step, while both lanes
  // of a pair hold the same elements)
  static_assert(M == 1 || M == 2 || M == 4, "DPP partner");
  constexpr int ctrl = M == 1 ? 0xB1 : M == 2 ? 0x4E : 0x141;
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(x));
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(u & 0xffffffffu), ctrl, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(u >> 32), ctrl, 0xF, 0xF, false);
  return __longlong_as_double(static_cast<long long>(
      (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo)));
}

template <int M, int N>
__device__ __forceinline__ void butterfly_step(double (&acc)[8], int lane) {
  // N live accumulators -> N/2: keep the lower half if bit M of the lane is
  // clear, else the upper half; send the other half to the partner
  const bool upper = (lane & M) != 0;
#pragma unroll
  for (int j = 0; j < N / 2; ++j) {
    const double keep = upper ? acc[j + N / 2] : acc[j];
    const double send = upper ? acc[j] : acc[j + N / 2];
    acc[j] = keep + dpp_partner<M>(send);
  }
}

template <typename T, int R>
__global__ __launch_bounds__(kPoolThreads) void pool16_kernel(PoolArgs a) {
  constexpr int V = PoolIO<T>::kVec;
  constexpr int C = 64 / R;                  // padded columns per wave
  constexpr int GROUPS = (kPoolThreads / 64) * R;
  constexpr int OUT = V / R;                 // doubles each lane writes
  static_assert(V == 8 && (R == 1 || R == 2 || R == 4 || R == 8), "lane layout");
  __shared__ double red[kPoolThreads / 64][C * V];
  const int64_t item = blockIdx.x;  // (batch, block)
  const int which = blockIdx.y;     // tensor 0 / 1
  const int64_t n = item / a.num_blocks;
  const int64_t b = item - n * a.num_blocks;
  const int cols = static_cast<int>(a.head_dim / V);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane / R;
  const int grp = wave * R + lane % R;
  const uint16_t* src = static_cast<const uint16_t*>(a.src[which]) + n * a.batch_stride + col * V;
  const int64_t row0 = b * a.block_size;
  int64_t row_end = row0 + a.block_size;
  if (row_end > a.valid_rows) row_end = a.valid_rows;

  double acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0;
  if (col < cols) {
    // Unrolled by 8, then 4, so a lane's loads of a block are in flight
    // together (8 rows per lane at D = 128, block 128).
    int64_t r = row0 + grp;
    for (; r + 7 * GROUPS < row_end; r += 8 * GROUPS) {
      u32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = load16(src + (r + u * GROUPS) * a.row_stride);
#pragma unroll
      for (int u = 0; u < 8; ++u) PoolIO<T>::add(acc, v[u]);
    }
    for (; r + 3 * GROUPS < row_end; r += 4 * GROUPS) {
      u32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = load16(src + (r + u * GROUPS) * a.row_stride);
#pragma unroll
      for (int u = 0; u < 4; ++u) PoolIO<T>::add(acc, v[u]);
    }
    for (; r < row_end; r += GROUPS) PoolIO<T>::add(acc, load16(src + r * a.row_stride));
  }
  // butterfly over the R row groups of the wave, highest lane bit first
  // (the step with mask M starts with 16 M / R live accumulators)
  if constexpr (R >= 8) butterfly_step<4, 64 / R>(acc, lane);
  if constexpr (R >= 4) butterfly_step<2, 32 / R>(acc, lane);
  if constexpr (R >= 2) butterfly_step<1, 16 / R>(acc, lane);
#pragma unroll
  for (int j = 0; j < OUT; ++j) red[wave][lane * OUT + j] = acc[j];
  __syncthreads();
  const int total = cols * V;
  uint16_t* dst = static_cast<uint16_t*>(a.dst[which]) + n * a.out_batch_stride + b * a.head_dim;
  for (int e = tid; e < total; e += kPoolThreads) {
    double s = red[0][e];
#pragma unroll
    for (int w = 1; w < kPoolThreads / 64; ++w) s += red[w][e];
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

template <typename T>
void launch_pool16(int lanes_per_col, dim3 grid, const PoolArgs& a, hipStream_t stream) {
  switch (lanes_per_col) {
    case 8: hipLaunchKernelGGL((pool16_kernel<T, 8>), grid, dim3(kPoolThreads), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((pool16_kernel<T, 4>), grid, dim3(kPoolThreads), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((pool16_kernel<T, 2>), grid, dim3(kPoolThreads), 0, stream, a); break;
    default: hipLaunchKernelGGL((pool16_kernel<T, 1>), grid, dim3(kPoolThreads), 0, stream, a); break;
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
  // 16-byte path: D a multiple of 8 whose 16-byte columns, padded to a power
  // of two, number 8..64 (D = 40..512); R row groups of each column per wave
  int padded = 8;
  while (padded <= 64 && padded * 8 < a.head_dim) padded *= 2;
  const bool vec_ok = (a.head_dim % 8 == 0) && padded <= 64 &&
                      (a.row_stride % 8 == 0) && (a.batch_stride % 8 == 0);
  const int lanes_per_col = 64 / padded;
  bool aligned = true;
  for (int i = 0; i < tensors; ++i)
    aligned = aligned && (reinterpret_cast<uintptr_t>(a.src[i]) % 16 == 0);
  switch (dtype) {
    case FPV2_BF16:
      if (vec_ok && aligned)
        launch_pool16<bf16_t>(lanes_per_col, grid, a, stream);
      else
        hipLaunchKernelGGL(pool_generic_kernel<bf16_t>, grid, dim3(kPoolThreads), 0, stream, a);
      break;
    case FPV2_F16:
      if (vec_ok && aligned)
        launch_pool16<f16_t>(lanes_per_col, grid, a, stream);
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
