/*
 * fpv2_decoder.h — decoder-layer operations of the end-to-end prefill
 * harness (random-init Qwen3 architecture), exported by libfpv2_hip.so.
 *
 * These are not part of FPV2 itself.  The reference's end-to-end numbers
 * (README.md:30-46) run Qwen3 through mlx-lm (an external dependency, absent
 * from the reference tree), whose model code computes the RMSNorms and the
 * rotary embedding with fused Metal kernels (mx.fast.rms_norm, mx.fast.rope)
 * and the SwiGLU gate with nn.silu.  These entry points are the fused gfx950
 * counterparts used by fpv2/prefill_harness.py, so that the harness's
 * prefill time is not dominated by float32 elementwise chains.
 *
 * Conventions as in fpv2.h: device pointers, element strides, a hipStream_t
 * passed as void*, FPV2_BF16 or FPV2_F16 data, return FPV2_OK or a negative
 * fpv2_status with fpv2_last_error() set.  Rows are contiguous; for
 * fpv2_add_rms_norm and fpv2_silu_mul, row strides and `cols` must be
 * multiples of 8 elements and the pointers 16-byte aligned (16-byte vector
 * accesses).
 */
#ifndef FPV2_DECODER_H_
#define FPV2_DECODER_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Largest row length of fpv2_add_rms_norm (elements). */
#define FPV2_MAX_NORM_COLS 16384

/*
 * Residual add and RMSNorm of rows of `cols` elements:
 *   if delta != NULL:  x[r] = round(x[r] + delta[r])      (in place)
 *   y[r] = round(x[r] * rsqrt(mean(x[r]^2) + eps) * weight)
 * computed in float32 from the stored (rounded) x.  Counterpart of
 * mlx-lm's `h = x + r; mx.fast.rms_norm(h, w, eps)` pair in the Qwen3
 * block.  y must not alias x or delta.
 */
int fpv2_add_rms_norm(void* x, const void* delta, const void* weight, void* y,
                      int dtype, int64_t rows, int64_t cols,
                      int64_t x_row_stride, int64_t delta_row_stride,
                      int64_t y_row_stride, float eps, void* stream);

/*
 * Per-head RMSNorm and rotate-half rotary embedding of the query and key
 * heads of fused projection rows qkv[r] = [q heads | k heads | v heads],
 * with the value heads copied alongside:
 *   n = round(x * rsqrt(mean(x^2) + eps) * weight)       (norm output dtype)
 *   out[j]        = round(n[j] cos[r][j]        - n[j+D/2] sin[r][j])
 *   out[j + D/2]  = round(n[j+D/2] cos[r][j+D/2] + n[j] sin[r][j+D/2])
 * Query head h of row r goes to q_out + r*q_row_stride + h*q_head_stride,
 * key head h to k_out + r*kv_row_stride + h*kv_head_stride, and value head h
 * (unchanged) to v_out at the same offsets; v_out may be NULL (no copy).
 * With kv strides of a [kv_heads, capacity, D] cache, K and V land in the
 * cache directly.  cos / sin are float32 [rows, D] contiguous, 16-byte
 * aligned; head_dim a multiple of 8, <= 256; every stride a multiple of 4;
 * qkv, the weights and the outputs 8-byte aligned.
 * Counterpart of mlx-lm's q_norm / k_norm followed by nn.RoPE
 * (traditional = false) in the Qwen3 attention, and of its KV-cache update.
 */
int fpv2_qk_norm_rope(const void* qkv, const void* q_weight,
                      const void* k_weight, const float* cos, const float* sin,
                      void* q_out, void* k_out, void* v_out, int dtype,
                      int64_t rows, int64_t query_heads, int64_t kv_heads,
                      int64_t head_dim, int64_t qkv_row_stride,
                      int64_t q_head_stride, int64_t q_row_stride,
                      int64_t kv_head_stride, int64_t kv_row_stride, float eps,
                      void* stream);

/*
 * SwiGLU gate: out[r][c] = round(silu(g) * u) with g = gate_up[r][c],
 * u = gate_up[r][cols + c], silu(g) = g / (1 + exp(-g)) in float32.
 * Counterpart of mlx-lm's `nn.silu(gate) * up` in the Qwen3 MLP.
 */
int fpv2_silu_mul(const void* gate_up, void* out, int dtype, int64_t rows,
                  int64_t cols, int64_t in_row_stride, int64_t out_row_stride,
                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FPV2_DECODER_H_ */
