/* C-ABI of the RMSNorm family around the MoE block (libsmel_moe.so, HIP for gfx950).
 *
 * Same conventions as smel_moe.h: raw device pointers, element counts and strides in elements, 0 on success or an
 * SMEL_E* / hipError_t code with the message in smel_last_error(), every kernel on `stream`, no allocation, no host
 * synchronisation. Rows are 16-bit floats, `dtype` 0 = bf16, 1 = fp16; weights have the rows' dtype and `cols`
 * elements; rstd is one fp32 per row. 1 <= cols <= 16384 (the reference's MAX_COLS). fp32 math with the reference's
 * rounding points; each row's sum is a fixed-order reduction (bitwise repeatable).
 * `w_mode`: 0 = no weight (w may be null), 1 = w, 2 = 1 + w (Qwen3.5/3.6's plus_one).
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "smel_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* y[r] = x[r] rstd[r] w', rstd[r] = 1 / sqrt(mean(x[r]^2) + eps); x rows at stride x_stride (>= cols), y and rstd
 * contiguous. Replaces `_rms_fwd` smel/norm.py:50-62 (launched by `_RMSNorm.forward` :157-171). */
int smel_rmsnorm_fwd(const uint16_t* x, int64_t rows, int64_t cols, int64_t x_stride, const uint16_t* w,
                     int32_t w_mode, float eps, int32_t dtype, uint16_t* y, float* rstd, hipStream_t stream);

/* dx = rstd (g - xhat mean(g xhat)) (+ ds), xhat = x rstd, g = dy w'; x at stride x_stride, dy / ds / dx contiguous,
 * ds may be null. Replaces `_rms_bwd` smel/norm.py:64-82 (`_RMSNorm.backward` :173-183 with ds null,
 * `_AddRMSNorm.backward` :204-219 with x = s and ds = the gradient of s). */
int smel_rmsnorm_bwd(const uint16_t* dy, const uint16_t* x, int64_t rows, int64_t cols, int64_t x_stride,
                     const uint16_t* w, int32_t w_mode, const float* rstd, const uint16_t* ds, int32_t dtype,
                     uint16_t* dx, hipStream_t stream);

/* s = round(h + x) (the residual stream), y = s rstd w' with rstd of s; all contiguous, w_mode 1 or 2 in the
 * reference (0 accepted). Replaces `_add_rms_fwd` smel/norm.py:84-100 (`_AddRMSNorm.forward` :186-202). */
int smel_add_rmsnorm_fwd(const uint16_t* h, const uint16_t* x, int64_t rows, int64_t cols, const uint16_t* w,
                         int32_t w_mode, float eps, int32_t dtype, uint16_t* s, uint16_t* y, float* rstd,
                         hipStream_t stream);

/* y = round(round(w round(x rstd)) silu(z)), the sigmoid on the hardware exp2 and reciprocal (the reference's
 * tl.sigmoid is Triton's fast form too); all contiguous, w required. Replaces `_gated_fwd`
 * smel/norm.py:102-119 (`_GatedRMSNorm.forward` :222-236). */
int smel_gated_rmsnorm_fwd(const uint16_t* x, const uint16_t* z, int64_t rows, int64_t cols, const uint16_t* w,
                           float eps, int32_t dtype, uint16_t* y, float* rstd, hipStream_t stream);

/* dz = dout y silu'(z); dn = round(round(dout silu(z)) w); dx = rstd (dn - xhat mean(dn xhat)); all contiguous.
 * Replaces `_gated_bwd` smel/norm.py:121-145 (`_GatedRMSNorm.backward` :238-249). */
int smel_gated_rmsnorm_bwd(const uint16_t* dout, const uint16_t* x, const uint16_t* z, int64_t rows, int64_t cols,
                           const uint16_t* w, const float* rstd, int32_t dtype, uint16_t* dx, uint16_t* dz,
                           hipStream_t stream);

#ifdef __cplusplus
}
#endif
