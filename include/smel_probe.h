/* C-ABI of the peak probes (libsmel_moe.so): the achievable MFMA rate and HBM bandwidth of the GPU this library runs
 * on, measured by kernels that do nothing else, so that a kernel's roofline fraction can be read against what the
 * chip delivers as well as against its published peaks.
 *
 * These entry points have no counterpart in the reference (it reports no roofline); they are for the benchmark and
 * the profiles, not for the MoE layer. Same conventions as smel_moe.h (0 on success, SMEL_E* or hipError_t codes,
 * message in smel_last_error()); asynchronous on `stream`, no allocation.
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "smel_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* `blocks` workgroups of 4 waves, each wave issuing `iters` x 8 independent v_mfma_f32_32x32x16_bf16 (32768 FLOP
 * each) with nothing else in the loop: FLOP = blocks * 4 * iters * 8 * 32768. out: blocks * 256 floats (one word per
 * lane keeps the accumulators live). */
int smel_probe_mfma(float* out, int32_t blocks, int32_t iters, hipStream_t stream);

/* Streaming read of `bytes` (a multiple of 16) from `src`, 16 bytes per lane per load, grid-stride over `grid`
 * workgroups of 256 lanes. out: grid * 256 words (one per lane, keeps the loads live). */
int smel_probe_read(const void* src, int64_t bytes, uint32_t* out, int32_t grid, hipStream_t stream);

/* Device copy src -> dst of `bytes` (a multiple of 16), 16 bytes per lane, grid-stride over `grid` workgroups. */
int smel_probe_copy(const void* src, void* dst, int64_t bytes, int32_t grid, hipStream_t stream);

#ifdef __cplusplus
}
#endif
