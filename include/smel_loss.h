/* C-ABI of the single-pass chunked cross-entropy's per-chunk kernels (libsmel_moe.so, HIP for gfx950).
 *
 * Same conventions as smel_moe.h. The two GEMMs of each (token chunk, vocabulary chunk) step (logits = h W_c^T and
 * p W_c) are plain library GEMMs; these kernels do everything between and after them without a host
 * synchronisation. `dtype` is that of the rows h, the GEMM outputs and p: 0 bf16, 1 fp32, 2 fp16.
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "smel_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One vocabulary chunk [v0, v0 + vc) for n token rows: logits [n][ld] (the GEMM output, first vc columns used),
 * z = softcap tanh(logit / softcap) (softcap 0: z = logit); per row the running max m and sum s (fp32, m = -inf and
 * s = 0 before the first chunk) move to nm = max(m, max z): r = exp(m - nm) (written to r[row]), s = s r +
 * sum exp(z - nm); with need_grad, p = exp(z - nm) (times 1 - (z / softcap)^2 with the cap) in `dtype`, laid out as
 * p_parts column slices [p_parts][n][vc / p_parts] (p_parts divides vc; 1 = plain [n][vc]) for a split-K gradient
 * GEMM; the
 * row whose target tgt[row] lies in the chunk gets tgt_logit = z at the target and (with the cap) tgt_d = its cap
 * derivative. Replaces the chunk loop body of `_ce_chunk`, smel/loss.py:62-84. */
int smel_ce_chunk_update(const void* logits, int64_t n, int64_t vc, int64_t ld, int64_t v0, const int64_t* tgt,
                         float softcap, int32_t dtype, int32_t need_grad, float* m, float* s, float* tgt_logit,
                         float* tgt_d, void* p, int32_t p_parts, float* r, hipStream_t stream);

/* acc [n][H] fp32 = acc r[row] + sum_k pw[k] (pw [parts][n][H] = the slices' products p_k W_c,k in `dtype`, summed
 * in k order): the gradient accumulator's rescale and add, smel/loss.py:85. */
int smel_ce_acc_update(float* acc, const float* r, const void* pw, int32_t parts, int64_t n, int64_t H, int32_t dtype,
                       hipStream_t stream);

#ifdef __cplusplus
}
#endif
