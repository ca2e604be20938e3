/* C-ABI of the single-pass chunked cross-entropy (libsmel_moe.so, HIP for gfx950): both GEMMs of every
 * (token pass, vocabulary chunk) step on MFMA, the online softmax in the logits GEMM's epilogue, no [tokens, vocab]
 * logits in memory. Replaces _ce_chunk / _ChunkedCE of smel/loss.py:50-146.
 *
 * Same conventions as smel_moe.h. `dtype` is that of the token rows h, the head rows and the softmax terms: 0 bf16,
 * 1 fp32, 2 fp16. Row-major operands must be runs of 16-byte multiples at 16-byte aligned addresses.
 *
 * One pass over n token rows: smel_ce_begin, then per vocabulary chunk [v0, v0 + vc) smel_ce_logits, smel_ce_stats
 * and (with the gradient) smel_ce_grad, then smel_ce_finish and smel_ce_loss_sum. The per-row state (running maximum
 * m as a power-of-two exponent, running sum s, target logit tz and cap derivative td) lives in caller buffers of n
 * floats; the window statistics in [nwin][ldn] buffers (nwin = ceil(vc / 256) * 2 windows of 128 columns).
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "smel_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* m = m0 (or -inf without m0), s = 0, tz = 0, td = 1 for n rows (the state before the first chunk; m0 presets the
 * final maximum for the two-pass form). Replaces the state initialisation of `_ce_chunk`, smel/loss.py:56-61. */
int smel_ce_begin(float* m, float* s, float* tz, float* td, const float* m0, int64_t n, hipStream_t stream);

/* One vocabulary chunk: z = cap(h W^T) for the n token rows h [n][ldh] and the vc head rows W [vc][ldw] (row 0 =
 * vocabulary id v0), the logits rounded to `dtype` before the cap (softcap 0: none, else z = c tanh(z / c)). Per
 * window of 128 columns and row: win_e = ceil(max z log2 e) (-inf for a window past the chunk) and win_s = sum of
 * exp(z - win_e ln 2); with P (may be null: no gradient), P [n][ldp] (ldp >= vc rounded up to 256) = those terms
 * times the cap derivative 1 - (z / c)^2, in `dtype`, zero past the chunk. A row whose target tgt lies in the chunk
 * gets tz = its z and td = its cap derivative. Replaces the chunk loop body of `_ce_chunk`, smel/loss.py:62-84
 * (the logits GEMM included). */
int smel_ce_logits(const void* W, int64_t ldw, int64_t vc, int64_t v0, const void* h, int64_t ldh, int64_t n,
                   int64_t H, const int64_t* tgt, float softcap, int32_t dtype, void* P, int64_t ldp, float* win_e,
                   float* win_s, int64_t ldn, float* tz, float* td, hipStream_t stream);

/* Folds a chunk's window statistics into the running state: E = max win_e, nE = max(m, E), s = s 2^(m - nE) +
 * sum win_s 2^(win_e - nE), m = nE, r = 2^(m_old - nE) (0 on the first chunk) and per window shift = nE - win_e
 * (255: the window's terms count as zero). smel/loss.py:65-69, in base-2 exponents. */
int smel_ce_stats(const float* win_e, const float* win_s, int64_t nwin, int64_t ldn, int64_t n, float* m, float* s,
                  uint8_t* shift, float* r, hipStream_t stream);

/* The gradient GEMM of vocabulary chunk number `chunk` (0, 1, ... in order) over its vc columns, with the head
 * transposed: WT [H][ldwt], column 0 = vocabulary id v0 (ldwt covers vc rounded up to 16 bytes). The chunk's columns
 * are split in two halves: acc [n][H] fp32 = (chunk == 0 ? 0 : r (acc + part[(chunk - 1) % 2])) + sum over the
 * first half of (P[v] 2^-shift) W[v], and part[chunk % 2] = the same sum over the second half (part: [2][n][H]
 * fp32; the gradient sum after the last chunk is acc + part[last % 2]). smel/loss.py:83-85
 * (`acc * r + p.to(h.dtype) @ W`), the product on MFMA. */
int smel_ce_grad(const void* WT, int64_t ldwt, int64_t H, const void* P, int64_t ldp, int64_t vc,
                 const uint8_t* shift, int64_t ldn, const float* r, int64_t n, int32_t dtype, int32_t chunk,
                 float* acc, float* part, hipStream_t stream);

/* Per row: loss_rows = m ln 2 + log s - tz; with acc, g [n][ldg] in g_dtype = gscale ((acc + part) / s - td W[tgt])
 * (part: the last chunk's partial [n][H], may be null; no target row when tgt is outside [0, V)), the target row
 * read from trows [n][H] when given, else from W [V][ldw]. smel/loss.py:86-92. */
int smel_ce_finish(const float* m, const float* s, const float* tz, const float* td, const float* acc,
                   const float* part, const void* W, int64_t ldw, const void* trows, const int64_t* tgt, int64_t V,
                   int64_t n, int64_t H, int32_t dtype, float gscale, void* g, int64_t ldg, int32_t g_dtype,
                   float* loss_rows, hipStream_t stream);

/* total = (accumulate ? total : 0) + scale * sum of loss_rows, in fixed order (smel/loss.py:136-140). */
int smel_ce_loss_sum(const float* loss_rows, int64_t n, float scale, int32_t accumulate, float* total,
                     hipStream_t stream);

/* x [n] in `dtype` *= *go (a device fp32 scalar): the backward's incoming gradient, smel/loss.py:144-146. */
int smel_ce_scale(void* x, int64_t n, int32_t dtype, const float* go, hipStream_t stream);

/* dst [C][ldd] = src [R][C] (pitch lds) transposed, dst columns R .. ldd - 1 zero: the head layout of smel_ce_grad
 * (made once per frozen head). */
int smel_ce_transpose(const void* src, int64_t R, int64_t C, int64_t lds, void* dst, int64_t ldd, int32_t dtype,
                      hipStream_t stream);

#ifdef __cplusplus
}
#endif
