/* C-ABI of the fp32 path of the MoE layer: the reference run on fp32 tensors (its fp32 models; _gmm falls to its
 * per-group matmul loop for any non-bf16 tensor, smel/moe.py:58-72, and the tests compare at 1e-5,
 * tests/test_moe.py:10-36). Every product is an fp32 MFMA (v_mfma_f32_32x32x2_f32) with fp32 accumulation; int4 banks
 * are dequantized to fp32 inside the GEMM (the reference's fp32 Int4Experts: w = q s + z in fp32, smel/quant.py:51-84).
 * Rows are in the sorted row space of smel_dispatch (include/smel_moe.h): the tile list {group, row0, row1, gk} and
 * the group kinds are the same as the bf16 GEMMs'. All pointers are device pointers; all matrices are row-major fp32
 * unless stated. Results are deterministic (fixed summation order, no atomics). Entry points return 0 or an error
 * code; smel_last_error() says why. */
#ifndef SMEL_F32_H
#define SMEL_F32_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One projection's weights for every group kind, fp32 path. A matrix is [R][C] as the reference stores it (gate_up
 * R = 2I, C = H; down R = H, C = I; a LoRA A [r][in], B [out][r]); matrix `idx` of a stack starts at idx * R * C. */
typedef struct smel_wset_f32 {
  const uint8_t* q4;      /* SMEL_KIND_INT4: the reference's int4 bank, q [E][R][C/2] (even column in the low nibble) */
  const uint16_t* scale;  /*   its bf16 scale [E][R][C/group]                                                       */
  const uint16_t* zero;   /*   its bf16 zero  [E][R][C/group]                                                       */
  const float* wf;        /* SMEL_KIND_BF16: a frozen bank of the activation dtype (BF16Experts of an fp32 model)   */
  const float* wsel;      /* SMEL_KIND_SEL: selected experts (or per-slot LoRA factors), [n_sel][R][C]             */
  const float* wsh;       /* SMEL_KIND_SHARED: one matrix [R][C] (shared expert, router, a dense LoRA factor)      */
  int64_t R, C;           /* one matrix                                                                             */
  int32_t group;          /* int4 group (even, divides C)                                                           */
  int32_t kinds;          /* bit (1 << kind) set for each kind whose tiles this launch computes; other tiles skipped */
  int32_t q4_round_bf16;  /* 1: the int4 dequant rounds to bf16 (an Int4Experts whose dtype is bf16), 0: fp32       */
  int32_t pad_;
} smel_wset_f32;

/* ---- (A5/A6/A10/A11/A12) replaces _gmm, smel/moe.py:58-72 (per-group x_g @ w_g.T / x_g @ w_g), for fp32 tensors.
 * For each tile {g, row0, row1, gk} of tiles[0 .. n_tiles[0]) (any tile height: the block walks it in 64-row steps)
 * whose kind (gk >> 16, gk = gkind[g] when gkind is given, else tile[3]) is in w->kinds, with W = matrix gk & 0xffff
 * of that kind:
 *   trans = 0:  C[r][n] = beta C[r][n] + alpha sum_k A[r][k] W[n][k]   (n < R, k < C: out = a W^T)
 *   trans = 1:  C[r][n] = beta C[r][n] + alpha sum_k A[r][k] W[k][n]   (n < C, k < R: out = a W)
 * for rows r in [row0, row1). beta is 0 or 1 (beta 0 never reads C). A [rows][lda], C [rows][ldc]. */
int smel_gmm_f32(const smel_wset_f32* w, int32_t trans, const int32_t* gkind, const int32_t* tiles,
                 const int32_t* n_tiles, int64_t max_tiles, const float* A, int64_t lda, float alpha, float beta,
                 float* C, int64_t ldc, hipStream_t stream);

/* ---- LoRA weight gradients (autograd of lora_linear / lora_gate_up, smel/lora.py:61-83, for fp32 tensors).
 * For each job j < n_jobs with rows [offsets[g], offsets[g+1]), g = job_group[j]:
 *   C_j[m][n] = alpha sum_r X[r][m] Y[r][n]   (m < M, n < N; C_j = C + j * c_stride, [M][N] row-major)
 * summed in row order within 16-row steps (a job with no rows writes zeros). X [rows][ldx], Y [rows][ldy]. */
int smel_wgrad_f32(const float* X, int64_t ldx, const float* Y, int64_t ldy, const int32_t* offsets,
                   const int32_t* job_group, int32_t n_jobs, int64_t M, int64_t N, float alpha, float* C,
                   int64_t c_stride, hipStream_t stream);

/* ---- the token gather of routed_experts (xs = x2d[order // K], smel/moe.py:216-221): out[p] = src[idx[p] / div]
 * for p < n_valid[0] (device int32; NULL: all n rows), a zero row where idx[p] < 0 or p >= n_valid[0] (the dispatch
 * leaves the order entries of dropped slots unwritten: n_valid = offsets + E); src [*][lds], out [n][cols]. */
int smel_gather_rows_f32(const float* src, int64_t lds, const int32_t* idx, int32_t div, const int32_t* n_valid,
                         int64_t n, int64_t cols, float* out, hipStream_t stream);

/* ---- act(g) * u and its backward (act / act_and_grad, smel/moe.py:91-107; FrozenExpertsFn, :110-143), fp32.
 * h [rows][ldh] holds g in columns [0, I) and u in [I, 2I); act 0 = silu, 1 = gelu_tanh.
 *   forward:  a[r][j] = act(g) u
 *   backward: dh[r][j] = da u act'(g),  dh[r][I + j] = da act(g)  (da [rows][ldda], dh [rows][lddh]) */
int smel_act_gate_f32(const float* h, int64_t ldh, int64_t rows, int64_t I, int32_t act, float* a, int64_t lda,
                      hipStream_t stream);
int smel_act_gate_bwd_f32(const float* h, int64_t ldh, const float* da, int64_t ldda, int64_t rows, int64_t I,
                          int32_t act, float* dh, int64_t lddh, hipStream_t stream);

/* ---- the combine of routed_experts (smel/moe.py:248-252) and its backward, fp32.
 *   forward:  out[t] = sum_k ys[inv[t K + k]] topv[t][k]   (k ascending; a slot with inv < 0 adds nothing)
 *   backward: dys[inv[t K + k]] = topv[t][k] dout[t],  dtopv[t][k] = <ys[inv[t K + k]], dout[t]>
 * ys / dys [T K][H], out / dout [T][H], topv / dtopv [T][K]. */
int smel_combine_f32(const float* ys, const float* topv, const int32_t* inv, int64_t T, int64_t K, int64_t H,
                     float* out, hipStream_t stream);
int smel_combine_bwd_f32(const float* ys, const float* dout, const float* topv, const int32_t* inv, int64_t T,
                         int64_t K, int64_t H, float* dys, float* dtopv, hipStream_t stream);
/* dX of the token gather: dx[t] = sum_k dxs[inv[t K + k]] (k ascending). */
int smel_dx_reduce_f32(const float* dxs, const int32_t* inv, int64_t T, int64_t K, int64_t H, float* dx,
                       hipStream_t stream);

/* ---- route (smel/moe.py:162-167) and route_gemma4's selection (:176-180) from fp32 logits [T][ldl], E <= 512,
 * K <= 16: probs = softmax (fp32), the K largest probabilities (descending, the lower expert id first among equal
 * ones), topv = p / sum of the K, times per_expert_scale[id] when pes [E] is given; topi int64 and int32. */
int smel_route_select_f32(const float* logits, int64_t ldl, int64_t T, int64_t E, int64_t K, const float* pes,
                          float* probs, float* topv, int64_t* topi, int32_t* topi32, hipStream_t stream);
/* Backward of that selection: dtopv [T][K] -> dlogits [T][E] (through the per-expert scale, the renorm, the gather
 * and the softmax; the softmax probabilities probs as the forward wrote them). */
int smel_route_bwd_f32(const float* dtopv, const float* probs, const int32_t* topi32, const float* pes, int64_t T,
                       int64_t K, int64_t E, float* dlogits, hipStream_t stream);

/* ---- route_gemma4's router input (smel/moe.py:172-174), fp32: r = (mean_j h[t][j]^2 + eps)^-1/2,
 * xn = ((h r) scale) * hs with hs = fp32(H^-1/2); rstd [T] = r kept for the backward.
 * Backward: g = (dxn hs) scale, dh = g r - h r^3 sum_j(g h) / H. */
int smel_route_prenorm_f32(const float* h, const float* scale, int64_t T, int64_t H, float eps, float hs, float* xn,
                           float* rstd, hipStream_t stream);
int smel_route_prenorm_bwd_f32(const float* h, const float* scale, const float* rstd, const float* dxn, int64_t T,
                               int64_t H, float hs, float* dh, hipStream_t stream);

/* ---- shared_mlp's gate (smel/moe.py:201) and moe_forward's sum (:263), fp32: s [T] = the gate logit x w_sg^T,
 *   forward:  out[t] = base[t] + y[t] sigmoid(s[t])   (base optional)
 *   backward: dy[t] = dout[t] sigmoid(s[t]),  ds[t] = <dout[t], y[t]> sigmoid (1 - sigmoid). */
int smel_gate_mul_f32(const float* y, const float* s, const float* base, int64_t T, int64_t H, float* out,
                      hipStream_t stream);
int smel_gate_mul_bwd_f32(const float* y, const float* s, const float* dout, int64_t T, int64_t H, float* dy,
                          float* ds, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SMEL_F32_H */
