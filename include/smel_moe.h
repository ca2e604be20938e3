/* C-ABI of the MI355X (gfx950) MoE-layer hot path of SMEL FT.
 *
 * Every entry point is stateless, allocates nothing, launches its kernels on the given HIP stream and never
 * synchronizes the host. Pointers are device pointers unless noted; bf16 tensors are passed as uint16_t bit
 * patterns. Return value: 0 on success, a positive hipError_t from the launch, or a negative SMEL_E* code for a
 * rejected argument (smel_last_error() then holds a message; it is thread-local).
 *
 * Row space shared by the grouped GEMMs: rows [0, TK) are the routed slots in expert-sorted order (TK = T*topk),
 * rows [TK, TK+T) are the shared expert's rows (one per token, token order) when the shared expert is fused in.
 * order[row] is the flat slot p = t*topk + k of a routed row. "Groups" are the experts 0..E-1 plus, when present,
 * the shared expert as group E; gkind[g] = (kind << 16) | index says where group g's weights live. A tile list entry
 * is {group, row0, row1, gk}: the GEMM / LoRA entry points take gk from there when their gkind argument is NULL
 * (smel_dispatch fills it when given gkind), which saves a dependent load per workgroup.
 */
#ifndef SMEL_MOE_H
#define SMEL_MOE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMEL_EINVAL (-1)       /* bad pointer / size / stride */
#define SMEL_EUNSUPPORTED (-2) /* shape outside what the kernels handle (message says which limit) */

/* group kinds (gkind >> 16) */
#define SMEL_KIND_INT4 0   /* frozen expert in the int4 bank (Int4Experts), index = expert id      */
#define SMEL_KIND_BF16 1   /* frozen expert in a bf16 bank (BF16Experts), index = expert id        */
#define SMEL_KIND_SEL 2    /* selected expert (bf16 copy + LoRA), index = slot j in sel_ids        */
#define SMEL_KIND_SHARED 3 /* shared expert (bf16 + LoRA), index 0                                 */

/* Weights of one projection (gate_up or down) for every group kind. A matrix is [R][C] in the reference
 * (gate_up: R = 2I, C = H; down: R = H, C = I; R a multiple of 32). The forward GEMM contracts over C (out = x W^T)
 * and reads the fragment layout of smel_pack_int4 / smel_pack_bf16; the backward GEMM contracts over R (dx = dy W)
 * and reads the transposed fragment layout of smel_pack_int4_t / smel_pack_bf16_t (below), one matrix after the
 * other for a stacked bank. */
typedef struct smel_wset {
  const uint8_t* q4;   /* int4 bank [E][R][C] packed by smel_pack_int4 (forward) / _int4_t (backward)   */
  const uint32_t* sz4; /* its scale/zero, packed by the same call                                      */
  const uint16_t* wb;  /* bf16 bank [E][R][C] (BF16Experts.gate_up / .down), smel_pack_bf16(_t)        */
  const uint16_t* wsel;/* selected experts [n_sel][R][C] (LayerExperts.sel_gate_up / sel_down), packed  */
  const uint16_t* wsh; /* shared expert [R][C], packed                                                 */
  /* LoRA as a K-extension of the GEMM (0-padded, built by smel_lora_prep), in 32-wide planes:
   *   forward  ext_*: [n][R][32]          (B factor per output row; gate_up with one plane: B_gate in cols 0..15,
   *                                        B_up in 16..31; with two planes: each in cols 0..r-1 of its own rows)
   *   backward ext_*: [n][planes][C][32]  (A factor per output column; gate_up with one plane: A_gate in 0..15, A_up
   *                                        in 16..31; with two planes: A_gate in plane 0, A_up in plane 1)
   * The ext rows passed to the GEMMs are [rows][32 * planes]. Two planes (SMEL_WSET_EXT2, gate_up LoRA of rank
   * 17..32): the forward's gate columns take plane 0 of the ext rows and its up columns plane 1; the backward adds
   * both planes' products. */
  const uint16_t* ext_sel;
  const uint16_t* ext_sh;
  int64_t R, C;
  int32_t group;       /* int4 group along C (a multiple of 32)                                        */
  int32_t flags;       /* SMEL_WSET_FAST_DQ: every scale/zero group of q4 passed smel_int4_fast_ok;
                        * SMEL_WSET_EXT2: the LoRA K-extension has two planes (see above)                */
} smel_wset;
#define SMEL_WSET_FAST_DQ 1
#define SMEL_WSET_EXT2 2
/* SMEL_WSET_XCD_CHUNK: the GEMM's tile list is in group order (smel_dispatch's tiles_grouped) and each of the 8
 * XCDs takes a contiguous chunk of it, so a group's tiles run side by side on one XCD and share its L2 (its weights
 * are streamed once for all of them); without it, tile t runs on XCD t % 8 in list order. */
#define SMEL_WSET_XCD_CHUNK 4
/* SMEL_WSET_MERGE_SHORT (smel_gmm_fwd, gate_up projection, group-ordered tile list, int4 bank with
 * SMEL_WSET_FAST_DQ, C a multiple of 64): the blocks of a full int4 tile also take the rows of the next tile when that is the same
 * group's last tile of at most 32 rows (the weights are streamed and dequantized once for up to 160 rows); that
 * tile's own blocks do nothing. */
#define SMEL_WSET_MERGE_SHORT 8
/* SMEL_WSET_MERGED_LIST (smel_gmm_fwd, either projection; an int4 bank needs SMEL_WSET_FAST_DQ and C a multiple of
 * 64): the tile list is smel_dispatch's tiles_merged, whose int4 tiles may hold up to 160 rows (a full tile and the
 * group's last tile of at most 32 rows); each is one tile (one weight stream and dequant), and no block idles.
 * Without it a tile of the list has at most 128 rows (rows past 128 are not computed). */
#define SMEL_WSET_MERGED_LIST 16

const char* smel_last_error(void);
int smel_abi_version(void);

/* ---- (A7) replaces dequant_int4 / _dq4_kernel, smel/quant.py:51-84.
 * q [rows][K/2], scale/zero [rows][K/group] -> out [rows][K]: w = RNE(q*s + z) (fp32 math). out_f32 = 1 writes fp32. */
int smel_dequant_int4(const uint8_t* q, const uint16_t* scale, const uint16_t* zero, void* out, int64_t rows,
                      int64_t K, int64_t group, int32_t out_f32, hipStream_t stream);

/* ---- (A8) replaces quantize_int4, smel/quant.py:5-44 (the on-disk format's producer, run on the GPU).
 * w [rows][K] (w_dtype 0 bf16, 1 fp32, 2 fp16) -> q [rows][K/2] (even column in the low nibble), scale/zero bf16
 * [rows][K/group]. Per group: the range [min, max] shrunk about its midpoint by each of the n_clip (1..8) factors in
 * clip[] (host array) in turn, the candidate with the smallest sum of squared errors kept (later ones only if strictly
 * better); every step is the reference's fp32 operation, the error sum in index order. group even, K % group == 0. */
int smel_quantize_int4(const void* w, int32_t w_dtype, int64_t rows, int64_t K, int32_t group, const float* clip,
                       int32_t n_clip, uint8_t* q, uint16_t* scale, uint16_t* zero, hipStream_t stream);

/* ---- Weight layouts of the grouped GEMMs (no counterpart in the reference, whose q/scale/zero and bf16 tensors
 * stay the source of truth and are not modified; a frozen bank is packed once when it is built).
 * A matrix of `rows` rows (a stacked bank: E*R rows) and K columns is cut into fragments of 32 rows and k-steps of
 * 64 columns; each (fragment f, k-step ks) is one 1-KB block per 64 lanes, lane 32*h + i holding row 32*f + i:
 *   SMEL_PACK_Q4   block (f, ks):        16 B = the 32 nibbles of k in [64 ks + 32 h, +32)
 *   SMEL_PACK_SZ   block (f, ks/4):      16 B = 4 words (ks%4 = 0..3), scale | zero << 16 of the group of 64 ks+32 h
 *   SMEL_PACK_BF16 block (f, ks, s<4):   16 B = the 8 bf16 of k in [64 ks + 32 h + 8 s, +8)
 * so a GEMM wave reads each block with one contiguous 1-KB load. Rows >= rows and columns >= K are zero.
 * smel_packed_bytes gives the size of each (or -1 for a bad argument). */
#define SMEL_PACK_Q4 0
#define SMEL_PACK_SZ 1
#define SMEL_PACK_BF16 2
int64_t smel_packed_bytes(int32_t what, int64_t rows, int64_t K);
/* q [rows][K/2], scale/zero [rows][K/group] bf16 (the Int4Experts dict of smel/moe.py:35-55, smel/quant.py:24-44)
 * -> qf (SMEL_PACK_Q4), szf (SMEL_PACK_SZ). K a multiple of 32, group a multiple of 32 dividing K. */
int smel_pack_int4(const uint8_t* q, const uint16_t* scale, const uint16_t* zero, int64_t rows, int64_t K,
                   int64_t group, uint8_t* qf, uint32_t* szf, hipStream_t stream);
/* w [rows][ld] bf16 (first K columns used) -> wf (SMEL_PACK_BF16). K and ld multiples of 8. */
int smel_pack_bf16(const uint16_t* w, int64_t rows, int64_t K, int64_t ld, uint16_t* wf, hipStream_t stream);

/* Transposed fragment layouts, read by smel_gmm_bwd (no counterpart in the reference either; the same source tensors,
 * one more derived copy per frozen bank, int4 stays int4). For n_mats matrices [R][C] (the contraction runs over R):
 * with p = a pair of 32 columns, ks = a 64-row step, lane l = 16 kq + i, substep s, 16-column fragment fr:
 *   SMEL_PACK_Q4   block (mat, p, ks) 1 KB:  lane chunk word 2 fr + s = the 8 nibbles (low first) of column
 *                                             32 p + 16 fr + i at rows 64 ks + 32 s + 8 kq + [0, 8)
 *   SMEL_PACK_SZ   block (mat, g, ks) 512 B: fp32 pair 16 kq + 8 s + t = (scale, zero) of row 64 ks + 32 s + 8 kq + t
 *                                             in column group g (C / group groups); packed with fast = 1 the pair
 *                                             is (scale, zero - 1024 scale) for even t and (scale / 16,
 *                                             zero - 64 scale) for odd t, each an exact fp32 value
 *   SMEL_PACK_BF16 block (mat, p, ks, 2 fr + s) 1 KB: lane chunk = the 8 bf16 of that column at those rows
 * Rows >= R are zero. smel_packed_t_bytes gives the size of each (-1 for a bad argument). */
int64_t smel_packed_t_bytes(int32_t what, int64_t n_mats, int64_t R, int64_t C, int64_t group);
/* q [n_mats][R][C/2], scale/zero [n_mats][R][C/group] -> qt, szt. C a multiple of 32, group a multiple of 32
 * dividing C. */
int smel_pack_int4_t(const uint8_t* q, const uint16_t* scale, const uint16_t* zero, int64_t n_mats, int64_t R,
                     int64_t C, int64_t group, int32_t fast, uint8_t* qt, float* szt, hipStream_t stream);
/* w [n_mats][R][ld] bf16 (first C columns) -> wt. C a multiple of 32. */
int smel_pack_bf16_t(const uint16_t* w, int64_t n_mats, int64_t R, int64_t C, int64_t ld, uint16_t* wt,
                     hipStream_t stream);
/* Scale / zero groups [n] bf16 (any bank's scale and zero tensors) -> *ok = 1 if every group has z - 1024 s, z - 64 s
 * and s / 16 exactly representable as normal (or zero) fp32 values, else 0. Such a bank dequantizes with the cheaper
 * fp16-magic form in the GEMMs (same values, bit for bit); pack it with fast = 1 and set SMEL_WSET_FAST_DQ.
 * ok is device memory; the result is there when the stream reaches it. */
int smel_int4_fast_ok(const uint16_t* scale, const uint16_t* zero, int64_t n, int32_t* ok, hipStream_t stream);

/* ---- (A1) replaces route, smel/moe.py:162-167, plus the shared-expert gate logit of smel/moe.py:201.
 * x [T][H], gate_w [E][H] bf16 (E <= 512), shared_gate_w [H] or NULL. Writes probs [T][E] fp32 (softmax of the
 * bf16-rounded logits), topv [T][K] bf16 (renormalised), topi [T][K] int64 and topi32 [T][K] int32 (descending,
 * lower expert id first among equal logits), and, if shared_gate_w, sgate [T] fp32 = sigmoid(bf16(x . w_sg)).
 * topv32 [T][K] (optional) receives fp32(topv), the combine weight of the reference (topv.float(), :252).
 * logits [T][smel_route_ld(E, shared_gate_w != NULL)] bf16 is the caller's workspace; it is left holding the
 * bf16 logits (expert e in column e, the shared-gate logit in column ceil32(E)). */
int smel_route(const uint16_t* x, const uint16_t* gate_w, const uint16_t* shared_gate_w, int64_t T, int64_t H,
               int64_t E, int64_t K, float* probs, uint16_t* topv, float* topv32, int64_t* topi, int32_t* topi32,
               float* sgate, uint16_t* logits, hipStream_t stream);
/* smel_route that also counts the dispatch's histograms of its own topi (route followed by the dispatch of
 * routed_experts, smel/moe.py:162-167 then :216-223): disp_ws [smel_dispatch_ws_size(T*K, E)] int32 is the workspace
 * the following smel_dispatch_counted of the same topi takes; it is cleared here and left holding the per-block expert
 * counts, so the dispatch skips its histogram launch. Results otherwise those of smel_route. */
int smel_route_counted(const uint16_t* x, const uint16_t* gate_w, const uint16_t* shared_gate_w, int64_t T, int64_t H,
                       int64_t E, int64_t K, float* probs, uint16_t* topv, float* topv32, int64_t* topi,
                       int32_t* topi32, float* sgate, uint16_t* logits, int32_t* disp_ws, hipStream_t stream);
/* Row stride (elements) of smel_route's logits workspace (host-side, no GPU call); -1 for E <= 0. */
int64_t smel_route_ld(int64_t E, int32_t with_shared_gate);

/* Same selection from given bf16 logits [T][E], E <= 512 (bit-exact id checks against the CPU oracle). */
int smel_route_logits(const uint16_t* logits, int64_t T, int64_t E, int64_t K, float* probs, uint16_t* topv,
                      int64_t* topi, int32_t* topi32, hipStream_t stream);

/* ---- (A2) replaces route_gemma4, smel/moe.py:170-180 (the Gemma 4 router on the residual stream).
 * h [T][H] bf16, router_scale [H], proj_w [E][H], per_expert_scale [E] bf16 (E <= 512, H a multiple of 64):
 *   xn = bf16(bf16(bf16(h r) * router_scale) * H^-1/2), r = rstd[t] = (mean_j h[t][j]^2 + eps)^-1/2 (fp32),
 *   logits = bf16(xn proj_w^T), probs = softmax (fp32), top-k as smel_route, topv [T][K] fp32 = renormalised value
 *   * per_expert_scale[id]. xn [T][H], rstd [T] and logits [T][smel_route_ld(E, 0)] are caller workspaces, left
 *   holding those values (the backward reads rstd). */
int smel_route_gemma4(const uint16_t* h, const uint16_t* router_scale, const uint16_t* proj_w,
                      const uint16_t* per_expert_scale, int64_t T, int64_t H, int64_t E, int64_t K, float eps,
                      float* probs, float* topv, int64_t* topi, int32_t* topi32, uint16_t* xn, float* rstd,
                      uint16_t* logits, hipStream_t stream);
/* Backward of the router input of smel_route_gemma4 (autograd of smel/moe.py:172-174): dxn [T][H] bf16 = dL/dxn
 * (the router GEMM's dX) -> dh [T][H] bf16 = g r - h r^3 sum_j(g h)/H with g = bf16(bf16(dxn H^-1/2) router_scale).
 * The d(topv) -> dlogits step is smel_route_bwd with inv = NULL and per_expert_scale. */
int smel_route_gemma4_prenorm_bwd(const uint16_t* h, const uint16_t* router_scale, const float* rstd,
                                  const uint16_t* dxn, int64_t T, int64_t H, uint16_t* dh, hipStream_t stream);

/* ---- (A3) replaces the dispatch of routed_experts, smel/moe.py:216-223 and the inverse of :249-250.
 * ids [T*K] (int32 if ids_are_i64 == 0, else int64) -> counts [E], offsets [E+1], order [TK] (stable: experts
 * ascending, slot p ascending within one), inv [TK], and the GEMM tile list: tiles [max_tiles][4] = {group, row0,
 * row1, gk} over groups 0..E-1 (+ group E = shared rows [TK, TK+shared_rows) when shared_rows > 0), m_tile rows
 * each, gk = gkind[group] when gkind [E (+1)] is given (the GEMMs then need no gkind argument), else 0; n_tiles [1]
 * = how many are used. Order: the tiles of more than m_tile / 2 rows in group order, then the shorter (last) tiles
 * in group order. tiles_grouped (optional, [max_tiles][4]): the same tiles in group order (for SMEL_WSET_XCD_CHUNK).
 * err [1]: bit 0 set if an id is outside [0, E) (that slot is dropped, its
 * inv = -1), bit 1 if the tile list overflowed max_tiles. ws [smel_dispatch_ws_size(T*K, E)] int32 is the caller's
 * workspace. E <= 512.
 * merge_rows (0: off; m_tile < merge_rows <= 1.5 m_tile, needs gkind): also the merged list tiles_merged [max_tiles][4]
 * (n_tiles_merged [1] of them) for the forward GEMMs with SMEL_WSET_MERGED_LIST: a group of kind SMEL_KIND_INT4
 * whose last tile has at most merge_rows - m_tile rows gets it joined to the full tile before it (one tile of up to
 * merge_rows rows); order: those merged tiles, then the other tiles of more than m_tile / 2 rows, then the shorter
 * ones, each part in group order. */
int smel_dispatch(const void* ids, int32_t ids_are_i64, int64_t T, int64_t K, int64_t E, int64_t shared_rows,
                  int32_t m_tile, const int32_t* gkind, int32_t* counts, int32_t* offsets, int32_t* order,
                  int32_t* inv, int32_t* tiles, int32_t* tiles_grouped, int32_t* n_tiles, int32_t* err,
                  int32_t merge_rows, int32_t* tiles_merged, int32_t* n_tiles_merged, int32_t* ws, hipStream_t stream);
/* int32 elements of smel_dispatch's workspace (host-side, no GPU call); -1 for bad sizes. */
int64_t smel_dispatch_ws_size(int64_t TK, int64_t E);
/* smel_dispatch of the ids that smel_route_counted selected, with the workspace it filled: the histogram launch is
 * skipped (same results as smel_dispatch; ws must come from smel_route_counted of exactly these ids). */
int smel_dispatch_counted(const void* ids, int32_t ids_are_i64, int64_t T, int64_t K, int64_t E, int64_t shared_rows,
                          int32_t m_tile, const int32_t* gkind, int32_t* counts, int32_t* offsets, int32_t* order,
                          int32_t* inv, int32_t* tiles, int32_t* tiles_grouped, int32_t* n_tiles, int32_t* err,
                          int32_t merge_rows, int32_t* tiles_merged, int32_t* n_tiles_merged, int32_t* ws,
                          hipStream_t stream);
/* smel_dispatch without the workspace argument; it allocates nothing. No counterpart in the reference: it exists
 * for callers that cannot allocate device memory (code under HIP-graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). The workspace is a fixed array of smel_dispatch_noalloc_max_ws() int32 held by the library on
 * every GPU it runs on until the process ends; calls whose smel_dispatch_ws_size(T*K, E) exceeds it are rejected
 * (SMEL_EUNSUPPORTED). Every call on one GPU shares that GPU's array and each call rewrites all of the part it uses
 * before reading it, so nothing carries over between calls, but calls that overlap in time on one GPU (different
 * streams, or threads without ordering) race: order them on one stream. Results are those of smel_dispatch (without
 * the merged list: merge_rows 0). */
int smel_dispatch_noalloc(const void* ids, int32_t ids_are_i64, int64_t T, int64_t K, int64_t E, int64_t shared_rows,
                          int32_t m_tile, const int32_t* gkind, int32_t* counts, int32_t* offsets, int32_t* order,
                          int32_t* inv, int32_t* tiles, int32_t* tiles_grouped, int32_t* n_tiles, int32_t* err,
                          hipStream_t stream);
/* int32 capacity of smel_dispatch_noalloc's built-in workspace (host-side, no GPU call). */
int64_t smel_dispatch_noalloc_max_ws(void);
/* Upper bound of the tile-list length for smel_dispatch (host-side, no GPU call). */
int64_t smel_dispatch_max_tiles(int64_t TK, int64_t E, int64_t shared_rows, int32_t m_tile);

/* ---- LoRA factor layouts (smel/lora.py:14-58 params, fp32) -> the bf16 K-extension operands.
 * For n groups (n_sel selected slots, or 1 for the shared MLP) with rank r, hidden Hd, inter In, and `planes` 32-wide
 * planes for the gate_up side (1: r <= 16, gate and up packed in one plane; 2: r <= 32, gate in plane 0 and up in
 * plane 1; the down side always has one plane, r <= 32):
 *   planes = 1                                              planes = 2
 *   fwd_gu  [n][2In][32]: B_gate cols 0..r-1 of rows < In,   B_gate / B_up in cols 0..r-1 of their rows
 *                         B_up cols 16..16+r-1 of rows >= In
 *   a_gu    [n][32][Hd] : A_gate rows 0..r-1, A_up 16..       [2][n][32][Hd]: A_gate in plane 0, A_up in plane 1
 *   bt_gu   [n][32][2In]: B_gate^T rows 0.. / cols < In,     [2][n][32][2In]: plane 0 B_gate^T (cols < In), plane 1
 *                         B_up^T rows 16.. / cols >= In                        B_up^T (cols >= In)
 *   at_gu   [n][Hd][32] : a_gu transposed                    [n][2][Hd][32]: A_gate^T in plane 0, A_up^T in plane 1
 *   fwd_dn  [n][Hd][32] : B_down in cols 0..r-1
 *   a_dn    [n][32][In] : A_down rows 0..r-1                        (AD = act a_dn^T)
 *   bt_dn   [n][32][Hd] : B_down^T rows 0..r-1                       (DB = dy bt_dn^T)
 *   at_dn   [n][In][32] : a_dn transposed (backward ext of down)
 * Every other entry is 0. The LoRA of smel/lora.py takes any rank; ranks above 32 are rejected here. */
int smel_lora_prep(const float* A_gate, const float* B_gate, const float* A_up, const float* B_up,
                   const float* A_down, const float* B_down, int64_t n, int64_t r, int32_t planes, int64_t Hd,
                   int64_t In, uint16_t* fwd_gu, uint16_t* fwd_dn, uint16_t* a_gu, uint16_t* a_dn, uint16_t* bt_dn,
                   uint16_t* bt_gu, uint16_t* at_gu, uint16_t* at_dn, hipStream_t stream);
/* The same layouts for up to two LoRA sets of one layer (the selected experts' and the shared MLP's, same Hd, In and
 * planes) in one launch; a set with n = 0 is skipped. */
typedef struct smel_lora_set {
  const float *A_gate, *B_gate, *A_up, *B_up, *A_down, *B_down;
  int64_t n, r;
  uint16_t *fwd_gu, *fwd_dn, *a_gu, *a_dn, *bt_dn, *bt_gu, *at_gu, *at_dn;
} smel_lora_set;
int smel_lora_prep_sets(const smel_lora_set* sets, int32_t n_sets, int32_t planes, int64_t Hd, int64_t In,
                        hipStream_t stream);

/* ---- (A11/A12) LoRA down-projections of the rows of LoRA groups (SEL / SHARED tiles of the tile list):
 * ext[row * ldx + 0:32] = bf16(scale_g * A_src[src(row)][0:Kd] . wcat_g[0:32][0:Kd]) where src(row) = token of the row
 * if a_gather else row (A holds a_rows rows), wcat_g = wcat_sel + idx*32*Kd, scale_g = scale_sel (SEL) or wcat_sh,
 * scale_sh (SHARED). One call fills one 32-wide plane: ldx = 32 * planes, ext offset by 32 per plane. Rows of other
 * groups are left untouched. Kd must be a multiple of 32. */
int smel_lora_ext(const int32_t* tiles, const int32_t* n_tiles, int64_t max_tiles, const int32_t* gkind,
                  const uint16_t* A_src, int64_t lda, int64_t a_rows, int32_t a_gather, const int32_t* order,
                  int64_t TK, int64_t topk, const uint16_t* wcat_sel, const uint16_t* wcat_sh, int64_t Kd,
                  float scale_sel, float scale_sh, uint16_t* ext, int64_t ldx, hipStream_t stream);

/* ---- (A5/A6/A11) grouped expert GEMM, forward: out = A W^T per group, W from w (int4 dequantized in registers,
 * or bf16), plus the LoRA K-extension ext[row] . w.ext_*[n] for SEL/SHARED groups when ext != NULL.
 * epilogue 0: out[slot(row)][n] = bf16(acc), n < R                                  (down projection)
 * epilogue 1: gate/up pairs: g = bf16(acc[n]), u = bf16(acc[R/2 + n]), out[row][n] = bf16(act(g) u), n < R/2;
 *             if hsave: hsave[row][n] = g, hsave[row][R/2 + n] = u                  (gate_up projection)
 * A rows: A[token(row)] if a_gather else A[row]; A holds a_rows rows; K = w.C (multiple of 32). */
int smel_gmm_fwd(const smel_wset* w, const int32_t* gkind, const int32_t* tiles, const int32_t* n_tiles,
                 int64_t max_tiles, const uint16_t* A, int64_t lda, int64_t a_rows, int32_t a_gather,
                 const int32_t* order,
                 int64_t TK, int64_t topk, const uint16_t* ext, int32_t epilogue, int32_t act, uint16_t* out,
                 int64_t ldo, uint16_t* hsave, hipStream_t stream);
/* The down projection's LoRA rows without a separate smel_lora_ext launch (lora_linear's x A^T, smel/lora.py:61-69,
 * for the down LoRA of the selected / shared experts): */
typedef struct smel_fwd_lora_rows {
  const uint16_t* a_sel;  /* a_dn layout of the selected experts [n_sel][32][I] (smel_lora_prep), or NULL          */
  const uint16_t* a_sh;   /* a_dn layout of the shared expert [32][I], or NULL                                     */
  float scale_sel, scale_sh;
  float* part;            /* [rows][parts][32] fp32, 16-B aligned; NULL: off                                         */
  int32_t parts;          /* smel_gmm_fwd_nblocks(2 I, 1): the gate_up GEMM's column blocks                         */
  uint16_t* ext_out;      /* [rows][32] bf16, 16-B aligned, or NULL                                                 */
} smel_fwd_lora_rows;
/* smel_gmm_fwd with lr: the gate_up forward (epilogue 1) writes, for the rows of SEL / SHARED tiles whose LoRA set
 * is given, part[row][b][j] = scale * sum over column block b's columns c of h[row][c] a[j][c] (h = the bf16 SiLU-gate
 * output it stores); the down forward (epilogue 0, ext unused) takes ext[row][j] = bf16(sum_b part[row][b][j]) as
 * its K-extension rows and, if ext_out, stores them there (the LoRA gradients read them). */
int smel_gmm_fwd_lr(const smel_wset* w, const int32_t* gkind, const int32_t* tiles, const int32_t* n_tiles,
                    int64_t max_tiles, const uint16_t* A, int64_t lda, int64_t a_rows, int32_t a_gather,
                    const int32_t* order, int64_t TK, int64_t topk, const uint16_t* ext, int32_t epilogue, int32_t act,
                    uint16_t* out, int64_t ldo, uint16_t* hsave, const smel_fwd_lora_rows* lr, hipStream_t stream);
/* Column blocks of smel_gmm_fwd for R weight rows and the epilogue (host-side, no GPU call); -1 for R <= 0. */
int64_t smel_gmm_fwd_nblocks(int64_t R, int32_t epilogue);

/* ---- (A13) replaces the combine of routed_experts, smel/moe.py:248-252 (+ the shared add of :263):
 * out[t] = bf16( sum_k topv[t,k] * fp32(Y[t*K+k])  [+ sgate[t] * fp32(Ysh[t])] ), k in fixed order, topv fp32;
 * the shared expert's row Ysh[t] is Y[TK+t] (the fused shared expert) when Ysh is NULL, else row t of Ysh [T][H]
 * (a shared expert of another intermediate size, run as its own GEMMs). inv [T*K] (optional, smel_dispatch's): a slot
 * with inv < 0 (an expert id out of range, dropped by the dispatch) adds nothing. K <= 16. */
int smel_combine(const uint16_t* Y, const float* topv, const int32_t* inv, const float* sgate, const uint16_t* Ysh,
                 int64_t T, int64_t K, int64_t H, uint16_t* out, hipStream_t stream);

/* ---- (A10/A11 backward) grouped GEMM, backward: acc = A W per group (contraction over w.R), W in the transposed
 * layouts (smel_pack_int4_t / smel_pack_bf16_t), int4 re-dequantized in registers, plus ext[row] . w.ext_*[n][0:32]
 * for SEL/SHARED groups when ext != NULL. acc is rounded to bf16 before the epilogue (the reference's bf16 GEMM output).
 * epilogue 0: out[slot(row)][n] = bf16(acc), n < C                                   (dX of gate_up: dh W_gu)
 * epilogue 1: down backward, n < C = I: da = w(row) acc with w(row) = topv[p] (fp32) or sgate[t]; (g, u) = hsave[row];
 *             out[row][n] = bf16(da u act'(g)), out[row][I+n] = bf16(da act(g));
 *             dwp[row][j] = sum over column block j of acc * bf16(act(g) u)   (d row weight, reduced later in
 *             fixed order); dwp holds (rows) x smel_gmm_bwd_nblocks(C) floats; bf16(act(g) u) is recomputed from
 *             the saved bf16 (g, u) exactly as smel_gmm_fwd's epilogue 1 computed it (the value the forward stored)
 * A rows: A[token(row)] if a_gather else A[row]; A holds a_rows rows; the GEMM K = w.R. */
int smel_gmm_bwd(const smel_wset* w, const int32_t* gkind, const int32_t* tiles, const int32_t* n_tiles,
                 int64_t max_tiles, const uint16_t* A, int64_t lda, int64_t a_rows, int32_t a_gather,
                 const int32_t* order,
                 int64_t TK, int64_t topk, const uint16_t* ext, int32_t epilogue, int32_t act,
                 const uint16_t* hsave, const float* topv, const float* sgate, uint16_t* out, int64_t ldo,
                 float* dwp, hipStream_t stream);
/* number of column blocks (dwp row width) smel_gmm_bwd uses for a given C */
int64_t smel_gmm_bwd_nblocks(int64_t C);
/* The gate_up backward's LoRA rows without a separate smel_lora_ext launch (the autograd of lora_gate_up's B
 * products, smel/lora.py:72-83: DXA = s [dg B_g, du B_u] per row of a selected / shared expert with a LoRA): */
typedef struct smel_bwd_lora_rows {
  const uint16_t* bt_sel;  /* bt_gu layout of the selected experts [planes][n_sel][32][2 I] (smel_lora_prep), or NULL */
  const uint16_t* bt_sh;   /* bt_gu layout of the shared expert [planes][1][32][2 I], or NULL                         */
  float scale_sel, scale_sh;
  int32_t n_sel;           /* selected slots of bt_sel (its plane stride)                                             */
  int32_t planes;          /* 1 or 2, as the weight set's SMEL_WSET_EXT2                                              */
  float* part;             /* [rows][parts][planes][32] fp32, 16-B aligned; NULL: off                                 */
  int32_t parts;           /* smel_gmm_bwd_nblocks(I): the down backward's column blocks                              */
} smel_bwd_lora_rows;
/* smel_gmm_bwd with lr: the down backward (epilogue 1) writes, for the rows of SEL / SHARED tiles whose bt_* is given,
 * part[row][b][c][j] = scale * sum over column block b's columns n of (dg[row][n] bt[c][j][n] + du[row][n]
 * bt[c][j][I+n]) from the bf16 dg / du it stores; the gate_up backward (epilogue 0, ext NULL) takes
 * ext[row][32 c + j] = bf16(sum_b part[row][b][c][j]) (b ascending, fp32) as its K-extension rows. */
int smel_gmm_bwd_lr(const smel_wset* w, const int32_t* gkind, const int32_t* tiles, const int32_t* n_tiles,
                    int64_t max_tiles, const uint16_t* A, int64_t lda, int64_t a_rows, int32_t a_gather,
                    const int32_t* order, int64_t TK, int64_t topk, const uint16_t* ext, int32_t epilogue, int32_t act,
                    const uint16_t* hsave, const float* topv, const float* sgate, uint16_t* out, int64_t ldo,
                    float* dwp, const smel_bwd_lora_rows* lr, hipStream_t stream);
/* The same rows as bf16 [rows][32 * planes] for the LoRA gradients: ext[row][32 c + j] = bf16(sum_b part[row][b][c][j])
 * for the rows of SEL tiles (sel != 0) and SHARED tiles (sh != 0) of the tile list; other rows are left untouched. */
int smel_lora_rows_sum(const int32_t* tiles, const int32_t* n_tiles, int64_t max_tiles, const int32_t* gkind,
                       int32_t sel, int32_t sh, const float* part, int32_t parts, int32_t planes, uint16_t* ext,
                       hipStream_t stream);

/* ---- (A15) router backward (autograd of route + renorm + the shared gate, smel/moe.py:162-167, 201):
 * dtopv[t,k] = sum_j dwp[inv[t*K+k]][j]; d renorm; d gather; d softmax (probs) -> dlogits [T][ldl] bf16 with
 * dlogits[t][E] = d shared-gate logit (sum_j dwp[TK+t][j] * sg (1-sg), or with dwp_sh != NULL sum_j dwp_sh[t][j] over
 * its nblk_sh columns: the shared expert run as its own GEMMs) when sgate != NULL, zero padding to ldl.
 * dtopv_out [T][K] fp32 (optional) receives dtopv. inv = NULL: dwp rows are the slots t*K+k themselves (TK = T*K).
 * per_expert_scale [E] bf16 (optional, route_gemma4): the routed value was renorm * per_expert_scale[id], so dtopv
 * is multiplied by it before the renorm backward. */
int smel_route_bwd(const float* dwp, int64_t nblk, const int32_t* inv, const float* probs, const int32_t* topi32,
                   const float* sgate, const float* dwp_sh, int64_t nblk_sh, int64_t T, int64_t K, int64_t E,
                   int64_t TK, uint16_t* dlogits, int64_t ldl, float* dtopv_out, const uint16_t* per_expert_scale,
                   hipStream_t stream);

/* d(combine weight) of routed_experts when topv is an input: dtopv[p] = sum_j dwp[inv[p]][j], fp32 [TK]. */
int smel_dtopv(const float* dwp, int64_t nblk, const int32_t* inv, int64_t TK, float* dtopv, hipStream_t stream);

/* ---- dX of the layer: dx[t] = bf16( sum_k DXS[t*K+k] + [shared row] + [DXR[t]] ), fixed order, fp32; the shared row
 * (with_shared) is DXS[TK+t], or DXSH[t] when dxsh is given; slots with inv < 0 (inv optional, as in smel_combine)
 * add nothing. K <= 16. */
int smel_dx_reduce(const uint16_t* dxs, const uint16_t* dxr, const int32_t* inv, int32_t with_shared,
                   const uint16_t* dxsh, int64_t T, int64_t K, int64_t H, uint16_t* dx, hipStream_t stream);

/* ---- LoRA weight gradients (autograd of smel/lora.py:61-83 for the selected experts and the shared MLP), up to six
 * products in one launch (four; six when the gate_up side has two planes, one job per plane). For job j and every
 * LoRA group lora_groups[i] (expert id, or E for the shared rows [TK, TK+T)):
 *   R[p][q] = sum_{rows of the group} alpha(row) * L[row * ldl + p] * Rm[src(row)][q],  p < 32, q < Q
 * summed in one fixed order (deterministic). src(row) = token of the row if r_gather else row; Rm holds r_rows rows;
 * alpha = the row weight (topv[p] fp32 / sgate[t]) if use_w, else 1 (folded into L before its bf16 rounding).
 * Each R[p][q] with p in [p0, p0+np) and q in [q0, q0+nq) of a destination is stored (fp32) at
 *   ptr[slot * s_idx + (p - p0) * s_p + (q - q0) * s_q],
 * dest[0][h] for groups i < n_sel (slot = i, the selected experts' LoRA tensors), dest[1][h] for the others (slot 0,
 * the shared MLP's), h = 0, 1 for the two halves (gate / up) of a gate_up product; ptr NULL = not stored. Q must be a
 * multiple of 16. */
typedef struct smel_wg_dest {
  float* ptr;
  int64_t s_idx, s_p, s_q;
  int32_t p0, np, q0, nq;
} smel_wg_dest;
typedef struct smel_wg_job {
  const uint16_t* L;   /* bf16 LoRA K-extension rows of the direction, ldl elements apart (32 p's used)   */
  const uint16_t* Rm;  /* right operand rows, ldr elements apart                                          */
  int64_t ldr, r_rows;
  int32_t r_gather, use_w;
  int64_t Q;
  int64_t ldl;         /* 32 or 64 (a plane of two-plane ext rows; L then points at the plane's column 0) */
  smel_wg_dest dest[2][2];
} smel_wg_job;
/* Groups of more than 512 rows are cut into 512-row chunks whose fp32 partial tiles go to the caller's workspace ws
 * (ws_floats >= smel_lora_wgrad_ws_floats(jobs, n_jobs, n_lora, max_rows), max_rows >= the rows of all LoRA groups
 * together) and are summed in chunk order by a second launch. */
int64_t smel_lora_wgrad_ws_floats(const smel_wg_job* jobs, int32_t n_jobs, int64_t n_lora, int64_t max_rows);
int smel_lora_wgrad(const smel_wg_job* jobs, int32_t n_jobs, const int32_t* lora_groups, int64_t n_lora,
                    int64_t n_sel, const int32_t* offsets, int64_t E, int64_t T, int64_t TK, int64_t topk,
                    const int32_t* order, const float* topv, const float* sgate, int64_t max_rows, float* ws,
                    int64_t ws_floats, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
