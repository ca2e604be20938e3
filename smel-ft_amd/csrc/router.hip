// Router: logits = x W_r^T (bf16 MFMA, fp32 accumulation, bf16-rounded like F.linear in bf16), softmax in fp32,
// top-k (descending, lower expert id first among equal logits), renormalisation; and its backward.
// Reference: route, smel/moe.py:162-167; the shared-expert gate logit of shared_mlp, smel/moe.py:201.
#include <math.h>

#include "abi_util.h"
#include "common.h"

namespace {

constexpr int MAXE = 512;      // experts handled by the selection (up to 8 logits per lane)

// Selection over one token's logits (held in LDS or global), by one wave; NPL = logits per lane (E <= 64 NPL).
// Writes probs, topi, topi32 and the renormalised values: topv bf16 and topv32 = the same rounded value as fp32
// (route), or topv_f32 = fp32 value times per_expert_scale[id] (route_gemma4).
template <int NPL, typename Get>
SMEL_DEV void select_topk(Get logit, int E, int K, int64_t t, float* __restrict__ probs, uint16_t* __restrict__ topv,
                          float* __restrict__ topv32, int64_t* __restrict__ topi, int32_t* __restrict__ topi32,
                          float* __restrict__ topv_f32, const uint16_t* __restrict__ pes,
                          int32_t* __restrict__ hist) {
  const int l = lane_id();
  float v[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = l + 64 * j;
    v[j] = e < E ? logit(e) : -INFINITY;
  }
  float m = v[0];
#pragma unroll
  for (int j = 1; j < NPL; ++j) m = fmaxf(m, v[j]);
  m = wave_max(m);
  float ex[NPL], s = 0.f;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    ex[j] = (l + 64 * j) < E ? expf(v[j] - m) : 0.f;
    s += ex[j];
  }
  s = wave_sum(s);
  const float inv_s = 1.0f / s;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = l + 64 * j;
    if (e < E) probs[t * E + e] = ex[j] * inv_s;
  }
  // top-k: K rounds of a wave-wide max over 32-bit keys (bf16 logit in an order-preserving form above 0xffff - e):
  // one compare per step for (value desc, index asc); a taken expert's key becomes 0
  uint32_t key[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = l + 64 * j;
    uint32_t b = __float_as_uint(v[j]) >> 16;   // the logit's bf16 bits
    if (b == 0x8000u) b = 0u;                   // -0 ties with +0
    const uint32_t ord = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
    key[j] = e < E ? (ord << 16) | (0xffffu - (uint32_t)e) : 0u;
  }
  float pk[16];
  int ik[16];
  float psum = 0.f;
  for (int k = 0; k < K; ++k) {
    uint32_t best = key[0];
#pragma unroll
    for (int j = 1; j < NPL; ++j) best = max(best, key[j]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) best = max(best, (uint32_t)__shfl_xor((int)best, o, 64));
    const int bi = (int)(0xffffu - (best & 0xffffu));
#pragma unroll
    for (int j = 0; j < NPL; ++j)
      if (bi == l + 64 * j) key[j] = 0u;
    const uint32_t ob = best >> 16;
    const float bv = __uint_as_float(((ob & 0x8000u) ? (ob & 0x7fffu) : (~ob & 0xffffu)) << 16);
    ik[k] = bi;
    pk[k] = expf(bv - m) * inv_s;   // the same expression as probs[t][bi]
    psum += pk[k];
  }
  if (l < K) {
    float p = 0.f;
    int i = 0;
    for (int k = 0; k < K; ++k)
      if (k == l) {
        p = pk[k];
        i = ik[k];
      }
    if (topv_f32) {
      topv_f32[t * K + l] = pes ? (p / psum) * bf2f(pes[i]) : p / psum;   // route_gemma4: fp32, x per-expert scale
    } else {
      const uint16_t b = f2bf(p / psum);
      topv[t * K + l] = b;
      if (topv32) topv32[t * K + l] = bf2f(b);   // the combine weight the reference uses: fp32 of the bf16 value
    }
    topi[t * K + l] = i;
    topi32[t * K + l] = i;
    // the dispatch's per-block histogram: an integer count, the same whatever order the adds land in
    if (hist) atomicAdd(&hist[(int)((t * K + l) / DISPATCH_SLOTS) * E + i], 1);
  }
}

// ---- logits GEMM: logits[t][c] = bf16(x[t] . w_c) for c < E (w_c = gate row c), at c = E32 = ceil32(E) the
// shared-gate logit x[t] . w_sg (when sg), other columns 0. Block = 64 tokens x 96 columns, 4 waves; wave w takes
// tokens 16 w .. 16 w + 15 against all 96 columns (v_mfma_f32_16x16x32_bf16, 6 column fragments) over the whole
// hidden dim, so no partial sums are reduced. Per 64-wide k-step the block stages the 96 weight rows once in LDS
// (LDS-DMA, 8-stage ring, XOR-swizzled 16-B chunks) and each wave loads its own 16 x rows into registers seven steps
// ahead (a step's MFMA work is short next to a load's latency, so the depth sets the kernel's speed): x is read once
// per column block and the weights once per 64 tokens. Grid = ceil(T / 64) x ceil(ldl / 96).
constexpr int RT = 64;
constexpr int RC = 96;
constexpr int RKT = 64;
constexpr int RSTAGE = RC * RKT;   // bf16 elements of one weight stage (12 KB)
// Vector-memory operations per wave in each issue group of the logits loop (the issue code is written with these
// counts; the wait is computed from them): 2 x-row loads into registers, 3 weight-row LDS-DMAs
constexpr int RVM_X = 2;
constexpr int RVM_W = RSTAGE * 2 / (4 * 1024);
constexpr int RNST = 8;                        // ring stages: loads run RNST - 1 steps ahead
constexpr int R_WAIT = (RNST - 2) * (RVM_X + RVM_W);   // steps j+1 .. j+RNST-2 may be in flight while step j computes

SMEL_DEV f32x4_t mfma16r(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}

__global__ __launch_bounds__(256) void route_logits_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ gw,
                                                           const uint16_t* __restrict__ sg, int T, int H, int E,
                                                           int ldl, uint16_t* __restrict__ logits,
                                                           int32_t* __restrict__ zero_ws, int zero_n) {
  __shared__ __attribute__((aligned(1024))) uint16_t WS[RNST][RSTAGE];
  if (zero_ws) {   // the dispatch workspace the selection counts into (the selection runs after this launch)
    const int nblk = gridDim.x * gridDim.y, b = blockIdx.y * gridDim.x + blockIdx.x;
    for (int i = b * 256 + (int)threadIdx.x; i < zero_n; i += nblk * 256) zero_ws[i] = 0;
  }
  const int tid = threadIdx.x, l = lane_id(), kq = l >> 4, li = l & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t0 = blockIdx.x * RT, c0 = blockIdx.y * RC;
  const int E32 = (E + 31) / 32 * 32;
  const int nk = H / RKT;
  // weight staging: wave-load ii of wave w fills weight rows 8 g .. 8 g + 7 (g = 3 w + ii) of a stage; lane i writes
  // physical chunk i % 8 of row 8 g + i / 8 = logical chunk (i % 8) ^ swz(row). A group of 8 rows is all gate rows or
  // all past E32 (E32 and c0 are multiples of 8), so one descriptor serves the wave-load.
  const rsrc_t rg = make_rsrc(gw, (uint64_t)E * H * 2);
  const rsrc_t rsg = make_rsrc(sg ? sg : gw, sg ? (uint64_t)H * 2 : 0);
  rsrc_t rb[RVM_W];
  uint32_t boff[RVM_W];
#pragma unroll
  for (int ii = 0; ii < RVM_W; ++ii) {
    const int row = 8 * (RVM_W * w + ii) + (l >> 3);
    const int c = c0 + row;
    const int ch = (l & 7) ^ swz(row);
    const bool gate = c0 + 8 * (RVM_W * w + ii) < E32;   // uniform
    rb[ii] = gate ? rg : rsg;
    boff[ii] = gate ? (c < E ? (uint32_t)c * H * 2 + 16 * ch : OOB) : ((sg && c == E32) ? 16u * ch : OOB);
  }
  // x rows of this wave: lane (kq, li) holds token 16 w + li, k = 32 s + 8 kq + [0, 8) in substep s
  const rsrc_t rx = make_rsrc(x, (uint64_t)T * H * 2);
  const int tok = t0 + 16 * w + li;
  const uint32_t xoff = tok < T ? (uint32_t)tok * H * 2 + 16 * kq : OOB;
  auto issue = [&](int j, u32x4_t* xa) {
    const bool in = j < nk;
    const uint32_t k2 = (uint32_t)j * RKT * 2;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < RVM_X; ++s) xa[s] = ld16(rx, in ? xoff + k2 + 64 * s : OOB);
#pragma unroll
    for (int ii = 0; ii < RVM_W; ++ii)
      ld16_lds(rb[ii], &WS[j % RNST][(RVM_W * w + ii) * 512], in ? boff[ii] + k2 : OOB);
    __builtin_amdgcn_sched_barrier(0);
  };
  // weight fragment reads: column fragment f, substep s, lane (kq, li) -> row 16 f + li, logical chunk 4 s + kq
  uint32_t brd[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) brd[s] = li * RKT + 8 * ((4 * s + kq) ^ swz(li));
  f32x4_t acc[6];
#pragma unroll
  for (int f = 0; f < 6; ++f) acc[f] = f32x4_t{};
  u32x4_t X[RNST][RVM_X];   // x rows of the steps in flight, register set j % RNST
  auto compute = [&](int j, const u32x4_t* xa) {
    const uint16_t* S = WS[j % RNST];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int f = 0; f < 6; ++f)
        acc[f] = mfma16r(xa[s], *reinterpret_cast<const u32x4_t*>(S + brd[s] + f * 16 * RKT), acc[f]);
  };
  // RNST - 1 steps ahead; per step and wave 2 x loads (registers) + 3 weight DMAs: before step j only steps
  // j+1 .. j+RNST-2 may still be in flight
#pragma unroll
  for (int s = 0; s < RNST - 1; ++s) issue(s, X[s]);
  for (int j = 0; j < nk; j += RNST) {
#pragma unroll
    for (int u = 0; u < RNST; ++u) {
      wait_vm_lds<R_WAIT>();
      __builtin_amdgcn_s_barrier();
      issue(j + u + RNST - 1, X[(u + RNST - 1) % RNST]);
      compute(j + u, X[u]);
    }
  }
  wait_vm<0>();   // the trailing (out-of-range) loads
  // D[4 kq + r][li] of fragment f: token 16 w + 4 kq + r, column c0 + 16 f + li
#pragma unroll
  for (int f = 0; f < 6; ++f) {
    const int c = c0 + 16 * f + li;
    if (c >= ldl) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 16 * w + 4 * kq + r;
      if (t < T) logits[(int64_t)t * ldl + c] = f2bf(acc[f][r]);
    }
  }
}

// ---- selection: one wave per token over its bf16 logits row (probs, top-k, renorm; shared-gate sigmoid).
template <int NPL>
__global__ __launch_bounds__(256) void route_select(const uint16_t* __restrict__ logits, int ldl, int T, int E, int K,
                                                    int sg_col, float* __restrict__ probs,
                                                    uint16_t* __restrict__ topv, float* __restrict__ topv32,
                                                    int64_t* __restrict__ topi, int32_t* __restrict__ topi32,
                                                    float* __restrict__ sgate, float* __restrict__ topv_f32,
                                                    const uint16_t* __restrict__ pes, int32_t* __restrict__ hist) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const uint16_t* row = logits + t * ldl;
  select_topk<NPL>([&](int e) { return bf2f(row[e]); }, E, K, t, probs, topv, topv32, topi, topi32, topv_f32, pes,
                   hist);
  if (sgate && lane_id() == 0) sgate[t] = 1.0f / (1.0f + expf(-bf2f(row[sg_col])));
}

// The selection launch for E experts: 4 logits per lane up to 256 experts, 8 up to 512.
void launch_select(hipStream_t stream, const uint16_t* logits, int ldl, int T, int E, int K, int sg_col, float* probs,
                   uint16_t* topv, float* topv32, int64_t* topi, int32_t* topi32, float* sgate, float* topv_f32,
                   const uint16_t* pes, int32_t* hist = nullptr) {
  const unsigned grid = (unsigned)((T + 3) / 4);
  if (E <= 256)
    route_select<4><<<grid, 256, 0, stream>>>(logits, ldl, T, E, K, sg_col, probs, topv, topv32, topi, topi32, sgate,
                                               topv_f32, pes, hist);
  else
    route_select<8><<<grid, 256, 0, stream>>>(logits, ldl, T, E, K, sg_col, probs, topv, topv32, topi, topi32, sgate,
                                               topv_f32, pes, hist);
}

// Backward of route (+ shared gate): one wave per token.
//   dtopv[k] = sum_j dwp[inv[t*K+k]][j]  (d of the combine weight; dwp holds per-column-block partials)
//   renorm:  topv_k = p_k / S  ->  dp_k = (dtopv_k - sum_j dtopv_j topv_j) / S
//   softmax: dlogit_e = p_e (dp_e - sum_k dp_k p_{i_k}),  dp_e = 0 off the top-k
//   shared gate: dlogit_sg = (sum_j dwp[TK+t][j]) * sg (1 - sg)
__global__ __launch_bounds__(256) void route_bwd(const float* __restrict__ dwp, int nblk,
                                                 const int32_t* __restrict__ inv, const float* __restrict__ probs,
                                                 const int32_t* __restrict__ topi32, const float* __restrict__ sgate,
                                                 const float* __restrict__ dwp_sh, int nblk_sh, int T, int K, int E,
                                                 int TK,
                                                 uint16_t* __restrict__ dlogits, int ldl,
                                                 float* __restrict__ dtopv_out, const uint16_t* __restrict__ pes) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int l = lane_id();
  // per-k quantities, lane k holds slot k
  float dtv = 0.f, p = 0.f;
  int idx = -1;
  if (l < K) {
    // -1 for a slot the dispatch dropped (id out of range); no inv = dwp rows are the slots themselves
    const int row = inv ? inv[t * K + l] : (int)(t * K + l);
    if (row >= 0)
      for (int j = 0; j < nblk; ++j) dtv += dwp[(int64_t)row * nblk + j];
    idx = topi32[t * K + l];
    if (idx >= 0 && idx < E) p = probs[t * E + idx];
    else idx = -1;
    if (dtopv_out) dtopv_out[t * K + l] = dtv;
    if (pes && idx >= 0) dtv *= bf2f(pes[idx]);   // route_gemma4's topv = renorm * per_expert_scale[i]
  }
  // S = sum_k p_k ; topv_k = p_k / S (recomputed in fp32, not the bf16-rounded copy)
  float S = 0.f, dot = 0.f;
  for (int k = 0; k < K; ++k) S += __shfl(p, k, 64);
  const float tv = (l < K) ? p / S : 0.f;
  for (int k = 0; k < K; ++k) dot += __shfl(dtv * tv, k, 64);
  const float dp = (l < K) ? (dtv - dot) / S : 0.f;
  float pdp = 0.f;   // sum_k dp_k p_k
  for (int k = 0; k < K; ++k) pdp += __shfl(dp * p, k, 64);
  // every lane gets the K (id, dp) pairs before any lane-divergent code (a shuffle only reads active lanes)
  int ik[16];
  float dk[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    ik[k] = k < K ? __shfl(idx, k, 64) : -1;
    dk[k] = k < K ? __shfl(dp, k, 64) : 0.f;
  }
  for (int e = l; e < ldl; e += 64) {
    float g = 0.f;
    if (e < E) {
      float dpe = 0.f;
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (ik[k] == e) dpe = dk[k];
      g = probs[t * E + e] * (dpe - pdp);
    } else if (e == E && sgate) {
      float ds = 0.f;
      if (dwp_sh)   // the shared expert ran as its own GEMMs: its row-weight partials, [T][nblk_sh]
        for (int j = 0; j < nblk_sh; ++j) ds += dwp_sh[t * nblk_sh + j];
      else
        for (int j = 0; j < nblk; ++j) ds += dwp[(int64_t)(TK + t) * nblk + j];
      const float sgv = sgate[t];
      g = ds * sgv * (1.0f - sgv);
    }
    dlogits[t * ldl + e] = f2bf(g);
  }
}

// ---- Gemma 4 router input (smel/moe.py:170-180): one wave per token of the residual stream h [T][H]:
//   r = (mean(h^2) + eps)^-1/2 (fp32), xn = bf16(bf16(bf16(h r) * router.scale) * H^-1/2)  (the reference's roundings:
//   .type_as(h), then two bf16 products); rstd[t] = r is kept for the backward.
__global__ __launch_bounds__(256) void route_prenorm(const uint16_t* __restrict__ h, const uint16_t* __restrict__ scale,
                                                     int T, int H, float eps, float hs, uint16_t* __restrict__ xn,
                                                     float* __restrict__ rstd) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int l = lane_id();
  const u32x4_t* row = reinterpret_cast<const u32x4_t*>(h + t * H);
  const int nc = H / 8;
  float ss = 0.f;
  for (int c = l; c < nc; c += 64) {
    const u32x4_t v = row[c];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = bf_lo(v[j]), b = bf_hi(v[j]);
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / (float)H + eps);
  const u32x4_t* sc = reinterpret_cast<const u32x4_t*>(scale);
  u32x4_t* out = reinterpret_cast<u32x4_t*>(xn + t * H);
  for (int c = l; c < nc; c += 64) {
    const u32x4_t v = row[c], g = sc[c];
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = bf2f(f2bf(bf2f(f2bf(bf_lo(v[j]) * r)) * bf_lo(g[j]))) * hs;
      const float b = bf2f(f2bf(bf2f(f2bf(bf_hi(v[j]) * r)) * bf_hi(g[j]))) * hs;
      o[j] = pack2bf(a, b);
    }
    out[c] = u32x4_t{o[0], o[1], o[2], o[3]};
  }
  if (l == 0) rstd[t] = r;
}

// Backward of route_prenorm given dxn = dL/dxn [T][H] bf16 (the router GEMM's dX): g = bf16(bf16(dxn H^-1/2) scale)
// (the bf16 products' backward), then the RMSNorm backward in fp32: dh = g r - h r^3 sum(g h) / H.
__global__ __launch_bounds__(256) void route_prenorm_bwd(const uint16_t* __restrict__ h,
                                                         const uint16_t* __restrict__ scale,
                                                         const float* __restrict__ rstd,
                                                         const uint16_t* __restrict__ dxn, int T, int H, float hs,
                                                         uint16_t* __restrict__ dh) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int l = lane_id();
  const u32x4_t* hr = reinterpret_cast<const u32x4_t*>(h + t * H);
  const u32x4_t* dr = reinterpret_cast<const u32x4_t*>(dxn + t * H);
  const u32x4_t* sc = reinterpret_cast<const u32x4_t*>(scale);
  const int nc = H / 8;
  auto gval = [&](uint32_t d, uint32_t s, int hi_half) {
    const float dv = hi_half ? bf_hi(d) : bf_lo(d), sv = hi_half ? bf_hi(s) : bf_lo(s);
    return bf2f(f2bf(bf2f(f2bf(dv * hs)) * sv));
  };
  float dot = 0.f;
  for (int c = l; c < nc; c += 64) {
    const u32x4_t v = hr[c], d = dr[c], g = sc[c];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dot = fmaf(gval(d[j], g[j], 0), bf_lo(v[j]), dot);
      dot = fmaf(gval(d[j], g[j], 1), bf_hi(v[j]), dot);
    }
  }
  dot = wave_sum(dot);
  const float r = rstd[t];
  const float c3 = r * r * r * dot / (float)H;
  u32x4_t* out = reinterpret_cast<u32x4_t*>(dh + t * H);
  for (int c = l; c < nc; c += 64) {
    const u32x4_t v = hr[c], d = dr[c], g = sc[c];
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack2bf(gval(d[j], g[j], 0) * r - bf_lo(v[j]) * c3, gval(d[j], g[j], 1) * r - bf_hi(v[j]) * c3);
    out[c] = u32x4_t{o[0], o[1], o[2], o[3]};
  }
}

__global__ __launch_bounds__(256) void dtopv_kernel(const float* __restrict__ dwp, int nblk,
                                                    const int32_t* __restrict__ inv, int TK, float* __restrict__ out) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= TK) return;
  const int row = inv[p];
  float v = 0.f;
  if (row >= 0)
    for (int j = 0; j < nblk; ++j) v += dwp[(int64_t)row * nblk + j];
  out[p] = v;
}

void launch_logits(hipStream_t stream, const uint16_t* x, const uint16_t* gw, const uint16_t* sg, int T, int H, int E,
                   int ldl, uint16_t* logits, int32_t* zero_ws = nullptr, int zero_n = 0) {
  const dim3 grid((unsigned)((T + RT - 1) / RT), (unsigned)((ldl + RC - 1) / RC));
  route_logits_kernel<<<grid, 256, 0, stream>>>(x, gw, sg, T, H, E, ldl, logits, zero_ws, zero_n);
}


}  // namespace

extern "C" int smel_dtopv(const float* dwp, int64_t nblk, const int32_t* inv, int64_t TK, float* dtopv,
                          hipStream_t stream) {
  SMEL_REQUIRE(nblk > 0 && TK >= 0, SMEL_EINVAL, "dtopv: bad sizes");
  if (TK == 0) return 0;
  SMEL_REQUIRE(dwp && inv && dtopv, SMEL_EINVAL, "dtopv: null pointer");
  dtopv_kernel<<<(unsigned)((TK + 255) / 256), 256, 0, stream>>>(dwp, (int)nblk, inv, (int)TK, dtopv);
  return smel::launch_status();
}

extern "C" int64_t smel_route_ld(int64_t E, int32_t with_shared_gate) {
  return E <= 0 ? -1 : (E + 31) / 32 * 32 + (with_shared_gate ? 32 : 0);
}

namespace {
int route_impl(const uint16_t* x, const uint16_t* gate_w, const uint16_t* shared_gate_w, int64_t T, int64_t H,
               int64_t E, int64_t K, float* probs, uint16_t* topv, float* topv32, int64_t* topi, int32_t* topi32,
               float* sgate, uint16_t* logits, int32_t* disp_ws, hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && H > 0 && E > 0 && K > 0, SMEL_EINVAL, "route: bad sizes");
  SMEL_REQUIRE(E <= MAXE, SMEL_EUNSUPPORTED, "route: E=%lld > %d experts", (long long)E, MAXE);
  SMEL_REQUIRE(K <= E && K <= 16, SMEL_EUNSUPPORTED, "route: top_k=%lld must be <= min(E, 16)", (long long)K);
  SMEL_REQUIRE(H % 64 == 0, SMEL_EUNSUPPORTED, "route: hidden %lld must be a multiple of 64", (long long)H);
  SMEL_REQUIRE(!shared_gate_w || sgate, SMEL_EINVAL, "route: sgate output needed with shared_gate_w");
  SMEL_REQUIRE(T * H * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "route: x larger than 2 GiB");
  SMEL_REQUIRE(T * K < (1ll << 30), SMEL_EUNSUPPORTED, "route: T*K too large");
  if (T == 0) return 0;
  SMEL_REQUIRE(x && gate_w && probs && topv && topi && topi32 && logits, SMEL_EINVAL, "route: null pointer");
  const int64_t ldl = smel_route_ld(E, shared_gate_w != nullptr);
  // the dispatch workspace: [ceil(T K / 1024)][E] histogram counts, then one bad-id flag per block (smel_dispatch)
  const int64_t nb = (T * K + DISPATCH_SLOTS - 1) / DISPATCH_SLOTS;
  launch_logits(stream, x, gate_w, shared_gate_w, (int)T, (int)H, (int)E, (int)ldl, logits, disp_ws,
                (int)(disp_ws ? nb * E + nb : 0));
  launch_select(stream, logits, (int)ldl, (int)T, (int)E, (int)K, (int)((E + 31) / 32 * 32), probs, topv, topv32,
                topi, topi32, shared_gate_w ? sgate : nullptr, nullptr, nullptr, disp_ws);
  return smel::launch_status();
}
}  // namespace

extern "C" int smel_route(const uint16_t* x, const uint16_t* gate_w, const uint16_t* shared_gate_w, int64_t T,
                          int64_t H, int64_t E, int64_t K, float* probs, uint16_t* topv, float* topv32, int64_t* topi,
                          int32_t* topi32, float* sgate, uint16_t* logits, hipStream_t stream) {
  return route_impl(x, gate_w, shared_gate_w, T, H, E, K, probs, topv, topv32, topi, topi32, sgate, logits, nullptr,
                    stream);
}

extern "C" int smel_route_counted(const uint16_t* x, const uint16_t* gate_w, const uint16_t* shared_gate_w,
                                  int64_t T, int64_t H, int64_t E, int64_t K, float* probs, uint16_t* topv,
                                  float* topv32, int64_t* topi, int32_t* topi32, float* sgate, uint16_t* logits,
                                  int32_t* disp_ws, hipStream_t stream) {
  SMEL_REQUIRE(disp_ws || T == 0, SMEL_EINVAL, "route_counted: null dispatch workspace");
  return route_impl(x, gate_w, shared_gate_w, T, H, E, K, probs, topv, topv32, topi, topi32, sgate, logits, disp_ws,
                    stream);
}

extern "C" int smel_route_logits(const uint16_t* logits, int64_t T, int64_t E, int64_t K, float* probs,
                                 uint16_t* topv, int64_t* topi, int32_t* topi32, hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && E > 0 && K > 0, SMEL_EINVAL, "route_logits: bad sizes");
  SMEL_REQUIRE(E <= MAXE, SMEL_EUNSUPPORTED, "route_logits: E=%lld > %d", (long long)E, MAXE);
  SMEL_REQUIRE(K <= E && K <= 16, SMEL_EUNSUPPORTED, "route_logits: top_k=%lld must be <= min(E, 16)",
               (long long)K);
  if (T == 0) return 0;
  SMEL_REQUIRE(logits && probs && topv && topi && topi32, SMEL_EINVAL, "route_logits: null pointer");
  launch_select(stream, logits, (int)E, (int)T, (int)E, (int)K, 0, probs, topv, nullptr, topi, topi32, nullptr,
                nullptr, nullptr);
  return smel::launch_status();
}

extern "C" int smel_route_bwd(const float* dwp, int64_t nblk, const int32_t* inv, const float* probs,
                              const int32_t* topi32, const float* sgate, const float* dwp_sh, int64_t nblk_sh,
                              int64_t T, int64_t K, int64_t E, int64_t TK, uint16_t* dlogits, int64_t ldl,
                              float* dtopv_out, const uint16_t* per_expert_scale, hipStream_t stream) {
  SMEL_REQUIRE(!dwp_sh || nblk_sh > 0, SMEL_EINVAL, "route_bwd: nblk_sh must be positive with dwp_sh");
  SMEL_REQUIRE(T >= 0 && K > 0 && K <= 16 && E > 0 && nblk > 0, SMEL_EINVAL, "route_bwd: bad sizes");
  SMEL_REQUIRE(ldl >= E + (sgate ? 1 : 0), SMEL_EINVAL, "route_bwd: ldl %lld too small", (long long)ldl);
  if (T == 0) return 0;
  SMEL_REQUIRE(dwp && probs && topi32 && dlogits, SMEL_EINVAL, "route_bwd: null pointer");
  SMEL_REQUIRE(inv || TK == T * K, SMEL_EINVAL, "route_bwd: without inv, dwp rows are the T*K slots");
  route_bwd<<<(unsigned)((T + 3) / 4), 256, 0, stream>>>(dwp, (int)nblk, inv, probs, topi32, sgate, dwp_sh,
                                                         (int)nblk_sh, (int)T, (int)K, (int)E, (int)TK, dlogits,
                                                         (int)ldl, dtopv_out, per_expert_scale);
  return smel::launch_status();
}

extern "C" int smel_route_gemma4(const uint16_t* h, const uint16_t* router_scale, const uint16_t* proj_w,
                                 const uint16_t* per_expert_scale, int64_t T, int64_t H, int64_t E, int64_t K,
                                 float eps, float* probs, float* topv, int64_t* topi, int32_t* topi32, uint16_t* xn,
                                 float* rstd, uint16_t* logits, hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && H > 0 && E > 0 && K > 0, SMEL_EINVAL, "route_gemma4: bad sizes");
  SMEL_REQUIRE(E <= MAXE, SMEL_EUNSUPPORTED, "route_gemma4: E=%lld > %d experts", (long long)E, MAXE);
  SMEL_REQUIRE(K <= E && K <= 16, SMEL_EUNSUPPORTED, "route_gemma4: top_k=%lld must be <= min(E, 16)",
               (long long)K);
  SMEL_REQUIRE(H % 64 == 0, SMEL_EUNSUPPORTED, "route_gemma4: hidden %lld must be a multiple of 64", (long long)H);
  SMEL_REQUIRE(T * H * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "route_gemma4: h larger than 2 GiB");
  if (T == 0) return 0;
  SMEL_REQUIRE(h && router_scale && proj_w && per_expert_scale && probs && topv && topi && topi32 && xn && rstd &&
                   logits,
               SMEL_EINVAL, "route_gemma4: null pointer");
  const int64_t ldl = smel_route_ld(E, 0);
  const unsigned tg = (unsigned)((T + 3) / 4);
  // H^-1/2 as the reference's Python float (a double) rounded to fp32 for the bf16 product
  route_prenorm<<<tg, 256, 0, stream>>>(h, router_scale, (int)T, (int)H, eps, (float)pow((double)H, -0.5), xn, rstd);
  launch_logits(stream, xn, proj_w, nullptr, (int)T, (int)H, (int)E, (int)ldl, logits);
  launch_select(stream, logits, (int)ldl, (int)T, (int)E, (int)K, 0, probs, nullptr, nullptr, topi, topi32, nullptr,
                topv, per_expert_scale);
  return smel::launch_status();
}

extern "C" int smel_route_gemma4_prenorm_bwd(const uint16_t* h, const uint16_t* router_scale, const float* rstd,
                                             const uint16_t* dxn, int64_t T, int64_t H, uint16_t* dh,
                                             hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && H > 0 && H % 8 == 0, SMEL_EINVAL, "route_gemma4_prenorm_bwd: bad sizes");
  if (T == 0) return 0;
  SMEL_REQUIRE(h && router_scale && rstd && dxn && dh, SMEL_EINVAL, "route_gemma4_prenorm_bwd: null pointer");
  route_prenorm_bwd<<<(unsigned)((T + 3) / 4), 256, 0, stream>>>(h, router_scale, rstd, dxn, (int)T, (int)H,
                                                                  (float)pow((double)H, -0.5), dh);
  return smel::launch_status();
}
