// Router: logits = x W_r^T (bf16 MFMA, fp32 accumulation, bf16-rounded like F.linear in bf16), softmax in fp32,
// top-k (descending, lower expert id first among equal logits), renormalisation; and its backward.
// Reference: route, smel/moe.py:162-167; the shared-expert gate logit of shared_mlp, smel/moe.py:201.
#include "abi_util.h"
#include "common.h"

namespace {

constexpr int TB = 32;         // tokens per block (one 32-row MFMA slice)
constexpr int MAXE = 256;      // experts handled by one block
constexpr int LG_STRIDE = MAXE + 33;

// Selection over one token's logits (held in LDS or global), by one wave. Writes probs, topv, topi, topi32.
template <typename Get>
SMEL_DEV void select_topk(Get logit, int E, int K, int64_t t, float* __restrict__ probs, uint16_t* __restrict__ topv,
                          int64_t* __restrict__ topi, int32_t* __restrict__ topi32) {
  const int l = lane_id();
  float v[MAXE / 64];
#pragma unroll
  for (int j = 0; j < MAXE / 64; ++j) {
    const int e = l + 64 * j;
    v[j] = e < E ? logit(e) : -INFINITY;
  }
  float m = v[0];
#pragma unroll
  for (int j = 1; j < MAXE / 64; ++j) m = fmaxf(m, v[j]);
  m = wave_max(m);
  float ex[MAXE / 64], s = 0.f;
#pragma unroll
  for (int j = 0; j < MAXE / 64; ++j) {
    ex[j] = (l + 64 * j) < E ? expf(v[j] - m) : 0.f;
    s += ex[j];
  }
  s = wave_sum(s);
  const float inv_s = 1.0f / s;
#pragma unroll
  for (int j = 0; j < MAXE / 64; ++j) {
    const int e = l + 64 * j;
    if (e < E) probs[t * E + e] = ex[j] * inv_s;
  }
  // top-k: K rounds of a (value desc, index asc) arg-max across the wave
  unsigned taken = 0;
  float pk[16];
  int ik[16];
  float psum = 0.f;
  for (int k = 0; k < K; ++k) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < MAXE / 64; ++j) {
      const int e = l + 64 * j;
      if (e < E && !(taken >> j & 1u) && (v[j] > bv || (v[j] == bv && e < bi))) {
        bv = v[j];
        bi = e;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if ((bi & 63) == l) taken |= 1u << (bi >> 6);
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
    topv[t * K + l] = f2bf(p / psum);
    topi[t * K + l] = i;
    topi32[t * K + l] = i;
  }
}

// One block = 32 tokens, 8 waves: wave w computes expert columns of fragments (w&3), (w&3)+4, (w&3)+8 (32 columns
// each; the column E is the shared-expert gate when sg != nullptr) over the even (w < 4) or odd (w >= 4) 64-wide
// k-steps; the two halves are added (odd into even, fixed order) through LDS. H % 64 == 0.
__global__ __launch_bounds__(512) void route_fwd(const uint16_t* __restrict__ x, const uint16_t* __restrict__ gw,
                                                 const uint16_t* __restrict__ sg, int T, int H, int E, int K,
                                                 float* __restrict__ probs, uint16_t* __restrict__ topv,
                                                 int64_t* __restrict__ topi, int32_t* __restrict__ topi32,
                                                 float* __restrict__ sgate) {
  __shared__ float lg[TB * LG_STRIDE];
  const int l = lane_id(), wv = threadIdx.x >> 6, w = wv & 3, kh = wv >> 2, hi = l >> 5, r32 = l & 31;
  const int t0 = blockIdx.x * TB;
  const int ncol = E + (sg ? 1 : 0);
  const int nfrag = (ncol + 31) / 32;
  f32x16_t acc[3];
  uint32_t boff[3];
  const rsrc_t rg = make_rsrc(gw, (uint64_t)E * H * 2);
  const rsrc_t rsg = make_rsrc(sg, sg ? (uint64_t)H * 2 : 0);
  bool bsg[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    acc[i] = f32x16_t{};
    const int f = w + 4 * i;
    const int e = 32 * f + r32;
    bsg[i] = f < nfrag && e == E && sg;
    boff[i] = (f < nfrag && e < E) ? (uint32_t)e * H * 2 : (bsg[i] ? 0u : OOB);
  }
  const int t = t0 + r32;
  const rsrc_t rx = make_rsrc(x, (uint64_t)T * H * 2);
  const uint32_t aoff = t < T ? (uint32_t)t * H * 2 : OOB;
  // loads of step k0 + 128 are in flight while step k0 multiplies
  u32x4_t a[4], b[3][4], an[4], bn[3][4];
  auto load = [&](int k0, u32x4_t* av, u32x4_t (*bv)[4]) {
    const uint32_t ko = (uint32_t)(k0 + 32 * hi) * 2;
    const bool ok = k0 < H;
#pragma unroll
    for (int s = 0; s < 4; ++s) av[s] = ld16(rx, ok ? aoff + ko + 16 * s : OOB);
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int s = 0; s < 4; ++s) bv[i][s] = ld16(bsg[i] ? rsg : rg, ok ? boff[i] + ko + 16 * s : OOB);
  };
  load(64 * kh, a, b);
  for (int k0 = 64 * kh; k0 < H; k0 += 128) {
    load(k0 + 128, an, bn);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (w + 4 * i >= nfrag) continue;   // wave-uniform
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[i] = mfma32(a[s], b[i][s], acc[i]);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      a[s] = an[s];
#pragma unroll
      for (int i = 0; i < 3; ++i) b[i][s] = bn[i][s];
    }
  }
  // odd-step partial sums -> LDS, then the even-step waves add them and round the logits to bf16
  if (kh == 1) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int f = w + 4 * i;
      if (f >= nfrag) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) lg[acc_row(r, l) * LG_STRIDE + 32 * f + r32] = acc[i][r];
    }
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int f = w + 4 * i;
      if (f >= nfrag) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float* p = lg + acc_row(r, l) * LG_STRIDE + 32 * f + r32;
        *p = bf2f(f2bf(acc[i][r] + *p));
      }
    }
  }
  __syncthreads();
  for (int j = 0; j < TB / 8; ++j) {
    const int row = wv * (TB / 8) + j;
    const int64_t tt = t0 + row;
    if (tt >= T) break;
    const float* lrow = lg + row * LG_STRIDE;
    select_topk([&](int e) { return lrow[e]; }, E, K, tt, probs, topv, topi, topi32);
    if (sg && l == 0) sgate[tt] = 1.0f / (1.0f + expf(-lrow[E]));
  }
}

__global__ __launch_bounds__(256) void route_from_logits(const uint16_t* __restrict__ logits, int T, int E, int K,
                                                         float* __restrict__ probs, uint16_t* __restrict__ topv,
                                                         int64_t* __restrict__ topi, int32_t* __restrict__ topi32) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const uint16_t* row = logits + t * E;
  select_topk([&](int e) { return bf2f(row[e]); }, E, K, t, probs, topv, topi, topi32);
}

// Backward of route (+ shared gate): one wave per token.
//   dtopv[k] = sum_j dwp[inv[t*K+k]][j]  (d of the combine weight; dwp holds per-column-block partials)
//   renorm:  topv_k = p_k / S  ->  dp_k = (dtopv_k - sum_j dtopv_j topv_j) / S
//   softmax: dlogit_e = p_e (dp_e - sum_k dp_k p_{i_k}),  dp_e = 0 off the top-k
//   shared gate: dlogit_sg = (sum_j dwp[TK+t][j]) * sg (1 - sg)
__global__ __launch_bounds__(256) void route_bwd(const float* __restrict__ dwp, int nblk,
                                                 const int32_t* __restrict__ inv, const float* __restrict__ probs,
                                                 const int32_t* __restrict__ topi32, const uint16_t* __restrict__ topv,
                                                 const float* __restrict__ sgate, int T, int K, int E, int TK,
                                                 uint16_t* __restrict__ dlogits, int ldl,
                                                 float* __restrict__ dtopv_out) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int l = lane_id();
  // per-k quantities, lane k holds slot k
  float dtv = 0.f, p = 0.f;
  int idx = -1;
  if (l < K) {
    const int row = inv[t * K + l];   // -1 for a slot the dispatch dropped (id out of range)
    if (row >= 0)
      for (int j = 0; j < nblk; ++j) dtv += dwp[(int64_t)row * nblk + j];
    idx = topi32[t * K + l];
    if (idx >= 0 && idx < E) p = probs[t * E + idx];
    else idx = -1;
    if (dtopv_out) dtopv_out[t * K + l] = dtv;
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
      for (int j = 0; j < nblk; ++j) ds += dwp[(int64_t)(TK + t) * nblk + j];
      const float sgv = sgate[t];
      g = ds * sgv * (1.0f - sgv);
    }
    dlogits[t * ldl + e] = f2bf(g);
  }
  (void)topv;
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

}  // namespace

extern "C" int smel_dtopv(const float* dwp, int64_t nblk, const int32_t* inv, int64_t TK, float* dtopv,
                          hipStream_t stream) {
  SMEL_REQUIRE(nblk > 0 && TK >= 0, SMEL_EINVAL, "dtopv: bad sizes");
  if (TK == 0) return 0;
  SMEL_REQUIRE(dwp && inv && dtopv, SMEL_EINVAL, "dtopv: null pointer");
  dtopv_kernel<<<(unsigned)((TK + 255) / 256), 256, 0, stream>>>(dwp, (int)nblk, inv, (int)TK, dtopv);
  return smel::launch_status();
}

extern "C" int smel_route(const uint16_t* x, const uint16_t* gate_w, const uint16_t* shared_gate_w, int64_t T,
                          int64_t H, int64_t E, int64_t K, float* probs, uint16_t* topv, int64_t* topi,
                          int32_t* topi32, float* sgate, hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && H > 0 && E > 0 && K > 0, SMEL_EINVAL, "route: bad sizes");
  SMEL_REQUIRE(E <= MAXE, SMEL_EUNSUPPORTED, "route: E=%lld > %d experts", (long long)E, MAXE);
  SMEL_REQUIRE(K <= E && K <= 16, SMEL_EUNSUPPORTED, "route: top_k=%lld must be <= min(E, 16)", (long long)K);
  SMEL_REQUIRE(H % 64 == 0, SMEL_EUNSUPPORTED, "route: hidden %lld must be a multiple of 64", (long long)H);
  SMEL_REQUIRE(!shared_gate_w || sgate, SMEL_EINVAL, "route: sgate output needed with shared_gate_w");
  if (T == 0) return 0;
  SMEL_REQUIRE(x && gate_w && probs && topv && topi && topi32, SMEL_EINVAL, "route: null pointer");
  route_fwd<<<(unsigned)((T + TB - 1) / TB), 512, 0, stream>>>(x, gate_w, shared_gate_w, (int)T, (int)H, (int)E,
                                                                 (int)K, probs, topv, topi, topi32, sgate);
  return smel::launch_status();
}

extern "C" int smel_route_logits(const uint16_t* logits, int64_t T, int64_t E, int64_t K, float* probs,
                                 uint16_t* topv, int64_t* topi, int32_t* topi32, hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && E > 0 && K > 0, SMEL_EINVAL, "route_logits: bad sizes");
  SMEL_REQUIRE(E <= MAXE, SMEL_EUNSUPPORTED, "route_logits: E=%lld > %d", (long long)E, MAXE);
  SMEL_REQUIRE(K <= E && K <= 16, SMEL_EUNSUPPORTED, "route_logits: top_k=%lld must be <= min(E, 16)",
               (long long)K);
  if (T == 0) return 0;
  SMEL_REQUIRE(logits && probs && topv && topi && topi32, SMEL_EINVAL, "route_logits: null pointer");
  route_from_logits<<<(unsigned)((T + 3) / 4), 256, 0, stream>>>(logits, (int)T, (int)E, (int)K, probs, topv, topi,
                                                                  topi32);
  return smel::launch_status();
}

extern "C" int smel_route_bwd(const float* dwp, int64_t nblk, const int32_t* inv, const float* probs,
                              const int32_t* topi32, const uint16_t* topv, const float* sgate, int64_t T, int64_t K,
                              int64_t E, int64_t TK, uint16_t* dlogits, int64_t ldl, float* dtopv_out,
                              hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && K > 0 && K <= 16 && E > 0 && nblk > 0, SMEL_EINVAL, "route_bwd: bad sizes");
  SMEL_REQUIRE(ldl >= E + (sgate ? 1 : 0), SMEL_EINVAL, "route_bwd: ldl %lld too small", (long long)ldl);
  if (T == 0) return 0;
  SMEL_REQUIRE(dwp && inv && probs && topi32 && dlogits, SMEL_EINVAL, "route_bwd: null pointer");
  route_bwd<<<(unsigned)((T + 3) / 4), 256, 0, stream>>>(dwp, (int)nblk, inv, probs, topi32, topv, sgate, (int)T,
                                                         (int)K, (int)E, (int)TK, dlogits, (int)ldl, dtopv_out);
  return smel::launch_status();
}
