// fp32 path of the MoE layer (include/smel_f32.h): the reference's layer on fp32 tensors, whose _gmm falls to a
// per-group matmul loop for any non-bf16 tensor (smel/moe.py:58-72). Grouped GEMMs on v_mfma_f32_32x32x2_f32 over the
// same tile lists and group kinds as the bf16 GEMMs, LoRA weight gradients as row-group reductions on the same MFMA,
// and the fp32 element-wise steps around them (gather, act-gate, combine, dX reduce, router selection and backward,
// the Gemma router input, the shared-expert gate). Everything sums in a fixed order: no atomics.
#include <math.h>

#include "../../include/smel_f32.h"
#include "abi_util.h"
#include "common.h"

namespace {

constexpr int FB = 64;        // output tile 64 x 64: 4 waves, each a 32 x 32 quadrant
constexpr int FK = 16;        // k-step staged in LDS
constexpr int FLD = FB + 4;   // LDS pitch (floats) of a [k][64] stage: the transposing stores hit distinct banks

SMEL_DEV f32x16_t mfma_f32(float a, float b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// One staged k-step on a wave's quadrant (wm, wn): lane l supplies A[i = l % 32][k = 2 s + l / 32] and
// B[k][j = l % 32]; both stages are [k][64] with the row (column) index contiguous.
SMEL_DEV void mma_step(const float* __restrict__ As, const float* __restrict__ Bs, int wm, int wn, f32x16_t& acc) {
  const int l = lane_id(), i = l & 31, kh = l >> 5;
#pragma unroll
  for (int s = 0; s < FK / 2; ++s)
    acc = mfma_f32(As[(2 * s + kh) * FLD + 32 * wm + i], Bs[(2 * s + kh) * FLD + 32 * wn + i], acc);
}

// ---------------------------------------------------------------------------------------------- weight matrices

// One matrix [R][C] of a weight set: fp32 values, or the reference's int4 format dequantized as w = q s + z in fp32
// (q s is exact in fp32, so this equals the separate product and sum), optionally rounded to bf16. Offsets inside a
// matrix are 32-bit (one matrix is below 2^31 elements); the group index is a shift when the group is a power of two.
struct WMat {
  const float* f;
  const uint8_t* q;
  const uint16_t* s;
  const uint16_t* z;
  int C;
  int gpr;      // groups per row, C / group
  int group;
  int gshift;   // log2(group), or -1
  int rbf;
};

SMEL_DEV int gidx(const WMat& m, int row, int col) {
  return row * m.gpr + (m.gshift >= 0 ? col >> m.gshift : col / m.group);
}

SMEL_DEV float dq(const WMat& m, uint32_t q, int gi) {
  const float v = fmaf((float)q, bf2f(m.s[gi]), bf2f(m.z[gi]));
  return m.rbf ? bf2f(f2bf(v)) : v;
}

SMEL_DEV float w_at(const WMat& m, int row, int col) {
  if (m.f) return m.f[row * m.C + col];
  const uint32_t b = m.q[row * (m.C >> 1) + (col >> 1)];
  return dq(m, (b >> (4 * (col & 1))) & 0xfu, gidx(m, row, col));
}

// Elements [row][col .. col + 3] (col a multiple of 4, col + 3 < C, C a multiple of 4): one 16-byte load for fp32,
// one 16-bit load of nibbles for int4 (one scale / zero pair when the group is a multiple of 4).
SMEL_DEV void w_quad(const WMat& m, int row, int col, float v[4]) {
  if (m.f) {
    const float4 x = *reinterpret_cast<const float4*>(m.f + row * m.C + col);
    v[0] = x.x, v[1] = x.y, v[2] = x.z, v[3] = x.w;
    return;
  }
  const uint32_t qq = *reinterpret_cast<const uint16_t*>(m.q + row * (m.C >> 1) + (col >> 1));
  if ((m.group & 3) == 0) {
    const int gi = gidx(m, row, col);
    const float sc = bf2f(m.s[gi]), ze = bf2f(m.z[gi]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = fmaf((float)((qq >> (4 * i)) & 0xfu), sc, ze);
      v[i] = m.rbf ? bf2f(f2bf(x)) : x;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = dq(m, (qq >> (4 * i)) & 0xfu, gidx(m, row, col + i));
  }
}

SMEL_DEV bool resolve(const smel_wset_f32& w, int kind, int idx, WMat& m) {
  m.C = (int)w.C;
  m.group = w.group > 0 ? w.group : 1;
  m.gpr = (int)(w.C / m.group);
  m.gshift = (m.group & (m.group - 1)) == 0 ? __builtin_ctz((unsigned)m.group) : -1;
  m.rbf = w.q4_round_bf16;
  m.f = nullptr;
  m.q = nullptr;
  m.s = m.z = nullptr;
  const int64_t n = w.R * w.C;
  switch (kind) {
    case SMEL_KIND_INT4:
      if (!w.q4) return false;
      m.q = w.q4 + (int64_t)idx * (n >> 1);
      m.s = w.scale + (int64_t)idx * w.R * m.gpr;
      m.z = w.zero + (int64_t)idx * w.R * m.gpr;
      return true;
    case SMEL_KIND_BF16: m.f = w.wf ? w.wf + (int64_t)idx * n : nullptr; break;
    case SMEL_KIND_SEL: m.f = w.wsel ? w.wsel + (int64_t)idx * n : nullptr; break;
    default: m.f = w.wsh ? w.wsh + (int64_t)idx * n : nullptr; break;
  }
  return m.f != nullptr;
}

// ---------------------------------------------------------------------------------------------- grouped GEMM
// Block = one tile of the list x 64 output columns; the tile's rows in 64-row chunks. Each k-step: every thread
// loads 4 A values (row t / 4, k 4 (t % 4) ..) and 4 W values, stores them into the [k][64] stages, and the next
// step's loads are issued before this step's MFMAs (two LDS stages, one barrier per step).
// VEC: A rows and fp32 weights may be read as aligned float4 (lda, C multiples of 4, 16-byte aligned bases).
template <int TRANS, bool VEC>
__global__ __launch_bounds__(256) void gmm_f32_kernel(smel_wset_f32 w, const int32_t* __restrict__ gkind,
                                                      const int32_t* __restrict__ tiles,
                                                      const int32_t* __restrict__ n_tiles,
                                                      const float* __restrict__ A, int64_t lda, float alpha,
                                                      int beta1, float* __restrict__ C, int64_t ldc) {
  __shared__ __align__(16) float As[2][FK * FLD];
  __shared__ __align__(16) float Bs[2][FK * FLD];
  const int ti = blockIdx.x;
  if (ti >= n_tiles[0]) return;
  const int g = tiles[4 * ti], r0 = tiles[4 * ti + 1], r1 = tiles[4 * ti + 2];
  const int gk = gkind ? gkind[g] : tiles[4 * ti + 3];
  const int kind = gk >> 16, idx = gk & 0xffff;
  if (!((w.kinds >> kind) & 1)) return;
  WMat m;
  if (!resolve(w, kind, idx, m)) return;
  const int64_t N = TRANS ? w.C : w.R, K = TRANS ? w.R : w.C;
  const int64_t n0 = (int64_t)blockIdx.y * FB;
  if (n0 >= N) return;
  const int t = threadIdx.x, wv = t >> 6, wm = wv & 1, wn = wv >> 1;
  const int nk = (int)((K + FK - 1) / FK);
  // this thread's load coordinates: A (and W for TRANS = 0) row t / 4, k quad t % 4; W for TRANS = 1: k t / 16,
  // column quad t % 16
  const int am = t >> 2, akq = 4 * (t & 3);
  const int bk1 = t >> 4, bn1 = 4 * (t & 15);
  const bool qvec = (w.C & 3) == 0 && (m.f ? VEC : true);
  for (int mr0 = r0; mr0 < r1; mr0 += FB) {
    const int mr1 = min(r1, mr0 + FB);
    float ra[4], rb[4];
    auto load = [&](int64_t k0) {
      const int64_t row = mr0 + am, k = k0 + akq;
      if (VEC && row < mr1 && k + 3 < K) {
        const float4 v = *reinterpret_cast<const float4*>(A + row * lda + k);
        ra[0] = v.x, ra[1] = v.y, ra[2] = v.z, ra[3] = v.w;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) ra[i] = (row < mr1 && k + i < K) ? A[row * lda + k + i] : 0.f;
      }
      // weights: whole quads through w_quad when the matrix's rows are multiples of 4 (and, for fp32, its base
      // 16-byte aligned: VEC), the guarded element path otherwise
      if (TRANS == 0) {   // W [N][K]: row n0 + t / 4, k quad
        const int n = (int)(n0 + am), kq = (int)k;
        if (qvec && n < N && kq + 3 < K) {
          w_quad(m, n, kq, rb);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) rb[i] = (n < N && kq + i < K) ? w_at(m, n, kq + i) : 0.f;
        }
      } else {            // W [K][N]: row k0 + t / 16, column quad
        const int kk = (int)(k0 + bk1), n = (int)(n0 + bn1);
        if (qvec && kk < K && n + 3 < N) {
          w_quad(m, kk, n, rb);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) rb[i] = (kk < K && n + i < N) ? w_at(m, kk, n + i) : 0.f;
        }
      }
    };
    auto store = [&](int buf) {
#pragma unroll
      for (int i = 0; i < 4; ++i) As[buf][(akq + i) * FLD + am] = ra[i];
      if (TRANS == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) Bs[buf][(akq + i) * FLD + am] = rb[i];
      } else {
        *reinterpret_cast<float4*>(&Bs[buf][bk1 * FLD + bn1]) = make_float4(rb[0], rb[1], rb[2], rb[3]);
      }
    };
    f32x16_t acc = {};
    if (nk > 0) {
      load(0);
      store(0);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      if (kt + 1 < nk) load((int64_t)(kt + 1) * FK);
      mma_step(As[kt & 1], Bs[kt & 1], wm, wn, acc);
      if (kt + 1 < nk) store((kt + 1) & 1);
      __syncthreads();
    }
    const int l = lane_id();
    const int64_t col = n0 + 32 * wn + (l & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = mr0 + 32 * wm + acc_row(r, l);
      if (row < mr1 && col < N) {
        float* p = C + row * ldc + col;
        *p = beta1 ? *p + alpha * acc[r] : alpha * acc[r];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------- weight gradients
// Block = (64 x 64 output tile, job); the job's rows are the contraction, 16 per staged step: X rows give the
// [k][m] stage and Y rows the [k][n] stage directly (both row-contiguous).
template <bool VEC>
__global__ __launch_bounds__(256) void wgrad_f32_kernel(const float* __restrict__ X, int64_t ldx,
                                                        const float* __restrict__ Y, int64_t ldy,
                                                        const int32_t* __restrict__ offsets,
                                                        const int32_t* __restrict__ job_group, int64_t M, int64_t N,
                                                        float alpha, float* __restrict__ C, int64_t c_stride) {
  __shared__ __align__(16) float As[2][FK * FLD];
  __shared__ __align__(16) float Bs[2][FK * FLD];
  const int j = blockIdx.y;
  const int nbn = (int)((N + FB - 1) / FB);
  const int64_t m0 = (int64_t)(blockIdx.x / nbn) * FB, n0 = (int64_t)(blockIdx.x % nbn) * FB;
  const int g = job_group[j];
  const int64_t r0 = offsets[g], r1 = offsets[g + 1];
  const int t = threadIdx.x, wv = t >> 6, wm = wv & 1, wn = wv >> 1;
  const int kl = t >> 4, q4 = 4 * (t & 15);
  const int nk = r1 > r0 ? (int)((r1 - r0 + FK - 1) / FK) : 0;
  float ra[4], rb[4];
  auto load = [&](int64_t k0) {
    const int64_t r = r0 + k0 + kl;
    const int64_t mm = m0 + q4, nn = n0 + q4;
    if (VEC && r < r1 && mm + 3 < M) {
      const float4 v = *reinterpret_cast<const float4*>(X + r * ldx + mm);
      ra[0] = v.x, ra[1] = v.y, ra[2] = v.z, ra[3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) ra[i] = (r < r1 && mm + i < M) ? X[r * ldx + mm + i] : 0.f;
    }
    if (VEC && r < r1 && nn + 3 < N) {
      const float4 v = *reinterpret_cast<const float4*>(Y + r * ldy + nn);
      rb[0] = v.x, rb[1] = v.y, rb[2] = v.z, rb[3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) rb[i] = (r < r1 && nn + i < N) ? Y[r * ldy + nn + i] : 0.f;
    }
  };
  auto store = [&](int buf) {
    *reinterpret_cast<float4*>(&As[buf][kl * FLD + q4]) = make_float4(ra[0], ra[1], ra[2], ra[3]);
    *reinterpret_cast<float4*>(&Bs[buf][kl * FLD + q4]) = make_float4(rb[0], rb[1], rb[2], rb[3]);
  };
  f32x16_t acc = {};
  if (nk > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load((int64_t)(kt + 1) * FK);
    mma_step(As[kt & 1], Bs[kt & 1], wm, wn, acc);
    if (kt + 1 < nk) store((kt + 1) & 1);
    __syncthreads();
  }
  const int l = lane_id();
  const int64_t col = n0 + 32 * wn + (l & 31);
  float* Cj = C + (int64_t)j * c_stride;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = m0 + 32 * wm + acc_row(r, l);
    if (row < M && col < N) Cj[row * N + col] = alpha * acc[r];
  }
}

// ---------------------------------------------------------------------------------------------- element-wise

// Sum over a 256-thread block, the same order every time (each wave's tree, then the waves in order).
SMEL_DEV float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

SMEL_DEV float sigmoid32(float x) { return 1.0f / (1.0f + expf(-x)); }

// act(g) as torch computes it in fp32 (F.silu: g / (1 + e^-g); F.gelu tanh), and (act, act') as act_and_grad
SMEL_DEV float act32(float g, int act) {
  if (act == 0) return g / (1.0f + expf(-g));
  const float c = 0.7978845608028654f;
  return 0.5f * g * (1.0f + tanhf(c * (g + 0.044715f * g * g * g)));
}
SMEL_DEV void act_grad32(float g, int act, float& a, float& da) {
  if (act == 0) {
    const float s = sigmoid32(g);
    a = g * s;
    da = s * (1.0f + g * (1.0f - s));
    return;
  }
  const float c = 0.7978845608028654f;
  const float th = tanhf(c * (g + 0.044715f * g * g * g));
  a = 0.5f * g * (1.0f + th);
  da = 0.5f * (1.0f + th) + 0.5f * g * (1.0f - th * th) * c * (1.0f + 3.0f * 0.044715f * g * g);
}

__global__ __launch_bounds__(256) void gather_rows_f32_kernel(const float* __restrict__ src, int64_t lds,
                                                              const int32_t* __restrict__ idx, int div,
                                                              const int32_t* __restrict__ n_valid, int64_t cols,
                                                              float* __restrict__ out) {
  const int64_t p = blockIdx.x;
  const int i = (n_valid && p >= n_valid[0]) ? -1 : idx[p];
  const float* s = i >= 0 ? src + (int64_t)(i / div) * lds : nullptr;
  float* o = out + p * cols;
  for (int64_t c = threadIdx.x; c < cols; c += 256) o[c] = s ? s[c] : 0.f;
}

__global__ __launch_bounds__(256) void act_gate_f32_kernel(const float* __restrict__ h, int64_t ldh, int64_t I, int act,
                                                           float* __restrict__ a, int64_t lda) {
  const int64_t r = blockIdx.x;
  for (int64_t j = threadIdx.x; j < I; j += 256) a[r * lda + j] = act32(h[r * ldh + j], act) * h[r * ldh + I + j];
}

__global__ __launch_bounds__(256) void act_gate_bwd_f32_kernel(const float* __restrict__ h, int64_t ldh,
                                                               const float* __restrict__ da, int64_t ldda, int64_t I,
                                                               int act, float* __restrict__ dh, int64_t lddh) {
  const int64_t r = blockIdx.x;
  for (int64_t j = threadIdx.x; j < I; j += 256) {
    const float g = h[r * ldh + j], u = h[r * ldh + I + j], d = da[r * ldda + j];
    float a, dg;
    act_grad32(g, act, a, dg);
    dh[r * lddh + j] = d * u * dg;
    dh[r * lddh + I + j] = d * a;
  }
}

__global__ __launch_bounds__(256) void combine_f32_kernel(const float* __restrict__ ys, const float* __restrict__ topv,
                                                          const int32_t* __restrict__ inv, int K, int64_t H,
                                                          float* __restrict__ out) {
  const int64_t t = blockIdx.x;
  for (int64_t c = threadIdx.x; c < H; c += 256) {
    float acc = 0.f;
    for (int k = 0; k < K; ++k) {
      const int p = inv[t * K + k];
      if (p >= 0) acc += ys[(int64_t)p * H + c] * topv[t * K + k];
    }
    out[t * H + c] = acc;
  }
}

__global__ __launch_bounds__(256) void combine_bwd_f32_kernel(const float* __restrict__ ys,
                                                              const float* __restrict__ dout,
                                                              const float* __restrict__ topv,
                                                              const int32_t* __restrict__ inv, int K, int64_t H,
                                                              float* __restrict__ dys, float* __restrict__ dtopv) {
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  for (int k = 0; k < K; ++k) {
    const int p = inv[t * K + k];   // block-uniform
    float dot = 0.f;
    if (p >= 0) {
      const float tv = topv[t * K + k];
      for (int64_t c = threadIdx.x; c < H; c += 256) {
        const float d = dout[t * H + c];
        dys[(int64_t)p * H + c] = tv * d;
        dot += ys[(int64_t)p * H + c] * d;
      }
    }
    dot = block_sum(dot, red);
    if (threadIdx.x == 0) dtopv[t * K + k] = dot;
  }
}

__global__ __launch_bounds__(256) void dx_reduce_f32_kernel(const float* __restrict__ dxs,
                                                            const int32_t* __restrict__ inv, int K, int64_t H,
                                                            float* __restrict__ dx) {
  const int64_t t = blockIdx.x;
  for (int64_t c = threadIdx.x; c < H; c += 256) {
    float acc = 0.f;
    for (int k = 0; k < K; ++k) {
      const int p = inv[t * K + k];
      if (p >= 0) acc += dxs[(int64_t)p * H + c];
    }
    dx[t * H + c] = acc;
  }
}

// One wave per token. The top-k compares the fp32 probabilities themselves (the reference's torch.topk(probs)):
// 64-bit keys (probability bits, then the complement of the expert id, so equal values take the lower id first).
template <int NPL>
__global__ __launch_bounds__(256) void route_select_f32_kernel(const float* __restrict__ logits, int64_t ldl, int T,
                                                               int E, int K, const float* __restrict__ pes,
                                                               float* __restrict__ probs, float* __restrict__ topv,
                                                               int64_t* __restrict__ topi,
                                                               int32_t* __restrict__ topi32) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int l = lane_id();
  float v[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = l + 64 * j;
    v[j] = e < E ? logits[t * ldl + e] : -INFINITY;
  }
  float mx = v[0];
#pragma unroll
  for (int j = 1; j < NPL; ++j) mx = fmaxf(mx, v[j]);
  mx = wave_max(mx);
  float ex[NPL], s = 0.f;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    ex[j] = (l + 64 * j) < E ? expf(v[j] - mx) : 0.f;
    s += ex[j];
  }
  s = wave_sum(s);
  uint64_t key[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = l + 64 * j;
    const float p = ex[j] / s;
    if (e < E) probs[t * E + e] = p;
    key[j] = e < E ? ((uint64_t)__float_as_uint(p) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e) : 0ull;
  }
  float pk[16];
  int ik[16];
  float psum = 0.f;
  for (int k = 0; k < K; ++k) {
    uint64_t best = key[0];
#pragma unroll
    for (int j = 1; j < NPL; ++j) best = key[j] > best ? key[j] : best;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(best >> 32), o, 64);
      const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)best, o, 64);
      const uint64_t other = ((uint64_t)hi << 32) | lo;
      best = other > best ? other : best;
    }
    const int bi = (int)(0xffffffffu - (uint32_t)best);
#pragma unroll
    for (int j = 0; j < NPL; ++j)
      if (bi == l + 64 * j) key[j] = 0ull;
    ik[k] = bi;
    pk[k] = __uint_as_float((uint32_t)(best >> 32));
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
    const float tv = p / psum;
    topv[t * K + l] = pes ? tv * pes[i] : tv;
    topi[t * K + l] = i;
    topi32[t * K + l] = i;
  }
}

// dtopv -> dlogits, one wave per token (the fp32 form of route_bwd in router.hip):
//   per-expert scale: d(renorm)_k = dtopv_k pes[i_k];  renorm: dp_k = (d_k - sum_j d_j tv_j) / S, tv_j = p_j / S;
//   softmax: dlogit_e = p_e (dp_e - sum_k dp_k p_{i_k}),  dp_e = 0 off the top-k.
__global__ __launch_bounds__(256) void route_bwd_f32_kernel(const float* __restrict__ dtopv,
                                                            const float* __restrict__ probs,
                                                            const int32_t* __restrict__ topi32,
                                                            const float* __restrict__ pes, int T, int K, int E,
                                                            float* __restrict__ dlogits) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int l = lane_id();
  float d = 0.f, p = 0.f;
  int idx = -1;
  if (l < K) {
    idx = topi32[t * K + l];
    if (idx >= 0 && idx < E) {
      p = probs[t * E + idx];
      d = dtopv[t * K + l];
      if (pes) d *= pes[idx];
    } else {
      idx = -1;
    }
  }
  float S = 0.f, dot = 0.f, pdp = 0.f;
  for (int k = 0; k < K; ++k) S += __shfl(p, k, 64);
  const float tv = (l < K) ? p / S : 0.f;
  for (int k = 0; k < K; ++k) dot += __shfl(d * tv, k, 64);
  const float dp = (l < K) ? (d - dot) / S : 0.f;
  for (int k = 0; k < K; ++k) pdp += __shfl(dp * p, k, 64);
  int ik[16];
  float dk[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    ik[k] = k < K ? __shfl(idx, k, 64) : -1;
    dk[k] = k < K ? __shfl(dp, k, 64) : 0.f;
  }
  for (int e = l; e < E; e += 64) {
    float dpe = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k)
      if (ik[k] == e) dpe = dk[k];
    dlogits[t * E + e] = probs[t * E + e] * (dpe - pdp);
  }
}

__global__ __launch_bounds__(256) void route_prenorm_f32_kernel(const float* __restrict__ h,
                                                                const float* __restrict__ scale, int64_t H, float eps,
                                                                float hs, float* __restrict__ xn,
                                                                float* __restrict__ rstd) {
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  float ss = 0.f;
  for (int64_t j = threadIdx.x; j < H; j += 256) ss += h[t * H + j] * h[t * H + j];
  ss = block_sum(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)H + eps);
  if (threadIdx.x == 0) rstd[t] = r;
  for (int64_t j = threadIdx.x; j < H; j += 256) xn[t * H + j] = ((h[t * H + j] * r) * scale[j]) * hs;
}

__global__ __launch_bounds__(256) void route_prenorm_bwd_f32_kernel(const float* __restrict__ h,
                                                                    const float* __restrict__ scale,
                                                                    const float* __restrict__ rstd,
                                                                    const float* __restrict__ dxn, int64_t H, float hs,
                                                                    float* __restrict__ dh) {
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  const float r = rstd[t];
  float dot = 0.f;
  for (int64_t j = threadIdx.x; j < H; j += 256) dot += (dxn[t * H + j] * hs) * scale[j] * h[t * H + j];
  dot = block_sum(dot, red);
  const float c = r * r * r * dot / (float)H;
  for (int64_t j = threadIdx.x; j < H; j += 256) {
    const float g = (dxn[t * H + j] * hs) * scale[j];
    dh[t * H + j] = g * r - h[t * H + j] * c;
  }
}

__global__ __launch_bounds__(256) void gate_mul_f32_kernel(const float* __restrict__ y, const float* __restrict__ s,
                                                           const float* __restrict__ base, int64_t H,
                                                           float* __restrict__ out) {
  const int64_t t = blockIdx.x;
  const float sg = sigmoid32(s[t]);
  for (int64_t c = threadIdx.x; c < H; c += 256) {
    const float v = y[t * H + c] * sg;
    out[t * H + c] = base ? base[t * H + c] + v : v;
  }
}

__global__ __launch_bounds__(256) void gate_mul_bwd_f32_kernel(const float* __restrict__ y,
                                                               const float* __restrict__ s,
                                                               const float* __restrict__ dout, int64_t H,
                                                               float* __restrict__ dy, float* __restrict__ ds) {
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  const float sg = sigmoid32(s[t]);
  float dot = 0.f;
  for (int64_t c = threadIdx.x; c < H; c += 256) {
    const float d = dout[t * H + c];
    dy[t * H + c] = d * sg;
    dot += d * y[t * H + c];
  }
  dot = block_sum(dot, red);
  if (threadIdx.x == 0) ds[t] = dot * sg * (1.0f - sg);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

// ---------------------------------------------------------------------------------------------- C-ABI

extern "C" int smel_gmm_f32(const smel_wset_f32* w, int32_t trans, const int32_t* gkind, const int32_t* tiles,
                            const int32_t* n_tiles, int64_t max_tiles, const float* A, int64_t lda, float alpha,
                            float beta, float* C, int64_t ldc, hipStream_t stream) {
  SMEL_REQUIRE(w && tiles && n_tiles && A && C, SMEL_EINVAL, "smel_gmm_f32: null pointer");
  SMEL_REQUIRE(trans == 0 || trans == 1, SMEL_EINVAL, "smel_gmm_f32: trans must be 0 or 1");
  SMEL_REQUIRE(beta == 0.f || beta == 1.f, SMEL_EINVAL, "smel_gmm_f32: beta must be 0 or 1");
  SMEL_REQUIRE(w->R > 0 && w->C > 0 && max_tiles >= 0 && max_tiles < (1 << 30), SMEL_EINVAL,
               "smel_gmm_f32: bad sizes R=%lld C=%lld max_tiles=%lld", (long long)w->R, (long long)w->C,
               (long long)max_tiles);
  SMEL_REQUIRE(w->R * w->C < (1LL << 31), SMEL_EUNSUPPORTED, "smel_gmm_f32: one weight matrix of 2^31 elements or more");
  const int64_t N = trans ? w->C : w->R, K = trans ? w->R : w->C;
  SMEL_REQUIRE(lda >= K && ldc >= N, SMEL_EINVAL, "smel_gmm_f32: lda %lld < K %lld or ldc %lld < N %lld",
               (long long)lda, (long long)K, (long long)ldc, (long long)N);
  const int32_t known = (1 << SMEL_KIND_INT4) | (1 << SMEL_KIND_BF16) | (1 << SMEL_KIND_SEL) | (1 << SMEL_KIND_SHARED);
  SMEL_REQUIRE((w->kinds & ~known) == 0 && w->kinds != 0, SMEL_EINVAL, "smel_gmm_f32: bad kinds mask %d", w->kinds);
  SMEL_REQUIRE(!(w->kinds & (1 << SMEL_KIND_INT4)) ||
                   (w->q4 && w->scale && w->zero && w->group > 0 && w->group % 2 == 0 && w->C % w->group == 0),
               SMEL_EINVAL, "smel_gmm_f32: int4 tiles need q4 / scale / zero and an even group dividing C");
  SMEL_REQUIRE(!(w->kinds & (1 << SMEL_KIND_BF16)) || w->wf, SMEL_EINVAL, "smel_gmm_f32: no dense bank (wf)");
  SMEL_REQUIRE(!(w->kinds & (1 << SMEL_KIND_SEL)) || w->wsel, SMEL_EINVAL, "smel_gmm_f32: no selected weights");
  SMEL_REQUIRE(!(w->kinds & (1 << SMEL_KIND_SHARED)) || w->wsh, SMEL_EINVAL, "smel_gmm_f32: no shared weights");
  if (max_tiles == 0) return 0;
  const bool vec = aligned16(A) && lda % 4 == 0 && w->C % 4 == 0 && (!w->wf || aligned16(w->wf)) &&
                   (!w->wsel || aligned16(w->wsel)) && (!w->wsh || aligned16(w->wsh));
  const dim3 grid((unsigned)max_tiles, (unsigned)((N + FB - 1) / FB));
  const int b1 = beta != 0.f;
  if (trans == 0) {
    if (vec) gmm_f32_kernel<0, true><<<grid, 256, 0, stream>>>(*w, gkind, tiles, n_tiles, A, lda, alpha, b1, C, ldc);
    else gmm_f32_kernel<0, false><<<grid, 256, 0, stream>>>(*w, gkind, tiles, n_tiles, A, lda, alpha, b1, C, ldc);
  } else {
    if (vec) gmm_f32_kernel<1, true><<<grid, 256, 0, stream>>>(*w, gkind, tiles, n_tiles, A, lda, alpha, b1, C, ldc);
    else gmm_f32_kernel<1, false><<<grid, 256, 0, stream>>>(*w, gkind, tiles, n_tiles, A, lda, alpha, b1, C, ldc);
  }
  return smel::launch_status();
}

extern "C" int smel_wgrad_f32(const float* X, int64_t ldx, const float* Y, int64_t ldy, const int32_t* offsets,
                              const int32_t* job_group, int32_t n_jobs, int64_t M, int64_t N, float alpha, float* C,
                              int64_t c_stride, hipStream_t stream) {
  SMEL_REQUIRE(X && Y && offsets && job_group && C, SMEL_EINVAL, "smel_wgrad_f32: null pointer");
  SMEL_REQUIRE(M > 0 && N > 0 && ldx >= M && ldy >= N && n_jobs >= 0 && n_jobs < 65536 && c_stride >= M * N,
               SMEL_EINVAL, "smel_wgrad_f32: bad sizes");
  if (n_jobs == 0) return 0;
  const int64_t tiles = ((M + FB - 1) / FB) * ((N + FB - 1) / FB);
  SMEL_REQUIRE(tiles < (1 << 30), SMEL_EINVAL, "smel_wgrad_f32: output too large");
  const bool vec = aligned16(X) && aligned16(Y) && ldx % 4 == 0 && ldy % 4 == 0;
  const dim3 grid((unsigned)tiles, (unsigned)n_jobs);
  if (vec)
    wgrad_f32_kernel<true><<<grid, 256, 0, stream>>>(X, ldx, Y, ldy, offsets, job_group, M, N, alpha, C, c_stride);
  else
    wgrad_f32_kernel<false><<<grid, 256, 0, stream>>>(X, ldx, Y, ldy, offsets, job_group, M, N, alpha, C, c_stride);
  return smel::launch_status();
}

extern "C" int smel_gather_rows_f32(const float* src, int64_t lds, const int32_t* idx, int32_t div,
                                    const int32_t* n_valid, int64_t n, int64_t cols, float* out, hipStream_t stream) {
  SMEL_REQUIRE(src && idx && out && div > 0 && n >= 0 && cols > 0 && lds >= cols && n < (1LL << 31), SMEL_EINVAL,
               "smel_gather_rows_f32: bad arguments");
  if (n == 0) return 0;
  gather_rows_f32_kernel<<<(unsigned)n, 256, 0, stream>>>(src, lds, idx, div, n_valid, cols, out);
  return smel::launch_status();
}

extern "C" int smel_act_gate_f32(const float* h, int64_t ldh, int64_t rows, int64_t I, int32_t act, float* a,
                                 int64_t lda, hipStream_t stream) {
  SMEL_REQUIRE(h && a && rows >= 0 && I > 0 && ldh >= 2 * I && lda >= I && (act == 0 || act == 1) &&
                   rows < (1LL << 31),
               SMEL_EINVAL, "smel_act_gate_f32: bad arguments");
  if (rows == 0) return 0;
  act_gate_f32_kernel<<<(unsigned)rows, 256, 0, stream>>>(h, ldh, I, act, a, lda);
  return smel::launch_status();
}

extern "C" int smel_act_gate_bwd_f32(const float* h, int64_t ldh, const float* da, int64_t ldda, int64_t rows,
                                     int64_t I, int32_t act, float* dh, int64_t lddh, hipStream_t stream) {
  SMEL_REQUIRE(h && da && dh && rows >= 0 && I > 0 && ldh >= 2 * I && ldda >= I && lddh >= 2 * I &&
                   (act == 0 || act == 1) && rows < (1LL << 31),
               SMEL_EINVAL, "smel_act_gate_bwd_f32: bad arguments");
  if (rows == 0) return 0;
  act_gate_bwd_f32_kernel<<<(unsigned)rows, 256, 0, stream>>>(h, ldh, da, ldda, I, act, dh, lddh);
  return smel::launch_status();
}

extern "C" int smel_combine_f32(const float* ys, const float* topv, const int32_t* inv, int64_t T, int64_t K,
                                int64_t H, float* out, hipStream_t stream) {
  SMEL_REQUIRE(ys && topv && inv && out && T >= 0 && K > 0 && K <= 64 && H > 0 && T < (1LL << 31), SMEL_EINVAL,
               "smel_combine_f32: bad arguments");
  if (T == 0) return 0;
  combine_f32_kernel<<<(unsigned)T, 256, 0, stream>>>(ys, topv, inv, (int)K, H, out);
  return smel::launch_status();
}

extern "C" int smel_combine_bwd_f32(const float* ys, const float* dout, const float* topv, const int32_t* inv,
                                    int64_t T, int64_t K, int64_t H, float* dys, float* dtopv, hipStream_t stream) {
  SMEL_REQUIRE(ys && dout && topv && inv && dys && dtopv && T >= 0 && K > 0 && K <= 64 && H > 0 && T < (1LL << 31),
               SMEL_EINVAL, "smel_combine_bwd_f32: bad arguments");
  if (T == 0) return 0;
  combine_bwd_f32_kernel<<<(unsigned)T, 256, 0, stream>>>(ys, dout, topv, inv, (int)K, H, dys, dtopv);
  return smel::launch_status();
}

extern "C" int smel_dx_reduce_f32(const float* dxs, const int32_t* inv, int64_t T, int64_t K, int64_t H, float* dx,
                                  hipStream_t stream) {
  SMEL_REQUIRE(dxs && inv && dx && T >= 0 && K > 0 && K <= 64 && H > 0 && T < (1LL << 31), SMEL_EINVAL,
               "smel_dx_reduce_f32: bad arguments");
  if (T == 0) return 0;
  dx_reduce_f32_kernel<<<(unsigned)T, 256, 0, stream>>>(dxs, inv, (int)K, H, dx);
  return smel::launch_status();
}

extern "C" int smel_route_select_f32(const float* logits, int64_t ldl, int64_t T, int64_t E, int64_t K,
                                     const float* pes, float* probs, float* topv, int64_t* topi, int32_t* topi32,
                                     hipStream_t stream) {
  SMEL_REQUIRE(logits && probs && topv && topi && topi32, SMEL_EINVAL, "smel_route_select_f32: null pointer");
  SMEL_REQUIRE(E > 0 && E <= 512, SMEL_EUNSUPPORTED, "smel_route_select_f32: E=%lld outside 1..512", (long long)E);
  SMEL_REQUIRE(K > 0 && K <= 16 && K <= E, SMEL_EUNSUPPORTED, "smel_route_select_f32: top-k %lld outside 1..16",
               (long long)K);
  SMEL_REQUIRE(T >= 0 && ldl >= E && T < (1LL << 31), SMEL_EINVAL, "smel_route_select_f32: bad sizes");
  if (T == 0) return 0;
  const unsigned grid = (unsigned)((T + 3) / 4);
  if (E <= 256)
    route_select_f32_kernel<4><<<grid, 256, 0, stream>>>(logits, ldl, (int)T, (int)E, (int)K, pes, probs, topv, topi,
                                                         topi32);
  else
    route_select_f32_kernel<8><<<grid, 256, 0, stream>>>(logits, ldl, (int)T, (int)E, (int)K, pes, probs, topv, topi,
                                                         topi32);
  return smel::launch_status();
}

extern "C" int smel_route_bwd_f32(const float* dtopv, const float* probs, const int32_t* topi32, const float* pes,
                                  int64_t T, int64_t K, int64_t E, float* dlogits, hipStream_t stream) {
  SMEL_REQUIRE(dtopv && probs && topi32 && dlogits, SMEL_EINVAL, "smel_route_bwd_f32: null pointer");
  SMEL_REQUIRE(E > 0 && K > 0 && K <= 16 && T >= 0 && T < (1LL << 31), SMEL_EINVAL, "smel_route_bwd_f32: bad sizes");
  if (T == 0) return 0;
  route_bwd_f32_kernel<<<(unsigned)((T + 3) / 4), 256, 0, stream>>>(dtopv, probs, topi32, pes, (int)T, (int)K, (int)E,
                                                                    dlogits);
  return smel::launch_status();
}

extern "C" int smel_route_prenorm_f32(const float* h, const float* scale, int64_t T, int64_t H, float eps, float hs,
                                      float* xn, float* rstd, hipStream_t stream) {
  SMEL_REQUIRE(h && scale && xn && rstd && T >= 0 && H > 0 && T < (1LL << 31), SMEL_EINVAL,
               "smel_route_prenorm_f32: bad arguments");
  if (T == 0) return 0;
  route_prenorm_f32_kernel<<<(unsigned)T, 256, 0, stream>>>(h, scale, H, eps, hs, xn, rstd);
  return smel::launch_status();
}

extern "C" int smel_route_prenorm_bwd_f32(const float* h, const float* scale, const float* rstd, const float* dxn,
                                          int64_t T, int64_t H, float hs, float* dh, hipStream_t stream) {
  SMEL_REQUIRE(h && scale && rstd && dxn && dh && T >= 0 && H > 0 && T < (1LL << 31), SMEL_EINVAL,
               "smel_route_prenorm_bwd_f32: bad arguments");
  if (T == 0) return 0;
  route_prenorm_bwd_f32_kernel<<<(unsigned)T, 256, 0, stream>>>(h, scale, rstd, dxn, H, hs, dh);
  return smel::launch_status();
}

extern "C" int smel_gate_mul_f32(const float* y, const float* s, const float* base, int64_t T, int64_t H, float* out,
                                 hipStream_t stream) {
  SMEL_REQUIRE(y && s && out && T >= 0 && H > 0 && T < (1LL << 31), SMEL_EINVAL, "smel_gate_mul_f32: bad arguments");
  if (T == 0) return 0;
  gate_mul_f32_kernel<<<(unsigned)T, 256, 0, stream>>>(y, s, base, H, out);
  return smel::launch_status();
}

extern "C" int smel_gate_mul_bwd_f32(const float* y, const float* s, const float* dout, int64_t T, int64_t H,
                                     float* dy, float* ds, hipStream_t stream) {
  SMEL_REQUIRE(y && s && dout && dy && ds && T >= 0 && H > 0 && T < (1LL << 31), SMEL_EINVAL,
               "smel_gate_mul_bwd_f32: bad arguments");
  if (T == 0) return 0;
  gate_mul_bwd_f32_kernel<<<(unsigned)T, 256, 0, stream>>>(y, s, dout, H, dy, ds);
  return smel::launch_status();
}
