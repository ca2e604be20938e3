// Single-pass chunked cross-entropy over a frozen lm_head (smel/loss.py:50-92): the per-chunk online softmax state
// and the gradient terms, between the two GEMMs of each (token chunk, vocabulary chunk) step.
//
//   ce_chunk_update  (one block per token row): z = cap(logit) (cap = c tanh(z / c), or none), chunk max cm,
//                    new running max nm = max(m, cm), rescale r = exp(m - nm), softmax terms e = exp(z - nm),
//                    s = s r + sum(e), p = e (1 - (z / c)^2 with the cap) written in the rows' dtype for the
//                    gradient GEMM p W, and the target's capped logit and cap derivative when it lies in the chunk
//                    (smel/loss.py:62-84; no host synchronisation: the reference's `inside.any()` / `nonzero`
//                    become a comparison in the kernel)
//   ce_acc_update    acc = acc r + (p W) (smel/loss.py:85): one pass over the fp32 accumulator, summing the parts of
//                    the gradient GEMM in fixed order. The gradient GEMM p W has a long K (the vocabulary chunk) and
//                    a small output ([tokens, H]: 32 tiles of 256 x 256 at 1024 tokens, too few for 256 CUs), so p is
//                    written split into `parts` column slices [parts][n][vc / parts] and multiplied slice by slice
//                    in one batched GEMM (a split K)
// fp32 math; the GEMM outputs arrive rounded to the rows' dtype, as the reference's `(h @ W.t()).float()`.
// 16-bit rows move through 16-byte loads and stores (8 values per thread and step) when the chunk allows it.
#include "../../include/smel_loss.h"
#include "abi_util.h"
#include "common.h"

namespace {

template <int DT>
SMEL_DEV float ld_t(const void* p, int64_t i) {
  if constexpr (DT == 0) return __uint_as_float((uint32_t) static_cast<const uint16_t*>(p)[i] << 16);
  else if constexpr (DT == 1) return static_cast<const float*>(p)[i];
  else return (float)static_cast<const _Float16*>(p)[i];
}
template <int DT>
SMEL_DEV void st_t(void* p, int64_t i, float v) {
  if constexpr (DT == 0) static_cast<uint16_t*>(p)[i] = f2bf(v);
  else if constexpr (DT == 1) static_cast<float*>(p)[i] = v;
  else static_cast<_Float16*>(p)[i] = (_Float16)v;
}

SMEL_DEV float capf(float z, float c) { return c != 0.f ? c * tanhf(z / c) : z; }

// block-wide reduction of 256 threads: fixed order (xor butterfly per wave, then the four wave values in order)
template <bool MAX>
SMEL_DEV float block_reduce(float v, float* red) {
  for (int o = 1; o < 64; o <<= 1) {
    const float u = __shfl_xor(v, o, 64);
    v = MAX ? fmaxf(v, u) : v + u;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return MAX ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) : ((red[0] + red[1]) + red[2]) + red[3];
}

// 8 values of a 16-bit row from one 16-byte load
template <int DT>
SMEL_DEV void ld8(const void* p, int64_t i, float v[8]) {
  const u32x4_t q = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p) + i);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[2 * k] = DT == 0 ? bf_lo(q[k]) : h_lo(q[k]);
    v[2 * k + 1] = DT == 0 ? bf_hi(q[k]) : h_hi(q[k]);
  }
}

// VEC: 16-bit rows whose chunk width, row stride and base pointers are multiples of 8 elements / 16 bytes
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void ce_chunk_update_kernel(const void* __restrict__ lg, int64_t ld, int vc,
                                                              int64_t v0, const int64_t* __restrict__ tgt, float cap,
                                                              int need_grad, float* m, float* s, float* tgt_logit,
                                                              float* tgt_d, void* p, float* r_out, int64_t n, int sw) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t base = row * ld;
  // p in the split layout [vc / sw][n][sw]: column j of the row goes to part j / sw, column j % sw
  auto p_at = [&](int j) { return (int64_t)(j / sw) * n * sw + row * (int64_t)sw + (j % sw); };
  float cm = -INFINITY;
  if constexpr (VEC) {
    for (int c = threadIdx.x; c < vc / 8; c += 256) {
      float v[8];
      ld8<DT>(lg, base + 8 * c, v);
#pragma unroll
      for (int k = 0; k < 8; ++k) cm = fmaxf(cm, capf(v[k], cap));
    }
  } else {
    for (int j = threadIdx.x; j < vc; j += 256) cm = fmaxf(cm, capf(ld_t<DT>(lg, base + j), cap));
  }
  cm = block_reduce<true>(cm, red);
  const float m_old = m[row];
  const float nm = fmaxf(m_old, cm);
  const float r = expf(m_old - nm);   // exp(-inf) = 0 on the first chunk
  float sum = 0.f;
  if constexpr (VEC) {
    for (int c = threadIdx.x; c < vc / 8; c += 256) {
      float v[8];
      ld8<DT>(lg, base + 8 * c, v);
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 8; k += 2) {
        float q2[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const float z = capf(v[k + u], cap);
          const float e = expf(z - nm);
          sum += e;
          q2[u] = cap != 0.f ? e * (1.f - (z / cap) * (z / cap)) : e;
        }
        o[k / 2] = DT == 0 ? pack2bf(q2[0], q2[1])
                           : (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)q2[0]) |
                                 ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)q2[1]) << 16);
      }
      if (need_grad)
        *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(p) + p_at(8 * c)) =
            u32x4_t{o[0], o[1], o[2], o[3]};
    }
  } else {
    for (int j = threadIdx.x; j < vc; j += 256) {
      const float z = capf(ld_t<DT>(lg, base + j), cap);
      const float e = expf(z - nm);
      sum += e;
      if (need_grad) {
        const float q = cap != 0.f ? e * (1.f - (z / cap) * (z / cap)) : e;
        st_t<DT>(p, p_at(j), q);
      }
    }
  }
  sum = block_reduce<false>(sum, red);
  if (threadIdx.x == 0) {
    s[row] = s[row] * r + sum;
    m[row] = nm;
    r_out[row] = r;
    const int64_t t = tgt[row] - v0;
    if (t >= 0 && t < vc) {
      const float z = capf(ld_t<DT>(lg, base + t), cap);
      tgt_logit[row] = z;
      if (cap != 0.f) tgt_d[row] = 1.f - (z / cap) * (z / cap);
    }
  }
}

template <int DT>
__global__ __launch_bounds__(256) void ce_acc_update_kernel(float* __restrict__ acc, const float* __restrict__ r,
                                                            const void* __restrict__ pw, int64_t n, int64_t H,
                                                            int parts) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n * H) return;
  float v = ld_t<DT>(pw, i);
  for (int k = 1; k < parts; ++k) v += ld_t<DT>(pw, (int64_t)k * n * H + i);   // the split products, in order
  acc[i] = acc[i] * r[i / H] + v;
}

// the same for 16-bit products with H % 8 == 0 and 16-byte aligned buffers: 8 elements per thread
template <int DT>
__global__ __launch_bounds__(256) void ce_acc_update8_kernel(float* __restrict__ acc, const float* __restrict__ r,
                                                             const void* __restrict__ pw, int64_t n, int64_t H,
                                                             int parts) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i >= n * H) return;
  float v[8];
  ld8<DT>(pw, i, v);
  for (int k = 1; k < parts; ++k) {
    float u[8];
    ld8<DT>(pw, (int64_t)k * n * H + i, u);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] += u[e];
  }
  const float rr = r[i / H];
  f32x4_t* const a4 = reinterpret_cast<f32x4_t*>(acc + i);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const f32x4_t a = a4[h];
    a4[h] = f32x4_t{a[0] * rr + v[4 * h], a[1] * rr + v[4 * h + 1], a[2] * rr + v[4 * h + 2], a[3] * rr + v[4 * h + 3]};
  }
}

}  // namespace

extern "C" int smel_ce_chunk_update(const void* logits, int64_t n, int64_t vc, int64_t ld, int64_t v0,
                                    const int64_t* tgt, float softcap, int32_t dtype, int32_t need_grad, float* m,
                                    float* s, float* tgt_logit, float* tgt_d, void* p, int32_t p_parts, float* r,
                                    hipStream_t stream) {
  SMEL_REQUIRE(p_parts >= 1 && vc % p_parts == 0, SMEL_EINVAL, "ce_chunk_update: %d parts do not divide %lld columns",
               p_parts, (long long)vc);
  SMEL_REQUIRE(n >= 0 && vc >= 1 && vc <= INT32_MAX && ld >= vc, SMEL_EINVAL,
               "ce_chunk_update: bad sizes n=%lld vc=%lld ld=%lld", (long long)n, (long long)vc, (long long)ld);
  SMEL_REQUIRE(dtype >= 0 && dtype <= 2, SMEL_EINVAL, "ce_chunk_update: dtype %d (0 bf16, 1 fp32, 2 fp16)", dtype);
  SMEL_REQUIRE(n < (int64_t)1 << 31, SMEL_EUNSUPPORTED, "ce_chunk_update: %lld rows", (long long)n);
  if (n == 0) return 0;
  SMEL_REQUIRE(logits && tgt && m && s && tgt_logit && tgt_d && r && (!need_grad || p), SMEL_EINVAL,
               "ce_chunk_update: null pointer");
  const dim3 g((unsigned)n), b(256);
  const int sw = (int)(vc / p_parts);
  const bool vec = dtype != 1 && sw % 8 == 0 && ld % 8 == 0 && (uintptr_t)logits % 16 == 0 &&
                   (!need_grad || (uintptr_t)p % 16 == 0);
#define SMEL_CE_LAUNCH(D, V)                                                                                     \
  ce_chunk_update_kernel<D, V><<<g, b, 0, stream>>>(logits, ld, (int)vc, v0, tgt, softcap, need_grad, m, s, tgt_logit, \
                                                    tgt_d, p, r, n, sw)
  if (dtype == 0 && vec)
    SMEL_CE_LAUNCH(0, true);
  else if (dtype == 0)
    SMEL_CE_LAUNCH(0, false);
  else if (dtype == 2 && vec)
    SMEL_CE_LAUNCH(2, true);
  else if (dtype == 2)
    SMEL_CE_LAUNCH(2, false);
  else
    SMEL_CE_LAUNCH(1, false);
#undef SMEL_CE_LAUNCH
  return smel::launch_status();
}

extern "C" int smel_ce_acc_update(float* acc, const float* r, const void* pw, int32_t parts, int64_t n, int64_t H,
                                  int32_t dtype, hipStream_t stream) {
  SMEL_REQUIRE(n >= 0 && H >= 1 && parts >= 1, SMEL_EINVAL, "ce_acc_update: bad sizes");
  SMEL_REQUIRE(dtype >= 0 && dtype <= 2, SMEL_EINVAL, "ce_acc_update: dtype %d", dtype);
  if (n == 0) return 0;
  SMEL_REQUIRE(acc && r && pw, SMEL_EINVAL, "ce_acc_update: null pointer");
  const bool vec = dtype != 1 && H % 8 == 0 && (uintptr_t)acc % 16 == 0 && (uintptr_t)pw % 16 == 0;
  const int64_t blocks = vec ? (n * H / 8 + 255) / 256 : (n * H + 255) / 256;
  SMEL_REQUIRE(blocks < (int64_t)1 << 31, SMEL_EUNSUPPORTED, "ce_acc_update: too large");
  const dim3 g((unsigned)blocks), b(256);
  if (vec && dtype == 0)
    ce_acc_update8_kernel<0><<<g, b, 0, stream>>>(acc, r, pw, n, H, parts);
  else if (vec)
    ce_acc_update8_kernel<2><<<g, b, 0, stream>>>(acc, r, pw, n, H, parts);
  else if (dtype == 0)
    ce_acc_update_kernel<0><<<g, b, 0, stream>>>(acc, r, pw, n, H, parts);
  else if (dtype == 1)
    ce_acc_update_kernel<1><<<g, b, 0, stream>>>(acc, r, pw, n, H, parts);
  else
    ce_acc_update_kernel<2><<<g, b, 0, stream>>>(acc, r, pw, n, H, parts);
  return smel::launch_status();
}
