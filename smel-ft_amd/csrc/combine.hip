// Deterministic, atomic-free reductions over the K slots of a token: the weighted combine of the forward
// (smel/moe.py:248-252, plus the shared expert of :263) and the dX gather-reduce of the backward (the autograd of
// xs = x2d[tok] in smel/moe.py:223, which sums each token's K slot gradients). Fixed k order, fp32 accumulation.
// HBM-bound: the combine reads K+1 bf16 rows and writes one per token. A slot whose expert id was out of range was
// dropped by the dispatch (inv = -1, no GEMM wrote its row): it adds nothing here.
#include "abi_util.h"
#include "common.h"

namespace {

// One block per token, 8 columns (16 B) per thread per step.
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ Y, const float* __restrict__ topv,
                                                      const int32_t* __restrict__ inv,
                                                      const float* __restrict__ sgate,
                                                      const uint16_t* __restrict__ Ysh, int T, int K, int H,
                                                      uint16_t* __restrict__ out) {
  const int64_t t = blockIdx.x;
  float wk[16];
  uint32_t live = 0;   // bit k: slot k has a row
  for (int k = 0; k < K; ++k) {
    wk[k] = topv[t * K + k];
    if (!inv || inv[t * K + k] >= 0) live |= 1u << k;
  }
  const float ws = sgate ? sgate[t] : 0.f;
  const int64_t TK = (int64_t)T * K;
  const uint16_t* const ysh = Ysh ? Ysh + t * H : Y + (TK + t) * H;   // the shared expert's row
  for (int c = threadIdx.x * 8; c < H; c += blockDim.x * 8) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = 0; k < K; ++k) {
      if (!(live >> k & 1)) continue;   // uniform over the block
      const u32x4_t y = *reinterpret_cast<const u32x4_t*>(Y + (t * K + k) * H + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = fmaf(wk[k], bf_lo(y[j]), acc[2 * j]);
        acc[2 * j + 1] = fmaf(wk[k], bf_hi(y[j]), acc[2 * j + 1]);
      }
    }
    if (sgate) {
      const u32x4_t y = *reinterpret_cast<const u32x4_t*>(ysh + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = fmaf(ws, bf_lo(y[j]), acc[2 * j]);
        acc[2 * j + 1] = fmaf(ws, bf_hi(y[j]), acc[2 * j + 1]);
      }
    }
    *reinterpret_cast<u32x4_t*>(out + t * H + c) =
        u32x4_t{pack2bf(acc[0], acc[1]), pack2bf(acc[2], acc[3]), pack2bf(acc[4], acc[5]), pack2bf(acc[6], acc[7])};
  }
}

__global__ __launch_bounds__(256) void dx_reduce_kernel(const uint16_t* __restrict__ dxs,
                                                        const uint16_t* __restrict__ dxr,
                                                        const int32_t* __restrict__ inv, int with_shared,
                                                        const uint16_t* __restrict__ dxsh, int T, int K, int H,
                                                        uint16_t* __restrict__ dx) {
  const int64_t t = blockIdx.x;
  const int64_t TK = (int64_t)T * K;
  uint32_t live = 0;
  for (int k = 0; k < K; ++k)
    if (!inv || inv[t * K + k] >= 0) live |= 1u << k;
  for (int c = threadIdx.x * 8; c < H; c += blockDim.x * 8) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    auto add_row = [&](const uint16_t* p) {
      const u32x4_t y = *reinterpret_cast<const u32x4_t*>(p + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] += bf_lo(y[j]);
        acc[2 * j + 1] += bf_hi(y[j]);
      }
    };
    for (int k = 0; k < K; ++k)
      if (live >> k & 1) add_row(dxs + (t * K + k) * H);
    if (with_shared) add_row(dxsh ? dxsh + t * H : dxs + (TK + t) * H);
    if (dxr) add_row(dxr + t * H);
    *reinterpret_cast<u32x4_t*>(dx + t * H + c) =
        u32x4_t{pack2bf(acc[0], acc[1]), pack2bf(acc[2], acc[3]), pack2bf(acc[4], acc[5]), pack2bf(acc[6], acc[7])};
  }
}

}  // namespace

extern "C" int smel_combine(const uint16_t* Y, const float* topv, const int32_t* inv, const float* sgate,
                            const uint16_t* Ysh, int64_t T, int64_t K, int64_t H, uint16_t* out, hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && K > 0 && K <= 16 && H > 0, SMEL_EINVAL, "combine: bad sizes");
  SMEL_REQUIRE(H % 8 == 0, SMEL_EUNSUPPORTED, "combine: hidden %lld must be a multiple of 8", (long long)H);
  if (T == 0) return 0;
  SMEL_REQUIRE(Y && topv && out, SMEL_EINVAL, "combine: null pointer");
  combine_kernel<<<(unsigned)T, 256, 0, stream>>>(Y, topv, inv, sgate, Ysh, (int)T, (int)K, (int)H, out);
  return smel::launch_status();
}

extern "C" int smel_dx_reduce(const uint16_t* dxs, const uint16_t* dxr, const int32_t* inv, int32_t with_shared,
                              const uint16_t* dxsh, int64_t T, int64_t K, int64_t H, uint16_t* dx,
                              hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && K > 0 && H > 0, SMEL_EINVAL, "dx_reduce: bad sizes");
  SMEL_REQUIRE(H % 8 == 0, SMEL_EUNSUPPORTED, "dx_reduce: hidden %lld must be a multiple of 8", (long long)H);
  if (T == 0) return 0;
  SMEL_REQUIRE(dxs && dx, SMEL_EINVAL, "dx_reduce: null pointer");
  dx_reduce_kernel<<<(unsigned)T, 256, 0, stream>>>(dxs, dxr, inv, with_shared, dxsh, (int)T, (int)K, (int)H,
                                                      dx);
  return smel::launch_status();
}
