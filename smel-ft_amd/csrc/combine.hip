// Deterministic, atomic-free reductions over the K slots of a token: the weighted combine of the forward
// (smel/moe.py:248-252, plus the shared expert of :263) and the dX gather-reduce of the backward (the autograd of
// xs = x2d[tok] in smel/moe.py:223, which sums each token's K slot gradients). Fixed k order, fp32 accumulation.
// HBM-bound: the combine reads K+1 bf16 rows and writes one per token. A slot whose expert id was out of range was
// dropped by the dispatch (inv = -1, no GEMM wrote its row): it adds nothing here.
#include "abi_util.h"
#include "common.h"

namespace {

// One block per token, 8 columns (16 B) per thread per step. Every row of a step is loaded before the first is
// used (a dropped slot's load is out of range and reads zeros), so a thread has all of its token's rows in flight
// at once; the sums still run in the fixed k order. KM = the largest K the instance takes.
template <int KM>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ Y, const float* __restrict__ topv,
                                                      const int32_t* __restrict__ inv,
                                                      const float* __restrict__ sgate,
                                                      const uint16_t* __restrict__ Ysh, int T, int K, int H,
                                                      uint16_t* __restrict__ out) {
  const int64_t t = blockIdx.x;
  const rsrc_t ry = make_rsrc(Y + t * K * H, (uint64_t)K * H * 2);   // the token's K slot rows
  float wk[KM];
  uint32_t base[KM];   // byte offset of slot k's row, OOB for a dropped or absent slot
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    const bool live = k < K && (!inv || inv[t * K + k] >= 0);
    wk[k] = live ? topv[t * K + k] : 0.f;
    base[k] = live ? (uint32_t)(k * H * 2) : OOB;
  }
  const float ws = sgate ? sgate[t] : 0.f;
  const int64_t TK = (int64_t)T * K;
  const uint16_t* const ysh = Ysh ? Ysh + t * H : Y + (TK + t) * H;   // the shared expert's row
  const rsrc_t rs = make_rsrc(ysh, sgate ? (uint64_t)H * 2 : 0);
  for (int c = threadIdx.x * 8; c < H; c += blockDim.x * 8) {
    u32x4_t y[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) y[k] = ld16(ry, base[k] == OOB ? OOB : base[k] + 2 * c);
    const u32x4_t ys = ld16(rs, 2 * c);
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < KM; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = fmaf(wk[k], bf_lo(y[k][j]), acc[2 * j]);
        acc[2 * j + 1] = fmaf(wk[k], bf_hi(y[k][j]), acc[2 * j + 1]);
      }
    if (sgate) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = fmaf(ws, bf_lo(ys[j]), acc[2 * j]);
        acc[2 * j + 1] = fmaf(ws, bf_hi(ys[j]), acc[2 * j + 1]);
      }
    }
    *reinterpret_cast<u32x4_t*>(out + t * H + c) =
        u32x4_t{pack2bf(acc[0], acc[1]), pack2bf(acc[2], acc[3]), pack2bf(acc[4], acc[5]), pack2bf(acc[6], acc[7])};
  }
}

// Same load pattern: the K slot rows, then the shared expert's row and the router's dX row, all in flight at once;
// summed in that order.
template <int KM>
__global__ __launch_bounds__(256) void dx_reduce_kernel(const uint16_t* __restrict__ dxs,
                                                        const uint16_t* __restrict__ dxr,
                                                        const int32_t* __restrict__ inv, int with_shared,
                                                        const uint16_t* __restrict__ dxsh, int T, int K, int H,
                                                        uint16_t* __restrict__ dx) {
  const int64_t t = blockIdx.x;
  const int64_t TK = (int64_t)T * K;
  const rsrc_t rk = make_rsrc(dxs + t * K * H, (uint64_t)K * H * 2);
  uint32_t base[KM];
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    const bool live = k < K && (!inv || inv[t * K + k] >= 0);
    base[k] = live ? (uint32_t)(k * H * 2) : OOB;
  }
  const rsrc_t rs = make_rsrc(dxsh ? dxsh + t * H : dxs + (TK + t) * H, with_shared ? (uint64_t)H * 2 : 0);
  const rsrc_t rr = make_rsrc(dxr ? dxr + t * H : dxs, dxr ? (uint64_t)H * 2 : 0);
  for (int c = threadIdx.x * 8; c < H; c += blockDim.x * 8) {
    u32x4_t y[KM + 2];
#pragma unroll
    for (int k = 0; k < KM; ++k) y[k] = ld16(rk, base[k] == OOB ? OOB : base[k] + 2 * c);
    y[KM] = ld16(rs, 2 * c);
    y[KM + 1] = ld16(rr, 2 * c);
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    auto add_row = [&](const u32x4_t& v) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] += bf_lo(v[j]);
        acc[2 * j + 1] += bf_hi(v[j]);
      }
    };
#pragma unroll
    for (int k = 0; k < KM; ++k)
      if (base[k] != OOB) add_row(y[k]);
    if (with_shared) add_row(y[KM]);
    if (dxr) add_row(y[KM + 1]);
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
  SMEL_REQUIRE((int64_t)K * H * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "combine: K x hidden too large");
  if (K <= 8)
    combine_kernel<8><<<(unsigned)T, 256, 0, stream>>>(Y, topv, inv, sgate, Ysh, (int)T, (int)K, (int)H, out);
  else
    combine_kernel<16><<<(unsigned)T, 256, 0, stream>>>(Y, topv, inv, sgate, Ysh, (int)T, (int)K, (int)H, out);
  return smel::launch_status();
}

extern "C" int smel_dx_reduce(const uint16_t* dxs, const uint16_t* dxr, const int32_t* inv, int32_t with_shared,
                              const uint16_t* dxsh, int64_t T, int64_t K, int64_t H, uint16_t* dx,
                              hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && K > 0 && K <= 16 && H > 0, SMEL_EINVAL, "dx_reduce: bad sizes");
  SMEL_REQUIRE(H % 8 == 0, SMEL_EUNSUPPORTED, "dx_reduce: hidden %lld must be a multiple of 8", (long long)H);
  if (T == 0) return 0;
  SMEL_REQUIRE(dxs && dx, SMEL_EINVAL, "dx_reduce: null pointer");
  SMEL_REQUIRE((int64_t)K * H * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "dx_reduce: K x hidden too large");
  if (K <= 8)
    dx_reduce_kernel<8><<<(unsigned)T, 256, 0, stream>>>(dxs, dxr, inv, with_shared, dxsh, (int)T, (int)K, (int)H,
                                                         dx);
  else
    dx_reduce_kernel<16><<<(unsigned)T, 256, 0, stream>>>(dxs, dxr, inv, with_shared, dxsh, (int)T, (int)K, (int)H,
                                                          dx);
  return smel::launch_status();
}
