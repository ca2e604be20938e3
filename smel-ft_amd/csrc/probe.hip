// Peak probes (include/smel_probe.h): an MFMA-only loop and 16-byte-per-lane streaming read / copy kernels.
#include "../../include/smel_probe.h"
#include "abi_util.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kLanes = 256;
constexpr int kChains = 8;   // independent accumulators per wave: enough to cover the 32x32x16 MFMA's latency

__global__ __launch_bounds__(kLanes) void mfma_loop_kernel(float* __restrict__ out, int iters) {
  f32x16 acc[kChains];
  for (int j = 0; j < kChains; ++j) acc[j] = f32x16{};
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(threadIdx.x * 1e-3f + i);
    b[i] = (__bf16)(0.5f * i);
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kChains; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
  }
  float t = 0.f;
  for (int j = 0; j < kChains; ++j) t += acc[j][0] + acc[j][7];
  out[(size_t)blockIdx.x * kLanes + threadIdx.x] = t;
}

__global__ __launch_bounds__(kLanes) void read_kernel(const u32x4* __restrict__ src, int64_t n,
                                                      uint32_t* __restrict__ out) {
  uint32_t acc = 0;
  const int64_t step = (int64_t)gridDim.x * kLanes;
  for (int64_t i = (int64_t)blockIdx.x * kLanes + threadIdx.x; i < n; i += step) {
    u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  out[(size_t)blockIdx.x * kLanes + threadIdx.x] = acc;
}

__global__ __launch_bounds__(kLanes) void copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                      int64_t n) {
  const int64_t step = (int64_t)gridDim.x * kLanes;
  for (int64_t i = (int64_t)blockIdx.x * kLanes + threadIdx.x; i < n; i += step) dst[i] = src[i];
}

}  // namespace

extern "C" int smel_probe_mfma(float* out, int32_t blocks, int32_t iters, hipStream_t stream) {
  SMEL_REQUIRE(out != nullptr, SMEL_EINVAL, "probe_mfma: null output");
  SMEL_REQUIRE(blocks > 0 && blocks <= (1 << 20) && iters >= 0, SMEL_EINVAL, "probe_mfma: bad blocks=%d iters=%d",
               blocks, iters);
  mfma_loop_kernel<<<blocks, kLanes, 0, stream>>>(out, iters);
  return smel::launch_status();
}

extern "C" int smel_probe_read(const void* src, int64_t bytes, uint32_t* out, int32_t grid, hipStream_t stream) {
  SMEL_REQUIRE(src != nullptr && out != nullptr, SMEL_EINVAL, "probe_read: null pointer");
  SMEL_REQUIRE(bytes >= 0 && bytes % 16 == 0, SMEL_EINVAL, "probe_read: bytes=%lld is not a multiple of 16",
               (long long)bytes);
  SMEL_REQUIRE(grid > 0 && grid <= 65536, SMEL_EINVAL, "probe_read: bad grid %d", grid);
  read_kernel<<<grid, kLanes, 0, stream>>>(static_cast<const u32x4*>(src), bytes / 16, out);
  return smel::launch_status();
}

extern "C" int smel_probe_copy(const void* src, void* dst, int64_t bytes, int32_t grid, hipStream_t stream) {
  SMEL_REQUIRE(src != nullptr && dst != nullptr, SMEL_EINVAL, "probe_copy: null pointer");
  SMEL_REQUIRE(bytes >= 0 && bytes % 16 == 0, SMEL_EINVAL, "probe_copy: bytes=%lld is not a multiple of 16",
               (long long)bytes);
  SMEL_REQUIRE(grid > 0 && grid <= 65536, SMEL_EINVAL, "probe_copy: bad grid %d", grid);
  if (bytes == 0) return 0;
  copy_kernel<<<grid, kLanes, 0, stream>>>(static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), bytes / 16);
  return smel::launch_status();
}
