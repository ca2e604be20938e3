// Standalone int4 group dequant (the reference's _dq4_kernel, smel/quant.py:51-67): w = RNE(q*s + z) in fp32.
// HBM-bound: reads K/2 + 4K/group bytes and writes 2K (bf16) or 4K (fp32) bytes per row. Used for the bit-exact
// checks and by callers that want dense weights; the GEMMs dequantize in registers and never call it.
#include "abi_util.h"
#include "common.h"

namespace {

// One thread per 32-bit word of q (8 nibbles, 8 consecutive columns inside one group).
template <bool F32>
__global__ __launch_bounds__(256) void dequant_words(const uint32_t* __restrict__ q, const uint16_t* __restrict__ s,
                                                     const uint16_t* __restrict__ z, void* __restrict__ out,
                                                     int64_t n_words, int64_t words_per_row, int64_t groups,
                                                     int64_t group) {
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < n_words; w += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = w / words_per_row;
    const int64_t k0 = (w - row * words_per_row) * 8;
    const int64_t gi = row * groups + k0 / group;
    const float sc = bf2f(s[gi]), ze = bf2f(z[gi]);
    const uint32_t b = q[w];
    if (F32) {
      float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + w * 8);
      o[0] = make_float4(fmaf(nib(b, 0), sc, ze), fmaf(nib(b, 1), sc, ze), fmaf(nib(b, 2), sc, ze),
                         fmaf(nib(b, 3), sc, ze));
      o[1] = make_float4(fmaf(nib(b, 4), sc, ze), fmaf(nib(b, 5), sc, ze), fmaf(nib(b, 6), sc, ze),
                         fmaf(nib(b, 7), sc, ze));
    } else {
      uint32_t v[4];
      dq8(b, sc, ze, v);
      reinterpret_cast<uint4*>(static_cast<uint16_t*>(out))[w] = make_uint4(v[0], v[1], v[2], v[3]);
    }
  }
}

// Fallback: one thread per byte (any even K / even group).
template <bool F32>
__global__ __launch_bounds__(256) void dequant_bytes(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                                     const uint16_t* __restrict__ z, void* __restrict__ out,
                                                     int64_t n_bytes, int64_t half_k, int64_t groups, int64_t group) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_bytes; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / half_k;
    const int64_t k = (i - row * half_k) * 2;
    const int64_t gi = row * groups + k / group;
    const float sc = bf2f(s[gi]), ze = bf2f(z[gi]);
    const uint32_t b = q[i];
    const float lo = fmaf((float)(b & 0xf), sc, ze), hi = fmaf((float)(b >> 4), sc, ze);
    if (F32) {
      static_cast<float*>(out)[2 * i] = lo;
      static_cast<float*>(out)[2 * i + 1] = hi;
    } else {
      reinterpret_cast<uint32_t*>(out)[i] = pack2bf(lo, hi);
    }
  }
}

// sz[(r*2 + h)*nks + ks] = scale | zero << 16 of the group holding column 64*ks + 32*h.
__global__ __launch_bounds__(256) void pack_sz(const uint16_t* __restrict__ s, const uint16_t* __restrict__ z,
                                               int64_t rows, int64_t K, int64_t group, int64_t nks,
                                               uint32_t* __restrict__ out) {
  const int64_t G = K / group;
  const int64_t n = rows * 2 * nks;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t ks = i % nks;
    const int64_t h = (i / nks) & 1;
    const int64_t r = i / (2 * nks);
    const int64_t k = 64 * ks + 32 * h;
    uint32_t v = 0;
    if (k < K) {
      const int64_t gi = r * G + k / group;
      v = (uint32_t)s[gi] | ((uint32_t)z[gi] << 16);
    }
    out[i] = v;
  }
}

}  // namespace

extern "C" int smel_int4_pack_sz(const uint16_t* scale, const uint16_t* zero, int64_t rows, int64_t K, int64_t group,
                                 uint32_t* sz, hipStream_t stream) {
  SMEL_REQUIRE(rows >= 0 && K > 0 && group > 0 && K % group == 0 && group % 32 == 0, SMEL_EUNSUPPORTED,
               "int4_pack_sz: K=%lld, group=%lld (group must be a multiple of 32 dividing K)", (long long)K,
               (long long)group);
  if (rows == 0) return 0;
  SMEL_REQUIRE(scale && zero && sz, SMEL_EINVAL, "int4_pack_sz: null pointer");
  const int64_t nks = (K + 63) / 64;
  const int64_t n = rows * 2 * nks;
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 256 * 64);
  pack_sz<<<blocks, 256, 0, stream>>>(scale, zero, rows, K, group, nks, sz);
  return smel::launch_status();
}

extern "C" int smel_dequant_int4(const uint8_t* q, const uint16_t* scale, const uint16_t* zero, void* out,
                                 int64_t rows, int64_t K, int64_t group, int32_t out_f32, hipStream_t stream) {
  SMEL_REQUIRE(rows >= 0 && K > 0 && group > 0, SMEL_EINVAL, "dequant_int4: bad sizes rows=%lld K=%lld group=%lld",
               (long long)rows, (long long)K, (long long)group);
  SMEL_REQUIRE(K % group == 0 && group % 2 == 0, SMEL_EINVAL, "dequant_int4: K=%lld must be a multiple of the even "
               "group %lld", (long long)K, (long long)group);
  if (rows == 0) return 0;
  SMEL_REQUIRE(q && scale && zero && out, SMEL_EINVAL, "dequant_int4: null pointer");
  const int64_t groups = K / group;
  const bool words = (K % 8 == 0) && (group % 8 == 0) && ((uintptr_t)q % 4 == 0) &&
                     ((uintptr_t)out % (out_f32 ? 16 : 16) == 0);
  if (words) {
    const int64_t n = rows * K / 8;
    const int blocks = (int)std::min<int64_t>((n + 255) / 256, 256 * 64);
    if (out_f32)
      dequant_words<true><<<blocks, 256, 0, stream>>>((const uint32_t*)q, scale, zero, out, n, K / 8, groups, group);
    else
      dequant_words<false><<<blocks, 256, 0, stream>>>((const uint32_t*)q, scale, zero, out, n, K / 8, groups, group);
  } else {
    const int64_t n = rows * K / 2;
    const int blocks = (int)std::min<int64_t>((n + 255) / 256, 256 * 64);
    if (out_f32)
      dequant_bytes<true><<<blocks, 256, 0, stream>>>(q, scale, zero, out, n, K / 2, groups, group);
    else
      dequant_bytes<false><<<blocks, 256, 0, stream>>>(q, scale, zero, out, n, K / 2, groups, group);
  }
  return smel::launch_status();
}
