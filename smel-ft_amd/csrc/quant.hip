// Group-wise asymmetric int4 quantization of frozen experts on the GPU (smel/quant.py:5-44): per group of `group`
// consecutive weights, the [min, max] range shrunk about its midpoint by each clip factor in turn, the candidate
// with the smallest squared error kept (a later factor only if strictly better), q packed two per byte (even column
// in the low nibble), scale and zero as bf16.
//
// Every operation is the reference's fp32 operation in the reference's order, each rounded on its own (no fused
// multiply-add: contraction is off in this file): mid = (mn + mx) / 2, bounds mid + (b - mid) c, scale =
// bf16(max((mx - mn) / 15, 1e-8)), zero = bf16(mn), q = clamp(rint((w - zero) / scale), 0, 15), err = sum of
// (q scale + zero - w)^2. The one order the reference leaves to its library is that of the error sum; here it is
// the group's index order, so a candidate can differ from the reference's only where two candidates' errors agree
// to the last bits of fp32.
//
// One thread per group (the error sum runs in index order within the thread). Groups of 32, 64 and 128 are loaded
// once with 16-byte loads into registers; other even sizes re-read the group from the cache for each candidate.
// Offline format producer: runs once per bank, not on the training step.
#include "abi_util.h"
#include "common.h"

#pragma clang fp contract(off)

namespace {

constexpr int MAX_CLIP = 8;

struct QArgs {
  const void* w;
  int dt;   // 0 bf16, 1 fp32, 2 fp16
  int group, nclip;
  int64_t groups;
  float clip[MAX_CLIP];
  uint8_t* q;
  uint16_t* scale;
  uint16_t* zero;
};

SMEL_DEV float ldw(const QArgs& a, int64_t i) {
  if (a.dt == 0) return __uint_as_float((uint32_t)static_cast<const uint16_t*>(a.w)[i] << 16);
  if (a.dt == 1) return static_cast<const float*>(a.w)[i];
  return (float)static_cast<const _Float16*>(a.w)[i];
}

SMEL_DEV float bf16_round(float f) { return __uint_as_float((uint32_t)f2bf(f) << 16); }

SMEL_DEV float qval(float w, float s, float z) { return fminf(fmaxf(rintf((w - z) / s), 0.f), 15.f); }

// the whole search for one group held in registers v[0..G)
template <int G>
SMEL_DEV void search(const float (&v)[G], const QArgs& a, float& best_s, float& best_z) {
  float mn0 = v[0], mx0 = v[0];
#pragma unroll
  for (int j = 1; j < G; ++j) {
    mn0 = fminf(mn0, v[j]);
    mx0 = fmaxf(mx0, v[j]);
  }
  const float mid = (mn0 + mx0) / 2.f;
  float best_err = 0.f;
  for (int c = 0; c < a.nclip; ++c) {
    const float cf = a.clip[c];
    const float mn = mid + (mn0 - mid) * cf;
    const float mx = mid + (mx0 - mid) * cf;
    const float s = bf16_round(fmaxf((mx - mn) / 15.f, 1e-8f));
    const float z = bf16_round(mn);
    float err = 0.f;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float d = qval(v[j], s, z) * s + z - v[j];
      err = err + d * d;
    }
    if (c == 0 || err < best_err) {
      best_err = err;
      best_s = s;
      best_z = z;
    }
  }
}

template <int G>
__global__ __launch_bounds__(256) void quantize_int4_reg_kernel(QArgs a) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gi >= a.groups) return;
  const int64_t base = gi * G;
  float v[G];
  if (a.dt == 1) {
    const f32x4_t* p = reinterpret_cast<const f32x4_t*>(static_cast<const float*>(a.w) + base);
#pragma unroll
    for (int j = 0; j < G / 4; ++j) {
      const f32x4_t x = p[j];
      v[4 * j] = x[0], v[4 * j + 1] = x[1], v[4 * j + 2] = x[2], v[4 * j + 3] = x[3];
    }
  } else {
    const u32x4_t* p = reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(a.w) + base);
#pragma unroll
    for (int j = 0; j < G / 8; ++j) {
      const u32x4_t x = p[j];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (a.dt == 0) {
          v[8 * j + 2 * k] = bf_lo(x[k]);
          v[8 * j + 2 * k + 1] = bf_hi(x[k]);
        } else {
          v[8 * j + 2 * k] = h_lo(x[k]);
          v[8 * j + 2 * k + 1] = h_hi(x[k]);
        }
      }
    }
  }
  float s, z;
  search<G>(v, a, s, z);
  uint32_t packed[G / 8];
#pragma unroll
  for (int j = 0; j < G / 8; ++j) {
    uint32_t wv = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) wv |= (uint32_t)qval(v[8 * j + k], s, z) << (4 * k);
    packed[j] = wv;
  }
  uint32_t* const qo = reinterpret_cast<uint32_t*>(a.q + base / 2);
#pragma unroll
  for (int j = 0; j < G / 32; ++j)
    reinterpret_cast<u32x4_t*>(qo)[j] = u32x4_t{packed[4 * j], packed[4 * j + 1], packed[4 * j + 2], packed[4 * j + 3]};
  if constexpr (G % 32 != 0) {
#pragma unroll
    for (int j = (G / 32) * 4; j < G / 8; ++j) qo[j] = packed[j];
  }
  a.scale[gi] = f2bf(s);
  a.zero[gi] = f2bf(z);
}

__global__ __launch_bounds__(256) void quantize_int4_kernel(QArgs a) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gi >= a.groups) return;
  const int64_t base = gi * a.group;
  float mn0 = ldw(a, base), mx0 = mn0;
  for (int j = 1; j < a.group; ++j) {
    const float v = ldw(a, base + j);
    mn0 = fminf(mn0, v);
    mx0 = fmaxf(mx0, v);
  }
  const float mid = (mn0 + mx0) / 2.f;
  float best_err = 0.f, best_s = 0.f, best_z = 0.f;
  for (int c = 0; c < a.nclip; ++c) {
    const float cf = a.clip[c];
    const float mn = mid + (mn0 - mid) * cf;
    const float mx = mid + (mx0 - mid) * cf;
    const float s = bf16_round(fmaxf((mx - mn) / 15.f, 1e-8f));
    const float z = bf16_round(mn);
    float err = 0.f;
    for (int j = 0; j < a.group; ++j) {
      const float v = ldw(a, base + j);
      const float d = qval(v, s, z) * s + z - v;
      err = err + d * d;
    }
    if (c == 0 || err < best_err) {
      best_err = err;
      best_s = s;
      best_z = z;
    }
  }
  uint8_t* const qo = a.q + base / 2;
  for (int j = 0; j < a.group; j += 2) {
    const uint32_t q0 = (uint32_t)qval(ldw(a, base + j), best_s, best_z);
    const uint32_t q1 = (uint32_t)qval(ldw(a, base + j + 1), best_s, best_z);
    qo[j / 2] = (uint8_t)(q0 | (q1 << 4));
  }
  a.scale[gi] = f2bf(best_s);
  a.zero[gi] = f2bf(best_z);
}

}  // namespace

extern "C" int smel_quantize_int4(const void* w, int32_t w_dtype, int64_t rows, int64_t K, int32_t group,
                                  const float* clip, int32_t n_clip, uint8_t* q, uint16_t* scale, uint16_t* zero,
                                  hipStream_t stream) {
  SMEL_REQUIRE(rows >= 0 && K > 0, SMEL_EINVAL, "quantize_int4: bad sizes rows=%lld K=%lld", (long long)rows,
               (long long)K);
  SMEL_REQUIRE(group > 0 && group % 2 == 0 && K % group == 0, SMEL_EINVAL,
               "quantize_int4: K=%lld is not a multiple of the even group %d", (long long)K, group);
  SMEL_REQUIRE(w_dtype >= 0 && w_dtype <= 2, SMEL_EINVAL, "quantize_int4: w_dtype %d (0 bf16, 1 fp32, 2 fp16)",
               w_dtype);
  SMEL_REQUIRE(n_clip >= 1 && n_clip <= MAX_CLIP && clip, SMEL_EINVAL, "quantize_int4: %d clip factors (1..%d)",
               n_clip, MAX_CLIP);
  if (rows == 0) return 0;
  SMEL_REQUIRE(w && q && scale && zero, SMEL_EINVAL, "quantize_int4: null pointer");
  QArgs a{};
  a.w = w;
  a.dt = w_dtype;
  a.group = group;
  a.nclip = n_clip;
  a.groups = rows * (K / group);
  for (int i = 0; i < n_clip; ++i) a.clip[i] = clip[i];
  a.q = q;
  a.scale = scale;
  a.zero = zero;
  const int64_t blocks = (a.groups + 255) / 256;
  SMEL_REQUIRE(blocks < (int64_t)1 << 31, SMEL_EUNSUPPORTED, "quantize_int4: too many groups");
  // registers + 16-byte loads when every group starts 16-byte aligned (the q row of a group is group/2 bytes)
  const int esz = w_dtype == 1 ? 4 : 2;
  const bool aligned = ((uintptr_t)w % 16 == 0) && ((uintptr_t)q % 16 == 0) && (group * esz) % 16 == 0 &&
                       (group / 2) % 16 == 0;
  const dim3 g((unsigned)blocks), b(256);
  if (aligned && group == 32)
    quantize_int4_reg_kernel<32><<<g, b, 0, stream>>>(a);
  else if (aligned && group == 64)
    quantize_int4_reg_kernel<64><<<g, b, 0, stream>>>(a);
  else if (aligned && group == 128)
    quantize_int4_reg_kernel<128><<<g, b, 0, stream>>>(a);
  else
    quantize_int4_kernel<<<g, b, 0, stream>>>(a);
  return smel::launch_status();
}
