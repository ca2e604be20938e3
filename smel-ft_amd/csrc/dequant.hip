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

// ---- fragment layouts of the GEMM weight operands (one 1-KB block = what one wave loads with one 16-B load per
// lane; lane l = 32 h + i holds row 32 f + i of fragment f, k-half h of a 64-wide k-step):
//   int4 q : block (f, ks)       lane chunk = 32 nibbles, k = 64 ks + 32 h + [0, 32)
//   sz     : block (f, ks / 4)   lane chunk = 4 words (ks % 4 = 0..3): scale | zero << 16 of the group of 64 ks + 32 h
//   bf16   : block (f, ks, s)    lane chunk = 8 bf16, k = 64 ks + 32 h + 8 s + [0, 8)
// Rows >= rows and k >= K are zero.

__global__ __launch_bounds__(256) void pack_q4(const uint8_t* __restrict__ q, int64_t rows, int64_t K, int64_t nks,
                                               u32x4_t* __restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t lane = i & 63, blk = i >> 6;
    const int64_t f = blk / nks, ks = blk - f * nks;
    const int64_t r = 32 * f + (lane & 31), k = 64 * ks + 32 * (lane >> 5);
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (r < rows && k < K) v = *reinterpret_cast<const u32x4_t*>(q + r * (K / 2) + k / 2);
    out[i] = v;
  }
}

__global__ __launch_bounds__(256) void pack_sz(const uint16_t* __restrict__ s, const uint16_t* __restrict__ z,
                                               int64_t rows, int64_t K, int64_t group, int64_t nks4,
                                               u32x4_t* __restrict__ out, int64_t n) {
  const int64_t G = K / group;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t lane = i & 63, blk = i >> 6;
    const int64_t f = blk / nks4, run = blk - f * nks4;
    const int64_t r = 32 * f + (lane & 31);
    uint32_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t k = 64 * (4 * run + j) + 32 * (lane >> 5);
      v[j] = 0;
      if (r < rows && k < K) {
        const int64_t gi = r * G + k / group;
        v[j] = (uint32_t)s[gi] | ((uint32_t)z[gi] << 16);
      }
    }
    out[i] = u32x4_t{v[0], v[1], v[2], v[3]};
  }
}

__global__ __launch_bounds__(256) void pack_bf16(const uint16_t* __restrict__ w, int64_t rows, int64_t K, int64_t ld,
                                                 int64_t nks, u32x4_t* __restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t lane = i & 63, blk = i >> 6;
    const int64_t sub = blk & 3, fk = blk >> 2;
    const int64_t f = fk / nks, ks = fk - f * nks;
    const int64_t r = 32 * f + (lane & 31), k = 64 * ks + 32 * (lane >> 5) + 8 * sub;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (r < rows && k < K) v = *reinterpret_cast<const u32x4_t*>(w + r * ld + k);
    out[i] = v;
  }
}

// ---- transposed fragment layouts (the backward GEMM's weight operand: contraction over the matrix's rows R, output
// columns C; v_mfma_f32_16x16x32_bf16 with lane l = 16 kq + i holding column i of a 16-column fragment and, in
// substep s of a 64-row step, rows k = 32 s + 8 kq + [0, 8)):
//   int4 q : block (e, p, ks) = 1 KB, column pair p = 32 columns; lane chunk = 4 words, word (2 fr + s) = the 8
//            nibbles (row order, low nibble first) of column 32 p + 16 fr + i at rows 64 ks + 32 s + 8 kq + [0, 8)
//   sz     : block (e, g, ks) = 512 B, group g of C; fp32 pair 16 kq + 8 s + t = (scale, zero') of row
//            64 ks + 32 s + 8 kq + t (a lane reads the 64 B of its kq and substep); zero' = zero - 1024 scale for a
//            fast bank (the constant of the fp16-magic dequant, exact by smel_int4_fast_ok), else zero. fp32 here
//            because these values change along the contraction, so each lane needs eight pairs per substep: stored
//            ready to use, they cost no unpacking
//   bf16   : block (e, p, ks, 2 fr + s) = 1 KB; lane chunk = the 8 bf16 of column 32 p + 16 fr + i at those rows
// Rows >= R and columns >= C are zero.

__global__ __launch_bounds__(256) void pack_q4_t(const uint8_t* __restrict__ q, int64_t R, int64_t C, int64_t np,
                                                 int64_t nks, u32x4_t* __restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t lane = i & 63, blk = i >> 6;
    const int64_t ks = blk % nks, ep = blk / nks;
    const int64_t p = ep % np, e = ep / np;
    const int kq = (int)(lane >> 4), li = (int)(lane & 15);
    uint32_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int fr = j >> 1, sub = j & 1;
      const int64_t col = 32 * p + 16 * fr + li;
      const int64_t k0 = 64 * ks + 32 * sub + 8 * kq;
      uint32_t word = 0;
      if (col < C) {
        for (int t = 0; t < 8; ++t) {
          const int64_t k = k0 + t;
          if (k < R) {
            const uint32_t b = q[(e * R + k) * (C / 2) + col / 2];
            word |= ((col & 1) ? (b >> 4) : (b & 15u)) << (4 * t);
          }
        }
      }
      v[j] = word;
    }
    out[i] = u32x4_t{v[0], v[1], v[2], v[3]};
  }
}

__global__ __launch_bounds__(256) void pack_sz_t(const uint16_t* __restrict__ s, const uint16_t* __restrict__ z,
                                                 int64_t R, int64_t G, int64_t nks, int fast, float2* __restrict__ out,
                                                 int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t pos = i & 63, blk = i >> 6;
    const int64_t ks = blk % nks, eg = blk / nks;
    const int64_t g = eg % G, e = eg / G;
    const int64_t kq = pos >> 4, sub = (pos >> 3) & 1, t = pos & 7;
    const int64_t k = 64 * ks + 32 * sub + 8 * kq + t;
    float2 v = make_float2(0.f, 0.f);
    if (k < R) {
      const int64_t gi = (e * R + k) * G + g;
      const float sc = bf2f(s[gi]), ze = bf2f(z[gi]);
      // fast: the backward reads rows t = 0, 2, 4, 6 of a word as fp16 1024 + q and rows 1, 3, 5, 7 as 1024 + 16 q
      // (a nibble in bits 4..7 needs no shift): (s, z - 1024 s), resp. (s / 16, z - 64 s)
      if (!fast)
        v = make_float2(sc, ze);
      else if (t & 1)
        v = make_float2(sc * 0.0625f, fmaf(-64.f, sc, ze));
      else
        v = make_float2(sc, fmaf(-1024.f, sc, ze));
    }
    out[i] = v;
  }
}

// fp32 value d, exactly: a normal or zero fp32?
SMEL_DEV bool f32_exact(double d) {
  const float f = (float)d;
  return (double)f == d && (d == 0.0 || (fabs(d) >= 1.1754943508222875e-38 && fabs(d) <= 3.4028234663852886e38));
}
// z - m exactly an fp32 (z, m bf16 values, m possibly scaled by a power of two): with exponents at most 40 apart the
// difference (at most 49 significant bits) is exact in double, so the fp32 round trip decides; further apart, the
// exact difference needs more than 24 bits unless one side is zero.
SMEL_DEV bool diff_exact(double z, double m) {
  if (z == 0.0 || m == 0.0) return f32_exact(z - m);
  if (abs(ilogb(z) - ilogb(m)) > 40) return false;
  return f32_exact(z - m);
}
__global__ __launch_bounds__(256) void fast_ok_init(int32_t* ok) { *ok = 1; }
__global__ __launch_bounds__(256) void fast_ok_check(const uint16_t* __restrict__ s, const uint16_t* __restrict__ z,
                                                     int64_t n, int32_t* ok) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const double sc = bf2f(s[i]), ze = bf2f(z[i]);
    const bool good = f32_exact(sc) && f32_exact(sc / 16.0) && diff_exact(ze, 1024.0 * sc) &&
                      diff_exact(ze, 64.0 * sc) && f32_exact(1024.0 * sc);
    if (!good) *ok = 0;   // every writer stores the same value
  }
}

__global__ __launch_bounds__(256) void pack_bf16_t(const uint16_t* __restrict__ w, int64_t R, int64_t C, int64_t ld,
                                                   int64_t np, int64_t nks, u32x4_t* __restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t lane = i & 63, blk = i >> 6;
    const int j = (int)(blk & 3);
    const int64_t pk = blk >> 2;
    const int64_t ks = pk % nks, ep = pk / nks;
    const int64_t p = ep % np, e = ep / np;
    const int fr = j >> 1, sub = j & 1;
    const int kq = (int)(lane >> 4), li = (int)(lane & 15);
    const int64_t col = 32 * p + 16 * fr + li;
    const int64_t k0 = 64 * ks + 32 * sub + 8 * kq;
    uint32_t v[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t lo = 0, hi = 0;
      if (col < C && k0 + 2 * t < R) lo = w[(e * R + k0 + 2 * t) * ld + col];
      if (col < C && k0 + 2 * t + 1 < R) hi = w[(e * R + k0 + 2 * t + 1) * ld + col];
      v[t] = lo | (hi << 16);
    }
    out[i] = u32x4_t{v[0], v[1], v[2], v[3]};
  }
}

inline int pack_blocks(int64_t n) { return (int)std::min<int64_t>((n + 255) / 256, 256 * 64); }

}  // namespace

extern "C" int64_t smel_packed_bytes(int32_t what, int64_t rows, int64_t K) {
  if (rows < 0 || K <= 0) return -1;
  const int64_t nf = (rows + 31) / 32, nks = (K + 63) / 64;
  switch (what) {
    case SMEL_PACK_Q4: return nf * nks * 1024;
    case SMEL_PACK_SZ: return nf * ((nks + 3) / 4) * 1024;
    case SMEL_PACK_BF16: return nf * nks * 4096;
    default: return -1;
  }
}

extern "C" int64_t smel_packed_t_bytes(int32_t what, int64_t n_mats, int64_t R, int64_t C, int64_t group) {
  if (n_mats < 0 || R <= 0 || C <= 0) return -1;
  const int64_t np = (C + 31) / 32, nks = (R + 63) / 64;
  switch (what) {
    case SMEL_PACK_Q4: return n_mats * np * nks * 1024;
    case SMEL_PACK_SZ: return (group > 0 && C % group == 0) ? n_mats * (C / group) * nks * 512 : -1;
    case SMEL_PACK_BF16: return n_mats * np * nks * 4096;
    default: return -1;
  }
}

extern "C" int smel_pack_int4_t(const uint8_t* q, const uint16_t* scale, const uint16_t* zero, int64_t n_mats,
                                int64_t R, int64_t C, int64_t group, int32_t fast, uint8_t* qt, float* szt,
                                hipStream_t stream) {
  SMEL_REQUIRE(n_mats >= 0 && R > 0 && C > 0 && group > 0 && C % 32 == 0 && C % group == 0 && group % 32 == 0,
               SMEL_EUNSUPPORTED, "pack_int4_t: C=%lld, group=%lld (C a multiple of 32, group a multiple of 32 "
               "dividing C)", (long long)C, (long long)group);
  if (n_mats == 0) return 0;
  SMEL_REQUIRE(q && scale && zero && qt && szt, SMEL_EINVAL, "pack_int4_t: null pointer");
  SMEL_REQUIRE((uintptr_t)qt % 16 == 0 && (uintptr_t)szt % 8 == 0, SMEL_EUNSUPPORTED,
               "pack_int4_t: qt must be 16-byte and szt 8-byte aligned");
  SMEL_REQUIRE(fast == 0 || fast == 1, SMEL_EINVAL, "pack_int4_t: fast %d", fast);
  const int64_t np = C / 32, nks = (R + 63) / 64, G = C / group;
  const int64_t nq = n_mats * np * nks * 64, nsz = n_mats * G * nks * 64;
  pack_q4_t<<<pack_blocks(nq), 256, 0, stream>>>(q, R, C, np, nks, reinterpret_cast<u32x4_t*>(qt), nq);
  pack_sz_t<<<pack_blocks(nsz), 256, 0, stream>>>(scale, zero, R, G, nks, fast, reinterpret_cast<float2*>(szt), nsz);
  return smel::launch_status();
}

extern "C" int smel_int4_fast_ok(const uint16_t* scale, const uint16_t* zero, int64_t n, int32_t* ok,
                                 hipStream_t stream) {
  SMEL_REQUIRE(n >= 0 && ok && (n == 0 || (scale && zero)), SMEL_EINVAL, "int4_fast_ok: null pointer or n < 0");
  fast_ok_init<<<1, 1, 0, stream>>>(ok);
  int st = smel::launch_status();
  if (st || n == 0) return st;
  fast_ok_check<<<pack_blocks(n), 256, 0, stream>>>(scale, zero, n, ok);
  return smel::launch_status();
}

extern "C" int smel_pack_bf16_t(const uint16_t* w, int64_t n_mats, int64_t R, int64_t C, int64_t ld, uint16_t* wt,
                                hipStream_t stream) {
  SMEL_REQUIRE(n_mats >= 0 && R > 0 && C > 0 && C % 32 == 0 && ld >= C, SMEL_EUNSUPPORTED,
               "pack_bf16_t: C=%lld, ld=%lld (C a multiple of 32, ld >= C)", (long long)C, (long long)ld);
  if (n_mats == 0) return 0;
  SMEL_REQUIRE(w && wt, SMEL_EINVAL, "pack_bf16_t: null pointer");
  SMEL_REQUIRE((uintptr_t)wt % 16 == 0, SMEL_EUNSUPPORTED, "pack_bf16_t: wt must be 16-byte aligned");
  const int64_t np = C / 32, nks = (R + 63) / 64;
  const int64_t n = n_mats * np * nks * 4 * 64;
  pack_bf16_t<<<pack_blocks(n), 256, 0, stream>>>(w, R, C, ld, np, nks, reinterpret_cast<u32x4_t*>(wt), n);
  return smel::launch_status();
}

extern "C" int smel_pack_int4(const uint8_t* q, const uint16_t* scale, const uint16_t* zero, int64_t rows, int64_t K,
                              int64_t group, uint8_t* qf, uint32_t* szf, hipStream_t stream) {
  SMEL_REQUIRE(rows >= 0 && K > 0 && group > 0 && K % 32 == 0 && K % group == 0 && group % 32 == 0,
               SMEL_EUNSUPPORTED, "pack_int4: K=%lld, group=%lld (K a multiple of 32, group a multiple of 32 dividing K)",
               (long long)K, (long long)group);
  if (rows == 0) return 0;
  SMEL_REQUIRE(q && scale && zero && qf && szf, SMEL_EINVAL, "pack_int4: null pointer");
  SMEL_REQUIRE((uintptr_t)q % 16 == 0 && (uintptr_t)qf % 16 == 0 && (uintptr_t)szf % 16 == 0, SMEL_EUNSUPPORTED,
               "pack_int4: q, qf and szf must be 16-byte aligned");
  const int64_t nf = (rows + 31) / 32, nks = (K + 63) / 64, nks4 = (nks + 3) / 4;
  const int64_t nq = nf * nks * 64, nsz = nf * nks4 * 64;
  pack_q4<<<pack_blocks(nq), 256, 0, stream>>>(q, rows, K, nks, reinterpret_cast<u32x4_t*>(qf), nq);
  pack_sz<<<pack_blocks(nsz), 256, 0, stream>>>(scale, zero, rows, K, group, nks4, reinterpret_cast<u32x4_t*>(szf),
                                                nsz);
  return smel::launch_status();
}

extern "C" int smel_pack_bf16(const uint16_t* w, int64_t rows, int64_t K, int64_t ld, uint16_t* wf,
                              hipStream_t stream) {
  SMEL_REQUIRE(rows >= 0 && K > 0 && K % 8 == 0 && ld >= K && ld % 8 == 0, SMEL_EUNSUPPORTED,
               "pack_bf16: K=%lld, ld=%lld (K and ld multiples of 8, ld >= K)", (long long)K, (long long)ld);
  if (rows == 0) return 0;
  SMEL_REQUIRE(w && wf, SMEL_EINVAL, "pack_bf16: null pointer");
  SMEL_REQUIRE((uintptr_t)w % 16 == 0 && (uintptr_t)wf % 16 == 0, SMEL_EUNSUPPORTED,
               "pack_bf16: w and wf must be 16-byte aligned");
  const int64_t nf = (rows + 31) / 32, nks = (K + 63) / 64;
  const int64_t n = nf * nks * 4 * 64;
  pack_bf16<<<pack_blocks(n), 256, 0, stream>>>(w, rows, K, ld, nks, reinterpret_cast<u32x4_t*>(wf), n);
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
