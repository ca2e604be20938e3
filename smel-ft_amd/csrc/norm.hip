// RMSNorm family of the frozen layers around the MoE block, for bf16 or fp16 rows, forward and backward:
//   rmsnorm        y = x rstd w'           w' = 1 + w, w or 1            (smel/norm.py:50-62, backward :64-82)
//   add_rmsnorm    s = h + x (rounded), y = rmsnorm(s)                    (smel/norm.py:84-100; backward is rmsnorm's
//                                                                          with the gradient of s's other use added)
//   gated_rmsnorm  y = w norm(x) silu(z)   (Gated DeltaNet output norm)   (smel/norm.py:102-145)
// fp32 math with the reference's rounding points (the 16-bit rounding of n and w n in the gated norm, of s in the
// residual add). Saved for backward: the input and one fp32 rstd per row.
//
// Layout: a row is split into 16-byte chunks of 8 elements and belongs to `lpr` threads of a 256-thread block (a
// power of two: fewer than 64 for short rows, so one wave holds several rows; one wave for up to 2048 elements; the
// whole block above that); thread i of a row takes chunks i, i + lpr, ...: each pass reads lpr * 16 contiguous
// bytes of the row. The whole row stays in registers as 16-bit values (CPL <= 8 chunks per thread), so every tensor
// is read once and written once. The row sum is a fixed xor-butterfly over the row's lanes, then (block rows) the
// four wave sums in wave order through LDS: deterministic, no atomics. HBM-bound.
#include "../../include/smel_norm.h"
#include "abi_util.h"
#include "common.h"

namespace {

enum { M_FWD = 0, M_ADD = 1, M_BWD = 2, M_GFWD = 3, M_GBWD = 4 };

// storage type: 0 = bf16, 1 = fp16
template <int DT>
SMEL_DEV float e2f(uint32_t b16) {
  if constexpr (DT == 0)
    return __uint_as_float(b16 << 16);
  else {   // volatile: converted where used, so the row stays packed in registers between the two passes
    float f;
    asm volatile("v_cvt_f32_f16 %0, %1" : "=v"(f) : "v"(b16));
    return f;
  }
}
template <int DT>
SMEL_DEV uint32_t f2e(float f) {
  if constexpr (DT == 0)
    return f2bf(f);
  else
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
template <int DT>
SMEL_DEV float rnd(float f) {
  return e2f<DT>(f2e<DT>(f));
}
template <int DT>
SMEL_DEV float elem(const u32x4_t& q, int j) {
  return e2f<DT>((j & 1) ? q[j >> 1] >> 16 : q[j >> 1] & 0xffffu);
}

struct NormArgs {
  const uint16_t* a;   // x (fwd, bwd, gated) or h (add); row stride a_stride
  const uint16_t* b;   // add: x, bwd: dy, gated fwd: z, gated bwd: dout
  const uint16_t* c;   // bwd: ds (may be null), gated bwd: z
  const uint16_t* w;   // weight [cols] (null with w_mode 0)
  const float* rstd_in;
  uint16_t* o0;        // fwd / gated fwd: y, add: s, bwd / gated bwd: dx
  uint16_t* o1;        // add: y, gated bwd: dz
  float* rstd_out;
  int64_t rows, a_stride;
  int cols, w_mode, lpr, vec;
  float eps;
};

// 8 elements starting at e0 (< cols); vec: 16-byte aligned with 8 in range, else element by element, zero past cols
SMEL_DEV u32x4_t load8(const uint16_t* __restrict__ p, int e0, int cols, int vec) {
  if (vec) return *reinterpret_cast<const u32x4_t*>(p + e0);
  uint32_t h[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = e0 + j < cols ? p[e0 + j] : 0u;
  return u32x4_t{h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16};
}
SMEL_DEV void store8(uint16_t* __restrict__ p, int e0, int cols, int vec, const uint32_t v[8]) {
  if (vec) {
    *reinterpret_cast<u32x4_t*>(p + e0) = u32x4_t{v[0] | v[1] << 16, v[2] | v[3] << 16, v[4] | v[5] << 16,
                                                  v[6] | v[7] << 16};
    return;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (e0 + j < cols) p[e0 + j] = (uint16_t)v[j];
}

template <int DT>
SMEL_DEV void weff8(const NormArgs& p, int e0, float w[8]) {
  if (p.w_mode == 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = 1.f;
    return;
  }
  const u32x4_t q = load8(p.w, e0, p.cols, p.vec);
#pragma unroll
  for (int j = 0; j < 8; ++j) w[j] = p.w_mode == 2 ? 1.f + elem<DT>(q, j) : elem<DT>(q, j);
}

// exp on the hardware's exp2 and the division on its reciprocal (no range-reduction branches per element)
SMEL_DEV float sigmoid_f(float z) { return __builtin_amdgcn_rcpf(1.f + exp_fast(-z)); }

// sum over the lpr threads of a row (every thread of the block calls it; lpr is uniform)
SMEL_DEV float row_sum(float v, int lpr, float* red) {
  for (int o = 1; o < lpr && o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  if (lpr > 64) {
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = ((red[0] + red[1]) + red[2]) + red[3];
  }
  return v;
}

template <int MODE, int DT, int CPL>
__global__ __launch_bounds__(256) void norm_kernel(NormArgs p) {
  __shared__ float red[4];
  const int lpr = p.lpr;
  const int64_t row = (int64_t)blockIdx.x * (256 / lpr) + threadIdx.x / lpr;
  const int li = threadIdx.x & (lpr - 1);
  const bool live = row < p.rows;
  const int n = p.cols, nch = (n + 7) >> 3;
  const uint16_t* const ra = p.a + (live ? row : 0) * p.a_stride;
  const int64_t ro = (live ? row : 0) * (int64_t)n;   // row offset of the contiguous tensors
  const bool two = MODE != M_FWD;
  const bool three = MODE == M_GBWD;
  u32x4_t A[CPL], B[CPL], C[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int ck = li + lpr * k;
    A[k] = B[k] = C[k] = u32x4_t{0, 0, 0, 0};
    if (live && ck < nch) {
      A[k] = load8(ra, 8 * ck, n, p.vec);
      if (two) B[k] = load8(p.b + ro, 8 * ck, n, p.vec);
      if (three) C[k] = load8(p.c + ro, 8 * ck, n, p.vec);
    }
  }
  float rstd;
  if constexpr (MODE == M_FWD || MODE == M_ADD || MODE == M_GFWD) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int ck = li + lpr * k;
      if constexpr (MODE == M_ADD) {   // s = h + x, rounded like the 16-bit residual stream; stored, then normed
        if (live && ck < nch) {
          uint32_t sv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) sv[j] = f2e<DT>(elem<DT>(A[k], j) + elem<DT>(B[k], j));
          store8(p.o0 + ro, 8 * ck, n, p.vec, sv);
          A[k] = u32x4_t{sv[0] | sv[1] << 16, sv[2] | sv[3] << 16, sv[4] | sv[5] << 16, sv[6] | sv[7] << 16};
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = elem<DT>(A[k], j);
        ss = fmaf(v, v, ss);
      }
    }
    ss = row_sum(ss, lpr, red);
    rstd = 1.f / sqrtf(ss / (float)n + p.eps);
    if (live && li == 0) p.rstd_out[row] = rstd;
  } else {
    rstd = live ? p.rstd_in[row] : 0.f;
  }

  if constexpr (MODE == M_FWD || MODE == M_ADD || MODE == M_GFWD) {
    uint16_t* const out = (MODE == M_ADD ? p.o1 : p.o0) + ro;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int ck = li + lpr * k;
      if (!(live && ck < nch)) continue;
      float w[8];
      weff8<DT>(p, 8 * ck, w);
      uint32_t y[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float x = elem<DT>(A[k], j);
        if constexpr (MODE == M_GFWD) {
          const float z = elem<DT>(B[k], j);
          const float yv = rnd<DT>(w[j] * rnd<DT>(x * rstd));
          y[j] = f2e<DT>(yv * (z * sigmoid_f(z)));
        } else {
          y[j] = f2e<DT>(x * rstd * w[j]);
        }
      }
      store8(out, 8 * ck, n, p.vec, y);
    }
    return;
  }

  // backward: dx = rstd (g - xhat mean(g xhat)), g = dy w' (plain) or the gradient of the rounded n (gated)
  if constexpr (MODE == M_BWD || MODE == M_GBWD) {
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int ck = li + lpr * k;
      if (!(live && ck < nch)) continue;
      float w[8];
      weff8<DT>(p, 8 * ck, w);
      uint32_t dz[8], dnv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float xhat = elem<DT>(A[k], j) * rstd;
        const float d = elem<DT>(B[k], j);
        float g;
        if constexpr (MODE == M_GBWD) {
          const float z = elem<DT>(C[k], j);
          const float yv = rnd<DT>(w[j] * rnd<DT>(xhat));
          const float sg = sigmoid_f(z);
          dz[j] = f2e<DT>(d * yv * (sg * (1.f + z * (1.f - sg))));
          dnv[j] = f2e<DT>(rnd<DT>(d * (z * sg)) * w[j]);
          g = e2f<DT>(dnv[j]);
        } else {
          g = d * w[j];
        }
        dot = fmaf(g, xhat, dot);
      }
      if constexpr (MODE == M_GBWD) {   // dn is a 16-bit value: it replaces z in the row's registers
        store8(p.o1 + ro, 8 * ck, n, p.vec, dz);
        C[k] = u32x4_t{dnv[0] | dnv[1] << 16, dnv[2] | dnv[3] << 16, dnv[4] | dnv[5] << 16, dnv[6] | dnv[7] << 16};
      }
    }
    dot = row_sum(dot, lpr, red);
    const float cm = dot / (float)n;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int ck = li + lpr * k;
      if (!(live && ck < nch)) continue;
      float w[8];
      if (MODE == M_BWD) weff8<DT>(p, 8 * ck, w);
      u32x4_t ds = u32x4_t{0, 0, 0, 0};
      if (MODE == M_BWD && p.c) ds = load8(p.c + ro, 8 * ck, n, p.vec);
      uint32_t dx[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float xhat = elem<DT>(A[k], j) * rstd;
        const float g = MODE == M_GBWD ? elem<DT>(C[k], j) : elem<DT>(B[k], j) * w[j];
        float v = rstd * (g - xhat * cm);
        if (MODE == M_BWD && p.c) v += elem<DT>(ds, j);
        dx[j] = f2e<DT>(v);
      }
      store8(p.o0 + ro, 8 * ck, n, p.vec, dx);
    }
  }
}

constexpr int MAX_COLS = 16384;

bool aligned16(const void* q) { return ((uintptr_t)q & 15) == 0; }

template <int MODE, int DT>
int launch_dt(NormArgs& p, hipStream_t stream) {
  const int nch = (p.cols + 7) / 8;   // <= 2048
  int cpl = 1;
  p.lpr = 1;
  while (p.lpr < nch && p.lpr < 64) p.lpr *= 2;
  if (nch > 4 * 64) p.lpr = 256;
  // forward passes of short rows (head dims): two chunks per thread (measured 2-7% faster; the backward, which
  // holds two or three tensors per chunk, is faster with one)
  if ((MODE == M_FWD || MODE == M_ADD || MODE == M_GFWD) && p.lpr >= 16 && nch <= 64) p.lpr /= 2;
  while (cpl * p.lpr < nch) cpl *= 2;
  const int64_t rows_per_block = 256 / p.lpr;
  const int64_t blocks = (p.rows + rows_per_block - 1) / rows_per_block;
  SMEL_REQUIRE(blocks < (int64_t)1 << 31, SMEL_EUNSUPPORTED, "rmsnorm: %lld rows is too many", (long long)p.rows);
  if (blocks == 0) return 0;
  const dim3 g((unsigned)blocks), b(256);
  switch (cpl) {
    case 1: norm_kernel<MODE, DT, 1><<<g, b, 0, stream>>>(p); break;
    case 2: norm_kernel<MODE, DT, 2><<<g, b, 0, stream>>>(p); break;
    case 4: norm_kernel<MODE, DT, 4><<<g, b, 0, stream>>>(p); break;
    default: norm_kernel<MODE, DT, 8><<<g, b, 0, stream>>>(p); break;
  }
  return smel::launch_status();
}

// shared checks; vec = every tensor of the call allows 16-byte chunks
template <int MODE>
int launch(NormArgs& p, int dtype, const char* name, hipStream_t stream) {
  SMEL_REQUIRE(p.rows >= 0 && p.cols >= 1, SMEL_EINVAL, "%s: bad sizes rows=%lld cols=%d", name, (long long)p.rows,
               p.cols);
  SMEL_REQUIRE(p.cols <= MAX_COLS, SMEL_EUNSUPPORTED, "%s: %d columns, at most %d", name, p.cols, MAX_COLS);
  SMEL_REQUIRE(p.rows <= 1 || p.a_stride >= p.cols, SMEL_EINVAL, "%s: row stride %lld < cols %d", name,
               (long long)p.a_stride, p.cols);
  SMEL_REQUIRE(p.w_mode >= 0 && p.w_mode <= 2, SMEL_EINVAL, "%s: w_mode %d", name, p.w_mode);
  SMEL_REQUIRE(p.w_mode == 0 || p.w, SMEL_EINVAL, "%s: null weight with w_mode %d", name, p.w_mode);
  SMEL_REQUIRE(dtype == 0 || dtype == 1, SMEL_EINVAL, "%s: dtype %d (0 = bf16, 1 = fp16)", name, dtype);
  if (p.rows == 0) return 0;
  const void* ptrs[] = {p.a, p.b, p.c, p.w, p.o0, p.o1};
  bool vec = p.cols % 8 == 0 && (p.rows <= 1 || p.a_stride % 8 == 0);
  for (const void* q : ptrs) vec = vec && aligned16(q);   // null pointers are aligned
  p.vec = vec;
  return dtype == 0 ? launch_dt<MODE, 0>(p, stream) : launch_dt<MODE, 1>(p, stream);
}

NormArgs blank(int64_t rows, int64_t cols, int64_t a_stride, const uint16_t* w, int w_mode, float eps) {
  NormArgs p{};
  p.rows = rows;
  p.cols = cols > MAX_COLS ? MAX_COLS + 1 : (int)cols;
  p.a_stride = a_stride;
  p.w = w;
  p.w_mode = w_mode;
  p.eps = eps;
  return p;
}

}  // namespace

extern "C" int smel_rmsnorm_fwd(const uint16_t* x, int64_t rows, int64_t cols, int64_t x_stride, const uint16_t* w,
                                int32_t w_mode, float eps, int32_t dtype, uint16_t* y, float* rstd,
                                hipStream_t stream) {
  NormArgs p = blank(rows, cols, x_stride, w, w_mode, eps);
  SMEL_REQUIRE(rows == 0 || (x && y && rstd), SMEL_EINVAL, "rmsnorm_fwd: null pointer");
  p.a = x;
  p.o0 = y;
  p.rstd_out = rstd;
  return launch<M_FWD>(p, dtype, "rmsnorm_fwd", stream);
}

extern "C" int smel_rmsnorm_bwd(const uint16_t* dy, const uint16_t* x, int64_t rows, int64_t cols, int64_t x_stride,
                                const uint16_t* w, int32_t w_mode, const float* rstd, const uint16_t* ds,
                                int32_t dtype, uint16_t* dx, hipStream_t stream) {
  NormArgs p = blank(rows, cols, x_stride, w, w_mode, 0.f);
  SMEL_REQUIRE(rows == 0 || (dy && x && rstd && dx), SMEL_EINVAL, "rmsnorm_bwd: null pointer");
  p.a = x;
  p.b = dy;
  p.c = ds;
  p.rstd_in = rstd;
  p.o0 = dx;
  return launch<M_BWD>(p, dtype, "rmsnorm_bwd", stream);
}

extern "C" int smel_add_rmsnorm_fwd(const uint16_t* h, const uint16_t* x, int64_t rows, int64_t cols,
                                    const uint16_t* w, int32_t w_mode, float eps, int32_t dtype, uint16_t* s,
                                    uint16_t* y, float* rstd, hipStream_t stream) {
  NormArgs p = blank(rows, cols, cols, w, w_mode, eps);
  SMEL_REQUIRE(rows == 0 || (h && x && s && y && rstd), SMEL_EINVAL, "add_rmsnorm_fwd: null pointer");
  p.a = h;
  p.b = x;
  p.o0 = s;
  p.o1 = y;
  p.rstd_out = rstd;
  return launch<M_ADD>(p, dtype, "add_rmsnorm_fwd", stream);
}

extern "C" int smel_gated_rmsnorm_fwd(const uint16_t* x, const uint16_t* z, int64_t rows, int64_t cols,
                                      const uint16_t* w, float eps, int32_t dtype, uint16_t* y, float* rstd,
                                      hipStream_t stream) {
  NormArgs p = blank(rows, cols, cols, w, 1, eps);
  SMEL_REQUIRE(rows == 0 || (x && z && w && y && rstd), SMEL_EINVAL, "gated_rmsnorm_fwd: null pointer");
  p.a = x;
  p.b = z;
  p.o0 = y;
  p.rstd_out = rstd;
  return launch<M_GFWD>(p, dtype, "gated_rmsnorm_fwd", stream);
}

extern "C" int smel_gated_rmsnorm_bwd(const uint16_t* dout, const uint16_t* x, const uint16_t* z, int64_t rows,
                                      int64_t cols, const uint16_t* w, const float* rstd, int32_t dtype, uint16_t* dx,
                                      uint16_t* dz, hipStream_t stream) {
  NormArgs p = blank(rows, cols, cols, w, 1, 0.f);
  SMEL_REQUIRE(rows == 0 || (dout && x && z && w && rstd && dx && dz), SMEL_EINVAL,
               "gated_rmsnorm_bwd: null pointer");
  p.a = x;
  p.b = dout;
  p.c = z;
  p.rstd_in = rstd;
  p.o0 = dx;
  p.o1 = dz;
  return launch<M_GBWD>(p, dtype, "gated_rmsnorm_bwd", stream);
}
