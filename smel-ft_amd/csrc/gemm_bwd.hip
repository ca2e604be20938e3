// Grouped expert GEMM, backward (acc = A W per group, contraction over the weight's row dim): dA of the down
// projection (fused with the SiLU-gate backward, the d(combine weight) partials and the topv / shared-gate scaling)
// and dX of the gate_up projection. Frozen int4 experts are re-dequantized group by group; the int4 groups run along
// the output columns here, so each 64-row step of the weight is dequantized cooperatively into LDS, transposed to
// k-contiguous bf16 for the MFMA B operand. Reference: FrozenExpertsFn.backward, smel/moe.py:128-143, and the
// autograd of _selected_expert / lora_gate_up / lora_linear / the combine, smel/moe.py:204-252, smel/lora.py:61-83.
//
// Block = 4 waves, tile = up to 128 rows (4 slices of 32) x 256 columns (64 per wave). A rows staged in LDS (token
// gather fused for the down backward, which reads dout rows); W step [64][256] staged transposed in LDS.
#include "abi_util.h"
#include "common.h"

namespace {

constexpr int MT = 128;
constexpr int NT = 256;
constexpr int KT = 64;
constexpr int AS = KT + 8;   // A rows in LDS (bf16)
constexpr int BS = KT + 8;   // transposed W rows in LDS (bf16)

struct BwdArgs {
  smel_wset w;
  const int32_t* gkind;
  const int4* tiles;
  const int32_t* n_tiles;
  const uint16_t* A;
  int64_t lda;
  const int32_t* order;
  const uint16_t* ext;
  const uint16_t* hsave;
  const uint16_t* topv;
  const float* sgate;
  uint16_t* out;
  int64_t ldo;
  float* dwp;
  int a_gather, TK, topk, act;
  int Kd, N;   // Kd = w.R (contraction), N = w.C
};

// Stage W[k0 .. k0+63][n0 .. n0+255] of one group into Bt[n][k] (bf16, k contiguous). Thread -> (k pair, 32 cols).
template <bool Q4>
SMEL_DEV void stage_w(const BwdArgs& a, int kind, int idx, int k0, int n0, uint16_t* Bt) {
  const int tid = threadIdx.x;
  const int kp = tid & 31, c32 = tid >> 5;
  const int ka = k0 + 2 * kp;
  const int nc = n0 + 32 * c32;
  const smel_wset& w = a.w;
  uint32_t* dst = reinterpret_cast<uint32_t*>(Bt + (32 * c32) * BS + 2 * kp);
  const bool ok = ka + 1 < a.Kd && nc < a.N;   // Kd is a multiple of 32, so k pairs are whole
  if (Q4) {
    u32x4_t q0 = u32x4_t{}, q1 = u32x4_t{};
    float s0 = 0.f, z0 = 0.f, s1 = 0.f, z1 = 0.f;
    if (ok) {
      const int64_t r0 = (int64_t)idx * w.R + ka;
      q0 = *reinterpret_cast<const u32x4_t*>(w.q4 + r0 * (w.C / 2) + nc / 2);
      q1 = *reinterpret_cast<const u32x4_t*>(w.q4 + (r0 + 1) * (w.C / 2) + nc / 2);
      const int64_t g0 = r0 * (w.C / w.group) + nc / w.group;
      const int64_t g1 = (r0 + 1) * (w.C / w.group) + nc / w.group;
      s0 = bf2f(w.s4[g0]);
      z0 = bf2f(w.z4[g0]);
      s1 = bf2f(w.s4[g1]);
      z1 = bf2f(w.z4[g1]);
    }
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v0 = fmaf(nib(q0[wd], j), s0, z0);
        const float v1 = fmaf(nib(q1[wd], j), s1, z1);
        dst[(8 * wd + j) * (BS / 2)] = pack2bf(v0, v1);
      }
    }
  } else {
    const uint16_t* base = kind == SMEL_KIND_BF16 ? w.wb : (kind == SMEL_KIND_SEL ? w.wsel : w.wsh);
    const int64_t mi = kind == SMEL_KIND_SHARED ? 0 : idx;
    u32x4_t r0[4], r1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r0[i] = r1[i] = u32x4_t{};
    if (ok) {
      const uint16_t* p0 = base + (mi * w.R + ka) * w.C + nc;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        r0[i] = *reinterpret_cast<const u32x4_t*>(p0 + 8 * i);
        r1[i] = *reinterpret_cast<const u32x4_t*>(p0 + w.C + 8 * i);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t x0 = r0[i][j], x1 = r1[i][j];
        dst[(8 * i + 2 * j) * (BS / 2)] = (x0 & 0xffffu) | (x1 << 16);
        dst[(8 * i + 2 * j + 1) * (BS / 2)] = (x0 >> 16) | (x1 & 0xffff0000u);
      }
    }
  }
}

template <int EPI, bool Q4>
SMEL_DEV void run_tile(const BwdArgs& a, int kind, int idx, int row0, int nrows, uint16_t* As, uint16_t* Bt) {
  const int tid = threadIdx.x, l = lane_id(), w = tid >> 6, hi = l >> 5, r32 = l & 31;
  const int nb = blockIdx.y;
  const int n0 = nb * NT;
  const int Kd = a.Kd;
  const int cw = n0 + w * 64;                 // this wave's first column
  const bool fv0 = cw < a.N, fv1 = cw + 32 < a.N;
  const int ar = tid >> 1, ap = tid & 1;
  const uint16_t* arow = nullptr;
  if (ar < nrows) {
    const int grow = row0 + ar;
    const int src = a.a_gather ? row_token(grow, a.order, a.TK, a.topk) : grow;
    arow = a.A + (int64_t)src * a.lda;
  }
  const int nslice = (nrows + 31) >> 5;
  f32x16_t acc[4][2];
#pragma unroll
  for (int m = 0; m < 4; ++m) acc[m][0] = acc[m][1] = f32x16_t{};

  for (int k0 = 0; k0 < Kd; k0 += KT) {
    {
      const bool ok = arow && (k0 + 32 * ap + 32 <= Kd);
      uint16_t* dst = As + ar * AS + 32 * ap;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<u32x4_t*>(dst + 8 * i) =
            ok ? *reinterpret_cast<const u32x4_t*>(arow + k0 + 32 * ap + 8 * i) : u32x4_t{};
    }
    stage_w<Q4>(a, kind, idx, k0, n0, Bt);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4_t b0 = *reinterpret_cast<const u32x4_t*>(Bt + (w * 64 + r32) * BS + 32 * hi + 8 * s);
      const u32x4_t b1 = *reinterpret_cast<const u32x4_t*>(Bt + (w * 64 + 32 + r32) * BS + 32 * hi + 8 * s);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m < nslice) {
          const u32x4_t af = *reinterpret_cast<const u32x4_t*>(As + (m * 32 + r32) * AS + 32 * hi + 8 * s);
          if (fv0) acc[m][0] = mfma32(af, b0, acc[m][0]);
          if (fv1) acc[m][1] = mfma32(af, b1, acc[m][1]);
        }
      }
    }
    __syncthreads();
  }
  // ---- LoRA K-extension: ext[row][0:32] . Eb[0:32][n]
  const uint16_t* eb = kind == SMEL_KIND_SEL ? (a.w.ext_sel ? a.w.ext_sel + (int64_t)idx * 32 * a.N : nullptr)
                                               : (kind == SMEL_KIND_SHARED ? a.w.ext_sh : nullptr);
  if (a.ext && eb) {
    u32x4_t b0[2], b1[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      uint32_t v0[4] = {0, 0, 0, 0}, v1[4] = {0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = 16 * hi + 8 * s + 2 * j;
        if (fv0) {
          const uint16_t* p = eb + (int64_t)k * a.N + cw + r32;
          v0[j] = (uint32_t)p[0] | ((uint32_t)p[a.N] << 16);
        }
        if (fv1) {
          const uint16_t* p = eb + (int64_t)k * a.N + cw + 32 + r32;
          v1[j] = (uint32_t)p[0] | ((uint32_t)p[a.N] << 16);
        }
      }
      b0[s] = u32x4_t{v0[0], v0[1], v0[2], v0[3]};
      b1[s] = u32x4_t{v1[0], v1[1], v1[2], v1[3]};
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (m >= nslice) continue;
      const int row = m * 32 + r32;
      const uint16_t* er = a.ext + (int64_t)(row0 + row) * 32;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const u32x4_t af = row < nrows ? *reinterpret_cast<const u32x4_t*>(er + 16 * hi + 8 * s) : u32x4_t{};
        if (fv0) acc[m][0] = mfma32(af, b0[s], acc[m][0]);
        if (fv1) acc[m][1] = mfma32(af, b1[s], acc[m][1]);
      }
    }
  }
  // ---- epilogue
  if (EPI == 0) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (m >= nslice) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m * 32 + acc_row(r, l);
        if (row >= nrows) continue;
        const int64_t orow = (int64_t)row_slot(row0 + row, a.order, a.TK) * a.ldo;
        if (fv0) a.out[orow + cw + r32] = f2bf(acc[m][0][r]);
        if (fv1) a.out[orow + cw + 32 + r32] = f2bf(acc[m][1][r]);
      }
    }
    return;
  }
  // down backward: columns n < I of dh = [dg | du]
  float* red = reinterpret_cast<float*>(As);   // [4 waves][MT]
  const int I = a.N;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    if (m >= nslice) continue;   // block-uniform
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m * 32 + acc_row(r, l);
      const bool rv = row < nrows;
      const int grow = row0 + row;
      float wrow = 0.f;
      if (rv) wrow = grow < a.TK ? bf2f(a.topv[a.order[grow]]) : a.sgate[grow - a.TK];
      float part = 0.f;
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const bool fv = f == 0 ? fv0 : fv1;
        const int n = cw + 32 * f + r32;
        if (rv && fv) {
          const float g = bf2f(a.hsave[(int64_t)grow * 2 * I + n]);
          const float u = bf2f(a.hsave[(int64_t)grow * 2 * I + I + n]);
          float av, dav;
          act_and_grad_f(g, a.act, av, dav);
          const float abf = bf2f(f2bf(act_f(g, a.act) * u));   // the forward's rounded activation
          const float accv = acc[m][f][r];
          part += accv * abf;
          const float da = wrow * accv;
          a.out[(int64_t)grow * a.ldo + n] = f2bf(da * u * dav);
          a.out[(int64_t)grow * a.ldo + I + n] = f2bf(da * av);
        }
      }
      part = half_sum(part);
      if (r32 == 0) red[w * MT + row] = part;
    }
  }
  __syncthreads();
  if (tid < MT && tid < nrows) {
    const float v = ((red[tid] + red[MT + tid]) + red[2 * MT + tid]) + red[3 * MT + tid];
    a.dwp[(int64_t)(row0 + tid) * gridDim.y + nb] = v;
  }
}

template <int EPI>
__global__ __launch_bounds__(256) void gmm_bwd_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[MT * AS];
  __shared__ __attribute__((aligned(16))) uint16_t Bt[NT * BS];
  if ((int)blockIdx.x >= a.n_tiles[0]) return;
  const int4 t = a.tiles[blockIdx.x];
  const int gk = a.gkind[t.x];
  const int kind = gk >> 16, idx = gk & 0xffff;
  const int nrows = t.z - t.y;
  if (nrows <= 0) return;
  if (kind == SMEL_KIND_INT4)
    run_tile<EPI, true>(a, kind, idx, t.y, nrows, As, Bt);
  else
    run_tile<EPI, false>(a, kind, idx, t.y, nrows, As, Bt);
}

}  // namespace

extern "C" int64_t smel_gmm_bwd_nblocks(int64_t C) { return (C + NT - 1) / NT; }

extern "C" int smel_gmm_bwd(const smel_wset* w, const int32_t* gkind, const int32_t* tiles, const int32_t* n_tiles,
                            int64_t max_tiles, const uint16_t* A, int64_t lda, int32_t a_gather,
                            const int32_t* order, int64_t TK, int64_t topk, const uint16_t* ext, int32_t epilogue,
                            int32_t act, const uint16_t* hsave, const uint16_t* topv, const float* sgate,
                            uint16_t* out, int64_t ldo, float* dwp, hipStream_t stream) {
  SMEL_REQUIRE(w && gkind && tiles && n_tiles && A && out, SMEL_EINVAL, "gmm_bwd: null pointer");
  SMEL_REQUIRE(w->R > 0 && w->C > 0 && max_tiles >= 0 && lda >= w->R && topk > 0, SMEL_EINVAL,
               "gmm_bwd: bad sizes");
  SMEL_REQUIRE(w->R % 32 == 0 && w->C % 32 == 0, SMEL_EUNSUPPORTED,
               "gmm_bwd: weight dims %lldx%lld must be multiples of 32", (long long)w->R, (long long)w->C);
  SMEL_REQUIRE(!w->q4 || (w->group % 32 == 0 && w->C % w->group == 0), SMEL_EUNSUPPORTED,
               "gmm_bwd: int4 group %d must be a multiple of 32 dividing the columns", w->group);
  SMEL_REQUIRE(lda % 8 == 0 && ((uintptr_t)A % 16) == 0, SMEL_EUNSUPPORTED, "gmm_bwd: A rows must be 16-B aligned");
  SMEL_REQUIRE(epilogue == 0 || (epilogue == 1 && hsave && dwp && (topv || TK == 0)), SMEL_EINVAL,
               "gmm_bwd: epilogue %d needs hsave, dwp and topv", epilogue);
  SMEL_REQUIRE(!a_gather || order || TK == 0, SMEL_EINVAL, "gmm_bwd: gather needs order");
  if (max_tiles == 0) return 0;
  BwdArgs a;
  a.w = *w;
  a.gkind = gkind;
  a.tiles = reinterpret_cast<const int4*>(tiles);
  a.n_tiles = n_tiles;
  a.A = A;
  a.lda = lda;
  a.order = order;
  a.ext = ext;
  a.hsave = hsave;
  a.topv = topv;
  a.sgate = sgate;
  a.out = out;
  a.ldo = ldo;
  a.dwp = dwp;
  a.a_gather = a_gather;
  a.TK = (int)TK;
  a.topk = (int)topk;
  a.act = act;
  a.Kd = (int)w->R;
  a.N = (int)w->C;
  dim3 grid((unsigned)max_tiles, (unsigned)smel_gmm_bwd_nblocks(w->C));
  if (epilogue == 1)
    gmm_bwd_kernel<1><<<grid, 256, 0, stream>>>(a);
  else
    gmm_bwd_kernel<0><<<grid, 256, 0, stream>>>(a);
  return smel::launch_status();
}
