// Grouped expert GEMM, backward (acc = A W per group, contraction over the weight's row dim): dA of the down
// projection (fused with the SiLU-gate backward, the d(combine weight) partials and the topv / shared-gate scaling)
// and dX of the gate_up projection. Frozen int4 experts are re-dequantized group by group; the int4 groups run along
// the output columns here, so each 64-row step of the weight is dequantized cooperatively into LDS, transposed to
// k-contiguous bf16 for the MFMA B operand. Reference: FrozenExpertsFn.backward, smel/moe.py:128-143, and the
// autograd of _selected_expert / lora_gate_up / lora_linear / the combine, smel/moe.py:204-252, smel/lora.py:61-83.
//
// Block = 4 waves, tile = up to 128 rows (4 slices of 32) x 256 columns (64 per wave). Per 64-row step of W: the raw
// A rows and raw W rows of the next step are loaded into registers while the current step's MFMAs run; then A is
// written to LDS and W is dequantized (int4) and written transposed: thread (k pair, 32 columns) packs W[k][n] and
// W[k+1][n] into one 32-bit LDS word of row n, so a wave's stores cover 32 consecutive words of a row.
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
  int64_t a_rows;
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
  int nblk;    // column blocks per tile
};

// Raw W data of one thread for one step: rows (ka, ka+1), 32 columns.
template <bool Q4>
struct WRegs;
template <>
struct WRegs<true> {
  u32x4_t q[2];
  uint32_t s[2], z[2];
};
template <>
struct WRegs<false> {
  u32x4_t v[2][4];
};

template <int EPI, bool Q4, int NS>
SMEL_DEV void run_tile(const BwdArgs& a, int kind, int idx, int row0, int nrows, int nb, uint16_t* As,
                       uint16_t* Bt) {
  const int tid = threadIdx.x, l = lane_id(), w = tid >> 6, hi = l >> 5, r32 = l & 31;
  const int n0 = nb * NT;
  const int Kd = a.Kd;
  const smel_wset& ws = a.w;
  const int cw = n0 + w * 64;                 // this wave's first column
  const bool fv0 = cw < a.N, fv1 = cw + 32 < a.N;
  // ---- staging roles: A (tile row, 32-wide half), W (k pair, 32 columns)
  const int ar = tid >> 1, ap = tid & 1;
  const int kp = tid & 31, c32 = tid >> 5;
  const int nc = n0 + 32 * c32;
  const rsrc_t ra = make_rsrc(a.A, (uint64_t)a.a_rows * a.lda * 2);
  uint32_t aoff = OOB;
  if (ar < nrows) {
    const int grow = row0 + ar;
    const int src = a.a_gather ? row_token(grow, a.order, a.TK, a.topk) : grow;
    aoff = (uint32_t)src * (uint32_t)a.lda * 2 + 64 * ap;
  }
  // W rows (ka, ka+1) = lanes (i, i+1) of fragment ka / 32 in the packed layout; columns [nc, nc+32) = half h of
  // k-step ks of that layout.
  const int pk = (a.N + 63) / 64, pk4 = (pk + 3) / 4, nfr = Kd / 32;   // k-steps of the packed layout (along C)
  const int cks = nc / 64, ch = (nc / 32) & 1;
  const bool cok = nc < a.N;
  rsrc_t rw, rsz;
  uint32_t wbase, sbase = 0;   // byte offset of this thread's first chunk at k0 = 0
  if constexpr (Q4) {
    rw = make_rsrc(ws.q4 + (int64_t)idx * nfr * pk * 1024, (uint64_t)nfr * pk * 1024);
    rsz = make_rsrc(ws.sz4 + (int64_t)idx * nfr * pk4 * 256, (uint64_t)nfr * pk4 * 1024);
    wbase = (uint32_t)((cks * 64 + 32 * ch + (2 * kp) % 32) * 16);
    sbase = (uint32_t)(((cks >> 2) * 64 + 32 * ch + (2 * kp) % 32) * 16 + 4 * (cks & 3));
  } else {
    const uint16_t* base = kind == SMEL_KIND_BF16 ? ws.wb : (kind == SMEL_KIND_SEL ? ws.wsel : ws.wsh);
    const int64_t mi = kind == SMEL_KIND_SHARED ? 0 : idx;
    rw = make_rsrc(base + mi * nfr * pk * 2048, (uint64_t)nfr * pk * 4096);
    rsz = rw;
    wbase = (uint32_t)((cks * 4 * 64 + 32 * ch + (2 * kp) % 32) * 16);
  }

  f32x16_t acc[NS][2];
#pragma unroll
  for (int m = 0; m < NS; ++m) acc[m][0] = acc[m][1] = f32x16_t{};

  u32x4_t areg[4];
  WRegs<Q4> wr;
  auto load_step = [&](int k0) {
    const uint32_t ao = (k0 + 32 * ap + 32 <= Kd) ? aoff + k0 * 2 : OOB;
#pragma unroll
    for (int i = 0; i < 4; ++i) areg[i] = ld16(ra, ao + 16 * i);
    const int ka = k0 + 2 * kp;
    const bool ok = cok && ka + 1 < Kd;
    const int fr = ka / 32;
    if constexpr (Q4) {
      const uint32_t o = (uint32_t)fr * pk * 1024 + wbase;
      wr.q[0] = ld16(rw, ok ? o : OOB);
      wr.q[1] = ld16(rw, ok ? o + 16 : OOB);
      const uint32_t so = (uint32_t)fr * pk4 * 1024 + sbase;
      const uint32_t p0 = ld4(rsz, ok ? so : OOB), p1 = ld4(rsz, ok ? so + 16 : OOB);
      wr.s[0] = p0 & 0xffffu;
      wr.z[0] = p0 >> 16;
      wr.s[1] = p1 & 0xffffu;
      wr.z[1] = p1 >> 16;
    } else {
      const uint32_t o = (uint32_t)fr * pk * 4096 + wbase;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wr.v[0][i] = ld16(rw, ok ? o + 1024 * i : OOB);
        wr.v[1][i] = ld16(rw, ok ? o + 1024 * i + 16 : OOB);
      }
    }
  };
  auto store_step = [&]() {
    uint16_t* adst = As + ar * AS + 32 * ap;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4_t*>(adst + 8 * i) = areg[i];
    uint32_t* dst = reinterpret_cast<uint32_t*>(Bt + (32 * c32) * BS + 2 * kp);
    if constexpr (Q4) {
      const float s0 = bf2f(wr.s[0]), z0 = bf2f(wr.z[0]), s1 = bf2f(wr.s[1]), z1 = bf2f(wr.z[1]);
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        const uint32_t l0 = wr.q[0][wd] & 0x0f0f0f0fu, h0 = (wr.q[0][wd] >> 4) & 0x0f0f0f0fu;
        const uint32_t l1 = wr.q[1][wd] & 0x0f0f0f0fu, h1 = (wr.q[1][wd] >> 4) & 0x0f0f0f0fu;
        uint32_t* d = dst + (8 * wd) * (BS / 2);
        d[0 * (BS / 2)] = pack2bf(fmaf(ub0(l0), s0, z0), fmaf(ub0(l1), s1, z1));
        d[1 * (BS / 2)] = pack2bf(fmaf(ub0(h0), s0, z0), fmaf(ub0(h1), s1, z1));
        d[2 * (BS / 2)] = pack2bf(fmaf(ub1(l0), s0, z0), fmaf(ub1(l1), s1, z1));
        d[3 * (BS / 2)] = pack2bf(fmaf(ub1(h0), s0, z0), fmaf(ub1(h1), s1, z1));
        d[4 * (BS / 2)] = pack2bf(fmaf(ub2(l0), s0, z0), fmaf(ub2(l1), s1, z1));
        d[5 * (BS / 2)] = pack2bf(fmaf(ub2(h0), s0, z0), fmaf(ub2(h1), s1, z1));
        d[6 * (BS / 2)] = pack2bf(fmaf(ub3(l0), s0, z0), fmaf(ub3(l1), s1, z1));
        d[7 * (BS / 2)] = pack2bf(fmaf(ub3(h0), s0, z0), fmaf(ub3(h1), s1, z1));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t x0 = wr.v[0][i][j], x1 = wr.v[1][i][j];
          dst[(8 * i + 2 * j) * (BS / 2)] = __builtin_amdgcn_perm(x1, x0, 0x05040100u);
          dst[(8 * i + 2 * j + 1) * (BS / 2)] = __builtin_amdgcn_perm(x1, x0, 0x07060302u);
        }
      }
    }
  };

  const int nk = (Kd + KT - 1) / KT;
  load_step(0);
  const uint16_t* Ab = As + r32 * AS + 32 * hi;
  const uint16_t* Bb = Bt + (w * 64 + r32) * BS + 32 * hi;
  for (int i = 0; i < nk; ++i) {
    store_step();
    __syncthreads();
    if (i + 1 < nk) load_step((i + 1) * KT);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4_t b0 = *reinterpret_cast<const u32x4_t*>(Bb + 8 * s);
      const u32x4_t b1 = *reinterpret_cast<const u32x4_t*>(Bb + 32 * BS + 8 * s);
#pragma unroll
      for (int m = 0; m < NS; ++m) {
        const u32x4_t af = *reinterpret_cast<const u32x4_t*>(Ab + m * 32 * AS + 8 * s);
        acc[m][0] = mfma32(af, b0, acc[m][0]);
        acc[m][1] = mfma32(af, b1, acc[m][1]);
      }
    }
    __syncthreads();
  }
  // ---- LoRA K-extension: ext[row][0:32] . Eb[0:32][n]
  const uint16_t* eb = kind == SMEL_KIND_SEL ? (ws.ext_sel ? ws.ext_sel + (int64_t)idx * 32 * a.N : nullptr)
                                             : (kind == SMEL_KIND_SHARED ? ws.ext_sh : nullptr);
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
    const rsrc_t rx = make_rsrc(a.ext + (int64_t)row0 * 32, (uint64_t)nrows * 64);
#pragma unroll
    for (int m = 0; m < NS; ++m) {
      const int row = m * 32 + r32;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const u32x4_t af = ld16(rx, row < nrows ? (uint32_t)row * 64 + 32 * hi + 16 * s : OOB);
        acc[m][0] = mfma32(af, b0[s], acc[m][0]);
        acc[m][1] = mfma32(af, b1[s], acc[m][1]);
      }
    }
  }
  // ---- epilogue
  if (EPI == 0) {
#pragma unroll
    for (int m = 0; m < NS; ++m) {
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
  float* red = reinterpret_cast<float*>(As);   // [4 waves][MT]; As is free after the last barrier
  const int I = a.N;
#pragma unroll
  for (int m = 0; m < NS; ++m) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m * 32 + acc_row(r, l);
      const bool rv = row < nrows;
      const int grow = row0 + row;
      float wrow_ = 0.f;
      if (rv) wrow_ = grow < a.TK ? bf2f(a.topv[a.order[grow]]) : a.sgate[grow - a.TK];
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
          const float da = wrow_ * accv;
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
    a.dwp[(int64_t)(row0 + tid) * a.nblk + nb] = v;
  }
}

template <int EPI, bool Q4>
SMEL_DEV void run_tile_ns(const BwdArgs& a, int kind, int idx, int row0, int nrows, int nb, uint16_t* As,
                          uint16_t* Bt) {
  switch ((nrows + 31) >> 5) {
    case 1: run_tile<EPI, Q4, 1>(a, kind, idx, row0, nrows, nb, As, Bt); break;
    case 2: run_tile<EPI, Q4, 2>(a, kind, idx, row0, nrows, nb, As, Bt); break;
    case 3: run_tile<EPI, Q4, 3>(a, kind, idx, row0, nrows, nb, As, Bt); break;
    default: run_tile<EPI, Q4, 4>(a, kind, idx, row0, nrows, nb, As, Bt); break;
  }
}

template <int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gmm_bwd_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[MT * AS];
  __shared__ __attribute__((aligned(16))) uint16_t Bt[NT * BS];
  int tile, nb;
  if (!xcd_tile(a.n_tiles[0], a.nblk, tile, nb)) return;
  const int4 t = a.tiles[tile];
  const int gk = a.gkind[t.x];
  const int kind = gk >> 16, idx = gk & 0xffff;
  const int nrows = min(t.z - t.y, MT);
  if (nrows <= 0) return;
  if (kind == SMEL_KIND_INT4)
    run_tile_ns<EPI, true>(a, kind, idx, t.y, nrows, nb, As, Bt);
  else
    run_tile_ns<EPI, false>(a, kind, idx, t.y, nrows, nb, As, Bt);
}

}  // namespace

extern "C" int64_t smel_gmm_bwd_nblocks(int64_t C) { return (C + NT - 1) / NT; }

extern "C" int smel_gmm_bwd(const smel_wset* w, const int32_t* gkind, const int32_t* tiles, const int32_t* n_tiles,
                            int64_t max_tiles, const uint16_t* A, int64_t lda, int64_t a_rows, int32_t a_gather,
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
  SMEL_REQUIRE(!w->q4 || w->sz4, SMEL_EINVAL, "gmm_bwd: an int4 bank needs its packed scale/zero (smel_pack_int4)");
  SMEL_REQUIRE(lda % 8 == 0 && ((uintptr_t)A % 16) == 0, SMEL_EUNSUPPORTED, "gmm_bwd: A rows must be 16-B aligned");
  SMEL_REQUIRE(epilogue == 0 || (epilogue == 1 && hsave && dwp && (topv || TK == 0)), SMEL_EINVAL,
               "gmm_bwd: epilogue %d needs hsave, dwp and topv", epilogue);
  SMEL_REQUIRE(!a_gather || order || TK == 0, SMEL_EINVAL, "gmm_bwd: gather needs order");
  SMEL_REQUIRE(a_rows >= 0 && a_rows * lda * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "gmm_bwd: A larger than 2 GiB");
  SMEL_REQUIRE(w->R * w->C * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "gmm_bwd: one weight matrix larger than 2 GiB");
  if (max_tiles == 0) return 0;
  BwdArgs a;
  a.w = *w;
  a.gkind = gkind;
  a.tiles = reinterpret_cast<const int4*>(tiles);
  a.n_tiles = n_tiles;
  a.A = A;
  a.lda = lda;
  a.a_rows = a_rows;
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
  a.nblk = (int)smel_gmm_bwd_nblocks(w->C);
  const unsigned grid = (unsigned)(xcd_grid(max_tiles) * a.nblk);
  if (epilogue == 1)
    gmm_bwd_kernel<1><<<grid, 256, 0, stream>>>(a);
  else
    gmm_bwd_kernel<0><<<grid, 256, 0, stream>>>(a);
  return smel::launch_status();
}
