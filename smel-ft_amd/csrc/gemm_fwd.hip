// Grouped expert GEMM, forward (out = A W^T per group): the gate_up and down projections of every expert, frozen
// (int4 group-64, dequantized in registers inside the main loop — no bf16 copy of a frozen expert is ever written)
// or selected / shared (bf16 + LoRA as a 32-wide K-extension), with the token gather fused into the A load and the
// SiLU-gate fused into the gate_up epilogue.
// Reference: frozen_experts_forward / _gmm / _selected_expert / lora_gate_up / lora_linear,
// smel/moe.py:58-72, 110-117, 204-211 and smel/lora.py:61-83.
//
// Block = 4 waves, tile = up to 128 rows of one group (4 slices of 32) x (gate_up: 32 gate + 32 up columns per wave;
// down: 64 columns per wave). A (activation rows) is staged through LDS, double-buffered, and shared by the 4 waves;
// every wave streams its own weight rows straight into registers (16 B of int4 = 32 k per lane per step) and
// dequantizes them there, so each weight element of a tile is read and dequantized once. MFMA 32x32x16 bf16.
// Lane k-mapping inside a 64-wide step: lane half h = lane/32 carries k = 32h + 8s + [0,8) in substep s, for A and
// B alike (one 16-B read per lane per operand).
#include "abi_util.h"
#include "common.h"

namespace {

constexpr int MT = 128;
constexpr int KT = 64;
constexpr int AS = KT + 8;   // LDS row stride in bf16 (144 B: an odd number of 16-B units)

struct FwdArgs {
  smel_wset w;
  const int32_t* gkind;
  const int4* tiles;
  const int32_t* n_tiles;
  const uint16_t* A;
  int64_t lda;
  int64_t a_rows;       // rows of A (bounds of the A buffer)
  const int32_t* order;
  const uint16_t* ext;
  uint16_t* out;
  int64_t ldo;
  uint16_t* hsave;
  int a_gather, TK, topk, act;
  int N, K;   // N = w.R (weight rows), K = w.C
  int nblk;   // column blocks per tile
};

// Weight rows of one wave for one k-step: int4 (16 B = 32 nibbles per lane and fragment, plus its group's scale and
// zero) or bf16 (64 B per lane and fragment).
template <bool Q4>
struct BRegs;
template <>
struct BRegs<true> {
  u32x4_t q[2];
  u32x4_t sz[2];   // packed (scale, zero) of 4 consecutive k-steps (the 4-aligned run holding this step)
};
template <>
struct BRegs<false> {
  u32x4_t v[2][4];
};

template <int EPI, bool Q4, int NS>
SMEL_DEV void run_tile(const FwdArgs& a, int kind, int idx, int row0, int nrows, int nb, uint16_t* As) {
  const int tid = threadIdx.x, l = lane_id(), w = tid >> 6, hi = l >> 5, r32 = l & 31;
  const int K = a.K;
  const smel_wset& ws = a.w;
  // ---- this wave's two weight rows (per lane): gate/up pair for epilogue 1, two adjacent 32-column blocks else
  int n0, n1;
  bool fv0, fv1;
  if (EPI == 1) {
    const int I = a.N / 2;
    const int c0 = nb * 128 + w * 32;
    fv0 = fv1 = c0 < I;
    n0 = c0 + r32;
    n1 = I + c0 + r32;
  } else {
    const int c0 = nb * 256 + w * 64;
    fv0 = c0 < a.N;
    fv1 = c0 + 32 < a.N;
    n0 = c0 + r32;
    n1 = c0 + 32 + r32;
  }
  // ---- buffer resources: the weight matrix of this group, the A matrix
  rsrc_t rw, rsz;
  uint32_t wo0, wo1, so0 = 0, so1 = 0;
  const int nks = (ws.C + 63) / 64;   // k-steps of one weight row (packed scale/zero entries per lane half)
  if constexpr (Q4) {
    const int64_t mat = (int64_t)idx * ws.R;
    rw = make_rsrc(ws.q4 + mat * (ws.C / 2), (uint64_t)ws.R * (ws.C / 2));
    rsz = make_rsrc(ws.sz4 + mat * 2 * nks, (uint64_t)ws.R * 2 * nks * 4);
    wo0 = fv0 ? (uint32_t)n0 * (ws.C / 2) : OOB;
    wo1 = fv1 ? (uint32_t)n1 * (ws.C / 2) : OOB;
    so0 = fv0 ? (uint32_t)(n0 * 2 + hi) * nks * 4 : OOB;
    so1 = fv1 ? (uint32_t)(n1 * 2 + hi) * nks * 4 : OOB;
  } else {
    const uint16_t* base = kind == SMEL_KIND_BF16 ? ws.wb : (kind == SMEL_KIND_SEL ? ws.wsel : ws.wsh);
    const int64_t mi = kind == SMEL_KIND_SHARED ? 0 : idx;
    rw = make_rsrc(base + mi * ws.R * ws.C, (uint64_t)ws.R * ws.C * 2);
    rsz = rw;
    wo0 = fv0 ? (uint32_t)n0 * ws.C * 2 : OOB;
    wo1 = fv1 ? (uint32_t)n1 * ws.C * 2 : OOB;
  }
  const rsrc_t ra = make_rsrc(a.A, (uint64_t)a.a_rows * a.lda * 2);
  // A staging: 8 consecutive lanes read one row's 128 contiguous bytes of the k-step (16 B each), so a 16-lane
  // quarter-wave touches 2 rows; thread t covers rows t/8 + 32 i, i = 0..3, at 16-byte chunk t%8.
  const int ach = tid & 7, arow0 = tid >> 3;
  uint32_t aoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ar = arow0 + 32 * i;
    aoff[i] = OOB;
    if (ar < nrows) {
      const int grow = row0 + ar;
      const int src = a.a_gather ? row_token(grow, a.order, a.TK, a.topk) : grow;
      aoff[i] = (uint32_t)src * (uint32_t)a.lda * 2 + 16 * ach;
    }
  }

  f32x16_t acc[NS][2];
#pragma unroll
  for (int m = 0; m < NS; ++m) acc[m][0] = acc[m][1] = f32x16_t{};

  u32x4_t areg[4];
  BRegs<Q4> bc, bn;
  auto load_a = [&](int k0) {
    const bool ok = k0 + 8 * ach + 8 <= K;   // K % 32 == 0: a 16-B chunk is all in or all out
#pragma unroll
    for (int i = 0; i < 4; ++i) areg[i] = ld16(ra, ok ? aoff[i] + k0 * 2 : OOB);
  };
  auto store_a = [&](int buf) {
    uint16_t* dst = As + buf * (MT * AS) + arow0 * AS + 8 * ach;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4_t*>(dst + 32 * i * AS) = areg[i];
  };
  auto load_b = [&](int k0, BRegs<Q4>& b) {
    const int kk = k0 + 32 * hi;
    const bool ok = kk + 32 <= K;
    if constexpr (Q4) {
      b.q[0] = ld16(rw, ok ? wo0 + kk / 2 : OOB);
      b.q[1] = ld16(rw, ok ? wo1 + kk / 2 : OOB);
      const int ks = k0 / KT;
      if ((ks & 3) == 0) {   // a new run of 4 k-steps: one 16-B load of packed (scale, zero) per fragment
        b.sz[0] = ld16(rsz, so0 + ks * 4);
        b.sz[1] = ld16(rsz, so1 + ks * 4);
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        b.v[0][s] = ld16(rw, ok ? wo0 + kk * 2 + 16 * s : OOB);
        b.v[1][s] = ld16(rw, ok ? wo1 + kk * 2 + 16 * s : OOB);
      }
    }
  };
  auto frag = [&](const BRegs<Q4>& b, int f, int s, int j) -> u32x4_t {
    if constexpr (Q4) {
      const uint32_t p = j == 0 ? b.sz[f][0] : j == 1 ? b.sz[f][1] : j == 2 ? b.sz[f][2] : b.sz[f][3];
      uint32_t o[4];
      dq8(b.q[f][s], bf_lo(p), bf_hi(p), o);   // OOB rows load q = s = z = 0 -> exact zeros
      return u32x4_t{o[0], o[1], o[2], o[3]};
    } else {
      return b.v[f][s];
    }
  };

  const int nk = (K + KT - 1) / KT;
  if constexpr (Q4 && EPI == 1) {
    // int4 weights: a 4-deep ring of register sets (the loads of step i+4 are issued at step i, so an HBM fetch has
    // about four steps to land); the loop is unrolled by 4 so each set keeps one role. Packed (scale, zero) runs of
    // 4 steps are double-buffered (szc for the current run, szn loaded one run ahead). A: one step ahead via LDS.
    u32x4_t q0[2], q1[2], q2[2], q3[2], szc[2], szn[2];
    auto load_q = [&](int k0, u32x4_t* q) {
      const int kk = k0 + 32 * hi;
      const bool ok = k0 < K && kk + 32 <= K;
      q[0] = ld16(rw, ok ? wo0 + kk / 2 : OOB);
      q[1] = ld16(rw, ok ? wo1 + kk / 2 : OOB);
    };
    auto load_sz = [&](int ks, u32x4_t* z) {
      const bool ok = ks < nks;
      z[0] = ld16(rsz, ok ? so0 + ks * 4 : OOB);
      z[1] = ld16(rsz, ok ? so1 + ks * 4 : OOB);
    };
    auto step = [&](int i, const u32x4_t* q, int j) {
      const int buf = i & 1;
      const bool more = i + 1 < nk;
      if (more) load_a((i + 1) * KT);
      const uint16_t* Ab = As + buf * (MT * AS) + r32 * AS + 32 * hi;
      const uint32_t p0 = szc[0][j], p1 = szc[1][j];
      const float s0 = bf_lo(p0), z0 = bf_hi(p0), s1 = bf_lo(p1), z1 = bf_hi(p1);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        uint32_t o0[4], o1[4];
        dq8(q[0][s], s0, z0, o0);   // OOB rows load q = s = z = 0 -> exact zeros
        dq8(q[1][s], s1, z1, o1);
        const u32x4_t b0 = u32x4_t{o0[0], o0[1], o0[2], o0[3]};
        const u32x4_t b1 = u32x4_t{o1[0], o1[1], o1[2], o1[3]};
#pragma unroll
        for (int m = 0; m < NS; ++m) {
          const u32x4_t af = *reinterpret_cast<const u32x4_t*>(Ab + m * 32 * AS + 8 * s);
          acc[m][0] = mfma32(af, b0, acc[m][0]);
          acc[m][1] = mfma32(af, b1, acc[m][1]);
        }
      }
      if (more) store_a(buf ^ 1);
      __syncthreads();
    };
    load_a(0);
    load_q(0, q0);
    load_q(KT, q1);
    load_q(2 * KT, q2);
    load_q(3 * KT, q3);
    load_sz(0, szc);
    load_sz(4, szn);
    store_a(0);
    __syncthreads();
    for (int i = 0; i < nk; i += 4) {
      step(i, q0, 0);
      load_q((i + 4) * KT, q0);
      if (i + 1 >= nk) break;
      step(i + 1, q1, 1);
      load_q((i + 5) * KT, q1);
      if (i + 2 >= nk) break;
      step(i + 2, q2, 2);
      load_q((i + 6) * KT, q2);
      if (i + 3 >= nk) break;
      step(i + 3, q3, 3);
      load_q((i + 7) * KT, q3);
      szc[0] = szn[0];
      szc[1] = szn[1];
      load_sz(i + 8, szn);
    }
  } else {
    load_a(0);
    load_b(0, bc);
    store_a(0);
    __syncthreads();
    int buf = 0;
    for (int i = 0; i < nk; ++i) {
      const bool more = i + 1 < nk;
      if (more) {
        load_a((i + 1) * KT);
        load_b((i + 1) * KT, bn);
      }
      const uint16_t* Ab = As + buf * (MT * AS) + r32 * AS + 32 * hi;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4_t b0 = frag(bc, 0, s, i & 3);
        const u32x4_t b1 = frag(bc, 1, s, i & 3);
#pragma unroll
        for (int m = 0; m < NS; ++m) {
          const u32x4_t af = *reinterpret_cast<const u32x4_t*>(Ab + m * 32 * AS + 8 * s);
          acc[m][0] = mfma32(af, b0, acc[m][0]);
          acc[m][1] = mfma32(af, b1, acc[m][1]);
        }
      }
      if (more) {
        store_a(buf ^ 1);
        if constexpr (Q4) {
          bc.q[0] = bn.q[0];
          bc.q[1] = bn.q[1];
          if (((i + 1) & 3) == 0) {
            bc.sz[0] = bn.sz[0];
            bc.sz[1] = bn.sz[1];
          }
        } else {
          bc = bn;
        }
      }
      __syncthreads();
      buf ^= 1;
    }
  }
  // ---- LoRA K-extension: ext[row][0:32] . Bext[n][0:32]
  const uint16_t* eb = kind == SMEL_KIND_SEL ? (ws.ext_sel ? ws.ext_sel + (int64_t)idx * a.N * 32 : nullptr)
                                             : (kind == SMEL_KIND_SHARED ? ws.ext_sh : nullptr);
  if (a.ext && eb) {
    const rsrc_t re = make_rsrc(eb, (uint64_t)a.N * 64);
    const rsrc_t rx = make_rsrc(a.ext + (int64_t)row0 * 32, (uint64_t)nrows * 64);
    u32x4_t b0[2], b1[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      b0[s] = ld16(re, fv0 ? (uint32_t)n0 * 64 + 32 * hi + 16 * s : OOB);
      b1[s] = ld16(re, fv1 ? (uint32_t)n1 * 64 + 32 * hi + 16 * s : OOB);
    }
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
#pragma unroll
  for (int m = 0; m < NS; ++m) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m * 32 + acc_row(r, l);
      if (row >= nrows) continue;
      const int grow = row0 + row;
      if (EPI == 1) {
        if (!fv0) continue;
        const int I = a.N / 2;
        const uint16_t gb = f2bf(acc[m][0][r]), ub = f2bf(acc[m][1][r]);
        const float av = act_f(bf2f(gb), a.act) * bf2f(ub);
        a.out[(int64_t)grow * a.ldo + n0] = f2bf(av);
        if (a.hsave) {
          a.hsave[(int64_t)grow * a.N + n0] = gb;
          a.hsave[(int64_t)grow * a.N + I + n0] = ub;
        }
      } else {
        const int64_t orow = (int64_t)row_slot(grow, a.order, a.TK) * a.ldo;
        if (fv0) a.out[orow + n0] = f2bf(acc[m][0][r]);
        if (fv1) a.out[orow + n1] = f2bf(acc[m][1][r]);
      }
    }
  }
}

template <int EPI, bool Q4>
SMEL_DEV void run_tile_ns(const FwdArgs& a, int kind, int idx, int row0, int nrows, int nb, uint16_t* As) {
  switch ((nrows + 31) >> 5) {
    case 1: run_tile<EPI, Q4, 1>(a, kind, idx, row0, nrows, nb, As); break;
    case 2: run_tile<EPI, Q4, 2>(a, kind, idx, row0, nrows, nb, As); break;
    case 3: run_tile<EPI, Q4, 3>(a, kind, idx, row0, nrows, nb, As); break;
    default: run_tile<EPI, Q4, 4>(a, kind, idx, row0, nrows, nb, As); break;
  }
}

template <int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gmm_fwd_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2 * MT * AS];
  int tile, nb;
  if (!xcd_tile(a.n_tiles[0], a.nblk, tile, nb)) return;
  const int4 t = a.tiles[tile];
  const int gk = a.gkind[t.x];
  const int kind = gk >> 16, idx = gk & 0xffff;
  const int nrows = min(t.z - t.y, MT);
  if (nrows <= 0) return;
  if (kind == SMEL_KIND_INT4)
    run_tile_ns<EPI, true>(a, kind, idx, t.y, nrows, nb, As);
  else
    run_tile_ns<EPI, false>(a, kind, idx, t.y, nrows, nb, As);
}

}  // namespace

extern "C" int smel_gmm_fwd(const smel_wset* w, const int32_t* gkind, const int32_t* tiles, const int32_t* n_tiles,
                            int64_t max_tiles, const uint16_t* A, int64_t lda, int64_t a_rows, int32_t a_gather,
                            const int32_t* order, int64_t TK, int64_t topk, const uint16_t* ext, int32_t epilogue,
                            int32_t act, uint16_t* out, int64_t ldo, uint16_t* hsave, hipStream_t stream) {
  SMEL_REQUIRE(w && gkind && tiles && n_tiles && A && out, SMEL_EINVAL, "gmm_fwd: null pointer");
  SMEL_REQUIRE(w->R > 0 && w->C > 0 && max_tiles >= 0 && lda >= w->C && topk > 0, SMEL_EINVAL,
               "gmm_fwd: bad sizes");
  SMEL_REQUIRE(w->C % 32 == 0, SMEL_EUNSUPPORTED, "gmm_fwd: K=%lld must be a multiple of 32", (long long)w->C);
  SMEL_REQUIRE(w->R % 32 == 0 && (epilogue == 0 || (w->R / 2) % 32 == 0), SMEL_EUNSUPPORTED,
               "gmm_fwd: N=%lld must be a multiple of 32 (64 for gate_up)", (long long)w->R);
  SMEL_REQUIRE(!w->q4 || (w->group % 32 == 0 && w->C % w->group == 0), SMEL_EUNSUPPORTED,
               "gmm_fwd: int4 group %d must be a multiple of 32 dividing K", w->group);
  SMEL_REQUIRE(!w->q4 || w->sz4, SMEL_EINVAL, "gmm_fwd: an int4 bank needs its packed scale/zero (smel_int4_pack_sz)");
  SMEL_REQUIRE(lda % 8 == 0 && ((uintptr_t)A % 16) == 0, SMEL_EUNSUPPORTED, "gmm_fwd: A rows must be 16-B aligned");
  SMEL_REQUIRE(epilogue == 0 || epilogue == 1, SMEL_EINVAL, "gmm_fwd: epilogue %d", epilogue);
  SMEL_REQUIRE(!a_gather || order || TK == 0, SMEL_EINVAL, "gmm_fwd: gather needs order");
  SMEL_REQUIRE(act == 0 || act == 1, SMEL_EINVAL, "gmm_fwd: act %d", act);
  SMEL_REQUIRE(a_rows >= 0 && a_rows * lda * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "gmm_fwd: A larger than 2 GiB");
  if (max_tiles == 0) return 0;
  FwdArgs a;
  a.w = *w;
  a.gkind = gkind;
  a.tiles = reinterpret_cast<const int4*>(tiles);
  a.n_tiles = n_tiles;
  a.A = A;
  a.lda = lda;
  a.a_rows = a_rows;
  a.order = order;
  a.ext = ext;
  a.out = out;
  a.ldo = ldo;
  a.hsave = hsave;
  a.a_gather = a_gather;
  a.TK = (int)TK;
  a.topk = (int)topk;
  a.act = act;
  a.N = (int)w->R;
  a.K = (int)w->C;
  a.nblk = (int)(epilogue == 1 ? (w->R / 2 + 127) / 128 : (w->R + 255) / 256);
  const unsigned grid = (unsigned)(xcd_grid(max_tiles) * a.nblk);
  if (epilogue == 1)
    gmm_fwd_kernel<1><<<grid, 256, 0, stream>>>(a);
  else
    gmm_fwd_kernel<0><<<grid, 256, 0, stream>>>(a);
  return smel::launch_status();
}
