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
  const int32_t* order;
  const uint16_t* ext;
  uint16_t* out;
  int64_t ldo;
  uint16_t* hsave;
  int a_gather, TK, topk, act;
  int N, K;   // N = w.R (weight rows), K = w.C
};

struct BSrc {
  const uint8_t* q;      // int4 row base (bytes), or nullptr
  const uint16_t* sz_s;  // scale row base
  const uint16_t* sz_z;  // zero row base
  const uint16_t* wb;    // bf16 row base, or nullptr
};

template <bool Q4>
SMEL_DEV BSrc weight_row(const FwdArgs& a, int kind, int idx, int n, bool valid) {
  BSrc b{nullptr, nullptr, nullptr, nullptr};
  if (!valid) return b;
  const smel_wset& w = a.w;
  if (Q4) {
    const int64_t r = (int64_t)idx * w.R + n;
    b.q = w.q4 + r * (w.C / 2);
    b.sz_s = w.s4 + r * (w.C / w.group);
    b.sz_z = w.z4 + r * (w.C / w.group);
  } else {
    const uint16_t* base = kind == SMEL_KIND_BF16 ? w.wb : (kind == SMEL_KIND_SEL ? w.wsel : w.wsh);
    const int64_t mi = kind == SMEL_KIND_SHARED ? 0 : idx;
    b.wb = base + (mi * w.R + n) * w.C;
  }
  return b;
}

// Raw weight data of one fragment for one k-step.
struct BRaw {
  u32x4_t v[4];   // int4: v[0] holds 32 nibbles; bf16: v[0..3] hold 32 bf16
  float s, z;
};

template <bool Q4>
SMEL_DEV void load_b(const BSrc& b, int kk, int group, BRaw& r) {
  if (Q4) {
    if (b.q) {
      r.v[0] = *reinterpret_cast<const u32x4_t*>(b.q + kk / 2);
      r.s = bf2f(b.sz_s[kk / group]);
      r.z = bf2f(b.sz_z[kk / group]);
    } else {
      r.v[0] = u32x4_t{};
      r.s = r.z = 0.f;   // dequantizes to exact zeros
    }
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      r.v[s] = b.wb ? *reinterpret_cast<const u32x4_t*>(b.wb + kk + 8 * s) : u32x4_t{};
  }
}

template <bool Q4>
SMEL_DEV void make_frags(const BRaw& r, u32x4_t f[4]) {
  if (Q4) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      uint32_t o[4];
      dq8(r.v[0][s], r.s, r.z, o);
      f[s] = u32x4_t{o[0], o[1], o[2], o[3]};
    }
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) f[s] = r.v[s];
  }
}

template <int EPI, bool Q4>
SMEL_DEV void run_tile(const FwdArgs& a, int kind, int idx, int row0, int nrows, uint16_t* As) {
  const int tid = threadIdx.x, l = lane_id(), w = tid >> 6, hi = l >> 5, r32 = l & 31;
  const int nb = blockIdx.y;
  const int K = a.K;
  // ---- this wave's two weight rows (per lane)
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
  const BSrc bs0 = weight_row<Q4>(a, kind, idx, n0, fv0);
  const BSrc bs1 = weight_row<Q4>(a, kind, idx, n1, fv1);
  // ---- A staging: thread -> (tile row, 32-wide half of the k-step)
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

  u32x4_t areg[4];
  auto load_a = [&](int k0) {
    const bool ok = arow && (k0 + 32 * ap + 32 <= K);
#pragma unroll
    for (int i = 0; i < 4; ++i) areg[i] = ok ? *reinterpret_cast<const u32x4_t*>(arow + k0 + 32 * ap + 8 * i) : u32x4_t{};
  };
  auto store_a = [&](int buf) {
    uint16_t* dst = As + buf * (MT * AS) + ar * AS + 32 * ap;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4_t*>(dst + 8 * i) = areg[i];
  };
  BRaw braw[2];
  auto load_bs = [&](int k0) {
    const int kk = k0 + 32 * hi;
    const bool ok = kk + 32 <= K;
    load_b<Q4>(ok ? bs0 : BSrc{nullptr, nullptr, nullptr, nullptr}, kk, a.w.group, braw[0]);
    load_b<Q4>(ok ? bs1 : BSrc{nullptr, nullptr, nullptr, nullptr}, kk, a.w.group, braw[1]);
  };

  load_a(0);
  store_a(0);
  load_bs(0);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < K; k0 += KT) {
    u32x4_t bf0[4], bf1[4];
    make_frags<Q4>(braw[0], bf0);
    make_frags<Q4>(braw[1], bf1);
    const bool more = k0 + KT < K;
    if (more) {
      load_a(k0 + KT);
      load_bs(k0 + KT);
    }
    const uint16_t* Ab = As + buf * (MT * AS);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m < nslice) {
          const u32x4_t af = *reinterpret_cast<const u32x4_t*>(Ab + (m * 32 + r32) * AS + 32 * hi + 8 * s);
          if (fv0) acc[m][0] = mfma32(af, bf0[s], acc[m][0]);
          if (fv1) acc[m][1] = mfma32(af, bf1[s], acc[m][1]);
        }
      }
    }
    if (more) store_a(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  // ---- LoRA K-extension: ext[row][0:32] . Bext[n][0:32]
  const uint16_t* eb = kind == SMEL_KIND_SEL ? (a.w.ext_sel ? a.w.ext_sel + (int64_t)idx * a.N * 32 : nullptr)
                                               : (kind == SMEL_KIND_SHARED ? a.w.ext_sh : nullptr);
  if (a.ext && eb) {
    u32x4_t b0[2], b1[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      b0[s] = fv0 ? *reinterpret_cast<const u32x4_t*>(eb + (int64_t)n0 * 32 + 16 * hi + 8 * s) : u32x4_t{};
      b1[s] = fv1 ? *reinterpret_cast<const u32x4_t*>(eb + (int64_t)n1 * 32 + 16 * hi + 8 * s) : u32x4_t{};
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
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    if (m >= nslice) continue;
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

template <int EPI>
__global__ __launch_bounds__(256) void gmm_fwd_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2 * MT * AS];
  if ((int)blockIdx.x >= a.n_tiles[0]) return;
  const int4 t = a.tiles[blockIdx.x];
  const int gk = a.gkind[t.x];
  const int kind = gk >> 16, idx = gk & 0xffff;
  const int nrows = t.z - t.y;
  if (nrows <= 0) return;
  if (kind == SMEL_KIND_INT4)
    run_tile<EPI, true>(a, kind, idx, t.y, nrows, As);
  else
    run_tile<EPI, false>(a, kind, idx, t.y, nrows, As);
}

}  // namespace

extern "C" int smel_gmm_fwd(const smel_wset* w, const int32_t* gkind, const int32_t* tiles, const int32_t* n_tiles,
                            int64_t max_tiles, const uint16_t* A, int64_t lda, int32_t a_gather,
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
  SMEL_REQUIRE(lda % 8 == 0 && ((uintptr_t)A % 16) == 0, SMEL_EUNSUPPORTED, "gmm_fwd: A rows must be 16-B aligned");
  SMEL_REQUIRE(epilogue == 0 || epilogue == 1, SMEL_EINVAL, "gmm_fwd: epilogue %d", epilogue);
  SMEL_REQUIRE(!a_gather || order || TK == 0, SMEL_EINVAL, "gmm_fwd: gather needs order");
  SMEL_REQUIRE(act == 0 || act == 1, SMEL_EINVAL, "gmm_fwd: act %d", act);
  if (max_tiles == 0) return 0;
  FwdArgs a;
  a.w = *w;
  a.gkind = gkind;
  a.tiles = reinterpret_cast<const int4*>(tiles);
  a.n_tiles = n_tiles;
  a.A = A;
  a.lda = lda;
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
  if (epilogue == 1) {
    dim3 grid((unsigned)max_tiles, (unsigned)((w->R / 2 + 127) / 128));
    gmm_fwd_kernel<1><<<grid, 256, 0, stream>>>(a);
  } else {
    dim3 grid((unsigned)max_tiles, (unsigned)((w->R + 255) / 256));
    gmm_fwd_kernel<0><<<grid, 256, 0, stream>>>(a);
  }
  return smel::launch_status();
}
