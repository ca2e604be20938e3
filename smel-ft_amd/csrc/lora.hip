// LoRA pieces of the selected experts and the shared MLP (smel/lora.py:14-83): layout of the fp32 factors into the
// bf16 K-extension operands, the rank-32 down-projections of LoRA rows (x A^T, act A_d^T, dy B_d, dh B^T) and the
// factor gradients as fixed-order row reductions.
#include "abi_util.h"
#include "common.h"

namespace {

__global__ __launch_bounds__(256) void lora_prep_kernel(const float* __restrict__ Ag, const float* __restrict__ Bg,
                                                        const float* __restrict__ Au, const float* __restrict__ Bu,
                                                        const float* __restrict__ Ad, const float* __restrict__ Bd,
                                                        int n, int r, int Hd, int In, uint16_t* __restrict__ fwd_gu,
                                                        uint16_t* __restrict__ fwd_dn, uint16_t* __restrict__ a_gu,
                                                        uint16_t* __restrict__ a_dn, uint16_t* __restrict__ bt_dn,
                                                        uint16_t* __restrict__ bt_gu, uint16_t* __restrict__ at_gu,
                                                        uint16_t* __restrict__ at_dn) {
  const int which = blockIdx.y;
  int64_t total;
  switch (which) {
    case 0: total = (int64_t)n * 2 * In * 32; break;
    case 1: total = (int64_t)n * Hd * 32; break;
    case 2: total = (int64_t)n * 32 * Hd; break;
    case 3: total = (int64_t)n * 32 * In; break;
    case 4: total = (int64_t)n * 32 * Hd; break;
    case 5: total = (int64_t)n * 32 * 2 * In; break;
    case 6: total = (int64_t)n * Hd * 32; break;
    default: total = (int64_t)n * In * 32; break;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    float v = 0.f;
    if (which == 0) {            // fwd_gu [n][2In][32]
      const int c = i % 32;
      const int64_t rowg = i / 32;
      const int row = rowg % (2 * In);
      const int g = rowg / (2 * In);
      if (row < In && c < r) v = Bg[((int64_t)g * In + row) * r + c];
      if (row >= In && c >= 16 && c < 16 + r) v = Bu[((int64_t)g * In + row - In) * r + c - 16];
      fwd_gu[i] = f2bf(v);
    } else if (which == 1) {     // fwd_dn [n][Hd][32]
      const int c = i % 32;
      const int64_t rowg = i / 32;
      if (c < r) v = Bd[rowg * r + c];
      fwd_dn[i] = f2bf(v);
    } else if (which == 2) {     // a_gu [n][32][Hd]
      const int h = i % Hd;
      const int j = (i / Hd) % 32;
      const int g = i / ((int64_t)Hd * 32);
      if (j < r) v = Ag[((int64_t)g * r + j) * Hd + h];
      if (j >= 16 && j < 16 + r) v = Au[((int64_t)g * r + j - 16) * Hd + h];
      a_gu[i] = f2bf(v);
    } else if (which == 3) {     // a_dn [n][32][In]
      const int c = i % In;
      const int j = (i / In) % 32;
      const int g = i / ((int64_t)In * 32);
      if (j < r) v = Ad[((int64_t)g * r + j) * In + c];
      a_dn[i] = f2bf(v);
    } else if (which == 4) {     // bt_dn [n][32][Hd] = B_down^T
      const int h = i % Hd;
      const int j = (i / Hd) % 32;
      const int g = i / ((int64_t)Hd * 32);
      if (j < r) v = Bd[((int64_t)g * Hd + h) * r + j];
      bt_dn[i] = f2bf(v);
    } else if (which == 5) {     // bt_gu [n][32][2In]
      const int c = i % (2 * In);
      const int j = (i / (2 * In)) % 32;
      const int g = i / ((int64_t)2 * In * 32);
      if (j < r && c < In) v = Bg[((int64_t)g * In + c) * r + j];
      if (j >= 16 && j < 16 + r && c >= In) v = Bu[((int64_t)g * In + c - In) * r + j - 16];
      bt_gu[i] = f2bf(v);
    } else if (which == 6) {     // at_gu [n][Hd][32]: a_gu transposed (the backward GEMM's K-extension)
      const int j = i % 32;
      const int64_t hg = i / 32;
      const int h = hg % Hd;
      const int g = hg / Hd;
      if (j < r) v = Ag[((int64_t)g * r + j) * Hd + h];
      if (j >= 16 && j < 16 + r) v = Au[((int64_t)g * r + j - 16) * Hd + h];
      at_gu[i] = f2bf(v);
    } else {                     // at_dn [n][In][32]: a_dn transposed
      const int j = i % 32;
      const int64_t cg = i / 32;
      const int c = cg % In;
      const int g = cg / In;
      if (j < r) v = Ad[((int64_t)g * r + j) * In + c];
      at_dn[i] = f2bf(v);
    }
  }
}

// ext[row][0:32] = bf16(scale * A_src[src(row)] . wcat^T) for the rows of SEL / SHARED tiles. Block = one 32-row
// slice of a tile; its 8 waves take the 64-wide k-steps j = w, w + 8, ... issuing all loads of up to XPRE of their
// steps before the MFMAs (one memory latency per XPRE steps, not one per step); the partial sums are added in wave
// order through LDS.
constexpr int XW = 8;
constexpr int XPRE = 4;

__global__ __launch_bounds__(512) void lora_ext_kernel(const int4* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
                                                       const int32_t* __restrict__ gkind, const uint16_t* __restrict__ A,
                                                       int64_t lda, int64_t a_rows, int a_gather,
                                                       const int32_t* __restrict__ order, int TK, int topk,
                                                       const uint16_t* __restrict__ wsel, const uint16_t* __restrict__ wsh,
                                                       int Kd, float ssel, float ssh, uint16_t* __restrict__ ext) {
  __shared__ float red[XW * 64 * 16];
  if ((int)blockIdx.x >= n_tiles[0]) return;
  const int4 t = tiles[blockIdx.x];
  const int gk = gkind[t.x];
  const int kind = gk >> 16, idx = gk & 0xffff;
  if (kind != SMEL_KIND_SEL && kind != SMEL_KIND_SHARED) return;
  const int m = blockIdx.y;
  const int nrows = min(t.z - t.y, 128);
  if (m * 32 >= nrows) return;
  const uint16_t* wc = kind == SMEL_KIND_SEL ? (wsel ? wsel + (int64_t)idx * 32 * Kd : nullptr) : wsh;
  if (!wc) return;   // this group has no LoRA
  const int l = lane_id(), w = threadIdx.x >> 6, hi = l >> 5, r32 = l & 31;
  const float scale = kind == SMEL_KIND_SEL ? ssel : ssh;
  const int row = m * 32 + r32;
  const rsrc_t ra = make_rsrc(A, (uint64_t)a_rows * lda * 2);
  const rsrc_t rb = make_rsrc(wc, (uint64_t)32 * Kd * 2);
  uint32_t ao = OOB;
  if (row < nrows) {
    const int grow = t.y + row;
    ao = (uint32_t)(a_gather ? row_token(grow, order, TK, topk) : grow) * (uint32_t)lda * 2;
  }
  const uint32_t bo = (uint32_t)r32 * Kd * 2;
  const int nk = (Kd + 63) / 64;
  f32x16_t acc = f32x16_t{};
  for (int j0 = w; j0 < nk; j0 += XW * XPRE) {
    u32x4_t av[XPRE][4], bv[XPRE][4];
#pragma unroll
    for (int p = 0; p < XPRE; ++p) {
      const int kk = (j0 + XW * p) * 64 + 32 * hi;
      const bool ok = kk + 32 <= Kd;   // Kd % 32 == 0: a lane half's 32 k are all in or all out
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        av[p][s] = ld16(ra, ok ? ao + kk * 2 + 16 * s : OOB);
        bv[p][s] = ld16(rb, ok ? bo + kk * 2 + 16 * s : OOB);
      }
    }
    __builtin_amdgcn_sched_barrier(0);   // every load of the batch is issued before the first MFMA waits
#pragma unroll
    for (int p = 0; p < XPRE; ++p)
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = mfma32(av[p][s], bv[p][s], acc);
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) red[(w * 16 + r) * 64 + l] = acc[r];   // lane-contiguous: no bank conflicts
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = red[r * 64 + l];
#pragma unroll
      for (int ww = 1; ww < XW; ++ww) v += red[(ww * 16 + r) * 64 + l];
      const int orow = m * 32 + acc_row(r, l);
      if (orow < nrows) ext[(int64_t)(t.y + orow) * 32 + r32] = f2bf(scale * v);
    }
  }
}

// part[i][c][p][q] = sum over rows c*CH .. c*CH+CH-1 of group lora_groups[i]: alpha(row) L[row][p] Rm[src(row)][q],
// as an MFMA GEMM with the row index as the contraction dim: per 64-row step, L and Rm are staged transposed in LDS
// (k-pair packing: the values of rows 2j and 2j+1 share one 32-bit word), then each wave multiplies the 32 x 64 L^T
// tile by its 64 x 32 slice of the Rm tile. Block = 4 waves = 32 p x 128 q. The LDS tiles are double-buffered and
// the raw rows of step j+1 are loaded into registers before step j's MFMAs, so one barrier per step suffices and a
// load's latency overlaps a step of work.
constexpr int WG_CH = 256;    // rows per chunk
constexpr int WG_QB = 128;    // columns per block
constexpr int WG_S = 64 + 8;  // LDS row stride (bf16)

__global__ __launch_bounds__(256) void lora_wgrad_part(const int32_t* __restrict__ groups, const int32_t* __restrict__ offsets,
                                                       int E, int T, int TK, int topk, const int32_t* __restrict__ order,
                                                       const uint16_t* __restrict__ L, const uint16_t* __restrict__ Rm,
                                                       int64_t ldr, int64_t r_rows, int r_gather, int use_w,
                                                       const uint16_t* __restrict__ topv, const float* __restrict__ sgate,
                                                       int Q, float* __restrict__ part, int chunks) {
  __shared__ __attribute__((aligned(16))) uint16_t LT[2][32 * WG_S];
  __shared__ __attribute__((aligned(16))) uint16_t RT[2][WG_QB * WG_S];
  const int i = blockIdx.x, c = blockIdx.z;
  const int g = groups[i];
  const int r0 = g < E ? offsets[g] : TK;
  const int r1 = g < E ? offsets[g + 1] : TK + T;
  const int a0 = r0 + c * WG_CH;
  if (a0 >= r1) return;
  const int a1 = min(r1, a0 + WG_CH);
  const int q0 = blockIdx.y * WG_QB;
  const int tid = threadIdx.x, l = lane_id(), w = tid >> 6, hi = l >> 5, r32 = l & 31;
  const int kp = tid & 31, grp = tid >> 5;   // k pair, and 4 p's (L) / 16 q's (Rm) per thread
  const int qq = q0 + 16 * grp;
  const bool qok = qq < Q;
  const rsrc_t rr = make_rsrc(Rm, (uint64_t)r_rows * ldr * 2);
  f32x16_t acc = f32x16_t{};
  // raw data of one step for this thread: L rows (ra, ra+1) x 4 p, Rm rows (ra, ra+1) x 16 q, the row weights
  uint2 lv0, lv1;
  u32x4_t x0[2], x1[2];
  float al0, al1;
  auto row_info = [&](int row, uint32_t& roff, float& alpha) {
    roff = OOB;
    alpha = 0.f;
    if (row < a1) {
      int src = row;
      alpha = 1.f;
      if (row < TK) {
        const int p = order[row];
        if (r_gather) src = p / topk;
        if (use_w) alpha = bf2f(topv[p]);
      } else {
        if (r_gather) src = row - TK;
        if (use_w) alpha = sgate[row - TK];
      }
      roff = (uint32_t)src * (uint32_t)ldr * 2;
    }
  };
  auto load = [&](int k0) {
    const int ra = k0 + 2 * kp;
    uint32_t o0, o1;
    row_info(ra, o0, al0);
    row_info(ra + 1, o1, al1);
    lv0 = ra < a1 ? *reinterpret_cast<const uint2*>(L + (int64_t)ra * 32 + 4 * grp) : make_uint2(0, 0);
    lv1 = ra + 1 < a1 ? *reinterpret_cast<const uint2*>(L + (int64_t)(ra + 1) * 32 + 4 * grp) : make_uint2(0, 0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      x0[h] = ld16(rr, qok ? o0 + (uint32_t)(qq + 8 * h) * 2 : OOB);
      x1[h] = ld16(rr, qok ? o1 + (uint32_t)(qq + 8 * h) * 2 : OOB);
    }
  };
  auto stage = [&](int buf) {
    // L^T: alpha folded in (fp32, one bf16 rounding)
    uint32_t* d = reinterpret_cast<uint32_t*>(LT[buf] + (4 * grp) * WG_S + 2 * kp);
    d[0 * (WG_S / 2)] = pack2bf(al0 * bf_lo(lv0.x), al1 * bf_lo(lv1.x));
    d[1 * (WG_S / 2)] = pack2bf(al0 * bf_hi(lv0.x), al1 * bf_hi(lv1.x));
    d[2 * (WG_S / 2)] = pack2bf(al0 * bf_lo(lv0.y), al1 * bf_lo(lv1.y));
    d[3 * (WG_S / 2)] = pack2bf(al0 * bf_hi(lv0.y), al1 * bf_hi(lv1.y));
    uint32_t* e = reinterpret_cast<uint32_t*>(RT[buf] + (16 * grp) * WG_S + 2 * kp);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        e[(8 * h + 2 * j) * (WG_S / 2)] = __builtin_amdgcn_perm(x1[h][j], x0[h][j], 0x05040100u);
        e[(8 * h + 2 * j + 1) * (WG_S / 2)] = __builtin_amdgcn_perm(x1[h][j], x0[h][j], 0x07060302u);
      }
  };
  load(a0);
  int buf = 0;
  for (int k0 = a0; k0 < a1; k0 += 64) {
    stage(buf);
    if (k0 + 64 < a1) load(k0 + 64);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4_t af = *reinterpret_cast<const u32x4_t*>(LT[buf] + r32 * WG_S + 32 * hi + 8 * s);
      const u32x4_t bfr = *reinterpret_cast<const u32x4_t*>(RT[buf] + (32 * w + r32) * WG_S + 32 * hi + 8 * s);
      acc = mfma32(af, bfr, acc);
    }
    buf ^= 1;
  }
  const int q = q0 + 32 * w + r32;
  if (q < Q) {
    float* dst = part + ((int64_t)i * chunks + c) * 32 * Q + q;
#pragma unroll
    for (int r = 0; r < 16; ++r) dst[(int64_t)acc_row(r, l) * Q] = acc[r];
  }
}

__global__ __launch_bounds__(256) void lora_wgrad_sum(const int32_t* __restrict__ groups,
                                                      const int32_t* __restrict__ offsets, int E, int T, int TK,
                                                      int Q, const float* __restrict__ part, int chunks,
                                                      float* __restrict__ out) {
  const int i = blockIdx.y;
  const int g = groups[i];
  const int rows = g < E ? offsets[g + 1] - offsets[g] : T;
  const int nch = min((rows + WG_CH - 1) / WG_CH, chunks);
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < (int64_t)32 * Q; e += (int64_t)gridDim.x * blockDim.x) {
    float v = 0.f;
    for (int c = 0; c < nch; ++c) v += part[((int64_t)i * chunks + c) * 32 * Q + e];
    out[(int64_t)i * 32 * Q + e] = v;
  }
}

}  // namespace

extern "C" int smel_lora_prep(const float* A_gate, const float* B_gate, const float* A_up, const float* B_up,
                              const float* A_down, const float* B_down, int64_t n, int64_t r, int64_t Hd, int64_t In,
                              uint16_t* fwd_gu, uint16_t* fwd_dn, uint16_t* a_gu, uint16_t* a_dn, uint16_t* bt_dn,
                              uint16_t* bt_gu, uint16_t* at_gu, uint16_t* at_dn, hipStream_t stream) {
  SMEL_REQUIRE(n >= 0 && r > 0 && Hd > 0 && In > 0, SMEL_EINVAL, "lora_prep: bad sizes");
  SMEL_REQUIRE(r <= 16, SMEL_EUNSUPPORTED, "lora_prep: rank %lld > 16", (long long)r);
  if (n == 0) return 0;
  SMEL_REQUIRE(A_gate && B_gate && A_up && B_up && A_down && B_down && fwd_gu && fwd_dn && a_gu && a_dn && bt_dn &&
                   bt_gu && at_gu && at_dn, SMEL_EINVAL, "lora_prep: null pointer");
  dim3 grid(256, 8);
  lora_prep_kernel<<<grid, 256, 0, stream>>>(A_gate, B_gate, A_up, B_up, A_down, B_down, (int)n, (int)r, (int)Hd,
                                             (int)In, fwd_gu, fwd_dn, a_gu, a_dn, bt_dn, bt_gu, at_gu, at_dn);
  return smel::launch_status();
}

extern "C" int smel_lora_ext(const int32_t* tiles, const int32_t* n_tiles, int64_t max_tiles, const int32_t* gkind,
                             const uint16_t* A_src, int64_t lda, int64_t a_rows, int32_t a_gather,
                             const int32_t* order, int64_t TK, int64_t topk, const uint16_t* wcat_sel,
                             const uint16_t* wcat_sh, int64_t Kd, float scale_sel, float scale_sh, uint16_t* ext,
                             hipStream_t stream) {
  SMEL_REQUIRE(tiles && n_tiles && gkind && A_src && ext, SMEL_EINVAL, "lora_ext: null pointer");
  SMEL_REQUIRE(Kd > 0 && Kd % 32 == 0, SMEL_EUNSUPPORTED, "lora_ext: K %lld must be a multiple of 32", (long long)Kd);
  SMEL_REQUIRE(lda % 8 == 0 && ((uintptr_t)A_src % 16) == 0, SMEL_EUNSUPPORTED, "lora_ext: A rows must be 16-B aligned");
  SMEL_REQUIRE(!a_gather || order || TK == 0, SMEL_EINVAL, "lora_ext: gather needs order");
  SMEL_REQUIRE(a_rows >= 0 && a_rows * lda * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "lora_ext: A larger than 2 GiB");
  if (max_tiles == 0) return 0;
  dim3 grid((unsigned)max_tiles, 4);
  lora_ext_kernel<<<grid, 512, 0, stream>>>(reinterpret_cast<const int4*>(tiles), n_tiles, gkind, A_src, lda, a_rows,
                                            a_gather, order, (int)TK, (int)topk, wcat_sel, wcat_sh, (int)Kd, scale_sel,
                                            scale_sh, ext);
  return smel::launch_status();
}

extern "C" int64_t smel_lora_wgrad_part_chunks(int64_t max_group_rows) {
  return (max_group_rows + WG_CH - 1) / WG_CH;
}

extern "C" int smel_lora_wgrad(const int32_t* lora_groups, int64_t n_lora, const int32_t* offsets, int64_t E,
                               int64_t T, int64_t TK, int64_t topk, const int32_t* order, const uint16_t* L,
                               const uint16_t* Rm, int64_t ldr, int64_t r_rows, int32_t r_gather, int32_t use_w,
                               const uint16_t* topv, const float* sgate, int64_t Q, float* part,
                               int64_t part_chunks, float* out, hipStream_t stream) {
  SMEL_REQUIRE(n_lora >= 0 && Q > 0 && part_chunks >= 0, SMEL_EINVAL, "lora_wgrad: bad sizes");
  if (n_lora == 0 || part_chunks == 0) return 0;
  SMEL_REQUIRE(lora_groups && offsets && L && Rm && part && out, SMEL_EINVAL, "lora_wgrad: null pointer");
  SMEL_REQUIRE(!(r_gather || use_w) || order || TK == 0, SMEL_EINVAL, "lora_wgrad: needs order");
  SMEL_REQUIRE(ldr % 8 == 0 && Q % 16 == 0 && ((uintptr_t)Rm % 16) == 0, SMEL_EUNSUPPORTED,
               "lora_wgrad: Rm rows must be 16-B aligned and Q a multiple of 16");
  SMEL_REQUIRE(r_rows * ldr * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "lora_wgrad: Rm larger than 2 GiB");
  dim3 g1((unsigned)n_lora, (unsigned)((Q + WG_QB - 1) / WG_QB), (unsigned)part_chunks);
  lora_wgrad_part<<<g1, 256, 0, stream>>>(lora_groups, offsets, (int)E, (int)T, (int)TK, (int)topk, order, L, Rm, ldr,
                                          r_rows, r_gather, use_w, topv, sgate, (int)Q, part, (int)part_chunks);
  int st = smel::launch_status();
  if (st) return st;
  dim3 g2((unsigned)std::min<int64_t>((32 * Q + 255) / 256, 1024), (unsigned)n_lora);
  lora_wgrad_sum<<<g2, 256, 0, stream>>>(lora_groups, offsets, (int)E, (int)T, (int)TK, (int)Q, part,
                                         (int)part_chunks, out);
  return smel::launch_status();
}
