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
                                                        uint16_t* __restrict__ bt_gu) {
  const int which = blockIdx.y;
  int64_t total;
  switch (which) {
    case 0: total = (int64_t)n * 2 * In * 32; break;
    case 1: total = (int64_t)n * Hd * 32; break;
    case 2: total = (int64_t)n * 32 * Hd; break;
    case 3: total = (int64_t)n * 32 * In; break;
    case 4: total = (int64_t)n * 32 * Hd; break;
    default: total = (int64_t)n * 32 * 2 * In; break;
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
    } else {                     // bt_gu [n][32][2In]
      const int c = i % (2 * In);
      const int j = (i / (2 * In)) % 32;
      const int g = i / ((int64_t)2 * In * 32);
      if (j < r && c < In) v = Bg[((int64_t)g * In + c) * r + j];
      if (j >= 16 && j < 16 + r && c >= In) v = Bu[((int64_t)g * In + c - In) * r + j - 16];
      bt_gu[i] = f2bf(v);
    }
  }
}

// ext[row][0:32] = bf16(scale * A_src[src(row)] . wcat^T) for the rows of SEL / SHARED tiles. Block = one 32-row
// slice of a tile; its 4 waves take every 4th 64-wide k-step (loads of the next step in flight during the MFMAs) and
// their partial sums are added in wave order through LDS.
__global__ __launch_bounds__(256) void lora_ext_kernel(const int4* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
                                                       const int32_t* __restrict__ gkind, const uint16_t* __restrict__ A,
                                                       int64_t lda, int64_t a_rows, int a_gather,
                                                       const int32_t* __restrict__ order, int TK, int topk,
                                                       const uint16_t* __restrict__ wsel, const uint16_t* __restrict__ wsh,
                                                       int Kd, float ssel, float ssh, uint16_t* __restrict__ ext) {
  __shared__ float red[4 * 64 * 16];
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
  f32x16_t acc = f32x16_t{};
  u32x4_t av[4], bv[4], an[4], bn[4];
  auto load = [&](int k0, u32x4_t* x, u32x4_t* y) {
    const int kk = k0 + 32 * hi;
    const bool ok = k0 < Kd && kk + 32 <= Kd;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      x[s] = ld16(ra, ok ? ao + kk * 2 + 16 * s : OOB);
      y[s] = ld16(rb, ok ? bo + kk * 2 + 16 * s : OOB);
    }
  };
  int k0 = 64 * w;
  load(k0, av, bv);
  for (; k0 < Kd; k0 += 256) {
    load(k0 + 256, an, bn);
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = mfma32(av[s], bv[s], acc);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      av[s] = an[s];
      bv[s] = bn[s];
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) red[(w * 64 + l) * 16 + r] = acc[r];
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float v = ((red[l * 16 + r] + red[(64 + l) * 16 + r]) + red[(128 + l) * 16 + r]) + red[(192 + l) * 16 + r];
      const int orow = m * 32 + acc_row(r, l);
      if (orow < nrows) ext[(int64_t)(t.y + orow) * 32 + r32] = f2bf(scale * v);
    }
  }
}

// part[i][c][p][q] = sum over rows c*CH .. c*CH+CH-1 of group lora_groups[i]: alpha(row) L[row][p] Rm[src(row)][q],
// as an MFMA GEMM with the row index as the contraction dim: per 64-row step, L and Rm are staged transposed in LDS
// (k-pair packing: the values of rows 2j and 2j+1 share one 32-bit word), then each wave multiplies the 32 x 64 L^T
// tile by its 64 x 32 slice of the Rm tile. Block = 4 waves = 32 p x 128 q.
constexpr int WG_CH = 1024;   // rows per chunk
constexpr int WG_QB = 128;    // columns per block
constexpr int WG_S = 64 + 8;  // LDS row stride (bf16)

__global__ __launch_bounds__(256) void lora_wgrad_part(const int32_t* __restrict__ groups, const int32_t* __restrict__ offsets,
                                                       int E, int T, int TK, int topk, const int32_t* __restrict__ order,
                                                       const uint16_t* __restrict__ L, const uint16_t* __restrict__ Rm,
                                                       int64_t ldr, int64_t r_rows, int r_gather, int use_w,
                                                       const uint16_t* __restrict__ topv, const float* __restrict__ sgate,
                                                       int Q, float* __restrict__ part, int chunks) {
  __shared__ __attribute__((aligned(16))) uint16_t LT[32 * WG_S];
  __shared__ __attribute__((aligned(16))) uint16_t RT[WG_QB * WG_S];
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
  const rsrc_t rr = make_rsrc(Rm, (uint64_t)r_rows * ldr * 2);
  f32x16_t acc = f32x16_t{};
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
  for (int k0 = a0; k0 < a1; k0 += 64) {
    const int ra = k0 + 2 * kp;
    uint32_t o0, o1;
    float al0, al1;
    row_info(ra, o0, al0);
    row_info(ra + 1, o1, al1);
    // L^T: rows ra, ra+1, p = 4*grp .. 4*grp+3 (alpha folded in, fp32 then one bf16 rounding)
    {
      const uint2 v0 = ra < a1 ? *reinterpret_cast<const uint2*>(L + (int64_t)ra * 32 + 4 * grp) : make_uint2(0, 0);
      const uint2 v1 = ra + 1 < a1 ? *reinterpret_cast<const uint2*>(L + (int64_t)(ra + 1) * 32 + 4 * grp)
                                   : make_uint2(0, 0);
      uint32_t* d = reinterpret_cast<uint32_t*>(LT + (4 * grp) * WG_S + 2 * kp);
      d[0 * (WG_S / 2)] = pack2bf(al0 * bf_lo(v0.x), al1 * bf_lo(v1.x));
      d[1 * (WG_S / 2)] = pack2bf(al0 * bf_hi(v0.x), al1 * bf_hi(v1.x));
      d[2 * (WG_S / 2)] = pack2bf(al0 * bf_lo(v0.y), al1 * bf_lo(v1.y));
      d[3 * (WG_S / 2)] = pack2bf(al0 * bf_hi(v0.y), al1 * bf_hi(v1.y));
    }
    // Rm^T: rows ra, ra+1, q = q0 + 16*grp .. +15
    {
      const int qq = q0 + 16 * grp;
      const bool qok = qq < Q;
      u32x4_t x0[2], x1[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        x0[h] = ld16(rr, qok ? o0 + (uint32_t)(qq + 8 * h) * 2 : OOB);
        x1[h] = ld16(rr, qok ? o1 + (uint32_t)(qq + 8 * h) * 2 : OOB);
      }
      uint32_t* d = reinterpret_cast<uint32_t*>(RT + (16 * grp) * WG_S + 2 * kp);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          d[(8 * h + 2 * j) * (WG_S / 2)] = __builtin_amdgcn_perm(x1[h][j], x0[h][j], 0x05040100u);
          d[(8 * h + 2 * j + 1) * (WG_S / 2)] = __builtin_amdgcn_perm(x1[h][j], x0[h][j], 0x07060302u);
        }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4_t af = *reinterpret_cast<const u32x4_t*>(LT + r32 * WG_S + 32 * hi + 8 * s);
      const u32x4_t bfr = *reinterpret_cast<const u32x4_t*>(RT + (32 * w + r32) * WG_S + 32 * hi + 8 * s);
      acc = mfma32(af, bfr, acc);
    }
    __syncthreads();
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
                              uint16_t* bt_gu, hipStream_t stream) {
  SMEL_REQUIRE(n >= 0 && r > 0 && Hd > 0 && In > 0, SMEL_EINVAL, "lora_prep: bad sizes");
  SMEL_REQUIRE(r <= 16, SMEL_EUNSUPPORTED, "lora_prep: rank %lld > 16", (long long)r);
  if (n == 0) return 0;
  SMEL_REQUIRE(A_gate && B_gate && A_up && B_up && A_down && B_down && fwd_gu && fwd_dn && a_gu && a_dn && bt_dn &&
                   bt_gu, SMEL_EINVAL, "lora_prep: null pointer");
  dim3 grid(256, 6);
  lora_prep_kernel<<<grid, 256, 0, stream>>>(A_gate, B_gate, A_up, B_up, A_down, B_down, (int)n, (int)r, (int)Hd,
                                             (int)In, fwd_gu, fwd_dn, a_gu, a_dn, bt_dn, bt_gu);
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
  lora_ext_kernel<<<grid, 256, 0, stream>>>(reinterpret_cast<const int4*>(tiles), n_tiles, gkind, A_src, lda, a_rows,
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
