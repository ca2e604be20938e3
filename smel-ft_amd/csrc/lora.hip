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

// ext[row][0:32] = bf16(scale * A_src[src(row)] . wcat^T) for the rows of SEL / SHARED tiles. Wave m = slice m.
__global__ __launch_bounds__(256) void lora_ext_kernel(const int4* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
                                                       const int32_t* __restrict__ gkind, const uint16_t* __restrict__ A,
                                                       int64_t lda, int a_gather, const int32_t* __restrict__ order,
                                                       int TK, int topk, const uint16_t* __restrict__ wsel,
                                                       const uint16_t* __restrict__ wsh, int Kd, float ssel, float ssh,
                                                       uint16_t* __restrict__ ext) {
  if ((int)blockIdx.x >= n_tiles[0]) return;
  const int4 t = tiles[blockIdx.x];
  const int gk = gkind[t.x];
  const int kind = gk >> 16, idx = gk & 0xffff;
  if (kind != SMEL_KIND_SEL && kind != SMEL_KIND_SHARED) return;
  const int l = lane_id(), m = threadIdx.x >> 6, hi = l >> 5, r32 = l & 31;
  const int nrows = t.z - t.y;
  if (m * 32 >= nrows) return;
  const uint16_t* wc = kind == SMEL_KIND_SEL ? (wsel ? wsel + (int64_t)idx * 32 * Kd : nullptr) : wsh;
  if (!wc) return;   // this group has no LoRA
  const float scale = kind == SMEL_KIND_SEL ? ssel : ssh;
  const int row = m * 32 + r32;
  const uint16_t* arow = nullptr;
  if (row < nrows) {
    const int grow = t.y + row;
    arow = A + (int64_t)(a_gather ? row_token(grow, order, TK, topk) : grow) * lda;
  }
  const uint16_t* brow = wc + (int64_t)r32 * Kd;
  f32x16_t acc = f32x16_t{};
  for (int k0 = 0; k0 < Kd; k0 += 64) {
    const int kk = k0 + 32 * hi;
    const bool ok = kk + 32 <= Kd;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4_t a = (ok && arow) ? *reinterpret_cast<const u32x4_t*>(arow + kk + 8 * s) : u32x4_t{};
      const u32x4_t b = ok ? *reinterpret_cast<const u32x4_t*>(brow + kk + 8 * s) : u32x4_t{};
      acc = mfma32(a, b, acc);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int orow = m * 32 + acc_row(r, l);
    if (orow < nrows) ext[(int64_t)(t.y + orow) * 32 + r32] = f2bf(scale * acc[r]);
  }
}

// part[i][c][p][q] = sum over rows c*256 .. c*256+255 of group lora_groups[i]: alpha(row) L[row][p] Rm[src(row)][q].
// Thread = (column q of a 64-wide block, 8 of the 32 p).
__global__ __launch_bounds__(256) void lora_wgrad_part(const int32_t* __restrict__ groups, const int32_t* __restrict__ offsets,
                                                       int E, int T, int TK, int topk, const int32_t* __restrict__ order,
                                                       const uint16_t* __restrict__ L, const uint16_t* __restrict__ Rm,
                                                       int64_t ldr, int r_gather, int use_w,
                                                       const uint16_t* __restrict__ topv, const float* __restrict__ sgate,
                                                       int Q, float* __restrict__ part, int chunks) {
  const int i = blockIdx.x, c = blockIdx.y;
  const int g = groups[i];
  const int r0 = g < E ? offsets[g] : TK;
  const int r1 = g < E ? offsets[g + 1] : TK + T;
  const int a0 = r0 + c * 256;
  if (a0 >= r1) return;
  const int a1 = min(r1, a0 + 256);
  const int q = blockIdx.z * 64 + (threadIdx.x & 63);
  if (q >= Q) return;
  const int pb = (threadIdx.x >> 6) * 8;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int row = a0; row < a1; ++row) {
    float alpha = 1.f;
    int src = row;
    if (r_gather || use_w) {
      if (row < TK) {
        const int p = order[row];
        if (r_gather) src = p / topk;
        if (use_w) alpha = bf2f(topv[p]);
      } else {
        if (r_gather) src = row - TK;
        if (use_w) alpha = sgate[row - TK];
      }
    }
    const float rv = alpha * bf2f(Rm[(int64_t)src * ldr + q]);
    const u32x4_t lv = *reinterpret_cast<const u32x4_t*>(L + (int64_t)row * 32 + pb);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] = fmaf(bf_lo(lv[j]), rv, acc[2 * j]);
      acc[2 * j + 1] = fmaf(bf_hi(lv[j]), rv, acc[2 * j + 1]);
    }
  }
  float* dst = part + (((int64_t)i * chunks + c) * 32 + pb) * Q + q;
#pragma unroll
  for (int j = 0; j < 8; ++j) dst[(int64_t)j * Q] = acc[j];
}

__global__ __launch_bounds__(256) void lora_wgrad_sum(const int32_t* __restrict__ groups,
                                                      const int32_t* __restrict__ offsets, int E, int T, int TK,
                                                      int Q, const float* __restrict__ part, int chunks,
                                                      float* __restrict__ out) {
  const int i = blockIdx.y;
  const int g = groups[i];
  const int rows = g < E ? offsets[g + 1] - offsets[g] : T;
  const int nch = min((rows + 255) / 256, chunks);
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
                             const uint16_t* A_src, int64_t lda, int32_t a_gather, const int32_t* order, int64_t TK,
                             int64_t topk, const uint16_t* wcat_sel, const uint16_t* wcat_sh, int64_t Kd,
                             float scale_sel, float scale_sh, uint16_t* ext, hipStream_t stream) {
  SMEL_REQUIRE(tiles && n_tiles && gkind && A_src && ext, SMEL_EINVAL, "lora_ext: null pointer");
  SMEL_REQUIRE(Kd > 0 && Kd % 32 == 0, SMEL_EUNSUPPORTED, "lora_ext: K %lld must be a multiple of 32", (long long)Kd);
  SMEL_REQUIRE(lda % 8 == 0 && ((uintptr_t)A_src % 16) == 0, SMEL_EUNSUPPORTED, "lora_ext: A rows must be 16-B aligned");
  SMEL_REQUIRE(!a_gather || order || TK == 0, SMEL_EINVAL, "lora_ext: gather needs order");
  if (max_tiles == 0) return 0;
  lora_ext_kernel<<<(unsigned)max_tiles, 256, 0, stream>>>(reinterpret_cast<const int4*>(tiles), n_tiles, gkind, A_src,
                                                            lda, a_gather, order, (int)TK, (int)topk, wcat_sel,
                                                            wcat_sh, (int)Kd, scale_sel, scale_sh, ext);
  return smel::launch_status();
}

extern "C" int64_t smel_lora_wgrad_part_chunks(int64_t max_group_rows) { return (max_group_rows + 255) / 256; }

extern "C" int smel_lora_wgrad(const int32_t* lora_groups, int64_t n_lora, const int32_t* offsets, int64_t E,
                               int64_t T, int64_t TK, int64_t topk, const int32_t* order, const uint16_t* L,
                               const uint16_t* Rm, int64_t ldr, int32_t r_gather, int32_t use_w,
                               const uint16_t* topv, const float* sgate, int64_t Q, float* part,
                               int64_t part_chunks, float* out, hipStream_t stream) {
  SMEL_REQUIRE(n_lora >= 0 && Q > 0 && part_chunks >= 0, SMEL_EINVAL, "lora_wgrad: bad sizes");
  if (n_lora == 0 || part_chunks == 0) return 0;
  SMEL_REQUIRE(lora_groups && offsets && L && Rm && part && out, SMEL_EINVAL, "lora_wgrad: null pointer");
  SMEL_REQUIRE(!(r_gather || use_w) || order || TK == 0, SMEL_EINVAL, "lora_wgrad: needs order");
  dim3 g1((unsigned)n_lora, (unsigned)part_chunks, (unsigned)((Q + 63) / 64));
  lora_wgrad_part<<<g1, 256, 0, stream>>>(lora_groups, offsets, (int)E, (int)T, (int)TK, (int)topk, order, L, Rm, ldr,
                                          r_gather, use_w, topv, sgate, (int)Q, part, (int)part_chunks);
  int st = smel::launch_status();
  if (st) return st;
  dim3 g2((unsigned)std::min<int64_t>((32 * Q + 255) / 256, 1024), (unsigned)n_lora);
  lora_wgrad_sum<<<g2, 256, 0, stream>>>(lora_groups, offsets, (int)E, (int)T, (int)TK, (int)Q, part,
                                         (int)part_chunks, out);
  return smel::launch_status();
}
