// Grouped expert GEMM, backward (acc = A W per group, contraction over the weight's row dim): dA of the down
// projection (fused with the SiLU-gate backward, the d(combine weight) partials and the topv / shared-gate scaling)
// and dX of the gate_up projection. Frozen int4 experts are re-dequantized group by group; the int4 groups run along
// the output columns here, so each 64-row step of the weight is dequantized cooperatively into LDS, transposed to
// k-contiguous bf16 for the MFMA B operand. Reference: FrozenExpertsFn.backward, smel/moe.py:128-143, and the
// autograd of _selected_expert / lora_gate_up / lora_linear / the combine, smel/moe.py:204-252, smel/lora.py:61-83.
//
// Block = 4 waves in a 2 x 2 grid, tile = up to 128 rows x 128 columns, each wave 64 rows (2 slices of 32) x 64
// columns (2 fragments). Per 64-row step of W (one barrier per step):
//  * A rows (gathered by token for the down projection) go global -> LDS by LDS-DMA into a ring of 3 stages,
//    2 steps ahead;
//  * W is read from the fragment layout of smel_pack_int4 / smel_pack_bf16 into registers 3 steps ahead; one step
//    ahead of its use, every thread dequantizes a row pair x 16 columns and writes them transposed (a 32-bit word =
//    the two rows of one column) into one of two W^T buffers [column][k];
//  * vmcnt retires in issue order: each step issues W before A and waits for exactly what the step uses.
#include "abi_util.h"
#include "common.h"

namespace {

constexpr int MT = 128;
constexpr int NT = 128;
constexpr int KT = 64;
constexpr int A_STAGE = MT * KT;   // bf16 elements of one A stage
constexpr int B_STAGE = NT * KT;   // bf16 elements of one W^T buffer: column n at n * KT

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

// Raw W data of one thread for one step, rows (ka, ka+1) x 16 columns: bf16 in v[row][0..1] (8 columns each), or
// int4: v[row][0] = the row's 16-B lane chunk of q (32 columns, this thread's 16 in words 2 hq, 2 hq + 1) and
// v[row][1] = its 16-B chunk of packed scale/zero (this k-step's word at index cks % 4).
struct WRegs {
  u32x4_t v[2][2];
};

template <int EPI, int NSW>
SMEL_DEV void run_tile(const BwdArgs& a, int kind, int idx, int row0, int nrows, int nb, uint16_t* S0, uint16_t* S1,
                       uint16_t* S2, uint16_t* B0, uint16_t* B1) {
  const int tid = threadIdx.x, l = lane_id(), hi = l >> 5, r32 = l & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = w >> 1, wc = w & 1;   // this wave: tile rows [64 wr, +64), columns [64 wc, +64)
  const int n0 = nb * NT;
  const int Kd = a.Kd;
  const smel_wset& ws = a.w;
  const int cw = n0 + wc * 64;         // this wave's first column
  const bool fv0 = cw < a.N, fv1 = cw + 32 < a.N;
  const int nk = (Kd + KT - 1) / KT;
  // ---- W staging role: rows (k0 + 2 kp, +1) x columns [nc, nc + 16)
  const int kp = tid & 31, cc = tid >> 5;
  const int nc = n0 + 16 * cc;
  const bool cok = nc < a.N;
  const int pk = (a.N + 63) / 64, pk4 = (pk + 3) / 4, nfr = Kd / 32;   // packed k-steps run along C here
  const int cks = nc / 64, ch = (nc >> 5) & 1;
  const int lane2 = 32 * ch + (2 * kp) % 32;   // packed lane of row ka (row ka + 1 is the next lane)
  const bool q4 = kind == SMEL_KIND_INT4;   // uniform: the tile's group kind
  const int hq = (nc >> 4) & 1;              // int4: which 8 bytes of the 16-B q chunk are this thread's
  const int zw = cks & 3;                     // int4: word of the packed scale/zero chunk
  rsrc_t rw, rsz;
  uint32_t wbase, sbase, wstep, sstep;
  if (q4) {
    rw = make_rsrc(ws.q4 + (int64_t)idx * nfr * pk * 1024, (uint64_t)nfr * pk * 1024);
    rsz = make_rsrc(ws.sz4 + (int64_t)idx * nfr * pk4 * 256, (uint64_t)nfr * pk4 * 1024);
    wbase = (uint32_t)((cks * 64 + lane2) * 16);
    sbase = (uint32_t)(((cks >> 2) * 64 + lane2) * 16);
    wstep = pk * 1024;
    sstep = pk4 * 1024;
  } else {
    const uint16_t* base = kind == SMEL_KIND_BF16 ? ws.wb : (kind == SMEL_KIND_SEL ? ws.wsel : ws.wsh);
    const int64_t mi = kind == SMEL_KIND_SHARED ? 0 : idx;
    rw = make_rsrc(base + mi * nfr * pk * 2048, (uint64_t)nfr * pk * 4096);
    rsz = rw;
    wbase = (uint32_t)(((cks * 4 + ((nc >> 3) & 3)) * 64 + lane2) * 16);
    sbase = wbase + 1024;   // the next 8 columns
    wstep = sstep = pk * 4096;
  }
  // Four 16-B loads per thread and step for either kind, at addresses chosen above (no branch here: a branch
  // between the two kinds' loads makes the compiler wait for the other branch's loads as well).
  auto issue_w = [&](int j, WRegs& r) {
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t fr = (uint32_t)((j * KT + 2 * kp) / 32);
    const bool ok = cok && j < nk;
    const uint32_t o = fr * wstep + wbase, so = fr * sstep + sbase;
    r.v[0][0] = ld16(rw, ok ? o : OOB);
    r.v[0][1] = ld16(rsz, ok ? so : OOB);
    r.v[1][0] = ld16(rw, ok ? o + 16 : OOB);
    r.v[1][1] = ld16(rsz, ok ? so + 16 : OOB);
  };
  // W^T word of tile column n = 16 cc + c and k pair kp: element n * KT + 8 * ((kp / 4) ^ swz(n)) + 2 * (kp % 4);
  // swz(16 cc + c) = swz(c), a constant per c.
  uint32_t* const wt0 = reinterpret_cast<uint32_t*>(B0) + 16 * cc * (KT / 2) + (kp & 3);
  uint32_t* const wt1 = reinterpret_cast<uint32_t*>(B1) + 16 * cc * (KT / 2) + (kp & 3);
  const int kc = kp >> 2;
  auto store_w = [&](const WRegs& r, uint32_t* wt) {
    uint32_t word[16];
    if (q4) {
      const uint32_t p0 = zw == 0 ? r.v[0][1].x : zw == 1 ? r.v[0][1].y : zw == 2 ? r.v[0][1].z : r.v[0][1].w;
      const uint32_t p1 = zw == 0 ? r.v[1][1].x : zw == 1 ? r.v[1][1].y : zw == 2 ? r.v[1][1].z : r.v[1][1].w;
      const float s0 = bf_lo(p0), z0 = bf_hi(p0), s1 = bf_lo(p1), z1 = bf_hi(p1);
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const uint32_t q0 = hq ? r.v[0][0][2 + d] : r.v[0][0][d], q1 = hq ? r.v[1][0][2 + d] : r.v[1][0][d];
        const uint32_t l0 = q0 & 0x0f0f0f0fu, h0 = (q0 >> 4) & 0x0f0f0f0fu;
        const uint32_t l1 = q1 & 0x0f0f0f0fu, h1 = (q1 >> 4) & 0x0f0f0f0fu;
        uint32_t* o = word + 8 * d;
        o[0] = pack2bf(fmaf(ub0(l0), s0, z0), fmaf(ub0(l1), s1, z1));
        o[1] = pack2bf(fmaf(ub0(h0), s0, z0), fmaf(ub0(h1), s1, z1));
        o[2] = pack2bf(fmaf(ub1(l0), s0, z0), fmaf(ub1(l1), s1, z1));
        o[3] = pack2bf(fmaf(ub1(h0), s0, z0), fmaf(ub1(h1), s1, z1));
        o[4] = pack2bf(fmaf(ub2(l0), s0, z0), fmaf(ub2(l1), s1, z1));
        o[5] = pack2bf(fmaf(ub2(h0), s0, z0), fmaf(ub2(h1), s1, z1));
        o[6] = pack2bf(fmaf(ub3(l0), s0, z0), fmaf(ub3(l1), s1, z1));
        o[7] = pack2bf(fmaf(ub3(h0), s0, z0), fmaf(ub3(h1), s1, z1));
      }
    } else {
#pragma unroll
      for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t x0 = r.v[0][d][j], x1 = r.v[1][d][j];
          word[8 * d + 2 * j] = __builtin_amdgcn_perm(x1, x0, 0x05040100u);
          word[8 * d + 2 * j + 1] = __builtin_amdgcn_perm(x1, x0, 0x07060302u);
        }
    }
#pragma unroll
    for (int c = 0; c < 16; ++c) wt[c * (KT / 2) + 4 * (kc ^ swz(c))] = word[c];
  };
  // ---- A staging (as the forward kernel): wave-load ii of wave w fills rows 8 g .. 8 g + 7, g = 4 w + ii
  const rsrc_t ra = make_rsrc(a.A, (uint64_t)a.a_rows * a.lda * 2);
  const int li = tid & 63;
  uint32_t aoff[4];
  int akc[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const int g = 4 * w + ii;
    const int row = 8 * g + (li >> 3);
    const int c = (li & 7) ^ swz(row);
    akc[ii] = 8 * c;
    aoff[ii] = OOB;
    if (row < nrows) {
      const int grow = row0 + row;
      const int src = a.a_gather ? row_token(grow, a.order, a.TK, a.topk) : grow;
      aoff[ii] = (uint32_t)src * (uint32_t)a.lda * 2 + 16 * c;
    }
  }
  auto issue_a = [&](int j, uint16_t* S) {
    const int k0 = j * KT;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
      ld16_lds(ra, S + (4 * w + ii) * 512, (k0 + akc[ii] + 8 <= Kd) ? aoff[ii] + k0 * 2 : OOB);
    __builtin_amdgcn_sched_barrier(0);
  };
  // fragment reads: A row 64 wr + 32 m + r32, W^T column 64 wc + 32 f + r32, logical chunk 4 h + s
  uint32_t frd[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) frd[s] = r32 * KT + 8 * ((4 * hi + s) ^ swz(r32));
  const int abase = 64 * wr * KT, bbase = 64 * wc * KT;

  f32x16_t acc[NSW > 0 ? NSW : 1][2];
#pragma unroll
  for (int m = 0; m < (NSW > 0 ? NSW : 1); ++m) acc[m][0] = acc[m][1] = f32x16_t{};

  auto compute = [&](const uint16_t* Sa, const uint16_t* Bt) {
    if constexpr (NSW > 0) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4_t b0 = *reinterpret_cast<const u32x4_t*>(Bt + bbase + frd[s]);
        const u32x4_t b1 = *reinterpret_cast<const u32x4_t*>(Bt + bbase + 32 * KT + frd[s]);
#pragma unroll
        for (int m = 0; m < NSW; ++m) {
          const u32x4_t af = *reinterpret_cast<const u32x4_t*>(Sa + abase + m * 32 * KT + frd[s]);
          acc[m][0] = mfma32(af, b0, acc[m][0]);
          acc[m][1] = mfma32(af, b1, acc[m][1]);
        }
      }
    }
  };

  // Ring positions of step j: A stage j % 3 (loaded 2 steps ahead), W^T buffer j % 2 (W(j+1) is dequantized into
  // the other one during step j), W register set (j+1) % 6 dequantized and set (j+5) % 6 refilled (4 steps ahead).
  WRegs w0, w1, w2, w3, w4, w5;
  issue_w(0, w0);
  issue_w(1, w1);
  issue_w(2, w2);
  issue_w(3, w3);
  issue_a(0, S0);
  issue_w(4, w4);
  issue_a(1, S1);
  store_w(w0, wt0);
  auto step = [&](int j, uint16_t* Sa, uint16_t* Sa2, const uint16_t* Bc, uint32_t* wtn, const WRegs& wuse,
                  WRegs& wiss) {
    SMEL_WAIT_VM_LDS(8);   // A(j) and W(j+1) have landed: only step j-1's group may still be in flight
    __builtin_amdgcn_s_barrier();
    issue_w(j + 5, wiss);
    issue_a(j + 2, Sa2);
    store_w(wuse, wtn);    // W(j+1) -> the other W^T buffer
    compute(Sa, Bc);
  };
  // whole rounds of 6 steps without exits (so the loop header keeps the waits above), then the remaining steps
  int i = 0;
  for (; i + 6 <= nk; i += 6) {
    step(i, S0, S2, B0, wt1, w1, w5);
    step(i + 1, S1, S0, B1, wt0, w2, w0);
    step(i + 2, S2, S1, B0, wt1, w3, w1);
    step(i + 3, S0, S2, B1, wt0, w4, w2);
    step(i + 4, S1, S0, B0, wt1, w5, w3);
    step(i + 5, S2, S1, B1, wt0, w0, w4);
  }
  if (i < nk) {
    step(i, S0, S2, B0, wt1, w1, w5);
    if (i + 1 < nk) {
      step(i + 1, S1, S0, B1, wt0, w2, w0);
      if (i + 2 < nk) {
        step(i + 2, S2, S1, B0, wt1, w3, w1);
        if (i + 3 < nk) {
          step(i + 3, S0, S2, B1, wt0, w4, w2);
          if (i + 4 < nk) step(i + 4, S1, S0, B0, wt1, w5, w3);
        }
      }
    }
  }
  SMEL_WAIT_VM_LDS(0);
  __builtin_amdgcn_s_barrier();   // every wave is done with the ring: its LDS is reused below
  // ---- LoRA K-extension: ext[row][0:32] . Eb[0:32][n]
  const uint16_t* eb = kind == SMEL_KIND_SEL ? (ws.ext_sel ? ws.ext_sel + (int64_t)idx * 32 * a.N : nullptr)
                                             : (kind == SMEL_KIND_SHARED ? ws.ext_sh : nullptr);
  if (NSW > 0 && a.ext && eb) {
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
    for (int m = 0; m < (NSW > 0 ? NSW : 1); ++m) {
      const int row = 64 * wr + m * 32 + r32;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const u32x4_t af = ld16(rx, row < nrows ? (uint32_t)row * 64 + 32 * hi + 16 * s : OOB);
        acc[m][0] = mfma32(af, b0[s], acc[m][0]);
        acc[m][1] = mfma32(af, b1[s], acc[m][1]);
      }
    }
  }
  // ---- epilogue through LDS (the ring is free: see the barrier above): the wave results go into a row-major tile,
  // then each thread handles 8 columns of whole rows with 16-B accesses (one address per 8 outputs).
  const int ech = tid & 15;                // 8-column chunk of the block's 128 columns
  const int col0 = n0 + 8 * ech;
  if (EPI == 0) {
    // bf16 tile [128][128]: rows 0..63 in S0, 64..127 in S1; 16-B chunk c of row r at c ^ (r & 7)
#pragma unroll
    for (int m = 0; m < NSW; ++m) {
      uint16_t* D = wr == 0 ? S0 : S1;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lr = m * 32 + acc_row(r, l);   // row inside this wave's 64-row half
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          const int col = 64 * wc + 32 * f + r32;
          D[lr * 128 + 8 * ((col >> 3) ^ (lr & 7)) + (col & 7)] = f2bf(acc[m][f][r]);
        }
      }
    }
    __syncthreads();
    if (col0 < a.N) {
      for (int row = tid >> 4; row < nrows; row += 16) {
        const int lr = row & 63;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>((row < 64 ? S0 : S1) + lr * 128 + 8 * (ech ^ (lr & 7)));
        const int64_t orow = row_slot(row0 + row, a.order, a.TK);
        *reinterpret_cast<u32x4_t*>(a.out + orow * a.ldo + col0) = v;
      }
    }
    return;
  }
  // down backward, columns n < I of dh = [dg | du]: fp32 tile [128][128], 32 rows per array (S0, S1, S2, B0); 16-B
  // chunk c (4 floats) of row r at c ^ (r & 7). Then per row: da = w(row) acc, (g, u) = hsave, dg = da u act'(g),
  // du = da act(g), and the row's partial of sum_n acc * bf16(act(g) u) over this block's columns -> dwp.
  float* const Fa[4] = {reinterpret_cast<float*>(S0), reinterpret_cast<float*>(S1), reinterpret_cast<float*>(S2),
                        reinterpret_cast<float*>(B0)};
#pragma unroll
  for (int m = 0; m < NSW; ++m) {
    float* D = wr == 0 ? Fa[m] : Fa[2 + m];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int lr = acc_row(r, l);
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const int col = 64 * wc + 32 * f + r32;
        D[lr * 128 + 4 * ((col >> 2) ^ (lr & 7)) + (col & 3)] = acc[m][f][r];
      }
    }
  }
  __syncthreads();
  const int I = a.N;
  const bool cv = col0 < I;
  for (int row = tid >> 4; row < nrows; row += 16) {   // 16 threads per row, uniform trip count per row group
    const int lr = row & 31;
    const int q = row >> 5;   // a select, not an indexed local array (which would live in scratch memory)
    const float* D = (q == 0 ? Fa[0] : q == 1 ? Fa[1] : q == 2 ? Fa[2] : Fa[3]) + lr * 128;
    const f32x4_t x0 = *reinterpret_cast<const f32x4_t*>(D + 4 * ((2 * ech) ^ (lr & 7)));
    const f32x4_t x1 = *reinterpret_cast<const f32x4_t*>(D + 4 * ((2 * ech + 1) ^ (lr & 7)));
    const int grow = row0 + row;
    const float wrow_ = grow < a.TK ? bf2f(a.topv[a.order[grow]]) : a.sgate[grow - a.TK];
    float part = 0.f;
    if (cv) {
      const u32x4_t g2 = *reinterpret_cast<const u32x4_t*>(a.hsave + (int64_t)grow * 2 * I + col0);
      const u32x4_t u2 = *reinterpret_cast<const u32x4_t*>(a.hsave + (int64_t)grow * 2 * I + I + col0);
      const float accv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      uint32_t og[4], ou[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float dgv[2], duv[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float g = h ? bf_hi(g2[j]) : bf_lo(g2[j]);
          const float u = h ? bf_hi(u2[j]) : bf_lo(u2[j]);
          float av, dav;
          act_and_grad_f(g, a.act, av, dav);
          const float abf = bf2f(f2bf(act_f(g, a.act) * u));   // the forward's rounded activation
          const float acv = accv[2 * j + h];
          part += acv * abf;
          const float da = wrow_ * acv;
          dgv[h] = da * u * dav;
          duv[h] = da * av;
        }
        og[j] = pack2bf(dgv[0], dgv[1]);
        ou[j] = pack2bf(duv[0], duv[1]);
      }
      *reinterpret_cast<u32x4_t*>(a.out + (int64_t)grow * a.ldo + col0) = u32x4_t{og[0], og[1], og[2], og[3]};
      *reinterpret_cast<u32x4_t*>(a.out + (int64_t)grow * a.ldo + I + col0) = u32x4_t{ou[0], ou[1], ou[2], ou[3]};
    }
    // fixed-order sum over the row's 16 threads (lanes 16 q .. 16 q + 15 of a wave)
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) part += __shfl_xor(part, o, 64);
    if (ech == 0) a.dwp[(int64_t)grow * a.nblk + nb] = part;
  }
}

template <int EPI>
SMEL_DEV void run_tile_ns(const BwdArgs& a, int kind, int idx, int row0, int nrows, int nb, uint16_t* S0,
                          uint16_t* S1, uint16_t* S2, uint16_t* B0, uint16_t* B1) {
  // slices of 32 rows this wave computes (its 64-row half of the tile); every wave stages and syncs alike
  const int wr = __builtin_amdgcn_readfirstlane(threadIdx.x >> 7);
  const int nsw = min(2, max(0, (nrows - 64 * wr + 31) >> 5));
  switch (nsw) {
    case 0: run_tile<EPI, 0>(a, kind, idx, row0, nrows, nb, S0, S1, S2, B0, B1); break;
    case 1: run_tile<EPI, 1>(a, kind, idx, row0, nrows, nb, S0, S1, S2, B0, B1); break;
    default: run_tile<EPI, 2>(a, kind, idx, row0, nrows, nb, S0, S1, S2, B0, B1); break;
  }
}

template <int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gmm_bwd_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(1024))) uint16_t S0[A_STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t S1[A_STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t S2[A_STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t B0[B_STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t B1[B_STAGE];
  int tile, nb;
  if (!xcd_tile(a.n_tiles[0], a.nblk, tile, nb)) return;
  const int4 t = a.tiles[tile];
  const int gk = a.gkind[t.x];
  const int kind = gk >> 16, idx = gk & 0xffff;
  const int nrows = min(t.z - t.y, MT);
  if (nrows <= 0) return;
  run_tile_ns<EPI>(a, kind, idx, t.y, nrows, nb, S0, S1, S2, B0, B1);
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
  SMEL_REQUIRE(ldo % 8 == 0 && ((uintptr_t)out % 16) == 0 && ((uintptr_t)hsave % 16) == 0, SMEL_EUNSUPPORTED,
               "gmm_bwd: out / hsave rows must be 16-B aligned");
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
