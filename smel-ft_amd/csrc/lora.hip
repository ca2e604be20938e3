// LoRA pieces of the selected experts and the shared MLP (smel/lora.py:14-83): layout of the fp32 factors into the
// bf16 K-extension operands, the rank-32 down-projections of LoRA rows (x A^T, act A_d^T, dy B_d, dh B^T) and the
// factor gradients as fixed-order row reductions.
#include "abi_util.h"
#include "common.h"

namespace {

constexpr int PREP_MAX_SETS = 2;
constexpr int PCH = 128;   // columns (A factors) or rows (B factors) of one chunk
// block kinds: the A factors of gate / up (over Hd), A_down (over In), the B factors of gate / up (rows of In),
// B_down (rows of Hd)
enum { PK_AGU = 0, PK_ADN = 1, PK_BGU = 2, PK_BDN = 3, PK_N = 4 };
struct PrepArgs {
  smel_lora_set set[PREP_MAX_SETS];
  int first[PREP_MAX_SETS * PK_N + 1];   // first block of each (set, kind), then the total
  int planes, Hd, In;
};

// One block = one chunk of PCH columns (A factors) or rows (B factors) of one expert's fp32 factor(s). The chunk goes
// to LDS as [factor][rank][column] in one round of coalesced loads (every load issued before the first is used); the
// block then writes every layout that draws on it, the plain and the transposed one, two bf16 per 32-bit store with
// consecutive threads on consecutive words.
__global__ __launch_bounds__(256) void lora_prep_kernel(PrepArgs pa) {
  __shared__ float sa[2][32][PCH + 1];   // odd row length: the transposed reads and writes are conflict free
  const int tid = threadIdx.x, bid = blockIdx.x;
  int si = 0;
#pragma unroll
  for (int i = 1; i < PREP_MAX_SETS * PK_N; ++i)
    if (bid >= pa.first[i]) si = i;
  const smel_lora_set& S = pa.set[si / PK_N];
  const int kind = si % PK_N;
  const int n = (int)S.n, R = (int)S.r, P = pa.planes, Hd = pa.Hd, In = pa.In;
  const int X = (kind == PK_AGU || kind == PK_BDN) ? Hd : In;   // the dimension the chunks run over
  const int nch = (X + PCH - 1) / PCH;
  const int loc = bid - pa.first[si], g = loc / nch, x0 = (loc % nch) * PCH, w = min(PCH, X - x0);
  const int nf = (kind == PK_AGU || kind == PK_BGU) ? 2 : 1;   // factors in the chunk (gate and up)
  // gate_up side: with one plane, gate ranks sit at 0..r-1 and up ranks at 16..16+r-1 of it; with two planes, each
  // projection has its own plane and its ranks at 0..r-1. (plane, j) -> rank of gate / up, or -1.
  auto gate_rank = [&](int plane, int j) -> int { return (plane == 0 && j < R) ? j : -1; };
  auto up_rank = [&](int plane, int j) -> int {
    if (P == 1) return (j >= 16 && j < 16 + R) ? j - 16 : -1;
    return (plane == 1 && j < R) ? j : -1;
  };
  // ---- load, 16 B per lane: A factors [n][R][X] as (factor, rank, 4 columns) items, B factors [n][X][R] as the
  // chunk's w * R contiguous floats per factor; into sa[f][k][c]
  {
    const bool isA = kind == PK_AGU || kind == PK_ADN;
    const float* f0 = kind == PK_AGU ? S.A_gate : kind == PK_ADN ? S.A_down : kind == PK_BGU ? S.B_gate : S.B_down;
    const float* f1 = kind == PK_AGU ? S.A_up : S.B_up;
    constexpr int NI = 2 * 32 * PCH / 4 / 256;   // 16-B items per thread
    f32x4_t v[NI];
#pragma unroll
    for (int u = 0; u < NI; ++u) {
      const int q = u * 256 + tid, f = q / (8 * PCH), e = q % (8 * PCH);   // e: item inside one factor's chunk
      const float* src = f ? f1 : f0;
      bool ok;
      int64_t off;
      if (isA) {   // e = (rank k, 4-column group)
        const int k = e / (PCH / 4), c = 4 * (e % (PCH / 4));
        ok = f < nf && k < R && c < w;
        off = ((int64_t)g * R + k) * X + x0 + c;
      } else {     // e = float quad of the chunk's rows
        ok = f < nf && 4 * e < w * R;
        off = ((int64_t)g * X + x0) * R + 4 * e;
      }
      v[u] = ok ? *reinterpret_cast<const f32x4_t*>(src + off) : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    // B chunks hold ranks past R in no float: their slots must read 0
    if (!isA)
      for (int q = tid; q < 2 * 32 * PCH; q += 256) sa[q / (32 * PCH)][(q / PCH) % 32][q % PCH] = 0.f;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NI; ++u) {
      const int q = u * 256 + tid, f = q / (8 * PCH), e = q % (8 * PCH);
      if (isA) {
        const int k = e / (PCH / 4), c = 4 * (e % (PCH / 4));
#pragma unroll
        for (int t = 0; t < 4; ++t) sa[f][k][c + t] = v[u][t];
      } else if (4 * e < w * R) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int x = 4 * e + t;   // float x of the chunk = row x / R, rank x % R
          sa[f][x % R][x / R] = v[u][t];
        }
      }
    }
  }
  __syncthreads();
  // slot j of plane `plane` of the gate_up layouts: the gate or up factor's value at chunk column c, or 0
  auto gu = [&](int plane, int j, int c) -> float {
    const int kg = gate_rank(plane, j), ku = up_rank(plane, j);
    return kg >= 0 ? sa[0][kg][c] : (ku >= 0 ? sa[1][ku][c] : 0.f);
  };
  auto one = [&](int j, int c) -> float { return j < R ? sa[0][j][c] : 0.f; };
  // 16-B stores of 8 bf16. [..][X] rows (32 slots per plane): item (plane, slot j, 8 columns); [X][32] rows: item
  // (plane, column, 8 slots)
  auto pack8 = [&](float a0, float a1, float a2, float a3, float a4, float a5, float a6, float a7) {
    return u32x4_t{pack2bf(a0, a1), pack2bf(a2, a3), pack2bf(a4, a5), pack2bf(a6, a7)};
  };
  auto rows_along_x = [&](uint16_t* dst, int planes_, int64_t plane_stride, int64_t row0, int ldx, auto value) {
    for (int q = tid; q < planes_ * 32 * (PCH / 8); q += 256) {
      const int c = 8 * (q % (PCH / 8)), j = (q / (PCH / 8)) % 32, pl = q / (32 * (PCH / 8));
      if (c < w)
        *reinterpret_cast<u32x4_t*>(dst + pl * plane_stride + (row0 + j) * (int64_t)ldx + x0 + c) =
            pack8(value(pl, j, c), value(pl, j, c + 1), value(pl, j, c + 2), value(pl, j, c + 3), value(pl, j, c + 4),
                  value(pl, j, c + 5), value(pl, j, c + 6), value(pl, j, c + 7));
    }
  };
  auto slots_along_row = [&](uint16_t* dst, int planes_, int64_t plane_stride, int64_t xrow0, auto value) {
    for (int q = tid; q < planes_ * PCH * 4; q += 256) {
      const int j = 8 * (q % 4), c = (q / 4) % PCH, pl = q / (PCH * 4);
      if (c < w)
        *reinterpret_cast<u32x4_t*>(dst + pl * plane_stride + (xrow0 + x0 + c) * 32 + j) =
            pack8(value(pl, j, c), value(pl, j + 1, c), value(pl, j + 2, c), value(pl, j + 3, c), value(pl, j + 4, c),
                  value(pl, j + 5, c), value(pl, j + 6, c), value(pl, j + 7, c));
    }
  };
  switch (kind) {
    case PK_AGU:
      // a_gu [planes][n][32][Hd] and at_gu [n][planes][Hd][32]
      rows_along_x(S.a_gu, P, (int64_t)n * 32 * Hd, (int64_t)g * 32, Hd,
                   [&](int pl, int j, int c) { return gu(pl, j, c); });
      slots_along_row(S.at_gu, P, (int64_t)Hd * 32, (int64_t)g * P * Hd,
                      [&](int pl, int j, int c) { return gu(pl, j, c); });
      break;
    case PK_ADN:
      // a_dn [n][32][In] and at_dn [n][In][32]
      rows_along_x(S.a_dn, 1, 0, (int64_t)g * 32, In, [&](int, int j, int c) { return one(j, c); });
      slots_along_row(S.at_dn, 1, 0, (int64_t)g * In, [&](int, int j, int c) { return one(j, c); });
      break;
    case PK_BGU:
      // fwd_gu [n][2In][32]: gate rows < In (ranks at slots 0..r-1), up rows >= In (plane 1 with two planes, else
      // the up slots of the one plane); bt_gu [planes][n][32][2In]: gate columns < In, up columns >= In
      slots_along_row(S.fwd_gu, 2, (int64_t)In * 32, (int64_t)g * 2 * In, [&](int half, int j, int c) {
        if (!half) return one(j, c);
        const int k = up_rank(P - 1, j);
        return k >= 0 ? sa[1][k][c] : 0.f;
      });
      for (int half = 0; half < 2; ++half)
        rows_along_x(S.bt_gu + half * In, P, (int64_t)n * 32 * 2 * In, (int64_t)g * 32, 2 * In, [&](int pl, int j, int c) {
          const int k = half ? up_rank(pl, j) : gate_rank(pl, j);
          return k >= 0 ? sa[half][k][c] : 0.f;
        });
      break;
    default:
      // fwd_dn [n][Hd][32] and bt_dn [n][32][Hd]
      slots_along_row(S.fwd_dn, 1, 0, (int64_t)g * Hd, [&](int, int j, int c) { return one(j, c); });
      rows_along_x(S.bt_dn, 1, 0, (int64_t)g * 32, Hd, [&](int, int j, int c) { return one(j, c); });
      break;
  }
}

// ext[row * ldx + 0:32] = bf16(scale * A_src[src(row)] . wcat^T) for the rows of SEL / SHARED tiles (one 32-wide
// plane per call). Persistent: one block per CU first builds, in LDS, the list of this call's tiles that carry a LoRA
// (the tile list holds each tile's kind; all tile entries are loaded at once, one memory latency), then takes the
// (LoRA tile, 32-row slice) items blockIdx.x, blockIdx.x + gridDim.x, ... A slice's 8 waves take the 64-wide k-steps
// j = w, w + 8, ..., issuing all loads of up to XPRE of their steps before the MFMAs (one memory latency per XPRE
// steps, not one per step); the partial sums are added in wave order through LDS. The 16x16x32 MFMA layout lets four
// lanes share a row, so each load takes 64 contiguous bytes of 16 rows (32 bytes of 32 rows with 32x32x16).
SMEL_DEV f32x4_t mfma16x(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}
constexpr int XW = 8;
constexpr int XPRE = 4;
constexpr int XT_PER = 8;              // tile entries each thread scans
constexpr int XLT = 512 * XT_PER;      // tiles one call may hold

__global__ __launch_bounds__(512) void lora_ext_kernel(const int4* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
                                                       const int32_t* __restrict__ gkind, const uint16_t* __restrict__ A,
                                                       int64_t lda, int64_t a_rows, int a_gather,
                                                       const int32_t* __restrict__ order, int TK, int topk,
                                                       const uint16_t* __restrict__ wsel, const uint16_t* __restrict__ wsh,
                                                       int Kd, float ssel, float ssh, uint16_t* __restrict__ ext,
                                                       int ldx, int max_tiles) {
  __shared__ float red[XW * 64 * 16];
  __shared__ int4 lt[XLT];   // the call's LoRA tiles (whole entries: no second load per item)
  __shared__ int wcnt[XT_PER][XW];
  const int tid = threadIdx.x, l = lane_id(), w = tid >> 6, kq = l >> 4, li = l & 15;
  // ---- the LoRA tiles of this call, in tile order
  const int nt = min(n_tiles[0], max_tiles);
  bool fl[XT_PER];
  int4 te[XT_PER];
#pragma unroll
  for (int p = 0; p < XT_PER; ++p) {
    const int i = p * 512 + tid;
    fl[p] = false;
    te[p] = int4{0, 0, 0, 0};
    if (i < nt) {
      int4 t = tiles[i];
      if (gkind) t.w = gkind[t.x];   // the group kind, in the entry's fourth field from here on
      const int kind = t.w >> 16;
      fl[p] = (kind == SMEL_KIND_SEL && wsel) || (kind == SMEL_KIND_SHARED && wsh);
      te[p] = t;
    }
  }
  uint64_t msk[XT_PER];
#pragma unroll
  for (int p = 0; p < XT_PER; ++p) {
    msk[p] = __ballot(fl[p]);
    if (l == 0) wcnt[p][w] = __popcll(msk[p]);
  }
  __syncthreads();
  int total = 0;
#pragma unroll
  for (int p = 0; p < XT_PER; ++p) {
    int off = total;
#pragma unroll
    for (int v = 0; v < XW; ++v) {
      off += v < w ? wcnt[p][v] : 0;
      total += wcnt[p][v];
    }
    if (fl[p]) lt[off + __popcll(msk[p] & ((1ull << l) - 1ull))] = te[p];
  }
  __syncthreads();
  // ---- (tile, slice) items
  const rsrc_t ra = make_rsrc(A, (uint64_t)a_rows * lda * 2);
  const int nk = (Kd + 63) / 64;
  for (int item = blockIdx.x; item < 4 * total; item += gridDim.x) {
    const int4 t = lt[item >> 2];
    const int kind = t.w >> 16, idx = t.w & 0xffff;
    const int m = item & 3;
    const int nrows = min(t.z - t.y, 128);
    if (m * 32 >= nrows) continue;   // uniform over the block
    const uint16_t* wc = kind == SMEL_KIND_SEL ? wsel + (int64_t)idx * 32 * Kd : wsh;
    const float scale = kind == SMEL_KIND_SEL ? ssel : ssh;
    // v_mfma_f32_16x16x32_bf16: lane (kq, i) holds row 16 fr + i of the slice and factor row 16 fc + i, k = 32 s +
    // 8 kq + [0, 8) of each 64-wide step, so a load takes 64 contiguous bytes of 16 rows (4 lanes per row)
    const rsrc_t rb = make_rsrc(wc, (uint64_t)32 * Kd * 2);
    uint32_t ao[2], bo[2];
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const int row = m * 32 + 16 * f + li;
      ao[f] = OOB;
      if (row < nrows) {
        const int grow = t.y + row;
        ao[f] = (uint32_t)(a_gather ? row_token(grow, order, TK, topk) : grow) * (uint32_t)lda * 2 + 16 * kq;
      }
      bo[f] = (uint32_t)(16 * f + li) * Kd * 2 + 16 * kq;
    }
    f32x4_t acc[2][2];
#pragma unroll
    for (int f = 0; f < 2; ++f) acc[f][0] = acc[f][1] = f32x4_t{};
    for (int j0 = w; j0 < nk; j0 += XW * XPRE) {
      u32x4_t av[XPRE][2][2], bv[XPRE][2][2];   // [step][fragment][substep]
      // the factor rows first: they do not wait for the row's token (a gathered row's address does)
#pragma unroll
      for (int p = 0; p < XPRE; ++p)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int kk = (j0 + XW * p) * 64 + 32 * s2;
          const bool ok = kk + 32 <= Kd;   // Kd % 32 == 0: a 32-wide substep is all in or all out
#pragma unroll
          for (int f = 0; f < 2; ++f) bv[p][f][s2] = ld16(rb, ok ? bo[f] + kk * 2 : OOB);
        }
#pragma unroll
      for (int p = 0; p < XPRE; ++p)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int kk = (j0 + XW * p) * 64 + 32 * s2;
          const bool ok = kk + 32 <= Kd;
#pragma unroll
          for (int f = 0; f < 2; ++f) av[p][f][s2] = ld16(ra, (ok && ao[f] != OOB) ? ao[f] + kk * 2 : OOB);
        }
      __builtin_amdgcn_sched_barrier(0);   // every load of the batch is issued before the first MFMA waits
#pragma unroll
      for (int p = 0; p < XPRE; ++p)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
          for (int fr = 0; fr < 2; ++fr)
#pragma unroll
            for (int fc = 0; fc < 2; ++fc) acc[fr][fc] = mfma16x(av[p][fr][s2], bv[p][fc][s2], acc[fr][fc]);
    }
    // element q = 8 fr + 4 fc + r of a lane: row 16 fr + 4 kq + r of the slice, factor row (ext column) 16 fc + i
#pragma unroll
    for (int q = 0; q < 16; ++q) red[(w * 16 + q) * 64 + l] = acc[q >> 3][(q >> 2) & 1][q & 3];   // lane-contiguous
    lds_barrier();
    // wave w sums elements 2w and 2w + 1 over the waves, in wave order, and stores those values
    static_assert(2 * XW == 16, "two accumulator elements per wave");
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int q = 2 * w + rr;
      float v = red[q * 64 + l];
#pragma unroll
      for (int ww = 1; ww < XW; ++ww) v += red[(ww * 16 + q) * 64 + l];
      const int orow = m * 32 + 16 * (q >> 3) + 4 * kq + (q & 3);
      if (orow < nrows) ext[(int64_t)(t.y + orow) * ldx + 16 * ((q >> 2) & 1) + li] = f2bf(scale * v);
    }
    lds_barrier();   // red is reused by the next item
  }
}

// LoRA factor gradients, all products of a backward (four, or six with two-plane gate_up operands) in one launch.
// Item = (WG_CBI adjacent 128-column blocks of a job, 512-row chunk slot of a LoRA group); persistent blocks (at most
// two per CU) take the items that are in use, counted on the device from the group offsets. An item's column blocks
// share its row table and run as one sequence of 64-row steps, so each next one's first loads go out during the
// previous one's last steps (an item's time is mostly its fixed latency, not its steps). out[p][q] = sum over ALL rows of group i
// of alpha(row) L[row * ldl + p] Rm[src(row)][q], p < 32, as an MFMA GEMM with the row index as the contraction dim:
// per 64-row step, L and Rm are staged transposed in LDS (k-pair packing: the values of rows 2j and 2j+1 share one
// 32-bit word), then each wave multiplies the 32 x 64 L^T tile by its 64 x 32 slice of the Rm tile. The LDS tiles
// are double-buffered and the raw rows of step j+1 are loaded into registers before step j's MFMAs, so one barrier
// per step suffices. Rows are summed in one fixed order (deterministic), and
// each (p, q) goes straight to the gradient tensor the job's destination descriptor names.
constexpr int WG_QB = 128;    // columns per block
constexpr int WG_S = 64 + 8;  // LDS row stride (bf16)
constexpr int WG_PF = 4;      // 64-row steps in flight
constexpr int WG_CH = 512;    // rows per chunk block
constexpr int WG_MAXG = 256;  // LoRA groups per call
constexpr int WG_WIN = WG_CH; // rows per index window
constexpr int WG_MAXJ = 6;    // jobs per launch (four, or six with two-plane gate_up operands)
constexpr int WG_CBI = 4;     // adjacent column blocks per item (a divisor of the jobs' 4, 8 and 16)

struct WgArgs {
  smel_wg_job job[WG_MAXJ];
  int qb0[WG_MAXJ];            // first 128-column block of each job in the partial-tile space
  int nqb;                     // 128-column blocks of all jobs
  int pb0[WG_MAXJ];            // first column-block group (WG_CBI blocks) of each job
  int npb;                     // column-block groups of all jobs
  int tot;                     // partial-tile slots per column block
  float* ws;                   // partial tiles [sum of column blocks][tot][32 * 128]
  const int32_t* groups;
  int n_lora, n_sel;
  const int32_t* offsets;
  int E, T, TK, topk;
  const int32_t* order;
  const float* topv;
  const float* sgate;
};

// The LoRA groups' first row G0, row count GN and first chunk slot GC (GC[n] = slots used), into LDS: thread i loads
// group i's offsets (all groups at once, one memory latency). Returns the number of groups.
SMEL_DEV int wg_table(const WgArgs& a, int* G0, int* GN, int* GC) {
  const int tid = threadIdx.x;
  if (tid < a.n_lora) {
    const int g = a.groups[tid];
    G0[tid] = g < a.E ? a.offsets[g] : a.TK;
    GN[tid] = g < a.E ? a.offsets[g + 1] - a.offsets[g] : a.T;
  }
  __syncthreads();
  if (tid == 0) {
    // the host's row bound caps the slots (monotone, <= tot): nothing is read or written out of range
    int c = 0;
    for (int i = 0; i < a.n_lora; ++i) {
      GC[i] = min(c, a.tot);
      c += max(1, (GN[i] + WG_CH - 1) / WG_CH);
    }
    GC[a.n_lora] = min(c, a.tot);
  }
  __syncthreads();
  return a.n_lora;
}

// R[p][q] of one 32 x 32 wave tile (acc of wave w, lane l; column block q0) -> the job's destination for group i's
// class (selected slot i, or the shared set) and p-range. Registers 4 j .. 4 j + 3 of a lane hold four consecutive p's,
// so a destination with p contiguous (s_p = 1: the B factors' [out][r] layout) takes them as one 16-B store.
SMEL_DEV void wg_store(const smel_wg_job& J, int n_sel, int i, int q0, int w, int l, const f32x16_t& acc) {
  const int q = q0 + 32 * w + (l & 31);
  if (q >= J.Q) return;
  const int cls = i < n_sel ? 0 : 1;
  const int64_t slot = cls == 0 ? i : 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const smel_wg_dest& d = J.dest[cls][h];
    if (!d.ptr || q < d.q0 || q >= d.q0 + d.nq) continue;
    float* const base = d.ptr + slot * d.s_idx + (int64_t)(q - d.q0) * d.s_q;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = acc_row(4 * j, l);   // p .. p + 3 in registers 4 j .. 4 j + 3
      float* const o = base + (int64_t)(p - d.p0) * d.s_p;
      if (d.s_p == 1 && p >= d.p0 && p + 4 <= d.p0 + d.np && ((uintptr_t)o & 15) == 0) {
        *reinterpret_cast<f32x4_t*>(o) = f32x4_t{acc[4 * j], acc[4 * j + 1], acc[4 * j + 2], acc[4 * j + 3]};
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (p + t >= d.p0 && p + t < d.p0 + d.np) o[t * d.s_p] = acc[4 * j + t];
      }
    }
  }
}

__global__ __launch_bounds__(256) void lora_wgrad_kernel(WgArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t LT[2][32 * WG_S];
  __shared__ __attribute__((aligned(16))) uint16_t RT[2][WG_QB * WG_S];
  __shared__ uint32_t TOFF[WG_WIN];
  __shared__ float TAL[WG_WIN];
  __shared__ int G0[WG_MAXG], GN[WG_MAXG], GC[WG_MAXG + 1];
  // the groups' rows, loaded in parallel (one memory latency), and their chunk slots: group i owns slots
  // [GC[i], GC[i+1]), one per 512-row chunk (at least one)
  const int ng = wg_table(a, G0, GN, GC);
  const int used = GC[ng];
  // persistent: items (column-block group of all jobs, chunk slot), the slots in use only
  static_assert(WG_WIN == WG_CH, "one row window per chunk");
  for (int it = blockIdx.x; it < a.npb * used; it += gridDim.x) {   // uniform
    const int pg = it / used, sl = it - pg * used;
    int jb = 0;
#pragma unroll
    for (int j = 1; j < WG_MAXJ; ++j)
      if (pg >= a.pb0[j]) jb = j;
    const smel_wg_job& J = a.job[jb];
    const int qb = WG_CBI * (pg - a.pb0[jb]);                               // the item's first column block
    const int ncb = min(WG_CBI, (int)((J.Q + WG_QB - 1) / WG_QB) - qb);     // 1 .. WG_CBI
    int i = 0;
    while (GC[i + 1] <= sl) ++i;
    const int c = sl - GC[i];
    const int nch = GC[i + 1] - GC[i];
    const int g0 = G0[i], g1 = G0[i] + GN[i];
    // this block: rows [a0, a1) = chunk c of the group
    const int a0 = g0 + c * WG_CH;
    const int a1 = min(g1, a0 + WG_CH);
    const int q0 = qb * WG_QB;
    const int Q = (int)J.Q;
    const int tid = threadIdx.x, l = lane_id(), w = tid >> 6, hi = l >> 5, r32 = l & 31;
    const int kp = tid & 31, grp = tid >> 5;   // k pair, and 4 p's (L) / 16 q's (Rm) per thread
    const int qq = q0 + 16 * grp;             // in the item's first column block
    const rsrc_t rr = make_rsrc(J.Rm, (uint64_t)J.r_rows * J.ldr * 2);
    const int64_t ldr = J.ldr;
    const int r_gather = J.r_gather, use_w = J.use_w;
    const uint16_t* __restrict__ Lp = J.L;
    f32x16_t acc[WG_CBI];   // the item's column blocks
#pragma unroll
    for (int cb = 0; cb < WG_CBI; ++cb) acc[cb] = f32x16_t{};
    // raw data of one step for this thread: L rows (ra, ra+1) x 4 p, Rm rows (ra, ra+1) x 16 q, the row weights;
    // WG_PF steps are in flight (a register ring rotated by unrolling): a long group (the shared MLP's T rows) is bound
    // by the load latency, not by its few MFMAs.
    struct Raw {
      uint2 lv0, lv1;
      u32x4_t x0[2], x1[2];
      float al0, al1;
    };
    Raw rw[WG_PF];
    // per window of WG_WIN rows: source-row byte offset and row weight of every row, built once into LDS so that the
    // prefetched loads depend on LDS reads only (a load whose address came from a global load would make the wait for
    // it drain every load in flight, vmcnt retiring in order)
    // a thread's WG_WIN / 256 rows: all their slot loads, then all their weight loads (two memory round trips)
    auto build = [&](int w0, int w1) {
      constexpr int BR = WG_WIN / 256;
      int pv[BR];
#pragma unroll
      for (int u = 0; u < BR; ++u) {
        const int row = w0 + tid + 256 * u;
        pv[u] = (row < w1 && row < a.TK) ? a.order[row] : 0;
      }
      float al[BR];
#pragma unroll
      for (int u = 0; u < BR; ++u) {
        const int row = w0 + tid + 256 * u;
        al[u] = 1.f;
        if (use_w && row < w1) al[u] = row < a.TK ? a.topv[pv[u]] : a.sgate[row - a.TK];
      }
#pragma unroll
      for (int u = 0; u < BR; ++u) {
        const int row = w0 + tid + 256 * u;
        if (row < w1) {
          const int src = !r_gather ? row : (row < a.TK ? pv[u] / a.topk : row - a.TK);
          TOFF[row - w0] = (uint32_t)src * (uint32_t)ldr * 2;
          TAL[row - w0] = al[u];
        }
      }
    };
    const uint32_t ldl2 = (uint32_t)J.ldl * 2;              // L row pitch in bytes
    const rsrc_t rl = make_rsrc(Lp, (uint64_t)a1 * ldl2);  // L rows [0, a1): a row past the group reads zeros
    // branch-free: rows past the window, and a column block past the item's, get out-of-range offsets (zeros) and
    // weight 0
    auto load = [&](int k0, int w0, int w1, int cb, Raw& R) {
      const int qc = qq + WG_QB * cb;
      const bool qok = cb < ncb && qc < Q;
      const int ra = k0 + 2 * kp;
      const bool v0 = ra < w1, v1 = ra + 1 < w1;
      const int t0 = v0 ? ra - w0 : 0, t1 = v1 ? ra + 1 - w0 : 0;
      const uint32_t o0 = v0 ? TOFF[t0] : OOB, o1 = v1 ? TOFF[t1] : OOB;
      R.al0 = v0 ? TAL[t0] : 0.f;
      R.al1 = v1 ? TAL[t1] : 0.f;
      const u32x2_t l0 = ld8(rl, v0 ? (uint32_t)ra * ldl2 + 8 * grp : OOB);
      const u32x2_t l1 = ld8(rl, v1 ? (uint32_t)(ra + 1) * ldl2 + 8 * grp : OOB);
      R.lv0 = make_uint2(l0.x, l0.y);
      R.lv1 = make_uint2(l1.x, l1.y);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        R.x0[h] = ld16(rr, qok ? o0 + (uint32_t)(qc + 8 * h) * 2 : OOB);
        R.x1[h] = ld16(rr, qok ? o1 + (uint32_t)(qc + 8 * h) * 2 : OOB);
      }
    };
    auto stage = [&](int buf, const Raw& R) {
      // L^T: alpha folded in (fp32, one bf16 rounding)
      uint32_t* d = reinterpret_cast<uint32_t*>(LT[buf] + (4 * grp) * WG_S + 2 * kp);
      d[0 * (WG_S / 2)] = pack2bf(R.al0 * bf_lo(R.lv0.x), R.al1 * bf_lo(R.lv1.x));
      d[1 * (WG_S / 2)] = pack2bf(R.al0 * bf_hi(R.lv0.x), R.al1 * bf_hi(R.lv1.x));
      d[2 * (WG_S / 2)] = pack2bf(R.al0 * bf_lo(R.lv0.y), R.al1 * bf_lo(R.lv1.y));
      d[3 * (WG_S / 2)] = pack2bf(R.al0 * bf_hi(R.lv0.y), R.al1 * bf_hi(R.lv1.y));
      uint32_t* e = reinterpret_cast<uint32_t*>(RT[buf] + (16 * grp) * WG_S + 2 * kp);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          e[(8 * h + 2 * j) * (WG_S / 2)] = __builtin_amdgcn_perm(R.x1[h][j], R.x0[h][j], 0x05040100u);
          e[(8 * h + 2 * j + 1) * (WG_S / 2)] = __builtin_amdgcn_perm(R.x1[h][j], R.x0[h][j], 0x07060302u);
        }
    };
    for (int w0 = a0; w0 < a1; w0 += WG_WIN) {   // uniform
      const int w1 = min(a1, w0 + WG_WIN);
      __syncthreads();   // the previous window's table and tiles are no longer read
      build(w0, w1);
      __syncthreads();
      // virtual steps: [cb S, (cb + 1) S) are column block cb's 64-row steps (S = whole rounds of WG_PF)
      const int S = (w1 - w0 + 64 * WG_PF - 1) / (64 * WG_PF) * WG_PF;
      auto vload = [&](int v, Raw& R) {
        const int cb = v / S;   // >= ncb past the last step: zeros
        load(w0 + 64 * (v - cb * S), w0, w1, cb, R);
      };
#pragma unroll
      for (int u = 0; u < WG_PF; ++u) vload(u, rw[u]);
      // WG_PF steps per round, branch-free (a step past the window stages zeros and adds nothing), so the compiler's
      // wait for a ring slot counts exactly the loads issued after it
      auto round = [&](int v0, f32x16_t& ac) {
#pragma unroll
        for (int u = 0; u < WG_PF; ++u) {
          const int buf = u & 1;
          stage(buf, rw[u]);
          vload(v0 + u + WG_PF, rw[u]);   // the next column block's first steps during this one's last round
          __syncthreads();
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const u32x4_t af = *reinterpret_cast<const u32x4_t*>(LT[buf] + r32 * WG_S + 32 * hi + 8 * s);
            const u32x4_t bfr = *reinterpret_cast<const u32x4_t*>(RT[buf] + (32 * w + r32) * WG_S + 32 * hi + 8 * s);
            ac = mfma32(af, bfr, ac);
          }
        }
      };
#pragma unroll
      for (int cb = 0; cb < WG_CBI; ++cb)
        if (cb < ncb)   // uniform
          for (int v0 = cb * S; v0 < (cb + 1) * S; v0 += WG_PF) round(v0, acc[cb]);
    }
    auto put = [&](const f32x16_t& ac, int qbc) {
      if (nch == 1) {
        wg_store(J, a.n_sel, i, qbc * WG_QB, w, l, ac);
      } else {
        // a group of several chunks: this chunk's partial tile, summed in chunk order by lora_wgrad_reduce
        float* tile = a.ws + ((int64_t)(a.qb0[jb] + qbc) * a.tot + sl) * (32 * WG_QB);
#pragma unroll
        for (int r = 0; r < 16; ++r) tile[r * 256 + tid] = ac[r];
      }
    };
#pragma unroll
    for (int cb = 0; cb < WG_CBI; ++cb)
      if (cb < ncb) put(acc[cb], qb + cb);
  }
}

// The multi-chunk groups: sum the partial tiles in chunk order, store like lora_wgrad_kernel. Block = (one column
// block of all jobs, one LoRA group); blocks of groups with at most one chunk leave at once. The chunks' loads go out
// four chunks at a time (one memory round trip per four chunks), the sum keeps chunk order.
__global__ __launch_bounds__(256) void lora_wgrad_reduce(WgArgs a) {
  __shared__ int G0[WG_MAXG], GN[WG_MAXG], GC[WG_MAXG + 1];
  const int qbg = blockIdx.x, i = blockIdx.y;
  int jb = 0;
#pragma unroll
  for (int j = 1; j < WG_MAXJ; ++j)
    if (qbg >= a.qb0[j]) jb = j;
  const smel_wg_job& J = a.job[jb];
  const int qb = qbg - a.qb0[jb];
  wg_table(a, G0, GN, GC);
  const int tid = threadIdx.x;
  const int nch = GC[i + 1] - GC[i];
  if (nch <= 1) return;   // uniform
  const float* tile = a.ws + ((int64_t)qbg * a.tot + GC[i]) * (32 * WG_QB);
  f32x16_t acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = tile[r * 256 + tid];
  for (int c0 = 1; c0 < nch; c0 += 4) {
    float v[4][16];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        v[u][r] = c0 + u < nch ? tile[(int64_t)(c0 + u) * (32 * WG_QB) + r * 256 + tid] : 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (c0 + u < nch)   // uniform
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] += v[u][r];
  }
  wg_store(J, a.n_sel, i, qb * WG_QB, tid >> 6, lane_id(), acc);
}

// LoRA rows from per-column-block fp32 partials (smel_gmm_bwd_lr's): ext[row][32 c + j] = bf16(sum_b part[row][b][c][j])
// with b ascending from 0.f, the order the gate_up backward sums them in, so both see the same bf16 rows. One block
// per tile of the list; a thread takes 8 values (two 16-B loads per partial, one 16-B store).
__global__ __launch_bounds__(256) void lora_rows_sum_kernel(const int4* __restrict__ tiles,
                                                            const int32_t* __restrict__ n_tiles,
                                                            const int32_t* __restrict__ gkind, int sel, int sh,
                                                            const float* __restrict__ part, int parts, int planes,
                                                            uint16_t* __restrict__ ext) {
  const int tt = blockIdx.x;
  if (tt >= n_tiles[0]) return;
  const int4 t = tiles[tt];
  const int gk = gkind ? gkind[t.x] : t.w;
  const int kind = gk >> 16;
  if (!((kind == SMEL_KIND_SEL && sel) || (kind == SMEL_KIND_SHARED && sh))) return;
  const int nrows = min(t.z - t.y, 128);
  const int W = 4 * planes;   // 8-value chunks per row
  for (int i = threadIdx.x; i < nrows * W; i += blockDim.x) {
    const int row = i / W, ch = i - row * W;
    const int c = ch >> 2, j0 = 8 * (ch & 3);
    const int64_t grow = t.y + row;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < parts; ++p) {
      const float* src = part + ((grow * parts + p) * planes + c) * 32 + j0;
      const f32x4_t x0 = *reinterpret_cast<const f32x4_t*>(src), x1 = *reinterpret_cast<const f32x4_t*>(src + 4);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[q] += x0[q];
        v[4 + q] += x1[q];
      }
    }
    *reinterpret_cast<u32x4_t*>(ext + grow * 32 * planes + 32 * c + j0) =
        u32x4_t{pack2bf(v[0], v[1]), pack2bf(v[2], v[3]), pack2bf(v[4], v[5]), pack2bf(v[6], v[7])};
  }
}

}  // namespace

extern "C" int smel_lora_prep_sets(const smel_lora_set* sets, int32_t n_sets, int32_t planes, int64_t Hd,
                                   int64_t In, hipStream_t stream) {
  SMEL_REQUIRE(sets && n_sets >= 1 && n_sets <= PREP_MAX_SETS, SMEL_EINVAL, "lora_prep: %d sets (1 or 2)", n_sets);
  SMEL_REQUIRE(Hd > 0 && In > 0, SMEL_EINVAL, "lora_prep: bad sizes");
  SMEL_REQUIRE(planes == 1 || planes == 2, SMEL_EINVAL, "lora_prep: planes %d (1 or 2)", planes);
  PrepArgs pa{};
  pa.planes = planes;
  pa.Hd = (int)Hd;
  pa.In = (int)In;
  int nz = 0;
  for (int i = 0; i < n_sets; ++i) {
    const smel_lora_set& S = sets[i];
    SMEL_REQUIRE(S.n >= 0 && S.r > 0, SMEL_EINVAL, "lora_prep: set %d: bad sizes", i);
    SMEL_REQUIRE(S.r <= 16 * planes, SMEL_EUNSUPPORTED, "lora_prep: set %d: rank %lld > %d (%d plane%s)", i,
                 (long long)S.r, 16 * planes, planes, planes == 1 ? "; 2 planes take up to 32" : "s");
    if (S.n == 0) continue;
    SMEL_REQUIRE(S.A_gate && S.B_gate && S.A_up && S.B_up && S.A_down && S.B_down && S.fwd_gu && S.fwd_dn && S.a_gu &&
                     S.a_dn && S.bt_dn && S.bt_gu && S.at_gu && S.at_dn,
                 SMEL_EINVAL, "lora_prep: set %d: null pointer", i);
    SMEL_REQUIRE(S.n * planes * 32 * std::max(Hd, 2 * In) < (1ll << 31), SMEL_EUNSUPPORTED,
                 "lora_prep: set %d: layouts too large", i);
    SMEL_REQUIRE(((uintptr_t)S.fwd_gu | (uintptr_t)S.fwd_dn | (uintptr_t)S.a_gu | (uintptr_t)S.a_dn |
                  (uintptr_t)S.bt_dn | (uintptr_t)S.bt_gu | (uintptr_t)S.at_gu | (uintptr_t)S.at_dn) % 16 == 0,
                 SMEL_EUNSUPPORTED, "lora_prep: set %d: outputs must be 16-byte aligned", i);
    SMEL_REQUIRE(((uintptr_t)S.A_gate | (uintptr_t)S.B_gate | (uintptr_t)S.A_up | (uintptr_t)S.B_up |
                  (uintptr_t)S.A_down | (uintptr_t)S.B_down) % 16 == 0,
                 SMEL_EUNSUPPORTED, "lora_prep: set %d: factors must be 16-byte aligned", i);
    pa.set[nz++] = S;   // empty sets are left out of the launch
  }
  if (nz == 0) return 0;
  SMEL_REQUIRE(Hd % 32 == 0 && In % 32 == 0, SMEL_EUNSUPPORTED,
               "lora_prep: Hd=%lld and In=%lld must be multiples of 32 (as the GEMMs' dimensions)", (long long)Hd,
               (long long)In);
  // blocks: per set, n experts x chunks of each kind
  const int64_t ch_h = (Hd + PCH - 1) / PCH, ch_i = (In + PCH - 1) / PCH;
  int64_t b = 0;
  for (int i = 0; i < PREP_MAX_SETS; ++i)
    for (int k = 0; k < PK_N; ++k) {
      pa.first[i * PK_N + k] = (int)b;
      if (i < nz) b += pa.set[i].n * ((k == PK_AGU || k == PK_BDN) ? ch_h : ch_i);
    }
  pa.first[PREP_MAX_SETS * PK_N] = (int)b;
  SMEL_REQUIRE(b < (1ll << 31), SMEL_EUNSUPPORTED, "lora_prep: too many blocks");
  if (b == 0) return 0;
  lora_prep_kernel<<<(unsigned)b, 256, 0, stream>>>(pa);
  return smel::launch_status();
}

extern "C" int smel_lora_prep(const float* A_gate, const float* B_gate, const float* A_up, const float* B_up,
                              const float* A_down, const float* B_down, int64_t n, int64_t r, int32_t planes,
                              int64_t Hd, int64_t In, uint16_t* fwd_gu, uint16_t* fwd_dn, uint16_t* a_gu,
                              uint16_t* a_dn, uint16_t* bt_dn, uint16_t* bt_gu, uint16_t* at_gu, uint16_t* at_dn,
                              hipStream_t stream) {
  const smel_lora_set S{A_gate, B_gate, A_up, B_up, A_down, B_down, n, r, fwd_gu, fwd_dn, a_gu, a_dn,
                        bt_dn, bt_gu, at_gu, at_dn};
  return smel_lora_prep_sets(&S, 1, planes, Hd, In, stream);
}

extern "C" int smel_lora_ext(const int32_t* tiles, const int32_t* n_tiles, int64_t max_tiles, const int32_t* gkind,
                             const uint16_t* A_src, int64_t lda, int64_t a_rows, int32_t a_gather,
                             const int32_t* order, int64_t TK, int64_t topk, const uint16_t* wcat_sel,
                             const uint16_t* wcat_sh, int64_t Kd, float scale_sel, float scale_sh, uint16_t* ext,
                             int64_t ldx, hipStream_t stream) {
  SMEL_REQUIRE(tiles && n_tiles && A_src && ext, SMEL_EINVAL, "lora_ext: null pointer");
  SMEL_REQUIRE(ldx == 32 || ldx == 64, SMEL_EINVAL, "lora_ext: ext row stride %lld (32 or 64)", (long long)ldx);
  SMEL_REQUIRE(Kd > 0 && Kd % 32 == 0, SMEL_EUNSUPPORTED, "lora_ext: K %lld must be a multiple of 32", (long long)Kd);
  SMEL_REQUIRE(lda % 8 == 0 && ((uintptr_t)A_src % 16) == 0, SMEL_EUNSUPPORTED, "lora_ext: A rows must be 16-B aligned");
  SMEL_REQUIRE(!a_gather || order || TK == 0, SMEL_EINVAL, "lora_ext: gather needs order");
  SMEL_REQUIRE(a_rows >= 0 && a_rows * lda * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "lora_ext: A larger than 2 GiB");
  SMEL_REQUIRE(max_tiles <= XLT, SMEL_EUNSUPPORTED, "lora_ext: at most %d tiles per call (got %lld)", XLT,
               (long long)max_tiles);
  if (max_tiles == 0 || (!wcat_sel && !wcat_sh)) return 0;
  lora_ext_kernel<<<smel::cu_count(), 512, 0, stream>>>(reinterpret_cast<const int4*>(tiles), n_tiles, gkind, A_src,
                                                        lda, a_rows, a_gather, order, (int)TK, (int)topk, wcat_sel,
                                                        wcat_sh, (int)Kd, scale_sel, scale_sh, ext, (int)ldx,
                                                        (int)max_tiles);
  return smel::launch_status();
}

extern "C" int smel_lora_rows_sum(const int32_t* tiles, const int32_t* n_tiles, int64_t max_tiles, const int32_t* gkind,
                                  int32_t sel, int32_t sh, const float* part, int32_t parts, int32_t planes,
                                  uint16_t* ext, hipStream_t stream) {
  SMEL_REQUIRE(parts >= 1 && (planes == 1 || planes == 2) && max_tiles >= 0, SMEL_EINVAL,
               "lora_rows_sum: parts %d, planes %d", parts, planes);
  if (max_tiles == 0 || (!sel && !sh)) return 0;
  SMEL_REQUIRE(tiles && n_tiles && part && ext, SMEL_EINVAL, "lora_rows_sum: null pointer");
  SMEL_REQUIRE(((uintptr_t)part % 16) == 0 && ((uintptr_t)ext % 16) == 0, SMEL_EUNSUPPORTED,
               "lora_rows_sum: part and ext must be 16-B aligned");
  lora_rows_sum_kernel<<<(unsigned)max_tiles, 256, 0, stream>>>(reinterpret_cast<const int4*>(tiles), n_tiles, gkind,
                                                               sel, sh, part, parts, planes, ext);
  return smel::launch_status();
}

namespace {
int64_t wg_qblocks(const smel_wg_job* jobs, int n_jobs) {
  int64_t n = 0;
  for (int j = 0; j < n_jobs; ++j) n += (jobs[j].Q + WG_QB - 1) / WG_QB;
  return n;
}
int64_t wg_tot(int64_t n_lora, int64_t max_rows) { return n_lora + (max_rows + WG_CH - 1) / WG_CH; }
}  // namespace

extern "C" int64_t smel_lora_wgrad_ws_floats(const smel_wg_job* jobs, int32_t n_jobs, int64_t n_lora,
                                             int64_t max_rows) {
  if (!jobs || n_jobs < 0 || n_jobs > WG_MAXJ || n_lora < 0 || max_rows < 0) return -1;
  return wg_qblocks(jobs, n_jobs) * wg_tot(n_lora, max_rows) * 32 * WG_QB;
}

extern "C" int smel_lora_wgrad(const smel_wg_job* jobs, int32_t n_jobs, const int32_t* lora_groups, int64_t n_lora,
                               int64_t n_sel, const int32_t* offsets, int64_t E, int64_t T, int64_t TK, int64_t topk,
                               const int32_t* order, const float* topv, const float* sgate, int64_t max_rows,
                               float* ws, int64_t ws_floats, hipStream_t stream) {
  SMEL_REQUIRE(jobs && n_jobs >= 0 && n_jobs <= WG_MAXJ && n_lora >= 0 && n_sel >= 0 && n_sel <= n_lora &&
                   max_rows >= 0,
               SMEL_EINVAL, "lora_wgrad: bad job / group counts");
  if (n_jobs == 0 || n_lora == 0) return 0;
  SMEL_REQUIRE(lora_groups && offsets, SMEL_EINVAL, "lora_wgrad: null pointer");
  SMEL_REQUIRE(n_lora <= WG_MAXG, SMEL_EUNSUPPORTED, "lora_wgrad: %lld LoRA groups > %d", (long long)n_lora, WG_MAXG);
  SMEL_REQUIRE(ws && ws_floats >= smel_lora_wgrad_ws_floats(jobs, n_jobs, n_lora, max_rows), SMEL_EINVAL,
               "lora_wgrad: workspace smaller than smel_lora_wgrad_ws_floats");
  WgArgs a;
  a.tot = (int)wg_tot(n_lora, max_rows);
  a.ws = ws;
  int qbs = 0, pbs = 0;
  for (int j = 0; j < WG_MAXJ; ++j) {
    a.qb0[j] = qbs;
    a.pb0[j] = pbs;
    if (j < n_jobs) {
      const smel_wg_job& J = jobs[j];
      SMEL_REQUIRE(J.L && J.Rm && J.Q > 0, SMEL_EINVAL, "lora_wgrad: job %d: null operand or Q", j);
      SMEL_REQUIRE((J.ldl == 32 || J.ldl == 64) && ((uintptr_t)J.L % 8) == 0, SMEL_EINVAL,
                   "lora_wgrad: job %d: L row stride %lld (32 or 64) or L not 8-B aligned", j, (long long)J.ldl);
      SMEL_REQUIRE(!(J.r_gather || J.use_w) || order || TK == 0, SMEL_EINVAL, "lora_wgrad: job %d needs order", j);
      SMEL_REQUIRE(J.ldr % 8 == 0 && J.Q % 16 == 0 && ((uintptr_t)J.Rm % 16) == 0, SMEL_EUNSUPPORTED,
                   "lora_wgrad: job %d: Rm rows must be 16-B aligned and Q a multiple of 16", j);
      SMEL_REQUIRE(J.r_rows * J.ldr * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "lora_wgrad: job %d: Rm larger than 2 GiB",
                   j);
      for (int c = 0; c < 2; ++c)
        for (int h = 0; h < 2; ++h) {
          const smel_wg_dest& d = J.dest[c][h];
          SMEL_REQUIRE(!d.ptr || (d.p0 >= 0 && d.np >= 0 && d.p0 + d.np <= 32 && d.q0 >= 0 && d.nq >= 0 &&
                                  d.q0 + d.nq <= J.Q),
                       SMEL_EINVAL, "lora_wgrad: job %d: destination [%d][%d] outside the 32 x Q result", j, c, h);
        }
      a.job[j] = J;
      const int nqbj = (int)((J.Q + WG_QB - 1) / WG_QB);
      qbs += nqbj;
      pbs += (nqbj + WG_CBI - 1) / WG_CBI;
    } else {
      a.job[j] = smel_wg_job{};
      a.job[j].Q = WG_QB;
      a.job[j].ldl = 32;
    }
  }
  a.nqb = qbs;
  a.npb = pbs;
  a.groups = lora_groups;
  a.n_lora = (int)n_lora;
  a.n_sel = (int)n_sel;
  a.offsets = offsets;
  a.E = (int)E;
  a.T = (int)T;
  a.TK = (int)TK;
  a.topk = (int)topk;
  a.order = order;
  a.topv = topv;
  a.sgate = sgate;
  // persistent blocks over the (column-block group, chunk slot) items in use: at most two per CU
  const int64_t bound = (int64_t)pbs * a.tot;
  lora_wgrad_kernel<<<(unsigned)std::min<int64_t>(bound, 2 * smel::cu_count()), 256, 0, stream>>>(a);
  int st = smel::launch_status();
  if (st) return st;
  lora_wgrad_reduce<<<dim3((unsigned)qbs, (unsigned)n_lora), 256, 0, stream>>>(a);
  return smel::launch_status();
}
