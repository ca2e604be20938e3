// Grouped expert GEMM, backward (acc = A W per group, contraction over the weight's row dim): dA of the down
// projection (fused with the SiLU-gate backward, the d(combine weight) partials and the topv / shared-gate scaling)
// and dX of the gate_up projection. Frozen int4 experts are re-dequantized step by step in registers. Reference:
// FrozenExpertsFn.backward, smel/moe.py:128-143, and the autograd of _selected_expert / lora_gate_up / lora_linear /
// the combine, smel/moe.py:204-252, smel/lora.py:61-83.
//
// The weights come in the transposed fragment layout of smel_pack_int4_t / smel_pack_bf16_t, so every wave streams its
// own 64 output columns straight into registers and dequantizes them there, as the forward kernel does; the int4
// scale / zero vary along the contraction here, so each lane needs one (scale, zero) pair per row it holds: those
// 64-pair runs (fp32, ready to use) go global -> LDS by LDS-DMA beside the A rows.
//
// Block = 4 waves, tile = up to 128 rows of one group (4 slices of 32) x 256 columns (64 per wave).
// MFMA v_mfma_f32_16x16x32_bf16: lane l = 16 kq + i carries, in substep s of a 64-wide k-step, k = 32 s + 8 kq +
// [0, 8) for A and B alike (so a lane needs 16 scale/zero words per k-step, not 32 as with 32x32x16), and
// accumulates D[4 kq + r][i]. Per k-step:
//  * A rows (gathered by token for the down projection) go global -> LDS (16-B LDS-DMA) into a ring of 4 stages,
//    XOR-swizzled as in the forward kernel; each wave DMAs its own scale/zero words (4 B per lane) into the stage;
//  * int4: weights (a 4-deep register ring of 2 loads), scale/zero and A all run 3 k-steps ahead; bf16: weights 1
//    step ahead (8 loads), A 3 steps ahead;
//  * vmcnt retires in issue order: each step issues its weight loads before its LDS-DMAs and waits for exactly the
//    loads of the step it is about to use.

#include "abi_util.h"
#include "common.h"

namespace {

constexpr int MT = 128;
constexpr int KT = 64;
constexpr int NB = 256;            // output columns per block
constexpr int A_BYTES = MT * KT * 2;         // A rows of one stage
// scale/zero of one stage: 4 waves x 64 rows x (scale, zero) fp32, per group (two groups per wave when the int4 group
// is 32 wide: SZ2)
constexpr int z_bytes(bool sz2) { return 4 * 512 * (sz2 ? 2 : 1); }
constexpr int q_stage(bool sz2) { return A_BYTES + z_bytes(sz2); }
// 4 stages; the epilogue's staged tile (4 x A_BYTES) and its 512-B row table fit inside
constexpr int smem_bytes(bool sz2) { return 4 * q_stage(sz2); }
static_assert(smem_bytes(false) <= 80 * 1024 && 4 * A_BYTES + 512 <= smem_bytes(false), "two blocks per CU");

// Vector-memory operations per wave in each issue group of the main loops; the issue code below is written with
// these counts and every wait is computed from them (vmcnt retires in issue order).
constexpr int VM_A = A_BYTES / (4 * 1024);                 // A rows of a stage: 1-KB LDS-DMA wave-loads, 4 waves
constexpr int VM_Q = 2;                                     // int4: 16-B words of the two column pairs
constexpr int vm_sz(bool sz2) { return sz2 ? 4 : 2; }       // int4: 256-B scale/zero runs, per group
constexpr int vm_q4(bool sz2) { return VM_Q + vm_sz(sz2) + VM_A; }
constexpr int VM_B = 2 * 4;                                 // bf16: 2 substeps x 4 column fragments
// int4: steps j+1 and j+2 may be in flight while step j computes; bf16: issue order ... W(j+1), A(j+3), so before
// step j only A(j+2) may be
constexpr int q4_wait(bool sz2) { return 2 * vm_q4(sz2); }
constexpr int BF_WAIT = VM_A;

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
  const float* topv;
  const float* sgate;
  uint16_t* out;
  int64_t ldo;
  float* dwp;
  int a_gather, TK, topk, act;
  int Kd, N;   // Kd = w.R (contraction), N = w.C
  int nblk;    // column blocks per tile
  smel_bwd_lora_rows lr;   // gate_up LoRA rows: partials produced by the down backward, taken by the gate_up backward
  bool lr_on;
};

SMEL_DEV f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}

// 8 nibbles of one word (rows k0 .. k0+7, low nibble first) with per-row scale sc[t] / zero ze[t] -> 4 packed bf16
// pairs in row order, w = RNE(q*s + z) with fp32 arithmetic (the reference's dequant value).
SMEL_DEV void dq8r(uint32_t b, const float* sc, const float* ze, uint32_t out[4]) {
  const uint32_t lo = b & 0x0f0f0f0fu;          // rows 0,2,4,6
  const uint32_t hi = (b >> 4) & 0x0f0f0f0fu;   // rows 1,3,5,7
  out[0] = pack2bf(fmaf(ub0(lo), sc[0], ze[0]), fmaf(ub0(hi), sc[1], ze[1]));
  out[1] = pack2bf(fmaf(ub1(lo), sc[2], ze[2]), fmaf(ub1(hi), sc[3], ze[3]));
  out[2] = pack2bf(fmaf(ub2(lo), sc[4], ze[4]), fmaf(ub2(hi), sc[5], ze[5]));
  out[3] = pack2bf(fmaf(ub3(lo), sc[6], ze[6]), fmaf(ub3(hi), sc[7], ze[7]));
}
// 4-byte-per-lane LDS-DMA: lane i writes bytes [4 i, 4 i + 4) after the wave-uniform LDS address.
SMEL_DEV void ld4_lds(rsrc_t r, const void* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(lds), 4, off, 0, 0, 0);
}

template <int EPI, bool Q4, int NS, bool SZ2, bool FAST>
SMEL_DEV void run_tile(const BwdArgs& a, int kind, int idx, int row0, int nrows, int nb, uint8_t* smem) {
  // LDS rings of 4 stages. int4: [A rows 16 KB | scale/zero pairs of 4 waves x 64 rows (x 2 groups for SZ2), 2 KB
  // (4 KB)]; bf16: A rows. The weights go to registers. The epilogue reuses the first 64 KB.
  constexpr int QS = q_stage(SZ2), ZW = SZ2 ? 1024 : 512;   // stage bytes, scale/zero bytes per wave
  auto St = [&](int st) {
    return reinterpret_cast<uint16_t*>(smem + st * (Q4 ? QS : A_BYTES));
  };
  auto Zt = [&](int st) { return smem + st * QS + A_BYTES; };
  auto Et = [&](int m) { return reinterpret_cast<uint16_t*>(smem + m * A_BYTES); };
  const int tid = threadIdx.x, l = lane_id(), kq = l >> 4, li = l & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int Kd = a.Kd, N = a.N;
  const smel_wset& ws = a.w;
  // What the epilogue needs per tile row, fetched now (thread t < MT: row t) so that no load sits between its
  // stores: the output slot for the gate_up backward, the combine weight for the down backward.
  int ep_slot = 0;
  float ep_w = 0.f;
  if (tid < nrows) {
    const int grow = row0 + tid;
    if (EPI == 0)
      ep_slot = row_slot(grow, a.order, a.TK);
    else
      ep_w = grow < a.TK ? a.topv[a.order[grow]] : a.sgate[grow - a.TK];
  }
  const int cw = nb * NB + w * 64;   // this wave's first output column
  const int nk = (Kd + KT - 1) / KT;
  const int np = N / 32;             // column pairs of one matrix
  const int p0 = cw / 32;
  // Weight / scale-zero offsets need no validity flags: each descriptor covers exactly the rest of one matrix, so a
  // column pair or group past its end reads as zero (hardware out-of-range handling). The second column pair gets a
  // descriptor of its own (scalar registers) at the first pair's lane offset, which saves a vector register.
  rsrc_t rw, rw1, rsz, rsz1;
  uint32_t wo, so = 0;
  if constexpr (Q4) {
    const int G = N / ws.group;
    const uint8_t* qb = ws.q4 + (int64_t)idx * np * nk * 1024;
    const int64_t qbytes = (int64_t)np * nk * 1024;
    rw = make_rsrc(qb, (uint64_t)qbytes);
    rw1 = make_rsrc(qb + (int64_t)nk * 1024, (uint64_t)(qbytes - (int64_t)nk * 1024));
    const uint8_t* zb = reinterpret_cast<const uint8_t*>(ws.sz4) + (int64_t)idx * G * nk * 512;
    const int64_t zbytes = (int64_t)G * nk * 512;
    const int64_t zstep = (int64_t)((cw + 32) / ws.group - cw / ws.group) * nk * 512;   // 0 or one group
    rsz = make_rsrc(zb, (uint64_t)zbytes);
    rsz1 = make_rsrc(zb + zstep, (uint64_t)(zbytes - zstep));
    wo = (uint32_t)(p0 * nk * 1024 + l * 16);
    so = (uint32_t)((cw / ws.group) * nk * 512 + 4 * l);
  } else {
    const uint16_t* base = kind == SMEL_KIND_BF16 ? ws.wb : (kind == SMEL_KIND_SEL ? ws.wsel : ws.wsh);
    const int64_t mi = kind == SMEL_KIND_SHARED ? 0 : idx;
    const uint16_t* wb = base + mi * np * nk * 2048;
    const int64_t wbytes = (int64_t)np * nk * 4096;
    rw = make_rsrc(wb, (uint64_t)wbytes);
    rw1 = make_rsrc(wb + (int64_t)nk * 2048, (uint64_t)(wbytes - (int64_t)nk * 4096));
    rsz = rsz1 = rw;
    wo = (uint32_t)(p0 * nk * 4096 + l * 16);
  }
  // ---- A staging: wave-load ii of wave w fills rows 8 g .. 8 g + 7 (g = 4 w + ii) of a stage, 1 KB; lane i writes
  // physical chunk i % 8 of row 8 g + i / 8, i.e. logical chunk c = (i % 8) ^ swz(row). Kd is a multiple of 64, so a
  // k-step is all in or all out.
  const rsrc_t ra = make_rsrc(a.A, (uint64_t)a.a_rows * a.lda * 2);
  uint32_t aoff[VM_A];
#pragma unroll
  for (int ii = 0; ii < VM_A; ++ii) {
    const int g = VM_A * w + ii;
    const int row = 8 * g + (l >> 3);
    const int c = (l & 7) ^ swz(row);
    aoff[ii] = OOB;
    if (row < nrows) {
      const int grow = row0 + row;
      const int src = a.a_gather ? row_token(grow, a.order, a.TK, a.topk) : grow;
      aoff[ii] = (uint32_t)src * (uint32_t)a.lda * 2 + 16 * c;
    }
  }
  // All loads of step j: int4 -> q (2 x 16 B per lane) into the registers qd, scale/zero pairs (2 x 256 B per group)
  // into stage st; A (4 x 1 KB) into stage st.
  auto issue_lds = [&](int j, int st, u32x4_t* qd) {
    const bool in = j < nk;
    const uint32_t k2 = (uint32_t)j * KT * 2;
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (Q4) {
      static_assert(VM_Q == 2, "one word per column pair, 2 pairs");
      qd[0] = ld16(rw, in ? wo + j * 1024 : OOB);
      qd[1] = ld16(rw1, in ? wo + j * 1024 : OOB);
      // vm_sz(SZ2) runs of 256 B: (scale, zero) of the 64 rows, per group of the wave's columns
#pragma unroll
      for (int z = 0; z < vm_sz(SZ2); ++z)
        ld4_lds(z < 2 ? rsz : rsz1, Zt(st) + w * ZW + 256 * z, in ? so + j * 512 + 256 * (z & 1) : OOB);
    }
#pragma unroll
    for (int ii = 0; ii < VM_A; ++ii) ld16_lds(ra, St(st) + (VM_A * w + ii) * 512, in ? aoff[ii] + k2 : OOB);
    __builtin_amdgcn_sched_barrier(0);
  };
  // A fragment reads: lane (kq, li) of row-fragment rf, substep s reads logical chunk 4 s + kq of row 16 rf + li
  // (swz of that row depends on li only)
  uint32_t ard[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) ard[s] = li * KT + 8 * ((4 * s + kq) ^ swz(li));

  constexpr int NRF = 2 * NS;   // 16-row fragments
  f32x4_t acc[NRF][4];
#pragma unroll
  for (int m = 0; m < NRF; ++m)
#pragma unroll
    for (int f = 0; f < 4; ++f) acc[m][f] = f32x4_t{};

  if constexpr (Q4) {
    // One k-step = 2 substeps of 32. The A fragments, this lane's q words and its scale/zero pairs come from the
    // stage. The compiler would run a substep's four dequants (VALU) back to back and then its MFMAs, so the order is
    // fixed by sched_barrier fences: each group of MFMAs on column fragment f runs beside half of the dequant of
    // fragment f+1, and the second half of substep 0 (MFMAs only) also prepares substep 1's scale/zero and first
    // fragment. 16 A registers live at a time (first half rows, then second half rows).
    const uint32_t magic = FAST ? f16_magic() : 0u;
    auto compute = [&](int st, const u32x4_t* qv) {
      const uint16_t* S = St(st);
      const float* Z = reinterpret_cast<const float*>(Zt(st) + w * ZW) + 32 * kq;
      const u32x4_t q0 = qv[0], q1 = qv[1];
      float sc[8], ze[8];
      u32x4_t b[4];
      auto unpack = [&](const float* zp) {   // 8 (scale, zero) pairs, used as they are
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const f32x4_t z4 = *reinterpret_cast<const f32x4_t*>(zp + 4 * v);
          sc[2 * v] = z4[0];
          ze[2 * v] = z4[1];
          sc[2 * v + 1] = z4[2];
          ze[2 * v + 1] = z4[3];
        }
      };
      // half h of column fragment f's dequant in substep s. Fast bank: B words h and h + 2 (rows 2h, 2h+1 and
      // 2h+4, 2h+5): byte h of each half-word holds rows 2h (+4) in its low nibble, read as fp16 1024 + q with the
      // pair (s, z - 1024 s), and rows 2h+1 (+5) in its high nibble, read in place as fp16 1024 + 16 q with the pair
      // (s / 16, z - 64 s): 17 VALU per 8 weights. Exact path: the whole fragment with h = 0.
      auto dqh = [&](int s, int f, int h) {
        const uint32_t qw = (f < 2 ? q0 : q1)[2 * (f & 1) + s];
        if constexpr (FAST) {
          const uint32_t qb = h ? qw >> 8 : qw;
          const uint32_t x0 = (qb & 0x000F000Fu) | magic;
          const uint32_t x1 = (qb & 0x00F000F0u) | magic;
          const int j = 2 * h;
          b[f][h] = pack2bf(fmaf(h_lo(x0), sc[j], ze[j]), fmaf(h_lo(x1), sc[j + 1], ze[j + 1]));
          b[f][h + 2] = pack2bf(fmaf(h_hi(x0), sc[j + 4], ze[j + 4]), fmaf(h_hi(x1), sc[j + 5], ze[j + 5]));
        } else if (h == 0) {
          uint32_t o[4];
          dq8r(qw, sc, ze, o);   // rows / columns outside the matrix hold q = s = z = 0
          b[f] = u32x4_t{o[0], o[1], o[2], o[3]};
        }
      };
      constexpr int H1 = (NRF + 1) / 2, HA = (H1 + 1) / 2;   // first-half row fragments, in two MFMA groups
      constexpr int H2 = NRF - H1;                            // second-half row fragments
      auto rda = [&](int s, int m) { return *reinterpret_cast<const u32x4_t*>(S + ard[s] + m * 16 * KT); };
      // A fragments: the first half's and the second half's in separate registers, each read about two column
      // fragments of MFMAs before its first use (the second half during the first half's MFMAs, the next substep's
      // first half during the second half's), so no MFMA group waits for its LDS reads
      u32x4_t af1[H1], af2[H2 > 0 ? H2 : 1];
      unpack(Z);
      dqh(0, 0, 0);
      dqh(0, 0, 1);
#pragma unroll
      for (int m = 0; m < H1; ++m) af1[m] = rda(0, m);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          if (SZ2 && f == 1) unpack(Z + 128 + 16 * s);   // fragments 2, 3 are the wave's second scale/zero group
#pragma unroll
          for (int m = 0; m < HA; ++m) acc[m][f] = mfma16(af1[m], b[f], acc[m][f]);
          if (f < 3) dqh(s, f + 1, 0);
          if (f == 1) {
#pragma unroll
            for (int m = 0; m < H2; ++m) af2[m] = rda(s, H1 + m);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int m = HA; m < H1; ++m) acc[m][f] = mfma16(af1[m], b[f], acc[m][f]);
          if (f < 3) dqh(s, f + 1, 1);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int f = 0; f < 4; ++f) {
#pragma unroll
          for (int m = 0; m < H2; ++m) acc[H1 + m][f] = mfma16(af2[m], b[f], acc[H1 + m][f]);
          if (s == 0) {   // substep 1's first fragment: b[0] is free once these MFMAs on it are issued
            if (f == 0) unpack(Z + 16);
            if (f == 1) dqh(1, 0, 0);
            if (f == 2) dqh(1, 0, 1);
            if (f == 1) {   // substep 1's first-half A fragments (their registers' MFMAs are all issued)
#pragma unroll
              for (int m = 0; m < H1; ++m) af1[m] = rda(1, m);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    // 4-stage ring (q: 4 register sets), three steps ahead: before step j, steps j+1 and j+2 may be in flight.
    u32x4_t qa[VM_Q], qb[VM_Q], qc[VM_Q], qe[VM_Q];
    u32x4_t* const qs[4] = {qa, qb, qc, qe};
    auto step = [&](int j, int st) {
      wait_vm_lds<q4_wait(SZ2)>();
      __builtin_amdgcn_s_barrier();
      issue_lds(j + 3, (st + 3) & 3, qs[(st + 3) & 3]);
      compute(st, qs[st]);
    };
    issue_lds(0, 0, qa);
    issue_lds(1, 1, qb);
    issue_lds(2, 2, qc);
    int i = 0;
    for (; i + 4 <= nk; i += 4) {   // whole rounds of 4 steps, then the 0-3 remaining ones
      step(i, 0);
      step(i + 1, 1);
      step(i + 2, 2);
      step(i + 3, 3);
    }
    if (i < nk) {
      step(i, 0);
      if (i + 1 < nk) {
        step(i + 1, 1);
        if (i + 2 < nk) step(i + 2, 2);
      }
    }
  } else {
    auto mma = [&](const uint16_t* S, int s, const u32x4_t* b) {
#pragma unroll
      for (int m = 0; m < NRF; ++m) {
        const u32x4_t af = *reinterpret_cast<const u32x4_t*>(S + ard[s] + m * 16 * KT);
#pragma unroll
        for (int f = 0; f < 4; ++f) acc[m][f] = mfma16(af, b[f], acc[m][f]);
      }
    };
    // bf16 weights: 8 loads per wave and step (2 pairs x 2 fragments x 2 substeps), one step ahead in two
    // alternating register sets; A three steps ahead in a 4-stage ring. Issue order W(j+1), A(j+3): before step j
    // only A(j+2)'s 4 loads may still be in flight.
    u32x4_t bA[2][4], bB[2][4];   // [substep][column fragment]
    static_assert(VM_B == 2 * 4, "2 substeps x 4 column fragments");
    auto issue_b = [&](int j, u32x4_t (*b)[4]) {
      const bool in = j < nk;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int fr = 0; fr < 2; ++fr) {
          b[s][fr] = ld16(rw, in ? wo + j * 4096 + (2 * fr + s) * 1024 : OOB);
          b[s][2 + fr] = ld16(rw1, in ? wo + j * 4096 + (2 * fr + s) * 1024 : OOB);
        }
    };
    // The step's 2 NRF A-fragment reads in (substep, fragment) order through a ring of three registers, two reads
    // ahead of the MFMAs that use them (the weights sit in registers already); the fences keep the scheduler from
    // sinking the reads back to their uses.
    auto compute = [&](int st, u32x4_t (*b)[4]) {
      const uint16_t* S = St(st);
      constexpr int NR = 2 * NRF;
      auto rd = [&](int r) {
        return *reinterpret_cast<const u32x4_t*>(S + ard[r / NRF] + (r % NRF) * 16 * KT);
      };
      u32x4_t ar[3];
      ar[0] = rd(0);
      ar[1] = rd(1);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int s = r / NRF, m = r % NRF;
        if (r + 2 < NR) ar[(r + 2) % 3] = rd(r + 2);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < 4; ++f) acc[m][f] = mfma16(ar[r % 3], b[s][f], acc[m][f]);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    issue_lds(0, 0, nullptr);
    issue_lds(1, 1, nullptr);
    issue_b(0, bA);
    issue_lds(2, 2, nullptr);
    for (int i = 0; i < nk; i += 4) {
      wait_vm_lds<BF_WAIT>();
      __builtin_amdgcn_s_barrier();
      issue_b(i + 1, bB);
      issue_lds(i + 3, 3, nullptr);
      compute(0, bA);
      wait_vm_lds<BF_WAIT>();
      __builtin_amdgcn_s_barrier();
      issue_b(i + 2, bA);
      issue_lds(i + 4, 0, nullptr);
      if (i + 1 < nk) compute(1, bB);   // steps past K: loads of zeros, no compute
      wait_vm_lds<BF_WAIT>();
      __builtin_amdgcn_s_barrier();
      issue_b(i + 3, bB);
      issue_lds(i + 5, 1, nullptr);
      if (i + 2 < nk) compute(2, bA);
      wait_vm_lds<BF_WAIT>();
      __builtin_amdgcn_s_barrier();
      issue_b(i + 4, bA);
      issue_lds(i + 6, 2, nullptr);
      if (i + 3 < nk) compute(3, bB);
    }
  }
  wait_vm<0>();   // the ring's trailing (out-of-range) loads
  // ---- LoRA K-extension: ext[row][32 c : 32 c + 32] . Eb[c][n][0:32], one 32-wide substep per plane c (two planes
  // for a gate_up LoRA of rank 17..32: the gate and the up products add up)
  const int planes = (ws.flags & SMEL_WSET_EXT2) ? 2 : 1;   // uniform
  const uint16_t* eb = kind == SMEL_KIND_SEL ? (ws.ext_sel ? ws.ext_sel + (int64_t)idx * planes * N * 32 : nullptr)
                                             : (kind == SMEL_KIND_SHARED ? ws.ext_sh : nullptr);
  // xpart: the rows come as the down backward's per-column-block fp32 partials, summed here in block order
  const bool xpart = EPI == 0 && a.lr_on;
  if ((a.ext || xpart) && eb) {
    const uint32_t xb = 64u * planes;   // ext row bytes
    const rsrc_t re = make_rsrc(eb, (uint64_t)planes * N * 64);
    const rsrc_t rx = make_rsrc(a.ext ? a.ext + (int64_t)row0 * (xb / 2) : nullptr, a.ext ? (uint64_t)nrows * xb : 0);
    // partials: summed once per tile into a bf16 tile X [128][32 planes] in ring stage 0 (free now), every load of a
    // thread in flight at once, then read like the ext rows
    uint16_t* const X = reinterpret_cast<uint16_t*>(smem);
    if (xpart) {
      const int P = a.lr.parts;
      const rsrc_t rp = make_rsrc(a.lr.part + (int64_t)row0 * P * planes * 32, (uint64_t)nrows * P * planes * 128);
      __syncthreads();   // every wave's ring loads have landed and its fragment reads returned
      const int xr = tid >> 2, xj = 8 * (tid & 3);   // rows xr and xr + 64, values xj .. xj + 7 of a plane
      for (int c = 0; c < planes; ++c) {
        float v[2][8] = {};
        for (int p0 = 0; p0 < P; p0 += 2) {
          u32x4_t x[2][2][2];
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              const int row = xr + 64 * h, p = p0 + q;
              const uint32_t o =
                  (row < nrows && p < P) ? (uint32_t)(((row * P + p) * planes + c) * 128 + 4 * xj) : OOB;
              x[h][q][0] = ld16(rp, o);
              x[h][q][1] = ld16(rp, o == OOB ? OOB : o + 16);
            }
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int q = 0; q < 2; ++q)   // p ascending; a p past P reads zeros
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                v[h][t] += __uint_as_float(x[h][q][0][t]);
                v[h][4 + t] += __uint_as_float(x[h][q][1][t]);
              }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<u32x4_t*>(X + (xr + 64 * h) * 32 * planes + 32 * c + xj) =
              u32x4_t{pack2bf(v[h][0], v[h][1]), pack2bf(v[h][2], v[h][3]), pack2bf(v[h][4], v[h][5]),
                      pack2bf(v[h][6], v[h][7])};
      }
      __syncthreads();
    }
    for (int c = 0; c < planes; ++c) {
      u32x4_t b[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int n = cw + 16 * f + li;
        b[f] = ld16(re, (cw + 16 * f < N) ? (uint32_t)(c * N + n) * 64 + 16 * kq : OOB);
      }
#pragma unroll
      for (int m = 0; m < NRF; ++m) {
        const int row = m * 16 + li;
        u32x4_t af;
        if (xpart) {
          af = *reinterpret_cast<const u32x4_t*>(X + row * 32 * planes + 32 * c + 8 * kq);
        } else {
          af = ld16(rx, row < nrows ? (uint32_t)row * xb + 64 * c + 16 * kq : OOB);
        }
#pragma unroll
        for (int f = 0; f < 4; ++f) acc[m][f] = mfma16(af, b[f], acc[m][f]);
      }
    }
  }
  // ---- epilogue through LDS (the ring is free after the loop): every lane writes its results, rounded to bf16, into a
  // row-major tile [128][256] (rows 32 m .. 32 m + 31 in stage m; 16-B chunk c of row r at c ^ (r & 7)), then each
  // thread handles 8 columns of whole rows with 16-B accesses.
  __syncthreads();   // every wave is done with the ring (its loads landed, its reads returned)
#pragma unroll
  for (int m = 0; m < NRF; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * m + 4 * kq + r;   // D[4 kq + r][li] of the fragment
      const int lr = row & 31;
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int col = 64 * w + 16 * f + li;
        Et(row >> 5)[lr * 256 + 8 * ((col >> 3) ^ (lr & 7)) + (col & 7)] = f2bf(acc[m][f][r]);
      }
    }
  // per-row slot / weight table right after the staged tile (inside the ring, free now)
  int* const rowmap = reinterpret_cast<int*>(smem + 4 * A_BYTES);
  if (tid < MT) {
    if (EPI == 0)
      rowmap[tid] = ep_slot;
    else
      reinterpret_cast<float*>(rowmap)[tid] = ep_w;
  }
  __syncthreads();
  // thread -> (row, 8-column chunk): 32 threads per row, 8 rows per pass
  const int ch = tid & 31;
  const int col0 = nb * NB + 8 * ch;
  if (EPI == 0) {
    if (col0 < N) {
      for (int row = tid >> 5; row < nrows; row += 8) {
        const int lr = row & 31;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(Et(row >> 5) + lr * 256 + 8 * (ch ^ (lr & 7)));
        const int64_t orow = rowmap[row];
        *reinterpret_cast<u32x4_t*>(a.out + orow * a.ldo + col0) = v;
      }
    }
    return;
  }
  // down backward, columns n < I of dh = [dg | du]: per row, da = w(row) acc, (g, u) = hsave, dg = da u act'(g),
  // du = da act(g), and the row's partial of sum_n acc * bf16(act(g) u) over this block's columns -> dwp. The
  // forward's activation bf16(act(g) u) is recomputed from the saved bf16 (g, u) with the forward epilogue's own
  // operations (act_f and act_and_grad_f share the sigmoid / tanh form), so it is the value the forward stored.
  const int I = N;
  const bool cv = col0 < I;
  const float* const wmap = reinterpret_cast<const float*>(rowmap);
  // 32 threads per row, 8 rows per pass; the saved (g, u) of PB passes are loaded before any of them is used, so the
  // stores of one batch never wait for the loads of the next row.
  constexpr int PB = 8;
  const int act = a.act;
  {
    for (int rb = tid >> 5; rb < nrows; rb += 8 * PB) {
      u32x4_t g2s[PB], u2s[PB];
#pragma unroll
      for (int p = 0; p < PB; ++p) {
        const int64_t grow = row0 + rb + 8 * p;
        g2s[p] = u2s[p] = u32x4_t{};
        if (cv && rb + 8 * p < nrows) {
          g2s[p] = *reinterpret_cast<const u32x4_t*>(a.hsave + grow * 2 * I + col0);
          u2s[p] = *reinterpret_cast<const u32x4_t*>(a.hsave + grow * 2 * I + I + col0);
        }
      }
#pragma unroll
      for (int p = 0; p < PB; ++p) {
        const int row = rb + 8 * p;
        if (row >= nrows) break;   // uniform over the row's 32 threads
        const int lr = row & 31;
        const u32x4_t av = *reinterpret_cast<const u32x4_t*>(Et(row >> 5) + lr * 256 + 8 * (ch ^ (lr & 7)));
        const int grow = row0 + row;
        const float wrow_ = wmap[row];
        float part = 0.f;
        if (cv) {
          const u32x4_t g2 = g2s[p], u2 = u2s[p];
          uint32_t og[4], ou[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float dgv[2], duv[2], avl[2], dav[2], uv[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              uv[h] = h ? bf_hi(u2[j]) : bf_lo(u2[j]);
              act_and_grad_f(h ? bf_hi(g2[j]) : bf_lo(g2[j]), act, avl[h], dav[h]);
            }
            const uint32_t a2 = pack2bf(avl[0] * uv[0], avl[1] * uv[1]);   // the forward's rounded activation
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const float acv = h ? bf_hi(av[j]) : bf_lo(av[j]);
              part += acv * (h ? bf_hi(a2) : bf_lo(a2));
              const float da = wrow_ * acv;
              dgv[h] = da * uv[h] * dav[h];
              duv[h] = da * avl[h];
            }
            og[j] = pack2bf(dgv[0], dgv[1]);
            ou[j] = pack2bf(duv[0], duv[1]);
          }
          *reinterpret_cast<u32x4_t*>(a.out + (int64_t)grow * a.ldo + col0) = u32x4_t{og[0], og[1], og[2], og[3]};
          *reinterpret_cast<u32x4_t*>(a.out + (int64_t)grow * a.ldo + I + col0) =
              u32x4_t{ou[0], ou[1], ou[2], ou[3]};
        }
        // fixed-order sum over the row's 32 threads (lanes 32 h .. 32 h + 31 of a wave)
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) part += __shfl_xor(part, o, 64);
        if (ch == 0) a.dwp[(int64_t)grow * a.nblk + nb] = part;
      }
    }
  }
  // ---- the gate_up backward's LoRA rows of this tile (SEL / SHARED with a LoRA): this block's partial of
  // s [dg, du] bt^T over its columns, part[row][nb][c][j]. The K of 512 (this block's 256 dg columns, then its 256 du
  // columns, read back from the rows just stored) goes in 4 chunks of 128 columns through LDS: the dh rows and bt rows
  // of every chunk are loaded coalesced (16-B pieces of whole row segments) into registers at once, then per chunk
  // wave w multiplies rows 32 w .. 32 w + 31 by them (MFMA 32x32x16, one accumulator per plane).
  if (!a.lr_on) return;
  const uint16_t* bt = kind == SMEL_KIND_SEL ? a.lr.bt_sel : (kind == SMEL_KIND_SHARED ? a.lr.bt_sh : nullptr);
  if (!bt) return;   // uniform
  const int64_t I2 = 2 * (int64_t)I;
  const int64_t pstride = (kind == SMEL_KIND_SEL ? (int64_t)a.lr.n_sel : 1) * 32 * I2;   // one plane
  if (kind == SMEL_KIND_SEL) bt += (int64_t)idx * 32 * I2;
  const float sc = kind == SMEL_KIND_SEL ? a.lr.scale_sel : a.lr.scale_sh;
  const int P = a.lr.parts, gplanes = a.lr.planes;   // the gate_up side's planes
  constexpr int DP = 128 + 8;                         // LDS row pitch (bf16): 272 B
  uint16_t* const D = reinterpret_cast<uint16_t*>(smem);   // dh chunk [128][DP]
  uint16_t* const Bs = D + MT * DP;                         // bt chunk [planes][32][DP]
  static_assert(MT * DP * 2 + 2 * 32 * DP * 2 <= smem_bytes(false), "LoRA-row chunks fit in the ring");
  const rsrc_t rd = make_rsrc(a.out + (int64_t)row0 * a.ldo, (uint64_t)nrows * a.ldo * 2);
  const rsrc_t rb0 = make_rsrc(bt, (uint64_t)32 * I2 * 2);
  const rsrc_t rb1 = make_rsrc(gplanes > 1 ? bt + pstride : bt, gplanes > 1 ? (uint64_t)32 * I2 * 2 : 0);
  const int gch = tid & 15, grow = tid >> 4;   // this thread's 16-B pieces: rows grow + 16 i, columns 8 gch ..
  // chunk q: columns (q < 2 ? 0 : I) + nb * 256 + 128 (q & 1) + [0, 128); I is a multiple of 32, so a piece is in or out
  auto piece_ok = [&](int q) { return nb * NB + 128 * (q & 1) + 8 * gch < I; };
  auto piece_col = [&](int q) { return (q >= 2 ? I : 0) + nb * NB + 128 * (q & 1) + 8 * gch; };
  // the bt rows of all 4 chunks before the barrier (they do not depend on this block's stores), the dh rows of all
  // 4 chunks right after it: one memory round trip for the whole projection
  u32x4_t pd[4][8], pb[4][2][2];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t o = piece_ok(q) ? (uint32_t)((grow + 16 * i) * I2 + piece_col(q)) * 2 : OOB;
      pb[q][0][i] = ld16(rb0, o);
      pb[q][1][i] = ld16(rb1, o);
    }
  const int h5 = l >> 5, r32 = l & 31;
  f32x16_t px0 = f32x16_t{}, px1 = f32x16_t{};
  __syncthreads();   // the block's dg / du stores are visible to all of its waves; the staged tile's reads are done
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = grow + 16 * i;
      pd[q][i] = ld16(rd, piece_ok(q) && row < nrows ? (uint32_t)(row * a.ldo + piece_col(q)) * 2 : OOB);
    }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4_t*>(D + (grow + 16 * i) * DP + 8 * gch) = pd[q][i];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      *reinterpret_cast<u32x4_t*>(Bs + (grow + 16 * i) * DP + 8 * gch) = pb[q][0][i];
      *reinterpret_cast<u32x4_t*>(Bs + (32 + grow + 16 * i) * DP + 8 * gch) = pb[q][1][i];
    }
    lds_barrier();
    if (w < NS) {
      const uint16_t* Ar = D + (32 * w + r32) * DP + 8 * h5;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const u32x4_t af = *reinterpret_cast<const u32x4_t*>(Ar + 16 * s);
        px0 = mfma32(af, *reinterpret_cast<const u32x4_t*>(Bs + r32 * DP + 16 * s + 8 * h5), px0);
        if (gplanes > 1)   // uniform
          px1 = mfma32(af, *reinterpret_cast<const u32x4_t*>(Bs + (32 + r32) * DP + 16 * s + 8 * h5), px1);
      }
    }
    lds_barrier();   // this chunk's reads are done before the next one is stored
  }
  if (w >= NS) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int orow = 32 * w + acc_row(r, l);
    if (orow < nrows) {
      float* const o = a.lr.part + (((int64_t)(row0 + orow) * P + nb) * gplanes) * 32 + r32;
      o[0] = sc * px0[r];
      if (gplanes > 1) o[32] = sc * px1[r];
    }
  }
}

template <int EPI, bool Q4, bool SZ2, bool FAST>
SMEL_DEV void run_tile_ns(const BwdArgs& a, int kind, int idx, int row0, int nrows, int nb, uint8_t* smem) {
  switch ((nrows + 31) >> 5) {
    case 1: run_tile<EPI, Q4, 1, SZ2, FAST>(a, kind, idx, row0, nrows, nb, smem); break;
    case 2: run_tile<EPI, Q4, 2, SZ2, FAST>(a, kind, idx, row0, nrows, nb, smem); break;
    case 3: run_tile<EPI, Q4, 3, SZ2, FAST>(a, kind, idx, row0, nrows, nb, smem); break;
    default: run_tile<EPI, Q4, 4, SZ2, FAST>(a, kind, idx, row0, nrows, nb, smem); break;
  }
}

template <int EPI, bool SZ2>
SMEL_DEV void gmm_bwd_body(const BwdArgs& a, uint8_t* smem) {
  int tile, nb;
  if (!((a.w.flags & SMEL_WSET_XCD_CHUNK) ? xcd_tile_chunk(a.n_tiles[0], a.nblk, tile, nb)
                                          : xcd_tile(a.n_tiles[0], a.nblk, tile, nb)))
    return;
  const int4 t = a.tiles[tile];
  const int gk = a.gkind ? a.gkind[t.x] : t.w;   // the tile list may carry the group kind itself
  const int kind = gk >> 16, idx = gk & 0xffff;
  const int nrows = min(t.z - t.y, MT);
  if (nrows <= 0) return;
  if (kind == SMEL_KIND_INT4) {
    if (a.w.flags & SMEL_WSET_FAST_DQ)
      run_tile_ns<EPI, true, SZ2, true>(a, kind, idx, t.y, nrows, nb, smem);
    else
      run_tile_ns<EPI, true, SZ2, false>(a, kind, idx, t.y, nrows, nb, smem);
  } else {
    run_tile_ns<EPI, false, false, false>(a, kind, idx, t.y, nrows, nb, smem);
  }
}

template <int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gmm_bwd_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[smem_bytes(false)];
  gmm_bwd_body<EPI, false>(a, smem);
}

// An int4 group of 32 columns (the 64 columns of a wave span two scale/zero groups): the larger ring allows one
// block per CU.
template <int EPI>
__global__ __launch_bounds__(256) void gmm_bwd_kernel_sz2(BwdArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[smem_bytes(true)];
  gmm_bwd_body<EPI, true>(a, smem);
}

}  // namespace

extern "C" int64_t smel_gmm_bwd_nblocks(int64_t C) { return (C + NB - 1) / NB; }

extern "C" int smel_gmm_bwd_lr(const smel_wset* w, const int32_t* gkind, const int32_t* tiles,
                               const int32_t* n_tiles, int64_t max_tiles, const uint16_t* A, int64_t lda,
                               int64_t a_rows, int32_t a_gather, const int32_t* order, int64_t TK, int64_t topk,
                               const uint16_t* ext, int32_t epilogue, int32_t act, const uint16_t* hsave,
                               const float* topv, const float* sgate, uint16_t* out, int64_t ldo, float* dwp,
                               const smel_bwd_lora_rows* lr, hipStream_t stream) {
  SMEL_REQUIRE(w && tiles && n_tiles && A && out, SMEL_EINVAL, "gmm_bwd: null pointer");
  SMEL_REQUIRE(w->R > 0 && w->C > 0 && max_tiles >= 0 && lda >= w->R && topk > 0, SMEL_EINVAL,
               "gmm_bwd: bad sizes");
  SMEL_REQUIRE(w->R % 64 == 0 && w->C % 32 == 0, SMEL_EUNSUPPORTED,
               "gmm_bwd: weight dims %lldx%lld must be multiples of 64 x 32", (long long)w->R, (long long)w->C);
  SMEL_REQUIRE(!w->q4 || (w->group % 32 == 0 && w->C % w->group == 0), SMEL_EUNSUPPORTED,
               "gmm_bwd: int4 group %d must be a multiple of 32 dividing the columns", w->group);
  SMEL_REQUIRE(!w->q4 || w->sz4, SMEL_EINVAL,
               "gmm_bwd: an int4 bank needs its transposed scale/zero (smel_pack_int4_t)");
  SMEL_REQUIRE(lda % 8 == 0 && ((uintptr_t)A % 16) == 0, SMEL_EUNSUPPORTED, "gmm_bwd: A rows must be 16-B aligned");
  SMEL_REQUIRE(ldo % 8 == 0 && ((uintptr_t)out % 16) == 0 && ((uintptr_t)hsave % 16) == 0, SMEL_EUNSUPPORTED,
               "gmm_bwd: out / hsave rows must be 16-B aligned");
  SMEL_REQUIRE(epilogue == 0 || (epilogue == 1 && hsave && dwp && (topv || TK == 0)), SMEL_EINVAL,
               "gmm_bwd: epilogue %d needs hsave, dwp and topv", epilogue);
  SMEL_REQUIRE(!a_gather || order || TK == 0, SMEL_EINVAL, "gmm_bwd: gather needs order");
  SMEL_REQUIRE(!(w->flags & SMEL_WSET_EXT2) || epilogue == 0, SMEL_EINVAL,
               "gmm_bwd: a two-plane LoRA extension belongs to the gate_up backward (epilogue 0)");
  SMEL_REQUIRE(act == 0 || act == 1, SMEL_EINVAL, "gmm_bwd: act %d", act);
  SMEL_REQUIRE(a_rows >= 0 && a_rows * lda * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "gmm_bwd: A larger than 2 GiB");
  SMEL_REQUIRE(w->R * w->C * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "gmm_bwd: one weight matrix larger than 2 GiB");
  if (lr && lr->part) {
    SMEL_REQUIRE(lr->planes == 1 || lr->planes == 2, SMEL_EINVAL, "gmm_bwd: LoRA-row planes %d", lr->planes);
    SMEL_REQUIRE(((uintptr_t)lr->part % 16) == 0, SMEL_EUNSUPPORTED, "gmm_bwd: LoRA-row partials must be 16-B aligned");
    if (epilogue == 1) {
      SMEL_REQUIRE(lr->parts == smel_gmm_bwd_nblocks(w->C), SMEL_EINVAL,
                   "gmm_bwd: %d LoRA-row partials per row (the down backward's column blocks: %lld)", lr->parts,
                   (long long)smel_gmm_bwd_nblocks(w->C));
      SMEL_REQUIRE(ldo >= 2 * w->C && (!lr->bt_sel || lr->n_sel > 0), SMEL_EINVAL,
                   "gmm_bwd: LoRA rows need the dh rows [rows][2 I] and the selected slots' count");
    } else {
      SMEL_REQUIRE(!ext && lr->parts >= 1, SMEL_EINVAL, "gmm_bwd: LoRA-row partials replace ext (pass NULL)");
      SMEL_REQUIRE(lr->planes == ((w->flags & SMEL_WSET_EXT2) ? 2 : 1), SMEL_EINVAL,
                   "gmm_bwd: LoRA-row planes %d against the weight set's extension", lr->planes);
    }
  }
  if (max_tiles == 0) return 0;
  BwdArgs a;
  a.lr_on = lr && lr->part;
  if (a.lr_on) a.lr = *lr;
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
  const bool sz2 = w->q4 && w->group % 64 != 0;
  if (sz2) {
    if (epilogue == 1)
      gmm_bwd_kernel_sz2<1><<<grid, 256, 0, stream>>>(a);
    else
      gmm_bwd_kernel_sz2<0><<<grid, 256, 0, stream>>>(a);
  } else {
    if (epilogue == 1)
      gmm_bwd_kernel<1><<<grid, 256, 0, stream>>>(a);
    else
      gmm_bwd_kernel<0><<<grid, 256, 0, stream>>>(a);
  }
  return smel::launch_status();
}

extern "C" int smel_gmm_bwd(const smel_wset* w, const int32_t* gkind, const int32_t* tiles, const int32_t* n_tiles,
                            int64_t max_tiles, const uint16_t* A, int64_t lda, int64_t a_rows, int32_t a_gather,
                            const int32_t* order, int64_t TK, int64_t topk, const uint16_t* ext, int32_t epilogue,
                            int32_t act, const uint16_t* hsave, const float* topv, const float* sgate,
                            uint16_t* out, int64_t ldo, float* dwp, hipStream_t stream) {
  return smel_gmm_bwd_lr(w, gkind, tiles, n_tiles, max_tiles, A, lda, a_rows, a_gather, order, TK, topk, ext,
                         epilogue, act, hsave, topv, sgate, out, ldo, dwp, nullptr, stream);
}
