// Grouped expert GEMM, forward (out = A W^T per group): the gate_up and down projections of every expert, frozen
// (int4 group-64, dequantized in registers inside the main loop — no bf16 copy of a frozen expert is ever written)
// or selected / shared (bf16 + LoRA as a 32-wide K-extension), with the token gather fused into the A load and the
// SiLU-gate fused into the gate_up epilogue.
// Reference: frozen_experts_forward / _gmm / _selected_expert / lora_gate_up / lora_linear,
// smel/moe.py:58-72, 110-117, 204-211 and smel/lora.py:61-83.
//
// Block = 4 waves, tile = up to 128 rows of one group (4 slices of 32) x (gate_up: 32 gate + 32 up columns per wave;
// down: 64 columns per wave); a tile of an int4 group also takes up to 160 rows (5 slices) when a full tile and the
// group's last tile of at most 32 rows are merged (SMEL_WSET_MERGED_LIST, both projections; SMEL_WSET_MERGE_SHORT,
// gate_up only): the weights are then streamed and dequantized once for all of the group's rows. MFMA 32x32x16 bf16.
// Per 64-wide k-step:
//  * A (activation rows, gathered by token) goes global -> LDS directly (16-B LDS-DMA loads, 1 KB per wave-load, no
//    registers), into a ring of 4 stages; each 128-B row's 16-B chunks are XOR-swizzled so the fragment reads are
//    bank-conflict free. Every wave reads all rows of a stage.
//  * every wave streams its own two 32-row weight fragments straight into registers from the fragment layout of
//    smel_pack_int4 / smel_pack_bf16 (one contiguous 1-KB load per fragment and k-step) and dequantizes int4 there,
//    so each weight element of a tile is read and dequantized once (dq8, or dq8f for a bank with the
//    SMEL_WSET_FAST_DQ flag: the same values in fewer instructions).
//  * loads run 3 k-steps ahead (int4: a 4-deep register ring; bf16: 1 step ahead, as its fragments are 4x larger).
//    vmcnt retires in issue order, so each step issues its weight loads before its A loads and waits, before one
//    barrier, for exactly the loads of the step it is about to use.
// Lane k-mapping inside a k-step: lane half h = lane/32 carries k = 32h + 8s + [0,8) in substep s, for A and B alike.
#include "abi_util.h"
#include "common.h"

namespace {

constexpr int MT = 128;            // rows of a tile of the tile list
constexpr int MT_MERGED = 160;     // rows of a merged tile: a full tile + a last tile of <= 32 rows
constexpr int KT = 64;
// An A stage holds MT_MERGED rows (row r at r * KT bf16, no padding; the four stages are contiguous). The gate_up
// epilogue keeps the g and u tiles of 160 x 128 in them; the down epilogue its output tile. A tile of at most MT rows
// leaves rows MT.. of every stage alone: the down projection keeps its LoRA rows (stages 0 and 1) and its rows'
// output slots (stage 2) there.
constexpr int STAGE = MT_MERGED * KT;   // bf16 elements of a stage
constexpr int SPARE = MT * KT;          // first element of a stage's rows past MT

// Vector-memory operations per wave in each issue group of the main loops; the issue code below is written with
// these counts and every wait is computed from them (vmcnt retires in issue order).
// A rows of a stage: 1-KB LDS-DMA wave-loads of 8 rows; with 4 waves, 4 per wave cover 128 rows, 5 cover 160.
constexpr int vm_a(int ns) { return ns > 4 ? 5 : 4; }
constexpr int VM_Q = 2;                           // int4: one 16-B word per weight fragment, 2 fragments
constexpr int VM_SZ = 2;                          // int4: a scale/zero run (16 B) or pair (4 B), per fragment
constexpr int VM_B = 2 * 4;                       // bf16: 4 substep chunks per fragment, 2 fragments
// int4, tiles of up to 4 slices: the group of step j carries the packed scale/zero run of steps j..j+3 iff j % 4 ==
// 0; after the barrier of step j the group of step j+3 is issued; while step j (round position pos = j % 4) computes,
// the groups of steps j+1 and j+2 may still be in flight (four sets of weight registers)
constexpr int q4_group(int j, int vma) { return VM_Q + (j % 4 == 0 ? VM_SZ : 0) + vma; }
constexpr int q4_wait(int pos, int vma) { return q4_group(pos + 1, vma) + q4_group(pos + 2, vma); }
// int4, 5-slice (merged) tiles, whose accumulators leave room for three sets of weight registers only: after the
// barrier of step j the group [q, scale/zero of step j+2 | A of step j+3] is issued. Before step j computes it needs
// q(j) (group of step j-2) and A(j) (group of step j-3): A(j+1) and the whole group of step j-1 may still be in flight.
constexpr int q4_wait_w2(int vma) { return vma + (VM_Q + VM_SZ + vma); }
// bf16: issue order ... B(j+1), A(j+3): before step j only the last group, A(j+2), may be in flight

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
  smel_fwd_lora_rows lr;   // down-LoRA rows: produced by the gate_up epilogue, taken by the down K-extension
  bool lr_on;
};

template <int EPI, bool Q4, int NS, bool FAST>
SMEL_DEV void run_tile(const FwdArgs& a, int kind, int idx, int row0, int nrows, int nb, uint16_t* S0, uint16_t* S1,
                       uint16_t* S2, uint16_t* S3, int* rowmap, uint16_t* X) {
  static_assert(NS * 32 <= MT_MERGED, "the tile's rows fit the A stages");
  constexpr int VMA = vm_a(NS);               // A wave-loads per wave and stage
  constexpr int BF_WAIT = VMA;                // bf16: issue order ... B(j+1), A(j+3): before step j only A(j+2)
  const int tid = threadIdx.x, l = lane_id(), hi = l >> 5, r32 = l & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = a.K;
  const smel_wset& ws = a.w;
  // output slot of tile row t (thread t < MT) for the down projection, fetched now so that no load sits between the
  // epilogue's stores
  int ep_slot = 0;
  if (EPI == 0 && NS <= 4 && tid < nrows) ep_slot = row_slot(row0 + tid, a.order, a.TK);
  // ---- this wave's two 32-row weight fragments: gate/up pair for epilogue 1, two adjacent fragments else
  int n0, n1, fr0, fr1;
  bool fv0, fv1;
  if (EPI == 1) {
    const int I = a.N / 2;
    const int c0 = nb * 128 + w * 32;
    fv0 = fv1 = c0 < I;
    n0 = c0 + r32;
    n1 = I + c0 + r32;
    fr0 = c0 / 32;
    fr1 = (I + c0) / 32;
  } else {
    const int c0 = nb * 256 + w * 64;
    fv0 = c0 < a.N;
    fv1 = c0 + 32 < a.N;
    n0 = c0 + r32;
    n1 = c0 + 32 + r32;
    fr0 = c0 / 32;
    fr1 = c0 / 32 + 1;
  }
  const int nk = (K + KT - 1) / KT, nk4 = (nk + 3) / 4;
  const int nfr = a.N / 32;   // fragments of one matrix
  rsrc_t rw, rsz;
  uint32_t wo0, wo1, so0 = OOB, so1 = OOB;
  if constexpr (Q4) {
    rw = make_rsrc(ws.q4 + (int64_t)idx * nfr * nk * 1024, (uint64_t)nfr * nk * 1024);
    rsz = make_rsrc(ws.sz4 + (int64_t)idx * nfr * nk4 * 256, (uint64_t)nfr * nk4 * 1024);
    wo0 = fv0 ? (uint32_t)(fr0 * nk * 1024 + l * 16) : OOB;
    wo1 = fv1 ? (uint32_t)(fr1 * nk * 1024 + l * 16) : OOB;
    so0 = fv0 ? (uint32_t)(fr0 * nk4 * 1024 + l * 16) : OOB;
    so1 = fv1 ? (uint32_t)(fr1 * nk4 * 1024 + l * 16) : OOB;
  } else {
    const uint16_t* base = kind == SMEL_KIND_BF16 ? ws.wb : (kind == SMEL_KIND_SEL ? ws.wsel : ws.wsh);
    const int64_t mi = kind == SMEL_KIND_SHARED ? 0 : idx;
    rw = make_rsrc(base + mi * nfr * nk * 2048, (uint64_t)nfr * nk * 4096);
    rsz = rw;
    wo0 = fv0 ? (uint32_t)(fr0 * nk * 4096 + l * 16) : OOB;
    wo1 = fv1 ? (uint32_t)(fr1 * nk * 4096 + l * 16) : OOB;
  }
  // ---- down LoRA rows from the gate_up forward's per-column-block partials (LoRA tiles of the down projection):
  // summed in block order into the bf16 tile X [128][32] before the main loop (no accumulator is live yet; rows 0..63
  // at X, rows 64..127 at X + STAGE: the spare rows of stages 0 and 1); the same rows in every column block of the
  // tile, column block 0 also stores them for the LoRA gradients
  if (EPI == 0 && a.lr_on && a.lr.part &&
      ((kind == SMEL_KIND_SEL && ws.ext_sel) || (kind == SMEL_KIND_SHARED && ws.ext_sh))) {
    const int P = a.lr.parts;
    const rsrc_t rp = make_rsrc(a.lr.part + (int64_t)row0 * P * 32, (uint64_t)nrows * P * 128);
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {   // 256 threads x 8 values x 2 passes = 128 rows x 32
      const int row = (tid >> 2) + 64 * pass, k0 = 8 * (tid & 3);
      float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int p = 0; p < P; ++p) {
        const uint32_t o = row < nrows ? (uint32_t)((row * P + p) * 32 + k0) * 4 : OOB;
        const u32x4_t x0 = ld16(rp, o), x1 = ld16(rp, o == OOB ? OOB : o + 16);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          v[t] += __uint_as_float(x0[t]);
          v[4 + t] += __uint_as_float(x1[t]);
        }
      }
      const u32x4_t h = u32x4_t{pack2bf(v[0], v[1]), pack2bf(v[2], v[3]), pack2bf(v[4], v[5]), pack2bf(v[6], v[7])};
      *reinterpret_cast<u32x4_t*>(X + pass * STAGE + (row & 63) * 32 + k0) = h;
      if (nb == 0 && a.lr.ext_out && row < nrows)
        *reinterpret_cast<u32x4_t*>(a.lr.ext_out + (int64_t)(row0 + row) * 32 + k0) = h;
    }
    lds_barrier();
  }
  // ---- A staging: wave-load ii of wave w fills rows 8 g .. 8 g + 7 (g = VMA w + ii) of a stage, 1 KB; lane i writes
  // physical chunk i % 8 of row 8 g + i / 8, i.e. logical chunk c = (i % 8) ^ swz(row).
  const rsrc_t ra = make_rsrc(a.A, (uint64_t)a.a_rows * a.lda * 2);
  const int li = tid & 63;
  // Tiles of up to 4 slices keep each chunk's first k (akc) for the K tail; a merged 5-slice tile exists only for K a
  // multiple of 64 (every chunk of an in-range step is inside the row) and keeps no such registers.
  constexpr bool TAIL = NS <= 4;
  uint32_t aoff[VMA];
  int akc[TAIL ? VMA : 1];   // first k of this lane's chunk
#pragma unroll
  for (int ii = 0; ii < VMA; ++ii) {
    const int row = 8 * (VMA * w + ii) + (li >> 3);
    const int c = (li & 7) ^ swz(row);
    if constexpr (TAIL) akc[ii] = 8 * c;
    aoff[ii] = OOB;
    if (row < nrows) {
      const int grow = row0 + row;
      const int src = a.a_gather ? row_token(grow, a.order, a.TK, a.topk) : grow;
      aoff[ii] = (uint32_t)src * (uint32_t)a.lda * 2 + 16 * c;
    }
  }
  auto issue_a = [&](int j, uint16_t* S) {
    const int k0 = j * KT;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ii = 0; ii < VMA; ++ii) {
      if constexpr (TAIL)
        ld16_lds(ra, S + (VMA * w + ii) * 512, (k0 + akc[ii] + 8 <= K) ? aoff[ii] + k0 * 2 : OOB);
      else
        ld16_lds(ra, S + (VMA * w + ii) * 512, aoff[ii] + k0 * 2);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // A fragment reads: lane (r32, h) of slice m, substep s reads logical chunk 4 h + s of row 32 m + r32
  uint32_t ard[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) ard[s] = r32 * KT + 8 * ((4 * hi + s) ^ swz(r32));

  f32x16_t acc[NS][2];
#pragma unroll
  for (int m = 0; m < NS; ++m) acc[m][0] = acc[m][1] = f32x16_t{};

  // A fragment of slice m, substep s from a stage
  auto rd = [&](const uint16_t* S, int s, int m) {
    return *reinterpret_cast<const u32x4_t*>(S + ard[s] + m * 32 * KT);
  };
  auto mma = [&](const uint16_t* S, int s, const u32x4_t& b0, const u32x4_t& b1) {
#pragma unroll
    for (int m = 0; m < NS; ++m) {
      const u32x4_t af = *reinterpret_cast<const u32x4_t*>(S + ard[s] + m * 32 * KT);
      acc[m][0] = mfma32(af, b0, acc[m][0]);
      acc[m][1] = mfma32(af, b1, acc[m][1]);
    }
  };

  if constexpr (Q4 && NS <= 4) {
    // Group of loads for step j: q (2), then, when j % 4 == 0, the packed (scale, zero) run of steps j..j+3 (2),
    // then A (VMA). Groups j+1, j+2 are in flight while step j computes; group j+3 is issued after its barrier.
    static_assert(VM_Q == 2 && VM_SZ == 2, "one q word and one scale/zero run per fragment, 2 fragments");
    u32x4_t q0[VM_Q], q1[VM_Q], q2[VM_Q], q3[VM_Q], szc[VM_SZ], szn[VM_SZ];
    const uint32_t wof[VM_Q] = {wo0, wo1}, sof[VM_SZ] = {so0, so1};
    auto issue = [&](int j, u32x4_t* q, u32x4_t* z, uint16_t* S) {
      const bool in = j < nk;
#pragma unroll
      for (int f = 0; f < VM_Q; ++f) q[f] = ld16(rw, in ? wof[f] + j * 1024 : OOB);
      if (z) {   // exactly the steps with j % 4 == 0 (q4_group)
        const bool zin = (j >> 2) < nk4;
#pragma unroll
        for (int f = 0; f < VM_SZ; ++f) z[f] = ld16(rsz, zin ? sof[f] + (j >> 2) * 1024 : OOB);
      }
      issue_a(j, S);   // sched barriers keep the group's loads in this order, ahead of the step's compute
    };
    const uint32_t magic = FAST ? f16_magic() : 0u;
    auto compute = [&](const uint16_t* S, const u32x4_t* q, int p) {
      const uint32_t p0 = p == 0 ? szc[0][0] : p == 1 ? szc[0][1] : p == 2 ? szc[0][2] : szc[0][3];
      const uint32_t p1 = p == 0 ? szc[1][0] : p == 1 ? szc[1][1] : p == 2 ? szc[1][2] : szc[1][3];
      const float s0 = bf_lo(p0), z0 = bf_hi(p0), s1 = bf_lo(p1), z1 = bf_hi(p1);
      const FastSZ f0 = fast_sz(s0, z0), f1 = fast_sz(s1, z1);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        uint32_t o0[4], o1[4];
        if constexpr (FAST) {
          dq8f(q[0][s], f0, magic, o0);
          dq8f(q[1][s], f1, magic, o1);
        } else {
          dq8(q[0][s], s0, z0, o0);   // rows / k outside the matrix hold q = s = z = 0 -> exact zeros
          dq8(q[1][s], s1, z1, o1);
        }
        mma(S, s, u32x4_t{o0[0], o0[1], o0[2], o0[3]}, u32x4_t{o1[0], o1[1], o1[2], o1[3]});
      }
    };
    issue(0, q0, szc, S0);
    issue(1, q1, nullptr, S1);
    issue(2, q2, nullptr, S2);
    // ceil(nk / 4) * 4 steps of loads and barriers (a load past K reads zeros); the computes of steps past K are
    // skipped (uniform branches)
    for (int i = 0; i < nk; i += 4) {
      wait_vm_lds<q4_wait(0, VMA)>();
      __builtin_amdgcn_s_barrier();
      issue(i + 3, q3, nullptr, S3);
      compute(S0, q0, 0);
      wait_vm_lds<q4_wait(1, VMA)>();
      __builtin_amdgcn_s_barrier();
      issue(i + 4, q0, szn, S0);
      if (i + 1 < nk) compute(S1, q1, 1);
      wait_vm_lds<q4_wait(2, VMA)>();
      __builtin_amdgcn_s_barrier();
      issue(i + 5, q1, nullptr, S1);
      if (i + 2 < nk) compute(S2, q2, 2);
      wait_vm_lds<q4_wait(3, VMA)>();
      __builtin_amdgcn_s_barrier();
      issue(i + 6, q2, nullptr, S2);
      if (i + 3 < nk) compute(S3, q3, 3);
      szc[0] = szn[0];
      szc[1] = szn[1];
    }
  } else if constexpr (Q4) {
    // 5-slice (merged) tiles: 160 accumulators leave room for three sets of weight registers only, so the weights
    // (q and the step's (scale, zero) pair of each fragment, 4 B: word j % 4 of the packed run) are loaded two steps
    // ahead and A three. In issue order: A(0), [q/z(0) A(1)], [q/z(1) A(2)], then after the barrier of step j
    // [q/z(j+2) A(j+3)].
    static_assert(VM_Q == 2 && VM_SZ == 2, "one q word and one scale/zero pair per fragment, 2 fragments");
    u32x4_t q0[VM_Q], q1[VM_Q], q2[VM_Q], q3[VM_Q];
    uint32_t z0[VM_SZ], z1[VM_SZ], z2[VM_SZ], z3[VM_SZ];
    const uint32_t wof[VM_Q] = {wo0, wo1}, sof[VM_SZ] = {so0, so1};
    auto issue_w = [&](int j, u32x4_t* q, uint32_t* z) {
      const bool in = j < nk;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int f = 0; f < VM_Q; ++f) q[f] = ld16(rw, in ? wof[f] + j * 1024 : OOB);
#pragma unroll
      for (int f = 0; f < VM_SZ; ++f) z[f] = ld4(rsz, in ? sof[f] + (j >> 2) * 1024 + 4 * (j & 3) : OOB);
    };
    const uint32_t magic = FAST ? f16_magic() : 0u;
    // The A fragment of slice m + 1 (or of the next substep's slice 0) is read from LDS before slice m's two MFMAs
    // run, so each read has a pair of MFMAs to land instead of being waited for at once; the fences keep the
    // scheduler from sinking the reads back to their uses.
    auto compute = [&](const uint16_t* S, const u32x4_t* q, const uint32_t* z) {
      const float s0 = bf_lo(z[0]), z0v = bf_hi(z[0]), s1 = bf_lo(z[1]), z1v = bf_hi(z[1]);
      const FastSZ f0 = fast_sz(s0, z0v), f1 = fast_sz(s1, z1v);
      u32x4_t a_cur = rd(S, 0, 0);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        uint32_t o0[4], o1[4];
        if constexpr (FAST) {
          dq8f(q[0][s], f0, magic, o0);
          dq8f(q[1][s], f1, magic, o1);
        } else {
          dq8(q[0][s], s0, z0v, o0);
          dq8(q[1][s], s1, z1v, o1);
        }
        const u32x4_t b0 = u32x4_t{o0[0], o0[1], o0[2], o0[3]}, b1 = u32x4_t{o1[0], o1[1], o1[2], o1[3]};
#pragma unroll
        for (int m = 0; m < NS; ++m) {
          u32x4_t a_nxt = a_cur;
          if (m + 1 < NS) a_nxt = rd(S, s, m + 1);
          else if (s + 1 < 4) a_nxt = rd(S, s + 1, 0);
          __builtin_amdgcn_sched_barrier(0);
          acc[m][0] = mfma32(a_cur, b0, acc[m][0]);
          acc[m][1] = mfma32(a_cur, b1, acc[m][1]);
          __builtin_amdgcn_sched_barrier(0);
          a_cur = a_nxt;
        }
      }
    };
    issue_a(0, S0);
    issue_w(0, q0, z0);
    issue_a(1, S1);
    issue_w(1, q1, z1);
    issue_a(2, S2);
    for (int i = 0; i < nk; i += 4) {
      wait_vm_lds<q4_wait_w2(VMA)>();
      __builtin_amdgcn_s_barrier();
      issue_w(i + 2, q2, z2);
      issue_a(i + 3, S3);
      compute(S0, q0, z0);
      wait_vm_lds<q4_wait_w2(VMA)>();
      __builtin_amdgcn_s_barrier();
      issue_w(i + 3, q3, z3);
      issue_a(i + 4, S0);
      if (i + 1 < nk) compute(S1, q1, z1);
      wait_vm_lds<q4_wait_w2(VMA)>();
      __builtin_amdgcn_s_barrier();
      issue_w(i + 4, q0, z0);
      issue_a(i + 5, S1);
      if (i + 2 < nk) compute(S2, q2, z2);
      wait_vm_lds<q4_wait_w2(VMA)>();
      __builtin_amdgcn_s_barrier();
      issue_w(i + 5, q1, z1);
      issue_a(i + 6, S2);
      if (i + 3 < nk) compute(S3, q3, z3);
    }
  } else {
    // bf16 weights: 8 loads per fragment pair and step, one step ahead in two alternating register sets; A three
    // steps ahead. Issue order B(j+1), A(j+3): before step j only A(j+2) may still be in flight.
    static_assert(VM_B == 2 * 4, "2 fragments x 4 substep chunks");
    u32x4_t bA[2][4], bB[2][4];
    auto issue_b = [&](int j, u32x4_t (*b)[4]) {
      const bool in = j < nk;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        b[0][s] = ld16(rw, in ? wo0 + j * 4096 + s * 1024 : OOB);
        b[1][s] = ld16(rw, in ? wo1 + j * 4096 + s * 1024 : OOB);
      }
    };
    // The step's 4 NS A-fragment reads in (substep, slice) order through a ring of three registers, two reads ahead of
    // the MFMA pair that uses them (the weights sit in registers already, so nothing else delays the MFMAs); the
    // fences keep the scheduler from sinking the reads back to their uses.
    auto compute = [&](const uint16_t* S, u32x4_t (*b)[4]) {
      constexpr int NR = 4 * NS;
      u32x4_t ar[3];
      ar[0] = rd(S, 0, 0);
      if (NR > 1) ar[1] = rd(S, 1 / NS, 1 % NS);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int s = r / NS, m = r % NS;
        if (r + 2 < NR) ar[(r + 2) % 3] = rd(S, (r + 2) / NS, (r + 2) % NS);
        __builtin_amdgcn_sched_barrier(0);
        acc[m][0] = mfma32(ar[r % 3], b[0][s], acc[m][0]);
        acc[m][1] = mfma32(ar[r % 3], b[1][s], acc[m][1]);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    issue_a(0, S0);
    issue_a(1, S1);
    issue_b(0, bA);
    issue_a(2, S2);
    for (int i = 0; i < nk; i += 4) {
      wait_vm_lds<BF_WAIT>();
      __builtin_amdgcn_s_barrier();
      issue_b(i + 1, bB);
      issue_a(i + 3, S3);
      compute(S0, bA);
      wait_vm_lds<BF_WAIT>();
      __builtin_amdgcn_s_barrier();
      issue_b(i + 2, bA);
      issue_a(i + 4, S0);
      if (i + 1 < nk) compute(S1, bB);   // steps past K: loads of zeros, no compute
      wait_vm_lds<BF_WAIT>();
      __builtin_amdgcn_s_barrier();
      issue_b(i + 3, bB);
      issue_a(i + 5, S1);
      if (i + 2 < nk) compute(S2, bA);
      wait_vm_lds<BF_WAIT>();
      __builtin_amdgcn_s_barrier();
      issue_b(i + 4, bA);
      issue_a(i + 6, S2);
      if (i + 3 < nk) compute(S3, bB);
    }
  }
  wait_vm<0>();   // the ring's trailing (out-of-range) loads
  // ---- LoRA K-extension: ext[row][0:32] . Bext[n][0:32]. Two planes (gate_up LoRA of rank 17..32): ext rows are
  // 64 wide, the gate fragment (0) takes plane 0 and the up fragment (1) plane 1.
  const uint16_t* eb = kind == SMEL_KIND_SEL ? (ws.ext_sel ? ws.ext_sel + (int64_t)idx * a.N * 32 : nullptr)
                                             : (kind == SMEL_KIND_SHARED ? ws.ext_sh : nullptr);
  const bool xrows = EPI == 0 && a.lr_on && a.lr.part;   // K-extension rows in X (filled at the tile's start)
  if ((a.ext || xrows) && eb) {
    const bool two = (ws.flags & SMEL_WSET_EXT2) != 0;   // uniform
    const uint32_t xb = two ? 128u : 64u;                 // ext row bytes
    const rsrc_t re = make_rsrc(eb, (uint64_t)a.N * 64);
    const rsrc_t rx = make_rsrc(a.ext + (int64_t)row0 * (xb / 2), (uint64_t)nrows * xb);
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
        const uint32_t o = row < nrows ? (uint32_t)row * xb + 32 * hi + 16 * s : OOB;
        const u32x4_t af =
            xrows ? *reinterpret_cast<const u32x4_t*>(X + (m >> 1) * STAGE + (row & 63) * 32 + 16 * hi + 8 * s)
                  : ld16(rx, o);
        const u32x4_t af1 = two ? ld16(rx, o == OOB ? OOB : o + 64) : af;
        acc[m][0] = mfma32(af, b0[s], acc[m][0]);
        acc[m][1] = mfma32(af1, b1[s], acc[m][1]);
      }
    }
  }
  // ---- epilogue through LDS (the ring is free after the loop): every lane writes its bf16 results into a row-major
  // tile, then each thread stores 16-B chunks of whole rows, i.e. one address per 8 outputs instead of one per
  // output. Tile rows are 128 B-chunked and XOR-swizzled like the A stages (phys chunk = c ^ (row & 7)).
  __syncthreads();   // every wave is done with the ring (its loads landed, its reads returned)
  if constexpr (EPI == 1) {
    // the down LoRA's A factor of this tile's group (SEL / SHARED with a LoRA), if the partials are wanted
    const uint16_t* xa = nullptr;
    float xscale = 0.f;
    if (a.lr_on && a.lr.part) {
      if (kind == SMEL_KIND_SEL && a.lr.a_sel) {
        xa = a.lr.a_sel + (int64_t)idx * 32 * (a.N / 2);
        xscale = a.lr.scale_sel;
      } else if (kind == SMEL_KIND_SHARED && a.lr.a_sh) {
        xa = a.lr.a_sh;
        xscale = a.lr.scale_sh;
      }
    }
    // g tile [160][128] in S0 (rows 0..HALF-1) / S1 (rows HALF..), u tile in S2 / S3 (a stage holds HALF rows of 128
    // columns); column = 32 w + r32 inside the block's 128. Which stage a row goes to is known at compile time: HALF is
    // a multiple of 8 and a lane's part of acc_row is below 8.
    constexpr int HALF = MT_MERGED / 2;
    const int col = 32 * w + r32;
#pragma unroll
    for (int m = 0; m < NS; ++m) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool lo = m * 32 + 8 * (r >> 2) < HALF;
        uint16_t* G = lo ? S0 : S1;
        uint16_t* U = lo ? S2 : S3;
        const int row = m * 32 + acc_row(r, l), lr = lo ? row : row - HALF;
        const int e = lr * 128 + 8 * ((col >> 3) ^ (row & 7)) + (col & 7);
        G[e] = f2bf(acc[m][0][r]);
        U[e] = f2bf(acc[m][1][r]);
      }
    }
    __syncthreads();
    // thread -> (row, 8-column chunk): 16 threads per row, 16 rows per pass
    const int I = a.N / 2;
    const int ch = tid & 15;
    const int col0 = nb * 128 + 8 * ch;
    if (col0 < I) {
      for (int row = tid >> 4; row < nrows; row += 16) {
        const bool lo = row < HALF;
        const int lr = lo ? row : row - HALF;
        const int e = lr * 128 + 8 * (ch ^ (row & 7));
        const u32x4_t g = *reinterpret_cast<const u32x4_t*>((lo ? S0 : S1) + e);
        const u32x4_t u = *reinterpret_cast<const u32x4_t*>((lo ? S2 : S3) + e);
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = pack2bf(act_f(bf_lo(g[j]), a.act) * bf_lo(u[j]), act_f(bf_hi(g[j]), a.act) * bf_hi(u[j]));
        const int64_t grow = row0 + row;
        *reinterpret_cast<u32x4_t*>(a.out + grow * a.ldo + col0) = u32x4_t{o[0], o[1], o[2], o[3]};
        if (a.hsave) {
          *reinterpret_cast<u32x4_t*>(a.hsave + grow * a.N + col0) = g;
          *reinterpret_cast<u32x4_t*>(a.hsave + grow * a.N + I + col0) = u;
        }
        if (xa)   // h replaces g in the tile (each chunk is read and written by this thread only)
          *reinterpret_cast<u32x4_t*>((lo ? S0 : S1) + e) = u32x4_t{o[0], o[1], o[2], o[3]};
      }
    }
    if (xa) {
      // partial down-LoRA projection of the tile's rows over this block's 128 columns of h:
      // part[row][nb][j] = scale * sum_c h[row][c] a[j][c]; wave w takes rows 32 w .. 32 w + 31
      __syncthreads();
      if (w < NS) {
        const rsrc_t rb = make_rsrc(xa, (uint64_t)32 * I * 2);
        f32x16_t px = f32x16_t{};
        const int row = 32 * w + r32;
        const uint16_t* Hh = row < HALF ? S0 : S1;
        const int lr_ = row < HALF ? row : row - HALF;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int c = 64 * kk + 32 * hi + 8 * s;   // column inside the block's 128
            const u32x4_t af = *reinterpret_cast<const u32x4_t*>(Hh + lr_ * 128 + 8 * ((c >> 3) ^ (row & 7)));
            const int gc = nb * 128 + c;
            const u32x4_t bf = ld16(rb, gc < I ? (uint32_t)(r32 * I + gc) * 2 : OOB);
            px = mfma32(af, bf, px);
          }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int orow = 32 * w + acc_row(r, l);
          if (orow < nrows)
            a.lr.part[((int64_t)(row0 + orow) * a.lr.parts + nb) * 32 + r32] = xscale * px[r];
        }
      }
    }
  } else if constexpr (NS == 5) {
    // merged tile: out tile [160][256] over the four contiguous stages, row r at S0 + 256 r; column = 64 w + 32 f +
    // r32 inside the block's 256. Thread -> (row, two 8-column chunks): 16 threads per row, 16 rows per pass; the
    // output slots of a thread's 10 rows are loaded before the tile goes to LDS (no row table: the tile fills the LDS)
    const int ch = tid & 15;
    int slot[MT_MERGED / 16];
#pragma unroll
    for (int p = 0; p < MT_MERGED / 16; ++p) {
      const int row = (tid >> 4) + 16 * p;
      slot[p] = row < nrows ? row_slot(row0 + row, a.order, a.TK) : 0;
    }
#pragma unroll
    for (int m = 0; m < NS; ++m) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m * 32 + acc_row(r, l);
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          const int col = 64 * w + 32 * f + r32;
          S0[row * 256 + 8 * ((col >> 3) ^ (row & 7)) + (col & 7)] = f2bf(acc[m][f][r]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < MT_MERGED / 16; ++p) {
      const int row = (tid >> 4) + 16 * p;
      if (row < nrows) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int c = ch + 16 * h, col0 = nb * 256 + 8 * c;
          if (col0 < a.N) {
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(S0 + row * 256 + 8 * (c ^ (row & 7)));
            *reinterpret_cast<u32x4_t*>(a.out + (int64_t)slot[p] * a.ldo + col0) = v;
          }
        }
      }
    }
  } else {
    // out tile [128][256]: rows 32 m .. 32 m + 31 in stage m; column = 64 w + 32 f + r32 inside the block's 256
    uint16_t* const St[4] = {S0, S1, S2, S3};
    if (tid < MT) rowmap[tid] = ep_slot;
#pragma unroll
    for (int m = 0; m < NS; ++m) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lr = acc_row(r, l);   // row inside the stage (= row & 31)
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          const int col = 64 * w + 32 * f + r32;
          St[m][lr * 256 + 8 * ((col >> 3) ^ (lr & 7)) + (col & 7)] = f2bf(acc[m][f][r]);
        }
      }
    }
    __syncthreads();
    // thread -> (row, 8-column chunk): 32 threads per row, 8 rows per pass; rows go to their slot's output row
    const int ch = tid & 31;
    const int col0 = nb * 256 + 8 * ch;
    if (col0 < a.N) {
      for (int row = tid >> 5; row < nrows; row += 8) {
        const int lr = row & 31;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(St[row >> 5] + lr * 256 + 8 * (ch ^ (lr & 7)));
        const int64_t orow = rowmap[row];
        *reinterpret_cast<u32x4_t*>(a.out + orow * a.ldo + col0) = v;
      }
    }
  }
}

template <int EPI, bool Q4, bool FAST>
SMEL_DEV void run_tile_ns(const FwdArgs& a, int kind, int idx, int row0, int nrows, int nb, uint16_t* S0,
                          uint16_t* S1, uint16_t* S2, uint16_t* S3, int* rowmap, uint16_t* X) {
  switch ((nrows + 31) >> 5) {
    case 1: run_tile<EPI, Q4, 1, FAST>(a, kind, idx, row0, nrows, nb, S0, S1, S2, S3, rowmap, X); break;
    case 2: run_tile<EPI, Q4, 2, FAST>(a, kind, idx, row0, nrows, nb, S0, S1, S2, S3, rowmap, X); break;
    case 3: run_tile<EPI, Q4, 3, FAST>(a, kind, idx, row0, nrows, nb, S0, S1, S2, S3, rowmap, X); break;
    case 4: run_tile<EPI, Q4, 4, FAST>(a, kind, idx, row0, nrows, nb, S0, S1, S2, S3, rowmap, X); break;
    default:   // 5 slices: only a merged int4 tile (fast dequant form) has more rows
      if constexpr (Q4 && FAST)
        run_tile<EPI, Q4, 5, FAST>(a, kind, idx, row0, nrows, nb, S0, S1, S2, S3, rowmap, X);
      break;
  }
}

template <int EPI>
SMEL_DEV void gmm_fwd_body(const FwdArgs& a, uint16_t* S0, uint16_t* S1, uint16_t* S2, uint16_t* S3, int* rowmap,
                           uint16_t* X) {
  int tile, nb;
  const int n_t = a.n_tiles[0];
  if (!((a.w.flags & SMEL_WSET_XCD_CHUNK) ? xcd_tile_chunk(n_t, a.nblk, tile, nb) : xcd_tile(n_t, a.nblk, tile, nb)))
    return;
  const int4 t = a.tiles[tile];
  const int gk = a.gkind ? a.gkind[t.x] : t.w;   // the tile list may carry the group kind itself
  const int kind = gk >> 16, idx = gk & 0xffff;
  int row1 = t.z;
  // a tile of up to 160 rows: a merged list's int4 tile (its rows beyond 128 are the group's short last tile), or a
  // gate_up tile that takes the next one below (group-ordered list, SMEL_WSET_MERGE_SHORT). Both need the fast
  // dequant form and K a multiple of 64 (the 5-slice tile has no registers for the other form or for a K tail).
  const bool five = kind == SMEL_KIND_INT4 && (a.w.flags & SMEL_WSET_FAST_DQ) && (a.K & (KT - 1)) == 0;
  if (EPI == 1 && five && (a.w.flags & SMEL_WSET_MERGE_SHORT)) {
    // In a group-ordered list, a group's last tile of at most MT_MERGED - MT rows right after a full tile of the same
    // group is taken by the full tile's blocks (one weight stream and dequant for both); its own blocks exit.
    if (t.z - t.y <= MT_MERGED - MT && tile > 0) {
      const int4 p = a.tiles[tile - 1];
      if (p.x == t.x && p.z == t.y && p.z - p.y == MT) return;
    }
    if (t.z - t.y == MT && tile + 1 < n_t) {
      const int4 q = a.tiles[tile + 1];
      if (q.x == t.x && q.y == t.z && q.z - q.y <= MT_MERGED - MT) row1 = q.z;
    }
  }
  const bool merged = five && (a.w.flags & (EPI == 1 ? SMEL_WSET_MERGE_SHORT | SMEL_WSET_MERGED_LIST
                                                      : SMEL_WSET_MERGED_LIST));
  const int nrows = min(row1 - t.y, merged ? MT_MERGED : MT);
  if (nrows <= 0) return;
  if (kind == SMEL_KIND_INT4) {
    if (a.w.flags & SMEL_WSET_FAST_DQ)
      run_tile_ns<EPI, true, true>(a, kind, idx, t.y, nrows, nb, S0, S1, S2, S3, rowmap, X);
    else
      run_tile_ns<EPI, true, false>(a, kind, idx, t.y, nrows, nb, S0, S1, S2, S3, rowmap, X);
  } else {
    run_tile_ns<EPI, false, false>(a, kind, idx, t.y, min(nrows, MT), nb, S0, S1, S2, S3, rowmap, X);
  }
}

// Four contiguous A stages of 160 rows (80 KiB, two blocks per CU), nothing else in LDS. The down projection
// (epilogue 0) keeps a tile's LoRA rows and its rows' output slots in the stages' spare rows (a tile of at most 128
// rows; a merged tile of more is an int4 tile, without either).
template <int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gmm_fwd_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(1024))) uint16_t ring[4 * STAGE];
  uint16_t* const S0 = ring;
  if constexpr (EPI == 0)
    gmm_fwd_body<EPI>(a, S0, S0 + STAGE, S0 + 2 * STAGE, S0 + 3 * STAGE,
                      reinterpret_cast<int*>(S0 + 2 * STAGE + SPARE), S0 + SPARE);
  else
    gmm_fwd_body<EPI>(a, S0, S0 + STAGE, S0 + 2 * STAGE, S0 + 3 * STAGE, nullptr, nullptr);
}

}  // namespace

extern "C" int64_t smel_gmm_fwd_nblocks(int64_t R, int32_t epilogue) {
  if (R <= 0) return -1;
  return epilogue == 1 ? (R / 2 + 127) / 128 : (R + 255) / 256;
}

extern "C" int smel_gmm_fwd_lr(const smel_wset* w, const int32_t* gkind, const int32_t* tiles,
                               const int32_t* n_tiles, int64_t max_tiles, const uint16_t* A, int64_t lda,
                               int64_t a_rows, int32_t a_gather, const int32_t* order, int64_t TK, int64_t topk,
                               const uint16_t* ext, int32_t epilogue, int32_t act, uint16_t* out, int64_t ldo,
                               uint16_t* hsave, const smel_fwd_lora_rows* lr, hipStream_t stream) {
  SMEL_REQUIRE(w && tiles && n_tiles && A && out, SMEL_EINVAL, "gmm_fwd: null pointer");
  SMEL_REQUIRE(w->R > 0 && w->C > 0 && max_tiles >= 0 && lda >= w->C && topk > 0, SMEL_EINVAL,
               "gmm_fwd: bad sizes");
  SMEL_REQUIRE(w->C % 32 == 0, SMEL_EUNSUPPORTED, "gmm_fwd: K=%lld must be a multiple of 32", (long long)w->C);
  SMEL_REQUIRE(w->R % 32 == 0 && (epilogue == 0 || (w->R / 2) % 32 == 0), SMEL_EUNSUPPORTED,
               "gmm_fwd: N=%lld must be a multiple of 32 (64 for gate_up)", (long long)w->R);
  SMEL_REQUIRE(!w->q4 || (w->group % 32 == 0 && w->C % w->group == 0), SMEL_EUNSUPPORTED,
               "gmm_fwd: int4 group %d must be a multiple of 32 dividing K", w->group);
  SMEL_REQUIRE(!w->q4 || w->sz4, SMEL_EINVAL, "gmm_fwd: an int4 bank needs its packed scale/zero (smel_pack_int4)");
  SMEL_REQUIRE(lda % 8 == 0 && ((uintptr_t)A % 16) == 0, SMEL_EUNSUPPORTED, "gmm_fwd: A rows must be 16-B aligned");
  SMEL_REQUIRE(ldo % 8 == 0 && ((uintptr_t)out % 16) == 0 && ((uintptr_t)hsave % 16) == 0, SMEL_EUNSUPPORTED,
               "gmm_fwd: out / hsave rows must be 16-B aligned");
  SMEL_REQUIRE(epilogue == 0 || epilogue == 1, SMEL_EINVAL, "gmm_fwd: epilogue %d", epilogue);
  SMEL_REQUIRE(!(w->flags & SMEL_WSET_EXT2) || epilogue == 1, SMEL_EINVAL,
               "gmm_fwd: a two-plane LoRA extension belongs to the gate_up projection (epilogue 1)");
  SMEL_REQUIRE(!(w->flags & SMEL_WSET_MERGED_LIST) || !w->q4 || ((w->flags & SMEL_WSET_FAST_DQ) && w->C % 64 == 0),
               SMEL_EINVAL,
               "gmm_fwd: a merged tile list (SMEL_WSET_MERGED_LIST) on an int4 bank needs its fast dequant form and K "
               "a multiple of 64");
  SMEL_REQUIRE(!a_gather || order || TK == 0, SMEL_EINVAL, "gmm_fwd: gather needs order");
  SMEL_REQUIRE(act == 0 || act == 1, SMEL_EINVAL, "gmm_fwd: act %d", act);
  SMEL_REQUIRE(a_rows >= 0 && a_rows * lda * 2 < (1ll << 31), SMEL_EUNSUPPORTED, "gmm_fwd: A larger than 2 GiB");
  if (lr && lr->part) {
    SMEL_REQUIRE(epilogue == 1 ? lr->parts == smel_gmm_fwd_nblocks(w->R, 1) : lr->parts >= 1, SMEL_EINVAL,
                 "gmm_fwd: %d LoRA-row partials per row (the gate_up GEMM's column blocks)", lr->parts);
    SMEL_REQUIRE(((uintptr_t)lr->part % 16) == 0 && ((uintptr_t)lr->ext_out % 16) == 0, SMEL_EUNSUPPORTED,
                 "gmm_fwd: LoRA-row partials and rows must be 16-B aligned");
    SMEL_REQUIRE(epilogue == 1 || !(w->flags & SMEL_WSET_EXT2), SMEL_EINVAL,
                 "gmm_fwd: the down projection's LoRA has one plane");
  }
  if (max_tiles == 0) return 0;
  FwdArgs a;
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

extern "C" int smel_gmm_fwd(const smel_wset* w, const int32_t* gkind, const int32_t* tiles, const int32_t* n_tiles,
                            int64_t max_tiles, const uint16_t* A, int64_t lda, int64_t a_rows, int32_t a_gather,
                            const int32_t* order, int64_t TK, int64_t topk, const uint16_t* ext, int32_t epilogue,
                            int32_t act, uint16_t* out, int64_t ldo, uint16_t* hsave, hipStream_t stream) {
  return smel_gmm_fwd_lr(w, gkind, tiles, n_tiles, max_tiles, A, lda, a_rows, a_gather, order, TK, topk, ext,
                         epilogue, act, out, ldo, hsave, nullptr, stream);
}
