// Single-pass chunked cross-entropy over a frozen lm_head (smel/loss.py:50-156), both GEMMs on MFMA.
//
// Per vocabulary chunk [v0, v0 + vc) and pass of n token rows:
//   ce_logits  (MFMA, 256 vocabulary x 256 token tile, 8 waves): z = h W_c^T rounded to the rows' dtype (the
//              reference's `(h @ W.t())`), capped (z -> c tanh(z / c)), and per window of 128 columns and token row
//              the window's maximum rounded up to a whole power of two, e = ceil(max z * log2 e), the sum of
//              exp(z - e ln 2) and the softmax terms p = exp(z - e ln 2) (times the cap derivative 1 - (z / c)^2) in
//              the rows' dtype, [n][vc] row-major; the target's capped logit and cap derivative where the target
//              lies in the tile. The logits never reach memory.
//   ce_stats   per row: chunk maximum E = max e, chunk sum, the running maximum nE = max(m, E) and sum
//              s = s 2^(m - nE) + sum_w s_w 2^(e_w - nE), the accumulator's rescale r = 2^(m - nE), and per window
//              the shift nE - e_w of its softmax terms. Every rescale is an exact power of two.
//   ce_grad    (MFMA, 256 hidden x 256 token tile, 8 waves, the chunk's columns in two K halves):
//              acc = r (acc + part_prev) + sum_v p'_v W_v over the first half, part = the second half's sum, with
//              p' = p 2^-(shift): each 16-byte fragment of p is shifted in registers as it leaves LDS (bf16: one
//              saturating 16-bit subtract of the exponent per value pair; fp16 / fp32: ldexp), so the products are
//              the reference's `p.to(h.dtype) @ W` terms at the running maximum (smel/loss.py:85).
//   ce_finish  per row: loss = nE ln 2 + log s - z_target, gradient row = (acc + part) / s - d_target W[target]
//              (smel/loss.py:87-92), scaled and stored in the requested dtype; ce_loss_sum adds the rows' losses
//              in fixed order.
// The head operand of ce_grad is the head transposed ([H][V], one copy per frozen head, made by ce_transpose), so
// both GEMMs read K-contiguous rows. No atomics: every output element has one writer and fixed-order sums.
// Both GEMMs are bound by the rate at which a CU brings operands in from L2 (about 14 B per clock here), so their
// tiles are the largest the registers hold (256 x 256, 131 FLOP per loaded byte in bf16).
#include <algorithm>
#include <type_traits>

#include "../../include/smel_loss.h"
#include "abi_util.h"
#include "common.h"

namespace {

constexpr int WIN = 128;    // vocabulary columns of one statistics window
// build-time tuning of the two GEMMs: k-step bytes, ring stages (a stage holds 256 + 256 rows) and waves per block;
// deeper rings and 64-byte k-steps measured no faster
#ifndef SMEL_CE_LG_KB
#define SMEL_CE_LG_KB 128
#define SMEL_CE_LG_NST 2
#define SMEL_CE_GR_KB 128
#define SMEL_CE_GR_NST 2
#endif
#ifndef SMEL_CE_LG_NW
#define SMEL_CE_LG_NW 8
#endif
#ifndef SMEL_CE_GR_NW
#define SMEL_CE_GR_NW 8
#endif

constexpr int VT = 256;     // vocabulary columns of a logits tile (two windows)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr int SHIFT_ZERO = 255;   // a shift that turns every softmax term of the window into zero

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

template <int DT>
constexpr int ebytes() {
  return DT == 1 ? 4 : 2;
}

// One 16-byte chunk per lane of A and B into a 32x32 fp32 accumulator: 16-bit types in one 32x32x16 MFMA; fp32 in
// four 32x32x2 MFMAs, the j-th value of both chunks in the j-th (the k order inside a chunk is the same for A and B).
template <int DT>
SMEL_DEV void mma(f32x16_t& c, const u32x4_t& a, const u32x4_t& b) {
  if constexpr (DT == 0) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                0, 0, 0);
  } else if constexpr (DT == 2) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                               0, 0);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[j]), __uint_as_float(b[j]), c, 0, 0, 0);
  }
}

// fp32 value rounded to the rows' dtype and back (the reference's 16-bit GEMM output)
template <int DT>
SMEL_DEV float round_t(float v) {
  if constexpr (DT == 0) return bf2f(f2bf(v));
  else if constexpr (DT == 2) return (float)(_Float16)v;
  else return v;
}
// two values in the rows' dtype, packed (16-bit) — fp32 keeps them apart
SMEL_DEV uint32_t pack2h(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}

// 16-byte chunk of softmax terms times 2^-sh (sh >= 0). bf16 (all terms are >= 0 and at most ~1): subtracting
// sh << 7 from the bit pattern moves the exponent, exactly for every result in the normal range; the saturating
// subtract turns a result below it into zero or a value under 2^-126. fp16 / fp32: ldexp, exact.
// The results go to a separate vector: hipcc of ROCm 7.2 miscompiles an in-place update v[i] = f(bit_cast(v[i])) of
// an ext-vector element in an unrolled loop (every later element got the first element's result).
template <int DT>
SMEL_DEV u32x4_t shift_chunk(const u32x4_t v, uint32_t sh) {
  u32x4_t o;
  if constexpr (DT == 0) {
    const unsigned short d = (unsigned short)(sh << 7);
    const u16x2_t dd = {d, d};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t x = v[i];
      o[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2_t, x), dd));
    }
  } else if constexpr (DT == 2) {
    const int e = -(int)sh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t x = v[i];
      o[i] = pack2h(ldexpf(h_lo(x), e), ldexpf(h_hi(x), e));
    }
  } else {
    const int e = -(int)sh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t x = v[i];
      o[i] = __float_as_uint(ldexpf(__uint_as_float(x), e));
    }
  }
  return o;
}

// ------------------------------------------------------------------------------------------------ GEMM main loop
// C[i][j] += sum_k A[i][k] B[j][k] over one tile: A 256 rows, B 64 NB rows, both K-contiguous (row pitch in bytes
// given by the caller's offsets). 4 waves: wave w computes A rows 128 (w & 1) + [0, 128) x B rows 32 NB (w >> 1) +
// [0, 32 NB) as 4 x NB MFMA tiles of 32 x 32. Per k-step (KB bytes of every row: 128 or 64) the operands go
// global -> LDS directly (16-byte LDS-DMA loads, 1 KB per wave-load), into a ring of NST stages loaded NST - 1 steps
// ahead. The 16-byte chunks of each LDS row are XOR-swizzled (logical chunk c of row r at phys(c, r)) so that the
// fragment reads of 8 or 16 consecutive rows at one logical chunk hit distinct banks (32 or 64 four-byte banks).
// Lane half h carries chunk NSUB h + s in substep s, for A and B alike.
template <int KB_, int NB, int NST, int NW = 4>
struct Ring {
  static constexpr int KB = KB_;            // bytes of one k-step of a row
  static constexpr int NSTAGE = NST;
  static constexpr int NWAVES = NW;         // 2 x NW / 2 waves: A halves x B parts
  static constexpr int RPW = 1024 / KB;     // rows of one 1-KB wave-load
  static constexpr int CPR = KB / 16;       // 16-byte chunks per row
  static constexpr int NSUB = CPR / 2;      // MFMA substeps per k-step
  static constexpr int B_ROWS = 32 * NB * (NW / 2);
  static constexpr int A_BYTES = 256 * KB, B_BYTES = B_ROWS * KB, STAGE = A_BYTES + B_BYTES, BYTES = NST * STAGE;
  static constexpr int VM_A = 256 / RPW / NW, VM_B = B_ROWS / RPW / NW;   // wave-loads per wave and stage
  static_assert(VM_A % 2 == 0 && VM_B % 2 == 0, "even wave-load counts (the 128-byte swizzle parity)");
  static constexpr int VM_STEP = VM_A + VM_B;
  static_assert(KB == 128 || KB == 64, "k-steps of 128 or 64 bytes");
  // the row swizzle: 128-byte rows (8 chunks) c ^ (r % 8) ^ (r / 8 % 2); 64-byte rows (4 chunks)
  // c ^ ((r / 2 ^ r / 4) % 4); both depend on r % 16 only
  static SMEL_DEV int phys(int c, int r) {
    if constexpr (KB == 128) return c ^ (r & 7) ^ ((r >> 3) & 1);
    else return c ^ (((r >> 1) ^ (r >> 2)) & 3);
  }
  // wave-load ii of wave w (rows RPW g .. RPW g + RPW - 1, g = VM w + ii): this lane's row in the operand tile and
  // the byte offset of the logical chunk it loads (physical chunk lane % CPR of that row)
  static SMEL_DEV int ld_row(int vm, int w, int ii, int lane) { return RPW * (vm * w + ii) + lane / CPR; }
  static SMEL_DEV uint32_t ld_chunk(int vm, int w, int ii, int lane) {
    return 16u * (uint32_t)phys(lane % CPR, ld_row(vm, w, ii, lane));
  }
};

// Row offsets (bytes from the operand base) of this lane's wave-loads, OOB for rows at or past `valid`.
template <class R, int VM>
SMEL_DEV void row_offsets(uint32_t (&off)[VM], int w, int lane, int valid, uint32_t pitch_bytes) {
#pragma unroll
  for (int ii = 0; ii < VM; ++ii) {
    const int row = R::ld_row(VM, w, ii, lane);
    off[ii] = row < valid ? (uint32_t)row * pitch_bytes : OOB;
  }
}

// The main loop over kbytes (a multiple of 16) of every row, in the k-step order rot, rot + 1, ..., nk - 1, 0, ...,
// rot - 1: a tile's sum over k is then taken in an order fixed by `rot`, and tiles running side by side with different
// rotations read different 128-byte columns of their rows at any moment (with row pitches that are multiples of
// 2 KB, the rows of one column all fall on one L2 channel). `pre(kk, first)` runs before the operand loads of the
// step after the current one are issued (kk = that step's k-step index; first: before the loop, for the first
// step) and may issue its own loads: they retire before the next step's wait. `fix(n, kk, v)` transforms a B fragment
// of tile column n in k-step kk as it leaves LDS.
template <int DT, class R, int NB, class Pre, class Fix>
SMEL_DEV void nt_loop(f32x16_t (&acc)[4][NB], uint8_t* smem, rsrc_t ra, const uint32_t (&aoff)[R::VM_A], rsrc_t rb,
                      const uint32_t (&boff)[R::VM_B], int kbytes, int rot, Pre&& pre, Fix&& fix) {
  constexpr int KB = R::KB, NST = R::NSTAGE;
  const int lane = lane_id(), h = lane >> 5, r32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = w & 1, wn = w >> 1;
  const int nk = (kbytes + KB - 1) / KB;
  if (nk <= 0) return;   // an empty K range (a half of a one-step chunk): the tile's sum is zero
  rot = __builtin_amdgcn_readfirstlane(rot % nk);
  auto kstep = [&](int j) { return j + rot < nk ? j + rot : j + rot - nk; };
  auto issue = [&](int j) {
    uint8_t* S = smem + (j % NST) * R::STAGE;
    const uint32_t k0 = (uint32_t)kstep(j) * KB;
    const bool tail = (int)k0 + KB > kbytes;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ii = 0; ii < R::VM_A; ++ii) {
      const uint32_t cb = R::ld_chunk(R::VM_A, w, ii, lane);
      const bool ok = !tail || (int)(k0 + cb) + 16 <= kbytes;
      ld16_lds(ra, S + (R::VM_A * w + ii) * 1024, ok ? aoff[ii] + k0 + cb : OOB);
    }
#pragma unroll
    for (int ii = 0; ii < R::VM_B; ++ii) {
      const uint32_t cb = R::ld_chunk(R::VM_B, w, ii, lane);
      const bool ok = !tail || (int)(k0 + cb) + 16 <= kbytes;
      ld16_lds(rb, S + R::A_BYTES + (R::VM_B * w + ii) * 1024, ok ? boff[ii] + k0 + cb : OOB);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // fragment read offsets inside a stage: substep s reads logical chunk NSUB h + s of its rows
  uint32_t pcb[R::NSUB];
#pragma unroll
  for (int s = 0; s < R::NSUB; ++s) pcb[s] = (uint32_t)r32 * KB + 16u * (uint32_t)R::phys(R::NSUB * h + s, r32);
  pre(kstep(0), true);
#pragma unroll
  for (int s = 0; s < NST - 1; ++s)
    if (s < nk) issue(s);
  for (int j = 0; j < nk; ++j) {
    // this wave's loads of step j have landed (later steps' may still be in flight: no __syncthreads, which would
    // wait for all of them) and its LDS reads of the stage the next issue overwrites have returned; then the barrier
    __builtin_amdgcn_sched_barrier(0);
    if (j + NST - 2 < nk) wait_vm_lds<(NST - 2) * R::VM_STEP>();
    else wait_vm_lds<0>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < nk) pre(kstep(j + 1), false);
    if (j + NST - 1 < nk) issue(j + NST - 1);
    const int kk = kstep(j);
    const uint8_t* A = smem + (j % NST) * R::STAGE + wm * 128 * KB;
    const uint8_t* B = smem + (j % NST) * R::STAGE + R::A_BYTES + wn * 32 * NB * KB;
    // fragments in two register sets: those of substep s + 1 are read from LDS before the MFMAs of substep s are
    // issued (the order is pinned), so their LDS latency runs under those MFMAs
    u32x4_t af[2][4], bf[2][NB];
    auto read = [&](int s, int set) {
#pragma unroll
      for (int m = 0; m < 4; ++m) af[set][m] = *reinterpret_cast<const u32x4_t*>(A + m * 32 * KB + pcb[s]);
#pragma unroll
      for (int n = 0; n < NB; ++n) bf[set][n] = *reinterpret_cast<const u32x4_t*>(B + n * 32 * KB + pcb[s]);
    };
    read(0, 0);
#pragma unroll
    for (int s = 0; s < R::NSUB; ++s) {
      const int cur = s & 1;
      if (s + 1 < R::NSUB) read(s + 1, cur ^ 1);
      __builtin_amdgcn_sched_barrier(0);
      u32x4_t bx[NB];
#pragma unroll
      for (int n = 0; n < NB; ++n) bx[n] = fix(n, kk, bf[cur][n]);
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < NB; ++n) mma<DT>(acc[m][n], af[cur][m], bx[n]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// ------------------------------------------------------------------------------------------------ ce_logits
struct LogitsArgs {
  const void* W;        // head rows of the chunk (row 0 = vocabulary id v0), pitch ldw elements
  const void* h;        // token rows, pitch ldh elements
  const int64_t* tgt;   // target id per token row
  void* P;              // softmax terms [n][ldp] in the rows' dtype, or null (statistics only)
  float *win_e, *win_s; // [nwin][ldn] window maxima (power-of-two exponents) and sums
  float *tz, *td;       // target logit and cap derivative per row (written where the target lies in the chunk)
  int64_t ldw, ldh, ldp, ldn, v0;
  int vc, n, K;         // chunk columns, token rows, hidden size
  float cap;
  int n_vt, n_tt;       // 256-column vocabulary tiles, 256-row token tiles
};

constexpr int LG_NW = SMEL_CE_LG_NW, LG_NB = 8 / (LG_NW / 2);   // waves; token slices of 32 per wave

template <int DT, bool CAP>
__global__ __launch_bounds__(64 * LG_NW) __attribute__((amdgpu_waves_per_eu(LG_NW / 4, LG_NW / 4))) void
ce_logits_kernel(LogitsArgs a) {
  using R = Ring<SMEL_CE_LG_KB, LG_NB, SMEL_CE_LG_NST, LG_NW>;
  static_assert(R::B_ROWS == 256, "256-row token tiles");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[R::BYTES];
  const int b = blockIdx.x, x = b % NXCD, jj = b / NXCD;
  // blocks b, b + 8, ... run on one XCD: it takes vocabulary tiles x, x + 8, ... with all token tiles of each in a
  // row, so one vocabulary tile's head rows are read from that XCD's L2 by all its token tiles
  const int tt = jj % a.n_tt, vt = (jj / a.n_tt) * NXCD + x;
  if (vt >= a.n_vt) return;
  constexpr int E = ebytes<DT>();
  const int lane = lane_id(), h = lane >> 5, r32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = w & 1, wn = w >> 1;
  const int a0 = vt * VT, b0 = tt * 256;
  const int kbytes = a.K * E;
  const int a_valid = min(VT, a.vc - a0), b_valid = min(256, a.n - b0);
  const rsrc_t ra = make_rsrc(static_cast<const uint8_t*>(a.W) + (int64_t)a0 * a.ldw * E,
                              (uint64_t)(a_valid - 1) * a.ldw * E + kbytes);
  const rsrc_t rb = make_rsrc(static_cast<const uint8_t*>(a.h) + (int64_t)b0 * a.ldh * E,
                              (uint64_t)(b_valid - 1) * a.ldh * E + kbytes);
  uint32_t aoff[R::VM_A], boff[R::VM_B];
  row_offsets<R>(aoff, w, lane, a_valid, (uint32_t)(a.ldw * E));
  row_offsets<R>(boff, w, lane, b_valid, (uint32_t)(a.ldh * E));
  // this lane's token rows' targets, loaded before the main loop (the epilogue would wait on them)
  int tg[LG_NB];   // target - v0 - c0 (the window's first column), -1 when outside [0, 2^31)
#pragma unroll
  for (int n = 0; n < LG_NB; ++n) {
    const int tok = b0 + 32 * LG_NB * wn + 32 * n + r32;
    const int64_t t = tok < a.n ? a.tgt[tok] - a.v0 - (a0 + 128 * wm) : -1;
    tg[n] = t >= 0 && t < INT32_MAX ? (int)t : -1;
  }
  f32x16_t acc[4][LG_NB];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int n = 0; n < LG_NB; ++n) acc[m][n] = f32x16_t{};
  nt_loop<DT, R, LG_NB>(acc, smem, ra, aoff, rb, boff, kbytes, 5 * (b / NXCD), [](int, bool) {},
                    [](int, int, const u32x4_t& v) { return v; });
  __syncthreads();   // every wave is done with the operand ring: the epilogue may use the LDS

  // ---- epilogue. acc[m][n][r] = z at vocabulary column c0 + 32 m + 8 (r / 4) + 4 h + r % 4 of token row
  // b0 + 32 NB wn + 32 n + r32: each token row's 128 columns of this wave (one window) are 64 values in this lane and
  // 64 in lane ^ 32.
  const int c0 = a0 + 128 * wm;              // first chunk column of the window
  const int win = vt * 2 + wm;
  const int ncol = a.vc - c0;                // valid columns of the window (may be <= 0 or > 128)
  const float cap = a.cap;
  const float inv_cap = cap != 0.f ? 1.f / cap : 0.f;
  auto col_of = [&](int m, int r) { return 32 * m + 8 * (r >> 2) + 4 * h + (r & 3); };
  // FULL: every column of the window lies in the chunk (all tiles but the chunk's last): no masking
  auto slice = [&](int n, auto full_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
    const int tok = b0 + 32 * LG_NB * wn + 32 * n + r32;
    const bool tok_ok = tok < a.n;
    float mx = -INFINITY;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float z = round_t<DT>(acc[m][n][r]);
        if constexpr (CAP) z = cap * tanhf(z * inv_cap);
        if constexpr (!FULL)
          if (col_of(m, r) >= ncol) z = -INFINITY;
        acc[m][n][r] = z;
        mx = fmaxf(mx, z);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float e = mx == -INFINITY ? -INFINITY : ceilf(mx * LOG2E);
    const float ne = mx == -INFINITY ? 0.f : -e;
    float sum = 0.f;
    uint8_t* prow = a.P ? static_cast<uint8_t*>(a.P) + ((int64_t)tok * a.ldp + c0) * E : nullptr;
    // 16-bit terms go through this wave's LDS region first ([32 rows][272 B]), then out as whole 256-byte row
    // segments (16 lanes per row, 16 B each); fp32 terms are stored directly
    uint8_t* stg = smem + w * 16384;
    constexpr int SP = 272;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float z = acc[m][n][4 * q + i];
          float ez;
          if constexpr (FULL) ez = __builtin_amdgcn_exp2f(fmaf(z, LOG2E, ne));
          else ez = z != -INFINITY ? __builtin_amdgcn_exp2f(fmaf(z, LOG2E, ne)) : 0.f;
          sum += ez;
          if constexpr (CAP) p[i] = (FULL || z != -INFINITY) ? ez * (1.f - (z * inv_cap) * (z * inv_cap)) : 0.f;
          else p[i] = ez;
        }
        if constexpr (DT == 1) {
          if (prow && tok_ok)
            *reinterpret_cast<f32x4_t*>(prow + (32 * m + 8 * q + 4 * h) * E) = f32x4_t{p[0], p[1], p[2], p[3]};
        } else {
          uint8_t* d = stg + r32 * SP + (32 * m + 8 * q + 4 * h) * 2;
          if constexpr (DT == 0) *reinterpret_cast<u32x2_t*>(d) = u32x2_t{pack2bf(p[0], p[1]), pack2bf(p[2], p[3])};
          else *reinterpret_cast<u32x2_t*>(d) = u32x2_t{pack2h(p[0], p[1]), pack2h(p[2], p[3])};
        }
      }
    if constexpr (DT != 1) {
      if (a.P) {   // the slice's 32 token rows x 256 B: chunk k = 64 j + lane is row k / 16, 16-byte piece k % 16
        const int tok_s = b0 + 32 * LG_NB * wn + 32 * n;
        uint8_t* pbase = static_cast<uint8_t*>(a.P) + ((int64_t)tok_s * a.ldp + c0) * E;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int k = 64 * j + lane, row = k >> 4, piece = k & 15;
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(stg + row * SP + piece * 16);
          if (tok_s + row < a.n) *reinterpret_cast<u32x4_t*>(pbase + (int64_t)row * a.ldp * E + piece * 16) = v;
        }
      }
    }
    sum += __shfl_xor(sum, 32, 64);
    if (h == 0 && tok_ok) {
      a.win_e[(int64_t)win * a.ldn + tok] = e;
      a.win_s[(int64_t)win * a.ldn + tok] = sum;
    }
    // the target: at most one window of the whole vocabulary holds it; a wave with such a row puts its capped
    // logits of this slice in LDS ([32 rows][128], free after the main loop) and the row's lane h = 0 reads its one
    const int tc64 = tok_ok ? tg[n] : -1;
    const bool here = tc64 >= 0 && tc64 < 128 && tc64 < ncol;
    if (__builtin_amdgcn_ballot_w64(here)) {
      static_assert(LG_NW * 16384 <= R::BYTES, "per-wave staging / target scratch in the operand ring");
      float* zb = reinterpret_cast<float*>(smem + w * 16384) + r32 * 128;
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) zb[col_of(m, r)] = acc[m][n][r];
      __builtin_amdgcn_wave_barrier();
      const bool mine = here && h == 0;
      const float zt = mine ? zb[(int)tc64] : 0.f;
      __builtin_amdgcn_wave_barrier();
      if (mine) {
        a.tz[tok] = zt;
        a.td[tok] = CAP ? 1.f - (zt * inv_cap) * (zt * inv_cap) : 1.f;
      }
    }
  };
  if (ncol >= 128) {
#pragma unroll
    for (int n = 0; n < LG_NB; ++n) slice(n, std::true_type{});
  } else {
#pragma unroll
    for (int n = 0; n < LG_NB; ++n) slice(n, std::false_type{});
  }
}

// ------------------------------------------------------------------------------------------------ ce_grad
// Tiles of 256 hidden x 256 token rows (the tile size sets the FLOPs per byte loaded, which bounds these GEMMs), the
// chunk's K range split in two halves so that 4092 x 2048 outputs still give 256 workgroups: the first half adds
// into the accumulator, acc = r (acc + part_prev) + sum_first_half, the second half writes its sum to a partial
// buffer part[c % 2] (c = chunk index; the next chunk's first half folds it in, the finish adds the last one).
struct GradArgs {
  const void* WT;        // transposed head [H][ldwt], column 0 = vocabulary id v0 of the chunk
  const void* P;         // softmax terms [n][ldp]
  const uint8_t* shift;  // [nwin][ldn]
  const float* r;        // accumulator rescale per row
  float* acc;            // [n][H] fp32
  float* part;           // [2][n][H] fp32 partials of the second halves
  int64_t ldwt, ldp, ldn;
  int H, n, kbytes, first, parity;
  int n_ht, n_tt;        // 256-row hidden tiles, 256-row token tiles
};

constexpr int GR_NW = SMEL_CE_GR_NW, GR_NB = 8 / (GR_NW / 2);
constexpr int GR_SP = 528;   // epilogue staging row pitch: 128 fp32 + 16 B (rows start on different banks)

template <int DT>
__global__ __launch_bounds__(64 * GR_NW) __attribute__((amdgpu_waves_per_eu(GR_NW / 4, GR_NW / 4))) void
ce_grad_kernel(GradArgs a) {
  using R = Ring<SMEL_CE_GR_KB, GR_NB, SMEL_CE_GR_NST, GR_NW>;
  static_assert(R::B_ROWS == 256, "256-row token tiles");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[R::BYTES > GR_NW * 32 * GR_SP ? R::BYTES : GR_NW * 32 * GR_SP];
  // the list (half, token tile, hidden tile), XCD x a contiguous run of it: one XCD's tiles share their token
  // tiles' softmax terms and the hidden tiles' head columns of one K half in its L2
  const int n_tiles = a.n_ht * a.n_tt;
  int item, unused;
  if (!xcd_tile_chunk(2 * n_tiles, 1, item, unused)) return;
  const int half = item / n_tiles, tile = item % n_tiles;
  const int tt = tile / a.n_ht, ht = tile % a.n_ht;
  constexpr int E = ebytes<DT>();
  const int lane = lane_id(), h = lane >> 5, r32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = w & 1, wn = w >> 1;
  const int a0 = ht * 256, b0 = tt * 256;
  const int a_valid = min(256, a.H - a0), b_valid = min(256, a.n - b0);
  // the halves: k-steps [0, nk / 2) and [nk / 2, nk) of the chunk
  const int nk = (a.kbytes + R::KB - 1) / R::KB;
  const int klo = half ? (nk / 2) * R::KB : 0;
  const int kbytes = half ? a.kbytes - klo : (nk / 2) * R::KB;
  const rsrc_t ra = make_rsrc(static_cast<const uint8_t*>(a.WT) + (int64_t)a0 * a.ldwt * E,
                              (uint64_t)(a_valid - 1) * a.ldwt * E + a.kbytes);
  const rsrc_t rb = make_rsrc(static_cast<const uint8_t*>(a.P) + (int64_t)b0 * a.ldp * E,
                              (uint64_t)(b_valid - 1) * a.ldp * E + a.kbytes);
  uint32_t aoff[R::VM_A], boff[R::VM_B];
  row_offsets<R>(aoff, w, lane, a_valid, (uint32_t)(a.ldwt * E));
  row_offsets<R>(boff, w, lane, b_valid, (uint32_t)(a.ldp * E));
#pragma unroll
  for (int ii = 0; ii < R::VM_A; ++ii) aoff[ii] += (uint32_t)klo;   // an OOB offset stays past the buffer
#pragma unroll
  for (int ii = 0; ii < R::VM_B; ++ii) boff[ii] += (uint32_t)klo;
  f32x16_t acc[4][GR_NB];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int n = 0; n < GR_NB; ++n) acc[m][n] = f32x16_t{};
  // shifts of this lane's token rows: the window of k-step kk (of the chunk) is kk * KB / (WIN * E)
  constexpr int STEPS_PER_WIN = WIN * E / R::KB;
  const int kbase = klo / R::KB;
  const int tok0 = b0 + 32 * GR_NB * wn + r32;
  uint32_t sh_cur[GR_NB], sh_next[GR_NB];
  auto load_sh = [&](int win, uint32_t (&dst)[GR_NB]) {
#pragma unroll
    for (int n = 0; n < GR_NB; ++n) {
      const int tok = tok0 + 32 * n;
      dst[n] = tok < a.n ? (uint32_t)a.shift[(int64_t)win * a.ldn + tok] : (uint32_t)SHIFT_ZERO;
    }
  };
  int cur_win = 0;
  auto pre = [&](int kk, bool first) {   // the shifts of k-step kk's window, loaded where a window starts
    const int kg = kbase + kk;
    if (first) {
      cur_win = kg / STEPS_PER_WIN;
      load_sh(cur_win, sh_cur);
    } else if (kg % STEPS_PER_WIN == 0) {
      load_sh(kg / STEPS_PER_WIN, sh_next);
    }
  };
  auto fix = [&](int n, int kk, const u32x4_t& v) {
    const int wj = (kbase + kk) / STEPS_PER_WIN;
    if (n == 0 && wj != cur_win) {
      cur_win = wj;
#pragma unroll
      for (int q = 0; q < GR_NB; ++q) sh_cur[q] = sh_next[q];
    }
    return shift_chunk<DT>(v, sh_cur[n]);
  };
  nt_loop<DT, R, GR_NB>(acc, smem, ra, aoff, rb, boff, kbytes, 5 * (int)(blockIdx.x / NXCD), pre, fix);

  // ---- epilogue: acc[m][n][r] = term of hidden column a0 + 128 wm + 32 m + 8 (r / 4) + 4 h + r % 4 and token
  // row tok0 + 32 n. Per token slice the wave stages its 32 rows x 128 columns in LDS (the ring is free) and writes
  // them out as whole 512-byte row segments (32 lanes per row, 16 B each), the accumulator update alike.
  __syncthreads();
  uint8_t* stg = smem + w * (32 * GR_SP);
  const size_t nh = (size_t)a.n * a.H;
  const float* prev = a.part + (size_t)(a.parity ^ 1) * nh;
  float* mine = a.part + (size_t)a.parity * nh;
  const int col0 = a0 + 128 * wm;
#pragma unroll
  for (int n = 0; n < GR_NB; ++n) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f32x4_t*>(stg + r32 * GR_SP + (32 * m + 8 * q + 4 * h) * 4) =
            f32x4_t{acc[m][n][4 * q], acc[m][n][4 * q + 1], acc[m][n][4 * q + 2], acc[m][n][4 * q + 3]};
    const int tok_s = b0 + 32 * GR_NB * wn + 32 * n;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const int k = 64 * jj + lane, row = k >> 5, piece = k & 31;
      const int tok = tok_s + row, col = col0 + 4 * piece;
      f32x4_t v = *reinterpret_cast<const f32x4_t*>(stg + row * GR_SP + piece * 16);
      if (tok >= a.n || col >= a.H) continue;
      const size_t at = (size_t)tok * a.H + col;
      if (half) {
        *reinterpret_cast<f32x4_t*>(mine + at) = v;
        continue;
      }
      if (!a.first) {
        const float rr = a.r[tok];
        const f32x4_t o = *reinterpret_cast<const f32x4_t*>(a.acc + at);
        const f32x4_t pp = *reinterpret_cast<const f32x4_t*>(prev + at);
        v = f32x4_t{fmaf(o[0] + pp[0], rr, v[0]), fmaf(o[1] + pp[1], rr, v[1]), fmaf(o[2] + pp[2], rr, v[2]),
                    fmaf(o[3] + pp[3], rr, v[3])};
      }
      *reinterpret_cast<f32x4_t*>(a.acc + at) = v;
    }
  }
}

// ------------------------------------------------------------------------------------------------ small kernels
__global__ __launch_bounds__(256) void ce_begin_kernel(float* m, float* s, float* tz, float* td, const float* m0,
                                                       int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  m[i] = m0 ? m0[i] : -INFINITY;
  s[i] = 0.f;
  tz[i] = 0.f;
  td[i] = 1.f;
}

SMEL_DEV float pow2i(float e) { return ldexpf(1.f, (int)e); }

// 16 rows per block, 16 threads per row (windows w = q mod 16): each thread loads its windows' maxima and sums once
// (up to ST_W of them in registers, any further ones again from memory), partial maxima and sums are combined in
// fixed order through LDS
constexpr int ST_ROWS = 16, ST_Q = 16, ST_W = 16;
__global__ __launch_bounds__(256) void ce_stats_kernel(const float* __restrict__ win_e, const float* __restrict__ win_s,
                                                       int nwin, int64_t ldn, int64_t n, float* m, float* s,
                                                       uint8_t* shift, float* r_out) {
  __shared__ float red[ST_Q][ST_ROWS];
  const int q = threadIdx.x / ST_ROWS, t = threadIdx.x % ST_ROWS;
  const int64_t row = (int64_t)blockIdx.x * ST_ROWS + t;
  const bool ok = row < n;
  float ev[ST_W], sv[ST_W];
  float E = -INFINITY;
#pragma unroll
  for (int i = 0; i < ST_W; ++i) {
    const int w = q + ST_Q * i;
    const bool in = ok && w < nwin;
    ev[i] = in ? win_e[(int64_t)w * ldn + row] : -INFINITY;
    sv[i] = in ? win_s[(int64_t)w * ldn + row] : 0.f;
    E = fmaxf(E, ev[i]);
  }
  if (ok)
    for (int w = q + ST_Q * ST_W; w < nwin; w += ST_Q) E = fmaxf(E, win_e[(int64_t)w * ldn + row]);
  red[q][t] = E;
  lds_barrier();
#pragma unroll
  for (int k = 0; k < ST_Q; ++k) E = fmaxf(E, red[k][t]);
  lds_barrier();
  const float mo = ok ? m[row] : -INFINITY;
  const float nE = fmaxf(mo, E);   // finite: every chunk has a valid column
  float S = 0.f;
  auto fold = [&](int w, float e, float sw) {
    int sh = SHIFT_ZERO;
    if (e != -INFINITY) {
      const float d = nE - e;
      sh = d < (float)SHIFT_ZERO ? (int)d : SHIFT_ZERO;
      S += ldexpf(sw, -(int)fminf(d, 300.f));
    }
    shift[(int64_t)w * ldn + row] = (uint8_t)sh;
  };
  if (ok) {
#pragma unroll
    for (int i = 0; i < ST_W; ++i) {
      const int w = q + ST_Q * i;
      if (w < nwin) fold(w, ev[i], sv[i]);
    }
    for (int w = q + ST_Q * ST_W; w < nwin; w += ST_Q) fold(w, win_e[(int64_t)w * ldn + row], win_s[(int64_t)w * ldn + row]);
  }
  red[q][t] = S;
  lds_barrier();
  if (q == 0 && ok) {
    S = 0.f;
#pragma unroll
    for (int k = 0; k < ST_Q; ++k) S += red[k][t];
    const float r = mo == -INFINITY ? 0.f : ldexpf(1.f, -(int)fminf(nE - mo, 300.f));
    s[row] = s[row] * r + S;
    m[row] = nE;
    r_out[row] = r;
  }
}

template <int DT>
SMEL_DEV float ld_t(const void* p, int64_t i) {
  if constexpr (DT == 0) return bf2f(static_cast<const uint16_t*>(p)[i]);
  else if constexpr (DT == 1) return static_cast<const float*>(p)[i];
  else return (float)static_cast<const _Float16*>(p)[i];
}
template <int DT>
SMEL_DEV void st_t(void* p, int64_t i, float v) {
  if constexpr (DT == 0) static_cast<uint16_t*>(p)[i] = f2bf(v);
  else if constexpr (DT == 1) static_cast<float*>(p)[i] = v;
  else static_cast<_Float16*>(p)[i] = (_Float16)v;
}

// one block per row: loss and (with acc) the gradient row; trows (optional) holds the target rows already in the
// rows' dtype, else they are read from W at the target id
template <int DT, int GT>
__global__ __launch_bounds__(256) void ce_finish_kernel(const float* __restrict__ m, const float* __restrict__ s,
                                                        const float* __restrict__ tz, const float* __restrict__ td,
                                                        const float* __restrict__ acc,
                                                        const float* __restrict__ part, const void* __restrict__ W,
                                                        int64_t ldw, const void* __restrict__ trows,
                                                        const int64_t* __restrict__ tgt, int64_t V, int64_t H,
                                                        float gscale, void* g, int64_t ldg, float* loss_rows,
                                                        bool vec) {
  const int64_t row = blockIdx.x;
  const float sr = s[row];
  const int64_t t = tgt[row];
  const bool ok = t >= 0 && t < V;
  if (threadIdx.x == 0) loss_rows[row] = (m[row] * LN2 + logf(sr)) - tz[row];
  if (!acc) return;
  const float inv = 1.f / sr, d = ok ? td[row] : 0.f;
  const void* wsrc = trows ? trows : W;
  const int64_t wrow = trows ? row * H : (ok ? t : 0) * ldw;
  if (DT == 0 && GT == 0 && vec) {
    // 8 columns per thread and pass: 2 x 16-B loads of acc (and of part), one of the bf16 target row, one 16-B store
    for (int64_t c = 8 * (int64_t)threadIdx.x; c < H; c += 8 * 256) {
      const f32x4_t a0 = *reinterpret_cast<const f32x4_t*>(acc + row * H + c);
      const f32x4_t a1 = *reinterpret_cast<const f32x4_t*>(acc + row * H + c + 4);
      f32x4_t p0 = f32x4_t{0.f, 0.f, 0.f, 0.f}, p1 = p0;
      if (part) {
        p0 = *reinterpret_cast<const f32x4_t*>(part + row * H + c);
        p1 = *reinterpret_cast<const f32x4_t*>(part + row * H + c + 4);
      }
      const u32x4_t wv = ok ? *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(wsrc) + wrow + c)
                            : u32x4_t{0u, 0u, 0u, 0u};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float x0 = k < 2 ? a0[2 * k] + p0[2 * k] : a1[2 * k - 4] + p1[2 * k - 4];
        const float x1 = k < 2 ? a0[2 * k + 1] + p0[2 * k + 1] : a1[2 * k - 3] + p1[2 * k - 3];
        o[k] = pack2bf((x0 * inv - d * bf_lo(wv[k])) * gscale, (x1 * inv - d * bf_hi(wv[k])) * gscale);
      }
      *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(g) + row * ldg + c) = u32x4_t{o[0], o[1], o[2], o[3]};
    }
    return;
  }
  for (int64_t c = threadIdx.x; c < H; c += 256) {
    const float wv = ok ? ld_t<DT>(wsrc, wrow + c) : 0.f;
    const float v = (acc[row * H + c] + (part ? part[row * H + c] : 0.f)) * inv - d * wv;
    st_t<GT>(g, row * ldg + c, v * gscale);
  }
}

// total (+)= scale * sum of the rows' losses, in fixed order (one block)
__global__ __launch_bounds__(256) void ce_loss_sum_kernel(const float* __restrict__ loss_rows, int64_t n, float scale,
                                                          int accumulate, float* total) {
  __shared__ float red[256];
  float v = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 256) v += loss_rows[i];
  red[threadIdx.x] = v;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) *total = (accumulate ? *total : 0.f) + red[0] * scale;
}

// x *= *go for n values of the rows' dtype (the backward's incoming gradient, a device scalar)
template <int DT>
__global__ __launch_bounds__(256) void ce_scale_kernel(void* x, int64_t n, const float* __restrict__ go) {
  const float f = *go;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    st_t<DT>(x, i, ld_t<DT>(x, i) * f);
}

// dst [C][ldd] = src [R][C] (pitch lds) transposed, 64 x 64 tiles through LDS; dst columns R .. ldd - 1 zeroed
template <int E>
__global__ __launch_bounds__(256) void ce_transpose_kernel(const uint8_t* __restrict__ src, int64_t R, int64_t C,
                                                           int64_t lds, uint8_t* __restrict__ dst, int64_t ldd) {
  __shared__ uint8_t tile[64][64 * E + 4];
  const int64_t r0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int rr = i / 64, cc = i % 64;
    const int64_t r = r0 + rr, c = c0 + cc;
    uint8_t* t = &tile[rr][cc * E];
    if (r < R && c < C) {
      for (int b = 0; b < E; ++b) t[b] = src[(r * lds + c) * E + b];
    } else {
      for (int b = 0; b < E; ++b) t[b] = 0;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int cc = i / 64, rr = i % 64;
    const int64_t r = r0 + rr, c = c0 + cc;
    if (c < C && r < ldd)
      for (int b = 0; b < E; ++b) dst[(c * ldd + r) * E + b] = tile[rr][cc * E + b];
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// ------------------------------------------------------------------------------------------------ C-ABI
#define SMEL_DT_OK(dt) ((dt) >= 0 && (dt) <= 2)

extern "C" int smel_ce_begin(float* m, float* s, float* tz, float* td, const float* m0, int64_t n,
                             hipStream_t stream) {
  SMEL_REQUIRE(n >= 0, SMEL_EINVAL, "ce_begin: n=%lld", (long long)n);
  if (n == 0) return 0;
  SMEL_REQUIRE(m && s && tz && td, SMEL_EINVAL, "ce_begin: null pointer");
  ce_begin_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream>>>(m, s, tz, td, m0, n);
  return smel::launch_status();
}

extern "C" int smel_ce_logits(const void* W, int64_t ldw, int64_t vc, int64_t v0, const void* h, int64_t ldh,
                              int64_t n, int64_t H, const int64_t* tgt, float softcap, int32_t dtype, void* P,
                              int64_t ldp, float* win_e, float* win_s, int64_t ldn, float* tz, float* td,
                              hipStream_t stream) {
  SMEL_REQUIRE(SMEL_DT_OK(dtype), SMEL_EINVAL, "ce_logits: dtype %d (0 bf16, 1 fp32, 2 fp16)", dtype);
  const int E = dtype == 1 ? 4 : 2;
  SMEL_REQUIRE(n >= 0 && vc >= 1 && H >= 1 && v0 >= 0, SMEL_EINVAL, "ce_logits: bad sizes n=%lld vc=%lld H=%lld",
               (long long)n, (long long)vc, (long long)H);
  if (n == 0) return 0;
  SMEL_REQUIRE(W && h && tgt && win_e && win_s && tz && td, SMEL_EINVAL, "ce_logits: null pointer");
  SMEL_REQUIRE((H * E) % 16 == 0 && (ldw * E) % 16 == 0 && (ldh * E) % 16 == 0 && ldw >= H && ldh >= H &&
                   aligned16(W) && aligned16(h),
               SMEL_EUNSUPPORTED, "ce_logits: rows must be 16-byte aligned runs (H=%lld, ldw=%lld, ldh=%lld)",
               (long long)H, (long long)ldw, (long long)ldh);
  const int64_t vcp = (vc + VT - 1) / VT * VT;
  SMEL_REQUIRE(!P || (ldp >= vcp && (ldp * E) % 16 == 0 && aligned16(P)), SMEL_EINVAL,
               "ce_logits: softmax rows need %lld columns, 16-byte aligned (ldp=%lld)", (long long)vcp, (long long)ldp);
  SMEL_REQUIRE(ldn >= n, SMEL_EINVAL, "ce_logits: statistics pitch %lld < %lld rows", (long long)ldn, (long long)n);
  SMEL_REQUIRE((ldw * E) * 256 < ((int64_t)1 << 31) && (ldh * E) * 256 < ((int64_t)1 << 31) && vc < INT32_MAX &&
                   n < INT32_MAX,
               SMEL_EUNSUPPORTED, "ce_logits: tile offsets exceed 31 bits");
  LogitsArgs a;
  a.W = W;
  a.h = h;
  a.tgt = tgt;
  a.P = P;
  a.win_e = win_e;
  a.win_s = win_s;
  a.tz = tz;
  a.td = td;
  a.ldw = ldw;
  a.ldh = ldh;
  a.ldp = ldp;
  a.ldn = ldn;
  a.v0 = v0;
  a.vc = (int)vc;
  a.n = (int)n;
  a.K = (int)H;
  a.cap = softcap;
  a.n_vt = (int)(vcp / VT);
  a.n_tt = (int)((n + 255) / 256);
  const int64_t blocks = xcd_grid(a.n_vt) * a.n_tt;
  SMEL_REQUIRE(blocks < INT32_MAX, SMEL_EUNSUPPORTED, "ce_logits: grid too large");
  const dim3 g((unsigned)blocks), b(64 * LG_NW);
  const bool cap = softcap != 0.f;
  if (dtype == 0 && cap) ce_logits_kernel<0, true><<<g, b, 0, stream>>>(a);
  else if (dtype == 0) ce_logits_kernel<0, false><<<g, b, 0, stream>>>(a);
  else if (dtype == 1 && cap) ce_logits_kernel<1, true><<<g, b, 0, stream>>>(a);
  else if (dtype == 1) ce_logits_kernel<1, false><<<g, b, 0, stream>>>(a);
  else if (cap) ce_logits_kernel<2, true><<<g, b, 0, stream>>>(a);
  else ce_logits_kernel<2, false><<<g, b, 0, stream>>>(a);
  return smel::launch_status();
}

extern "C" int smel_ce_stats(const float* win_e, const float* win_s, int64_t nwin, int64_t ldn, int64_t n, float* m,
                             float* s, uint8_t* shift, float* r, hipStream_t stream) {
  SMEL_REQUIRE(n >= 0 && nwin >= 1 && ldn >= n, SMEL_EINVAL, "ce_stats: bad sizes");
  if (n == 0) return 0;
  SMEL_REQUIRE(win_e && win_s && m && s && shift && r, SMEL_EINVAL, "ce_stats: null pointer");
  SMEL_REQUIRE(nwin < INT32_MAX, SMEL_EUNSUPPORTED, "ce_stats: too many windows");
  ce_stats_kernel<<<dim3((unsigned)((n + ST_ROWS - 1) / ST_ROWS)), dim3(256), 0, stream>>>(win_e, win_s, (int)nwin,
                                                                                        ldn, n, m, s, shift, r);
  return smel::launch_status();
}

extern "C" int smel_ce_grad(const void* WT, int64_t ldwt, int64_t H, const void* P, int64_t ldp, int64_t vc,
                            const uint8_t* shift, int64_t ldn, const float* r, int64_t n, int32_t dtype, int32_t chunk,
                            float* acc, float* part, hipStream_t stream) {
  SMEL_REQUIRE(SMEL_DT_OK(dtype), SMEL_EINVAL, "ce_grad: dtype %d (0 bf16, 1 fp32, 2 fp16)", dtype);
  const int E = dtype == 1 ? 4 : 2;
  SMEL_REQUIRE(n >= 0 && vc >= 1 && H >= 1 && ldn >= n && chunk >= 0, SMEL_EINVAL, "ce_grad: bad sizes");
  if (n == 0) return 0;
  SMEL_REQUIRE(WT && P && shift && acc && part && (chunk == 0 || r), SMEL_EINVAL, "ce_grad: null pointer");
  const int64_t kbytes = (vc * E + 15) / 16 * 16;
  SMEL_REQUIRE(H % 4 == 0 && aligned16(acc) && aligned16(part) && aligned16(WT) && aligned16(P) &&
                   (ldwt * E) % 16 == 0 && (ldp * E) % 16 == 0 && ldp * E >= kbytes && ldwt * E >= kbytes,
               SMEL_EUNSUPPORTED, "ce_grad: rows must be 16-byte aligned runs covering the chunk (H=%lld)",
               (long long)H);
  SMEL_REQUIRE((ldwt * E) * 256 < ((int64_t)1 << 31) && (ldp * E) * 256 < ((int64_t)1 << 31) && H < INT32_MAX &&
                   n < INT32_MAX,
               SMEL_EUNSUPPORTED, "ce_grad: tile offsets exceed 31 bits");
  GradArgs a;
  a.WT = WT;
  a.P = P;
  a.shift = shift;
  a.r = r;
  a.acc = acc;
  a.part = part;
  a.ldwt = ldwt;
  a.ldp = ldp;
  a.ldn = ldn;
  a.H = (int)H;
  a.n = (int)n;
  a.kbytes = (int)kbytes;
  a.first = chunk == 0;
  a.parity = chunk & 1;
  a.n_ht = (int)((H + 255) / 256);
  a.n_tt = (int)((n + 255) / 256);
  const int64_t items = 2 * (int64_t)a.n_ht * a.n_tt;
  SMEL_REQUIRE(items < INT32_MAX, SMEL_EUNSUPPORTED, "ce_grad: grid too large");
  const dim3 g((unsigned)xcd_grid(items)), b(64 * GR_NW);
  if (dtype == 0) ce_grad_kernel<0><<<g, b, 0, stream>>>(a);
  else if (dtype == 1) ce_grad_kernel<1><<<g, b, 0, stream>>>(a);
  else ce_grad_kernel<2><<<g, b, 0, stream>>>(a);
  return smel::launch_status();
}

extern "C" int smel_ce_finish(const float* m, const float* s, const float* tz, const float* td, const float* acc,
                              const float* part, const void* W, int64_t ldw, const void* trows, const int64_t* tgt, int64_t V, int64_t n,
                              int64_t H, int32_t dtype, float gscale, void* g, int64_t ldg, int32_t g_dtype,
                              float* loss_rows, hipStream_t stream) {
  SMEL_REQUIRE(SMEL_DT_OK(dtype) && SMEL_DT_OK(g_dtype), SMEL_EINVAL, "ce_finish: dtype %d / %d", dtype, g_dtype);
  SMEL_REQUIRE(n >= 0 && H >= 1 && V >= 1, SMEL_EINVAL, "ce_finish: bad sizes");
  if (n == 0) return 0;
  SMEL_REQUIRE(m && s && tz && td && tgt && loss_rows && (!acc || (g && ldg >= H && (W || trows))), SMEL_EINVAL,
               "ce_finish: null pointer");
  SMEL_REQUIRE(n < INT32_MAX, SMEL_EUNSUPPORTED, "ce_finish: too many rows");
  const dim3 gr((unsigned)n), b(256);
  // 16-byte accesses when every row of acc, part, the target rows and g starts on 16 bytes
  const auto al16 = [](const void* p) { return ((uintptr_t)p % 16) == 0; };
  const bool vec = acc && H % 8 == 0 && al16(acc) && al16(part) && al16(g) && ldg % 8 == 0 &&
                   (trows ? al16(trows) : (al16(W) && ldw % 8 == 0));
#define SMEL_FIN(D, G) \
  ce_finish_kernel<D, G><<<gr, b, 0, stream>>>(m, s, tz, td, acc, part, W, ldw, trows, tgt, V, H, gscale, g, ldg, \
                                               loss_rows, vec)
#define SMEL_FIN_G(D)            \
  if (g_dtype == 0) SMEL_FIN(D, 0); \
  else if (g_dtype == 1) SMEL_FIN(D, 1); \
  else SMEL_FIN(D, 2);
  if (dtype == 0) {
    SMEL_FIN_G(0)
  } else if (dtype == 1) {
    SMEL_FIN_G(1)
  } else {
    SMEL_FIN_G(2)
  }
#undef SMEL_FIN_G
#undef SMEL_FIN
  return smel::launch_status();
}

extern "C" int smel_ce_loss_sum(const float* loss_rows, int64_t n, float scale, int32_t accumulate, float* total,
                                hipStream_t stream) {
  SMEL_REQUIRE(n >= 0 && total && (n == 0 || loss_rows), SMEL_EINVAL, "ce_loss_sum: bad arguments");
  ce_loss_sum_kernel<<<dim3(1), dim3(256), 0, stream>>>(loss_rows, n, scale, accumulate, total);
  return smel::launch_status();
}

extern "C" int smel_ce_scale(void* x, int64_t n, int32_t dtype, const float* go, hipStream_t stream) {
  SMEL_REQUIRE(SMEL_DT_OK(dtype) && n >= 0, SMEL_EINVAL, "ce_scale: dtype %d, n %lld", dtype, (long long)n);
  if (n == 0) return 0;
  SMEL_REQUIRE(x && go, SMEL_EINVAL, "ce_scale: null pointer");
  const dim3 g((unsigned)std::min<int64_t>((n + 255) / 256, 4096)), b(256);
  if (dtype == 0) ce_scale_kernel<0><<<g, b, 0, stream>>>(x, n, go);
  else if (dtype == 1) ce_scale_kernel<1><<<g, b, 0, stream>>>(x, n, go);
  else ce_scale_kernel<2><<<g, b, 0, stream>>>(x, n, go);
  return smel::launch_status();
}

extern "C" int smel_ce_transpose(const void* src, int64_t R, int64_t C, int64_t lds, void* dst, int64_t ldd,
                                 int32_t dtype, hipStream_t stream) {
  SMEL_REQUIRE(SMEL_DT_OK(dtype), SMEL_EINVAL, "ce_transpose: dtype %d", dtype);
  SMEL_REQUIRE(R >= 0 && C >= 0 && lds >= C && ldd >= R, SMEL_EINVAL, "ce_transpose: bad sizes");
  if (R == 0 || C == 0) return 0;
  SMEL_REQUIRE(src && dst, SMEL_EINVAL, "ce_transpose: null pointer");
  const int64_t gx = (ldd + 63) / 64, gy = (C + 63) / 64;
  SMEL_REQUIRE(gx < INT32_MAX && gy < 65536, SMEL_EUNSUPPORTED, "ce_transpose: too large");
  const dim3 g((unsigned)gx, (unsigned)gy), b(256);
  const auto* s8 = static_cast<const uint8_t*>(src);
  auto* d8 = static_cast<uint8_t*>(dst);
  if (dtype == 1) ce_transpose_kernel<4><<<g, b, 0, stream>>>(s8, R, C, lds, d8, ldd);
  else ce_transpose_kernel<2><<<g, b, 0, stream>>>(s8, R, C, lds, d8, ldd);
  return smel::launch_status();
}
