// Shared device helpers for the MoE-layer kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SMEL_DEV __device__ __forceinline__

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------------ bf16 <-> fp32
SMEL_DEV float bf2f(uint32_t h16) { return __uint_as_float(h16 << 16); }
SMEL_DEV float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
SMEL_DEV float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 (gfx950 converts in hardware, two values per v_cvt_pk_bf16_f32; NaN stays NaN).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
SMEL_DEV uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
SMEL_DEV uint32_t pack2bf(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

// ------------------------------------------------------------------------------------------------ wave helpers
SMEL_DEV int lane_id() { return __lane_id(); }

SMEL_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
SMEL_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// sum over the 32 lanes that share lane/32 (the two halves of a wave reduce independently)
SMEL_DEV float half_sum(float v) {
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ------------------------------------------------------------------------------------------------ MFMA
// v_mfma_f32_32x32x16_bf16: lane l supplies A[i = l%32][k in K-set(l/32)] and B[k in K-set(l/32)][j = l%32]
// (8 bf16 each); C lands as acc[r] = C[8*(r/4) + 4*(l/32) + r%4][l%32]. Which 8 k values a lane half carries is
// our choice as long as A and B agree.
SMEL_DEV f32x16_t mfma32(const u32x4_t& a, const u32x4_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}
SMEL_DEV int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// ------------------------------------------------------------------------------------------------ int4 dequant
// Byte n of x as fp32 (v_cvt_f32_ubyteN: one instruction, no separate extract).
SMEL_DEV float ub0(uint32_t x) { float f; asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(x)); return f; }
SMEL_DEV float ub1(uint32_t x) { float f; asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(x)); return f; }
SMEL_DEV float ub2(uint32_t x) { float f; asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(x)); return f; }
SMEL_DEV float ub3(uint32_t x) { float f; asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(x)); return f; }

// 8 nibbles of one uint32 (little-endian bytes; low nibble = even column) -> 4 packed bf16 pairs,
// w = RNE_bf16(q*s + z) with fp32 arithmetic (q*s is exact, so fma and mul+add agree): 23 VALU ops for 8 weights.
SMEL_DEV void dq8(uint32_t b, float s, float z, uint32_t out[4]) {
  const uint32_t lo = b & 0x0f0f0f0fu;          // columns 0,2,4,6
  const uint32_t hi = (b >> 4) & 0x0f0f0f0fu;   // columns 1,3,5,7
  out[0] = pack2bf(fmaf(ub0(lo), s, z), fmaf(ub0(hi), s, z));
  out[1] = pack2bf(fmaf(ub1(lo), s, z), fmaf(ub1(hi), s, z));
  out[2] = pack2bf(fmaf(ub2(lo), s, z), fmaf(ub2(hi), s, z));
  out[3] = pack2bf(fmaf(ub3(lo), s, z), fmaf(ub3(hi), s, z));
}

// Nibble j (0..7) of b as float.
SMEL_DEV float nib(uint32_t b, int j) { return (float)((b >> (4 * j)) & 0xfu); }

// ---- The same value in 17 instead of 23 VALU ops (banks whose scale/zero pass smel_int4_fast_ok).
// A nibble q ORed into the low mantissa bits of the fp16 1024.0 (0x6400) is the fp16 value 1024 + q, and in bits 4..7
// it is 1024 + 16 q: exact. v_fma_mix_f32 multiplies that fp16 half (either half of a register, no extraction) by an
// fp32 operand and adds an fp32 operand, rounded once:
//   fma(1024 + q, s, z - 1024 s)       = fl(q s + z)
//   fma(1024 + 16 q, s / 16, z - 64 s) = fl(q s + z)
// whenever z - 1024 s, z - 64 s and s / 16 are exact fp32 values (both sides then round the same real number), which
// smel_int4_fast_ok checks for every group of a bank when it is packed. One AND-OR per two weights replaces the
// nibble split and the byte-to-float conversions of dq8.
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
SMEL_DEV float h_lo(uint32_t x) { return (float)__builtin_bit_cast(h2_t, x)[0]; }
SMEL_DEV float h_hi(uint32_t x) { return (float)__builtin_bit_cast(h2_t, x)[1]; }
// fp16 pair (1024, 1024) in a vector register: v_and_or_b32 takes the mask from a scalar register and this constant
// from a vector one (one scalar operand per instruction), so it must not be folded into a literal.
SMEL_DEV uint32_t f16_magic() {
  uint32_t m;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(m));
  return m;
}
struct FastSZ {
  float a0, c0, a1, c1;   // s, z - 1024 s, s / 16, z - 64 s
};
SMEL_DEV FastSZ fast_sz(float s, float z) {
  return FastSZ{s, fmaf(-1024.f, s, z), s * 0.0625f, fmaf(-64.f, s, z)};
}
// dq8 for a fast bank: nibbles t = 0..7 of b (bits 4t) are columns 0..7.
SMEL_DEV void dq8f(uint32_t b, const FastSZ& p, uint32_t magic, uint32_t out[4]) {
  const uint32_t b8 = b >> 8;
  const uint32_t x0 = (b & 0x000F000Fu) | magic;    // columns 0, 4 at 1024 + q
  const uint32_t x1 = (b & 0x00F000F0u) | magic;    // columns 1, 5 at 1024 + 16 q
  const uint32_t x2 = (b8 & 0x000F000Fu) | magic;   // columns 2, 6
  const uint32_t x3 = (b8 & 0x00F000F0u) | magic;   // columns 3, 7
  out[0] = pack2bf(fmaf(h_lo(x0), p.a0, p.c0), fmaf(h_lo(x1), p.a1, p.c1));
  out[1] = pack2bf(fmaf(h_lo(x2), p.a0, p.c0), fmaf(h_lo(x3), p.a1, p.c1));
  out[2] = pack2bf(fmaf(h_hi(x0), p.a0, p.c0), fmaf(h_hi(x1), p.a1, p.c1));
  out[3] = pack2bf(fmaf(h_hi(x2), p.a0, p.c0), fmaf(h_hi(x3), p.a1, p.c1));
}

// ------------------------------------------------------------------------------------------------ activations
// act ids: 0 = silu, 1 = gelu_tanh (smel/moe.py:91-107)
// e^x as one v_exp_f32 (2^x; results below the normal range flush to 0, which cannot change 1 + e^x)
SMEL_DEV float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
// SiLU as g * sigmoid(g), the sigmoid by v_rcp_f32 (1 ulp): the results are rounded to bf16 next
SMEL_DEV float act_f(float g, int act) {
  if (act == 0) return g * __builtin_amdgcn_rcpf(1.0f + exp_fast(-g));
  const float c = 0.7978845608028654f;
  const float t = tanhf(c * (g + 0.044715f * g * g * g));
  return 0.5f * g * (1.0f + t);
}
SMEL_DEV void act_and_grad_f(float g, int act, float& a, float& da) {
  if (act == 0) {   // the same sigmoid as act_f
    const float s = __builtin_amdgcn_rcpf(1.0f + exp_fast(-g));
    a = g * s;
    da = s * (1.0f + g * (1.0f - s));
    return;
  }
  const float c = 0.7978845608028654f;
  const float t = tanhf(c * (g + 0.044715f * g * g * g));
  a = 0.5f * g * (1.0f + t);
  da = 0.5f * (1.0f + t) + 0.5f * g * (1.0f - t * t) * c * (1.0f + 3.0f * 0.044715f * g * g);
}

// ------------------------------------------------------------------------------------------------ buffer loads
// Raw buffer loads: a load whose byte offset is outside [0, bytes) returns zeros, so rows past a tile's end and
// columns past a matrix's end need no branch — their offset is set to OOB.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t OOB = 0x80000000u;
SMEL_DEV rsrc_t make_rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0x7fffffffull ? 0x7fffffffu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}
SMEL_DEV u32x4_t ld16(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
SMEL_DEV uint32_t ld2(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0); }
SMEL_DEV uint32_t ld4(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
SMEL_DEV u32x2_t ld8(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0); }

// Loads straight into LDS (gfx950: 16 B per lane): lane i of the wave writes bytes [16 i, 16 i + 16) after the
// wave-uniform LDS address `lds`; an out-of-range offset writes zeros. Completion is counted by vmcnt.
typedef __attribute__((address_space(3))) void* lds_ptr_t;
SMEL_DEV void ld16_lds(rsrc_t r, const void* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(lds), 16, off, 0, 0, 0);
}
// s_waitcnt on the vector-memory counter only (gfx9 encoding: vmcnt bits [3:0] and [15:14]).
#define SMEL_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
// ... and on LDS as well (lgkmcnt = 0): this wave's own LDS reads are done.
#define SMEL_WAIT_VM_LDS(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4))
// The same waits with the count checked at compile time. A pipelined main loop computes N from the per-group load
// counts its issue code is written with (constexpr), so a count cannot drift from the loads actually issued.
template <int N>
SMEL_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt counts 0..63 outstanding vector-memory operations");
  SMEL_WAIT_VM(N);
}
template <int N>
SMEL_DEV void wait_vm_lds() {
  static_assert(N >= 0 && N < 64, "vmcnt counts 0..63 outstanding vector-memory operations");
  SMEL_WAIT_VM_LDS(N);
}
// Workgroup barrier for hand-offs through LDS only: it orders the block's LDS accesses around the barrier and waits
// for none of the wave's global loads or stores. (__syncthreads also waits for every outstanding global access, a
// whole memory round trip after a store.) Only for code whose threads exchange nothing through global memory.
SMEL_DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Operand tiles in LDS hold rows of 64 bf16 (128 B) without padding; the physical 16-B chunk of logical chunk c of
// row r is c ^ swz(r), so 8 (or 16) lanes reading consecutive rows at one logical chunk touch distinct banks with 32
// (or 64) four-byte banks.
SMEL_DEV int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// ------------------------------------------------------------------------------------------------ XCD-aware tiles
// MI355X has 8 XCDs, each with its own L2; consecutive workgroup ids go to consecutive XCDs. A 1-D grid of
// xcd_grid(max_tiles) * nblk workgroups are mapped so that the nblk column blocks of one tile run back to back on one
// XCD (workgroups go to the XCDs round robin: block b to XCD b % 8): they share the tile's A rows in that XCD's L2.
// xcd_tile: tiles are taken in list order, tile t on XCD t % 8. xcd_tile_chunk: XCD x takes the contiguous chunk
// [x c, (x + 1) c) of the list (c = ceil(n_tiles / 8)) in order, so with a list in group order the tiles of one group
// run side by side on one XCD and share its weights in that XCD's L2.
constexpr int NXCD = 8;
// Slots per block of the dispatch's per-block expert histograms (the dispatch workspace holds [blocks][E] counts,
// then one bad-id flag per block); smel_route_counted writes the same histograms.
constexpr int DISPATCH_SLOTS = 1024;
inline int64_t xcd_grid(int64_t max_tiles) { return (max_tiles + NXCD - 1) / NXCD * NXCD; }
SMEL_DEV bool xcd_tile_chunk(int n_tiles, int nblk, int& tile, int& nb) {
  const int b = blockIdx.x;
  const int x = b % NXCD, j = b / NXCD;
  const int chunk = (n_tiles + NXCD - 1) / NXCD;
  const int r = j / nblk;
  if (r >= chunk) return false;
  const int t = x * chunk + r;
  if (t >= n_tiles) return false;
  tile = t;
  nb = j % nblk;
  return true;
}
SMEL_DEV bool xcd_tile(int n_tiles, int nblk, int& tile, int& nb) {
  const int b = blockIdx.x;
  const int x = b % NXCD, j = b / NXCD;
  const int t = (j / nblk) * NXCD + x;
  if (t >= n_tiles) return false;
  tile = t;
  nb = j % nblk;
  return true;
}

// ------------------------------------------------------------------------------------------------ row mapping
// Rows of the grouped GEMMs: [0, TK) are the routed slots in expert-sorted order, [TK, TK + T) the shared expert
// (one row per token, in token order). order[row] = flat slot p = t*K + k of a routed row.
SMEL_DEV int row_token(int row, const int32_t* __restrict__ order, int TK, int topk) {
  return row < TK ? order[row] / topk : row - TK;
}
SMEL_DEV int row_slot(int row, const int32_t* __restrict__ order, int TK) { return row < TK ? order[row] : row; }
