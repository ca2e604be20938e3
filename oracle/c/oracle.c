/* C restatement of the integer/byte parts of SMEL FT's MoE-layer hot path — TEST INFRASTRUCTURE ONLY.
 *
 * Loaded by tests/ through ctypes (oracle/intref.py) as a second, independent restatement beside the numpy/torch
 * one; never linked into or called by the product library.
 *
 *   oracle_bf16_rne           fp32 -> bf16 round-to-nearest-even (torch's .to(torch.bfloat16); NaN kept quiet)
 *   oracle_dequant_int4       w = q*s + z in fp32, one RNE to bf16 (smel/quant.py:51-67, the GPU-kernel form;
 *                             low nibble = even column, smel/quant.py:42)
 *   oracle_dispatch           stable counting sort of the flat expert ids (smel/moe.py:216-223) + inverse
 *                             permutation (smel/moe.py:249-250)
 *   oracle_topk               top-k by value, lower index first among equal values (the deterministic form of
 *                             torch.topk used in smel/moe.py:165)
 */
#include <stdint.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t oracle_bf16_rne_one(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* NaN: keep it quiet */
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

void oracle_bf16_rne(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = oracle_bf16_rne_one(x[i]);
}

static float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* q [rows, K/2] bytes, scale/zero [rows, K/group] bf16 bits -> out [rows, K] bf16 bits (or fp32 if out_f32). */
void oracle_dequant_int4(const uint8_t* q, const uint16_t* scale, const uint16_t* zero, void* out, int64_t rows,
                         int64_t K, int64_t group, int32_t out_f32) {
  const int64_t G = K / group;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t k = 0; k < K; ++k) {
      const uint8_t b = q[r * (K / 2) + k / 2];
      const uint32_t nib = (k & 1) ? (b >> 4) : (b & 0xF);
      const float s = bf16_to_f32(scale[r * G + k / group]);
      const float z = bf16_to_f32(zero[r * G + k / group]);
      const float w = (float)nib * s + z; /* q*s is exact in fp32, so this rounds once */
      if (out_f32)
        ((float*)out)[r * K + k] = w;
      else
        ((uint16_t*)out)[r * K + k] = oracle_bf16_rne_one(w);
    }
  }
}

/* topi [T*K] (any order of k within a token) -> counts [E], offsets [E+1], order [T*K], inv [T*K]. Returns 0, or -1
 * when an id is outside [0, E). */
int32_t oracle_dispatch(const int32_t* topi, int64_t TK, int64_t E, int32_t* counts, int32_t* offsets,
                        int32_t* order, int32_t* inv) {
  for (int64_t e = 0; e < E; ++e) counts[e] = 0;
  for (int64_t p = 0; p < TK; ++p) {
    if (topi[p] < 0 || topi[p] >= E) return -1;
    counts[topi[p]]++;
  }
  offsets[0] = 0;
  for (int64_t e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
  for (int64_t e = 0; e < E; ++e) counts[e] = 0; /* reuse as per-expert cursor */
  for (int64_t p = 0; p < TK; ++p) {
    const int32_t e = topi[p];
    const int32_t j = offsets[e] + counts[e]++;
    order[j] = (int32_t)p;
    inv[p] = j;
  }
  return 0;
}

/* p [rows, n] -> v [rows, k], idx [rows, k]: descending value, lower index first among equal values. */
void oracle_topk(const float* p, int64_t rows, int64_t n, int64_t k, float* v, int32_t* idx) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = p + r * n;
    for (int64_t j = 0; j < k; ++j) {
      int64_t best = -1;
      for (int64_t c = 0; c < n; ++c) {
        int taken = 0;
        for (int64_t t = 0; t < j; ++t) taken |= (idx[r * k + t] == c);
        if (taken) continue;
        if (best < 0 || row[c] > row[best]) best = c; /* strict: the first (lowest) index wins ties */
      }
      idx[r * k + j] = (int32_t)best;
      v[r * k + j] = row[best];
    }
  }
}
