// Dispatch: stable counting sort of the flat expert ids (the argsort(stable=True) + bincount of routed_experts,
// smel/moe.py:216-223, and the inverse permutation of :249-250), plus the GEMM tile list. No host sync: counts and
// offsets stay on the device and the grouped GEMMs read the tile list.
//
// One workgroup of 1024 threads (16 waves). Wave w owns the contiguous slot range [w*C, (w+1)*C). Pass 1 counts per
// (wave, expert) in LDS; a scan over waves and experts gives each (wave, expert) its first output position; pass 2
// walks the wave's range 64 slots at a time and ranks equal ids inside the step with ballots (a wave-level
// multisplit), so slot order inside an expert is ascending p — exactly the stable sort.
#include "abi_util.h"
#include "common.h"

namespace {

constexpr int NW = 16;        // waves
constexpr int MAXE = 512;

SMEL_DEV int block_exclusive_scan(int v, int* wsum /* [NW] LDS */, int& total) {
  const int l = lane_id(), w = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(inc, o, 64);
    if (l >= o) inc += y;
  }
  if (l == 63) wsum[w] = inc;
  __syncthreads();
  int base = 0, tot = 0;
  for (int j = 0; j < NW; ++j) {
    const int s = wsum[j];
    if (j < w) base += s;
    tot += s;
  }
  __syncthreads();
  total = tot;
  return base + inc - v;
}

__global__ __launch_bounds__(1024) void dispatch_kernel(const void* __restrict__ ids, int is64, int TK, int E,
                                                        int shared_rows, int m_tile, int max_tiles,
                                                        int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                        int32_t* __restrict__ order, int32_t* __restrict__ inv,
                                                        int32_t* __restrict__ tiles, int32_t* __restrict__ n_tiles,
                                                        int32_t* __restrict__ err) {
  __shared__ int hist[NW * MAXE];   // per-wave counts, then per-wave write cursors
  __shared__ int off_s[MAXE + 1];
  __shared__ int wsum[NW];
  __shared__ int bad;
  const int tid = threadIdx.x, l = lane_id(), w = tid >> 6;
  auto id_at = [&](int p) -> int {
    return is64 ? (int)static_cast<const int64_t*>(ids)[p] : static_cast<const int32_t*>(ids)[p];
  };
  for (int i = tid; i < NW * E; i += 1024) hist[i] = 0;
  if (tid == 0) bad = 0;
  __syncthreads();
  const int chunk = (TK + NW - 1) / NW;
  const int p0 = min(TK, w * chunk), p1 = min(TK, p0 + chunk);
  for (int p = p0 + l; p < p1; p += 64) {
    const int e = id_at(p);
    if (e >= 0 && e < E)
      atomicAdd(&hist[w * E + e], 1);
    else
      bad = 1;
  }
  __syncthreads();
  // per expert: exclusive prefix over waves (in place), total count
  int my_total = 0;
  for (int e = tid; e < E; e += 1024) {
    int run = 0;
    for (int j = 0; j < NW; ++j) {
      const int c = hist[j * E + e];
      hist[j * E + e] = run;
      run += c;
    }
    my_total = run;   // E <= 1024: one expert per thread
  }
  int total_rows;
  const int ex = block_exclusive_scan(tid < E ? my_total : 0, wsum, total_rows);
  if (tid < E) {
    off_s[tid] = ex;
    counts[tid] = my_total;
    offsets[tid] = ex;
  }
  if (tid == 0) {
    off_s[E] = total_rows;
    offsets[E] = total_rows;
  }
  __syncthreads();
  for (int i = tid; i < NW * E; i += 1024) hist[i] += off_s[i % E];
  __syncthreads();
  // pass 2: stable ranking inside 64-slot steps
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  for (int base = p0; base < p1; base += 64) {
    const int p = base + l;
    int e = p < p1 ? id_at(p) : -1;
    const bool ok = e >= 0 && e < E;
    uint64_t m = __ballot(ok);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = ok && ((e >> b) & 1);
      const uint64_t bb = __ballot(bit);
      m &= bit ? bb : ~bb;
    }
    if (ok) {
      const uint64_t lt = (l == 0) ? 0ull : (~0ull >> (64 - l));
      const int rank = __popcll(m & lt);
      const int pos = hist[w * E + e] + rank;
      order[pos] = p;
      inv[p] = pos;
      if ((m >> l) == 1ull) hist[w * E + e] += __popcll(m);   // highest lane of the group advances the cursor
    } else if (p < p1) {
      inv[p] = -1;
    }
  }
  // tile list over groups 0..E-1 (+ shared group E)
  const int G = E + (shared_rows > 0 ? 1 : 0);
  int nt = 0, rows = 0, row0 = 0;
  if (tid < G) {
    rows = tid < E ? off_s[tid + 1] - off_s[tid] : shared_rows;
    row0 = tid < E ? off_s[tid] : TK;
    nt = (rows + m_tile - 1) / m_tile;
  }
  int total_tiles;
  const int tbase = block_exclusive_scan(nt, wsum, total_tiles);
  if (tid < G) {
    for (int i = 0; i < nt && tbase + i < max_tiles; ++i) {
      int4 tl;
      tl.x = tid;
      tl.y = row0 + i * m_tile;
      tl.z = min(row0 + rows, row0 + (i + 1) * m_tile);
      tl.w = 0;
      reinterpret_cast<int4*>(tiles)[tbase + i] = tl;
    }
  }
  if (tid == 0) {
    n_tiles[0] = min(total_tiles, max_tiles);
    err[0] = bad | (total_tiles > max_tiles ? 2 : 0);
  }
}

}  // namespace

extern "C" int64_t smel_dispatch_max_tiles(int64_t TK, int64_t E, int64_t shared_rows, int32_t m_tile) {
  if (m_tile <= 0) return 0;
  return (TK + m_tile - 1) / m_tile + E + (shared_rows + m_tile - 1) / m_tile + 1;
}

extern "C" int smel_dispatch(const void* ids, int32_t ids_are_i64, int64_t T, int64_t K, int64_t E,
                             int64_t shared_rows, int32_t m_tile, int32_t* counts, int32_t* offsets, int32_t* order,
                             int32_t* inv, int32_t* tiles, int32_t* n_tiles, int32_t* err, hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && K > 0 && E > 0 && shared_rows >= 0 && m_tile > 0, SMEL_EINVAL, "dispatch: bad sizes");
  SMEL_REQUIRE(E <= MAXE, SMEL_EUNSUPPORTED, "dispatch: E=%lld > %d experts", (long long)E, MAXE);
  SMEL_REQUIRE(T * K < (1ll << 30), SMEL_EUNSUPPORTED, "dispatch: T*K too large");
  SMEL_REQUIRE(counts && offsets && tiles && n_tiles && err && (T == 0 || (ids && order && inv)), SMEL_EINVAL,
               "dispatch: null pointer");
  const int64_t mt = smel_dispatch_max_tiles(T * K, E, shared_rows, m_tile);
  dispatch_kernel<<<1, 1024, 0, stream>>>(ids, ids_are_i64 ? 1 : 0, (int)(T * K), (int)E, (int)shared_rows, m_tile,
                                          (int)mt, counts, offsets, order, inv, tiles, n_tiles, err);
  return smel::launch_status();
}
