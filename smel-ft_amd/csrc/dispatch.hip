// Dispatch: stable counting sort of the flat expert ids (the argsort(stable=True) + bincount of routed_experts,
// smel/moe.py:216-223, and the inverse permutation of :249-250), plus the GEMM tile list. No host sync: counts and
// offsets stay on the device and the grouped GEMMs read the tile list.
//
// Launches over blocks of 1024 slots (one per thread): (1) per-block expert histograms; (2) one block turns them into
// counts, offsets, each block's first output position per expert, and the tile list; (3) every block ranks its slots
// again — inside a wave by ballots over the id bits (a wave-level multisplit), across its 16 waves by a per-expert
// prefix — and scatters order / inv. Slots of one expert thus keep ascending p: the stable sort. With at most 64
// blocks (T * K <= 65536 slots) (2) and (3) are one launch: each block folds every block's histogram itself.
#include <mutex>

#include "abi_util.h"
#include "common.h"

// Workspace of smel_dispatch_noalloc (the allocation-free variant below): one copy of this array on every GPU the
// library runs on, held until the process ends. In host code the name is a host-side stand-in, not a device
// address: kernels only ever receive the address hipGetSymbolAddress returns for the current device.
constexpr int64_t SCRATCH_INTS = 1 << 18;   // 1 MiB: nb * (E + 1) ints for nb = ceil(T*K / 1024) blocks
static __device__ __align__(256) int32_t scratch[SCRATCH_INTS];

namespace {

constexpr int NW = 16;        // waves per block
constexpr int DB = NW * 64;   // slots per block
static_assert(DB == DISPATCH_SLOTS, "the histogram blocks smel_route_counted fills");
constexpr int MAXE = 512;
constexpr int HCH = 12288;    // histogram entries per LDS chunk of dispatch_scan (48 KB)

SMEL_DEV int block_exclusive_scan(int v, int* wsum /* [NW] LDS */, int& total) {
  const int l = lane_id(), w = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(inc, o, 64);
    if (l >= o) inc += y;
  }
  if (l == 63) wsum[w] = inc;
  lds_barrier();
  int base = 0, tot = 0;
  for (int j = 0; j < NW; ++j) {
    const int s = wsum[j];
    if (j < w) base += s;
    tot += s;
  }
  lds_barrier();
  total = tot;
  return base + inc - v;
}

// Exclusive scan of N triples at once over the block (the latency of one scan); v is replaced by its exclusive
// prefix, tot = the block totals. wsum is not reused afterwards, so there is no trailing barrier.
struct I3 {
  int a, b, c;
};
template <int N>
SMEL_DEV void block_exclusive_scan3(I3 (&v)[N], I3 (*wsum)[N] /* [NW][N] LDS */, I3 (&tot)[N]) {
  const int l = lane_id(), w = threadIdx.x >> 6;
  I3 inc[N];
#pragma unroll
  for (int n = 0; n < N; ++n) inc[n] = v[n];
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const int ya = __shfl_up(inc[n].a, o, 64), yb = __shfl_up(inc[n].b, o, 64), yc = __shfl_up(inc[n].c, o, 64);
      if (l >= o) {
        inc[n].a += ya;
        inc[n].b += yb;
        inc[n].c += yc;
      }
    }
  }
  if (l == 63)
#pragma unroll
    for (int n = 0; n < N; ++n) wsum[w][n] = inc[n];
  lds_barrier();
#pragma unroll
  for (int n = 0; n < N; ++n) {
    I3 base{0, 0, 0}, t{0, 0, 0};
    for (int j = 0; j < NW; ++j) {
      const I3 s = wsum[j][n];
      if (j < w) {
        base.a += s.a;
        base.b += s.b;
        base.c += s.c;
      }
      t.a += s.a;
      t.b += s.b;
      t.c += s.c;
    }
    tot[n] = t;
    v[n] = I3{base.a + inc[n].a - v[n].a, base.b + inc[n].b - v[n].b, base.c + inc[n].c - v[n].c};
  }
}

SMEL_DEV int id_at(const void* ids, int is64, int p) {
  return is64 ? (int)static_cast<const int64_t*>(ids)[p] : static_cast<const int32_t*>(ids)[p];
}

SMEL_DEV int tiles_of(int rows, int m_tile) { return (rows + m_tile - 1) / m_tile; }
SMEL_DEV int long_tiles_of(int rows, int m_tile) {   // tiles of more than m_tile / 2 rows
  const int nt = tiles_of(rows, m_tile);
  return nt - ((nt > 0 && rows - (nt - 1) * m_tile <= m_tile / 2) ? 1 : 0);
}

// The merged tile list (tiles_m, merge_rows > m_tile), for the gate_up forward: an int4 group's last tile of at most
// merge_rows - m_tile rows joins the full tile before it (one tile, one weight stream and dequant for both). Order:
// the merged tiles, then the other tiles of more than m_tile / 2 rows, then the shorter ones, each part in group
// order (the costliest tiles start first, the short ones fill the last round). A group's counts: {merged (0 or 1),
// full or long (the tiles before the last, and the last when long), short (0 or 1)}.
SMEL_DEV I3 merged_counts(int rows, int m_tile, int merge_rows, bool int4) {
  const int nt = tiles_of(rows, m_tile);
  if (nt == 0) return I3{0, 0, 0};
  const int rem = rows - (nt - 1) * m_tile;
  const int a = (merge_rows > m_tile && int4 && nt >= 2 && rem <= merge_rows - m_tile) ? 1 : 0;
  const int last_long = (!a && rem > m_tile / 2) ? 1 : 0;
  return I3{a, nt - 1 - a + last_long, (!a && !last_long) ? 1 : 0};
}
struct TileLds {
  int lb[MAXE + 1], sb[MAXE + 1], mb[MAXE + 1], ma[MAXE + 1], row0[MAXE + 1], rows[MAXE + 1], nt[MAXE + 1],
      gk[MAXE + 1];
};
// Tile list over groups 0..E-1 (+ shared group E): the tiles of more than m_tile / 2 rows first (in group order), then
// the shorter last tiles of the groups (in group order). The grouped GEMMs start tiles in list order, so the short
// tiles fill the last round of workgroups instead of holding long ones back. tiles_g (optional): the same tiles in
// group order, a group's tiles next to each other.
// Group g = tid: rows from row0, nt tiles of which nlong long; lbase / sbase = its first position among the long /
// short tiles; n_long / n_short = the totals. The groups' values go through LDS, then thread q writes long tile q and
// short tile q (its group found by a binary search over the first positions), so no thread loops over a large
// group's tiles. Every thread of the block calls it (one barrier inside).
// Merged list (tiles_m != nullptr): mc / mpos = this group's merged_counts and their exclusive positions, mtot the
// totals.
SMEL_DEV void store_tiles(TileLds& t, int tid, int G, int rows, int row0, int nt, int lbase, int sbase, int n_long,
                          int n_short, int m_tile, int max_tiles, int gkv, int bad, int32_t* __restrict__ tiles,
                          int32_t* __restrict__ tiles_g, int32_t* __restrict__ n_tiles, int32_t* __restrict__ err,
                          I3 mc, I3 mpos, I3 mtot, int32_t* __restrict__ tiles_m, int32_t* __restrict__ n_tiles_m) {
  if (tid < G) {
    t.lb[tid] = lbase;
    t.sb[tid] = sbase;
    t.mb[tid] = mpos.b;
    t.ma[tid] = mc.a;
    t.row0[tid] = row0;
    t.rows[tid] = rows;
    t.nt[tid] = nt;
    t.gk[tid] = gkv;
  }
  lds_barrier();
  // the last group whose first position is <= q: the group of position q (groups without such tiles share their
  // first position with the next group)
  auto group_of = [&](const int* first, int q) {
    int lo = 0, hi = G - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (first[mid] <= q)
        lo = mid;
      else
        hi = mid - 1;
    }
    return lo;
  };
  // merged list: a long tile is also the merged list's full / long tile i of its group (at mtot.a + mb[g] + i), except
  // the one that a merged group's short last tile joins (that one the group's own thread writes)
  auto put = [&](int g, int i, int pos, bool is_long) {
    if (tiles_m && is_long && !(t.ma[g] && i >= t.nt[g] - 2)) {
      const int mp = mtot.a + t.mb[g] + i;
      if (mp < max_tiles) {
        const int r0 = t.row0[g];
        reinterpret_cast<int4*>(tiles_m)[mp] =
            int4{g, r0 + i * m_tile, min(r0 + t.rows[g], r0 + (i + 1) * m_tile), t.gk[g]};
      }
    }
    if (pos >= max_tiles) return;
    const int r0 = t.row0[g];
    int4 tl;
    tl.x = g;
    tl.y = r0 + i * m_tile;
    tl.z = min(r0 + t.rows[g], r0 + (i + 1) * m_tile);
    tl.w = t.gk[g];
    reinterpret_cast<int4*>(tiles)[pos] = tl;
    const int gpos = t.lb[g] + t.sb[g] + i;   // a group's tiles next to each other
    if (tiles_g && gpos < max_tiles) reinterpret_cast<int4*>(tiles_g)[gpos] = tl;
  };
  for (int q = tid; q < n_long; q += DB) {
    const int g = group_of(t.lb, q);
    put(g, q - t.lb[g], q, true);
  }
  for (int q = tid; q < n_short; q += DB) {   // only a group's last tile can be short
    const int g = group_of(t.sb, q);
    put(g, t.nt[g] - 1, n_long + q, false);
  }
  if (tid == 0) {
    const int total_tiles = n_long + n_short;
    n_tiles[0] = min(total_tiles, max_tiles);
    err[0] = bad | (total_tiles > max_tiles ? 2 : 0);
  }
  if (!tiles_m) return;   // uniform
  auto putm = [&](int g, int y, int z, int pos) {
    if (pos >= max_tiles) return;
    int4 tl;
    tl.x = g;
    tl.y = y;
    tl.z = z;
    tl.w = t.gk[g];
    reinterpret_cast<int4*>(tiles_m)[pos] = tl;
  };
  if (tid < G) {   // the group's merged tile and short tile (at most one of each), from its own thread
    if (mc.a) putm(tid, row0 + (nt - 2) * m_tile, row0 + rows, mpos.a);
    if (mc.c) putm(tid, row0 + (nt - 1) * m_tile, row0 + rows, mtot.a + mtot.b + mpos.c);
  }
  if (tid == 0) n_tiles_m[0] = min(mtot.a + mtot.b + mtot.c, max_tiles);   // never longer than tiles
}

// The tile list from the offsets off_s[0..E] (LDS). Called by every thread of one block (block scans inside).
SMEL_DEV void write_tiles(TileLds& tl, int tid, int E, int TK, int shared_rows, int m_tile, int max_tiles, int gkv,
                          const int* off_s, int bad, int* wsum, I3 (*wsum3)[1], int32_t* __restrict__ tiles,
                          int32_t* __restrict__ tiles_g, int32_t* __restrict__ n_tiles, int32_t* __restrict__ err,
                          int merge_rows, bool has_gk, int32_t* __restrict__ tiles_m, int32_t* __restrict__ n_tiles_m) {
  const int G = E + (shared_rows > 0 ? 1 : 0);
  int nt = 0, rows = 0, row0 = 0, nlong = 0;
  if (tid < G) {
    rows = tid < E ? off_s[tid + 1] - off_s[tid] : shared_rows;
    row0 = tid < E ? off_s[tid] : TK;
    nt = tiles_of(rows, m_tile);
    nlong = long_tiles_of(rows, m_tile);
  }
  int n_long, n_short;
  const int lbase = block_exclusive_scan(nlong, wsum, n_long);
  const int sbase = block_exclusive_scan(nt - nlong, wsum, n_short);
  const I3 mc = merged_counts(rows, m_tile, tiles_m ? merge_rows : 0, has_gk && (gkv >> 16) == SMEL_KIND_INT4);
  I3 mv[1] = {mc}, mtot[1];
  block_exclusive_scan3<1>(mv, wsum3, mtot);
  store_tiles(tl, tid, G, rows, row0, nt, lbase, sbase, n_long, n_short, m_tile, max_tiles, gkv, bad, tiles, tiles_g,
              n_tiles, err, mc, mv[0], mtot[0], tiles_m, n_tiles_m);
}

// (1) hist[b][e] = slots of block b routed to expert e; bad[b] = 1 if block b holds an id outside [0, E)
__global__ __launch_bounds__(1024) void dispatch_hist(const void* __restrict__ ids, int is64, int TK, int E,
                                                      int32_t* __restrict__ hist, int32_t* __restrict__ bad) {
  __shared__ int h[MAXE];
  __shared__ int bad_s;
  const int tid = threadIdx.x, b = blockIdx.x;
  for (int e = tid; e < E; e += DB) h[e] = 0;
  if (tid == 0) bad_s = 0;
  lds_barrier();
  const int p = b * DB + tid;
  if (p < TK) {
    const int e = id_at(ids, is64, p);
    if (e >= 0 && e < E)
      atomicAdd(&h[e], 1);   // LDS counter: the total does not depend on the order
    else
      bad_s = 1;
  }
  lds_barrier();
  for (int e = tid; e < E; e += DB) hist[b * E + e] = h[e];
  if (tid == 0) bad[b] = bad_s;
}

// (2) one block: counts, offsets, hist -> base[b][e] (first output position of block b's slots of expert e), tiles
__global__ __launch_bounds__(1024) void dispatch_scan(int nb, int TK, int E, int shared_rows, int m_tile,
                                                      int max_tiles, const int32_t* __restrict__ gkind,
                                                      int32_t* __restrict__ hist,
                                                      const int32_t* __restrict__ bad, int32_t* __restrict__ counts,
                                                      int32_t* __restrict__ offsets, int32_t* __restrict__ tiles,
                                                      int32_t* __restrict__ tiles_g, int32_t* __restrict__ n_tiles,
                                                      int32_t* __restrict__ err, int merge_rows,
                                                      int32_t* __restrict__ tiles_m,
                                                      int32_t* __restrict__ n_tiles_m) {
  __shared__ int wsum[NW];
  __shared__ I3 wsum3[NW][1];
  __shared__ int off_s[MAXE + 1];
  __shared__ int bad_s;
  __shared__ int hs[HCH];
  __shared__ TileLds tl;
  const int tid = threadIdx.x;
  if (tid == 0) bad_s = 0;
  // the bad-id flags and the group kinds are needed only at the end: their loads go out with the first histogram
  // chunk's
  int badv = 0;
  for (int b = tid; b < nb; b += DB) badv |= bad[b];
  const int G = E + (shared_rows > 0 ? 1 : 0);   // groups: the experts, then the shared expert
  const int gkv = (gkind && tid < G) ? gkind[tid] : 0;
  // the histograms go through LDS in chunks of whole blocks, loaded by all threads at once (one memory latency per
  // chunk instead of one per block and expert column); with a single chunk the second pass reuses it
  const int ch = HCH / E;   // blocks per chunk
  const bool one = nb <= ch;
  int total = 0;
  for (int b0 = 0; b0 < nb; b0 += ch) {
    const int n = min(ch, nb - b0) * E;
    lds_barrier();
    for (int i = tid; i < n; i += DB) hs[i] = hist[b0 * E + i];
    lds_barrier();
    if (tid < E)
      for (int b = 0; b < n / E; ++b) total += hs[b * E + tid];
  }
  int total_rows;
  const int ex = block_exclusive_scan(tid < E ? total : 0, wsum, total_rows);
  if (tid < E) {
    off_s[tid] = ex;
    counts[tid] = total;
    offsets[tid] = ex;
  }
  int run = ex;
  for (int b0 = 0; b0 < nb; b0 += ch) {
    const int n = min(ch, nb - b0) * E;
    if (!one) {
      lds_barrier();
      for (int i = tid; i < n; i += DB) hs[i] = hist[b0 * E + i];
      lds_barrier();
    }
    if (tid < E)
      for (int b = 0; b < n / E; ++b) {
        const int c = hs[b * E + tid];
        hs[b * E + tid] = run;
        run += c;
      }
    lds_barrier();
    for (int i = tid; i < n; i += DB) hist[b0 * E + i] = hs[i];
  }
  if (tid == 0) {
    off_s[E] = total_rows;
    offsets[E] = total_rows;
  }
  if (badv) bad_s = 1;
  lds_barrier();
  write_tiles(tl, tid, E, TK, shared_rows, m_tile, max_tiles, gkv, off_s, bad_s, wsum, wsum3, tiles, tiles_g, n_tiles,
              err, merge_rows, gkind != nullptr, tiles_m, n_tiles_m);
}

// Stable scatter of block b's slots: order[pos] = p, inv[p] = pos (-1 for an id outside [0, E)); base(x) = the first
// output position of this block's slots of expert x. Every thread of the block calls it.
// e = the thread's slot id (loaded by the caller, -1 past TK).
template <typename Base>
SMEL_DEV void scatter_block(int e, int TK, int E, int b, Base base, int* cnt /* [NW * MAXE] LDS */,
                            int32_t* __restrict__ order, int32_t* __restrict__ inv) {
  const int tid = threadIdx.x, l = lane_id(), w = tid >> 6;
  for (int i = tid; i < NW * E; i += DB) cnt[i] = 0;
  lds_barrier();
  const int p = b * DB + tid;
  const bool ok = e >= 0 && e < E;
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  uint64_t m = __ballot(ok);
  for (int bit = 0; bit < nbits; ++bit) {
    const bool v = ok && ((e >> bit) & 1);
    const uint64_t bb = __ballot(v);
    m &= v ? bb : ~bb;
  }
  const uint64_t lt = (l == 0) ? 0ull : (~0ull >> (64 - l));
  const int rank = ok ? __popcll(m & lt) : 0;
  if (ok && (m >> l) == 1ull) cnt[w * E + e] = __popcll(m);   // the group's highest lane records its size
  lds_barrier();
  for (int x = tid; x < E; x += DB) {
    int run = base(x);
    for (int j = 0; j < NW; ++j) {
      const int c = cnt[j * E + x];
      cnt[j * E + x] = run;
      run += c;
    }
  }
  lds_barrier();
  if (ok) {
    const int pos = cnt[w * E + e] + rank;
    order[pos] = p;
    inv[p] = pos;
  } else if (p < TK) {
    inv[p] = -1;
  }
}

// (3) the scatter after dispatch_scan: base[b][e] comes from the scan
__global__ __launch_bounds__(1024) void dispatch_scatter(const void* __restrict__ ids, int is64, int TK, int E,
                                                         const int32_t* __restrict__ base,
                                                         int32_t* __restrict__ order, int32_t* __restrict__ inv) {
  __shared__ int cnt[NW * MAXE];   // per-wave counts, then per-wave first positions
  const int b = blockIdx.x, p = b * DB + threadIdx.x;
  const int e = p < TK ? id_at(ids, is64, p) : -1;
  scatter_block(e, TK, E, b, [&](int x) { return base[b * E + x]; }, cnt, order, inv);
}

// (2+3) for at most SCAN_FUSE_NB blocks, the scan and the scatter in one launch: every block folds all blocks'
// histograms itself (the totals, and the prefix over the blocks before it, per expert) and scatters its slots; block
// 0 also writes counts, offsets, the tile lists, n_tiles and err. No block waits for another. Order of the work: every
// load first (the slot id, the histograms), the ranking of the block's slots, one scan of (offsets, long tiles, short
// tiles), then only stores and LDS traffic (so no wait on a load queued behind a store).
constexpr int SCAN_FUSE_NB = 64;
__global__ __launch_bounds__(1024) void dispatch_scan_scatter(const void* __restrict__ ids, int is64, int nb, int TK,
                                                              int E, int shared_rows, int m_tile, int max_tiles,
                                                              const int32_t* __restrict__ gkind,
                                                              const int32_t* __restrict__ hist,
                                                              const int32_t* __restrict__ bad,
                                                              int32_t* __restrict__ counts,
                                                              int32_t* __restrict__ offsets,
                                                              int32_t* __restrict__ tiles,
                                                              int32_t* __restrict__ tiles_g,
                                                              int32_t* __restrict__ n_tiles,
                                                              int32_t* __restrict__ err, int32_t* __restrict__ order,
                                                              int32_t* __restrict__ inv, int merge_rows,
                                                              int32_t* __restrict__ tiles_m,
                                                              int32_t* __restrict__ n_tiles_m) {
  __shared__ int cnt[NW * MAXE];   // per-wave counts, then per-wave first positions
  __shared__ I3 wsum[NW][2];
  __shared__ int bad_s;
  __shared__ TileLds tl;
  const int tid = threadIdx.x, l = lane_id(), w = tid >> 6, b = blockIdx.x;
  const bool lead = b == 0;   // uniform
  const int G = E + (shared_rows > 0 ? 1 : 0);
  const int p = b * DB + tid;
  const int e = p < TK ? id_at(ids, is64, p) : -1;
  int badv = 0, gkv = 0;
  if (lead) {
    for (int bb = tid; bb < nb; bb += DB) badv |= bad[bb];
    gkv = (gkind && tid < G) ? gkind[tid] : 0;
  }
  int c[SCAN_FUSE_NB];
  if (tid < E) {
#pragma unroll
    for (int i = 0; i < SCAN_FUSE_NB; ++i) {   // branch-free: rows past nb re-read the last one and count zero
      const int v = hist[min(i, nb - 1) * E + tid];
      c[i] = i < nb ? v : 0;
    }
  }
  for (int i = tid; i < NW * E; i += DB) cnt[i] = 0;
  if (tid == 0) bad_s = 0;
  lds_barrier();
  // rank of the slot among the block's slots of its expert: inside the wave by ballots over the id bits, the wave's
  // count per expert recorded by the group's highest lane
  const bool ok = e >= 0 && e < E;
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  uint64_t m = __ballot(ok);
  for (int bit = 0; bit < nbits; ++bit) {
    const bool v = ok && ((e >> bit) & 1);
    const uint64_t bb = __ballot(v);
    m &= v ? bb : ~bb;
  }
  const uint64_t lt = (l == 0) ? 0ull : (~0ull >> (64 - l));
  const int rank = ok ? __popcll(m & lt) : 0;
  if (ok && (m >> l) == 1ull) cnt[w * E + e] = __popcll(m);
  if (badv) bad_s = 1;
  // per expert: the total over all blocks, the prefix over blocks 0 .. b-1; per group: its tiles
  int total = 0, pre = 0;
  if (tid < E) {
#pragma unroll
    for (int i = 0; i < SCAN_FUSE_NB; ++i) {
      total += c[i];
      pre += i < b ? c[i] : 0;
    }
  }
  const int rows = tid < E ? total : (tid < G ? shared_rows : 0);
  const int nt = tiles_of(rows, m_tile), nlong = long_tiles_of(rows, m_tile);
  // (offsets, long tiles, short tiles) and, for the lead block's merged list, its three tile classes: one scan
  const I3 mc = merged_counts(rows, m_tile, lead && tiles_m ? merge_rows : 0, gkind && (gkv >> 16) == SMEL_KIND_INT4);
  I3 sv[2] = {I3{tid < E ? total : 0, nlong, nt - nlong}, mc}, stot[2];
  block_exclusive_scan3<2>(sv, wsum, stot);   // its barrier also completes cnt, bad_s
  const I3 ex = sv[0], tot = stot[0];
  if (lead) {
    if (tid < E) {
      counts[tid] = total;
      offsets[tid] = ex.a;
    }
    if (tid == 0) offsets[E] = tot.a;
    store_tiles(tl, tid, G, rows, tid < E ? ex.a : TK, nt, ex.b, ex.c, tot.b, tot.c, m_tile, max_tiles, gkv, bad_s,
                tiles, tiles_g, n_tiles, err, mc, sv[1], stot[1], tiles_m, n_tiles_m);
  }
  // first output position of wave j's slots of expert tid
  if (tid < E) {
    int run = ex.a + pre;
    for (int j = 0; j < NW; ++j) {
      const int cj = cnt[j * E + tid];
      cnt[j * E + tid] = run;
      run += cj;
    }
  }
  lds_barrier();
  if (ok) {
    const int pos = cnt[w * E + e] + rank;
    order[pos] = p;
    inv[p] = pos;
  } else if (p < TK) {
    inv[p] = -1;
  }
}

}  // namespace

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch[MAX_DEVICES] = {};

// Device address of the current device's `scratch` array, looked up on the first call on that device (with it
// current) and kept; nullptr with the error message set if the lookup fails.
int32_t* scratch_on_device() {
  int dev = -1;
  const hipError_t e0 = hipGetDevice(&dev);
  if (e0 != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
    smel::set_error("dispatch_noalloc: no usable current device (%s)", hipGetErrorString(e0));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      smel::set_error("dispatch_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                      hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev] = static_cast<int32_t*>(p);
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" int64_t smel_dispatch_max_tiles(int64_t TK, int64_t E, int64_t shared_rows, int32_t m_tile) {
  if (m_tile <= 0) return 0;
  return (TK + m_tile - 1) / m_tile + E + (shared_rows + m_tile - 1) / m_tile + 1;
}

extern "C" int64_t smel_dispatch_ws_size(int64_t TK, int64_t E) {
  if (TK < 0 || E <= 0) return -1;
  const int64_t nb = (TK + DB - 1) / DB;
  return nb * E + nb;
}

namespace {
int dispatch_impl(const void* ids, int32_t ids_are_i64, int64_t T, int64_t K, int64_t E, int64_t shared_rows,
                  int32_t m_tile, const int32_t* gkind, int32_t* counts, int32_t* offsets, int32_t* order, int32_t* inv,
                  int32_t* tiles, int32_t* tiles_grouped, int32_t* n_tiles, int32_t* err, int32_t merge_rows,
                  int32_t* tiles_merged, int32_t* n_tiles_merged, int32_t* ws, bool counted, hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && K > 0 && E > 0 && shared_rows >= 0 && m_tile > 0, SMEL_EINVAL, "dispatch: bad sizes");
  SMEL_REQUIRE(merge_rows == 0 || (merge_rows > m_tile && 2 * merge_rows <= 3 * m_tile && tiles_merged &&
                                   n_tiles_merged && gkind),
               SMEL_EINVAL,
               "dispatch: a merged tile list needs m_tile < merge_rows <= 1.5 m_tile (got %d, m_tile %d), its outputs "
               "and the group kinds", merge_rows, m_tile);
  if (merge_rows == 0) tiles_merged = n_tiles_merged = nullptr;
  SMEL_REQUIRE(E <= MAXE, SMEL_EUNSUPPORTED, "dispatch: E=%lld > %d experts", (long long)E, MAXE);
  SMEL_REQUIRE(T * K < (1ll << 30), SMEL_EUNSUPPORTED, "dispatch: T*K too large");
  SMEL_REQUIRE(counts && offsets && tiles && n_tiles && err && (T == 0 || (ids && order && inv && ws)), SMEL_EINVAL,
               "dispatch: null pointer");
  const int64_t TK = T * K;
  const int64_t mt = smel_dispatch_max_tiles(TK, E, shared_rows, m_tile);
  const int nb = (int)((TK + DB - 1) / DB);
  int32_t* hist = ws;
  int32_t* bad = ws ? ws + (int64_t)nb * E : nullptr;
  if (nb > 0 && !counted) {
    dispatch_hist<<<nb, DB, 0, stream>>>(ids, ids_are_i64 ? 1 : 0, (int)TK, (int)E, hist, bad);
    const int st = smel::launch_status();
    if (st) return st;
  }
  if (nb > 0 && nb <= SCAN_FUSE_NB) {
    dispatch_scan_scatter<<<nb, DB, 0, stream>>>(ids, ids_are_i64 ? 1 : 0, nb, (int)TK, (int)E, (int)shared_rows,
                                                 m_tile, (int)mt, gkind, hist, bad, counts, offsets, tiles,
                                                 tiles_grouped, n_tiles, err, order, inv, merge_rows, tiles_merged,
                                                 n_tiles_merged);
    return smel::launch_status();
  }
  dispatch_scan<<<1, DB, 0, stream>>>(nb, (int)TK, (int)E, (int)shared_rows, m_tile, (int)mt, gkind, hist, bad,
                                      counts, offsets, tiles, tiles_grouped, n_tiles, err, merge_rows, tiles_merged,
                                      n_tiles_merged);
  if (nb > 0) {
    const int st = smel::launch_status();
    if (st) return st;
    dispatch_scatter<<<nb, DB, 0, stream>>>(ids, ids_are_i64 ? 1 : 0, (int)TK, (int)E, hist, order, inv);
  }
  return smel::launch_status();
}
}  // namespace

extern "C" int smel_dispatch(const void* ids, int32_t ids_are_i64, int64_t T, int64_t K, int64_t E,
                             int64_t shared_rows, int32_t m_tile, const int32_t* gkind, int32_t* counts,
                             int32_t* offsets, int32_t* order, int32_t* inv, int32_t* tiles, int32_t* tiles_grouped,
                             int32_t* n_tiles, int32_t* err, int32_t merge_rows, int32_t* tiles_merged,
                             int32_t* n_tiles_merged, int32_t* ws, hipStream_t stream) {
  return dispatch_impl(ids, ids_are_i64, T, K, E, shared_rows, m_tile, gkind, counts, offsets, order, inv, tiles,
                       tiles_grouped, n_tiles, err, merge_rows, tiles_merged, n_tiles_merged, ws, false, stream);
}

extern "C" int smel_dispatch_counted(const void* ids, int32_t ids_are_i64, int64_t T, int64_t K, int64_t E,
                                     int64_t shared_rows, int32_t m_tile, const int32_t* gkind, int32_t* counts,
                                     int32_t* offsets, int32_t* order, int32_t* inv, int32_t* tiles,
                                     int32_t* tiles_grouped, int32_t* n_tiles, int32_t* err, int32_t merge_rows,
                                     int32_t* tiles_merged, int32_t* n_tiles_merged, int32_t* ws,
                                     hipStream_t stream) {
  return dispatch_impl(ids, ids_are_i64, T, K, E, shared_rows, m_tile, gkind, counts, offsets, order, inv, tiles,
                       tiles_grouped, n_tiles, err, merge_rows, tiles_merged, n_tiles_merged, ws, true, stream);
}

extern "C" int64_t smel_dispatch_noalloc_max_ws(void) { return SCRATCH_INTS; }

extern "C" int smel_dispatch_noalloc(const void* ids, int32_t ids_are_i64, int64_t T, int64_t K, int64_t E,
                                     int64_t shared_rows, int32_t m_tile, const int32_t* gkind, int32_t* counts,
                                     int32_t* offsets, int32_t* order, int32_t* inv, int32_t* tiles,
                                     int32_t* tiles_grouped, int32_t* n_tiles, int32_t* err, hipStream_t stream) {
  SMEL_REQUIRE(T >= 0 && K > 0 && E > 0 && T * K < (1ll << 30), SMEL_EINVAL, "dispatch_noalloc: bad sizes");
  const int64_t need = smel_dispatch_ws_size(T * K, E);
  SMEL_REQUIRE(need >= 0 && need <= SCRATCH_INTS, SMEL_EUNSUPPORTED,
               "dispatch_noalloc: T*K=%lld slots over E=%lld experts need %lld workspace ints, more than the %lld of "
               "the built-in scratch array (use smel_dispatch with a workspace)",
               (long long)(T * K), (long long)E, (long long)need, (long long)SCRATCH_INTS);
  int32_t* ws = scratch_on_device();
  if (!ws) return SMEL_EINVAL;
  return smel_dispatch(ids, ids_are_i64, T, K, E, shared_rows, m_tile, gkind, counts, offsets, order, inv, tiles,
                       tiles_grouped, n_tiles, err, 0, nullptr, nullptr, ws, stream);
}
