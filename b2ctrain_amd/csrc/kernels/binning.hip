// Binning and sorting (replaces src/gpu/binning.cu:10-143 and its CUB calls).
//
// * Radix sort: stable LSD key/value sort, 8-bit digits, reduce-then-scan (no inter-workgroup spin
//   waits). Per tile of 256 * KPT keys: an LDS digit histogram (upsweep), a per-digit exclusive scan over
//   tiles, then a stable scatter. In the scatter each wave owns a contiguous 64 * KPT stretch of the tile
//   and ranks it round by round in input order (ballot "match" masks for the lanes below with the same
//   digit, plus the wave's running per-digit count in LDS), so no block barrier sits inside the ranking
//   loop; keys and values are staged in LDS sorted by digit and written out in runs. Every thread loads
//   its KPT keys before it computes anything, so the loads of a tile are all in flight at once. KPT is 16
//   for large sorts and 4 for small ones (enough workgroups to cover the chip).
// * Count scan: reduce-then-scan of tile_count gathered in depth order, four contiguous entries a thread;
//   each workgroup of the second pass sums its predecessors' totals itself (no middle kernel).
// * Emit: small splats one thread each over the set bits of their hit mask; splats whose bbox exceeds 64
//   tiles one wave per chunk of the bbox, in row-major order.
#pragma clang fp contract(off)
#include "b2c_kernels.h"
#include "device_math.h"

#include <algorithm>

namespace b2c {
namespace dev {
namespace {

constexpr int SORT_THREADS = 256;
constexpr int KPT_BIG = 16;  // keys per thread of a large sort (4096-key tiles)
constexpr int KPT_SMALL = 8;  // below BIG_SORT_MIN keys (2048-key tiles)
constexpr uint32_t BIG_SORT_MIN = 1u << 22;
constexpr int KPT_HUGE = 32;  // from HUGE_SORT_MIN keys (8192-key tiles)
constexpr uint32_t HUGE_SORT_MIN = 1u << 25;
constexpr int RADIX = 256;
constexpr int NWAVES = SORT_THREADS / 64;
constexpr int SCAN_PER = 4;                         // count scan: contiguous entries per thread
constexpr int SCAN_TILE = SORT_THREADS * SCAN_PER;  // entries per workgroup

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// Lanes of this wave whose `bits`-bit digit equals mine (among lanes with `active` set).
__device__ __forceinline__ uint64_t match_digit(uint32_t d, int bits, bool active) {
  uint64_t m = ballot64(active);
  for (int b = 0; b < bits; b++) {
    const uint64_t bal = ballot64(((d >> b) & 1u) != 0u);
    m &= ((d >> b) & 1u) ? bal : ~bal;
  }
  return m;
}

// Inclusive scan within a wave64 (Hillis-Steele over shuffles).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    uint32_t t = __shfl_up(v, o);
    if (l >= o) v += t;
  }
  return v;
}

// Exclusive scan over a 256-thread block; returns the exclusive prefix, writes the block total.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* s_wsum, uint32_t& total) {
  const int w = threadIdx.x >> 6, l = lane_id();
  uint32_t inc = wave_incl_scan(v);
  if (l == 63) s_wsum[w] = inc;
  __syncthreads();
  uint32_t wbase = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < NWAVES; k++) {
    uint32_t s = s_wsum[k];
    if (k < w) wbase += s;
    tot += s;
  }
  __syncthreads();
  total = tot;
  return wbase + inc - v;
}

__device__ __forceinline__ uint32_t live_count(uint32_t cap, const uint32_t* n_dev) {
  if (!n_dev) return cap;
  uint32_t n = *n_dev;
  return n < cap ? n : cap;
}

// Tile of keys this workgroup sorts. Workgroup w runs on XCD w mod 8, so XCD x takes the contiguous tiles
// [x per, (x + 1) per), per = ceil(nblocks / 8): a histogram row holds one entry per tile, and the entries of
// neighbouring tiles, which share a cache line, are then written and read within one XCD's L2 instead of
// as partial lines from eight. The grid has 8 per workgroups; those mapped past nblocks return.
__device__ __forceinline__ uint32_t sort_tile(uint32_t nblocks) {
  const uint32_t per = (nblocks + 7u) / 8u;
  return (blockIdx.x & 7u) * per + (blockIdx.x >> 3);
}

// Per-tile digit histogram (R = 256 or 512 digits). Thread t loads the KPT consecutive keys [t KPT, t KPT +
// KPT) of the tile (16-byte loads) and counts runs of one digit in registers, adding each run to the LDS
// histogram with one atomic: tile keys in emit order come in runs (a splat's tiles along a bbox row), which
// would otherwise serialise on the same LDS word.
template <int KPT, int R>
__global__ void __launch_bounds__(SORT_THREADS) radix_upsweep(const uint32_t* __restrict__ keys, uint32_t cap,
                                                              const uint32_t* __restrict__ n_dev, int shift, int bits,
                                                              uint32_t* __restrict__ block_hist, uint32_t nblocks) {
  static_assert(KPT % 4 == 0, "keys are loaded four at a time");
  constexpr uint32_t TILE = SORT_THREADS * KPT;
  __shared__ uint32_t hist[R];
  const uint32_t tile = sort_tile(nblocks);
  if (tile >= nblocks) return;
  const uint32_t n = live_count(cap, n_dev);
  for (int t = threadIdx.x; t < R; t += SORT_THREADS) hist[t] = 0;
  __syncthreads();
  const uint32_t base = tile * TILE;
  if (base < n) {  // a tile past the live count (n_dev) reports zeros
    const uint32_t dmask = (1u << bits) - 1u;
    const uint32_t first = base + threadIdx.x * (uint32_t)KPT;
    uint32_t key[KPT];
    if (first + KPT <= n) {
#pragma unroll
      for (int q = 0; q < KPT / 4; q++) {
        const uint4 v = reinterpret_cast<const uint4*>(keys + first)[q];
        key[4 * q] = v.x; key[4 * q + 1] = v.y; key[4 * q + 2] = v.z; key[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int r = 0; r < KPT; r++) key[r] = first + r < n ? keys[first + r] : 0u;
    }
    uint32_t run_d = (key[0] >> shift) & dmask, run_c = first < n ? 1u : 0u;
#pragma unroll
    for (int r = 1; r < KPT; r++) {
      const uint32_t d = (key[r] >> shift) & dmask;
      const uint32_t live = first + r < n ? 1u : 0u;
      if (d == run_d) {
        run_c += live;
      } else {
        if (run_c) atomicAdd(&hist[run_d], run_c);
        run_d = d;
        run_c = live;
      }
    }
    if (run_c) atomicAdd(&hist[run_d], run_c);
  }
  __syncthreads();
  for (int t = threadIdx.x; t < R; t += SORT_THREADS) block_hist[(size_t)t * nblocks + tile] = hist[t];
}

// One workgroup per digit: exclusive scan of the digit's per-tile counts (each thread a contiguous run of
// tiles), total into digit_total. Runs of up to SCAN_KEEP tiles (sorts of up to 2048 tiles: 8M keys at
// 4096-key tiles) are read once and kept in registers; longer ones are read twice.
constexpr uint32_t SCAN_KEEP = 8;
__global__ void __launch_bounds__(SORT_THREADS) radix_scan_digits(uint32_t* __restrict__ block_hist, uint32_t nblocks,
                                                                  uint32_t* __restrict__ digit_total) {
  __shared__ uint32_t s_wsum[NWAVES];
  uint32_t* row = block_hist + (size_t)blockIdx.x * nblocks;
  const uint32_t per = (nblocks + SORT_THREADS - 1) / SORT_THREADS;
  const uint32_t lo = min(nblocks, threadIdx.x * per), hi = min(nblocks, lo + per);
  uint32_t tot;
  if (per <= SCAN_KEEP) {  // uniform: the run stays in registers (one memory round trip)
    uint32_t v[SCAN_KEEP];
    uint32_t sum = 0;
#pragma unroll
    for (uint32_t k = 0; k < SCAN_KEEP; k++) {
      v[k] = lo + k < hi ? row[lo + k] : 0u;
      sum += v[k];
    }
    uint32_t run = block_excl_scan(sum, s_wsum, tot);
#pragma unroll
    for (uint32_t k = 0; k < SCAN_KEEP; k++) {
      if (lo + k < hi) row[lo + k] = run;
      run += v[k];
    }
  } else {
    uint32_t sum = 0;
    for (uint32_t j = lo; j < hi; j++) sum += row[j];
    uint32_t run = block_excl_scan(sum, s_wsum, tot);
    for (uint32_t j = lo; j < hi; j++) {
      const uint32_t v = row[j];
      row[j] = run;
      run += v;
    }
  }
  if (threadIdx.x == 0) digit_total[blockIdx.x] = tot;
}

// Stable scatter of one digit pass over tiles of 256 * KPT keys. Wave w owns keys [w * 64 KPT, (w + 1) *
// 64 KPT) of the tile and ranks them in input order (ballot match masks within a round, the wave's running
// per-digit counts in LDS across rounds); per-wave offsets then give each key its position in an LDS
// staging buffer sorted by digit, which is written out in order: each digit's keys of this tile form one
// contiguous run in the output, so consecutive lanes write consecutive addresses. NV = 1 or 2 value arrays
// ride along with the keys. R = 256 or 512 digits (8- or 9-bit passes); thread t owns digits t R/256 ...
template <int NV, int KPT, int R>
__global__ void __launch_bounds__(SORT_THREADS) radix_scatter(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, const uint32_t* __restrict__ vals2_in,
    uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out, uint32_t* __restrict__ vals2_out, uint32_t cap,
    const uint32_t* __restrict__ n_dev, int shift, int bits, const uint32_t* __restrict__ block_hist, uint32_t nblocks,
    const uint32_t* __restrict__ digit_total) {
  constexpr uint32_t TILE = SORT_THREADS * KPT, CHUNK = 64 * KPT;
  __shared__ uint32_t s_key[TILE];
  __shared__ uint32_t s_val[TILE];  // one value array staged at a time (with NV = 2 the second follows the first)
  constexpr int DPT = R / SORT_THREADS;  // digits per thread
  // global position of the tile's first key of each digit minus its local (staging) offset: staging slot j
  // of digit d goes to s_gdelta[d] + j
  __shared__ uint32_t s_gdelta[R];
  __shared__ uint32_t s_wcnt[NWAVES][R];
  __shared__ uint32_t s_wsum[NWAVES];
  const uint32_t tile = sort_tile(nblocks);
  if (tile >= nblocks) return;
  const uint32_t n = live_count(cap, n_dev);
  const uint32_t base = tile * TILE;
  if (base >= n) return;
  const uint32_t tile_n = min(TILE, n - base);
  const int w = threadIdx.x >> 6, lane = lane_id();
  const uint32_t dmask = (1u << bits) - 1u;
  // 1. all loads of this thread in flight at once
  uint32_t key[KPT], val[NV][KPT];
#pragma unroll
  for (int r = 0; r < KPT; r++) {
    const uint32_t li = w * CHUNK + (uint32_t)r * 64 + lane;
    const bool valid = li < tile_n;
    key[r] = valid ? keys_in[base + li] : 0u;
    val[0][r] = valid ? (vals_in ? vals_in[base + li] : base + li) : 0u;  // no values: sort the positions
    if constexpr (NV > 1) val[1][r] = valid ? vals2_in[base + li] : 0u;
  }
  uint32_t loff_d[DPT];  // local (staging) offset of each of this thread's digits
  {  // 2. thread t owns digits t DPT .. t DPT + DPT - 1: global base and local offset of each in this tile
    uint32_t tot_d[DPT], mine[DPT], cnt[DPT], tot_sum = 0, cnt_sum = 0;
#pragma unroll
    for (int j = 0; j < DPT; j++) {
      const uint32_t d = threadIdx.x * DPT + j;
      tot_d[j] = digit_total[d];
      mine[j] = block_hist[(size_t)d * nblocks + tile];
      const uint32_t next = tile + 1 < nblocks ? block_hist[(size_t)d * nblocks + tile + 1] : tot_d[j];
      cnt[j] = next - mine[j];
      tot_sum += tot_d[j];
      cnt_sum += cnt[j];
    }
    uint32_t tot;
    uint32_t digit_start = block_excl_scan(tot_sum, s_wsum, tot);
    uint32_t loff = block_excl_scan(cnt_sum, s_wsum, tot);
#pragma unroll
    for (int j = 0; j < DPT; j++) {
      const uint32_t d = threadIdx.x * DPT + j;
      s_gdelta[d] = digit_start + mine[j] - loff;
      loff_d[j] = loff;
      digit_start += tot_d[j];
      loff += cnt[j];
#pragma unroll
      for (int k = 0; k < NWAVES; k++) s_wcnt[k][d] = 0u;
    }
  }
  __syncthreads();
  // 3. rank within the wave: rank = keys of the same digit earlier in this wave's stretch. All lanes read
  //    the running count before the round's leaders advance it (LDS instructions of a wave run in order).
  uint32_t rank[KPT];
  uint32_t* wc = s_wcnt[w];
#pragma unroll
  for (int r = 0; r < KPT; r++) {
    const bool valid = w * CHUNK + (uint32_t)r * 64 + lane < tile_n;
    const uint32_t d = (key[r] >> shift) & dmask;
    const uint64_t peers = match_digit(d, bits, valid);
    const uint32_t lt = popc64(peers & lanemask_lt());
    const uint32_t before = wc[d];
    if (valid && lt == 0) wc[d] = before + popc64(peers);
    rank[r] = before + lt;
  }
  __syncthreads();
  // 4. per-wave counts become staging offsets
#pragma unroll
  for (int j = 0; j < DPT; j++) {
    const uint32_t d = threadIdx.x * DPT + j;
    uint32_t run = loff_d[j];
#pragma unroll
    for (int k = 0; k < NWAVES; k++) {
      const uint32_t c = s_wcnt[k][d];
      s_wcnt[k][d] = run;
      run += c;
    }
  }
  __syncthreads();
  // 5. stage sorted by digit: the keys and the first value array (the staging offsets go to rank[])
#pragma unroll
  for (int r = 0; r < KPT; r++) {
    if (w * CHUNK + (uint32_t)r * 64 + lane < tile_n) {
      const uint32_t lp = wc[(key[r] >> shift) & dmask] + rank[r];
      rank[r] = lp;
      s_key[lp] = key[r];
      s_val[lp] = val[0][r];
    }
  }
  __syncthreads();
  // 6. write out in digit runs
  for (uint32_t j = threadIdx.x; j < tile_n; j += SORT_THREADS) {
    const uint32_t k = s_key[j];
    const uint32_t g = s_gdelta[(k >> shift) & dmask] + j;
    keys_out[g] = k;
    vals_out[g] = s_val[j];
  }
  if constexpr (NV > 1) {  // 7. the second value array through the same staging buffer
    __syncthreads();
#pragma unroll
    for (int r = 0; r < KPT; r++)
      if (w * CHUNK + (uint32_t)r * 64 + lane < tile_n) s_val[rank[r]] = val[1][r];
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < tile_n; j += SORT_THREADS) {
      vals2_out[s_gdelta[(s_key[j] >> shift) & dmask] + j] = s_val[j];
    }
  }
}

__global__ void __launch_bounds__(256) depth_keys_kernel(int n, const uint32_t* __restrict__ tile_count,
                                                         const uint32_t* depth_bits, uint32_t* keys,
                                                         uint32_t* __restrict__ vals) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  keys[i] = tile_count[i] ? depth_bits[i] : 0xFFFFFFFFu;  // in place when keys is depth_bits
  vals[i] = (uint32_t)i;
}

// ---- count scan in depth order ----
// Thread t of workgroup b owns entries [b * SCAN_TILE + 4t, +4): the order gather and the count gathers
// are issued before any arithmetic.
__device__ __forceinline__ void gather_counts(int n, const uint32_t* __restrict__ order,
                                              const uint32_t* __restrict__ tile_count, uint32_t first, uint32_t* c) {
  uint32_t o[SCAN_PER];
#pragma unroll
  for (int k = 0; k < SCAN_PER; k++) o[k] = first + k < (uint32_t)n ? order[first + k] : 0xFFFFFFFFu;
#pragma unroll
  for (int k = 0; k < SCAN_PER; k++) c[k] = o[k] != 0xFFFFFFFFu ? tile_count[o[k]] : 0u;
}

__global__ void __launch_bounds__(SORT_THREADS) scan_reduce(int n, const uint32_t* __restrict__ order,
                                                            const uint32_t* __restrict__ tile_count,
                                                            uint32_t* __restrict__ block_sums) {
  __shared__ uint32_t s_wsum[NWAVES];
  uint32_t c[SCAN_PER];
  gather_counts(n, order, tile_count, blockIdx.x * (uint32_t)SCAN_TILE + threadIdx.x * SCAN_PER, c);
  uint32_t acc = 0;
#pragma unroll
  for (int k = 0; k < SCAN_PER; k++) acc += c[k];
  uint32_t tot;
  block_excl_scan(acc, s_wsum, tot);
  if (threadIdx.x == 0) block_sums[blockIdx.x] = tot;
}

// Each workgroup sums the totals of the workgroups before it (at most a few thousand, read from L2) as its
// offset, then scans its own entries; the last workgroup writes the grand total to total_dev.
__global__ void __launch_bounds__(SORT_THREADS) scan_down(int n, const uint32_t* __restrict__ order,
                                                          const uint32_t* __restrict__ tile_count,
                                                          const uint32_t* __restrict__ block_sums,
                                                          uint32_t* __restrict__ tile_off,
                                                          uint32_t* __restrict__ total_dev, uint32_t* total_host) {
  __shared__ uint32_t s_wsum[NWAVES];
  const uint32_t first = blockIdx.x * (uint32_t)SCAN_TILE + threadIdx.x * SCAN_PER;
  uint32_t c[SCAN_PER];
  gather_counts(n, order, tile_count, first, c);
  uint32_t before = 0;
  for (uint32_t j = threadIdx.x; j < blockIdx.x; j += SORT_THREADS) before += block_sums[j];
  uint32_t offset;
  block_excl_scan(before, s_wsum, offset);
  uint32_t acc = 0;
#pragma unroll
  for (int k = 0; k < SCAN_PER; k++) acc += c[k];
  uint32_t tot;
  uint32_t run = offset + block_excl_scan(acc, s_wsum, tot);
#pragma unroll
  for (int k = 0; k < SCAN_PER; k++) {
    run += c[k];
    if (first + k < (uint32_t)n) tile_off[first + k] = run;
  }
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) {
    *total_dev = offset + tot;
    // straight into the caller's pinned host word (a system-scope vector store), instead of a copy launch
    if (total_host) __hip_atomic_store(total_host, offset + tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// Position of the k-th set bit (k counted from 0) of m, by halving: five popcounts.
__device__ __forceinline__ uint32_t select_bit(uint32_t m, uint32_t k) {
  uint32_t pos = 0;
#pragma unroll
  for (int half = 16; half >= 1; half >>= 1) {
    const uint32_t low = (uint32_t)__builtin_popcount(m & ((1u << half) - 1u));
    const bool up = k >= low;
    k = up ? k - low : k;
    m = up ? m >> half : m;
    pos = up ? pos + half : pos;
  }
  return pos;
}

// Position of the k-th set bit (k < popcount) of the 64-bit mask (hi, lo).
__device__ __forceinline__ uint32_t select_bit64(uint32_t lo, uint32_t hi, uint32_t k) {
  const uint32_t pl = (uint32_t)__builtin_popcount(lo);
  const bool up = k >= pl;
  return select_bit(up ? hi : lo, up ? k - pl : k) + (up ? 32u : 0u);
}

// Small splats: each wave takes 64 consecutive depth ranks, whose slot ranges [tile_off - count, tile_off)
// are adjacent (big splats' ranges, filled by emit_big_kernel, interleave). The wave's intersections are
// dealt to the lanes round-robin: intersection q belongs to the last rank whose running start is <= q (a
// binary search over the wave's 64 starts in LDS) and is the k-th set bit of that splat's hit mask
// (row-major bbox order; a bbox of up to 64 tiles: the mask of hit_info or of hit_wide). Every lane does
// the same work and consecutive lanes write consecutive slots. Big splats only record their base.
__global__ void __launch_bounds__(256) emit_small_kernel(b2c_emit_args a, uint32_t* __restrict__ big_base) {
  __shared__ uint32_t s_start[4][64], s_base[4][64], s_mask[4][64], s_mask_hi[4][64], s_info[4][64], s_id[4][64];
  const int w = threadIdx.x >> 6, lane = lane_id();
  const int r = blockIdx.x * 256 + threadIdx.x;
  uint32_t i = 0, cnt = 0, base = 0;
  uint2 hi = make_uint2(0u, 0u), wide = make_uint2(0u, 0u);
  bool big = false;
  if (r < a.n) {
    i = a.order[r];
    cnt = a.tile_count[i];
    if (cnt) {
      base = a.tile_off[r] - cnt;
      hi = reinterpret_cast<const uint2*>(a.hit_info)[i];
      if (hi.x == 0xFFFFFFFFu) {
        wide = reinterpret_cast<const uint2*>(a.hit_wide)[i];
        big = (wide.x | wide.y) == 0u;  // a splat with hits and no mask: over 64 bbox tiles
        if (big) big_base[i] = base;
      } else {
        wide = make_uint2(hi.x, 0u);
      }
    }
  }
  const uint32_t c = (cnt && !big && base + cnt <= a.cap) ? cnt : 0u;
  const uint32_t incl = wave_incl_scan(c);
  const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
  s_start[w][lane] = incl - c;
  s_base[w][lane] = base;
  s_mask[w][lane] = wide.x;
  s_mask_hi[w][lane] = wide.y;
  s_info[w][lane] = hi.y;
  s_id[w][lane] = i;
  __syncthreads();
  for (uint32_t q = (uint32_t)lane; q < total; q += 64u) {
    int j = 0;  // last lane with start <= q (the lanes after the owner start past q)
#pragma unroll
    for (int step = 32; step >= 1; step >>= 1)
      if (s_start[w][j + step] <= q) j += step;
    const uint32_t k = q - s_start[w][j];
    const uint32_t info = s_info[w][j];
    const uint32_t min_x = info & 0xFFFu, min_y = (info >> 12) & 0xFFFu, bw = info >> 24;
    const uint32_t bit = select_bit64(s_mask[w][j], s_mask_hi[w][j], k);
    const uint32_t row = bit / bw;
    const uint32_t slot = s_base[w][j] + k;
    a.keys[slot] = (min_y + row) * (uint32_t)a.tiles_x + min_x + (bit - row * bw);
    a.vals[slot] = s_id[w][j];
  }
}

// Big splats: one wave per (big-list entry, chunk), the chunk's tiles tested 64 at a time; hits go to
// the entry's slots at the chunk's offset (counted by b2c_hip_project with the same test, in the same
// order), so each chunk writes its own stretch independently.
__global__ void __launch_bounds__(256) emit_big_kernel(b2c_emit_args a, const uint32_t* __restrict__ big_base) {
  const int lane = lane_id();
  // wave-uniform (the compiler cannot see that threadIdx.x >> 6 is): the per-item chain uses scalar loads
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)((blockIdx.x * 256u + threadIdx.x) >> 6));
  const uint32_t nwaves = (gridDim.x * 256u) >> 6;
  const uint32_t items = *a.big_items_count;
  const uint32_t sentinel = (uint32_t)(a.tiles_x * a.tiles_y);
  for (uint32_t it = wave; it < items; it += nwaves) {
    // three dependent memory round trips: the item; the entry's bbox, splat and chunk offsets; the splat's
    // count, base and record. An entry past the capacity gets an empty range rather than a branch, so the
    // compiler cannot sink the last loads behind the capacity check (a fourth round trip).
    const uint32_t code = a.big_items[it];
    const uint32_t e = code >> 5, k = code & 31u;
    const uint4 info = reinterpret_cast<const uint4*>(a.big_info)[e];
    const uint32_t i = a.big_list[e];
    // the chunk's offset in the splat's slots: the hits of the chunks before it (lane j holds chunk j's)
    const uint32_t* chunk = a.big_chunk + (size_t)e * B2C_BIG_CHUNKS;
    const uint32_t own = chunk[k];
    uint32_t before = (uint32_t)lane < k ? chunk[lane] : 0u;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) before += __shfl_xor(before, o);  // every lane gets the sum
    const uint32_t off = before, off_next = before + own;
    const uint32_t cnt = a.tile_count[i];
    const uint32_t base = big_base[i];
    const SplatRecGeom g = splat_rec_geom(a.raster_rec, i);
    // the record is used here, so its loads share the third round trip (instead of being sunk into the
    // tile loop's guard)
    asm volatile("" : : "v"(g.mx), "v"(g.my), "v"(g.conic.c00), "v"(g.conic.c01), "v"(g.conic.c11), "v"(g.power));
    const bool fits = base + cnt <= a.cap;
    const uint32_t begin = k * info.w, end = fits ? min(begin + info.w, info.z) : begin;
    const uint32_t off_end = fits ? (end < info.z ? off_next : cnt) : off;
    const int min_x = (int)(info.x & 0xFFFFu), min_y = (int)(info.x >> 16), bw = (int)info.y;
    uint32_t written = off;
    for (uint32_t b0 = begin; b0 < end; b0 += 64) {
      const uint32_t b = b0 + (uint32_t)lane;
      bool h = false;
      int tx = 0, ty = 0;
      if (b < end) {
        tx = min_x + (int)(b % (uint32_t)bw);
        ty = min_y + (int)(b / (uint32_t)bw);
        const float rx = tx * (float)RT_W, ry = ty * (float)RT_W;
        h = tile_hit(rx, ry, rx + RT_W, ry + RT_W, g.mx, g.my, g.conic, g.power);
      }
      const uint64_t mk = ballot64(h);
      if (h) {
        const uint32_t slot = written + mbcnt64(mk);
        if (slot < off_end) {
          a.keys[base + slot] = (uint32_t)(ty * a.tiles_x + tx);
          a.vals[base + slot] = i;
        }
      }
      written += popc64(mk);
    }
    for (uint32_t s = written + lane; s < off_end; s += 64) {
      a.keys[base + s] = sentinel;
      a.vals[base + s] = i;
    }
  }
}

// Per-tile [first, last) of the sorted keys (binning.cu:95-105), every tile written: the thread at each key
// boundary writes the bounds of the runs on either side and clears the tiles with no key between them (the
// first and last threads those before the first key and after the last), so the ranges need no clearing
// beforehand; with no keys at all the grid clears every tile. tile_end keeps a copy of `last` that the
// forward does not shrink, and tile_end[n_tiles] = where the sentinel keys start (m if there are none).
// With slot_sorted set (an index sort: the sorted emit positions), also gathers the splat ids into list
// order: vals_sorted[i] = vals[slot_sorted[i]].
__device__ __forceinline__ void clear_tiles(uint2* ranges, uint32_t* tile_end, uint32_t lo, uint32_t hi) {
  for (uint32_t t = lo; t < hi; t++) {
    ranges[t] = make_uint2(0u, 0u);
    if (tile_end) tile_end[t] = 0u;
  }
}

constexpr uint32_t RANGE_KEYS = 4;

__global__ void __launch_bounds__(256) tile_ranges_kernel(uint32_t cap, const uint32_t* __restrict__ m_dev,
                                                          const uint32_t* __restrict__ keys,
                                                          const uint32_t* __restrict__ slot_sorted,
                                                          const uint32_t* __restrict__ vals,
                                                          uint32_t* __restrict__ vals_sorted, uint32_t n_tiles,
                                                          uint2* __restrict__ ranges, uint32_t* __restrict__ tile_end) {
  const uint32_t m = live_count(cap, m_dev);
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (m == 0) {
    for (uint32_t t = i; t < n_tiles; t += gridDim.x * 256u) {
      ranges[t] = make_uint2(0u, 0u);
      if (tile_end) tile_end[t] = 0u;
    }
    if (i == 0 && tile_end) tile_end[n_tiles] = 0u;
    return;
  }
  // RANGE_KEYS consecutive keys per thread (one 16-byte load where all are live), and the key before them
  const uint32_t i0 = i * RANGE_KEYS;
  if (i0 >= m) return;
  uint32_t k[RANGE_KEYS];
  if (i0 + RANGE_KEYS <= m) {
    const uint4 q = reinterpret_cast<const uint4*>(keys)[i];
    k[0] = q.x; k[1] = q.y; k[2] = q.z; k[3] = q.w;
  } else {
#pragma unroll
    for (uint32_t j = 0; j < RANGE_KEYS; j++) k[j] = i0 + j < m ? keys[i0 + j] : 0u;
  }
  uint32_t prev = i0 == 0 ? 0xFFFFFFFFu : keys[i0 - 1];
#pragma unroll
  for (uint32_t j = 0; j < RANGE_KEYS; j++) {
    const uint32_t ii = i0 + j;
    if (ii >= m) break;
    if (slot_sorted) vals_sorted[ii] = vals[slot_sorted[ii]];
    const uint32_t tile = k[j];
    if (ii == 0 || tile != prev) {
      // tiles after the previous run (or from 0) up to this run (or the end), which no key names
      clear_tiles(ranges, tile_end, ii == 0 ? 0u : min(prev + 1u, n_tiles), min(tile, n_tiles));
      if (tile < n_tiles) ranges[tile].x = ii;
      if (ii > 0 && prev < n_tiles) {
        ranges[prev].y = ii;
        if (tile_end) tile_end[prev] = ii;
      }
      // start of the run of sentinel keys (emit shortfall of big splats), which sorts last
      if (tile_end && tile >= n_tiles && (ii == 0 || prev < n_tiles)) tile_end[n_tiles] = ii;
    }
    if (ii == m - 1 && tile < n_tiles) {
      ranges[tile].y = m;
      clear_tiles(ranges, tile_end, tile + 1u, n_tiles);
      if (tile_end) {
        tile_end[tile] = m;
        tile_end[n_tiles] = m;  // no sentinel keys
      }
    }
    prev = tile;
  }
}

inline int sort_kpt(uint32_t n) { return n >= HUGE_SORT_MIN ? KPT_HUGE : n >= BIG_SORT_MIN ? KPT_BIG : KPT_SMALL; }
inline uint32_t sort_blocks(uint32_t n, int kpt) {
  const uint32_t tile = (uint32_t)(SORT_THREADS * kpt);
  return (n + tile - 1) / tile;
}
inline uint32_t scan_blocks(uint32_t n) { return (n + SCAN_TILE - 1) / SCAN_TILE; }

template <int KPT, int R>
void sort_pass(const uint32_t* src_k, const uint32_t* src_v, const uint32_t* src_v2, uint32_t* dk, uint32_t* dv,
               uint32_t* dv2, uint32_t n, const uint32_t* n_dev, int shift, int bits, uint32_t* block_hist,
               uint32_t* digit_total, hipStream_t stream) {
  const uint32_t nb = sort_blocks(n, KPT);
  const dim3 grid(8u * ((nb + 7u) / 8u));  // sort_tile's XCD-contiguous mapping
  radix_upsweep<KPT, R><<<grid, dim3(SORT_THREADS), 0, stream>>>(src_k, n, n_dev, shift, bits, block_hist, nb);
  radix_scan_digits<<<dim3(R), dim3(SORT_THREADS), 0, stream>>>(block_hist, nb, digit_total);
  if (src_v2)
    radix_scatter<2, KPT, R><<<grid, dim3(SORT_THREADS), 0, stream>>>(src_k, src_v, src_v2, dk, dv, dv2, n, n_dev,
                                                                       shift, bits, block_hist, nb, digit_total);
  else
    radix_scatter<1, KPT, R><<<grid, dim3(SORT_THREADS), 0, stream>>>(src_k, src_v, nullptr, dk, dv, nullptr, n,
                                                                       n_dev, shift, bits, block_hist, nb, digit_total);
}

}  // namespace
}  // namespace dev
}  // namespace b2c

using namespace b2c::dev;

extern "C" size_t b2c_radix_sort_temp_bytes(uint32_t n) {
  // the larger of the small-tile 8-bit and the large-tile 9-bit histograms, so the bound is monotone in n
  // whichever tile size and digit width a sort of n picks
  const size_t nb_small = sort_blocks(n > 0 ? n : 1, KPT_SMALL), nb_big = sort_blocks(n > 0 ? n : 1, KPT_BIG);
  const size_t hist = std::max(nb_small * RADIX, nb_big * 2 * RADIX);
  return (hist + 2 * RADIX) * sizeof(uint32_t);
}

extern "C" int b2c_hip_radix_sort_kv2(const uint32_t* keys_in, const uint32_t* vals_in, const uint32_t* vals2_in,
                                      uint32_t* keys_out, uint32_t* vals_out, uint32_t* vals2_out, uint32_t* keys_alt,
                                      uint32_t* vals_alt, uint32_t* vals2_alt, uint32_t n, const uint32_t* n_dev,
                                      int begin_bit, int end_bit, void* temp, size_t temp_bytes, hipStream_t stream) {
  if (n == 0 || end_bit <= begin_bit) return 0;
  if (temp_bytes < b2c_radix_sort_temp_bytes(n) || begin_bit < 0 || end_bit > 32) return (int)hipErrorInvalidValue;
  // the histogram pass reads the keys 16 bytes at a time
  if ((reinterpret_cast<uintptr_t>(keys_in) | reinterpret_cast<uintptr_t>(keys_out) | reinterpret_cast<uintptr_t>(keys_alt)) % 16u)
    return (int)hipErrorInvalidValue;
  const bool two = vals2_in != nullptr;
  if (two && (!vals2_out || !vals2_alt)) return (int)hipErrorInvalidValue;
  const int kpt = sort_kpt(n);
  uint32_t* block_hist = static_cast<uint32_t*>(temp);
  uint32_t* digit_total = block_hist + (size_t)sort_blocks(n, kpt) * (kpt != KPT_SMALL ? 2 * RADIX : RADIX);
  // 8-bit digits; a large sort whose key width is a few bits over a multiple of 8 (17-bit tile keys at 4K)
  // widens the first passes to 9 bits instead of running a pass for the remainder
  const int width = end_bit - begin_bit;
  int passes = (width + 7) / 8, wide = 0;
  if (kpt != KPT_SMALL && (width + 8) / 9 < passes) {
    passes = (width + 8) / 9;
    wide = width - 8 * passes;  // passes of 9 bits, the rest 8 (fewer where the width runs out)
  }
  const uint32_t* src_k = keys_in;
  const uint32_t* src_v = vals_in;
  const uint32_t* src_v2 = vals2_in;
  int shift = begin_bit;
  for (int p = 0; p < passes; p++) {
    // 8-bit passes split the width evenly (13 bits: 7 + 6, not 8 + 5): the first pass's digit runs per
    // tile are then twice as long, whole cache lines of keys instead of halves
    const int even = (end_bit - shift + (passes - p) - 1) / (passes - p);
    const int want = p < wide ? 9 : (even < 8 ? even : 8);
    const int bits = end_bit - shift < want ? end_bit - shift : want;
    // route the passes so that the last one lands in the output buffers
    const bool to_out = ((passes - 1 - p) % 2) == 0;
    uint32_t* dk = to_out ? keys_out : keys_alt;
    uint32_t* dv = to_out ? vals_out : vals_alt;
    uint32_t* dv2 = two ? (to_out ? vals2_out : vals2_alt) : nullptr;
    if (kpt == KPT_HUGE && bits > 8)
      sort_pass<KPT_HUGE, 2 * RADIX>(src_k, src_v, src_v2, dk, dv, dv2, n, n_dev, shift, bits, block_hist, digit_total,
                                     stream);
    else if (kpt == KPT_HUGE)
      sort_pass<KPT_HUGE, RADIX>(src_k, src_v, src_v2, dk, dv, dv2, n, n_dev, shift, bits, block_hist, digit_total,
                                 stream);
    else if (kpt == KPT_BIG && bits > 8)
      sort_pass<KPT_BIG, 2 * RADIX>(src_k, src_v, src_v2, dk, dv, dv2, n, n_dev, shift, bits, block_hist, digit_total,
                                    stream);
    else if (kpt == KPT_BIG)
      sort_pass<KPT_BIG, RADIX>(src_k, src_v, src_v2, dk, dv, dv2, n, n_dev, shift, bits, block_hist, digit_total,
                                stream);
    else
      sort_pass<KPT_SMALL, RADIX>(src_k, src_v, src_v2, dk, dv, dv2, n, n_dev, shift, bits, block_hist, digit_total,
                                  stream);
    int e = (int)hipGetLastError();
    if (e) return e;
    shift += bits;
    src_k = dk;
    src_v = dv;
    src_v2 = dv2;
  }
  return 0;
}

extern "C" int b2c_hip_radix_sort_pairs(const uint32_t* keys_in, const uint32_t* vals_in, uint32_t* keys_out,
                                        uint32_t* vals_out, uint32_t* keys_alt, uint32_t* vals_alt, uint32_t n,
                                        const uint32_t* n_dev, int begin_bit, int end_bit, void* temp, size_t temp_bytes,
                                        hipStream_t stream) {
  return b2c_hip_radix_sort_kv2(keys_in, vals_in, nullptr, keys_out, vals_out, nullptr, keys_alt, vals_alt, nullptr, n,
                                n_dev, begin_bit, end_bit, temp, temp_bytes, stream);
}

extern "C" int b2c_hip_depth_keys(int n, const uint32_t* tile_count, const uint32_t* depth_bits, uint32_t* keys, uint32_t* vals,
                                  hipStream_t stream) {
  if (n <= 0) return 0;
  depth_keys_kernel<<<dim3((n + 255) / 256), dim3(256), 0, stream>>>(n, tile_count, depth_bits,
                                                                      keys, vals);
  return (int)hipGetLastError();
}

extern "C" size_t b2c_scan_temp_bytes(uint32_t n) { return ((size_t)scan_blocks(n > 0 ? n : 1) + 1) * sizeof(uint32_t); }

extern "C" int b2c_hip_scan_counts_host(int n, const uint32_t* order, const uint32_t* tile_count, uint32_t* tile_off,
                                        uint32_t* total_dev, uint32_t* total_host, void* temp, size_t temp_bytes,
                                        hipStream_t stream) {
  if (n <= 0) {
    if (total_host) return (int)hipErrorInvalidValue;  // nothing would write it
    return b2c_hip_fill_u32(total_dev, 0u, 1, stream);
  }
  if (temp_bytes < b2c_scan_temp_bytes((uint32_t)n)) return (int)hipErrorInvalidValue;
  const uint32_t nb = scan_blocks((uint32_t)n);
  uint32_t* block_sums = static_cast<uint32_t*>(temp);
  scan_reduce<<<dim3(nb), dim3(SORT_THREADS), 0, stream>>>(n, order, tile_count, block_sums);
  scan_down<<<dim3(nb), dim3(SORT_THREADS), 0, stream>>>(n, order, tile_count, block_sums, tile_off, total_dev,
                                                          total_host);
  return (int)hipGetLastError();
}

extern "C" int b2c_hip_scan_counts(int n, const uint32_t* order, const uint32_t* tile_count, uint32_t* tile_off,
                                   uint32_t* total_dev, void* temp, size_t temp_bytes, hipStream_t stream) {
  return b2c_hip_scan_counts_host(n, order, tile_count, tile_off, total_dev, nullptr, temp, temp_bytes, stream);
}

extern "C" int b2c_hip_emit(const b2c_emit_args* a, hipStream_t stream) {
  if (a->n <= 0) return 0;
  if (!a->big_info || !a->big_chunk || !a->big_items || !a->big_items_count || !a->hit_wide)
    return (int)hipErrorInvalidValue;
  emit_small_kernel<<<dim3((a->n + 255) / 256), dim3(256), 0, stream>>>(*a, a->big_base);
  emit_big_kernel<<<dim3(B2C_BIG_GRID), dim3(256), 0, stream>>>(*a, a->big_base);
  return (int)hipGetLastError();
}

extern "C" int b2c_hip_tile_ranges(uint32_t m, const uint32_t* m_dev, const uint32_t* keys_sorted,
                                   const uint32_t* slot_sorted, const uint32_t* vals, uint32_t* vals_sorted,
                                   uint32_t n_tiles, uint32_t* ranges, uint32_t* tile_end, hipStream_t stream) {
  if (n_tiles == 0) return 0;
  if (slot_sorted && (!vals || !vals_sorted)) return (int)hipErrorInvalidValue;
  if (reinterpret_cast<uintptr_t>(keys_sorted) % 16u) return (int)hipErrorInvalidValue;  // read 16 bytes at a time
  // at least enough threads to clear every tile when there are no keys
  const uint32_t threads = max((m + RANGE_KEYS - 1u) / RANGE_KEYS, min(n_tiles, 65536u));
  tile_ranges_kernel<<<dim3((threads + 255) / 256), dim3(256), 0, stream>>>(m, m_dev, keys_sorted, slot_sorted, vals,
                                                                            vals_sorted, n_tiles,
                                                                            reinterpret_cast<uint2*>(ranges), tile_end);
  return (int)hipGetLastError();
}
