// Spatial-hash binning for gfx950: cell keys, a stable LSD radix sort (per
// pass: tile histograms, the first pass's counted with the keys, a per-digit
// scan over the tiles, a ballot-ranked scatter), bin_offsets from sorted run
// heads, the grid-mode block table, the
// permutation and its inverse, and the bin/unbin row moves.
//
// Replaces the reference's atomic counting sort (sphops/sph_cuda.cu:32-206,
// 1926-2056).  Results are deterministic: within a cell particles keep their
// input order, which is one of the orders the reference's atomic race can
// produce.  No dense per-cell counter array is touched: bin_offsets is
// written once per cell straight from the sorted keys.
#include "sphops_internal.hpp"

namespace sphops {

namespace {

constexpr int kThreads = 256;
constexpr int kItems = 16;
constexpr int kTile = kThreads * kItems;  // 4096 keys per radix / scan tile
constexpr int kRadixBits = 10;  // cell keys below 2^30 sort in 3 passes (cfg5's 2e8 cells: 28 bits)
constexpr int kBins = kRadixBins;
static_assert(kBins == 1 << kRadixBits, "kRadixBins must match kRadixBits");
constexpr int kChunkLog2 = 10;            // cells per bin_offsets workgroup
constexpr int kChunk = 1 << kChunkLog2;

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = __lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// ------------------------------------------------------------------ keys

// The sort moves one 64-bit word per particle: its cell key in the high half
// (the sort key) and its index in the low half (B*G and B*N are below 2^32).
__device__ __forceinline__ uint32_t kv_key(uint64_t v) { return (uint32_t)(v >> 32); }
__device__ __forceinline__ uint32_t kv_val(uint64_t v) { return (uint32_t)v; }

// The tile-counting kernels (keys, radix and class histograms) run one
// workgroup of kCountThreads per tile: a tile's loads in flight need more
// waves than one 256-thread workgroup per CU has.
constexpr int kCountThreads = 1024;
constexpr int kCountItems = kTile / kCountThreads;
static_assert(kCountItems * kCountThreads == kTile, "a counting workgroup covers one tile");

// Keys of the kTile particles of radix tile blockIdx.x, and the tile's counts
// of the first radix digit (the low kRadixBits of the key), laid out as
// k_radix_hist writes them: the sort's first pass then needs no pass of its
// own over the keys to count them.
template <int D, bool PERIODIC>
__global__ __launch_bounds__(kCountThreads) void k_cell_keys(GridParams g, const float* __restrict__ pos,
                                                           uint64_t* __restrict__ kv, uint32_t n,
                                                           uint32_t* __restrict__ hist, uint32_t ntiles) {
  __shared__ uint32_t h[kBins];
  for (int d = threadIdx.x; d < kBins; d += kCountThreads) h[d] = 0;
  __syncthreads();
  const uint32_t base = blockIdx.x * kTile;
#pragma unroll
  for (int i = 0; i < kCountItems; ++i) {
    const uint32_t k = base + i * kCountThreads + threadIdx.x;
    if (k < n) {
      float x[3];
      load_pos<D>(pos, k, x);
      int c[3];
      pos2cell<D, PERIODIC>(g, x, c);
      const uint32_t key = (k / g.N) * g.G + cell_hash<D>(g, c);
      kv[k] = ((uint64_t)key << 32) | k;
      atomicAdd(&h[key & (kBins - 1)], 1u);
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < kBins; d += kCountThreads) hist[d * ntiles + blockIdx.x] = h[d];
}

// ------------------------------------------------------- device-wide scan

// Exclusive scan of the 4096 values owned by one workgroup (16 consecutive
// values per thread).  Returns the workgroup total; `vals` are replaced by
// their exclusive prefix.  T: uint32_t, or uint64_t for two 32-bit counts
// scanned together (low and high halves; neither total reaches 2^32).
template <class T>
__device__ T block_exclusive_scan(T (&v)[kItems], T* sm /*[kThreads/64]*/) {
  T run = 0;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    T t = v[i];
    v[i] = run;
    run += t;
  }
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
  T incl = run;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    T y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63) sm[wave] = incl;
  __syncthreads();
  T wave_base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) {
    T s = sm[w];
    if (w < wave) wave_base += s;
    total += s;
  }
  __syncthreads();
  const T base = wave_base + incl - run;
#pragma unroll
  for (int i = 0; i < kItems; ++i) v[i] += base;
  return total;
}

template <class T>
__global__ __launch_bounds__(kThreads) void k_scan_reduce(const T* __restrict__ in, uint64_t n,
                                                          T* __restrict__ partials) {
  __shared__ T sm[kThreads / 64];
  const uint64_t base = (uint64_t)blockIdx.x * kTile + (uint64_t)threadIdx.x * kItems;
  T s = 0;
#pragma unroll
  for (int i = 0; i < kItems; ++i)
    if (base + i < n) s += in[base + i];
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
  if (lane == 0) sm[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    T t = 0;
    for (int w = 0; w < kThreads / 64; ++w) t += sm[w];
    partials[blockIdx.x] = t;
  }
}

// Scan one tile in place-or-out, adding partials[tile] (if given).  When
// `total_out` is non-null the grand total is stored there by the last tile.
template <class T>
__global__ __launch_bounds__(kThreads) void k_scan_apply(const T* in, T* out, uint64_t n,
                                                         const T* __restrict__ partials, T* total_out) {
  __shared__ T sm[kThreads / 64];
  const uint64_t base = (uint64_t)blockIdx.x * kTile + (uint64_t)threadIdx.x * kItems;
  T v[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) v[i] = (base + i < n) ? in[base + i] : T(0);
  const T tot = block_exclusive_scan<T>(v, sm);
  const T off = partials ? partials[blockIdx.x] : T(0);
#pragma unroll
  for (int i = 0; i < kItems; ++i)
    if (base + i < n) out[base + i] = v[i] + off;
  if (total_out && blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) *total_out = off + tot;
}

// Scan one tile with its offset computed in place: the sum of partials[0 ..
// tile), reduced by the workgroup (no separate scan of the partials).
template <class T>
__global__ __launch_bounds__(kThreads) void k_scan_apply_flat(const T* in, T* out, uint64_t n,
                                                              const T* __restrict__ partials, T* total_out) {
  __shared__ T sm[kThreads / 64];
  const uint32_t tile = blockIdx.x;
  T pre = 0;
  for (uint32_t i = threadIdx.x; i < tile; i += kThreads) pre += partials[i];
  const int lane = __lane_id(), wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) pre += __shfl_down(pre, off, 64);
  if (lane == 0) sm[wave] = pre;
  __syncthreads();
  T off = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) off += sm[w];
  __syncthreads();
  const uint64_t base = (uint64_t)tile * kTile + (uint64_t)threadIdx.x * kItems;
  T v[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) v[i] = (base + i < n) ? in[base + i] : T(0);
  const T tot = block_exclusive_scan<T>(v, sm);
#pragma unroll
  for (int i = 0; i < kItems; ++i)
    if (base + i < n) out[base + i] = v[i] + off;
  if (total_out && tile == gridDim.x - 1 && threadIdx.x == 0) *total_out = off + tot;
}

// Tile counts up to this take the two-launch scan (partial sums, then each
// tile reduces the partials before it); larger ones recurse.
constexpr uint64_t kFlatScanTiles = 8192;

}  // namespace

static_assert(kScanTile == (uint64_t)kTile, "scan_tmp_elems assumes the scan tile");

namespace {

// out[i] = sum_{j<i} in[j]; optionally *total = sum of all.  `tmp` holds
// scan_tmp_elems(n) words.  `in` may equal `out`.
void device_exclusive_scan(const uint32_t* in, uint32_t* out, uint64_t n, uint32_t* tmp, uint32_t* total,
                           hipStream_t st) {
  if (n == 0) return;
  const uint64_t tiles = (n + kTile - 1) / kTile;
  if (tiles == 1) {
    hipLaunchKernelGGL(k_scan_apply<uint32_t>, dim3(1), dim3(kThreads), 0, st, in, out, n, nullptr, total);
    SPHOPS_LAUNCHED();
    return;
  }
  uint32_t* partials = tmp;
  hipLaunchKernelGGL(k_scan_reduce<uint32_t>, dim3((uint32_t)tiles), dim3(kThreads), 0, st, in, n, partials);
  SPHOPS_LAUNCHED();
  if (tiles <= kFlatScanTiles) {
    hipLaunchKernelGGL(k_scan_apply_flat<uint32_t>, dim3((uint32_t)tiles), dim3(kThreads), 0, st, in, out, n,
                       partials, total);
    SPHOPS_LAUNCHED();
    return;
  }
  device_exclusive_scan(partials, partials, tiles, tmp + tiles + kTile, nullptr, st);
  hipLaunchKernelGGL(k_scan_apply<uint32_t>, dim3((uint32_t)tiles), dim3(kThreads), 0, st, in, out, n, partials,
                     total);
  SPHOPS_LAUNCHED();
}

// The same over 64-bit words, for at most kFlatScanTiles tiles: the partial
// sums take 2 * tiles words of `tmp` (dual_scan_fits checks both bounds).
bool dual_scan_fits(const Grid& g, uint64_t n) {
  const uint64_t tiles = (n + kTile - 1) / kTile;
  return tiles <= kFlatScanTiles && 2 * tiles <= g.scan_tmp_len;
}

void device_exclusive_scan64(const uint64_t* in, uint64_t* out, uint64_t n, uint32_t* tmp, uint64_t* total,
                             hipStream_t st) {
  if (n == 0) return;
  const uint64_t tiles = (n + kTile - 1) / kTile;
  if (tiles == 1) {
    hipLaunchKernelGGL(k_scan_apply<uint64_t>, dim3(1), dim3(kThreads), 0, st, in, out, n, nullptr, total);
    SPHOPS_LAUNCHED();
    return;
  }
  uint64_t* partials = reinterpret_cast<uint64_t*>(tmp);
  hipLaunchKernelGGL(k_scan_reduce<uint64_t>, dim3((uint32_t)tiles), dim3(kThreads), 0, st, in, n, partials);
  SPHOPS_LAUNCHED();
  hipLaunchKernelGGL(k_scan_apply_flat<uint64_t>, dim3((uint32_t)tiles), dim3(kThreads), 0, st, in, out, n,
                     partials, total);
  SPHOPS_LAUNCHED();
}

// ------------------------------------------------------------ radix sort

__global__ __launch_bounds__(kCountThreads) void k_radix_hist(const uint64_t* __restrict__ kv, uint32_t n,
                                                              int shift, uint32_t* __restrict__ hist,
                                                              uint32_t ntiles) {
  __shared__ uint32_t h[kBins];
  for (int d = threadIdx.x; d < kBins; d += kCountThreads) h[d] = 0;
  __syncthreads();
  const uint32_t base = blockIdx.x * kTile;
#pragma unroll
  for (int i = 0; i < kCountItems; ++i) {
    const uint32_t idx = base + i * kCountThreads + threadIdx.x;
    if (idx < n) atomicAdd(&h[(kv_key(kv[idx]) >> shift) & (kBins - 1)], 1u);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < kBins; d += kCountThreads) hist[d * ntiles + blockIdx.x] = h[d];
}

// Per digit d (a wave each, four digits a workgroup): the tile counts
// hist[d * ntiles + t] are replaced by their exclusive prefix over the tiles,
// and the digit's total goes to tot[d].  The scatter adds the totals of the
// smaller digits, which gives the exclusive prefix over digit-major order
// that a device-wide scan of the histograms would.
__global__ __launch_bounds__(kThreads) void k_radix_colscan(uint32_t* __restrict__ hist, uint32_t ntiles,
                                                            uint32_t* __restrict__ tot) {
  const uint32_t d = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (d >= (uint32_t)kBins) return;  // wave-uniform
  const uint32_t lane = __lane_id();
  uint32_t* __restrict__ h = hist + (uint64_t)d * ntiles;
  uint32_t carry = 0;
  for (uint32_t t0 = 0; t0 < ntiles; t0 += 4 * 64) {
    uint32_t v[4], sum = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t t = t0 + lane * 4 + u;
      v[u] = t < ntiles ? h[t] : 0u;
      sum += v[u];
    }
    uint32_t incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t y = __shfl_up(incl, off, 64);
      if ((int)lane >= off) incl += y;
    }
    uint32_t run = carry + incl - sum;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t t = t0 + lane * 4 + u;
      if (t < ntiles) h[t] = run;
      run += v[u];
    }
    carry += (uint32_t)__shfl(incl, 63, 64);
  }
  if (lane == 0) tot[d] = carry;
}

// Stable scatter of one radix digit.  Wave w of the tile owns keys
// [w*1024, (w+1)*1024) and walks them 64 at a time in index order; lanes with
// equal digits find each other with 8 ballots, so each key's rank among the
// equal-digit keys before it is exact and no atomics are involved.
__global__ __launch_bounds__(kThreads) void k_radix_scatter(const uint64_t* __restrict__ kin,
                                                            uint64_t* __restrict__ kout, uint32_t n, int shift,
                                                            const uint32_t* __restrict__ hist_scan,
                                                            const uint32_t* __restrict__ tot, uint32_t ntiles) {
  static_assert(kBins == 4 * kThreads, "four digits a thread in the digit prefix");
  __shared__ uint32_t wcnt[kThreads / 64][kBins];
  __shared__ uint32_t gbase[kBins];
  __shared__ uint32_t wsum[kThreads / 64];
  const int wave = threadIdx.x >> 6, lane = __lane_id();
  for (int i = threadIdx.x; i < (kThreads / 64) * kBins; i += kThreads) (&wcnt[0][0])[i] = 0;
  {
    // digit d's first slot: the totals of the digits below d (exclusive
    // prefix over the workgroup, four consecutive digits a thread) plus the
    // counts of d in the tiles before this one
    const int d0 = 4 * threadIdx.x;
    uint32_t v[4], sum = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v[u] = tot[d0 + u];
      sum += v[u];
    }
    uint32_t incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    uint32_t run = incl - sum;
    for (int w = 0; w < wave; ++w) run += wsum[w];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      gbase[d0 + u] = run + hist_scan[(uint64_t)(d0 + u) * ntiles + blockIdx.x];
      run += v[u];
    }
  }
  __syncthreads();

  const uint32_t base = blockIdx.x * kTile + wave * (kTile / (kThreads / 64));
  const uint64_t below_mask = lanemask_lt();
  uint64_t word[kItems];
  uint32_t rank[kItems];
#pragma unroll
  for (int t = 0; t < kItems; ++t) {
    const uint32_t idx = base + t * 64 + lane;
    const bool valid = idx < n;
    word[t] = valid ? kin[idx] : 0ull;
    const uint32_t digit = (kv_key(word[t]) >> shift) & (kBins - 1);
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
      const bool bit = (digit >> b) & 1u;
      const uint64_t bb = __ballot(bit);
      peers &= bit ? bb : ~bb;
    }
    const uint32_t before = (uint32_t)__popcll(peers & below_mask);
    const uint32_t prior = wcnt[wave][digit];
    if (valid && before == 0) wcnt[wave][digit] = prior + (uint32_t)__popcll(peers);
    rank[t] = prior + before;
  }
  __syncthreads();
  // exclusive prefix of the per-wave counts, digit by digit
  for (int d = threadIdx.x; d < kBins; d += kThreads) {
    uint32_t run = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
      const uint32_t c = wcnt[w][d];
      wcnt[w][d] = run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < kItems; ++t) {
    const uint32_t idx = base + t * 64 + lane;
    if (idx < n) {
      const uint32_t digit = (kv_key(word[t]) >> shift) & (kBins - 1);
      kout[gbase[digit] + wcnt[wave][digit] + rank[t]] = word[t];
    }
  }
}

// ------------------------------------------------------- bin_offsets

__global__ __launch_bounds__(kThreads) void k_fill_u32(uint32_t* __restrict__ p, uint64_t n, uint32_t v) {
  const uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) p[i] = v;
}

// chunk_lo[c] = number of sorted keys below the first cell of chunk c
// (c = 0 .. nch), by binary search over the sorted keys.
__global__ __launch_bounds__(kThreads) void k_chunk_lo(const uint64_t* __restrict__ kv, uint32_t n,
                                                       uint32_t* __restrict__ chunk_lo, uint32_t nch) {
  const uint32_t c = blockIdx.x * kThreads + threadIdx.x;
  if (c > nch) return;
  const uint64_t target = (uint64_t)c << kChunkLog2;
  uint32_t lo = 0, hi = n;
  while (lo < hi) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    if ((uint64_t)kv_key(kv[mid]) < target) lo = mid + 1;
    else hi = mid;
  }
  chunk_lo[c] = lo;
}

// bin_offsets[c] = number of sorted keys < c, for the 1024 cells of a chunk.
// Run heads inside the chunk mark their cell; empty cells take the next run
// head (suffix minimum), the chunk end being the sentinel.  A workgroup
// handles kChunksPerBlock consecutive chunks (most of them empty at large
// cell counts, where the kernel is a 16-byte-per-lane store stream).
constexpr int kChunksPerBlock = 4;

__device__ __forceinline__ void bin_offsets_block(const uint64_t* __restrict__ kv,
                                                  const uint32_t* __restrict__ chunk_lo, uint32_t nch,
                                                  int32_t* __restrict__ bo, uint64_t ncells_p1, uint32_t blk) {
  __shared__ uint32_t first[kChunk];
  __shared__ uint32_t wmin[kThreads / 64];
  const int t = threadIdx.x;
  for (int i = 0; i < kChunksPerBlock; ++i) {
    const uint32_t ch = blk * kChunksPerBlock + (uint32_t)i;
    if (ch >= nch) break;  // uniform over the workgroup
    const uint32_t lo = chunk_lo[ch], hi = chunk_lo[ch + 1];
    const uint64_t c0 = (uint64_t)ch << kChunkLog2;
    uint32_t s[4];
    if (lo == hi) {  // uniform over the workgroup
#pragma unroll
      for (int q = 0; q < 4; ++q) s[q] = lo;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) first[t * 4 + q] = hi;
      __syncthreads();
      for (uint32_t p = lo + t; p < hi; p += kThreads) {
        const uint32_t key = kv_key(kv[p]);
        if (p == lo || kv_key(kv[p - 1]) != key) first[key - (uint32_t)c0] = p;
      }
      __syncthreads();
#pragma unroll
      for (int q = 0; q < 4; ++q) s[q] = first[t * 4 + q];
      s[2] = min(s[2], s[3]);
      s[1] = min(s[1], s[2]);
      s[0] = min(s[0], s[1]);
      // exclusive suffix minimum over threads
      const int lane = __lane_id(), wave = t >> 6;
      uint32_t incl = s[0];
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_down(incl, off, 64);
        if (lane + off < 64) incl = min(incl, y);
      }
      if (lane == 0) wmin[wave] = incl;
      __syncthreads();
      uint32_t after = hi;
      for (int w = wave + 1; w < kThreads / 64; ++w) after = min(after, wmin[w]);
      uint32_t nxt = __shfl_down(incl, 1, 64);
      if (lane == 63) nxt = hi;
      after = min(after, nxt);
#pragma unroll
      for (int q = 0; q < 4; ++q) s[q] = min(s[q], after);
      __syncthreads();  // `first` and `wmin` are reused by the next chunk
    }
    const uint64_t c = c0 + (uint64_t)t * 4;
    if (c + 3 < ncells_p1) {
      // non-temporal: the table is far larger than the caches, and kept out
      // of them it leaves no dirty lines for the kernels after it to evict
      typedef int v4i __attribute__((ext_vector_type(4)));
      const v4i v = {(int)s[0], (int)s[1], (int)s[2], (int)s[3]};
      __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(bo + c));
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (c + q < ncells_p1) bo[c + q] = (int)s[q];
    }
  }
}

__global__ __launch_bounds__(kThreads) void k_bin_offsets(const uint64_t* __restrict__ kv,
                                                          const uint32_t* __restrict__ chunk_lo, uint32_t nch,
                                                          int32_t* __restrict__ bo, uint64_t ncells_p1) {
  bin_offsets_block(kv, chunk_lo, nch, bo, ncells_p1, blockIdx.x);
}

// First and one-past-last sorted position of the run of `key` (its cell)
// that contains position k, from the sorted keys alone: a galloping search
// away from k, then a binary search in the last step's window; about
// 2 log2(run length) loads, near k.
__device__ __forceinline__ uint32_t run_start(const uint64_t* __restrict__ kv, uint32_t k, uint32_t key) {
  uint32_t hi = k, lo = 0, step = 1;  // key(hi) == key; lo: a smaller key, once found
  bool found = false;
  while (step <= hi) {
    const uint32_t probe = hi - step;
    if (kv_key(kv[probe]) < key) {
      lo = probe;
      found = true;
      break;
    }
    hi = probe;
    step <<= 1;
  }
  if (!found) {
    if (kv_key(kv[0]) == key) return 0;
    lo = 0;  // key(0) < key
  }
  while (hi - lo > 1) {  // key(lo) < key == key(hi)
    const uint32_t mid = lo + ((hi - lo) >> 1);
    if (kv_key(kv[mid]) < key) lo = mid;
    else hi = mid;
  }
  return hi;
}

__device__ __forceinline__ uint32_t run_end(const uint64_t* __restrict__ kv, uint32_t n, uint32_t k,
                                            uint32_t key) {
  uint32_t lo = k, hi = n, step = 1;  // key(lo) == key; hi: a larger key, once found
  bool found = false;
  while (lo + step < n) {
    const uint32_t probe = lo + step;
    if (kv_key(kv[probe]) > key) {
      hi = probe;
      found = true;
      break;
    }
    lo = probe;
    step <<= 1;
  }
  if (!found) {
    if (kv_key(kv[n - 1]) == key) return n;
    hi = n - 1;  // key(n - 1) > key
  }
  while (hi - lo > 1) {  // key(lo) == key < key(hi)
    const uint32_t mid = lo + ((hi - lo) >> 1);
    if (kv_key(kv[mid]) > key) hi = mid;
    else lo = mid;
  }
  return hi;
}

// Cell count from which the permutation and block-row kernels find a cell's
// bounds in the sorted keys near k (run_start / run_end, which the previous
// kernels left in cache) instead of loading them from bin_offsets, whose
// entries are then scattered over a large array (2^22 cells = 16 MB, four
// times an XCD's L2): 0.339 -> 0.326 ms for instantiate at cfg5, while at
// cfg1 the dependent loads of the search cost 5 us more than the cached
// bin_offsets loads.
constexpr uint64_t kRunSearchMinCells = 1ull << 22;

// Permutation (destination slot of every input particle), in grid mode
// (BLOCKS) the block-start flags of the block table: sorted position k starts
// a block when its offset in its cell is a multiple of maxp; and with UNITS
// the work split of the neighbour-list fill, which depends on the cell runs
// alone: unit_len[k] = particles of the unit starting at k (a run of up to
// kUnitParticles particles of a cell with two or more, starting at a
// multiple of kUnitParticles in the cell), 0 for the other particles of such
// a cell, -1 for a particle alone in its cell; the unit-start flag is 1
// where unit_len > 0.  When both are made they go to flags64 as masks, per
// wave of 64 sorted positions w: flags64[2w] the block starts, flags64[2w + 1]
// the unit starts (bit l: position 64w + l), and flags64[2 nw + w] their
// counts (blocks in the low half, units in the high half; nw = the number of
// waves), which one scan of nw words turns into each wave's first block row
// and unit slot; else one flag per position to flags32.  The cell's first
// position comes from bin_offsets or, with bo null, from the sorted keys.
template <bool BLOCKS, bool UNITS>
__device__ __forceinline__ void permutation_block(const uint64_t* __restrict__ kv, uint32_t n, uint32_t N,
                                                  int32_t* __restrict__ perm, const int32_t* __restrict__ bo,
                                                  uint32_t maxp, uint32_t* __restrict__ flags32,
                                                  uint64_t* __restrict__ flags64, int32_t* __restrict__ unit_len,
                                                  int32_t* __restrict__ inv, uint32_t blk) {
  const uint32_t k = blk * kThreads + threadIdx.x;
  if (k >= n) return;
  const uint64_t w = kv[k];
  const uint32_t src = kv_val(w);
  const uint32_t cloud = (src / N) * N;
  perm[src] = (int32_t)(k - cloud);
  if (inv != nullptr) inv[k] = (int32_t)(src - cloud);
  if constexpr (BLOCKS || UNITS) {
    const uint32_t key = kv_key(w);
    const uint32_t rs = bo != nullptr ? (uint32_t)bo[key] : run_start(kv, k, key);
    const uint32_t bf = BLOCKS && (k - rs) % maxp == 0 ? 1u : 0u;
    uint32_t uf = 0;
    if constexpr (UNITS) {
      const bool alone = k == rs && (k + 1 == n || kv_key(kv[k + 1]) != key);
      int32_t ul = -1;
      if (!alone) {
        ul = 0;
        if ((k - rs) % (uint32_t)kUnitParticles == 0) {
          uint32_t len = 1;
          while (len < (uint32_t)kUnitParticles && k + len < n && kv_key(kv[k + len]) == key) ++len;
          ul = (int32_t)len;
          uf = 1;
        }
      }
      unit_len[k] = ul;
    }
    if constexpr (BLOCKS && UNITS) {
      // k runs over 64 consecutive positions a wave (kThreads is a multiple
      // of 64): its lane 0 holds the wave's first position, which is below n
      // whenever any lane of the wave is
      const uint64_t bm = __ballot(bf != 0u), um = __ballot(uf != 0u);
      if (__lane_id() == 0) {
        const uint32_t w = k >> 6, nw = (n + 63) >> 6;
        flags64[2 * (uint64_t)w] = bm;
        flags64[2 * (uint64_t)w + 1] = um;
        flags64[2 * (uint64_t)nw + w] = (uint64_t)__popcll(bm) | ((uint64_t)__popcll(um) << 32);
      }
    } else {
      flags32[k] = BLOCKS ? bf : uf;
    }
  }
}

template <bool BLOCKS, bool UNITS>
__global__ __launch_bounds__(kThreads) void k_permutation(const uint64_t* __restrict__ kv, uint32_t n,
                                                          uint32_t N, int32_t* __restrict__ perm,
                                                          const int32_t* __restrict__ bo, uint32_t maxp,
                                                          uint32_t* __restrict__ flags32,
                                                          uint64_t* __restrict__ flags64,
                                                          int32_t* __restrict__ unit_len,
                                                          int32_t* __restrict__ inv) {
  permutation_block<BLOCKS, UNITS>(kv, n, N, perm, bo, maxp, flags32, flags64, unit_len, inv, blockIdx.x);
}

// bin_offsets and the permutation in one launch, for grids whose permutation
// finds cell bounds in the sorted keys (it does not read bin_offsets): one
// permutation workgroup after every `every` chunk workgroups, so that the
// latency-bound permutation runs under the bin_offsets store stream instead
// of after it (the dispatcher starts workgroups in order; with all
// permutation workgroups first the two did not overlap).
template <bool BLOCKS, bool UNITS>
__global__ __launch_bounds__(kThreads) void k_offsets_permutation(
    const uint64_t* __restrict__ kv, const uint32_t* __restrict__ chunk_lo, uint32_t nch, int32_t* __restrict__ bo,
    uint64_t ncells_p1, uint32_t nb_bo, uint32_t n, uint32_t N, int32_t* __restrict__ perm, uint32_t maxp,
    uint32_t* __restrict__ flags32, uint64_t* __restrict__ flags64, int32_t* __restrict__ unit_len,
    int32_t* __restrict__ inv, uint32_t nb_perm, uint32_t every) {
  const uint32_t b = blockIdx.x, q = b / (every + 1), r = b % (every + 1);
  if (q < nb_perm) {
    if (r == every)
      permutation_block<BLOCKS, UNITS>(kv, n, N, perm, nullptr, maxp, flags32, flags64, unit_len, inv, q);
    else if (q * every + r < nb_bo) bin_offsets_block(kv, chunk_lo, nch, bo, ncells_p1, q * every + r);
  } else {
    const uint32_t c = nb_perm * every + (b - nb_perm * (every + 1));
    if (c < nb_bo) bin_offsets_block(kv, chunk_lo, nch, bo, ncells_p1, c);
  }
}

// Rows {global_cell, offset_in_cell, count, batch} (sphops/utils.cuh:295-301)
// of the blocks starting at sorted position i < n (row rowidx[i]; position i
// starts a block when rowidx[i + 1] > rowidx[i], the scan having counted its
// flag), zero rows r in [total, max_blocks) (thread i handles position i and
// row i), and the block count into total_out.  Cell bounds as in
// k_permutation.  With UNITS the flags are k_permutation's masks (`masks`,
// 2 nw words) and the scan its per-wave counts (`scan64`, nw + 1 words, the
// totals last; a position's row and slot are its wave's plus the starts
// below it in the wave): the fill's units are written too, units[slot] = {k,
// unit_len[k]}, and their number into unit_total.
template <bool UNITS>
__global__ __launch_bounds__(kThreads) void k_block_rows(const uint64_t* __restrict__ kv, uint32_t n,
                                                         const int32_t* __restrict__ bo,
                                                         const uint32_t* __restrict__ rowidx32,
                                                         const uint64_t* __restrict__ masks,
                                                         const uint64_t* __restrict__ scan64, uint32_t maxp,
                                                         uint32_t G, int4* __restrict__ info,
                                                         const uint32_t* __restrict__ total32, uint64_t max_blocks,
                                                         int32_t* __restrict__ total_out,
                                                         const int32_t* __restrict__ unit_len,
                                                         uint2* __restrict__ units, int32_t* __restrict__ unit_total) {
  const uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  const uint32_t nw = (n + 63) >> 6;
  const uint32_t t = UNITS ? (uint32_t)scan64[nw] : *total32;
  if (i == 0) {
    if (total_out) *total_out = (int32_t)t;
    if constexpr (UNITS) *unit_total = (int32_t)(scan64[nw] >> 32);
  }
  if (i < max_blocks && i >= t) info[i] = make_int4(0, 0, 0, 0);
  if (i >= n) return;
  const uint32_t k = (uint32_t)i;
  uint32_t row;
  if constexpr (UNITS) {
    const uint32_t w = k >> 6;
    const uint64_t below = (1ull << (k & 63u)) - 1ull;
    const uint64_t bm = masks[2 * (uint64_t)w], um = masks[2 * (uint64_t)w + 1], sk = scan64[w];
    if ((um >> (k & 63u)) & 1ull)
      units[(uint32_t)(sk >> 32) + (uint32_t)__popcll(um & below)] = make_uint2(k, (uint32_t)unit_len[k]);
    if (((bm >> (k & 63u)) & 1ull) == 0ull) return;  // not a block start
    row = (uint32_t)sk + (uint32_t)__popcll(bm & below);
  } else {
    row = rowidx32[k];
    if (rowidx32[k + 1] == row) return;  // not a block start
  }
  const uint32_t key = kv_key(kv[k]);
  const uint32_t rs = bo != nullptr ? (uint32_t)bo[key] : run_start(kv, k, key);
  const uint32_t re = bo != nullptr ? (uint32_t)bo[key + 1] : run_end(kv, n, k, key);
  const uint32_t off = k - rs;
  info[row] = make_int4((int)key, (int)off, (int)min(maxp, re - k), (int)(key / G));
}

// ----------------------------------------------------------- bin / unbin

// One group of `lanes` threads moves one particle row.  forward: scatter
// in[b,i] -> out[b,perm[b,i]];  backward: gather out[b,i] = in[b,perm[b,i]].
// Null mass pointers leave the mass rows out.
template <int P, bool VEC4>
__global__ __launch_bounds__(kThreads) void k_move_rows(const float* __restrict__ in_pos,
                                                        const float* __restrict__ in_state,
                                                        const float* __restrict__ in_mass,
                                                        const int32_t* __restrict__ perm, float* __restrict__ out_pos,
                                                        float* __restrict__ out_state, float* __restrict__ out_mass,
                                                        uint32_t n, uint32_t N, uint32_t C, int lanes_log2,
                                                        int forward) {
  const uint64_t gid = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  const uint64_t k = gid >> lanes_log2;
  const uint32_t q = (uint32_t)(gid & ((1u << lanes_log2) - 1));
  if (k >= n) return;
  const uint64_t b = k / N;
  const uint64_t slot = b * N + (uint32_t)perm[k];
  const uint64_t src = forward ? k : slot;
  const uint64_t dst = forward ? slot : k;
  if (q == 0) {
    if constexpr (P == 2)
      reinterpret_cast<float2*>(out_pos)[dst] = reinterpret_cast<const float2*>(in_pos)[src];
    else
      reinterpret_cast<float4*>(out_pos)[dst] = reinterpret_cast<const float4*>(in_pos)[src];
    if (in_mass != nullptr) out_mass[dst] = in_mass[src];
  }
  const uint32_t lanes = 1u << lanes_log2;
  if constexpr (VEC4) {
    const uint32_t U = C >> 2;
    const float4* s4 = reinterpret_cast<const float4*>(in_state) + src * U;
    float4* d4 = reinterpret_cast<float4*>(out_state) + dst * U;
    for (uint32_t u = q; u < U; u += lanes) d4[u] = s4[u];
  } else {
    const float* s1 = in_state + src * C;
    float* d1 = out_state + dst * C;
    for (uint32_t u = q; u < C; u += lanes) d1[u] = s1[u];
  }
}

template <int D>
void launch_keys(const Grid& g, const float* pos, uint32_t n, hipStream_t st) {
  const uint32_t ntiles = (uint32_t)g.n_tiles;
  if (g.periodic)
    hipLaunchKernelGGL((k_cell_keys<D, true>), dim3(ntiles), dim3(kCountThreads), 0, st, g.p, pos, g.kv[0], n, g.hist,
                       ntiles);
  else
    hipLaunchKernelGGL((k_cell_keys<D, false>), dim3(ntiles), dim3(kCountThreads), 0, st, g.p, pos, g.kv[0], n, g.hist,
                       ntiles);
  SPHOPS_LAUNCHED();
}

inline dim3 blocks_for(uint64_t n) { return dim3((uint32_t)((n + kThreads - 1) / kThreads)); }

}  // namespace

namespace {
// Words from device memory into (device-visible) pinned host memory, with
// system-scope stores so that the host sees them once the kernel is done.
__global__ __launch_bounds__(kThreads) void k_words_to_host(const uint32_t* __restrict__ src, uint32_t* dst,
                                                            uint32_t words) {
  const uint32_t i = threadIdx.x;
  if (i < words) __hip_atomic_store(dst + i, src[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
}  // namespace

void copy_words_to_host(const uint32_t* src, uint32_t* dst_device_view, uint32_t words, hipStream_t st) {
  if (words == 0) return;
  hipLaunchKernelGGL(k_words_to_host, dim3(1), dim3(kThreads), 0, st, src, dst_device_view, words);
  SPHOPS_LAUNCHED();
}

// A fill kernel rather than hipMemsetAsync, so that a step captured in a HIP
// graph holds no memset nodes.
void fill_u32(uint32_t* p, uint64_t n, uint32_t v, hipStream_t st) {
  if (n == 0) return;
  hipLaunchKernelGGL(k_fill_u32, dim3((uint32_t)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, st, p, n, v);
  SPHOPS_LAUNCHED();
}

// ------------------------------------------------ neighbour-list schedule
//
// Stable partition of the binned particles into kNumClasses classes by
// neighbour-list length (kListClasses), which the pair kernels serve with
// groups of kListGroups (or kSplitGroups) lanes per particle.  The partition
// is done per tile of 4096 binned particles and the tiles stay in order
// (tile-major: every class of a region of space is processed together, so
// neighbour rows shared between classes are reused from the same L2).

namespace {

// Class of a list (or candidate) length: the number of bounds it exceeds.
__device__ __forceinline__ uint32_t length_class(int32_t len, const ClassBounds& cb) {
  uint32_t q = 0;
#pragma unroll
  for (int i = 0; i < kNumClasses - 1; ++i) q += (len > cb.t[i]) ? 1u : 0u;
  return q;
}

// Length of item idx: from CSR offsets (CSR) or a plain length array.
// A plain length of -1 marks an item that is not scheduled; below -1 it
// encodes a particle whose list row was not stored, -1 - (its stencil
// candidates), scheduled by its candidates (the pair kernels walk them).
template <bool CSR>
__device__ __forceinline__ int32_t item_length(const int32_t* __restrict__ src, uint32_t idx) {
  if constexpr (CSR) return src[idx + 1] - src[idx];
  const int32_t v = src[idx];
  return v >= -1 ? v : -1 - v;
}

// Per tile of kTile items: the number of items of each class, written to
// cnt[tile * kNumClasses + class].
// Items of negative length are skipped: they get no class and no slot.
template <bool CSR>
__global__ __launch_bounds__(kCountThreads) void k_class_count(const int32_t* __restrict__ src, uint32_t n,
                                                               ClassBounds cb, uint32_t* __restrict__ cnt) {
  __shared__ uint32_t h[kNumClasses];
  if (threadIdx.x < kNumClasses) h[threadIdx.x] = 0;
  __syncthreads();
  const uint32_t base = blockIdx.x * kTile;
  uint32_t c[kNumClasses] = {};
#pragma unroll
  for (int i = 0; i < kCountItems; ++i) {
    const uint32_t idx = base + i * kCountThreads + threadIdx.x;
    const int32_t len = idx < n ? item_length<CSR>(src, idx) : -1;
    if (len >= 0) {
      const uint32_t k = length_class(len, cb);
#pragma unroll
      for (int q = 0; q < kNumClasses; ++q) c[q] += (k == (uint32_t)q);
    }
  }
#pragma unroll
  for (int q = 0; q < kNumClasses; ++q) {
    uint32_t v = c[q];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
    if (__lane_id() == 0) atomicAdd(&h[q], v);
  }
  __syncthreads();
  if (threadIdx.x < kNumClasses) cnt[blockIdx.x * kNumClasses + threadIdx.x] = h[threadIdx.x];
}

// Waves of a segment of c items at g lanes per item (64 / g items a wave).
__device__ __forceinline__ uint32_t seg_waves(uint32_t c, int32_t g) {
  const uint32_t per = (uint32_t)(kWave / g);
  return (c + per - 1) / per;
}

// Stable scatter of a tile's items into order, class by class, and the wave
// descriptors of the tile's segments.  The tile first finds its segment
// offsets (segment s = tile * kNumClasses + class, in tile-major order): the
// sum of the counts of all earlier tiles, reduced by the workgroup, plus the
// tile's own earlier classes; it writes them to seg (and the last tile the
// item total to seg[nseg]).  The same reduction gives the first wave of each
// of its segments in the descriptor table of each group-size table (the
// waves of all earlier segments), and the last tile writes the tables' wave
// totals.  Same tile walk as the radix scatter: wave w owns items
// [w*1024, (w+1)*1024) in index order; three ballots identify lanes of the
// same class.  Descriptor {first slot in order, group size << 8 | items}:
// one per 64-lane wave of a segment.
template <bool CSR>
__global__ __launch_bounds__(kThreads) void k_class_scatter(const int32_t* __restrict__ src, uint32_t n,
                                                            ClassBounds cb, const uint32_t* __restrict__ cnt,
                                                            uint32_t* __restrict__ seg,
                                                            int32_t* __restrict__ order, GroupSizes gs1,
                                                            GroupSizes gs2, int tables, uint2* __restrict__ waves1,
                                                            uint2* __restrict__ waves2,
                                                            int32_t* __restrict__ total1,
                                                            int32_t* __restrict__ total2) {
  __shared__ uint32_t wcnt[kThreads / 64][kNumClasses];
  __shared__ uint32_t gbase[kNumClasses], gcnt[kNumClasses];
  __shared__ uint32_t wbase[2][kNumClasses];
  __shared__ uint32_t part[3][kThreads / 64];
  const int wave = threadIdx.x >> 6, lane = __lane_id();
  if (threadIdx.x < (kThreads / 64) * kNumClasses) (&wcnt[0][0])[threadIdx.x] = 0;
  {
    const uint32_t before = blockIdx.x * (uint32_t)kNumClasses;
    uint32_t s = 0, w1 = 0, w2 = 0;
    for (uint32_t i = threadIdx.x; i < before; i += kThreads) {
      const uint32_t c = cnt[i];
      s += c;
      w1 += seg_waves(c, gs1.g[i % kNumClasses]);
      if (tables == 2) w2 += seg_waves(c, gs2.g[i % kNumClasses]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      s += __shfl_down(s, off, 64);
      w1 += __shfl_down(w1, off, 64);
      w2 += __shfl_down(w2, off, 64);
    }
    if (lane == 0) {
      part[0][wave] = s;
      part[1][wave] = w1;
      part[2][wave] = w2;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t run = 0, r1 = 0, r2 = 0;
      for (int w = 0; w < kThreads / 64; ++w) {
        run += part[0][w];
        r1 += part[1][w];
        r2 += part[2][w];
      }
      for (int q = 0; q < kNumClasses; ++q) {
        const uint32_t c = cnt[before + q];
        gbase[q] = run;
        gcnt[q] = c;
        seg[before + q] = run;
        run += c;
        wbase[0][q] = r1;
        r1 += seg_waves(c, gs1.g[q]);
        wbase[1][q] = r2;
        if (tables == 2) r2 += seg_waves(c, gs2.g[q]);
      }
      if (blockIdx.x == gridDim.x - 1) {
        seg[before + kNumClasses] = run;
        *total1 = (int32_t)r1;
        if (tables == 2) *total2 = (int32_t)r2;
      }
    }
  }
  __syncthreads();
  const uint32_t base = blockIdx.x * kTile + wave * (kTile / (kThreads / 64));
  const uint64_t below_mask = lanemask_lt();
  uint32_t cls[kItems], rank[kItems];
#pragma unroll
  for (int t = 0; t < kItems; ++t) {
    const uint32_t idx = base + t * 64 + lane;
    const int32_t len = idx < n ? item_length<CSR>(src, idx) : -1;
    const bool valid = len >= 0;
    const uint32_t k = valid ? length_class(len, cb) : 0u;
    cls[t] = k;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 3; ++bit) {
      const uint64_t bb = __ballot((k >> bit) & 1u);
      peers &= ((k >> bit) & 1u) ? bb : ~bb;
    }
    const uint32_t before = (uint32_t)__popcll(peers & below_mask);
    const uint32_t prior = wcnt[wave][k];
    if (valid && before == 0) wcnt[wave][k] = prior + (uint32_t)__popcll(peers);
    rank[t] = prior + before;
  }
  __syncthreads();
  if (threadIdx.x < kNumClasses) {
    uint32_t run = 0;
    for (int w = 0; w < kThreads / 64; ++w) {
      const uint32_t c = wcnt[w][threadIdx.x];
      wcnt[w][threadIdx.x] = run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < kItems; ++t) {
    const uint32_t idx = base + t * 64 + lane;
    if (idx < n && item_length<CSR>(src, idx) >= 0) order[gbase[cls[t]] + wcnt[wave][cls[t]] + rank[t]] = (int32_t)idx;
  }
  // the descriptors of the tile's segments, table by table
  for (int tb = 0; tb < tables; ++tb) {
    const GroupSizes& gs = tb == 0 ? gs1 : gs2;
    uint2* __restrict__ waves = tb == 0 ? waves1 : waves2;
#pragma unroll
    for (int q = 0; q < kNumClasses; ++q) {
      const uint32_t lo = gbase[q], c = gcnt[q];
      const uint32_t per = (uint32_t)(kWave / gs.g[q]);
      const uint32_t nw = (c + per - 1) / per;
      for (uint32_t u = threadIdx.x; u < nw; u += kThreads)
        waves[wbase[tb][q] + u] = make_uint2(lo + u * per, ((uint32_t)gs.g[q] << 8) | min(per, c - u * per));
    }
  }
}

// Tile-major schedule: per tile of 4096 binned particles a stable partition
// by length class, tiles in order, plus one descriptor per 64-lane wave.
template <bool CSR>
void tiled_schedule(const Grid& g, const int32_t* src, const ClassBounds& cb, const GroupSizes& gs, int32_t* order,
                    uint2* waves, int32_t* wave_total, hipStream_t st, const GroupSizes* gs2 = nullptr,
                    uint2* waves2 = nullptr, int32_t* wave_total2 = nullptr) {
  const uint32_t n = (uint32_t)g.n_keys;
  const uint32_t ntiles = (uint32_t)g.n_tiles;
  const uint32_t nseg = (uint32_t)kNumClasses * ntiles;
  // hist holds 256 * ntiles words: item counts per segment, then their
  // offsets (nseg + 1, the last is the number of scheduled items)
  uint32_t* cnt = g.hist;
  uint32_t* seg = cnt + nseg;
  hipLaunchKernelGGL((k_class_count<CSR>), dim3(ntiles), dim3(kCountThreads), 0, st, src, n, cb, cnt);
  SPHOPS_LAUNCHED();
  const int tables = waves2 != nullptr ? 2 : 1;  // a second table: same order, other group sizes
  const GroupSizes gsb = gs2 != nullptr ? *gs2 : gs;
  hipLaunchKernelGGL((k_class_scatter<CSR>), dim3(ntiles), dim3(kThreads), 0, st, src, n, cb, cnt, seg, order, gs,
                     gsb, tables, waves, tables == 2 ? waves2 : waves, wave_total,
                     tables == 2 ? wave_total2 : wave_total);
  SPHOPS_LAUNCHED();
}

}  // namespace

uint64_t neighbour_wave_capacity(const Grid& g) { return g.n_keys + (uint64_t)kNumClasses * g.n_tiles; }

void run_split_schedule(const Grid& g, const int32_t* len, int32_t* order, uint2* waves, int32_t* wave_total,
                        hipStream_t st) {
  tiled_schedule<false>(g, len, kListClasses, kSplitGroups, order, waves, wave_total, st);
}

void run_neighbour_schedule(const Grid& g, const int32_t* ncnt, int32_t* order, uint2* waves, int32_t* wave_total,
                            uint2* waves2, int32_t* wave_total2, hipStream_t st) {
  tiled_schedule<false>(g, ncnt, kListClasses, kListGroups, order, waves, wave_total, st, &kSplitGroups, waves2,
                        wave_total2);
}

namespace {
__global__ __launch_bounds__(kThreads) void k_unit_write(const int32_t* __restrict__ unit_len,
                                                         const uint32_t* __restrict__ slot, uint32_t n,
                                                         uint2* __restrict__ units) {
  const uint32_t k = blockIdx.x * kThreads + threadIdx.x;
  if (k >= n) return;
  const int32_t len = unit_len[k];
  if (len > 0) units[slot[k]] = make_uint2(k, (uint32_t)len);
}
}  // namespace

void run_unit_schedule(const Grid& g, hipStream_t st) {
  const uint32_t n = (uint32_t)g.n_keys;
  device_exclusive_scan(g.flags, g.flags, n, g.scan_tmp, reinterpret_cast<uint32_t*>(g.unit_total), st);
  hipLaunchKernelGGL(k_unit_write, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, st, g.unit_len, g.flags,
                     n, g.units);
  SPHOPS_LAUNCHED();
}

void exclusive_scan_u32(const Grid& g, uint32_t* data, uint64_t n, uint32_t* total, hipStream_t st) {
  device_exclusive_scan(data, data, n, g.scan_tmp, total, st);
}

void run_instantiate(Grid& g, const float* pos, int32_t* perm, int32_t* bo, int32_t* block_info,
                     int32_t* total_blocks, hipStream_t st, int32_t* inv) {
  const uint32_t n = (uint32_t)g.n_keys;
  const uint64_t ncp1 = g.n_cells + 1;
  if (n == 0) {
    hipLaunchKernelGGL(k_fill_u32, blocks_for(ncp1), dim3(kThreads), 0, st, reinterpret_cast<uint32_t*>(bo),
                       ncp1, 0u);
    SPHOPS_LAUNCHED();
    if (!g.particle_mode) {
      hipLaunchKernelGGL(k_fill_u32, blocks_for(g.max_blocks * 4 + 1), dim3(kThreads), 0, st,
                         reinterpret_cast<uint32_t*>(block_info), g.max_blocks * 4, 0u);
      SPHOPS_LAUNCHED();
    }
    if (total_blocks) fill_u32(reinterpret_cast<uint32_t*>(total_blocks), 1, 0u, st);
    return;
  }
  // 1. keys, with the first pass's digit counts
  if ((uint64_t)n > g.n_tiles * kTile) throw Error("instantiate: more keys than radix tiles");
  if (g.dim == 2) launch_keys<2>(g, pos, n, st);
  else launch_keys<3>(g, pos, n, st);

  // 2. stable LSD radix sort of (key, index)
  int bits = 1;
  while (bits < 32 && (g.n_cells - 1) >> bits) ++bits;
  const int passes = (bits + kRadixBits - 1) / kRadixBits;
  const uint32_t ntiles = (uint32_t)g.n_tiles;
  uint32_t* digit_totals = g.hist + (uint64_t)kBins * ntiles;  // the histograms' last kBins words
  int cur = 0;
  for (int p = 0; p < passes; ++p) {
    const int shift = p * kRadixBits;
    if (p > 0) {  // the first pass's counts come from k_cell_keys
      hipLaunchKernelGGL(k_radix_hist, dim3(ntiles), dim3(kCountThreads), 0, st, g.kv[cur], n, shift, g.hist,
                         ntiles);
      SPHOPS_LAUNCHED();
    }
    hipLaunchKernelGGL(k_radix_colscan, dim3(kBins / (kThreads / 64)), dim3(kThreads), 0, st, g.hist, ntiles,
                       digit_totals);
    SPHOPS_LAUNCHED();
    hipLaunchKernelGGL(k_radix_scatter, dim3(ntiles), dim3(kThreads), 0, st, g.kv[cur], g.kv[cur ^ 1], n, shift,
                       g.hist, digit_totals, ntiles);
    SPHOPS_LAUNCHED();
    cur ^= 1;
  }
  const uint64_t* skv = g.kv[cur];

  // 3. bin_offsets via per-chunk key ranges
  const uint32_t nch = (uint32_t)g.n_chunks;
  hipLaunchKernelGGL(k_chunk_lo, blocks_for((uint64_t)nch + 1), dim3(kThreads), 0, st, skv, n, g.chunk_lo, nch);
  SPHOPS_LAUNCHED();
  const uint32_t nb_bo = (nch + kChunksPerBlock - 1) / kChunksPerBlock;

  // 4. permutation (destination slot of each input particle), with the
  // block-start flags in grid mode and, when the grid has the fill's
  // buffers, the fill's work split (unit_len, the units and their count);
  // on large grids it takes cell bounds from the sorted keys and runs in
  // the bin_offsets launch
  const int32_t* cell_bo = g.n_cells >= kRunSearchMinCells ? nullptr : bo;
  const bool units = g.unit_len != nullptr && g.units != nullptr && g.unit_total != nullptr;
  // the masks of the block and unit starts and their per-wave counts take
  // 3 nw + 1 words of the other sort buffer (n + 1 words, free after the sort)
  const uint32_t nw = (n + 63) / 64;
  const bool dual = units && !g.particle_mode && n >= 64 && dual_scan_fits(g, nw);
  uint64_t* f64 = g.kv[cur ^ 1];
  const uint32_t nb_perm = blocks_for(n).x;
  if (cell_bo != nullptr) {
    hipLaunchKernelGGL(k_bin_offsets, dim3(nb_bo), dim3(kThreads), 0, st, skv, g.chunk_lo, nch, bo, ncp1);
    SPHOPS_LAUNCHED();
  }
  const uint32_t every = std::max<uint32_t>(1u, nb_bo / std::max<uint32_t>(nb_perm, 1u));
  // the interleaved launch covers nb_perm * (every + 1) workgroups, or more
  // when the chunks outnumber the permutation's (every rounds down)
  const uint32_t nb_all = std::max(nb_bo + nb_perm, nb_perm * (every + 1));
#define SPHOPS_PERM(BL, UN, F32, F64)                                                                              \
  do {                                                                                                              \
    if (cell_bo != nullptr)                                                                                         \
      hipLaunchKernelGGL((k_permutation<BL, UN>), blocks_for(n), dim3(kThreads), 0, st, skv, n, g.p.N, perm,       \
                         cell_bo, g.p.maxp, F32, F64, UN ? g.unit_len : nullptr, inv);                              \
    else                                                                                                            \
      hipLaunchKernelGGL((k_offsets_permutation<BL, UN>), dim3(nb_all), dim3(kThreads), 0, st, skv, g.chunk_lo,    \
                         nch, bo, ncp1, nb_bo, n, g.p.N, perm, g.p.maxp, F32, F64, UN ? g.unit_len : nullptr, inv,  \
                         nb_perm, every);                                                                           \
  } while (0)
  if (g.particle_mode) {
    if (units) SPHOPS_PERM(false, true, g.flags, nullptr);
    else SPHOPS_PERM(false, false, nullptr, nullptr);
  } else {
    if (dual) SPHOPS_PERM(true, true, nullptr, f64);
    else SPHOPS_PERM(true, false, g.flags, nullptr);
  }
#undef SPHOPS_PERM
  SPHOPS_LAUNCHED();

  // 5. block table (grid mode) and the fill's units
  if (!g.particle_mode) {
    const dim3 rows_grid = blocks_for(std::max<uint64_t>(n, g.max_blocks));
    if (dual) {
      uint64_t* counts = f64 + 2 * (uint64_t)nw;
      device_exclusive_scan64(counts, counts, nw, g.scan_tmp, counts + nw, st);
      hipLaunchKernelGGL(k_block_rows<true>, rows_grid, dim3(kThreads), 0, st, skv, n, cell_bo, nullptr, f64, counts,
                         g.p.maxp, g.p.G, reinterpret_cast<int4*>(block_info), nullptr, g.max_blocks, total_blocks,
                         g.unit_len, g.units, g.unit_total);
    } else {
      device_exclusive_scan(g.flags, g.flags, n, g.scan_tmp, g.flags + n, st);
      hipLaunchKernelGGL(k_block_rows<false>, rows_grid, dim3(kThreads), 0, st, skv, n, cell_bo, g.flags, nullptr,
                         nullptr,
                         g.p.maxp, g.p.G, reinterpret_cast<int4*>(block_info), g.flags + n, g.max_blocks,
                         total_blocks, nullptr, nullptr, nullptr);
    }
    SPHOPS_LAUNCHED();
  } else {
    if (units) {
      device_exclusive_scan(g.flags, g.flags, n, g.scan_tmp, reinterpret_cast<uint32_t*>(g.unit_total), st);
      hipLaunchKernelGGL(k_unit_write, blocks_for(n), dim3(kThreads), 0, st, g.unit_len, g.flags, n, g.units);
      SPHOPS_LAUNCHED();
    }
    if (total_blocks) fill_u32(reinterpret_cast<uint32_t*>(total_blocks), 1, 0u, st);
  }
  // the fill's work split now describes this snapshot's cell runs (and a
  // fill prepared for an earlier snapshot must be prepared again)
  g.split_key[0] = g.split_key[1] = nullptr;
  g.split_bo = (units && (dual || g.particle_mode)) ? bo : nullptr;
}

void run_bin_particles(const Grid& g, const float* in_pos, const float* in_state, const float* in_mass,
                       const int32_t* perm, float* out_pos, float* out_state, float* out_mass, uint32_t C,
                       bool forward, hipStream_t st) {
  const uint32_t n = (uint32_t)g.n_keys;
  if (n == 0) return;
  const bool vec4 = (C % 4 == 0) && (reinterpret_cast<uintptr_t>(in_state) % 16 == 0) &&
                    (reinterpret_cast<uintptr_t>(out_state) % 16 == 0);
  const uint32_t units = vec4 ? C / 4 : C;
  int lanes_log2 = 0;
  while ((1u << lanes_log2) < units && lanes_log2 < 4) ++lanes_log2;
  const uint64_t threads = (uint64_t)n << lanes_log2;
  const dim3 grid = blocks_for(threads);
  const int fw = forward ? 1 : 0;
#define SPHOPS_MOVE(P, V)                                                                                 \
  hipLaunchKernelGGL((k_move_rows<P, V>), grid, dim3(kThreads), 0, st, in_pos, in_state, in_mass, perm, \
                     out_pos, out_state, out_mass, n, g.p.N, C, lanes_log2, fw)
  if (g.dim == 2) {
    if (vec4) SPHOPS_MOVE(2, true); else SPHOPS_MOVE(2, false);
  } else {
    if (vec4) SPHOPS_MOVE(4, true); else SPHOPS_MOVE(4, false);
  }
#undef SPHOPS_MOVE
  SPHOPS_LAUNCHED();
}

}  // namespace sphops
