// Cell-tiled pass-B backward (blur + gradient_hybrid, C = 16) for the
// particles of well-filled cells.
//
// The lane-split list kernel (k_blur_hybrid_bwd_quad) loads every neighbour
// row from L2 once per directed pair: 336 bytes per pair at C = 16, and its
// time follows the number of vector-memory instructions that takes.  Here a
// unit of up to kTileP particles of one cell -- which share the cell's
// stencil -- is served by one workgroup that streams the stencil's rows
// (positions and volumes, s, the two upstream gradients) through LDS in
// chunks of kTileRows contiguous rows, so each row is loaded once per unit
// and read from LDS by every pair that needs it.
//
// Work balance: the pairs of a chunk (every unit particle's list entries
// that fall in the chunk's rows, particle-major) are cut into 64 equal runs,
// one per lane quad; the four lanes of a quad hold the four channel slices
// of a pair.  A run may start or end inside a particle's pairs.  A quad adds
// its partial sums for a particle straight into the particle's LDS
// accumulator when the particle starts inside its run (no other quad starts
// with it, so no two quads write one accumulator), and into its own slot
// when the particle is the first of its run; after a barrier the slots are
// added to the accumulators particle by particle in quad order.  Every sum
// runs in a fixed order: results are deterministic, with no atomics on
// floating-point data.
//
// Included by perception_kernels.hpp after the list-build kernels (it uses
// their Walker, fetch_ranges and row helpers); not a standalone header.
#pragma once

namespace sphops {
namespace pk {

constexpr int kTileThreads = 256;                   // one workgroup, 64 lane quads
constexpr int kTileQuads = kTileThreads / 4;
constexpr int kTileP = 32;                          // particles per unit
constexpr int kTileRows = 112;                      // stencil rows per chunk
constexpr int kTileMinOcc = 8;                      // cells with this many particles or more are tiled
constexpr int kTileWorkgroups = 1024;               // persistent launch
constexpr int kTileMaxRanges = 27;

// ---------------------------------------------------------------- units
//
// Per binned particle k: whether its cell is tiled (at least kTileMinOcc
// particles), the first particle of every run of kTileP particles of a tiled
// cell (flag = 1, unit_len = particles of the unit), and the list length the
// split schedule of the remaining particles takes (-1 for tiled particles:
// not scheduled).
template <int D, bool P>
__device__ __forceinline__ void tile_flags_of(const GridParams& g, const int32_t* __restrict__ bo, uint32_t k,
                                              const float* xi, const int32_t* __restrict__ ncnt,
                                              uint32_t* __restrict__ flags, int32_t* __restrict__ unit_len,
                                              int32_t* __restrict__ sparse_len) {
  int c[3];
  pos2cell<D, P>(g, xi, c);
  const uint32_t h = (k / g.N) * g.G + cell_hash<D>(g, c);
  const int32_t cs = bo[h], ce = bo[h + 1];
  const bool tiled = ce - cs >= kTileMinOcc;
  const int32_t off = (int32_t)k - cs;
  const bool first = tiled && off % kTileP == 0;
  flags[k] = first ? 1u : 0u;
  unit_len[k] = first ? min(kTileP, ce - (int32_t)k) : 0;
  sparse_len[k] = tiled ? -1 : ncnt[k];
}

template <int D, bool P>
__global__ __launch_bounds__(kThreads) void k_tile_flags(GridParams g, const int32_t* __restrict__ bo,
                                                         const float4* __restrict__ xw,
                                                         const int32_t* __restrict__ ncnt,
                                                         uint32_t* __restrict__ flags, int32_t* __restrict__ unit_len,
                                                         int32_t* __restrict__ sparse_len) {
  const uint32_t n = g.B * g.N;
  const uint32_t k = blockIdx.x * kThreads + threadIdx.x;
  if (k >= n) return;
  float xi[3];
  unpack(xw[k], xi);
  tile_flags_of<D, P>(g, bo, k, xi, ncnt, flags, unit_len, sparse_len);
}

[[maybe_unused]] static __global__ __launch_bounds__(kThreads) void k_tile_units(const int32_t* __restrict__ unit_len,
                                                         const uint32_t* __restrict__ slot, uint32_t n,
                                                         uint2* __restrict__ units) {
  const uint32_t k = blockIdx.x * kThreads + threadIdx.x;
  if (k >= n) return;
  const int32_t len = unit_len[k];
  if (len > 0) units[slot[k]] = make_uint2(k, (uint32_t)len);
}

// ------------------------------------------------------------ the kernel

// Sum over the four lanes of a quad, delivered to all four.
static __device__ __forceinline__ float quad_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
  return v;
}

template <int D, bool P, bool FULL>
struct TileShared {
  static constexpr int C = 16, CW = 4;
  static constexpr int kS = C + 4;            // row strides (floats): an odd number of 16-byte units
  static constexpr int kG2 = C * D + 4;
  static constexpr int kAcc = 2 * C + 3 + (FULL ? 7 : 0);
  static constexpr int kAccS = kAcc | 1;
  static constexpr int kOwn = FULL ? kTileP : 1;
  float4 xw[kTileRows];
  float s[FULL ? kTileRows : 1][kS];
  float gb[kTileRows][kS];
  float g2[kTileRows][kG2];
  float4 own_xw[kTileP];
  float own_s[kOwn][kS];
  float own_gb[kOwn][kS];
  float own_g2[kOwn][kG2];
  float acc[kTileP][kAccS];
  float slot[kTileQuads][kAccS];
  uint8_t jl[kTileP * kTileRows];            // the chunk's pairs, particle-major: row within the chunk
  int32_t cum[2][kTileP + 1];                // per chunk (two in flight): pairs of the particles before
  int32_t wtot[kTileThreads / 64];
  uint32_t gidx[2][kTileRows];               // global row of each chunk row (two chunks in flight)
  uint32_t ra[kTileMaxRanges], rb[kTileMaxRanges], pre[kTileMaxRanges + 1];
};

// Row staging of one chunk: every thread's share of the chunk's rows (the
// packed position, blur and gradient upstream rows, and s with FULL), loaded
// into registers in one batch and written to LDS later.
template <int D, bool FULL>
struct TileStage {
  static constexpr int C = 16;
  static constexpr int kXw = (kTileRows + kTileThreads - 1) / kTileThreads;
  static constexpr int kGb = (kTileRows * C / 4 + kTileThreads - 1) / kTileThreads;
  static constexpr int kG2 = (kTileRows * C * D / 4 + kTileThreads - 1) / kTileThreads;
  static constexpr int kSs = FULL ? kGb : 0;
  float4 xw[kXw], gb[kGb], g2[kG2], s[kSs > 0 ? kSs : 1];

  __device__ __forceinline__ void load(const OpPtrs& a, const uint32_t* gidx, uint32_t nr, int tid) {
#pragma unroll
    for (int q = 0; q < kXw; ++q) {
      const uint32_t i = tid + q * kTileThreads;
      if (i < nr) xw[q] = a.xw[gidx[i]];
    }
#pragma unroll
    for (int q = 0; q < kGb; ++q) {
      const uint32_t i = tid + q * kTileThreads;
      if (i < nr * (C / 4)) {
        gb[q] = reinterpret_cast<const float4*>(a.g)[(uint64_t)gidx[i / (C / 4)] * (C / 4) + i % (C / 4)];
        if constexpr (FULL)
          s[q] = reinterpret_cast<const float4*>(a.s)[(uint64_t)gidx[i / (C / 4)] * (C / 4) + i % (C / 4)];
      }
    }
#pragma unroll
    for (int q = 0; q < kG2; ++q) {
      const uint32_t i = tid + q * kTileThreads;
      if (i < nr * (C * D / 4))
        g2[q] = reinterpret_cast<const float4*>(a.g2)[(uint64_t)gidx[i / (C * D / 4)] * (C * D / 4) + i % (C * D / 4)];
    }
  }

  template <class SH>
  __device__ __forceinline__ void store(SH& sh, uint32_t nr, int tid) const {
#pragma unroll
    for (int q = 0; q < kXw; ++q) {
      const uint32_t i = tid + q * kTileThreads;
      if (i < nr) sh.xw[i] = xw[q];
    }
#pragma unroll
    for (int q = 0; q < kGb; ++q) {
      const uint32_t i = tid + q * kTileThreads;
      if (i < nr * (C / 4)) {
        *reinterpret_cast<float4*>(&sh.gb[i / (C / 4)][4 * (i % (C / 4))]) = gb[q];
        if constexpr (FULL) *reinterpret_cast<float4*>(&sh.s[i / (C / 4)][4 * (i % (C / 4))]) = s[q];
      }
    }
#pragma unroll
    for (int q = 0; q < kG2; ++q) {
      const uint32_t i = tid + q * kTileThreads;
      if (i < nr * (C * D / 4)) *reinterpret_cast<float4*>(&sh.g2[i / (C * D / 4)][4 * (i % (C * D / 4))]) = g2[q];
    }
  }
};

// Global rows of chunk c of the stencil (its rows concatenated in range
// order): gidx[i] for i < the chunk's row count, which is returned.
template <class SH>
__device__ __forceinline__ uint32_t tile_chunk_rows(SH& sh, int R, uint32_t c, uint32_t* gidx, int tid) {
  const uint32_t T = sh.pre[R];
  const uint32_t p0 = c * kTileRows;
  const uint32_t nr = p0 < T ? min((uint32_t)kTileRows, T - p0) : 0u;
  if ((uint32_t)tid < nr) {
    const uint32_t pos = p0 + tid;
    int r = 0;
    while (sh.pre[r + 1] <= pos) ++r;
    gidx[tid] = sh.ra[r] + (pos - sh.pre[r]);
  }
  return nr;
}

// Accumulator layout (per particle, and per slot): [0, C) dsb, [C, 2C) dsg,
// [2C, 2C+3) sum_j v_j grad W, and with FULL [2C+3, 2C+6) dx of blur,
// [2C+6, 2C+9) dx of the gradient, [2C+9] drho of the gradient.
template <int D, bool P, bool FULL>
__global__ __launch_bounds__(kTileThreads, 2) void k_blur_hybrid_bwd_tiled(GridParams g, OpPtrs a,
                                                                           const int32_t* __restrict__ bo) {
  using SH = TileShared<D, P, FULL>;
  constexpr int C = SH::C, CW = SH::CW;
  constexpr int kTestSub = kTileThreads / kTileP;              // threads testing one particle's candidates
  constexpr int kTestPer = (kTileRows + kTestSub - 1) / kTestSub;  // candidates per thread and chunk
  static_assert(kTestPer <= 32, "test mask is 32 bits");
  __shared__ SH sh;
  const int tid = threadIdx.x;
  const int lane = __lane_id(), wave = tid >> 6;
  const int quad = tid >> 2, sl = tid & 3;
  const uint32_t c0 = (uint32_t)sl * CW;
  const float4* __restrict__ xw = a.xw;
  const uint32_t nunits = (uint32_t)*a.tile_count;
  const int R = g.morton ? Walker<D, P>::kCellRanges : Walker<D, P>::kRowRanges;
  const int tp = tid / kTestSub, tsub = tid % kTestSub;        // tester: particle, sub-lane

  for (uint32_t u = blockIdx.x; u < nunits; u += gridDim.x) {
    const uint2 ud = a.tile_units[u];
    const uint32_t k0 = ud.x;
    const int n = (int)ud.y;
    // ---- the cell's stencil ranges; the unit's own rows; zero accumulators
    if (tid < R) {
      float x0[3];
      unpack(xw[k0], x0);
      Walker<D, P> w;
      w.init(g, x0, k0);
      w.fetch(g, bo, tid);
      sh.ra[tid] = w.j;
      sh.rb[tid] = w.jend;
    }
    if (tid < n) sh.own_xw[tid] = xw[k0 + tid];
    if constexpr (FULL) {
      const float4* ssrc = reinterpret_cast<const float4*>(a.s) + (uint64_t)k0 * (C / 4);
      const float4* gsrc = reinterpret_cast<const float4*>(a.g) + (uint64_t)k0 * (C / 4);
      for (int i = tid; i < n * (C / 4); i += kTileThreads) {
        *reinterpret_cast<float4*>(&sh.own_s[i / (C / 4)][4 * (i % (C / 4))]) = ssrc[i];
        *reinterpret_cast<float4*>(&sh.own_gb[i / (C / 4)][4 * (i % (C / 4))]) = gsrc[i];
      }
      const float4* g2src = reinterpret_cast<const float4*>(a.g2) + (uint64_t)k0 * (C * D / 4);
      for (int i = tid; i < n * (C * D / 4); i += kTileThreads)
        *reinterpret_cast<float4*>(&sh.own_g2[i / (C * D / 4)][4 * (i % (C * D / 4))]) = g2src[i];
    }
    for (int i = tid; i < kTileP * SH::kAccS; i += kTileThreads) (&sh.acc[0][0])[i] = 0.0f;
    __syncthreads();

    if (tid == 0) {  // prefix of the range lengths: the stencil rows concatenated in range order
      uint32_t run = 0;
      for (int rr = 0; rr < R; ++rr) {
        sh.pre[rr] = run;
        run += sh.rb[rr] - sh.ra[rr];
      }
      sh.pre[R] = run;
    }
    __syncthreads();
    const uint32_t nchunks = (sh.pre[R] + kTileRows - 1) / kTileRows;
    uint32_t nr_next = tile_chunk_rows(sh, R, 0, sh.gidx[0], tid);
    __syncthreads();
    TileStage<D, FULL> stage;
    stage.load(a, sh.gidx[0], nr_next, tid);

    for (uint32_t ck = 0;; ++ck) {
      const bool more = ck < nchunks;
      const uint32_t nr = nr_next;
      // ---- phase A: rows of chunk ck (loaded during the previous chunk)
      // into LDS; the next chunk's global rows; the previous chunk's slots
      if (more) {
        stage.store(sh, nr, tid);
        nr_next = tile_chunk_rows(sh, R, ck + 1, sh.gidx[(ck + 1) & 1], tid);
      }
      if (ck > 0) {
        const int32_t* cp = sh.cum[(ck - 1) & 1];
        const int32_t Pk = cp[n];
        const int32_t Rq = (Pk + kTileQuads - 1) / kTileQuads;
        for (int i = tid; i < n * SH::kAcc; i += kTileThreads) {
          const int p = i / SH::kAcc, x = i % SH::kAcc;
          const int32_t plo = cp[p], phi = cp[p + 1];
          if (phi <= plo) continue;
          float v = sh.acc[p][x];
          for (int32_t q = (plo + Rq - 1) / Rq; q * Rq < phi; ++q) v += sh.slot[q][x];
          sh.acc[p][x] = v;
        }
      }
      __syncthreads();
      if (!more) break;

      // ---- phase T: in-radius test of every (unit particle, chunk row),
      // compacted particle-major into sh.jl
      uint32_t mask = 0;
      if (tp < n) {
        float xi[3];
        unpack(sh.own_xw[tp], xi);
#pragma unroll
        for (int q = 0; q < kTestPer; ++q) {
          const uint32_t i = (uint32_t)(tsub + q * kTestSub);
          if (i < nr) {
            float xj[3], rr[3];
            unpack(sh.xw[i], xj);
            if (displacement<D, P>(g, xi, xj, rr) < g.eps2) mask |= 1u << q;
          }
        }
      }
      const uint32_t cnt = (uint32_t)__popc(mask);
      // exclusive scan of cnt over the workgroup in thread order (= particle-major)
      uint32_t incl = cnt;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t v = __shfl_up(incl, off, 64);
        if (lane >= off) incl += v;
      }
      if (lane == 63) sh.wtot[wave] = (int32_t)incl;
      __syncthreads();
      uint32_t base = 0;
      for (int w = 0; w < wave; ++w) base += (uint32_t)sh.wtot[w];
      uint32_t at = base + incl - cnt;
      int32_t* cum = sh.cum[ck & 1u];
      if (tsub == 0 && tp <= n) cum[tp] = (int32_t)at;  // tp == n: the total (its threads count 0)
      if (tid == kTileThreads - 1 && n == kTileP) cum[n] = (int32_t)(base + incl);
      while (mask) {
        const int q = __ffs(mask) - 1;
        mask &= mask - 1;
        sh.jl[at++] = (uint8_t)(tsub + q * kTestSub);
      }
      __syncthreads();

      // ---- phase B: the next chunk's rows start loading; the quads' runs of
      // this chunk's pairs
      stage.load(a, sh.gidx[(ck + 1) & 1], nr_next, tid);
      const int32_t Pk = cum[n];
      const int32_t Rq = (Pk + kTileQuads - 1) / kTileQuads;
      int32_t pi = quad * Rq;
      const int32_t pe = min(Pk, pi + Rq);
      if (pi < pe) {
        int p = 0;
        while (cum[p + 1] <= pi) ++p;
        const int pfirst = p;
        float xi[3], vi = 0.0f;
        float si[FULL ? CW : 1] = {}, gbi[FULL ? CW : 1] = {}, ggi[FULL ? CW * D : 1] = {};
        auto load_own = [&](int pp) {
          const float4 pw = sh.own_xw[pp];
          xi[0] = pw.x;
          xi[1] = pw.y;
          xi[2] = pw.z;
          vi = pw.w;
          if constexpr (FULL) {
            load_span<CW, true>(&sh.own_s[pp][c0], si);
            load_span<CW, true>(&sh.own_gb[pp][c0], gbi);
            load_span<CW * D, true>(&sh.own_g2[pp][c0 * D], ggi);
          }
        };
        load_own(p);
        float dsb[CW] = {}, dsg[CW] = {}, wsum[3] = {};
        float dxb[3] = {}, dxg[3] = {}, drg = 0.0f;
        auto flush = [&](int pp) {
          float* dst = (pp == pfirst) ? sh.slot[quad] : sh.acc[pp];
          const bool add = pp != pfirst;
#pragma unroll
          for (int f = 0; f < CW; ++f) {
            float* q1 = &dst[c0 + f];
            float* q2 = &dst[C + c0 + f];
            *q1 = add ? *q1 + dsb[f] : dsb[f];
            *q2 = add ? *q2 + dsg[f] : dsg[f];
            dsb[f] = 0.0f;
            dsg[f] = 0.0f;
          }
          constexpr int NR = FULL ? 10 : 3;
          float red[NR];
#pragma unroll
          for (int e = 0; e < 3; ++e) red[e] = wsum[e];  // identical in the four lanes
          if constexpr (FULL) {
#pragma unroll
            for (int e = 0; e < 3; ++e) {
              red[3 + e] = quad_sum(dxb[e]);
              red[6 + e] = quad_sum(dxg[e]);
            }
            red[9] = quad_sum(drg);
          }
          if (sl == 0) {
#pragma unroll
            for (int x = 0; x < NR; ++x) {
              float* q = &dst[2 * C + x];
              *q = add ? *q + red[x] : red[x];
            }
          }
#pragma unroll
          for (int e = 0; e < 3; ++e) {
            wsum[e] = 0.0f;
            dxb[e] = 0.0f;
            dxg[e] = 0.0f;
          }
          drg = 0.0f;
        };
        for (; pi < pe; ++pi) {
          if (pi >= cum[p + 1]) {
            flush(p);
            do {
              ++p;
            } while (cum[p + 1] <= pi);
            load_own(p);
          }
          const uint32_t jl = sh.jl[pi];
          const float4 pj = sh.xw[jl];
          float xj[3], rr[3], rbk[3];
          unpack(pj, xj);
          const float vj = pj.w;
          const float d2 = displacement<D, P>(g, xi, xj, rr);
          const float db = back_disp<D, P>(g, xi, xj, rr, d2, rbk);
          const float W = poly6(g.eps2, db);
          float d, dinv;
          const float mag = spiky_mag(g.eps, db, &d, &dinv);
          float w[3];
#pragma unroll
          for (int q = 0; q < D; ++q) {
            w[q] = mag * rbk[q];
            wsum[q] += vj * w[q];
          }
          float gbj[CW], ggj[CW * D];
          load_span<CW, true>(&sh.gb[jl][c0], gbj);
          load_span<CW * D, true>(&sh.g2[jl][c0 * D], ggj);
          if constexpr (!FULL) {
#pragma unroll
            for (int f = 0; f < CW; ++f) {
              dsb[f] += W * gbj[f];
#pragma unroll
              for (int q = 0; q < D; ++q) dsg[f] += ggj[f * D + q] * w[q];
            }
          } else {
            float t2 = 0.0f, ja = 0.0f, jb = 0.0f;
            if (db != 0.0f && db < g.eps2) {
              const float tt = g.eps2 - db;
              t2 = tt * tt;
              const float di = dinv;
              ja = 3.0f * (g.eps - d) * (g.eps - d) * di;
              jb = 3.0f * (g.eps2 - db) * di * di * di;
            }
            float sj[CW];
            load_span<CW, true>(&sh.s[jl][c0], sj);
            float A = 0.0f, Bv = 0.0f;
            float u1[D] = {}, u2[D] = {};
#pragma unroll
            for (int f = 0; f < CW; ++f) {
              dsb[f] += W * gbj[f];
              A += gbi[f] * sj[f];
              Bv += gbj[f] * si[f];
              const float df = si[f] - sj[f];
#pragma unroll
              for (int q = 0; q < D; ++q) {
                dsg[f] += ggj[f * D + q] * w[q];
                u1[q] += df * ggj[f * D + q];
                u2[q] += df * ggi[f * D + q];
              }
            }
            const float m6 = -6.0f * t2 * (A * vj + Bv * vi);
            float uu[D], uw = 0.0f, rv = 0.0f;
#pragma unroll
            for (int q = 0; q < D; ++q) {
              dxb[q] += m6 * rbk[q];
              uw += u1[q] * w[q];
              uu[q] = vi * u1[q] + vj * u2[q];
              rv += rbk[q] * uu[q];
            }
            drg += uw;
#pragma unroll
            for (int q = 0; q < D; ++q) dxg[q] += ja * uu[q] - jb * rbk[q] * rv;
          }
        }
        flush(p);
      }
      __syncthreads();
    }

    // ---- outputs of the unit's particles
    for (int i = tid; i < n * C; i += kTileThreads) {
      const int p = i / C, f = i % C;
      const uint32_t kk = k0 + (uint32_t)p;
      const float vi = sh.own_xw[p].w;
      float t = vi * sh.acc[p][C + f];
#pragma unroll
      for (int q = 0; q < D; ++q) t += a.g2[((uint64_t)kk * C + f) * D + q] * sh.acc[p][2 * C + q];
      a.out1[(uint64_t)kk * C + f] = sh.acc[p][f] * (vi * g.c6) + t * g.cs;
    }
    if constexpr (FULL) {
      if (tid < n) {
        const uint32_t kk = k0 + (uint32_t)tid;
        const float mi = a.m[kk], ri = a.rho[kk];
        const float mr2 = mi / (ri * ri);
        float drb = 0.0f;
        for (int f = 0; f < C; ++f) drb += sh.own_s[tid][f] * sh.acc[tid][f];
        a.out2[kk] = -mr2 * (drb * g.c6 + sh.acc[tid][2 * C + 9] * g.cs);
        float dx[D];
#pragma unroll
        for (int q = 0; q < D; ++q) dx[q] = sh.acc[tid][2 * C + 3 + q] * g.c6 + sh.acc[tid][2 * C + 6 + q] * g.cs;
        store_pos_grad<D>(a.out0, kk, dx, 1.0f);
      }
    }
    __syncthreads();
  }
}

}  // namespace pk
}  // namespace sphops
