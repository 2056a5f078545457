// Pass-B backward over the pairs inside one cell, each pair evaluated once
// for both of its ends (no reference counterpart: the reference evaluates
// every ordered pair from its target's side, sphops/sph_cuda.cu:723-1416).
//
// The list fill (FillTiles) keeps a tiled cell's own-cell entries at the end
// of its particles' rows; the lane-split list kernel skips them, and this
// kernel adds what those pairs contribute.  Both ends of such a pair lie in
// one cell, so the cell's rows fit in LDS, and the two directed pairs (i, j)
// and (j, i) share their geometry (r, W, the spiky magnitude and the
// Jacobian coefficients) and most of their channel products:
//   blur:      dL/ds_i += W g_j,          dL/ds_j += W g_i,
//              the dL/dx factor k6 t2 (v_j g_i.s_j + v_i g_j.s_i) is the same
//              for both ends, and r_b flips sign;
//   gradient:  dL/ds_i += g2_j . w,       dL/ds_j -= g2_i . w   (w = K r_b),
//              u_j = -u_i, u_j . r_b(j) = u_i . r_b(i), dL/dx_j = -dL/dx_i,
//              the dL/drho terms are u1 . w and u2 . w.
// (Variable names as in k_blur_hybrid_bwd_quad, whose directed terms these
// are.)  So one unordered pair costs about 0.65 of two directed ones in VALU
// work, and its neighbour rows come from LDS instead of L2.
//
// One workgroup (four waves) per cell of at most kCellMax particles, cells
// taken in turn from the fill's table.  The cell's particles are cut into
// blocks of 16, one particle per lane quad (four channel slices of four
// channels, C = 16).  Pairs of blocks follow a round-robin tournament: in
// each round every block is in at most one pair, so the four waves never
// touch the same accumulators; a barrier separates rounds.  A wave serving
// blocks (A, B) keeps A's rows and A's accumulators in registers and takes
// B's rows from LDS, pairing quad q with particle (q + t) mod 16 of B at
// step t: within a step the B particles are distinct, so each quad adds its
// j-side terms to B's LDS accumulators with a plain read-modify-write, and a
// wave's LDS operations complete in issue order.  The pairs inside one block
// (the diagonal) take steps t = 1 .. 8 (t = 8 for the first eight quads
// only) and the self pair at t = 0.  Every sum is taken in a fixed order:
// results are deterministic.  The outputs, already written by the list
// kernel, receive the cell's contributions for the particles whose rows
// skipped their own cell (own[k] > 0).
#pragma once

namespace sphops {
namespace pk {

// Cells of 16 to 64 particles (the best of the thresholds measured at cfg5:
// 8-128 with two workgroups per CU, 16-128, and 16-64 with four).
constexpr int kCellMax = 64;         // particles per tiled cell (4 blocks of 16)
constexpr int kCellMin = 16;         // cells with fewer particles keep their pairs in the list
constexpr int kCellThreads = 256;    // four waves: up to four block pairs per round
constexpr uint32_t kCellWorkgroups = 1024;

template <int D, bool FULL, int PARTS>
struct CellLds {
  static constexpr bool kB = (PARTS & 1) != 0, kG = (PARTS & 2) != 0;
  static constexpr int kNG = D;  // float4 pieces of a particle's upstream2 slice (4 channels x D)
  float4 xv[kCellMax];                                // (x, y, z, m / rho)
  float4 s[FULL ? kCellMax * 4 : 1];                  // [p * 4 + slice]
  float4 gb[kB ? kCellMax * 4 : 1];
  float4 gg[kG ? kNG : 1][kG ? kCellMax * 4 : 1];     // piece m of [p * 4 + slice]
  float4 dsb[kB ? kCellMax * 4 : 1];                  // j-side accumulators, per slice
  float4 dsg[kG ? kCellMax * 4 : 1];
  float4 dxr[FULL ? kCellMax * 4 : 1];                // (dL/dx partial, dL/drho gradient partial)
  float4 ws[kG ? kCellMax * 4 : 1];                   // (sum v K, 0); equal in every slice
};

// Block-pair work of one wave: A's particle i = 16 A + q in registers
// against B's particles (B == A: the diagonal).
template <int D, bool FULL, int PARTS>
__device__ __forceinline__ void cell_block_pair(const GridParams& g, CellLds<D, FULL, PARTS>& L, uint32_t n, int A,
                                                int B, float k6) {
  constexpr bool kB = (PARTS & 1) != 0, kG = (PARTS & 2) != 0;
  constexpr int CW = 4;
  const int lane = __lane_id();
  const int q = lane >> 2, slice = lane & 3;
  const uint32_t i = (uint32_t)(16 * A + q);
  if (i >= n) return;
  const bool diag = A == B;
  const uint32_t si4 = i * 4 + slice;
  const float4 pxi = L.xv[i];
  const float xi[3] = {pxi.x, pxi.y, pxi.z};
  const float vi = pxi.w;
  float si[FULL ? CW : 1] = {}, gbi[kB ? CW : 1] = {}, ggi[kG ? CW * D : 1] = {};
  if constexpr (FULL) {
    const float4 t = L.s[si4];
    si[0] = t.x; si[1] = t.y; si[2] = t.z; si[3] = t.w;
  }
  if constexpr (kB) {
    const float4 t = L.gb[si4];
    gbi[0] = t.x; gbi[1] = t.y; gbi[2] = t.z; gbi[3] = t.w;
  }
  if constexpr (kG) {
#pragma unroll
    for (int m = 0; m < D; ++m) {
      const float4 t = L.gg[m][si4];
      ggi[4 * m + 0] = t.x; ggi[4 * m + 1] = t.y; ggi[4 * m + 2] = t.z; ggi[4 * m + 3] = t.w;
    }
  }
  float dsb[CW] = {}, dsg[CW] = {}, dxm[D] = {}, wsum[D] = {};
  float drg = 0.0f;
  const int steps = diag ? 9 : 16;
  for (int t = 0; t < steps; ++t) {
    const uint32_t j = (uint32_t)(16 * B + ((q + t) & 15));
    if (j >= n || (diag && t == 8 && q >= 8)) continue;
    const bool jside = !(diag && t == 0);  // the self pair adds to i once
    const uint32_t sj4 = j * 4 + slice;
    const float4 pxj = L.xv[j];
    const float xj[3] = {pxj.x, pxj.y, pxj.z};
    const float vj = pxj.w;
    float sj[FULL ? CW : 1] = {}, gbj[kB ? CW : 1] = {}, ggj[kG ? CW * D : 1] = {};
    if constexpr (FULL) {
      const float4 u = L.s[sj4];
      sj[0] = u.x; sj[1] = u.y; sj[2] = u.z; sj[3] = u.w;
    }
    if constexpr (kB) {
      const float4 u = L.gb[sj4];
      gbj[0] = u.x; gbj[1] = u.y; gbj[2] = u.z; gbj[3] = u.w;
    }
    if constexpr (kG) {
#pragma unroll
      for (int m = 0; m < D; ++m) {
        const float4 u = L.gg[m][sj4];
        ggj[4 * m + 0] = u.x; ggj[4 * m + 1] = u.y; ggj[4 * m + 2] = u.z; ggj[4 * m + 3] = u.w;
      }
    }
    // geometry (the directed pair (i, j) of the list kernel: rb = x_i - x_j)
    float r[3] = {0.0f, 0.0f, 0.0f}, rb[3] = {0.0f, 0.0f, 0.0f};
    const float d2 = displacement<D, false>(g, xi, xj, r);
    const bool inr = d2 < g.eps2;  // the fill's test: the pair is in i's and j's rows
#pragma unroll
    for (int e = 0; e < D; ++e) rb[e] = -r[e];
    float d, dinv;
    const float mag = spiky_mag(g.eps, d2, &d, &dinv);
    const bool jac = inr && d2 != 0.0f;
    const float W = inr ? poly6(g.eps2, d2) : 0.0f;
    const float tt = g.eps2 - d2;
    const float t2 = jac ? tt * tt : 0.0f;
    const float ja = jac ? 3.0f * (g.eps - d) * (g.eps - d) * dinv : 0.0f;
    const float jb = jac ? 3.0f * tt * dinv * dinv * dinv : 0.0f;
    float w[D];
#pragma unroll
    for (int e = 0; e < D; ++e) w[e] = inr ? mag * rb[e] : 0.0f;
    // j-side accumulators
    float4 ab = make_float4(0.0f, 0.0f, 0.0f, 0.0f), ag = ab, ax = ab, aw = ab;
    if (jside) {
      if constexpr (kB) ab = L.dsb[sj4];
      if constexpr (kG) {
        ag = L.dsg[sj4];
        aw = L.ws[sj4];
      }
      if constexpr (FULL) ax = L.dxr[sj4];
    }
    float jb4[CW] = {ab.x, ab.y, ab.z, ab.w}, jg4[CW] = {ag.x, ag.y, ag.z, ag.w};
    float jx[4] = {ax.x, ax.y, ax.z, ax.w};
    float coef = 0.0f;
    if constexpr (kB) {
      float Av = 0.0f, Bv = 0.0f;
#pragma unroll
      for (int f = 0; f < CW; ++f) {
        dsb[f] += W * gbj[f];
        jb4[f] += W * gbi[f];
        if constexpr (FULL) {
          Av += gbi[f] * sj[f];
          Bv += gbj[f] * si[f];
        }
      }
      if constexpr (FULL) coef = k6 * t2 * (Av * vj + Bv * vi);
    }
    float dxp[D] = {};  // dL/dx term of the pair for i (j receives its negative)
    if constexpr (kG) {
      float u1[D] = {}, u2[D] = {};
#pragma unroll
      for (int f = 0; f < CW; ++f) {
        float df = 0.0f;
        if constexpr (FULL) df = si[f] - sj[f];
#pragma unroll
        for (int e = 0; e < D; ++e) {
          dsg[f] += ggj[f * D + e] * w[e];
          jg4[f] -= ggi[f * D + e] * w[e];
          if constexpr (FULL) {
            u1[e] += df * ggj[f * D + e];
            u2[e] += df * ggi[f * D + e];
          }
        }
      }
#pragma unroll
      for (int e = 0; e < D; ++e) {
        wsum[e] += vj * w[e];
      }
      aw.x -= vi * w[0];
      aw.y -= vi * w[1];
      if constexpr (D == 3) aw.z -= vi * w[2];
      if constexpr (FULL) {
        float u[D], uw = 0.0f, uw2 = 0.0f, rv = 0.0f;
#pragma unroll
        for (int e = 0; e < D; ++e) {
          uw += u1[e] * w[e];
          uw2 += u2[e] * w[e];
          u[e] = vi * u1[e] + vj * u2[e];
          rv += rb[e] * u[e];
        }
        drg += uw;
        jx[3] += uw2;
        coef -= jb * rv;
#pragma unroll
        for (int e = 0; e < D; ++e) dxp[e] = ja * u[e] + coef * rb[e];
      }
    } else if constexpr (FULL) {
#pragma unroll
      for (int e = 0; e < D; ++e) dxp[e] = coef * rb[e];
    }
    if constexpr (FULL) {
#pragma unroll
      for (int e = 0; e < D; ++e) {
        dxm[e] += dxp[e];
        jx[e] -= dxp[e];
      }
    }
    if (jside) {
      if constexpr (kB) L.dsb[sj4] = make_float4(jb4[0], jb4[1], jb4[2], jb4[3]);
      if constexpr (kG) {
        L.dsg[sj4] = make_float4(jg4[0], jg4[1], jg4[2], jg4[3]);
        L.ws[sj4] = aw;
      }
      if constexpr (FULL) L.dxr[sj4] = make_float4(jx[0], jx[1], D == 3 ? jx[2] : 0.0f, jx[3]);
    }
  }
  // i's register sums into its accumulators (no other wave touches block A
  // in this round; this wave's own j-side updates of A came before)
  if constexpr (kB) {
    float4 v = L.dsb[si4];
    v.x += dsb[0]; v.y += dsb[1]; v.z += dsb[2]; v.w += dsb[3];
    L.dsb[si4] = v;
  }
  if constexpr (kG) {
    float4 v = L.dsg[si4];
    v.x += dsg[0]; v.y += dsg[1]; v.z += dsg[2]; v.w += dsg[3];
    L.dsg[si4] = v;
    float4 ws = L.ws[si4];
    ws.x += wsum[0]; ws.y += wsum[1];
    if constexpr (D == 3) ws.z += wsum[2];
    L.ws[si4] = ws;
  }
  if constexpr (FULL) {
    float4 v = L.dxr[si4];
    v.x += dxm[0]; v.y += dxm[1];
    if constexpr (D == 3) v.z += dxm[2];
    v.w += drg;
    L.dxr[si4] = v;
  }
}

// PARTS and FULL as for k_blur_hybrid_bwd_quad (C = 16, clamped grids).
template <int D, bool FULL, int PARTS>
__global__ __launch_bounds__(kCellThreads, 4) void k_cell_pairs_bwd(GridParams g, OpPtrs a) {
  constexpr bool kB = (PARTS & 1) != 0, kG = (PARTS & 2) != 0;
  constexpr int CW = 4;
  __shared__ CellLds<D, FULL, PARTS> L;
  const uint32_t ncells = (uint32_t)*a.cell_count;
  const int tid = threadIdx.x, wv = tid >> 6;
  const float k6 = kG ? -6.0f * (g.c6 / g.cs) : -6.0f;
  const float4* __restrict__ s4 = reinterpret_cast<const float4*>(a.s);
  const float4* __restrict__ g4 = reinterpret_cast<const float4*>(a.g);
  const float4* __restrict__ gg4 = reinterpret_cast<const float4*>(a.g2);
  for (uint32_t c = blockIdx.x; c < ncells; c += gridDim.x) {
    const uint2 cd = a.cells[c];
    const uint32_t cs = cd.x, n = cd.y;
    // stage the cell's rows (contiguous in the binned arrays) and clear the
    // accumulators
    for (uint32_t e = tid; e < n; e += kCellThreads) L.xv[e] = a.xw[cs + e];
    for (uint32_t e = tid; e < 4 * n; e += kCellThreads) {
      if constexpr (FULL) L.s[e] = s4[(uint64_t)cs * 4 + e];
      if constexpr (kB) {
        L.gb[e] = g4[(uint64_t)cs * 4 + e];
        L.dsb[e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
      if constexpr (kG) {
        L.dsg[e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        L.ws[e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
      if constexpr (FULL) L.dxr[e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if constexpr (kG) {
      for (uint32_t e = tid; e < 4 * D * n; e += kCellThreads) L.gg[e % D][e / D] = gg4[(uint64_t)cs * 4 * D + e];
    }
    __syncthreads();
    // rounds of the tournament over nb blocks (nb odd: a dummy player, whose
    // partner serves its own block's pairs that round; nb even: a last round
    // for the diagonals)
    const int nb = (int)((n + 15) >> 4);
    const int np = nb + (nb & 1), m = np - 1;
    for (int r = 0; r < m; ++r) {
      if (wv < np / 2) {
        int A = wv == 0 ? r : (r + wv) % m;
        int B = wv == 0 ? m : (r - wv + m) % m;
        if (A == nb) A = B;
        if (B == nb) B = A;
        cell_block_pair<D, FULL, PARTS>(g, L, n, A, B, k6);
      }
      __syncthreads();
    }
    if ((nb & 1) == 0) {
      for (int A = wv; A < nb; A += kCellThreads / kWave) cell_block_pair<D, FULL, PARTS>(g, L, n, A, A, k6);
      __syncthreads();
    }
    // add the cell's sums to the outputs of the particles whose rows skipped
    // their own cell; four adjacent lanes hold one particle's slices
    for (uint32_t e = tid; e < 4 * ((n + 15) & ~15u); e += kCellThreads) {
      const uint32_t p = e >> 2;
      const int slice = (int)(e & 3);
      const bool live = p < n && a.nown[cs + p] > 0;
      const uint32_t k = cs + p;
      float drb = 0.0f, drg = 0.0f, dx[D] = {};
      if (p < n) {
        const float vi = L.xv[p].w;
        float o[CW] = {};
        if constexpr (kB) {
          const float4 b = L.dsb[e];
          const float sb = vi * g.c6;
          o[0] = b.x * sb; o[1] = b.y * sb; o[2] = b.z * sb; o[3] = b.w * sb;
          if constexpr (FULL) {
            const float4 si = L.s[e];
            drb = si.x * b.x + si.y * b.y + si.z * b.z + si.w * b.w;
          }
        }
        if constexpr (kG) {
          const float4 gs = L.dsg[e];
          const float4 ws = L.ws[p * 4];  // slice 0's copy
          const float dsgv[CW] = {gs.x, gs.y, gs.z, gs.w};
          const float wsv[3] = {ws.x, ws.y, ws.z};
          float ggi[CW * D];
#pragma unroll
          for (int mm = 0; mm < D; ++mm) {
            const float4 t = L.gg[mm][e];
            ggi[4 * mm + 0] = t.x; ggi[4 * mm + 1] = t.y; ggi[4 * mm + 2] = t.z; ggi[4 * mm + 3] = t.w;
          }
#pragma unroll
          for (int f = 0; f < CW; ++f) {
            float tv = vi * dsgv[f];
#pragma unroll
            for (int d = 0; d < D; ++d) tv += ggi[f * D + d] * wsv[d];
            o[f] = kB ? o[f] + tv * g.cs : tv * g.cs;
          }
        }
        if (live) {
          float4* out1 = reinterpret_cast<float4*>(a.out1) + (uint64_t)k * 4 + slice;
          float4 v = *out1;
          v.x += o[0]; v.y += o[1]; v.z += o[2]; v.w += o[3];
          *out1 = v;
        }
        if constexpr (FULL) {
          const float4 xr = L.dxr[e];
          dx[0] = xr.x; dx[1] = xr.y;
          if constexpr (D == 3) dx[2] = xr.z;
          drg = xr.w;
        }
      }
      if constexpr (FULL) {
        // sums over the four slices (lanes 4p .. 4p + 3)
        drb += quad_get<1>(drb) + quad_get<2>(drb) + quad_get<3>(drb);
        drg += quad_get<1>(drg) + quad_get<2>(drg) + quad_get<3>(drg);
#pragma unroll
        for (int d = 0; d < D; ++d) dx[d] += quad_get<1>(dx[d]) + quad_get<2>(dx[d]) + quad_get<3>(dx[d]);
        if (live && slice == 0) {
          const float mi = a.m[k], ri = a.rho[k];
          const float mr2 = mi / (ri * ri);
          float dr = 0.0f;
          if constexpr (kB) dr = drb * g.c6;
          if constexpr (kG) dr = kB ? dr + drg * g.cs : drg * g.cs;
          a.out2[k] += -mr2 * dr;
          store_pos_grad<D, true>(a.out0, k, dx, kG ? g.cs : g.c6);
        }
      }
    }
    __syncthreads();  // before the next cell overwrites the LDS
  }
}

}  // namespace pk
}  // namespace sphops
