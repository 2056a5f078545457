// SPH neighbour perception kernels (forward and gather-form backward) for gfx950.
//
// One lane owns one binned particle i and writes only i's outputs: no atomics,
// deterministic results.  Neighbour data is read through a packed float4 per
// particle (x, y, z|0, weight), weight = mass or mass/rho depending on the
// operator, so one 16-byte load gives a neighbour's position and weight.
//
// Three traversals of i's neighbours:
//  * kList     — walk i's precomputed in-radius list (row nptr[i], ncnt[i]
//                entries, built once per snapshot by the fill kernel below);
//                no distance tests, no divergence beyond list length.
//  * kStencil  — test every candidate of the 3^D cell stencil, four loads in
//                flight per lane, and call the operator for in-radius pairs.
//  * kStencil2 — the same scan, but in-radius neighbours are first appended to
//                the lane's column of a per-wave LDS list and processed after,
//                so channel loops run with the wave converged.
// The stencil is read as contiguous slices of the sorted arrays through
// bin_offsets: in grid mode 3^(D-1) rows of up to three x-adjacent cells (plus
// the periodic wrap cell), as the reference traverses them
// (sphops/sph_cuda.cu:1561-1640); in particle mode the 3^D Morton cells
// (sphops/sph_cuda.cu:324-346).  Operator formulas are the reference's
// (sphops/sph_cuda.cu:218-721, 1160-1375; sphops/utils.cuh:199-279) with
// per-pair work hoisted out of the channel loops.
#pragma once

#include "sphops_internal.hpp"

#include <type_traits>

namespace sphops {
namespace pk {

constexpr int kThreads = 256;
constexpr int kCap = 32;

enum Trav { kList = 0, kStencil = 1, kStencil2 = 2 };
enum Weight { kWNone = 0, kWMass = 1, kWVolume = 2 };

// ------------------------------------------------------------- traversal

template <int D, bool PERIODIC>
struct Walker {
  int c[3];
  uint32_t base;  // b * G
  int r;          // next range to fetch
  uint32_t j, jend;

  static constexpr int kRowRanges = (D == 2 ? 3 : 9) * (PERIODIC ? 2 : 1);
  static constexpr int kCellRanges = (D == 2 ? 9 : 27);

  __device__ __forceinline__ void init(const GridParams& g, const float* xi, uint32_t k) {
    pos2cell<D, PERIODIC>(g, xi, c);
    base = (k / g.N) * g.G;
    r = 0;
    j = 0;
    jend = 0;
  }

  __device__ __forceinline__ bool fetch(const GridParams& g, const int32_t* __restrict__ bo, int rr) {
    int nc[3] = {c[0], c[1], D == 3 ? c[2] : 0};
    if (!g.morton) {
      if (rr >= kRowRanges) return false;
      const int row = PERIODIC ? (rr >> 1) : rr;
      const int chunk = PERIODIC ? (rr & 1) : 0;
      j = jend = 0;
      if constexpr (D == 2) {
        nc[1] = c[1] + row - 1;
      } else {
        nc[1] = c[1] + row % 3 - 1;
        nc[2] = c[2] + row / 3 - 1;
      }
#pragma unroll
      for (int d = 1; d < D; ++d) {
        if (PERIODIC) {
          nc[d] = bound_axis(nc[d], g.gs[d], true);
        } else if (nc[d] < 0 || nc[d] >= g.gs[d]) {
          return true;
        }
      }
      int x0, x1;
      if (chunk == 0) {
        x0 = max(0, c[0] - 1);
        x1 = min(g.gs[0] - 1, c[0] + 1);
      } else if (c[0] == 0) {
        x0 = x1 = g.gs[0] - 1;
      } else if (c[0] == g.gs[0] - 1) {
        x0 = x1 = 0;
      } else {
        return true;
      }
      nc[0] = x0;
      const uint32_t h0 = cell_hash<D>(g, nc);
      const uint32_t h1 = h0 + (uint32_t)(x1 - x0);
      j = (uint32_t)bo[base + h0];
      jend = (uint32_t)bo[base + h1 + 1];
      return true;
    }
    if (rr >= kCellRanges) return false;
    j = jend = 0;
    nc[0] = c[0] + rr % 3 - 1;
    nc[1] = c[1] + (rr / 3) % 3 - 1;
    if constexpr (D == 3) nc[2] = c[2] + rr / 9 - 1;
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (PERIODIC) {
        nc[d] = bound_axis(nc[d], g.gs[d], true);
      } else if (nc[d] < 0 || nc[d] >= g.gs[d]) {
        return true;
      }
    }
    const uint32_t h = cell_hash<D>(g, nc);
    j = (uint32_t)bo[base + h];
    jend = (uint32_t)bo[base + h + 1];
    return true;
  }

  // Position on the next candidate; false once the stencil is exhausted.
  __device__ __forceinline__ bool next(const GridParams& g, const int32_t* __restrict__ bo) {
    while (j >= jend) {
      if (!fetch(g, bo, r)) return false;
      ++r;
    }
    return true;
  }
};

// ------------------------------------------------------------- row loads

template <int N, bool VEC>
__device__ __forceinline__ void load_span(const float* __restrict__ p, float* v) {
  if constexpr (VEC) {
    const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int u = 0; u < N / 4; ++u) {
      const float4 t = q[u];
      v[4 * u + 0] = t.x;
      v[4 * u + 1] = t.y;
      v[4 * u + 2] = t.z;
      v[4 * u + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int u = 0; u < N; ++u) v[u] = p[u];
  }
}

// CM channels in registers; EXACT means C == CM (rows loaded as 16-byte
// vectors when CM % 4 == 0), otherwise C <= CM with predication.
template <int CM, bool EXACT>
struct Chan {
  static constexpr bool kVec = EXACT && (CM % 4 == 0);
  __device__ static __forceinline__ uint32_t stride(uint32_t C) { return EXACT ? (uint32_t)CM : C; }
  __device__ static __forceinline__ void load(const float* __restrict__ p, uint64_t row, uint32_t C, float* v) {
    if constexpr (EXACT) {
      load_span<CM, kVec>(p + row * CM, v);
    } else {
#pragma unroll
      for (int f = 0; f < CM; ++f) v[f] = (f < (int)C) ? p[row * C + f] : 0.0f;
    }
  }
  template <int D>
  __device__ static __forceinline__ void load_cd(const float* __restrict__ p, uint64_t row, uint32_t C, float* v) {
    if constexpr (EXACT) {
      load_span<CM * D, (CM * D) % 4 == 0 && kVec>(p + row * CM * D, v);
    } else {
#pragma unroll
      for (int f = 0; f < CM * D; ++f) v[f] = (f < (int)C * D) ? p[row * C * D + f] : 0.0f;
    }
  }
};

// Backward outputs: store, or (ACC) add to what an earlier launch on the
// same stream stored; each element has one owning lane.
template <bool ACC>
__device__ __forceinline__ void put(float* __restrict__ out, uint64_t i, float v) {
  if constexpr (ACC) v += out[i];
  out[i] = v;
}

template <int D, bool ACC = false>
__device__ __forceinline__ void store_pos_grad(float* __restrict__ out, uint32_t k, const float* v, float scale) {
  if constexpr (D == 2) {
    float2 o = make_float2(v[0] * scale, v[1] * scale);
    if constexpr (ACC) {
      const float2 p = reinterpret_cast<const float2*>(out)[k];
      o.x += p.x;
      o.y += p.y;
    }
    reinterpret_cast<float2*>(out)[k] = o;
  } else {
    float4 o = make_float4(v[0] * scale, v[1] * scale, v[2] * scale, 0.0f);
    if constexpr (ACC) {
      const float4 p = reinterpret_cast<const float4*>(out)[k];
      o.x += p.x;
      o.y += p.y;
      o.z += p.z;
    }
    reinterpret_cast<float4*>(out)[k] = o;
  }
}

// Adjugate inverse of a symmetric 2x2 / 3x3 matrix read from its upper
// triangle, identity when |det| < tol (sphops/sph_cuda.cu:3095-3179).
template <int D>
__device__ __forceinline__ void safe_inv_sym(const float* M, float tol, float* L) {
  if constexpr (D == 2) {
    const float a = M[0], b = M[1], d = M[3];
    const float det = a * d - b * b;
    if (fabsf(det) < tol) {
      L[0] = 1.0f; L[1] = 0.0f; L[2] = 0.0f; L[3] = 1.0f;
      return;
    }
    const float id = 1.0f / det;
    L[0] = d * id; L[1] = -b * id; L[2] = -b * id; L[3] = a * id;
  } else {
    const float a = M[0], b = M[1], c = M[2], d = M[4], e = M[5], f = M[8];
    const float t1 = d * f - e * e, t2 = c * e - b * f, t3 = b * e - c * d;
    const float det = a * t1 + b * t2 + c * t3;
    if (fabsf(det) < tol) {
#pragma unroll
      for (int q = 0; q < 9; ++q) L[q] = (q % 4 == 0) ? 1.0f : 0.0f;
      return;
    }
    const float id = 1.0f / det;
    const float u = (b * c - a * e) * id;
    L[0] = t1 * id; L[1] = t2 * id; L[2] = t3 * id;
    L[3] = t2 * id; L[4] = (a * f - c * c) * id; L[5] = u;
    L[6] = t3 * id; L[7] = u; L[8] = (a * d - b * b) * id;
  }
}

// displacement x_i - x_j as the reference's backward evaluates it
template <int D, bool P>
__device__ __forceinline__ float back_disp(const GridParams& g, const float* xi, const float* xj, const float* r_fwd,
                                           float d2_fwd, float* rb) {
  if constexpr (!P) {
#pragma unroll
    for (int e = 0; e < D; ++e) rb[e] = -r_fwd[e];
    return d2_fwd;
  } else {
    return displacement<D, P>(g, xj, xi, rb);
  }
}

// Sum over aligned groups of G lanes (G a wave-uniform power of two <= 64),
// delivered to each group's first lane; the other lanes keep partial sums.
// A fixed tree: lane i adds lane i+1, then i+2, i+4, ... (DPP row_shl inside
// 16-lane rows, with no LDS round trip; a bpermute for the 16 and 32 steps).
// Every step shuffles all accumulators before adding, so the shuffles of one
// step overlap.  The order is fixed, so results are deterministic.
template <int STEP>
__device__ __forceinline__ float grp_fetch(float v) {
  if constexpr (STEP < 16) {
    // DPP row_shl:STEP (0x100 + STEP), all rows and banks, 0 past the row end
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x100 + STEP, 0xF, 0xF, true));
  } else {
    return __shfl_down(v, STEP, kWave);
  }
}

template <int STEP>
__device__ __forceinline__ void grp_add(float& v) { v += grp_fetch<STEP>(v); }

template <int STEP, int N>
__device__ __forceinline__ void grp_add(float (&v)[N]) {
  float t[N];
#pragma unroll
  for (int q = 0; q < N; ++q) t[q] = grp_fetch<STEP>(v[q]);
#pragma unroll
  for (int q = 0; q < N; ++q) v[q] += t[q];
}

template <class... A>
__device__ __forceinline__ void grp_sum(int G, A&... v) {
  if (G > 1) (grp_add<1>(v), ...);
  if (G > 2) (grp_add<2>(v), ...);
  if (G > 4) (grp_add<4>(v), ...);
  if (G > 8) (grp_add<8>(v), ...);
  if (G > 16) (grp_add<16>(v), ...);
  if (G > 32) (grp_add<32>(v), ...);
}

// ------------------------------------------------------------- operators
//
// Interface: init(g, a, k) at the owning lane, pair(g, a, xi, xj, wj, r, d2, j)
// for every in-radius neighbour j (r = x_j - x_i wrapped, d2 = |r|^2 in fp32,
// wj = the packed weight of j), finish(g, a, k).  kWeightKind selects what the
// packed float4 carries in .w.

template <int D, bool P>
struct OpCount {
  static constexpr int kWeightKind = kWNone;
  static constexpr bool kChannels = false;
  float acc = 0.0f;
  __device__ void init(const GridParams&, const OpPtrs&, uint32_t) {}
  __device__ void pair(const GridParams&, const OpPtrs&, const float*, const float*, float, const float*, float,
                       uint32_t) {
    acc += 1.0f;
  }
  __device__ void reduce(int G) { (void)G; }
  __device__ void finish(const GridParams&, const OpPtrs& a, uint32_t k) { a.out0[k] = acc; }
};

template <int D, bool P>
struct OpDensity {
  static constexpr int kWeightKind = kWMass;
  static constexpr bool kChannels = false;
  float acc = 0.0f;
  __device__ void init(const GridParams&, const OpPtrs&, uint32_t) {}
  __device__ void pair(const GridParams& g, const OpPtrs&, const float*, const float*, float wj, const float*,
                       float d2, uint32_t) {
    acc += poly6(g.eps2, d2) * wj;
  }
  __device__ void reduce(int G) { grp_sum(G, acc); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) { a.out0[k] = acc * g.c6; }
};

template <int D, bool P>
struct OpDensityGradient {
  static constexpr int kWeightKind = kWMass;
  static constexpr bool kChannels = false;
  float acc[D] = {};
  __device__ void init(const GridParams&, const OpPtrs&, uint32_t) {}
  __device__ void pair(const GridParams& g, const OpPtrs&, const float*, const float*, float wj, const float* r,
                       float d2, uint32_t) {
    float d;
    const float t = spiky_mag(g.eps, d2, &d) * wj;
#pragma unroll
    for (int e = 0; e < D; ++e) acc[e] += t * r[e];
  }
  __device__ void reduce(int G) { grp_sum(G, acc); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) {
#pragma unroll
    for (int e = 0; e < D; ++e) a.out0[(uint64_t)k * D + e] = acc[e] * g.cs;
  }
};

template <int D, bool P>
struct OpMomentMatrix {
  static constexpr int kWeightKind = kWVolume;
  static constexpr bool kChannels = false;
  float acc[D * D] = {};
  __device__ void init(const GridParams&, const OpPtrs&, uint32_t) {}
  __device__ void pair(const GridParams& g, const OpPtrs&, const float*, const float*, float wj, const float* r,
                       float d2, uint32_t) {
    float d;
    const float t = spiky_mag(g.eps, d2, &d) * wj;
#pragma unroll
    for (int p = 0; p < D; ++p)
#pragma unroll
      for (int q = 0; q < D; ++q) acc[p * D + q] += t * r[p] * r[q];
  }
  __device__ void reduce(int G) { grp_sum(G, acc); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) {
#pragma unroll
    for (int q = 0; q < D * D; ++q) a.out0[(uint64_t)k * D * D + q] = acc[q] * g.cs;
  }
};

template <int D, bool P, int CM, bool EX>
struct OpBlur {
  static constexpr int kWeightKind = kWVolume;
  static constexpr bool kChannels = true;
  using Ch = Chan<CM, EX>;
  float acc[CM] = {};
  __device__ void init(const GridParams&, const OpPtrs&, uint32_t) {}
  __device__ void pair(const GridParams& g, const OpPtrs& a, const float*, const float*, float wj, const float*,
                       float d2, uint32_t j) {
    const float w = poly6(g.eps2, d2) * wj;
    float sj[CM];
    Ch::load(a.s, j, a.C, sj);
#pragma unroll
    for (int f = 0; f < CM; ++f) acc[f] += w * sj[f];
  }
  __device__ void reduce(int G) { grp_sum(G, acc); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) {
    const uint32_t C = EX ? CM : a.C;
#pragma unroll
    for (int f = 0; f < CM; ++f)
      if (f < (int)C) a.out0[(uint64_t)k * Ch::stride(a.C) + f] = acc[f] * g.c6;
  }
};

template <int D, bool P, int CM, bool EX>
struct OpGradient {
  static constexpr int kWeightKind = kWVolume;
  static constexpr bool kChannels = true;
  using Ch = Chan<CM, EX>;
  float si[CM];
  float acc[CM * D] = {};
  __device__ void init(const GridParams&, const OpPtrs& a, uint32_t k) { Ch::load(a.s, k, a.C, si); }
  __device__ void pair(const GridParams& g, const OpPtrs& a, const float*, const float*, float wj, const float* r,
                       float d2, uint32_t j) {
    float d;
    const float t = spiky_mag(g.eps, d2, &d) * wj;
    float sj[CM];
    Ch::load(a.s, j, a.C, sj);
#pragma unroll
    for (int f = 0; f < CM; ++f) {
      const float q = t * (sj[f] - si[f]);
#pragma unroll
      for (int e = 0; e < D; ++e) acc[f * D + e] += q * r[e];
    }
  }
  __device__ void reduce(int G) { grp_sum(G, acc); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) {
    const uint32_t C = EX ? CM : a.C;
#pragma unroll
    for (int f = 0; f < CM * D; ++f)
      if (f < (int)(C * D)) a.out0[(uint64_t)k * Ch::stride(a.C) * D + f] = acc[f] * g.cs;
  }
};

// gradient_hybrid forward fused: raw gradient and moment matrix in one sweep,
// then raw @ safe_inv(M) in registers (sphops/sph.py:474-484).
template <int D, bool P, int CM, bool EX>
struct OpGradientHybrid {
  static constexpr int kWeightKind = kWVolume;
  static constexpr bool kChannels = true;
  using Ch = Chan<CM, EX>;
  float si[CM];
  float acc[CM * D] = {};
  float M[D * D] = {};
  __device__ void init(const GridParams&, const OpPtrs& a, uint32_t k) { Ch::load(a.s, k, a.C, si); }
  __device__ void pair(const GridParams& g, const OpPtrs& a, const float*, const float*, float wj, const float* r,
                       float d2, uint32_t j) {
    float d;
    const float t = spiky_mag(g.eps, d2, &d) * wj;
#pragma unroll
    for (int p = 0; p < D; ++p)
#pragma unroll
      for (int q = p; q < D; ++q) M[p * D + q] += t * r[p] * r[q];
    float sj[CM];
    Ch::load(a.s, j, a.C, sj);
#pragma unroll
    for (int f = 0; f < CM; ++f) {
      const float q = t * (sj[f] - si[f]);
#pragma unroll
      for (int e = 0; e < D; ++e) acc[f * D + e] += q * r[e];
    }
  }
  __device__ void reduce(int G) { grp_sum(G, acc, M); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) {
    float Ms[D * D], L[D * D];
#pragma unroll
    for (int p = 0; p < D; ++p)
#pragma unroll
      for (int q = 0; q < D; ++q) Ms[p * D + q] = (q >= p ? M[p * D + q] : M[q * D + p]) * g.cs;
    safe_inv_sym<D>(Ms, a.tol, L);
    const uint32_t C = EX ? CM : a.C;
#pragma unroll
    for (int f = 0; f < CM; ++f) {
      if (f >= (int)C) continue;
      float raw[D];
#pragma unroll
      for (int e = 0; e < D; ++e) raw[e] = acc[f * D + e] * g.cs;
#pragma unroll
      for (int e = 0; e < D; ++e) {
        float o = 0.0f;
#pragma unroll
        for (int q = 0; q < D; ++q) o += raw[q] * L[q * D + e];
        a.out0[(uint64_t)k * Ch::stride(a.C) * D + f * D + e] = o;
      }
    }
  }
};

// ------------------------------------------------------- fused forward
//
// Operators that share a neighbour pass: density with density gradient
// (both weighted by mass), blur with gradient_hybrid (both weighted by
// volume m/rho and both reading s_j).  out0 gets the first, out3 the second.

template <int D, bool P>
struct OpDensityPair {
  static constexpr int kWeightKind = kWMass;
  static constexpr bool kChannels = false;
  float rho = 0.0f;
  float grad[D] = {};
  __device__ void init(const GridParams&, const OpPtrs&, uint32_t) {}
  __device__ void pair(const GridParams& g, const OpPtrs&, const float*, const float*, float wj, const float* r,
                       float d2, uint32_t) {
    rho += poly6(g.eps2, d2) * wj;
    float d;
    const float t = spiky_mag(g.eps, d2, &d) * wj;
#pragma unroll
    for (int e = 0; e < D; ++e) grad[e] += t * r[e];
  }
  __device__ void reduce(int G) { grp_sum(G, rho, grad); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) {
    a.out0[k] = rho * g.c6;
#pragma unroll
    for (int e = 0; e < D; ++e) a.out3[(uint64_t)k * D + e] = grad[e] * g.cs;
  }
};

template <int D, bool P, int CM, bool EX>
struct OpBlurGradientHybrid {
  static constexpr int kWeightKind = kWVolume;
  static constexpr bool kChannels = true;
  using Ch = Chan<CM, EX>;
  float si[CM];
  float blur[CM] = {};
  float acc[CM * D] = {};
  float M[D * D] = {};
  __device__ void init(const GridParams&, const OpPtrs& a, uint32_t k) { Ch::load(a.s, k, a.C, si); }
  __device__ void pair(const GridParams& g, const OpPtrs& a, const float*, const float*, float wj, const float* r,
                       float d2, uint32_t j) {
    const float w = poly6(g.eps2, d2) * wj;
    float d;
    const float t = spiky_mag(g.eps, d2, &d) * wj;
#pragma unroll
    for (int p = 0; p < D; ++p)
#pragma unroll
      for (int q = p; q < D; ++q) M[p * D + q] += t * r[p] * r[q];
    float sj[CM];
    Ch::load(a.s, j, a.C, sj);
#pragma unroll
    for (int f = 0; f < CM; ++f) {
      blur[f] += w * sj[f];
      const float q = t * (sj[f] - si[f]);
#pragma unroll
      for (int e = 0; e < D; ++e) acc[f * D + e] += q * r[e];
    }
  }
  __device__ void reduce(int G) { grp_sum(G, blur, acc, M); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) {
    const uint32_t C = EX ? CM : a.C;
#pragma unroll
    for (int f = 0; f < CM; ++f)
      if (f < (int)C) a.out0[(uint64_t)k * Ch::stride(a.C) + f] = blur[f] * g.c6;
    float Ms[D * D], L[D * D];
#pragma unroll
    for (int p = 0; p < D; ++p)
#pragma unroll
      for (int q = 0; q < D; ++q) Ms[p * D + q] = (q >= p ? M[p * D + q] : M[q * D + p]) * g.cs;
    safe_inv_sym<D>(Ms, a.tol, L);
#pragma unroll
    for (int f = 0; f < CM; ++f) {
      if (f >= (int)C) continue;
      float raw[D];
#pragma unroll
      for (int e = 0; e < D; ++e) raw[e] = acc[f * D + e] * g.cs;
#pragma unroll
      for (int e = 0; e < D; ++e) {
        float o = 0.0f;
#pragma unroll
        for (int q = 0; q < D; ++q) o += raw[q] * L[q * D + e];
        a.out3[(uint64_t)k * Ch::stride(a.C) * D + f * D + e] = o;
      }
    }
  }
};

// ---------------------------------------------------------- backward ops

template <int D, bool P>
struct OpDensityBwd {
  static constexpr int kWeightKind = kWMass;
  static constexpr bool kChannels = false;
  float gi = 0.0f, mi = 0.0f;
  float dx[D] = {};
  __device__ void init(const GridParams&, const OpPtrs& a, uint32_t k) {
    gi = a.g[k];
    mi = a.m[k];
  }
  struct Nbr {  // the neighbour's upstream, loaded ahead by k_pairs_grouped
    float g;
  };
  __device__ static void fetch(const OpPtrs& a, uint32_t j, Nbr& n) { n.g = a.g[j]; }
  __device__ void pair(const GridParams& g, const OpPtrs& a, const float* xi, const float* xj, float wj,
                       const float* r, float d2, uint32_t j) {
    Nbr n;
    fetch(a, j, n);
    pair(g, a, xi, xj, wj, r, d2, j, n);
  }
  __device__ void pair(const GridParams& g, const OpPtrs&, const float* xi, const float* xj, float wj,
                       const float* r, float d2, uint32_t, const Nbr& n) {
    float rb[3];
    const float db = back_disp<D, P>(g, xi, xj, r, d2, rb);
    if (db == 0.0f || !(db < g.eps2)) return;
    const float t = g.eps2 - db;
    const float coef = gi * wj + n.g * mi;
    const float mag = -coef * 6.0f * t * t;
#pragma unroll
    for (int e = 0; e < D; ++e) dx[e] += mag * rb[e];
  }
  __device__ void reduce(int G) { grp_sum(G, dx); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) { store_pos_grad<D>(a.out0, k, dx, g.c6); }
};

template <int D, bool P>
struct OpDensityGradientBwd {
  static constexpr int kWeightKind = kWMass;
  static constexpr bool kChannels = false;
  float gi[D], mi = 0.0f;
  float dx[D] = {};
  __device__ void init(const GridParams&, const OpPtrs& a, uint32_t k) {
#pragma unroll
    for (int e = 0; e < D; ++e) gi[e] = a.g[(uint64_t)k * D + e];
    mi = a.m[k];
  }
  struct Nbr {  // the neighbour's upstream, loaded ahead by k_pairs_grouped
    float g[D];
  };
  __device__ static void fetch(const OpPtrs& a, uint32_t j, Nbr& n) {
#pragma unroll
    for (int e = 0; e < D; ++e) n.g[e] = a.g[(uint64_t)j * D + e];
  }
  __device__ void pair(const GridParams& g, const OpPtrs& a, const float* xi, const float* xj, float wj,
                       const float* r, float d2, uint32_t j) {
    Nbr n;
    fetch(a, j, n);
    pair(g, a, xi, xj, wj, r, d2, j, n);
  }
  __device__ void pair(const GridParams& g, const OpPtrs&, const float* xi, const float* xj, float wj,
                       const float* r, float d2, uint32_t, const Nbr& n) {
    float rb[3];
    const float db = back_disp<D, P>(g, xi, xj, r, d2, rb);
    float diff[D];
#pragma unroll
    for (int e = 0; e < D; ++e) diff[e] = n.g[e] * mi - gi[e] * wj;
    spiky_jacobian_apply<D>(rb, db, g.eps, g.eps2, diff, dx);
  }
  __device__ void reduce(int G) { grp_sum(G, dx); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) { store_pos_grad<D>(a.out0, k, dx, g.cs); }
};

template <int D, bool P>
struct OpMomentMatrixBwd {
  static constexpr int kWeightKind = kWVolume;
  static constexpr bool kChannels = false;
  float gi[D * D], vi = 0.0f, mr2 = 0.0f;
  float dx[D] = {};
  float drho = 0.0f;
  __device__ void init(const GridParams&, const OpPtrs& a, uint32_t k) {
#pragma unroll
    for (int q = 0; q < D * D; ++q) gi[q] = a.g[(uint64_t)k * D * D + q];
    const float mi = a.m[k], ri = a.rho[k];
    vi = mi / ri;
    mr2 = mi / (ri * ri);
  }
  __device__ void pair(const GridParams& g, const OpPtrs& a, const float* xi, const float* xj, float vj,
                       const float* r, float d2, uint32_t j) {
    float rb[3];
    const float db = back_disp<D, P>(g, xi, xj, r, d2, rb);
    float d;
    const float mag = spiky_mag(g.eps, db, &d);
    float w[D];
#pragma unroll
    for (int e = 0; e < D; ++e) w[e] = mag * rb[e];
    float gd[D * D];
#pragma unroll
    for (int p = 0; p < D; ++p) {
#pragma unroll
      for (int q = 0; q < D; ++q) {
        const float gj = a.g[(uint64_t)j * D * D + p * D + q];
        drho += gj * rb[p] * w[q];
        const float c = gi[p * D + q] * vj + gj * vi;
        dx[p] += w[q] * c;
        gd[p * D + q] = rb[p] * c;
      }
    }
#pragma unroll
    for (int p = 0; p < D; ++p) spiky_jacobian_apply<D>(rb, db, g.eps, g.eps2, &gd[p * D], dx);
  }
  __device__ void reduce(int G) { grp_sum(G, dx, drho); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) {
    store_pos_grad<D>(a.out0, k, dx, g.cs);
    a.out2[k] = -drho * mr2 * g.cs;
  }
};

template <int D, bool P, int CM, bool EX, bool FULL>
struct OpBlurBwd {
  static constexpr int kWeightKind = kWVolume;
  static constexpr bool kChannels = true;
  using Ch = Chan<CM, EX>;
  float vi = 0.0f, mr2 = 0.0f;
  float si[FULL ? CM : 1], gi[FULL ? CM : 1];
  float ds[CM] = {};
  float dx[D] = {};
  float drho = 0.0f;
  __device__ void init(const GridParams&, const OpPtrs& a, uint32_t k) {
    const float mi = a.m[k], ri = a.rho[k];
    vi = mi / ri;
    mr2 = mi / (ri * ri);
    if constexpr (FULL) {
      Ch::load(a.s, k, a.C, si);
      Ch::load(a.g, k, a.C, gi);
    }
  }
  __device__ void pair(const GridParams& g, const OpPtrs& a, const float* xi, const float* xj, float vj,
                       const float* r, float d2, uint32_t j) {
    float rb[3];
    const float db = back_disp<D, P>(g, xi, xj, r, d2, rb);
    const float W = poly6(g.eps2, db);
    float gj[CM];
    Ch::load(a.g, j, a.C, gj);
#pragma unroll
    for (int f = 0; f < CM; ++f) ds[f] += W * gj[f];
    if constexpr (FULL) {
      float sj[CM];
      Ch::load(a.s, j, a.C, sj);
      float A = 0.0f, Bv = 0.0f;
#pragma unroll
      for (int f = 0; f < CM; ++f) {
        A += gi[f] * sj[f];
        Bv += gj[f] * si[f];
      }
      drho += W * Bv;
      if (db != 0.0f && db < g.eps2) {
        const float t = g.eps2 - db;
        const float mag = -6.0f * t * t * (A * vj + Bv * vi);
#pragma unroll
        for (int e = 0; e < D; ++e) dx[e] += mag * rb[e];
      }
    }
  }
  __device__ void reduce(int G) { grp_sum(G, ds, dx, drho); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) {
    const uint32_t C = EX ? CM : a.C;
    const float sc = vi * g.c6;
#pragma unroll
    for (int f = 0; f < CM; ++f)
      if (f < (int)C) a.out1[(uint64_t)k * Ch::stride(a.C) + f] = ds[f] * sc;
    if constexpr (FULL) {
      a.out2[k] = -drho * mr2 * g.c6;
      store_pos_grad<D>(a.out0, k, dx, g.c6);
    }
  }
};

template <int D, bool P, int CM, bool EX, bool FULL, bool ACC = false>
struct OpGradientBwd {
  static constexpr int kWeightKind = kWVolume;
  static constexpr bool kChannels = true;
  using Ch = Chan<CM, EX>;
  float vi = 0.0f, mr2 = 0.0f;
  float gi[CM * D];
  float si[FULL ? CM : 1];
  float ds[CM] = {};
  float wsum[D] = {};
  float dx[D] = {};
  float drho = 0.0f;
  __device__ void init(const GridParams&, const OpPtrs& a, uint32_t k) {
    const float mi = a.m[k], ri = a.rho[k];
    vi = mi / ri;
    mr2 = mi / (ri * ri);
    Ch::template load_cd<D>(a.g, k, a.C, gi);
    if constexpr (FULL) Ch::load(a.s, k, a.C, si);
  }
  __device__ void pair(const GridParams& g, const OpPtrs& a, const float* xi, const float* xj, float vj,
                       const float* r, float d2, uint32_t j) {
    float rb[3];
    const float db = back_disp<D, P>(g, xi, xj, r, d2, rb);
    float d;
    const float mag = spiky_mag(g.eps, db, &d);
    float w[D];
#pragma unroll
    for (int e = 0; e < D; ++e) w[e] = mag * rb[e];
#pragma unroll
    for (int e = 0; e < D; ++e) wsum[e] += vj * w[e];
    float gj[CM * D];
    Ch::template load_cd<D>(a.g, j, a.C, gj);
    if constexpr (!FULL) {
#pragma unroll
      for (int f = 0; f < CM; ++f) {
        float pf = 0.0f;
#pragma unroll
        for (int e = 0; e < D; ++e) pf += gj[f * D + e] * w[e];
        ds[f] += pf;
      }
    } else {
      float sj[CM];
      Ch::load(a.s, j, a.C, sj);
      float u1[D] = {}, u2[D] = {};
#pragma unroll
      for (int f = 0; f < CM; ++f) {
        float pf = 0.0f;
        const float df = si[f] - sj[f];
#pragma unroll
        for (int e = 0; e < D; ++e) {
          pf += gj[f * D + e] * w[e];
          u1[e] += df * gj[f * D + e];
          u2[e] += df * gi[f * D + e];
        }
        ds[f] += pf;
      }
      float u[D], uw = 0.0f;
#pragma unroll
      for (int e = 0; e < D; ++e) {
        uw += u1[e] * w[e];
        u[e] = vi * u1[e] + vj * u2[e];
      }
      drho += uw;
      spiky_jacobian_apply<D>(rb, db, g.eps, g.eps2, u, dx);
    }
  }
  __device__ void reduce(int G) { grp_sum(G, ds, wsum, dx, drho); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) {
    const uint32_t C = EX ? CM : a.C;
#pragma unroll
    for (int f = 0; f < CM; ++f) {
      if (f >= (int)C) continue;
      float t = vi * ds[f];
#pragma unroll
      for (int e = 0; e < D; ++e) t += gi[f * D + e] * wsum[e];
      put<ACC>(a.out1, (uint64_t)k * Ch::stride(a.C) + f, t * g.cs);
    }
    if constexpr (FULL) {
      put<ACC>(a.out2, k, -drho * mr2 * g.cs);
      store_pos_grad<D, ACC>(a.out0, k, dx, g.cs);
    }
  }
};

// ------------------------------------------------------ fused backward
//
// Backward of the fused pairs: upstream a.g for the first operator, a.g2
// for the second; the gradients of both are summed into one set of outputs.

template <int D, bool P>
struct OpDensityPairBwd {
  static constexpr int kWeightKind = kWMass;
  static constexpr bool kChannels = false;
  float gi = 0.0f, gdi[D], mi = 0.0f;
  float dx_w[D] = {}, dx_k[D] = {};
  __device__ void init(const GridParams&, const OpPtrs& a, uint32_t k) {
    gi = a.g[k];
#pragma unroll
    for (int e = 0; e < D; ++e) gdi[e] = a.g2[(uint64_t)k * D + e];
    mi = a.m[k];
  }
  struct Nbr {  // the neighbour's two upstreams, loaded ahead by k_pairs_grouped
    float g, g2[D];
  };
  __device__ static void fetch(const OpPtrs& a, uint32_t j, Nbr& n) {
    n.g = a.g[j];
#pragma unroll
    for (int e = 0; e < D; ++e) n.g2[e] = a.g2[(uint64_t)j * D + e];
  }
  __device__ void pair(const GridParams& g, const OpPtrs& a, const float* xi, const float* xj, float wj,
                       const float* r, float d2, uint32_t j) {
    Nbr n;
    fetch(a, j, n);
    pair(g, a, xi, xj, wj, r, d2, j, n);
  }
  __device__ void pair(const GridParams& g, const OpPtrs&, const float* xi, const float* xj, float wj,
                       const float* r, float d2, uint32_t, const Nbr& n) {
    float rb[3];
    const float db = back_disp<D, P>(g, xi, xj, r, d2, rb);
    if (db != 0.0f && db < g.eps2) {
      const float t = g.eps2 - db;
      const float mag = -(gi * wj + n.g * mi) * 6.0f * t * t;
#pragma unroll
      for (int e = 0; e < D; ++e) dx_w[e] += mag * rb[e];
    }
    float diff[D];
#pragma unroll
    for (int e = 0; e < D; ++e) diff[e] = n.g2[e] * mi - gdi[e] * wj;
    spiky_jacobian_apply<D>(rb, db, g.eps, g.eps2, diff, dx_k);
  }
  __device__ void reduce(int G) { grp_sum(G, dx_w, dx_k); }
  __device__ void finish(const GridParams& g, const OpPtrs& a, uint32_t k) {
    float dx[D];
#pragma unroll
    for (int e = 0; e < D; ++e) dx[e] = dx_w[e] * g.c6 + dx_k[e] * g.cs;
    store_pos_grad<D>(a.out0, k, dx, 1.0f);
  }
};

// ---- stencil walk for particles whose row did not fit

// Candidates of particle k in stencil order, for a lane whose requests never
// decrease (t, then a larger t, ...): the cursor keeps the range it stopped
// in, so a row of n candidates costs one walk over its stencil ranges, not
// one walk per candidate.  Only for particles the fill could not store
// (count < 0).
template <int D, bool P>
struct StencilCursor {
  Walker<D, P> w;
  uint32_t before;  // candidates in the ranges before the current one

  __device__ __forceinline__ void init(const GridParams& g, const float* xi, uint32_t k) {
    w.init(g, xi, k);
    before = 0;
  }
  // Candidate number t (0-based); k itself past the stencil, which cannot
  // happen for t below the particle's candidate count.
  __device__ __forceinline__ uint32_t at(const GridParams& g, const int32_t* __restrict__ bo, uint32_t k,
                                         uint32_t t) {
    while (t - before >= w.jend - w.j) {
      before += w.jend - w.j;
      w.j = w.jend = 0;
      if (!w.fetch(g, bo, w.r)) return k;
      ++w.r;
    }
    return w.j + (t - before);
  }
};

// Row of particle k: its list entries, or (count < 0) its stencil candidates.
struct Row {
  int32_t start, end;
  bool stencil;
  __device__ __forceinline__ static Row of(const OpPtrs& a, uint32_t k) {
    const int32_t c = a.ncnt[k];
    if (c >= 0) return Row{a.nptr[k], a.nptr[k] + c, false};
    return Row{0, -1 - c, true};
  }
};

// ---------------------------------------------------------------- driver

// (x, y, z|0, weight) per particle into the scratch array the pair kernels read.
template <int D, int WK>
__global__ __launch_bounds__(kThreads) void k_pack(const float* __restrict__ x, const float* __restrict__ m,
                                                   const float* __restrict__ rho, float4* __restrict__ xw,
                                                   uint32_t n) {
  const uint32_t k = blockIdx.x * kThreads + threadIdx.x;
  if (k >= n) return;
  float p[3];
  load_pos<D>(x, k, p);
  float w = 0.0f;
  if constexpr (WK == kWMass) w = m[k];
  if constexpr (WK == kWVolume) w = m[k] / rho[k];
  xw[k] = make_float4(p[0], p[1], D == 3 ? p[2] : 0.0f, w);
}

__device__ __forceinline__ void unpack(const float4 v, float* p) {
  p[0] = v.x;
  p[1] = v.y;
  p[2] = v.z;
}

template <int D, bool P, int TRAV, class OP>
__global__ __launch_bounds__(kThreads) void k_pairs(GridParams g, const int32_t* __restrict__ bo, OpPtrs a) {
  const uint32_t n = g.B * g.N;
  // particles dealt to the XCDs in chunks (xcd_block_id_chunked), as the
  // schedules are: contiguous eighths would give some XCDs only sparse regions
  const uint32_t b = xcd_block_id_chunked((n + kThreads - 1) / kThreads);
  const uint32_t k = b == 0xFFFFFFFFu ? n : b * kThreads + threadIdx.x;
  const bool active = k < n;
  const float4* __restrict__ xw = a.xw;
  OP op;
  float xi[3] = {0.0f, 0.0f, 0.0f};
  if (active) {
    unpack(xw[k], xi);
    op.init(g, a, k);
  }
  if constexpr (TRAV == kList) {
    const Row row = active ? Row::of(a, k) : Row{0, 0, false};
    if (row.stencil) {
      StencilCursor<D, P> cur;
      cur.init(g, xi, k);
      for (int t = 0; t < row.end; ++t) {
        const uint32_t j = cur.at(g, a.bo, k, (uint32_t)t);
        const float4 pj = xw[j];
        float xj[3], r[3];
        unpack(pj, xj);
        const float d2 = displacement<D, P>(g, xi, xj, r);
        if (d2 < g.eps2) op.pair(g, a, xi, xj, pj.w, r, d2, j);
      }
    } else if (active) {
      const int32_t* __restrict__ nidx = a.nidx;
      int t = row.start;
      const int end = row.end;
      for (; t + 1 < end; t += 2) {
        const uint32_t j0 = (uint32_t)nidx[t], j1 = (uint32_t)nidx[t + 1];
        const float4 p0 = xw[j0], p1 = xw[j1];
        float x0[3], x1[3], r0[3], r1[3];
        unpack(p0, x0);
        unpack(p1, x1);
        const float d0 = displacement<D, P>(g, xi, x0, r0);
        const float d1 = displacement<D, P>(g, xi, x1, r1);
        op.pair(g, a, xi, x0, p0.w, r0, d0, j0);
        op.pair(g, a, xi, x1, p1.w, r1, d1, j1);
      }
      if (t < end) {
        const uint32_t j0 = (uint32_t)nidx[t];
        const float4 p0 = xw[j0];
        float x0[3], r0[3];
        unpack(p0, x0);
        const float d0 = displacement<D, P>(g, xi, x0, r0);
        op.pair(g, a, xi, x0, p0.w, r0, d0, j0);
      }
    }
  } else {
    Walker<D, P> w;
    if (active) w.init(g, xi, k);
    bool more = active && w.next(g, bo);
    if constexpr (TRAV == kStencil) {
      while (more) {
        const uint32_t last = w.jend - 1;
        float4 p[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) p[q] = xw[min(w.j + q, last)];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (w.j + q <= last) {
            float xj[3], r[3];
            unpack(p[q], xj);
            const float d2 = displacement<D, P>(g, xi, xj, r);
            if (d2 < g.eps2) op.pair(g, a, xi, xj, p[q].w, r, d2, w.j + q);
          }
        }
        w.j = min(w.j + 4, w.jend);
        more = w.next(g, bo);
      }
    } else {
      __shared__ uint32_t list[kThreads / kWave][kCap][kWave];
      const int wv = threadIdx.x >> 6, ln = __lane_id();
      while (__any(more)) {
        int cnt = 0;
        while (more && cnt <= kCap - 4) {
          const uint32_t last = w.jend - 1;
          float4 p[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) p[q] = xw[min(w.j + q, last)];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if (w.j + q <= last) {
              float xj[3], r[3];
              unpack(p[q], xj);
              const float d2 = displacement<D, P>(g, xi, xj, r);
              if (d2 < g.eps2) list[wv][cnt++][ln] = w.j + q;
            }
          }
          w.j = min(w.j + 4, w.jend);
          more = w.next(g, bo);
        }
        for (int t = 0; t < cnt; ++t) {
          const uint32_t j = list[wv][t][ln];
          const float4 pj = xw[j];
          float xj[3], r[3];
          unpack(pj, xj);
          const float d2 = displacement<D, P>(g, xi, xj, r);
          op.pair(g, a, xi, xj, pj.w, r, d2, j);
        }
      }
    }
  }
  if (active) op.finish(g, a, k);
}

// The number of live waves: the device count when the caller passed one (the
// launch is then sized by an upper bound), else the host count.
__device__ __forceinline__ uint32_t wave_limit(uint32_t host, const int32_t* dev) {
  return dev ? (uint32_t)*dev : host;
}

// The schedule's waves are served in rounds of (at most) the launched waves:
// this wave's first index, with the XCD mapping in chunks (xcd_block_id_chunked)
// taken over the workgroups the round needs, so that a launch larger than the
// schedule still spreads its live waves over all eight XCDs, and every XCD
// serves a share of every region of space; and the round's stride.
// Any launch (a multiple of eight workgroups) serves every live wave, so the
// launch can be sized from an estimate and the count read on the device.
__device__ __forceinline__ uint32_t schedule_blocks(uint32_t live) {
  const uint32_t per = kThreads / kWave;
  return min((live + per - 1) / per, gridDim.x);
}
__device__ __forceinline__ uint32_t schedule_wave(uint32_t live) {
  const uint32_t per = kThreads / kWave;
  const uint32_t b = xcd_block_id_chunked(schedule_blocks(live));
  return b == 0xFFFFFFFFu ? b : b * per + (threadIdx.x >> 6);
}
__device__ __forceinline__ uint32_t schedule_stride(uint32_t live) {
  return schedule_blocks(live) * (kThreads / kWave);
}

// Ops that declare a neighbour record (Nbr, fetch) have it loaded ahead of
// their pair() calls by the list loop below.
template <class T, class = void>
struct has_nbr : std::false_type {};
template <class T>
struct has_nbr<T, std::void_t<typename T::Nbr>> : std::true_type {};

// List traversal with a group of G lanes per particle, G by list-length class:
// wave w serves the particles a.order[first .. first + n) of its descriptor
// a.waves[w] = {first, G << 8 | n}; lane `sub` of a group takes pairs sub,
// sub+G, ... of the particle's list, so consecutive lanes read consecutive
// neighbours; the group then sums its partials.
template <int D, bool P, class OP>
__global__ __launch_bounds__(kThreads) void k_pairs_grouped(GridParams g, OpPtrs a) {
  const uint32_t live = wave_limit(a.nwaves, a.nwaves_dev);
  const uint32_t stride = schedule_stride(live);
  for (uint32_t wave = schedule_wave(live); wave < live; wave += stride) {
    const uint2 wd = a.waves[wave];
    const int G = (int)(wd.y >> 8);
    const int lane = __lane_id();
    const uint32_t slot = (uint32_t)(lane / G);
    const int sub = lane & (G - 1);
    const bool active = slot < (wd.y & 0xFFu);
    const uint32_t k = active ? (uint32_t)a.order[wd.x + slot] : 0u;
    const float4* __restrict__ xw = a.xw;
    OP op;
    float xi[3] = {0.0f, 0.0f, 0.0f};
    if (active) {
      unpack(xw[k], xi);
      op.init(g, a, k);
      const int32_t* __restrict__ nidx = a.nidx;
      const Row row = Row::of(a, k);
      const int end = row.end;
      int t = row.start + sub;
      if (row.stencil) {
        StencilCursor<D, P> cur;
        cur.init(g, xi, k);
        for (; t < end; t += G) {
          const uint32_t j = cur.at(g, a.bo, k, (uint32_t)t);
          const float4 pj = xw[j];
          float xj[3], r[3];
          unpack(pj, xj);
          const float d2 = displacement<D, P>(g, xi, xj, r);
          if (d2 < g.eps2) op.pair(g, a, xi, xj, pj.w, r, d2, j);
        }
      }
      if (t < end) {
        // list rows: four entries per step, in the order above; their
        // indices are loaded one step ahead (clamped into the row) and
        // their positions together, so a step waits for memory once
        uint32_t jn[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) jn[q] = (uint32_t)nidx[min(t + q * G, end - 1)];
        for (; t < end; t += 4 * G) {
          uint32_t j[4];
          float4 p[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            j[q] = jn[q];
            jn[q] = (uint32_t)nidx[min(t + (4 + q) * G, end - 1)];
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) p[q] = xw[j[q]];
          if constexpr (has_nbr<OP>::value) {  // the op's neighbour data too
            typename OP::Nbr nb[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) OP::fetch(a, j[q], nb[q]);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              if (t + q * G < end) {
                float xj[3], r[3];
                unpack(p[q], xj);
                const float d2 = displacement<D, P>(g, xi, xj, r);
                op.pair(g, a, xi, xj, p[q].w, r, d2, j[q], nb[q]);
              }
            }
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              if (t + q * G < end) {
                float xj[3], r[3];
                unpack(p[q], xj);
                const float d2 = displacement<D, P>(g, xi, xj, r);
                op.pair(g, a, xi, xj, p[q].w, r, d2, j[q]);
              }
            }
          }
        }
      }
    }
    op.reduce(G);
    if (active && sub == 0) op.finish(g, a, k);
  }
}

// ------------------------------------------------ lane-split channel kernels
//
// A group of G >= 4 lanes serves one particle as G/4 pair streams x 4 channel
// slices: lane sub = 4 * stream + slice walks the stream's pairs and handles
// channels [slice*CW, (slice+1)*CW) of C = 4*CW.  The four lanes of a stream
// read adjacent pieces of each neighbour's rows, so a wave's row loads are
// contiguous per neighbour, and a lane holds a quarter of the channel state.
// Channel sums are reduced over the streams (into the group's first four
// lanes, one per slice); sums over channels (dL/dx, dL/drho) over the whole
// group into its first lane.

struct VolumeWeights {  // packing of (x, m / rho) for the kernels below
  static constexpr int kWeightKind = kWVolume;
};

template <class... A>
__device__ __forceinline__ void grp_sum_streams(int G, A&... v) {
  if (G > 4) (grp_add<4>(v), ...);
  if (G > 8) (grp_add<8>(v), ...);
  if (G > 16) (grp_add<16>(v), ...);
  if (G > 32) (grp_add<32>(v), ...);
}

// Pass-B backward (blur with upstream a.g + gradient_hybrid with upstream
// a.g2, the straight-through gradient backward) in one pass on the lane-split
// layout; with FULL also dL/drho and dL/dx, summed over both operators.  The
// four slice lanes of a stream take the stream's pairs four at a time: lane q evaluates the geometry of the q-th pair (index, weight, W,
// grad W, the Jacobian coefficients) and the quad exchanges it by DPP
// quad_perm broadcasts, so each pair's geometry is evaluated once instead of
// in all four slices.  Terms summed over channels (dL/dx, dL/drho) stay
// per-lane partial sums over the lane's slice, reduced at the end; sum_j v_j
// grad W is accumulated by the owning lane only.
template <int Q>
__device__ __forceinline__ float quad_get(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), Q * 0x55, 0xF, 0xF, false));
}
template <int Q>
__device__ __forceinline__ uint32_t quad_get(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, Q * 0x55, 0xF, 0xF, false);
}

// Start of the channel slice [c0, c0 + CW) of row j of a (rows, stride)
// float array: with OFF32 a 32-bit byte offset from the (uniform) base, so
// the load takes a scalar base and one vector offset register; the launcher
// selects OFF32 only when every byte offset of the array fits in 32 bits.
template <bool OFF32>
__device__ __forceinline__ const float* row_slice(const float* __restrict__ base, uint32_t j, uint32_t stride,
                                                  uint32_t c0) {
  if constexpr (OFF32) return reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + (j * stride + c0) * 4u);
  return base + (uint64_t)j * stride + c0;
}

// PARTS: 3 for the fused pair, 1 for blur alone (upstream a.g), 2 for the
// gradient alone (upstream a.g2); the other operator's loads and terms are
// left out.
// The launch bound of 3 workgroups per CU (C = 16) still compiles to 122
// VGPRs and 4 waves per SIMD, but schedules the loop better than a bound of
// 4: 0.871 against 0.883 ms at cfg5.
template <int D, bool P, int CW, bool FULL, bool OFF32, int PARTS>
__global__ __launch_bounds__(kThreads, CW == 4 ? 3 : 2) void k_blur_hybrid_bwd_quad(GridParams g, OpPtrs a) {
  constexpr int C = 4 * CW;
  constexpr bool kB = (PARTS & 1) != 0, kG = (PARTS & 2) != 0;
  const uint32_t live = wave_limit(a.nwaves2, a.nwaves2_dev);
  const uint32_t stride = schedule_stride(live);
  for (uint32_t wave = schedule_wave(live); wave < live; wave += stride) {
    const uint2 wd = a.waves2[wave];
    const int G = (int)(wd.y >> 8);
    const int lane = __lane_id();
    const uint32_t slot = (uint32_t)(lane / G);
    const int sub = lane & (G - 1);
    const int slice = sub & 3, stream = sub >> 2, S = G >> 2;
    const bool active = slot < (wd.y & 0xFFu);
    const uint32_t k = active ? (uint32_t)a.order[wd.x + slot] : 0u;
    const uint32_t c0 = (uint32_t)slice * CW;
    const float4* __restrict__ xw = a.xw;
    float xi[3] = {0.0f, 0.0f, 0.0f};
    float vi = 0.0f, mr2 = 0.0f;
    float si[FULL ? CW : 1] = {}, gbi[FULL && kB ? CW : 1] = {};
    float ggi[kG ? CW * D : 1] = {};
    float dsb[CW] = {}, dsg[CW] = {};
    float wsum[D] = {};
    // dL/dx of both operators in one accumulator, in units of the spiky
    // coefficient (of poly6's for blur alone): blur's pair term enters
    // scaled by k6 = -6 c6 / cs
    float dxm[D] = {};
    float drb = 0.0f, drg = 0.0f;
    const float k6 = kG ? -6.0f * (g.c6 / g.cs) : -6.0f;
    if (active) {
      unpack(xw[k], xi);
      const float mi = a.m[k], ri = a.rho[k];
      vi = mi / ri;
      mr2 = mi / (ri * ri);
      if constexpr (kG) load_span<CW * D, true>(a.g2 + ((uint64_t)k * C + c0) * D, ggi);
      if constexpr (FULL) load_span<CW, true>(a.s + (uint64_t)k * C + c0, si);
      if constexpr (FULL && kB) load_span<CW, true>(a.g + (uint64_t)k * C + c0, gbi);
      const int32_t* __restrict__ nidx = a.nidx;
      const Row row = Row::of(a, k);
      const int start = row.start;
      // with cell tiles the row's last nown[k] entries (its own cell) are
      // served by k_cell_pairs_bwd
      const int end = row.end - (a.nown != nullptr ? a.nown[k] : 0);
      // rows walked on the stencil (count < 0, rare) take the general loop;
      // a wave without them the list-only one
      auto walk = [&](auto stencil_rows) {
        constexpr bool ST = decltype(stencil_rows)::value;
        StencilCursor<D, P> cur;
        if (ST && row.stencil) cur.init(g, xi, k);
        for (int t0 = start + stream; t0 < end; t0 += 4 * S) {
          // geometry of the pair this lane owns (all zero for a stencil
          // candidate out of radius)
          const int to = t0 + slice * S;
          uint32_t jo = k;
          float vo = 0.0f, Wo = 0.0f, t2o = 0.0f, jao = 0.0f, jbo = 0.0f;
          float rbo[3] = {0.0f, 0.0f, 0.0f}, wo[3] = {0.0f, 0.0f, 0.0f};
          float4 pj = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          float d2 = 0.0f, r[3] = {0.0f, 0.0f, 0.0f};
          bool inr = false;
          // list rows of the full backward take the pair with no branch (a
          // lane past the row's end takes the row's last entry; the quad
          // loop below stops before its pair, and its volume is zeroed for
          // wsum): 0.878 -> 0.861 ms at cfg5; the dL/ds-only variant, whose
          // time follows its loads, keeps the branch (0.673 against 0.697)
          constexpr bool kNoBranch = !ST && FULL;
          if constexpr (!kNoBranch) {
            if (to < end) {
              const uint32_t jc = ST && row.stencil ? cur.at(g, a.bo, k, (uint32_t)to) : (uint32_t)nidx[to];
              pj = xw[jc];
              float xj[3];
              unpack(pj, xj);
              d2 = displacement<D, P>(g, xi, xj, r);
              inr = !(ST && row.stencil) || d2 < g.eps2;
              if (inr) jo = jc;
            }
          } else {
            inr = to < end;
            jo = (uint32_t)nidx[min(to, end - 1)];
            pj = xw[jo];
            float xj[3];
            unpack(pj, xj);
            d2 = displacement<D, P>(g, xi, xj, r);
          }
          if (kNoBranch || inr) {
            float xj[3];
            unpack(pj, xj);
            vo = inr ? pj.w : 0.0f;
            const float db = back_disp<D, P>(g, xi, xj, r, d2, rbo);
            Wo = poly6(g.eps2, db);
            float d, dinv;
            const float mag = spiky_mag(g.eps, db, &d, &dinv);
    #pragma unroll
            for (int e = 0; e < D; ++e) {
              wo[e] = mag * rbo[e];
              wsum[e] += vo * wo[e];
            }
            const bool jac = db != 0.0f && db < g.eps2;  // Jacobian terms vanish outside (0, eps)
            const float tt = g.eps2 - db;
            const float di = dinv;
            t2o = jac ? tt * tt : 0.0f;
            jao = jac ? 3.0f * (g.eps - d) * (g.eps - d) * di : 0.0f;
            jbo = jac ? 3.0f * tt * di * di * di : 0.0f;
          }
    #pragma unroll
          for (int q = 0; q < 4; ++q) {
            if (t0 + q * S >= end) break;  // uniform over the quad
            uint32_t j;
            float vj, W, t2, ja, jb, rb[3], w[3];
    #define SPHOPS_QUAD_FETCH(QQ)                                                   \
      j = quad_get<QQ>(jo);                                                         \
      vj = quad_get<QQ>(vo);                                                        \
      W = quad_get<QQ>(Wo);                                                         \
      t2 = quad_get<QQ>(t2o);                                                       \
      ja = quad_get<QQ>(jao);                                                       \
      jb = quad_get<QQ>(jbo);                                                       \
      for (int e = 0; e < D; ++e) {                                                 \
        rb[e] = quad_get<QQ>(rbo[e]);                                               \
        w[e] = quad_get<QQ>(wo[e]);                                                 \
      }
            if (q == 0) { SPHOPS_QUAD_FETCH(0) }
            else if (q == 1) { SPHOPS_QUAD_FETCH(1) }
            else if (q == 2) { SPHOPS_QUAD_FETCH(2) }
            else { SPHOPS_QUAD_FETCH(3) }
    #undef SPHOPS_QUAD_FETCH
            float gbj[kB ? CW : 1], ggj[kG ? CW * D : 1];
            if constexpr (kB) load_span<CW, true>(row_slice<OFF32>(a.g, j, C, c0), gbj);
            if constexpr (kG) load_span<CW * D, true>(row_slice<OFF32>(a.g2, j, C * D, c0 * D), ggj);
            if constexpr (!FULL) {
    #pragma unroll
              for (int f = 0; f < CW; ++f) {
                if constexpr (kB) dsb[f] += W * gbj[f];
                if constexpr (kG) {
    #pragma unroll
                  for (int e = 0; e < D; ++e) dsg[f] += ggj[f * D + e] * w[e];
                }
              }
            } else {
              float sj[CW];
              load_span<CW, true>(row_slice<OFF32>(a.s, j, C, c0), sj);
              float coef = 0.0f;  // the pair's factor of rb in dL/dx
              if constexpr (kB) {
                float A = 0.0f, Bv = 0.0f;
    #pragma unroll
                for (int f = 0; f < CW; ++f) {
                  dsb[f] += W * gbj[f];
                  A += gbi[f] * sj[f];
                  Bv += gbj[f] * si[f];
                }
                coef = k6 * t2 * (A * vj + Bv * vi);  // t2 = 0 outside (0, eps)
                if constexpr (!kG) {
    #pragma unroll
                  for (int e = 0; e < D; ++e) dxm[e] += coef * rb[e];
                }
              }
              if constexpr (kG) {
                float u1[D] = {}, u2[D] = {};
    #pragma unroll
                for (int f = 0; f < CW; ++f) {
                  const float df = si[f] - sj[f];
    #pragma unroll
                  for (int e = 0; e < D; ++e) {
                    dsg[f] += ggj[f * D + e] * w[e];
                    u1[e] += df * ggj[f * D + e];
                    u2[e] += df * ggi[f * D + e];
                  }
                }
                float u[D], uw = 0.0f, rv = 0.0f;
    #pragma unroll
                for (int e = 0; e < D; ++e) {
                  uw += u1[e] * w[e];
                  u[e] = vi * u1[e] + vj * u2[e];
                  rv += rb[e] * u[e];
                }
                drg += uw;
                coef -= jb * rv;
    #pragma unroll
                for (int e = 0; e < D; ++e) dxm[e] += ja * u[e] + coef * rb[e];  // ja = jb = 0 outside
              }
            }
          }
        }
      };
      if (__ballot(row.stencil) != 0) walk(std::integral_constant<bool, true>{});
      else walk(std::integral_constant<bool, false>{});
      if constexpr (FULL && kB) {  // blur's dL/drho: sum_j W_j g_j . s_i = s_i . sum_j W_j g_j
  #pragma unroll
        for (int f = 0; f < CW; ++f) drb += si[f] * dsb[f];
      }
    }
    if constexpr (kB) grp_sum_streams(G, dsb);
    if constexpr (kG) {
      grp_sum_streams(G, dsg);
      grp_sum(G, wsum);
  #pragma unroll
      for (int e = 0; e < D; ++e) wsum[e] = quad_get<0>(wsum[e]);  // the group total, to the four slice lanes
    }
    if constexpr (FULL && kB && kG) grp_sum(G, dxm, drb, drg);
    else if constexpr (FULL && kB) grp_sum(G, dxm, drb);
    else if constexpr (FULL && kG) grp_sum(G, dxm, drg);
    if (active && stream == 0) {
      const float sb = vi * g.c6;
  #pragma unroll
      for (int f = 0; f < CW; ++f) {
        float o = 0.0f;
        if constexpr (kB) o = dsb[f] * sb;
        if constexpr (kG) {
          float t = vi * dsg[f];
  #pragma unroll
          for (int e = 0; e < D; ++e) t += ggi[f * D + e] * wsum[e];
          o = kB ? o + t * g.cs : t * g.cs;
        }
        a.out1[(uint64_t)k * C + c0 + f] = o;
      }
      if constexpr (FULL) {
        if (slice == 0) {
          float dr = 0.0f, dx[D];
          if constexpr (kB) dr = drb * g.c6;
          if constexpr (kG) dr = kB ? dr + drg * g.cs : drg * g.cs;
  #pragma unroll
          for (int e = 0; e < D; ++e) dx[e] = dxm[e] * (kG ? g.cs : g.c6);
          a.out2[k] = -mr2 * dr;
          store_pos_grad<D>(a.out0, k, dx, 1.0f);
        }
      }
    }
  }
}

// Pass-B forward (blur + gradient_hybrid) on the lane-split layout with the
// pair geometry shared per quad, as k_blur_hybrid_bwd_quad: lane q of a quad
// evaluates the q-th of four pairs (index, volume-weighted W and spiky
// magnitude, r), the quad exchanges them by DPP, and every lane accumulates
// its channel slice.  The moment matrix is accumulated by the owning lane,
// reduced over the group and handed to the four slice lanes.  PARTS: 3 for
// the fused pair (blur into a.out0, gradient_hybrid into a.out3), 1 for blur
// alone, 2 for gradient_hybrid alone (into a.out3).
template <int D, bool P, int CW, bool OFF32, int PARTS>
__global__ __launch_bounds__(kThreads, 6) void k_blur_hybrid_fwd_quad(GridParams g, OpPtrs a) {
  constexpr int C = 4 * CW;
  constexpr bool kB = (PARTS & 1) != 0, kG = (PARTS & 2) != 0;
  const uint32_t live = wave_limit(a.nwaves2, a.nwaves2_dev);
  const uint32_t stride = schedule_stride(live);
  for (uint32_t wave = schedule_wave(live); wave < live; wave += stride) {
    const uint2 wd = a.waves2[wave];
    const int G = (int)(wd.y >> 8);
    const int lane = __lane_id();
    const uint32_t slot = (uint32_t)(lane / G);
    const int sub = lane & (G - 1);
    const int slice = sub & 3, stream = sub >> 2, S = G >> 2;
    const bool active = slot < (wd.y & 0xFFu);
    const uint32_t k = active ? (uint32_t)a.order[wd.x + slot] : 0u;
    const uint32_t c0 = (uint32_t)slice * CW;
    const float4* __restrict__ xw = a.xw;
    float xi[3] = {0.0f, 0.0f, 0.0f};
    float si[CW] = {};
    float blur[CW] = {};
    float acc[CW * D] = {};
    float M[D * D] = {};
    if (active) {
      unpack(xw[k], xi);
      if constexpr (kG) load_span<CW, true>(a.s + (uint64_t)k * C + c0, si);
      const int32_t* __restrict__ nidx = a.nidx;
      const Row row = Row::of(a, k);
      const int start = row.start;
      const int end = row.end;
      // rows walked on the stencil (count < 0, rare) take the general loop;
      // a wave without them the list-only one
      auto walk = [&](auto stencil_rows) {
        constexpr bool ST = decltype(stencil_rows)::value;
        StencilCursor<D, P> cur;
        if (ST && row.stencil) cur.init(g, xi, k);
        // list rows: the next iteration's list entry is loaded one iteration
        // ahead (clamped into the row), and the body has no branch before
        // the row loads, so the position and row loads go out together
        uint32_t jnext = 0u;
        if constexpr (!ST) {
          if (end > start) jnext = (uint32_t)nidx[min(start + stream + slice * S, end - 1)];
        }
        for (int t0 = start + stream; t0 < end; t0 += 4 * S) {
          const int to = t0 + slice * S;
          uint32_t jo = k;
          // owned pair: volume-weighted W, and the volume-weighted spiky
          // magnitude times r (the moment matrix and gradient factor)
          float wo = 0.0f, tro[3] = {0.0f, 0.0f, 0.0f};
          float4 pj = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          float d2 = 0.0f, rr[3] = {0.0f, 0.0f, 0.0f};
          bool inr = false;
          if constexpr (ST) {
            if (to < end) {
              const uint32_t jc = row.stencil ? cur.at(g, a.bo, k, (uint32_t)to) : (uint32_t)nidx[to];
              pj = xw[jc];
              float xj[3];
              unpack(pj, xj);
              d2 = displacement<D, P>(g, xi, xj, rr);
              inr = !row.stencil || d2 < g.eps2;
              if (inr) jo = jc;
            }
          } else {
            inr = to < end;
            if (inr) jo = jnext;
            jnext = (uint32_t)nidx[min(to + 4 * S, end - 1)];
            pj = xw[jo];
            float xj[3];
            unpack(pj, xj);
            d2 = displacement<D, P>(g, xi, xj, rr);
          }
          // all four pairs are taken unconditionally (a pair past the row's
          // end has j = k and zero weights, so it adds nothing), and their
          // four row loads are issued before any of them is used
          float sj[4][CW];
          load_span<CW, true>(row_slice<OFF32>(a.s, quad_get<0>(jo), C, c0), sj[0]);
          load_span<CW, true>(row_slice<OFF32>(a.s, quad_get<1>(jo), C, c0), sj[1]);
          load_span<CW, true>(row_slice<OFF32>(a.s, quad_get<2>(jo), C, c0), sj[2]);
          load_span<CW, true>(row_slice<OFF32>(a.s, quad_get<3>(jo), C, c0), sj[3]);
          if (inr) {
            if constexpr (kB) wo = poly6(g.eps2, d2) * pj.w;
            if constexpr (kG) {
              float d;
              const float to_ = spiky_mag(g.eps, d2, &d) * pj.w;
    #pragma unroll
              for (int e = 0; e < D; ++e) tro[e] = to_ * rr[e];
    #pragma unroll
              for (int p = 0; p < D; ++p)
    #pragma unroll
                for (int q = p; q < D; ++q) M[p * D + q] += tro[p] * rr[q];
            }
          }
    #pragma unroll
          for (int q = 0; q < 4; ++q) {
            float w, tr[3];
    #define SPHOPS_QUAD_FETCH(QQ)             \
      w = quad_get<QQ>(wo);                   \
      for (int e = 0; e < D; ++e) tr[e] = quad_get<QQ>(tro[e]);
            if (q == 0) { SPHOPS_QUAD_FETCH(0) }
            else if (q == 1) { SPHOPS_QUAD_FETCH(1) }
            else if (q == 2) { SPHOPS_QUAD_FETCH(2) }
            else { SPHOPS_QUAD_FETCH(3) }
    #undef SPHOPS_QUAD_FETCH
    #pragma unroll
            for (int f = 0; f < CW; ++f) {
              if constexpr (kB) blur[f] += w * sj[q][f];
              if constexpr (kG) {
                const float df = sj[q][f] - si[f];
    #pragma unroll
                for (int e = 0; e < D; ++e) acc[f * D + e] += df * tr[e];
              }
            }
          }
        }
      };
      if (__ballot(row.stencil) != 0) walk(std::integral_constant<bool, true>{});
      else walk(std::integral_constant<bool, false>{});
    }
    if constexpr (kB) grp_sum_streams(G, blur);
    if constexpr (kG) {
      grp_sum_streams(G, acc);
      grp_sum(G, M);
  #pragma unroll
      for (int q = 0; q < D * D; ++q) M[q] = quad_get<0>(M[q]);  // the group total, to the four slice lanes
    }
    if (active && stream == 0) {
      if constexpr (kB) {
  #pragma unroll
        for (int f = 0; f < CW; ++f) a.out0[(uint64_t)k * C + c0 + f] = blur[f] * g.c6;
      }
    }
    if (kG && active && stream == 0) {
      float Ms[D * D], L[D * D];
  #pragma unroll
      for (int p = 0; p < D; ++p)
  #pragma unroll
        for (int q = 0; q < D; ++q) Ms[p * D + q] = (q >= p ? M[p * D + q] : M[q * D + p]) * g.cs;
      safe_inv_sym<D>(Ms, a.tol, L);
  #pragma unroll
      for (int f = 0; f < CW; ++f) {
        float raw[D];
  #pragma unroll
        for (int e = 0; e < D; ++e) raw[e] = acc[f * D + e] * g.cs;
  #pragma unroll
        for (int e = 0; e < D; ++e) {
          float o = 0.0f;
  #pragma unroll
          for (int q = 0; q < D; ++q) o += raw[q] * L[q * D + e];
          a.out3[((uint64_t)k * C + c0 + f) * D + e] = o;
        }
      }
    }
  }
}

// ------------------------------------------------- neighbour-list build
//
// Row i of the list holds particle i's in-radius neighbours in stencil order:
// the order of the concatenated stencil ranges Walker::fetch(0), fetch(1), ...
// visits.  Work split (k_fill_split, then run_unit_schedule): the particles
// of a cell with two or more particles form units, runs of up to
// kUnitParticles consecutive particles of one cell, which share the cell's
// stencil; a particle alone in its cell is "lone".  k_fill serves every unit
// with one wave, then every chunk of 64 consecutive particles for its lone
// members, a lane each (a wave for a lone particle with many candidates).

// unit_len[k] = particles of the unit starting at k (> 0), 0 for the other
// particles of a cell with two or more, -1 for a lone particle; flags[k] = 1
// where a unit starts (scanned by run_unit_schedule).
template <int D, bool P>
__global__ __launch_bounds__(kThreads) void k_fill_split(GridParams g, const int32_t* __restrict__ bo,
                                                         const float* __restrict__ x,
                                                         int32_t* __restrict__ unit_len,
                                                         uint32_t* __restrict__ flags) {
  const uint32_t n = g.B * g.N;
  const uint32_t k = blockIdx.x * kThreads + threadIdx.x;
  if (k >= n) return;
  float xi[3];
  load_pos<D>(x, k, xi);
  Walker<D, P> w;
  w.init(g, xi, k);
  const uint32_t h = w.base + cell_hash<D>(g, w.c);
  const int32_t cs = bo[h], ce = bo[h + 1];
  const int32_t off = (int32_t)k - cs;
  const int32_t ul = ce - cs < 2 ? -1 : off % kUnitParticles == 0 ? min(kUnitParticles, ce - (int32_t)k) : 0;
  unit_len[k] = ul;
  flags[k] = ul > 0 ? 1u : 0u;
}

// Stencil ranges per particle.
template <int D, bool P>
__host__ __device__ constexpr int ranges_per_particle(bool morton) {
  return morton ? Walker<D, P>::kCellRanges : Walker<D, P>::kRowRanges;
}

// ---- row allocation
//
// Rows hold a particle's in-radius neighbours only.  A unit of particles, or
// a wave's lone particles, first counts its hits, then takes one block of
// the index buffer with an atomic add on a 64-bit counter and writes its rows
// there.  The buffer is cut into S equal slices of `slen` entries (S a power
// of two, smask = S - 1), slice s allocated by the counter at
// stripes[s * kStripeWords], zero before the fill; wave w takes its blocks
// from slice w & smask, or, when a block does not fit there, from one of
// kFillProbes - 1 further slices spread over the buffer (an odd stride of
// about S / kFillProbes slices: neighbouring slices serve neighbouring waves,
// which work on the same dense region and fill up together).  Row contents and order (stencil order) are
// fixed; only where a row lands depends on the order in which blocks reach a
// counter, which no result depends on.  A block that fits nowhere is not
// written: its particles' counts are set to -1 - (their stencil candidates)
// and the pair kernels walk their stencils instead (StencilCursor).
// Counter words: [0] entries taken (a failed attempt's block included), [1]
// entries of failed attempts, [2] entries of blocks not written.
constexpr uint32_t kFillProbes = 8;
struct FillStripes {
  unsigned long long* ctr;  // kFillStripes * kStripeWords
  uint32_t smask;
  uint64_t slen;
  // Block of `need` entries for wave `wave` (lane 0's value is used, the
  // result is wave-uniform): its first index-buffer position, or ~0 if it
  // does not fit.
  __device__ __forceinline__ uint64_t take(uint32_t wave, uint32_t need) const {
    if (need == 0) return 0;
    const bool first = __lane_id() == 0;
    const uint32_t probes = min(kFillProbes, smask + 1);
    const uint32_t stride = ((smask + 1) / probes) | 1u;  // odd: the probed slices are distinct
    for (uint32_t i = 0; i < probes; ++i) {
      const uint32_t s = (wave + i * stride) & smask;
      unsigned long long* c = ctr + (uint64_t)s * kStripeWords;
      unsigned long long b = 0;
      if (first) b = atomicAdd(c, (unsigned long long)need);
      b = __shfl(b, 0, kWave);
      if (b + need <= slen) return (uint64_t)s * slen + b;
      if (first) atomicAdd(c + 1, (unsigned long long)need);
    }
    if (first) atomicAdd(ctr + (uint64_t)(wave & smask) * kStripeWords + 2, (unsigned long long)need);
    return ~0ull;
  }
};

// Lane t's value of v (t wave-uniform).
__device__ __forceinline__ float lane_float(float v, uint32_t t) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)t));
}

// Index-buffer store at element offset `at` (< 2^30, so the byte offset fits
// 32 bits and the store takes the buffer base as a scalar).
__device__ __forceinline__ void store_entry(int32_t* __restrict__ nidx, uint32_t at, int32_t j) {
  *reinterpret_cast<int32_t*>(reinterpret_cast<char*>(nidx) + at * 4u) = j;
}

// Rounds of 64 candidates whose hit bytes a unit keeps in LDS for its write
// pass (later rounds are tested again).
constexpr int kFillRounds = 48;

// Rows of the unit i0 .. i0 + ni - 1 (ni <= kUnitParticles particles of one
// cell, or one lone particle), one wave.  Lane r < R fetches stencil range r
// of the cell; round q tests candidate positions 64q .. 64q + 63 of the
// concatenated ranges, lane l taking position 64q + l, against every
// particle of the unit (wave-uniform positions).  Pass one counts the hits
// per particle and keeps, per lane and round, the byte of the unit's
// particles its candidate hit (`hits`, this wave's kFillRounds * 64 bytes of
// LDS); the unit takes one block of the index buffer; pass two writes each
// particle's row, ranking the hits of a round with mbcnt.
template <int D, bool P, int R, bool OT>
__device__ __forceinline__ void unit_rows(const GridParams& g, const float4* __restrict__ xw,
                                          const int32_t* __restrict__ bo, uint32_t i0, uint32_t ni,
                                          uint32_t wave, uint8_t* __restrict__ hits,
                                          int32_t* __restrict__ nidx, int32_t* __restrict__ nstart,
                                          int32_t* __restrict__ ncnt, const FillStripes& fs,
                                          const FillTiles& ft) {
  const uint32_t lane = (uint32_t)__lane_id();
  const float4 pt = xw[i0 + min(lane, ni - 1u)];
  float xs[kUnitParticles][3];
#pragma unroll
  for (int t = 0; t < kUnitParticles; ++t) {
    xs[t][0] = lane_float(pt.x, t);
    xs[t][1] = lane_float(pt.y, t);
    xs[t][2] = lane_float(pt.z, t);
  }
  // stencil range `lane` of the cell: start and length
  uint32_t lo = 0, len = 0;
  if ((int)lane < R) {
    Walker<D, P> w;
    w.init(g, xs[0], i0);
    w.fetch(g, bo, (int)lane);
    lo = w.j;
    len = w.jend - w.j;
  }
  // the unit's own cell [cs, ce) and whether it is a tile (wave-uniform)
  uint32_t cs = 0, ce = 0;
  bool tiled = false;
  if constexpr (OT) {
    Walker<D, P> w;
    w.init(g, xs[0], i0);
    const uint32_t h = w.base + cell_hash<D>(g, w.c);
    cs = (uint32_t)__builtin_amdgcn_readfirstlane(bo[h]);
    ce = (uint32_t)__builtin_amdgcn_readfirstlane(bo[h + 1]);
    tiled = ce - cs >= ft.tmin && ce - cs <= ft.tmax;
    if (tiled && i0 == cs && lane == 0) ft.cells[atomicAdd(ft.count, 1)] = make_uint2(cs, ce - cs);
  }
  // Many ranges (particle mode, periodic grids): empty ones are dropped and a
  // range that starts where the previous kept one ends is merged into it, so
  // the concatenation (the candidate sequence, rows included) is unchanged
  // and the mapping below steps over the `nr` kept ranges only.  Kept range
  // m goes through this wave's LDS area (rewritten by pass one) to lane m.
  uint32_t nr = (uint32_t)R;
  if constexpr (R > 9) {
    const uint64_t below = (1ull << lane) - 1ull;
    const uint64_t ne = __ballot(len > 0);
    const uint64_t before = ne & below;
    const int prev = before ? 63 - __clzll(before) : 0;
    const uint32_t prev_end = (uint32_t)__shfl((int)(lo + len), prev, kWave);
    const bool head = len > 0 && (before == 0 || prev_end != lo);
    const uint64_t heads = __ballot(head);
    nr = (uint32_t)__popcll(heads);
    // last nonempty range before the next head: the kept range's end
    const uint64_t later = heads & ~(below | (1ull << lane));
    const uint64_t upto = later ? ne & ((1ull << __builtin_ctzll(later)) - 1ull) : ne;
    const int last = upto ? 63 - __clzll(upto) : 0;
    const uint32_t end = (uint32_t)__shfl((int)(lo + len), last, kWave);
    uint2* kept = reinterpret_cast<uint2*>(hits);
    if (head) kept[__popcll(heads & below)] = make_uint2(lo, end - lo);
    const uint2 mine = kept[min(lane, (uint32_t)R - 1u)];
    lo = lane < nr ? mine.x : 0u;
    len = lane < nr ? mine.y : 0u;
  }
  // exclusive prefix of the lengths (R <= 32 lanes) and the candidate total
  uint32_t pre = len;
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) {
    const uint32_t v = __shfl_up(pre, off, kWave);
    if ((int)lane >= off) pre += v;
  }
  const uint32_t ncand = (uint32_t)__builtin_amdgcn_readlane((int)pre, 31);
  pre -= len;
  // a tile's own cell is one contiguous piece of one stencil range: its
  // candidate positions [po0, po0 + ce - cs), so only the rounds overlapping
  // it count and place own-cell hits apart
  uint32_t po0 = 0, po1 = 0;
  if constexpr (OT) {
    if (tiled) {
      const uint64_t at_r = __ballot((int)lane < 32 && len > 0 && cs >= lo && cs < lo + len);
      const int r0 = at_r ? __builtin_ctzll(at_r) : 0;
      po0 = (uint32_t)__shfl((int)(pre + cs - lo), r0, kWave);
      po1 = po0 + (ce - cs);
    }
  }
  // candidate at position p < ncand: p + offs of the last range starting at
  // or before p.  The starts do not decrease, so that offset is offs of range
  // 0 plus the steps dof[r] = offs[r] - offs[r - 1] of the ranges 1 .. r
  // starting at or before p (a sum, which the compiler keeps in registers).
  const int32_t offs = (int32_t)(lo - pre);
  const int32_t dof = offs - __shfl_up(offs, 1, kWave);
  const int32_t off0 = __builtin_amdgcn_readlane(offs, 0);
  // wave-uniform values: in grid mode (R <= 9) kept in vector registers (the
  // scalar file holds the unit's positions); the 27 single-cell ranges of
  // particle mode would take 54 vector registers and most of the occupancy,
  // so they are read into scalar registers
  uint32_t spre[R];
  int32_t sdof[R];
#pragma unroll
  for (int r = 1; r < R; ++r) {
    if constexpr (R > 9) {
      spre[r] = (uint32_t)__builtin_amdgcn_readlane((int)pre, r);
      sdof[r] = __builtin_amdgcn_readlane(dof, r);
    } else {
      spre[r] = (uint32_t)__shfl((int)pre, r, kWave);
      sdof[r] = __shfl(dof, r, kWave);
    }
  }
  auto candidate = [&](uint32_t p) -> uint32_t {
    int32_t o = off0;
#pragma unroll
    for (int r = 1; r < R; ++r) {
      if constexpr (R > 9) {
        if ((uint32_t)r >= nr) break;  // wave-uniform
      }
      o += p >= spre[r] ? sdof[r] : 0;
    }
    return p < ncand ? (uint32_t)((int32_t)p + o) : i0;
  };
  const uint32_t rounds = (ncand + kWave - 1) / kWave;
  // pass one: count, keeping the hit bytes; the next round's positions are
  // loaded while this round is tested
  uint32_t cnt[kUnitParticles] = {}, cown[kUnitParticles] = {};
  uint32_t jn = candidate(lane);
  float4 nx = xw[jn];
  for (uint32_t rd = 0; rd < rounds; ++rd) {
    const uint32_t p = rd * kWave + lane;
    float xj[3];
    unpack(nx, xj);
    if (p >= ncand) xj[0] = __int_as_float(0x7FC00000);  // NaN: never in radius
    const bool own = OT && tiled && jn >= cs && jn < ce;
    if (rd + 1 < rounds) {
      jn = candidate(p + kWave);
      nx = xw[jn];
    }
    uint32_t bits = 0;
#pragma unroll
    for (int t = 0; t < kUnitParticles; ++t) {
      if (t < (int)ni) {
        float r[3];
        const bool in = displacement<D, P>(g, xs[t], xj, r) < g.eps2;
        cnt[t] += (uint32_t)__popcll(__ballot(in));
        if constexpr (OT) {
          if (tiled && rd * kWave < po1 && rd * kWave + kWave > po0)
            cown[t] += (uint32_t)__popcll(__ballot(in && own));
        }
        bits |= (in ? 1u : 0u) << t;
      }
    }
    if (rd < (uint32_t)kFillRounds) hits[rd * kWave + lane] = (uint8_t)bits;
  }
  // the unit's block of the index buffer
  uint32_t tot = 0;
#pragma unroll
  for (int t = 0; t < kUnitParticles; ++t) tot += cnt[t];
  const uint64_t b = fs.take(wave, tot);
  if (b == ~0ull) {
    if (lane < ni) {
      nstart[i0 + lane] = 0;
      ncnt[i0 + lane] = -1 - (int32_t)ncand;
      if constexpr (OT) ft.own[i0 + lane] = 0;
    }
    return;
  }
  // at[t]: next slot of particle t's row; ao[t]: next slot of its own-cell
  // entries, which a tile's rows keep last
  uint32_t at[kUnitParticles], ao[kUnitParticles];
  int32_t mine_start = 0, mine_cnt = 0, mine_own = 0;
  {
    uint32_t run = (uint32_t)b;
#pragma unroll
    for (int t = 0; t < kUnitParticles; ++t) {
      at[t] = run;
      run += cnt[t];
      ao[t] = run - cown[t];
      if ((int)lane == t) {
        mine_start = (int32_t)at[t];
        mine_cnt = (int32_t)cnt[t];
        mine_own = (int32_t)cown[t];
      }
    }
  }
  // pass two: write the rows
  for (uint32_t rd = 0; rd < rounds; ++rd) {
    const uint32_t p = rd * kWave + lane;
    const uint32_t j = candidate(p);
    uint32_t bits;
    if (rd < (uint32_t)kFillRounds) {
      bits = hits[rd * kWave + lane];
    } else {
      float xj[3];
      unpack(xw[j], xj);
      if (p >= ncand) xj[0] = __int_as_float(0x7FC00000);
      bits = 0;
#pragma unroll
      for (int t = 0; t < kUnitParticles; ++t) {
        float r[3];
        if (t < (int)ni && displacement<D, P>(g, xs[t], xj, r) < g.eps2) bits |= 1u << t;
      }
    }
    if (OT && tiled && rd * kWave < po1 && rd * kWave + kWave > po0) {
      const bool own = j >= cs && j < ce;
#pragma unroll
      for (int t = 0; t < kUnitParticles; ++t) {
        if (t < (int)ni) {
          const bool in = (bits >> t) & 1u;
          const uint64_t m = __ballot(in && !own), mo = __ballot(in && own);
          const uint64_t mm = own ? mo : m;
          const uint32_t rank =
              __builtin_amdgcn_mbcnt_hi((uint32_t)(mm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mm, 0u));
          if (in) store_entry(nidx, (own ? ao[t] : at[t]) + rank, (int32_t)j);
          at[t] += (uint32_t)__popcll(m);
          ao[t] += (uint32_t)__popcll(mo);
        }
      }
      continue;
    }
#pragma unroll
    for (int t = 0; t < kUnitParticles; ++t) {
      if (t < (int)ni) {
        const bool in = (bits >> t) & 1u;
        const uint64_t m = __ballot(in);
        const uint32_t rank =
            __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if (in) store_entry(nidx, at[t] + rank, (int32_t)j);
        at[t] += (uint32_t)__popcll(m);
      }
    }
  }
  if (lane < ni) {
    nstart[i0 + lane] = mine_start;
    ncnt[i0 + lane] = mine_cnt;
    if constexpr (OT) ft.own[i0 + lane] = mine_own;
  }
}

// Lone particles of the chunk of 64 particles starting at k0, one lane each:
// a first walk over the stencil counts the candidates and marks the in-radius
// ones among the first 64 (a 64-bit mask, the first four also kept in
// registers), the wave takes one block for all of its rows, and the rows are
// written from the registers or, for more than four hits, by a second walk.
// A lone particle with more than 64 candidates is served afterwards by the
// whole wave (unit_rows, ni = 1).
template <int D, bool P, int R, bool OT>
__device__ __forceinline__ void lone_rows(const GridParams& g, const float4* __restrict__ xw,
                                          const int32_t* __restrict__ bo, const int32_t* __restrict__ unit_len,
                                          uint32_t k0, uint32_t wave, uint8_t* __restrict__ hits,
                                          int32_t* __restrict__ nidx, int32_t* __restrict__ nstart,
                                          int32_t* __restrict__ ncnt, const FillStripes& fs,
                                          const FillTiles& ft) {
  const uint32_t n = g.B * g.N;
  const uint32_t lane = (uint32_t)__lane_id();
  const uint32_t k = k0 + lane;
  const bool lone = k < n && unit_len[k] < 0;
  float xi[3] = {0.0f, 0.0f, 0.0f};
  uint64_t mask = 0;
  uint32_t cand = 0, c = 0;
  int32_t h0 = 0, h1 = 0, h2 = 0, h3 = 0;
  Walker<D, P> w{};
  // ranges fetched kFetch at a time (their loads in flight together): three
  // for the many single-cell ranges of particle mode and periodic grids, one
  // for the nine stencil rows of a clamped grid, whose register budget the
  // unit path needs; a clamped grid's walk loads two candidate positions
  // at a time instead (more would cost the unit path a wave per SIMD)
  constexpr int kFetch = R > 9 ? 3 : 1;
  constexpr int kLoneLoads = R > 9 ? 1 : 2;
  static_assert(R % kFetch == 0, "ranges come in whole fetch groups");
  if (lone) {
    unpack(xw[k], xi);
    w.init(g, xi, k);
#pragma unroll 1
    for (int r0 = 0; r0 < R; r0 += kFetch) {
      uint32_t rlo[kFetch], rhi[kFetch];
#pragma unroll
      for (int u = 0; u < kFetch; ++u) {
        w.fetch(g, bo, r0 + u);
        rlo[u] = w.j;
        rhi[u] = w.jend;
      }
#pragma unroll
      for (int u = 0; u < kFetch; ++u) {
        const uint32_t len = rhi[u] - rlo[u];
        const uint32_t take = cand < (uint32_t)kWave ? min(len, (uint32_t)kWave - cand) : 0u;
        // kLoneLoads candidate positions in flight per step (the last one
        // repeated past the range's end, so every load stays in it)
        for (uint32_t q = 0; q < take; q += kLoneLoads) {
          float4 pj[kLoneLoads];
#pragma unroll
          for (int v = 0; v < kLoneLoads; ++v) pj[v] = xw[rlo[u] + min(q + (uint32_t)v, take - 1u)];
#pragma unroll
          for (int v = 0; v < kLoneLoads; ++v) {
            float xj[3], rr[3];
            unpack(pj[v], xj);
            if (q + (uint32_t)v < take && displacement<D, P>(g, xi, xj, rr) < g.eps2) {
              mask |= 1ull << (cand + q + (uint32_t)v);
              const int32_t j = (int32_t)(rlo[u] + q + (uint32_t)v);
              h0 = c == 0 ? j : h0;
              h1 = c == 1 ? j : h1;
              h2 = c == 2 ? j : h2;
              h3 = c == 3 ? j : h3;
              ++c;
            }
          }
        }
        cand += len;
      }
    }
  }
  const bool light = lone && cand <= (uint32_t)kWave;
  const uint32_t cnt = light ? c : 0u;
  if constexpr (OT) {
    if (lone) ft.own[k] = 0;  // a lone particle's cell is never a tile
  }
  uint32_t incl = cnt;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint32_t v = __shfl_up(incl, off, kWave);
    if ((int)lane >= off) incl += v;
  }
  const uint32_t wtot = __shfl(incl, kWave - 1, kWave);
  const uint64_t b = fs.take(wave, wtot);
  if (light) {
    if (b == ~0ull) {
      nstart[k] = 0;
      ncnt[k] = -1 - (int32_t)cand;
    } else {
      uint32_t at = (uint32_t)b + incl - cnt;
      nstart[k] = (int32_t)at;
      ncnt[k] = (int32_t)cnt;
      if (cnt <= 4) {
        if (cnt > 0) store_entry(nidx, at, h0);
        if (cnt > 1) store_entry(nidx, at + 1, h1);
        if (cnt > 2) store_entry(nidx, at + 2, h2);
        if (cnt > 3) store_entry(nidx, at + 3, h3);
      } else {
        uint32_t pos = 0;
#pragma unroll 1
        for (int r = 0; r < R && pos < (uint32_t)kWave && (mask >> pos) != 0; ++r) {
          w.fetch(g, bo, r);
          for (uint32_t j = w.j; j < w.jend; ++j, ++pos)
            if ((mask >> pos) & 1ull) store_entry(nidx, at++, (int32_t)j);
        }
      }
    }
  }
  uint64_t heavy = __ballot(lone && !light);
  while (heavy) {
    const uint32_t l = (uint32_t)__builtin_ctzll(heavy);
    heavy &= heavy - 1;
    unit_rows<D, P, R, OT>(g, xw, bo, k0 + l, 1, wave, hits, nidx, nstart, ncnt, fs, ft);
  }
}

// The list fill: a persistent grid whose waves take the chunks of 64
// particles c = wave, wave + (waves in the grid), ... (k0 = 64 c) and the
// units (units[u] = {first particle, particles}) from kFillStripes queues:
// queue q holds the units u = q, q + kFillStripes, ... (a sample of the whole
// cloud, so the queues carry about equal work), its counter at word
// kUnitQueueWord of stripe q, and the waves w = q mod kFillStripes take its
// units one at a time until it is empty.  A unit's cost runs from one round
// to dozens (crowded cells sit together), so a fixed share per wave leaves
// the waves that drew crowded cells running long after the others.  Even
// waves take their chunks first, odd waves their units first, so that the
// memory-bound lone walks overlap the ALU-bound units.  Which wave writes a
// row changes only where the row lands in the index buffer.
template <int D, bool P, int R, bool OT>
__device__ __forceinline__ void fill_items(const GridParams& g, const float4* __restrict__ xw,
                                           const int32_t* __restrict__ bo, const int32_t* __restrict__ unit_len,
                                           const uint2* __restrict__ units, uint32_t nunits, uint8_t* hits,
                                           int32_t* __restrict__ nidx, int32_t* __restrict__ nstart,
                                           int32_t* __restrict__ ncnt, const FillStripes& fs,
                                           const FillTiles& ft) {
  const uint32_t n = g.B * g.N;
  const uint32_t nchunks = (n + kWave - 1) / kWave;
  const uint32_t nwaves = gridDim.x * (kThreads / kWave);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(xcd_block_id() * (kThreads / kWave) + (threadIdx.x >> 6));
  const bool chunks_first = (wave & 1u) == 0;
  for (int phase = 0; phase < 2; ++phase) {
    if ((phase == 0) == chunks_first) {
      for (uint32_t c = wave; c < nchunks; c += nwaves)
        lone_rows<D, P, R, OT>(g, xw, bo, unit_len, c * kWave, wave, hits, nidx, nstart, ncnt, fs, ft);
    } else {
      const uint32_t q = wave & (kFillStripes - 1u);
      const uint32_t in_queue = q < nunits ? (nunits - q + kFillStripes - 1u) / kFillStripes : 0u;
      unsigned long long* __restrict__ next = fs.ctr + (uint64_t)q * kStripeWords + kUnitQueueWord;
      for (;;) {
        uint32_t i = 0;
        if (__lane_id() == 0) i = (uint32_t)atomicAdd(next, 1ull);
        i = (uint32_t)__builtin_amdgcn_readfirstlane((int)__shfl((int)i, 0, kWave));
        if (i >= in_queue) break;
        const uint2 ud = units[i * kFillStripes + q];
        unit_rows<D, P, R, OT>(g, xw, bo, __builtin_amdgcn_readfirstlane(ud.x),
                               __builtin_amdgcn_readfirstlane(ud.y), wave, hits, nidx, nstart, ncnt, fs, ft);
      }
    }
  }
}

// M: particle mode (stencil of single cells) or grid mode (stencil rows);
// OT: cell tiles (FillTiles).
template <int D, bool P, bool M, bool OT>
__global__ __launch_bounds__(kThreads) void k_fill(GridParams g, const float4* __restrict__ xw,
                                                   const int32_t* __restrict__ bo,
                                                   const int32_t* __restrict__ unit_len,
                                                   const uint2* __restrict__ units,
                                                   const int32_t* __restrict__ unit_total,
                                                   int32_t* __restrict__ nidx, int32_t* __restrict__ nstart,
                                                   int32_t* __restrict__ ncnt, FillStripes fs, FillTiles ft) {
  __shared__ __align__(16) uint8_t hits[kThreads / kWave][kFillRounds * kWave];
  uint8_t* mine = hits[threadIdx.x >> 6];
  const uint32_t nunits = (uint32_t)*unit_total;
  fill_items<D, P, M ? Walker<D, P>::kCellRanges : Walker<D, P>::kRowRanges, OT>(
      g, xw, bo, unit_len, units, nunits, mine, nidx, nstart, ncnt, fs, ft);
}

// total[0] = in-radius pairs (blocks written or not), total[1] = pairs of
// the blocks not written, from the counters' words (see FillStripes); the
// counters, and the unit queues of all kFillStripes stripes, are then reset
// to zero for the next fill.  One workgroup of
// kThreads >= kFillStripes.
static_assert(kThreads >= kFillStripes, "k_fill_totals reads one counter per thread");
[[maybe_unused]] static __global__ __launch_bounds__(kThreads) void k_fill_totals(unsigned long long* __restrict__ ctr,
                                                                 uint32_t stripes,
                                                                 unsigned long long* __restrict__ total) {
  __shared__ unsigned long long part[2][kThreads / kWave];
  const uint32_t s = threadIdx.x;
  unsigned long long a = 0, o = 0;
  if (s < stripes) {
    unsigned long long* c = ctr + (uint64_t)s * kStripeWords;
    a = c[0] - c[1] + c[2];
    o = c[2];
    c[0] = c[1] = c[2] = 0ull;
  }
  if (s < kFillStripes) ctr[(uint64_t)s * kStripeWords + kUnitQueueWord] = 0ull;  // the fill's unit queues
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    a += __shfl_down(a, off, kWave);
    o += __shfl_down(o, off, kWave);
  }
  if (__lane_id() == 0) {
    part[0][s / kWave] = a;
    part[1][s / kWave] = o;
  }
  __syncthreads();
  if (s == 0) {
    unsigned long long sa = 0, so = 0;
    for (uint32_t w = 0; w < kThreads / kWave; ++w) {
      sa += part[0][w];
      so += part[1][w];
    }
    total[0] = sa;
    total[1] = so;
  }
}


}  // namespace pk
}  // namespace sphops

#include "perception_tiled.hpp"
#include "perception_cells.hpp"

namespace sphops {
namespace pk {

inline dim3 grid_for(uint64_t n) { return dim3((uint32_t)((n + kThreads - 1) / kThreads)); }
// One workgroup per kThreads items, rounded up to a multiple of the eight
// XCDs (what xcd_block_id_chunked needs to cover every item).
inline dim3 grid_for_xcds(uint64_t n) { return dim3((uint32_t)(((n + kThreads - 1) / kThreads + 7) / 8 * 8)); }

// The (x, weight) records the pair kernels read: packed into the caller's
// buffer (or the grid's scratch), or the caller's buffer as it is when it
// already holds them (a backward reusing its forward's records).
template <int D, class OP>
void pack_for(const Grid& g, OpPtrs& a, hipStream_t st) {
  if (a.xw_buf != nullptr && a.xw_ready) {
    a.xw = a.xw_buf;
    return;
  }
  float4* dst = a.xw_buf != nullptr ? a.xw_buf : g.packed;
  constexpr int WK = OP::kWeightKind;
  hipLaunchKernelGGL((k_pack<D, WK>), grid_for(g.n_keys), dim3(kThreads), 0, st, a.x, a.m, a.rho, dst,
                     (uint32_t)g.n_keys);
  SPHOPS_LAUNCHED();
  a.xw = dst;
}

constexpr uint32_t kPersistentWorkgroups = 2048;
// Workgroups of the list fill (timed at cfg5, with the unit queues too: 4096
// beats 2048, 3072, 6144 and 8192).
constexpr uint32_t kFillWorkgroups = 4096;
static_assert(kFillWorkgroups * (kThreads / kWave) >= kFillStripes, "every unit queue of the fill has a wave");

// Work split of the list fill (unit table and lone marks, in the grid's
// scratch), read by neighbour_fill.
template <int D, bool P>
void neighbour_candidates(const Grid& g, const int32_t* bo, const float* x, hipStream_t st) {
  const uint32_t n = (uint32_t)g.n_keys;
  hipLaunchKernelGGL((k_fill_split<D, P>), grid_for(n), dim3(kThreads), 0, st, g.p, bo, x, g.unit_len, g.flags);
  SPHOPS_LAUNCHED();
  run_unit_schedule(g, st);
}

// Fill the rows (compact, allocated from the striped counters) with the work
// split neighbour_candidates left in the grid; used[0..1] receive the pair
// totals (k_fill_totals).
// With ft.own set, the rows keep the own-cell entries of the tiles last
// (FillTiles); ft.count is cleared here.
template <int D, bool P>
void neighbour_fill(const Grid& g, const int32_t* bo, const float* x, int32_t* nstart, int32_t* nidx,
                    int32_t* ncnt, unsigned long long* used, int64_t cap, const FillTiles& ft, hipStream_t st) {
  const uint32_t n = (uint32_t)g.n_keys;
  // 3D positions are already 16-byte (x, y, z, w) records; the fill reads
  // x, y and z only, so they need no packing
  const float4* xw = reinterpret_cast<const float4*>(x);
  if constexpr (D == 2) {
    hipLaunchKernelGGL((k_pack<D, kWNone>), grid_for(n), dim3(kThreads), 0, st, x, nullptr, nullptr, g.packed, n);
    SPHOPS_LAUNCHED();
    xw = g.packed;
  }
  // S slices of at least kStripeMinEntries entries and, for n particles,
  // about n / (kStripeMinUnits * kUnitParticles) units or more each (one
  // slice for small buffers)
  uint32_t S = 1;
  while (S < kFillStripes && (int64_t)(2 * S) * kStripeMinEntries <= cap &&
         (uint64_t)(2 * S) * kStripeMinUnits * kUnitParticles <= n)
    S *= 2;
  // the counters are zero here: zeroed at grid creation and by the totals
  // kernel of every fill
  FillStripes fs{g.stripes, S - 1, (uint64_t)(cap / S)};
  const bool ot = ft.own != nullptr;
  if (ot) fill_u32(reinterpret_cast<uint32_t*>(ft.count), 1, 0u, st);
#define SPHOPS_FILL(M, OT)                                                                                      \
  hipLaunchKernelGGL((k_fill<D, P, M, OT>), dim3(kFillWorkgroups), dim3(kThreads), 0, st, g.p, xw, bo, g.unit_len, \
                     g.units, g.unit_total, nidx, nstart, ncnt, fs, ft)
  if (g.particle_mode) {
    if (ot) SPHOPS_FILL(true, true);
    else SPHOPS_FILL(true, false);
  } else {
    if (ot) SPHOPS_FILL(false, true);
    else SPHOPS_FILL(false, false);
  }
#undef SPHOPS_FILL
  SPHOPS_LAUNCHED();
  hipLaunchKernelGGL(k_fill_totals, dim3(1), dim3(kThreads), 0, st, g.stripes, S, used);
  SPHOPS_LAUNCHED();
}

// Workgroups for a schedule of `waves` waves, rounded up to a multiple of 8
// (schedule_wave's mapping covers the live waves with that many).
inline uint32_t launch_groups(uint32_t waves) {
  const uint32_t per = kThreads / kWave;
  return ((waves + per - 1) / per + 7u) & ~7u;
}

// Launch of a schedule whose wave count the kernel reads on the device
// (`dev`): `waves` is only an estimate, and the kernels loop until every
// live wave is served, so at least 64 workgroups go out even when the
// estimate is zero.
inline uint32_t schedule_groups(uint32_t waves, const int32_t* dev) {
  const uint32_t w = launch_groups(waves);
  return dev != nullptr ? std::max<uint32_t>(w, 64u) : w;
}

template <int D, bool P, class OP>
void launch_pairs(const Grid& g, const int32_t* bo, OpPtrs a, hipStream_t st) {
  const uint64_t n = g.n_keys;
  if (n == 0) return;
  pack_for<D, OP>(g, a, st);
  if (a.nidx != nullptr && a.waves != nullptr) {
    const uint32_t wgs = schedule_groups(a.nwaves, a.nwaves_dev);
    if (wgs == 0) return;
    hipLaunchKernelGGL((k_pairs_grouped<D, P, OP>), dim3(wgs), dim3(kThreads), 0, st, g.p, a);
  } else if (a.nidx != nullptr) {
    hipLaunchKernelGGL((k_pairs<D, P, kList, OP>), grid_for_xcds(n), dim3(kThreads), 0, st, g.p, bo, a);
  } else if (OP::kChannels) {
    hipLaunchKernelGGL((k_pairs<D, P, kStencil2, OP>), grid_for_xcds(n), dim3(kThreads), 0, st, g.p, bo, a);
  } else {
    hipLaunchKernelGGL((k_pairs<D, P, kStencil, OP>), grid_for_xcds(n), dim3(kThreads), 0, st, g.p, bo, a);
  }
  SPHOPS_LAUNCHED();
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Lane-split kernels serve rows of 16 or 32 channels read as 16-byte vectors
// (the fused pass B, forward and backward).
inline bool split_ok(const OpPtrs& a) {
  return a.nidx != nullptr && a.waves2 != nullptr && (a.C == 16 || a.C == 32) && aligned16(a.s) &&
         aligned16(a.g) && aligned16(a.g2);
}

// Byte offsets into the (B*N, C*D) gradient rows fit in 32 bits.
inline bool row_offsets_fit_32(const Grid& g, uint32_t C) {
  return g.n_keys * (uint64_t)C * 3u * 4u <= 0xFFFFFFFFull;
}

// PARTS as for k_blur_hybrid_fwd_quad.
template <int D, bool P, int PARTS = 3>
void launch_blur_hybrid_fwd_quad(const Grid& g, OpPtrs a, hipStream_t st) {
  if (g.n_keys == 0) return;
  const uint32_t wgs = schedule_groups(a.nwaves2, a.nwaves2_dev);
  pack_for<D, VolumeWeights>(g, a, st);
  if (wgs == 0) return;
  const bool off32 = row_offsets_fit_32(g, a.C);
#define SPHOPS_FWD_QUAD(CW, O32) \
  hipLaunchKernelGGL((k_blur_hybrid_fwd_quad<D, P, CW, O32, PARTS>), dim3(wgs), dim3(kThreads), 0, st, g.p, a)
  if (a.C == 16) {
    if (off32) SPHOPS_FWD_QUAD(4, true);
    else SPHOPS_FWD_QUAD(4, false);
  } else {
    if (off32) SPHOPS_FWD_QUAD(8, true);
    else SPHOPS_FWD_QUAD(8, false);
  }
#undef SPHOPS_FWD_QUAD
  SPHOPS_LAUNCHED();
}

// The lane-split pass-B backward over the schedule a.waves2 (positions and
// volumes already packed into a.xw); PARTS as for k_blur_hybrid_bwd_quad.
template <int D, bool P, bool FULL, int PARTS = 3>
void launch_blur_hybrid_bwd_quad_packed(const Grid& g, const OpPtrs& a, hipStream_t st) {
  const uint32_t wgs = schedule_groups(a.nwaves2, a.nwaves2_dev);
  if (wgs == 0) return;
  const bool off32 = row_offsets_fit_32(g, a.C);
#define SPHOPS_BWD_QUAD(CW, O32) \
  hipLaunchKernelGGL((k_blur_hybrid_bwd_quad<D, P, CW, FULL, O32, PARTS>), dim3(wgs), dim3(kThreads), 0, st, g.p, a)
  if (a.C == 16) {
    if (off32) SPHOPS_BWD_QUAD(4, true);
    else SPHOPS_BWD_QUAD(4, false);
  } else {
    if (off32) SPHOPS_BWD_QUAD(8, true);
    else SPHOPS_BWD_QUAD(8, false);
  }
#undef SPHOPS_BWD_QUAD
  SPHOPS_LAUNCHED();
}

template <int D, bool P, bool FULL, int PARTS = 3>
void launch_blur_hybrid_bwd_quad(const Grid& g, OpPtrs a, hipStream_t st) {
  if (g.n_keys == 0) return;
  pack_for<D, VolumeWeights>(g, a, st);
  // the cell kernel serves the tiles' own-cell pairs (3D clamped grids, C =
  // 16); otherwise the rows are read whole
  const bool cells = a.nown != nullptr && a.cells != nullptr && a.cell_count != nullptr && D == 3 && !P &&
                     a.C == 16 && aligned16(a.out1);
  if (!cells) a.nown = nullptr;
  launch_blur_hybrid_bwd_quad_packed<D, P, FULL, PARTS>(g, a, st);
  if constexpr (D == 3 && !P) {
    if (cells) {
      hipLaunchKernelGGL((k_cell_pairs_bwd<D, FULL, PARTS>), dim3(kCellWorkgroups), dim3(kCellThreads), 0, st, g.p,
                         a);
      SPHOPS_LAUNCHED();
    }
  }
}

// Pass-B backward with cell tiles: the tiled kernel serves the particles of
// the units, the lane-split list kernel the others (their own schedule).
template <int D, bool P, bool FULL>
void launch_blur_hybrid_bwd_tiles(const Grid& g, const int32_t* bo, OpPtrs a, hipStream_t st) {
  if (g.n_keys == 0) return;
  pack_for<D, VolumeWeights>(g, a, st);
  hipLaunchKernelGGL((k_blur_hybrid_bwd_tiled<D, P, FULL>), dim3(kTileWorkgroups), dim3(kTileThreads), 0, st, g.p,
                     a, bo);
  SPHOPS_LAUNCHED();
  OpPtrs b = a;
  b.order = a.order_sparse;
  b.waves2 = a.waves_sparse;
  b.nwaves2 = a.nwaves_sparse;
  b.nwaves2_dev = a.nwaves_sparse_dev;
  launch_blur_hybrid_bwd_quad_packed<D, P, FULL>(g, b, st);
}

// Cell tiles of a snapshot (see perception_tiled.hpp): units of up to kTileP
// particles of cells with at least kTileMinOcc, their count on the device,
// and the lane-split schedule of the particles outside them.
template <int D, bool P>
void neighbour_tiles(const Grid& g, const int32_t* bo, const float* x, const int32_t* ncnt, uint2* units,
                     int32_t* unit_count, int32_t* order_sparse, uint2* waves_sparse, int32_t* wave_count_sparse,
                     hipStream_t st) {
  const uint32_t n = (uint32_t)g.n_keys;
  hipLaunchKernelGGL((k_pack<D, kWNone>), grid_for(n), dim3(kThreads), 0, st, x, nullptr, nullptr, g.packed, n);
  SPHOPS_LAUNCHED();
  hipLaunchKernelGGL((k_tile_flags<D, P>), grid_for(n), dim3(kThreads), 0, st, g.p, bo, g.packed, ncnt, g.flags,
                     g.unit_len, g.sparse_len);
  SPHOPS_LAUNCHED();
  exclusive_scan_u32(g, g.flags, n, reinterpret_cast<uint32_t*>(unit_count), st);
  hipLaunchKernelGGL(k_tile_units, grid_for(n), dim3(kThreads), 0, st, g.unit_len, g.flags, n, units);
  SPHOPS_LAUNCHED();
  run_split_schedule(g, g.sparse_len, order_sparse, waves_sparse, wave_count_sparse, st);
}

// Pick the register-channel configuration for C.
template <int D, bool P, template <int, bool, int, bool> class OPT>
void launch_channels(const Grid& g, const int32_t* bo, const OpPtrs& a, hipStream_t st) {
  const uint32_t C = a.C;
  const bool al = aligned16(a.s) && aligned16(a.g) && aligned16(a.g2);
  if (al && C == 16) return launch_pairs<D, P, OPT<D, P, 16, true>>(g, bo, a, st);
  if (al && C == 12) return launch_pairs<D, P, OPT<D, P, 12, true>>(g, bo, a, st);
  if (al && C == 32) return launch_pairs<D, P, OPT<D, P, 32, true>>(g, bo, a, st);
  if (C <= 8) return launch_pairs<D, P, OPT<D, P, 8, false>>(g, bo, a, st);
  if (C <= 16) return launch_pairs<D, P, OPT<D, P, 16, false>>(g, bo, a, st);
  if (C <= 32) return launch_pairs<D, P, OPT<D, P, 32, false>>(g, bo, a, st);
  return launch_pairs<D, P, OPT<D, P, 64, false>>(g, bo, a, st);
}

template <int D, bool P, int CM, bool EX> using BlurBwdFull = OpBlurBwd<D, P, CM, EX, true>;
template <int D, bool P, int CM, bool EX> using BlurBwdDs = OpBlurBwd<D, P, CM, EX, false>;
template <int D, bool P, int CM, bool EX> using GradientBwdFull = OpGradientBwd<D, P, CM, EX, true>;
template <int D, bool P, int CM, bool EX> using GradientBwdDs = OpGradientBwd<D, P, CM, EX, false>;
template <int D, bool P, int CM, bool EX> using GradientBwdFullAcc = OpGradientBwd<D, P, CM, EX, true, true>;
template <int D, bool P, int CM, bool EX> using GradientBwdDsAcc = OpGradientBwd<D, P, CM, EX, false, true>;

template <int D, bool P>
void forward_dispatch(const Grid& g, Op op, const int32_t* bo, const OpPtrs& a_in, hipStream_t st) {
  OpPtrs a = a_in;
  a.bo = bo;
  switch (op) {
    case Op::Count: return launch_pairs<D, P, OpCount<D, P>>(g, bo, a, st);
    case Op::Density: return launch_pairs<D, P, OpDensity<D, P>>(g, bo, a, st);
    case Op::DensityGradient: return launch_pairs<D, P, OpDensityGradient<D, P>>(g, bo, a, st);
    case Op::MomentMatrix: return launch_pairs<D, P, OpMomentMatrix<D, P>>(g, bo, a, st);
    // blur alone stays on the grouped kernel (a row per lane), which is faster
    // for it than the lane-split kernel (0.28 against 0.30 ms at cfg5)
    case Op::Blur: return launch_channels<D, P, OpBlur>(g, bo, a, st);
    case Op::Gradient: return launch_channels<D, P, OpGradient>(g, bo, a, st);
    case Op::GradientHybrid: {
      // over a neighbour list with 16 or 32 channels: the lane-split kernel
      // with the gradient_hybrid part only (its output in out3)
      OpPtrs b = a;
      b.out3 = a.out0;
      if (split_ok(b)) return launch_blur_hybrid_fwd_quad<D, P, 2>(g, b, st);
      return launch_channels<D, P, OpGradientHybrid>(g, bo, a, st);
    }
    case Op::DensityPair: return launch_pairs<D, P, OpDensityPair<D, P>>(g, bo, a, st);
    case Op::BlurGradientHybrid:
      if (split_ok(a)) return launch_blur_hybrid_fwd_quad<D, P>(g, a, st);
      return launch_channels<D, P, OpBlurGradientHybrid>(g, bo, a, st);
    case Op::NeighbourCandidates:
      if (g.n_keys) neighbour_candidates<D, P>(g, bo, a.x, st);
      return;
    case Op::NeighbourFill:
      if (g.n_keys) neighbour_fill<D, P>(g, a.bo, a.x, a.iout3, a.iout, a.iout2, a.used, a.cap, a.fill_tiles, st);
      return;
    case Op::NeighbourTiles:
      if (g.n_keys)
        neighbour_tiles<D, P>(g, bo, a.x, a.ncnt, const_cast<uint2*>(a.tile_units), const_cast<int32_t*>(a.tile_count),
                              const_cast<int32_t*>(a.order_sparse), const_cast<uint2*>(a.waves_sparse),
                              const_cast<int32_t*>(a.nwaves_sparse_dev), st);
      return;
  }
  throw Error("unknown forward operator");
}

template <int D, bool P>
void backward_dispatch(const Grid& g, Op op, bool full, const int32_t* bo, const OpPtrs& a_in, hipStream_t st) {
  OpPtrs a = a_in;
  a.bo = bo;
  switch (op) {
    case Op::Density: return launch_pairs<D, P, OpDensityBwd<D, P>>(g, bo, a, st);
    case Op::DensityGradient: return launch_pairs<D, P, OpDensityGradientBwd<D, P>>(g, bo, a, st);
    case Op::MomentMatrix: return launch_pairs<D, P, OpMomentMatrixBwd<D, P>>(g, bo, a, st);
    case Op::Blur:
      // over a neighbour list with 16 or 32 channels: the lane-split kernel
      // with the blur terms only
      if (split_ok(a)) {
        if (full) return launch_blur_hybrid_bwd_quad<D, P, true, 1>(g, a, st);
        return launch_blur_hybrid_bwd_quad<D, P, false, 1>(g, a, st);
      }
      if (full) return launch_channels<D, P, BlurBwdFull>(g, bo, a, st);
      return launch_channels<D, P, BlurBwdDs>(g, bo, a, st);
    case Op::Gradient:
    case Op::GradientHybrid: {
      // the same with the gradient terms only (its upstream in g2)
      OpPtrs b = a;
      b.g2 = a.g;
      b.g = nullptr;
      if (split_ok(b)) {
        if (full) return launch_blur_hybrid_bwd_quad<D, P, true, 2>(g, b, st);
        return launch_blur_hybrid_bwd_quad<D, P, false, 2>(g, b, st);
      }
      if (full) return launch_channels<D, P, GradientBwdFull>(g, bo, a, st);
      return launch_channels<D, P, GradientBwdDs>(g, bo, a, st);
    }
    case Op::DensityPair: return launch_pairs<D, P, OpDensityPairBwd<D, P>>(g, bo, a, st);
    case Op::BlurGradientHybrid: {
      if (split_ok(a) && a.C == 16 && a.tile_units != nullptr && a.waves_sparse != nullptr) {
        if (full) return launch_blur_hybrid_bwd_tiles<D, P, true>(g, bo, a, st);
        return launch_blur_hybrid_bwd_tiles<D, P, false>(g, bo, a, st);
      }
      if (split_ok(a)) {
        if (full) return launch_blur_hybrid_bwd_quad<D, P, true>(g, a, st);
        return launch_blur_hybrid_bwd_quad<D, P, false>(g, a, st);
      }
      // blur's backward stores, the gradient's backward (upstream2) adds
      OpPtrs b = a;
      b.g2 = nullptr;
      backward_dispatch<D, P>(g, Op::Blur, full, bo, b, st);
      b.g = a.g2;
      if (full) return launch_channels<D, P, GradientBwdFullAcc>(g, bo, b, st);
      return launch_channels<D, P, GradientBwdDsAcc>(g, bo, b, st);
    }
    default:
      break;
  }
  throw Error("operator has no backward");
}

}  // namespace pk
}  // namespace sphops
