// Device-side grid semantics and SPH pair kernels for the gfx950 sphops path.
//
// Grid semantics follow the reference's GridConfig (sphops/utils.cuh:303-524):
// cell = floor(x * inv_eps) + G/2 with flush-to-zero behaviour of the
// reference's fast-math build, clamp or periodic wrap per axis, row-major hash
// (grid mode) or 10-bit Morton interleave (particle mode).  Pair kernels follow
// sphops/utils.cuh:199-279: poly6 W = max(0, (h^2 - |r|^2)^3), spiky
// K = 3 (h - |r|)^2 / |r| * r and its Jacobian.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <float.h>
#include <limits.h>

namespace sphops {

constexpr int kWave = 64;

// Everything a kernel needs to know about the grid.  Passed by value.
struct GridParams {
  int gs[3];          // cells per axis (gs[2] == 1 in 2D)
  int half_gs[3];     // gs/2 (integer division), the cell-index offset
  float eps;          // interaction radius h (fp32)
  float inv_eps;      // 1.0f / eps computed on the host in fp32
  float eps2;         // eps * eps in fp32
  float L[3];         // periodic box per axis: float(gs) * eps
  float half_L[3];    // 0.5f * L
  float c6;           // poly6 coefficient
  float cs;           // spiky coefficient
  uint32_t N;         // particles per cloud
  uint32_t B;         // clouds
  uint32_t G;         // cells per cloud
  uint32_t maxp;      // max particles per block-table row
  int morton;         // 1: particle mode (Morton hash), 0: grid mode
};

// ------------------------------------------------------------------ cells

// __float2int_rd(x * inv_eps) of a flush-to-zero build, saturating, NaN -> 0.
__device__ __forceinline__ int floor_cell(float x, float inv_eps) {
  float xz = (fabsf(x) < FLT_MIN) ? 0.0f : x;
  float p = xz * inv_eps;
  if (fabsf(p) < FLT_MIN) p = 0.0f;
  if (p != p) return 0;
  if (p >= 2147483648.0f) return INT_MAX;
  if (p < -2147483648.0f) return INT_MIN;
  return (int)floorf(p);
}

__device__ __forceinline__ int wrap_add(int a, int b) {
  return (int)((unsigned)a + (unsigned)b);
}

__device__ __forceinline__ int bound_axis(int c, int g, bool periodic) {
  if (periodic) {
    int m = c % g;
    return m < 0 ? m + g : m;
  }
  return min(max(c, 0), g - 1);
}

// Spread the 10 low bits of v: one zero bit between them (2D) or two (3D).
template <int D>
__device__ __forceinline__ uint32_t spread_bits(uint32_t v) {
  v &= 0x3FFu;
  if constexpr (D == 2) {
    v = (v | (v << 8)) & 0x00FF00FFu;
    v = (v | (v << 4)) & 0x0F0F0F0Fu;
    v = (v | (v << 2)) & 0x33333333u;
    v = (v | (v << 1)) & 0x55555555u;
  } else {
    v = (v | (v << 16)) & 0x030000FFu;
    v = (v | (v << 8)) & 0x0300F00Fu;
    v = (v | (v << 4)) & 0x030C30C3u;
    v = (v | (v << 2)) & 0x09249249u;
  }
  return v;
}

template <int D>
__device__ __forceinline__ uint32_t cell_hash(const GridParams& g, const int* c) {
  if (g.morton) {
    uint32_t h = spread_bits<D>((uint32_t)c[0]) | (spread_bits<D>((uint32_t)c[1]) << 1);
    if constexpr (D == 3) h |= spread_bits<D>((uint32_t)c[2]) << 2;
    return h;
  }
  if constexpr (D == 2) return (uint32_t)(c[1] * g.gs[0] + c[0]);
  return (uint32_t)((c[2] * g.gs[1] + c[1]) * g.gs[0] + c[0]);
}

template <int D, bool PERIODIC>
__device__ __forceinline__ void pos2cell(const GridParams& g, const float* x, int* c) {
#pragma unroll
  for (int d = 0; d < D; ++d)
    c[d] = bound_axis(wrap_add(floor_cell(x[d], g.inv_eps), g.half_gs[d]), g.gs[d], PERIODIC);
}

// ------------------------------------------------------------ positions

template <int D> struct PosT;
template <> struct PosT<2> { using type = float2; };
template <> struct PosT<3> { using type = float4; };

template <int D>
__device__ __forceinline__ void load_pos(const float* __restrict__ X, uint32_t k, float* p) {
  if constexpr (D == 2) {
    float2 v = reinterpret_cast<const float2*>(X)[k];
    p[0] = v.x; p[1] = v.y;
  } else {
    float4 v = reinterpret_cast<const float4*>(X)[k];
    p[0] = v.x; p[1] = v.y; p[2] = v.z;
  }
}

// Periodic minimum image of one displacement component (utils.cuh:321-331).
__device__ __forceinline__ float wrap_periodic(float d, float L, float half_L) {
#pragma clang fp contract(off)
  if (L <= 0.0f) return d;
  float t = fmodf(d + half_L, L);
  if (t < 0.0f) t += L;
  return t - half_L;
}

// r = to - from (wrapped when periodic) and |r|^2, in fp32 with no fused
// multiply-add, so the in-radius decision is reproducible on the CPU.
template <int D, bool PERIODIC>
__device__ __forceinline__ float displacement(const GridParams& g, const float* from, const float* to, float* r) {
#pragma clang fp contract(off)
#pragma unroll
  for (int d = 0; d < D; ++d) {
    float v = to[d] - from[d];
    if constexpr (PERIODIC) v = wrap_periodic(v, g.L[d], g.half_L[d]);
    r[d] = v;
  }
  float acc = r[0] * r[0];
#pragma unroll
  for (int d = 1; d < D; ++d) acc = acc + r[d] * r[d];
  return acc;
}

// -------------------------------------------------------------- kernels

__device__ __forceinline__ float poly6(float eps2, float d2) {
  float t = eps2 - d2;
  return fmaxf(0.0f, t * t * t);
}

// Hardware reciprocal square root and reciprocal (v_rsq_f32 / v_rcp_f32,
// 1 ulp): the pair kernels take 1/|r| from one v_rsq and |r| = |r|^2 / |r|
// as their product (one quarter-rate instruction instead of v_sqrt and
// v_rcp); the in-radius decision never depends on them (it compares |r|^2
// with eps^2).
__device__ __forceinline__ float fast_rsq(float v) { return __builtin_amdgcn_rsqf(v); }
__device__ __forceinline__ float fast_rcp(float v) { return __builtin_amdgcn_rcpf(v); }

// Spiky magnitude 3 (h - d)^2 / d for 0 < d < h, else 0; returns d = |r|
// (0 for d2 = 0) and, if asked, 1/d (meaningful for d2 > 0 only).
__device__ __forceinline__ float spiky_mag(float eps, float d2, float* d_out, float* di_out = nullptr) {
  const float di = fast_rsq(d2);
  const float d = d2 == 0.0f ? 0.0f : d2 * di;
  *d_out = d;
  if (di_out != nullptr) *di_out = di;
  if (d2 == 0.0f || !(d < eps)) return 0.0f;
  const float t = eps - d;
  return 3.0f * t * t * di;
}

// grad_out += J(r) * v with J = dK/dr (utils.cuh:242-260); no-op outside (0, h).
template <int D>
__device__ __forceinline__ void spiky_jacobian_apply(const float* r, float d2, float eps, float eps2,
                                                     const float* v, float* out) {
  if (d2 == 0.0f || !(d2 < eps2)) return;
  const float di = fast_rsq(d2);
  const float d = d2 * di;
  const float a = 3.0f * (eps - d) * (eps - d) * di;   // diagonal part
  const float b = 3.0f * (eps2 - d2) * di * di * di;   // r r^T part
  float rv = 0.0f;
#pragma unroll
  for (int e = 0; e < D; ++e) rv += r[e] * v[e];
#pragma unroll
  for (int e = 0; e < D; ++e) out[e] += a * v[e] - b * r[e] * rv;
}

// ------------------------------------------------------------ utilities

// Map hardware workgroup ids so that each XCD (workgroups are dealt round
// robin over the 8 XCDs) gets one contiguous range of logical ids; neighbour
// data of adjacent sorted particles then shares one L2.
__device__ __forceinline__ uint32_t xcd_block_id() {
  const uint32_t nb = gridDim.x, x = blockIdx.x;
  const uint32_t xcd = x & 7u, q = nb >> 3, rem = nb & 7u;
  return xcd * q + min(xcd, rem) + (x >> 3);
}

// The same mapping over the first nb_live logical ids of a launch of at least
// 8 * ceil(nb_live / 8) workgroups (a launch sized by an upper bound);
// workgroups past them get UINT32_MAX.
__device__ __forceinline__ uint32_t xcd_block_id(uint32_t nb_live) {
  const uint32_t x = blockIdx.x;
  const uint32_t xcd = x & 7u, q = nb_live >> 3, rem = nb_live & 7u;
  const uint32_t k = x >> 3;
  return k < q + (xcd < rem ? 1u : 0u) ? xcd * q + min(xcd, rem) + k : 0xFFFFFFFFu;
}

// The first nb_live logical ids dealt to the eight XCDs in chunks of
// kXcdChunk consecutive ids, the XCDs taking turns chunk by chunk: a chunk
// keeps neighbouring ids (neighbouring space) on one XCD's L2, and the turns
// give every XCD a share of every part of the id range, so that no XCD draws
// only the costly ones (contiguous eighths leave the XCDs that get the sparse
// regions idle for up to half the launch).  Workgroup x runs on XCD x mod 8
// and is its XCD's (x / 8)-th; a launch of at least 8 * ceil(nb_live / 8)
// workgroups covers every id, the workgroups past them get UINT32_MAX.
constexpr uint32_t kXcdChunk = 64;
__device__ __forceinline__ uint32_t xcd_block_id_chunked(uint32_t nb_live) {
  const uint32_t x = blockIdx.x, xcd = x & 7u, k = x >> 3;
  const uint32_t per_xcd = (nb_live + 7u) >> 3;
  if (k >= per_xcd) return 0xFFFFFFFFu;
  const uint32_t whole = per_xcd / kXcdChunk * kXcdChunk;  // ids of each XCD in whole chunks
  const uint32_t id = k < whole ? ((k / kXcdChunk) * 8u + xcd) * kXcdChunk + k % kXcdChunk
                                : 8u * whole + xcd * (per_xcd - whole) + (k - whole);
  return id < nb_live ? id : 0xFFFFFFFFu;
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

}  // namespace sphops
