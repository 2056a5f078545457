// Fused perception features of NPA.perceive (models/npa.py:87-137 of the
// reference), forward and backward, for gfx950.
//
// The reference builds the MLP input z from the perception operators with a
// chain of torch elementwise ops: grad_s * coef, log-normalisation
// log(1 + |v|) * v / max(|v|, 1e-12) over the spatial axis
// (models/npa.py:83-85), density_gradient * coef^(1+D) / N and its
// log-normalisation, then torch.cat([s, blur, grad_s.view(B, N, C*D),
// grad_rho], -1).  Here one kernel writes z from the four operator outputs
// and one kernel maps dL/dz back to them.  Both are bound by HBM: z and the
// operator outputs are read or written once each, through an LDS tile.
#include "sphops_internal.hpp"

namespace sphops {

namespace {

constexpr int kThreads = 256;
constexpr float kNormEps = 1e-12f;  // torch.nn.functional.normalize's default eps

// v <- log(1 + |v|) * v / max(|v|, eps)
template <int D>
__device__ __forceinline__ void log_normalize(float* v) {
  float n2 = 0.0f;
#pragma unroll
  for (int e = 0; e < D; ++e) n2 += v[e] * v[e];
  const float u = sqrtf(n2);
  const float f = log1pf(u) / fmaxf(u, kNormEps);
#pragma unroll
  for (int e = 0; e < D; ++e) v[e] *= f;
}

// w <- J^T w for the log-normalisation at v (J symmetric):
// J = (phi / m) I + (phi' / m - phi / m^2) v v^T / u, phi = log(1 + u),
// m = max(u, eps), phi' = 1 / (1 + u) (the v v^T / u term is absent at u = 0,
// where torch's norm has a zero gradient; for u >= eps, m = u).
template <int D>
__device__ __forceinline__ void log_normalize_backward(const float* v, float* w) {
  float n2 = 0.0f, vw = 0.0f;
#pragma unroll
  for (int e = 0; e < D; ++e) {
    n2 += v[e] * v[e];
    vw += v[e] * w[e];
  }
  const float u = sqrtf(n2);
  const float m = fmaxf(u, kNormEps);
  const float phi = log1pf(u);
  const float a = phi / m;
  float b = 0.0f;
  if (u > 0.0f) {
    const float dm = u >= kNormEps ? phi / (m * m) : 0.0f;  // d(1/m)/du * phi; m is constant below eps
    b = (1.0f / ((1.0f + u) * m) - dm) / u;
  }
#pragma unroll
  for (int e = 0; e < D; ++e) w[e] = a * w[e] + b * vw * v[e];
}

// Particles per workgroup: a tile of T rows of z (W floats each) lives in LDS,
// so every global access is a contiguous, coalesced run: the tile's slices of
// s, blur, grad_s, grad_rho (and of d_s ... on the way back) and its rows of z.
constexpr uint32_t kTileFloats = 5120;  // 20 KiB; W <= 5 * 64 + 3 for C <= 64

__host__ __device__ inline uint32_t feature_width(uint32_t C, int D, int flags) {
  return 2u * C + ((flags & SPHOPS_GLUE_STATE_GRAD) ? C * (uint32_t)D : 0u) +
         ((flags & SPHOPS_GLUE_DENSITY_GRAD) ? (uint32_t)D : 0u);
}

inline uint32_t tile_particles(uint32_t W) { return std::min<uint32_t>(64u, kTileFloats / W); }

// i / d and i % d for i < 2^24: a float quotient, then one correction step
__device__ __forceinline__ uint32_t div_small(uint32_t i, uint32_t d, float inv_d, uint32_t& r) {
  uint32_t q = (uint32_t)(((float)i + 0.5f) * inv_d);
  int32_t rr = (int32_t)i - (int32_t)(q * d);
  if (rr < 0) {
    --q;
    rr += (int32_t)d;
  } else if (rr >= (int32_t)d) {
    ++q;
    rr -= (int32_t)d;
  }
  r = (uint32_t)rr;
  return q;
}

// A tile's rows of z and its slices of s, blur, grad_s, grad_rho hold the same
// number of floats, t * W.  Index i of that range maps to one source (or
// destination) float and one element of the LDS tile: seg_of() gives both.
// Each thread moves the indices tid + kThreads * m, all loads issued before
// the LDS writes, so a wave keeps kSlots loads in flight.
constexpr int kSlots = (int)(kTileFloats / kThreads);
static_assert(kSlots * kThreads == (int)kTileFloats, "tile must split evenly over the threads");

struct TileMap {
  uint32_t C, CD, D, W, o, tC, tCD;  // o: offset of the density gradient in a row of z
  float invC, invCD;
  // segment of index i (0 s, 1 blur, 2 grad_s, 3 grad_rho), its offset j in
  // that segment's slice, and the matching element of the tile
  __device__ __forceinline__ int seg_of(uint32_t i, uint32_t& j, uint32_t& e) const {
    uint32_t r;
    if (i < 2u * tC) {
      const int sgm = i < tC ? 0 : 1;
      j = sgm ? i - tC : i;
      const uint32_t p = div_small(j, C, invC, r);
      e = p * W + (sgm ? C : 0u) + r;
      return sgm;
    }
    if (i < 2u * tC + tCD) {
      j = i - 2u * tC;
      const uint32_t p = div_small(j, CD, invCD, r);
      e = p * W + 2u * C + r;
      return 2;
    }
    j = i - 2u * tC - tCD;
    const uint32_t p = j / D;
    e = p * W + o + (j - p * D);
    return 3;
  }
};

template <int D>
__device__ __forceinline__ TileMap tile_map(uint32_t C, uint32_t t, int flags) {
  const bool sg = flags & SPHOPS_GLUE_STATE_GRAD;
  TileMap m;
  m.C = C;
  m.CD = C * D;
  m.D = D;
  m.W = feature_width(C, D, flags);
  m.o = 2u * C + (sg ? m.CD : 0u);
  m.tC = t * C;
  m.tCD = sg ? t * m.CD : 0u;
  m.invC = 1.0f / (float)C;
  m.invCD = 1.0f / (float)m.CD;
  return m;
}

template <int D>
__global__ __launch_bounds__(kThreads) void k_glue_forward(const float* __restrict__ s, const float* __restrict__ blur,
                                                           const float* __restrict__ grad_s,
                                                           const float* __restrict__ grad_rho, float* __restrict__ z,
                                                           uint64_t n, uint32_t C, uint32_t T, float coef_s,
                                                           float coef_rho, float total_mass, int flags) {
  __shared__ float tile[kTileFloats];
  const bool lng = flags & SPHOPS_GLUE_LOG_NORM_GRAD, lnd = flags & SPHOPS_GLUE_LOG_NORM_DENSITY_GRAD;
  const uint64_t k0 = (uint64_t)blockIdx.x * T;
  const uint32_t t = (uint32_t)min<uint64_t>(T, n - k0);
  const TileMap mp = tile_map<D>(C, t, flags);
  const uint32_t tW = t * mp.W, tid = threadIdx.x;
  const float inv_mass = 1.0f / total_mass;
  s += k0 * C;
  blur += k0 * C;
  grad_s += k0 * mp.CD;
  grad_rho += k0 * D;
  float val[kSlots];
#pragma unroll
  for (int m = 0; m < kSlots; ++m) {
    const uint32_t i = tid + kThreads * m;
    if (i < tW) {
      uint32_t j, e;
      const int g = mp.seg_of(i, j, e);
      const float* src = g == 0 ? s : g == 1 ? blur : g == 2 ? grad_s : grad_rho;
      val[m] = src[j];
    }
  }
#pragma unroll
  for (int m = 0; m < kSlots; ++m) {
    const uint32_t i = tid + kThreads * m;
    if (i < tW) {
      uint32_t j, e;
      const int g = mp.seg_of(i, j, e);
      // grad_rho * coef_rho / N as torch rounds it: (g * coef_rho) * fp32(1 / N)
      tile[e] = g < 2 ? val[m] : g == 2 ? val[m] * coef_s : val[m] * coef_rho * inv_mass;
    }
  }
  __syncthreads();
  if (mp.tCD && lng) {
    for (uint32_t v = tid; v < mp.tC; v += kThreads) {
      uint32_t c;
      const uint32_t p = div_small(v, C, mp.invC, c);
      log_normalize<D>(&tile[p * mp.W + 2u * C + c * D]);
    }
  }
  if ((flags & SPHOPS_GLUE_DENSITY_GRAD) && lnd) {
    for (uint32_t p = tid; p < t; p += kThreads) log_normalize<D>(&tile[p * mp.W + mp.o]);
  }
  __syncthreads();
  float* zt = z + k0 * mp.W;
#pragma unroll
  for (int m = 0; m < kSlots; ++m) {
    const uint32_t i = tid + kThreads * m;
    if (i < tW) zt[i] = tile[i];
  }
}

template <int D>
__global__ __launch_bounds__(kThreads) void k_glue_backward(const float* __restrict__ dz,
                                                            const float* __restrict__ grad_s,
                                                            const float* __restrict__ grad_rho,
                                                            float* __restrict__ d_s, float* __restrict__ d_blur,
                                                            float* __restrict__ d_grad_s,
                                                            float* __restrict__ d_grad_rho, uint64_t n, uint32_t C,
                                                            uint32_t T, float coef_s, float coef_rho,
                                                            float total_mass, int flags) {
  __shared__ float tile[kTileFloats];
  const bool lng = flags & SPHOPS_GLUE_LOG_NORM_GRAD, lnd = flags & SPHOPS_GLUE_LOG_NORM_DENSITY_GRAD;
  const uint64_t k0 = (uint64_t)blockIdx.x * T;
  const uint32_t t = (uint32_t)min<uint64_t>(T, n - k0);
  const TileMap mp = tile_map<D>(C, t, flags);
  const uint32_t tW = t * mp.W, tid = threadIdx.x;
  const float inv_mass = 1.0f / total_mass;
  const float* dzt = dz + k0 * mp.W;
  {
    float val[kSlots];
#pragma unroll
    for (int m = 0; m < kSlots; ++m) {
      const uint32_t i = tid + kThreads * m;
      if (i < tW) val[m] = dzt[i];
    }
#pragma unroll
    for (int m = 0; m < kSlots; ++m) {
      const uint32_t i = tid + kThreads * m;
      if (i < tW) tile[i] = val[m];
    }
  }
  __syncthreads();
  // J^T of the log-normalisations, in place; the scale factors fold in below
  if (mp.tCD && lng && d_grad_s) {
    for (uint32_t v = tid; v < mp.tC; v += kThreads) {
      uint32_t c;
      const uint32_t p = div_small(v, C, mp.invC, c);
      float g[D];
#pragma unroll
      for (int e = 0; e < D; ++e) g[e] = grad_s[(k0 * C + v) * D + e] * coef_s;
      log_normalize_backward<D>(g, &tile[p * mp.W + 2u * C + c * D]);
    }
  }
  if ((flags & SPHOPS_GLUE_DENSITY_GRAD) && lnd && d_grad_rho) {
    for (uint32_t p = tid; p < t; p += kThreads) {
      float g[D];
#pragma unroll
      for (int e = 0; e < D; ++e) g[e] = grad_rho[(k0 + p) * D + e] * coef_rho * inv_mass;
      log_normalize_backward<D>(g, &tile[p * mp.W + mp.o]);
    }
  }
  __syncthreads();
  float* dst0 = d_s ? d_s + k0 * C : nullptr;
  float* dst1 = d_blur ? d_blur + k0 * C : nullptr;
  float* dst2 = d_grad_s ? d_grad_s + k0 * mp.CD : nullptr;
  float* dst3 = d_grad_rho ? d_grad_rho + k0 * D : nullptr;
#pragma unroll
  for (int m = 0; m < kSlots; ++m) {
    const uint32_t i = tid + kThreads * m;
    if (i < tW) {
      uint32_t j, e;
      const int g = mp.seg_of(i, j, e);
      float* dst = g == 0 ? dst0 : g == 1 ? dst1 : g == 2 ? dst2 : dst3;
      if (dst) dst[j] = g < 2 ? tile[e] : g == 2 ? tile[e] * coef_s : tile[e] * inv_mass * coef_rho;
    }
  }
}


// ---- Euler update of step_euler (models/npa.py:125-133, 178-200) --------
// From the MLP output y = [a (D), ds (C)] per particle: dx = alpha * a * eps /
// (1 + |a|), x_out = x_bin + dt * pad(dx) * m (+ noise * noise_std * sqrt_dt
// * m), s_out = s_bin + dt * ds * m, |dx| per particle.  One launch, two
// kinds of waves: the first n * C threads stream the state channels (thread
// (k, c)), the next n threads each take one particle's position row and |dx|,
// so no wave carries the position arithmetic as a divergent branch.

template <int D>
__device__ __forceinline__ float scaled_step(const float* a, float alpha, float eps, float* dx) {
  float n2 = 0.0f;
#pragma unroll
  for (int e = 0; e < D; ++e) n2 += a[e] * a[e];
  const float den = 1.0f + sqrtf(n2);
  float d2 = 0.0f;
#pragma unroll
  for (int e = 0; e < D; ++e) {
    dx[e] = alpha * a[e] * eps / den;  // ((alpha * a) * eps) / (1 + |a|), the reference's order
    d2 += dx[e] * dx[e];
  }
  return sqrtf(d2);
}

template <int D, typename I>
__global__ __launch_bounds__(kThreads) void k_euler_forward(const float* __restrict__ y,
                                                            const float* __restrict__ x_bin,
                                                            const float* __restrict__ s_bin,
                                                            const float* __restrict__ mask,
                                                            const float* __restrict__ noise, float* __restrict__ x_out,
                                                            float* __restrict__ s_out, float* __restrict__ dx_norm,
                                                            uint64_t n, uint32_t C, uint32_t P, float alpha, float eps,
                                                            float dt, float noise_std, float sqrt_dt) {
  const I t = (I)blockIdx.x * kThreads + threadIdx.x;
  const I nC = (I)n * C;
  if (t < nC) {
    const I k = t / C;  // 32-bit division whenever n * C fits
    const uint32_t c = (uint32_t)(t - k * C);
    const float m = mask ? mask[k] : 1.0f;
    s_out[t] = s_bin[t] + dt * y[(uint64_t)k * (D + C) + D + c] * m;
    return;
  }
  const I k = t - nC;
  if (k >= (I)n) return;
  const float m = mask ? mask[k] : 1.0f;
  const float* yr = y + (uint64_t)k * (D + C);
  float a[D], dx[D];
#pragma unroll
  for (int e = 0; e < D; ++e) a[e] = yr[e];
  const float dn = scaled_step<D>(a, alpha, eps, dx);
  constexpr int PW = D == 2 ? 2 : 4;  // position row width (the C ABI checks P == PW)
#pragma unroll
  for (int e = 0; e < PW; ++e) {
    const uint64_t o = (uint64_t)k * PW + e;
    float xo = x_bin[o] + dt * (e < D ? dx[e < D ? e : 0] : 0.0f) * m;  // lanes >= D: the zero padding
    if (noise) xo += noise[o] * noise_std * sqrt_dt * m;
    x_out[o] = xo;
  }
  if (dx_norm) dx_norm[k] = dn;
}

// dL/dy from dL/dx_out, dL/ds_out and dL/d|dx| (each may be NULL: zero);
// threads as in k_euler_forward (state channels, then one per particle).
// With kappa = alpha * eps, u = |a|, g = dt * m * dL/dx_out[:D] + dL/d|dx| *
// dx / |dx|: dL/da = kappa * (g / (1 + u) - (a.g) a / (u (1 + u)^2)), whose
// second term and the |dx| term vanish at a = 0 (torch's norm has a zero
// gradient there).  With r = 1 / (1 + u): dx = kappa a r and |dx| = |kappa|
// u r, so the |dx| term of g is dL/d|dx| sign(kappa) a / u.
template <int D, typename I>
__global__ __launch_bounds__(kThreads) void k_euler_backward(const float* __restrict__ y,
                                                             const float* __restrict__ mask,
                                                             const float* __restrict__ d_x_out,
                                                             const float* __restrict__ d_s_out,
                                                             const float* __restrict__ d_dx_norm,
                                                             float* __restrict__ d_y, uint64_t n, uint32_t C,
                                                             uint32_t P, float alpha, float eps, float dt) {
  const I t = (I)blockIdx.x * kThreads + threadIdx.x;
  const I nC = (I)n * C;
  if (t < nC) {
    const I k = t / C;
    const uint32_t c = (uint32_t)(t - k * C);
    const float m = mask ? mask[k] : 1.0f;
    d_y[(uint64_t)k * (D + C) + D + c] = d_s_out ? dt * m * d_s_out[t] : 0.0f;
    return;
  }
  const I k = t - nC;
  if (k >= (I)n) return;
  const float m = mask ? mask[k] : 1.0f;
  const float* yr = y + (uint64_t)k * (D + C);
  float a[D], g[D];
  float u2 = 0.0f;
#pragma unroll
  for (int e = 0; e < D; ++e) {
    a[e] = yr[e];
    u2 += a[e] * a[e];
  }
  const float u = sqrtf(u2);
  const float kappa = alpha * eps;
  const float r = 1.0f / (1.0f + u);
  const float iu = u > 0.0f ? 1.0f / u : 0.0f;
  const float gn = (d_dx_norm && kappa != 0.0f) ? (kappa < 0.0f ? -d_dx_norm[k] : d_dx_norm[k]) * iu : 0.0f;
  float ag = 0.0f;
#pragma unroll
  for (int e = 0; e < D; ++e) {
    g[e] = (d_x_out ? dt * m * d_x_out[(uint64_t)k * P + e] : 0.0f) + gn * a[e];
    ag += a[e] * g[e];
  }
  const float b = ag * r * iu;
#pragma unroll
  for (int e = 0; e < D; ++e) d_y[(uint64_t)k * (D + C) + e] = kappa * r * (g[e] - b * a[e]);
}

}  // namespace

void run_glue_forward(int dim, const float* s, const float* blur, const float* grad_s, const float* grad_rho,
                      float* z, uint64_t n, uint32_t C, float coef_s, float coef_rho, float total_mass, int flags,
                      hipStream_t st) {
  if (n == 0) return;
  const uint32_t T = tile_particles(feature_width(C, dim, flags));
  const dim3 grid((uint32_t)((n + T - 1) / T));
  if (dim == 2) {
    hipLaunchKernelGGL(k_glue_forward<2>, grid, dim3(kThreads), 0, st, s, blur, grad_s, grad_rho, z, n, C, T, coef_s,
                       coef_rho, total_mass, flags);
  } else {
    hipLaunchKernelGGL(k_glue_forward<3>, grid, dim3(kThreads), 0, st, s, blur, grad_s, grad_rho, z, n, C, T, coef_s,
                       coef_rho, total_mass, flags);
  }
  SPHOPS_LAUNCHED();
}

void run_glue_backward(int dim, const float* dz, const float* grad_s, const float* grad_rho, float* d_s,
                       float* d_blur, float* d_grad_s, float* d_grad_rho, uint64_t n, uint32_t C, float coef_s,
                       float coef_rho, float total_mass, int flags, hipStream_t st) {
  if (n == 0) return;
  const uint32_t T = tile_particles(feature_width(C, dim, flags));
  const dim3 grid((uint32_t)((n + T - 1) / T));
  if (dim == 2) {
    hipLaunchKernelGGL(k_glue_backward<2>, grid, dim3(kThreads), 0, st, dz, grad_s, grad_rho, d_s, d_blur, d_grad_s,
                       d_grad_rho, n, C, T, coef_s, coef_rho, total_mass, flags);
  } else {
    hipLaunchKernelGGL(k_glue_backward<3>, grid, dim3(kThreads), 0, st, dz, grad_s, grad_rho, d_s, d_blur, d_grad_s,
                       d_grad_rho, n, C, T, coef_s, coef_rho, total_mass, flags);
  }
  SPHOPS_LAUNCHED();
}

void run_euler_forward(int dim, const float* y, const float* x_bin, const float* s_bin, const float* mask,
                       const float* noise, float* x_out, float* s_out, float* dx_norm, uint64_t n, uint32_t C,
                       uint32_t P, float alpha, float eps, float dt, float noise_std, float sqrt_dt, hipStream_t st) {
  if (n == 0) return;
  const uint64_t threads = n * (C + 1ull);  // n * C state threads, then n particle threads
  const dim3 grid((uint32_t)((threads + kThreads - 1) / kThreads));
  const bool narrow = threads + kThreads <= 0xFFFFFFFFull;
  auto kern = dim == 2 ? (narrow ? k_euler_forward<2, uint32_t> : k_euler_forward<2, uint64_t>)
                       : (narrow ? k_euler_forward<3, uint32_t> : k_euler_forward<3, uint64_t>);
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, st, y, x_bin, s_bin, mask, noise, x_out, s_out, dx_norm, n, C, P,
                     alpha, eps, dt, noise_std, sqrt_dt);
  SPHOPS_LAUNCHED();
}

void run_euler_backward(int dim, const float* y, const float* mask, const float* d_x_out, const float* d_s_out,
                        const float* d_dx_norm, float* d_y, uint64_t n, uint32_t C, uint32_t P, float alpha,
                        float eps, float dt, hipStream_t st) {
  if (n == 0) return;
  const uint64_t threads = n * (C + 1ull);
  const dim3 grid((uint32_t)((threads + kThreads - 1) / kThreads));
  const bool narrow = threads + kThreads <= 0xFFFFFFFFull;
  auto kern = dim == 2 ? (narrow ? k_euler_backward<2, uint32_t> : k_euler_backward<2, uint64_t>)
                       : (narrow ? k_euler_backward<3, uint32_t> : k_euler_backward<3, uint64_t>);
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, st, y, mask, d_x_out, d_s_out, d_dx_norm, d_y, n, C, P, alpha, eps,
                     dt);
  SPHOPS_LAUNCHED();
}

}  // namespace sphops
