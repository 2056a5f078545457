// Fused perception features of NPA.perceive (models/npa.py:87-137 of the
// reference), forward and backward, for gfx950.
//
// The reference builds the MLP input z from the perception operators with a
// chain of torch elementwise ops: grad_s * coef, log-normalisation
// log(1 + |v|) * v / max(|v|, 1e-12) over the spatial axis
// (models/npa.py:83-85), density_gradient * coef^(1+D) / N and its
// log-normalisation, then torch.cat([s, blur, grad_s.view(B, N, C*D),
// grad_rho], -1).  Here one kernel writes z from the four operator outputs
// and one kernel maps dL/dz back to them.  One thread serves one (particle,
// channel): it moves channel c of s and blur and the D components of
// grad_s[c]; channel 0 also serves the density gradient.
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

template <int D>
__global__ __launch_bounds__(kThreads) void k_glue_forward(const float* __restrict__ s, const float* __restrict__ blur,
                                                           const float* __restrict__ grad_s,
                                                           const float* __restrict__ grad_rho, float* __restrict__ z,
                                                           uint64_t n, uint32_t C, float coef_s, float coef_rho,
                                                           float total_mass, int flags) {
  const uint64_t t = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= n * C) return;
  const uint64_t k = t / C;
  const uint32_t c = (uint32_t)(t - k * C);
  const bool sg = flags & SPHOPS_GLUE_STATE_GRAD, lng = flags & SPHOPS_GLUE_LOG_NORM_GRAD;
  const bool dg = flags & SPHOPS_GLUE_DENSITY_GRAD, lnd = flags & SPHOPS_GLUE_LOG_NORM_DENSITY_GRAD;
  const uint64_t W = 2u * C + (sg ? (uint64_t)C * D : 0u) + (dg ? D : 0u);
  float* zr = z + k * W;
  zr[c] = s[k * C + c];
  zr[C + c] = blur[k * C + c];
  if (sg) {
    float v[D];
#pragma unroll
    for (int e = 0; e < D; ++e) v[e] = grad_s[(k * C + c) * D + e] * coef_s;
    if (lng) log_normalize<D>(v);
#pragma unroll
    for (int e = 0; e < D; ++e) zr[2u * C + c * D + e] = v[e];
  }
  if (dg && c == 0) {
    float v[D];
#pragma unroll
    for (int e = 0; e < D; ++e) v[e] = grad_rho[k * D + e] * coef_rho / total_mass;
    if (lnd) log_normalize<D>(v);
    const uint64_t o = 2u * C + (sg ? (uint64_t)C * D : 0u);
#pragma unroll
    for (int e = 0; e < D; ++e) zr[o + e] = v[e];
  }
}

template <int D>
__global__ __launch_bounds__(kThreads) void k_glue_backward(const float* __restrict__ dz,
                                                            const float* __restrict__ grad_s,
                                                            const float* __restrict__ grad_rho,
                                                            float* __restrict__ d_s, float* __restrict__ d_blur,
                                                            float* __restrict__ d_grad_s,
                                                            float* __restrict__ d_grad_rho, uint64_t n, uint32_t C,
                                                            float coef_s, float coef_rho, float total_mass,
                                                            int flags) {
  const uint64_t t = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= n * C) return;
  const uint64_t k = t / C;
  const uint32_t c = (uint32_t)(t - k * C);
  const bool sg = flags & SPHOPS_GLUE_STATE_GRAD, lng = flags & SPHOPS_GLUE_LOG_NORM_GRAD;
  const bool dg = flags & SPHOPS_GLUE_DENSITY_GRAD, lnd = flags & SPHOPS_GLUE_LOG_NORM_DENSITY_GRAD;
  const uint64_t W = 2u * C + (sg ? (uint64_t)C * D : 0u) + (dg ? D : 0u);
  const float* dr = dz + k * W;
  if (d_s) d_s[k * C + c] = dr[c];
  if (d_blur) d_blur[k * C + c] = dr[C + c];
  if (sg && d_grad_s) {
    float w[D];
#pragma unroll
    for (int e = 0; e < D; ++e) w[e] = dr[2u * C + c * D + e];
    if (lng) {
      float v[D];
#pragma unroll
      for (int e = 0; e < D; ++e) v[e] = grad_s[(k * C + c) * D + e] * coef_s;
      log_normalize_backward<D>(v, w);
    }
#pragma unroll
    for (int e = 0; e < D; ++e) d_grad_s[(k * C + c) * D + e] = w[e] * coef_s;
  }
  if (dg && d_grad_rho && c == 0) {
    const uint64_t o = 2u * C + (sg ? (uint64_t)C * D : 0u);
    float w[D];
#pragma unroll
    for (int e = 0; e < D; ++e) w[e] = dr[o + e];
    if (lnd) {
      float v[D];
#pragma unroll
      for (int e = 0; e < D; ++e) v[e] = grad_rho[k * D + e] * coef_rho / total_mass;
      log_normalize_backward<D>(v, w);
    }
#pragma unroll
    for (int e = 0; e < D; ++e) d_grad_rho[k * D + e] = w[e] * coef_rho / total_mass;
  }
}

inline dim3 blocks(uint64_t n) { return dim3((uint32_t)((n + kThreads - 1) / kThreads)); }

}  // namespace

void run_glue_forward(int dim, const float* s, const float* blur, const float* grad_s, const float* grad_rho,
                      float* z, uint64_t n, uint32_t C, float coef_s, float coef_rho, float total_mass, int flags,
                      hipStream_t st) {
  if (n == 0) return;
  if (dim == 2) {
    hipLaunchKernelGGL(k_glue_forward<2>, blocks(n * C), dim3(kThreads), 0, st, s, blur, grad_s, grad_rho, z, n, C,
                       coef_s, coef_rho, total_mass, flags);
  } else {
    hipLaunchKernelGGL(k_glue_forward<3>, blocks(n * C), dim3(kThreads), 0, st, s, blur, grad_s, grad_rho, z, n, C,
                       coef_s, coef_rho, total_mass, flags);
  }
  SPHOPS_LAUNCHED();
}

void run_glue_backward(int dim, const float* dz, const float* grad_s, const float* grad_rho, float* d_s,
                       float* d_blur, float* d_grad_s, float* d_grad_rho, uint64_t n, uint32_t C, float coef_s,
                       float coef_rho, float total_mass, int flags, hipStream_t st) {
  if (n == 0) return;
  if (dim == 2) {
    hipLaunchKernelGGL(k_glue_backward<2>, blocks(n * C), dim3(kThreads), 0, st, dz, grad_s, grad_rho, d_s, d_blur,
                       d_grad_s, d_grad_rho, n, C, coef_s, coef_rho, total_mass, flags);
  } else {
    hipLaunchKernelGGL(k_glue_backward<3>, blocks(n * C), dim3(kThreads), 0, st, dz, grad_s, grad_rho, d_s, d_blur,
                       d_grad_s, d_grad_rho, n, C, coef_s, coef_rho, total_mass, flags);
  }
  SPHOPS_LAUNCHED();
}

}  // namespace sphops
