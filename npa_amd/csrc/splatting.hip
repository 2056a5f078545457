// Differentiable 2D Gaussian splatting of particles into images
// (utils/splatting.py:6-117 of the reference), forward and backward, for
// gfx950.
//
// The reference evaluates a (2r+1)^2 patch of Gaussian weights around each
// particle's pixel, optionally normalises them to sum to K over the patch,
// and scatter-adds w and w * rgb into the image with float atomics
// (torch.scatter_add_), so its sums come in no fixed order.  Here:
//  * forward: a per-particle pass writes each particle's patch centre,
//    offset and normalised colour (32 bytes); then one workgroup per 16 x 16
//    pixel tile gathers.  It walks the image's particles in chunks of 256,
//    ranks the ones whose patch overlaps the tile by ballot (keeping
//    particle order) into LDS, and each thread sums its pixel over that
//    list.  Every pixel's sum runs in ascending
//    particle order: deterministic, no atomics, no zero-fill pass (each tile
//    writes all of its pixels);
//  * backward: one wave per particle sweeps its own patch, reading dL/dimage
//    there, and reduces across the wave, so every gradient is also a fixed-
//    order sum.  The patch normalisation's sum and its derivative are
//    separable (a product of two 1D sums), which costs 4(2r+1) exponentials
//    per particle instead of (2r+1)^2.
#include "sphops_internal.hpp"

namespace sphops {

namespace {

constexpr int kTile = 16;               // pixels per tile side; one thread per pixel
constexpr int kTileThreads = kTile * kTile;
constexpr int kWavesPerTile = kTileThreads / 64;
constexpr int kBwdWaves = 4;            // particles per backward workgroup

// pos = (x - lo) / (hi - lo) * (img_size - 1) per axis; with y_up, pos_y =
// (img_size - 1) - pos_y (utils/splatting.py:33-37).  Each step is in fp32
// as torch evaluates it; torch divides a tensor by a Python scalar as a
// product with the scalar's fp32 reciprocal, and so does this code.
// Returns false for particles whose patch cannot reach the image (and for
// NaN positions); otherwise the patch centre pixel (bx, by) = floor(pos) and
// the fractional offset (fx, fy) = pos - floor(pos).
__device__ __forceinline__ bool particle_setup(const SplatParams& sp, float x0, float x1, int& bx, int& by, float& fx,
                                               float& fy) {
  const float px = (x0 - sp.lo) * sp.inv_span * sp.scale;
  float py = (x1 - sp.lo) * sp.inv_span * sp.scale;
  if (sp.y_up) py = sp.scale - py;
  const float lim_lo = -(float)sp.r - 1.0f, lim_hi = (float)(sp.H + sp.r);
  if (!(px >= lim_lo && px < lim_hi && py >= lim_lo && py < lim_hi)) return false;
  const float fbx = floorf(px), fby = floorf(py);
  bx = (int)fbx;
  by = (int)fby;
  fx = px - fbx;
  fy = py - fby;
  return true;
}

// exp(-(a^2 + b^2) / (2 sigma^2)).  The argument is never below -25 (a patch
// corner: |offset|^2 <= 2 r^2, r = ceil(5 sigma)), where the hardware 2^x on
// x log2(e) is within 1e-6 relative of expf.
__device__ __forceinline__ float gauss(float a, float b, float inv_two_s2) {
  return __expf(-(a * a + b * b) * inv_two_s2);
}

__device__ __forceinline__ uint32_t rank_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Per particle, once: the patch centre, the fractional offset and the
// colour scaled by the normalisation, so the tiles read 32 bytes a particle
// and evaluate one exponential per (pixel, particle).  rec[2i] = (fx, fy,
// bx, by) with bx = kNoPatch for a particle that cannot reach the image;
// rec[2i + 1] = (k r, k g, k b, k), k = K / (1e-8 + S) (1 without
// normalisation).
constexpr int kNoPatch = INT32_MIN;

__global__ __launch_bounds__(256) void k_splat_prep(SplatParams sp, const float* __restrict__ x,
                                                    const float* __restrict__ color, int64_t n,
                                                    float4* __restrict__ rec) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  int bx = 0, by = 0;
  float fx = 0.0f, fy = 0.0f;
  const bool live = particle_setup(sp, x[2 * i], x[2 * i + 1], bx, by, fx, fy);
  float k = 1.0f;
  if (live && sp.normalize) {
    float sx = 0.0f, sy = 0.0f;
    for (int d = -sp.r; d <= sp.r; ++d) {
      sx += gauss((float)d - fx, 0.0f, sp.inv_two_s2);
      sy += gauss((float)d - fy, 0.0f, sp.inv_two_s2);
    }
    k = sp.K / (1e-8f + sx * sy);
  }
  const float* c = color + i * sp.ncolor + (sp.ncolor - 3);
  rec[2 * i] = make_float4(fx, fy, __int_as_float(live ? bx : kNoPatch), __int_as_float(by));
  rec[2 * i + 1] = make_float4(c[0] * k, c[1] * k, c[2] * k, k);
}

__global__ __launch_bounds__(kTileThreads) void k_splat_forward(SplatParams sp, const float4* __restrict__ rec,
                                                                const int32_t* __restrict__ starts,
                                                                float* __restrict__ out) {
  __shared__ float4 geo[kTileThreads];  // fx, fy, bx, by (bits)
  __shared__ float4 col[kTileThreads];  // k r, k g, k b, k
  __shared__ int wave_hits[kWavesPerTile];
  const int b = blockIdx.z;
  const int tx0 = blockIdx.x * kTile, ty0 = blockIdx.y * kTile;
  const int px = tx0 + (threadIdx.x % kTile), py = ty0 + (threadIdx.x / kTile);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int r = sp.r;
  float acc_r = 0.0f, acc_g = 0.0f, acc_b = 0.0f, acc_d = 0.0f;
  const int p0 = starts[b], p1 = starts[b + 1];
  for (int c0 = p0; c0 < p1; c0 += kTileThreads) {
    const int i = c0 + (int)threadIdx.x;
    float4 q = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    bool hit = false;
    if (i < p1) {
      q = rec[2 * (int64_t)i];
      const int bx = __float_as_int(q.z), by = __float_as_int(q.w);
      hit = bx != kNoPatch && bx + r >= tx0 && bx - r < tx0 + kTile && by + r >= ty0 && by - r < ty0 + kTile;
    }
    const uint64_t m = __ballot(hit);
    if (lane == 0) wave_hits[wave] = __popcll(m);
    __syncthreads();
    int base = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kWavesPerTile; ++w) {
      base += w < wave ? wave_hits[w] : 0;
      total += wave_hits[w];
    }
    if (hit) {
      const int slot = base + (int)rank_below(m);
      geo[slot] = q;
      col[slot] = rec[2 * (int64_t)i + 1];
    }
    __syncthreads();
    for (int k = 0; k < total; ++k) {
      const float4 g4 = geo[k];
      const int dx = px - __float_as_int(g4.z), dy = py - __float_as_int(g4.w);
      if (dx >= -r && dx <= r && dy >= -r && dy <= r) {
        const float4 c = col[k];
        const float g = gauss((float)dx - g4.x, (float)dy - g4.y, sp.inv_two_s2);
        acc_r += c.x * g;
        acc_g += c.y * g;
        acc_b += c.z * g;
        acc_d += c.w * g;
      }
    }
    __syncthreads();
  }
  if (px < sp.H && py < sp.H) {
    reinterpret_cast<float4*>(out)[((int64_t)b * sp.H + py) * sp.H + px] = make_float4(acc_r, acc_g, acc_b, acc_d);
  }
}

// The image a particle belongs to: the last b with starts[b] <= i.
__device__ __forceinline__ int image_of(const int32_t* starts, int images, int i) {
  int lo = 0, hi = images - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (starts[mid] <= i) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Per particle, with g_q the patch weights, w_q = g_q K / n (n = 1e-8 + S,
// S = sum of g over the whole patch; w = g and n = 1 without normalisation),
// d_q = dL/dimage at pixel q (r, g, b, density) and G_q = rgb . d_q.rgb +
// d_q.density = dL/dw_q, over the pixels q of the patch inside the image:
//   dL/drgb = sum_q w_q d_q.rgb,
//   dL/dg_q = G_q K / n  (q inside) - (K / n^2) sum_p G_p g_p  (every q),
//   dg_q/dfx = g_q * 2 (q_x - fx) / (2 sigma^2), the same for y,
// and dL/dx = dL/dfx * (img_size - 1) / (hi - lo) (floor has no gradient), the y term
// negated with y_up.  Only the colour row's last three channels get a
// gradient.
__global__ __launch_bounds__(64 * kBwdWaves) void k_splat_backward(SplatParams sp, const float* __restrict__ x,
                                                                   const float* __restrict__ color,
                                                                   const int32_t* __restrict__ starts, int images,
                                                                   int64_t n, const float* __restrict__ d_img,
                                                                   float* __restrict__ d_x,
                                                                   float* __restrict__ d_color) {
  const int64_t i = (int64_t)blockIdx.x * kBwdWaves + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (i >= n) return;
  int bx = 0, by = 0;
  float fx = 0.0f, fy = 0.0f;
  const bool live = particle_setup(sp, x[2 * i], x[2 * i + 1], bx, by, fx, fy);
  const float* c = color + i * sp.ncolor + (sp.ncolor - 3);
  const float cr = c[0], cg = c[1], cb = c[2];
  const int r = sp.r, P = 2 * r + 1, H = sp.H;
  float s_dr = 0.0f, s_dg = 0.0f, s_db = 0.0f;  // sum g d.rgb
  float s_gg = 0.0f, s_ggx = 0.0f, s_ggy = 0.0f;  // sum G g, G g (qx - fx), G g (qy - fy)
  float sx = 1.0f, sy = 1.0f, sxa = 0.0f, sya = 0.0f;  // separable patch sums for the normaliser
  if (live) {
    const int b = image_of(starts, images, (int)i);
    const float4* dimg = reinterpret_cast<const float4*>(d_img) + (int64_t)b * H * H;
    for (int q = lane; q < P * P; q += 64) {
      const int qy = q / P, qx = q - qy * P;
      const int ix = bx + qx - r, iy = by + qy - r;
      if (ix >= 0 && ix < H && iy >= 0 && iy < H) {
        const float ax = (float)(qx - r) - fx, ay = (float)(qy - r) - fy;
        const float g = gauss(ax, ay, sp.inv_two_s2);
        const float4 d = dimg[(int64_t)iy * H + ix];
        const float G = cr * d.x + cg * d.y + cb * d.z + d.w;
        s_dr += g * d.x;
        s_dg += g * d.y;
        s_db += g * d.z;
        s_gg += G * g;
        s_ggx += G * g * ax;
        s_ggy += G * g * ay;
      }
    }
    if (sp.normalize) {
      sx = sy = 0.0f;
      for (int d = lane; d < P; d += 64) {
        const float ax = (float)(d - r) - fx, ay = (float)(d - r) - fy;
        const float gx = gauss(ax, 0.0f, sp.inv_two_s2), gy = gauss(ay, 0.0f, sp.inv_two_s2);
        sx += gx;
        sy += gy;
        sxa += gx * ax;
        sya += gy * ay;
      }
    }
  }
  s_dr = wave_sum(s_dr);
  s_dg = wave_sum(s_dg);
  s_db = wave_sum(s_db);
  s_gg = wave_sum(s_gg);
  s_ggx = wave_sum(s_ggx);
  s_ggy = wave_sum(s_ggy);
  float dfx = 0.0f, dfy = 0.0f, dr = 0.0f, dg = 0.0f, db = 0.0f;
  if (live) {
    const float k2 = 2.0f * sp.inv_two_s2;
    if (sp.normalize) {
      sx = wave_sum(sx);
      sy = wave_sum(sy);
      sxa = wave_sum(sxa);
      sya = wave_sum(sya);
      const float nrm = 1e-8f + sx * sy;
      const float kn = sp.K / nrm;
      const float dnrm = -kn / nrm * s_gg;  // dL/dn... times dn/dg_q = 1 for every q
      dr = kn * s_dr;
      dg = kn * s_dg;
      db = kn * s_db;
      dfx = k2 * (kn * s_ggx + dnrm * sxa * sy);
      dfy = k2 * (kn * s_ggy + dnrm * sx * sya);
    } else {
      dr = s_dr;
      dg = s_dg;
      db = s_db;
      dfx = k2 * s_ggx;
      dfy = k2 * s_ggy;
    }
    if (sp.y_up) dfy = -dfy;
  }
  const float jac = sp.inv_span * sp.scale;
  if (lane == 0) {
    d_x[2 * i] = dfx * jac;
    d_x[2 * i + 1] = dfy * jac;
  }
  for (int j = lane; j < sp.ncolor; j += 64) {
    const int k = j - (sp.ncolor - 3);
    d_color[i * sp.ncolor + j] = k == 0 ? dr : k == 1 ? dg : k == 2 ? db : 0.0f;
  }
}

}  // namespace

void run_splat_forward(const SplatParams& sp, const float* x, const float* color, const int32_t* starts, int images,
                       int64_t n, float4* rec, float* out, hipStream_t st) {
  if (images == 0 || sp.H == 0) return;
  if (n > 0) {
    hipLaunchKernelGGL(k_splat_prep, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, sp, x, color, n, rec);
    SPHOPS_LAUNCHED();
  }
  const dim3 grid((uint32_t)((sp.H + kTile - 1) / kTile), (uint32_t)((sp.H + kTile - 1) / kTile), (uint32_t)images);
  hipLaunchKernelGGL(k_splat_forward, grid, dim3(kTileThreads), 0, st, sp, rec, starts, out);
  SPHOPS_LAUNCHED();
}

void run_splat_backward(const SplatParams& sp, const float* x, const float* color, const int32_t* starts, int images,
                        int64_t n, const float* d_img, float* d_x, float* d_color, hipStream_t st) {
  if (n == 0) return;
  const dim3 grid((uint32_t)((n + kBwdWaves - 1) / kBwdWaves));
  hipLaunchKernelGGL(k_splat_backward, grid, dim3(64 * kBwdWaves), 0, st, sp, x, color, starts, images, n, d_img, d_x,
                     d_color);
  SPHOPS_LAUNCHED();
}

}  // namespace sphops
