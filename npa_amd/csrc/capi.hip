// extern "C" entry points of libsphops_hip.so (declared in include/sphops_hip.h).
#include <atomic>
#include <cmath>
#include <string>

#include "../../include/sphops_hip.h"
#include "perception_kernels.hpp"

namespace sphops {

void run_forward_2d(const Grid& g, Op op, const int32_t* bo, const OpPtrs& a, hipStream_t st);
void run_forward_3d(const Grid& g, Op op, const int32_t* bo, const OpPtrs& a, hipStream_t st);
void run_backward_2d(const Grid& g, Op op, bool full, const int32_t* bo, const OpPtrs& a, hipStream_t st);
void run_backward_3d(const Grid& g, Op op, bool full, const int32_t* bo, const OpPtrs& a, hipStream_t st);

namespace {

thread_local std::string g_last_error;

template <class F>
int guarded(F&& f) {
  try {
    f();
    g_last_error.clear();
    return 0;
  } catch (const std::exception& e) {
    g_last_error = e.what();
  } catch (...) {
    g_last_error = "unknown error";
  }
  return -1;
}

// The message is turned into a std::string only on failure, so a passing
// check allocates nothing.
void require(bool ok, const char* msg) {
  if (!ok) throw Error(msg);
}
void require(bool ok, const std::string& msg) {
  if (!ok) throw Error(msg);
}

template <class T>
T* dalloc(uint64_t n) {
  void* p = nullptr;
  SPHOPS_HIP(hipMalloc(&p, sizeof(T) * (n ? n : 1)));
  return static_cast<T*>(p);
}

uint32_t spread_host(uint32_t v, int dim) {
  uint32_t out = 0;
  for (int b = 0; b < 10; ++b) out |= ((v >> b) & 1u) << (b * dim);
  return out;
}

// Validates the grid arguments and fills the parameters and scratch sizes of
// `g` (HashGrid::_init, sphops/sph_cuda.cu:1836-1878; Python checks of
// sphops/sph.py:48-78).  Allocates nothing.
void setup_grid(Grid& g, int dim, int boundary, int mode, const int32_t* grid_size, float eps,
                uint32_t particle_count, uint32_t batch_size, uint32_t max_particles_per_block) {
  require(dim == 2 || dim == 3, "dim must be 2 or 3");
  require(boundary == SPHOPS_CLAMPED || boundary == SPHOPS_PERIODIC, "boundary must be clamped or periodic");
  require(mode == SPHOPS_MODE_GRID || mode == SPHOPS_MODE_PARTICLE, "mode must be grid or particle");
  require(grid_size != nullptr, "grid_size must not be NULL");
  require(std::isfinite(eps) && eps > 0.0f, "eps must be a positive finite number");
  require(max_particles_per_block >= 1, "max_particles_per_block must be >= 1");
  uint64_t G = 1;
  for (int d = 0; d < dim; ++d) {
    require(grid_size[d] >= 1, "grid sizes must be >= 1");
    if (boundary == SPHOPS_PERIODIC)
      require(grid_size[d] >= 3, "periodic grids need at least 3 cells per axis (fewer double-count neighbours)");
    G *= (uint64_t)grid_size[d];
  }
  const uint64_t BG = G * batch_size, BN = (uint64_t)particle_count * batch_size;
  require(BG + 1 < (1ull << 32), "batch_size * cell_count must be below 2^32 - 1");
  require(BN < (1ull << 31), "batch_size * particle_count must be below 2^31");
  if (mode == SPHOPS_MODE_PARTICLE) {
    uint32_t hmax = 0;
    for (int d = 0; d < dim; ++d) {
      const int gsz = grid_size[d];
      require((gsz & (gsz - 1)) == 0, "particle mode needs power-of-two grid sizes");
      require(gsz <= 1024, "particle mode supports at most 1024 cells per axis");
      hmax |= spread_host((uint32_t)gsz - 1, dim) << d;
    }
    require(hmax < G, "particle mode: the Morton hash of this grid shape exceeds the cell count "
                      "(use equal sizes, or sizes non-increasing along x, y, z)");
  }
  g.dim = dim;
  g.periodic = boundary == SPHOPS_PERIODIC;
  g.particle_mode = mode == SPHOPS_MODE_PARTICLE;
  auto& p = g.p;
  for (int d = 0; d < 3; ++d) {
    p.gs[d] = d < dim ? grid_size[d] : 1;
    p.half_gs[d] = p.gs[d] / 2;
  }
  p.eps = eps;
  p.inv_eps = 1.0f / eps;
  p.eps2 = eps * eps;
  for (int d = 0; d < 3; ++d) {
    p.L[d] = static_cast<float>(p.gs[d]) * eps;
    p.half_L[d] = 0.5f * p.L[d];
  }
  // coefficients exactly as HashGrid::_init derives them (fp32 powers of
  // 1/eps, double constant, rounded to fp32)
  const float ie = p.inv_eps, ie2 = ie * ie, ie4 = ie2 * ie2;
  if (dim == 2) {
    const float ie5 = ie4 * ie, ie8 = ie4 * ie4;
    p.c6 = (float)(4.0 / M_PI * (double)ie8);
    p.cs = (float)(10.0 / M_PI * (double)ie5);
  } else {
    const float ie6 = ie4 * ie2, ie9 = ie4 * ie4 * ie;
    p.c6 = (float)((315.0 / (64.0 * M_PI)) * (double)ie9);
    p.cs = (float)((15.0 / M_PI) * (double)ie6);
  }
  p.N = particle_count;
  p.B = batch_size;
  p.G = (uint32_t)G;
  p.maxp = max_particles_per_block;
  p.morton = g.particle_mode ? 1 : 0;
  if (!g.particle_mode) {
    const uint64_t per = std::min<uint64_t>(particle_count,
                                            G + (particle_count + max_particles_per_block - 1) /
                                                    max_particles_per_block);
    g.max_blocks = per * batch_size;
  } else {
    g.max_blocks = 1;
  }
  g.n_keys = BN;
  g.n_cells = BG;
  g.n_tiles = (BN + 4095) / 4096;
  g.n_chunks = (BG + 1 + 1023) / 1024;
}

void free_grid(Grid* g) {
  if (!g) return;
  for (int i = 0; i < 2; ++i) {
    (void)hipFree(g->kv[i]);
  }
  (void)hipFree(g->hist);
  (void)hipFree(g->scan_tmp);
  (void)hipFree(g->chunk_lo);
  (void)hipFree(g->flags);
  (void)hipFree(g->packed);
  (void)hipFree(g->sparse_len);
  (void)hipFree(g->unit_len);
  (void)hipFree(g->units);
  (void)hipFree(g->unit_total);
  (void)hipFree(g->stripes);
  delete g;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// The splat constants as utils/splatting.py:40-76 computes them in Python
// (double) before torch rounds them to fp32.
SplatParams splat_params(int64_t images, int64_t particles, int ncolor, int img_size, double sigma, double lo,
                         double hi, int normalize_color, int y_up, double pixel_size) {
  require(images >= 0 && images <= 65535, "images must be in [0, 65535]");
  require(particles >= 0 && particles < (int64_t)1 << 31, "particles must be in [0, 2^31)");
  require(ncolor >= 3, "color needs at least 3 channels (the last three are r, g, b)");
  require(img_size >= 1 && img_size <= 16384, "img_size must be in [1, 16384]");
  require(hi != lo, "hi must differ from lo");
  double s = sigma;
  if (normalize_color) s = sigma * img_size * pixel_size / (hi - lo);
  require(std::isfinite(s) && s > 0.0, "sigma (in pixels) must be positive and finite");
  const double r = std::max(1.0, std::ceil(5.0 * s));
  require(r <= kMaxSplatRadius, "splat radius ceil(5 sigma) exceeds " + std::to_string(kMaxSplatRadius) + " pixels");
  const double kk = img_size * pixel_size / (hi - lo);
  SplatParams sp;
  sp.H = img_size;
  sp.r = (int)r;
  sp.lo = (float)lo;
  sp.inv_span = 1.0f / (float)(hi - lo);
  sp.scale = (float)(img_size - 1);
  sp.inv_two_s2 = 1.0f / (float)(2.0 * s * s);
  sp.K = (float)(kk * kk);
  sp.normalize = normalize_color ? 1 : 0;
  sp.y_up = y_up ? 1 : 0;
  sp.ncolor = ncolor;
  return sp;
}

void check_channels(uint32_t C) {
  require(C >= 1 && C <= kMaxChannels,
          "feature_dim must be in [1, " + std::to_string(kMaxChannels) + "], got " + std::to_string(C));
}

void forward(const Grid& g, Op op, const int32_t* bo, const OpPtrs& a, hipStream_t st) {
  if (g.dim == 2) run_forward_2d(g, op, bo, a, st);
  else run_forward_3d(g, op, bo, a, st);
}

void backward(const Grid& g, Op op, bool full, const int32_t* bo, const OpPtrs& a, hipStream_t st) {
  if (g.dim == 2) run_backward_2d(g, op, full, bo, a, st);
  else run_backward_3d(g, op, full, bo, a, st);
}

__global__ __launch_bounds__(256) void k_safe_inv2(const float4* __restrict__ in, float4* __restrict__ out,
                                                   uint64_t count, float tol) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  const float4 m = in[i];
  float M[4] = {m.x, m.y, m.z, m.w}, L[4];
  pk::safe_inv_sym<2>(M, tol, L);
  out[i] = make_float4(L[0], L[1], L[2], L[3]);
}

__global__ __launch_bounds__(256) void k_safe_inv3(const float* __restrict__ in, float* __restrict__ out,
                                                   uint64_t count, float tol) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  float M[9], L[9];
#pragma unroll
  for (int q = 0; q < 9; ++q) M[q] = in[i * 9 + q];
  pk::safe_inv_sym<3>(M, tol, L);
#pragma unroll
  for (int q = 0; q < 9; ++q) out[i * 9 + q] = L[q];
}

}  // namespace

void run_safe_inv(const float* in, float* out, uint64_t count, int dim, float tol, hipStream_t st) {
  if (count == 0) return;
  const dim3 grid((uint32_t)((count + 255) / 256));
  if (dim == 2) {
    require(pk::aligned16(in) && pk::aligned16(out), "safe_inv_sym_mat: 2x2 matrices must be 16-byte aligned");
    hipLaunchKernelGGL(k_safe_inv2, grid, dim3(256), 0, st, reinterpret_cast<const float4*>(in),
                       reinterpret_cast<float4*>(out), count, tol);
  } else {
    hipLaunchKernelGGL(k_safe_inv3, grid, dim3(256), 0, st, in, out, count, tol);
  }
  SPHOPS_LAUNCHED();
}

}  // namespace sphops

using sphops::Grid;
using sphops::Op;
using sphops::OpPtrs;
using sphops::guarded;
using sphops::require;
using sphops::spread_host;
using sphops::dalloc;

struct sphops_grid : Grid {};

extern "C" {

int sphops_abi_version(void) { return SPHOPS_ABI_VERSION; }

const char* sphops_last_error(void) { return sphops::g_last_error.c_str(); }

int sphops_grid_create(int dim, int boundary, int mode, const int32_t* grid_size, float eps, uint32_t particle_count,
                       uint32_t batch_size, uint32_t max_particles_per_block, sphops_grid** out) {
  return guarded([&] {
    require(out != nullptr, "out must not be NULL");
    *out = nullptr;
    sphops_grid shape;
    sphops::setup_grid(shape, dim, boundary, mode, grid_size, eps, particle_count, batch_size,
                       max_particles_per_block);
    auto* g = new sphops_grid(shape);
    const uint64_t BN = g->n_keys;
    try {
      SPHOPS_HIP(hipGetDevice(&g->device));
      for (int i = 0; i < 2; ++i) {
        g->kv[i] = dalloc<uint64_t>(BN + 1);
      }
      g->hist = dalloc<uint32_t>(sphops::hist_words(*g));
      g->scan_tmp_len = sphops::scan_tmp_elems(sphops::scan_words(*g));
      g->scan_tmp = dalloc<uint32_t>(g->scan_tmp_len);
      g->chunk_lo = dalloc<uint32_t>(g->n_chunks + 1);
      g->flags = dalloc<uint32_t>(BN + 1);
      g->packed = dalloc<float4>(BN);
      g->sparse_len = dalloc<int32_t>(BN);
      g->unit_len = dalloc<int32_t>(BN);
      g->units = dalloc<uint2>(BN);
      g->unit_total = dalloc<int32_t>(1);
      g->stripes = dalloc<unsigned long long>((uint64_t)sphops::kFillStripes * sphops::kStripeWords);
      // zero once here (and wait, so that a fill on any stream sees it);
      // every fill's totals kernel leaves them zero again
      SPHOPS_HIP(hipMemset(g->stripes, 0, sizeof(unsigned long long) * sphops::kFillStripes * sphops::kStripeWords));
      SPHOPS_HIP(hipDeviceSynchronize());
    } catch (...) {
      sphops::free_grid(g);
      throw;
    }
    *out = g;
  });
}

void sphops_grid_destroy(sphops_grid* grid) { sphops::free_grid(grid); }

int64_t sphops_grid_max_blocks(const sphops_grid* grid) { return grid ? (int64_t)grid->max_blocks : -1; }

int sphops_grid_coefficients(const sphops_grid* grid, float* poly6, float* spiky) {
  return guarded([&] {
    require(grid != nullptr, "grid must not be NULL");
    if (poly6) *poly6 = grid->p.c6;
    if (spiky) *spiky = grid->p.cs;
  });
}

static void check_initialize_args(const Grid& g, const float* positions, const int32_t* permutation,
                                  const int32_t* bin_offsets, const int32_t* block_info) {
  require(bin_offsets != nullptr, "bin_offsets must not be NULL");
  require(g.n_keys == 0 || (positions && permutation), "positions and permutation must not be NULL");
  require(g.particle_mode || block_info != nullptr || g.max_blocks == 0,
          "block_info must not be NULL in grid mode");
  require(sphops::pk::aligned16(bin_offsets), "bin_offsets must be 16-byte aligned");
  require(g.particle_mode || sphops::pk::aligned16(block_info), "block_info must be 16-byte aligned");
  require(g.dim == 2 || sphops::pk::aligned16(positions), "3D positions must be 16-byte aligned");
}

int sphops_initialize(sphops_grid* grid, const float* positions, int32_t* permutation, int32_t* bin_offsets,
                      int32_t* block_info, int32_t* total_blocks, void* stream) {
  return guarded([&] {
    require(grid != nullptr, "grid must not be NULL");
    check_initialize_args(*grid, positions, permutation, bin_offsets, block_info);
    sphops::run_instantiate(*grid, positions, permutation, bin_offsets, block_info, total_blocks,
                            sphops::as_stream(stream));
  });
}

int sphops_initialize_inverse(sphops_grid* grid, const float* positions, int32_t* permutation,
                              int32_t* inverse, int32_t* bin_offsets, int32_t* block_info,
                              int32_t* total_blocks, void* stream) {
  return guarded([&] {
    require(grid != nullptr, "grid must not be NULL");
    check_initialize_args(*grid, positions, permutation, bin_offsets, block_info);
    require(grid->n_keys == 0 || inverse != nullptr, "inverse must not be NULL");
    sphops::run_instantiate(*grid, positions, permutation, bin_offsets, block_info, total_blocks,
                            sphops::as_stream(stream), inverse);
  });
}

static int move_rows(const sphops_grid* grid, const float* ip, const float* is, const float* im, const int32_t* perm,
                     float* op, float* os, float* om, uint32_t C, bool fwd, void* stream) {
  return guarded([&] {
    require(grid != nullptr, "grid must not be NULL");
    sphops::check_channels(C == 0 ? 1 : C);
    require(grid->n_keys == 0 || (ip && is && perm && op && os), "null buffer");
    require((im == nullptr) == (om == nullptr), "the mass rows are moved both or neither (both NULL)");
    sphops::run_bin_particles(*grid, ip, is, im, perm, op, os, om, C, fwd, sphops::as_stream(stream));
  });
}

int sphops_bin_particles(const sphops_grid* grid, const float* in_pos, const float* in_state, const float* in_mass,
                         const int32_t* permutation, float* out_pos, float* out_state, float* out_mass,
                         uint32_t feature_dim, void* stream) {
  return move_rows(grid, in_pos, in_state, in_mass, permutation, out_pos, out_state, out_mass, feature_dim, true,
                   stream);
}

int sphops_backward_bin_particles(const sphops_grid* grid, const float* grad_out_pos, const float* grad_out_state,
                                  const float* grad_out_mass, const int32_t* permutation, float* grad_in_pos,
                                  float* grad_in_state, float* grad_in_mass, uint32_t feature_dim, void* stream) {
  return move_rows(grid, grad_out_pos, grad_out_state, grad_out_mass, permutation, grad_in_pos, grad_in_state,
                   grad_in_mass, feature_dim, false, stream);
}

static int fwd_op(const sphops_grid* grid, Op op, const int32_t* bo, OpPtrs a, void* stream) {
  return guarded([&] {
    require(grid != nullptr, "grid must not be NULL");
    const bool chan = op == Op::Blur || op == Op::Gradient || op == Op::GradientHybrid || op == Op::BlurGradientHybrid;
    if (grid->n_keys == 0) {  // no particles: nothing to read or write (empty tensors may be NULL)
      require(bo != nullptr, "null buffer");
      if (chan) sphops::check_channels(a.C);
      return;
    }
    require(bo != nullptr && a.x != nullptr && a.out0 != nullptr, "null buffer");
    if (chan) {
      sphops::check_channels(a.C);
      require(a.s != nullptr, "state must not be NULL");
    }
    if (op != Op::Count) require(a.m != nullptr, "mass must not be NULL");
    if (chan || op == Op::MomentMatrix) require(a.rho != nullptr, "rho must not be NULL");
    if (op == Op::DensityPair || op == Op::BlurGradientHybrid) require(a.out3 != nullptr, "out2 must not be NULL");
    require(grid->dim == 2 || sphops::pk::aligned16(a.x), "3D positions must be 16-byte aligned");
    sphops::forward(*grid, op, bo, a, sphops::as_stream(stream));
  });
}

int sphops_count_forward(const sphops_grid* grid, const float* x, float* count, const int32_t* bo, const int32_t*,
                         void* stream) {
  OpPtrs a;
  a.x = x;
  a.out0 = count;
  return fwd_op(grid, Op::Count, bo, a, stream);
}

int sphops_density_forward(const sphops_grid* grid, const float* x, const float* mass, float* rho, const int32_t* bo,
                           const int32_t*, void* stream) {
  OpPtrs a;
  a.x = x;
  a.m = mass;
  a.out0 = rho;
  return fwd_op(grid, Op::Density, bo, a, stream);
}

int sphops_blur_forward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                        const float* state_in, float* state_out, uint32_t C, const int32_t* bo, const int32_t*,
                        void* stream) {
  OpPtrs a;
  a.x = x;
  a.rho = rho;
  a.m = mass;
  a.s = state_in;
  a.out0 = state_out;
  a.C = C;
  return fwd_op(grid, Op::Blur, bo, a, stream);
}

int sphops_gradient_forward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                            const float* state_in, float* out, uint32_t C, const int32_t* bo, const int32_t*,
                            void* stream) {
  OpPtrs a;
  a.x = x;
  a.rho = rho;
  a.m = mass;
  a.s = state_in;
  a.out0 = out;
  a.C = C;
  return fwd_op(grid, Op::Gradient, bo, a, stream);
}

int sphops_density_gradient_forward(const sphops_grid* grid, const float* x, const float* mass, float* out,
                                    const int32_t* bo, const int32_t*, void* stream) {
  OpPtrs a;
  a.x = x;
  a.m = mass;
  a.out0 = out;
  return fwd_op(grid, Op::DensityGradient, bo, a, stream);
}

int sphops_moment_matrix_forward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                                 float* out, const int32_t* bo, const int32_t*, void* stream) {
  OpPtrs a;
  a.x = x;
  a.rho = rho;
  a.m = mass;
  a.out0 = out;
  return fwd_op(grid, Op::MomentMatrix, bo, a, stream);
}

int sphops_gradient_hybrid_forward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                                   const float* state_in, float* out, uint32_t C, float tol, const int32_t* bo,
                                   const int32_t*, void* stream) {
  OpPtrs a;
  a.x = x;
  a.rho = rho;
  a.m = mass;
  a.s = state_in;
  a.out0 = out;
  a.C = C;
  a.tol = tol;
  return fwd_op(grid, Op::GradientHybrid, bo, a, stream);
}

static int bwd_op(const sphops_grid* grid, Op op, bool full, const int32_t* bo, OpPtrs a, void* stream) {
  return guarded([&] {
    require(grid != nullptr, "grid must not be NULL");
    if (grid->n_keys == 0) {  // no particles: nothing to read or write (empty tensors may be NULL)
      require(bo != nullptr, "null buffer");
      if (op == Op::Blur || op == Op::Gradient || op == Op::BlurGradientHybrid) sphops::check_channels(a.C);
      return;
    }
    require(bo != nullptr && a.x != nullptr && a.m != nullptr && a.g != nullptr, "null buffer");
    if (op == Op::Blur || op == Op::Gradient || op == Op::BlurGradientHybrid) {
      sphops::check_channels(a.C);
      require(a.rho != nullptr && a.s != nullptr && a.out1 != nullptr, "null buffer");
      if (full) require(a.out0 != nullptr && a.out2 != nullptr, "null buffer");
    } else if (op == Op::MomentMatrix) {
      require(a.rho != nullptr && a.out0 != nullptr && a.out2 != nullptr, "null buffer");
    } else {
      require(a.out0 != nullptr, "null buffer");
    }
    require(grid->dim == 2 || (sphops::pk::aligned16(a.x) && (!a.out0 || sphops::pk::aligned16(a.out0))),
            "3D positions must be 16-byte aligned");
    sphops::backward(*grid, op, full, bo, a, sphops::as_stream(stream));
  });
}

int sphops_density_backward(const sphops_grid* grid, const float* x, const float* mass, const float* dL_rho,
                            float* grad_x, const int32_t* bo, const int32_t*, int dLdx, void* stream) {
  if (!dLdx) return 0;
  OpPtrs a;
  a.x = x;
  a.m = mass;
  a.g = dL_rho;
  a.out0 = grad_x;
  return bwd_op(grid, Op::Density, true, bo, a, stream);
}

int sphops_blur_backward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                         const float* state_in, const float* dL, float* grad_x, float* grad_s, float* grad_rho,
                         uint32_t C, const int32_t* bo, const int32_t*, int dLdx, int dLds, int dLdrho,
                         void* stream) {
  if (!dLdx && !dLds && !dLdrho) return 0;
  const bool ds_only = dLds && !dLdx && !dLdrho;
  OpPtrs a;
  a.x = x;
  a.rho = rho;
  a.m = mass;
  a.s = state_in;
  a.g = dL;
  a.out0 = grad_x;
  a.out1 = grad_s;
  a.out2 = grad_rho;
  a.C = C;
  return bwd_op(grid, Op::Blur, !ds_only, bo, a, stream);
}

int sphops_density_gradient_backward(const sphops_grid* grid, const float* x, const float* mass, const float* dL,
                                     float* grad_x, const int32_t* bo, const int32_t*, int dLdx, void* stream) {
  if (!dLdx) return 0;
  OpPtrs a;
  a.x = x;
  a.m = mass;
  a.g = dL;
  a.out0 = grad_x;
  return bwd_op(grid, Op::DensityGradient, true, bo, a, stream);
}

int sphops_gradient_backward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                             const float* state_in, const float* dL, float* grad_x, float* grad_s, float* grad_rho,
                             uint32_t C, const int32_t* bo, const int32_t*, int dLdx, int dLds, int dLdrho,
                             void* stream) {
  if (!dLdx && !dLds && !dLdrho) return 0;
  const bool ds_only = dLds && !dLdx && !dLdrho;
  OpPtrs a;
  a.x = x;
  a.rho = rho;
  a.m = mass;
  a.s = state_in;
  a.g = dL;
  a.out0 = grad_x;
  a.out1 = grad_s;
  a.out2 = grad_rho;
  a.C = C;
  return bwd_op(grid, Op::Gradient, !ds_only, bo, a, stream);
}

int sphops_moment_matrix_backward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                                  const float* dL, float* grad_x, float* grad_rho, const int32_t* bo, const int32_t*,
                                  int dLdx, int dLdrho, void* stream) {
  if (!dLdx && !dLdrho) return 0;
  OpPtrs a;
  a.x = x;
  a.rho = rho;
  a.m = mass;
  a.g = dL;
  a.out0 = grad_x;
  a.out2 = grad_rho;
  return bwd_op(grid, Op::MomentMatrix, true, bo, a, stream);
}

static OpPtrs from_args(const sphops_args* a) {
  OpPtrs p;
  p.x = a->x;
  p.m = a->mass;
  p.rho = a->rho;
  p.s = a->state;
  p.g = a->upstream;
  p.out0 = a->out;
  p.out1 = a->grad_state;
  p.out2 = a->grad_rho;
  p.C = a->feature_dim;
  p.tol = a->tol;
  p.nptr = a->nbr_start;
  p.ncnt = a->nbr_count;
  p.nidx = a->nbr_index;
  p.order = a->nbr_order;
  p.waves = reinterpret_cast<const uint2*>(a->nbr_waves);
  p.nwaves = (uint32_t)std::max(a->nbr_wave_count, 0);
  p.waves2 = reinterpret_cast<const uint2*>(a->nbr_waves_split);
  p.nwaves2 = (uint32_t)std::max(a->nbr_wave_count_split, 0);
  p.g2 = a->upstream2;
  p.out3 = a->out2;
  p.nwaves_dev = a->nbr_wave_count_device;
  p.nwaves2_dev = a->nbr_wave_count_split_device;
  p.tile_units = reinterpret_cast<const uint2*>(a->tile_units);
  p.tile_count = a->tile_unit_count;
  p.order_sparse = a->nbr_order_sparse;
  p.waves_sparse = reinterpret_cast<const uint2*>(a->nbr_waves_sparse);
  p.nwaves_sparse = (uint32_t)std::max(a->nbr_wave_count_sparse, 0);
  p.nwaves_sparse_dev = a->nbr_wave_count_sparse_device;
  p.xw_buf = reinterpret_cast<float4*>(a->packed);
  p.xw_ready = a->packed_valid != 0;
  p.nown = a->nbr_own;
  p.cells = reinterpret_cast<const uint2*>(a->cells);
  p.cell_count = a->cell_count;
  return p;
}

static void check_list(const sphops_args* a) {
  require(a->nbr_index == nullptr || (a->nbr_start != nullptr && a->nbr_count != nullptr),
          "nbr_index needs nbr_start and nbr_count");
  require(a->nbr_order == nullptr || a->nbr_index != nullptr, "nbr_order needs nbr_index");
  require(a->nbr_waves == nullptr || a->nbr_order != nullptr, "nbr_waves needs nbr_order");
  require(a->nbr_order == nullptr || a->nbr_waves != nullptr, "nbr_order needs nbr_waves");
  require(a->nbr_wave_count >= 0 && a->nbr_wave_count_split >= 0, "negative wave count");
  require(a->nbr_waves_split == nullptr || a->nbr_waves != nullptr, "nbr_waves_split needs nbr_waves");
  require(a->nbr_wave_count_device == nullptr || a->nbr_waves != nullptr, "nbr_wave_count_device needs nbr_waves");
  require(a->nbr_wave_count_split_device == nullptr || a->nbr_waves_split != nullptr,
          "nbr_wave_count_split_device needs nbr_waves_split");
  const bool tiles = a->tile_units != nullptr;
  require(!tiles || (a->tile_unit_count != nullptr && a->nbr_order_sparse != nullptr &&
                     a->nbr_waves_sparse != nullptr && a->nbr_waves_split != nullptr),
          "tile_units needs tile_unit_count, nbr_order_sparse, nbr_waves_sparse and the split schedule");
  require(a->nbr_wave_count_sparse >= 0, "negative wave count");
  require(a->packed == nullptr || sphops::pk::aligned16(a->packed), "packed must be 16-byte aligned");
  require(a->packed_valid == 0 || a->packed != nullptr, "packed_valid needs packed");
  const int cell_ptrs = (a->nbr_own != nullptr) + (a->cells != nullptr) + (a->cell_count != nullptr);
  require(cell_ptrs == 0 || cell_ptrs == 3, "nbr_own, cells and cell_count go together");
  require(cell_ptrs == 0 || a->nbr_index != nullptr, "cell tiles need the neighbour list (nbr_index)");
}

int sphops_forward(const sphops_grid* grid, int op, const sphops_args* args, void* stream) {
  if (args == nullptr) {
    sphops::g_last_error = "args must not be NULL";
    return -1;
  }
  if (op < SPHOPS_OP_COUNT || op > SPHOPS_OP_BLUR_GRADIENT_HYBRID) {
    sphops::g_last_error = "unknown operator " + std::to_string(op);
    return -1;
  }
  int st = guarded([&] { check_list(args); });
  if (st) return st;
  return fwd_op(grid, static_cast<Op>(op), args->bin_offsets, from_args(args), stream);
}

int sphops_backward(const sphops_grid* grid, int op, int dLdx, int dLds, int dLdrho, const sphops_args* args,
                    void* stream) {
  if (args == nullptr) {
    sphops::g_last_error = "args must not be NULL";
    return -1;
  }
  if (op <= SPHOPS_OP_COUNT || op > SPHOPS_OP_BLUR_GRADIENT_HYBRID) {
    sphops::g_last_error = "operator " + std::to_string(op) + " has no backward";
    return -1;
  }
  int st = guarded([&] { check_list(args); });
  if (st) return st;
  const Op o = static_cast<Op>(op);
  OpPtrs a = from_args(args);
  if (o == Op::DensityPair || o == Op::BlurGradientHybrid) {
    st = guarded([&] { require(a.g != nullptr && a.g2 != nullptr, "fused backward needs upstream and upstream2"); });
    if (st) return st;
  }
  switch (o) {
    case Op::Density:
    case Op::DensityGradient:
    case Op::DensityPair:
      if (!dLdx) return 0;
      return bwd_op(grid, o, true, args->bin_offsets, a, stream);
    case Op::MomentMatrix:
      if (!dLdx && !dLdrho) return 0;
      return bwd_op(grid, o, true, args->bin_offsets, a, stream);
    default: {
      if (!dLdx && !dLds && !dLdrho) return 0;
      const bool ds_only = dLds && !dLdx && !dLdrho;
      return bwd_op(grid, o == Op::GradientHybrid ? Op::Gradient : o, !ds_only, args->bin_offsets, a, stream);
    }
  }
}

int sphops_neighbor_candidates(const sphops_grid* grid, const float* x, const int32_t* bo, int split_from_initialize,
                               void* stream) {
  return guarded([&] {
    require(grid != nullptr, "grid must not be NULL");
    require(bo != nullptr && (x != nullptr || grid->n_keys == 0), "null buffer");
    require(grid->dim == 2 || sphops::pk::aligned16(x), "3D positions must be 16-byte aligned");
    if (grid->n_keys == 0) return;
    // the split depends on the cell runs alone: the grid still holds the one
    // its last instantiate derived when the caller vouches for bo and no
    // build has replaced it since
    if (!split_from_initialize || grid->split_bo != bo) {
      OpPtrs a;
      a.x = x;
      sphops::forward(*grid, Op::NeighbourCandidates, bo, a, sphops::as_stream(stream));
      grid->split_bo = nullptr;
    }
    grid->split_key[0] = x;
    grid->split_key[1] = bo;
  });
}

static int neighbor_fill(const sphops_grid* grid, const float* x, const int32_t* bo, int32_t* nbr_start,
                         int32_t* nbr_index, int64_t index_capacity, int32_t* nbr_count, int64_t* nbr_total,
                         const sphops::FillTiles& ft, void* stream) {
  return guarded([&] {
    require(grid != nullptr, "grid must not be NULL");
    require(bo != nullptr && nbr_total != nullptr && (x != nullptr || grid->n_keys == 0), "null buffer");
    require(grid->dim == 2 || sphops::pk::aligned16(x), "3D positions must be 16-byte aligned");
    require(index_capacity >= 0, "negative index capacity");
    require(index_capacity <= sphops::kMaxListEntries, "index_capacity above 2^30 entries");
    const hipStream_t st = sphops::as_stream(stream);
    if (grid->n_keys == 0) {
      sphops::fill_u32(reinterpret_cast<uint32_t*>(nbr_total), 4, 0u, st);
      return;
    }
    require(nbr_start != nullptr && nbr_count != nullptr && (nbr_index != nullptr || index_capacity == 0),
            "null buffer");
    require(grid->split_key[0] == x && grid->split_key[1] == bo,
            "sphops_neighbor_fill must follow sphops_neighbor_candidates on the same grid with the same "
            "positions and bin_offsets");
    OpPtrs a;
    a.x = x;
    a.iout3 = nbr_start;
    a.iout = nbr_index;
    a.iout2 = nbr_count;
    a.used = reinterpret_cast<unsigned long long*>(nbr_total);
    a.cap = index_capacity;
    a.fill_tiles = ft;
    sphops::forward(*grid, Op::NeighbourFill, bo, a, st);
  });
}

int sphops_neighbor_fill(const sphops_grid* grid, const float* x, const int32_t* bo, int32_t* nbr_start,
                         int32_t* nbr_index, int64_t index_capacity, int32_t* nbr_count, int64_t* nbr_total,
                         void* stream) {
  return neighbor_fill(grid, x, bo, nbr_start, nbr_index, index_capacity, nbr_count, nbr_total, sphops::FillTiles{},
                       stream);
}

int sphops_neighbor_fill_tiled(const sphops_grid* grid, const float* x, const int32_t* bo, int32_t* nbr_start,
                               int32_t* nbr_index, int64_t index_capacity, int32_t* nbr_count, int64_t* nbr_total,
                               int32_t* nbr_own, uint32_t* cells, int32_t* cell_count, void* stream) {
  int st = guarded([&] {
    require(grid != nullptr, "grid must not be NULL");
    require(cell_count != nullptr && (grid->n_keys == 0 || (nbr_own != nullptr && cells != nullptr)),
            "null buffer");
    if (grid->n_keys == 0) sphops::fill_u32(reinterpret_cast<uint32_t*>(cell_count), 1, 0u, sphops::as_stream(stream));
  });
  if (st) return st;
  sphops::FillTiles ft{};
  if (grid->n_keys != 0) {
    ft.own = nbr_own;
    ft.cells = reinterpret_cast<uint2*>(cells);
    ft.count = cell_count;
    ft.tmin = (uint32_t)sphops::pk::kCellMin;
    ft.tmax = (uint32_t)sphops::pk::kCellMax;
  }
  return neighbor_fill(grid, x, bo, nbr_start, nbr_index, index_capacity, nbr_count, nbr_total, ft, stream);
}

int64_t sphops_neighbor_cell_capacity(const sphops_grid* grid) {
  if (grid == nullptr) {
    sphops::g_last_error = "grid must not be NULL";
    return -1;
  }
  return (int64_t)(grid->n_keys / sphops::pk::kCellMin + 1);
}

int sphops_neighbor_schedule(const sphops_grid* grid, const int32_t* nbr_count, int32_t* nbr_order,
                             uint32_t* nbr_waves, int32_t* wave_count, uint32_t* nbr_waves_split,
                             int32_t* wave_count_split, void* stream) {
  return guarded([&] {
    require(grid != nullptr, "grid must not be NULL");
    require(nbr_count != nullptr && wave_count != nullptr &&
                ((nbr_order != nullptr && nbr_waves != nullptr) || grid->n_keys == 0),
            "null buffer");
    const hipStream_t st = sphops::as_stream(stream);
    require((nbr_waves_split == nullptr) == (wave_count_split == nullptr),
            "nbr_waves_split and wave_count_split go together");
    if (grid->n_keys == 0) {
      sphops::fill_u32(reinterpret_cast<uint32_t*>(wave_count), 1, 0u, st);
      if (wave_count_split) sphops::fill_u32(reinterpret_cast<uint32_t*>(wave_count_split), 1, 0u, st);
      return;
    }
    sphops::run_neighbour_schedule(*grid, nbr_count, nbr_order, reinterpret_cast<uint2*>(nbr_waves), wave_count,
                                   reinterpret_cast<uint2*>(nbr_waves_split), wave_count_split, st);
  });
}

int sphops_neighbor_tiles(const sphops_grid* grid, const float* x, const int32_t* bo, const int32_t* nbr_count,
                          uint32_t* tile_units, int32_t* tile_unit_count, int32_t* nbr_order_sparse,
                          uint32_t* nbr_waves_sparse, int32_t* wave_count_sparse, void* stream) {
  return guarded([&] {
    require(grid != nullptr, "grid must not be NULL");
    require(bo != nullptr && tile_unit_count != nullptr && wave_count_sparse != nullptr, "null buffer");
    const hipStream_t st = sphops::as_stream(stream);
    if (grid->n_keys == 0) {
      sphops::fill_u32(reinterpret_cast<uint32_t*>(tile_unit_count), 1, 0u, st);
      sphops::fill_u32(reinterpret_cast<uint32_t*>(wave_count_sparse), 1, 0u, st);
      return;
    }
    require(x != nullptr && nbr_count != nullptr && tile_units != nullptr && nbr_order_sparse != nullptr &&
                nbr_waves_sparse != nullptr,
            "null buffer");
    require(grid->dim == 2 || sphops::pk::aligned16(x), "3D positions must be 16-byte aligned");
    OpPtrs a;
    a.x = x;
    a.ncnt = nbr_count;
    a.tile_units = reinterpret_cast<const uint2*>(tile_units);
    a.tile_count = tile_unit_count;
    a.order_sparse = nbr_order_sparse;
    a.waves_sparse = reinterpret_cast<const uint2*>(nbr_waves_sparse);
    a.nwaves_sparse_dev = wave_count_sparse;
    sphops::forward(*grid, Op::NeighbourTiles, bo, a, st);
    // the tile build overwrote the fill's work split in the grid scratch: a
    // later fill needs sphops_neighbor_candidates again
    grid->split_key[0] = grid->split_key[1] = nullptr;
    grid->split_bo = nullptr;
  });
}

int64_t sphops_neighbor_tile_capacity(const sphops_grid* grid) {
  if (grid == nullptr) {
    sphops::g_last_error = "grid must not be NULL";
    return -1;
  }
  return (int64_t)(grid->n_keys / sphops::pk::kTileMinOcc + 1);
}

int64_t sphops_neighbor_wave_capacity(const sphops_grid* grid) {
  if (grid == nullptr) {
    sphops::g_last_error = "grid must not be NULL";
    return -1;
  }
  return (int64_t)sphops::neighbour_wave_capacity(*grid);
}

int sphops_copy_words_to_host(const void* device_src, void* host_dst, uint32_t words, void* stream) {
  return guarded([&] {
    require(words <= 256, "sphops_copy_words_to_host: at most 256 words");
    if (words == 0) return;
    require(device_src != nullptr && host_dst != nullptr, "null buffer");
    void* dev_view = nullptr;
    SPHOPS_HIP(hipHostGetDevicePointer(&dev_view, host_dst, 0));
    sphops::copy_words_to_host(static_cast<const uint32_t*>(device_src), static_cast<uint32_t*>(dev_view), words,
                               sphops::as_stream(stream));
  });
}

int sphops_safe_inv_sym_mat(const float* in, float* out, int64_t count, int dim, float tol, void* stream) {
  return guarded([&] {
    require(dim == 2 || dim == 3, "safe_inverse only supports 2x2 or 3x3 matrices.");
    require(count >= 0, "count must be >= 0");
    require(count == 0 || (in && out), "null buffer");
    sphops::run_safe_inv(in, out, (uint64_t)count, dim, tol, sphops::as_stream(stream));
  });
}

int sphops_perception_features_forward(int dim, const float* s, const float* blur, const float* grad_s,
                                       const float* grad_rho, float* z, int64_t particles, uint32_t C, float coef_s,
                                       float coef_rho, float total_mass, int flags, void* stream) {
  return guarded([&] {
    require(dim == 2 || dim == 3, "dim must be 2 or 3");
    require(particles >= 0, "particles must be >= 0");
    sphops::check_channels(C);
    require(particles == 0 || (s && blur && z), "null buffer");
    require(particles == 0 || !(flags & SPHOPS_GLUE_STATE_GRAD) || grad_s, "grad_s must not be NULL");
    require(particles == 0 || !(flags & SPHOPS_GLUE_DENSITY_GRAD) || grad_rho, "grad_rho must not be NULL");
    sphops::run_glue_forward(dim, s, blur, grad_s, grad_rho, z, (uint64_t)particles, C, coef_s, coef_rho,
                             total_mass, flags, sphops::as_stream(stream));
  });
}

int sphops_perception_features_backward(int dim, const float* dz, const float* grad_s, const float* grad_rho,
                                        float* d_s, float* d_blur, float* d_grad_s, float* d_grad_rho,
                                        int64_t particles, uint32_t C, float coef_s, float coef_rho,
                                        float total_mass, int flags, void* stream) {
  return guarded([&] {
    require(dim == 2 || dim == 3, "dim must be 2 or 3");
    require(particles >= 0, "particles must be >= 0");
    sphops::check_channels(C);
    require(particles == 0 || dz, "null buffer");
    require(particles == 0 || !d_grad_s || !(flags & SPHOPS_GLUE_LOG_NORM_GRAD) || grad_s,
            "grad_s must not be NULL");
    require(particles == 0 || !d_grad_rho || !(flags & SPHOPS_GLUE_LOG_NORM_DENSITY_GRAD) || grad_rho,
            "grad_rho must not be NULL");
    sphops::run_glue_backward(dim, dz, grad_s, grad_rho, d_s, d_blur, d_grad_s, d_grad_rho, (uint64_t)particles, C,
                              coef_s, coef_rho, total_mass, flags, sphops::as_stream(stream));
  });
}

int sphops_euler_update_forward(int dim, int P, const float* y, const float* x_bin, const float* s_bin,
                                const float* mask, const float* noise, float* x_out, float* s_out, float* dx_norm,
                                int64_t particles, uint32_t C, float alpha, float eps, float dt, float noise_std,
                                float sqrt_dt, void* stream) {
  return guarded([&] {
    require(dim == 2 || dim == 3, "dim must be 2 or 3");
    require(P == (dim == 2 ? 2 : 4), "P must be 2 in 2D and 4 in 3D");
    require(particles >= 0, "particles must be >= 0");
    sphops::check_channels(C);
    require(particles == 0 || (y && x_bin && s_bin && x_out && s_out), "null buffer");
    sphops::run_euler_forward(dim, y, x_bin, s_bin, mask, noise, x_out, s_out, dx_norm, (uint64_t)particles, C,
                              (uint32_t)P, alpha, eps, dt, noise_std, sqrt_dt, sphops::as_stream(stream));
  });
}

int sphops_euler_update_backward(int dim, int P, const float* y, const float* mask, const float* d_x_out,
                                 const float* d_s_out, const float* d_dx_norm, float* d_y, int64_t particles,
                                 uint32_t C, float alpha, float eps, float dt, void* stream) {
  return guarded([&] {
    require(dim == 2 || dim == 3, "dim must be 2 or 3");
    require(P == (dim == 2 ? 2 : 4), "P must be 2 in 2D and 4 in 3D");
    require(particles >= 0, "particles must be >= 0");
    sphops::check_channels(C);
    require(particles == 0 || (y && d_y), "null buffer");
    sphops::run_euler_backward(dim, y, mask, d_x_out, d_s_out, d_dx_norm, d_y, (uint64_t)particles, C, (uint32_t)P,
                               alpha, eps, dt, sphops::as_stream(stream));
  });
}

int sphops_splat_forward(const float* x, const float* color, const int32_t* starts, int64_t images,
                         int64_t particles, int ncolor, int img_size, double sigma, double lo, double hi,
                         int normalize_color, int y_up, double pixel_size, float* out, void* workspace,
                         void* stream) {
  return guarded([&] {
    const sphops::SplatParams sp = sphops::splat_params(images, particles, ncolor, img_size, sigma, lo, hi,
                                                        normalize_color, y_up, pixel_size);
    require(images == 0 || (starts && out), "null buffer");
    require(particles == 0 || (x && color && workspace), "null buffer");
    require(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "workspace must be 16-byte aligned");
    sphops::run_splat_forward(sp, x, color, starts, (int)images, particles, static_cast<float4*>(workspace), out,
                              sphops::as_stream(stream));
  });
}

int64_t sphops_splat_workspace_bytes(int64_t particles) { return particles > 0 ? 32 * particles : 0; }

int sphops_splat_backward(const float* x, const float* color, const int32_t* starts, int64_t images,
                          int64_t particles, int ncolor, int img_size, double sigma, double lo, double hi,
                          int normalize_color, int y_up, double pixel_size, const float* d_out, float* d_x,
                          float* d_color, void* stream) {
  return guarded([&] {
    const sphops::SplatParams sp = sphops::splat_params(images, particles, ncolor, img_size, sigma, lo, hi,
                                                        normalize_color, y_up, pixel_size);
    require(particles == 0 || (x && color && starts && d_out && d_x && d_color), "null buffer");
    require(particles == 0 || images >= 1, "particles need at least one image");
    sphops::run_splat_backward(sp, x, color, starts, (int)images, particles, d_out, d_x, d_color,
                               sphops::as_stream(stream));
  });
}

int64_t sphops_linear_weight_grad_workspace_bytes(int64_t rows, int in_features, int out_features) {
  if (rows < 0 || in_features < 1 || out_features < 1) return 0;
  return 4 * sphops::linear_grad_chunks(rows, in_features, out_features) * ((int64_t)in_features * out_features + out_features);
}

}  // extern "C"

namespace {

int linear_weight_grad(const float* x, const float* dy, float* dw, float* db, int64_t rows, int in_features,
                       int out_features, void* workspace, bool relu_x, void* stream) {
  return guarded([&] {
    require(rows >= 0 && rows <= sphops::kMaxLinearRows, "rows must be in [0, " +
                                                             std::to_string(sphops::kMaxLinearRows) + "]");
    require(in_features >= 1 && out_features >= 1 && in_features <= sphops::kMaxLinearFeatures &&
                out_features <= sphops::kMaxLinearFeatures,
            "in_features and out_features must be in [1, " + std::to_string(sphops::kMaxLinearFeatures) + "]");
    require(sphops::linear_grad_fits(rows, in_features, out_features),
            "layer too large: more than 2^25 (row chunk, 32-row output band) pairs");
    require(dw != nullptr && (rows == 0 || (x && dy && workspace)), "null buffer");
    sphops::run_linear_weight_grad(x, dy, dw, db, rows, in_features, out_features,
                                   static_cast<float*>(workspace), relu_x, sphops::as_stream(stream));
  });
}

}  // namespace

extern "C" {

int sphops_linear_weight_grad(const float* x, const float* dy, float* dw, float* db, int64_t rows,
                              int in_features, int out_features, void* workspace, void* stream) {
  return linear_weight_grad(x, dy, dw, db, rows, in_features, out_features, workspace, false, stream);
}

int sphops_relu_linear_weight_grad(const float* a, const float* dy, float* dw, float* db, int64_t rows,
                                   int in_features, int out_features, void* workspace, void* stream) {
  return linear_weight_grad(a, dy, dw, db, rows, in_features, out_features, workspace, true, stream);
}

int sphops_relu_linear_forward(const float* a, const float* w, const float* b, float* y, int64_t rows,
                               int in_features, int out_features, void* stream) {
  return guarded([&] {
    require(rows >= 0, "rows must be >= 0");
    require(in_features >= 4 && in_features <= sphops::kMaxReluLinearIn && in_features % 4 == 0,
            "in_features must be a multiple of 4 in [4, " + std::to_string(sphops::kMaxReluLinearIn) + "]");
    require(out_features >= 1 && out_features <= sphops::kMaxReluLinearOut,
            "out_features must be in [1, " + std::to_string(sphops::kMaxReluLinearOut) + "]");
    require(sphops::relu_linear_forward_fits(rows), "too many rows");
    require(rows == 0 || (a && w && y), "null buffer");
    require(reinterpret_cast<uintptr_t>(a) % 16 == 0, "a must be 16-byte aligned");
    sphops::run_relu_linear_forward(a, w, b, y, rows, in_features, out_features, sphops::as_stream(stream));
  });
}

int sphops_relu_linear_input_grad(const float* dy, const float* w, const float* h, float* dx, int64_t rows,
                                  int in_features, int out_features, void* stream) {
  return guarded([&] {
    require(rows >= 0, "rows must be >= 0");
    require(in_features >= 1 && in_features <= sphops::kMaxLinearFeatures && out_features >= 1 &&
                out_features <= sphops::kMaxReluLinearOut,
            "in_features must be in [1, " + std::to_string(sphops::kMaxLinearFeatures) + "] and out_features in [1, " +
                std::to_string(sphops::kMaxReluLinearOut) + "]");
    require(sphops::relu_linear_input_grad_fits(rows, in_features), "too many rows x in_features");
    require(rows == 0 || (dy && w && h && dx), "null buffer");
    sphops::run_relu_linear_input_grad(dy, w, h, dx, rows, in_features, out_features, sphops::as_stream(stream));
  });
}

}  // extern "C"

// ------------------------------------------------ binning without allocation
//
// sphops_initialize_noalloc runs sphops_initialize's kernels with their
// scratch (sort keys and values, radix histograms, scan partials, chunk
// tables, block flags) carved from `scratch`, a file-scope device array, so a
// call allocates nothing, on the device or the host.  Each GPU the library
// runs on holds its own copy of the array until the process ends.  Host code
// never uses the array's name as an address: the device address comes from
// hipGetSymbolAddress, once per device, on the first call with that device
// current.  Every call on one GPU shares that GPU's array; each call writes
// (or clears) every word it later reads, so the previous call's contents do
// not matter, but calls that overlap on one GPU race.

namespace {

constexpr uint64_t kNoAllocMaxKeys = 1ull << 20;   // B * N
constexpr uint64_t kNoAllocMaxCells = 1ull << 28;  // B * G
constexpr int kNoAllocMaxDevices = 64;

// Word offsets of the scratch pieces for a grid of n_keys particles, n_tiles
// radix tiles and n_chunks cell chunks; each piece starts on 256 bytes.
struct NoAllocLayout {
  uint64_t kv[2], hist, flags, chunk_lo, scan, scan_len, words;
};

constexpr uint64_t pad_words(uint64_t w) { return (w + 63) & ~uint64_t(63); }

constexpr NoAllocLayout noalloc_layout(uint64_t n_keys, uint64_t n_tiles, uint64_t n_chunks) {
  NoAllocLayout l{};
  uint64_t at = 0;
  for (int i = 0; i < 2; ++i) {  // 64-bit words
    l.kv[i] = at;
    at += pad_words(2 * (n_keys + 1));
  }
  l.hist = at;
  at += pad_words(sphops::hist_words(n_tiles));
  l.flags = at;
  at += pad_words(n_keys + 1);
  l.chunk_lo = at;
  at += pad_words(n_chunks + 1);
  l.scan = at;
  l.scan_len = sphops::scan_tmp_elems(sphops::scan_words(n_keys, n_tiles, n_chunks));
  at += pad_words(l.scan_len);
  l.words = at;
  return l;
}

// Every piece grows with its size, so the largest grid the entry point
// accepts bounds every layout: about 22 MiB.
constexpr uint64_t kNoAllocWords =
    noalloc_layout(kNoAllocMaxKeys, (kNoAllocMaxKeys + 4095) / 4096, (kNoAllocMaxCells + 1 + 1023) / 1024).words;

std::atomic<uint32_t*> g_scratch_addr[kNoAllocMaxDevices];

}  // namespace

static __device__ __align__(256) uint32_t scratch[kNoAllocWords];

namespace {

// Device address of `scratch` on the current device (looked up once per device).
uint32_t* scratch_on_current_device(int* device) {
  int dev = 0;
  SPHOPS_HIP(hipGetDevice(&dev));
  require(dev >= 0 && dev < kNoAllocMaxDevices, "sphops_initialize_noalloc: device ordinal above 63");
  uint32_t* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    void* q = nullptr;
    SPHOPS_HIP(hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)));
    p = static_cast<uint32_t*>(q);
    g_scratch_addr[dev].store(p, std::memory_order_release);
  }
  *device = dev;
  return p;
}

}  // namespace

extern "C" {

int sphops_initialize_noalloc(int dim, int boundary, int mode, const int32_t* grid_size, float eps,
                              uint32_t particle_count, uint32_t batch_size, uint32_t max_particles_per_block,
                              const float* positions, int32_t* permutation, int32_t* bin_offsets,
                              int32_t* block_info, int32_t* total_blocks, void* stream) {
  return guarded([&] {
    Grid g;
    sphops::setup_grid(g, dim, boundary, mode, grid_size, eps, particle_count, batch_size, max_particles_per_block);
    require(g.n_keys <= kNoAllocMaxKeys, "sphops_initialize_noalloc: batch_size * particle_count above 2^20");
    require(g.n_cells <= kNoAllocMaxCells, "sphops_initialize_noalloc: batch_size * cell_count above 2^28");
    check_initialize_args(g, positions, permutation, bin_offsets, block_info);
    const NoAllocLayout l = noalloc_layout(g.n_keys, g.n_tiles, g.n_chunks);
    require(l.words <= kNoAllocWords, "sphops_initialize_noalloc: scratch layout exceeds the static array");
    uint32_t* s = scratch_on_current_device(&g.device);
    for (int i = 0; i < 2; ++i) {
      g.kv[i] = reinterpret_cast<uint64_t*>(s + l.kv[i]);
    }
    g.hist = s + l.hist;
    g.flags = s + l.flags;
    g.chunk_lo = s + l.chunk_lo;
    g.scan_tmp = s + l.scan;
    g.scan_tmp_len = l.scan_len;
    sphops::run_instantiate(g, positions, permutation, bin_offsets, block_info, total_blocks,
                            sphops::as_stream(stream));
  });
}

}  // extern "C"

