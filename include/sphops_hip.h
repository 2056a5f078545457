/*
 * sphops_hip.h — C ABI of the MI355X (gfx950) sphops library, libsphops_hip.so.
 *
 * This replaces the reference's nanobind module `sph_cuda`
 * (TheDevilWillBeBee/NPA, sphops/sph_cuda.cu:3380-3441): the eight HashGrid
 * classes become one opaque handle created with (dim, boundary, mode), and every
 * method becomes a function taking raw device pointers.  Shapes are fixed by the
 * handle (B clouds of N particles, G cells per cloud) plus an explicit
 * feature_dim where the reference read it from an array shape.
 *
 * Conventions
 *  - All pointers are device pointers to contiguous row-major fp32 / int32
 *    buffers allocated by the caller (the library never allocates user
 *    tensors; sphops/sph.py allocates every output with torch.empty*).
 *  - Positions are float2 per particle in 2D and float4 (x, y, z, unused w) in
 *    3D, as in the reference (positions shape (B, N, 2) or (B, N, 4)).
 *  - `stream` is a hipStream_t; work is enqueued on it and the call returns
 *    without synchronising.
 *  - Return value 0 means success; nonzero means failure, with a message in
 *    sphops_last_error() (thread-local).  Shape checking is the caller's job
 *    (the reference's validate_array_shape, sphops/utils.cuh:526-566, lives in
 *    the Python layer).
 *  - Results are deterministic: no floating-point atomics are used.
 */
#ifndef SPHOPS_HIP_H
#define SPHOPS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPHOPS_ABI_VERSION 21

#define SPHOPS_CLAMPED 0
#define SPHOPS_PERIODIC 1
#define SPHOPS_MODE_GRID 0     /* row-major cell hash  (reference "grid" mode)     */
#define SPHOPS_MODE_PARTICLE 1 /* Morton cell hash     (reference "particle" mode) */

typedef struct sphops_grid sphops_grid;

/* ABI version of the loaded library (SPHOPS_ABI_VERSION). */
int sphops_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* sphops_last_error(void);

/* A grid of no particles (particle_count or batch_size 0) is valid: every
 * call then validates its other arguments and launches nothing, and the
 * per-particle buffers (positions, states, outputs, block_info with no rows)
 * may be NULL, as torch passes them for empty tensors.  bin_offsets is
 * always B*G+1 entries and receives zeros. */

/* HashGrid{2D,3D}{Periodic,Box} / VHashGrid... constructors
 * (sphops/sph_cuda.cu:3049-3093 classes, HashGrid::_init sph_cuda.cu:1836-1899;
 * Python entry sphops/sph.py:48-78).  grid_size has `dim` entries. */
int sphops_grid_create(int dim, int boundary, int mode, const int32_t* grid_size, float eps,
                       uint32_t particle_count, uint32_t batch_size, uint32_t max_particles_per_block,
                       sphops_grid** out);
void sphops_grid_destroy(sphops_grid* grid);

/* Read-only properties (sph_cuda.cu:3229-3237 `max_blocks`, and the kernel
 * coefficients HashGrid::_init derives, sph_cuda.cu:1862-1878). */
int64_t sphops_grid_max_blocks(const sphops_grid* grid);
int sphops_grid_coefficients(const sphops_grid* grid, float* poly6, float* spiky);

/* HashGrid::initialize (sph_cuda.cu:1926-1992): cell keys, stable sort,
 * permutation (B,N), bin_offsets (B*G+1, global values), block_info
 * (max_blocks,4; grid mode only, ignored in particle mode).  total_blocks
 * (one int32, may be NULL) receives the number of block_info rows in use, kept
 * per snapshot instead of inside the grid. */
int sphops_initialize(sphops_grid* grid, const float* positions, int32_t* permutation, int32_t* bin_offsets,
                      int32_t* block_info, int32_t* total_blocks, void* stream);

/* sphops_initialize that also writes the inverse permutation (B,N int32):
 * inverse[b*N + i] = the index within cloud b of the particle binned to slot
 * i, so permutation[b*N + inverse[b*N + i]] == i.  No counterpart in the
 * reference.  sphops_bin_particles with the inverse in place of the
 * permutation is then the unbin (sphops_backward_bin_particles) done as a
 * scatter, which moves the rows faster than the gather.  The outputs other
 * than inverse are sphops_initialize's, bit for bit. */
int sphops_initialize_inverse(sphops_grid* grid, const float* positions, int32_t* permutation,
                              int32_t* inverse, int32_t* bin_offsets, int32_t* block_info,
                              int32_t* total_blocks, void* stream);

/* sphops_initialize without a grid object and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * (or host) memory while they run -- code under HIP-graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  The grid is described by
 * the arguments of sphops_grid_create; the outputs are sphops_initialize's,
 * bit for bit.  The sort, scan and block-table scratch comes from one static
 * device array per GPU (about 22 MiB, held until the process ends), so
 * batch_size * particle_count must be at most 2^20 and batch_size * cell count
 * at most 2^28; larger grids fail with an error and no work queued.  Calls
 * that overlap on one GPU share the array and race: serialise them (one
 * stream, or events). */
int sphops_initialize_noalloc(int dim, int boundary, int mode, const int32_t* grid_size, float eps,
                              uint32_t particle_count, uint32_t batch_size, uint32_t max_particles_per_block,
                              const float* positions, int32_t* permutation, int32_t* bin_offsets,
                              int32_t* block_info, int32_t* total_blocks, void* stream);

/* HashGrid::bin_particles (sph_cuda.cu:1994-2024): out[b, perm[b,i]] = in[b,i]. */
int sphops_bin_particles(const sphops_grid* grid, const float* in_pos, const float* in_state,
                         const float* in_mass, const int32_t* permutation, float* out_pos, float* out_state,
                         float* out_mass, uint32_t feature_dim, void* stream);

/* HashGrid::backward_bin_particles (sph_cuda.cu:2026-2056): out[b,i] = in[b, perm[b,i]]
 * (also the reference's unbin_particles, sphops/sph.py:187-198).  In both
 * directions the two mass pointers may be NULL together (no reference
 * counterpart): the mass rows are then not moved, as for a backward whose
 * mass needs no gradient. */
int sphops_backward_bin_particles(const sphops_grid* grid, const float* grad_out_pos,
                                  const float* grad_out_state, const float* grad_out_mass,
                                  const int32_t* permutation, float* grad_in_pos, float* grad_in_state,
                                  float* grad_in_mass, uint32_t feature_dim, void* stream);

/* Forward operators on binned particles (sph_cuda.cu:2058-2499).  `block_info`
 * is accepted for interface parity and may be NULL: neighbour ranges are read
 * from bin_offsets alone. */
int sphops_count_forward(const sphops_grid* grid, const float* x, float* count, const int32_t* bin_offsets,
                         const int32_t* block_info, void* stream);
int sphops_density_forward(const sphops_grid* grid, const float* x, const float* mass, float* rho,
                           const int32_t* bin_offsets, const int32_t* block_info, void* stream);
int sphops_blur_forward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                        const float* state_in, float* state_out, uint32_t feature_dim, const int32_t* bin_offsets,
                        const int32_t* block_info, void* stream);
int sphops_gradient_forward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                            const float* state_in, float* state_gradient_out, uint32_t feature_dim,
                            const int32_t* bin_offsets, const int32_t* block_info, void* stream);
int sphops_density_gradient_forward(const sphops_grid* grid, const float* x, const float* mass,
                                    float* density_gradient_out, const int32_t* bin_offsets,
                                    const int32_t* block_info, void* stream);
int sphops_moment_matrix_forward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                                 float* moment_matrix_out, const int32_t* bin_offsets, const int32_t* block_info,
                                 void* stream);

/* gradient_hybrid forward value raw @ safe_inv(M, tol) in one pass.  No native
 * counterpart in the reference: it replaces the Python composite
 * moment_matrix -> safe_inv_sym_mat -> gradient -> matmul (sphops/sph.py:474-484);
 * its backward is sphops_gradient_backward (straight-through). */
int sphops_gradient_hybrid_forward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                                   const float* state_in, float* out, uint32_t feature_dim, float tol,
                                   const int32_t* bin_offsets, const int32_t* block_info, void* stream);

/* Backward operators (sph_cuda.cu:2501-3046).  The flags say which gradients
 * the caller needs, as the reference's dLdx/dLds/dLdrho arguments: all false is
 * a no-op; dLds alone selects the dL/ds-only kernel; anything else computes and
 * writes every gradient buffer of the operator. */
int sphops_density_backward(const sphops_grid* grid, const float* x, const float* mass, const float* dL_rho,
                            float* grad_x, const int32_t* bin_offsets, const int32_t* block_info, int dLdx,
                            void* stream);
int sphops_blur_backward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                         const float* state_in, const float* dL_blur, float* grad_x, float* grad_s,
                         float* grad_rho, uint32_t feature_dim, const int32_t* bin_offsets,
                         const int32_t* block_info, int dLdx, int dLds, int dLdrho, void* stream);
int sphops_density_gradient_backward(const sphops_grid* grid, const float* x, const float* mass,
                                     const float* dL_density_gradient, float* grad_x, const int32_t* bin_offsets,
                                     const int32_t* block_info, int dLdx, void* stream);
int sphops_gradient_backward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                             const float* state_in, const float* dL_gradient, float* grad_x, float* grad_s,
                             float* grad_rho, uint32_t feature_dim, const int32_t* bin_offsets,
                             const int32_t* block_info, int dLdx, int dLds, int dLdrho, void* stream);
int sphops_moment_matrix_backward(const sphops_grid* grid, const float* x, const float* rho, const float* mass,
                                  const float* dL_moment_matrix, float* grad_x, float* grad_rho,
                                  const int32_t* bin_offsets, const int32_t* block_info, int dLdx, int dLdrho,
                                  void* stream);

/* ---- generic operator interface (the path the Python layer uses) -------
 *
 * One entry point per direction for every perception operator, with an
 * optional per-snapshot neighbour list.  The reference has no counterpart:
 * its methods above traverse the cell stencil on every call.  Building the
 * list once per snapshot (sphops_neighbor_candidates, sphops_neighbor_fill,
 * sphops_neighbor_schedule) and passing it here makes every later operator
 * walk only in-radius pairs; the pair set is identical, only the fp32
 * summation order can differ.
 *
 * Two fused codes evaluate operators that the reference always runs over the
 * same neighbours one after the other (models/npa.py:106-126) in one pass:
 * DENSITY_PAIR = density (out) + density_gradient (out2), both mass-weighted;
 * BLUR_GRADIENT_HYBRID = blur (out) + gradient_hybrid (out2), both reading
 * x, rho, mass and state.  Their backward takes the first operator's
 * upstream in `upstream` and the second's in `upstream2` and writes the sum
 * of both operators' gradients. */

#define SPHOPS_OP_COUNT 0
#define SPHOPS_OP_DENSITY 1
#define SPHOPS_OP_DENSITY_GRADIENT 2
#define SPHOPS_OP_MOMENT_MATRIX 3
#define SPHOPS_OP_BLUR 4
#define SPHOPS_OP_GRADIENT 5
#define SPHOPS_OP_GRADIENT_HYBRID 6
#define SPHOPS_OP_DENSITY_PAIR 7
#define SPHOPS_OP_BLUR_GRADIENT_HYBRID 8

typedef struct sphops_args {
  const float* x;              /* binned positions (B,N,2|4) */
  const float* mass;           /* (B,N) */
  const float* rho;            /* (B,N): blur, gradient, gradient_hybrid, moment_matrix */
  const float* state;          /* (B,N,C): blur, gradient, gradient_hybrid */
  const float* upstream;       /* backward: dL/d(output), shaped like the forward output */
  float* out;                  /* forward: the output; backward: dL/dx (B,N,2|4) */
  float* grad_state;           /* backward: dL/ds (B,N,C) */
  float* grad_rho;             /* backward: dL/drho (B,N) */
  uint32_t feature_dim;        /* C */
  float tol;                   /* gradient_hybrid: safe-inverse threshold */
  const int32_t* bin_offsets;  /* (B*G+1) from sphops_initialize */
  const int32_t* nbr_start;    /* optional list row start per particle (sphops_neighbor_fill) */
  const int32_t* nbr_count;    /* optional list length per particle from sphops_neighbor_fill */
  const int32_t* nbr_index;    /* optional list entries from sphops_neighbor_fill; NULL: scan the stencil */
  const int32_t* nbr_order;    /* optional schedule from sphops_neighbor_schedule: particle order ... */
  const uint32_t* nbr_waves;   /* ... its wave descriptors (2 words per wave) ... */
  int32_t nbr_wave_count;      /* ... and the host copy of its wave count */
  const uint32_t* nbr_waves_split;  /* optional second descriptor table of the schedule ... */
  int32_t nbr_wave_count_split;     /* ... and its wave count (lane-split channel kernels) */
  const float* upstream2;      /* fused backward: dL/d(second output) */
  float* out2;                 /* fused forward: the second output */
  /* Optional device copies of the two wave counts (the wave_count and
   * wave_count_split words that sphops_neighbor_schedule writes).  When set,
   * the kernels read the counts there, and nbr_wave_count(_split) need only
   * bound them (sphops_neighbor_wave_capacity), so the caller never reads a
   * count back: a step can be captured in a HIP graph. */
  const int32_t* nbr_wave_count_device;
  const int32_t* nbr_wave_count_split_device;
  /* Optional cell tiles from sphops_neighbor_tiles, used by the
   * BLUR_GRADIENT_HYBRID backward at C = 16 (with the split schedule above):
   * the units ({first particle, particles} pairs) and their device count,
   * and the split schedule of the particles outside the units (order, wave
   * descriptors, a bound of the wave count for the launch, the device count). */
  const uint32_t* tile_units;
  const int32_t* tile_unit_count;
  const int32_t* nbr_order_sparse;
  const uint32_t* nbr_waves_sparse;
  int32_t nbr_wave_count_sparse;
  const int32_t* nbr_wave_count_sparse_device;
  /* Optional (x, y, z|0, weight) records of the call's particles, B*N
   * 16-byte-aligned float4, with the operator's neighbour weight: the mass
   * for DENSITY, DENSITY_GRADIENT and DENSITY_PAIR, mass / rho for BLUR,
   * GRADIENT, GRADIENT_HYBRID, MOMENT_MATRIX and BLUR_GRADIENT_HYBRID (no
   * reference counterpart).  With packed_valid = 0 the call writes them there
   * instead of the grid's scratch; with packed_valid = 1 it reads them as they
   * are, which is how a backward reuses what its forward wrote for the same
   * x, mass and rho (one packing pass fewer).  NULL: the grid's scratch. */
  float* packed;
  int32_t packed_valid;
  /* Optional cell tiles from sphops_neighbor_fill_tiled (no reference
   * counterpart; all three or none): the own-cell entry counts, the cell
   * table ({first particle, particles} pairs) and its device count.  The
   * BLUR, GRADIENT(_HYBRID) and BLUR_GRADIENT_HYBRID backward with 16
   * channels on 3D clamped grids then take each tiled cell's inner pairs from
   * a kernel that evaluates each pair once for both ends; every other
   * operator reads the rows whole. */
  const int32_t* nbr_own;
  const uint32_t* cells;
  const int32_t* cell_count;
} sphops_args;

/* Forward operator `op` (SPHOPS_OP_*) on binned particles. */
int sphops_forward(const sphops_grid* grid, int op, const sphops_args* args, void* stream);

/* Backward of operator `op` (not COUNT); flags as in the per-operator
 * functions above.  For SPHOPS_OP_GRADIENT_HYBRID it is the gradient
 * operator's backward (straight-through, sphops/sph.py:482); the fused codes
 * need both upstreams (pass zeros, or better the single operator, when one
 * output has no gradient). */
int sphops_backward(const sphops_grid* grid, int op, int dLdx, int dLds, int dLdrho, const sphops_args* args,
                    void* stream);

/* First step of the neighbour list: the split of the fill's work (units of
 * up to 8 particles of one cell with two or more particles, which share the
 * cell's 3^D stencil, the cells the reference traverses; particles alone in
 * their cell), left in the grid's scratch for sphops_neighbor_fill.  The
 * split depends on the cell runs alone, and sphops_initialize derives it from
 * the sorted keys as it writes bin_offsets: with split_from_initialize = 1
 * the caller states that bin_offsets is, unmodified, what this grid's last
 * sphops_initialize wrote, and the call then reuses that split (no kernel
 * runs); with 0, or when the grid's scratch no longer holds that split (a
 * later build on another bin_offsets, sphops_neighbor_tiles), it is computed
 * from x and bin_offsets. */
int sphops_neighbor_candidates(const sphops_grid* grid, const float* x, const int32_t* bin_offsets,
                               int split_from_initialize, void* stream);

/* In-radius neighbours (pairs |r| < eps incl. self) of every binned particle,
 * in stencil order: row i is nbr_index[nbr_start[i] .. nbr_start[i] +
 * nbr_count[i]) (nbr_start and nbr_count have B*N entries).  Rows are
 * compact, allocated in blocks from counters that each own an equal slice of
 * nbr_index (up to 256 slices of at least 2^15 entries), so nbr_index needs
 * the number of in-radius pairs plus a margin for uneven slices.  nbr_total
 * (two device int64) receives the number of in-radius pairs, stored or not,
 * and the number of pairs in rows that were not stored (0: the list is
 * complete).  A row that does not fit in its slice is not stored: its
 * nbr_count is -1 - (the particle's stencil candidates), and every operator
 * walks that particle's stencil instead, so results never depend on the
 * capacity (a caller sizes the next snapshot's buffer from nbr_total, read
 * back whenever convenient).  Where a row lands depends on the order blocks
 * are taken; rows, their order and all results do not.  index_capacity is at
 * most 2^30.  Must follow
 * sphops_neighbor_candidates on the same grid with the same x and bin_offsets
 * (checked by pointer; their contents must not change in between), with no
 * other candidates call on that grid in between. */
int sphops_neighbor_fill(const sphops_grid* grid, const float* x, const int32_t* bin_offsets, int32_t* nbr_start,
                         int32_t* nbr_index, int64_t index_capacity, int32_t* nbr_count, int64_t* nbr_total,
                         void* stream);

/* sphops_neighbor_fill with cell tiles (no reference counterpart): the rows
 * of the particles of every cell holding 16 to 64 particles keep their
 * own-cell entries (self included) last, in stencil order like the rest of
 * the row; nbr_own (B*N) receives how many (0 for every other particle and for
 * rows not stored), cells (capacity sphops_neighbor_cell_capacity pairs) one
 * {first particle, particles} pair per such cell in no fixed order, and
 * cell_count (one device int32) their number.  The rows hold the same
 * entries as sphops_neighbor_fill's, so every operator accepts the list;
 * the backward operators that know the tiles (sphops_args.nbr_own) skip the
 * last nbr_own entries and evaluate those pairs per cell instead. */
int sphops_neighbor_fill_tiled(const sphops_grid* grid, const float* x, const int32_t* bin_offsets,
                               int32_t* nbr_start, int32_t* nbr_index, int64_t index_capacity, int32_t* nbr_count,
                               int64_t* nbr_total, int32_t* nbr_own, uint32_t* cells, int32_t* cell_count,
                               void* stream);

/* Capacity (cell descriptors) the cells buffer of sphops_neighbor_fill_tiled needs. */
int64_t sphops_neighbor_cell_capacity(const sphops_grid* grid);

/* Schedule for list traversal.  The binned particles are cut into tiles of
 * 4096; within a tile they are partitioned (stably) by list length into eight
 * classes (<=6, <=12, <=24, ..., <=384, >384 neighbours), served by groups of
 * 1, 1, 2, 4, ..., 64 lanes per particle; tiles stay in order, so each region
 * of space is processed in one stretch.  From the list lengths nbr_count
 * (B*N), nbr_order (B*N) receives the particles in that order, nbr_waves
 * (2 words per wave, capacity sphops_neighbor_wave_capacity) one descriptor
 * per 64-lane wave {first slot in nbr_order, group size << 8 | particles in
 * the wave}, wave_count (one device int32) the number of waves.  Optionally
 * (both non-NULL) nbr_waves_split / wave_count_split receive a second table
 * over the same order with 4, 4, 4, 4, 16, 32, 64, 64 lanes per particle,
 * used by the kernels that split 16 or 32 channels over four lanes (the
 * fused blur + gradient_hybrid pass). */
int sphops_neighbor_schedule(const sphops_grid* grid, const int32_t* nbr_count, int32_t* nbr_order,
                             uint32_t* nbr_waves, int32_t* wave_count, uint32_t* nbr_waves_split,
                             int32_t* wave_count_split, void* stream);

/* Cell tiles of a snapshot for the pass-B backward (no reference
 * counterpart).  Cells holding at least 8 binned particles are cut into units of up to 32
 * consecutive particles: tile_units receives {first particle, particles} per
 * unit (capacity sphops_neighbor_tile_capacity pairs), tile_unit_count (one
 * device int32) their number.  The backward then stages each unit's stencil
 * rows in LDS once instead of loading a neighbour's rows once per pair.  The
 * other particles get the split schedule of sphops_neighbor_schedule, over
 * their own order: nbr_order_sparse (B*N), nbr_waves_sparse (capacity
 * sphops_neighbor_wave_capacity), wave_count_sparse (device int32).  Needs
 * the snapshot's x_bin, bin_offsets and list lengths (sphops_neighbor_fill).
 * It overwrites the fill's work split in the grid scratch: call it after the
 * snapshot's last fill; a later fill fails until sphops_neighbor_candidates
 * runs again. */
int sphops_neighbor_tiles(const sphops_grid* grid, const float* x, const int32_t* bin_offsets,
                          const int32_t* nbr_count, uint32_t* tile_units, int32_t* tile_unit_count,
                          int32_t* nbr_order_sparse, uint32_t* nbr_waves_sparse, int32_t* wave_count_sparse,
                          void* stream);

/* Capacity (unit descriptors) tile_units must have for this grid. */
int64_t sphops_neighbor_tile_capacity(const sphops_grid* grid);

/* Number of wave descriptors nbr_waves must hold for this grid (B*N + 8 per tile of 4096). */
int64_t sphops_neighbor_wave_capacity(const sphops_grid* grid);

/* Copy of `words` (at most 256) 32-bit words from device memory into pinned
 * host memory allocated with hipHostMalloc (torch's pin_memory), written by
 * one small kernel on `stream` with system-scope stores (no reference
 * counterpart): the host reads them once an event recorded after the call
 * has completed.  The Python layer reads the list totals back this way;
 * unlike an asynchronous device-to-host copy it adds no copy engine
 * dependency to the stream. */
int sphops_copy_words_to_host(const void* device_src, void* host_dst, uint32_t words, void* stream);

/* Module function safe_inv_sym_mat (sph_cuda.cu:3181-3226): `count` symmetric
 * dim x dim matrices (dim 2 or 3), identity where |det| < tol. */
int sphops_safe_inv_sym_mat(const float* in_matrix, float* out_matrix, int64_t count, int dim, float tol,
                            void* stream);

/* Perception features of NPA.perceive (models/npa.py:87-137; no counterpart
 * in the reference's native module: the reference builds them with torch
 * elementwise ops and torch.cat).  For `particles` rows of C channels in D =
 * dim dimensions, z (particles, W) receives, in order:
 *   s (C), blur (C),
 *   if STATE_GRAD: grad_s * coef_s (C x D, row-major), log-normalised per
 *     channel over D when LOG_NORM_GRAD,
 *   if DENSITY_GRAD: grad_rho * coef_rho / total_mass (D), log-normalised when
 *     LOG_NORM_DENSITY_GRAD,
 * so W = 2C + (STATE_GRAD ? C*D : 0) + (DENSITY_GRAD ? D : 0).  The
 * log-normalisation is log(1 + |v|) * v / max(|v|, 1e-12)
 * (models/npa.py:83-85).  grad_s / grad_rho may be NULL when their flag is
 * off. */
#define SPHOPS_GLUE_STATE_GRAD 1
#define SPHOPS_GLUE_LOG_NORM_GRAD 2
#define SPHOPS_GLUE_DENSITY_GRAD 4
#define SPHOPS_GLUE_LOG_NORM_DENSITY_GRAD 8
int sphops_perception_features_forward(int dim, const float* s, const float* blur, const float* grad_s,
                                       const float* grad_rho, float* z, int64_t particles, uint32_t C, float coef_s,
                                       float coef_rho, float total_mass, int flags, void* stream);

/* Backward of sphops_perception_features_forward: from dL/dz (particles, W)
 * and the forward's grad_s / grad_rho, writes dL/ds, dL/dblur (particles, C),
 * dL/dgrad_s (particles, C, D) and dL/dgrad_rho (particles, D); any output may
 * be NULL (not computed). */
int sphops_perception_features_backward(int dim, const float* dz, const float* grad_s, const float* grad_rho,
                                        float* d_s, float* d_blur, float* d_grad_s, float* d_grad_rho,
                                        int64_t particles, uint32_t C, float coef_s, float coef_rho,
                                        float total_mass, int flags, void* stream);

/* Euler update of step_euler (models/npa.py:154-204, with the position-step
 * scaling of NPA.forward, models/npa.py:125-133; no counterpart in the
 * reference's native module).  y (particles, dim + C) is the MLP output
 * [a, ds]; x_bin (particles, P) with P = dim (2D) or 4 (3D, lane 3 padding);
 * s_bin (particles, C); mask (particles) or NULL (all ones); noise
 * (particles, P) standard normals or NULL.  Writes
 *   dx = alpha * a * eps / (1 + |a|),
 *   x_out = x_bin + dt * [dx, 0] * mask (+ noise * noise_std * sqrt_dt * mask),
 *   s_out = s_bin + dt * ds * mask,
 *   dx_norm = |dx| (particles), unless NULL. */
int sphops_euler_update_forward(int dim, int P, const float* y, const float* x_bin, const float* s_bin,
                                const float* mask, const float* noise, float* x_out, float* s_out, float* dx_norm,
                                int64_t particles, uint32_t C, float alpha, float eps, float dt, float noise_std,
                                float sqrt_dt, void* stream);

/* Backward of sphops_euler_update_forward with respect to y: from dL/dx_out
 * (particles, P), dL/ds_out (particles, C) and dL/d dx_norm (particles), any
 * of them NULL (zero), writes dL/dy (particles, dim + C).  The gradients with
 * respect to x_bin and s_bin are dL/dx_out and dL/ds_out themselves. */
int sphops_euler_update_backward(int dim, int P, const float* y, const float* mask, const float* d_x_out,
                                 const float* d_s_out, const float* d_dx_norm, float* d_y, int64_t particles,
                                 uint32_t C, float alpha, float eps, float dt, void* stream);

/* Differentiable 2D Gaussian splatting (utils/splatting.py:6-117; no
 * counterpart in the reference's native module: the reference scatters with
 * torch.scatter_add_).  Particles of image b are rows starts[b] ..
 * starts[b + 1] - 1 of x (particles, 2) and color (particles, ncolor);
 * starts (images + 1 int32, device) is ascending with starts[0] = 0 and
 * starts[images] = particles.  out (images, img_size, img_size, 4) receives
 * [r, g, b, density] per pixel: the sum over particles of w and w * rgb
 * (rgb = the last three colour channels), with w the particle's Gaussian
 * weight at the pixel over a (2r+1)^2 patch around floor(pos),
 * pos = (x - lo) / (hi - lo) * (img_size - 1) (y flipped with y_up), all as
 * the reference's splat_particles with the same arguments computes them.
 * Sums run in ascending particle order (deterministic).  workspace holds
 * sphops_splat_workspace_bytes(particles) bytes of per-particle records. */
int sphops_splat_forward(const float* x, const float* color, const int32_t* starts, int64_t images,
                         int64_t particles, int ncolor, int img_size, double sigma, double lo, double hi,
                         int normalize_color, int y_up, double pixel_size, float* out, void* workspace,
                         void* stream);

/* Bytes of the workspace sphops_splat_forward needs for `particles`
 * particles (32 per particle; the caller allocates it, 16-byte aligned). */
int64_t sphops_splat_workspace_bytes(int64_t particles);

/* Backward of sphops_splat_forward: from dL/dout (images, img_size, img_size,
 * 4), writes dL/dx (particles, 2) and dL/dcolor (particles, ncolor; zero
 * except the last three channels). */
int sphops_splat_backward(const float* x, const float* color, const int32_t* starts, int64_t images,
                          int64_t particles, int ncolor, int img_size, double sigma, double lo, double hi,
                          int normalize_color, int y_up, double pixel_size, const float* d_out, float* d_x,
                          float* d_color, void* stream);

/* Weight and bias gradients of a linear layer y = x W^T + b over `rows` rows
 * (no counterpart in the reference's native module: the NPA MLP is
 * torch.nn.Linear, models/npa.py:63-78).  x (rows, in_features) and dy
 * (rows, out_features) row-major fp32; writes dw = dy^T x (out_features,
 * in_features) and, unless NULL, db = the column sums of dy (out_features).
 * in_features and out_features are at most 32768.  Computed on the fp32
 * matrix cores; deterministic (chunk partial sums added in a fixed order).
 * workspace holds
 * sphops_linear_weight_grad_workspace_bytes(rows, in_features, out_features)
 * bytes. */
int sphops_linear_weight_grad(const float* x, const float* dy, float* dw, float* db, int64_t rows,
                              int in_features, int out_features, void* workspace, void* stream);
int64_t sphops_linear_weight_grad_workspace_bytes(int64_t rows, int in_features, int out_features);

/* Input gradient through a ReLU and a linear layer, y = relu(a) W^T + b
 * (torch.nn.ReLU then torch.nn.Linear, models/npa.py:65-68; no counterpart in
 * the reference's native module): dx = 0 where h <= 0, else dy W, with
 * h = relu(a) (rows, in_features), dy (rows, out_features), w (out_features,
 * in_features) and dx (rows, in_features) row-major fp32.  The zeroing follows
 * torch's threshold_backward(grad, h, 0).  in_features is at most 32768 and
 * out_features at most 64.  dy W runs on the fp32 matrix cores;
 * deterministic. */
int sphops_relu_linear_input_grad(const float* dy, const float* w, const float* h, float* dx, int64_t rows,
                                  int in_features, int out_features, void* stream);

/* Forward through a ReLU and a linear layer (torch.nn.ReLU then
 * torch.nn.Linear, models/npa.py:65-68; no counterpart in the reference's
 * native module): y = relu(a) W^T + b, with a (rows, in_features), w
 * (out_features, in_features), b (out_features, or NULL) and y (rows,
 * out_features) row-major fp32; relu as torch's (NaN stays NaN).  in_features
 * is a multiple of 4 up to 256, out_features at most 64, and a is 16-byte
 * aligned.  relu(a) is not written; the backward takes a itself:
 * sphops_relu_linear_input_grad(dy, w, a, ...) (a <= 0 exactly where
 * relu(a) <= 0) and sphops_relu_linear_weight_grad.  On the fp32 matrix
 * cores; deterministic. */
int sphops_relu_linear_forward(const float* a, const float* w, const float* b, float* y, int64_t rows,
                               int in_features, int out_features, void* stream);

/* sphops_linear_weight_grad with x = relu(a): dw = dy^T relu(a), db = the
 * column sums of dy; the same workspace size. */
int sphops_relu_linear_weight_grad(const float* a, const float* dy, float* dw, float* db, int64_t rows,
                                   int in_features, int out_features, void* workspace, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPHOPS_HIP_H */
