// Host-side internals shared by the sphops translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdexcept>
#include <string>

#include "sphops_device.hpp"
#include "sphops_hip.h"

namespace sphops {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

#define SPHOPS_HIP(call)                                                                  \
  do {                                                                                    \
    hipError_t e_ = (call);                                                               \
    if (e_ != hipSuccess)                                                                 \
      throw ::sphops::Error(std::string("HIP error at ") + __FILE__ + ":" +               \
                            std::to_string(__LINE__) + " - " + hipGetErrorString(e_));    \
  } while (0)

#define SPHOPS_LAUNCHED() SPHOPS_HIP(hipGetLastError())

// Grid object: static parameters plus the scratch buffers binning needs
// (the reference's HashGrid::_init allocations, sphops/sph_cuda.cu:1880-1895).
struct Grid {
  GridParams p{};
  int dim = 2;
  bool periodic = false;
  bool particle_mode = false;
  uint64_t max_blocks = 1;
  int device = 0;

  // scratch, sized at creation for B*N keys and B*G+1 cells
  uint64_t n_keys = 0;        // B*N
  uint64_t n_cells = 0;       // B*G
  uint64_t n_tiles = 0;       // radix tiles
  uint64_t n_chunks = 0;      // cell chunks for bin_offsets
  // radix-sort ping-pong buffers of B*N + 1 words (cell key << 32 | particle
  // index); after the sort the free one holds instantiate's flag scan
  uint64_t* kv[2] = {nullptr, nullptr};
  uint32_t* hist = nullptr;       // 256 * n_tiles (+1)
  uint32_t* scan_tmp = nullptr;   // partial sums for device scans
  uint64_t scan_tmp_len = 0;
  uint32_t* chunk_lo = nullptr;   // n_chunks + 1: sorted keys below each chunk's first cell
  uint32_t* flags = nullptr;      // B*N + 1 (block starts, then their scan)
  float4* packed = nullptr;       // B*N (x, y, z|0, weight) read by the pair kernels
  // work split of the neighbour-list fill:
  int32_t* sparse_len = nullptr;  // B*N: list length of the particles outside the cell tiles, -1 for the others
  int32_t* unit_len = nullptr;    // B*N: particles of the unit starting here (> 0), 0, or -1 (lone particle)
  uint2* units = nullptr;         // B*N: unit descriptors {first particle, particles}
  int32_t* unit_total = nullptr;  // number of units (device)
  unsigned long long* stripes = nullptr;  // kFillStripes * kStripeWords: row-allocation counters of the fill
  // (positions, bin_offsets) of the last neighbour_candidates call: the fill
  // reads the work split and ranges that call left and must get the same
  mutable const void* split_key[2] = {nullptr, nullptr};
  // bin_offsets written by the last instantiate when the work split
  // (unit_len, units, unit_total) still holds what that call derived from the
  // sorted keys; null once a build has replaced it
  mutable const int32_t* split_bo = nullptr;
};

// binning.hip
// inv (B*N, or null): the inverse permutation, inv[b*N + slot] = the index
// within cloud b of the particle binned to that slot
void run_instantiate(Grid& g, const float* pos, int32_t* perm, int32_t* bin_offsets,
                     int32_t* block_info, int32_t* total_blocks, hipStream_t st, int32_t* inv = nullptr);
void run_bin_particles(const Grid& g, const float* in_pos, const float* in_state, const float* in_mass,
                       const int32_t* perm, float* out_pos, float* out_state, float* out_mass,
                       uint32_t C, bool forward, hipStream_t st);
// Words of partial sums a device scan of n words needs (every recursion
// level padded to a tile of 4096).
constexpr uint64_t kScanTile = 4096;
constexpr uint64_t scan_tmp_elems(uint64_t n) {
  uint64_t total = 0;
  while (n > kScanTile) {
    n = (n + kScanTile - 1) / kScanTile;
    total += n + kScanTile;
  }
  return total + 1;
}

// Words of the longest device scan run on a grid's scratch: the radix
// histograms, the block flags (B*N + 1) and the chunk starts.
constexpr uint64_t scan_words(uint64_t n_keys, uint64_t n_tiles, uint64_t n_chunks) {
  const uint64_t a = 1024ull * n_tiles, b = n_keys + 1, c = n_chunks + 1;
  return a > b ? (a > c ? a : c) : (b > c ? b : c);
}
inline uint64_t scan_words(const Grid& g) { return scan_words(g.n_keys, g.n_tiles, g.n_chunks); }
// in-place exclusive scan of n <= B*N+1 words with the grid's scratch
void exclusive_scan_u32(const Grid& g, uint32_t* data, uint64_t n, uint32_t* total, hipStream_t st);

// perception.hip
enum class Op : int {
  Count = 0,
  Density = 1,
  DensityGradient = 2,
  MomentMatrix = 3,
  Blur = 4,
  Gradient = 5,
  GradientHybrid = 6,
  DensityPair = 7,      // density + density gradient in one pass
  BlurGradientHybrid = 8,  // blur + gradient_hybrid in one pass
  NeighbourCandidates = 9,  // scanned stencil candidate counts (int32, the list's row offsets)
  NeighbourFill = 10,       // in-radius neighbour indices and counts (int32)
  NeighbourTiles = 11,      // cell tiles of the pass-B backward and the schedule of the other particles
};

// Cell tiles of the list (OT = true in the fill): the rows of the particles
// of a cell holding tmin .. tmax particles keep their own-cell entries (self
// included) last, own[k] receives their number (0 for every other particle
// and for rows walked on the stencil), and each such cell is appended to
// cells as {first particle, particles}, count[0] cells in all (appended in
// no fixed order; capacity B*N / tmin).  The pair kernels that know the
// cells (the pass-B backward) skip a row's last own[k] entries and take
// those pairs from the cell kernel, which evaluates each pair of a cell once
// for both of its ends; the other kernels read the whole row.
struct FillTiles {
  int32_t* own;
  uint2* cells;
  int32_t* count;
  uint32_t tmin, tmax;
};

struct OpPtrs {
  const float* x = nullptr;
  const float* m = nullptr;
  const float* rho = nullptr;
  const float* s = nullptr;
  const float* g = nullptr;   // upstream gradient (backward)
  const float* g2 = nullptr;  // second upstream gradient (fused backward)
  float* out0 = nullptr;      // forward output / grad_x
  float* out1 = nullptr;      // grad_s
  float* out2 = nullptr;      // grad_rho
  float* out3 = nullptr;      // second forward output (fused forward)
  int32_t* iout = nullptr;    // neighbour indices (list build)
  int32_t* iout2 = nullptr;   // neighbour counts (list build)
  int32_t* iout3 = nullptr;   // list row starts (list build)
  unsigned long long* used = nullptr;  // entries the fill asked for (list build)
  int64_t cap = 0;            // capacity of iout for the fill
  const int32_t* bo = nullptr;     // bin_offsets (set by the dispatch; the stencil walk of unstored rows)
  const int32_t* nptr = nullptr;  // list row start per particle (B*N)
  const int32_t* ncnt = nullptr;  // list length per particle (B*N)
  const int32_t* nidx = nullptr;  // neighbour indices; non-null selects list traversal
  const float4* xw = nullptr;     // packed positions and weights (set by the launcher)
  float4* xw_buf = nullptr;       // caller's buffer for them (null: the grid's scratch) ...
  bool xw_ready = false;          // ... already holding this call's records
  const int32_t* order = nullptr; // particles in schedule order (optional, list traversal)
  const uint2* waves = nullptr;   // per-wave descriptors {first slot in order, group size << 8 | particles}
  uint32_t nwaves = 0;
  const uint2* waves2 = nullptr;  // descriptors for lane-split channel kernels (group sizes kSplitGroups)
  uint32_t nwaves2 = 0;
  // optional device copies of the wave counts; when set the kernels read them
  // and nwaves / nwaves2 only size the launch (an upper bound)
  const int32_t* nwaves_dev = nullptr;
  const int32_t* nwaves2_dev = nullptr;
  // optional cell tiles of the pass-B backward (sphops_neighbor_tiles): the
  // units, their device count, and the split schedule of the other particles
  const uint2* tile_units = nullptr;
  const int32_t* tile_count = nullptr;
  const int32_t* order_sparse = nullptr;
  const uint2* waves_sparse = nullptr;
  uint32_t nwaves_sparse = 0;
  const int32_t* nwaves_sparse_dev = nullptr;
  // cell tiles: written by the list fill (fill_tiles.own non-null) and read
  // by the pass-B backward (nown, cells, cell_count, all three or none)
  FillTiles fill_tiles{};
  const int32_t* nown = nullptr;
  const uint2* cells = nullptr;
  const int32_t* cell_count = nullptr;
  uint32_t C = 0;
  float tol = 1e-3f;
};

void run_forward(const Grid& g, Op op, const int32_t* bin_offsets, const OpPtrs& a, hipStream_t st);
// full = false selects the dL/ds-only variant (Blur, Gradient)
void run_backward(const Grid& g, Op op, bool full, const int32_t* bin_offsets, const OpPtrs& a,
                  hipStream_t st);
// Pair-kernel schedule: per tile of 4096 binned particles, a stable partition
// by neighbour-list length class (kListClasses / kListGroups), tiles in
// order; one descriptor per wave {first slot in order, group size << 8 | particles}.
void run_neighbour_schedule(const Grid& g, const int32_t* ncnt, int32_t* order, uint2* waves, int32_t* wave_total,
                            uint2* waves2, int32_t* wave_total2, hipStream_t st);
// The split-group schedule alone (kSplitGroups) over lengths `len`; items of
// negative length are left out.
void run_split_schedule(const Grid& g, const int32_t* len, int32_t* order, uint2* waves, int32_t* wave_total,
                        hipStream_t st);
// upper bound of the number of waves a schedule can hold
uint64_t neighbour_wave_capacity(const Grid& g);
// Units of the cell-major fill: units[u] = {first particle, count} for every
// particle k with unit_len[k] > 0 (flags[k] = 1 there, 0 elsewhere), in
// particle order; their number goes to unit_total.  Scans flags in place.
void run_unit_schedule(const Grid& g, hipStream_t st);
// Neighbour-list fill: cells of two or more particles are filled cell-major
// in units of at most kUnitParticles particles of one cell, one wave per
// unit; particles alone in their cell one lane each.
// Largest neighbour-list index buffer (entries): byte offsets into it fit in 32 bits.
constexpr int64_t kMaxListEntries = (int64_t)1 << 30;
constexpr int32_t kUnitParticles = 8;
// Row allocation of the fill: up to kFillStripes counters, each owning an
// equal slice of the index buffer of at least kStripeMinEntries entries and
// serving about kStripeMinUnits units or more (so that slices fill evenly);
// a wave takes its blocks from counter (wave id mod stripes).  One counter
// for the whole device serialises the atomics of ~10^5 units; striped, they
// spread over as many addresses.  Counters lie kStripeWords 64-bit words
// apart (256 bytes).
constexpr uint32_t kFillStripes = 256;
constexpr uint32_t kStripeWords = 32;
// word of a stripe's 256-byte record that counts the units taken from the
// list fill's unit queue of that stripe (a cache line apart from the row
// counters at words 0-2)
constexpr uint32_t kUnitQueueWord = 16;
constexpr int64_t kStripeMinEntries = (int64_t)1 << 15;
constexpr uint64_t kStripeMinUnits = 64;
// Work classes of the list traversal: class q holds
// the items whose length is <= t[q] (and above the previous bound), the last
// class the rest; each class is served by groups of g[q] lanes per particle
// (a power of two <= 64).  Bounds double from class to class, and so do the
// group sizes up to their cap, so a class spans a factor of two in items per
// lane.  The tables were chosen by timing the cfg5 workload on an MI355X.
constexpr int kNumClasses = 8;
struct ClassBounds {
  int32_t t[kNumClasses - 1];
};
struct GroupSizes {
  int32_t g[kNumClasses];
};
// pair lists: about 6-12 pairs per lane
constexpr ClassBounds kListClasses{{6, 12, 24, 48, 96, 192, 384}};
constexpr GroupSizes kListGroups{{1, 1, 2, 4, 8, 16, 32, 64}};
// lane-split channel kernels: four lanes (channel slices) per pair stream,
// 1, 1, 1, 1, 4, 8, 16, 16 streams per particle (about 12-48 pairs each)
constexpr GroupSizes kSplitGroups{{4, 4, 4, 4, 16, 32, 64, 64}};
void run_safe_inv(const float* in, float* out, uint64_t count, int dim, float tol, hipStream_t st);
void fill_u32(uint32_t* p, uint64_t n, uint32_t v, hipStream_t st);
// words (<= 256) from device memory to pinned host memory (its device view)
void copy_words_to_host(const uint32_t* src, uint32_t* dst_device_view, uint32_t words, hipStream_t st);
// perceive_glue.hip: perception features of NPA.perceive (include/sphops_hip.h)
void run_glue_forward(int dim, const float* s, const float* blur, const float* grad_s, const float* grad_rho,
                      float* z, uint64_t n, uint32_t C, float coef_s, float coef_rho, float total_mass, int flags,
                      hipStream_t st);
void run_glue_backward(int dim, const float* dz, const float* grad_s, const float* grad_rho, float* d_s,
                       float* d_blur, float* d_grad_s, float* d_grad_rho, uint64_t n, uint32_t C, float coef_s,
                       float coef_rho, float total_mass, int flags, hipStream_t st);
void run_euler_forward(int dim, const float* y, const float* x_bin, const float* s_bin, const float* mask,
                       const float* noise, float* x_out, float* s_out, float* dx_norm, uint64_t n, uint32_t C,
                       uint32_t P, float alpha, float eps, float dt, float noise_std, float sqrt_dt, hipStream_t st);
void run_euler_backward(int dim, const float* y, const float* mask, const float* d_x_out, const float* d_s_out,
                        const float* d_dx_norm, float* d_y, uint64_t n, uint32_t C, uint32_t P, float alpha,
                        float eps, float dt, hipStream_t st);
// splatting.hip: 2D Gaussian splatting (utils/splatting.py:6-117)
struct SplatParams {
  int H;             // image side (img_size)
  int r;             // patch radius
  float lo;          // world lower bound
  float inv_span;    // 1 / (hi - lo), both in fp32
  float scale;       // img_size - 1
  float inv_two_s2;  // 1 / (2 sigma^2), sigma in pixels
  float K;           // (img_size * pixel_size / (hi - lo))^2: patch weight total when normalising
  int normalize;     // normalize_color
  int y_up;
  int ncolor;        // colour row width; the last three channels are r, g, b
};
constexpr int kMaxSplatRadius = 255;
void run_splat_forward(const SplatParams& sp, const float* x, const float* color, const int32_t* starts, int images,
                       int64_t n, float4* rec, float* out, hipStream_t st);
void run_splat_backward(const SplatParams& sp, const float* x, const float* color, const int32_t* starts, int images,
                        int64_t n, const float* d_img, float* d_x, float* d_color, hipStream_t st);

// linear_grad.hip: weight / bias gradients of a linear layer over many rows
constexpr int64_t kMaxChunkRows = 8192;
constexpr int64_t kMaxLinearRows = kMaxChunkRows * 65535;
constexpr int kMaxLinearFeatures = 32768;  // keeps chunk byte offsets below 2^31
constexpr int64_t kMaxLinearWaves = int64_t(1) << 25;  // one wave per (row chunk, output job); 2^31 threads
int64_t linear_grad_chunks(int64_t rows, int nin, int nout);
bool linear_grad_fits(int64_t rows, int nin, int nout);
void run_linear_weight_grad(const float* x, const float* dy, float* dw, float* db, int64_t rows, int nin, int nout,
                            float* work, bool relu_x, hipStream_t st);
constexpr int kMaxReluLinearOut = 64;  // two 32-wide tiles of W kept in registers
constexpr int kMaxReluLinearIn = 256;  // forward: W's columns for one output in registers
bool relu_linear_forward_fits(int64_t rows);
void run_relu_linear_forward(const float* a, const float* w, const float* b, float* y, int64_t rows, int nin,
                             int nout, hipStream_t st);
bool relu_linear_input_grad_fits(int64_t rows, int nin);
void run_relu_linear_input_grad(const float* dy, const float* w, const float* h, float* dx, int64_t rows, int nin,
                                int nout, hipStream_t st);

constexpr uint32_t kMaxChannels = 64;
constexpr int kRadixBins = 1024;  // digit values per radix-sort pass (10 bits)
// Words of the radix histograms: kRadixBins tile counts per tile of 4096
// keys, then the kRadixBins digit totals.
constexpr uint64_t hist_words(uint64_t n_tiles) { return (uint64_t)kRadixBins * (n_tiles + 1); }
inline uint64_t hist_words(const Grid& g) { return hist_words(g.n_tiles); }

}  // namespace sphops
