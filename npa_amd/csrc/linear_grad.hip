// Weight and bias gradients of a linear layer over very many rows, for the
// NPA MLP (models/npa.py:63-78 of the reference, torch.nn.Linear), for gfx950.
//
// dW = dY^T X (out x in) and db = sum over rows of dY, with X (rows x in) and
// dY (rows x out) row-major fp32.  The output is small (128 x 83 for the NPA
// MLP's first layer) and the reduction is long (one row per particle, 10^6
// at the 3D stress size); the library GEMM picks a handful of output tiles
// for that shape and leaves most of the GPU idle.  Here the reduction runs on
// the fp32 matrix cores (v_mfma_f32_32x32x2_f32: a 32 x 32 tile, two rows per
// instruction):
// * the rows are split into chunks and the output into jobs of one 32-row
//   band of dW by up to four 32-column tiles; each wave takes one (chunk,
//   job), reads its rows straight from HBM (lanes 0-31 one row, lanes 32-63
//   the next, 32 consecutive columns each, through buffer loads whose range
//   check zeroes what lies past the chunk or the layer) 16 rows ahead of the
//   matrix instructions, and keeps its tiles in registers;
// * the waves of one workgroup share a chunk when a chunk has four or more
//   jobs, so the X columns they all read come from one L1;
// * each wave writes its tiles (and, for the jobs of the first column tile,
//   the column sums of its dY band) as the chunk's partial sums, and a second
//   kernel adds the partials in a fixed order, so the result is
//   deterministic.
#include "sphops_internal.hpp"
#include "sphops_device.hpp"

namespace sphops {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMT = 32;             // matrix-core tile side
constexpr int kPairs = 8;           // row pairs per load group (16 rows)
constexpr int kGroupRows = 2 * kPairs;
constexpr int kMaxTilesPerJob = 4;  // column tiles per wave
constexpr int kWaveTarget = 2048;   // waves per launch at large row counts (two per SIMD)
constexpr int64_t kMinChunkRows = 128;
constexpr int kReduceWaves = 16;    // chunk-sum workgroup: 16 waves x 64 elements

struct LinearPlan {
  int o_tiles, i_tiles, i_groups, ti, jobs;
  int64_t chunk_rows, chunks;
};

LinearPlan linear_plan(int64_t rows, int nin, int nout) {
  LinearPlan p;
  p.o_tiles = (nout + kMT - 1) / kMT;
  p.i_tiles = (nin + kMT - 1) / kMT;
  p.i_groups = (p.i_tiles + kMaxTilesPerJob - 1) / kMaxTilesPerJob;
  p.ti = (p.i_tiles + p.i_groups - 1) / p.i_groups;
  p.jobs = p.o_tiles * p.i_groups;
  const int64_t want = std::max<int64_t>(1, kWaveTarget / p.jobs);
  int64_t c = (rows + want - 1) / want;
  c = (c + kGroupRows - 1) / kGroupRows * kGroupRows;
  p.chunk_rows = std::min<int64_t>(kMaxChunkRows, std::max<int64_t>(kMinChunkRows, c));
  p.chunks = rows > 0 ? (rows + p.chunk_rows - 1) / p.chunk_rows : 0;
  return p;
}

// Operands are read through buffer resources that span one chunk's rows:
// the hardware returns 0 for a byte offset at or past the resource's size, so
// rows past the chunk and lanes whose column lies past the layer (offset
// kOffLane) load zeros with no select after the load, and the next group's
// loads stay in flight under the current group's matrix instructions.  The
// offsets stay below 2^32 for features up to kMaxLinearFeatures.
constexpr uint32_t kOffLane = 0x80000000u;
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 buffer descriptor word 3: 32-bit raw data

__device__ __forceinline__ __amdgpu_buffer_rsrc_t chunk_rsrc(const float* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes, kRsrcWord3);
}

__device__ __forceinline__ float load_b32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// Wave `wid` = chunk * jobs + job.  Job j covers dW rows o0 = 32 (j / i_groups)
// .. +31 and columns i0 = 32 TI (j % i_groups) .. + 32 TI - 1.  For the matrix
// instruction, lane l supplies A[m = l % 32][k = l / 32] = dY[row_k][o0 + m]
// and B[k = l / 32][n = l % 32] = X[row_k][i0 + 32 t + n]; result register r
// of lane l holds tile row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
template <int TI, bool RELU_X>
__global__ __launch_bounds__(256) void k_linear_mfma(const float* __restrict__ x, const float* __restrict__ dy,
                                                     float* __restrict__ part, int64_t rows, int nin, int nout,
                                                     int i_groups, int jobs, int64_t chunk_rows,
                                                     uint32_t total_waves) {
  const uint32_t wid = __builtin_amdgcn_readfirstlane(xcd_block_id() * 4u + threadIdx.x / 64u);
  if (wid >= total_waves) return;
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int64_t chunk = wid / (uint32_t)jobs;
  const int job = (int)(wid % (uint32_t)jobs);
  const int o0 = (job / i_groups) * kMT, i0 = (job % i_groups) * TI * kMT;
  const int64_t r0 = chunk * chunk_rows, r1 = min<int64_t>(rows, r0 + chunk_rows);
  const bool a_col = o0 + c < nout;
  const __amdgpu_buffer_rsrc_t ra = chunk_rsrc(dy + r0 * nout, (r1 - r0) * nout * 4);
  const __amdgpu_buffer_rsrc_t rb = chunk_rsrc(x + r0 * nin, (r1 - r0) * nin * 4);
  // byte offset of the lane's element in chunk row h
  const uint32_t la = a_col ? (uint32_t)(h * nout + o0 + c) * 4u : kOffLane;
  uint32_t lb[TI];
#pragma unroll
  for (int t = 0; t < TI; ++t) lb[t] = i0 + kMT * t + c < nin ? (uint32_t)(h * nin + i0 + kMT * t + c) * 4u : kOffLane;

  f32x16 acc[TI];
#pragma unroll
  for (int t = 0; t < TI; ++t) acc[t] = f32x16{};
  float accb = 0.0f;

  // two load groups in ping-pong: group g + 16 loads while group g computes
  float a0[kPairs], b0[kPairs][TI], a1[kPairs], b1[kPairs][TI];
  auto load = [&](int64_t g, float (&va)[kPairs], float (&vb)[kPairs][TI]) {
    const uint32_t lr = (uint32_t)(g - r0);
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      va[p] = load_b32(ra, la + (lr + 2 * p) * (uint32_t)nout * 4u);
#pragma unroll
      for (int t = 0; t < TI; ++t) vb[p][t] = load_b32(rb, lb[t] + (lr + 2 * p) * (uint32_t)nin * 4u);
    }
  };
  auto compute = [&](const float (&va)[kPairs], const float (&vb)[kPairs][TI]) {
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      accb += va[p];
#pragma unroll
      for (int t = 0; t < TI; ++t) {
        // relu(x) as torch computes it: NaN stays NaN
        const float bx = RELU_X ? (vb[p][t] <= 0.0f ? 0.0f : vb[p][t]) : vb[p][t];
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[p], bx, acc[t], 0, 0, 0);
      }
    }
  };
  // Past the chunk's last row the loads return zeros, which add nothing.  The
  // scheduling barriers keep the compiler from sinking a group's loads down
  // to their first use, which would leave them no time in flight.
  load(r0, a0, b0);
  for (int64_t g = r0; g < r1; g += 2 * kGroupRows) {
    load(g + kGroupRows, a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    compute(a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    load(g + 2 * kGroupRows, a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    compute(a1, b1);
    __builtin_amdgcn_sched_barrier(0);
  }

  const int64_t nw = (int64_t)nout * nin;
  float* pw = part + chunk * (nw + nout);
#pragma unroll
  for (int t = 0; t < TI; ++t) {
    const int col = i0 + kMT * t + c;
    if (col >= nin) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = o0 + 8 * (r / 4) + 4 * h + (r % 4);
      if (m < nout) pw[(int64_t)m * nin + col] = acc[t][r];
    }
  }
  if (job % i_groups == 0) {
    accb += __shfl_xor(accb, 32);
    if (h == 0 && a_col) pw[nw + o0 + c] = accb;
  }
}

// out[e] = sum over chunks of part[chunk * n + e] (n = out * in + out: dW
// then db), in a fixed order: wave q of the workgroup keeps eight running
// sums over chunks q + 16 (8 s + k), k = 0..7, adds them k = 0..7, and wave 0
// adds the 16 waves' sums q = 0..15.
__global__ __launch_bounds__(64 * kReduceWaves) void k_chunk_reduce(const float* __restrict__ part,
                                                                    float* __restrict__ dw,
                                                                    float* __restrict__ db, int64_t nw, int nout,
                                                                    int64_t chunks) {
  __shared__ float red[kReduceWaves][64];
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int64_t n = nw + nout;
  const int64_t e = (int64_t)blockIdx.x * 64 + lane;
  float s[8] = {};
  if (e < n) {
    int64_t c = q;
    for (; c + 7 * kReduceWaves < chunks; c += 8 * kReduceWaves) {
#pragma unroll
      for (int k = 0; k < 8; ++k) s[k] += part[(c + k * kReduceWaves) * n + e];
    }
    for (int k = 0; c < chunks; c += kReduceWaves, ++k) s[k] += part[c * n + e];
  }
  float total = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) total += s[k];
  red[q][lane] = total;
  __syncthreads();
  if (q == 0 && e < n) {
    float t = 0.0f;
#pragma unroll
    for (int k = 0; k < kReduceWaves; ++k) t += red[k][lane];
    if (e < nw) dw[e] = t;
    else if (db) db[e - nw] = t;
  }
}

template <int TI>
void launch_mfma(const LinearPlan& p, const float* x, const float* dy, float* part, int64_t rows, int nin, int nout,
                 bool relu_x, hipStream_t st) {
  const uint32_t waves = (uint32_t)(p.jobs * p.chunks);
  if (relu_x)
    hipLaunchKernelGGL((k_linear_mfma<TI, true>), dim3((waves + 3) / 4), dim3(256), 0, st, x, dy, part, rows, nin,
                       nout, p.i_groups, p.jobs, p.chunk_rows, waves);
  else
    hipLaunchKernelGGL((k_linear_mfma<TI, false>), dim3((waves + 3) / 4), dim3(256), 0, st, x, dy, part, rows, nin,
                       nout, p.i_groups, p.jobs, p.chunk_rows, waves);
  SPHOPS_LAUNCHED();
}

// Input gradient through a ReLU and a linear layer, y = relu(a) W^T + b:
// dA[r][n] = 0 where h[r][n] = relu(a)[r][n] <= 0 (torch's threshold_backward),
// else (dY W)[r][n].  It replaces the dH = dY W product and the elementwise
// ReLU backward, so dH never goes to memory: per row it reads dY and h and
// writes dA.  dY W runs on the matrix cores (K = nout padded to 2 KS): one
// wave per (TILES tiles of 32 rows, 128 columns) keeps W's four 32-column
// tiles as B operands in registers; for row tile i, lane l supplies A[m = l %
// 32][k = l / 32] = dY[32 i + m][2 s + k] at step s, and result register j of
// column tile t holds row 8 (j / 4) + 4 (l / 32) + j % 4, column 32 t + l % 32,
// where h is read and dA written.  Buffer resources over the wave's rows
// return zeros past the rows, past nout and past nin, and drop the stores
// there.
constexpr int kRLTiles = 4;

// Row tiles per wave: kRLTiles for long inputs, one (four times the waves)
// below 2^17 rows, where a quarter as many waves would leave most SIMDs idle.
int relu_linear_tiles(int64_t rows) { return rows >= (int64_t(1) << 17) ? kRLTiles : 1; }

template <int KS, int TILES>
__global__ __launch_bounds__(256) void k_relu_linear_dx(const float* __restrict__ dy, const float* __restrict__ w,
                                                        const float* __restrict__ h, float* __restrict__ dx,
                                                        int64_t rows, int nin, int nout, int col_blocks,
                                                        uint32_t total_waves) {
  const uint32_t wid = __builtin_amdgcn_readfirstlane(xcd_block_id() * 4u + threadIdx.x / 64u);
  if (wid >= total_waves) return;
  const int lane = threadIdx.x & 63, c = lane & 31, hh = lane >> 5;
  const int n0 = (int)(wid % (uint32_t)col_blocks) * 128;
  const int64_t r0 = (int64_t)(wid / (uint32_t)col_blocks) * (TILES * kMT);
  const int64_t nr = min<int64_t>(TILES * kMT, rows - r0);
  const __amdgpu_buffer_rsrc_t rdy = chunk_rsrc(dy + r0 * nout, nr * nout * 4);
  const __amdgpu_buffer_rsrc_t rh = chunk_rsrc(h + r0 * nin, nr * nin * 4);
  const __amdgpu_buffer_rsrc_t rdx = chunk_rsrc(dx + r0 * nin, nr * nin * 4);

  float bw[4][KS];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int n = n0 + kMT * t + c;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int k = 2 * s + hh;
      bw[t][s] = (k < nout && n < nin) ? w[(int64_t)k * nin + n] : 0.0f;
    }
  }
  // byte offsets: the lane's dY entries (row c of the tile, k = 2 s + hh) and
  // its h / dA column in each column tile
  uint32_t ka[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) ka[s] = 2 * s + hh < nout ? (uint32_t)(c * nout + 2 * s + hh) * 4u : kOffLane;
  uint32_t cn[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) cn[t] = n0 + kMT * t + c < nin ? (uint32_t)(n0 + kMT * t + c) * 4u : kOffLane;

  for (int i = 0; i < TILES; ++i) {
    if (i * kMT >= nr) break;  // uniform
    const uint32_t ra = (uint32_t)(i * kMT * nout) * 4u;
    float a[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) a[s] = load_b32(rdy, ka[s] + ra);
    float hv[4][16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t rr = (uint32_t)(i * kMT + 8 * (j / 4) + 4 * hh + (j % 4)) * (uint32_t)nin * 4u;
#pragma unroll
      for (int t = 0; t < 4; ++t) hv[t][j] = load_b32(rh, cn[t] + rr);
    }
    f32x16 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = f32x16{};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], bw[t][s], acc[t], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t rr = (uint32_t)(i * kMT + 8 * (j / 4) + 4 * hh + (j % 4)) * (uint32_t)nin * 4u;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float v = hv[t][j] <= 0.0f ? 0.0f : acc[t][j];
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rdx, cn[t] + rr, 0, 0);
      }
    }
  }
}

template <int KS>
void launch_relu_dx(const float* dy, const float* w, const float* h, float* dx, int64_t rows, int nin, int nout,
                    hipStream_t st) {
  const int col_blocks = (nin + 127) / 128;
  const int tiles = relu_linear_tiles(rows);
  const int64_t rows_per_wave = tiles * kMT;
  const uint32_t waves = (uint32_t)(((rows + rows_per_wave - 1) / rows_per_wave) * col_blocks);
  if (tiles == kRLTiles)
    hipLaunchKernelGGL((k_relu_linear_dx<KS, kRLTiles>), dim3((waves + 3) / 4), dim3(256), 0, st, dy, w, h, dx, rows,
                       nin, nout, col_blocks, waves);
  else
    hipLaunchKernelGGL((k_relu_linear_dx<KS, 1>), dim3((waves + 3) / 4), dim3(256), 0, st, dy, w, h, dx, rows, nin,
                       nout, col_blocks, waves);
  SPHOPS_LAUNCHED();
}

// Forward through a ReLU and a linear layer, y = relu(a) W^T + b, for at most
// 64 outputs and in_features a multiple of 4 up to 256, on the matrix cores:
// one wave per TILES tiles of 32 rows keeps W's 32-output tiles as B
// operands in registers.  Lane l (row m = l % 32 of the tile, half q = l / 32)
// loads a[m][8 g + 4 q .. + 3] as one 16-byte load per g; at step (g, j) it
// supplies A[m][q] = relu(a[m][8 g + 4 q + j]) and B[q][n] = W[n][8 g + 4 q +
// j], so the steps cover every k once.  relu(a) never goes to memory.
template <int G, int NT, int TILES>
__global__ __launch_bounds__(256) void k_relu_linear_fwd(const float* __restrict__ a, const float* __restrict__ w,
                                                         const float* __restrict__ b, float* __restrict__ y,
                                                         int64_t rows, int nin, int nout, uint32_t total_waves) {
  const uint32_t wid = __builtin_amdgcn_readfirstlane(xcd_block_id() * 4u + threadIdx.x / 64u);
  if (wid >= total_waves) return;
  const int lane = threadIdx.x & 63, c = lane & 31, hq = lane >> 5;
  const int64_t r0 = (int64_t)wid * (TILES * kMT);
  const int64_t nr = min<int64_t>(TILES * kMT, rows - r0);
  const __amdgpu_buffer_rsrc_t ra = chunk_rsrc(a + r0 * nin, nr * nin * 4);
  const __amdgpu_buffer_rsrc_t ry = chunk_rsrc(y + r0 * nout, nr * nout * 4);
  float wr[NT][G][4];
  float bias[NT];
  uint32_t yc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = kMT * t + c;
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = 8 * g + 4 * hq + j;
        wr[t][g][j] = (n < nout && k < nin) ? w[(int64_t)n * nin + k] : 0.0f;
      }
    }
    bias[t] = (b != nullptr && n < nout) ? b[n] : 0.0f;
    yc[t] = n < nout ? (uint32_t)n * 4u : kOffLane;
  }
  // the lane's 16-byte column block of each row; blocks past nin read zeros
  uint32_t ka[G];
#pragma unroll
  for (int g = 0; g < G; ++g) ka[g] = 8 * g + 4 * hq < nin ? (uint32_t)(8 * g + 4 * hq) * 4u : kOffLane;

  // Tile i + 1 loads while tile i computes.  Tiles past the wave's rows load
  // zeros and their stores are dropped by the range check, so the four tiles
  // run unconditionally.
  auto load = [&](int i, f32x4 (&av)[G]) {
    const uint32_t ro = (uint32_t)((i * kMT + c) * nin) * 4u;
#pragma unroll
    for (int g = 0; g < G; ++g)
      av[g] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, ka[g] + ro, 0, 0));
  };
  auto compute_store = [&](int i, const f32x4 (&av)[G]) {
    f32x16 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x16{};
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v = av[g][j] <= 0.0f ? 0.0f : av[g][j];  // torch's relu: NaN stays NaN
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(v, wr[t][g][j], acc[t], 0, 0, 0);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t rr = (uint32_t)((i * kMT + 8 * (j / 4) + 4 * hq + (j % 4)) * nout) * 4u;
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc[t][j] + bias[t]), ry, yc[t] + rr, 0,
                                              0);
      }
    }
  };
  f32x4 av0[G], av1[G];
  load(0, av0);
#pragma unroll
  for (int i = 0; i < TILES; i += 2) {
    if (i + 1 < TILES) load(i + 1, av1);
    __builtin_amdgcn_sched_barrier(0);
    compute_store(i, av0);
    __builtin_amdgcn_sched_barrier(0);
    if (i + 2 < TILES) load(i + 2, av0);
    __builtin_amdgcn_sched_barrier(0);
    if (i + 1 < TILES) compute_store(i + 1, av1);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int G, int NT>
void launch_relu_fwd_nt(const float* a, const float* w, const float* b, float* y, int64_t rows, int nin, int nout,
                        hipStream_t st) {
  const int tiles = relu_linear_tiles(rows);
  const int64_t rows_per_wave = tiles * kMT;
  const uint32_t waves = (uint32_t)((rows + rows_per_wave - 1) / rows_per_wave);
  if (tiles == kRLTiles)
    hipLaunchKernelGGL((k_relu_linear_fwd<G, NT, kRLTiles>), dim3((waves + 3) / 4), dim3(256), 0, st, a, w, b, y,
                       rows, nin, nout, waves);
  else
    hipLaunchKernelGGL((k_relu_linear_fwd<G, NT, 1>), dim3((waves + 3) / 4), dim3(256), 0, st, a, w, b, y, rows, nin,
                       nout, waves);
  SPHOPS_LAUNCHED();
}

template <int G>
void launch_relu_fwd(const float* a, const float* w, const float* b, float* y, int64_t rows, int nin, int nout,
                     hipStream_t st) {
  if (nout <= kMT) launch_relu_fwd_nt<G, 1>(a, w, b, y, rows, nin, nout, st);
  else launch_relu_fwd_nt<G, 2>(a, w, b, y, rows, nin, nout, st);
}

}  // namespace

int64_t linear_grad_chunks(int64_t rows, int nin, int nout) { return linear_plan(rows, nin, nout).chunks; }

bool linear_grad_fits(int64_t rows, int nin, int nout) {
  const LinearPlan p = linear_plan(rows, nin, nout);
  return (int64_t)p.jobs * p.chunks <= kMaxLinearWaves;
}

void run_linear_weight_grad(const float* x, const float* dy, float* dw, float* db, int64_t rows, int nin, int nout,
                            float* work, bool relu_x, hipStream_t st) {
  const LinearPlan p = linear_plan(rows, nin, nout);
  if (p.chunks > 0) {
    switch (p.ti) {
      case 1: launch_mfma<1>(p, x, dy, work, rows, nin, nout, relu_x, st); break;
      case 2: launch_mfma<2>(p, x, dy, work, rows, nin, nout, relu_x, st); break;
      case 3: launch_mfma<3>(p, x, dy, work, rows, nin, nout, relu_x, st); break;
      default: launch_mfma<4>(p, x, dy, work, rows, nin, nout, relu_x, st); break;
    }
  }
  const int64_t nw = (int64_t)nout * nin;
  hipLaunchKernelGGL(k_chunk_reduce, dim3((uint32_t)((nw + nout + 63) / 64)), dim3(64 * kReduceWaves), 0, st, work,
                     dw, db, nw, nout, p.chunks);
  SPHOPS_LAUNCHED();
}

}  // namespace sphops

namespace sphops {

bool relu_linear_input_grad_fits(int64_t rows, int nin) {
  const int64_t rows_per_wave = relu_linear_tiles(rows) * kMT;
  return ((rows + rows_per_wave - 1) / rows_per_wave) * ((nin + 127) / 128) <= kMaxLinearWaves;
}

// K = nout padded to a multiple of 2 (the instruction's two rows) from a short
// list, so the padding wastes at most a quarter of the matrix work
void run_relu_linear_input_grad(const float* dy, const float* w, const float* h, float* dx, int64_t rows, int nin,
                                int nout, hipStream_t st) {
  if (rows == 0) return;
  if (nout <= 4) launch_relu_dx<2>(dy, w, h, dx, rows, nin, nout, st);
  else if (nout <= 8) launch_relu_dx<4>(dy, w, h, dx, rows, nin, nout, st);
  else if (nout <= 12) launch_relu_dx<6>(dy, w, h, dx, rows, nin, nout, st);
  else if (nout <= 16) launch_relu_dx<8>(dy, w, h, dx, rows, nin, nout, st);
  else if (nout <= 20) launch_relu_dx<10>(dy, w, h, dx, rows, nin, nout, st);
  else if (nout <= 24) launch_relu_dx<12>(dy, w, h, dx, rows, nin, nout, st);
  else if (nout <= 32) launch_relu_dx<16>(dy, w, h, dx, rows, nin, nout, st);
  else if (nout <= 48) launch_relu_dx<24>(dy, w, h, dx, rows, nin, nout, st);
  else launch_relu_dx<kMaxReluLinearOut / 2>(dy, w, h, dx, rows, nin, nout, st);
}

}  // namespace sphops

namespace sphops {

bool relu_linear_forward_fits(int64_t rows) {
  const int64_t rows_per_wave = relu_linear_tiles(rows) * kMT;
  return (rows + rows_per_wave - 1) / rows_per_wave <= kMaxLinearWaves;
}

// in_features padded to a multiple of 8 (16-byte blocks of two lane halves)
void run_relu_linear_forward(const float* a, const float* w, const float* b, float* y, int64_t rows, int nin,
                             int nout, hipStream_t st) {
  if (rows == 0) return;
  const int g = (nin + 7) / 8;
  if (g <= 4) launch_relu_fwd<4>(a, w, b, y, rows, nin, nout, st);
  else if (g <= 8) launch_relu_fwd<8>(a, w, b, y, rows, nin, nout, st);
  else if (g <= 12) launch_relu_fwd<12>(a, w, b, y, rows, nin, nout, st);
  else if (g <= 16) launch_relu_fwd<16>(a, w, b, y, rows, nin, nout, st);
  else if (g <= 24) launch_relu_fwd<24>(a, w, b, y, rows, nin, nout, st);
  else launch_relu_fwd<kMaxReluLinearIn / 8>(a, w, b, y, rows, nin, nout, st);
}

}  // namespace sphops
