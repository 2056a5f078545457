// Weight and bias gradients of a linear layer over very many rows, for the
// NPA MLP (models/npa.py:63-78 of the reference, torch.nn.Linear), for gfx950.
//
// dW = dY^T X (out x in) and db = sum over rows of dY, with X (rows x in) and
// dY (rows x out) row-major fp32.  The output is small (128 x 83 for the NPA
// MLP's first layer) and the reduction is long (one row per particle, 10^6
// at the 3D stress size); the library GEMM picks a handful of output tiles
// for that shape and leaves most of the GPU idle.  Here the rows are split
// into chunks: workgroup (tile, chunk) stages 32 rows at a time of its
// 128 x 128 output tile's dY and X columns in LDS, and each thread
// accumulates an 8 x 8 block of the tile in registers.  Each row of X and dY
// is read from HBM once per tile (once in all for layers up to 128 x 128).
// The per-chunk partial sums go to a workspace and a second kernel adds them
// in chunk order, so the result is deterministic.
#include "sphops_internal.hpp"

namespace sphops {

namespace {

constexpr int kLT = 128;        // output tile side (out and in)
constexpr int kLR = 32;         // rows staged per LDS round
constexpr int kLThreads = 256;  // 16 x 16 threads, 8 x 8 outputs each
constexpr int kLB = 8;

__global__ __launch_bounds__(kLThreads) void k_linear_partial(const float* __restrict__ x,
                                                              const float* __restrict__ dy,
                                                              float* __restrict__ part_w,
                                                              float* __restrict__ part_b, int64_t rows, int nin,
                                                              int nout, int tiles_in, int64_t chunk_rows) {
  __shared__ float4 sy[kLR][kLT / 4];  // dY rows, this tile's out columns
  __shared__ float4 sx[kLR][kLT / 4];  // X rows, this tile's in columns
  const int tile = blockIdx.x;
  const int o0 = (tile / tiles_in) * kLT, i0 = (tile % tiles_in) * kLT;
  const int64_t chunk = blockIdx.y;
  const int64_t r0 = chunk * chunk_rows;
  const int64_t r1 = min<int64_t>(rows, r0 + chunk_rows);
  const int tid = threadIdx.x;
  const int to = (tid / 16) * kLB, ti = (tid % 16) * kLB;  // this thread's 8 x 8 block in the tile
  float acc[kLB][kLB] = {};
  float accb[kLB] = {};
  const bool bias_lane = i0 == 0 && part_b != nullptr && ti == 0;
  float* sy1 = reinterpret_cast<float*>(&sy[0][0]);
  float* sx1 = reinterpret_cast<float*>(&sx[0][0]);
  for (int64_t rb = r0; rb < r1; rb += kLR) {
    const int nr = (int)min<int64_t>(kLR, r1 - rb);
    // stage kLR rows x kLT columns of each operand (zeros past the edges)
    for (int e = tid; e < kLR * kLT; e += kLThreads) {
      const int r = e / kLT, c = e % kLT;
      const bool rowok = r < nr;
      sy1[e] = (rowok && o0 + c < nout) ? dy[(rb + r) * nout + o0 + c] : 0.0f;
      sx1[e] = (rowok && i0 + c < nin) ? x[(rb + r) * nin + i0 + c] : 0.0f;
    }
    __syncthreads();
    for (int r = 0; r < nr; ++r) {
      const float4 a0 = sy[r][to / 4], a1 = sy[r][to / 4 + 1];
      const float4 b0 = sx[r][ti / 4], b1 = sx[r][ti / 4 + 1];
      const float a[kLB] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      const float b[kLB] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int u = 0; u < kLB; ++u) {
#pragma unroll
        for (int v = 0; v < kLB; ++v) acc[u][v] += a[u] * b[v];
      }
      if (bias_lane) {
#pragma unroll
        for (int u = 0; u < kLB; ++u) accb[u] += a[u];
      }
    }
    __syncthreads();
  }
  float* pw = part_w + chunk * (int64_t)nout * nin;
#pragma unroll
  for (int u = 0; u < kLB; ++u) {
    const int o = o0 + to + u;
    if (o >= nout) continue;
#pragma unroll
    for (int v = 0; v < kLB; ++v) {
      const int i = i0 + ti + v;
      if (i < nin) pw[(int64_t)o * nin + i] = acc[u][v];
    }
    if (bias_lane) part_b[chunk * nout + o] = accb[u];
  }
}

// out[e] = sum over chunks c of part[c * n + e], in a fixed order: eight
// running sums over chunks c = 8q + k (k = 0..7, eight loads in flight),
// then added k = 0..7.
__global__ __launch_bounds__(256) void k_chunk_sum(const float* __restrict__ part, float* __restrict__ out,
                                                   int64_t n, int64_t chunks) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  float s[8] = {};
  int64_t c = 0;
  for (; c + 8 <= chunks; c += 8) {
#pragma unroll
    for (int k = 0; k < 8; ++k) s[k] += part[(c + k) * n + e];
  }
  for (int k = 0; c < chunks; ++c, ++k) s[k] += part[c * n + e];
  float total = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) total += s[k];
  out[e] = total;
}

}  // namespace

// Rows per chunk: enough chunks to fill the GPU (about 1024 workgroups per
// output tile), at least 256 rows (so the partial sums stay small next to the
// inputs) and at most kMaxChunkRows, a multiple of kLR.
int64_t linear_grad_chunk_rows(int64_t rows) {
  int64_t c = (rows + 1023) / 1024;
  c = (c + kLR - 1) / kLR * kLR;
  return std::min<int64_t>(kMaxChunkRows, std::max<int64_t>(256, c));
}

int64_t linear_grad_chunks(int64_t rows) {
  return rows > 0 ? (rows + linear_grad_chunk_rows(rows) - 1) / linear_grad_chunk_rows(rows) : 0;
}

void run_linear_weight_grad(const float* x, const float* dy, float* dw, float* db, int64_t rows, int nin, int nout,
                            float* work, hipStream_t st) {
  const int64_t chunks = linear_grad_chunks(rows);
  const int64_t nw = (int64_t)nout * nin;
  float* part_w = work;
  float* part_b = db ? work + chunks * nw : nullptr;
  if (chunks > 0) {
    const int tiles_in = (nin + kLT - 1) / kLT, tiles_out = (nout + kLT - 1) / kLT;
    hipLaunchKernelGGL(k_linear_partial, dim3((uint32_t)(tiles_in * tiles_out), (uint32_t)chunks),
                       dim3(kLThreads), 0, st, x, dy, part_w, part_b, rows, nin, nout, tiles_in,
                       linear_grad_chunk_rows(rows));
    SPHOPS_LAUNCHED();
  }
  hipLaunchKernelGGL(k_chunk_sum, dim3((uint32_t)((nw + 255) / 256)), dim3(256), 0, st, part_w, dw, nw, chunks);
  SPHOPS_LAUNCHED();
  if (db) {
    hipLaunchKernelGGL(k_chunk_sum, dim3((uint32_t)((nout + 255) / 256)), dim3(256), 0, st, part_b, db,
                       (int64_t)nout, chunks);
    SPHOPS_LAUNCHED();
  }
}

}  // namespace sphops
