// Backward perception kernels instantiated for 2D, clamped grids; the
// periodic ones are instantiated in perception_bwd_2d_periodic.hip, so the
// two halves compile in parallel.
#include "perception_kernels.hpp"

namespace sphops {

void run_backward_2d_periodic(const Grid& g, Op op, bool full, const int32_t* bo, const OpPtrs& a, hipStream_t st);

void run_backward_2d(const Grid& g, Op op, bool full, const int32_t* bo, const OpPtrs& a, hipStream_t st) {
  if (g.periodic) run_backward_2d_periodic(g, op, full, bo, a, st);
  else pk::backward_dispatch<2, false>(g, op, full, bo, a, st);
}

}  // namespace sphops
