// Backward perception kernels instantiated for 2D, periodic grids (called
// from run_backward_2d in perception_bwd_2d.hip).
#include "perception_kernels.hpp"

namespace sphops {

void run_backward_2d_periodic(const Grid& g, Op op, bool full, const int32_t* bo, const OpPtrs& a, hipStream_t st) {
  pk::backward_dispatch<2, true>(g, op, full, bo, a, st);
}

}  // namespace sphops
