// Backward perception kernels instantiated for 3D, periodic grids (called
// from run_backward_3d in perception_bwd_3d.hip).
#include "perception_kernels.hpp"

namespace sphops {

void run_backward_3d_periodic(const Grid& g, Op op, bool full, const int32_t* bo, const OpPtrs& a, hipStream_t st) {
  pk::backward_dispatch<3, true>(g, op, full, bo, a, st);
}

}  // namespace sphops
