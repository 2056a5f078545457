// Backward perception kernels instantiated for 3D (clamped and periodic).
#include "perception_kernels.hpp"

namespace sphops {

void run_backward_3d(const Grid& g, Op op, bool full, const int32_t* bo, const OpPtrs& a, hipStream_t st) {
  if (g.periodic) pk::backward_dispatch<3, true>(g, op, full, bo, a, st);
  else pk::backward_dispatch<3, false>(g, op, full, bo, a, st);
}

}  // namespace sphops
