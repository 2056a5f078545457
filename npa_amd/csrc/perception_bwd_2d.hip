// Backward perception kernels instantiated for 2D (clamped and periodic).
#include "perception_kernels.hpp"

namespace sphops {

void run_backward_2d(const Grid& g, Op op, bool full, const int32_t* bo, const OpPtrs& a, hipStream_t st) {
  if (g.periodic) pk::backward_dispatch<2, true>(g, op, full, bo, a, st);
  else pk::backward_dispatch<2, false>(g, op, full, bo, a, st);
}

}  // namespace sphops
