// Forward perception kernels instantiated for 2D (clamped and periodic).
#include "perception_kernels.hpp"

namespace sphops {

void run_forward_2d(const Grid& g, Op op, const int32_t* bo, const OpPtrs& a, hipStream_t st) {
  if (g.periodic) pk::forward_dispatch<2, true>(g, op, bo, a, st);
  else pk::forward_dispatch<2, false>(g, op, bo, a, st);
}

}  // namespace sphops
