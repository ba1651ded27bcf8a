// The input-projection workers (frnn_proj.h) in a launch of their own: the
// forward's fallback where they cannot run beside the recurrence (it fills the
// GPU, or needs successive launches), and frnn_fwd_projected with
// FRNN_PROJ_OVERLAP=0.
#include "frnn_proj.h"

namespace frnn {

template <int MMA>
__global__ void __launch_bounds__(256) proj_alone_kernel(ProjArgs a) {
  extern __shared__ float lds[];
  proj_wg_worker<MMA>(a, reinterpret_cast<char*>(lds));
}

int proj_lds_bytes() { return kProjLds; }

const void* proj_kernel(int mma) {
  switch (mma) {
    case MMA_BF16: return reinterpret_cast<const void*>(&proj_alone_kernel<MMA_BF16>);
    case MMA_F16: return reinterpret_cast<const void*>(&proj_alone_kernel<MMA_F16>);
  }
  return nullptr;
}

}  // namespace frnn
