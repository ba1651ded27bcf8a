// Recurrence kernels of the elman cell: every (operand type, k-tiles per wave) variant.
#include "frnn_kernels.h"
#include "frnn_recurrence.h"

namespace frnn {

template <int MMA, int KTW>
static const void* pick(bool fwd) {
  return fwd ? reinterpret_cast<const void*>(&fwd_kernel<CELL_ELMAN, MMA, KTW, 1>)
             : reinterpret_cast<const void*>(&bwd_kernel<CELL_ELMAN, MMA, KTW, 1>);
}

template <int MMA>
static const void* by_ktw(int ktw, bool fwd) {
  switch (ktw) {
    case 1: return pick<MMA, 1>(fwd);
    case 2: return pick<MMA, 2>(fwd);
    case 4: return pick<MMA, 4>(fwd);
    case 6: return pick<MMA, 6>(fwd);
    case 8: return pick<MMA, 8>(fwd);
  }
  return nullptr;
}

const void* elman_kernel(int mma, int ktw, bool forward) {
  return mma == MMA_BF16 ? by_ktw<MMA_BF16>(ktw, forward) : by_ktw<MMA_F32>(ktw, forward);
}

}  // namespace frnn
