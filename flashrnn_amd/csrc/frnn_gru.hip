// Recurrence kernels of the gru cell: every built (operand type, contraction
// split, k-tiles per wave, hidden tiles per workgroup) variant. The planner
// picks KS = min(4, largest power of two <= D/32), 8 for the backward where
// D/32 >= 8; one-tile workgroups (widths up to 512) use k-tile classes 1, 2, 4;
// two-tile workgroups (widths 544-768) use classes 6 and 8 with KS = 3, BF16 only.
#include "frnn_kernels.h"
#include "frnn_bwd_rs.h"
#include "frnn_recurrence.h"

namespace frnn {

template <int MMA, int KTW, int NDT, int KS>
static const void* pick(bool fwd, bool proj) {
  // projection-gated forwards (frnn_proj.h): 16-bit operands
  if constexpr (MMA != MMA_F32)
    if (fwd && proj) return reinterpret_cast<const void*>(&fwd_kernel<CELL_GRU, MMA, KTW, 1, NDT, KS, true>);
  if (proj) return nullptr;
  return fwd ? reinterpret_cast<const void*>(&fwd_kernel<CELL_GRU, MMA, KTW, 1, NDT, KS, false>)
             : reinterpret_cast<const void*>(&bwd_kernel<CELL_GRU, MMA, KTW, 1, NDT, KS>);
}

template <int MMA>
static const void* by_shape(int ks, int ktw, int ndt, bool fwd, bool proj) {
  if (ndt == 1 && ks == 1 && ktw == 1) return pick<MMA, 1, 1, 1>(fwd, proj);
  if (ndt == 1 && ks == 2 && ktw == 1) return pick<MMA, 1, 1, 2>(fwd, proj);
  if (ndt == 1 && ks == 2 && ktw == 2) return pick<MMA, 2, 1, 2>(fwd, proj);
  if (ndt == 1 && ks == 4 && ktw == 1) return pick<MMA, 1, 1, 4>(fwd, proj);
  if (ndt == 1 && ks == 4 && ktw == 2) return pick<MMA, 2, 1, 4>(fwd, proj);
  if (ndt == 1 && ks == 4 && ktw == 4) return pick<MMA, 4, 1, 4>(fwd, proj);
  if (ndt == 1 && ks == 8 && ktw == 1) return pick<MMA, 1, 1, 8>(fwd, proj);
  if (ndt == 1 && ks == 8 && ktw == 2) return pick<MMA, 2, 1, 8>(fwd, proj);
  if constexpr (MMA != MMA_F32) {  // two-tile workgroups: only a 16-bit slice fits beside the runs
    if (ndt == 2 && ks == 3 && ktw == 6) return pick<MMA, 6, 2, 3>(fwd, proj);
    if (ndt == 2 && ks == 3 && ktw == 8) return pick<MMA, 8, 2, 3>(fwd, proj);
  }
  return nullptr;
}

const void* gru_kernel(int mma, int ks, int ktw, int ndt, bool forward, bool proj) {
  switch (mma) {
    case MMA_BF16: return by_shape<MMA_BF16>(ks, ktw, ndt, forward, proj);
    case MMA_F16: return by_shape<MMA_F16>(ks, ktw, ndt, forward, proj);
    case MMA_F32: return by_shape<MMA_F32>(ks, ktw, ndt, forward, proj);
  }
  return nullptr;
}

long gru_lds_floats(bool forward, int ks) {
  return forward ? Lds<CELL_GRU, 1>::fwd(ks) : Lds<CELL_GRU, 1>::bwd(ks);
}

template <int MMA, int NDT, int KS, int PTM>
static const void* pick_rs() {
  return reinterpret_cast<const void*>(&bwd_rs_kernel<CELL_GRU, MMA, NDT, KS, PTM>);
}

// Reduce-scatter backward: two-tile workgroups (widths 544-1024), where it
// replaces the all-gather backward (see frnn_bwd_rs.h).
template <int MMA>
static const void* rs_by_shape(int ndt, int ks, int ptm) {
  if (ndt == 2 && ks == 3 && ptm == 8) return pick_rs<MMA, 2, 3, 8>();
  // four compute waves per tile (ten waves: two compute waves on every SIMD
  // instead of three SIMDs with two and one with the two I/O waves)
  if (ndt == 2 && ks == 4 && ptm == 6) return pick_rs<MMA, 2, 4, 6>();
  return nullptr;
}

const void* gru_rs_kernel(int mma, int ndt, int ks, int ptm) {
  switch (mma) {
    case MMA_BF16: return rs_by_shape<MMA_BF16>(ndt, ks, ptm);
    case MMA_F16: return rs_by_shape<MMA_F16>(ndt, ks, ptm);
  }
  return nullptr;
}

long gru_rs_lds_floats(int ndt) {
  return ndt == 1 ? RsShape<CELL_GRU, 1>::floats() : RsShape<CELL_GRU, 2>::floats();
}

}  // namespace frnn
