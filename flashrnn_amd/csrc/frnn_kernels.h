// Kernel argument blocks and kernel lookup, shared by the kernels and the launcher.
#pragma once

#include <stdint.h>

#include "frnn_plan.h"

namespace frnn {

struct FwdArgs {
  Plan p;
  const void* wx;
  const void* R;
  const void* bias;
  const void* s0;
  void* states;
  void* carry;
  void* save;               // lane-native saved values (training, dtype p.dt_save) or null
  char* xbuf;               // exchange, both parities
  long long xbytes;
  uint32_t* claim;          // zeroed slot counters (XCD-local exchange)
  uint32_t* status;
  uint32_t spin_limit;
  unsigned long long* prof;  // phase profile (8 words) or null
};

struct BwdArgs {
  Plan p;
  const void* R;
  const void* save;         // lane-native saved values (dtype p.dt_save)
  const void* d_states;     // may be null
  const void* d_carry;      // may be null
  void* dwx;
  void* ds0;
  float* dcand;             // GRU: cotangent of the R-only candidate gate [B,T,N,D] (dR GEMM operand)
  float* dbpart;
  char* xbuf;
  long long xbytes;
  uint32_t* claim;          // zeroed slot counters (XCD-local exchange)
  uint32_t* status;
  uint32_t spin_limit;
  unsigned long long* prof;  // phase profile (8 words, after the forward's 8) or null
};

// dR[g,n,o,p] = sum over (b,t) of dG[b,t,g,n,o] h_{t-1}[b,n,p], read from the
// public dWx (GRU: gate 0 from dcand) and the forward's state output (h_{-1} = s0).
struct GemmArgs {
  Plan p;
  const void* dwx;
  const float* dcand;
  const void* states;
  const void* s0;
  float* part;
  const float* dbpart;
  void* dR;
  void* db;
  const void* zero;     // 256 zero bytes (the DMA path's source for k beyond B*T)
  const void* dcand16;  // GRU, DMA path: dcand in the MMA type
};

// dR GEMM whose operand tiles are loaded by LDS-DMA several stages ahead: 16-bit
// operands in the MMA's type (dWx, states and s0 alike; the GRU's candidate gate
// from its 16-bit copy dcand16), D % 64 == 0; null otherwise.
const void* gemm_dma_kernel(int mma);
// FP32 -> 16-bit copy (the DMA GEMM's h_{-1} rows when s0 is FP32).
const void* to16_kernel();

// Persistent recurrence kernel for (mma, k-tiles per wave) of one cell; null if not built.
const void* lstm_kernel(int mma, int ks, int ktw, int ndt, bool forward);
const void* gru_kernel(int mma, int ks, int ktw, int ndt, bool forward);
const void* elman_kernel(int mma, int ks, int ktw, int ndt, bool forward);
const void* slstm_kernel(int mma, int ks, int ktw, int ndt, bool forward);
// LDS floats per hidden-tile team of the persistent kernels (KS compute waves).
long lstm_lds_floats(bool forward, int ks);
long gru_lds_floats(bool forward, int ks);
long elman_lds_floats(bool forward, int ks);
long slstm_lds_floats(bool forward, int ks);

inline long recurrence_lds_floats(int cell, bool forward, int ks) {
  switch (cell) {
    case 0: return lstm_lds_floats(forward, ks);
    case 1: return gru_lds_floats(forward, ks);
    case 2: return elman_lds_floats(forward, ks);
    case 3: return slstm_lds_floats(forward, ks);
  }
  return 0;
}

inline const void* recurrence_kernel(int cell, int mma, int ks, int ktw, int ndt, bool forward) {
  switch (cell) {
    case 0: return lstm_kernel(mma, ks, ktw, ndt, forward);
    case 1: return gru_kernel(mma, ks, ktw, ndt, forward);
    case 2: return elman_kernel(mma, ks, ktw, ndt, forward);
    case 3: return slstm_kernel(mma, ks, ktw, ndt, forward);
  }
  return nullptr;
}
// Reduce-scatter backward kernels (frnn_bwd_rs.h) for (mma, hidden tiles per
// workgroup, compute waves per tile, output-tile class); null if not built.
const void* lstm_rs_kernel(int mma, int ndt, int ks, int ptm);
const void* gru_rs_kernel(int mma, int ndt, int ks, int ptm);
const void* elman_rs_kernel(int mma, int ndt, int ks, int ptm);
const void* slstm_rs_kernel(int mma, int ndt, int ks, int ptm);
long lstm_rs_lds_floats(int ndt);
long gru_rs_lds_floats(int ndt);
long elman_rs_lds_floats(int ndt);
long slstm_rs_lds_floats(int ndt);
inline const void* rs_kernel(int cell, int mma, int ndt, int ks, int ptm) {
  switch (cell) {
    case 0: return lstm_rs_kernel(mma, ndt, ks, ptm);
    case 1: return gru_rs_kernel(mma, ndt, ks, ptm);
    case 2: return elman_rs_kernel(mma, ndt, ks, ptm);
    case 3: return slstm_rs_kernel(mma, ndt, ks, ptm);
  }
  return nullptr;
}
inline long rs_lds_floats(int cell, int ndt) {
  switch (cell) {
    case 0: return lstm_rs_lds_floats(ndt);
    case 1: return gru_rs_lds_floats(ndt);
    case 2: return elman_rs_lds_floats(ndt);
    case 3: return slstm_rs_lds_floats(ndt);
  }
  return 0;
}

// dR GEMM: wide = 64x64 workgroup tiles (4 waves, D % 64 == 0), else 32x32 (1 wave).
const void* gemm_kernel(int mma, bool wide);
const void* reduce_kernel();
const void* zero_kernel();

}  // namespace frnn
